"""The oracle and the input generators against the committed golden fixtures
(``tests/golden``, written by ``tests/golden/make_golden.py``).

Integer, byte and bf16-code outputs must match bit for bit. The oracle sums in
float64 and rounds to fp32, so GEMM sums do not depend on the BLAS build; the
SwiGLU and scoring functions go through numpy's ``exp``, whose last bit may
differ between CPU builds, so the routed layer is compared normwise to 1e-3 (a
single bf16 rounding flip moves one element by 2^-8) and the router weights to
rtol 1e-12."""

import json
import os

import numpy as np
import pytest

from oracle import lru as L
from oracle import moe as M
from oracle import mxfp4 as Q
from oracle import routing as RT

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def load(name):
    return np.load(os.path.join(GOLDEN, name), allow_pickle=False)


def test_dequant_known_answer():
    f = load("dequant_kat.npz")
    assert np.array_equal(Q.dequant_fp4_weight(f["packed"], f["scales"]), f["out_bf16"])


@pytest.mark.parametrize("rule", ["ceil_div6", "ocp_floor"])
def test_round_fp4_sweep(rule):
    f = load("fp4_round_sweep.npz")
    dq, _, sc = Q.dynamic_mx_quant(f["x_bf16"], rule)
    assert np.all(sc == 127)
    assert np.array_equal(Q.bf16_bits_to_f32(dq), f["out_f32"])
    # the sweep row itself: the reference's own -6..6 step 0.01 values, rounded to bf16
    assert f["x_bf16"].shape[1] >= 1201 + 1201 // 31


def test_act_quant_fp8():
    f = load("act_quant_fp8.npz")
    rt, codes, s, k = Q.act_quant(f["x_bf16"], 128)
    assert np.array_equal(rt, f["rt_bf16"])
    assert np.array_equal(codes, f["codes"])
    assert np.array_equal(s.astype(np.float32), f["scale_f32"])
    assert np.array_equal(k.astype(np.int32), f["scale_exp"])


@pytest.mark.parametrize("rule", ["ceil_div6", "ocp_floor"])
def test_fp4_act_quant(rule):
    f = load("fp4_act_quant.npz")
    dq, packed, sc = Q.dynamic_mx_quant(f["x_bf16"], rule)
    assert np.array_equal(dq, f[f"{rule}_dq_bf16"])
    assert np.array_equal(packed, f[f"{rule}_packed"])
    assert np.array_equal(sc, f[f"{rule}_scale"])


@pytest.mark.parametrize("bm", [16, 64])
def test_moe_align(bm):
    f = load("moe_align.npz")
    r = RT.moe_align(f["topk_ids"], f["topk_w"], int(f["n_experts"]), bm)
    for key in ("order", "row", "counts", "sorted_ids", "block_expert", "expert_start"):
        assert np.array_equal(np.asarray(r[key], np.int64), f[f"bm{bm}_{key}"]), key
    assert np.array_equal(np.asarray(r["s_w"], np.float32), f[f"bm{bm}_s_w"])
    assert int(r["num_post_padded"]) == int(f[f"bm{bm}_num_post_padded"])
    assert f[f"bm{bm}_counts"][9] == 0  # the fixture keeps one expert empty


@pytest.mark.parametrize("scoring", ["softmax", "sigmoid", "sqrtsoftplus"])
def test_route(scoring):
    f = load("route.npz")
    w, ids, _ = RT.route(f["x_bf16"], f["gate_w"], int(f["topk"]), scoring, bias=f["bias"], renormalize=True,
                         scale=float(f["scale"]))
    assert np.array_equal(ids, f[f"{scoring}_ids"])
    np.testing.assert_allclose(w, f[f"{scoring}_w"], rtol=1e-12)


def _layer_inputs(f):
    from dsv4_hip import synth
    import torch
    T, D, I, E = (int(f[k]) for k in ("T", "D", "I", "E"))
    x = synth.bf16_normal(np.random.default_rng(int(f["x_seed"])), (T, D))
    xb = x.view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(xb, f["x_bf16"]), "the bf16 input generator changed"
    experts = {e: synth.expert_weights(e, D, I) for e in range(E)}
    import hashlib
    for e, d in experts.items():
        for name, arr in d.items():
            got = hashlib.sha256(np.ascontiguousarray(arr).tobytes()).hexdigest()
            assert got == str(f[f"sha_e{e}_{name}"]), f"the expert generator changed (expert {e}, {name})"
    return xb, experts


def _normrel(a, b):
    return float(np.abs(a - b).max() / max(np.abs(b).max(), 1e-30))


def test_routed_layer():
    f = load("routed_layer.npz")
    xb, experts = _layer_inputs(f)
    E = int(f["E"])
    y = M.routed_bf16(xb, f["topk_ids"], f["topk_w"], experts, n_experts=E)["y"]
    assert _normrel(Q.bf16_bits_to_f32(y), Q.bf16_bits_to_f32(f["y_bf16"])) <= 1e-3
    for rule in ("ocp_floor", "ceil_div6"):
        y4 = M.routed_a4w4(xb, f["topk_ids"], f["topk_w"], experts, n_experts=E, rule=rule)["y"]
        assert _normrel(Q.bf16_bits_to_f32(y4), Q.bf16_bits_to_f32(f[f"y_a4w4_{rule}"])) <= 1e-3


def test_lru_known_answer_oracle_and_native():
    with open(os.path.join(GOLDEN, "lru_kat.json")) as fh:
        kat = json.load(fh)
    o = L.LRUOracle(kat["capacity"])
    from dsv4_hip.slots import HostLRU
    nat = HostLRU(kat["capacity"])
    for step in kat["trace"]:
        key = tuple(step["key"])
        hit, ev = o.access(key)
        assert hit == step["hit"] and (None if ev is None else list(ev)) == step["evicted"]
        nhit, _, nev = nat.access(1000 * key[0] + key[1])
        want_ev = None if step["evicted"] is None else 1000 * step["evicted"][0] + step["evicted"][1]
        assert nhit == step["hit"]
        assert (nev is None) == (want_ev is None)
    s = o.stats()
    assert [list(k) for k in o.cache.keys()] == kat["cached_after"]
    assert nat.keys() == [1000 * k[0] + k[1] for k in kat["cached_after"]]
    assert (s["hits"], s["misses"], s["evictions"]) == (kat["hits"], kat["misses"], kat["evictions"])
    assert s["hit_rate"] == kat["hit_rate"]
    z = L.LRUOracle(0)
    z.access((0, 0))
    z.access((0, 0))
    assert z.stats()["misses"] == kat["capacity0_misses"] and z.stats()["cached"] == kat["capacity0_cached"]
