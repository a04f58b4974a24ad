"""GPU parity against the committed golden fixtures (``tests/golden``): the HIP
path is checked against stored answers, without running the oracle.

Bar: bit-exact for dequant, both activation quantisers, the fp4 rounding sweep
and moe_align; router ids exact (the fixture's biased scores are >1e-4 apart)
and weights within 2e-5 relative (fp32 logits against float64); the routed
layer within 1e-2 (bf16 profile) and 2e-2 (a4w4) max-relative."""

import os

import numpy as np
import pytest
import torch

from dsv4_hip import ops, synth, PROFILE_A4W4, PROFILE_BF16, RULE_CEIL_DIV6, RULE_OCP_FLOOR

pytestmark = pytest.mark.gpu

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
RULES = {"ceil_div6": RULE_CEIL_DIV6, "ocp_floor": RULE_OCP_FLOOR}


def load(name):
    return np.load(os.path.join(GOLDEN, name), allow_pickle=False)


def _bf16_dev(bits, dev):
    return torch.from_numpy(np.ascontiguousarray(bits).view(np.int16)).view(torch.bfloat16).to(dev)


def _bits(t):
    return t.detach().cpu().view(torch.int16).numpy().view(np.uint16)


def _f32(bits):
    return (np.asarray(bits, np.uint16).astype(np.uint32) << 16).view(np.float32)


def test_dequant_known_answer(gpu):
    f = load("dequant_kat.npz")
    out = ops.dequant_mxfp4(torch.from_numpy(f["packed"]).to(gpu).view(torch.int8),
                            torch.from_numpy(f["scales"]).to(gpu))
    torch.cuda.synchronize()
    assert np.array_equal(_bits(out), f["out_bf16"])


@pytest.mark.parametrize("rule", ["ceil_div6", "ocp_floor"])
def test_round_fp4_sweep(gpu, rule):
    f = load("fp4_round_sweep.npz")
    x = _bf16_dev(f["x_bf16"], gpu)
    p, s, d = ops.mxfp4_act_quant(x, RULES[rule], dq=torch.empty_like(x))
    torch.cuda.synchronize()
    assert np.all(s.cpu().numpy() == 127)
    assert np.array_equal(_f32(_bits(d)), f["out_f32"])


def test_act_quant_fp8(gpu):
    f = load("act_quant_fp8.npz")
    x = _bf16_dev(f["x_bf16"], gpu)
    r = ops.fp8_act_quant(x, 128, rt=torch.empty_like(x), want_codes=True, want_scale=True, want_e8m0x4=True)
    torch.cuda.synchronize()
    assert np.array_equal(_bits(r["rt"]), f["rt_bf16"])
    assert np.array_equal(r["codes"].cpu().numpy(), f["codes"])
    assert np.array_equal(r["scale"].cpu().numpy(), f["scale_f32"])
    assert np.array_equal(r["e8m0x4"].cpu().numpy(), np.repeat((f["scale_exp"] + 127).astype(np.uint8), 4, axis=-1))
    # the inplace form (the reference's act_quant(x, ..., inplace=True))
    ops.fp8_act_quant(x, 128, rt=x)
    torch.cuda.synchronize()
    assert np.array_equal(_bits(x), f["rt_bf16"])


@pytest.mark.parametrize("rule", ["ceil_div6", "ocp_floor"])
def test_fp4_act_quant(gpu, rule):
    f = load("fp4_act_quant.npz")
    x = _bf16_dev(f["x_bf16"], gpu)
    p, s, d = ops.mxfp4_act_quant(x, RULES[rule], dq=torch.empty_like(x))
    torch.cuda.synchronize()
    assert np.array_equal(p.cpu().numpy(), f[f"{rule}_packed"])
    assert np.array_equal(s.cpu().numpy(), f[f"{rule}_scale"])
    assert np.array_equal(_bits(d), f[f"{rule}_dq_bf16"])


@pytest.mark.parametrize("bm", [16, 64])
@pytest.mark.parametrize("id_dtype", [torch.int64, torch.int32])
def test_moe_align(gpu, bm, id_dtype):
    f = load("moe_align.npz")
    E = int(f["n_experts"])
    ids = torch.from_numpy(f["topk_ids"]).to(id_dtype).to(gpu)
    res = ops.moe_align(ids, torch.from_numpy(f["topk_w"]).to(gpu), E, bm)
    torch.cuda.synchronize()
    for key in ("order", "row", "counts", "expert_start"):
        assert np.array_equal(getattr(res, key).cpu().numpy().astype(np.int64), f[f"bm{bm}_{key}"]), key
    assert np.array_equal(res.s_w.cpu().numpy(), f[f"bm{bm}_s_w"])
    P = int(res.num_post_padded.item())
    assert P == int(f[f"bm{bm}_num_post_padded"])
    assert np.array_equal(res.sorted_ids.cpu().numpy()[:P].astype(np.int64), f[f"bm{bm}_sorted_ids"])
    assert np.array_equal(res.block_expert.cpu().numpy()[:P // bm].astype(np.int64), f[f"bm{bm}_block_expert"])
    assert int(res.status.item()) == 0


@pytest.mark.parametrize("scoring", ["softmax", "sigmoid", "sqrtsoftplus"])
def test_route(gpu, scoring):
    f = load("route.npz")
    w, ids = ops.route(_bf16_dev(f["x_bf16"], gpu), torch.from_numpy(f["gate_w"]).to(gpu), int(f["topk"]), scoring,
                       bias=torch.from_numpy(f["bias"]).to(gpu), renormalize=True, scale=float(f["scale"]))
    torch.cuda.synchronize()
    assert np.array_equal(ids.cpu().numpy().astype(np.int64), f[f"{scoring}_ids"])
    np.testing.assert_allclose(w.cpu().numpy(), f[f"{scoring}_w"], rtol=2e-5, atol=1e-7)


def _normrel(a, b):
    return float(np.abs(a - b).max() / max(np.abs(b).max(), 1e-30))


@pytest.mark.parametrize("profile,rule,tol", [("bf16", "ocp_floor", 1e-2), ("a4w4", "ocp_floor", 2e-2),
                                              ("a4w4", "ceil_div6", 2e-2)])
def test_routed_layer(gpu, profile, rule, tol):
    f = load("routed_layer.npz")
    T, D, I, E = (int(f[k]) for k in ("T", "D", "I", "E"))
    x = synth.bf16_normal(np.random.default_rng(int(f["x_seed"])), (T, D))
    assert np.array_equal(x.view(torch.int16).numpy().view(np.uint16), f["x_bf16"])
    import hashlib
    devw = {}
    for e in range(E):
        d = synth.expert_weights(e, D, I)
        for name, arr in d.items():
            assert hashlib.sha256(np.ascontiguousarray(arr).tobytes()).hexdigest() == str(f[f"sha_e{e}_{name}"])
        devw[e] = {k: torch.from_numpy(v).to(gpu) for k, v in d.items()}
    runner = ops.LayerRunner(gpu, E, D, I)
    y = runner.forward(x.to(gpu), torch.from_numpy(f["topk_ids"]).to(gpu), torch.from_numpy(f["topk_w"]).to(gpu),
                       ops.expert_table(devw, E, gpu), profile=PROFILE_BF16 if profile == "bf16" else PROFILE_A4W4,
                       rule=RULES[rule])
    torch.cuda.synchronize()
    want = f["y_bf16"] if profile == "bf16" else f[f"y_a4w4_{rule}"]
    r = _normrel(_f32(_bits(y)), _f32(want))
    assert r <= tol, r
