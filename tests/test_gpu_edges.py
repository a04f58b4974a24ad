"""GPU edge cases of the routed layer against the oracle: one token with one
pick, the largest expert count (512), experts whose table entry is empty (they
contribute zeros) and routed ids outside [0, E) (skipped by the align, counted
in its status, and adding nothing to the combine)."""

import numpy as np
import pytest
import torch

from oracle import moe as M
from oracle import mxfp4 as Q
from dsv4_hip import ops, synth, AFMT_E2M1, AFMT_E4M3, PROFILE_A4W4, PROFILE_BF16, RULE_OCP_FLOOR

pytestmark = pytest.mark.gpu

TOL = {"bf16": 1e-2, "a4w4": 2e-2}


def rel(a, b):
    return float(np.abs(a - b).max() / max(np.abs(b).max(), 1e-30))


def _bits(t):
    return t.detach().cpu().view(torch.int16).numpy().view(np.uint16)


def _ref(profile, xb, ids, w, host, E):
    if profile == "bf16":
        return M.routed_bf16(xb, ids, w, host, n_experts=E)["y"]
    return M.routed_a4w4(xb, ids, w, host, n_experts=E, rule="ocp_floor")["y"]


def _run(profile, x, ids, w, table, E, D, I, dev):
    runner = ops.LayerRunner(dev, E, D, I)
    prof = PROFILE_BF16 if profile == "bf16" else PROFILE_A4W4
    y = runner.forward(x.to(dev), torch.from_numpy(ids).to(dev), torch.from_numpy(w).to(dev), table, profile=prof,
                       rule=RULE_OCP_FLOOR)
    torch.cuda.synchronize()
    return Q.bf16_bits_to_f32(_bits(y))


@pytest.mark.parametrize("profile", ["bf16", "a4w4"])
@pytest.mark.parametrize("T,K,E,D,I", [(1, 1, 16, 512, 512), (1, 8, 256, 4096, 2048), (16, 8, 512, 512, 512),
                                       (5, 3, 48, 1024, 1024)])
def test_layer_small_and_wide(gpu, profile, T, K, E, D, I):
    ids = synth.zipf_topk(T, K, E, synth.rank_permutation(E, 3), np.random.default_rng(T + E))
    w = synth.routing_weights(T, K, 9)
    x = synth.bf16_normal(np.random.default_rng(2), (T, D))
    xb = x.view(torch.int16).numpy().view(np.uint16)
    host = {int(e): synth.expert_weights(int(e), D, I) for e in np.unique(ids)}
    devw = {e: {k: torch.from_numpy(v).to(gpu) for k, v in d.items()} for e, d in host.items()}
    got = _run(profile, x, ids, w, ops.expert_table(devw, E, gpu), E, D, I, gpu)
    want = Q.bf16_bits_to_f32(_ref(profile, xb, ids, w, host, E))
    assert rel(got, want) <= TOL[profile], rel(got, want)


def _zero_expert(D, I):
    z = synth.expert_weights(0, D, I)
    return {k: np.zeros_like(v) if k.endswith("p") else v for k, v in z.items()}


@pytest.mark.parametrize("profile", ["bf16", "a4w4"])
def test_missing_experts_contribute_zeros(gpu, profile):
    # the table's entries for two routed experts are empty (null pointers): their
    # rows are zero, as an expert with all-zero weights gives in the oracle
    T, K, E, D, I = 12, 4, 32, 1024, 512
    ids = synth.zipf_topk(T, K, E, synth.rank_permutation(E, 3), np.random.default_rng(5))
    w = synth.routing_weights(T, K, 6)
    x = synth.bf16_normal(np.random.default_rng(7), (T, D))
    xb = x.view(torch.int16).numpy().view(np.uint16)
    used = np.unique(ids)
    missing = set(int(e) for e in used[:2])
    host = {int(e): synth.expert_weights(int(e), D, I) for e in used}
    devw = {e: {k: torch.from_numpy(v).to(gpu) for k, v in d.items()} for e, d in host.items() if e not in missing}
    got = _run(profile, x, ids, w, ops.expert_table(devw, E, gpu), E, D, I, gpu)
    ref_host = {e: (_zero_expert(D, I) if e in missing else d) for e, d in host.items()}
    want = Q.bf16_bits_to_f32(_ref(profile, xb, ids, w, ref_host, E))
    assert rel(got, want) <= TOL[profile], rel(got, want)
    full = Q.bf16_bits_to_f32(_ref(profile, xb, ids, w, host, E))
    assert not np.allclose(got, full)                  # the missing experts did matter


@pytest.mark.parametrize("n_rows_T", [12, 400])   # single-workgroup align / chunked align
def test_out_of_range_ids_add_nothing(gpu, n_rows_T):
    T, K, E, D, I = n_rows_T, 8, 32, 1024, 512
    ids = synth.zipf_topk(T, K, E, synth.rank_permutation(E, 3), np.random.default_rng(11))
    w = synth.routing_weights(T, K, 12)
    bad = ids.copy()
    bad[0, 3] = E          # above the range
    bad[T - 1, 0] = -1     # below it
    x = synth.bf16_normal(np.random.default_rng(13), (T, D))
    xb = x.view(torch.int16).numpy().view(np.uint16)
    host = {int(e): synth.expert_weights(int(e), D, I) for e in np.unique(ids)}
    devw = {e: {k: torch.from_numpy(v).to(gpu) for k, v in d.items()} for e, d in host.items()}
    got = _run("bf16", x, bad, w, ops.expert_table(devw, E, gpu), E, D, I, gpu)
    # oracle: the two entries go to an extra expert with all-zero weights
    ref_ids = bad.copy()
    ref_ids[ref_ids < 0] = E
    ref_ids[ref_ids >= E] = E
    ref_host = dict(host)
    ref_host[E] = _zero_expert(D, I)
    want = Q.bf16_bits_to_f32(M.routed_bf16(xb, ref_ids, w, ref_host, n_experts=E + 1)["y"])
    assert rel(got, want) <= TOL["bf16"], rel(got, want)
    al = ops.moe_align(torch.from_numpy(bad).to(gpu), torch.from_numpy(w).to(gpu), E, 16)
    torch.cuda.synchronize()
    assert int(al.status.item()) == 2


@pytest.mark.parametrize("bm", [16, 64, 128, 256])
@pytest.mark.parametrize("profile", ["bf16", "a4w4"])
def test_missing_experts_gemm_rows(gpu, profile, bm):
    # every kernel (16-row, 64/128-row tiled, 256-row large-tile) on a table with three
    # routed experts empty, among them the one with the most rows: their rows of h and
    # of the down output are exactly zero, every other row bit for bit what the full
    # table gives
    T, K, E, D, I = 300, 6, 24, 2048, 1024
    ids = synth.zipf_topk(T, K, E, synth.rank_permutation(E, 3), np.random.default_rng(21))
    w = synth.routing_weights(T, K, 22)
    x = synth.bf16_normal(np.random.default_rng(23), (T, D)).to(gpu)
    counts = np.bincount(ids.reshape(-1), minlength=E)
    used = np.unique(ids)
    missing = {int(np.argmax(counts)), int(used[0]), int(used[-1])}
    devw = {int(e): {k: torch.from_numpy(v).to(gpu) for k, v in synth.expert_weights(int(e), D, I).items()}
            for e in used}
    full = ops.expert_table(devw, E, gpu)
    part = ops.expert_table({e: d for e, d in devw.items() if e not in missing}, E, gpu)
    al = ops.moe_align(torch.from_numpy(ids).to(gpu), torch.from_numpy(w).to(gpu), E, bm)
    wf = torch.from_numpy(w.reshape(-1)).to(gpu)
    if profile == "bf16":
        q = ops.fp8_act_quant(x, 128, want_codes=True, want_e8m0x4=True)
        a, a_s, afmt = q["codes"], q["e8m0x4"], AFMT_E4M3
    else:
        a, a_s, _ = ops.mxfp4_act_quant(x, RULE_OCP_FLOOR)
        afmt = AFMT_E2M1
    h_full = ops.gemm_gateup(afmt, a, a_s, K, al, full, D, I, wf, 10.0)
    h_part = ops.gemm_gateup(afmt, a, a_s, K, al, part, D, I, wf, 10.0)
    if profile == "bf16":
        q = ops.fp8_act_quant(h_full, 128, want_codes=True, want_e8m0x4=True)
        ha, has = q["codes"], q["e8m0x4"]
    else:
        ha, has, _ = ops.mxfp4_act_quant(h_full, RULE_OCP_FLOOR)
    o_full = ops.gemm_down(afmt, ha, has, al, full, I, D)
    o_part = ops.gemm_down(afmt, ha, has, al, part, I, D)
    torch.cuda.synchronize()
    gone = torch.from_numpy(np.isin(ids.reshape(-1), list(missing))).to(gpu)
    print(f"{profile} bm={bm}: {int(gone.sum())} of {T * K} rows on missing experts {sorted(missing)}")
    for name, got, ref in (("h", h_part, h_full), ("down", o_part, o_full)):
        assert float(got[gone].float().abs().max()) == 0.0, f"{name}: rows of missing experts are not zero"
        assert torch.equal(got.view(torch.int16)[~gone], ref.view(torch.int16)[~gone]), \
            f"{name}: rows of present experts differ"
