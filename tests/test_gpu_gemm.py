"""GPU parity of the grouped GEMMs and the fused routed layer.

Tolerance: normwise max relative error
    rel = max|gpu - oracle| / max|oracle|
<= 1e-2 for the bf16 profile and <= 2e-2 for the a4w4 profile. Stage tests
feed the GPU kernel and the oracle the *same* quantised operands, so the only
difference is fp32 summation order and the bf16 roundings that follow it; they
must also meet a per-element bar (``_parity``). a4w4: the down GEMM bit for
bit (every product and partial sum is exact), h within one bf16 ulp (the
kernel's expf and numpy's exp may round apart). bf16 profile (E4M3 x E2M1 MFMA): each down
output within one bf16 ulp plus 2^-10 of its sum of absolute products (the
MFMA drops products far below the largest of their group), the gate/up
GEMM's h within one ulp plus that bound carried through SwiGLU from its gate
and up values. The end-to-end tests start from the same bf16 x and routing:
a4w4 bit for bit; bf16 per element within 3e-2 of max(|ref|, rms(ref)).
"""

import numpy as np
import pytest
import torch

from oracle import mxfp4 as Q
from oracle import moe as M
from _parity import check_bound, elementwise_rel, gemm_bound, swiglu_bound
from dsv4_hip import (ops, synth, AFMT_E2M1, AFMT_E4M3, PROFILE_A4W4, PROFILE_BF16, PROFILE_BF16_PURE,
                      RULE_OCP_FLOOR, RULE_CEIL_DIV6)

pytestmark = pytest.mark.gpu

TOL = {"bf16": 1e-2, "a4w4": 2e-2, "bf16_pure": 1e-2}
# per-element relative error with a floor of rms(output) (_parity.elementwise_rel); a4w4: bit for bit;
# the pure-bf16 variant has no quantisation step for a 1-ulp difference to move
ELEM_TOL = {"bf16": 3e-2, "a4w4": 0.0, "bf16_pure": 2e-2}


def rel(a, b):
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    return float(np.abs(a - b).max() / max(np.abs(b).max(), 1e-30))


def _bits(t):
    return t.detach().cpu().contiguous().view(torch.int16).numpy().view(np.uint16)


def _dev_bf16(bits, dev):
    return torch.from_numpy(np.ascontiguousarray(bits, np.uint16).view(np.int16)).view(torch.bfloat16).to(dev)


def _dev(a, dev):
    return torch.from_numpy(np.ascontiguousarray(a)).to(dev)


def make_layer(E, D, I, experts_needed, dev):
    host = {e: synth.expert_weights(int(e), D, I) for e in experts_needed}
    devw = {e: {k: _dev(v, dev) for k, v in d.items()} for e, d in host.items()}
    return host, devw, ops.expert_table(devw, E, dev)


def _case(T, K, E, D, I, seed, dev):
    ids = synth.zipf_topk(T, K, E, synth.rank_permutation(E, 3), np.random.default_rng(seed))
    w = synth.routing_weights(T, K, seed + 1)
    x = synth.bf16_normal(np.random.default_rng(seed + 2), (T, D))
    xb = x.view(torch.int16).numpy().view(np.uint16)
    host, devw, table = make_layer(E, D, I, np.unique(ids), dev)
    return ids, w, xb, host, devw, table


@pytest.mark.parametrize("profile", ["bf16", "a4w4"])
@pytest.mark.parametrize("T,K,E,D,I,bm", [(24, 4, 16, 1024, 512, 16), (200, 8, 16, 512, 512, 16),
                                          (8, 8, 256, 4096, 2048, 16), (200, 8, 16, 512, 512, 64),
                                          (200, 8, 16, 1024, 512, 128), (300, 6, 24, 2048, 1024, 64),
                                          (200, 8, 16, 1024, 1024, 256), (300, 6, 24, 2048, 1024, 256),
                                          (640, 8, 8, 4096, 2048, 256)])
def test_grouped_gemm_stages(gpu, profile, T, K, E, D, I, bm):
    # bm 16 runs the single-wave decode kernel, 64/128 the LDS-tiled kernel, 256 the
    # large-tile kernel (256 x 256 workgroup tiles, 32x32x64 MFMA) in half-block
    # workgroups (E4M3 always, E2M1 below 32,768 routed rows)
    _stage_case(gpu, profile, T, K, E, D, I, bm)


def test_grouped_gemm_stages_whole_blocks_a4w4(gpu):
    # from 32,768 routed rows the E2M1 large-tile kernel runs one 8-wave workgroup
    # per whole 256-row block (csrc/gemm_big.hip launch_moe_gemm_big); every element
    # of both stages against the oracle, the down GEMM bit for bit
    _stage_case(gpu, "a4w4", 4096, 8, 16, 1024, 1024, 256)


def _stage_case(gpu, profile, T, K, E, D, I, bm):
    ids, w, xb, host, devw, table = _case(T, K, E, D, I, 31 + T, gpu)
    al = ops.moe_align(_dev(ids, gpu), _dev(w, gpu), E, bm)
    R = T * K
    if profile == "bf16":
        rt, codes, s, k = Q.act_quant(xb, 128)
        a_f = Q.bf16_bits_to_f32(rt)
        a = _dev(codes, gpu)
        a_s = _dev(np.repeat((k + 127).astype(np.uint8), 4, axis=-1), gpu)
        afmt = AFMT_E4M3
    else:
        _, packed, sc = Q.ocp_mx_quant(xb, 32)
        a_f = Q.fp4_codes_to_f32(packed, sc)
        a, a_s, afmt = _dev(packed, gpu), _dev(sc, gpu), AFMT_E2M1
    h = ops.gemm_gateup(afmt, a, a_s, K, al, table, D, I, _dev(w.reshape(-1), gpu), 10.0)
    torch.cuda.synchronize()
    # oracle gate/up + SwiGLU for each flat row on the same quantised x
    flat_e = ids.reshape(-1)
    h_ref = np.zeros((R, I), np.float32)
    g_all, u_all = np.zeros((R, I), np.float32), np.zeros((R, I), np.float32)
    g_abs, u_abs = np.zeros((R, I), np.float32), np.zeros((R, I), np.float32)
    for e in np.unique(flat_e):
        rows = np.nonzero(flat_e == e)[0]
        w1 = Q.dequant_fp4_weight_f32(host[e]["w1p"], host[e]["w1s"])
        w3 = Q.dequant_fp4_weight_f32(host[e]["w3p"], host[e]["w3s"])
        xa = a_f[rows // K]
        g = Q.f32_to_bf16_f32(M.matmul_nt(xa, w1))
        u = Q.f32_to_bf16_f32(M.matmul_nt(xa, w3))
        g_all[rows], u_all[rows] = g, u
        g_abs[rows], u_abs[rows] = M.matmul_nt(np.abs(xa), np.abs(w1)), M.matmul_nt(np.abs(xa), np.abs(w3))
        h_ref[rows] = M.swiglu(g, u, w.reshape(-1)[rows], 10.0)
    h_gpu = Q.bf16_bits_to_f32(_bits(h))
    h_want = Q.f32_to_bf16_f32(h_ref)
    print(f"gate/up {profile} T={T} bm={bm}: normwise rel {rel(h_gpu, h_want):.3e}")
    assert rel(h_gpu, h_want) <= TOL[profile]
    # a4w4: g and u are exact; h may still flip one ulp where the kernel's expf and
    # numpy's exp round differently, so both profiles take the SwiGLU bound
    check_bound(h_gpu, h_want, swiglu_bound(g_all, u_all, w.reshape(-1), 10.0, h_want,
                                            g_abs if profile == "bf16" else None,
                                            u_abs if profile == "bf16" else None),
                f"gate/up {profile} bm={bm}")
    # down GEMM on the oracle's quantised h
    hb = Q.f32_to_bf16_bits(h_ref)
    if profile == "bf16":
        hrt, hc, hs, hk = Q.act_quant(hb, 128)
        ha_f = Q.bf16_bits_to_f32(hrt)
        ha, has = _dev(hc, gpu), _dev(np.repeat((hk + 127).astype(np.uint8), 4, axis=-1), gpu)
    else:
        _, hp, hsc = Q.ocp_mx_quant(hb, 32)
        ha_f = Q.fp4_codes_to_f32(hp, hsc)
        ha, has = _dev(hp, gpu), _dev(hsc, gpu)
    out = ops.gemm_down(afmt, ha, has, al, table, I, D)
    torch.cuda.synchronize()
    out_ref = np.zeros((R, D), np.float32)
    out_abs = np.zeros((R, D), np.float32)
    for e in np.unique(flat_e):
        rows = np.nonzero(flat_e == e)[0]
        w2 = Q.dequant_fp4_weight_f32(host[e]["w2p"], host[e]["w2s"])
        out_ref[rows] = M.matmul_nt(ha_f[rows], w2)
        out_abs[rows] = M.matmul_nt(np.abs(ha_f[rows]), np.abs(w2))
    out_gpu, out_want = Q.bf16_bits_to_f32(_bits(out)), Q.f32_to_bf16_f32(out_ref)
    print(f"down {profile} T={T} bm={bm}: normwise rel {rel(out_gpu, out_want):.3e}")
    assert rel(out_gpu, out_want) <= TOL[profile]
    if profile == "a4w4":
        assert np.array_equal(out_gpu, out_want), "a4w4 down: not bit-exact"
    else:
        check_bound(out_gpu, out_want, gemm_bound(out_want, out_abs), f"down {profile} bm={bm}")


def test_grouped_gemm_empty_group_pattern(gpu):
    # _bench_gmm.py:8-22: groups [2, 0, 3] -> expert 1 receives no rows
    E, D, I, K = 3, 512, 512, 1
    ids = np.array([[0], [0], [2], [2], [2]], np.int64)
    w = np.ones((5, 1), np.float32)
    xb = synth.bf16_normal(np.random.default_rng(0), (5, D)).view(torch.int16).numpy().view(np.uint16)
    host, devw, table = make_layer(E, D, I, [0, 2], gpu)
    al = ops.moe_align(_dev(ids, gpu), _dev(w, gpu), E, 16)
    rt, codes, s, k = Q.act_quant(xb, 128)
    h = ops.gemm_gateup(AFMT_E4M3, _dev(codes, gpu), _dev(np.repeat((k + 127).astype(np.uint8), 4, -1), gpu), K,
                        al, table, D, I, _dev(w.reshape(-1), gpu), 10.0)
    torch.cuda.synchronize()
    a_f = Q.bf16_bits_to_f32(rt)
    for e, rows in ((0, [0, 1]), (2, [2, 3, 4])):
        w1 = Q.dequant_fp4_weight_f32(host[e]["w1p"], host[e]["w1s"])
        w3 = Q.dequant_fp4_weight_f32(host[e]["w3p"], host[e]["w3s"])
        g = Q.f32_to_bf16_f32(M.matmul_nt(a_f[rows], w1))
        u = Q.f32_to_bf16_f32(M.matmul_nt(a_f[rows], w3))
        ref = M.swiglu(g, u, np.ones(len(rows), np.float32), 10.0)
        assert rel(Q.bf16_bits_to_f32(_bits(h))[rows], ref) <= 1e-2


@pytest.mark.parametrize("profile", ["bf16", "a4w4", "bf16_pure"])
@pytest.mark.parametrize("T,K,E,D,I", [(8, 8, 256, 4096, 2048), (64, 6, 32, 1024, 512), (100, 6, 32, 1024, 512),
                                       (256, 8, 32, 2048, 1024), (400, 8, 256, 1024, 512)])
def test_layer_forward_vs_oracle(gpu, profile, T, K, E, D, I):
    # 16-row blocks up to 2047 routed rows (h quantised in the gate/up epilogue for a4w4,
    # by a separate launch for FP8); 256 tokens x top-8 = 2048 routed rows: 64-row M blocks
    # (tiled kernel, h quantised in the epilogue in both profiles); 3200 routed rows: the
    # chunked two-launch align. The pure-bf16 variant takes the same block sizes (no h
    # quantisation: its down GEMM reads bf16 h).
    ids, w, xb, host, devw, table = _case(T, K, E, D, I, 77 + T, gpu)
    runner = ops.LayerRunner(gpu, E, D, I)
    x = _dev_bf16(xb, gpu)
    prof = {"bf16": PROFILE_BF16, "a4w4": PROFILE_A4W4, "bf16_pure": PROFILE_BF16_PURE}[profile]
    y = runner.forward(x, _dev(ids, gpu), _dev(w, gpu), table, profile=prof, rule=RULE_OCP_FLOOR)
    torch.cuda.synchronize()
    if profile == "bf16":
        ref = M.routed_bf16(xb, ids, w, host, n_experts=E)
    elif profile == "bf16_pure":
        ref = M.routed_bf16(xb, ids, w, host, n_experts=E, fp8_act=False)
    else:
        ref = M.routed_a4w4(xb, ids, w, host, n_experts=E, rule="ocp_floor")
    got = Q.bf16_bits_to_f32(_bits(y))
    want = Q.bf16_bits_to_f32(ref["y"])
    er = elementwise_rel(got, want)
    print(f"layer {profile} T={T} K={K} E={E} D={D} I={I}: normwise rel {rel(got, want):.3e}, "
          f"elementwise rel {er:.3e}")
    assert rel(got, want) <= TOL[profile], rel(got, want)
    assert er <= ELEM_TOL[profile], er
    if profile == "a4w4":
        assert np.array_equal(_bits(y), ref["y"])


def test_layer_forward_ceil_rule_and_int32_ids(gpu):
    T, K, E, D, I = 16, 4, 16, 512, 512
    ids, w, xb, host, devw, table = _case(T, K, E, D, I, 5, gpu)
    runner = ops.LayerRunner(gpu, E, D, I)
    y = runner.forward(_dev_bf16(xb, gpu), _dev(ids.astype(np.int32), gpu), _dev(w, gpu), table,
                       profile=PROFILE_A4W4, rule=RULE_CEIL_DIV6)
    torch.cuda.synchronize()
    ref = M.routed_a4w4(xb, ids, w, host, n_experts=E, rule="ceil_div6")
    assert rel(Q.bf16_bits_to_f32(_bits(y)), Q.bf16_bits_to_f32(ref["y"])) <= TOL["a4w4"]


# ---- the pure-bf16 variant: bf16 activations as they are on the bf16 MFMA ----
# Products of a bf16 value and an exactly dequantised E2M1 weight are exact in fp32 and
# the MFMA accumulates in fp32, so each output is within one bf16 ulp of the float64
# oracle plus 2^-16 of its sum of absolute products (fp32 summation over K <= 4096).
PURE_ACC_REL = 2.0 ** -16


_PURE_SHAPES = [(24, 4, 16, 1024, 512), (8, 8, 256, 4096, 2048), (200, 8, 16, 512, 512), (300, 8, 8, 2048, 1024)]


@pytest.mark.parametrize("T,K,E,D,I,block_m", [s + (bm,) for bm in (16, 64) for s in _PURE_SHAPES] +
                         [(40, 4, 8, 1024, 384, 64)] +
                         [(8, 8, 256, 4096, 2048, 256), (300, 8, 8, 2048, 1024, 256), (1024, 8, 8, 1024, 1024, 256)])
def test_grouped_gemm_stages_bf16_pure(gpu, T, K, E, D, I, block_m):
    # 16-row blocks: the single-wave kernel; 64-row blocks: the LDS-tiled kernel
    # (bf16 A tile in LDS, weight fragments dequantised once per 32-k half, weight
    # scales through a per-wave LDS table; 8-wave workgroups where the columns
    # divide by 256 (gate/up) or 512 (down), 4-wave ones otherwise: I = 384 runs a
    # 4-wave gate/up, and no down, whose reduction length must be a multiple of 256); 256-row
    # blocks: the large-tile bf16 kernel (32x32x16 bf16 MFMAs, weight fragments
    # dequantised in registers per 16-k chunk; hidden and inter multiples of 1024)
    from dsv4_hip import AFMT_BF16
    ids, w, xb, host, devw, table = _case(T, K, E, D, I, 71 + T, gpu)
    al = ops.moe_align(_dev(ids, gpu), _dev(w, gpu), E, block_m)
    R = T * K
    x = _dev_bf16(xb, gpu)
    h = ops.gemm_gateup(AFMT_BF16, x, None, K, al, table, D, I, _dev(w.reshape(-1), gpu), 10.0)
    torch.cuda.synchronize()
    a_f = Q.bf16_bits_to_f32(xb)
    flat_e = ids.reshape(-1)
    h_ref = np.zeros((R, I), np.float32)
    g_all, u_all = np.zeros((R, I), np.float32), np.zeros((R, I), np.float32)
    g_abs, u_abs = np.zeros((R, I), np.float32), np.zeros((R, I), np.float32)
    for e in np.unique(flat_e):
        rows = np.nonzero(flat_e == e)[0]
        w1 = Q.dequant_fp4_weight_f32(host[e]["w1p"], host[e]["w1s"])
        w3 = Q.dequant_fp4_weight_f32(host[e]["w3p"], host[e]["w3s"])
        xa = a_f[rows // K]
        g = Q.f32_to_bf16_f32(M.matmul_nt(xa, w1))
        u = Q.f32_to_bf16_f32(M.matmul_nt(xa, w3))
        g_all[rows], u_all[rows] = g, u
        g_abs[rows], u_abs[rows] = M.matmul_nt(np.abs(xa), np.abs(w1)), M.matmul_nt(np.abs(xa), np.abs(w3))
        h_ref[rows] = M.swiglu(g, u, w.reshape(-1)[rows], 10.0)
    h_gpu = Q.bf16_bits_to_f32(_bits(h))
    h_want = Q.f32_to_bf16_f32(h_ref)
    print(f"pure bf16 gate/up T={T} block_m={block_m}: normwise rel {rel(h_gpu, h_want):.3e}")
    check_bound(h_gpu, h_want, swiglu_bound(g_all, u_all, w.reshape(-1), 10.0, h_want, g_abs, u_abs,
                                            acc_rel=PURE_ACC_REL), f"pure bf16 gate/up T={T} block_m={block_m}")
    if I % 256:
        return
    # down on the oracle's bf16 h, as it is
    hb = Q.f32_to_bf16_bits(h_ref)
    out = ops.gemm_down(AFMT_BF16, _dev_bf16(hb, gpu), None, al, table, I, D)
    torch.cuda.synchronize()
    hf = Q.bf16_bits_to_f32(hb)
    out_ref = np.zeros((R, D), np.float32)
    out_abs = np.zeros((R, D), np.float32)
    for e in np.unique(flat_e):
        rows = np.nonzero(flat_e == e)[0]
        w2 = Q.dequant_fp4_weight_f32(host[e]["w2p"], host[e]["w2s"])
        out_ref[rows] = M.matmul_nt(hf[rows], w2)
        out_abs[rows] = M.matmul_nt(np.abs(hf[rows]), np.abs(w2))
    out_gpu, out_want = Q.bf16_bits_to_f32(_bits(out)), Q.f32_to_bf16_f32(out_ref)
    print(f"pure bf16 down T={T} block_m={block_m}: normwise rel {rel(out_gpu, out_want):.3e}")
    check_bound(out_gpu, out_want, gemm_bound(out_want, out_abs, acc_rel=PURE_ACC_REL),
                f"pure bf16 down T={T} block_m={block_m}")


@pytest.mark.parametrize("block_m", [16, 64, 256])
def test_dequant_in_the_bf16_gemm_every_byte_and_scale(gpu, block_m):
    # one-hot activations pick single weight elements: out[f][n] = W[n][k(f)] exactly, so
    # every packed byte value with every E8M0 byte 0..252 goes through the GEMM's
    # dequantisation and must equal the oracle's bf16 dequant (up to the sign of zero).
    # Above 252 some weights are infinite, and 0 x inf would turn whole output columns
    # into NaN, as it does in any dot product with them.
    from dsv4_hip import AFMT_BF16
    D, I, E = (1024, 1024, 1) if block_m == 256 else (512, 512, 1)  # the large-tile kernel: I % 1024 == 0
    rng = np.random.default_rng(5)
    w2p = rng.integers(0, 256, (D, I // 2), dtype=np.uint8)
    w2s = np.tile(np.arange(253, dtype=np.uint8), (D * (I // 32)) // 253 + 1)[:D * (I // 32)].reshape(D, I // 32)
    rng.shuffle(w2s.reshape(-1))
    ex = {k: torch.zeros(16, dtype=torch.uint8, device=gpu) for k in ("w1p", "w1s", "w3p", "w3s")}
    ex["w2p"], ex["w2s"] = _dev(w2p, gpu), _dev(w2s, gpu)
    table = ops.expert_table({0: ex}, E, gpu)
    R = I  # row f picks k = f
    ids = np.zeros((R, 1), np.int64)
    al = ops.moe_align(_dev(ids, gpu), None, E, block_m)
    one = np.zeros((R, I), np.float32)
    one[np.arange(R), np.arange(R)] = 1.0
    out = ops.gemm_down(AFMT_BF16, _dev_bf16(Q.f32_to_bf16_bits(one), gpu), None, al, table, I, D)
    torch.cuda.synchronize()
    want = Q.dequant_fp4_weight_f32(w2p, w2s).T   # [k, n]
    got = Q.bf16_bits_to_f32(_bits(out))
    assert np.isfinite(want).all()
    bad = got != want
    if bad.any():
        k, n = np.nonzero(bad)
        sb = w2s[n, k // 32]
        print(f"{int(bad.sum())} differ; scale bytes {np.unique(sb)[:20]}; |want| max {np.abs(want[bad]).max():.3e}; "
              f"got {got[bad][:8]} want {want[bad][:8]}")
    assert not bad.any(), "dequantised weights differ"
    print(f"{want.size} weight elements checked, scale bytes 0..252")
