"""Per-element parity bars for the GEMM tests (test helpers, no GPU code).

When the GPU kernel and the oracle receive the same quantised operands, every
product is exact on both sides; the oracle sums them in float64 and rounds
once. The scaled MFMA (v_mfma_scale_f32_16x16x128_f8f6f4) does not accumulate
like an IEEE fp32 sum either: measured on gfx950 with E4M3 x E2M1 operands, it
drops products that lie more than about 10-13 binades below the largest
product of their group of consecutive k (448 + 127 * 2^-9 comes out as
448 + 120 * 2^-9; FP8 subnormals on their own are kept). The bar for a GEMM
output is therefore one bf16 ulp (the two sums may round to neighbouring bf16
values) plus ``acc_rel`` times the sum of the absolute products of that
output (``abs_sum``), and a floor relative to the largest output for sums
that cancel. E2M1 x E2M1 products span only ~7 binades, nothing is dropped and
every partial sum is exact in fp32 for the synthetic operands, so the a4w4
profile is checked bit for bit instead. For the SwiGLU output h =
silu(min(g, L)) * clamp(u, -L, L) * w, the bf16 gate g and up u carry the
same bound; it reaches h to first order through the derivatives.
"""

import numpy as np

# share of the sum of absolute products an E4M3 x E2M1 MFMA output may be off by
ACC_REL = 2.0 ** -10


def bf16_ulp(v):
    """Spacing of bf16 numbers at |v| (v float array): 2^(floor(log2|v|) - 7)."""
    a = np.abs(np.asarray(v, np.float64))
    e = np.floor(np.log2(np.maximum(a, 2.0 ** -126)))
    return np.exp2(e - 7)


def ulp_bound(want, n_ulp=1.0, floor_frac=2.0 ** -10):
    """n_ulp bf16 ulps of max(|want|, floor_frac * max|want|), per element."""
    w = np.abs(np.asarray(want, np.float64))
    floor = floor_frac * max(float(w.max()) if w.size else 0.0, 1e-30)
    return n_ulp * bf16_ulp(np.maximum(w, floor))


def gemm_bound(want, abs_sum, acc_rel=ACC_REL, floor_frac=2.0 ** -10):
    """One bf16 ulp of max(|want|, floor) plus acc_rel * sum_k |a_k b_k|."""
    return ulp_bound(want, 1.0, floor_frac) + acc_rel * np.asarray(abs_sum, np.float64)


def swiglu_bound(g, u, w, limit, h, g_abs_sum=None, u_abs_sum=None, acc_rel=ACC_REL, floor_frac=2.0 ** -10):
    """Bound on |h_gpu - h_ref| for h = silu(min(g, L)) * clamp(u, +-L) * w when
    g and u are bf16 GEMM outputs that may each be off by ``gemm_bound`` (their
    sums of absolute products given) (rows: g, u [R, I]; w [R])."""
    g = np.asarray(g, np.float64)
    u = np.asarray(u, np.float64)
    w = np.asarray(w, np.float64)[:, None]
    fg = floor_frac * max(np.abs(g).max(), 1e-30)
    fu = floor_frac * max(np.abs(u).max(), 1e-30)
    eg = bf16_ulp(np.maximum(np.abs(g), fg)) + (0.0 if g_abs_sum is None else acc_rel * np.asarray(g_abs_sum))
    eu = bf16_ulp(np.maximum(np.abs(u), fu)) + (0.0 if u_abs_sum is None else acc_rel * np.asarray(u_abs_sum))
    gc = np.minimum(g, limit) if limit else g
    uc = np.clip(u, -limit, limit) if limit else u
    sig = 1.0 / (1.0 + np.exp(-gc))
    dsilu = sig * (1.0 + gc * (1.0 - sig))
    # a value within its own error of the clamp may land on either side of it
    dh_dg = np.abs(w * uc * dsilu) * ((g - eg < limit) if limit else 1.0)
    dh_du = np.abs(w * gc * sig) * ((np.abs(u) - eu < limit) if limit else 1.0)
    return ulp_bound(h, 1.0, floor_frac) + dh_dg * eg + dh_du * eu


def check_bound(got, want, bound, what):
    """Asserts |got - want| <= bound everywhere; returns the worst |err| / bound."""
    err = np.abs(np.asarray(got, np.float64) - np.asarray(want, np.float64))
    ratio = err / np.maximum(bound, 1e-300)
    worst = float(ratio.max()) if ratio.size else 0.0
    n_bad = int((ratio > 1.0).sum())
    print(f"{what}: worst |err|/bound = {worst:.3f}, elements over = {n_bad} of {ratio.size}", flush=True)
    assert n_bad == 0, f"{what}: {n_bad} element(s) over the bound (worst ratio {worst:.2f})"
    return worst


def elementwise_rel(got, want, floor_frac=1.0):
    """max |got - want| / max(|want|, floor_frac * rms(want)): a per-element
    relative error whose floor keeps near-zero outputs from dominating."""
    g = np.asarray(got, np.float64)
    w = np.asarray(want, np.float64)
    rms = float(np.sqrt((w * w).mean())) if w.size else 0.0
    return float((np.abs(g - w) / np.maximum(np.abs(w), max(floor_frac * rms, 1e-30))).max())
