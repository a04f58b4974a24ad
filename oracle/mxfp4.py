"""numpy restatement of the reference's FP4/FP8 arithmetic (test oracle only).

Follows ``npu_ops.py`` of the reference:

* ``FP4_TABLE`` / ``FP4_POS``           - ``npu_ops.py:19-26``
* ``e8m0_to_fp32``                      - ``npu_ops.py:35-44``
* ``fast_pow2_scale``                   - ``npu_ops.py:47-50``
* ``round_fp4``                         - ``npu_ops.py:53-67``
* ``act_quant`` (FP8 E4M3, per-128)     - ``npu_ops.py:73-104``
* ``fp4_act_quant`` (ceil(amax/6) rule) - ``npu_ops.py:107-121``
* ``dequant_fp4_weight``                - ``npu_ops.py:129-158``

bf16 tensors are carried as ``uint16`` bit patterns; float conversions follow
torch's CPU rules (round-to-nearest-even, NaN -> 0x7FC0).
"""

import numpy as np

FP4_TABLE = np.array([0.0, 0.5, 1.0, 1.5, 2.0, 3.0, 4.0, 6.0,
                      0.0, -0.5, -1.0, -1.5, -2.0, -3.0, -4.0, -6.0], dtype=np.float32)
FP4_POS = np.array([0.0, 0.5, 1.0, 1.5, 2.0, 3.0, 4.0, 6.0], dtype=np.float32)
FP8_MAX = 448.0
FP4_MAX = 6.0

# The reference multiplies fp32 tensors by Python floats; torch evaluates those
# products in fp32 with the scalar rounded to fp32 first.
_F32_INV_448 = np.float32(1.0 / FP8_MAX)
_F32_INV_6 = np.float32(1.0 / FP4_MAX)


# ---------------------------------------------------------------------------
# bf16 helpers
# ---------------------------------------------------------------------------
def f32_to_bf16_bits(x):
    """fp32 -> bf16 bit pattern, round-to-nearest-even; NaN -> 0x7FC0 (torch CPU rule)."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    u = x.view(np.uint32).astype(np.uint64)
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    r[np.isnan(x)] = 0x7FC0
    return r


def bf16_bits_to_f32(b):
    b = np.ascontiguousarray(b, dtype=np.uint16)
    return (b.astype(np.uint32) << 16).view(np.float32)


def f32_to_bf16_f32(x):
    """Round fp32 values to bf16 and return them as fp32 (``t.to(bf16).float()``)."""
    return bf16_bits_to_f32(f32_to_bf16_bits(x))


# ---------------------------------------------------------------------------
# scale helpers
# ---------------------------------------------------------------------------
def e8m0_to_fp32(scale_u8):
    """UE8M0 byte -> 2**(byte-127) as fp32 (byte 0 -> 2**-127 subnormal, 255 -> +inf).

    Restates ``npu_ops.py:35-44`` (``torch.pow(2.0, u - 127)``)."""
    u = np.asarray(scale_u8, dtype=np.uint8).astype(np.int32)
    with np.errstate(over="ignore"):
        return np.ldexp(np.float32(1.0), u - 127).astype(np.float32)


def _ceil_log2_f32(v):
    """Exact ceil(log2 v) for positive finite fp32 v (normal or subnormal)."""
    m, e = np.frexp(v.astype(np.float64))  # v = m * 2**e, m in [0.5, 1)
    return np.where(m == 0.5, e - 1, e).astype(np.int32)


def fast_pow2_scale(amax, max_inv):
    """``npu_ops.py:47-50``: 2**ceil(log2(max(amax*max_inv, 2**-126))), fp32 arithmetic.

    Returns (scale fp32, exponent int32)."""
    with np.errstate(over="ignore"):
        v = (np.asarray(amax, np.float32) * np.float32(max_inv)).astype(np.float32)
    v = np.maximum(v, np.float32(2.0 ** -126))
    k = _ceil_log2_f32(v)
    return np.ldexp(np.float32(1.0), k).astype(np.float32), k


# ---------------------------------------------------------------------------
# FP8 E4M3 (OCP "fn") conversion used by act_quant
# ---------------------------------------------------------------------------
def f32_to_e4m3fn_code(v):
    """fp32 -> float8_e4m3fn byte, round-to-nearest-even, for |v| <= 448.

    The sign bit follows the fp32 sign bit (so -0.0 and negative values that
    round to zero give 0x80), as torch's ``.to(torch.float8_e4m3fn)`` does."""
    v = np.asarray(v, dtype=np.float32)
    a = np.abs(v).astype(np.float64)
    if np.any(a > FP8_MAX) or np.any(np.isnan(a)):
        raise ValueError("f32_to_e4m3fn_code expects finite |v| <= 448")
    _, e = np.frexp(a)
    E = np.where(a < 2.0 ** -6, -6, e - 1)          # binade exponent, subnormals share -6
    r = np.rint(np.ldexp(a, 3 - E))                  # mantissa in units of 2**(E-3), RNE
    code = ((E + 7) << 3) + r.astype(np.int64) - 8   # carry into the exponent is automatic
    code = np.where(a == 0, 0, code)
    sign = np.signbit(v).astype(np.int64) << 7
    return (code | sign).astype(np.uint8)


def e4m3fn_code_to_f32(c):
    c = np.asarray(c, dtype=np.uint8).astype(np.int64)
    s = c >> 7
    e = (c >> 3) & 15
    m = c & 7
    mag = np.where(e == 0, np.ldexp(m.astype(np.float64), -9),
                   np.ldexp(1.0 + m / 8.0, e - 7))
    mag = np.where((e == 15) & (m == 7), np.nan, mag)
    return np.where(s == 1, -mag, mag).astype(np.float32)


# ---------------------------------------------------------------------------
# act_quant: per-block FP8 round trip (npu_ops.py:73-104)
# ---------------------------------------------------------------------------
def act_quant(x_bf16, block_size=128):
    """FP8 E4M3 quantisation of a bf16 matrix with a power-of-two scale per block.

    Returns ``(rt_bf16_bits, codes_u8, scale_f32, scale_exp)``:
    ``rt`` is the inplace round trip (what ``act_quant(x, 128, "ue8m0", None,
    True)`` writes into ``x``), ``codes`` the e4m3fn bytes, ``scale`` the fp32
    power-of-two scale per block and ``scale_exp`` its log2.
    """
    xb = np.asarray(x_bf16, dtype=np.uint16)
    shape = xb.shape
    N = shape[-1]
    assert N % block_size == 0, (N, block_size)
    xf = bf16_bits_to_f32(xb).reshape(-1, N // block_size, block_size)
    amax = np.abs(xf).max(axis=-1, keepdims=True)
    amax = np.maximum(amax, np.float32(1e-4))                   # clamp(min=1e-4)
    s, k = fast_pow2_scale(amax, 1.0 / FP8_MAX)                # npu_ops.py:91
    y = np.clip(xf / s, -FP8_MAX, FP8_MAX).astype(np.float32)  # npu_ops.py:94
    codes = f32_to_e4m3fn_code(y)
    rt = (e4m3fn_code_to_f32(codes) * s).astype(np.float32)    # npu_ops.py:96
    return (f32_to_bf16_bits(rt).reshape(shape), codes.reshape(shape),
            s.reshape(*shape[:-1], N // block_size), k.reshape(*shape[:-1], N // block_size))


# ---------------------------------------------------------------------------
# FP4 E2M1 rounding and activation quantisation
# ---------------------------------------------------------------------------
def round_fp4(v):
    """``npu_ops.py:53-67``: nearest E2M1 magnitude via searchsorted; ties -> even index.

    Returns (value fp32 with the reference's sign rule, index 0..7)."""
    v = np.asarray(v, dtype=np.float32)
    a = np.abs(v)
    idx = np.searchsorted(FP4_POS, a, side="left")
    idx = np.clip(idx, 1, 7)
    lo = FP4_POS[idx - 1]
    hi = FP4_POS[idx]
    d_lo = (a - lo).astype(np.float32)
    d_hi = (hi - a).astype(np.float32)
    take_hi = (d_hi < d_lo) | ((d_hi == d_lo) & (((idx - 1) % 2) == 1))
    val = np.where(take_hi, hi, lo).astype(np.float32)
    mag_idx = np.where(take_hi, idx, idx - 1)
    sign = np.where(v < 0, np.float32(-1.0), np.float32(1.0))
    return (val * sign).astype(np.float32), mag_idx.astype(np.int64)


def _pack_nibbles(codes):
    """[..., K] nibbles -> [..., K/2] bytes, low nibble = even k (npu_ops.py:146)."""
    c = codes.astype(np.uint8)
    return (c[..., 0::2] | (c[..., 1::2] << 4)).astype(np.uint8)


def fp4_act_quant(x_bf16, block_size=32):
    """``npu_ops.py:107-121`` (scale = 2**ceil(log2(amax/6)), no saturation needed).

    Returns ``(dq_bf16_bits, packed_u8, scale_e8m0_u8)``: ``dq`` is what the
    reference's inplace call writes; ``packed``/``scale`` are the same values in
    MXFP4 storage (nibble sign bit set exactly when the reference's value is
    negative, including -0.0)."""
    xb = np.asarray(x_bf16, dtype=np.uint16)
    shape = xb.shape
    N = shape[-1]
    assert N % block_size == 0, (N, block_size)
    xf = bf16_bits_to_f32(xb).reshape(-1, N // block_size, block_size)
    amax = np.abs(xf).max(axis=-1, keepdims=True)
    amax = np.maximum(amax, np.float32(FP4_MAX * 2.0 ** -126))
    s, k = fast_pow2_scale(amax, 1.0 / FP4_MAX)
    v = np.clip(xf / s, -FP4_MAX, FP4_MAX).astype(np.float32)
    q, mag_idx = round_fp4(v)
    dq = (q * s).astype(np.float32)
    nib = mag_idx | (np.signbit(q).astype(np.int64) << 3)
    packed = _pack_nibbles(nib.reshape(*shape))
    scale = (k + 127).astype(np.uint8).reshape(*shape[:-1], N // block_size)
    return f32_to_bf16_bits(dq).reshape(shape), packed, scale


def _ocp_round_e2m1(a):
    """Nearest-even E2M1 magnitude for a in [0, 6] (OCP MX v1.0 conversion)."""
    a = a.astype(np.float64)
    _, e = np.frexp(a)
    E = np.where(a < 1.0, 0, e - 1)
    r = np.rint(np.ldexp(a, 1 - E))
    idx = ((E + 1) << 1) + r.astype(np.int64) - 2
    idx = np.where(a == 0, 0, idx)
    return idx


def ocp_mx_quant(x_bf16, block_size=32):
    """OCP MX v1.0 MXFP4 quantisation: shared exponent floor(log2 amax) - 2,
    elements saturate to +-6, round-to-nearest-even; an all-zero block gets
    exponent -127 (byte 0). This is the rule stated for the a4w4 profile in
    place of the closed ``npu_dynamic_mx_quant`` (``deepseek_v4.py:212,240``).

    Returns ``(dq_bf16_bits, packed_u8, scale_e8m0_u8)``."""
    xb = np.asarray(x_bf16, dtype=np.uint16)
    shape = xb.shape
    N = shape[-1]
    assert N % block_size == 0, (N, block_size)
    xf = bf16_bits_to_f32(xb).reshape(-1, N // block_size, block_size)
    amax = np.abs(xf).max(axis=-1, keepdims=True).astype(np.float64)
    _, e = np.frexp(amax)
    shared = np.where(amax == 0, -127, np.clip(e - 1 - 2, -127, 127)).astype(np.int64)
    X = np.ldexp(1.0, shared)
    a = np.minimum(np.abs(xf).astype(np.float64) / X, FP4_MAX)
    idx = _ocp_round_e2m1(a)
    sign = np.signbit(xf).astype(np.int64)
    nib = idx | (sign << 3)
    dq = np.where(sign == 1, -1.0, 1.0) * FP4_POS[idx].astype(np.float64) * X
    packed = _pack_nibbles(nib.reshape(*shape))
    scale = (shared + 127).astype(np.uint8).reshape(*shape[:-1], N // block_size)
    return f32_to_bf16_bits(dq.astype(np.float32)).reshape(shape), packed, scale


def dynamic_mx_quant(x_bf16, rule="ocp_floor"):
    """MXFP4 activation quantisation, per 32 elements, under either scale rule.

    ``"ceil_div6"`` = the reference's own torch rule (``fp4_act_quant``);
    ``"ocp_floor"`` = OCP MX floor rule."""
    if rule == "ceil_div6":
        return fp4_act_quant(x_bf16, 32)
    if rule == "ocp_floor":
        return ocp_mx_quant(x_bf16, 32)
    raise ValueError(f"unknown scale rule {rule!r}")


# ---------------------------------------------------------------------------
# weight dequant (npu_ops.py:129-158)
# ---------------------------------------------------------------------------
_TBL256 = np.stack([FP4_TABLE[np.arange(256) & 0xF], FP4_TABLE[np.arange(256) >> 4]], axis=-1)


def dequant_fp4_weight_f32(w_packed, scale):
    """[N, K/2] packed + [N, K/32] UE8M0 -> fp32 [N, K] (before the bf16 cast)."""
    u = np.asarray(w_packed).view(np.uint8)
    N, K2 = u.shape
    K = 2 * K2
    vals = _TBL256[u.astype(np.int32)]                       # [N, K/2, 2]
    s = e8m0_to_fp32(np.asarray(scale).view(np.uint8))[..., None]   # [N, K/32, 1]
    with np.errstate(invalid="ignore", over="ignore"):
        return (vals.reshape(N, K // 32, 32) * s).reshape(N, K).astype(np.float32)


def dequant_fp4_weight(w_packed, scale):
    """``dequant_fp4_weight(w, s, torch.bfloat16)`` as bf16 bit patterns [N, K]."""
    return f32_to_bf16_bits(dequant_fp4_weight_f32(w_packed, scale))


def fp4_codes_to_f32(packed, scale, block=32):
    """Dequantise MXFP4 activations/weights (same math as the weight dequant)."""
    return dequant_fp4_weight_f32(packed, scale)


def dequant_fp8_weight_f32(codes, scale, block=128):
    """``npu_ops.py:161-167`` dequant_fp8_weight before its bf16 cast: E4M3 code
    value times ``2^(s-127)`` of its 128x128 block. ``codes`` [N, K] uint8,
    ``scale`` [ceil(N/128), ceil(K/128)] uint8. Exact in bf16 for the scale
    range of the checkpoints (a 4-bit significand times a power of two)."""
    c = np.asarray(codes, np.uint8)
    N, K = c.shape
    v = e4m3fn_code_to_f32(c)
    s = e8m0_to_fp32(np.asarray(scale, np.uint8))
    s = np.repeat(np.repeat(s, block, axis=0)[:N], block, axis=1)[:, :K]
    with np.errstate(invalid="ignore", over="ignore"):
        return (v * s).astype(np.float32)
