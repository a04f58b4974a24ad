"""Pins the numpy oracle's FP4/FP8 arithmetic (CPU only).

Each check is independent of the oracle's own formulas:
  * the reference's own self-test vectors and brute-force references
    (test_npu_ops.py:50-96, 154-195), restated with torch library routines;
  * torch's float8_e4m3fn cast and torch.pow (library routines);
  * exhaustive byte x scale tables and brute force on the E2M1 grid.
"""

import math

import numpy as np
import pytest
import torch

from oracle import mxfp4 as Q

FP4_T = torch.tensor(Q.FP4_TABLE)


def bf16_bits(t):
    return t.contiguous().view(torch.int16).numpy().view(np.uint16)


def same_bf16(a, b):
    """Bitwise equality, except that any two NaNs match: torch's CPU fp32->bf16
    conversion itself yields 0x7FC0 (scalar path) or 0xFFFF (vectorised path)."""
    a = np.asarray(a, np.uint16)
    b = np.asarray(b, np.uint16)
    nan_a = (a & 0x7FFF) > 0x7F80
    nan_b = (b & 0x7FFF) > 0x7F80
    return bool(np.array_equal(nan_a, nan_b) and np.array_equal(a[~nan_a], b[~nan_b]))


# --- _round_fp4: sweep -6..6 step 0.01 vs brute force (test_npu_ops.py:154-165)
def test_round_fp4_sweep_vs_bruteforce():
    vals = torch.arange(-6.0, 6.001, 0.01, dtype=torch.float32)
    got, _ = Q.round_fp4(vals.numpy())
    ref = []
    for v in vals:
        dists = (FP4_T - v).abs()
        mn = dists.min()
        ties = torch.nonzero(dists <= mn + 1e-9).flatten()
        idx = ties[0] if len(ties) == 1 else next((int(i) for i in ties if int(i) % 2 == 0), int(ties[0]))
        ref.append(float(FP4_T[idx]))
    assert np.array_equal(np.abs(got), np.abs(np.array(ref, np.float32)))
    assert np.allclose(got, ref, atol=1e-6)


def test_round_fp4_ties_go_to_even_mantissa():
    # midpoints of the E2M1 grid: 0.25 0.75 1.25 1.75 2.5 3.5 5
    mids = np.array([0.25, 0.75, 1.25, 1.75, 2.5, 3.5, 5.0], np.float32)
    got, idx = Q.round_fp4(mids)
    assert list(got) == [0.0, 1.0, 1.0, 2.0, 2.0, 4.0, 4.0]
    assert all(i % 2 == 0 for i in idx)


# --- act_quant (test_npu_ops.py:50-61, 167-178): restated with torch ops
def _torch_act_quant_inplace(x, block_size):
    xf = x.float()
    N = x.shape[-1]
    xb = xf.reshape(-1, N // block_size, block_size)
    amax = xb.abs().amax(-1, keepdim=True).clamp(min=1e-4)
    s = torch.pow(2.0, torch.ceil(torch.log2(amax / 448.0)))
    y8 = torch.clamp(xb / s, -448.0, 448.0).to(torch.float8_e4m3fn)
    return (y8.float() * s).reshape_as(x).to(x.dtype), s


@pytest.mark.parametrize("seed,scale", [(0, 3.0), (1, 1e-3), (2, 300.0), (3, 1e-6)])
def test_act_quant_matches_torch_restatement(seed, scale):
    torch.manual_seed(seed)
    x = (torch.randn(64, 512) * scale).to(torch.bfloat16)
    ref, s_ref = _torch_act_quant_inplace(x, 128)
    rt, codes, s, k = Q.act_quant(bf16_bits(x), 128)
    assert np.array_equal(rt, bf16_bits(ref))
    assert np.array_equal(s.reshape(64, 4), s_ref.reshape(64, 4).numpy())
    # the scale is an exact power of two and the codes decode to the round trip
    assert np.array_equal(np.ldexp(np.float32(1), k), s)
    assert np.array_equal(Q.f32_to_bf16_bits(Q.e4m3fn_code_to_f32(codes).reshape(64, 4, 128)
                                             * s.reshape(64, 4, 1)).reshape(64, 512), rt)


def test_e4m3_conversion_vs_torch_cast_exhaustive():
    # every finite bf16 pattern with |v| <= 448, plus values between bf16 neighbours
    b = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    v = Q.bf16_bits_to_f32(b)
    v = v[np.isfinite(v) & (np.abs(v) <= 448)]
    extra = (v[:-1] + np.float32(1e-7) * np.abs(v[:-1])).astype(np.float32)
    extra = extra[np.abs(extra) <= 448]
    v = np.concatenate([v, extra])
    ours = Q.f32_to_e4m3fn_code(v)
    ref = torch.from_numpy(v).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    assert np.array_equal(ours, ref)


def test_act_quant_scale_is_bitexact_ceil_log2():
    # amax * fp32(1/448) never lands near a power of two for bf16 amax unless exactly on it
    b = np.arange(0x0080, 0x7f80, dtype=np.uint32).astype(np.uint16)  # positive normal bf16
    amax = Q.bf16_bits_to_f32(b)
    amax = np.maximum(amax, np.float32(1e-4))
    s, k = Q.fast_pow2_scale(amax, 1.0 / 448.0)
    ref = torch.pow(2.0, torch.ceil(torch.log2(torch.clamp(torch.from_numpy(amax) * (1.0 / 448.0),
                                                             min=2.0 ** -126)))).numpy()
    assert np.array_equal(s, ref)


# --- fp4_act_quant (test_npu_ops.py:64-83, 180-183): brute force
def _bruteforce_fp4_quant(x, block_size):
    xf = x.float()
    N = x.shape[-1]
    xb = xf.reshape(-1, N // block_size, block_size)
    amax = xb.abs().amax(-1, keepdim=True).clamp(min=6 * 2.0 ** -126)
    s = torch.pow(2.0, torch.ceil(torch.log2(amax / 6.0)))
    v = torch.clamp(xb / s, -6.0, 6.0)
    flat = v.reshape(-1)
    d = (flat.unsqueeze(-1) - FP4_T.unsqueeze(0)).abs()
    mn = d.min(dim=-1, keepdim=True).values
    cand = (d <= mn + 1e-9)
    idxs = torch.arange(16)
    big = torch.where(cand, (idxs % 2 == 0).float(), torch.full_like(d, -1e9))
    pick = big.argmax(dim=-1)
    q = FP4_T[pick]
    s = s.expand(-1, -1, block_size).reshape(-1)
    return (q * s).reshape_as(x).to(x.dtype)


@pytest.mark.parametrize("seed,scale", [(0, 2.0), (5, 1e-30), (6, 1e30)])
def test_fp4_act_quant_vs_bruteforce(seed, scale):
    torch.manual_seed(seed)
    x2 = (torch.randn(64, 256) * scale).to(torch.bfloat16)
    dq, packed, sc = Q.fp4_act_quant(bf16_bits(x2), 32)
    ref = _bruteforce_fp4_quant(x2, 32)
    # the brute force reference picks +0 for tiny negatives; compare values, then signs of nonzeros
    assert np.array_equal(Q.bf16_bits_to_f32(dq), ref.float().numpy())
    # packed + scale decode back to the same values
    back = Q.fp4_codes_to_f32(packed, sc)
    assert np.array_equal(back, Q.bf16_bits_to_f32(dq))


def test_fp4_act_quant_negative_zero_rule():
    # values that round to zero keep the reference's sign rule: -0.0 iff x/s < 0
    x = np.zeros((1, 32), np.float32)
    x[0, 0] = 6.0
    x[0, 1] = -0.25    # x/s = -0.25 -> rounds to 0 (tie to even) with sign -> -0.0
    x[0, 2] = -0.0     # v = -0.0 is not < 0 -> +0.0
    dq, packed, _ = Q.fp4_act_quant(Q.f32_to_bf16_bits(x), 32)
    assert dq[0, 1] == 0x8000 and dq[0, 2] == 0x0000
    assert (packed[0, 0] >> 4) == 0x8 and (packed[0, 1] & 0xF) == 0x0


# --- OCP floor rule: brute force per block
def test_ocp_floor_rule_bruteforce():
    rng = np.random.default_rng(11)
    x = (rng.standard_normal((32, 128)) * np.exp(rng.uniform(-8, 8, (32, 1)))).astype(np.float32)
    x[3] = 0.0
    xb = Q.f32_to_bf16_bits(x)
    dq, packed, sc = Q.ocp_mx_quant(xb, 32)
    xf = Q.bf16_bits_to_f32(xb)
    mags = [0.0, 0.5, 1.0, 1.5, 2.0, 3.0, 4.0, 6.0]
    for r in range(32):
        for b in range(4):
            blk = xf[r, 32 * b:32 * b + 32].astype(np.float64)
            amax = np.abs(blk).max()
            if amax == 0:
                shared = -127
            else:
                shared = max(min(math.frexp(amax)[1] - 1 - 2, 127), -127)
            assert sc[r, b] == shared + 127
            X = 2.0 ** shared
            for j, v in enumerate(blk):
                a = min(abs(v) / X, 6.0)
                d = [abs(a - m) for m in mags]
                best = min(d)
                cands = [i for i in range(8) if d[i] == best]
                i = cands[0] if len(cands) == 1 else [c for c in cands if c % 2 == 0][0]
                want = (-1.0 if math.copysign(1, v) < 0 else 1.0) * mags[i] * X
                got = float(Q.bf16_bits_to_f32(dq[r:r + 1, 32 * b + j:32 * b + j + 1])[0, 0])
                assert got == want and math.copysign(1, got) == math.copysign(1, want), (r, b, j, v)
            if amax > 0:
                # the block maximum lands in [4, 6] on the E2M1 grid
                assert 4.0 <= amax / X < 8.0


# --- dequant (test_npu_ops.py:86-96, 185-195)
def _loop_dequant(w_packed, scale):
    u = w_packed.view(torch.uint8)
    N, Kh = u.shape
    K = Kh * 2
    vals = torch.empty(N, K, dtype=torch.float32)
    for j in range(Kh):
        vals[:, 2 * j] = FP4_T[(u[:, j] & 0x0F).long()]
        vals[:, 2 * j + 1] = FP4_T[((u[:, j] >> 4) & 0x0F).long()]
    s = torch.pow(2.0, scale.view(torch.uint8).to(torch.int32).float() - 127.0)
    s = s.unsqueeze(-1).expand(N, K // 32, 32).reshape(N, K)
    return vals * s


def test_dequant_reference_selftest_vector():
    N, Kh = 8, 128
    rng = np.random.default_rng(0)
    packed = torch.from_numpy(rng.integers(0, 256, (N, Kh), dtype=np.uint8))
    scale_bytes = rng.integers(120, 134, (N, (Kh * 2) // 32), dtype=np.uint8)
    ref = _loop_dequant(packed.view(torch.int8), torch.from_numpy(scale_bytes))
    ours = Q.dequant_fp4_weight(packed.numpy(), scale_bytes)
    assert np.array_equal(ours, bf16_bits(ref.to(torch.bfloat16)))


def test_dequant_exhaustive_byte_scale_table():
    # every byte (both nibbles) under every scale byte, vs torch.pow / FP4_TABLE, bitwise
    b = np.tile(np.arange(256, dtype=np.uint8), (256, 16))          # [256 scales, 4096 bytes]
    s = np.repeat(np.arange(256, dtype=np.uint8)[:, None], 256, axis=1)  # [256, 256] one per 32 elements
    ours = Q.dequant_fp4_weight(b, s)
    u = torch.from_numpy(b)
    lo = FP4_T[(u & 0xF).long()]
    hi = FP4_T[(u >> 4).long()]
    vals = torch.stack([lo, hi], -1).reshape(256, 8192)
    sc = torch.pow(2.0, torch.from_numpy(s).int().float() - 127.0).repeat_interleave(32, dim=1)
    ref = (vals * sc).to(torch.bfloat16)
    assert same_bf16(ours, bf16_bits(ref))
    # spot facts: nibble 8 -> +0.0; scale 255 -> inf/NaN pattern; scale 0 -> subnormal
    assert ours[127, 16] == 0x0000 and ours[127, 17] == 0x0000  # byte 0x08 at k=16: low nib 8
    assert ours[255, 2] == 0x7F80 and ours[255, 0] == 0x7FC0      # byte 1 low nib 1 -> +inf; byte 0 -> NaN
    assert ours[0, 2] == 0x0020                                    # 0.5 * 2^-127 = 2^-128


def test_e8m0_to_fp32_edges():
    got = Q.e8m0_to_fp32(np.array([0, 1, 127, 254, 255], np.uint8))
    ref = torch.pow(2.0, torch.tensor([0, 1, 127, 254, 255]).float() - 127.0).numpy()
    assert np.array_equal(got, ref)


def test_bf16_rounding_matches_torch():
    rng = np.random.default_rng(2)
    v = rng.standard_normal(100000).astype(np.float32) * np.float32(1e3)
    v = np.concatenate([v, np.array([np.inf, -np.inf, np.nan, 3.3895314e38, -0.0], np.float32)])
    assert same_bf16(Q.f32_to_bf16_bits(v), bf16_bits(torch.from_numpy(v).to(torch.bfloat16)))
