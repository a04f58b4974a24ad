// Per-thread bodies of the activation quantisers, shared by the standalone
// kernels (quant.hip) and the fused align + quantise launch (align.hip).
// One thread owns 8 consecutive bf16 elements (group g); the lanes of one
// quantisation block are consecutive lanes of one wave (16 lanes per 128-element
// FP8 block, 4 lanes per 32-element MXFP4 block), so the block's amax is a
// wave-local xor reduction. The caller maps lanes to groups so that g % 16
// (resp. g % 4) equals the lane's position in its block.
#pragma once
#include "common.h"

namespace dsv4 {

// act_quant (npu_ops.py:73-104): per-128 block of one row,
//   amax = max(max|x|, 1e-4); s = 2^ceil(log2(max(amax * fp32(1/448), 2^-126)))
//   code = e4m3fn(clamp(x / s, +-448)) (RNE); rt = bf16(e4m3(code) * s)
// block exponent k of a 128-element FP8 block with abs-max amax (scale 2^k)
DSV4_DEV int fp8_block_exp(float amax) {
  amax = fmaxf(amax, 1e-4f);
  float vs = fmaxf(amax * (1.0f / 448.0f), 1.1754943508222875e-38f);
  return ceil_log2(vs);
}

// E4M3fn code of element f of a block with inverse scale inv = 2^-k
DSV4_DEV uint32_t fp8_code(float f, float inv) {
  float y = fminf(fmaxf(f * inv, -448.0f), 448.0f);
  uint32_t neg = __float_as_uint(y) >> 31;
  return e4m3_mag_code(fabsf(y)) | (neg << 7);
}

// `live` must be the same for the 16 lanes of a block.
DSV4_DEV void fp8_quant_group(const uint4* __restrict__ x, int64_t g, bool live, uint4* __restrict__ rt,
                              uint2* __restrict__ codes, float* __restrict__ scale_f32,
                              uint32_t* __restrict__ scale_e8m0x4) {
  uint4 v = live ? x[g] : make_uint4(0, 0, 0, 0);
  uint32_t w[4] = {v.x, v.y, v.z, v.w};
  float f[8];
  float amax = 0.0f;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    f[2 * i] = bf16_to_f32(w[i] & 0xffffu);
    f[2 * i + 1] = bf16_to_f32(w[i] >> 16);
    amax = fmaxf(amax, fmaxf(fabsf(f[2 * i]), fabsf(f[2 * i + 1])));
  }
  amax = wave_max_xor(amax, 16);
  const int k = fp8_block_exp(amax);
  float s = pow2f(k), inv = pow2f(-k);
  uint32_t c[8];
  uint32_t o[4];
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    c[i] = fp8_code(f[i], inv);
    const uint32_t neg = c[i] >> 7, mag = c[i] & 0x7fu;
    float q = e4m3_mag_value(mag) * s;
    uint32_t b = f32_to_bf16(neg ? -q : q);
    if (i & 1) o[i >> 1] |= b << 16; else o[i >> 1] = b;
  }
  if (!live) return;
  if (rt) rt[g] = make_uint4(o[0], o[1], o[2], o[3]);
  if (codes) codes[g] = make_uint2(c[0] | (c[1] << 8) | (c[2] << 16) | (c[3] << 24),
                                   c[4] | (c[5] << 8) | (c[6] << 16) | (c[7] << 24));
  if ((g & 15) == 0) {
    const int64_t blk = g >> 4;
    if (scale_f32) scale_f32[blk] = s;
    if (scale_e8m0x4) scale_e8m0x4[blk] = (uint32_t)(k + 127) * 0x01010101u;
  }
}

// MXFP4 activation quant, per 32 elements.
//  rule 0 "ceil_div6" (npu_ops.py:107-121):
//     amax = max(max|x|, 6*2^-126); s = 2^ceil(log2(max(amax*fp32(1/6), 2^-126)))
//     v = clamp(x/s, +-6); q = E2M1-RNE(|v|); sign = (v < 0); dq = bf16(+-q * s)
//  rule 1 "ocp_floor" (OCP MX v1.0): shared = floor(log2 amax) - 2 clamped to
//     [-127, 127] (-127 for an all-zero block); q = E2M1-RNE(min(|x|/2^shared, 6));
//     sign = signbit(x)
// Outputs: packed nibbles (low = even element), E8M0 scale byte, optional bf16 dq.
// shared exponent of an MXFP4 block with abs-max `amax` (rule 0 / 1 as above)
DSV4_DEV int mxfp4_block_exp(float amax, int rule) {
  if (rule == 0) {
    amax = fmaxf(amax, 6.0f * 1.1754943508222875e-38f);
    float vs = fmaxf(amax * (1.0f / 6.0f), 1.1754943508222875e-38f);
    return ceil_log2(vs);
  }
  return (amax == 0.0f) ? -127 : min(max(floor_log2(amax) - 2, -127), 127);
}

// sign-magnitude E2M1 nibble of element f of a block with inverse scale inv = 2^-k
DSV4_DEV uint32_t mxfp4_nibble(float f, float inv, int rule) {
  float y = f * inv;
  uint32_t neg;
  float a;
  if (rule == 0) {
    y = fminf(fmaxf(y, -6.0f), 6.0f);
    neg = (y < 0.0f) ? 1u : 0u;
    a = fabsf(y);
  } else {
    neg = __float_as_uint(f) >> 31;
    a = fminf(fabsf(y), 6.0f);
  }
  return e2m1_mag_code(a) | (neg << 3);
}

// `live` must be the same for the 4 lanes of a block.
DSV4_DEV void mxfp4_quant_group(const uint4* __restrict__ x, int64_t g, bool live, int rule,
                                uint32_t* __restrict__ packed, uint8_t* __restrict__ scale,
                                uint4* __restrict__ dq) {
  uint4 v = live ? x[g] : make_uint4(0, 0, 0, 0);
  uint32_t w[4] = {v.x, v.y, v.z, v.w};
  float f[8];
  float amax = 0.0f;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    f[2 * i] = bf16_to_f32(w[i] & 0xffffu);
    f[2 * i + 1] = bf16_to_f32(w[i] >> 16);
    amax = fmaxf(amax, fmaxf(fabsf(f[2 * i]), fabsf(f[2 * i + 1])));
  }
  amax = wave_max_xor(amax, 4);
  const int k = mxfp4_block_exp(amax, rule);
  float s = pow2f(k), inv = pow2f(-k);
  uint32_t pk = 0;
  uint32_t o[4];
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const uint32_t nib = mxfp4_nibble(f[i], inv, rule);
    pk |= nib << (4 * i);
    const uint32_t neg = nib >> 3, mag = nib & 7u;
    float q = e2m1_mag_value(mag) * s;
    uint32_t b = f32_to_bf16(neg ? -q : q);
    if (i & 1) o[i >> 1] |= b << 16; else o[i >> 1] = b;
  }
  if (!live) return;
  packed[g] = pk;
  if (dq) dq[g] = make_uint4(o[0], o[1], o[2], o[3]);
  if ((g & 3) == 0) scale[g >> 2] = (uint8_t)(k + 127);
}

}  // namespace dsv4
