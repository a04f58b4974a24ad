// Shared device helpers for the MI355X (gfx950) MoE expert path.
//
// Number formats (all byte-exact against the reference's torch arithmetic):
//   bf16   : carried as uint16_t bit patterns; fp32 -> bf16 is round-to-nearest-even
//            with NaN -> 0x7FC0 (torch's CPU rule, c10/util/BFloat16.h).
//   E2M1   : FP4 nibble s.e1e0.m; two per byte, low nibble = even k
//            (npu_ops.py:146); nibble 8 decodes to +0.0 (npu_ops.py:20-24).
//   E8M0   : one byte per 32 elements, value 2^(b-127); b=0 -> 2^-127 (fp32
//            subnormal), b=255 -> +inf (npu_ops.py:35-44, torch.pow).
//   E4M3fn : OCP FP8 used by act_quant (npu_ops.py:94), max 448, RNE.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#define DSV4_DEV __device__ __forceinline__

namespace dsv4 {

DSV4_DEV float bf16_to_f32(uint32_t h) { return __uint_as_float(h << 16); }

DSV4_DEV uint32_t f32_to_bf16(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return 0x7fc0u;
  return (u + 0x7fffu + ((u >> 16) & 1u)) >> 16;
}

// Exact power of two 2^k as fp32 for k in [-149, 128] (128 -> +inf).
DSV4_DEV float pow2f(int k) {
  if (k >= 128) return __uint_as_float(0x7f800000u);
  if (k >= -126) return __uint_as_float((uint32_t)(k + 127) << 23);
  if (k >= -149) return __uint_as_float(1u << (k + 149));
  return 0.0f;
}

// floor(log2(a)) for positive finite a (normal or subnormal).
DSV4_DEV int floor_log2(float a) { return __builtin_amdgcn_frexp_expf(a) - 1; }

// ceil(log2(v)) for positive finite v.
DSV4_DEV int ceil_log2(float v) {
  int e = __builtin_amdgcn_frexp_expf(v);        // v = m * 2^e, m in [0.5, 1)
  float m = __builtin_amdgcn_frexp_mantf(v);
  return (m == 0.5f) ? e - 1 : e;
}

// E8M0 byte -> fp32 scale (npu_ops.py:35-44).
DSV4_DEV float e8m0_to_f32(uint32_t b) { return pow2f((int)b - 127); }

// |v| (already divided by the block scale, |v| <= 448) -> E4M3fn magnitude code
// with round-to-nearest-even. The binade exponent is clamped at -6 so that the
// subnormal range uses the same formula; a carry out of the mantissa moves into
// the exponent field by the addition itself.
DSV4_DEV uint32_t e4m3_mag_code(float a) {
  int E = (a < 0.015625f) ? -6 : floor_log2(a);
  float r = __builtin_rintf(a * pow2f(3 - E));
  int code = ((E + 7) << 3) + (int)r - 8;
  return (a == 0.0f) ? 0u : (uint32_t)code;
}
DSV4_DEV float e4m3_mag_value(uint32_t c) {
  uint32_t e = (c >> 3) & 15u, m = c & 7u;
  return (e == 0) ? (float)m * 0.001953125f : pow2f((int)e - 7) * (1.0f + 0.125f * (float)m);
}

// |v| in [0, 6] -> E2M1 magnitude index 0..7 (round-to-nearest-even on the
// E2M1 grid; equal to the reference's searchsorted/tie-to-even rule,
// npu_ops.py:53-67).
DSV4_DEV uint32_t e2m1_mag_code(float a) {
  int E = (a < 1.0f) ? 0 : floor_log2(a);
  float r = __builtin_rintf(a * pow2f(1 - E));
  int code = ((E + 1) << 1) + (int)r - 2;
  return (a == 0.0f) ? 0u : (uint32_t)code;
}
DSV4_DEV float e2m1_mag_value(uint32_t c) {
  // 0, .5, 1, 1.5, 2, 3, 4, 6
  return (c < 2) ? 0.5f * (float)c : pow2f((int)(c >> 1) - 1) * (1.0f + 0.5f * (float)(c & 1));
}

// Wave helpers (wave64).
DSV4_DEV float wave_max_xor(float v, int width) {
  for (int o = width >> 1; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
  return v;
}

}  // namespace dsv4

// Status codes returned by every extern "C" entry point.
enum {
  DSV4_OK = 0,
  DSV4_ERR_NULL = -1,       // a required pointer is null
  DSV4_ERR_SHAPE = -2,      // a size is negative, zero where it must not be, or misaligned
  DSV4_ERR_UNSUPPORTED = -3,// a mode / dtype / size is outside what the kernels support
  DSV4_ERR_HIP = -4,        // a HIP runtime call failed
  DSV4_ERR_STATE = -5,      // handle / slot-manager state error
};
