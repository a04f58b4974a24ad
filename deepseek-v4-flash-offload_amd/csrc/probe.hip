// MFMA issue-rate probe (a measurement helper; the grouped GEMMs do not use it).
//
// Each wave runs `iters` iterations of independent accumulation chains of one
// scaled MFMA shape on register operands: no memory traffic inside the loop, so
// the launch measures what the matrix cores sustain for that shape and operand
// format pair at the clock the chip holds under a pure-MFMA load. Both shapes do
// 262,144 dense FLOPs per wave per iteration (16x16x128: four chains; 32x32x64:
// two chains), and with 8 workgroups of 4 waves per CU every SIMD always has
// independent MFMAs to issue.
#include "common.h"
#include "kernels.h"

namespace {

typedef int v8i __attribute__((ext_vector_type(8)));
typedef float v4f __attribute__((ext_vector_type(4)));
typedef float v16f __attribute__((ext_vector_type(16)));

constexpr double kFlopPerWaveIter = 262144.0;

template <int FA, int FB>
__global__ __launch_bounds__(256) void mfma_rate_16(float* out, int iters, int seed) {
  v8i a, b;
  for (int i = 0; i < 8; ++i) {
    a[i] = seed * (int)(threadIdx.x + i);
    b[i] = seed ^ (int)(threadIdx.x * 7 + i);
  }
  v4f c0 = {0, 0, 0, 0}, c1 = c0, c2 = c0, c3 = c0;
  for (int it = 0; it < iters; ++it) {
    c0 = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(a, b, c0, FA, FB, 0, 127, 0, 127);
    c1 = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(a, b, c1, FA, FB, 0, 127, 0, 127);
    c2 = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(a, b, c2, FA, FB, 0, 127, 0, 127);
    c3 = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(a, b, c3, FA, FB, 0, 127, 0, 127);
  }
  const v4f s = c0 + c1 + c2 + c3;
  out[blockIdx.x * 256 + threadIdx.x] = s[0] + s[1] + s[2] + s[3];
}

template <int FA, int FB>
__global__ __launch_bounds__(256) void mfma_rate_32(float* out, int iters, int seed) {
  v8i a, b;
  for (int i = 0; i < 8; ++i) {
    a[i] = seed * (int)(threadIdx.x + i);
    b[i] = seed ^ (int)(threadIdx.x * 7 + i);
  }
  v16f c0 = {}, c1 = {};
  for (int it = 0; it < iters; ++it) {
    c0 = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(a, b, c0, FA, FB, 0, 127, 0, 127);
    c1 = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(a, b, c1, FA, FB, 0, 127, 0, 127);
  }
  float s = 0.0f;
  for (int i = 0; i < 16; ++i) s += c0[i] + c1[i];
  out[blockIdx.x * 256 + threadIdx.x] = s;
}

template <int FA, int FB>
void launch_rate(int shape, int n_wg, int iters, float* out, hipStream_t st) {
  if (shape == 0) hipLaunchKernelGGL((mfma_rate_16<FA, FB>), dim3(n_wg), dim3(256), 0, st, out, iters, 3);
  else hipLaunchKernelGGL((mfma_rate_32<FA, FB>), dim3(n_wg), dim3(256), 0, st, out, iters, 3);
}

}  // namespace

hipError_t launch_mfma_rate_probe(int shape, int fmt_a, int fmt_b, int n_wg, int iters, float* out, double* flop,
                                  hipStream_t st) {
  if ((shape != 0 && shape != 1) || n_wg <= 0 || iters <= 0 || !out) return hipErrorInvalidValue;
  if (fmt_a == 4 && fmt_b == 4) launch_rate<4, 4>(shape, n_wg, iters, out, st);
  else if (fmt_a == 0 && fmt_b == 4) launch_rate<0, 4>(shape, n_wg, iters, out, st);
  else if (fmt_a == 0 && fmt_b == 0) launch_rate<0, 0>(shape, n_wg, iters, out, st);
  else return hipErrorInvalidValue;
  if (flop) *flop = kFlopPerWaveIter * iters * n_wg * 4.0;
  return hipGetLastError();
}
