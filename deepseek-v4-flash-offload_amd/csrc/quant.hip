// MXFP4 weight dequant, FP8 activation round trip and MXFP4 activation quant.
//
// All three are HBM-bound streaming kernels: one thread owns 8 consecutive
// elements (16 B of bf16), consecutive lanes own consecutive 8-element groups,
// so every load and store instruction of a wave covers one contiguous span.
#include "common.h"
#include "kernels.h"
#include "quant_dev.h"

using namespace dsv4;

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

// ---------------------------------------------------------------------------
// MXFP4 weight -> bf16 (npu_ops.py:142-158).
// Group g = 8 elements = packed dword g; its scale is byte g/4 (32 elements per
// scale). The hardware scaled convert produces LUT[nibble] * 2^(s-127) rounded
// to bf16, which equals the reference's fp32 product (exact: <= 2 significant
// bits) except for nibble 8, which the hardware decodes to -0.0 (the reference
// table holds +0.0), and for scale byte 255, where the reference multiplies by
// +inf. Both are corrected here.
// ---------------------------------------------------------------------------
DSV4_DEV uint32_t fix_neg_zero(uint32_t r) {
  uint32_t t = r & 0x7fff7fffu;
  uint32_t nz = (t + 0x7fff7fffu) & 0x80008000u;  // bit 15 of a half set iff that half != +-0
  return r & (0x7fff7fffu | nz);
}

DSV4_DEV uint32_t inf_scale_pair(uint32_t byte) {
  uint32_t r = 0;
  for (int h = 0; h < 2; ++h) {
    uint32_t nib = (byte >> (4 * h)) & 15u;
    uint32_t v = ((nib & 7u) == 0) ? 0x7fc0u : ((nib & 8u) ? 0xff80u : 0x7f80u);
    r |= v << (16 * h);
  }
  return r;
}

DSV4_DEV u32x4 dequant8(uint32_t p, uint32_t s) {
  float sc = e8m0_to_f32(s);
  u32x4 r;
  r.x = fix_neg_zero(__builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(p, sc, 0)));
  r.y = fix_neg_zero(__builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(p, sc, 1)));
  r.z = fix_neg_zero(__builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(p, sc, 2)));
  r.w = fix_neg_zero(__builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(p, sc, 3)));
  if (s == 255u) {
    r.x = inf_scale_pair(p & 0xffu);
    r.y = inf_scale_pair((p >> 8) & 0xffu);
    r.z = inf_scale_pair((p >> 16) & 0xffu);
    r.w = inf_scale_pair(p >> 24);
  }
  return r;
}

// Four 8-element groups per thread, spaced one grid-stride apart, so each
// load/store instruction of a wave still covers one contiguous span while four
// independent loads are in flight per lane. Output is written with
// non-temporal stores (it is not re-read by this kernel). The launcher sizes
// the grid so that 4 * grid * 256 >= n_groups; the guards only bite in the
// last workgroups.
constexpr int kDequantGroupsPerThread = 4;

__global__ __launch_bounds__(256) void mxfp4_dequant_kernel(const uint32_t* __restrict__ packed,
                                                             const uint8_t* __restrict__ scales,
                                                             u32x4* __restrict__ out, int64_t n_groups) {
  const int64_t stride = (int64_t)gridDim.x * 256;
  const int64_t g0 = (int64_t)blockIdx.x * 256 + threadIdx.x;
  uint32_t p[kDequantGroupsPerThread], s[kDequantGroupsPerThread];
#pragma unroll
  for (int i = 0; i < kDequantGroupsPerThread; ++i) {
    const int64_t g = g0 + i * stride;
    if (g < n_groups) {
      p[i] = __builtin_nontemporal_load(packed + g);
      s[i] = scales[g >> 2];
    }
  }
#pragma unroll
  for (int i = 0; i < kDequantGroupsPerThread; ++i) {
    const int64_t g = g0 + i * stride;
    if (g < n_groups) __builtin_nontemporal_store(dequant8(p[i], s[i]), out + g);
  }
}

// Several tensors in one launch (an expert's w1, w2, w3), each in the checkpoint
// layout or the MFMA-tiled one (dsv4_mxfp4_tile_weights). A workgroup takes 256
// consecutive 16-byte packed chunks (32 elements, one E8M0 scale each) of one
// tensor in SOURCE order - one contiguous 4 KB load - and dequantises each into its
// 64 output bytes in LDS, placed so that the 16 KB then leave in whole contiguous
// runs: a checkpoint-layout source maps to 16 KB of contiguous output; a tiled one
// to two 16-row x 256-k units, each 16 row segments of 512 bytes. (Writing each
// chunk's 64 bytes straight from its lane scatters 16-byte pieces over 16 rows per
// store instruction: measured at 0.6 TB/s.) Tiled chunk c of a tensor holds
// packed[16 nt + r][16 (8 j + 2 g + ji) .. +16) with c = ((nt K/256 + j) 2 + ji) 64 +
// r + 16 g. Workgroup w belongs to the last job q with wg_start[q] <= w (uniform).
__global__ __launch_bounds__(256) void mxfp4_dequant_multi_kernel(Dsv4DequantJobs J) {
  __shared__ __attribute__((aligned(16))) u32x4 buf[256 * 4];  // 16 KB of bf16 output
  const int t = threadIdx.x;
  int q = 0;
#pragma unroll
  for (int jb = 1; jb < kDequantMaxJobs; ++jb)
    if (jb < J.n && (int64_t)blockIdx.x >= J.wg_start[jb]) q = jb;
  const uint8_t* pk = J.packed[0];
  const uint8_t* sc = J.scales[0];
  uint16_t* ot = J.out[0];
  int64_t kc = J.kc[0], nchunks = J.start[1] - J.start[0], wg0 = J.wg_start[0];
  int tl = J.tiled[0];
#pragma unroll
  for (int jb = 1; jb < kDequantMaxJobs; ++jb)
    if (jb == q) {
      pk = J.packed[jb];
      sc = J.scales[jb];
      ot = J.out[jb];
      kc = J.kc[jb];
      nchunks = J.start[jb + 1] - J.start[jb];
      wg0 = J.wg_start[jb];
      tl = J.tiled[jb];
    }
  const int64_t c0 = ((int64_t)blockIdx.x - wg0) * 256;  // first chunk of this workgroup
  const int64_t c = c0 + t;
  const int64_t nst = kc >> 3;  // 256-k stages per row (tiled sources)
  if (c < nchunks) {
    int64_t nat = c;  // checkpoint-layout chunk index n * K/32 + cb
    int lpos = 4 * t;  // u32x4 slot of the chunk's first 16 output bytes in buf
    if (tl) {
      const int L = (int)(c & 63), ji = (int)((c >> 6) & 1);
      const int64_t u = c >> 7;  // 16-row x 256-k unit = nt * nst + j
      const int r = L & 15, cb8 = 2 * (L >> 4) + ji;
      nat = (16 * (u / nst) + r) * kc + 8 * (u % nst) + cb8;
      lpos = ((t >> 7) * 512 + r * 32 + cb8 * 4);
    }
    const u32x4 p = __builtin_nontemporal_load((const u32x4*)pk + c);
    const uint32_t s = sc[nat];
    buf[lpos] = dequant8(p.x, s);
    buf[lpos + 1] = dequant8(p.y, s);
    buf[lpos + 2] = dequant8(p.z, s);
    buf[lpos + 3] = dequant8(p.w, s);
  }
  __syncthreads();
  const int64_t nvalid = nchunks - c0;  // chunks of this workgroup (<= 256 in its last one)
#pragma unroll
  for (int pass = 0; pass < 4; ++pass) {
    const int slot = pass * 256 + t;  // 16-byte output piece of buf
    if (tl) {
      // unit (pass / 2) of the workgroup: rows 8 (pass % 2) + t / 32, bytes 16 (t % 32) of a 512-byte segment
      const int unit = pass >> 1;
      if (128 * unit >= nvalid) continue;
      const int64_t u = (c0 >> 7) + unit;
      const int r = 8 * (pass & 1) + (t >> 5);
      const int64_t n = 16 * (u / nst) + r;
      __builtin_nontemporal_store(buf[slot], (u32x4*)ot + n * (kc * 4) + 32 * (u % nst) + (t & 31));
    } else {
      if (slot / 4 >= nvalid) continue;
      __builtin_nontemporal_store(buf[slot], (u32x4*)ot + c0 * 4 + slot);
    }
  }
}

// ---------------------------------------------------------------------------
// Activation quantisers (bodies in quant_dev.h): one thread per 8-element group.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void fp8_act_quant_kernel(const uint4* __restrict__ x, int64_t n_groups,
                                                             uint4* __restrict__ rt, uint2* __restrict__ codes,
                                                             float* __restrict__ scale_f32,
                                                             uint32_t* __restrict__ scale_e8m0x4) {
  const int64_t g = (int64_t)blockIdx.x * 256 + threadIdx.x;
  fp8_quant_group(x, g, g < n_groups, rt, codes, scale_f32, scale_e8m0x4);  // n_groups % 16 == 0
}

__global__ __launch_bounds__(256) void mxfp4_act_quant_kernel(const uint4* __restrict__ x, int64_t n_groups,
                                                               int rule, uint32_t* __restrict__ packed,
                                                               uint8_t* __restrict__ scale,
                                                               uint4* __restrict__ dq) {
  const int64_t g = (int64_t)blockIdx.x * 256 + threadIdx.x;
  mxfp4_quant_group(x, g, g < n_groups, rule, packed, scale, dq);  // n_groups % 4 == 0
}

// ---------------------------------------------------------------------------
// launchers
// ---------------------------------------------------------------------------
// ---------------------------------------------------------------------------
// y[m] = bf16(x[m] @ dequant(W)^T) for a few activation rows (the config-0
// "dequant + bf16 GEMV" of the reference's CPU path: npu_ops.py:142-158 then
// F.linear). One wave per kGemvRows weight rows: per pass lane L takes 32-element
// block L (+64 per pass) of every one of its rows - the rows' 16 packed bytes
// and E8M0 byte are all loaded before any is used, so kGemvRows loads per lane
// are in flight - decodes them with the hardware scaled fp4 -> fp32 convert
// (exact) and accumulates x * w in fp32; wave sums give the dot products. x stays bf16 (no activation
// quantisation). HBM-bound on the weight bytes.
// ---------------------------------------------------------------------------
constexpr int kGemvRows = 8;

template <int MB>
__global__ __launch_bounds__(256) void mxfp4_gemv_kernel(const uint16_t* __restrict__ x, int M,
                                                         const uint8_t* __restrict__ packed,
                                                         const uint8_t* __restrict__ scales, int N, int K,
                                                         uint16_t* __restrict__ y) {
  const int lane = threadIdx.x & 63;
  const int n0 = (blockIdx.x * 4 + (threadIdx.x >> 6)) * kGemvRows;
  if (n0 >= N) return;
  const int nblk = K / 32;
  float acc[kGemvRows][MB];
#pragma unroll
  for (int r = 0; r < kGemvRows; ++r)
#pragma unroll
    for (int m = 0; m < MB; ++m) acc[r][m] = 0.f;
  for (int b = lane; b < nblk; b += 64) {
    u32x4 p[kGemvRows];
    uint32_t sb[kGemvRows];
#pragma unroll
    for (int r = 0; r < kGemvRows; ++r) {
      const int n = min(n0 + r, N - 1);  // rows past N repeat the last row; never stored
      p[r] = *(const u32x4*)(packed + (int64_t)n * (K / 2) + 16 * b);
      sb[r] = scales[(int64_t)n * nblk + b];
    }
    uint32_t xw[MB][16];  // the x rows' 32 bf16 values of this block, packed
#pragma unroll
    for (int m = 0; m < MB; ++m) {
      const u32x4* xr = (const u32x4*)(x + (int64_t)min(m, M - 1) * K + 32 * b);
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        const u32x4 v = xr[c];
        xw[m][4 * c] = v.x, xw[m][4 * c + 1] = v.y, xw[m][4 * c + 2] = v.z, xw[m][4 * c + 3] = v.w;
      }
    }
    // one x row: its 32 floats once per block; more rows: converted where used
    float xf1[32];
    if constexpr (MB == 1) {
#pragma unroll
      for (int j = 0; j < 16; ++j) {
        xf1[2 * j] = bf16_to_f32(xw[0][j] & 0xffffu);
        xf1[2 * j + 1] = bf16_to_f32(xw[0][j] >> 16);
      }
    }
#pragma unroll
    for (int r = 0; r < kGemvRows; ++r) {
      // hardware scaled convert: 2 nibbles (low first) -> LUT * 2^(s-127) in fp32, exact
      // (nibble 8 gives -0.0 where the table holds +0.0: the same contribution to a sum)
      const float sc = e8m0_to_f32(sb[r]);
      const uint32_t pw[4] = {p[r].x, p[r].y, p[r].z, p[r].w};
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        typedef float f32x2 __attribute__((ext_vector_type(2)));
        const f32x2 w0 = __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(pw[q], sc, 0);
        const f32x2 w1 = __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(pw[q], sc, 1);
        const f32x2 w2 = __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(pw[q], sc, 2);
        const f32x2 w3 = __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(pw[q], sc, 3);
        const float wv[8] = {w0.x, w0.y, w1.x, w1.y, w2.x, w2.y, w3.x, w3.y};
#pragma unroll
        for (int i = 0; i < 8; ++i) {
#pragma unroll
          for (int m = 0; m < MB; ++m) {
            float xv;
            if constexpr (MB == 1) {
              xv = xf1[8 * q + i];
            } else {
              const uint32_t d = xw[m][4 * q + i / 2];
              xv = bf16_to_f32((i & 1) ? (d >> 16) : (d & 0xffffu));
            }
            acc[r][m] = fmaf(xv, wv[i], acc[r][m]);
          }
        }
      }
    }
  }
#pragma unroll
  for (int r = 0; r < kGemvRows; ++r)
#pragma unroll
    for (int m = 0; m < MB; ++m) {
      float v = acc[r][m];
      for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
      if (lane == 0 && m < M && n0 + r < N) y[(int64_t)m * N + n0 + r] = (uint16_t)f32_to_bf16(v);
    }
}

// M = 1 or up to 4 rows per launch; more rows run as several launches
hipError_t launch_mxfp4_gemv(const uint16_t* x, int M, const uint8_t* packed, const uint8_t* scales, int N, int K,
                             uint16_t* y, hipStream_t st) {
  const dim3 grid((N + 4 * kGemvRows - 1) / (4 * kGemvRows));
  for (int m0 = 0; m0 < M; m0 += 4) {
    const int mc = min(4, M - m0);
    const uint16_t* xm = x + (int64_t)m0 * K;
    uint16_t* ym = y + (int64_t)m0 * N;
    if (mc == 1)
      hipLaunchKernelGGL((mxfp4_gemv_kernel<1>), grid, dim3(256), 0, st, xm, mc, packed, scales, N, K, ym);
    else
      hipLaunchKernelGGL((mxfp4_gemv_kernel<4>), grid, dim3(256), 0, st, xm, mc, packed, scales, N, K, ym);
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
  }
  return hipSuccess;
}

// ---------------------------------------------------------------------------
// MFMA-tiled layout of packed E2M1 weights W [N, K/2] (N % 16 == 0, K % 256 == 0):
//   tiled[nt][j][ji][g][r][e] = W[16 nt + r][128 j + 32 g + 16 ji + e]
// (nt: 16-row tile, j: 256-wide K stage, ji: MFMA of the stage, lane L = r + 16 g,
// e: byte of the lane's 16). Lane L of MFMA ji of stage j of a tile finds its
// operand at ((nt * K/256 + j) * 2 + ji) * 1024 + 16 L, so every weight load of
// the grouped GEMMs covers one contiguous 1 KB (eight whole 128-byte lines); in
// the checkpoint layout each load instruction touches 16 rows x 64 bytes.
// One thread moves one 16-byte chunk; `inverse` maps tiled back to natural.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void mxfp4_tile_kernel(const u32x4* __restrict__ src, u32x4* __restrict__ dst,
                                                         int64_t n_chunks, int64_t chunks_per_row, int nst,
                                                         int inverse) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;  // natural chunk index
  if (i >= n_chunks) return;
  const int64_t n = i / chunks_per_row;
  const int cb = (int)(i % chunks_per_row);
  const int j = cb >> 3, c = cb & 7, g = c >> 1, ji = c & 1;
  const int64_t nt = n >> 4;
  const int r = (int)(n & 15);
  const int64_t t = ((nt * nst + j) * 2 + ji) * 64 + (r + 16 * g);  // tiled chunk index
  if (inverse)
    dst[i] = src[t];
  else
    dst[t] = src[i];
}

hipError_t launch_mxfp4_tile(const uint8_t* src, uint8_t* dst, int64_t N, int64_t K, int inverse, hipStream_t st) {
  const int64_t chunks_per_row = K / 32;  // 16 bytes = 32 E2M1 values
  const int64_t n_chunks = N * chunks_per_row;
  if (n_chunks == 0) return hipSuccess;
  const int64_t grid = (n_chunks + 255) / 256;
  if (grid > 0x7fffffffLL || K / 256 > 0x7fffffffLL) return hipErrorInvalidValue;
  hipLaunchKernelGGL(mxfp4_tile_kernel, dim3((unsigned)grid), dim3(256), 0, st, (const u32x4*)src, (u32x4*)dst,
                     n_chunks, chunks_per_row, (int)(K / 256), inverse);
  return hipGetLastError();
}

hipError_t launch_mxfp4_dequant(const uint8_t* packed, const uint8_t* scales, uint16_t* out,
                                int64_t n_elems, hipStream_t st) {
  const int64_t n_groups = n_elems / 8;
  if (n_groups == 0) return hipSuccess;
  const int64_t per_wg = 256LL * kDequantGroupsPerThread;
  const int64_t grid = (n_groups + per_wg - 1) / per_wg;
  if (grid > 0x7fffffffLL) return hipErrorInvalidValue;
  hipLaunchKernelGGL(mxfp4_dequant_kernel, dim3((unsigned)grid), dim3(256), 0, st,
                     (const uint32_t*)packed, scales, (u32x4*)out, n_groups);
  return hipGetLastError();
}

hipError_t launch_mxfp4_dequant_multi(const Dsv4DequantJobs& jobs, hipStream_t st) {
  if (jobs.n < 1 || jobs.n > kDequantMaxJobs) return hipErrorInvalidValue;
  Dsv4DequantJobs J = jobs;
  int64_t grid = 0;
  for (int q = 0; q < J.n; ++q) {  // whole workgroups of 256 chunks per tensor
    J.wg_start[q] = grid;
    grid += (J.start[q + 1] - J.start[q] + 255) / 256;
  }
  if (grid == 0) return hipSuccess;
  if (grid > 0x7fffffffLL) return hipErrorInvalidValue;
  hipLaunchKernelGGL(mxfp4_dequant_multi_kernel, dim3((unsigned)grid), dim3(256), 0, st, J);
  return hipGetLastError();
}

hipError_t launch_fp8_act_quant(const uint16_t* x, int64_t n_elems, uint16_t* rt, uint8_t* codes,
                                float* scale_f32, uint8_t* scale_e8m0x4, hipStream_t st) {
  int64_t n_groups = n_elems / 8;
  if (n_groups == 0) return hipSuccess;
  int grid = (int)((n_groups + 255) / 256);
  hipLaunchKernelGGL(fp8_act_quant_kernel, dim3(grid), dim3(256), 0, st, (const uint4*)x, n_groups,
                     (uint4*)rt, (uint2*)codes, scale_f32, (uint32_t*)scale_e8m0x4);
  return hipGetLastError();
}

hipError_t launch_mxfp4_act_quant(const uint16_t* x, int64_t n_elems, int rule, uint8_t* packed,
                                  uint8_t* scale, uint16_t* dq, hipStream_t st) {
  int64_t n_groups = n_elems / 8;
  if (n_groups == 0) return hipSuccess;
  int grid = (int)((n_groups + 255) / 256);
  hipLaunchKernelGGL(mxfp4_act_quant_kernel, dim3(grid), dim3(256), 0, st, (const uint4*)x, n_groups,
                     rule, (uint32_t*)packed, scale, (uint4*)dq);
  return hipGetLastError();
}
