// Row gather (permute) and the deterministic unweighted combine (unpermute).
//
// permute   : x_sorted = x[row]           (deepseek_v4.py:171, 213-214)
// unpermute : y = zeros(fp32); y.index_add_(0, row, out.float()); y.bf16()
//             (deepseek_v4.py:195-197, 243-245)
// index_add_ accumulates each token's rows in ascending sorted position, which
// for the routed layout is ascending expert id. The combine below sums every
// token's rows in that order starting from +0.0f, one workgroup per token and
// no atomics, so the result is bit-identical to the reference's fp32 sum.
#include "common.h"
#include "kernels.h"

namespace {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

// Rows whose index is outside [0, n_src) are written as zeros.
__global__ __launch_bounds__(256) void gather_rows_kernel(const u32x4* __restrict__ src,
                                                          const int32_t* __restrict__ row, int64_t n_src,
                                                          int64_t n_rows, int64_t row_vecs,
                                                          u32x4* __restrict__ dst) {
  const int64_t total = n_rows * row_vecs;
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < total; i += (int64_t)gridDim.x * 256) {
    const int64_t r = i / row_vecs, c = i - r * row_vecs;
    const int64_t sr = row[r];
    dst[i] = (sr >= 0 && sr < n_src) ? src[sr * row_vecs + c] : u32x4{0u, 0u, 0u, 0u};
  }
}


DSV4_DEV void accumulate8(float* acc, u32x4 v) {
  acc[0] += dsv4::bf16_to_f32(v.x & 0xffffu); acc[1] += dsv4::bf16_to_f32(v.x >> 16);
  acc[2] += dsv4::bf16_to_f32(v.y & 0xffffu); acc[3] += dsv4::bf16_to_f32(v.y >> 16);
  acc[4] += dsv4::bf16_to_f32(v.z & 0xffffu); acc[5] += dsv4::bf16_to_f32(v.z >> 16);
  acc[6] += dsv4::bf16_to_f32(v.w & 0xffffu); acc[7] += dsv4::bf16_to_f32(v.w >> 16);
}

DSV4_DEV u32x4 pack8(const float* acc) {
  u32x4 r;
  r.x = dsv4::f32_to_bf16(acc[0]) | (dsv4::f32_to_bf16(acc[1]) << 16);
  r.y = dsv4::f32_to_bf16(acc[2]) | (dsv4::f32_to_bf16(acc[3]) << 16);
  r.z = dsv4::f32_to_bf16(acc[4]) | (dsv4::f32_to_bf16(acc[5]) << 16);
  r.w = dsv4::f32_to_bf16(acc[6]) | (dsv4::f32_to_bf16(acc[7]) << 16);
  return r;
}

// Order of n <= 64 entries held one per lane (lanes >= n ignored): returns the
// calling lane's rank under (key, lane) ordering. Registers only - no local
// arrays, which would be placed in scratch memory.
DSV4_DEV int wave_rank(long long key, int n) {
  const int lane = threadIdx.x & 63;
  int rank = 0;
  for (int j = 0; j < n; ++j) {
    const long long kj = __shfl(key, j, 64);
    rank += (kj < key || (kj == key && j < lane)) ? 1 : 0;
  }
  return rank;
}

// lane holding rank r (uniform result)
DSV4_DEV int wave_select_rank(int rank, int n, int r) {
  const int lane = threadIdx.x & 63;
  return __ffsll((unsigned long long)__ballot(lane < n && rank == r)) - 1;
}

// Workgroups of 64 lanes tile (token, 512-column chunk); each lane owns 8
// columns. The token's K entries are visited in (expert id, k) order. With
// shared rows (the shared expert's output, bf16 [T, D]) the routed sum is
// rounded to bf16 first and the shared row added to it, as the reference's
// `out + self.shared_experts(hs)` adds two bf16 tensors (deepseek_v4.py:262-264).
// Entries whose id is outside [0, E) were never aligned (moe_align counts them
// in its status) and contribute nothing.
template <typename IdT>
__global__ __launch_bounds__(64) void combine_flat_kernel(const u32x4* __restrict__ src,
                                                          const IdT* __restrict__ ids, int K, int D,
                                                          u32x4* __restrict__ y,
                                                          const u32x4* __restrict__ shared_rows, int E) {
  const int t = blockIdx.y;
  const int lane = threadIdx.x;
  const long long key = lane < K ? (long long)ids[(int64_t)t * K + lane] : 0;
  const int rank = wave_rank(key, K);
  // lane r receives the k of rank r (the inverse permutation, pushed by ds_permute)
  const int k_of_rank = __builtin_amdgcn_ds_permute((lane < K ? rank : lane) * 4, lane);
  const int valid = (key >= 0 && key < E) ? 1 : 0;
  const int vecs = D / 8;
  const int c = blockIdx.x * 64 + lane;
  const bool live = c < vecs;
  const u32x4* srow = src + (int64_t)t * K * vecs + (live ? c : 0);
  float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
  // 8 rows' loads in flight at once, then summed in rank order
  for (int r0 = 0; r0 < K; r0 += 8) {
    u32x4 v[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int k = __shfl(k_of_rank, min(r0 + i, K - 1), 64);
      const bool use = r0 + i < K && __shfl(valid, k, 64) != 0;
      v[i] = use ? srow[(int64_t)k * vecs] : u32x4{0u, 0u, 0u, 0u};
    }
#pragma unroll
    for (int i = 0; i < 8; ++i)
      if (r0 + i < K) accumulate8(acc, v[i]);
  }
  if (!live) return;
  if (shared_rows) {
#pragma unroll
    for (int i = 0; i < 8; ++i) acc[i] = dsv4::bf16_to_f32(dsv4::f32_to_bf16(acc[i]));
    accumulate8(acc, shared_rows[(int64_t)t * vecs + c]);
  }
  y[(int64_t)t * vecs + c] = pack8(acc);
}

__global__ __launch_bounds__(256) void expand_block_scales_kernel(const uint8_t* __restrict__ block, int64_t N,
                                                                  int64_t K32, int64_t KB,
                                                                  uint8_t* __restrict__ out) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= N * K32) return;
  const int64_t n = i / K32, k = i - n * K32;
  out[i] = block[(n / 128) * KB + k / 4];
}

__global__ __launch_bounds__(256) void bucket_rows_kernel(const int32_t* __restrict__ row, int R, int T, int Kmax,
                                                          int32_t* __restrict__ cnt, int32_t* __restrict__ pos,
                                                          int32_t* __restrict__ status) {
  const int u = blockIdx.x * 256 + threadIdx.x;
  if (u >= R) return;
  const int t = row[u];
  if (t < 0 || t >= T) { atomicAdd(status, 1); return; }
  const int s = atomicAdd(&cnt[t], 1);
  if (s < Kmax) pos[(int64_t)t * Kmax + s] = u; else atomicAdd(status, 1);
}

__global__ __launch_bounds__(256) void zero_i32_kernel(int32_t* p, int n) {
  const int i = blockIdx.x * 256 + threadIdx.x;
  if (i < n) p[i] = 0;
}

__global__ __launch_bounds__(256) void combine_rows_kernel(const u32x4* __restrict__ src,
                                                           const int32_t* __restrict__ cnt,
                                                           const int32_t* __restrict__ pos, int Kmax, int D,
                                                           u32x4* __restrict__ y) {
  const int t = blockIdx.x;
  const int n = min(cnt[t], Kmax);
  const int lane = threadIdx.x & 63;
  // each wave ranks the token's row positions itself (ascending position)
  const long long mypos = lane < n ? (long long)pos[(int64_t)t * Kmax + lane] : 0;
  const int rank = wave_rank(mypos, n);
  const int vecs = D / 8;
  for (int c0 = 0; c0 < vecs; c0 += 256) {
    const int c = c0 + threadIdx.x;
    float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
    for (int r = 0; r < n; ++r) {
      const long long row = __shfl(mypos, wave_select_rank(rank, n, r), 64);
      if (c < vecs) accumulate8(acc, src[row * vecs + c]);
    }
    if (c < vecs) y[(int64_t)t * vecs + c] = pack8(acc);
  }
}

}  // namespace

hipError_t launch_moe_gather_rows(const uint8_t* src, int64_t n_src, const int32_t* row, int64_t n_rows,
                                  int64_t row_bytes, uint8_t* dst, hipStream_t st) {
  const int64_t vecs = row_bytes / 16;
  const int64_t total = n_rows * vecs;
  if (total == 0) return hipSuccess;
  int64_t want = (total + 255) / 256;
  hipLaunchKernelGGL(gather_rows_kernel, dim3((int)(want < 16384 ? want : 16384)), dim3(256), 0, st,
                     (const u32x4*)src, row, n_src, n_rows, vecs, (u32x4*)dst);
  return hipGetLastError();
}

hipError_t launch_moe_combine_flat(const uint16_t* src, const void* topk_ids, int ids_int64, int T, int K,
                                   int D, uint16_t* y, hipStream_t st, const uint16_t* shared_rows, int E) {
  if (T == 0 || D == 0) return hipSuccess;
  const dim3 grid((D / 8 + 63) / 64, T);
  if (ids_int64)
    hipLaunchKernelGGL(combine_flat_kernel<long long>, grid, dim3(64), 0, st, (const u32x4*)src,
                       (const long long*)topk_ids, K, D, (u32x4*)y, (const u32x4*)shared_rows, E);
  else
    hipLaunchKernelGGL(combine_flat_kernel<int32_t>, grid, dim3(64), 0, st, (const u32x4*)src,
                       (const int32_t*)topk_ids, K, D, (u32x4*)y, (const u32x4*)shared_rows, E);
  return hipGetLastError();
}

hipError_t launch_expand_block_scales(const uint8_t* block, int64_t N, int64_t K, uint8_t* out, hipStream_t st) {
  const int64_t K32 = K / 32, KB = (K + 127) / 128, total = N * K32;
  if (total == 0) return hipSuccess;
  if ((total + 255) / 256 > 0x7fffffffLL) return hipErrorInvalidValue;
  hipLaunchKernelGGL(expand_block_scales_kernel, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, st, block, N,
                     K32, KB, out);
  return hipGetLastError();
}

hipError_t launch_moe_unpermute_rows(const uint16_t* src, const int32_t* row, int R, int T, int Kmax, int D,
                                     int32_t* work_cnt, int32_t* work_pos, int32_t* status, uint16_t* y,
                                     hipStream_t st) {
  if (T == 0) return hipSuccess;
  hipLaunchKernelGGL(zero_i32_kernel, dim3((T + 255) / 256), dim3(256), 0, st, work_cnt, T);
  hipLaunchKernelGGL(zero_i32_kernel, dim3(1), dim3(256), 0, st, status, 1);
  if (R > 0)
    hipLaunchKernelGGL(bucket_rows_kernel, dim3((R + 255) / 256), dim3(256), 0, st, row, R, T, Kmax, work_cnt,
                       work_pos, status);
  hipLaunchKernelGGL(combine_rows_kernel, dim3(T), dim3(256), 0, st, (const u32x4*)src, work_cnt, work_pos,
                     Kmax, D, (u32x4*)y);
  return hipGetLastError();
}
