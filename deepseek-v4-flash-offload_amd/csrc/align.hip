// moe_align: stable counting sort of the routed (token, k) entries by expert.
//
// Restates deepseek_v4.py:155-164 (flatten, argsort, bincount, nonzero) with
// the stable order (expert ascending, flat index ascending), and derives the
// padded block layout used by the grouped GEMM: each expert's rows are padded
// to a multiple of block_m so that an M block never straddles two experts.
//
// One workgroup (256 threads for decode-sized inputs, 1024 otherwise):
//   1. LDS histogram (atomic increments; counts are order-independent).
//   2. Three block-wide exclusive scans: unpadded offsets, padded offsets,
//      active-expert ranks.
//   3. Stable scatter in chunks of one entry per thread: within a wave,
//      entries with the same expert are found by a ballot match over the key
//      bits; the rank is the popcount of lower lanes; per-wave counts go
//      through LDS to rank across the waves; a running count per expert
//      carries across chunks.
#include "common.h"
#include "kernels.h"
#include "quant_dev.h"
#include "route_dev.h"

namespace {

// exclusive scan of one int per thread across the NT-thread workgroup; returns the total.
template <int NT>
__device__ int block_exclusive_scan(int v, int* lds_waves, int* out_total) {
  constexpr int kWaves = NT / 64;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  int incl = v;
  for (int o = 1; o < 64; o <<= 1) {
    int t = __shfl_up(incl, o, 64);
    if (lane >= o) incl += t;
  }
  if (lane == 63) lds_waves[wave] = incl;
  __syncthreads();
  if (wave == 0) {
    int w = (lane < kWaves) ? lds_waves[lane] : 0;
    int wi = w;
    for (int o = 1; o < 64; o <<= 1) {
      int t = __shfl_up(wi, o, 64);
      if (lane >= o) wi += t;
    }
    if (lane < kWaves) lds_waves[lane] = wi - w;
    if (lane == kWaves - 1) *out_total = wi;
  }
  __syncthreads();
  int r = lds_waves[wave] + incl - v;
  __syncthreads();
  return r;
}

// Padded layout from the per-expert counts (thread e < E holds count c of
// expert e; bad = out-of-range ids): unpadded and padded offsets, active ranks,
// block_expert, the padding sentinel, num_post_padded, the optional per-expert
// outputs, and off_u/off_p (LDS) for the scatter. n_shared > 0 adds the shared
// expert as one more group, placed first: n_shared rows with flat indices
// R .. R+n_shared-1 and block_expert = E in the leading blocks (its
// workgroups stream twice the bytes of a routed one, so they are dispatched
// first rather than left as the launch's tail). The routed experts follow;
// the padding sentinel is R + n_shared.
// write = false: only off_u/off_p (for workgroups that recompute the layout
// to scatter their own entries).
// hot (optional, chunked align only): experts with at least hot->hot_min rows get
// their own layout of kHotBlockM-row blocks (hot->sorted_ids / block_expert /
// num_post_padded) and no blocks in the main layout; off_p then holds -1 - (their
// padded offset in the hot layout), which tells the scatter where an entry goes.
template <int NT>
__device__ void align_layout(int c, int bad, int R, int E, int block_m, int max_blocks, int n_shared,
                             const Dsv4AlignOut& o, int* off_u, int* off_p, bool write = true,
                             const Dsv4AlignHot* hot = nullptr) {
  constexpr int kWaves = NT / 64;
  __shared__ int scan_tmp[kWaves];
  __shared__ int totals[4];
  const int tid = threadIdx.x;
  const bool is_hot = hot && hot->hot_min > 0 && c >= hot->hot_min;
  const int padded = is_hot ? 0 : ((c + block_m - 1) / block_m) * block_m;
  const int padded_h = is_hot ? ((c + kHotBlockM - 1) / kHotBlockM) * kHotBlockM : 0;
  const int shared_padded = ((n_shared + block_m - 1) / block_m) * block_m;
  const int ou = block_exclusive_scan<NT>(c, scan_tmp, &totals[0]);
  const int op = block_exclusive_scan<NT>(padded, scan_tmp, &totals[1]) + shared_padded;
  const int oa = block_exclusive_scan<NT>(c > 0 ? 1 : 0, scan_tmp, &totals[2]);
  const int oph = hot ? block_exclusive_scan<NT>(padded_h, scan_tmp, &totals[3]) : 0;
  if (tid < E) {
    off_u[tid] = ou;
    off_p[tid] = is_hot ? -1 - oph : op;
  }
  if (!write) {
    __syncthreads();
    return;
  }
  if (tid < E) {
    if (o.counts) o.counts[tid] = c;
    if (o.expert_start) o.expert_start[tid] = is_hot ? -1 : op;
    if (o.active) o.active[tid] = -1;
  }
  __syncthreads();
  const int pad_id = R + n_shared;  // padding sentinel
  const int total_padded = totals[1] + shared_padded;
  const int total_blocks = total_padded / block_m;
  const int cap = max_blocks * block_m;
  if (tid < E) {
    if (o.active && c > 0) o.active[oa] = tid;
    const int b0 = op / block_m, b1 = min((op + padded) / block_m, max_blocks);
    for (int b = b0; b < b1; ++b) o.block_expert[b] = tid;
    const int p1 = min(op + padded, cap);
    for (int p = op + c; p < p1; ++p) o.sorted_ids[p] = pad_id;
    if (is_hot) {
      const int cap_h = hot->max_blocks * kHotBlockM;
      const int h0 = oph / kHotBlockM, h1 = min((oph + padded_h) / kHotBlockM, hot->max_blocks);
      for (int b = h0; b < h1; ++b) hot->block_expert[b] = tid;
      const int q1 = min(oph + padded_h, cap_h);
      for (int q = oph + c; q < q1; ++q) hot->sorted_ids[q] = pad_id;
    }
  }
  if (hot && tid == 0) {
    const int total_h = totals[3];
    hot->num_post_padded[0] = min(total_h, hot->max_blocks * kHotBlockM);
  }
  // the shared expert's group: rows R + i in order, ahead of the routed experts
  for (int i = tid; i < shared_padded; i += NT) {
    if (i < cap) {
      o.sorted_ids[i] = i < n_shared ? R + i : pad_id;
      if (i % block_m == 0) o.block_expert[i / block_m] = E;
    }
  }
  if (tid == 0) {
    o.num_post_padded[0] = min(total_padded, cap);
    if (o.num_active) o.num_active[0] = totals[2];
    const bool hot_over = hot && totals[3] > hot->max_blocks * kHotBlockM;
    if (o.status) o.status[0] = bad + ((total_blocks > max_blocks || hot_over) ? (1 << 30) : 0);
  }
  __syncthreads();
}

// Stable scatter of entries [i0, i1): in chunks of one entry per thread,
// entries with the same expert are found within a wave by a ballot match over
// the key bits; the rank is the popcount of lower lanes; per-wave counts go
// through LDS to rank across the waves; running[e] (LDS, the rank of the
// range's first entry of expert e) carries across chunks. have_id0: the
// caller already holds ids[i0 + tid] in id0.
template <typename IdT, int NT>
__device__ void align_scatter_range(const IdT* __restrict__ ids, const float* __restrict__ topk_w, int i0, int i1,
                                    int K, int E, int block_m, int max_blocks, const int* off_u, const int* off_p,
                                    int* running, int* wcount, const Dsv4AlignOut& o, bool have_id0,
                                    long long id0, const Dsv4AlignHot* hot = nullptr) {
  constexpr int kWaves = NT / 64;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  int nbits = 0;
  while ((1 << nbits) < E + 1) ++nbits;
  const unsigned long long lt_mask = (lane == 0) ? 0ull : (~0ull >> (64 - lane));
  for (int base = i0; base < i1; base += NT) {
    const int i = base + tid;
    int e = E;
    if (i < i1) {
      long long ee = (have_id0 && base == i0) ? id0 : (long long)ids[i];
      if (ee >= 0 && ee < E) e = (int)ee;
    }
    unsigned long long peers = __ballot(1);
    for (int b = 0; b < nbits; ++b) {
      const int bit = (e >> b) & 1;
      const unsigned long long bal = __ballot(bit);
      peers &= bit ? bal : ~bal;
    }
    const int rank = __popcll(peers & lt_mask);
    if (rank == 0) wcount[wave * (E + 1) + e] = __popcll(peers);
    __syncthreads();
    if (i < i1 && e < E) {
      int r = running[e] + rank;
      for (int w = 0; w < wave; ++w) r += wcount[w * (E + 1) + e];
      const int u = off_u[e] + r;
      const int op = off_p[e];
      if (o.order) o.order[u] = i;
      if (o.s_e) o.s_e[u] = e;
      if (o.s_w) o.s_w[u] = topk_w ? topk_w[i] : 0.0f;
      if (o.row) o.row[u] = i / K;
      if (op >= 0) {
        const int p = op + r;
        if (p < max_blocks * block_m) o.sorted_ids[p] = i;
        if (o.padded_pos) o.padded_pos[i] = p;
      } else {  // hot layout (only when hot is given: off_p >= 0 otherwise)
        const int q = -1 - op + r;
        if (q < hot->max_blocks * kHotBlockM) hot->sorted_ids[q] = i;
        if (o.padded_pos) o.padded_pos[i] = -1 - q;
      }
    }
    __syncthreads();
    for (int ex = tid; ex < E + 1; ex += NT) {
      int s = 0;
      for (int w = 0; w < kWaves; ++w) { s += wcount[w * (E + 1) + ex]; wcount[w * (E + 1) + ex] = 0; }
      running[ex] += s;
    }
    __syncthreads();
  }
}

// One workgroup does it all (decode-sized inputs).
template <typename IdT, int NT>
__device__ void align_body(const IdT* __restrict__ ids, const float* __restrict__ topk_w, int R, int K, int E,
                           int block_m, int max_blocks, const Dsv4AlignOut& o, int n_shared = 0) {
  constexpr int kWaves = NT / 64;
  extern __shared__ int lds[];
  int* cnt = lds;                    // [E + 1] (slot E collects out-of-range ids)
  int* off_u = cnt + (E + 1);        // [E]
  int* off_p = off_u + E;            // [E]
  int* running = off_p + E;          // [E + 1]
  int* wcount = running + (E + 1);   // [kWaves][E + 1]

  const int tid = threadIdx.x;
  for (int i = tid; i < E + 1; i += NT) { cnt[i] = 0; running[i] = 0; }
  for (int i = tid; i < kWaves * (E + 1); i += NT) wcount[i] = 0;
  __syncthreads();

  // 1. histogram (the first chunk's ids stay in registers for the scatter)
  const long long id0 = tid < R ? (long long)ids[tid] : 0;
  for (int i = tid; i < R; i += NT) {
    long long e = i == tid ? id0 : (long long)ids[i];
    atomicAdd(&cnt[(e < 0 || e >= E) ? E : (int)e], 1);
  }
  __syncthreads();

  // 2. layout (E <= NT)
  align_layout<NT>(tid < E ? cnt[tid] : 0, cnt[E], R, E, block_m, max_blocks, n_shared, o, off_u, off_p);

  // 3. stable scatter
  align_scatter_range<IdT, NT>(ids, topk_w, 0, R, K, E, block_m, max_blocks, off_u, off_p, running, wcount, o,
                               true, id0);
}

// ---- chunked align for many entries: two launches ------------------------
// (1) per-chunk counts cc[c][E + 1] (slot E: out-of-range ids), in the same
//     launch as the quantisation of x; (2) every chunk's workgroup derives the
//     layout and its own per-expert start from cc and scatters its entries, so
//     the order is the single-workgroup order (expert ascending, flat index
//     ascending); workgroup 0 writes the layout outputs.
constexpr int kAlignChunk = 1024;  // entries per chunk

template <typename IdT, int NT>
__device__ void align_count_chunk(const IdT* __restrict__ ids, int R, int E, int c, int* cc) {
  extern __shared__ int lds[];
  int* cnt = lds;  // [E + 1]
  for (int i = threadIdx.x; i < E + 1; i += NT) cnt[i] = 0;
  __syncthreads();
  const int i1 = min(R, (c + 1) * kAlignChunk);
  for (int i = c * kAlignChunk + threadIdx.x; i < i1; i += NT) {
    const long long e = (long long)ids[i];
    atomicAdd(&cnt[(e < 0 || e >= E) ? E : (int)e], 1);
  }
  __syncthreads();
  for (int e = threadIdx.x; e < E + 1; e += NT) cc[(int64_t)c * (E + 1) + e] = cnt[e];
}

template <typename IdT, int NT, int QF>
__global__ __launch_bounds__(NT) void align_count_quant_kernel(const IdT* __restrict__ ids, int R, int E, int C,
                                                               int* __restrict__ cc, const uint4* __restrict__ x,
                                                               int64_t n_groups, int rule, void* q_codes,
                                                               void* q_scale) {
  if ((int)blockIdx.x < C) {
    align_count_chunk<IdT, NT>(ids, R, E, blockIdx.x, cc);
    return;
  }
  const int64_t g = (int64_t)(blockIdx.x - C) * NT + threadIdx.x;
  if (QF == 0)
    dsv4::fp8_quant_group(x, g, g < n_groups, nullptr, (uint2*)q_codes, nullptr, (uint32_t*)q_scale);
  else if (QF == 1)
    dsv4::mxfp4_quant_group(x, g, g < n_groups, rule, (uint32_t*)q_codes, (uint8_t*)q_scale, nullptr);
}

// Every chunk's workgroup sums the chunk counts itself (its exclusive
// per-expert start and the totals), rebuilds the layout offsets, and scatters
// its entries; workgroup 0 also writes the layout outputs.
template <typename IdT, int NT>
__global__ __launch_bounds__(NT) void align_scatter_kernel(const IdT* __restrict__ ids,
                                                           const float* __restrict__ topk_w, int R, int K, int E,
                                                           int C, int block_m, int max_blocks, int n_shared,
                                                           const int* __restrict__ cc, Dsv4AlignOut o,
                                                           Dsv4AlignHot hot) {
  const Dsv4AlignHot* hp = hot.hot_min > 0 ? &hot : nullptr;
  constexpr int kWaves = NT / 64;
  extern __shared__ int lds[];
  int* off_u = lds;                  // [E]
  int* off_p = off_u + E;            // [E]
  int* running = off_p + E;          // [E + 1]
  int* wcount = running + (E + 1);   // [kWaves][E + 1]
  __shared__ int bad;
  const int c = blockIdx.x, tid = threadIdx.x;
  int tot = 0;  // count of expert tid
  for (int e = tid; e <= E; e += NT) {
    int before = 0, all = 0;
    for (int c0 = 0; c0 < C; c0 += 16) {  // 16 independent loads in flight
      int v[16];
#pragma unroll
      for (int j = 0; j < 16; ++j) v[j] = c0 + j < C ? cc[(int64_t)(c0 + j) * (E + 1) + e] : 0;
#pragma unroll
      for (int j = 0; j < 16; ++j) {
        before += c0 + j < c ? v[j] : 0;
        all += v[j];
      }
    }
    running[e] = before;
    if (e == tid) tot = all;
    if (e == E) bad = all;  // slot E: out-of-range ids
  }
  for (int i = tid; i < kWaves * (E + 1); i += NT) wcount[i] = 0;
  __syncthreads();
  align_layout<NT>(tid < E ? tot : 0, bad, R, E, block_m, max_blocks, n_shared, o, off_u, off_p, c == 0, hp);
  align_scatter_range<IdT, NT>(ids, topk_w, c * kAlignChunk, min(R, (c + 1) * kAlignChunk), K, E, block_m,
                               max_blocks, off_u, off_p, running, wcount, o, false, 0, hp);
}

template <typename IdT, int NT>
__global__ __launch_bounds__(NT) void moe_align_kernel(const IdT* __restrict__ ids,
                                                       const float* __restrict__ topk_w, int R, int K,
                                                       int E, int block_m, int max_blocks,
                                                       Dsv4AlignOut o) {
  align_body<IdT, NT>(ids, topk_w, R, K, E, block_m, max_blocks, o);
}

// The layer's first launch: workgroup 0 aligns the routing while workgroups
// 1.. quantise the activations x (they are independent), which saves a
// dependent launch on the decode critical path. QF selects the quantiser:
// 0 = FP8 per 128 (bf16 profile, codes + E8M0 x4), 1 = MXFP4 per 32.
template <typename IdT, int NT, int QF>
__global__ __launch_bounds__(NT) void moe_align_quant_kernel(const IdT* __restrict__ ids,
                                                             const float* __restrict__ topk_w, int R, int K,
                                                             int E, int block_m, int max_blocks,
                                                             Dsv4AlignOut o, const uint4* __restrict__ x,
                                                             int64_t n_groups, int rule, void* q_codes,
                                                             void* q_scale, int n_shared) {
  if (blockIdx.x == 0) {
    align_body<IdT, NT>(ids, topk_w, R, K, E, block_m, max_blocks, o, n_shared);
    return;
  }
  const int64_t g = (int64_t)(blockIdx.x - 1) * NT + threadIdx.x;
  if (QF == 0)
    dsv4::fp8_quant_group(x, g, g < n_groups, nullptr, (uint2*)q_codes, nullptr, (uint32_t*)q_scale);
  else
    dsv4::mxfp4_quant_group(x, g, g < n_groups, rule, (uint32_t*)q_codes, (uint8_t*)q_scale, nullptr);
}

// Decode-sized router + align in the layer's first launch (the router's top-k
// and moe_align fused, so the routed ids never wait for another launch):
// workgroup 0's waves each select the top-k of one token at a time
// (route_topk_token, the router's own per-token code, writing ra.out_ids and
// ra.out_w), and after a barrier - which also makes those global writes
// visible to the whole workgroup - the same workgroup aligns them. Workgroups
// 1.. quantise x as in moe_align_quant_kernel.
template <int EPL, int NT, int QF>
__global__ __launch_bounds__(NT) void route_align_quant_kernel(RouteTopkArgs ra, int block_m, int max_blocks,
                                                               Dsv4AlignOut o, const uint4* __restrict__ x,
                                                               int64_t n_groups, int rule, void* q_codes,
                                                               void* q_scale, int n_shared) {
  if (blockIdx.x == 0) {
    for (int t = threadIdx.x >> 6; t < ra.T; t += NT / 64) dsv4::route_topk_token<EPL>(ra, t, threadIdx.x & 63);
    __syncthreads();
    align_body<int32_t, NT>(ra.out_ids, ra.out_w, ra.T * ra.K, ra.K, ra.E, block_m, max_blocks, o, n_shared);
    return;
  }
  const int64_t g = (int64_t)(blockIdx.x - 1) * NT + threadIdx.x;
  if (QF == 0)
    dsv4::fp8_quant_group(x, g, g < n_groups, nullptr, (uint2*)q_codes, nullptr, (uint32_t*)q_scale);
  else
    dsv4::mxfp4_quant_group(x, g, g < n_groups, rule, (uint32_t*)q_codes, (uint8_t*)q_scale, nullptr);
}

}  // namespace

hipError_t launch_moe_align(const void* topk_ids, int ids_int64, const float* topk_w, int R, int K, int E,
                            int block_m, int max_blocks, const Dsv4AlignOut& o, hipStream_t st) {
  // small problems (decode) run on 4 waves: fewer waves to synchronise; larger
  // ones (prefill, or E > 256) on 16 waves: fewer sequential 1024-entry chunks
  const bool small = E <= 256 && R <= 2048;
  const int nwaves = small ? 4 : 16;
  const size_t lds = sizeof(int) * (size_t)((E + 1) + E + E + (E + 1) + nwaves * (E + 1));
  if (small) {
    if (ids_int64)
      hipLaunchKernelGGL((moe_align_kernel<long long, 256>), dim3(1), dim3(256), lds, st,
                         (const long long*)topk_ids, topk_w, R, K, E, block_m, max_blocks, o);
    else
      hipLaunchKernelGGL((moe_align_kernel<int32_t, 256>), dim3(1), dim3(256), lds, st,
                         (const int32_t*)topk_ids, topk_w, R, K, E, block_m, max_blocks, o);
  } else {
    if (ids_int64)
      hipLaunchKernelGGL((moe_align_kernel<long long, 1024>), dim3(1), dim3(1024), lds, st,
                         (const long long*)topk_ids, topk_w, R, K, E, block_m, max_blocks, o);
    else
      hipLaunchKernelGGL((moe_align_kernel<int32_t, 1024>), dim3(1), dim3(1024), lds, st,
                         (const int32_t*)topk_ids, topk_w, R, K, E, block_m, max_blocks, o);
  }
  return hipGetLastError();
}

hipError_t launch_moe_align_quant(const void* topk_ids, int ids_int64, const float* topk_w, int R, int K, int E,
                                  int block_m, int max_blocks, const Dsv4AlignOut& o, const uint16_t* x,
                                  int64_t n_elems, int qfmt, int rule, void* q_codes, void* q_scale,
                                  hipStream_t st, int n_shared) {
  const bool small = E <= 256 && R <= 2048;
  const int nt = small ? 256 : 1024;
  const size_t lds = sizeof(int) * (size_t)((E + 1) + E + E + (E + 1) + (nt / 64) * (E + 1));
  const int64_t n_groups = n_elems / 8;
  const int64_t qwg = (n_groups + nt - 1) / nt;
  if (qwg + 1 > 0x7fffffffLL) return hipErrorInvalidValue;
  const dim3 grid((unsigned)(1 + qwg));
#define DSV4_AQ(IDT, NT_, QF)                                                                              \
  hipLaunchKernelGGL((moe_align_quant_kernel<IDT, NT_, QF>), grid, dim3(NT_), lds, st, (const IDT*)topk_ids, \
                     topk_w, R, K, E, block_m, max_blocks, o, (const uint4*)x, n_groups, rule, q_codes, q_scale, \
                     n_shared)
  if (small) {
    if (ids_int64) { if (qfmt == 0) DSV4_AQ(long long, 256, 0); else DSV4_AQ(long long, 256, 1); }
    else { if (qfmt == 0) DSV4_AQ(int32_t, 256, 0); else DSV4_AQ(int32_t, 256, 1); }
  } else {
    if (ids_int64) { if (qfmt == 0) DSV4_AQ(long long, 1024, 0); else DSV4_AQ(long long, 1024, 1); }
    else { if (qfmt == 0) DSV4_AQ(int32_t, 1024, 0); else DSV4_AQ(int32_t, 1024, 1); }
  }
#undef DSV4_AQ
  return hipGetLastError();
}

int64_t align_chunked_scratch_bytes(int R, int E) {
  const int64_t C = (R + kAlignChunk - 1) / kAlignChunk;
  return C * (E + 1) * (int64_t)sizeof(int);
}

hipError_t launch_moe_align_chunked(const void* topk_ids, int ids_int64, const float* topk_w, int R, int K, int E,
                                    int block_m, int max_blocks, const Dsv4AlignOut& o, const uint16_t* x,
                                    int64_t n_elems, int qfmt, int rule, void* q_codes, void* q_scale,
                                    hipStream_t st, int n_shared, void* scratch, const Dsv4AlignHot* hot) {
  const Dsv4AlignHot hv = hot ? *hot : Dsv4AlignHot{};
  const int C = (R + kAlignChunk - 1) / kAlignChunk;
  int* cc = (int*)scratch;
  const int64_t n_groups = x ? n_elems / 8 : 0;
  constexpr int NT1 = 256;
  const int64_t qwg = (n_groups + NT1 - 1) / NT1;
  if (C + qwg > 0x7fffffffLL) return hipErrorInvalidValue;
  const dim3 g1((unsigned)(C + qwg));
  const size_t lds1 = sizeof(int) * (size_t)(E + 1);
#define DSV4_CQ(IDT, QF)                                                                                    \
  hipLaunchKernelGGL((align_count_quant_kernel<IDT, NT1, QF>), g1, dim3(NT1), lds1, st, (const IDT*)topk_ids, \
                     R, E, C, cc, (const uint4*)x, n_groups, rule, q_codes, q_scale)
  const int qf = x ? qfmt : 2;  // 2: count only
  if (ids_int64) {
    if (qf == 0) DSV4_CQ(long long, 0); else if (qf == 1) DSV4_CQ(long long, 1); else DSV4_CQ(long long, 2);
  } else {
    if (qf == 0) DSV4_CQ(int32_t, 0); else if (qf == 1) DSV4_CQ(int32_t, 1); else DSV4_CQ(int32_t, 2);
  }
#undef DSV4_CQ
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  // the layout needs one thread per expert: 256 threads up to 256 experts, 1024 above
#define DSV4_SC(IDT, NT)                                                                                       \
  hipLaunchKernelGGL((align_scatter_kernel<IDT, NT>), dim3(C), dim3(NT),                                      \
                     sizeof(int) * (size_t)(E + E + (E + 1) + (NT / 64) * (E + 1)), st, (const IDT*)topk_ids, \
                     topk_w, R, K, E, C, block_m, max_blocks, n_shared, cc, o, hv)
  if (E <= 256) {
    if (ids_int64) DSV4_SC(long long, 256); else DSV4_SC(int32_t, 256);
  } else {
    if (ids_int64) DSV4_SC(long long, 1024); else DSV4_SC(int32_t, 1024);
  }
#undef DSV4_SC
  return hipGetLastError();
}

// 8 waves: one token per wave at decode batch sizes, and E <= 512 experts for
// the align's one-thread-per-expert layout step.
hipError_t launch_route_align_quant(const RouteTopkArgs& ra, int block_m, int max_blocks, const Dsv4AlignOut& o,
                                    const uint16_t* x, int64_t n_elems, int qfmt, int rule, void* q_codes,
                                    void* q_scale, hipStream_t st, int n_shared) {
  constexpr int NT = 512;
  if (ra.E > NT || ra.E <= 0 || (int64_t)ra.T * ra.K > 0x7fffffffLL) return hipErrorInvalidValue;
  const int E = ra.E;
  const size_t lds = sizeof(int) * (size_t)((E + 1) + E + E + (E + 1) + (NT / 64) * (E + 1));
  const int64_t n_groups = n_elems / 8;
  const int64_t qwg = (n_groups + NT - 1) / NT;
  if (qwg + 1 > 0x7fffffffLL) return hipErrorInvalidValue;
  const dim3 grid((unsigned)(1 + qwg));
#define DSV4_RAQ(EPL, QF)                                                                                  \
  hipLaunchKernelGGL((route_align_quant_kernel<EPL, NT, QF>), grid, dim3(NT), lds, st, ra, block_m, max_blocks, \
                     o, (const uint4*)x, n_groups, rule, q_codes, q_scale, n_shared)
#define DSV4_RAQ_E(QF)       \
  if (E <= 64)               \
    DSV4_RAQ(1, QF);         \
  else if (E <= 128)         \
    DSV4_RAQ(2, QF);         \
  else if (E <= 256)         \
    DSV4_RAQ(4, QF);         \
  else                       \
    DSV4_RAQ(8, QF)
  if (qfmt == 0) {
    DSV4_RAQ_E(0);
  } else {
    DSV4_RAQ_E(1);
  }
#undef DSV4_RAQ_E
#undef DSV4_RAQ
  return hipGetLastError();
}
