// Router of one MoE layer (OffloadDeepseekV4MoE._route, deepseek_v4.py:118-148):
//   logits = float(x) @ gate_wᵀ                      (fp32, [T, E])
//   scores = softmax | sigmoid | sqrt(softplus)(logits)
//   ids    = top-K of scores + bias, or tid2eid[input_ids] on hash layers
//   w      = scores[ids], / sum(w) when renormalising, * routed_scaling_factor
//
// Two launches:
//   route_logits_kernel - fp32 MFMA (v_mfma_f32_16x16x4_f32), or for bf16 x
//     from 256 tokens on bf16 MFMA on an exact three-way bf16 split of the
//     weight, one wave per
//     16x16 (small T) or 64x32 (T >= 256) tokens x experts x one K chunk. K is
//     split into S chunks so that enough waves run (decode-sized T has few
//     tiles to stream the 4 MiB gate matrix with); each chunk's partial logits
//     go to the workspace [S, T, E].
//   route_topk_kernel   - one wave per token: sums the S partials in chunk
//     order (deterministic), applies the score function, selects K experts by
//     repeated wave-wide argmax (ties to the lower id), gathers, renormalises.
#include "common.h"
#include "kernels.h"
#include "route_dev.h"

namespace dsv4 {
namespace {

typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));

constexpr int kRouteWaves = 4;  // waves per workgroup in both kernels

// The MFMAs of one step (32 k) on its x (xa, xb: 8 values of token row m per lane, fp32
// in both, or bf16 in xa) and weights (wa, wb: 8 fp32 values of expert row n per lane).
template <bool XF32, int MT, int NT, bool BF3>
DSV4_DEV void route_step(f32x4 (&acc)[MT][NT], const uint4 (&xa)[MT], const uint4 (&xb)[MT], const float4 (&wa)[NT],
                         const float4 (&wb)[NT]) {
  float xf[MT][8], wf[NT][8];
#pragma unroll
  for (int m = 0; m < MT; ++m) {
    const uint4 u = xa[m], v = xb[m];
    if (XF32) {
      xf[m][0] = __uint_as_float(u.x), xf[m][1] = __uint_as_float(u.y);
      xf[m][2] = __uint_as_float(u.z), xf[m][3] = __uint_as_float(u.w);
      xf[m][4] = __uint_as_float(v.x), xf[m][5] = __uint_as_float(v.y);
      xf[m][6] = __uint_as_float(v.z), xf[m][7] = __uint_as_float(v.w);
    } else {
      xf[m][0] = bf16_to_f32(u.x & 0xffffu), xf[m][1] = bf16_to_f32(u.x >> 16);
      xf[m][2] = bf16_to_f32(u.y & 0xffffu), xf[m][3] = bf16_to_f32(u.y >> 16);
      xf[m][4] = bf16_to_f32(u.z & 0xffffu), xf[m][5] = bf16_to_f32(u.z >> 16);
      xf[m][6] = bf16_to_f32(u.w & 0xffffu), xf[m][7] = bf16_to_f32(u.w >> 16);
    }
  }
#pragma unroll
  for (int n = 0; n < NT; ++n) {
    wf[n][0] = wa[n].x, wf[n][1] = wa[n].y, wf[n][2] = wa[n].z, wf[n][3] = wa[n].w;
    wf[n][4] = wb[n].x, wf[n][5] = wb[n].y, wf[n][6] = wb[n].z, wf[n][7] = wb[n].w;
  }
  if constexpr (BF3) {
#pragma unroll
    for (int n = 0; n < NT; ++n) {
      uint32_t hi[4], mid[4], lo[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        uint32_t h2[2], m2[2], l2[2];
#pragma unroll
        for (int h = 0; h < 2; ++h) {
          const float w = wf[n][2 * i + h];
          const uint32_t wh = __float_as_uint(w) & 0xffff0000u;
          const float r1 = w - __uint_as_float(wh);
          const uint32_t wm = __float_as_uint(r1) & 0xffff0000u;
          const float r2 = r1 - __uint_as_float(wm);
          h2[h] = wh >> 16;
          m2[h] = wm >> 16;
          l2[h] = __float_as_uint(r2) >> 16;
        }
        hi[i] = h2[0] | (h2[1] << 16);
        mid[i] = m2[0] | (m2[1] << 16);
        lo[i] = l2[0] | (l2[1] << 16);
      }
      const bf16x8 bh = __builtin_bit_cast(bf16x8, make_uint4(hi[0], hi[1], hi[2], hi[3]));
      const bf16x8 bm = __builtin_bit_cast(bf16x8, make_uint4(mid[0], mid[1], mid[2], mid[3]));
      const bf16x8 bl = __builtin_bit_cast(bf16x8, make_uint4(lo[0], lo[1], lo[2], lo[3]));
#pragma unroll
      for (int m = 0; m < MT; ++m) {
        const bf16x8 a = __builtin_bit_cast(bf16x8, xa[m]);
        acc[m][n] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, bl, acc[m][n], 0, 0, 0);
        acc[m][n] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, bm, acc[m][n], 0, 0, 0);
        acc[m][n] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, bh, acc[m][n], 0, 0, 0);
      }
    }
  } else {
#pragma unroll
    for (int i = 0; i < 8; ++i)
#pragma unroll
      for (int m = 0; m < MT; ++m)
#pragma unroll
        for (int n = 0; n < NT; ++n)
          acc[m][n] = __builtin_amdgcn_mfma_f32_16x16x4f32(xf[m][i], wf[n][i], acc[m][n], 0, 0, 0);
  }
}

// A wave computes (16*MT) tokens x (16*NT) experts of one K chunk as MT x NT
// tiles of v_mfma_f32_16x16x4_f32. Lane (r = l%16, g = l/16) loads, per step of
// 32 k, x[t][kb+8g, +8) for its MT token rows and W[e][kb+8g, +8) for its NT
// expert rows. The A operand in lane l is A[l%16][l/16] and the B operand
// B[l/16][l%16], so MFMA i, fed element i, reduces over the four k's
// {kb + 8g + i : g = 0..3}; the 8 MFMAs of a step cover [kb, kb+32).
// XF32: x is fp32 (the reference takes hs.float(), so fp32 hidden states are
// used as they are); otherwise bf16.
//
// BF3 (bf16 x only): each fp32 weight w is split exactly into three bf16
// planes, hi = w with its low 16 bits cleared, mid = the same of w - hi, lo =
// w - hi - mid (at most 8 significant bits left, so exact in bf16), and the
// step's 32 k run as three v_mfma_f32_16x16x32_bf16 (A = the bf16 x values, B
// = hi, mid, lo): every product is exact in fp32 and the accumulation is fp32,
// at about five times the fp32 MFMA's rate. Lane (r, g) feeds the same 8 k's
// to A and B, so the hardware's pairing of A and B elements is all that matters.
//
// NSTEP > 0: the chunk is exactly NSTEP steps. PF = 0: every one of its loads is issued
// before the first MFMA (decode-sized T: a few hundred waves each stream 16 expert
// rows, and a step-by-step prefetch would pay one memory latency per step). PF > 0:
// the loads run PF steps ahead of the MFMAs in a ring of PF + 1 steps (the large tile,
// whose whole chunk would not fit in registers; with one step ahead, each step waited
// for its loads).
template <bool XF32, int MT, int NT, bool BF3 = false, int NSTEP = 0, int PF = 0>
__global__ __launch_bounds__(64 * kRouteWaves) void route_logits_kernel(const void* __restrict__ xp,
                                                                         const float* __restrict__ w, int T,
                                                                         int D, int E, int kchunk,
                                                                         float* __restrict__ part) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int e0 = (blockIdx.x * kRouteWaves + wave) * 16 * NT;
  if (e0 >= E) return;
  const int t0 = blockIdx.y * 16 * MT, z = blockIdx.z;
  const int r = lane & 15, g = lane >> 4;
  const int64_t k0 = (int64_t)z * kchunk + 8 * g;
  bool live[MT];
  int64_t xoff[MT];
  const float* wr[NT];
#pragma unroll
  for (int m = 0; m < MT; ++m) {
    live[m] = t0 + 16 * m + r < T;
    xoff[m] = (int64_t)(live[m] ? t0 + 16 * m + r : 0) * D + k0;
  }
#pragma unroll
  for (int n = 0; n < NT; ++n) wr[n] = w + (int64_t)min(e0 + 16 * n + r, E - 1) * D + k0;
  // 8 x values of token row m at k offset kb: two uint4 of fp32, or one uint4 of bf16.
  // Rows past T read row 0 (no branch around the load): a token row of the product
  // depends on its own x row only, and those rows are never stored.
  auto load_x = [&](int m, int kb, uint4& a, uint4& b) {
    if (XF32) {
      const uint4* p = (const uint4*)((const float*)xp + xoff[m] + kb);
      a = p[0];
      b = p[1];
    } else {
      a = *(const uint4*)((const uint16_t*)xp + xoff[m] + kb);
      b = make_uint4(0u, 0u, 0u, 0u);
    }
  };
  f32x4 acc[MT][NT];
#pragma unroll
  for (int m = 0; m < MT; ++m)
#pragma unroll
    for (int n = 0; n < NT; ++n) acc[m][n] = f32x4{0.f, 0.f, 0.f, 0.f};
  auto step = [&](const uint4 (&xa)[MT], const uint4 (&xb)[MT], const float4 (&wa)[NT], const float4 (&wb)[NT]) {
    route_step<XF32, MT, NT, BF3>(acc, xa, xb, wa, wb);
  };
  if constexpr (NSTEP > 0 && PF > 0) {
    constexpr int RING = PF + 1;
    uint4 xa[RING][MT], xb[RING][MT];
    float4 wa[RING][NT], wb[RING][NT];
    auto issue = [&](int q) __attribute__((always_inline)) {
      const int r = q % RING;
#pragma unroll
      for (int m = 0; m < MT; ++m) load_x(m, 32 * q, xa[r][m], xb[r][m]);
#pragma unroll
      for (int n = 0; n < NT; ++n)
        wa[r][n] = *(const float4*)(wr[n] + 32 * q), wb[r][n] = *(const float4*)(wr[n] + 32 * q + 4);
    };
#pragma unroll
    for (int q = 0; q < PF && q < NSTEP; ++q) issue(q);
#pragma unroll
    for (int q = 0; q < NSTEP; ++q) {
      if (q + PF < NSTEP) issue(q + PF);  // resolved at compile time (q is unrolled)
      __builtin_amdgcn_sched_barrier(0);
      step(xa[q % RING], xb[q % RING], wa[q % RING], wb[q % RING]);
      __builtin_amdgcn_sched_barrier(0);
    }
  } else if constexpr (NSTEP > 0) {
    // the whole chunk's loads, then its MFMAs
    uint4 xa[NSTEP][MT], xb[NSTEP][MT];
    float4 wa[NSTEP][NT], wb[NSTEP][NT];
#pragma unroll
    for (int q = 0; q < NSTEP; ++q) {
#pragma unroll
      for (int m = 0; m < MT; ++m) load_x(m, 32 * q, xa[q][m], xb[q][m]);
#pragma unroll
      for (int n = 0; n < NT; ++n)
        wa[q][n] = *(const float4*)(wr[n] + 32 * q), wb[q][n] = *(const float4*)(wr[n] + 32 * q + 4);
    }
    __builtin_amdgcn_sched_barrier(0);  // (else the scheduler sinks each load to its use)
#pragma unroll
    for (int q = 0; q < NSTEP; ++q) step(xa[q], xb[q], wa[q], wb[q]);
  } else {
    // one step of loads in flight while the previous step's MFMAs run
    uint4 xa[MT], xb[MT];
    float4 wa[NT], wb[NT];
#pragma unroll
    for (int m = 0; m < MT; ++m) load_x(m, 0, xa[m], xb[m]);
#pragma unroll
    for (int n = 0; n < NT; ++n) wa[n] = *(const float4*)wr[n], wb[n] = *(const float4*)(wr[n] + 4);
    for (int kb = 0; kb < kchunk; kb += 32) {
      uint4 ca[MT], cb[MT];
      float4 cwa[NT], cwb[NT];
#pragma unroll
      for (int m = 0; m < MT; ++m) ca[m] = xa[m], cb[m] = xb[m];
#pragma unroll
      for (int n = 0; n < NT; ++n) cwa[n] = wa[n], cwb[n] = wb[n];
      if (kb + 32 < kchunk) {
#pragma unroll
        for (int m = 0; m < MT; ++m) load_x(m, kb + 32, xa[m], xb[m]);
#pragma unroll
        for (int n = 0; n < NT; ++n)
          wa[n] = *(const float4*)(wr[n] + kb + 32), wb[n] = *(const float4*)(wr[n] + kb + 36);
      }
      step(ca, cb, cwa, cwb);
    }
  }
  // C lane l holds C[4(l/16) + i][l%16]: token t0 + 16m + 4g + i, expert e0 + 16n + r.
  float* out = part + (int64_t)z * T * E;
#pragma unroll
  for (int n = 0; n < NT; ++n) {
    const int e = e0 + 16 * n + r;
    if (e >= E) continue;
#pragma unroll
    for (int m = 0; m < MT; ++m)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int t = t0 + 16 * m + 4 * g + i;
        if (t < T) out[(int64_t)t * E + e] = acc[m][n][i];
      }
  }
}

// Large token counts, E a multiple of 256: one workgroup of eight waves covers 64 tokens x
// all 256 experts of its group x one K chunk of NSTEP steps (a wave: 64 tokens x 32
// experts, as the tile above). The chunk's x rows are loaded once into LDS and read by
// the eight waves (with the tile above each x row was fetched by the eight waves of its
// expert tiles, half of the traffic the logits took from L2); the gate rows stream per
// wave, PF steps ahead. Rows past T read row 0 and are not stored.
constexpr int kRouteLdsWaves = 8;
template <bool XF32, bool BF3, int NSTEP, int PF>
__global__ __launch_bounds__(64 * kRouteLdsWaves) void route_logits_lds_kernel(const void* __restrict__ xp,
                                                                               const float* __restrict__ w, int T,
                                                                               int D, int E, float* __restrict__ part) {
  constexpr int MT = 4, NT = 2, KC = 32 * NSTEP;  // KC: k per chunk
  constexpr int ES = XF32 ? 4 : 2;                // x bytes per element
  constexpr int PITCH = KC * ES + 16;             // LDS row pitch: 16 rows of a read on distinct banks
  constexpr int CPR = KC * ES / 16;               // 16-byte pieces per x row
  __shared__ __attribute__((aligned(16))) uint8_t xs[64 * PITCH];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int e0 = blockIdx.x * 256 + wave * 32;
  const int t0 = blockIdx.y * 64, z = blockIdx.z;
  const int r = lane & 15, g = lane >> 4;
  const int64_t k0 = (int64_t)z * KC;
  const bool active = e0 < E;  // waves past E still load their share of x
  const float* wr[NT];
#pragma unroll
  for (int n = 0; n < NT; ++n) wr[n] = w + (int64_t)min(e0 + 16 * n + r, E - 1) * D + k0 + 8 * g;
  constexpr int RING = PF + 1;
  float4 wa[RING][NT], wb[RING][NT];
  auto issue_w = [&](int q) __attribute__((always_inline)) {
#pragma unroll
    for (int n = 0; n < NT; ++n)
      wa[q % RING][n] = *(const float4*)(wr[n] + 32 * q), wb[q % RING][n] = *(const float4*)(wr[n] + 32 * q + 4);
  };
  if (active) {
#pragma unroll
    for (int q = 0; q < PF && q < NSTEP; ++q) issue_w(q);
  }
  // the chunk's x rows into LDS: piece c = i * 512 + tid of row c / CPR
  constexpr int NPC = 64 * CPR / (64 * kRouteLdsWaves);
  static_assert(NPC * 64 * kRouteLdsWaves == 64 * CPR, "x pieces per thread");
  uint4 xl[NPC];
#pragma unroll
  for (int i = 0; i < NPC; ++i) {
    const int c = i * 64 * kRouteLdsWaves + tid, row = c / CPR, pc = c % CPR;
    const int t = t0 + row < T ? t0 + row : 0;
    xl[i] = *(const uint4*)((const uint8_t*)xp + ((int64_t)t * D + k0) * ES + 16 * pc);
  }
#pragma unroll
  for (int i = 0; i < NPC; ++i) {
    const int c = i * 64 * kRouteLdsWaves + tid, row = c / CPR, pc = c % CPR;
    *(uint4*)(xs + row * PITCH + 16 * pc) = xl[i];
  }
  __syncthreads();
  if (!active) return;
  f32x4 acc[MT][NT];
#pragma unroll
  for (int m = 0; m < MT; ++m)
#pragma unroll
    for (int n = 0; n < NT; ++n) acc[m][n] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int q = 0; q < NSTEP; ++q) {
    if (q + PF < NSTEP) issue_w(q + PF);  // resolved at compile time (q is unrolled)
    uint4 xa[MT], xb[MT];
#pragma unroll
    for (int m = 0; m < MT; ++m) {  // lane (r, g): x[16 m + r][32 q + 8 g, +8)
      const uint8_t* p = xs + (16 * m + r) * PITCH + (32 * q + 8 * g) * ES;
      xa[m] = *(const uint4*)p;
      xb[m] = XF32 ? *(const uint4*)(p + 16) : make_uint4(0u, 0u, 0u, 0u);
    }
    __builtin_amdgcn_sched_barrier(0);
    route_step<XF32, MT, NT, BF3>(acc, xa, xb, wa[q % RING], wb[q % RING]);
    __builtin_amdgcn_sched_barrier(0);
  }
  float* out = part + (int64_t)z * T * E;
#pragma unroll
  for (int n = 0; n < NT; ++n) {
    const int e = e0 + 16 * n + r;
    if (e >= E) continue;
#pragma unroll
    for (int m = 0; m < MT; ++m)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int t = t0 + 16 * m + 4 * g + i;
        if (t < T) out[(int64_t)t * E + e] = acc[m][n][i];
      }
  }
}

template <int EPL>
__global__ __launch_bounds__(64 * kRouteWaves) void route_topk_kernel(RouteTopkArgs a) {
  const int t = blockIdx.x * kRouteWaves + (threadIdx.x >> 6);
  if (t >= a.T) return;
  route_topk_token<EPL>(a, t, threadIdx.x & 63);
}

}  // namespace
}  // namespace dsv4

using namespace dsv4;

// Per-wave tile: 16 tokens x 16 experts for decode-sized T (more waves,
// shorter K loops); from 256 tokens on 64 x 32 (each weight fragment serves
// four token tiles, which halves the L2 bytes the gate weight costs).
struct RouteTile {
  int mt, nt;
};
static RouteTile route_tile(int T) { return T >= 256 ? RouteTile{4, 2} : RouteTile{1, 1}; }

// The decode-sized tile streams chunks of exactly this many k, every load issued up
// front (route_logits_kernel's NSTEP = kRouteSmallChunk / 32); the large tile, where
// the split gives chunks of this many k, runs them with its loads three steps ahead.
constexpr int kRouteSmallChunk = 256;
constexpr int kRouteLargeChunk = 512;
static bool route_small_chunks(int T, int D) { return route_tile(T).mt == 1 && D % kRouteSmallChunk == 0; }

// K split so that about 2048 waves (two per SIMD) run, with chunks of at least
// 256 k that stay multiples of 32; decode-sized T: chunks of exactly 256 k.
int route_split_k(int T, int D, int E) {
  if (route_small_chunks(T, D)) return D / kRouteSmallChunk;
  const RouteTile rt = route_tile(T);
  const int tt = 16 * rt.mt, te = 16 * rt.nt;
  const int tiles = ((E + te - 1) / te) * ((T + tt - 1) / tt);
  int S = 1;
  while (S < 16 && tiles * S < 2048 && D % (64 * S) == 0 && D / (2 * S) >= 256) S *= 2;
  return S;
}

hipError_t launch_route_logits(const void* x, int x_f32, const float* gate_w, int T, int D, int E, float* part,
                               int* S_out, hipStream_t st) {
  const int S = route_split_k(T, D, E);
  *S_out = S;
  const RouteTile rt = route_tile(T);
  const int tt = 16 * rt.mt, te = 16 * rt.nt;
  dim3 g1((E + te * kRouteWaves - 1) / (te * kRouteWaves), (T + tt - 1) / tt, S);
  dim3 b1(64 * kRouteWaves);
  if (rt.mt == 4) {
    constexpr int NS = kRouteLargeChunk / 32;
    if (D / S == kRouteLargeChunk && E % 256 == 0) {  // x through LDS, eight waves over 256 experts
      const dim3 g8(E / 256, (T + 63) / 64, S), b8(64 * kRouteLdsWaves);
      if (x_f32)
        hipLaunchKernelGGL((route_logits_lds_kernel<true, false, NS, 3>), g8, b8, 0, st, x, gate_w, T, D, E, part);
      else
        hipLaunchKernelGGL((route_logits_lds_kernel<false, true, NS, 3>), g8, b8, 0, st, x, gate_w, T, D, E, part);
    } else if (D / S == kRouteLargeChunk) {
      if (x_f32)
        hipLaunchKernelGGL((route_logits_kernel<true, 4, 2, false, NS, 3>), g1, b1, 0, st, x, gate_w, T, D, E, D / S,
                           part);
      else
        hipLaunchKernelGGL((route_logits_kernel<false, 4, 2, true, NS, 3>), g1, b1, 0, st, x, gate_w, T, D, E, D / S,
                           part);
    } else if (x_f32) {
      hipLaunchKernelGGL((route_logits_kernel<true, 4, 2>), g1, b1, 0, st, x, gate_w, T, D, E, D / S, part);
    } else {
      hipLaunchKernelGGL((route_logits_kernel<false, 4, 2, true>), g1, b1, 0, st, x, gate_w, T, D, E, D / S,
                         part);
    }
  } else if (route_small_chunks(T, D)) {
    constexpr int NS = kRouteSmallChunk / 32;
    if (x_f32)
      hipLaunchKernelGGL((route_logits_kernel<true, 1, 1, false, NS>), g1, b1, 0, st, x, gate_w, T, D, E, D / S,
                         part);
    else
      hipLaunchKernelGGL((route_logits_kernel<false, 1, 1, false, NS>), g1, b1, 0, st, x, gate_w, T, D, E, D / S,
                         part);
  } else {
    if (x_f32)
      hipLaunchKernelGGL((route_logits_kernel<true, 1, 1>), g1, b1, 0, st, x, gate_w, T, D, E, D / S, part);
    else
      hipLaunchKernelGGL((route_logits_kernel<false, 1, 1>), g1, b1, 0, st, x, gate_w, T, D, E, D / S, part);
  }
  return hipGetLastError();
}

hipError_t launch_route_topk(const RouteTopkArgs& ra, hipStream_t st) {
  const dim3 g2((ra.T + kRouteWaves - 1) / kRouteWaves), b2(64 * kRouteWaves);
  if (ra.E <= 64)
    hipLaunchKernelGGL(route_topk_kernel<1>, g2, b2, 0, st, ra);
  else if (ra.E <= 128)
    hipLaunchKernelGGL(route_topk_kernel<2>, g2, b2, 0, st, ra);
  else if (ra.E <= 256)
    hipLaunchKernelGGL(route_topk_kernel<4>, g2, b2, 0, st, ra);
  else
    hipLaunchKernelGGL(route_topk_kernel<8>, g2, b2, 0, st, ra);
  return hipGetLastError();
}

hipError_t launch_moe_route(const void* x, int x_f32, const float* gate_w, int T, int D, int E, int K, int scoring,
                            const float* bias, const void* tid2eid, int tid_is64, const void* input_ids,
                            int ids_is64, int64_t vocab, int renorm, float scale, float* out_w,
                            int32_t* out_ids, int32_t* status, float* part, hipStream_t st) {
  int S = 1;
  const hipError_t e = launch_route_logits(x, x_f32, gate_w, T, D, E, part, &S, st);
  if (e != hipSuccess) return e;
  const RouteTopkArgs ra{part, S, T, E, K, scoring, bias, tid2eid, tid_is64, input_ids, ids_is64,
                         vocab, renorm, scale, out_w, out_ids, status};
  return launch_route_topk(ra, st);
}
