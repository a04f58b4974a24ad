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

namespace dsv4 {
namespace {

typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));

constexpr int kRouteWaves = 4;  // waves per workgroup in both kernels

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
template <bool XF32, int MT, int NT, bool BF3 = false>
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
  // 8 x values of token row m at k offset kb: two uint4 of fp32, or one uint4 of bf16
  auto load_x = [&](int m, int kb, uint4& a, uint4& b) {
    if (!live[m]) {
      a = b = make_uint4(0u, 0u, 0u, 0u);
    } else if (XF32) {
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
  // one step of loads in flight while the previous step's MFMAs run
  uint4 xa[MT], xb[MT];
  float4 wa[NT], wb[NT];
#pragma unroll
  for (int m = 0; m < MT; ++m) load_x(m, 0, xa[m], xb[m]);
#pragma unroll
  for (int n = 0; n < NT; ++n) wa[n] = *(const float4*)wr[n], wb[n] = *(const float4*)(wr[n] + 4);
  for (int kb = 0; kb < kchunk; kb += 32) {
    float xf[MT][8], wf[NT][8];
    uint4 xa_cur[MT];
#pragma unroll
    for (int m = 0; m < MT; ++m) {
      const uint4 u = xa[m], v = xb[m];
      xa_cur[m] = u;
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
    if (kb + 32 < kchunk) {
#pragma unroll
      for (int m = 0; m < MT; ++m) load_x(m, kb + 32, xa[m], xb[m]);
#pragma unroll
      for (int n = 0; n < NT; ++n)
        wa[n] = *(const float4*)(wr[n] + kb + 32), wb[n] = *(const float4*)(wr[n] + kb + 36);
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
          const bf16x8 a = __builtin_bit_cast(bf16x8, xa_cur[m]);
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

DSV4_DEV float wave_sum(float v) {
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}

DSV4_DEV bool better(float ov, int oid, float v, int id) { return ov > v || (ov == v && oid < id); }

// One DPP step of the (value, id) reduction: the partner lane given by CTRL.
template <int CTRL>
DSV4_DEV void argmax_dpp(float& v, int& id) {
  const float ov = __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xf, 0xf, false));
  const int oid = __builtin_amdgcn_update_dpp(0, id, CTRL, 0xf, 0xf, false);
  if (better(ov, oid, v, id)) {
    v = ov;
    id = oid;
  }
}

// (value, id) maximum over the wave, uniform result; equal values go to the
// lower id. Within each 16-lane row: quad swaps (xor 1, xor 2), then the half-row
// and row mirrors (each lane meets the other quad, then the other half); the
// four rows' results are then read as scalars.
DSV4_DEV void wave_argmax(float& v, int& id) {
  argmax_dpp<0xb1>(v, id);   // quad_perm [1, 0, 3, 2]
  argmax_dpp<0x4e>(v, id);   // quad_perm [2, 3, 0, 1]
  argmax_dpp<0x141>(v, id);  // row_half_mirror
  argmax_dpp<0x140>(v, id);  // row_mirror
  float bv = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 0));
  int bid = __builtin_amdgcn_readlane(id, 0);
#pragma unroll
  for (int r = 1; r < 4; ++r) {
    const float rv = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 16 * r));
    const int rid = __builtin_amdgcn_readlane(id, 16 * r);
    if (better(rv, rid, bv, bid)) {
      bv = rv;
      bid = rid;
    }
  }
  v = bv;
  id = bid;
}

DSV4_DEV int64_t load_index(const void* p, int is64, int64_t i) {
  return is64 ? ((const int64_t*)p)[i] : (int64_t)((const int32_t*)p)[i];
}

// EPL experts per lane: expert e lives in lane e % 64, slot e / 64.
template <int EPL>
__global__ __launch_bounds__(64 * kRouteWaves) void route_topk_kernel(const float* __restrict__ part, int S, int T,
                                                                       int E, int K, int scoring,
                                                                       const float* __restrict__ bias,
                                                                       const void* tid2eid, int tid_is64,
                                                                       const void* input_ids, int ids_is64,
                                                                       int64_t vocab, int renorm, float scale,
                                                                       float* __restrict__ out_w,
                                                                       int32_t* __restrict__ out_ids,
                                                                       int32_t* status) {
  const int lane = threadIdx.x & 63;
  const int t = blockIdx.x * kRouteWaves + (threadIdx.x >> 6);
  if (t >= T) return;
  const float ninf = -__builtin_inff();
  float sc[EPL];
  // the S partials of each expert, summed in chunk order; up to 16 chunks' loads in flight
#pragma unroll
  for (int j = 0; j < EPL; ++j) sc[j] = 0.f;
  for (int z0 = 0; z0 < S; z0 += 16) {
    float v[16][EPL];
#pragma unroll
    for (int i = 0; i < 16; ++i)
#pragma unroll
      for (int j = 0; j < EPL; ++j) {
        const int e = lane + 64 * j;
        v[i][j] = (z0 + i < S && e < E) ? part[((int64_t)(z0 + i) * T + t) * E + e] : 0.f;
      }
#pragma unroll
    for (int i = 0; i < 16; ++i)
#pragma unroll
      for (int j = 0; j < EPL; ++j)
        if (z0 + i < S) sc[j] += v[i][j];
  }
  if (scoring == 0) {  // softmax over the E experts
    float m = ninf;
#pragma unroll
    for (int j = 0; j < EPL; ++j)
      if (lane + 64 * j < E) m = fmaxf(m, sc[j]);
    m = wave_max_xor(m, 64);
    float s = 0.f;
#pragma unroll
    for (int j = 0; j < EPL; ++j) {
      sc[j] = (lane + 64 * j < E) ? expf(sc[j] - m) : 0.f;
      s += sc[j];
    }
    s = wave_sum(s);
#pragma unroll
    for (int j = 0; j < EPL; ++j) sc[j] = sc[j] / s;
  } else if (scoring == 1) {  // sigmoid
#pragma unroll
    for (int j = 0; j < EPL; ++j) sc[j] = 1.f / (1.f + expf(-sc[j]));
  } else {  // sqrt(softplus), softplus threshold 20 as in F.softplus
#pragma unroll
    for (int j = 0; j < EPL; ++j) sc[j] = sqrtf(sc[j] > 20.f ? sc[j] : log1pf(expf(sc[j])));
  }

  int64_t tok = -1;
  if (tid2eid) {
    tok = load_index(input_ids, ids_is64, t);
    if (tok < 0 || tok >= vocab) {
      if (status && lane == 0) atomicAdd(status, 1);
      tok = -1;
    }
  }
  float choice[EPL];
#pragma unroll
  for (int j = 0; j < EPL; ++j) {
    const int e = lane + 64 * j;
    float c = sc[j] + (bias && e < E ? bias[e] : 0.f);
    if (c != c) c = __builtin_inff();  // topk ranks NaN above every number
    choice[j] = (e < E) ? c : ninf;
  }
  uint32_t taken = 0;
  float my_w = 0.f, sum = 0.f;
  int my_id = 0;
  for (int k = 0; k < K; ++k) {
    int id;
    if (tid2eid) {
      const int64_t v = (tok < 0) ? -1 : load_index(tid2eid, tid_is64, tok * K + k);
      id = (v >= 0 && v < E) ? (int)v : -1;
      if (id < 0 && tok >= 0 && status && lane == 0) atomicAdd(status, 1);
    } else {
      float v = ninf;
      id = 0x7fffffff;
#pragma unroll
      for (int j = 0; j < EPL; ++j) {
        const int e = lane + 64 * j;
        if (e < E && !(taken >> j & 1u) && (choice[j] > v || (choice[j] == v && e < id))) {
          v = choice[j];
          id = e;
        }
      }
      wave_argmax(v, id);
      if ((id & 63) == lane) taken |= 1u << (id >> 6);
    }
    float wk = 0.f;
    if (id >= 0 && id < E) {
      float mine = sc[0];
#pragma unroll
      for (int j = 1; j < EPL; ++j)
        if ((id >> 6) == j) mine = sc[j];
      wk = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(mine), id & 63));  // id is wave-uniform
    }
    sum += wk;
    if (lane == k) {
      my_w = wk;
      my_id = id;
    }
  }
  if (lane < K) {
    float wv = my_w;
    const bool bad_token = tid2eid && tok < 0;  // keeps its zero weights
    if (renorm && !bad_token) wv = wv / sum;
    out_w[(int64_t)t * K + lane] = wv * scale;
    out_ids[(int64_t)t * K + lane] = my_id;
  }
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

// K split so that about 2048 waves (two per SIMD) run, with chunks of at least
// 256 k that stay multiples of 32.
int route_split_k(int T, int D, int E) {
  const RouteTile rt = route_tile(T);
  const int tt = 16 * rt.mt, te = 16 * rt.nt;
  const int tiles = ((E + te - 1) / te) * ((T + tt - 1) / tt);
  int S = 1;
  while (S < 16 && tiles * S < 2048 && D % (64 * S) == 0 && D / (2 * S) >= 256) S *= 2;
  return S;
}

hipError_t launch_moe_route(const void* x, int x_f32, const float* gate_w, int T, int D, int E, int K, int scoring,
                            const float* bias, const void* tid2eid, int tid_is64, const void* input_ids,
                            int ids_is64, int64_t vocab, int renorm, float scale, float* out_w,
                            int32_t* out_ids, int32_t* status, float* part, hipStream_t st) {
  const int S = route_split_k(T, D, E);
  const RouteTile rt = route_tile(T);
  const int tt = 16 * rt.mt, te = 16 * rt.nt;
  dim3 g1((E + te * kRouteWaves - 1) / (te * kRouteWaves), (T + tt - 1) / tt, S);
  dim3 b1(64 * kRouteWaves);
  if (rt.mt == 4) {
    if (x_f32)
      hipLaunchKernelGGL((route_logits_kernel<true, 4, 2>), g1, b1, 0, st, x, gate_w, T, D, E, D / S, part);
    else
      hipLaunchKernelGGL((route_logits_kernel<false, 4, 2, true>), g1, b1, 0, st, x, gate_w, T, D, E, D / S,
                         part);
  } else {
    if (x_f32)
      hipLaunchKernelGGL((route_logits_kernel<true, 1, 1>), g1, b1, 0, st, x, gate_w, T, D, E, D / S, part);
    else
      hipLaunchKernelGGL((route_logits_kernel<false, 1, 1>), g1, b1, 0, st, x, gate_w, T, D, E, D / S, part);
  }
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  dim3 g2((T + kRouteWaves - 1) / kRouteWaves);
#define DSV4_TOPK(EPL)                                                                                      \
  hipLaunchKernelGGL(route_topk_kernel<EPL>, g2, dim3(64 * kRouteWaves), 0, st, part, S, T, E, K, scoring, \
                     bias, tid2eid, tid_is64, input_ids, ids_is64, vocab, renorm, scale, out_w, out_ids,  \
                     status)
  if (E <= 64)
    DSV4_TOPK(1);
  else if (E <= 128)
    DSV4_TOPK(2);
  else if (E <= 256)
    DSV4_TOPK(4);
  else
    DSV4_TOPK(8);
#undef DSV4_TOPK
  return hipGetLastError();
}
