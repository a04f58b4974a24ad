// Per-token top-k of the router (OffloadDeepseekV4MoE._route, deepseek_v4.py:126-148),
// shared by the router's own launch and the decode launch that also builds the
// expert layout (moe_align) from the ids it selects.
#pragma once
#include "common.h"
#include "kernels.h"

namespace dsv4 {

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

// One wave computes token t: sums the S partials of each expert in chunk order
// (deterministic), applies the score function, selects K experts by repeated
// wave-wide argmax (ties to the lower id) or reads them from tid2eid, gathers
// the unbiased scores, renormalises and scales. EPL experts per lane: expert e
// lives in lane e % 64, slot e / 64.
template <int EPL>
DSV4_DEV void route_topk_token(const RouteTopkArgs& a, int t, int lane) {
  const float* __restrict__ part = a.part;
  const int S = a.S, T = a.T, E = a.E, K = a.K, scoring = a.scoring;
  const float* __restrict__ bias = a.bias;
  const void* tid2eid = a.tid2eid;
  const int tid_is64 = a.tid_is64, ids_is64 = a.ids_is64, renorm = a.renorm;
  const void* input_ids = a.input_ids;
  const int64_t vocab = a.vocab;
  const float scale = a.scale;
  float* __restrict__ out_w = a.out_w;
  int32_t* __restrict__ out_ids = a.out_ids;
  int32_t* status = a.status;
  const float ninf = -__builtin_inff();
  // the bias and the token's input id are loaded with the partials (one memory
  // latency, not two or three)
  int64_t tok = tid2eid ? load_index(input_ids, ids_is64, t) : -1;
  // Loads read clamped indices (expert E - 1, chunk S - 1) and the values are dropped
  // afterwards, so no load sits behind a branch: each would be its own round trip.
  float bv[EPL];
#pragma unroll
  for (int j = 0; j < EPL; ++j) {
    const int e = lane + 64 * j;
    bv[j] = bias ? bias[min(e, E - 1)] : 0.f;
    if (e >= E) bv[j] = 0.f;
  }
  float sc[EPL];
  // the S partials of each expert, summed in chunk order; up to 16 chunks' loads in flight
#pragma unroll
  for (int j = 0; j < EPL; ++j) sc[j] = 0.f;
  for (int z0 = 0; z0 < S; z0 += 16) {
    float v[16][EPL];
#pragma unroll
    for (int i = 0; i < 16; ++i)
#pragma unroll
      for (int j = 0; j < EPL; ++j)
        v[i][j] = part[((int64_t)min(z0 + i, S - 1) * T + t) * E + min(lane + 64 * j, E - 1)];
#pragma unroll
    for (int i = 0; i < 16; ++i)
#pragma unroll
      for (int j = 0; j < EPL; ++j)
        if (z0 + i < S) sc[j] += v[i][j];
  }
#pragma unroll
  for (int j = 0; j < EPL; ++j)
    if (lane + 64 * j >= E) sc[j] = 0.f;
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

  if (tid2eid && (tok < 0 || tok >= vocab)) {
    if (status && lane == 0) atomicAdd(status, 1);
    tok = -1;
  }
  float choice[EPL];
#pragma unroll
  for (int j = 0; j < EPL; ++j) {
    const int e = lane + 64 * j;
    float c = sc[j] + bv[j];
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

}  // namespace dsv4
