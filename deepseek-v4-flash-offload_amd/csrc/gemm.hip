// Grouped expert GEMMs on gfx950 block-scaled MFMA (v_mfma_scale_f32_16x16x128_f8f6f4).
//
// Replaces the three npu_grouped_matmul calls of deepseek_v4.py:177-193 (bf16
// profile) and :218-232,241 (a4w4 profile). Weights stay in their checkpoint
// MXFP4 form ([N, K/2] E2M1 + [N, K/32] E8M0, read in place from the expert's
// slot through a device pointer table, no restacking) and feed the MFMA B
// operand directly; the hardware applies both E8M0 scales per 32-element block.
//
//  * bf16 profile: the reference quantises x (and h) with the per-128 FP8 round
//    trip (act_quant) and multiplies the bf16 result by the bf16-dequantised
//    weight. Both operands are exactly representable as (E4M3 code x 2^k) and
//    (E2M1 code x 2^s), so the FP8 x FP4 scaled MFMA computes the same products
//    exactly, accumulating in fp32 (summation order differs, hence the 1e-2
//    tolerance rather than bit equality on GEMM outputs).
//  * a4w4 profile: FP4 x FP4 with per-32 E8M0 scales on both operands.
//
// Work decomposition: one single-wave workgroup = one M block (16 padded rows of
// one expert, from moe_align) x NT = 4 output tiles of 16 columns (gate/up: 2
// gate + 2 up tiles of the same 32 intermediate columns). Small workgroups keep
// the per-CU load even (a decode step has ~40 active experts x 64 column
// chunks = ~2560 workgroups for 256 CUs). The A rows are gathered on load
// through sorted_ids (no permuted copy of x is materialised). The wave streams
// its weight rows straight from HBM into registers: every weight byte is used
// by exactly one wave, so staging it through LDS would only add traffic. The K
// loop runs in 256-wide stages with a two-stage register ring and no branches,
// so the loads of stage j+1 are in flight while stage j is multiplied.
//
// K mapping. One 256-wide stage is 2 MFMAs (ji = 0, 1) of 128 logical k. Logical
// 32-block b of MFMA ji is global 32-block 8*j + 2*b + ji, so the lane holding
// block b of a weight row (lane group g = b) reads 32 contiguous bytes per stage
// and the four lane groups of a row read its 128 contiguous bytes.
// Operand layouts (measured on gfx950):
//   E2M1 A/B: lane (r = l%16, g = l/16) holds logical k [32g, 32g+32) of row r
//             in 16 bytes, low nibble first.
//   E4M3 A  : lane (r, g) holds logical k [16g, 16g+16) in bytes 0-15 and
//             [64+16g, 64+16g+16) in bytes 16-31.
//   scales  : lane (r, g) supplies the E8M0 of logical block g of its row/col.
//   C       : lane l holds C[4*(l/16)+i][l%16], i = 0..3.
#include <type_traits>

#include "common.h"
#include "kernels.h"
#include "quant_dev.h"

namespace {

typedef int v8i __attribute__((ext_vector_type(8)));
typedef int v4i __attribute__((ext_vector_type(4)));
typedef float v4f __attribute__((ext_vector_type(4)));

#ifndef DSV4_GEMM_PREFETCH
#define DSV4_GEMM_PREFETCH 1
#endif
// The 16-row kernel loads MFMA-tiled routed weights non-temporally: each weight
// byte is read by one or a few row blocks, close together, and with one
// contiguous 1 KB per wave load this measured 8% faster for the decode shape
// than plain loads (on the checkpoint layout, 64 B from each of 16 rows per
// load, non-temporal loads measured 9% slower, so that layout keeps plain
// ones). The 64-row kernel keeps plain loads: its row blocks of one expert
// re-read the weights from L2 (there non-temporal loads measured 2-4% slower).
#ifndef DSV4_GEMM_NT_LOADS
#define DSV4_GEMM_NT_LOADS 1
#endif

constexpr int kBM = 16;
constexpr bool kNtLoads = DSV4_GEMM_NT_LOADS != 0;
constexpr int kNT = 4;        // 16-column output tiles per wave
#ifndef DSV4_GEMM_WAVES
#define DSV4_GEMM_WAVES 1
#endif
constexpr int kWaves = DSV4_GEMM_WAVES;  // waves per workgroup (they share nothing but the M block)
constexpr int kStageK = 256;  // reduction elements per pipeline stage

template <int AFMT>
struct AStage;
template <>
struct AStage<0> {  // E4M3: 32 bytes per lane per MFMA
  v8i d[2];
  uint32_t s;
};
template <>
struct AStage<1> {  // E2M1: 16 bytes per lane per MFMA
  v4i d[2];
  uint32_t s;
};
// bf16 activations (kAfmtBf16): for scaled-MFMA position ji, the lane's 32 bf16 of the
// 32-k block its weight chunk covers, as 4 x 16 bytes (one bf16 MFMA each)
template <>
struct AStage<kAfmtBf16> {
  v4i d[2][4];
  uint32_t s;
};
// B operand of one stage: E2M1 weights (16 bytes per lane per MFMA, kNT tiles)
// or, for the shared expert, E4M3 weights (32 bytes, laid out like the E4M3 A
// operand). An E4M3 stage holds kNT/2 tiles, so both take the same registers;
// the E4M3 path covers its kNT tiles in two passes over K.
template <bool B8>
struct BStageT {
  static constexpr int NTB = B8 ? kNT / 2 : kNT;
  typename std::conditional<B8, v8i, v4i>::type d[NTB][2];
  uint32_t s[NTB];
};
using BStage = BStageT<false>;

// Every operand lives in global memory; the casts keep the loads global_load_*
// (pointers read from the expert table would otherwise become flat accesses).
typedef __attribute__((address_space(1))) const v4i gv4i;
typedef __attribute__((address_space(1))) const uint16_t gu16;
DSV4_DEV v4i ld16(const uint8_t* p) { return *(gv4i*)p; }
// Weight bytes: non-temporal when the kernel reads each of them about once.
template <bool NT>
DSV4_DEV v4i ld16_w(const uint8_t* p) {
  if constexpr (NT) return __builtin_nontemporal_load((gv4i*)p);
  else return *(gv4i*)p;
}
DSV4_DEV uint32_t ld_u16(const uint8_t* p) { return *(gu16*)p; }

// ---------------------------------------------------------------------------
// Scale bytes, loaded once per row instead of once per stage. Per stage a lane
// needs 2 scale bytes of each of its rows (bytes 8j + 2g, +1: one per MFMA of
// the stage); fetching them stage by stage issues one L1->L2 request per row
// per stage for 2 bytes, and those requests, not the bytes, were measured to
// bound the weight stream (the per-CU pool of outstanding L1 misses fills with
// them). Instead the four lane groups of a row load the row's K/32 scale bytes
// once, each group a contiguous S = K/128 byte slice, and every stage fetches
// its two bytes from the holding lane with a cross-lane permute.
// ---------------------------------------------------------------------------
template <int NST>
struct RowScales {
  static constexpr int S = 2 * NST;  // bytes per lane group
  uint32_t w[S / 4 > 0 ? S / 4 : 1];
};

template <int NST>
DSV4_DEV void load_row_scales(RowScales<NST>& rs, const uint8_t* row, int g) {
  constexpr int S = RowScales<NST>::S;
  const uint8_t* p = row + g * S;
  if constexpr (S >= 16) {
#pragma unroll
    for (int i = 0; i < S / 16; ++i) {
      const v4i v = ld16(p + 16 * i);
      rs.w[4 * i] = (uint32_t)v.x;
      rs.w[4 * i + 1] = (uint32_t)v.y;
      rs.w[4 * i + 2] = (uint32_t)v.z;
      rs.w[4 * i + 3] = (uint32_t)v.w;
    }
  } else if constexpr (S == 8) {
    typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
    typedef __attribute__((address_space(1))) const u32x2 gu32x2;
    const u32x2 v = *(gu32x2*)p;
    rs.w[0] = v.x;
    rs.w[1] = v.y;
  } else {
    typedef __attribute__((address_space(1))) const uint32_t gu32;
    rs.w[0] = *(gu32*)p;
  }
}

// The 2 scale bytes (low byte: MFMA ji = 0) lane (r16, g) uses in stage j.
template <int NST>
DSV4_DEV uint32_t stage_scales(const RowScales<NST>& rs, int j, int r16, int g) {
  constexpr int S = RowScales<NST>::S;
  if constexpr (S >= 8) {
    // bytes [8j, 8j+8) sit in one lane group: dwords d0, d0 + 1
    const int holder = (8 * j) / S, d0 = ((8 * j) % S) / 4;
    const int src = r16 + 16 * holder;
    const uint32_t v0 = (uint32_t)__shfl((int)rs.w[d0], src, 64);
    const uint32_t v1 = (uint32_t)__shfl((int)rs.w[d0 + 1], src, 64);
    return (((g & 2) ? v1 : v0) >> (16 * (g & 1))) & 0xffffu;
  } else {  // S == 4 (K = 512): a stage spans two lane groups
    const int src = r16 + 16 * (2 * j + (g >> 1));
    const uint32_t v = (uint32_t)__shfl((int)rs.w[0], src, 64);
    return (v >> (16 * (g & 1))) & 0xffffu;
  }
}

template <int AFMT, bool SCALES = true>
DSV4_DEV void load_a(AStage<AFMT>& a, const uint8_t* abase, const uint8_t* asbase, int j, int g) {
  if constexpr (AFMT == kAfmtBf16) {  // k block 8j + 2g + ji: elements 256j + 64g + 32ji .. +32
    const uint8_t* p = abase + (int64_t)j * 512 + 128 * g;
#pragma unroll
    for (int ji = 0; ji < 2; ++ji)
#pragma unroll
      for (int m = 0; m < 4; ++m) a.d[ji][m] = ld16(p + 64 * ji + 16 * m);
    return;
  } else if constexpr (AFMT == 1) {
    const uint8_t* p = abase + (int64_t)j * 128 + g * 32;
    a.d[0] = ld16(p);
    a.d[1] = ld16(p + 16);
  } else {
    const uint8_t* p = abase + (int64_t)j * 256 + 16 * (g & 1) + 64 * (g >> 1);
#pragma unroll
    for (int ji = 0; ji < 2; ++ji) {
      const v4i lo = ld16(p + 32 * ji);        // logical block g>>1
      const v4i hi = ld16(p + 32 * ji + 128);  // logical block 2 + (g>>1)
      a.d[ji] = v8i{lo.x, lo.y, lo.z, lo.w, hi.x, hi.y, hi.z, hi.w};
    }
  }
  if constexpr (SCALES) a.s = ld_u16(asbase + j * 8 + 2 * g);
}

// E2M1 weight layouts: the lane's chunk for MFMA ji of stage j is at
// bt + j * stage_stride + ji * mfma_stride, bt being the lane's chunk of stage 0.
struct BLayout {
  int64_t stage_stride;  // checkpoint [N, K/2]: 128; MFMA-tiled: 2048
  int mfma_stride;       // checkpoint: 16; MFMA-tiled: 1024
};
// An expert table entry marks a packed weight field in the MFMA-tiled layout
// (mxfp4_tile_kernel) by bit 0 of its pointer (the fields are 16-byte aligned).
DSV4_DEV bool tiled_ptr(const uint8_t* p) { return ((uintptr_t)p & 1u) != 0; }
DSV4_DEV const uint8_t* untag(const uint8_t* p) { return (const uint8_t*)((uintptr_t)p & ~(uintptr_t)1); }
// The lane's stage-0 chunk of weight row `row` (16-row tile row / 16) and the strides.
// KNOWN_TILED: the caller has already found the tag set.
template <bool KNOWN_TILED = false>
DSV4_DEV const uint8_t* b_lane_base(const uint8_t* w, int64_t row, int64_t row_bytes, int nst, int lane,
                                    BLayout& lay) {
  if (KNOWN_TILED || tiled_ptr(w)) {
    lay = BLayout{2048, 1024};
    return untag(w) + (row >> 4) * (int64_t)nst * 2048 + 16 * lane;
  }
  lay = BLayout{128, 16};
  return w + row * row_bytes + 32 * (lane >> 4);
}

template <bool SCALES = true, bool B8 = false, bool NT = false>
DSV4_DEV void load_b(BStageT<B8>& b, const uint8_t* const* bt, const uint8_t* const* bst, int j, int g,
                     const BLayout& lay = BLayout{128, 16}) {
#pragma unroll
  for (int t = 0; t < BStageT<B8>::NTB; ++t) {
    if constexpr (B8) {  // E4M3 rows: the E4M3 A layout (two 16-byte halves per MFMA)
      const uint8_t* p = bt[t] + (int64_t)j * 256 + 16 * (g & 1) + 64 * (g >> 1);
#pragma unroll
      for (int ji = 0; ji < 2; ++ji) {
        const v4i lo = ld16_w<NT>(p + 32 * ji);
        const v4i hi = ld16_w<NT>(p + 32 * ji + 128);
        b.d[t][ji] = v8i{lo.x, lo.y, lo.z, lo.w, hi.x, hi.y, hi.z, hi.w};
      }
    } else {
      const uint8_t* p = bt[t] + j * lay.stage_stride;
      b.d[t][0] = ld16_w<NT>(p);
      b.d[t][1] = ld16_w<NT>(p + lay.mfma_stride);
    }
    if constexpr (SCALES) b.s[t] = ld_u16(bst[t] + j * 8 + 2 * g);
  }
}

template <bool B8>
DSV4_DEV v8i b_operand(const BStageT<B8>& b, int t, int ji) {
  if constexpr (B8) {
    return b.d[t][ji];
  } else {
    return v8i{b.d[t][ji].x, b.d[t][ji].y, b.d[t][ji].z, b.d[t][ji].w, 0, 0, 0, 0};
  }
}

template <int AFMT, bool B8 = false>
DSV4_DEV void compute(v4f* acc, const AStage<AFMT>& a, const BStageT<B8>& b) {
#pragma unroll
  for (int ji = 0; ji < 2; ++ji) {
    v8i av;
    if constexpr (AFMT == 1) {
      av = v8i{a.d[ji].x, a.d[ji].y, a.d[ji].z, a.d[ji].w, 0, 0, 0, 0};
    } else {
      av = a.d[ji];
    }
    const int sa = (int)((a.s >> (8 * ji)) & 0xffu);
#pragma unroll
    for (int t = 0; t < BStageT<B8>::NTB; ++t) {
      const v8i bv = b_operand<B8>(b, t, ji);
      const int sb = (int)((b.s[t] >> (8 * ji)) & 0xffu);
      acc[t] = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(av, bv, acc[t], AFMT == 0 ? 0 : 4, B8 ? 0 : 4, 0,
                                                                sa, 0, sb);
    }
  }
}

// bf16 activations: the lane's E2M1 chunk of weight row r16 for MFMA position ji holds
// the 32 k its A data holds (low nibble first), so each 4-byte word m of the chunk, with
// the row's E8M0 applied by the scaled convert (exact: at most two significant bits),
// is the B operand of the bf16 MFMA whose A operand is A word m: both sides feed the
// same 8 k's in the same lane positions, which is all the k pairing of the MFMA needs.
// (The convert decodes nibble 8 to -0, harmless in a product; a scale byte of 255 gives
// non-finite weights, as the reference's dequant does.)
template <bool B8>
DSV4_DEV void compute_bf16(v4f* acc, const AStage<kAfmtBf16>& a, const BStageT<B8>& b) {
  static_assert(!B8, "bf16 activations meet E2M1 weights only");
  typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
  typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
#pragma unroll
  for (int ji = 0; ji < 2; ++ji)
#pragma unroll
    for (int t = 0; t < kNT; ++t) {
      const float sc = dsv4::e8m0_to_f32((b.s[t] >> (8 * ji)) & 0xffu);
#pragma unroll
      for (int m = 0; m < 4; ++m) {
        const uint32_t w = (uint32_t)b.d[t][ji][m];
        const bf16x2 p0 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(w, sc, 0);
        const bf16x2 p1 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(w, sc, 1);
        const bf16x2 p2 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(w, sc, 2);
        const bf16x2 p3 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(w, sc, 3);
        const bf16x8 bw = bf16x8{p0[0], p0[1], p1[0], p1[1], p2[0], p2[1], p3[0], p3[1]};
        acc[t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a.d[ji][m]), bw, acc[t], 0, 0,
                                                         0);
      }
    }
}

// A row of flat index f: a routed entry reads row f / a_row_div, one of the
// trailing shared_a_rows shared-expert entries row f - (R - shared_a_rows), and
// padding (f >= R) row 0 (its products land only in rows that are never stored).
template <bool SH>
DSV4_DEV int64_t a_row(const Dsv4GemmArgs& p, int f) {
  if constexpr (!SH) return f < p.R ? (int64_t)(f / p.a_row_div) : 0;
  const int r0 = p.R - p.shared_a_rows;
  return f < r0 ? (int64_t)(f / p.a_row_div) : (f < p.R ? (int64_t)(f - r0) : 0);
}

// Epilogue of one 16-row subtile: lane holds rows row0 + 4*g + i (i = 0..3) of
// column r16 of each of the 4 tiles. Gate/up: hb receives the bf16 h values the
// SwiGLU produced (tiles t = 0, 1 are intermediate columns col0 + 16 t + r16) and
// fr the rows' flat indices; h is written unless the caller fuses its quantisation.
template <bool GATEUP, bool SH = false>
DSV4_DEV void store_tile(const Dsv4GemmArgs& p, const v4f* acc, int row0, int col0, int g, int r16,
                         uint32_t (*hb)[2] = nullptr, int* fr = nullptr) {
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int f = p.sorted_ids[row0 + 4 * g + i];
    if (fr) fr[i] = f;
    if (f >= p.R) continue;
    uint16_t* orow = p.out + (int64_t)f * p.N + col0 + r16;
    if (GATEUP) {
      // deepseek_v4.py:177-187: bf16 GEMM outputs -> fp32, clamp, silu(gate) * up * w
      // (shared-expert rows: w = 1, model_npu.py:478-489 applies no weight)
      const float w = (!SH || f < p.R - p.shared_a_rows) ? p.topk_w[f] : 1.0f;
#pragma unroll
      for (int t = 0; t < 2; ++t) {
        float gt = dsv4::bf16_to_f32(dsv4::f32_to_bf16(acc[t][i]));
        float up = dsv4::bf16_to_f32(dsv4::f32_to_bf16(acc[t + 2][i]));
        if (p.swiglu_limit > 0.0f) {
          up = fminf(fmaxf(up, -p.swiglu_limit), p.swiglu_limit);
          gt = fminf(gt, p.swiglu_limit);
        }
        const float h = gt / (1.0f + expf(-gt)) * up * w;
        const uint32_t b = dsv4::f32_to_bf16(h);
        if (hb) hb[i][t] = b;
        if (!p.hq_skip_h) orow[16 * t] = (uint16_t)b;
      }
    } else {
#pragma unroll
      for (int t = 0; t < kNT; ++t) orow[16 * t] = (uint16_t)dsv4::f32_to_bf16(acc[t][i]);
    }
  }
}

// MXFP4 quantisation of the h subtile a gate/up wave holds: its 32 intermediate
// columns are exactly one 32-element block of each row, spread over the 16
// lanes of lane group g (2 values each). Same arithmetic as mxfp4_quant_group.
DSV4_DEV void quantise_h_mxfp4(const Dsv4GemmArgs& p, const uint32_t (*hb)[2], const int* fr, int col0, int g,
                               int r16) {
  (void)g;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const float v0 = dsv4::bf16_to_f32(hb[i][0]), v1 = dsv4::bf16_to_f32(hb[i][1]);
    const float amax = dsv4::wave_max_xor(fmaxf(fabsf(v0), fabsf(v1)), 16);
    const int k = dsv4::mxfp4_block_exp(amax, p.hq_rule);
    const float inv = dsv4::pow2f(-k);
    const uint32_t n0 = dsv4::mxfp4_nibble(v0, inv, p.hq_rule), n1 = dsv4::mxfp4_nibble(v1, inv, p.hq_rule);
    const uint32_t o0 = (uint32_t)__shfl_xor((int)n0, 1, 64), o1 = (uint32_t)__shfl_xor((int)n1, 1, 64);
    const int f = fr[i];
    if (f < p.R) {
      uint8_t* row = p.hq_codes + (int64_t)f * (p.N / 2) + col0 / 2;
      if ((r16 & 1) == 0) {  // low nibble = even column
        row[r16 / 2] = (uint8_t)(n0 | (o0 << 4));
        row[8 + r16 / 2] = (uint8_t)(n1 | (o1 << 4));
      }
      if (r16 == 0) p.hq_scale[(int64_t)f * (p.N / 32) + col0 / 32] = (uint8_t)(k + 127);
    }
  }
}

// NTW: the block's routed weights are MFMA-tiled and loaded non-temporally.
template <int AFMT, bool GATEUP, int NST, bool SH, bool NTW>
__attribute__((always_inline)) DSV4_DEV void moe_gemm_block(const Dsv4GemmArgs& p, const int mb, const int e) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  // the shared expert's blocks carry id shared_expert and read its E4M3 weights
  const bool shared = SH && e == p.shared_expert;
  const Dsv4ExpertPtrs ex = shared ? p.shared : p.experts[e];
  // an expert whose weights are not in the table contributes zeros (never read null)
  const bool have_w = GATEUP ? (ex.w1p && ex.w1s && ex.w3p && ex.w3s) : (ex.w2p && ex.w2s);
  const int r16 = lane & 15, g = lane >> 4;

  // A operand row of this lane, gathered on load
  const int64_t arow = a_row<SH>(p, p.sorted_ids[mb * kBM + r16]);
  const uint8_t* abase = p.a + arow * p.a_row_bytes;
  const uint8_t* asbase = AFMT == kAfmtBf16 ? nullptr : p.a_scale + arow * (int64_t)(p.Kdim / 32);

  // weight rows of this lane's tiles (E2M1: K/2 bytes per row, E4M3: K)
  const int64_t brow_bytes = shared ? p.Kdim : p.Kdim / 2, bsrow = p.Kdim / 32;
  int col0;
  const uint8_t* bt[kNT];
  const uint8_t* bst[kNT];
  BLayout lay{128, 16};  // routed E2M1 weights: checkpoint or MFMA-tiled layout (table pointer bit 0)
  if (GATEUP) {
    col0 = blockIdx.x * (kWaves * 32) + wave * 32;  // 32 intermediate columns: 2 gate + 2 up tiles
#pragma unroll
    for (int t = 0; t < 2; ++t) {
      const int64_t row = col0 + 16 * t + r16;
      if (shared) {  // E4M3 rows, checkpoint layout (the E4M3 loads add their own offsets)
        bt[t] = ex.w1p + row * brow_bytes;
        bt[t + 2] = ex.w3p + row * brow_bytes;
      } else {  // w1 and w3 of an expert share one layout
        bt[t] = b_lane_base<NTW>(ex.w1p, row, brow_bytes, NST, lane, lay);
        bt[t + 2] = b_lane_base<NTW>(ex.w3p, row, brow_bytes, NST, lane, lay);
      }
      bst[t] = ex.w1s + row * bsrow;
      bst[t + 2] = ex.w3s + row * bsrow;
    }
  } else {
    col0 = blockIdx.x * (kWaves * 64) + wave * 64;
#pragma unroll
    for (int t = 0; t < kNT; ++t) {
      const int64_t row = col0 + 16 * t + r16;
      bt[t] = shared ? ex.w2p + row * brow_bytes : b_lane_base<NTW>(ex.w2p, row, brow_bytes, NST, lane, lay);
      bst[t] = ex.w2s + row * bsrow;
    }
  }

  v4f acc[kNT];
#pragma unroll
  for (int t = 0; t < kNT; ++t) acc[t] = v4f{0.f, 0.f, 0.f, 0.f};

  // NST = Kdim / 256 stages, fully unrolled into straight-line code. With
  // DSV4_GEMM_PREFETCH = P > 0 the loads of stage j+P are issued before the
  // MFMAs of stage j and a scheduling barrier keeps them there (a P+1 deep
  // register ring); with P = 0 the compiler schedules freely.
  // T0: first tile of this pass (E4M3 weights: two passes of kNT/2 tiles).
  // NT: non-temporal weight loads (MFMA-tiled routed weights only: on the
  // checkpoint layout they measured 9% slower than plain loads).
  auto kloop = [&](auto b8, auto t0c, auto ntc) {
    constexpr bool B8 = decltype(b8)::value;
    constexpr int t0 = decltype(t0c)::value;
    constexpr bool NT = decltype(ntc)::value;
    constexpr int NTB = BStageT<B8>::NTB;
    constexpr int P = DSV4_GEMM_PREFETCH;
    constexpr int RING = P + 1;
    const uint8_t* const* btp = bt + t0;
    const uint8_t* const* bstp = bst + t0;
    AStage<AFMT> a[RING];
    BStageT<B8> b[RING];
    RowScales<NST> as_row, bs_row[NTB];
    if constexpr (AFMT != kAfmtBf16) load_row_scales<NST>(as_row, asbase, g);
#pragma unroll
    for (int t = 0; t < NTB; ++t) load_row_scales<NST>(bs_row[t], bstp[t], g);
#pragma unroll
    for (int j = 0; j < P && j < NST; ++j) {
      load_a<AFMT, false>(a[j % RING], abase, asbase, j, g);
      load_b<false, B8, NT>(b[j % RING], btp, bstp, j, g, lay);
    }
#pragma unroll
    for (int j = 0; j < NST; ++j) {
      if (j + P < NST) {
        load_a<AFMT, false>(a[(j + P) % RING], abase, asbase, j + P, g);
        load_b<false, B8, NT>(b[(j + P) % RING], btp, bstp, j + P, g, lay);
      }
      if constexpr (P > 0) __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int t = 0; t < NTB; ++t) b[j % RING].s[t] = stage_scales<NST>(bs_row[t], j, r16, g);
      if constexpr (AFMT == kAfmtBf16) {
        compute_bf16<B8>(acc + t0, a[j % RING], b[j % RING]);
      } else {
        a[j % RING].s = stage_scales<NST>(as_row, j, r16, g);
        compute<AFMT, B8>(acc + t0, a[j % RING], b[j % RING]);
      }
      if constexpr (P > 0) __builtin_amdgcn_sched_barrier(0);
    }
  };
  // The strides stay opaque to the optimiser: as constants (2048, 1024: past
  // the loads' immediate-offset range) they led it to keep a 64-bit address
  // per stage live, +20 VGPRs in the down GEMM.
  if constexpr (NTW) asm volatile("" : "+s"(lay.stage_stride), "+s"(lay.mfma_stride));
  auto routed = [&] { kloop(std::false_type{}, std::integral_constant<int, 0>{}, std::integral_constant<bool, NTW>{}); };
  if (have_w) {
    if constexpr (AFMT == 0 && SH) {  // E4M3 weights only meet E4M3 activations (bf16 profile)
      if (shared) {
        kloop(std::true_type{}, std::integral_constant<int, 0>{}, std::false_type{});
        kloop(std::true_type{}, std::integral_constant<int, kNT / 2>{}, std::false_type{});
      } else {
        routed();
      }
    } else {
      routed();
    }
  }

  if (GATEUP && p.hq_mode == 2) {  // MXFP4 h: this wave holds whole 32-column blocks
    uint32_t hb[4][2];
    int fr[4];
    store_tile<GATEUP, SH>(p, acc, mb * kBM, col0, g, r16, hb, fr);
    quantise_h_mxfp4(p, hb, fr, col0, g, r16);
  } else {
    store_tile<GATEUP, SH>(p, acc, mb * kBM, col0, g, r16);
  }
}

// SH: the launch includes the shared expert's E4M3 blocks (a separate
// instantiation, so the routed-only kernels keep their register budget).
// The weight layout is chosen per block, before anything else, so the two
// bodies share no live values (a branch around the inner loop alone raised
// the register count by up to 100 VGPRs).
template <int AFMT, bool GATEUP, int NST, bool SH>
__global__ __launch_bounds__(64 * kWaves) void moe_gemm_kernel(Dsv4GemmArgs p) {
  const int mb = blockIdx.y;
  if (mb * kBM >= p.num_post_padded[0]) return;
  const int e = p.block_expert[mb];
  const bool shared = SH && e == p.shared_expert;
  if (kNtLoads && !shared && tiled_ptr(GATEUP ? p.experts[e].w1p : p.experts[e].w2p))
    moe_gemm_block<AFMT, GATEUP, NST, SH, true>(p, mb, e);
  else
    moe_gemm_block<AFMT, GATEUP, NST, SH, false>(p, mb, e);
}

// ---------------------------------------------------------------------------
// Tiled variant for many rows per expert (prefill): one workgroup = 4 waves =
// BM = 16*MT padded rows of one expert x 4 x 4 output tiles. The gathered A rows
// of each 256-wide K stage are loaded once into a double-buffered LDS tile that
// the four waves share; each wave streams its own four weight tiles from HBM
// (one-stage register prefetch, as above) and reuses every weight fragment
// across the MT row subtiles. One barrier per stage. The grid's x extent (N
// tiles) is a multiple of 8, so all M blocks of one (expert, N tile) land on the
// same XCD and re-read the weight tile from its L2.
// ---------------------------------------------------------------------------
// T0: first of the accumulator tiles this B stage feeds (E4M3 passes: 0, kNT/2)
// live: bit mt set when row subtile mt holds a routed row (wave-uniform)
template <int AFMT, int MT, bool B8 = false, int T0 = 0>
DSV4_DEV void compute_tiled(v4f (*acc)[kNT], const uint8_t* lds, const uint8_t* as_tab, int as_pitch, int j,
                            const BStageT<B8>& b, int r16, int g, uint32_t live) {
  constexpr int t0 = T0;
  constexpr int ASB = AFMT == 0 ? 256 : 128;
  constexpr int AROW = ASB + 16;
#pragma unroll
  for (int ji = 0; ji < 2; ++ji) {
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
      if (!((live >> mt) & 1u)) continue;
      const int row = 16 * mt + r16;
      const uint8_t* ap = lds + row * AROW;
      v8i av;
      if constexpr (AFMT == 1) {
        const v4i lo = *(const v4i*)(ap + (2 * g + ji) * 16);
        av = v8i{lo.x, lo.y, lo.z, lo.w, 0, 0, 0, 0};
      } else {
        const int o = 64 * (g >> 1) + 32 * ji + 16 * (g & 1);
        const v4i lo = *(const v4i*)(ap + o);
        const v4i hi = *(const v4i*)(ap + o + 128);
        av = v8i{lo.x, lo.y, lo.z, lo.w, hi.x, hi.y, hi.z, hi.w};
      }
      const int sa = as_tab[row * as_pitch + 8 * j + 2 * g + ji];
#pragma unroll
      for (int t = 0; t < BStageT<B8>::NTB; ++t) {
        const v8i bv = b_operand<B8>(b, t, ji);
        const int sb = (int)((b.s[t] >> (8 * ji)) & 0xffu);
        acc[mt][t0 + t] = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(av, bv, acc[mt][t0 + t],
                                                                           AFMT == 0 ? 0 : 4, B8 ? 0 : 4, 0, sa, 0,
                                                                           sb);
      }
    }
  }
}

// bf16 activations (pure-bf16 variant), in two phases per 32-k half ji of a
// stage: the weight fragments of the half are dequantised once (exactly, by
// the hardware converter) into bw, then each feeds the MT row subtiles, whose
// A fragments come from the LDS tile (rows of 512 bytes: the stage's 256 k).
// Lane (r16, g) of MFMA (ji, m) takes the 8 k of 32-k block 2g + ji at offset
// 8m, as in the 16-row kernel.
typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));

DSV4_DEV void dequant_half(bf16x8_t (*bw)[4], const BStageT<false>& b, int ji) {
#pragma unroll
  for (int t = 0; t < kNT; ++t) {
    const float sc = dsv4::e8m0_to_f32((b.s[t] >> (8 * ji)) & 0xffu);
#pragma unroll
    for (int m = 0; m < 4; ++m) {
      const uint32_t w = (uint32_t)b.d[t][ji][m];
      const bf16x2_t p0 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(w, sc, 0);
      const bf16x2_t p1 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(w, sc, 1);
      const bf16x2_t p2 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(w, sc, 2);
      const bf16x2_t p3 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(w, sc, 3);
      bw[t][m] = bf16x8_t{p0[0], p0[1], p1[0], p1[1], p2[0], p2[1], p3[0], p3[1]};
    }
  }
}

template <int MT>
DSV4_DEV void mfma_half_bf16(v4f (*acc)[kNT], const uint8_t* lds, const bf16x8_t (*bw)[4], int ji, int r16, int g,
                             uint32_t live) {
  constexpr int AROW = 512 + 16;
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) {
    if (!((live >> mt) & 1u)) continue;
    const uint8_t* ap = lds + (16 * mt + r16) * AROW + 64 * (2 * g + ji);
    v4i a[4];
#pragma unroll
    for (int m = 0; m < 4; ++m) a[m] = *(const v4i*)(ap + 16 * m);
#pragma unroll
    for (int t = 0; t < kNT; ++t)
#pragma unroll
      for (int m = 0; m < 4; ++m)
        acc[mt][t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, a[m]), bw[t][m],
                                                             acc[mt][t], 0, 0, 0);
  }
}

// LDS bytes of one A tile buffer (BM rows of one K stage, rows padded by 16 bytes)
template <int AFMT, int MT>
constexpr int tiled_a_buf_bytes() {
  return 16 * MT * ((AFMT == kAfmtBf16 ? 512 : AFMT == 0 ? 256 : 128) + 16);
}

// Row pitch of the bf16-activation kernel's weight-scale table in LDS (up to 32
// bytes per row): 10 dwords, so the 16 rows one read touches sit on distinct banks.
constexpr int kBfSclPitch = 40;

// One M block of the tiled kernel. NTW: non-temporal weight loads (the block's
// expert has no other M block, so nothing re-reads its weights).
template <int AFMT, bool GATEUP, int NST, int MT, int NW, bool SH, bool NTW>
__attribute__((always_inline)) DSV4_DEV void tiled_block(const Dsv4GemmArgs& p,
                                                         uint8_t (*a_lds)[tiled_a_buf_bytes<AFMT, MT>()],
                                                         uint8_t* as_tab) {
  constexpr int BM = 16 * MT;
  constexpr int NTH = 64 * NW;                // threads per workgroup
  constexpr bool ABF = AFMT == kAfmtBf16;     // bf16 activations: no A scales
  constexpr int ASB = ABF ? 512 : AFMT == 0 ? 256 : 128;  // A bytes per row per stage
  constexpr int AROW = ASB + 16;              // padded LDS row stride
  constexpr int LV = BM * ASB / (NTH * 16);   // 16-byte A chunks one thread moves per stage
  constexpr int KSB = 8 * NST;                // scale bytes per row (K / 32)
  constexpr int ASP = KSB + 16;               // A scale table pitch: 16 rows on distinct banks
  constexpr int AS_CHUNKS = ABF ? 0 : BM * KSB / 16;
  static_assert(LV >= 1 && LV * NTH * 16 == BM * ASB, "loader granularity");
  static_assert(NW % 4 == 0, "four gate/up waves make one 128-column FP8 block");
  static_assert(BM * AROW == tiled_a_buf_bytes<AFMT, MT>(), "A tile buffer size");

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int mb = blockIdx.y;
  if (mb * BM >= p.num_post_padded[0]) return;
  const int e = p.block_expert[mb];
  const bool shared = SH && e == p.shared_expert;
  const Dsv4ExpertPtrs ex = shared ? p.shared : p.experts[e];
  const bool have_w = GATEUP ? (ex.w1p && ex.w1s && ex.w3p && ex.w3s) : (ex.w2p && ex.w2s);
  const int r16 = lane & 15, g = lane >> 4;

  // Row subtiles holding at least one routed row (bit mt of live). An expert's
  // padding fills the end of its last block, so at 2048 tokens a third of the
  // 64-row blocks' 16-row subtiles are padding only: their A chunks and MFMAs
  // are skipped (wave-uniform branches; padding rows are never stored).
  uint32_t live = 0;
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) {
    const bool real = lane < 16 && p.sorted_ids[mb * BM + 16 * mt + lane] < p.R;
    live |= (__ballot(real) != 0 ? 1u : 0u) << mt;
  }

  // loader role: load v of wave w moves 1 KB of the stage's A tile = whole
  // 128-byte lines (4 rows x 256 B for E4M3, 8 rows x 128 B for E2M1), so each
  // line is one L1->L2 request; lane L carries 16-byte chunk (v*NW + w)*64 + L.
  // The 64 chunks of one load lie in one row subtile (64 / CPRW rows, dividing 16).
  constexpr int CPRW = ASB / 16;  // 16-byte chunks per A row per stage
  const uint8_t* lsrc[LV];
  int ldst[LV];
  bool lon[LV];
#pragma unroll
  for (int v = 0; v < LV; ++v) {
    const int id = (v * NW + wave) * 64 + lane, row = id / CPRW, ch = id % CPRW;
    const int64_t ar = a_row<SH>(p, p.sorted_ids[mb * BM + row]);
    lsrc[v] = p.a + ar * p.a_row_bytes + 16 * ch;
    ldst[v] = row * AROW + 16 * ch;
    lon[v] = (live >> (((v * NW + __builtin_amdgcn_readfirstlane(wave)) * 64 / CPRW) / 16)) & 1u;
  }

  const int64_t brow_bytes = shared ? p.Kdim : p.Kdim / 2, bsrow = p.Kdim / 32;
  int col0;
  const uint8_t* bt[kNT];
  const uint8_t* bst[kNT];
  BLayout lay{128, 16};  // routed E2M1 weights: checkpoint or MFMA-tiled layout (table pointer bit 0)
  if (GATEUP) {
    col0 = blockIdx.x * (NW * 32) + wave * 32;
#pragma unroll
    for (int t = 0; t < 2; ++t) {
      const int64_t row = col0 + 16 * t + r16;
      if (shared) {  // E4M3 rows, checkpoint layout (the E4M3 loads add their own offsets)
        bt[t] = ex.w1p + row * brow_bytes;
        bt[t + 2] = ex.w3p + row * brow_bytes;
      } else {  // w1 and w3 of an expert share one layout
        bt[t] = b_lane_base(ex.w1p, row, brow_bytes, NST, lane, lay);
        bt[t + 2] = b_lane_base(ex.w3p, row, brow_bytes, NST, lane, lay);
      }
      bst[t] = ex.w1s + row * bsrow;
      bst[t + 2] = ex.w3s + row * bsrow;
    }
  } else {
    col0 = blockIdx.x * (NW * 64) + wave * 64;
#pragma unroll
    for (int t = 0; t < kNT; ++t) {
      const int64_t row = col0 + 16 * t + r16;
      bt[t] = shared ? ex.w2p + row * brow_bytes : b_lane_base(ex.w2p, row, brow_bytes, NST, lane, lay);
      bst[t] = ex.w2s + row * bsrow;
    }
  }

  v4f acc[MT][kNT];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt)
#pragma unroll
    for (int t = 0; t < kNT; ++t) acc[mt][t] = v4f{0.f, 0.f, 0.f, 0.f};

  // bf16 activations: one weight stage in registers, whose half ji is reloaded
  // with the next stage's as soon as it is dequantised; the A tile moves in two
  // halves (the other LDS buffer is free for the whole stage). Two waves per SIMD.
  // The weight rows' scale bytes move SS stages at a time (8*SS bytes of each of
  // the wave's 64 rows, two 16-byte loads per lane) into a wave-private LDS table
  // that each stage reads its 2 bytes per tile from: fetched stage by stage they
  // cost one L1->L2 request per row per stage, as many requests as the weight
  // loads themselves, and a whole-K table per lane would not fit in registers
  // beside the dequantised fragments.
  auto kloop_bf16 = [&](const uint8_t* const* btp) {
    static_assert(LV % 2 == 0, "the A tile moves in two halves");
    constexpr int LH = LV / 2;
    constexpr int SS = NST < 4 ? NST : 4;  // stages per scale load
    constexpr int CR = SS / 2;             // 16-byte scale chunks per row per load
    uint8_t* stab = as_tab + __builtin_amdgcn_readfirstlane(wave) * (64 * kBfSclPitch);
    // lane chunk i*64 + lane = part (i*64 + lane) % CR of table row (i*64 + lane) / CR
    // = 16 t + r; chunk 1 (CR = 2) lies 32 table rows = two tiles further, at a
    // uniform distance in the global rows (w3 instead of w1, or 32 rows of w2)
    const int srow = lane / CR, spart = lane % CR, st = srow >> 4, sr = srow & 15;
    const uint8_t* ssrc = (GATEUP ? (st < 2 ? ex.w1s : ex.w3s) + (int64_t)(col0 + 16 * (st & 1) + sr) * bsrow
                                  : ex.w2s + (int64_t)(col0 + 16 * st + sr) * bsrow) +
                          16 * spart;
    const int64_t sstep = GATEUP ? (int64_t)((uintptr_t)ex.w3s - (uintptr_t)ex.w1s) : 32 * bsrow;
    const int sdst = srow * kBfSclPitch + 16 * spart;
    v4i sreg[CR];
    auto sload = [&](int s) __attribute__((always_inline)) {
#pragma unroll
      for (int i = 0; i < CR; ++i) sreg[i] = ld16((const uint8_t*)((uintptr_t)ssrc + i * sstep) + 8 * SS * s);
    };
    // the table rows are written and read by different lanes of the one wave,
    // whose LDS accesses complete in order
    auto sstore = [&]() __attribute__((always_inline)) {
#pragma unroll
      for (int i = 0; i < CR; ++i) {
        uint64_t* d = (uint64_t*)(stab + sdst + i * 32 * kBfSclPitch);
        d[0] = (uint64_t)(uint32_t)sreg[i].x | ((uint64_t)(uint32_t)sreg[i].y << 32);
        d[1] = (uint64_t)(uint32_t)sreg[i].z | ((uint64_t)(uint32_t)sreg[i].w << 32);
      }
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
      __builtin_amdgcn_wave_barrier();
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    };
    BStageT<false> b;
    auto sread = [&](int j) __attribute__((always_inline)) {
#pragma unroll
      for (int t = 0; t < kNT; ++t)
        b.s[t] = *(const uint16_t*)(stab + (16 * t + r16) * kBfSclPitch + 8 * (j % SS) + 2 * g);
    };
    v4i lreg[LH];
#pragma unroll
    for (int v = 0; v < LV; ++v)
      if (lon[v]) *(v4i*)&a_lds[0][ldst[v]] = ld16(lsrc[v]);
    load_b<false, false, NTW>(b, btp, nullptr, 0, g, lay);
    sload(0);
    sstore();
    sread(0);
    __syncthreads();
#pragma unroll
    for (int j = 0; j < NST; ++j) {
      const bool more = j + 1 < NST;
      uint8_t* nxt = a_lds[(j + 1) & 1];
      if (more) {
#pragma unroll
        for (int v = 0; v < LH; ++v)
          if (lon[v]) lreg[v] = ld16(lsrc[v] + (j + 1) * ASB);
      }
      if (j % SS == SS - 2 && j + 2 < NST) sload(j / SS + 1);  // the next SS stages' scales
      bf16x8_t bw[kNT][4];
#pragma unroll
      for (int ji = 0; ji < 2; ++ji) {
        dequant_half(bw, b, ji);
        if (more) {
#pragma unroll
          for (int t = 0; t < kNT; ++t) b.d[t][ji] = ld16_w<NTW>(btp[t] + (j + 1) * lay.stage_stride + ji * lay.mfma_stride);
          if (ji == 1) {
            if (j % SS == SS - 1) sstore();  // stage j's bytes were read during stage j - 1
            sread(j + 1);
          }
        }
        __builtin_amdgcn_sched_barrier(0);
        mfma_half_bf16<MT>(acc, a_lds[j & 1], bw, ji, r16, g, live);
        __builtin_amdgcn_sched_barrier(0);
        if (more) {
#pragma unroll
          for (int v = 0; v < LH; ++v)
            if (lon[ji * LH + v]) *(v4i*)&nxt[ldst[ji * LH + v]] = lreg[v];
          if (ji == 0) {
#pragma unroll
            for (int v = 0; v < LH; ++v)
              if (lon[LH + v]) lreg[v] = ld16(lsrc[LH + v] + (j + 1) * ASB);
          }
        }
      }
      __syncthreads();
    }
  };
  // uniform per workgroup (have_w, shared), so the barriers inside are reached by all
  auto kloop = [&](auto b8, auto t0c) {
    constexpr bool B8 = decltype(b8)::value;
    constexpr int t0 = decltype(t0c)::value;
    constexpr int NTB = BStageT<B8>::NTB;
    const uint8_t* const* btp = bt + t0;
    const uint8_t* const* bstp = bst + t0;
    if constexpr (ABF) {
      kloop_bf16(btp);
      return;
    }
    // scales of the whole K range, loaded once: the weight rows' by their lanes
    // (shared out per stage by permutes), the A rows' into an LDS table
    RowScales<NST> bs_row[NTB];
#pragma unroll
    for (int t = 0; t < NTB; ++t) load_row_scales<NST>(bs_row[t], bstp[t], g);
#pragma unroll
    for (int i = 0; i < (AS_CHUNKS + NTH - 1) / NTH; ++i) {
      const int c = i * NTH + tid;
      if (c < AS_CHUNKS && ((live >> (c / (KSB / 16) / 16)) & 1u)) {
        const int row = c / (KSB / 16), ch = c % (KSB / 16);
        const int64_t ar = a_row<SH>(p, p.sorted_ids[mb * BM + row]);
        *(v4i*)&as_tab[row * ASP + 16 * ch] = ld16(p.a_scale + ar * KSB + 16 * ch);
      }
    }
    v4i lreg[LV];
    BStageT<B8> b[2];
#pragma unroll
    for (int v = 0; v < LV; ++v)
      if (lon[v]) lreg[v] = ld16(lsrc[v]);
    load_b<false, B8, NTW>(b[0], btp, bstp, 0, g, lay);
#pragma unroll
    for (int v = 0; v < LV; ++v)
      if (lon[v]) *(v4i*)&a_lds[0][ldst[v]] = lreg[v];
    __syncthreads();
#pragma unroll
    for (int j = 0; j < NST; ++j) {
      if (j + 1 < NST) {
#pragma unroll
        for (int v = 0; v < LV; ++v)
          if (lon[v]) lreg[v] = ld16(lsrc[v] + (j + 1) * ASB);
        load_b<false, B8, NTW>(b[(j + 1) & 1], btp, bstp, j + 1, g, lay);
      }
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int t = 0; t < NTB; ++t) b[j & 1].s[t] = stage_scales<NST>(bs_row[t], j, r16, g);
      compute_tiled<AFMT, MT, B8, t0>(acc, a_lds[j & 1], as_tab, ASP, j, b[j & 1], r16, g, live);
      __builtin_amdgcn_sched_barrier(0);
      if (j + 1 < NST) {
#pragma unroll
        for (int v = 0; v < LV; ++v)
          if (lon[v]) *(v4i*)&a_lds[(j + 1) & 1][ldst[v]] = lreg[v];
      }
      __syncthreads();
    }
  };
  if (have_w) {
    if constexpr (AFMT == 0 && SH) {
      if (shared) {
        kloop(std::true_type{}, std::integral_constant<int, 0>{});
        // the second pass restages the A tiles: the LDS ring is free again
        kloop(std::true_type{}, std::integral_constant<int, kNT / 2>{});
      } else {
        kloop(std::false_type{}, std::integral_constant<int, 0>{});
      }
    } else {
      kloop(std::false_type{}, std::integral_constant<int, 0>{});
    }
  }

  if (GATEUP && p.hq_mode) {
    uint32_t hb[MT][4][2];
    int fr[MT][4];
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
      store_tile<GATEUP, SH>(p, acc[mt], mb * BM + 16 * mt, col0, g, r16, hb[mt], fr[mt]);
    if (p.hq_mode == 2) {
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) quantise_h_mxfp4(p, hb[mt], fr[mt], col0, g, r16);
    } else {
      // FP8 per 128: waves 4b..4b+3 hold the 128 columns of block b of each row;
      // row maxima meet in LDS (the K loop is done with a_lds)
      float* am = (float*)&a_lds[0][0];  // [NW waves][BM rows]
#pragma unroll
      for (int mt = 0; mt < MT; ++mt)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const float m = dsv4::wave_max_xor(
              fmaxf(fabsf(dsv4::bf16_to_f32(hb[mt][i][0])), fabsf(dsv4::bf16_to_f32(hb[mt][i][1]))), 16);
          if (r16 == 0) am[wave * BM + 16 * mt + 4 * g + i] = m;
        }
      __syncthreads();
#pragma unroll
      for (int mt = 0; mt < MT; ++mt)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int row = 16 * mt + 4 * g + i, f = fr[mt][i];
          const float* ab = am + (wave & ~3) * BM + row;
          const float amax = fmaxf(fmaxf(ab[0], ab[BM]), fmaxf(ab[2 * BM], ab[3 * BM]));
          const int k = dsv4::fp8_block_exp(amax);
          const float inv = dsv4::pow2f(-k);
          if (f < p.R) {
            uint8_t* crow = p.hq_codes + (int64_t)f * p.N + col0 + r16;
            crow[0] = (uint8_t)dsv4::fp8_code(dsv4::bf16_to_f32(hb[mt][i][0]), inv);
            crow[16] = (uint8_t)dsv4::fp8_code(dsv4::bf16_to_f32(hb[mt][i][1]), inv);
            if ((wave & 3) == 0 && r16 == 0)
              *(uint32_t*)(p.hq_scale + (int64_t)f * (p.N / 32) + (col0 & ~127) / 32) = (uint32_t)(k + 127) * 0x01010101u;
          }
        }
    }
  } else {
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) store_tile<GATEUP, SH>(p, acc[mt], mb * BM + 16 * mt, col0, g, r16);
  }
}

// Weights of an expert with several M blocks are re-read by each of them from L2
// and keep plain loads (non-temporal ones measured 2-4% slower for those);
// an expert with one M block (most experts below a few thousand tokens) reads
// its weights once, and non-temporal loads keep them from displacing the
// re-read lines: 2% off the 2048-token layer, 5% off the 512-token one
// (outputs bit-identical). The choice is made per block before anything else,
// so the two bodies share no live values.
template <int AFMT, bool GATEUP, int NST, int MT, int NW, bool SH>
__global__ __launch_bounds__(64 * NW, (MT <= 4 && NW == 4 ? 2 : 1)) void moe_gemm_tiled_kernel(Dsv4GemmArgs p) {
  constexpr int BM = 16 * MT;
  constexpr int ASP = 8 * NST + 16;  // A scale table pitch (K / 32 + 16 bytes)
  __shared__ __attribute__((aligned(16))) uint8_t a_lds[2][tiled_a_buf_bytes<AFMT, MT>()];
  __shared__ __attribute__((aligned(16))) uint8_t as_tab[AFMT == kAfmtBf16 ? NW * 64 * kBfSclPitch : BM * ASP];
  const int mb = blockIdx.y;
  const int npp = p.num_post_padded[0];
  if (mb * BM >= npp) return;
  const int e = p.block_expert[mb];
  const bool single = (mb == 0 || p.block_expert[mb - 1] != e) && ((mb + 1) * BM >= npp || p.block_expert[mb + 1] != e);
  if (single)
    tiled_block<AFMT, GATEUP, NST, MT, NW, SH, true>(p, a_lds, as_tab);
  else
    tiled_block<AFMT, GATEUP, NST, MT, NW, SH, false>(p, a_lds, as_tab);
}

}  // namespace

template <bool GATEUP, int NST, bool SH>
static void launch_nst_sh(const Dsv4GemmArgs& a, hipStream_t st) {
  const int cols_per_wave = GATEUP ? 32 : 64;
  if (a.block_m == kBM) {  // decode-shaped: single-wave workgroups
    const dim3 grid(a.N / (kWaves * cols_per_wave), a.max_blocks);
    if constexpr (!SH) {  // bf16 activations: routed experts only
      if (a.afmt == kAfmtBf16) {
        hipLaunchKernelGGL((moe_gemm_kernel<kAfmtBf16, GATEUP, NST, false>), grid, dim3(64 * kWaves), 0, st, a);
        return;
      }
    }
    if (a.afmt == 0)
      hipLaunchKernelGGL((moe_gemm_kernel<0, GATEUP, NST, SH>), grid, dim3(64 * kWaves), 0, st, a);
    else
      hipLaunchKernelGGL((moe_gemm_kernel<1, GATEUP, NST, false>), grid, dim3(64 * kWaves), 0, st, a);
    return;
  }
  // 4-wave workgroups for E4M3 and E2M1 activations (8-wave ones, sharing each
  // A tile across twice the columns, measured no faster); bf16 activations, with
  // twice the A bytes of E4M3 per row, take 8-wave workgroups where the columns
  // divide (1-3% faster at 512 and 2048 tokens, outputs bit-identical)
  const dim3 grid(a.N / (4 * cols_per_wave), a.max_blocks);
  if constexpr (!SH) {  // bf16 activations: 64-row blocks, routed experts only
    if (a.afmt == kAfmtBf16) {
      if (a.N % (8 * cols_per_wave) == 0) {
        const dim3 grid8(a.N / (8 * cols_per_wave), a.max_blocks);
        hipLaunchKernelGGL((moe_gemm_tiled_kernel<kAfmtBf16, GATEUP, NST, 4, 8, false>), grid8, dim3(512), 0, st, a);
      } else {
        hipLaunchKernelGGL((moe_gemm_tiled_kernel<kAfmtBf16, GATEUP, NST, 4, 4, false>), grid, dim3(256), 0, st, a);
      }
      return;
    }
  }
  if (a.block_m == 64) {
    if (a.afmt == 0)
      hipLaunchKernelGGL((moe_gemm_tiled_kernel<0, GATEUP, NST, 4, 4, SH>), grid, dim3(256), 0, st, a);
    else
      hipLaunchKernelGGL((moe_gemm_tiled_kernel<1, GATEUP, NST, 4, 4, false>), grid, dim3(256), 0, st, a);
  } else {
    if (a.afmt == 0)
      hipLaunchKernelGGL((moe_gemm_tiled_kernel<0, GATEUP, NST, 8, 4, SH>), grid, dim3(256), 0, st, a);
    else
      hipLaunchKernelGGL((moe_gemm_tiled_kernel<1, GATEUP, NST, 8, 4, false>), grid, dim3(256), 0, st, a);
  }
}

// The shared-expert instantiations exist for E4M3 activations (the bf16
// profile) only; the C ABI rejects a shared expert with E2M1 activations.
template <bool GATEUP, int NST>
static void launch_nst(const Dsv4GemmArgs& a, hipStream_t st) {
  if (a.has_shared && a.afmt == 0)
    launch_nst_sh<GATEUP, NST, true>(a, st);
  else
    launch_nst_sh<GATEUP, NST, false>(a, st);
}

template <bool GATEUP>
static hipError_t launch(const Dsv4GemmArgs& a, hipStream_t st) {
  if (a.block_m == kHotBlockM && !a.has_shared) return launch_moe_gemm_big(a, GATEUP, st);  // gemm_big.hip
  if (a.block_m != 16 && a.block_m != 64 && a.block_m != 128) return hipErrorInvalidValue;
  // bf16 activations: 16- or 64-row blocks, without a shared expert or a fused h quantisation
  if (a.afmt == kAfmtBf16 && (a.block_m == 128 || a.has_shared || (GATEUP && a.hq_mode))) return hipErrorInvalidValue;
  switch (a.Kdim / kStageK) {
    case 2: launch_nst<GATEUP, 2>(a, st); break;
    case 4: launch_nst<GATEUP, 4>(a, st); break;
    case 8: launch_nst<GATEUP, 8>(a, st); break;
    case 16: launch_nst<GATEUP, 16>(a, st); break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

// Reduction lengths 512..4096. Longer ones are not compiled: at K = 8192 the
// fully unrolled K loops of the 64/128-row kernels spill to scratch.
bool moe_gemm_supported_kdim(int kdim) {
  const int n = kdim / kStageK;
  return kdim % kStageK == 0 && (n == 2 || n == 4 || n == 8 || n == 16);
}

bool moe_gemm_supported_block_m(int bm) { return bm == 16 || bm == 64 || bm == 128 || bm == kHotBlockM; }

hipError_t launch_moe_gemm_gateup(const Dsv4GemmArgs& a, hipStream_t st) { return launch<true>(a, st); }

hipError_t launch_moe_gemm_down(const Dsv4GemmArgs& a, hipStream_t st) { return launch<false>(a, st); }
