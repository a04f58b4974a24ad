// Large-tile grouped GEMM for experts that receive many rows (prefill).
//
// moe_align gives every expert with at least `hot_min` routed rows its own
// layout of 256-row M blocks (the "hot" layout); this kernel runs those
// blocks against 256 weight rows (gate/up: 128 gate + the 128 matching up rows;
// down: 256 output rows of W2). Both operand tiles of each 64-k stage go through
// LDS - the A rows gathered through sorted_ids, the weight rows from the
// expert's slot - so every weight byte a workgroup brings from L2 serves 128 or
// 256 rows (the 16/64-row kernels re-read an expert's weights once per 16 or 64
// rows) and every A byte 256 weight rows. Two waves share each SIMD, each with
// 128 accumulator registers of v_mfma_scale_f32_32x32x64_f8f6f4 tiles, in one of
// two shapes picked per launch (Cfg):
//   whole blocks (E2M1 A from 32,768 rows): one workgroup of 8 waves per CU over
//                    the whole 256-row block; a wave owns 128 rows x 64 weight rows
//                    (4 x 2 tiles).
//   half blocks (E4M3 A; E2M1 A below 32,768 rows): two workgroups of 4 waves per
//                    CU, each over half a block (128 rows); a wave owns 64 rows x
//                    128 weight rows (2 x 4).
// A weight fragment read from LDS feeds TT MFMAs and an activation fragment WT.
// Two waves per SIMD let one wave's MFMAs run while the other waits at a barrier
// or on its LDS reads (against one 128 x 128 wave per SIMD, 256 accumulators in
// the AGPRs, the kernels took 4-8 % less time); two independent workgroups per CU
// also keep the MFMAs of one busy while the other crosses its stage barrier. The
// 32x32x64 form carries twice the FLOPs per operand byte of the 16x16x128 one (and
// ran fp4 x fp4 at 7.25 PFLOP/s against 6.7 in an MFMA-loop probe on this part).
//
// Operands move global -> LDS with global_load_lds_dwordx4 (lane i of one
// instruction writes its 16 bytes at the instruction's LDS base + 16 i): no
// staging registers, so a ring of NB stage slots keeps NB - 1 stages of loads
// in flight (96 KB per CU with E2M1 A on whole blocks, 2 x 32-36 KB on half blocks);
// the depth of the ring, and the second workgroup, hide the load latency.
// Each 1-KB chunk is laid out in the order the MFMA lanes read it, with an XOR
// swizzle that puts the 16 lanes of each ds_read_b128 pass on distinct banks.
//
// Operand layouts of the 32x32x64 scaled MFMA (measured on gfx950):
//   E2M1 A/B: lane (r = l%32, g = l/32) holds k [32g, 32g+32) of row r in 16
//             bytes, low nibble first.
//   E4M3 A  : lane (r, g) holds k [16g, 16g+16) in bytes 0-15 and
//             [32+16g, 32+16g+16) in bytes 16-31.
//   scales  : lane (r, g) supplies the E8M0 of 32-block g of its row/column.
//   C       : register i of lane l holds C[8(i/4) + 4(l/32) + i%4][l%32].
// Chunks of one stage (slot i = bytes [16 i, 16 i + 16) of a chunk):
//   E4M3 A chunk c : rows 16c + r (r < 16), 64 bytes each; slot 4r + (p ^ (r/4 % 4))
//                    holds bytes [16p, 16p + 16) of row r's stage.
//   E2M1 A chunk c : rows 32c + r (r < 32), 32 bytes each; slot 2r + (p ^ (r/8 % 2))
//                    holds bytes [16p, 16p + 16).
//   weight chunk c : weight rows 32c + 16h + r (h < 2, r < 16); slot 32h + 16j + r
//                    holds bytes [16j, 16j + 16) of the row's stage (in an
//                    MFMA-tiled slot, two whole 256-byte runs of each 16-row tile).
#include "common.h"
#include "kernels.h"
#include "quant_dev.h"

namespace {

typedef int v8i __attribute__((ext_vector_type(8)));
typedef int v4i __attribute__((ext_vector_type(4)));
typedef float v16f __attribute__((ext_vector_type(16)));
typedef __attribute__((address_space(1))) const v4i gv4i;
typedef __attribute__((address_space(1))) const void gvoid;
typedef __attribute__((address_space(3))) void lvoid;

constexpr int kHB = 256;     // rows per block of the hot layout
constexpr int kBN = 256;     // weight rows per block
constexpr int kKS = 64;      // k per stage
constexpr int kSS = 16;      // stages per scale super-stage (1024 k)

// Workgroup shapes. HALF: two workgroups per CU, each half a 256-row block, 4 waves of
// 64 rows x 128 weight rows; otherwise one workgroup per CU over the whole block, 8
// waves of 128 x 64. Either way two waves share a SIMD; two independent workgroups let
// one's MFMAs run while the other waits at its stage barrier. Measured (layer time, same
// runs): E4M3 at 16384 tokens 4.49-4.60 ms with the 8-wave shape against 4.27-4.29 with
// the half-block one; E2M1 at 16384 tokens 3.54-3.68 against 3.68-3.76, at 2048 tokens
// (16,384 routed rows, the hot experts' blocks too few to fill the CUs) 1.012-1.022
// against 0.981-0.984. launch_moe_gemm_big picks HALF for E4M3, and for E2M1 below
// 32,768 rows.
template <int AFMT, bool HALF>
struct Cfg {
  static constexpr int BM = HALF ? 128 : 256;  // rows per workgroup
  static constexpr int NT = HALF ? 256 : 512;  // threads
  static constexpr int NW = NT / 64;           // waves
  static constexpr int WM = 2, WN = NW / WM;   // wave grid over rows x weight rows
  static constexpr int TT = BM / WM / 32;      // 32-row token tiles per wave
  static constexpr int WT = kBN / WN / 32;     // 32-row weight tiles per wave
  static constexpr int WGS = HALF ? 2 : 1;     // workgroups per CU
};

template <int AFMT, bool HALF>
struct Big {
  using G = Cfg<AFMT, HALF>;
  static constexpr int kBM = G::BM;
  static constexpr int kNT = G::NT;
  static constexpr int ACH = kBM * (AFMT == 0 ? kKS : kKS / 2) / 1024;  // 1-KB A chunks per stage
  static constexpr int BCH = kBN * (kKS / 2) / 1024;  // 1-KB weight chunks per stage
  static constexpr int STAGE = (ACH + BCH) * 1024;
  static constexpr int NB = HALF ? (AFMT == 0 ? 3 : 4) : (AFMT == 0 ? 5 : 7);  // stage slots of the ring
  static constexpr int AV = ACH / Cfg<AFMT, HALF>::NW;      // A loads per thread per stage
  static constexpr int BV = BCH / Cfg<AFMT, HALF>::NW;      // weight loads per thread per stage
  static constexpr int L = AV + BV;
  typedef v16f Acc[G::TT][G::WT];  // a wave's accumulators
  // scales: one super-stage = 32 bytes per A row and per weight row (two 16-byte
  // pieces), loaded by LDS-DMA once per 16 stages into one of two buffers; a buffer
  // holds the A rows' then the weight rows' pieces, each half-major:
  // [half][row] x 16 bytes
  static constexpr int SCL = 2 * (kBM + kBN) * 16;
  static constexpr int AS_OFF = NB * STAGE;
  static constexpr int BS_OFF = kBM * 32;            // weight rows within a buffer
  static constexpr int SV = SCL / (kNT * 16);         // scale loads per thread per super-stage
  static constexpr int LDS = NB * STAGE + 2 * SCL;
  static_assert(LDS * Cfg<AFMT, HALF>::WGS <= 160 * 1024, "the stage ring and two scale super-stages must fit the LDS");
  static_assert(BCH == 8 && (ACH * 1024) == kBM * (AFMT == 0 ? kKS : kKS / 2), "chunking");
  static_assert(AV * G::NW == ACH && BV * G::NW == BCH && SV * kNT * 16 == SCL, "loads per thread");
  static_assert(L * NB + SV < 64, "vmcnt holds 6 bits");
};

DSV4_DEV bool tiled_ptr(const uint8_t* p) { return ((uintptr_t)p & 1u) != 0; }
DSV4_DEV const uint8_t* untag(const uint8_t* p) { return (const uint8_t*)((uintptr_t)p & ~(uintptr_t)1); }

// 16 bytes per lane from src to dst + 16 * lane (dst: the same for the whole wave)
DSV4_DEV void dma16(const uint8_t* src, uint8_t* dst) {
  __builtin_amdgcn_global_load_lds((gvoid*)src, (lvoid*)dst, 16, 0, 0);
}

// Waits until at most N of this wave's vector-memory loads are outstanding, then
// for every wave of the block. The direct-to-LDS loads are counted here by hand
// (a workgroup fence would make the compiler drain them all at every barrier);
// lgkmcnt(0) completes this wave's own LDS writes (the scales) first.
// The wait is the s_waitcnt builtin rather than inline assembly so that the
// compiler's own wait tracking sees it (it would otherwise keep counting the LDS
// reads before it as pending); the empty asm statements keep memory accesses from
// moving across the barrier.
template <int N>
DSV4_DEV void wait_loads_barrier() {
  static_assert(N >= 0 && N < 64, "vmcnt is 6 bits");
  // simm16: vmcnt [3:0] and [15:14], expcnt [6:4] (7: no wait), lgkmcnt [11:8] (0)
  constexpr int kEnc = (N & 15) | ((N >> 4) << 14) | (7 << 4);
  __builtin_amdgcn_sched_barrier(0);
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_waitcnt(kEnc);
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
  __builtin_amdgcn_sched_barrier(0);
}

// Issues the scale loads of super-stage ss into buffer `buf` (sc_src: this lane's
// pieces at super-stage 0, in load order (wave * SV + v) * 64 + lane).
template <int AFMT, bool HALF>
DSV4_DEV void big_dma_scales(uint8_t* lds, int buf, const uint8_t* const* sc_src, int wave, int ss) {
  using C = Big<AFMT, HALF>;
#pragma unroll
  for (int v = 0; v < C::SV; ++v) dma16(sc_src[v] + ss * 32, lds + C::AS_OFF + buf * C::SCL + (wave * C::SV + v) * 1024);
}

// Issues stage s's loads into ring slot `slot`: this wave's A chunks wave * AV + v and
// weight chunks wave * BV + v (a_src / b_src: this lane's piece at stage 0; bj / bg:
// the weight offset per 4 stages / per stage within them, no branch in the loop).
template <int AFMT, bool HALF>
DSV4_DEV void big_dma_stage(uint8_t* slot, const uint8_t* const* a_src, const uint8_t* const* b_src, int wave,
                            int bj, int bg, int s) {
  using C = Big<AFMT, HALF>;
  const int aoff = s * (AFMT == 0 ? kKS : kKS / 2);
#pragma unroll
  for (int v = 0; v < C::AV; ++v) dma16(a_src[v] + aoff, slot + (wave * C::AV + v) * 1024);
  // 4 stages = 256 k: 2048 bytes on in a tiled slot (128 row-major), 256 within it (32)
  const int boff = (s >> 2) * bj + (s & 3) * bg;
#pragma unroll
  for (int v = 0; v < C::BV; ++v) dma16(b_src[v] + boff, slot + (C::ACH + wave * C::BV + v) * 1024);
}

// The fragments of one stage for this wave: weight tiles nt (16 bytes each), A tiles
// mt (E4M3: 2 x 16 bytes, E2M1: 16 bytes).
template <int AFMT, bool HALF>
struct BigFrag {
  v4i b[Cfg<AFMT, HALF>::WT];
  v4i lo[Cfg<AFMT, HALF>::TT];
  v4i hi[AFMT == 0 ? Cfg<AFMT, HALF>::TT : 1];
};

// Reads one stage's fragments from ring slot L. a_lo / a_hi: this lane's byte offsets
// inside an A chunk, b_lane inside a weight chunk.
template <int AFMT, bool HALF>
DSV4_DEV void big_read(BigFrag<AFMT, HALF>& F, const uint8_t* L, int wm, const int* brow0, int r32, int a_lo,
                       int a_hi, int b_lane) {
  using C = Big<AFMT, HALF>;
#pragma unroll
  for (int nt = 0; nt < Cfg<AFMT, HALF>::WT; ++nt) F.b[nt] = *(const v4i*)(L + (C::ACH + brow0[nt] / 32) * 1024 + b_lane);
#pragma unroll
  for (int mt = 0; mt < Cfg<AFMT, HALF>::TT; ++mt) {
    const int row0 = (Cfg<AFMT, HALF>::BM / Cfg<AFMT, HALF>::WM) * wm + 32 * mt;
    if (AFMT == 0) {
      const uint8_t* ch = L + (row0 / 16 + (r32 >> 4)) * 1024;
      F.lo[mt] = *(const v4i*)(ch + a_lo);
      F.hi[mt] = *(const v4i*)(ch + a_hi);
    } else {
      F.lo[mt] = *(const v4i*)(L + (row0 / 32) * 1024 + a_lo);
    }
  }
}

// Scales of a group of four stages 4j .. 4j + 3 for this wave's tiles. A super-stage
// buffer holds, per A row and per weight row, the row's 32 E8M0 bytes of the 1024 k as
// two 16-byte pieces, half-major ([A rows][weight rows], each [half][row] x 16 bytes).
// Stage s of a super-stage uses, in lane (r32, g2), the row's byte q = 2 (s % 16) + g2:
// byte 2 (s % 8) + g2 of its piece s / 8. The group's bytes
// for both g2 are the 8 bytes at 2 (s % 8) (8-byte aligned): one ds_read_b64 per tile
// per four stages instead of one byte read per tile per stage. Shifted right by 8 g2,
// stage 4j + i's byte sits at bit 16 (i % 2) of word i / 2, which the MFMA picks with
// its scale byte select (op_sel = 2 (i % 2)).
template <int AFMT, bool HALF>
struct BigScl {
  uint64_t b[Cfg<AFMT, HALF>::WT], a[Cfg<AFMT, HALF>::TT];
};
template <int AFMT, bool HALF>
struct BigSclW {
  uint32_t b[Cfg<AFMT, HALF>::WT][2], a[Cfg<AFMT, HALF>::TT][2];
};

// Reads the raw scale groups of stages s0 .. s0 + 3 (s0 % 4 == 0, the stage within its
// super-stage) from super-stage buffer S.
template <int AFMT, bool HALF>
DSV4_DEV void big_read_scales(BigScl<AFMT, HALF>& R, const uint8_t* S, int s0, int wm, const int* brow0, int r32) {
  constexpr int kBM = Cfg<AFMT, HALF>::BM;
  const int off = 2 * (s0 & 7), half = s0 >> 3;  // byte within the row's 16-byte piece `half`
#pragma unroll
  for (int nt = 0; nt < Cfg<AFMT, HALF>::WT; ++nt)
    R.b[nt] = *(const uint64_t*)(S + kBM * 32 + (half * kBN + brow0[nt] + r32) * 16 + off);
#pragma unroll
  for (int mt = 0; mt < Cfg<AFMT, HALF>::TT; ++mt) {
    const int row0 = (kBM / Cfg<AFMT, HALF>::WM) * wm + 32 * mt;
    R.a[mt] = *(const uint64_t*)(S + (half * kBM + row0 + r32) * 16 + off);
  }
}

// This lane's scale words of a group: its bytes (g2) moved to bits 0, 16 of two words.
template <int AFMT, bool HALF>
DSV4_DEV void big_scale_words(BigSclW<AFMT, HALF>& W, const BigScl<AFMT, HALF>& R, int g2) {
  const int sh = 8 * g2;
#pragma unroll
  for (int nt = 0; nt < Cfg<AFMT, HALF>::WT; ++nt) {
    const uint64_t v = R.b[nt] >> sh;
    W.b[nt][0] = (uint32_t)v;
    W.b[nt][1] = (uint32_t)(v >> 32);
  }
#pragma unroll
  for (int mt = 0; mt < Cfg<AFMT, HALF>::TT; ++mt) {
    const uint64_t v = R.a[mt] >> sh;
    W.a[mt][0] = (uint32_t)v;
    W.a[mt][1] = (uint32_t)(v >> 32);
  }
}

// Instruction order of one stage after its barrier: each MFMA (64 cycles in the
// matrix pipe with FP8 A) followed by one of the stage's loads and two of the next
// stage's fragment reads, so the LDS and the memory pipe work under the MFMAs and
// the reads are done long before the next barrier waits for them.
template <int AFMT, bool HALF, int I>
DSV4_DEV void big_sched() {
  using G = Cfg<AFMT, HALF>;
  // ds_reads of big_read (+ big_read_scales in the last stage of a group)
  constexpr int kReads = G::WT + (AFMT == 0 ? 2 : 1) * G::TT + (I == 3 ? G::WT + G::TT : 0);
#pragma unroll
  for (int i = 0; i < G::TT * G::WT; ++i) {
    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);                      // MFMA
    if (i < Big<AFMT, HALF>::L) __builtin_amdgcn_sched_group_barrier(0x020, 1, 0);  // VMEM read
    if (2 * i < kReads) __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);    // DS read
  }
}

// One stage of MFMAs: TT x WT tiles of 32 x 32 per wave. The weights are the MFMA's A
// operand and the activations its B operand, so accumulator (tt, wt) holds weight
// columns x tokens: register r of lane l = weight column 8(r/4) + 4(l/32) + r%4 of
// weight tile wt, token l%32 of token tile tt (the E4M3 B layout is the A layout).
template <int AFMT, bool HALF, int I>
DSV4_DEV void big_mfma(typename Big<AFMT, HALF>::Acc& acc, const BigFrag<AFMT, HALF>& F, const BigSclW<AFMT, HALF>& W) {
#pragma unroll
  for (int tt = 0; tt < Cfg<AFMT, HALF>::TT; ++tt) {
    const v4i lo = F.lo[tt];
    const v4i hi = AFMT == 0 ? F.hi[tt] : v4i{0, 0, 0, 0};
    const v8i xf = v8i{lo.x, lo.y, lo.z, lo.w, hi.x, hi.y, hi.z, hi.w};
#pragma unroll
    for (int wt = 0; wt < Cfg<AFMT, HALF>::WT; ++wt) {
      const v8i wf = v8i{F.b[wt].x, F.b[wt].y, F.b[wt].z, F.b[wt].w, 0, 0, 0, 0};
      // stage I of the scale group: word I / 2, byte 2 (I % 2)
      acc[tt][wt] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(wf, xf, acc[tt][wt], 4, AFMT == 0 ? 0 : 4,
                                                                   2 * (I & 1), W.b[wt][I >> 1], 2 * (I & 1),
                                                                   W.a[tt][I >> 1]);
    }
  }
}

// ---- epilogue ---------------------------------------------------------------------
// Each lane holds, per token tile tt, 4-column runs of one token's row (columns
// 8q + 4(l/32) + e of every 32-column weight tile): SwiGLU, the quantisation blocks'
// maxima (in-lane, then across the lane pair l, l ^ 32, then - FP8 h only - across the
// WN waves of a token row through the LDS) and the packing all stay in registers.
// bf16 / E4M3 / E2M1 conversions use the gfx950 converters, which agree bit for bit
// with the library's software quantisers on every input they see here (RNE; E4M3 after
// the clamp to +-448; E2M1 with the sign of the input, whose -0 the rule-0 path
// turns into +0 as that rule wants).

// max of x over the lane pair (l, l ^ 32)
DSV4_DEV float max_pair(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_int(x), __float_as_int(x), false, false);
  return fmaxf(__int_as_float(r[0]), __int_as_float(r[1]));
}

// two floats -> packed bf16 (RNE), low half = a
DSV4_DEV uint32_t pk_bf16(float a, float b) {
  typedef __bf16 v2bf __attribute__((ext_vector_type(2)));
  const v2bf v = v2bf{(__bf16)a, (__bf16)b};
  return __builtin_bit_cast(uint32_t, v);
}
DSV4_DEV float bf16_lo(uint32_t w) { return __uint_as_float(w << 16); }
DSV4_DEV float bf16_hi(uint32_t w) { return __uint_as_float(w & 0xffff0000u); }

// silu(min(g, L)) * clamp(u, +-L) * w for bf16-rounded g, u, with silu(g) = g / (1 + e^-g)
// written exactly as the 16/64-row kernels' epilogue (expf, IEEE divide), so a token row
// gets the same h whichever kernel its expert runs on (deepseek_v4.py:184-187)
DSV4_DEV float big_swiglu(float gt, float up, float w, float limit) {
  if (limit > 0.0f) {
    up = fminf(fmaxf(up, -limit), limit);
    gt = fminf(gt, limit);
  }
  return gt / (1.0f + expf(-gt)) * up * w;
}

// 4 E4M3 codes of a * inv .. d * inv (inv = 2^-k), byte 0 = a
DSV4_DEV uint32_t pk_fp8x4(float a, float b, float c, float d, float inv) {
  const float m = 448.0f;
  const int lo = __builtin_amdgcn_cvt_pk_fp8_f32(fminf(fmaxf(a * inv, -m), m), fminf(fmaxf(b * inv, -m), m), 0, false);
  return (uint32_t)__builtin_amdgcn_cvt_pk_fp8_f32(fminf(fmaxf(c * inv, -m), m), fminf(fmaxf(d * inv, -m), m), lo, true);
}

// E2M1 nibble pair of a * inv, b * inv (low nibble = a) under scale rule `rule`
DSV4_DEV uint32_t pk_fp4x2(float a, float b, float inv, int rule) {
  float ya = fminf(fmaxf(a * inv, -6.0f), 6.0f), yb = fminf(fmaxf(b * inv, -6.0f), 6.0f);
  if (rule == 0) {  // the sign of a value that is exactly zero is +
    ya = ya == 0.0f ? 0.0f : ya;
    yb = yb == 0.0f ? 0.0f : yb;
  }
  return __builtin_amdgcn_cvt_scalef32_pk_fp4_f32(0u, ya, yb, 1.0f, 0) & 0xffu;
}

// Block -> tile mapping. Workgroups are dispatched to the 8 XCDs round-robin by
// linear id, and each XCD has its own L2, so with the plain mapping (N tiles fastest)
// every XCD would run 2 of the 16 N tiles of every M block and fetch every M block's
// A rows into its own L2. With N tiles a multiple of 8, each 32 consecutive
// workgroups of an XCD get 4 M extents x 8 N tiles instead: A rows shared 8 ways
// and weight tiles 4 ways within one L2. (An M extent is a hot-layout block, or
// half of one where a block takes two workgroups.) The grid's y extent is then
// padded to a multiple of 32; the padding workgroups exit at once.
DSV4_DEV void big_tile_of_block(int& mb, int& nt) {
  const int ntiles = gridDim.x;
  if (ntiles % 8 != 0) {
    mb = blockIdx.y;
    nt = blockIdx.x;
    return;
  }
  const int id = blockIdx.y * ntiles + blockIdx.x;
  const int x = id & 7, j = id >> 3;  // XCD, position in that XCD's sequence
  const int gi = j >> 5, w = j & 31;  // group of 32, place in it
  const int ngroups = ntiles >> 3;
  mb = 4 * ((gi / ngroups) * 8 + x) + (w >> 3);
  nt = 8 * (gi % ngroups) + (w & 7);
}

// Epilogue of a large-tile workgroup (every wave is past the operand ring, so the LDS is
// free): gate/up - SwiGLU x routing weight, bf16 h and/or its quantisation (hq_mode);
// down - bf16 outputs. acc[tt][wt]: register r of lane l = weight column 8(r/4) + 4(l/32) +
// r%4 of the wave's weight tile wt, token l%32 of its token tile tt. G: the workgroup shape
// (BM rows, WM x WN waves of TT x WT tiles).
template <class G, bool GATEUP>
DSV4_DEV void big_epilogue(const Dsv4GemmArgs& p, v16f (&acc)[G::TT][G::WT], uint8_t* lds, int c0, int wm, int wn,
                           int r32, int g2, const int* fr, const float* wr) {
  constexpr int kBM = G::BM, H = G::WT / 2;
  if (GATEUP) {
    const int cw = c0 + 32 * H * wn;  // this wave's first of 32 H intermediate columns
    // h for columns cw + 32 h + 8 q + 4 g2 + e of token tile tt, packed bf16 pairs
    uint32_t hp[G::TT][H][4][2];
    float rmax[G::TT][H];  // per 32-column block, this lane's half of it
#pragma unroll
    for (int tt = 0; tt < G::TT; ++tt)
#pragma unroll
      for (int h = 0; h < H; ++h) {
        float m = 0.0f;
#pragma unroll
        for (int q = 0; q < 4; ++q)
#pragma unroll
          for (int e = 0; e < 4; e += 2) {
            const int r = 4 * q + e;
            // gate (tile h) and up (tile H + h) of the same column, rounded to bf16
            const uint32_t gu0 = pk_bf16(acc[tt][h][r], acc[tt][H + h][r]);
            const uint32_t gu1 = pk_bf16(acc[tt][h][r + 1], acc[tt][H + h][r + 1]);
            const uint32_t hw = pk_bf16(big_swiglu(bf16_lo(gu0), bf16_hi(gu0), wr[tt], p.swiglu_limit),
                                        big_swiglu(bf16_lo(gu1), bf16_hi(gu1), wr[tt], p.swiglu_limit));
            hp[tt][h][q][e >> 1] = hw;
            m = fmaxf(m, fmaxf(fabsf(bf16_lo(hw)), fabsf(bf16_hi(hw))));
          }
        rmax[tt][h] = m;
      }
    if (!p.hq_skip_h && p.out) {
#pragma unroll
      for (int tt = 0; tt < G::TT; ++tt)
        if (fr[tt] < p.R)
#pragma unroll
          for (int h = 0; h < H; ++h)
#pragma unroll
            for (int q = 0; q < 4; ++q) {
              typedef uint32_t v2u __attribute__((ext_vector_type(2)));
              *(v2u*)(p.out + (int64_t)fr[tt] * p.N + cw + 32 * h + 8 * q + 4 * g2) =
                  v2u{hp[tt][h][q][0], hp[tt][h][q][1]};
            }
    }
    if (p.hq_mode == 2) {  // MXFP4 h: one 32-column block per (tt, h), half of it in each lane of a pair
#pragma unroll
      for (int tt = 0; tt < G::TT; ++tt)
#pragma unroll
        for (int h = 0; h < H; ++h) {
          const int k = dsv4::mxfp4_block_exp(max_pair(rmax[tt][h]), p.hq_rule);
          const float inv = dsv4::pow2f(-k);
          if (fr[tt] < p.R) {
            const int col = cw + 32 * h;
#pragma unroll
            for (int q = 0; q < 4; ++q) {
              const uint32_t w0 = hp[tt][h][q][0], w1 = hp[tt][h][q][1];
              const uint32_t nib = pk_fp4x2(bf16_lo(w0), bf16_hi(w0), inv, p.hq_rule) |
                                   pk_fp4x2(bf16_lo(w1), bf16_hi(w1), inv, p.hq_rule) << 8;
              *(uint16_t*)(p.hq_codes + (int64_t)fr[tt] * (p.N / 2) + (col + 8 * q + 4 * g2) / 2) = (uint16_t)nib;
            }
            if (g2 == 0) p.hq_scale[(int64_t)fr[tt] * (p.N / 32) + col / 32] = (uint8_t)(k + 127);
          }
        }
    } else if (p.hq_mode == 1) {  // FP8 h: one 128-column block per token, split over the WN waves of a row
      float* am = (float*)lds;     // [WN][kBM rows]
      float bm[G::TT];
#pragma unroll
      for (int tt = 0; tt < G::TT; ++tt) {
        float m = rmax[tt][0];
#pragma unroll
        for (int h = 1; h < H; ++h) m = fmaxf(m, rmax[tt][h]);
        if (g2 == 0) am[wn * kBM + (kBM / G::WM) * wm + 32 * tt + r32] = max_pair(m);
      }
      __syncthreads();
#pragma unroll
      for (int tt = 0; tt < G::TT; ++tt) {
        const int row = (kBM / G::WM) * wm + 32 * tt + r32;
        bm[tt] = am[row];
#pragma unroll
        for (int w = 1; w < G::WN; ++w) bm[tt] = fmaxf(bm[tt], am[w * kBM + row]);
      }
#pragma unroll
      for (int tt = 0; tt < G::TT; ++tt) {
        const int k = dsv4::fp8_block_exp(bm[tt]);
        const float inv = dsv4::pow2f(-k);
        if (fr[tt] < p.R) {
#pragma unroll
          for (int h = 0; h < H; ++h)
#pragma unroll
            for (int q = 0; q < 4; ++q) {
              const uint32_t w0 = hp[tt][h][q][0], w1 = hp[tt][h][q][1];
              *(uint32_t*)(p.hq_codes + (int64_t)fr[tt] * p.N + cw + 32 * h + 8 * q + 4 * g2) =
                  pk_fp8x4(bf16_lo(w0), bf16_hi(w0), bf16_lo(w1), bf16_hi(w1), inv);
            }
          if (g2 == 0)
#pragma unroll
            for (int h = 0; h < H; ++h) p.hq_scale[(int64_t)fr[tt] * (p.N / 32) + cw / 32 + h] = (uint8_t)(k + 127);
        }
      }
    }
  } else {
    const int cw = c0 + 32 * G::WT * wn;  // this wave's first output column
#pragma unroll
    for (int tt = 0; tt < G::TT; ++tt)
      if (fr[tt] < p.R)
#pragma unroll
        for (int wt = 0; wt < G::WT; ++wt)
#pragma unroll
          for (int q = 0; q < 4; ++q) {
            typedef uint32_t v2u __attribute__((ext_vector_type(2)));
            const int r = 4 * q;
            *(v2u*)(p.out + (int64_t)fr[tt] * p.N + cw + 32 * wt + 8 * q + 4 * g2) =
                v2u{pk_bf16(acc[tt][wt][r], acc[tt][wt][r + 1]), pk_bf16(acc[tt][wt][r + 2], acc[tt][wt][r + 3])};
          }
  }
}

template <int AFMT, bool HALF, bool GATEUP>
__global__ __launch_bounds__((Cfg<AFMT, HALF>::NT), (Cfg<AFMT, HALF>::WGS)) void moe_gemm_big_kernel(Dsv4GemmArgs p) {
  using C = Big<AFMT, HALF>;
  using G = Cfg<AFMT, HALF>;
  constexpr int kBM = G::BM, H = G::WT / 2;  // H: gate (and up) tiles per wave of gate/up
  __shared__ __attribute__((aligned(16))) uint8_t lds[C::LDS];
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // uniform: LDS-DMA destinations in SGPRs
  const int wm = wave / G::WN, wn = wave % G::WN;
  int hb, nt;
  big_tile_of_block(hb, nt);  // hb: this workgroup's share of a hot-layout block
  const int mb = hb / G::WGS;
  if (mb * kHB >= p.num_post_padded[0]) return;  // also every block of the grid's padding
  const int e = p.block_expert[mb];
  const Dsv4ExpertPtrs ex = p.experts[e];
  const bool have_w = GATEUP ? (ex.w1p && ex.w1s && ex.w3p && ex.w3s) : (ex.w2p && ex.w2s);
  const int NST = p.Kdim / kKS;
  const int wrow_bytes = p.Kdim / 2, srow = p.Kdim / 32;
  const int c0 = nt * (GATEUP ? 128 : 256);  // first intermediate column / output row of W2
  const int slot0 = mb * kHB + (hb % G::WGS) * kBM;

  // this lane's A piece per A load (stage 0): chunk wave * AV + v
  const uint8_t* a_src[C::AV];
#pragma unroll
  for (int v = 0; v < C::AV; ++v) {
    const int c = wave * C::AV + v;
    const int row = AFMT == 0 ? 16 * c + (lane >> 2) : 32 * c + (lane >> 1);
    const int piece = AFMT == 0 ? (lane & 3) ^ ((lane >> 4) & 3) : (lane & 1) ^ ((lane >> 4) & 1);
    const int f = p.sorted_ids[slot0 + row];
    const int arow = f < p.R ? f / p.a_row_div : 0;  // padding rows read row 0 (never stored)
    a_src[v] = p.a + (int64_t)arow * p.a_row_bytes + 16 * piece;
  }
  // this lane's weight piece per weight load: chunk wave * BV + v, slot `lane` =
  // 16-row tile q / 32 of the block, 16-byte half (q / 16) % 2, row q % 16
  const bool tiled = tiled_ptr(GATEUP ? ex.w1p : ex.w2p);
  const int bj = tiled ? 2048 : 4 * (kKS / 2), bg = tiled ? 256 : kKS / 2;
  const uint8_t* b_src[C::BV];
#pragma unroll
  for (int v = 0; v < C::BV; ++v) {
    const int q = (wave * C::BV + v) * 64 + lane;
    const int tile = q >> 5, ji = (q >> 4) & 1, r = q & 15;
    const int gtile = c0 / 16 + (GATEUP ? (tile & 7) : tile);
    const uint8_t* w = untag(GATEUP ? (tile < 8 ? ex.w1p : ex.w3p) : ex.w2p);
    b_src[v] = w + (tiled ? (int64_t)((gtile * (p.Kdim / 256)) * 2 + ji) * 1024 + 16 * r
                          : (int64_t)(16 * gtile + r) * wrow_bytes + 16 * ji);
  }
  // this lane's scale pieces (super-stage 0): piece q = (wave * SV + v) * 64 + lane of a
  // buffer: A rows for q < 2 kBM (half q / kBM, row q % kBM), weight rows after
  const uint8_t* sc_src[C::SV];
#pragma unroll
  for (int v = 0; v < C::SV; ++v) {
    const int q = (wave * C::SV + v) * 64 + lane;
    const bool arow_piece = q < 2 * kBM;
    const int w = arow_piece ? q : q - 2 * kBM, n = arow_piece ? kBM : kBN;
    const int half = w / n, row = w % n;
    if (arow_piece) {
      const int f = p.sorted_ids[slot0 + row];
      const int arow = f < p.R ? f / p.a_row_div : 0;
      sc_src[v] = p.a_scale + (int64_t)arow * srow + 16 * half;
    } else {
      const uint8_t* ws = GATEUP ? (row < 128 ? ex.w1s : ex.w3s) : ex.w2s;
      sc_src[v] = ws + (int64_t)(GATEUP ? c0 + (row & 127) : c0 + row) * srow + 16 * half;
    }
  }

  v16f acc[G::TT][G::WT];
#pragma unroll
  for (int mt = 0; mt < G::TT; ++mt)
#pragma unroll
    for (int nt = 0; nt < G::WT; ++nt) acc[mt][nt] = v16f{};
  const int r32 = lane & 31, g2 = lane >> 5;
  // flat index (and gate/up: routing weight) of this lane's token in each token tile
  int fr[G::TT];
  float wr[G::TT];
#pragma unroll
  for (int tt = 0; tt < G::TT; ++tt) {
    fr[tt] = p.sorted_ids[slot0 + (kBM / G::WM) * wm + 32 * tt + r32];
    wr[tt] = GATEUP && fr[tt] < p.R ? p.topk_w[fr[tt]] : 0.0f;
  }
  // first weight row of this wave's 32-row tile nt in the block
  // gate/up: tiles h < H = gate rows 32 (H wn + h).., tiles H + h = the matching up
  // rows 128 + 32 (H wn + h)..; down: output rows 32 (WT wn + nt)..
  int brow0[G::WT];
#pragma unroll
  for (int nt = 0; nt < G::WT; ++nt)
    brow0[nt] = GATEUP ? (nt / H) * 128 + 32 * (H * wn + nt % H) : 32 * (G::WT * wn + nt);
  // this lane's byte offsets inside a chunk (the swizzles of the layout comment)
  int a_lo, a_hi;
  if (AFMT == 0) {
    const int r = r32 & 15, x = (r >> 2) & 3;
    a_lo = 16 * (4 * r + (g2 ^ x));
    a_hi = 16 * (4 * r + ((2 + g2) ^ x));
  } else {
    a_lo = 16 * (2 * r32 + (g2 ^ ((r32 >> 3) & 1)));
    a_hi = 0;
  }
  const int b_lane = 16 * (32 * (r32 >> 4) + 16 * g2 + (r32 & 15));

  if (have_w) {  // uniform per workgroup: every wave reaches every barrier
    // Stage s lives in ring slot s % NB. Its fragments are read into registers during
    // stage s - 1 (while stage s - 1's MFMAs run), so once the barrier at the top of
    // stage s has passed - every wave holds its stage-s fragments - the slot takes the
    // loads of stage s + NB. The wait before that barrier lands stage s + 1 and leaves
    // the younger NB - 2 stages in flight. The loop has no branches (they would let
    // the compiler move the MFMAs away from their stage): past the last stage the loads
    // repeat stage NST - 1 into slots that are never read again, so every stage issues
    // the same number of loads and the wait count stays exact. Scales: super-stage ss
    // (stages 16ss..16ss+15) in LDS buffer ss % 2, loaded by LDS-DMA between stages
    // 16ss - 17 and 16ss - 16, once the buffer's previous super-stage has been read
    // (past the end: a repeat of the last one into the buffer no stage reads); those
    // loads are younger than the stage loads the next waits count, so the waits only
    // grow stricter. Scales in registers would make the compiler drain every load in
    // flight before storing them (it cannot see that 16 stages have passed). NST =
    // K / 64 is a multiple of 16.
    const int NSS = NST / kSS;
    big_dma_scales<AFMT, HALF>(lds, 0, sc_src, wave, 0);
#pragma unroll
    for (int t = 0; t < C::NB; ++t) big_dma_stage<AFMT, HALF>(lds + t * C::STAGE, a_src, b_src, wave, bj, bg, t);
    wait_loads_barrier<C::L * (C::NB - 1)>();
    BigFrag<AFMT, HALF> f0, f1;
    BigScl<AFMT, HALF> sr;   // raw scales of the next group of four stages
    BigSclW<AFMT, HALF> sw;  // this lane's scale words of the current group
    big_read<AFMT, HALF>(f0, lds, wm, brow0, r32, a_lo, a_hi, b_lane);
    big_read_scales<AFMT, HALF>(sr, lds + C::AS_OFF, 0, wm, brow0, r32);
    int slot = 0;  // ring slot of stage s
    // stage s (I = s % 4 of its scale group): multiply Fc (stage s), read stage s + 1
    // into Fn and, in the group's last stage, the next group's scales
    auto step = [&](auto I_, int s, BigFrag<AFMT, HALF>& Fc, BigFrag<AFMT, HALF>& Fn) __attribute__((always_inline)) {
      constexpr int I = decltype(I_)::value;
      const int nslot = slot + 1 == C::NB ? 0 : slot + 1;
      wait_loads_barrier<C::L * (C::NB - 2)>();
      if (I == 0) big_scale_words<AFMT, HALF>(sw, sr, g2);
      big_dma_stage<AFMT, HALF>(lds + slot * C::STAGE, a_src, b_src, wave, bj, bg, min(s + C::NB, NST - 1));
      const int s1 = s + 1;
      big_read<AFMT, HALF>(Fn, lds + nslot * C::STAGE, wm, brow0, r32, a_lo, a_hi, b_lane);
      if (I == 3) big_read_scales<AFMT, HALF>(sr, lds + C::AS_OFF + ((s1 / kSS) & 1) * C::SCL, s1 % kSS, wm, brow0, r32);
      big_mfma<AFMT, HALF, I>(acc, Fc, sw);
      big_sched<AFMT, HALF, I>();
      slot = nslot;
    };
    using I0 = std::integral_constant<int, 0>;
    using I1 = std::integral_constant<int, 1>;
    using I2 = std::integral_constant<int, 2>;
    using I3 = std::integral_constant<int, 3>;
#pragma unroll 1
    for (int ss = 0; ss < NSS; ++ss) {
      big_dma_scales<AFMT, HALF>(lds, (ss + 1) & 1, sc_src, wave, min(ss + 1, NSS - 1));
#pragma unroll 1
      for (int s = kSS * ss; s < kSS * (ss + 1); s += 4) {
        step(I0{}, s, f0, f1);
        step(I1{}, s + 1, f1, f0);
        step(I2{}, s + 2, f0, f1);
        step(I3{}, s + 3, f1, f0);
      }
    }
  }
  wait_loads_barrier<0>();  // every wave is done with the ring

  big_epilogue<G, GATEUP>(p, acc, lds, c0, wm, wn, r32, g2, fr, wr);
}


// ---- bf16 activations: the pure-bf16 variant ----------------------------------------
// Whole 256-row blocks x 256 weight rows, one workgroup of eight waves per CU (4 token
// groups x 2 weight groups: a wave owns 64 tokens x 128 weight rows = 2 x 4 tiles of
// 32 x 32), two waves per SIMD. Tokens (bf16, 128 bytes per row per 64-k stage) and the
// E2M1 weights (chunks as in the kernel above) move by LDS-DMA into a ring of three
// stages, the weight rows' E8M0 bytes per 1024-k super-stage. A stage's 64 k run as four
// 16-k chunks: in chunk c, lane (r, g) of weight tile wt turns the 4 bytes of its stage
// fragment at k 32 g + 8 c .. +8 into 8 bf16 with the hardware scaled converter (exact:
// an E2M1 value times 2^(s-127) is a bf16 value), takes the 8 bf16 of its token at the
// same k, and v_mfma_f32_32x32x16_bf16 sums the 16 k the two lane halves hold: both
// operands carry the same k in the same lane positions, so the instruction's own k order
// does not matter. Products are exact in fp32, sums fp32. A stage's fragments are read
// during the stage, after its barrier (two stages of loads stay in flight), the next
// chunk's tokens ahead of the current chunk's MFMAs.
//   token chunk c (1 KB): tokens 8c + r (r < 8); slot 8r + (p ^ r) holds bytes
//                         [16p, 16p + 16) of token r's stage (the 16 lanes of a read
//                         pass land on distinct bank groups, two tokens per group).
struct CfgBf {
  static constexpr int BM = 256, NT = 512, NW = 8, WM = 4, WN = 2, TT = 2, WT = 4;
};
namespace bfk {
constexpr int ACH = 32;                 // 1-KB token chunks per stage
constexpr int BCH = 8;                  // 1-KB weight chunks per stage
constexpr int STAGE = (ACH + BCH) * 1024;
constexpr int NB = 3;                   // ring slots
constexpr int SCL = 2 * kBN * 16;       // weight scales of one super-stage: [half][row] x 16 bytes
constexpr int AS_OFF = NB * STAGE;
constexpr int LDS = AS_OFF + 2 * SCL;
constexpr int AV = ACH / CfgBf::NW, BV = BCH / CfgBf::NW, L = AV + BV;  // loads per thread per stage
constexpr int SV = SCL / (CfgBf::NT * 16);                               // per super-stage
static_assert(LDS <= 160 * 1024, "ring and scale buffers fit the LDS");
static_assert(AV * CfgBf::NW == ACH && BV * CfgBf::NW == BCH && SV * CfgBf::NT * 16 == SCL, "loads per thread");
static_assert(L * (NB - 1) + SV < 64, "vmcnt holds 6 bits");
}  // namespace bfk

typedef __bf16 bfx8 __attribute__((ext_vector_type(8)));
typedef __bf16 bfx2 __attribute__((ext_vector_type(2)));

// 2^(b - 127) for an E8M0 byte b, branch-free: the byte is the fp32 exponent field
// (255 gives +inf, as the reference's pow does), except 0, the subnormal 2^-127
DSV4_DEV float e8m0_scale(uint32_t b) { return __uint_as_float(b ? b << 23 : 0x00400000u); }

// 8 bf16 of the 4 packed bytes w (low nibble first) times `scale` (exact)
DSV4_DEV bfx8 dequant8_bf16(uint32_t w, float scale) {
  const bfx2 a = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(w, scale, 0);
  const bfx2 b = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(w, scale, 1);
  const bfx2 c = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(w, scale, 2);
  const bfx2 d = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(w, scale, 3);
  return bfx8{a[0], a[1], b[0], b[1], c[0], c[1], d[0], d[1]};
}

template <bool GATEUP>
__global__ __launch_bounds__(512, 1) void moe_gemm_big_bf16_kernel(Dsv4GemmArgs p) {
  using G = CfgBf;
  constexpr int kBM = G::BM;
  __shared__ __attribute__((aligned(16))) uint8_t lds[bfk::LDS];
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // uniform: LDS-DMA destinations in SGPRs
  const int wm = wave / G::WN, wn = wave % G::WN;
  int mb, nt;
  big_tile_of_block(mb, nt);
  if (mb * kHB >= p.num_post_padded[0]) return;  // also every block of the grid's padding
  const int e = p.block_expert[mb];
  const Dsv4ExpertPtrs ex = p.experts[e];
  const bool have_w = GATEUP ? (ex.w1p && ex.w1s && ex.w3p && ex.w3s) : (ex.w2p && ex.w2s);
  const int NST = p.Kdim / kKS;
  const int wrow_bytes = p.Kdim / 2, srow = p.Kdim / 32;
  const int c0 = nt * (GATEUP ? 128 : 256);  // first intermediate column / output row of W2
  const int slot0 = mb * kHB;

  // this lane's token piece per token load (stage 0): chunk wave * AV + v, token 8c + lane / 8
  const uint8_t* a_src[bfk::AV];
#pragma unroll
  for (int v = 0; v < bfk::AV; ++v) {
    const int c = wave * bfk::AV + v, r = lane >> 3;
    const int f = p.sorted_ids[slot0 + 8 * c + r];
    const int arow = f < p.R ? f / p.a_row_div : 0;  // padding rows read row 0 (never stored)
    a_src[v] = p.a + (int64_t)arow * p.a_row_bytes + 16 * ((lane & 7) ^ r);
  }
  // weight pieces as in moe_gemm_big_kernel
  const bool tiled = tiled_ptr(GATEUP ? ex.w1p : ex.w2p);
  const int bj = tiled ? 2048 : 4 * (kKS / 2), bg = tiled ? 256 : kKS / 2;
  const uint8_t* b_src[bfk::BV];
#pragma unroll
  for (int v = 0; v < bfk::BV; ++v) {
    const int q = (wave * bfk::BV + v) * 64 + lane;
    const int tile = q >> 5, ji = (q >> 4) & 1, r = q & 15;
    const int gtile = c0 / 16 + (GATEUP ? (tile & 7) : tile);
    const uint8_t* w = untag(GATEUP ? (tile < 8 ? ex.w1p : ex.w3p) : ex.w2p);
    b_src[v] = w + (tiled ? (int64_t)((gtile * (p.Kdim / 256)) * 2 + ji) * 1024 + 16 * r
                          : (int64_t)(16 * gtile + r) * wrow_bytes + 16 * ji);
  }
  // this lane's weight-scale piece per super-stage: half q / kBN, row q % kBN of a buffer
  const uint8_t* sc_src[bfk::SV];
#pragma unroll
  for (int v = 0; v < bfk::SV; ++v) {
    const int q = (wave * bfk::SV + v) * 64 + lane;
    const int half = q / kBN, row = q % kBN;
    const uint8_t* ws = GATEUP ? (row < 128 ? ex.w1s : ex.w3s) : ex.w2s;
    sc_src[v] = ws + (int64_t)(GATEUP ? c0 + (row & 127) : c0 + row) * srow + 16 * half;
  }

  v16f acc[G::TT][G::WT];
#pragma unroll
  for (int tt = 0; tt < G::TT; ++tt)
#pragma unroll
    for (int wt = 0; wt < G::WT; ++wt) acc[tt][wt] = v16f{};
  const int r32 = lane & 31, g2 = lane >> 5;
  int fr[G::TT];
  float wr[G::TT];
#pragma unroll
  for (int tt = 0; tt < G::TT; ++tt) {
    fr[tt] = p.sorted_ids[slot0 + (kBM / G::WM) * wm + 32 * tt + r32];
    wr[tt] = GATEUP && fr[tt] < p.R ? p.topk_w[fr[tt]] : 0.0f;
  }
  constexpr int H = G::WT / 2;
  int brow0[G::WT];
#pragma unroll
  for (int wt = 0; wt < G::WT; ++wt)
    brow0[wt] = GATEUP ? (wt / H) * 128 + 32 * (H * wn + wt % H) : 32 * (G::WT * wn + wt);
  const int b_lane = 16 * (32 * (r32 >> 4) + 16 * g2 + (r32 & 15));
  // this lane's token in each tile: its chunk and row in the chunk (tiles start on chunk edges)
  int tchunk[G::TT];
#pragma unroll
  for (int tt = 0; tt < G::TT; ++tt) tchunk[tt] = ((kBM / G::WM) * wm + 32 * tt + r32) >> 3;
  const int tr = r32 & 7;

  if (have_w) {  // uniform per workgroup: every wave reaches every barrier
    // Stage s lives in ring slot s % NB. At the top of stage s this wave waits until its
    // own loads of stage s have landed (those of stage s + 1 may still fly), then the
    // barrier: every wave's share of stage s is in the LDS and every wave is done reading
    // stage s - 1, whose slot takes the loads of stage s + NB - 1. Past the last stage the
    // loads repeat stage NST - 1 into slots never read again (no branch in the loop).
    // Scales: super-stage ss in buffer ss % 2, loaded after the barrier of stage 16 ss
    // (stage 16 ss - 1, the last reader of that buffer's previous super-stage, is done).
    const int NSS = NST / kSS;
#pragma unroll
    for (int v = 0; v < bfk::SV; ++v) dma16(sc_src[v], lds + bfk::AS_OFF + (wave * bfk::SV + v) * 1024);
#pragma unroll
    for (int t = 0; t < bfk::NB - 1; ++t) {
#pragma unroll
      for (int v = 0; v < bfk::AV; ++v) dma16(a_src[v] + t * 128, lds + t * bfk::STAGE + (wave * bfk::AV + v) * 1024);
      const int boff = (t >> 2) * bj + (t & 3) * bg;
#pragma unroll
      for (int v = 0; v < bfk::BV; ++v)
        dma16(b_src[v] + boff, lds + t * bfk::STAGE + (bfk::ACH + wave * bfk::BV + v) * 1024);
    }
    int slot = 0, fill = bfk::NB - 1;
    // weight scales of the current group of four stages, this lane's bytes (g2) moved to
    // bits 16 i (stage 4j + i): one 8-byte read per tile per group (the row's bytes
    // 2 (s % 8) .. + 7 of its piece (s % 16) / 8 hold both g2's bytes of the group)
    uint64_t sr[G::WT];
    auto step = [&](auto I_, int s) __attribute__((always_inline)) {
      constexpr int I = decltype(I_)::value;  // s % 4
      wait_loads_barrier<bfk::L * (bfk::NB - 2)>();
      const int sl = min(s + bfk::NB - 1, NST - 1);
      uint8_t* fs = lds + fill * bfk::STAGE;
#pragma unroll
      for (int v = 0; v < bfk::AV; ++v) dma16(a_src[v] + sl * 128, fs + (wave * bfk::AV + v) * 1024);
      const int boff = (sl >> 2) * bj + (sl & 3) * bg;
#pragma unroll
      for (int v = 0; v < bfk::BV; ++v) dma16(b_src[v] + boff, fs + (bfk::ACH + wave * bfk::BV + v) * 1024);
      const uint8_t* Ls = lds + slot * bfk::STAGE;
      const uint8_t* S = lds + bfk::AS_OFF + ((s / kSS) & 1) * bfk::SCL;
      if (I == 0) {
        const int off = 2 * (s & 7), half = (s % kSS) >> 3;
#pragma unroll
        for (int wt = 0; wt < G::WT; ++wt)
          sr[wt] = *(const uint64_t*)(S + (half * kBN + brow0[wt] + r32) * 16 + off) >> (8 * g2);
      }
      v4i wf[G::WT];
      float wsc[G::WT];
#pragma unroll
      for (int wt = 0; wt < G::WT; ++wt) {
        wf[wt] = *(const v4i*)(Ls + (bfk::ACH + brow0[wt] / 32) * 1024 + b_lane);
        wsc[wt] = e8m0_scale((uint32_t)(sr[wt] >> (16 * I)) & 0xffu);
      }
      bfx8 tk[2][G::TT];
#pragma unroll
      for (int tt = 0; tt < G::TT; ++tt)
        tk[0][tt] = *(const bfx8*)(Ls + tchunk[tt] * 1024 + 16 * (8 * tr + ((4 * g2) ^ tr)));
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        if (c < 3) {
#pragma unroll
          for (int tt = 0; tt < G::TT; ++tt)
            tk[(c + 1) & 1][tt] = *(const bfx8*)(Ls + tchunk[tt] * 1024 + 16 * (8 * tr + ((4 * g2 + c + 1) ^ tr)));
        }
        bfx8 wb[G::WT];
#pragma unroll
        for (int wt = 0; wt < G::WT; ++wt) wb[wt] = dequant8_bf16((uint32_t)wf[wt][c], wsc[wt]);
#pragma unroll
        for (int tt = 0; tt < G::TT; ++tt)
#pragma unroll
          for (int wt = 0; wt < G::WT; ++wt)
            acc[tt][wt] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(wb[wt], tk[c & 1][tt], acc[tt][wt], 0, 0, 0);
      }
      slot = slot + 1 == bfk::NB ? 0 : slot + 1;
      fill = fill + 1 == bfk::NB ? 0 : fill + 1;
    };
    using I0 = std::integral_constant<int, 0>;
    using I1 = std::integral_constant<int, 1>;
    using I2 = std::integral_constant<int, 2>;
    using I3 = std::integral_constant<int, 3>;
    auto group = [&](int s) __attribute__((always_inline)) {
      step(I0{}, s);
      step(I1{}, s + 1);
      step(I2{}, s + 2);
      step(I3{}, s + 3);
    };
#pragma unroll 1
    for (int ss = 0; ss < NSS; ++ss) {
      group(kSS * ss);
      // the next super-stage's scales, once every wave is past stage 16 ss - 1 (the last
      // reader of that buffer); older than the loads the waits of stages 16 ss + 4 ..
      // leave in flight, so they have landed by stage 16 ss + 16
#pragma unroll
      for (int v = 0; v < bfk::SV; ++v)
        dma16(sc_src[v] + min(ss + 1, NSS - 1) * 32, lds + bfk::AS_OFF + ((ss + 1) & 1) * bfk::SCL + (wave * bfk::SV + v) * 1024);
#pragma unroll 1
      for (int s = kSS * ss + 4; s < kSS * (ss + 1); s += 4) group(s);
    }
  }
  wait_loads_barrier<0>();  // every wave is done with the ring
  big_epilogue<G, GATEUP>(p, acc, lds, c0, wm, wn, r32, g2, fr, wr);
}

}  // namespace

// K in whole 1024-k scale super-stages (the K = 512 GEMMs keep the 64-row kernel).
bool moe_gemm_big_supported(int kdim, int n, bool gateup) {
  return kdim >= 1024 && kdim % 1024 == 0 && n % (gateup ? 128 : 256) == 0;
}

template <int AFMT, bool HALF>
static void launch_big(const Dsv4GemmArgs& a, bool gateup, int ntiles, hipStream_t st) {
  using G = Cfg<AFMT, HALF>;
  // workgroups' M extent: WGS per hot-layout block, in whole groups of 32 for the XCD
  // grouping of big_tile_of_block
  const int m = G::WGS * a.max_blocks;
  const dim3 grid(ntiles, ntiles % 8 == 0 ? (m + 31) / 32 * 32 : m);
  if (gateup) hipLaunchKernelGGL((moe_gemm_big_kernel<AFMT, HALF, true>), grid, dim3(G::NT), 0, st, a);
  else hipLaunchKernelGGL((moe_gemm_big_kernel<AFMT, HALF, false>), grid, dim3(G::NT), 0, st, a);
}

hipError_t launch_moe_gemm_big(const Dsv4GemmArgs& a, bool gateup, hipStream_t st) {
  if (a.block_m != kHB || !moe_gemm_big_supported(a.Kdim, a.N, gateup)) return hipErrorInvalidValue;
  if (a.max_blocks <= 0) return hipSuccess;
  const int ntiles = a.N / (gateup ? 128 : 256);
  if (a.afmt == kAfmtBf16) {  // pure bf16: whole blocks, bf16 MFMA on in-register dequantised weights
    if (gateup && a.hq_mode) return hipErrorInvalidValue;
    const dim3 grid(ntiles, ntiles % 8 == 0 ? (a.max_blocks + 31) / 32 * 32 : a.max_blocks);
    if (gateup) hipLaunchKernelGGL((moe_gemm_big_bf16_kernel<true>), grid, dim3(CfgBf::NT), 0, st, a);
    else hipLaunchKernelGGL((moe_gemm_big_bf16_kernel<false>), grid, dim3(CfgBf::NT), 0, st, a);
    return hipGetLastError();
  }
  // workgroup shape (Cfg): half blocks for E4M3, and for E2M1 while the layer's rows
  // are too few to fill the CUs with whole blocks
  if (a.afmt == 0) launch_big<0, true>(a, gateup, ntiles, st);
  else if (a.R < 32768) launch_big<1, true>(a, gateup, ntiles, st);
  else launch_big<1, false>(a, gateup, ntiles, st);
  return hipGetLastError();
}
