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
// Work decomposition: one workgroup = 4 waves = one M block (16 padded rows of
// one expert, from moe_align) x one N tile. The A rows are gathered on load
// through sorted_ids (no permuted copy of x is materialised). Every wave owns
// two 16x16 output tiles and streams their weight rows straight from HBM into
// registers (each weight byte is used by exactly one wave, so LDS staging would
// only add traffic); the next 512-wide K step is prefetched while the current
// one is multiplied.
//
// K mapping. One 512-wide K step is 4 MFMAs (ji = 0..3) of 128 logical k each.
// Logical 32-block b of MFMA ji is global 32-block 16*jo + 4*b + ji, so the
// lane holding block b of a B row (lane group g = b) reads 64 contiguous bytes
// (4 x 16 B) per K step and its 4 scale bytes are one aligned dword.
// Operand layouts (measured on gfx950):
//   E2M1 A/B: lane (r = l%16, g = l/16) holds logical k [32g, 32g+32) of row r
//             in 16 bytes, low nibble first.
//   E4M3 A  : lane (r, g) holds logical k [16g, 16g+16) in bytes 0-15 and
//             [64+16g, 64+16g+16) in bytes 16-31.
//   scales  : lane (r, g) supplies the E8M0 of logical block g of its row/col.
//   C       : lane l holds C[4*(l/16)+i][l%16], i = 0..3.
#include "common.h"
#include "kernels.h"

namespace {

typedef int v8i __attribute__((ext_vector_type(8)));
typedef float v4f __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

constexpr int kBM = 16;

template <int AFMT>
struct AFrag {
  u32x4 v[AFMT == 0 ? 8 : 4];
  uint32_t s;
};
struct BFrag {
  u32x4 v[2][4];
  uint32_t s[2];
};

template <int AFMT>
DSV4_DEV void load_a(AFrag<AFMT>& a, const uint8_t* abase, const uint8_t* asbase, bool ok, int jo, int g) {
  if (!ok) {
#pragma unroll
    for (int i = 0; i < (AFMT == 0 ? 8 : 4); ++i) a.v[i] = u32x4{0u, 0u, 0u, 0u};
    a.s = 0x7f7f7f7fu;
    return;
  }
  if (AFMT == 1) {
    const u32x4* p = (const u32x4*)(abase + (int64_t)jo * 256 + g * 64);
#pragma unroll
    for (int ji = 0; ji < 4; ++ji) a.v[ji] = p[ji];
  } else {
    const uint8_t* p = abase + (int64_t)jo * 512 + 16 * (g & 1);
#pragma unroll
    for (int ji = 0; ji < 4; ++ji) {
      a.v[2 * ji] = *(const u32x4*)(p + 128 * (g >> 1) + 32 * ji);
      a.v[2 * ji + 1] = *(const u32x4*)(p + 128 * (2 + (g >> 1)) + 32 * ji);
    }
  }
  a.s = *(const uint32_t*)(asbase + jo * 16 + 4 * g);
}

DSV4_DEV void load_b(BFrag& b, const uint8_t* b0, const uint8_t* bs0, const uint8_t* b1, const uint8_t* bs1,
                     int jo, int g) {
  const u32x4* p0 = (const u32x4*)(b0 + (int64_t)jo * 256 + g * 64);
  const u32x4* p1 = (const u32x4*)(b1 + (int64_t)jo * 256 + g * 64);
#pragma unroll
  for (int ji = 0; ji < 4; ++ji) {
    b.v[0][ji] = __builtin_nontemporal_load(p0 + ji);
    b.v[1][ji] = __builtin_nontemporal_load(p1 + ji);
  }
  b.s[0] = *(const uint32_t*)(bs0 + jo * 16 + 4 * g);
  b.s[1] = *(const uint32_t*)(bs1 + jo * 16 + 4 * g);
}

template <int AFMT, int JI>
DSV4_DEV void mfma_step(v4f* acc, const AFrag<AFMT>& a, const BFrag& b) {
  v8i av;
  if (AFMT == 1) {
    av = v8i{(int)a.v[JI].x, (int)a.v[JI].y, (int)a.v[JI].z, (int)a.v[JI].w, 0, 0, 0, 0};
  } else {
    const u32x4 lo = a.v[2 * JI], hi = a.v[2 * JI + 1];
    av = v8i{(int)lo.x, (int)lo.y, (int)lo.z, (int)lo.w, (int)hi.x, (int)hi.y, (int)hi.z, (int)hi.w};
  }
  const int sa = (int)((a.s >> (8 * JI)) & 0xffu);
#pragma unroll
  for (int t = 0; t < 2; ++t) {
    const v8i bv = v8i{(int)b.v[t][JI].x, (int)b.v[t][JI].y, (int)b.v[t][JI].z, (int)b.v[t][JI].w, 0, 0, 0, 0};
    const int sb = (int)((b.s[t] >> (8 * JI)) & 0xffu);
    acc[t] = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(av, bv, acc[t], AFMT == 0 ? 0 : 4, 4, 0, sa, 0, sb);
  }
}

template <int AFMT>
DSV4_DEV void mfma_kstep(v4f* acc, const AFrag<AFMT>& a, const BFrag& b) {
  mfma_step<AFMT, 0>(acc, a, b);
  mfma_step<AFMT, 1>(acc, a, b);
  mfma_step<AFMT, 2>(acc, a, b);
  mfma_step<AFMT, 3>(acc, a, b);
}

template <int AFMT, bool GATEUP>
__global__ __launch_bounds__(256) void moe_gemm_kernel(Dsv4GemmArgs p) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int mb = blockIdx.y;
  if (mb * kBM >= p.num_post_padded[0]) return;
  const int e = p.block_expert[mb];
  const Dsv4ExpertPtrs ex = p.experts[e];
  const int r16 = lane & 15, g = lane >> 4;
  // An expert whose weights are not in the table contributes zeros (never read null).
  const bool have_w = GATEUP ? (ex.w1p && ex.w1s && ex.w3p && ex.w3s) : (ex.w2p && ex.w2s);

  // A operand row of this lane (gather on load).
  const int f_in = p.sorted_ids[mb * kBM + r16];
  const bool a_ok = f_in < p.R;
  const int64_t arow = a_ok ? (int64_t)(f_in / p.a_row_div) : 0;
  const uint8_t* abase = p.a + arow * p.a_row_bytes;
  const uint8_t* asbase = p.a_scale + arow * (int64_t)(p.Kdim / 32);

  // B rows of this lane's two 16-row weight tiles.
  const int64_t brow_bytes = p.Kdim / 2, bsrow = p.Kdim / 32;
  int col0;
  const uint8_t *b0, *bs0, *b1, *bs1;
  if (GATEUP) {
    col0 = blockIdx.x * 64 + wave * 16;  // output column of gate tile and up tile
    b0 = ex.w1p + (int64_t)(col0 + r16) * brow_bytes;
    bs0 = ex.w1s + (int64_t)(col0 + r16) * bsrow;
    b1 = ex.w3p + (int64_t)(col0 + r16) * brow_bytes;
    bs1 = ex.w3s + (int64_t)(col0 + r16) * bsrow;
  } else {
    col0 = blockIdx.x * 128 + wave * 32;
    b0 = ex.w2p + (int64_t)(col0 + r16) * brow_bytes;
    bs0 = ex.w2s + (int64_t)(col0 + r16) * bsrow;
    b1 = ex.w2p + (int64_t)(col0 + 16 + r16) * brow_bytes;
    bs1 = ex.w2s + (int64_t)(col0 + 16 + r16) * bsrow;
  }

  v4f acc[2] = {v4f{0.f, 0.f, 0.f, 0.f}, v4f{0.f, 0.f, 0.f, 0.f}};
  const int njo = have_w ? p.Kdim / 512 : 0;
  AFrag<AFMT> a0, a1;
  BFrag w0, w1;
  if (njo > 0) {
    load_a<AFMT>(a0, abase, asbase, a_ok, 0, g);
    load_b(w0, b0, bs0, b1, bs1, 0, g);
  }
  for (int jo = 0; jo < njo; jo += 2) {
    if (jo + 1 < njo) {
      load_a<AFMT>(a1, abase, asbase, a_ok, jo + 1, g);
      load_b(w1, b0, bs0, b1, bs1, jo + 1, g);
    }
    mfma_kstep<AFMT>(acc, a0, w0);
    if (jo + 2 < njo) {
      load_a<AFMT>(a0, abase, asbase, a_ok, jo + 2, g);
      load_b(w0, b0, bs0, b1, bs1, jo + 2, g);
    }
    if (jo + 1 < njo) mfma_kstep<AFMT>(acc, a1, w1);
  }

  // Epilogue: lane holds rows 4*g + i (i = 0..3) of column r16 of each tile.
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int f = p.sorted_ids[mb * kBM + 4 * g + i];
    if (f >= p.R) continue;
    if (GATEUP) {
      // deepseek_v4.py:177-187: bf16 GEMM outputs -> fp32, clamp, silu(gate)*up*w
      float gt = dsv4::bf16_to_f32(dsv4::f32_to_bf16(acc[0][i]));
      float up = dsv4::bf16_to_f32(dsv4::f32_to_bf16(acc[1][i]));
      if (p.swiglu_limit > 0.0f) {
        up = fminf(fmaxf(up, -p.swiglu_limit), p.swiglu_limit);
        gt = fminf(gt, p.swiglu_limit);
      }
      const float h = gt / (1.0f + __expf(-gt)) * up * p.topk_w[f];
      p.out[(int64_t)f * p.N + col0 + r16] = (uint16_t)dsv4::f32_to_bf16(h);
    } else {
      p.out[(int64_t)f * p.N + col0 + r16] = (uint16_t)dsv4::f32_to_bf16(acc[0][i]);
      p.out[(int64_t)f * p.N + col0 + 16 + r16] = (uint16_t)dsv4::f32_to_bf16(acc[1][i]);
    }
  }
}

}  // namespace

hipError_t launch_moe_gemm_gateup(const Dsv4GemmArgs& a, hipStream_t st) {
  dim3 grid(a.N / 64, a.max_blocks);
  if (a.afmt == 0)
    hipLaunchKernelGGL((moe_gemm_kernel<0, true>), grid, dim3(256), 0, st, a);
  else
    hipLaunchKernelGGL((moe_gemm_kernel<1, true>), grid, dim3(256), 0, st, a);
  return hipGetLastError();
}

hipError_t launch_moe_gemm_down(const Dsv4GemmArgs& a, hipStream_t st) {
  dim3 grid(a.N / 128, a.max_blocks);
  if (a.afmt == 0)
    hipLaunchKernelGGL((moe_gemm_kernel<0, false>), grid, dim3(256), 0, st, a);
  else
    hipLaunchKernelGGL((moe_gemm_kernel<1, false>), grid, dim3(256), 0, st, a);
  return hipGetLastError();
}
