// extern "C" entry points of libdsv4hip.so (declared in include/dsv4_moe.h).
//
// Every entry point validates its arguments on the host before anything is
// launched, returns DSV4_OK or a negative status, and leaves a message for
// dsv4_last_error(). Device buffers are owned by the caller; nothing here
// allocates device memory except the slot manager (slots.cpp). Kernels are
// enqueued on the caller's stream and nothing synchronises.
#include <hip/hip_runtime.h>
#include <stdarg.h>
#include <stdio.h>
#include <string.h>
#include <stdlib.h>
#include <algorithm>
#include <mutex>
#include <string>

#include "common.h"
#include "kernels.h"
#include "../../include/dsv4_moe.h"

static thread_local std::string g_last_error;

int dsv4_fail(int code, const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  g_last_error = buf;
  return code;
}

static int hip_status(hipError_t e, const char* where) {
  if (e == hipSuccess) return DSV4_OK;
  return dsv4_fail(DSV4_ERR_HIP, "%s: %s", where, hipGetErrorString(e));
}

#define REQUIRE(cond, code, ...) \
  do {                           \
    if (!(cond)) return dsv4_fail(code, __VA_ARGS__); \
  } while (0)

static inline bool aligned(const void* p, uintptr_t a) { return ((uintptr_t)p & (a - 1)) == 0; }
// Up to this many routed entries one workgroup aligns them (one launch, fused
// with the quantisation of x in the layer); above it, the chunked two-launch align.
static constexpr int64_t kAlignSmallRows = 2048;
static inline int64_t round_up(int64_t v, int64_t a) { return (v + a - 1) / a * a; }

extern "C" {

const char* dsv4_last_error(void) { return g_last_error.c_str(); }

int dsv4_abi_version(void) { return DSV4_ABI_VERSION; }

int dsv4_probe_mfma_rate(int shape, int fmt_a, int fmt_b, int n_wg, int iters, float* out, double* flop,
                         void* stream) {
  REQUIRE(shape == 0 || shape == 1, DSV4_ERR_UNSUPPORTED, "mfma probe: shape %d (0: 16x16x128, 1: 32x32x64)", shape);
  REQUIRE((fmt_a == 4 && fmt_b == 4) || (fmt_a == 0 && fmt_b == 4) || (fmt_a == 0 && fmt_b == 0),
          DSV4_ERR_UNSUPPORTED, "mfma probe: format pair (%d, %d)", fmt_a, fmt_b);
  REQUIRE(n_wg > 0 && iters > 0, DSV4_ERR_SHAPE, "mfma probe: n_wg=%d iters=%d", n_wg, iters);
  REQUIRE(out, DSV4_ERR_NULL, "mfma probe: null output");
  return hip_status(launch_mfma_rate_probe(shape, fmt_a, fmt_b, n_wg, iters, out, flop, (hipStream_t)stream),
                    "mfma probe launch");
}

// ---------------------------------------------------------------------------
int dsv4_mxfp4_dequant_bf16(const void* packed, const void* scales, void* out, int64_t n_rows, int64_t k,
                            void* stream) {
  REQUIRE(n_rows >= 0 && k >= 0, DSV4_ERR_SHAPE, "dequant: negative size");
  REQUIRE(k % 32 == 0, DSV4_ERR_SHAPE, "dequant: K=%lld must be a multiple of 32", (long long)k);
  if (n_rows == 0 || k == 0) return DSV4_OK;
  REQUIRE(packed && scales && out, DSV4_ERR_NULL, "dequant: null pointer");
  REQUIRE(aligned(packed, 4) && aligned(out, 16), DSV4_ERR_SHAPE, "dequant: misaligned buffer");
  return hip_status(launch_mxfp4_dequant((const uint8_t*)packed, (const uint8_t*)scales, (uint16_t*)out,
                                         n_rows * k, (hipStream_t)stream),
                    "dequant launch");
}

int dsv4_mxfp4_dequant_bf16_multi(int n, const void* const* packed, const void* const* scales, void* const* out,
                                  const int64_t* n_rows, const int64_t* k, void* stream) {
  REQUIRE(n >= 1 && n <= kDequantMaxJobs, DSV4_ERR_UNSUPPORTED, "dequant multi: %d tensors (1..%d)", n,
          kDequantMaxJobs);
  REQUIRE(packed && scales && out && n_rows && k, DSV4_ERR_NULL, "dequant multi: null host array");
  Dsv4DequantJobs J{};
  J.n = n;
  for (int i = 0; i < n; ++i) {
    REQUIRE(n_rows[i] >= 0 && k[i] >= 0, DSV4_ERR_SHAPE, "dequant multi: tensor %d has a negative size", i);
    REQUIRE(k[i] % 32 == 0, DSV4_ERR_SHAPE, "dequant multi: tensor %d: K=%lld must be a multiple of 32", i,
            (long long)k[i]);
    const uintptr_t pp = (uintptr_t)packed[i];
    const bool tiled = (pp & DSV4_TILED_WEIGHTS) != 0;  // MFMA-tiled layout, tagged as in dsv4_expert_ptrs
    const void* src = (const void*)(pp & ~(uintptr_t)DSV4_TILED_WEIGHTS);
    REQUIRE(!tiled || (n_rows[i] % 16 == 0 && k[i] % 256 == 0), DSV4_ERR_SHAPE,
            "dequant multi: tensor %d: tiled weights need rows %% 16 == 0 and K %% 256 == 0", i);
    const int64_t chunks = n_rows[i] * (k[i] / 32);
    if (chunks > 0) {
      REQUIRE(src && scales[i] && out[i], DSV4_ERR_NULL, "dequant multi: tensor %d: null pointer", i);
      REQUIRE(aligned(src, 16) && aligned(out[i], 16), DSV4_ERR_SHAPE,
              "dequant multi: tensor %d: packed and out need 16-byte alignment", i);
    }
    J.packed[i] = (const uint8_t*)src;
    J.scales[i] = (const uint8_t*)scales[i];
    J.out[i] = (uint16_t*)out[i];
    J.kc[i] = k[i] / 32;
    J.tiled[i] = tiled ? 1 : 0;
    J.start[i + 1] = J.start[i] + chunks;
  }
  return hip_status(launch_mxfp4_dequant_multi(J, (hipStream_t)stream), "dequant multi launch");
}

int dsv4_mxfp4_tile_weights(const void* src, void* dst, int64_t n_rows, int64_t k, int inverse, void* stream) {
  REQUIRE(n_rows >= 0 && k >= 0, DSV4_ERR_SHAPE, "tile weights: negative size");
  REQUIRE(n_rows % 16 == 0 && k % 256 == 0, DSV4_ERR_SHAPE,
          "tile weights: [%lld, %lld] needs rows %% 16 == 0 and K %% 256 == 0", (long long)n_rows, (long long)k);
  REQUIRE(inverse == 0 || inverse == 1, DSV4_ERR_UNSUPPORTED, "tile weights: inverse must be 0 or 1");
  if (n_rows == 0 || k == 0) return DSV4_OK;
  REQUIRE(src && dst, DSV4_ERR_NULL, "tile weights: null pointer");
  REQUIRE(aligned(src, 16) && aligned(dst, 16), DSV4_ERR_SHAPE, "tile weights: buffers must be 16-byte aligned");
  const int64_t bytes = n_rows * (k / 2);
  const uintptr_t s0 = (uintptr_t)src, d0 = (uintptr_t)dst;
  REQUIRE(s0 + bytes <= d0 || d0 + bytes <= s0, DSV4_ERR_SHAPE, "tile weights: src and dst overlap");
  return hip_status(launch_mxfp4_tile((const uint8_t*)src, (uint8_t*)dst, n_rows, k, inverse, (hipStream_t)stream),
                    "tile weights launch");
}

int dsv4_mxfp4_tile_host(const void* src, void* dst, int64_t n_rows, int64_t k) {
  REQUIRE(n_rows >= 0 && k >= 0, DSV4_ERR_SHAPE, "tile weights (host): negative size");
  REQUIRE(n_rows % 16 == 0 && k % 256 == 0, DSV4_ERR_SHAPE,
          "tile weights (host): [%lld, %lld] needs rows %% 16 == 0 and K %% 256 == 0", (long long)n_rows,
          (long long)k);
  if (n_rows == 0 || k == 0) return DSV4_OK;
  REQUIRE(src && dst, DSV4_ERR_NULL, "tile weights (host): null pointer");
  const uint8_t* s = (const uint8_t*)src;
  uint8_t* d = (uint8_t*)dst;
  const int64_t row_bytes = k / 2, nst = k / 256;
  REQUIRE(s + n_rows * row_bytes <= d || d + n_rows * row_bytes <= s, DSV4_ERR_SHAPE,
          "tile weights (host): src and dst overlap");
  for (int64_t nt = 0; nt < n_rows / 16; ++nt)  // destination order: tile, stage, MFMA, lane
    for (int64_t j = 0; j < nst; ++j)
      for (int ji = 0; ji < 2; ++ji)
        for (int g = 0; g < 4; ++g)
          for (int r = 0; r < 16; ++r, d += 16)
            memcpy(d, s + (16 * nt + r) * row_bytes + 128 * j + 32 * g + 16 * ji, 16);
  return DSV4_OK;
}

int dsv4_mxfp4_gemv_bf16(const void* x, int m, const void* packed, const void* scales, int n, int k, void* y,
                         void* stream) {
  REQUIRE(m >= 0 && n >= 0 && k >= 0, DSV4_ERR_SHAPE, "gemv: negative size");
  REQUIRE(m <= 16, DSV4_ERR_UNSUPPORTED, "gemv: %d activation rows (at most 16)", m);
  REQUIRE(k > 0 && k % 32 == 0, DSV4_ERR_SHAPE, "gemv: K=%d must be a positive multiple of 32", k);
  if (m == 0 || n == 0) return DSV4_OK;
  REQUIRE(x && packed && scales && y, DSV4_ERR_NULL, "gemv: null pointer");
  REQUIRE(aligned(x, 16) && aligned(packed, 16), DSV4_ERR_SHAPE, "gemv: x and packed need 16-byte alignment");
  return hip_status(launch_mxfp4_gemv((const uint16_t*)x, m, (const uint8_t*)packed, (const uint8_t*)scales, n, k,
                                      (uint16_t*)y, (hipStream_t)stream),
                    "gemv launch");
}

int dsv4_fp8_act_quant(const void* x, int64_t rows, int64_t cols, int block_size, void* rt, void* codes,
                       void* scale_f32, void* scale_e8m0x4, void* stream) {
  REQUIRE(rows >= 0 && cols >= 0, DSV4_ERR_SHAPE, "act_quant: negative size");
  REQUIRE(block_size == 128, DSV4_ERR_UNSUPPORTED, "act_quant: block_size %d unsupported (128 only)", block_size);
  REQUIRE(cols % block_size == 0, DSV4_ERR_SHAPE, "act_quant: last dim %lld not a multiple of %d",
          (long long)cols, block_size);
  if (rows == 0 || cols == 0) return DSV4_OK;
  REQUIRE(x, DSV4_ERR_NULL, "act_quant: null input");
  REQUIRE(rt || codes || scale_f32 || scale_e8m0x4, DSV4_ERR_NULL, "act_quant: no output requested");
  REQUIRE(aligned(x, 16) && aligned(rt, 16) && aligned(codes, 8) && aligned(scale_e8m0x4, 4) &&
              aligned(scale_f32, 4),
          DSV4_ERR_SHAPE, "act_quant: misaligned buffer");
  return hip_status(launch_fp8_act_quant((const uint16_t*)x, rows * cols, (uint16_t*)rt, (uint8_t*)codes,
                                         (float*)scale_f32, (uint8_t*)scale_e8m0x4, (hipStream_t)stream),
                    "act_quant launch");
}

int dsv4_mxfp4_act_quant(const void* x, int64_t rows, int64_t cols, int rule, void* packed, void* scale,
                         void* dq, void* stream) {
  REQUIRE(rows >= 0 && cols >= 0, DSV4_ERR_SHAPE, "mx_quant: negative size");
  REQUIRE(rule == DSV4_RULE_CEIL_DIV6 || rule == DSV4_RULE_OCP_FLOOR, DSV4_ERR_UNSUPPORTED,
          "mx_quant: unknown scale rule %d", rule);
  REQUIRE(cols % 32 == 0, DSV4_ERR_SHAPE, "mx_quant: last dim %lld not a multiple of 32", (long long)cols);
  if (rows == 0 || cols == 0) return DSV4_OK;
  REQUIRE(x && packed && scale, DSV4_ERR_NULL, "mx_quant: null pointer");
  REQUIRE(aligned(x, 16) && aligned(packed, 4) && aligned(dq, 16), DSV4_ERR_SHAPE, "mx_quant: misaligned buffer");
  return hip_status(launch_mxfp4_act_quant((const uint16_t*)x, rows * cols, rule, (uint8_t*)packed,
                                           (uint8_t*)scale, (uint16_t*)dq, (hipStream_t)stream),
                    "mx_quant launch");
}

// ---------------------------------------------------------------------------
int dsv4_moe_align_max_blocks(int R, int E, int block_m) {
  if (R < 0 || E <= 0 || block_m <= 0) return dsv4_fail(DSV4_ERR_SHAPE, "align: bad sizes");
  // sum_e ceil(c_e / B) <= R / B + #active <= R / B + min(E, R)
  const int64_t nb = (int64_t)R / block_m + (R < E ? R : E) + 1;
  return (int)nb;
}

int dsv4_moe_align(const void* topk_ids, int ids_int64, const float* topk_w, int T, int K, int E, int block_m,
                   int max_blocks, int32_t* sorted_ids, int32_t* block_expert, int32_t* num_post_padded,
                   int32_t* order, int32_t* s_e, float* s_w, int32_t* row, int32_t* counts,
                   int32_t* expert_start, int32_t* active, int32_t* num_active, int32_t* padded_pos,
                   int32_t* status, void* stream) {
  REQUIRE(T >= 0 && K > 0, DSV4_ERR_SHAPE, "align: bad T=%d K=%d", T, K);
  REQUIRE(E > 0 && E <= DSV4_MAX_EXPERTS, DSV4_ERR_UNSUPPORTED, "align: E=%d outside 1..%d", E,
          DSV4_MAX_EXPERTS);
  REQUIRE(block_m > 0 && block_m <= 1024, DSV4_ERR_SHAPE, "align: block_m=%d", block_m);
  const int64_t R = (int64_t)T * K;
  REQUIRE(R < (1 << 30), DSV4_ERR_SHAPE, "align: too many entries");
  REQUIRE(max_blocks >= dsv4_moe_align_max_blocks((int)R, E, block_m), DSV4_ERR_SHAPE,
          "align: max_blocks=%d below the bound %d", max_blocks, dsv4_moe_align_max_blocks((int)R, E, block_m));
  REQUIRE(sorted_ids && block_expert && num_post_padded, DSV4_ERR_NULL, "align: null padded-layout output");
  REQUIRE(R == 0 || topk_ids, DSV4_ERR_NULL, "align: null topk_ids");
  Dsv4AlignOut o{sorted_ids, block_expert, num_post_padded, order, s_e, s_w, row, counts,
                 expert_start, active, num_active, padded_pos, status};
  return hip_status(launch_moe_align(topk_ids, ids_int64, topk_w, (int)R, K, E, block_m, max_blocks, o,
                                     (hipStream_t)stream),
                    "align launch");
}

int64_t dsv4_moe_align_workspace_bytes(int T, int K, int E) {
  if (T <= 0 || K <= 0 || E <= 0) return 0;
  return align_chunked_scratch_bytes(T * K, E);
}

int dsv4_moe_align_ws(const void* topk_ids, int ids_int64, const float* topk_w, int T, int K, int E, int block_m,
                      int max_blocks, int32_t* sorted_ids, int32_t* block_expert, int32_t* num_post_padded,
                      int32_t* order, int32_t* s_e, float* s_w, int32_t* row, int32_t* counts,
                      int32_t* expert_start, int32_t* active, int32_t* num_active, int32_t* padded_pos,
                      int32_t* status, void* workspace, int64_t workspace_bytes, void* stream) {
  const int64_t R = (int64_t)T * K;
  if (R <= kAlignSmallRows || workspace == nullptr)
    return dsv4_moe_align(topk_ids, ids_int64, topk_w, T, K, E, block_m, max_blocks, sorted_ids, block_expert,
                          num_post_padded, order, s_e, s_w, row, counts, expert_start, active, num_active,
                          padded_pos, status, stream);
  REQUIRE(K > 0, DSV4_ERR_SHAPE, "align: bad K=%d", K);
  REQUIRE(E > 0 && E <= DSV4_MAX_EXPERTS, DSV4_ERR_UNSUPPORTED, "align: E=%d outside 1..%d", E,
          DSV4_MAX_EXPERTS);
  REQUIRE(block_m > 0 && block_m <= 1024, DSV4_ERR_SHAPE, "align: block_m=%d", block_m);
  REQUIRE(R < (1 << 30), DSV4_ERR_SHAPE, "align: too many entries");
  REQUIRE(max_blocks >= dsv4_moe_align_max_blocks((int)R, E, block_m), DSV4_ERR_SHAPE,
          "align: max_blocks=%d below the bound %d", max_blocks, dsv4_moe_align_max_blocks((int)R, E, block_m));
  REQUIRE(sorted_ids && block_expert && num_post_padded && topk_ids, DSV4_ERR_NULL, "align: null pointer");
  REQUIRE(workspace_bytes >= align_chunked_scratch_bytes((int)R, E) && aligned(workspace, 4), DSV4_ERR_SHAPE,
          "align: workspace %lld < %lld bytes", (long long)workspace_bytes,
          (long long)align_chunked_scratch_bytes((int)R, E));
  Dsv4AlignOut o{sorted_ids, block_expert, num_post_padded, order, s_e, s_w, row, counts,
                 expert_start, active, num_active, padded_pos, status};
  return hip_status(launch_moe_align_chunked(topk_ids, ids_int64, topk_w, (int)R, K, E, block_m, max_blocks, o,
                                             nullptr, 0, 0, 0, nullptr, nullptr, (hipStream_t)stream, 0, workspace),
                    "align launch");
}

int dsv4_moe_permute(const void* src, int64_t n_src, const int32_t* row, int64_t n_rows, int64_t row_bytes,
                     void* dst, void* stream) {
  REQUIRE(n_rows >= 0 && row_bytes >= 0 && n_src >= 0, DSV4_ERR_SHAPE, "permute: negative size");
  REQUIRE(row_bytes % 16 == 0, DSV4_ERR_SHAPE, "permute: row bytes %lld not a multiple of 16",
          (long long)row_bytes);
  if (n_rows == 0 || row_bytes == 0) return DSV4_OK;
  REQUIRE(src && row && dst, DSV4_ERR_NULL, "permute: null pointer");
  REQUIRE(aligned(src, 16) && aligned(dst, 16), DSV4_ERR_SHAPE, "permute: misaligned buffer");
  return hip_status(launch_moe_gather_rows((const uint8_t*)src, n_src, row, n_rows, row_bytes, (uint8_t*)dst,
                                           (hipStream_t)stream),
                    "permute launch");
}

int64_t dsv4_moe_unpermute_workspace_bytes(int T, int Kmax) {
  return (int64_t)sizeof(int32_t) * ((int64_t)T + (int64_t)T * Kmax + 1);
}

int dsv4_moe_unpermute(const void* out_sorted, const int32_t* row, int R, int T, int Kmax, int D, void* workspace,
                       void* y, int32_t* status_out, void* stream) {
  REQUIRE(R >= 0 && T >= 0 && D >= 0, DSV4_ERR_SHAPE, "unpermute: negative size");
  REQUIRE(Kmax > 0 && Kmax <= DSV4_UNPERMUTE_MAX_ROWS, DSV4_ERR_UNSUPPORTED, "unpermute: Kmax=%d outside 1..%d",
          Kmax, DSV4_UNPERMUTE_MAX_ROWS);
  REQUIRE(D % 8 == 0, DSV4_ERR_SHAPE, "unpermute: D=%d not a multiple of 8", D);
  if (T == 0 || D == 0) return DSV4_OK;
  REQUIRE(workspace && y && (R == 0 || (out_sorted && row)), DSV4_ERR_NULL, "unpermute: null pointer");
  REQUIRE(aligned(out_sorted, 16) && aligned(y, 16) && aligned(workspace, 4), DSV4_ERR_SHAPE,
          "unpermute: misaligned buffer");
  int32_t* cnt = (int32_t*)workspace;
  int32_t* pos = cnt + T;
  int32_t* status = status_out ? status_out : pos + (int64_t)T * Kmax;
  REQUIRE(aligned(status, 4), DSV4_ERR_SHAPE, "unpermute: misaligned status");
  return hip_status(launch_moe_unpermute_rows((const uint16_t*)out_sorted, row, R, T, Kmax, D, cnt, pos, status,
                                              (uint16_t*)y, (hipStream_t)stream),
                    "unpermute launch");
}

int dsv4_moe_combine(const void* out_flat, const void* topk_ids, int ids_int64, int T, int K, int D, void* y,
                     void* stream) {
  REQUIRE(T >= 0 && D >= 0, DSV4_ERR_SHAPE, "combine: negative size");
  REQUIRE(K > 0 && K <= DSV4_MAX_TOPK, DSV4_ERR_UNSUPPORTED, "combine: K=%d outside 1..%d", K, DSV4_MAX_TOPK);
  REQUIRE(D % 8 == 0, DSV4_ERR_SHAPE, "combine: D=%d not a multiple of 8", D);
  if (T == 0 || D == 0) return DSV4_OK;
  REQUIRE(out_flat && topk_ids && y, DSV4_ERR_NULL, "combine: null pointer");
  REQUIRE(aligned(out_flat, 16) && aligned(y, 16), DSV4_ERR_SHAPE, "combine: misaligned buffer");
  return hip_status(launch_moe_combine_flat((const uint16_t*)out_flat, topk_ids, ids_int64, T, K, D,
                                            (uint16_t*)y, (hipStream_t)stream),
                    "combine launch");
}

// ---------------------------------------------------------------------------
int64_t dsv4_moe_route_workspace_bytes(int T, int D, int E) {
  if (T <= 0 || D <= 0 || E <= 0) return 0;
  return (int64_t)route_split_k(T, D, E) * T * E * (int64_t)sizeof(float);
}

int dsv4_moe_route(const void* x, int x_f32, const float* gate_w, const float* bias, const void* tid2eid,
                   int tid2eid_int64, int64_t vocab, const void* input_ids, int input_ids_int64, int T, int D, int E,
                   int K, int scoring, int renormalize, float scale, float* out_w, int32_t* out_ids, int32_t* status,
                   void* workspace, void* stream) {
  REQUIRE(T >= 0, DSV4_ERR_SHAPE, "route: negative T");
  REQUIRE(D > 0 && D % 32 == 0, DSV4_ERR_SHAPE, "route: hidden size %d not a positive multiple of 32", D);
  REQUIRE(E >= 16 && E <= 512 && E % 16 == 0, DSV4_ERR_UNSUPPORTED,
          "route: %d experts unsupported (multiple of 16 in 16..512)", E);
  REQUIRE(K >= 1 && K <= E && K <= 64, DSV4_ERR_UNSUPPORTED, "route: top-k %d outside 1..min(E, 64)", K);
  REQUIRE(scoring >= 0 && scoring <= 2, DSV4_ERR_UNSUPPORTED,
          "route: scoring %d unknown (0 softmax, 1 sigmoid, 2 sqrtsoftplus)", scoring);
  if (T == 0) return DSV4_OK;
  REQUIRE(x && gate_w && out_w && out_ids && workspace, DSV4_ERR_NULL, "route: null pointer");
  if (tid2eid) {
    REQUIRE(input_ids, DSV4_ERR_NULL, "route: hash-layer routing needs input_ids");
    REQUIRE(vocab > 0, DSV4_ERR_SHAPE, "route: tid2eid needs vocab > 0");
  }
  REQUIRE(aligned(x, 16) && aligned(gate_w, 16) && aligned(workspace, 4), DSV4_ERR_SHAPE,
          "route: misaligned buffer (x and gate_w need 16 bytes)");
  REQUIRE(x_f32 == 0 || x_f32 == 1, DSV4_ERR_UNSUPPORTED, "route: x_f32 must be 0 (bf16) or 1 (fp32)");
  return hip_status(launch_moe_route(x, x_f32, gate_w, T, D, E, K, scoring, bias, tid2eid, tid2eid_int64,
                                     input_ids, input_ids_int64, vocab, renormalize, scale, out_w, out_ids, status,
                                     (float*)workspace, (hipStream_t)stream),
                    "route launch");
}

// ---------------------------------------------------------------------------
static_assert(DSV4_AFMT_BF16 == kAfmtBf16, "A format ids");

static int check_gemm_common(int afmt, const void* a, const void* a_scale, const int32_t* sorted_ids,
                             const int32_t* block_expert, const int32_t* npp, int R, int block_m, int max_blocks,
                             const void* experts, int Kdim, void* out) {
  REQUIRE(afmt == DSV4_AFMT_E4M3 || afmt == DSV4_AFMT_E2M1 || afmt == DSV4_AFMT_BF16, DSV4_ERR_UNSUPPORTED,
          "gemm: unknown A format %d", afmt);
  REQUIRE(afmt != DSV4_AFMT_BF16 || block_m == DSV4_GEMM_BLOCK_M || block_m == 64 || block_m == 256,
          DSV4_ERR_UNSUPPORTED, "gemm: bf16 activations need block_m %d, 64 or 256 (got %d)", DSV4_GEMM_BLOCK_M,
          block_m);
  REQUIRE(R >= 0 && max_blocks >= 0, DSV4_ERR_SHAPE, "gemm: negative size");
  REQUIRE(moe_gemm_supported_kdim(Kdim), DSV4_ERR_UNSUPPORTED,
          "gemm: reduction dim %d unsupported (512, 1024, 2048 or 4096)", Kdim);
  REQUIRE(a && (a_scale || afmt == DSV4_AFMT_BF16) && sorted_ids && block_expert && npp && experts && out,
          DSV4_ERR_NULL, "gemm: null pointer");
  REQUIRE(aligned(a, 16) && aligned(a_scale, 4) && aligned(experts, 8), DSV4_ERR_SHAPE,
          "gemm: misaligned buffer");
  return DSV4_OK;
}

// bytes per A row of a reduction of length k
static int64_t a_row_bytes(int afmt, int k) {
  return afmt == DSV4_AFMT_E4M3 ? (int64_t)k : afmt == DSV4_AFMT_E2M1 ? (int64_t)k / 2 : 2 * (int64_t)k;
}

int dsv4_moe_gemm_gateup(int afmt, const void* a, const void* a_scale, int a_row_div, const int32_t* sorted_ids,
                         const int32_t* block_expert, const int32_t* num_post_padded, int R, int block_m,
                         int max_blocks, const void* expert_table, int D, int I, const float* topk_w,
                         float swiglu_limit, void* h_out, void* stream) {
  REQUIRE(moe_gemm_supported_block_m(block_m), DSV4_ERR_UNSUPPORTED,
          "gemm: block_m %d unsupported (16, 64, 128 or 256)", block_m);
  REQUIRE(I > 0 && I % 128 == 0, DSV4_ERR_UNSUPPORTED, "gemm gate/up: I=%d not a multiple of 128", I);
  REQUIRE(a_row_div > 0, DSV4_ERR_SHAPE, "gemm gate/up: a_row_div=%d", a_row_div);
  if (R == 0 || max_blocks == 0) return DSV4_OK;
  int rc = check_gemm_common(afmt, a, a_scale, sorted_ids, block_expert, num_post_padded, R, block_m, max_blocks,
                             expert_table, D, h_out);
  if (rc) return rc;
  REQUIRE(topk_w, DSV4_ERR_NULL, "gemm gate/up: null routing weights");
  REQUIRE(block_m != 256 || moe_gemm_big_supported(D, I, true), DSV4_ERR_UNSUPPORTED,
          "gemm gate/up: 256-row blocks need D a multiple of 1024 and I of 128 (D=%d, I=%d)", D, I);
  Dsv4GemmArgs g{afmt, (const uint8_t*)a, a_row_bytes(afmt, D),
                 (const uint8_t*)a_scale, a_row_div, sorted_ids, block_expert, num_post_padded, R, block_m,
                 max_blocks, (const Dsv4ExpertPtrs*)expert_table, D, I, topk_w, swiglu_limit,
                 (uint16_t*)h_out};
  return hip_status(launch_moe_gemm_gateup(g, (hipStream_t)stream), "gemm gate/up launch");
}

int dsv4_moe_gemm_down(int afmt, const void* a, const void* a_scale, const int32_t* sorted_ids,
                       const int32_t* block_expert, const int32_t* num_post_padded, int R, int block_m,
                       int max_blocks, const void* expert_table, int I, int D, void* out, void* stream) {
  REQUIRE(moe_gemm_supported_block_m(block_m), DSV4_ERR_UNSUPPORTED,
          "gemm: block_m %d unsupported (16, 64, 128 or 256)", block_m);
  REQUIRE(D > 0 && D % 256 == 0, DSV4_ERR_UNSUPPORTED, "gemm down: D=%d not a multiple of 256", D);
  if (R == 0 || max_blocks == 0) return DSV4_OK;
  int rc = check_gemm_common(afmt, a, a_scale, sorted_ids, block_expert, num_post_padded, R, block_m, max_blocks,
                             expert_table, I, out);
  if (rc) return rc;
  REQUIRE(block_m != 256 || (moe_gemm_big_supported(I, D, false) && aligned(out, 16)), DSV4_ERR_UNSUPPORTED,
          "gemm down: 256-row blocks need I a multiple of 1024, D of 256 and a 16-byte aligned output");
  Dsv4GemmArgs g{afmt, (const uint8_t*)a, a_row_bytes(afmt, I),
                 (const uint8_t*)a_scale, 1, sorted_ids, block_expert, num_post_padded, R, block_m, max_blocks,
                 (const Dsv4ExpertPtrs*)expert_table, I, D, nullptr, 0.0f, (uint16_t*)out};
  return hip_status(launch_moe_gemm_down(g, (hipStream_t)stream), "gemm down launch");
}

// ---------------------------------------------------------------------------
// Fused routed layer: [align | quantise x] -> gate/up GEMM + SwiGLU (+ quantise
// h in the epilogue where a wave or workgroup holds whole quantisation blocks:
// MXFP4 always, FP8 in the 64/128-row kernel; a separate FP8 quantisation
// launch for 16-row blocks) -> down GEMM -> combine. No step needs ordering
// between workgroups of one launch: device-scope fences for such hand-offs were
// measured to cost far more than the launches they would save. Workspace
// regions are 256-byte aligned.
struct LayerWs {
  int64_t sorted_ids, block_expert, npp, status, xa, xs, h, ha, hs, out, align_scratch, route_part, total;
  int max_blocks;
  int bm;
  // hot layout (experts with at least hot_min rows, 256-row blocks, large-tile kernel); hot_min 0: none
  int hot_min, max_blocks_h;
  int64_t sorted_ids_h, block_expert_h, npp_h;
};

// Experts with at least hot_rows_threshold() routed rows run in 256-row blocks on
// the large-tile kernel in layers of at least hot_layer_rows() routed rows; the rest
// keep 64-row blocks. Measured with Zipf(1.1) routing over 256 experts (hidden 4096,
// inter 2048), top-8:
//   a4w4 (one 8-wave workgroup per hot block): the split lost 5-10 % at 2048 tokens
//   (the hot experts' blocks too few to fill a launch of their own) and gained 5.5 %
//   at 4096 tokens with a 256-row threshold (2 % ahead of 128); from 8192 tokens a
//   128-row threshold was 2-3 % faster than 256.
//   bf16 (two half-block workgroups per hot block, twice the workgroups per launch):
//   with a 128-row threshold the split gained 1.5-2 % at 2048 and 4096 tokens, where a
//   256-row threshold lost 1 % and 0.5-1.5 % against it.
//   a4w4 below 32,768 rows, where the large-tile launch takes half blocks as well and
//   runs beside the tiled one: a 128-row threshold gained 3 % at 2048 tokens (1.011-1.018
//   -> 0.981-0.984 ms), 256 lost 4 %.
//   pure bf16 (bf16 large-tile kernel, whole blocks, 128-row threshold): layer ms with
//   / without the split at 2048 tokens 1.682-1.689 / 1.570, 4096 2.588-2.604 / 2.451,
//   8192 4.087-4.096 / 4.106-4.112, 16384 7.20-7.33 / 7.41; bf16 MFMAs take the same
//   time on either kernel per useful FLOP until the hot experts fill many whole blocks,
//   so the pure variant splits from 65,536 routed rows.
// DSV4_HOT_LAYER_ROWS and DSV4_HOT_ROWS (0: never) override them, read once.
static int64_t hot_layer_rows(bool pure) {
  static const int64_t v = [] {
    const char* s = getenv("DSV4_HOT_LAYER_ROWS");
    return s ? (int64_t)atoll(s) : (int64_t)-1;
  }();
  return v >= 0 ? v : pure ? 65536 : 16384;
}

static int hot_rows_threshold(int64_t R, bool fp8) {
  static const int v = [] {
    const char* s = getenv("DSV4_HOT_ROWS");
    return s ? atoi(s) : -1;
  }();
  return v >= 0 ? v : (fp8 || R < 32768 || R >= 65536 ? 128 : 256);
}

// Rows per M block: 16 (decode kernel, ~1-4 rows per active expert) below 2048
// routed rows, 64 (tiled kernel, weight tiles reused across 4 row subtiles)
// from there on, where the Zipf-hot experts receive hundreds of rows.
static int layer_block_m(int64_t R) { return R >= 2048 ? 64 : DSV4_GEMM_BLOCK_M; }

static LayerWs layer_ws(int T, int K, int E, int D, int I, int profile, bool shared = false,
                        bool routed = false) {
  LayerWs w{};
  const int64_t R = (int64_t)T * K;
  const int64_t Rt = R + (shared ? T : 0);  // routed rows, then the shared expert's T rows
  const bool pure = profile == DSV4_PROFILE_BF16_PURE;  // bf16 x and h (16- and 64-row kernels)
  const int bm = layer_block_m(R);
  w.bm = bm;
  w.max_blocks = dsv4_moe_align_max_blocks((int)R, E, bm) + (shared ? (T + bm - 1) / bm : 0);
  const bool fp8 = profile == DSV4_PROFILE_BF16;
  int64_t o = 0;
  auto take = [&](int64_t bytes) { int64_t at = o; o = round_up(o + bytes, 256); return at; };
  w.sorted_ids = take(sizeof(int32_t) * (int64_t)w.max_blocks * bm);
  w.block_expert = take(sizeof(int32_t) * (int64_t)w.max_blocks);
  w.npp = take(sizeof(int32_t));
  w.status = take(sizeof(int32_t));
  w.xa = pure ? -1 : take(fp8 ? (int64_t)T * D : (int64_t)T * D / 2);
  w.xs = pure ? -1 : take((int64_t)T * D / 32);
  // bf16 h only where the gate/up cannot quantise it in its epilogue (FP8
  // blocks of 128 columns span four single-wave workgroups of the 16-row kernel)
  // and for the pure-bf16 variant, whose down GEMM reads it as it is
  w.h = ((fp8 && bm == DSV4_GEMM_BLOCK_M) || pure) ? take(2 * Rt * I) : -1;
  w.ha = pure ? -1 : take(fp8 ? Rt * I : Rt * I / 2);
  w.hs = pure ? -1 : take(Rt * I / 32);
  w.out = take(2 * Rt * D);
  w.align_scratch = R > kAlignSmallRows ? take(align_chunked_scratch_bytes((int)R, E)) : 0;
  w.route_part = routed ? take(dsv4_moe_route_workspace_bytes(T, D, E)) : -1;  // router partial logits
  const int hot = hot_rows_threshold(R, fp8 || pure);
  if (R >= hot_layer_rows(pure) && R > kAlignSmallRows && hot > 0 && moe_gemm_big_supported(D, I, true) &&
      moe_gemm_big_supported(I, D, false)) {
    w.hot_min = hot;
    // each hot expert holds >= hot_min rows: blocks <= R/256 + min(E, R/hot_min) + 1
    w.max_blocks_h = (int)(R / kHotBlockM + std::min<int64_t>(E, R / hot) + 1);
    w.sorted_ids_h = take(sizeof(int32_t) * (int64_t)w.max_blocks_h * kHotBlockM);
    w.block_expert_h = take(sizeof(int32_t) * (int64_t)w.max_blocks_h);
    w.npp_h = take(sizeof(int32_t));
  }
  w.total = o;
  return w;
}

// Router arguments of the layer entry that also routes (deepseek_v4.py:118-148).
struct LayerRoute {
  const float* gate_w;
  const float* bias;
  const void* tid2eid;
  int tid_is64;
  int64_t vocab;
  const void* input_ids;
  int ids_is64;
  int scoring;
  int renorm;
  float scale;
  float* out_w;      // [T, K] routing weights (written)
  int32_t* out_ids;  // [T, K] expert ids (written)
  int32_t* status;   // nullable: bad input ids / table entries
};

// Batches up to this many tokens route inside the layer's first launch (one
// token per wave of the align workgroup); larger ones route in the router's
// own two launches first.
constexpr int kFusedRouteTokens = 16;

// The routed layer, and with `shared` the shared expert as one more group of
// T rows (bf16 profile only; checked by the caller). With `route` the layer
// first routes x itself: topk_ids / topk_w are then the route's outputs.
// The hot layout's two large-tile launches run on a side stream, concurrently with the
// main layout's launches: the tiled kernel streams the cold experts' weights (bound by
// memory) while the large-tile kernel multiplies (bound by the MFMAs), and the two
// write disjoint rows of h and of the down outputs. One side stream (default priority)
// and a fork/join event pair per device, created on the device's first split layer;
// a per-device mutex orders the callers that share them. DSV4_HOT_CONCURRENT=0 keeps
// every launch on the caller's stream; read once.
struct SideStream {
  hipStream_t s;
  hipEvent_t fork, join;
  std::mutex mu;
};
static constexpr int kMaxSideDevices = 64;
static std::mutex g_side_mu;
static SideStream* g_side[kMaxSideDevices] = {};

static bool hot_concurrent() {
  static const bool v = [] {
    const char* s = getenv("DSV4_HOT_CONCURRENT");
    return !s || atoi(s) != 0;
  }();
  return v;
}

static int side_stream(void* stream, SideStream** out) {
  int cur = 0;
  hipError_t e = hipGetDevice(&cur);
  if (e != hipSuccess) return hip_status(e, "layer: hipGetDevice");
  hipDevice_t dev = cur;
  if (stream) {
    e = hipStreamGetDevice((hipStream_t)stream, &dev);
    if (e != hipSuccess) return hip_status(e, "layer: hipStreamGetDevice");
  }
  REQUIRE(dev >= 0 && dev < kMaxSideDevices, DSV4_ERR_UNSUPPORTED, "layer: device %d beyond %d", (int)dev,
          kMaxSideDevices);
  std::lock_guard<std::mutex> lock(g_side_mu);
  if (!g_side[dev]) {
    if (dev != cur) {
      e = hipSetDevice(dev);
      if (e != hipSuccess) return hip_status(e, "layer: hipSetDevice");
    }
    SideStream* ss = new SideStream();
    e = hipStreamCreateWithFlags(&ss->s, hipStreamNonBlocking);
    if (e == hipSuccess) e = hipEventCreateWithFlags(&ss->fork, hipEventDisableTiming);
    if (e == hipSuccess) e = hipEventCreateWithFlags(&ss->join, hipEventDisableTiming);
    if (dev != cur) (void)hipSetDevice(cur);
    if (e != hipSuccess) {
      delete ss;  // the handles made so far stay with the runtime until the process ends
      return hip_status(e, "layer: side stream / events");
    }
    g_side[dev] = ss;
  }
  *out = g_side[dev];
  return DSV4_OK;
}

static int layer_forward(int profile, int scale_rule, const void* x, const void* topk_ids, int ids_int64,
                         const float* topk_w, int T, int K, int E, int D, int I, const void* expert_table,
                         const Dsv4ExpertPtrs* shared, float swiglu_limit, void* workspace, int64_t workspace_bytes,
                         void* y, void* stream, const LayerRoute* route = nullptr, bool one_stream = false) {
  if (route) {
    topk_ids = route->out_ids;
    ids_int64 = 0;
    topk_w = route->out_w;
  }
  REQUIRE(profile == DSV4_PROFILE_BF16 || profile == DSV4_PROFILE_A4W4 || profile == DSV4_PROFILE_BF16_PURE,
          DSV4_ERR_UNSUPPORTED, "layer: unknown profile %d", profile);
  REQUIRE(profile != DSV4_PROFILE_BF16_PURE || !shared, DSV4_ERR_UNSUPPORTED,
          "layer: the fused shared expert needs the bf16 profile with its FP8 round trips");
  REQUIRE(T >= 0 && K > 0 && K <= DSV4_MAX_TOPK, DSV4_ERR_SHAPE, "layer: bad T=%d K=%d", T, K);
  REQUIRE(D % 512 == 0 && I % 512 == 0 && D > 0 && I > 0, DSV4_ERR_UNSUPPORTED,
          "layer: D=%d and I=%d must be multiples of 512", D, I);
  if (T == 0) return DSV4_OK;
  REQUIRE(x && topk_ids && topk_w && expert_table && workspace && y, DSV4_ERR_NULL, "layer: null pointer");
  const LayerWs w = layer_ws(T, K, E, D, I, profile, shared != nullptr, route != nullptr);
  REQUIRE(workspace_bytes >= w.total, DSV4_ERR_SHAPE, "layer: workspace %lld < %lld bytes",
          (long long)workspace_bytes, (long long)w.total);
  REQUIRE(aligned(workspace, 256), DSV4_ERR_SHAPE, "layer: workspace not 256-byte aligned");
  char* base = (char*)workspace;
  int32_t* sorted_ids = (int32_t*)(base + w.sorted_ids);
  int32_t* block_expert = (int32_t*)(base + w.block_expert);
  int32_t* npp = (int32_t*)(base + w.npp);
  int32_t* status = (int32_t*)(base + w.status);
  const int R = T * K;
  const int n_sh = shared ? T : 0;
  const int Rt = R + n_sh;
  const int bm = w.bm;
  REQUIRE(E > 0 && E <= DSV4_MAX_EXPERTS, DSV4_ERR_UNSUPPORTED, "layer: E=%d outside 1..%d", E, DSV4_MAX_EXPERTS);
  REQUIRE(scale_rule == DSV4_RULE_CEIL_DIV6 || scale_rule == DSV4_RULE_OCP_FLOOR || profile != DSV4_PROFILE_A4W4,
          DSV4_ERR_UNSUPPORTED, "layer: unknown scale rule %d", scale_rule);
  REQUIRE(aligned(x, 16), DSV4_ERR_SHAPE, "layer: x not 16-byte aligned");
  const bool fp8 = profile == DSV4_PROFILE_BF16;
  const bool pure = profile == DSV4_PROFILE_BF16_PURE;  // x and h stay bf16: no quantisation launches
  const int afmt = fp8 ? DSV4_AFMT_E4M3 : pure ? DSV4_AFMT_BF16 : DSV4_AFMT_E2M1;
  const int64_t x_elems = pure ? 0 : (int64_t)T * D;  // the align launch quantises x unless pure
  REQUIRE(moe_gemm_supported_kdim(D) && moe_gemm_supported_kdim(I), DSV4_ERR_UNSUPPORTED,
          "layer: no GEMM compiled for D=%d / I=%d", D, I);
  // routing layout and the activation quantisation of x share one launch
  Dsv4AlignOut ao{sorted_ids, block_expert, npp, nullptr, nullptr, nullptr, nullptr, nullptr,
                  nullptr,    nullptr,      nullptr, nullptr, status};
  int rc = DSV4_OK;
  bool aligned_already = false;
  if (route) {
    int S = 1;
    float* part = (float*)(base + w.route_part);
    rc = hip_status(launch_route_logits(x, 0, route->gate_w, T, D, E, part, &S, (hipStream_t)stream),
                    "route logits launch");
    if (rc) return rc;
    const RouteTopkArgs ra{part, S, T, E, K, route->scoring, route->bias, route->tid2eid, route->tid_is64,
                           route->input_ids, route->ids_is64, route->vocab, route->renorm, route->scale,
                           route->out_w, route->out_ids, route->status};
    if (T <= kFusedRouteTokens && R <= kAlignSmallRows) {  // top-k, align and x quantisation in one launch
      rc = hip_status(launch_route_align_quant(ra, bm, w.max_blocks, ao, pure ? nullptr : (const uint16_t*)x,
                                               x_elems, fp8 ? 0 : 1, scale_rule, pure ? nullptr : base + w.xa,
                                               pure ? nullptr : base + w.xs, (hipStream_t)stream, n_sh),
                      "route+align+quant launch");
      aligned_already = true;
    } else {
      rc = hip_status(launch_route_topk(ra, (hipStream_t)stream), "route top-k launch");
    }
    if (rc) return rc;
  }
  Dsv4AlignHot hot{};
  if (w.hot_min > 0)
    hot = Dsv4AlignHot{w.hot_min, w.max_blocks_h, (int32_t*)(base + w.sorted_ids_h), (int32_t*)(base + w.block_expert_h),
                       (int32_t*)(base + w.npp_h)};
  if (!aligned_already) rc = hip_status(
      R > kAlignSmallRows
          ? launch_moe_align_chunked(topk_ids, ids_int64, nullptr, R, K, E, bm, w.max_blocks, ao,
                                     pure ? nullptr : (const uint16_t*)x, x_elems, fp8 ? 0 : 1, scale_rule,
                                     pure ? nullptr : base + w.xa, pure ? nullptr : base + w.xs,
                                     (hipStream_t)stream, n_sh, base + w.align_scratch,
                                     w.hot_min > 0 ? &hot : nullptr)
          : launch_moe_align_quant(topk_ids, ids_int64, nullptr, R, K, E, bm, w.max_blocks, ao,
                                   pure ? nullptr : (const uint16_t*)x, x_elems, fp8 ? 0 : 1, scale_rule,
                                   pure ? nullptr : base + w.xa, pure ? nullptr : base + w.xs,
                                   (hipStream_t)stream, n_sh),
      "align+quant launch");
  if (rc) return rc;
  const Dsv4ExpertPtrs* table = (const Dsv4ExpertPtrs*)expert_table;
  // gate/up + SwiGLU, quantising h in the epilogue where the kernel holds whole blocks
  const bool hq_fused = !pure && (!fp8 || bm != DSV4_GEMM_BLOCK_M);
  Dsv4GemmArgs gu{};
  gu.afmt = afmt;
  gu.a = pure ? (const uint8_t*)x : (const uint8_t*)(base + w.xa);
  gu.a_row_bytes = a_row_bytes(afmt, D);
  gu.a_scale = pure ? nullptr : (const uint8_t*)(base + w.xs);
  gu.a_row_div = K;
  gu.sorted_ids = sorted_ids;
  gu.block_expert = block_expert;
  gu.num_post_padded = npp;
  gu.R = Rt;
  gu.block_m = bm;
  gu.max_blocks = w.max_blocks;
  gu.experts = table;
  gu.Kdim = D;
  gu.N = I;
  gu.topk_w = topk_w;
  gu.swiglu_limit = swiglu_limit;
  gu.out = hq_fused ? nullptr : (uint16_t*)(base + w.h);  // fused: h is never stored as bf16 (hq_skip_h)
  if (hq_fused) {
    gu.hq_mode = fp8 ? 1 : 2;
    gu.hq_rule = scale_rule;
    gu.hq_skip_h = 1;
    gu.hq_codes = (uint8_t*)(base + w.ha);
    gu.hq_scale = (uint8_t*)(base + w.hs);
  }
  if (shared) {  // rows R.. read x row f - R with routing weight 1
    gu.has_shared = 1;
    gu.shared_expert = E;
    gu.shared_a_rows = n_sh;
    gu.shared = *shared;
  }
  // the hot layout's 256-row blocks (routed rows only) on the large-tile kernel
  auto hot_args = [&](Dsv4GemmArgs g) {
    g.sorted_ids = hot.sorted_ids;
    g.block_expert = hot.block_expert;
    g.num_post_padded = hot.num_post_padded;
    g.block_m = kHotBlockM;
    g.max_blocks = hot.max_blocks;
    g.has_shared = 0;
    return g;
  };
  // concurrent split: h is quantised in the epilogues (no h-quantisation launch
  // between the two GEMMs reads the hot rows), so the hot rows' gate/up and down
  // need nothing from the main stream after the align
  // Under stream capture the layer keeps one stream: the shared side stream would
  // join the caller's capture, and another thread's layer on this device could then
  // put its work into that graph.
  // (the pure-bf16 variant has no h quantisation launch between the GEMMs either)
  const bool hot_side = w.hot_min > 0 && (hq_fused || pure);
  if (!one_stream && hot_side && hot_concurrent()) {
    hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
    if (hipStreamIsCapturing((hipStream_t)stream, &cs) != hipSuccess || cs != hipStreamCaptureStatusNone)
      one_stream = true;
  }
  SideStream* side = nullptr;
  std::unique_lock<std::mutex> side_lock;
  if (hot_side && !one_stream && hot_concurrent()) {
    rc = side_stream(stream, &side);
    if (rc) return rc;
    side_lock = std::unique_lock<std::mutex>(side->mu);
    rc = hip_status(hipEventRecord(side->fork, (hipStream_t)stream), "layer: fork record");
    if (!rc) rc = hip_status(hipStreamWaitEvent(side->s, side->fork, 0), "layer: fork wait");
    if (rc) return rc;
  }
  const hipStream_t hot_stream = side ? side->s : (hipStream_t)stream;
  // Once forked, the side stream is joined back into the caller's stream on every
  // path out, failures included, so the caller's stream still orders all of it.
  auto join = [&](int status_in) {
    if (!side) return status_in;
    int j = hip_status(hipEventRecord(side->join, side->s), "layer: join record");
    if (!j) j = hip_status(hipStreamWaitEvent((hipStream_t)stream, side->join, 0), "layer: join wait");
    side = nullptr;
    return status_in ? status_in : j;
  };
  if (side) {
    rc = hip_status(launch_moe_gemm_gateup(hot_args(gu), hot_stream), "gemm gate/up (large tiles) launch");
    if (rc) return join(rc);
  }
  rc = hip_status(launch_moe_gemm_gateup(gu, (hipStream_t)stream), "gemm gate/up launch");
  if (rc) return join(rc);
  if (w.hot_min > 0 && !side) {
    rc = hip_status(launch_moe_gemm_gateup(hot_args(gu), hot_stream), "gemm gate/up (large tiles) launch");
    if (rc) return rc;
  }
  if (!hq_fused && !pure) {  // FP8 blocks of 128 columns span four single-wave workgroups
    rc = dsv4_fp8_act_quant(base + w.h, Rt, I, 128, nullptr, base + w.ha, nullptr, base + w.hs, stream);
    if (rc) return join(rc);
  }
  Dsv4GemmArgs dn{};
  dn.afmt = afmt;
  dn.a = (const uint8_t*)(base + (pure ? w.h : w.ha));
  dn.a_row_bytes = a_row_bytes(afmt, I);
  dn.a_scale = pure ? nullptr : (const uint8_t*)(base + w.hs);
  dn.a_row_div = 1;
  dn.sorted_ids = sorted_ids;
  dn.block_expert = block_expert;
  dn.num_post_padded = npp;
  dn.R = Rt;
  dn.block_m = bm;
  dn.max_blocks = w.max_blocks;
  dn.experts = table;
  dn.Kdim = I;
  dn.N = D;
  dn.out = (uint16_t*)(base + w.out);
  if (shared) {  // h rows are indexed by flat index for every group
    dn.has_shared = 1;
    dn.shared_expert = E;
    dn.shared = *shared;
  }
  if (w.hot_min > 0) {
    rc = hip_status(launch_moe_gemm_down(hot_args(dn), hot_stream), "gemm down (large tiles) launch");
    if (rc) return join(rc);
  }
  rc = hip_status(launch_moe_gemm_down(dn, (hipStream_t)stream), "gemm down launch");
  rc = join(rc);  // the combine reads the hot rows' down outputs
  if (rc) return rc;
  // ids outside [0, E) were skipped by the align (never computed) and add nothing here
  REQUIRE(aligned(y, 16), DSV4_ERR_SHAPE, "layer: y not 16-byte aligned");
  const uint16_t* outp = (const uint16_t*)(base + w.out);
  return hip_status(launch_moe_combine_flat(outp, topk_ids, ids_int64, T, K, D, (uint16_t*)y, (hipStream_t)stream,
                                            shared ? outp + (int64_t)R * D : nullptr, E),
                    "combine launch");
}

int dsv4_moe_layer_workspace_bytes(int T, int K, int E, int D, int I, int profile, int64_t* bytes) {
  REQUIRE(bytes, DSV4_ERR_NULL, "workspace: null output");
  REQUIRE(T >= 0 && K > 0 && E > 0 && D > 0 && I > 0, DSV4_ERR_SHAPE, "workspace: bad sizes");
  REQUIRE(profile == DSV4_PROFILE_BF16 || profile == DSV4_PROFILE_A4W4 || profile == DSV4_PROFILE_BF16_PURE,
          DSV4_ERR_UNSUPPORTED,
          "workspace: unknown profile %d", profile);
  *bytes = layer_ws(T, K, E, D, I, profile).total;
  return DSV4_OK;
}

int dsv4_moe_layer_forward(int profile, int scale_rule, const void* x, const void* topk_ids, int ids_int64,
                           const float* topk_w, int T, int K, int E, int D, int I, const void* expert_table,
                           float swiglu_limit, void* workspace, int64_t workspace_bytes, void* y, void* stream) {
  return layer_forward(profile, scale_rule, x, topk_ids, ids_int64, topk_w, T, K, E, D, I, expert_table, nullptr,
                       swiglu_limit, workspace, workspace_bytes, y, stream);
}

// ---------------------------------------------------------------------------
// Allocation-free routed layer. Some callers cannot allocate device memory
// (code under HIP graph capture, tight serving loops, harnesses that forbid
// hipMalloc); for them the layer's workspace is `scratch`, a file-scope device
// array that each GPU holds once for the life of the process. In host code the
// name `scratch` is only a host-side stand-in for the symbol: its device
// address is looked up once per device with hipGetSymbolAddress, with that
// device current, and only that address is handed to kernels. The layer needs
// no zeroed workspace (every region is written before it is read), so nothing
// is cleared between calls; calls that overlap on one GPU (different streams)
// share the array and would race, so a call from a stream other than the
// device's last one is refused unless the caller declares it ordered.
static constexpr int64_t kScratchBytes = (int64_t)DSV4_NOALLOC_SCRATCH_BYTES;
static constexpr int kMaxDevices = 64;
static __device__ __align__(256) uint8_t scratch[kScratchBytes];
static std::mutex g_scratch_mu;
static void* g_scratch_ptr[kMaxDevices] = {};
static void* g_scratch_stream[kMaxDevices] = {};  // stream of the device's last call
static bool g_scratch_used[kMaxDevices] = {};

// Device address of `scratch` on the device that owns `stream` (looked up on
// that device's first call; later calls reuse it). Claims the array for
// `stream`: DSV4_ERR_STATE if the device's last call came from another stream
// and `ordered` is false.
static int scratch_address(void* stream, bool ordered, void** out) {
  int cur = 0;
  hipError_t e = hipGetDevice(&cur);
  if (e != hipSuccess) return hip_status(e, "no-alloc layer: hipGetDevice");
  hipDevice_t dev = cur;
  if (stream) {
    e = hipStreamGetDevice((hipStream_t)stream, &dev);
    if (e != hipSuccess) return hip_status(e, "no-alloc layer: hipStreamGetDevice");
  }
  REQUIRE(dev >= 0 && dev < kMaxDevices, DSV4_ERR_UNSUPPORTED, "no-alloc layer: device %d beyond %d", (int)dev,
          kMaxDevices);
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    if (dev != cur) {
      e = hipSetDevice(dev);
      if (e != hipSuccess) return hip_status(e, "no-alloc layer: hipSetDevice");
    }
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (dev != cur) (void)hipSetDevice(cur);
    if (e != hipSuccess) return hip_status(e, "no-alloc layer: hipGetSymbolAddress(scratch)");
    REQUIRE(p && aligned(p, 256), DSV4_ERR_STATE, "no-alloc layer: scratch address not 256-byte aligned");
    g_scratch_ptr[dev] = p;
  }
  REQUIRE(!g_scratch_used[dev] || g_scratch_stream[dev] == stream || ordered, DSV4_ERR_STATE,
          "no-alloc layer: device %d's scratch was last used from stream %p, this call comes from %p; calls on "
          "different streams race unless ordered (synchronize, or wait for an event, then pass "
          "DSV4_NOALLOC_STREAMS_ORDERED)",
          (int)dev, g_scratch_stream[dev], stream);
  g_scratch_used[dev] = true;
  g_scratch_stream[dev] = stream;
  *out = g_scratch_ptr[dev];
  return DSV4_OK;
}

int dsv4_moe_layer_forward_noalloc(int profile, int scale_rule, const void* x, const void* topk_ids, int ids_int64,
                                   const float* topk_w, int T, int K, int E, int D, int I, const void* expert_table,
                                   float swiglu_limit, void* y, int flags, void* stream) {
  REQUIRE(profile == DSV4_PROFILE_BF16 || profile == DSV4_PROFILE_A4W4 || profile == DSV4_PROFILE_BF16_PURE,
          DSV4_ERR_UNSUPPORTED, "no-alloc layer: unknown profile %d", profile);
  REQUIRE((flags & ~DSV4_NOALLOC_STREAMS_ORDERED) == 0, DSV4_ERR_UNSUPPORTED, "no-alloc layer: unknown flags 0x%x",
          flags);
  REQUIRE(T >= 0 && K > 0 && K <= DSV4_MAX_TOPK && E > 0 && D > 0 && I > 0, DSV4_ERR_SHAPE,
          "no-alloc layer: bad sizes T=%d K=%d E=%d D=%d I=%d", T, K, E, D, I);
  if (T == 0) return DSV4_OK;
  const int64_t need = layer_ws(T, K, E, D, I, profile).total;
  REQUIRE(need <= kScratchBytes, DSV4_ERR_UNSUPPORTED,
          "no-alloc layer: needs %lld bytes of workspace, the static scratch holds %lld (fewer tokens per call, "
          "or dsv4_moe_layer_forward with a caller workspace)",
          (long long)need, (long long)kScratchBytes);
  void* ws = nullptr;
  int rc = scratch_address(stream, (flags & DSV4_NOALLOC_STREAMS_ORDERED) != 0, &ws);
  if (rc) return rc;
  // one stream: this entry point creates nothing (no side stream or events)
  return layer_forward(profile, scale_rule, x, topk_ids, ids_int64, topk_w, T, K, E, D, I, expert_table, nullptr,
                       swiglu_limit, ws, kScratchBytes, y, stream, nullptr, true);
}

int dsv4_expand_block_scales(const void* block_scales, int64_t n_rows, int64_t k, void* out, void* stream) {
  REQUIRE(n_rows >= 0 && k >= 0, DSV4_ERR_SHAPE, "expand scales: negative size");
  REQUIRE(k % 32 == 0, DSV4_ERR_SHAPE, "expand scales: K=%lld not a multiple of 32", (long long)k);
  if (n_rows == 0 || k == 0) return DSV4_OK;
  REQUIRE(block_scales && out, DSV4_ERR_NULL, "expand scales: null pointer");
  return hip_status(launch_expand_block_scales((const uint8_t*)block_scales, n_rows, k, (uint8_t*)out,
                                               (hipStream_t)stream),
                    "expand scales launch");
}

int dsv4_moe_layer_shared_workspace_bytes(int T, int K, int E, int D, int I, int64_t* bytes) {
  REQUIRE(bytes, DSV4_ERR_NULL, "workspace: null output");
  REQUIRE(T >= 0 && K > 0 && E > 0 && D > 0 && I > 0, DSV4_ERR_SHAPE, "workspace: bad sizes");
  *bytes = layer_ws(T, K, E, D, I, DSV4_PROFILE_BF16, true).total;
  return DSV4_OK;
}

int dsv4_moe_layer_forward_shared(const void* x, const void* topk_ids, int ids_int64, const float* topk_w, int T,
                                  int K, int E, int D, int I, const void* expert_table, const void* sw1,
                                  const void* sw1s, const void* sw3, const void* sw3s, const void* sw2,
                                  const void* sw2s, float swiglu_limit, void* workspace, int64_t workspace_bytes,
                                  void* y, void* stream) {
  if (T == 0) return DSV4_OK;
  REQUIRE(sw1 && sw1s && sw3 && sw3s && sw2 && sw2s, DSV4_ERR_NULL, "layer: null shared-expert pointer");
  REQUIRE(aligned(sw1, 16) && aligned(sw3, 16) && aligned(sw2, 16) && aligned(sw1s, 4) && aligned(sw3s, 4) &&
              aligned(sw2s, 4),
          DSV4_ERR_SHAPE, "layer: misaligned shared-expert weights");
  const Dsv4ExpertPtrs sh{(const uint8_t*)sw1, (const uint8_t*)sw1s, (const uint8_t*)sw2,
                          (const uint8_t*)sw2s, (const uint8_t*)sw3, (const uint8_t*)sw3s};
  return layer_forward(DSV4_PROFILE_BF16, DSV4_RULE_OCP_FLOOR, x, topk_ids, ids_int64, topk_w, T, K, E, D, I,
                       expert_table, &sh, swiglu_limit, workspace, workspace_bytes, y, stream);
}

int dsv4_moe_routed_layer_workspace_bytes(int T, int K, int E, int D, int I, int profile, int with_shared,
                                          int64_t* bytes) {
  REQUIRE(bytes, DSV4_ERR_NULL, "workspace: null output");
  REQUIRE(T >= 0 && K > 0 && E > 0 && D > 0 && I > 0, DSV4_ERR_SHAPE, "workspace: bad sizes");
  REQUIRE(profile == DSV4_PROFILE_BF16 || profile == DSV4_PROFILE_A4W4 || profile == DSV4_PROFILE_BF16_PURE,
          DSV4_ERR_UNSUPPORTED, "workspace: unknown profile %d", profile);
  *bytes = layer_ws(T, K, E, D, I, profile, with_shared != 0, true).total;
  return DSV4_OK;
}

int dsv4_moe_routed_layer_forward(int profile, int scale_rule, const void* x, int T, int K, int E, int D, int I,
                                  const float* gate_w, const float* bias, const void* tid2eid, int tid2eid_int64,
                                  int64_t vocab, const void* input_ids, int input_ids_int64, int scoring,
                                  int renormalize, float routed_scale, const void* expert_table, const void* sw1,
                                  const void* sw1s, const void* sw3, const void* sw3s, const void* sw2,
                                  const void* sw2s, float swiglu_limit, float* topk_w_out, int32_t* topk_ids_out,
                                  int32_t* route_status, void* workspace, int64_t workspace_bytes, void* y,
                                  void* stream) {
  REQUIRE(T >= 0, DSV4_ERR_SHAPE, "routed layer: negative T");
  REQUIRE(E >= 16 && E <= 512 && E % 16 == 0, DSV4_ERR_UNSUPPORTED,
          "routed layer: %d experts unsupported (multiple of 16 in 16..512)", E);
  REQUIRE(K >= 1 && K <= E && K <= 64 && K <= DSV4_MAX_TOPK, DSV4_ERR_UNSUPPORTED,
          "routed layer: top-k %d outside 1..min(E, 64, %d)", K, DSV4_MAX_TOPK);
  REQUIRE(scoring >= 0 && scoring <= 2, DSV4_ERR_UNSUPPORTED,
          "routed layer: scoring %d unknown (0 softmax, 1 sigmoid, 2 sqrtsoftplus)", scoring);
  if (T == 0) return DSV4_OK;
  REQUIRE(gate_w && topk_w_out && topk_ids_out, DSV4_ERR_NULL, "routed layer: null router pointer");
  REQUIRE(aligned(gate_w, 16), DSV4_ERR_SHAPE, "routed layer: gate weight not 16-byte aligned");
  if (tid2eid) {
    REQUIRE(input_ids, DSV4_ERR_NULL, "routed layer: hash-layer routing needs input_ids");
    REQUIRE(vocab > 0, DSV4_ERR_SHAPE, "routed layer: tid2eid needs vocab > 0");
  }
  const bool has_shared = sw1 || sw1s || sw3 || sw3s || sw2 || sw2s;
  Dsv4ExpertPtrs sh{};
  if (has_shared) {
    REQUIRE(profile == DSV4_PROFILE_BF16, DSV4_ERR_UNSUPPORTED, "routed layer: the shared expert needs the bf16 profile");
    REQUIRE(sw1 && sw1s && sw3 && sw3s && sw2 && sw2s, DSV4_ERR_NULL, "routed layer: null shared-expert pointer");
    REQUIRE(aligned(sw1, 16) && aligned(sw3, 16) && aligned(sw2, 16) && aligned(sw1s, 4) && aligned(sw3s, 4) &&
                aligned(sw2s, 4),
            DSV4_ERR_SHAPE, "routed layer: misaligned shared-expert weights");
    sh = Dsv4ExpertPtrs{(const uint8_t*)sw1, (const uint8_t*)sw1s, (const uint8_t*)sw2,
                        (const uint8_t*)sw2s, (const uint8_t*)sw3, (const uint8_t*)sw3s};
  }
  const LayerRoute rt{gate_w, bias, tid2eid, tid2eid_int64, vocab, input_ids, input_ids_int64, scoring,
                      renormalize, routed_scale, topk_w_out, topk_ids_out, route_status};
  return layer_forward(profile, scale_rule, x, nullptr, 0, nullptr, T, K, E, D, I, expert_table,
                       has_shared ? &sh : nullptr, swiglu_limit, workspace, workspace_bytes, y, stream, &rt);
}

}  // extern "C"
