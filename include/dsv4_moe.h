/* C ABI of libdsv4hip.so - the MI355X (gfx950) routed-MoE expert path.
 *
 * Drop-in boundary for the expert hot path of the DeepSeek-V4 offload plugin.
 * Each entry point names the reference interface it replaces (file:line in the
 * reference repository). Conventions:
 *   - every pointer argument is a device pointer unless stated otherwise;
 *     buffers are owned by the caller (no allocation, no synchronisation);
 *   - `stream` is a hipStream_t passed as void* (NULL = default stream);
 *   - bf16 tensors are 16-bit patterns, row-major, contiguous;
 *   - MXFP4 tensors are the checkpoint layout: [N, K/2] bytes (two E2M1
 *     nibbles per byte, low nibble = even k) plus [N, K/32] E8M0 bytes;
 *   - return value: DSV4_OK (0) or a negative DSV4_ERR_* code, with a message
 *     available from dsv4_last_error() (thread-local).
 */
#ifndef DSV4_MOE_H
#define DSV4_MOE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* 2: dsv4_moe_unpermute gained `status_out` (before `stream`), dsv4_slots_invalidate
 *    gained `compute_stream`, dsv4_moe_layer_forward_noalloc gained `flags` (before
 *    `stream`), GEMM reduction lengths stop at 4096 (8192 dropped).
 *    Callers built against version 1 must not call a version-2 library. */
#define DSV4_ABI_VERSION 2

#define DSV4_MAX_EXPERTS 512
#define DSV4_MAX_TOPK 32
#define DSV4_GEMM_BLOCK_M 16 /* rows per M block for decode-sized calls; the GEMMs also take 64, 128 and 256 */

/* activation formats of the grouped GEMM A operand */
#define DSV4_AFMT_E4M3 0 /* one E4M3fn code per byte, E8M0 per 32 (bf16 profile) */
#define DSV4_AFMT_E2M1 1 /* two E2M1 codes per byte, E8M0 per 32 (a4w4 profile) */
#define DSV4_AFMT_BF16 2 /* bf16 rows as they are (a_scale unused), times the exactly dequantised \
                            bf16 weights on the bf16 MFMA: the pure-bf16 variant; block_m 16, 64 \
                            or 256 */

/* profiles of the routed layer */
#define DSV4_PROFILE_BF16 0 /* deepseek_v4.py:166-197 (FP8 round-trip activations) */
#define DSV4_PROFILE_A4W4 1 /* deepseek_v4.py:199-245 (MXFP4 activations)          */
#define DSV4_PROFILE_BF16_PURE 2 /* the bf16 profile without the FP8 round trips of x and h \
                                    (deepseek_v4.py:170,188 skipped): bf16 x bf16-dequantised \
                                    weights, fp32 accumulation; 16-/64-row blocks as the others */

/* MXFP4 activation scale rules */
#define DSV4_RULE_CEIL_DIV6 0 /* 2^ceil(log2(amax/6)), npu_ops.py:107-121 */
#define DSV4_RULE_OCP_FLOOR 1 /* 2^(floor(log2 amax)-2), OCP MX v1.0      */

/* status codes (csrc/common.h) */
#define DSV4_OK 0
#define DSV4_ERR_NULL (-1)
#define DSV4_ERR_SHAPE (-2)
#define DSV4_ERR_UNSUPPORTED (-3)
#define DSV4_ERR_HIP (-4)
#define DSV4_ERR_STATE (-5)

/* Per-expert weight pointers read by the grouped GEMMs (device array indexed
 * by expert id, 48 bytes per entry). Entries of experts that no token routes
 * to are never read. Packed fields are 16-byte aligned; a packed field whose
 * pointer has bit 0 set (DSV4_TILED_WEIGHTS) is in the MFMA-tiled layout of
 * dsv4_mxfp4_tile_weights instead of the checkpoint layout. The three packed
 * fields of one expert share a layout. */
typedef struct {
  const void* w1p; const void* w1s; /* gate  [I, D/2] + [I, D/32] */
  const void* w2p; const void* w2s; /* down  [D, I/2] + [D, I/32] */
  const void* w3p; const void* w3s; /* up    [I, D/2] + [I, D/32] */
} dsv4_expert_ptrs;
#define DSV4_TILED_WEIGHTS 1 /* OR into a packed-field pointer of dsv4_expert_ptrs */

const char* dsv4_last_error(void);
int dsv4_abi_version(void);

/* MXFP4 weight -> bf16, bit-exact with the reference's torch math.
 * Replaces npu_ops.dequant_fp4_weight (npu_ops.py:142-158).
 * packed [n_rows, k/2], scales [n_rows, k/32], out [n_rows, k]; k % 32 == 0. */
int dsv4_mxfp4_dequant_bf16(const void* packed, const void* scales, void* out, int64_t n_rows, int64_t k,
                            void* stream);

/* Up to 8 MXFP4 weights -> bf16 in one launch, each bit-exact as
 * dsv4_mxfp4_dequant_bf16. Replaces the three npu_ops.dequant_fp4_weight calls
 * with which the reference's ExpertBank.get fills a bf16 expert
 * (offload.py:77-84): w1, w2 and w3 of one expert in one call. `packed`,
 * `scales`, `out`, `n_rows` and `k` are host arrays of `n` (1..8) entries:
 * packed[i] [n_rows[i], k[i]/2], scales[i] [n_rows[i], k[i]/32], out[i]
 * [n_rows[i], k[i]] (device pointers, packed and out 16-byte aligned);
 * k[i] % 32 == 0. A packed pointer with DSV4_TILED_WEIGHTS set is read in the
 * MFMA-tiled layout (n_rows % 16 == 0, k % 256 == 0), as the slot records hold
 * it; the output is the checkpoint layout either way. */
int dsv4_mxfp4_dequant_bf16_multi(int n, const void* const* packed, const void* const* scales, void* const* out,
                                  const int64_t* n_rows, const int64_t* k, void* stream);

/* Packed E2M1 weights [n_rows, k/2] (checkpoint layout, npu_ops.py:142-158) to the
 * MFMA-tiled layout the grouped GEMMs stream fastest, or back (inverse = 1):
 *   tiled[nt][j][ji][g][r][e] = packed[16 nt + r][128 j + 32 g + 16 ji + e]
 * (16-row tiles nt, 256-wide K stages j, e < 16). A GEMM wave's weight load is
 * then one contiguous 1 KB instead of 16 rows x 64 bytes. No counterpart in the
 * reference (its weights stay in the checkpoint layout). n_rows % 16 == 0,
 * k % 256 == 0; src and dst must not overlap. Scales keep their layout. */
int dsv4_mxfp4_tile_weights(const void* src, void* dst, int64_t n_rows, int64_t k, int inverse, void* stream);
/* The same tiling on the host (src, dst: host memory), for records written to a
 * pinned pool before they are copied to the device. */
int dsv4_mxfp4_tile_host(const void* src, void* dst, int64_t n_rows, int64_t k);

/* y[m, n] = bf16(sum_k x[m, k] * dequant(packed, scales)[n, k]) with fp32
 * accumulation: the reference's CPU "dequant_fp4_weight + F.linear" check of a
 * single MXFP4 matrix (npu_ops.py:142-158), x kept in bf16 (no activation
 * quantisation). x bf16 [m, k] (m <= 16), packed [n, k/2], scales [n, k/32],
 * y bf16 [m, n]; k > 0, k % 32 == 0. */
int dsv4_mxfp4_gemv_bf16(const void* x, int m, const void* packed, const void* scales, int n, int k, void* y,
                         void* stream);

/* Per-128 FP8 E4M3 activation quantisation with power-of-two scales.
 * Replaces npu_ops.act_quant (npu_ops.py:73-104): `rt` receives the inplace
 * round trip (what act_quant(x, 128, "ue8m0", None, True) writes), `codes` the
 * E4M3fn bytes, `scale_f32` the fp32 scale per block ([rows, cols/128]) and
 * `scale_e8m0x4` the E8M0 byte of the block repeated for each 32 elements
 * ([rows, cols/32]). Any output may be NULL (at least one must not be). */
int dsv4_fp8_act_quant(const void* x, int64_t rows, int64_t cols, int block_size, void* rt, void* codes,
                       void* scale_f32, void* scale_e8m0x4, void* stream);

/* Per-32 MXFP4 activation quantisation: packed [rows, cols/2], E8M0 scale
 * [rows, cols/32], optional bf16 dequantised view `dq` [rows, cols].
 * rule DSV4_RULE_CEIL_DIV6 replaces npu_ops.fp4_act_quant (npu_ops.py:107-121;
 * `dq` is its inplace result); rule DSV4_RULE_OCP_FLOOR replaces the call sites
 * of torch_npu.npu_dynamic_mx_quant (deepseek_v4.py:212, 240). */
int dsv4_mxfp4_act_quant(const void* x, int64_t rows, int64_t cols, int rule, void* packed, void* scale, void* dq,
                         void* stream);

/* Router of one MoE layer, OffloadDeepseekV4MoE._route (deepseek_v4.py:118-148):
 *   logits = float(x) @ gate_wᵀ (fp32), scores = softmax (scoring 0) | sigmoid (1)
 *   | sqrt(softplus) (2, threshold 20 as F.softplus); ids = top-K of scores + bias
 *   (bias NULL: none), or on hash layers (tid2eid non-NULL) ids[t] =
 *   tid2eid[input_ids[t]] with tid2eid [vocab, K] int32/int64; out_w = scores[ids],
 *   divided by their sum when renormalize, times scale (routed_scaling_factor).
 * x [T, D] bf16 (x_f32 = 0) or fp32 (1); gate_w fp32 [E, D]; out_w fp32 [T, K]; out_ids int32 [T, K], each
 * token's ids in descending biased score with ties to the lower id (the reference's
 * topk(sorted=False) leaves order and tie rule open), or in table order on hash
 * layers. status [1] (nullable, zeroed by the caller) is incremented once per input
 * id outside [0, vocab) and per table entry outside [0, E); such picks get id -1
 * and weight 0.
 * Limits: D % 32 == 0, E % 16 == 0, 16 <= E <= 512, 1 <= K <= min(E, 64).
 * workspace: dsv4_moe_route_workspace_bytes(T, D, E) bytes (partial logits). */
int64_t dsv4_moe_route_workspace_bytes(int T, int D, int E);
int dsv4_moe_route(const void* x, int x_f32, const float* gate_w, const float* bias, const void* tid2eid,
                   int tid2eid_int64, int64_t vocab, const void* input_ids, int input_ids_int64, int T, int D, int E,
                   int K, int scoring, int renormalize, float scale, float* out_w, int32_t* out_ids, int32_t* status,
                   void* workspace, void* stream);

/* Upper bound of padded M blocks for R routed entries (host function). */
int dsv4_moe_align_max_blocks(int R, int E, int block_m);

/* Stable sort of the T*K routed entries by expert, with counts and the padded
 * block layout. Replaces the inline sort/count of deepseek_v4.py:155-164
 * (flat_e, argsort -> order, s_e, s_w, row = order // K, bincount -> counts,
 * nonzero -> active). Order is (expert asc, flat index asc) = argsort(stable).
 * topk_ids: [T, K] int32 or int64 (ids_int64 = 1). topk_w: [T, K] fp32 or NULL.
 * Required outputs: sorted_ids [max_blocks*block_m] (flat index t*K+k of each
 * padded slot, T*K marks padding), block_expert [max_blocks], num_post_padded
 * [1]. Optional (NULL to skip): order, s_e, s_w, row [T*K]; counts,
 * expert_start (first padded slot), active (ascending, -1 tail) [E];
 * num_active [1]; padded_pos [T*K] (padded slot of each flat index); status
 * [1] (number of out-of-range ids, plus 2^30 if max_blocks was too small). */
int dsv4_moe_align(const void* topk_ids, int ids_int64, const float* topk_w, int T, int K, int E, int block_m,
                   int max_blocks, int32_t* sorted_ids, int32_t* block_expert, int32_t* num_post_padded,
                   int32_t* order, int32_t* s_e, float* s_w, int32_t* row, int32_t* counts, int32_t* expert_start,
                   int32_t* active, int32_t* num_active, int32_t* padded_pos, int32_t* status, void* stream);

/* dsv4_moe_align with a workspace (dsv4_moe_align_workspace_bytes(T, K, E) bytes):
 * above 2048 entries the work is split over chunks of 1024 entries in two
 * launches (per-chunk counts; per-chunk layout and stable scatter) instead of
 * one workgroup; same outputs, bit for bit. A NULL workspace or at
 * most 2048 entries: the single-workgroup dsv4_moe_align. */
int64_t dsv4_moe_align_workspace_bytes(int T, int K, int E);
int dsv4_moe_align_ws(const void* topk_ids, int ids_int64, const float* topk_w, int T, int K, int E, int block_m,
                      int max_blocks, int32_t* sorted_ids, int32_t* block_expert, int32_t* num_post_padded,
                      int32_t* order, int32_t* s_e, float* s_w, int32_t* row, int32_t* counts,
                      int32_t* expert_start, int32_t* active, int32_t* num_active, int32_t* padded_pos,
                      int32_t* status, void* workspace, int64_t workspace_bytes, void* stream);

/* dst[i] = src[row[i]] for rows of row_bytes bytes (multiple of 16); src has
 * n_src rows and a row index outside [0, n_src) yields a zero row.
 * Replaces the gathers x_sorted = xq[row] (deepseek_v4.py:171, 213-214). */
int dsv4_moe_permute(const void* src, int64_t n_src, const int32_t* row, int64_t n_rows, int64_t row_bytes,
                     void* dst, void* stream);

/* y = bf16(zeros(T, D) fp32 .index_add_(0, row, out_sorted.float())), summed in
 * ascending sorted position per token, bit-exact. Replaces
 * deepseek_v4.py:195-197 / 243-245. Kmax (1..DSV4_UNPERMUTE_MAX_ROWS) bounds the
 * rows any one token may receive; a row beyond that bound, or whose token is
 * outside [0, T), is dropped and counted in `status` (device int32 [1],
 * overwritten; nullable), where index_add_ would have summed it or raised.
 * workspace: dsv4_moe_unpermute_workspace_bytes(T, Kmax) bytes of device memory. */
#define DSV4_UNPERMUTE_MAX_ROWS 64
int64_t dsv4_moe_unpermute_workspace_bytes(int T, int Kmax);
int dsv4_moe_unpermute(const void* out_sorted, const int32_t* row, int R, int T, int Kmax, int D, void* workspace,
                       void* y, int32_t* status, void* stream);

/* Same combine for rows stored by flat index (row t*K+k = the k-th pick of
 * token t): each token's rows are summed in ascending expert id, which is the
 * order index_add_ visits them in. Used by the fused layer. */
int dsv4_moe_combine(const void* out_flat, const void* topk_ids, int ids_int64, int T, int K, int D, void* y,
                     void* stream);

/* Grouped gate/up GEMM over all routed rows in one launch, fused with the
 * SwiGLU epilogue of deepseek_v4.py:184-187: h[f] = silu(min(g,L)) *
 * clamp(u,-L,L) * topk_w[f] where g/u are the bf16-rounded GEMM outputs.
 * Replaces the two npu_grouped_matmul calls of deepseek_v4.py:177-182
 * (afmt E4M3) / 231-232 (afmt E2M1). A rows are gathered on load: padded slot
 * p reads A row sorted_ids[p] / a_row_div. a: [rows, D] codes (E4M3) or
 * [rows, D/2] (E2M1), a_scale [rows, D/32]. h_out: bf16 [R, I] by flat index.
 * block_m (the moe_align block size) is 16 (single-wave workgroups, decode),
 * 64 or 128 (LDS-tiled workgroups: each weight fragment serves 4 or 8 row
 * tiles) or 256 (large-tile workgroups: 32x32x64 scaled MFMAs for E4M3/E2M1
 * A, 32x32x16 bf16 MFMAs on weights dequantised in registers for bf16 A; D a
 * multiple of 1024 for gate/up, I of 1024 and D of 256 for down); D and I must
 * be 256 * 2^n (512..4096) and I a multiple of 128. */
int dsv4_moe_gemm_gateup(int afmt, const void* a, const void* a_scale, int a_row_div, const int32_t* sorted_ids,
                         const int32_t* block_expert, const int32_t* num_post_padded, int R, int block_m,
                         int max_blocks, const void* expert_table, int D, int I, const float* topk_w,
                         float swiglu_limit, void* h_out, void* stream);

/* Grouped down GEMM: out[f] = bf16(a[f] @ W2[e]^T) for every routed row.
 * Replaces npu_grouped_matmul of deepseek_v4.py:190-193 / 241.
 * a: [R, I] (E4M3) or [R, I/2] (E2M1) by flat index, a_scale [R, I/32]. */
int dsv4_moe_gemm_down(int afmt, const void* a, const void* a_scale, const int32_t* sorted_ids,
                       const int32_t* block_expert, const int32_t* num_post_padded, int R, int block_m,
                       int max_blocks, const void* expert_table, int I, int D, void* out, void* stream);

/* The whole routed expert computation of one layer, i.e. the body of
 * OffloadDeepseekV4MoE._routed (deepseek_v4.py:150-197, profile BF16) or
 * _routed_mxfp4 (deepseek_v4.py:199-245, profile A4W4) after routing:
 * moe_align -> activation quant -> gate/up GEMM + SwiGLU -> h quant -> down
 * GEMM -> combine, as 4-5 launches on `stream` (align and the quantisation of
 * x share one; h is quantised in the gate/up epilogue except for the FP8
 * profile below 2048 routed rows). M blocks of 16 rows below 2048 routed rows,
 * 64 from there on. x [T, D] bf16, topk_ids/topk_w [T, K], y [T, D] bf16.
 * scale_rule applies to the A4W4 profile only. The workspace (size from
 * dsv4_moe_layer_workspace_bytes, 256-byte aligned) needs no initialisation.
 * A routed entry whose id is outside [0, E) contributes nothing (the
 * reference's engine lookup raises for it; check ids with dsv4_moe_align's
 * status where that matters), and an expert whose table entry holds null
 * weight pointers contributes zeros. */
int dsv4_moe_layer_workspace_bytes(int T, int K, int E, int D, int I, int profile, int64_t* bytes);
int dsv4_moe_layer_forward(int profile, int scale_rule, const void* x, const void* topk_ids, int ids_int64,
                           const float* topk_w, int T, int K, int E, int D, int I, const void* expert_table,
                           float swiglu_limit, void* workspace, int64_t workspace_bytes, void* y, void* stream);

/* dsv4_moe_layer_forward without a workspace argument and without allocating:
 * no counterpart in the reference. For callers that cannot allocate device
 * memory (code under HIP graph capture, serving loops, harnesses that forbid
 * hipMalloc). The workspace is a static device array of
 * DSV4_NOALLOC_SCRATCH_BYTES (64 MiB) that each GPU the library runs on holds
 * until the process ends; a call whose dsv4_moe_layer_workspace_bytes exceeds
 * it returns DSV4_ERR_UNSUPPORTED (about 500 tokens at top-8, hidden 4096,
 * inter 2048). The array is per device and shared by every call on it, and
 * keeps the last call's contents. Calls on one stream are ordered by it; calls
 * that overlap on one GPU (different streams, not ordered by the caller) race.
 * The library remembers the stream of each device's last call and rejects
 * (DSV4_ERR_STATE, before anything is enqueued) a call from another stream
 * unless `flags` holds DSV4_NOALLOC_STREAMS_ORDERED: the caller's promise that
 * this call is ordered after every earlier call on the device (a synchronize,
 * or an event the new stream waits for). Outputs equal dsv4_moe_layer_forward's
 * bit for bit. */
#define DSV4_NOALLOC_SCRATCH_BYTES (64 << 20)
#define DSV4_NOALLOC_STREAMS_ORDERED 1
int dsv4_moe_layer_forward_noalloc(int profile, int scale_rule, const void* x, const void* topk_ids, int ids_int64,
                                   const float* topk_w, int T, int K, int E, int D, int I, const void* expert_table,
                                   float swiglu_limit, void* y, int flags, void* stream);

/* The same layer with the shared expert folded in as one more group of the
 * grouped GEMMs (bf16 profile): OffloadDeepseekV4MoE.forward's
 * `out = self._routed(hs) + self.shared_experts(hs)` (deepseek_v4.py:262-264)
 * with shared_experts = model_npu.py:469-489 Expert(mode="fp8"): the FP8
 * round trip of x, E4M3 weights dequantised by 128x128 E8M0 block scales
 * (npu_ops.py:161-167), SwiGLU with swiglu_limit and no routing weight, the
 * FP8 round trip of h, and the down projection. The shared rows (flat indices
 * T*K .. T*K+T-1) run in the same launches as the routed ones; y =
 * bf16(bf16(routed sum) + shared row). sw1, sw3: E4M3 [I, D]; sw2: E4M3 [D, I];
 * sw1s, sw3s: E8M0 [I, D/32]; sw2s: E8M0 [D, I/32], the block scales repeated
 * per 32 along K (dsv4_expand_block_scales). */
int dsv4_moe_layer_shared_workspace_bytes(int T, int K, int E, int D, int I, int64_t* bytes);
int dsv4_moe_layer_forward_shared(const void* x, const void* topk_ids, int ids_int64, const float* topk_w, int T,
                                  int K, int E, int D, int I, const void* expert_table, const void* sw1,
                                  const void* sw1s, const void* sw3, const void* sw3s, const void* sw2,
                                  const void* sw2s, float swiglu_limit, void* workspace, int64_t workspace_bytes,
                                  void* y, void* stream);

/* The routed layer with its router: OffloadDeepseekV4MoE._routed(hs, input_ids)
 * (deepseek_v4.py:150-245) including its _route call (deepseek_v4.py:118-148),
 * and, with the six shared-expert pointers set (all null = none; bf16 profile
 * only), forward's `+ shared_experts(hs)` as in dsv4_moe_layer_forward_shared.
 * Routing arguments and outputs are those of dsv4_moe_route (x bf16 only);
 * topk_w_out / topk_ids_out receive the routing [T, K] the layer used. Up to 16
 * tokens, the router's top-k, the expert layout (moe_align) and the
 * quantisation of x run in one launch after the logits (the routed ids never
 * wait for a launch boundary); larger batches route in the router's two
 * launches first. The outputs equal dsv4_moe_route followed by
 * dsv4_moe_layer_forward(_shared) on its ids, bit for bit.
 * workspace: dsv4_moe_routed_layer_workspace_bytes(T, K, E, D, I, profile,
 * with_shared) bytes. */
int dsv4_moe_routed_layer_workspace_bytes(int T, int K, int E, int D, int I, int profile, int with_shared,
                                          int64_t* bytes);
int dsv4_moe_routed_layer_forward(int profile, int scale_rule, const void* x, int T, int K, int E, int D, int I,
                                  const float* gate_w, const float* bias, const void* tid2eid, int tid2eid_int64,
                                  int64_t vocab, const void* input_ids, int input_ids_int64, int scoring,
                                  int renormalize, float routed_scale, const void* expert_table, const void* sw1,
                                  const void* sw1s, const void* sw3, const void* sw3s, const void* sw2,
                                  const void* sw2s, float swiglu_limit, float* topk_w_out, int32_t* topk_ids_out,
                                  int32_t* route_status, void* workspace, int64_t workspace_bytes, void* y,
                                  void* stream);

/* out[n][j] = block_scales[n / 128][j / 4] for n < n_rows, j < k/32: the
 * 128x128 block scales of an FP8 weight [n_rows, k] (npu_ops.py:161-167,
 * dequant_fp8_weight) repeated per 32 along K, the layout the grouped GEMMs
 * read. block_scales: [ceil(n_rows/128), ceil(k/128)] E8M0; k % 32 == 0. */
int dsv4_expand_block_scales(const void* block_scales, int64_t n_rows, int64_t k, void* out, void* stream);

/* ------------------------------------------------------------------------
 * Expert slot cache (replaces ExpertBank's device caches, offload.py:22-151).
 * One device slot pool (caller-allocated, n_slots * record_bytes, 256-byte
 * aligned) + pinned host records (one per registered (layer, expert), the
 * expert's six packed tensors at fixed offsets) + a side copy stream.
 * ------------------------------------------------------------------------ */
typedef struct dsv4_slots dsv4_slots;

/* Pure LRU over `capacity` slots, host only (the policy of offload.py:86-100:
 * hit -> most recent, miss -> free slot or evict least recent; capacity 0
 * never caches). *hit = 1/0; *evicted = evicted key or -1. */
int dsv4_lru_create(int capacity, void** out);
int dsv4_lru_destroy(void* lru);
int dsv4_lru_access(void* lru, int64_t key, int* hit, int* slot, int64_t* evicted);
int dsv4_lru_keys(void* lru, int64_t* out, int max, int* n); /* least -> most recent */

/* pin_host: allocate host records page-locked (hipHostMalloc); on failure the
 * manager degrades to pageable memory, as ExpertBank.register does
 * (offload.py:62-67). */
int dsv4_slots_create(int device, int64_t record_bytes, int n_slots, void* device_pool, int pin_host,
                      dsv4_slots** out);
int dsv4_slots_destroy(dsv4_slots* s);
/* Host record of (layer, eid); create=1 allocates it (ExpertBank.register,
 * offload.py:59-68). *pinned tells whether it is page-locked. */
int dsv4_slots_host_record(dsv4_slots* s, int layer, int eid, int create, void** record, int* pinned);
int dsv4_slots_num_registered(dsv4_slots* s, int64_t* n);
/* Makes the n experts of `layer` resident and returns their slots (the batched
 * form of ExpertBank.get_packed, offload.py:103-129). Misses are copied on the
 * side copy stream; `compute_stream` waits for the copies the returned slots
 * depend on. Slots returned by the previous acquire are released first (their
 * readers are the work enqueued on compute_stream before this call). */
int dsv4_slots_acquire(dsv4_slots* s, int layer, const int32_t* eids, int n, void* compute_stream,
                       int32_t* slots, int* n_miss);
/* Starts copies for the non-resident experts of a later batch (no waits) and
 * sets *n_issued to the number started. The slots the last acquire returned
 * are never evicted for it (their readers may not be enqueued yet); when only
 * those are left the prefetch stops early. */
int dsv4_slots_prefetch(dsv4_slots* s, int layer, const int32_t* eids, int n, int* n_issued);
int dsv4_slots_release(dsv4_slots* s, void* compute_stream);
int dsv4_slots_copy_record(dsv4_slots* s, int layer, int eid, void* dst, void* stream);
int dsv4_slots_lookup(dsv4_slots* s, int layer, int eid, int32_t* slot);
int dsv4_slots_keys(dsv4_slots* s, int64_t* out, int max, int* n);
int dsv4_slots_sync(dsv4_slots* s);
/* Drops every resident expert (ExpertBank.invalidate, offload.py:131-133). The
 * slots of the last acquire are released on `compute_stream` first, so copies
 * into them made after this call wait for the reads already enqueued there. */
int dsv4_slots_invalidate(dsv4_slots* s, void* compute_stream);
/* stats[9] = hits, misses, evictions, prefetched, bytes_h2d, copies, cached, capacity, pinned */
int dsv4_slots_stats(dsv4_slots* s, int64_t* stats);
int dsv4_slots_reset_stats(dsv4_slots* s);

/* ---- Measurement helper (no counterpart in the reference) -------------------
 * One launch of an MFMA issue-rate loop, for the roofline of the grouped GEMMs:
 * n_wg workgroups of 4 waves, each wave running `iters` iterations of
 * independent chains of v_mfma_scale_f32_16x16x128_f8f6f4 (shape 0) or
 * v_mfma_scale_f32_32x32x64_f8f6f4 (shape 1) on register operands (no memory
 * traffic in the loop). fmt_a / fmt_b: DSV4_AFMT_E4M3 (0) or DSV4_AFMT_E2M1
 * (4); the pairs E2M1 x E2M1, E4M3 x E2M1 and E4M3 x E4M3. out: n_wg * 256
 * floats of device memory (one result per thread, so nothing is optimised
 * away). *flop (nullable): the dense FLOPs the launch performs. */
int dsv4_probe_mfma_rate(int shape, int fmt_a, int fmt_b, int n_wg, int iters, float* out, double* flop,
                         void* stream);

#ifdef __cplusplus
}
#endif

#endif /* DSV4_MOE_H */
