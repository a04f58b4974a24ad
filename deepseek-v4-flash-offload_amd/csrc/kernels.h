// Internal launcher declarations shared between the kernel files and the C ABI.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

// Per-expert device pointers of one expert's packed MXFP4 weights, in the
// checkpoint layout: w1/w3 [I, D/2] + [I, D/32], w2 [D, I/2] + [D, I/32].
struct Dsv4ExpertPtrs {
  const uint8_t* w1p;
  const uint8_t* w1s;
  const uint8_t* w2p;
  const uint8_t* w2s;
  const uint8_t* w3p;
  const uint8_t* w3s;
};

hipError_t launch_mxfp4_dequant(const uint8_t* packed, const uint8_t* scales, uint16_t* out,
                                int64_t n_elems, hipStream_t st);
// Up to kDequantMaxJobs tensors in one launch; start[j] = first 16-byte packed chunk
// (32 elements) of tensor j in the launch's numbering (start[0] = 0, start[n] = total);
// kc[j] = K/32 chunks per row; tiled[j]: packed in the MFMA-tiled layout (rows % 16 == 0,
// K % 256 == 0) instead of the checkpoint layout.
constexpr int kDequantMaxJobs = 8;
struct Dsv4DequantJobs {
  const uint8_t* packed[kDequantMaxJobs];
  const uint8_t* scales[kDequantMaxJobs];
  uint16_t* out[kDequantMaxJobs];
  int64_t start[kDequantMaxJobs + 1];
  int64_t kc[kDequantMaxJobs];
  int64_t wg_start[kDequantMaxJobs];  // first workgroup of tensor j (set by the launcher)
  int tiled[kDequantMaxJobs];
  int n;
};
hipError_t launch_mxfp4_dequant_multi(const Dsv4DequantJobs& jobs, hipStream_t st);
// packed E2M1 weights [N, K/2] <-> the MFMA-tiled layout (inverse = 1: tiled -> natural)
hipError_t launch_mxfp4_tile(const uint8_t* src, uint8_t* dst, int64_t N, int64_t K, int inverse, hipStream_t st);
// y[M, N] = bf16(x[M, K] @ dequant(packed, scales)^T), fp32 accumulation, M <= 16
hipError_t launch_mxfp4_gemv(const uint16_t* x, int M, const uint8_t* packed, const uint8_t* scales, int N, int K,
                             uint16_t* y, hipStream_t st);
hipError_t launch_fp8_act_quant(const uint16_t* x, int64_t n_elems, uint16_t* rt, uint8_t* codes,
                                float* scale_f32, uint8_t* scale_e8m0x4, hipStream_t st);
hipError_t launch_mxfp4_act_quant(const uint16_t* x, int64_t n_elems, int rule, uint8_t* packed,
                                  uint8_t* scale, uint16_t* dq, hipStream_t st);

struct Dsv4AlignOut {
  int32_t* sorted_ids;          // [max_blocks * block_m] flat index per padded slot, R = pad
  int32_t* block_expert;        // [max_blocks]
  int32_t* num_post_padded;     // [1]
  int32_t* order;               // [R] (nullable) stable argsort of flat expert ids
  int32_t* s_e;                 // [R] (nullable)
  float* s_w;                   // [R] (nullable)
  int32_t* row;                 // [R] (nullable)
  int32_t* counts;              // [E] (nullable)
  int32_t* expert_start;        // [E] (nullable) first padded slot
  int32_t* active;              // [E] (nullable) active experts ascending, -1 tail
  int32_t* num_active;          // [1] (nullable)
  int32_t* padded_pos;          // [R] (nullable) padded slot of each flat index
  int32_t* status;              // [1] (nullable) count of out-of-range expert ids
};
hipError_t launch_moe_align(const void* topk_ids, int ids_int64, const float* topk_w, int R, int K,
                            int E, int block_m, int max_blocks, const Dsv4AlignOut& o, hipStream_t st);

// align (workgroup 0) and activation quantisation (workgroups 1..) in one launch;
// qfmt 0 = FP8 per-128 codes + E8M0 x4 scales, 1 = MXFP4 per-32 (rule 0/1).
// n_shared > 0 adds a group of n_shared rows (flat indices R..) with
// block_expert E ahead of the routed experts; the padding sentinel becomes R + n_shared.
hipError_t launch_moe_align_quant(const void* topk_ids, int ids_int64, const float* topk_w, int R, int K, int E,
                                  int block_m, int max_blocks, const Dsv4AlignOut& o, const uint16_t* x,
                                  int64_t n_elems, int qfmt, int rule, void* q_codes, void* q_scale,
                                  hipStream_t st, int n_shared = 0);
// Second padded layout for experts with many rows: every expert with at least
// hot_min routed entries is laid out here in blocks of kHotBlockM rows (and gets
// no blocks in the main layout). hot_min = 0: none.
constexpr int kHotBlockM = 256;
struct Dsv4AlignHot {
  int hot_min;
  int max_blocks;
  int32_t* sorted_ids;       // [max_blocks * kHotBlockM]
  int32_t* block_expert;     // [max_blocks]
  int32_t* num_post_padded;  // [1]
};
// The same outputs from two launches for many entries: per-chunk counts (plus
// the quantisation of x when x is non-null), then per-chunk layout + scatter. scratch: align_chunked_scratch_bytes(R, E) bytes of device memory.
// hot (nullable): also the hot layout; the main layout's padded_pos then holds
// -1 - (hot position) for the hot experts' entries and expert_start -1 for them.
int64_t align_chunked_scratch_bytes(int R, int E);
hipError_t launch_moe_align_chunked(const void* topk_ids, int ids_int64, const float* topk_w, int R, int K, int E,
                                    int block_m, int max_blocks, const Dsv4AlignOut& o, const uint16_t* x,
                                    int64_t n_elems, int qfmt, int rule, void* q_codes, void* q_scale,
                                    hipStream_t st, int n_shared, void* scratch, const Dsv4AlignHot* hot = nullptr);
hipError_t launch_moe_gather_rows(const uint8_t* src, int64_t n_src, const int32_t* row, int64_t n_rows,
                                  int64_t row_bytes, uint8_t* dst, hipStream_t st);
// y[t] = bf16( sum over the token's entries, ordered by key, of rows of `src` (bf16) )
// mode 0: entry (t,k) -> src row t*K+k, key = topk_ids[t,k]   (flat-order combine)
// mode 1: entries from a per-token position list built from `row`, key = position
// Entries with ids outside [0, E) contribute nothing (E = INT_MAX: every id counts).
hipError_t launch_moe_combine_flat(const uint16_t* src, const void* topk_ids, int ids_int64, int T, int K,
                                   int D, uint16_t* y, hipStream_t st, const uint16_t* shared_rows = nullptr,
                                   int E = 0x7fffffff);
// out[n][k/32] = block[n/128][k/128]: 128x128 E8M0 block scales repeated per 32 along K
hipError_t launch_expand_block_scales(const uint8_t* block, int64_t N, int64_t K, uint8_t* out, hipStream_t st);
hipError_t launch_moe_unpermute_rows(const uint16_t* src, const int32_t* row, int R, int T, int Kmax, int D,
                                     int32_t* work_cnt, int32_t* work_pos, int32_t* status, uint16_t* y,
                                     hipStream_t st);

// A format of the 16- and 64-row grouped GEMMs: bf16 activations (2 bytes/elt, row-major,
// no a_scale) multiplied as they are - no FP8 round trip - against the exactly dequantised
// bf16 weights on the bf16 MFMA, fp32 accumulation (the "pure bf16" variant).
constexpr int kAfmtBf16 = 2;

struct Dsv4GemmArgs {
  int afmt;                       // 0: A is E4M3 codes (1 byte/elt); 1: A is packed E2M1 (2 elts/byte); kAfmtBf16
  const uint8_t* a;               // A codes, row-major
  int64_t a_row_bytes;
  const uint8_t* a_scale;         // E8M0 byte per 32 A elements, row-major [rows, Kdim/32]
  int a_row_div;                  // A row = flat_index / a_row_div (K of top-k for the gate/up GEMM, 1 for down)
  const int32_t* sorted_ids;      // padded slots -> flat index; >= R means padding
  const int32_t* block_expert;    // expert of each M block
  const int32_t* num_post_padded; // device scalar
  int R;
  int block_m;
  int max_blocks;
  const Dsv4ExpertPtrs* experts;  // device table indexed by expert id
  int Kdim;                       // reduction length
  int N;                          // output columns (I for gate/up, D for down)
  const float* topk_w;            // [R] routing weight by flat index (gate/up only)
  float swiglu_limit;             // <= 0 disables the clamp
  uint16_t* out;                  // bf16 [R, N] by flat index (gate/up: h, may be skipped, see hq_mode)
  // ---- gate/up only: quantise h for the down GEMM in the epilogue (zero = off).
  //   hq_mode 1: FP8 per 128 (codes [R, N] + E8M0 x4 [R, N/32]); only where a workgroup
  //   holds all 128 columns of a block (block_m 64/128 kernels). 2: MXFP4 per 32 with rule
  //   hq_rule (packed [R, N/2] + E8M0 [R, N/32]). hq_skip_h: do not write the bf16 h.
  int hq_mode;
  int hq_rule;
  int hq_skip_h;
  uint8_t* hq_codes;
  uint8_t* hq_scale;
  // ---- shared expert as one more group (zero = none; E4M3 activations only).
  //   M blocks whose block_expert is shared_expert read `shared`: E4M3 weights
  //   w1/w3 [N, K] / w2 [D, I] with E8M0 per 32 along K ([N, K/32], the 128x128
  //   block scales repeated). The last shared_a_rows flat indices below R are
  //   shared-expert rows: A row f - (R - shared_a_rows), routing weight 1.
  int has_shared;
  int shared_expert;
  int shared_a_rows;
  Dsv4ExpertPtrs shared;
};
hipError_t launch_moe_gemm_gateup(const Dsv4GemmArgs& a, hipStream_t st);
hipError_t launch_moe_gemm_down(const Dsv4GemmArgs& a, hipStream_t st);
// The large-tile kernel over a hot layout (block_m = kHotBlockM; no shared expert):
// gate/up (with the same epilogue options) or down.
bool moe_gemm_big_supported(int kdim, int n, bool gateup);
hipError_t launch_moe_gemm_big(const Dsv4GemmArgs& a, bool gateup, hipStream_t st);
// MFMA issue-rate probe (probe.hip): shape 0 = 16x16x128, 1 = 32x32x64
hipError_t launch_mfma_rate_probe(int shape, int fmt_a, int fmt_b, int n_wg, int iters, float* out, double* flop,
                                  hipStream_t st);
bool moe_gemm_supported_kdim(int kdim);  // reduction lengths with a compiled kernel (512..4096, powers of two)
bool moe_gemm_supported_block_m(int bm);  // 16 (decode kernel), 64 or 128 (tiled kernel), 256 (large-tile kernel)

// Router top-k of one layer (per-token arguments of route_topk_token).
struct RouteTopkArgs {
  const float* part;  // [S, T, E] partial logits (K chunks)
  int S, T, E, K, scoring;
  const float* bias;
  const void* tid2eid;
  int tid_is64;
  const void* input_ids;
  int ids_is64;
  int64_t vocab;
  int renorm;
  float scale;
  float* out_w;      // [T, K]
  int32_t* out_ids;  // [T, K]
  int32_t* status;
};

// Router: partial logits [S, T, E] in `part`, then scores / top-k / weights.
int route_split_k(int T, int D, int E);
hipError_t launch_moe_route(const void* x, int x_f32, const float* gate_w, int T, int D, int E, int K, int scoring,
                            const float* bias, const void* tid2eid, int tid_is64, const void* input_ids,
                            int ids_is64, int64_t vocab, int renorm, float scale, float* out_w,
                            int32_t* out_ids, int32_t* status, float* part, hipStream_t st);
// The two halves of launch_moe_route: the partial logits (returns the K split S
// through *S), and the per-token top-k over them.
hipError_t launch_route_logits(const void* x, int x_f32, const float* gate_w, int T, int D, int E, float* part,
                               int* S, hipStream_t st);
hipError_t launch_route_topk(const RouteTopkArgs& ra, hipStream_t st);
// Decode-sized routing straight into the layer's first launch: workgroup 0
// selects every token's top-k (ra.out_ids / ra.out_w) and then aligns them,
// workgroups 1.. quantise x (as launch_moe_align_quant; R = T * K <= 2048).
hipError_t launch_route_align_quant(const RouteTopkArgs& ra, int block_m, int max_blocks, const Dsv4AlignOut& o,
                                    const uint16_t* x, int64_t n_elems, int qfmt, int rule, void* q_codes,
                                    void* q_scale, hipStream_t st, int n_shared = 0);
