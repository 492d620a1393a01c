/*
 * mi_qmm.h -- C ABI of the MI355X (gfx950) affine quantized-matmul library.
 *
 * Drop-in boundary for the mlx-c calls that ddalcu/mlx-serve makes for every
 * quantized linear layer and MoE expert. Each entry point names the mlx-c
 * function it replaces (declared in the reference at src/mlx.zig). The argument
 * order follows the mlx-c call; mlx_array handles become raw device pointers
 * plus explicit shapes, and mlx_stream becomes a hipStream_t passed as void*.
 *
 * Conventions
 *   - All tensor arguments are DEVICE pointers to row-contiguous memory.
 *     Packed weights are uint32 [.., N, K*bits/32]; scales/biases [.., N, K/group_size].
 *   - Calls are asynchronous on `stream` (NULL = the default stream) and never
 *     synchronize the host. Indices may stay GPU-resident.
 *   - Return 0 on success. MI_ERR_UNSUPPORTED means "this library declines the
 *     call; use your fallback" (the reference expresses this by returning null
 *     from its kernel wrappers, src/transformer.zig:20317-20358). Other non-zero
 *     codes are errors, like mlx.check()'s error.MlxError (src/mlx.zig:547-550).
 *     mi_last_error() returns a thread-local message for the last failure.
 *   - dtype codes are mlx_dtype's values (src/mlx.zig:20-35).
 */
#ifndef MI_QMM_H
#define MI_QMM_H
#include <stdbool.h>
#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum {
  MI_OK = 0,
  MI_ERR_UNSUPPORTED = 1, /* decline: valid request outside this library's scope */
  MI_ERR_INVALID = 2,     /* bad pointer / shape / argument */
  MI_ERR_HIP = 3,         /* HIP runtime error (launch, allocation) */
  MI_ERR_WORKSPACE = 4,   /* workspace must grow but the stream is capturing */
};

/* Values match mlx_dtype (src/mlx.zig:20-35). */
enum {
  MI_DTYPE_UINT8 = 1,
  MI_DTYPE_UINT32 = 3,
  MI_DTYPE_FLOAT16 = 9,
  MI_DTYPE_FLOAT32 = 10,
  MI_DTYPE_BFLOAT16 = 12,
};

/* Mirrors mlx_optional_int (src/mlx.zig:40-50). has_value=false -> MLX default
 * (group_size 64, bits 4). */
typedef struct {
  int value;
  bool has_value;
} mi_optional_int;

/* Replaces mlx_quantized_matmul (src/mlx.zig:262), mode "affine", transpose=true:
 *   y[M,N] = x[M,K] @ dequant(w)[N,K]^T, dequant(w) = scale*q + bias per group.
 * x: x_dtype in {bfloat16, float32}; y has x's dtype. scales/biases: sb_dtype
 * bfloat16. bits in {2,3,4,5,6,8} (2/3/5/6: bfloat16 x only); group_size in
 * {32,64,128}; K % group_size == 0. Codes are one LSB-first bitstream per row (for 4
 * and 8 bits: value j of a word at bits j*bits).
 * mode "nvfp4" (4-bit e2m1, gs 16, e4m3 scales), "mxfp4" (4-bit e2m1, gs 32, e8m0
 * scales), "mxfp8" (8-bit e4m3, gs 32, e8m0 scales): bias-less (biases may be NULL),
 * scales MI_DTYPE_UINT8, x bfloat16; group_size/bits default to the mode's and must
 * match it. transpose=false and other modes return MI_ERR_UNSUPPORTED. */
int mi_quantized_matmul(void* y, const void* x, const uint32_t* w, const void* scales,
                        const void* biases, int64_t M, int64_t N, int64_t K, bool transpose,
                        mi_optional_int group_size, mi_optional_int bits, const char* mode,
                        int x_dtype, int sb_dtype, void* stream);

/* Replaces mlx_gather_qmm (src/mlx.zig:265), transpose=true, mode "affine":
 *   y[i] = x[lhs(i)] @ dequant(w[rhs(i)])^T      for i in [0, n_idx)
 * x: [x_batch, M, K]; w: [n_experts, N, K*bits/32]; scales/biases [n_experts, N, K/gs];
 * y: [n_idx, M, N]. Formats as mi_quantized_matmul; affine 2/3/5/6 bits at group sizes
 * other than 64 take at most 8 rows per pair, and they and the fp modes take bfloat16 x
 * only (else MI_ERR_UNSUPPORTED).
 * lhs_indices may be NULL: lhs(i) = i / lhs_div (lhs_div=1 is MLX's
 * default arange; lhs_div=top_k is one token broadcast over its top-k slots, the
 * reference's decode call). rhs_indices may be NULL: rhs(i) = i.
 * Indices are uint32 device arrays. sorted_indices=true groups consecutive equal
 * rhs values into one weight pass per run (any order stays correct; sorted order
 * is what makes it fast). Out-of-range indices write NaN rows, never read out of
 * bounds. Uses the per-device workspace (mi_workspace_reserve) for sorted work lists
 * and split-K partials. */
int mi_gather_qmm(void* y, const void* x, const uint32_t* w, const void* scales,
                  const void* biases, const uint32_t* lhs_indices, const uint32_t* rhs_indices,
                  int64_t n_idx, int64_t lhs_div, int64_t x_batch, int64_t M, int64_t N, int64_t K,
                  int64_t n_experts, bool transpose, mi_optional_int group_size,
                  mi_optional_int bits, const char* mode, bool sorted_indices, int x_dtype,
                  int sb_dtype, void* stream);

/* mi_gather_qmm without any device allocation. No counterpart in the reference: it is
 * for callers that cannot allocate (code under HIP graph capture, tight serving loops,
 * harnesses that forbid hipMalloc). Same arguments, results and kernels as
 * mi_gather_qmm; its work items and K-split partials live in a fixed per-device scratch
 * array of MI_GATHER_NOALLOC_SCRATCH_BYTES (64 MiB) inside the library: the array is
 * part of the library's code object, so it is reserved on every device when the library
 * loads (whether or not this entry point is called) and held until the process ends. A
 * call that would need more returns MI_ERR_WORKSPACE. Every call on a
 * device shares that device's scratch: calls that overlap on one device (different
 * streams, or concurrent host threads) race and must not be issued. */
#define MI_GATHER_NOALLOC_SCRATCH_BYTES ((int64_t)64 << 20)
int mi_gather_qmm_noalloc(void* y, const void* x, const uint32_t* w, const void* scales,
                          const void* biases, const uint32_t* lhs_indices,
                          const uint32_t* rhs_indices, int64_t n_idx, int64_t lhs_div,
                          int64_t x_batch, int64_t M, int64_t N, int64_t K, int64_t n_experts,
                          bool transpose, mi_optional_int group_size, mi_optional_int bits,
                          const char* mode, bool sorted_indices, int x_dtype, int sb_dtype,
                          void* stream);

/* Replaces mlx_dequantize (src/mlx.zig:271), same argument order (mlx_array handles become
 * pointers plus rows/K; the optional output dtype becomes out_dtype):
 *   affine: out[r,k] = scale[r,k/gs] * q[r,k] + bias[r,k/gs]
 * Modes "nvfp4" / "mxfp4" / "mxfp8" (uint8 scales, no biases): out = element(q) * scale,
 * exact in float32 and bfloat16. global_scale (nullable device pointer to one fp32, nvfp4
 * only; the reference passes none at every call site): out = (element(q) * scale) *
 * global_scale, the first product exact, one rounding. NULL for the other modes, else
 * MI_ERR_INVALID.
 * out_dtype float32: exact fp32 result. out_dtype bfloat16: rounded like MLX's
 * composed dequantize (a bf16 multiply then a bf16 add). */
int mi_dequantize(void* out, const uint32_t* w, const void* scales, const void* biases,
                  int64_t rows, int64_t K, mi_optional_int group_size, mi_optional_int bits,
                  const char* mode, const float* global_scale, int sb_dtype, int out_dtype,
                  void* stream);

/* Same as mi_dequantize with an explicit bf16 rounding: rounding 0 = one rounding
 * of s*q+b, 1 = op-by-op (the mi_dequantize default). No mlx-c counterpart: MLX's
 * rounding of a bf16 dequantize is not pinned by any data available to this
 * build, so both are offered. */
int mi_dequantize_rounding(void* out, const uint32_t* w, const void* scales, const void* biases,
                           int64_t rows, int64_t K, mi_optional_int group_size,
                           mi_optional_int bits, const char* mode, const float* global_scale,
                           int sb_dtype, int out_dtype, int rounding, void* stream);

/* Replaces mlx_quantize (src/mlx.zig:275), mode "affine", same argument order: w [rows,K]
 * (bfloat16 or float32) -> packed uint32 wq, scales/biases in bfloat16. global_scale must
 * be NULL (it belongs to nvfp4 quantization, which this library does not perform; the
 * reference passes none). */
int mi_quantize(uint32_t* wq, void* scales, void* biases, const void* w, int64_t rows, int64_t K,
                mi_optional_int group_size, mi_optional_int bits, const char* mode,
                const float* global_scale, int w_dtype, void* stream);

/* Solve (bits, group_size) from packed geometry, as affineParamsFromGeometry
 * (src/transformer.zig:16763-16782): bits = w_cols*32/in_dim, gs = in_dim/s_cols.
 * Returns 0, or MI_ERR_INVALID when the geometry is not an affine layout. Host only. */
int mi_affine_params_from_geometry(int64_t w_cols, int64_t s_cols, int64_t in_dim, int* bits,
                                   int* group_size);

/* Synthetic-input generator used by the benchmark (no reference counterpart):
 * out[i] = mean + std * N(0,1) as bfloat16 (dtype bfloat16) or float32, from a
 * counter-based SplitMix64 + Box-Muller stream keyed by seed. */
int mi_fill_randn(void* out, int64_t n, uint64_t seed, float mean, float stddev, int dtype,
                  void* stream);

/* ---------------------------------------------------------------- MoE glue ---
 * The steps on either side of gather_qmm in the reference's MoE layer (moeMLP2,
 * src/transformer.zig:14822-15192), on the GPU so the grouped launch needs no host sync. */

/* Replaces moeRoutingChain (src/transformer.zig:17022-17072): softmax over E fp32 logits
 * per token, top-k, weights renormalized over the k selected. inds/scores [T, k]; scores
 * in scores_dtype (float32, or bfloat16 rounded once). Slots are ordered by descending
 * logit, ties to the lower expert id (MLX's argpartition leaves the order unspecified).
 * E <= 1024, k <= min(64, E). */
int mi_moe_route_topk(uint32_t* inds, void* scores, const float* logits, int64_t T, int64_t E,
                      int k, int scores_dtype, void* stream);

/* Replaces groupLimitedRouting (src/transformer.zig:17242-17347; group mask groupLimitMask
 * :17138-17236), the DeepSeek-style router: fp32 logits [T, E] and expert bias [E] ->
 * inds [T, k] (descending masked key, ties to the lower id) and fp32 weights [T, k]:
 * sigmoid scores, +bias, groups of E/n_group ranked by the sum of their two largest biased
 * values, all but the topk_group best masked to -1e4, top-k of that; weights are the
 * unbiased scores of the selected, / (slot-order sum + 1e-20) when route_norm and k > 1,
 * times route_scale. E <= 1024, n_group <= 64, k <= min(64, E). */
int mi_moe_route_grouped(uint32_t* inds, float* scores, const float* logits, const float* bias,
                         int64_t T, int64_t E, int k, int n_group, int topk_group, bool route_norm,
                         float route_scale, void* stream);

/* Replaces the sort steps of the sorted MoE path (src/transformer.zig:14965-14993):
 * order = stable argsort(flat), inv = argsort(order), sorted = flat[order],
 * lhs = order / k. seg_offsets (may be NULL) receives n_experts+1 entries: the first
 * sorted position of each expert, then the number of in-range ids. Ids >= n_experts
 * sort last in index order. One block; n_experts <= 8192. */
int mi_moe_sort_dispatch(uint32_t* order, uint32_t* inv, uint32_t* sorted, uint32_t* lhs,
                         uint32_t* seg_offsets, const uint32_t* flat, int64_t n, int k,
                         int64_t n_experts, void* stream);

/* Replaces mlx_take_axis(axis 0) on row-major rows, as used to undo the expert sort
 * (src/transformer.zig:15037): out[r] = in[indices[r]]; rows of row_bytes bytes; indices
 * >= n_src give zero rows. n <= 65535 rows per call. */
/* mi_gather_qmm followed by mi_swiglu(gate, product) in one call: the up projection of the
 * sorted MoE path and its activation (src/transformer.zig:15009-15023), with the SwiGLU of :19846-19884 applied
 * as the product is written. gate has y's shape ([n_idx, M, N] bf16) and must not alias y.
 * Affine 4- and 8-bit weights, bf16 activations; other arguments as mi_gather_qmm.
 * Bit-equal to the two calls. */
int mi_gather_qmm_swiglu(void* y, const void* gate, const void* x, const uint32_t* w,
                         const void* scales, const void* biases, const uint32_t* lhs_indices,
                         const uint32_t* rhs_indices, int64_t n_idx, int64_t lhs_div,
                         int64_t x_batch, int64_t M, int64_t N, int64_t K, int64_t n_experts,
                         bool transpose, mi_optional_int group_size, mi_optional_int bits,
                         const char* mode, bool sorted_indices, int x_dtype, int sb_dtype,
                         void* stream);

/* Both projections before the activation of the sorted MoE path (src/transformer.zig:
 * 15009-15023: the gate and up gather_qmm calls and the SwiGLU after them) in one call:
 * y = SwiGLU(gather_qmm(x, w_gate, ...), gather_qmm(x, w_up, ...)), each product rounded to
 * bf16 first. Both banks share the indices, shapes and format; arguments otherwise as
 * mi_gather_qmm. On the grouped kernel and on one-row items this is one launch over both
 * banks; bit-equal to the split calls (mi_gather_qmm for gate, then mi_gather_qmm_swiglu for
 * up). Affine 4- and
 * 8-bit weights, bf16 activations. */
int mi_gather_qmm_gate_up_swiglu(void* y, const void* x, const uint32_t* w_gate,
                                 const void* s_gate, const void* b_gate, const uint32_t* w_up,
                                 const void* s_up, const void* b_up,
                                 const uint32_t* lhs_indices, const uint32_t* rhs_indices,
                                 int64_t n_idx, int64_t lhs_div, int64_t x_batch, int64_t M,
                                 int64_t N, int64_t K, int64_t n_experts, bool transpose,
                                 mi_optional_int group_size, mi_optional_int bits,
                                 const char* mode, bool sorted_indices, int x_dtype,
                                 int sb_dtype, void* stream);

int mi_take_rows(void* out, const void* in, const uint32_t* indices, int64_t n, int64_t n_src,
                 int64_t row_bytes, void* stream);

/* Replaces fusedSwiGLU (src/transformer.zig:19846-19884): y = bf16(bf16(g*sig(g)) * u),
 * sig(g) the sigmoid of the bf16 value g rounded to fp32 then bf16 (a table over every
 * bf16 pattern in the reference). dtype bfloat16 only. */
int mi_swiglu(void* y, const void* gate, const void* up, int64_t n, int dtype, void* stream);

/* The score-weighted sum over the k slots of each token (src/transformer.zig:15127-15140,
 * the composed pair gatherQmvDownReduce replicates at :20612-20621):
 * y[t, n] = sum_{s ascending} bf16(v[t*k+s, n] * score[t*k+s]), each add rounded to
 * bf16, from bf16 zero. v [T*k, N], scores [T*k], y [T, N]; bfloat16 only. */
int mi_moe_down_reduce(void* y, const void* v, const void* scores, int64_t T, int k, int64_t N,
                       int dtype, void* stream);

/* mi_take_rows(v, rows) followed by mi_moe_down_reduce in one pass: the un-sort of the
 * sorted dispatch (src/transformer.zig:15037) rides in the reduce (:15127-15140).
 * v [n_rows, N], rows [T*k] (uint32; an index >= n_rows reads as a zero row, as
 * mi_take_rows gives), scores [T*k], y [T, N]; bfloat16 only. Bit-equal to the two calls. */
int mi_moe_down_reduce_rows(void* y, const void* v, const void* scores, const uint32_t* rows,
                            int64_t n_rows, int64_t T, int k, int64_t N, int dtype,
                            void* stream);

/* Replaces gatherQmvGateUp (src/transformer.zig:20303-20396): for each token t and slot s,
 * g = x[t] @ dequant(w_gate[inds[t*k+s]])^T and u likewise, each rounded to bf16, then
 * y[t*k+s] = swiglu(g, u) exactly as mi_swiglu. x [T, K] bf16, y [T*k, N] bf16. Bit-equal
 * to two mi_gather_qmm calls followed by mi_swiglu. Formats: affine 4/8 bits, and the
 * bias-less modes nvfp4 / mxfp4 / mxfp8 (b_gate / b_up NULL, uint8 scales). */
int mi_gather_qmv_gate_up_swiglu(void* y, const void* x, const uint32_t* w_gate,
                                 const void* s_gate, const void* b_gate, const uint32_t* w_up,
                                 const void* s_up, const void* b_up, const uint32_t* inds,
                                 int64_t T, int k, int64_t N, int64_t K, int64_t n_experts,
                                 mi_optional_int group_size, mi_optional_int bits,
                                 const char* mode, void* stream);

/* Routing fused into the gate + up launch, as the reference's fused router feeds the
 * decode MoE (src/transformer.zig:17748; routing moeRoutingChain :17022-17072, then
 * gatherQmvGateUp :20303-20396): inds/scores [T, k] receive mi_moe_route_topk's result
 * for logits [T, E] fp32 (bit-equal), and y [T, k, N] the result of
 * mi_gather_qmv_gate_up_swiglu on those indices (bit-equal). One launch when the weights
 * are 4-bit gs 64 with K in one range, E <= 256 and scores_dtype bfloat16; otherwise the
 * two calls run in turn. */
int mi_moe_route_gate_up_swiglu(void* y, uint32_t* inds, void* scores, const float* logits,
                                const void* x, const uint32_t* w_gate, const void* s_gate,
                                const void* b_gate, const uint32_t* w_up, const void* s_up,
                                const void* b_up, int64_t T, int64_t E, int k, int64_t N,
                                int64_t K, mi_optional_int group_size, mi_optional_int bits,
                                const char* mode, int scores_dtype, void* stream);

/* Replaces gatherQmvDownReduce (src/transformer.zig:20675-20761): v[t*k+s] =
 * act[t*k+s] @ dequant(w_down[inds[t*k+s]])^T rounded to bf16, then y[t] as
 * mi_moe_down_reduce. act [T*k, K] bf16, scores [T*k] bf16, y [T, N] bf16. Bit-equal to
 * mi_gather_qmm followed by mi_moe_down_reduce. Formats as mi_gather_qmv_gate_up_swiglu. */
int mi_gather_qmv_down_reduce(void* y, const void* act, const uint32_t* w_down,
                              const void* s_down, const void* b_down, const uint32_t* inds,
                              const void* scores, int64_t T, int k, int64_t N, int64_t K,
                              int64_t n_experts, mi_optional_int group_size, mi_optional_int bits,
                              const char* mode, void* stream);

/* Grow the per-device workspace (sorted work lists, K-split partials) to at least
 * `bytes` ahead of HIP graph capture; calls that fit never allocate. No mlx-c
 * counterpart (MLX owns its allocator). An outgrown buffer that a call handed out during
 * a stream capture stays allocated (graphs captured then still use it) until
 * mi_workspace_release; one never used under capture is freed when it is outgrown. */
int mi_workspace_reserve(int64_t bytes, void* stream);

/* Free the workspace generations this device has outgrown. Growing never frees the
 * previous buffer, because a HIP graph captured while it was current keeps its address;
 * call this only when no such graph will be replayed again. Synchronizes the device when
 * there is something to free. No mlx-c counterpart (MLX owns its allocator). */
int mi_workspace_release(void* stream);

/* Thread-local text of the last non-zero return on this thread ("" if none). */
const char* mi_last_error(void);

/* Library version string. */
const char* mi_version(void);

/* Number of GEMMs this process has run through the vendor library (hipBLASLt). No
 * counterpart in the reference: a diagnostic for callers and tests that check no default
 * route reaches the library GEMM (only MI_QMM_DQGEMM=1 opts into it). */
int64_t mi_library_gemm_calls(void);

#ifdef __cplusplus
}
#endif
#endif
