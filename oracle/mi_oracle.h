/*
 * mi_oracle.h -- CPU restatement of MLX's affine quantized-matmul semantics.
 *
 * TEST INFRASTRUCTURE ONLY. This library is the checker for the HIP library
 * (libmi_qmm.so); only tests/, __graft_entry__.smoke() and bench.py's
 * cpu_baseline leg may load it. Nothing in the product path links it.
 *
 * Each function cites the reference call site whose semantics it restates
 * (paths relative to the ddalcu/mlx-serve tree). MLX itself (lib/mlx-src,
 * ml-explore/mlx v0.32.0) is an un-vendored submodule, so MLX's own algorithm
 * is restated from its published semantics; see the per-function notes for
 * which parts are pinned by what.
 */
#ifndef MI_ORACLE_H
#define MI_ORACLE_H
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- scalar helpers ---------------------------------------------------- */
float mo_bf16_to_f32(uint16_t h);
uint16_t mo_f32_to_bf16(float f); /* round-to-nearest-even, NaN kept quiet */
void mo_f32_to_bf16_array(const float* in, uint16_t* out, int64_t n);
void mo_bf16_to_f32_array(const uint16_t* in, float* out, int64_t n);

/* ---- deterministic input generator ------------------------------------ */
/* Counter-based SplitMix64 -> two uniforms -> Box-Muller in fp64 -> fp32.
 * Element 2j / 2j+1 take the cos / sin branch of pair j. */
uint64_t mo_splitmix64(uint64_t seed, uint64_t counter);
void mo_randn_f32(float* out, int64_t n, uint64_t seed, double mean, double stddev);
void mo_uniform_f64(double* out, int64_t n, uint64_t seed);

/* ---- affine packing (a1) ---------------------------------------------- */
/* value j of a word = (word >> (j*bits)) & (2^bits-1), LSB first. */
int mo_pack(const uint8_t* q, int64_t rows, int64_t K, int bits, uint32_t* wq);
int mo_unpack(const uint32_t* wq, int64_t rows, int64_t K, int bits, uint8_t* q);

/* ---- mx.quantize restatement (affine) ----------------------------------- */
/* w bf16 [rows,K] -> wq u32 [rows, K*bits/32], scales/biases bf16 [rows, K/gs]. */
int mo_quantize_bf16(const uint16_t* w, int64_t rows, int64_t K, int gs, int bits,
                     uint32_t* wq, uint16_t* scales, uint16_t* biases);

/* ---- mx.dequantize restatement (a2) ----------------------------------- */
enum { MO_DQ_F32 = 0, MO_DQ_BF16_FUSED = 1, MO_DQ_BF16_OPWISE = 2 };
int mo_dequantize(const uint32_t* wq, const uint16_t* scales, const uint16_t* biases,
                  int64_t rows, int64_t K, int gs, int bits, int kind, void* out);

/* ---- quantized_matmul truth (a3) -------------------------------------- */
/* y[M,N] = x[M,K] . dequant(W)[N,K]^T in fp64 over exactly dequantized weights.
 * x_f32 != 0: x is float32, else bf16. */
int mo_qmm_f64(const void* x, int x_f32, const uint32_t* wq, const uint16_t* scales,
               const uint16_t* biases, int64_t M, int64_t N, int64_t K, int gs, int bits,
               double* y);

/* fp32-accumulating multithreaded qmm (the timed CPU baseline). y is float32. */
int mo_qmm_f32(const uint16_t* x_bf16, const uint32_t* wq, const uint16_t* scales,
               const uint16_t* biases, int64_t M, int64_t N, int64_t K, int gs, int bits,
               float* y, int threads);

/* ---- gather_qmm truth (a5) -------------------------------------------- */
/* out[i] = x[lhs(i)] (M x K) . dequant(W[rhs(i)])^T, i in [0,n_idx).
 * lhs == NULL -> lhs(i) = i / lhs_div. Index out of range -> returns -2. */
int mo_gather_qmm_f64(const void* x, int x_f32, const uint32_t* wq, const uint16_t* scales,
                      const uint16_t* biases, const uint32_t* lhs, const uint32_t* rhs,
                      int64_t n_idx, int64_t lhs_div, int64_t M, int64_t N, int64_t K,
                      int64_t x_batch, int64_t n_experts, int gs, int bits, double* out);

/* ---- MoE routing (a8) -------------------------------------------------- */
/* softmax(logits) (fp32, max-subtracted) -> top-k by descending logit
 * (ties: lower index first) -> renormalised weights. */
int mo_route_softmax_topk(const float* logits, int64_t T, int64_t E, int k,
                          uint32_t* inds, float* scores);

/* ---- sorted dispatch glue (a6) ----------------------------------------- */
/* flat inds [n] -> order = stable argsort, inv = argsort(order),
 * sorted = flat[order], lhs = order / k. */
int mo_sort_dispatch(const uint32_t* flat, int64_t n, int k, uint32_t* order,
                     uint32_t* inv, uint32_t* sorted, uint32_t* lhs);

/* ---- fused decode contracts (a7) -------------------------------------- */
/* sigmoid over every bf16 pattern, rounded to bf16 (table SwiGLU). */
void mo_sigmoid_table_bf16(uint16_t* table /* 65536 */);
/* y = bf16(bf16(g * sig(g)) * u), elementwise over bf16 arrays. */
void mo_swiglu_bf16(const uint16_t* g, const uint16_t* u, int64_t n, uint16_t* y);
/* y[n] = ascending bf16 sum over slots of bf16(v[slot,n] * score[slot]). */
void mo_down_reduce_bf16(const uint16_t* v, const uint16_t* scores, int64_t topk,
                         int64_t N, uint16_t* y);

/* ---- geometry solve (a9) ---------------------------------------------- */
/* bits = w_cols*32/in_dim, gs = in_dim/s_cols; returns 0 or -1 when invalid. */
int mo_affine_params_from_geometry(int64_t w_cols, int64_t s_cols, int64_t in_dim,
                                   int* bits, int* gs);

/* ---- microscaling fp modes (f4) ------------------------------------------ */
/* mode 0 nvfp4, 1 mxfp4, 2 mxfp8; out fp32 (out_bf16 0) or bf16 bits. */
int mo_dequantize_fp(const uint32_t* wq, const uint8_t* scales, int64_t rows, int64_t K,
                     int mode, int out_bf16, void* out);
/* nvfp4 with the optional fp32 global scale (has_gscale 1; other modes: -1). */
int mo_dequantize_fp_gs(const uint32_t* wq, const uint8_t* scales, int64_t rows, int64_t K,
                        int mode, int out_bf16, int has_gscale, float gscale, void* out);

/* ---- group-limited routing (a8) ----------------------------------------- */
int mo_route_grouped_f64(const float* logits, const float* bias, int64_t T, int64_t E, int k,
                         int n_group, int topk_group, int route_norm, double route_scale,
                         uint32_t* inds, double* w);

#ifdef __cplusplus
}
#endif
#endif
