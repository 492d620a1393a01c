// Internal (host + device) declarations shared by the kernels and the C ABI layer.
#pragma once
#include <atomic>
#include <hip/hip_runtime.h>

#include <algorithm>
#include <stdint.h>

namespace mi {

// Small-M / gather kernel parameters (qmv.hip).
struct QmvParams {
  const uint32_t* w;       // [E, N, K*bits/32]
  const uint16_t* scales;  // [E, N, K/gs] bf16 bits
  const uint16_t* biases;  // [E, N, K/gs] bf16 bits
  const void* x;           // [x_batch, M, K] bf16 or f32
  void* y;                 // [n_pairs, M, N] same dtype as x
  const uint32_t* lhs;     // nullable: lhs(i) = i / lhs_div
  const uint32_t* rhs;     // nullable: rhs(i) = i
  const uint32_t* items;   // nullable: sorted work list, 4 u32 per item (expert, pos0, cnt, 0)
  const uint32_t* item_count;  // device count for `items`
  float* part;             // ks > 1: fp32 partials [ks][n_pairs*M][N] (summed by a 2nd kernel)
  // nullable, bf16 outputs only: y = swiglu(swiglu_gate, result) (the fused up projection)
  const uint16_t* swiglu_gate;
  // dual (one-row kernel, gs 64, one K range): w/scales/biases is the gate bank, these the
  // up bank, and y = swiglu(gate, up) in one launch
  const uint32_t* w2;
  const uint16_t* scales2;
  const uint16_t* biases2;
  int dual;
  // dual only, nullable: route inside the launch. Pairs are (token, slot) with
  // lhs = pair / route_k; each block runs the softmax top-k of its token's route_E logits
  // (route_E <= 256) to find its expert, and the blocks of row tile 0 write route_inds /
  // route_scores (bf16) of their pair.
  const float* route_logits;
  uint32_t* route_inds;
  uint16_t* route_scores;
  int route_E, route_k;
  int64_t n_pairs, lhs_div, x_batch, n_experts;
  int M, N, K;
  int bits, group_size, x_f32;
  int rpi;             // rows per work item (32: qmv, 16: qmv16)
  int items_per_pair;  // unsorted: ceil(M / rpi)
  int n_items_fixed;   // unsorted: n_pairs * items_per_pair
  int ks;              // K splits (grid.y)
  int gps;             // quantization groups per K split
  int row_blocks;      // grid.x: ceil(N / 32)
};

struct QmvConfig {
  int grid_z;  // items in the grid (capped; the kernel strides over the rest)
  int waves;   // waves per block (split the block's K range)
  int rows;    // max activation rows per item (<= 32; selects the template)
};

constexpr int kQmvMaxWaves = 4;  // waves per qmv block (weight-slice LDS is static)
int qmv_mr_for_rows(int rows);
int qmv_groups_per_wave(int bits, int gs);
size_t qmv_lds_bytes(int groups, int gs, int mr, int x_f32, int waves);
hipError_t launch_qmv(const QmvParams& P, const QmvConfig& C, hipStream_t s);
hipError_t launch_reduce_splits(const QmvParams& P, hipStream_t s);

// One-row decode kernel (qmv1.hip): 4-bit, bf16 x, items of exactly one row.
struct Qmv1Plan {
  int ks, gps, waves, nc, depth, tiles;
  size_t lds;
};
bool qmv1_supported(int N, int K, int gs, int bits, int x_f32);
Qmv1Plan qmv1_plan(int N, int K, int gs, int64_t n_items);
hipError_t launch_qmv1(const QmvParams& P, const Qmv1Plan& plan, int grid_z, hipStream_t s);
// dense one-row nvfp4 (fpm 0) / mxfp4 (fpm 1): the one-row kernel's fp instances
hipError_t launch_qmv1_fp(const QmvParams& P, const Qmv1Plan& plan, int fpm, hipStream_t s);
template <int GS>
hipError_t launch_qmv1_gs(const QmvParams& P, dim3 grid, int waves, int nc, int depth, size_t lds,
                          hipStream_t s);

// Few-row decode kernel (qmvm*.hip): 2 <= M <= 32 rows, gs 64, bf16 x and y; dense 4-/8-bit,
// gathers 4-bit.
struct QmvmParams {
  const void* x;
  const uint32_t* w;
  const uint16_t* scales;
  const uint16_t* biases;
  uint16_t* y;
  float* part;  // ks > 1: fp32 partials [ks][M][N]
  int M, N, K, group_size, kr, wr;
  uint32_t upr_mr, spr_mr;  // set by launch_qmvm: ceil(2^32 / d) for the staging divisions
};
struct QmvmPlan {
  int wr, ks, kr, waves, nc, xu, depth, tiles, mt, lds, sbf32, rows, bits;
  int fpm;  // -1 affine 4/8 bits; 0 nvfp4, 1 mxfp4, 2 mxfp8 (uint8 scales); 100 + b: affine b bits
  size_t part_bytes;
};
// rows = activation rows per call (dense) or per work item (gathers, n_items items).
bool qmvm_plan(int rows, int N, int K, int gs, int bits, int64_t n_items, QmvmPlan* out);
// The fp modes (fpm 0 nvfp4, 1 mxfp4, 2 mxfp8) at 1..32 rows per call or item.
bool qmvm_plan_fp(int rows, int N, int K, int fpm, int64_t n_items, QmvmPlan* out);
// Affine 2/3/5/6 bits (gs 64) at 1..32 rows per call or item.
bool qmvm_plan_odd(int rows, int N, int K, int gs, int bits, int64_t n_items, QmvmPlan* out);
hipError_t launch_qmvm(const QmvmParams& P, const QmvmPlan& plan, hipStream_t s);
hipError_t launch_qmvm_gather(const QmvParams& G, const QmvmPlan& plan, int grid_z, hipStream_t s);

// Grouped GEMM over sorted work items (gmm.hip): 4-bit affine gs 64, bf16 x; items of up to
// 32 * mt rows (mt = 1, 2) built by launch_build_items; grid_items blocks stride them.
bool gmm_supported(int64_t N, int64_t K, int bits, int gs, int x_f32, int64_t x_bytes);
hipError_t launch_gmm(const QmvParams& P, int mt, int grid_items, hipStream_t s);
// x-stationary instance for short K (the item's 64 x rows, all of K, in LDS): 64-row items,
// ns passes of 256 weight rows a block, plain bf16 outputs only
bool gmm_xs_fits(int64_t K);
hipError_t launch_gmm_xs(const QmvParams& P, int ns, int grid_items, hipStream_t s);

// Decode-width kernel (qmv16.hip): M <= 16 rows per item, 16-row weight tiles.
int qmv16_mp_for_rows(int rows);
int qmv16_groups_per_chunk(int bits, int gs);
bool qmv16_supported(int K, int gs, int bits);
size_t qmv16_lds_bytes(int groups, int gs, int bits, int mp, int x_f32, int waves);
hipError_t launch_qmv16(const QmvParams& P, const QmvConfig& C, hipStream_t s);

// Sorted gather: runs of equal rhs -> work items (moe.hip / segments.hip).
hipError_t launch_build_items(const uint32_t* rhs, int64_t n_pairs, int M, int rows_per_item,
                              uint32_t* items, uint32_t* item_count, int64_t max_items,
                              hipStream_t s);

// MoE glue (moe.hip).
hipError_t launch_route_topk(const float* logits, int64_t T, int E, int k, uint32_t* inds,
                             void* scores, int scores_bf16, hipStream_t s);
size_t sort_dispatch_lds_bytes(int E);
hipError_t launch_route_grouped(const float* logits, const float* bias, int64_t T, int E, int k,
                                int n_group, int topk_group, int route_norm, float route_scale,
                                uint32_t* inds, float* scores, hipStream_t s);
hipError_t launch_sort_dispatch(const uint32_t* flat, int64_t n, int k, int E, uint32_t* order,
                                uint32_t* inv, uint32_t* sorted, uint32_t* lhs, uint32_t* seg,
                                hipStream_t s);
hipError_t launch_take_rows(void* out, const void* in, const uint32_t* idx, int64_t n,
                            int64_t n_src, int64_t row_bytes, hipStream_t s);
hipError_t launch_swiglu(uint16_t* y, const uint16_t* g, const uint16_t* u, int64_t n,
                         hipStream_t s);
hipError_t launch_down_reduce(uint16_t* y, const uint16_t* v, const uint16_t* scores, int64_t T,
                              int k, int64_t N, hipStream_t s, const uint32_t* rows = nullptr,
                              int64_t n_rows = 0);
// nvfp4 (mode 0) / mxfp4 (1) / mxfp8 (2) dequantize, uint8 scales, no biases (quant.hip).
hipError_t launch_dequantize_fp(void* out, const uint32_t* w, const uint8_t* s, int64_t rows,
                                int64_t K, int mode, int out_f32, const float* gscale, hipStream_t st);
// Decode GEMV for 2/3/5/6-bit affine weights (fp_mode -1, bf16 scales/biases) and the
// nvfp4 / mxfp4 / mxfp8 modes (fp_mode 0/1/2, uint8 scales), 1..8 bf16 activation rows
// (qmv_any.hip). hipErrorNotSupported when the shape is outside its scope.
hipError_t launch_qmv_any(const uint16_t* x, const uint32_t* w, const void* s,
                          const uint16_t* b, uint16_t* y, int64_t M, int64_t N, int64_t K,
                          int gs, int bits, int fp_mode, hipStream_t st);
// The same kernel over gather pairs: block column i computes x[lhs(i)] @ W[rhs(i)]^T into
// y[i] (lhs(i) = lhs ? lhs[i] : i / lhs_div, rhs(i) = rhs ? rhs[i] : i; out-of-range ids
// give NaN rows).
hipError_t launch_qmv_any_gather(const uint16_t* x, const uint32_t* w, const void* s,
                                 const uint16_t* b, uint16_t* y, int64_t M, int64_t N, int64_t K,
                                 int gs, int bits, int fp_mode, const uint32_t* lhs,
                                 const uint32_t* rhs, int64_t n_pairs, int64_t lhs_div,
                                 int64_t x_batch, int64_t n_experts, hipStream_t st);
// Decode MoE down projection + score-weighted slot sum in one launch (moe_down.hip).
bool moe_down_supported(int64_t T, int k, int64_t N, int64_t K, int gs, int bits, int ws, int nc);
hipError_t launch_moe_down(uint16_t* y, const uint16_t* act, const uint32_t* w,
                           const uint16_t* scales, const uint16_t* biases, const uint32_t* inds,
                           const uint16_t* scores, int64_t T, int k, int64_t N, int64_t K,
                           int64_t E, int ws, int nc, hipStream_t s);

// Prefill GEMM (qmm.hip). Returns hipErrorNotSupported if the shape is not handled.
struct QmmParams {
  const uint32_t* w;
  const uint16_t* scales;
  const uint16_t* biases;
  const uint16_t* x;  // bf16 [M, K]
  uint16_t* y;        // bf16 [M, N]
  int M, N, K;
  int bits, group_size;
  // K split: grid.y = ks ranges of sup_per_split super-steps; ks > 1 writes fp32
  // partials [ks][M][N] to `part` and a fixed-order reduce produces y.
  float* part;
  int ks, sup_per_split, bm;
};
// Fills bm / ks / sup_per_split; returns the workspace bytes the call needs.
size_t qmm_plan(QmmParams& P);
hipError_t launch_qmm(const QmmParams& P, hipStream_t s);
bool qmm_supported(int M, int N, int K, int bits, int gs);

// Prefill GEMM for 4- and 8-bit weights, and for weights already dequantized to bf16
// (bits = 16) (prefill.hip): 256x256 tiles, weights dequantized in registers, x through an
// LDS ring; ks > 1 splits K (fp32 partials [ks][M][N] in `part`,
// summed in split order by a second kernel).
struct PrefillParams {
  const uint32_t* w;
  const uint16_t* scales;
  const uint16_t* biases;
  const uint16_t* x;  // bf16 [M, K]
  uint16_t* y;        // bf16 [M, N]
  int M, N, K;
  int group_size;
  float* part;
  int ks, sps;  // K splits and 64-wide steps per split
  int bits;     // 4, 8, or 16 (w holds bf16 [N, K])
};
bool prefill_supported(int64_t M, int64_t N, int64_t K, int bits, int gs);
size_t prefill_plan(PrefillParams& P);  // fills ks / sps; returns workspace bytes
hipError_t launch_prefill(const PrefillParams& P, hipStream_t s);

extern std::atomic<int64_t> g_library_gemms;  // dq_gemm calls (blas.cpp)

// Dequantize + hipBLASLt bf16 GEMM for large M (blas.cpp): y = x @ wd^T with wd the
// dequantized bf16 [N, K] weight; blas_ws is the library's scratch. 0 or -1 (err set).
constexpr size_t kDqGemmBlasWs = (size_t)32 << 20;
// y^T is N x M with leading dimension ldy (N for a whole y, the full width for a slice).
int dq_gemm(const uint16_t* x, const uint16_t* wd, uint16_t* y, int M, int N, int K, int ldy,
            void* blas_ws, size_t blas_ws_bytes, hipStream_t s, const char** err);

// Quantize / dequantize / generator (quant.hip).
hipError_t launch_dequantize(void* out, const uint32_t* w, const uint16_t* s, const uint16_t* b,
                             int64_t rows, int64_t K, int gs, int bits, int out_f32, int rounding,
                             hipStream_t st);
hipError_t launch_quantize(uint32_t* wq, uint16_t* s, uint16_t* b, const void* w, int w_f32,
                           int64_t rows, int64_t K, int gs, int bits, hipStream_t st);
hipError_t launch_randn(void* out, int64_t n, uint64_t seed, float mean, float stddev,
                        int out_f32, hipStream_t st);

}  // namespace mi
