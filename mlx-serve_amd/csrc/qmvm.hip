// Few-row decode GEMM on the 16x16x32 MFMA (qmvm_kernel.h): plan, launches, and the dense
// instances (the gather instances are in qmvm_gather.hip).
#include "qmvm_kernel.h"

#include <algorithm>
#include <cstdio>
#include <cstdlib>

namespace mi {

namespace qmvm_detail {
template void launch_family<4, 16, true, false>(const QmvmParams&, const QmvParams&, const QmvmPlan&,
                                             dim3, hipStream_t);
template void launch_family<4, 16, false, false>(const QmvmParams&, const QmvParams&,
                                              const QmvmPlan&, dim3, hipStream_t);
template void launch_family<4, 32, false, false>(const QmvmParams&, const QmvParams&,
                                              const QmvmPlan&, dim3, hipStream_t);
extern template void launch_family<4, 16, true, true>(const QmvmParams&, const QmvParams&,
                                                   const QmvmPlan&, dim3, hipStream_t);
extern template void launch_family<4, 16, false, true>(const QmvmParams&, const QmvParams&,
                                                    const QmvmPlan&, dim3, hipStream_t);
extern template void launch_family<4, 32, false, true>(const QmvmParams&, const QmvParams&,
                                                    const QmvmPlan&, dim3, hipStream_t);
extern template void launch_family<8, 16, true, false>(const QmvmParams&, const QmvParams&,
                                                    const QmvmPlan&, dim3, hipStream_t);
extern template void launch_family<8, 16, false, false>(const QmvmParams&, const QmvParams&,
                                                     const QmvmPlan&, dim3, hipStream_t);
extern template void launch_family<8, 32, false, false>(const QmvmParams&, const QmvParams&,
                                                     const QmvmPlan&, dim3, hipStream_t);
extern template void launch_family<4, 16, false, false, 0>(const QmvmParams&, const QmvParams&,
                                                        const QmvmPlan&, dim3, hipStream_t);
extern template void launch_family<4, 32, false, false, 0>(const QmvmParams&, const QmvParams&,
                                                        const QmvmPlan&, dim3, hipStream_t);
extern template void launch_family<4, 16, false, false, 1>(const QmvmParams&, const QmvParams&,
                                                        const QmvmPlan&, dim3, hipStream_t);
extern template void launch_family<4, 32, false, false, 1>(const QmvmParams&, const QmvParams&,
                                                        const QmvmPlan&, dim3, hipStream_t);
extern template void launch_family<4, 16, false, true, 0>(const QmvmParams&, const QmvParams&,
                                                       const QmvmPlan&, dim3, hipStream_t);
extern template void launch_family<4, 32, false, true, 0>(const QmvmParams&, const QmvParams&,
                                                       const QmvmPlan&, dim3, hipStream_t);
extern template void launch_family<4, 16, false, true, 1>(const QmvmParams&, const QmvParams&,
                                                       const QmvmPlan&, dim3, hipStream_t);
extern template void launch_family<4, 32, false, true, 1>(const QmvmParams&, const QmvParams&,
                                                       const QmvmPlan&, dim3, hipStream_t);
extern template void launch_family<8, 16, false, false, 2>(const QmvmParams&, const QmvParams&,
                                                        const QmvmPlan&, dim3, hipStream_t);
extern template void launch_family<8, 32, false, false, 2>(const QmvmParams&, const QmvParams&,
                                                        const QmvmPlan&, dim3, hipStream_t);
extern template void launch_family<8, 16, false, true, 2>(const QmvmParams&, const QmvParams&,
                                                        const QmvmPlan&, dim3, hipStream_t);
extern template void launch_family<8, 32, false, true, 2>(const QmvmParams&, const QmvParams&,
                                                        const QmvmPlan&, dim3, hipStream_t);
extern template void launch_family<4, 16, false, false, 102>(const QmvmParams&, const QmvParams&,
                                                           const QmvmPlan&, dim3, hipStream_t);
extern template void launch_family<4, 32, false, false, 102>(const QmvmParams&, const QmvParams&,
                                                           const QmvmPlan&, dim3, hipStream_t);
extern template void launch_family<4, 16, false, true, 102>(const QmvmParams&, const QmvParams&,
                                                           const QmvmPlan&, dim3, hipStream_t);
extern template void launch_family<4, 32, false, true, 102>(const QmvmParams&, const QmvParams&,
                                                           const QmvmPlan&, dim3, hipStream_t);
extern template void launch_family<4, 16, false, false, 103>(const QmvmParams&, const QmvParams&,
                                                           const QmvmPlan&, dim3, hipStream_t);
extern template void launch_family<4, 32, false, false, 103>(const QmvmParams&, const QmvParams&,
                                                           const QmvmPlan&, dim3, hipStream_t);
extern template void launch_family<4, 16, false, true, 103>(const QmvmParams&, const QmvParams&,
                                                           const QmvmPlan&, dim3, hipStream_t);
extern template void launch_family<4, 32, false, true, 103>(const QmvmParams&, const QmvParams&,
                                                           const QmvmPlan&, dim3, hipStream_t);
extern template void launch_family<4, 16, false, false, 105>(const QmvmParams&, const QmvParams&,
                                                           const QmvmPlan&, dim3, hipStream_t);
extern template void launch_family<4, 32, false, false, 105>(const QmvmParams&, const QmvParams&,
                                                           const QmvmPlan&, dim3, hipStream_t);
extern template void launch_family<4, 16, false, true, 105>(const QmvmParams&, const QmvParams&,
                                                           const QmvmPlan&, dim3, hipStream_t);
extern template void launch_family<4, 32, false, true, 105>(const QmvmParams&, const QmvParams&,
                                                           const QmvmPlan&, dim3, hipStream_t);
extern template void launch_family<4, 16, false, false, 106>(const QmvmParams&, const QmvParams&,
                                                           const QmvmPlan&, dim3, hipStream_t);
extern template void launch_family<4, 32, false, false, 106>(const QmvmParams&, const QmvParams&,
                                                           const QmvmPlan&, dim3, hipStream_t);
extern template void launch_family<4, 16, false, true, 106>(const QmvmParams&, const QmvParams&,
                                                           const QmvmPlan&, dim3, hipStream_t);
extern template void launch_family<4, 32, false, true, 106>(const QmvmParams&, const QmvParams&,
                                                           const QmvmPlan&, dim3, hipStream_t);
extern template void launch_family<4, 64, false, false>(const QmvmParams&, const QmvParams&,
                                                     const QmvmPlan&, dim3, hipStream_t);
extern template void launch_family<8, 64, false, false>(const QmvmParams&, const QmvParams&,
                                                     const QmvmPlan&, dim3, hipStream_t);
}  // namespace qmvm_detail

namespace {

// y[m, n] = sum over ranges r (in order) of part[r, m, n], rounded to bf16.
__global__ void qmvm_reduce_kernel(const float* __restrict__ part, uint16_t* __restrict__ y,
                                   int ks, int64_t mn) {
  const int64_t o = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (o >= mn) return;
  const float v = add_splits<8>(0.f, part + o, mn, 0, ks);
  y[o] = (uint16_t)f32_to_bf16_bits(v);
}

int env_or(const char* name, int dflt) {
  const char* v = std::getenv(name);
  return v ? std::atoi(v) : dflt;
}

// ceil(2^32 / d): umulhi(u, .) == u / d exactly for u < 2^19 and 2 <= d < 2^13 (the
// kernel does not use it for d == 1).
uint32_t div_magic(uint32_t d) {
  return d <= 1 ? 0xFFFFFFFFu : (uint32_t)((((uint64_t)1 << 32) + d - 1) / d);
}


template <bool GATHER>
void launch_any(QmvmParams P, const QmvParams& G, const QmvmPlan& pl, dim3 grid, hipStream_t s) {
  using namespace qmvm_detail;
  P.upr_mr = div_magic((uint32_t)(pl.kr / 8));
  P.spr_mr = div_magic((uint32_t)(pl.kr / P.group_size / 2));
  if (pl.fpm >= 100) {  // affine 2/3/5/6 bits
    const bool m16 = pl.mt == 16;
    switch (pl.fpm) {
      case 102: m16 ? launch_family<4, 16, false, GATHER, 102>(P, G, pl, grid, s)
                    : launch_family<4, 32, false, GATHER, 102>(P, G, pl, grid, s); break;
      case 103: m16 ? launch_family<4, 16, false, GATHER, 103>(P, G, pl, grid, s)
                    : launch_family<4, 32, false, GATHER, 103>(P, G, pl, grid, s); break;
      case 105: m16 ? launch_family<4, 16, false, GATHER, 105>(P, G, pl, grid, s)
                    : launch_family<4, 32, false, GATHER, 105>(P, G, pl, grid, s); break;
      default: m16 ? launch_family<4, 16, false, GATHER, 106>(P, G, pl, grid, s)
                   : launch_family<4, 32, false, GATHER, 106>(P, G, pl, grid, s); break;
    }
    return;
  }
  if (pl.fpm >= 0) {
    const bool m16 = pl.mt == 16;
    if (pl.fpm == 0)
      m16 ? launch_family<4, 16, false, GATHER, 0>(P, G, pl, grid, s)
          : launch_family<4, 32, false, GATHER, 0>(P, G, pl, grid, s);
    else if (pl.fpm == 2)
      m16 ? launch_family<8, 16, false, GATHER, 2>(P, G, pl, grid, s)
          : launch_family<8, 32, false, GATHER, 2>(P, G, pl, grid, s);
    else
      m16 ? launch_family<4, 16, false, GATHER, 1>(P, G, pl, grid, s)
          : launch_family<4, 32, false, GATHER, 1>(P, G, pl, grid, s);
    return;
  }
  if (pl.bits == 8) {
    if constexpr (!GATHER) {  // 8-bit instances are dense only
      if (pl.mt == 16 && pl.sbf32) launch_family<8, 16, true, false>(P, G, pl, grid, s);
      else if (pl.mt == 16) launch_family<8, 16, false, false>(P, G, pl, grid, s);
      else if (pl.mt == 32) launch_family<8, 32, false, false>(P, G, pl, grid, s);
      else launch_family<8, 64, false, false>(P, G, pl, grid, s);
    }
    return;
  }
  if (pl.mt == 16 && pl.sbf32) launch_family<4, 16, true, GATHER>(P, G, pl, grid, s);
  else if (pl.mt == 16) launch_family<4, 16, false, GATHER>(P, G, pl, grid, s);
  else if (pl.mt == 32) launch_family<4, 32, false, GATHER>(P, G, pl, grid, s);
  else if constexpr (!GATHER) launch_family<4, 64, false, false>(P, G, pl, grid, s);
}

}  // namespace

namespace {
// fpm -1: affine (gs 64, scale/bias pairs staged in LDS); 0 / 1 / 2: the fp modes (scales
// loaded with the weights: no staging, no even-group constraint); 100 + b: affine b = 2, 3,
// 5, 6 bits on the 4-bit layout (bits = 4 here), staged like the affine 4-bit plans.
bool plan_impl(int M, int N, int K, int gs, int bits, int64_t n_items, int fpm, QmvmPlan* out) {
  const bool fp = fpm >= 0 && fpm < 100, odd = fpm >= 100;
  if ((bits != 4 && bits != 8) || M < (fp || odd || bits == 8 ? 1 : 2) || M > (fp || odd ? 32 : 64))
    return false;
  if (odd && (int64_t)N * (K * (fpm - 100) / 8) >= ((int64_t)1 << 31)) return false;
  const int cv = 512 / bits;  // values per 64-byte chunk of a row
  if (K % cv != 0) return false;
  if (!fp && gs != 64) return false;  // the other group sizes take the general decode kernels
  if ((int64_t)N * (K * bits / 8) >= ((int64_t)1 << 31) || (int64_t)M * K * 2 >= ((int64_t)1 << 31))
    return false;
  static const int env_wr = env_or("MI_QMVM_WR", 0);
  static const int env_target = env_or("MI_QMVM_TARGET", 0);
  static const int env_depth = env_or("MI_QMVM_DEPTH", 0);
  static const int env_ks = env_or("MI_QMVM_KS", 0);  // K ranges (plan sweeps)
  const int mt = M <= 16 ? 16 : M <= 32 ? 32 : 64;
  const int mp = M < 32 ? M : 32;  // rows staged at once (64-row plans stage two passes)
  const size_t lds_max = 160 * 1024 - 512;  // the kernel's static row table
  const int nch = K / cv;
  const int target = env_target ? env_target : 8;
  // Weight tiles per block (WR): the staged activations are re-read from L2 once per
  // block, M / (4 WR) times the weight bytes, so take the most tiles that fit (measured:
  // 1 for M <= 2, 4 up to 16 rows, 8 above); then the
  // fewest K ranges (each range beyond one writes fp32 partials and needs the reduce
  // launch); then chunks per wave near `target` and more waves. Scale/bias pairs are
  // staged as fp32 (s, b - 128 s) when LDS allows, else as bf16 pairs.
  // 64-row plans: 4 tiles, so 8 waves still cover a K range of 2048 in one block
  // Gather items of 3..16 rows at K >= 4096: 16 tiles (one wave each, so K splits into
  // ranges of at most 8 chunks): configs[4] T=64 gate/up 1088 -> 1049 us per call (8 tiles:
  // 1077); at K = 2048 it is slower (436 -> 504 us).
  const bool long_gather = n_items > 1 && K >= 4096 && M > 2 && M <= 16 && !fp;
  // One byte a code (8-bit, mxfp8) doubles the weight bytes per staged activation, so fewer
  // tiles a block (more blocks) pay: 2 tiles for 8-bit up to 16 rows and mxfp8 up to 8
  // (Llama MLP 8-bit M=4 3526 -> 4032 GB/s, M=16 2981 -> 3072; mxfp8 M=8 2565 -> 2858; mxfp8
  // at 16 rows and both at 32 measured slower).
  const bool byte_few = bits == 8 && M > 2 && (M <= 8 || (fpm < 0 && M <= 16));
  const int wr0 = env_wr ? env_wr : long_gather ? 16 : byte_few ? 2
                  : M <= 2 ? 1 : M <= 16 ? 4 : M <= 32 ? 8 : 4;
  QmvmPlan best{};
  double best_cost = 1e30;
  // Up to 32 rows, a plan under 192 blocks (narrow shapes: N = 1536..7168 at K = 768..7168)
  // walks down the tile counts and takes the plan of the first that reaches 192 blocks
  // (else the last, one tile): more blocks outweigh the extra activation reads there, and
  // the cost model's K-split and chunk-count terms alone keep too many tiles a block.
  // Measured per launch, 8-bit: [2048,7168] 32 rows 14.5 -> 11.4 us (2 tiles), 16 rows
  // 10.6 -> 9.6 (1 tile); [1536,2048] 32 rows 12.0 -> 6.2, 16 rows 7.5 -> 4.8 (1 tile);
  // [7168,2048] 32 rows 13.0 -> 7.8 (2 tiles). Wide shapes such as [14336,4096] reach 192
  // blocks at the first tile count and keep their plan.
  static const int narrow = env_or("MI_QMVM_NARROW", 1);
  auto few_blocks = [&]() {
    return mt <= 32 && narrow && !env_wr &&
           (int64_t)best.tiles * best.ks * std::max<int64_t>(1, n_items) < 192;
  };
  for (int wr = wr0; wr >= 1 && (!best.nc || few_blocks()); wr >>= 1) {
    if (best.nc) best_cost = 1e30;  // a plan found at this tile count replaces it
    const int tiles = (N + 16 * wr - 1) / (16 * wr);
    for (int ks = 1; ks <= nch; ++ks) {
      if (nch % ks || (env_ks && ks != env_ks)) continue;
      const int chs = nch / ks;  // chunks per range
      const int nvals = chs * cv;
      if (!fp && (nvals / gs) % 2) continue;  // scale/bias pairs: an even group count
      const int max_waves = mt == 64 ? 8 : 16;  // the 64-row instances' launch bound
      for (int wk = 1; wk * wr <= max_waves; ++wk) {
        if (chs % wk) continue;
        const int nc = chs / wk;
        if (nc > 8) continue;
        const int waves = wk * wr;
        for (int f32 = mt == 16 && !fp && !odd ? 1 : 0; f32 >= 0; --f32) {
          qmvm_detail::QmvmLds L = qmvm_detail::qmvm_lds(mp, nvals, gs, 16 * wr, waves, mt, f32 != 0);
          if (fp) L.sbbytes = 0;
          if ((size_t)L.total() > lds_max) continue;
          const int units = mp * nvals / 8;
          const int xu = (units + 64 * waves - 1) / (64 * waves);
          if (xu > 8) continue;
          const int gr = nvals / gs;
          const int sload = 16 * wr * (gs <= 64 ? gr / 2 : gr);
          if (!fp && sload > 4 * 64 * waves) continue;
          const int64_t blocks = (int64_t)tiles * ks * std::max<int64_t>(1, n_items);
          const double cost = 3.0 * (ks - 1) + (blocks < 256 ? 4.0 * (256 - blocks) / 256 : 0) +
                              std::abs(nc - target) + 0.05 * (16 - waves) + (f32 ? 0 : 0.5);
          if (cost < best_cost) {
            best_cost = cost;
            best.wr = wr;
            best.ks = ks;
            best.kr = nvals;
            best.waves = waves;
            best.nc = nc;
            best.xu = xu <= 1 ? 1 : xu <= 2 ? 2 : xu <= 4 ? 4 : 8;
            best.lds = L.total();
            best.tiles = tiles;
            best.mt = mt;
            best.sbf32 = f32;
          }
          break;  // the fp32 layout fits: the bf16 one is not better
        }
      }
    }
  }
  if (!best.nc) return false;
  // two chunks in flight per wave, except where four measured faster on Llama MLP shapes:
  // 8-bit affine up to 16 rows (1-5%: M=8 18.99 -> 18.49 / 18.83 -> 17.83 us a gate / down
  // launch, M=4 3438 -> 3538 GB/s; at 32 rows four is 10% slower); mxfp4 at every row count
  // (5-7%: M=8 2402 -> 2583 GB/s) and mxfp8 (1-6%). nvfp4 is 5% slower with four.
  const bool deep = (bits == 8 && fpm < 0 && M <= 16) || fpm == 1 || fpm == 2;
  best.depth = env_depth ? env_depth : deep ? 4 : 2;
  best.rows = M;
  best.bits = bits;
  best.fpm = fpm;
  best.part_bytes = best.ks > 1 ? (size_t)best.ks * M * N * 4 : 0;
  static const int verbose = env_or("MI_QMVM_VERBOSE", 0);
  static int64_t last_key = -1;
  const int64_t key = ((int64_t)M << 40) ^ ((int64_t)N << 20) ^ K;
  if (verbose && key != last_key && (last_key = key, true))
    std::fprintf(stderr,
                 "qmvm M=%d N=%d K=%d: wr=%d ks=%d waves=%d nc=%d xu=%d depth=%d sbf32=%d lds=%d\n",
                 M, N, K, best.wr, best.ks, best.waves, best.nc, best.xu, best.depth, best.sbf32,
                 best.lds);
  *out = best;
  return true;
}
}  // namespace

bool qmvm_plan(int M, int N, int K, int gs, int bits, int64_t n_items, QmvmPlan* out) {
  return plan_impl(M, N, K, gs, bits, n_items, -1, out);
}

bool qmvm_plan_odd(int M, int N, int K, int gs, int bits, int64_t n_items, QmvmPlan* out) {
  if (bits != 2 && bits != 3 && bits != 5 && bits != 6) return false;
  return plan_impl(M, N, K, gs, 4, n_items, 100 + bits, out);
}

bool qmvm_plan_fp(int M, int N, int K, int fpm, int64_t n_items, QmvmPlan* out) {
  if (fpm < 0 || fpm > 2) return false;
  return plan_impl(M, N, K, fpm == 0 ? 16 : 32, fpm == 2 ? 8 : 4, n_items, fpm, out);
}

hipError_t launch_qmvm(const QmvmParams& P, const QmvmPlan& pl, hipStream_t s) {
  const QmvParams none{};
  launch_any<false>(P, none, pl, dim3((unsigned)pl.tiles, (unsigned)pl.ks), s);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess || pl.ks == 1) return e;
  const int64_t mn = (int64_t)P.M * P.N;
  hipLaunchKernelGGL(qmvm_reduce_kernel, dim3((unsigned)((mn + 255) / 256)), dim3(256), 0, s,
                     P.part, P.y, pl.ks, mn);
  return hipGetLastError();
}

hipError_t launch_qmvm_gather(const QmvParams& G, const QmvmPlan& pl, int grid_z, hipStream_t s) {
  if (pl.mt > 32) return hipErrorInvalidValue;  // gather items hold at most 32 rows
  QmvmParams P{G.x, G.w, G.scales, G.biases, (uint16_t*)G.y, G.part, pl.rows, G.N, G.K,
               G.group_size, pl.kr, pl.wr, 0, 0};
  launch_any<true>(P, G, pl, dim3((unsigned)pl.tiles, (unsigned)pl.ks, (unsigned)grid_z), s);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess || pl.ks == 1) return e;
  return launch_reduce_splits(G, s);
}

}  // namespace mi
