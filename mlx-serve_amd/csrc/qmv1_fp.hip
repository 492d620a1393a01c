// Instances of the one-row decode kernel for the bias-less 4-bit modes (nvfp4, mxfp4):
// dense calls of one activation row, the same plan as the affine group-size-64 instances.
#include "qmv1_kernel.h"

namespace mi {
namespace {

using qmv1_detail::qmv1_kernel;

template <int NC, int DEPTH, int FPM>
void launch_xu_fp(const QmvParams& P, dim3 grid, dim3 block, int xu, size_t lds, hipStream_t s) {
  switch (xu) {
    case 1: hipLaunchKernelGGL((qmv1_kernel<64, NC, 1, DEPTH, true, false, FPM>), grid, block, lds, s, P); break;
    case 2: hipLaunchKernelGGL((qmv1_kernel<64, NC, 2, DEPTH, true, false, FPM>), grid, block, lds, s, P); break;
    case 4: hipLaunchKernelGGL((qmv1_kernel<64, NC, 4, DEPTH, true, false, FPM>), grid, block, lds, s, P); break;
    default: hipLaunchKernelGGL((qmv1_kernel<64, NC, 8, DEPTH, true, false, FPM>), grid, block, lds, s, P); break;
  }
}

template <int NC, int FPM>
void launch_nc_fp(const QmvParams& P, dim3 grid, dim3 block, int xu, int depth, size_t lds,
                  hipStream_t s) {
  if (NC > 2 && depth == 2) launch_xu_fp<NC, 2, FPM>(P, grid, block, xu, lds, s);
  else launch_xu_fp<NC, 4, FPM>(P, grid, block, xu, lds, s);
}

template <int FPM>
void launch_fp(const QmvParams& P, const Qmv1Plan& pl, hipStream_t s) {
  const dim3 grid((unsigned)pl.tiles, (unsigned)P.ks, 1), block(64 * pl.waves);
  switch (pl.nc) {
    case 1: launch_nc_fp<1, FPM>(P, grid, block, pl.xu, pl.depth, pl.lds, s); break;
    case 2: launch_nc_fp<2, FPM>(P, grid, block, pl.xu, pl.depth, pl.lds, s); break;
    case 3: launch_nc_fp<3, FPM>(P, grid, block, pl.xu, pl.depth, pl.lds, s); break;
    case 4: launch_nc_fp<4, FPM>(P, grid, block, pl.xu, pl.depth, pl.lds, s); break;
    case 5: launch_nc_fp<5, FPM>(P, grid, block, pl.xu, pl.depth, pl.lds, s); break;
    case 6: launch_nc_fp<6, FPM>(P, grid, block, pl.xu, pl.depth, pl.lds, s); break;
    case 7: launch_nc_fp<7, FPM>(P, grid, block, pl.xu, pl.depth, pl.lds, s); break;
    case 8: launch_nc_fp<8, FPM>(P, grid, block, pl.xu, pl.depth, pl.lds, s); break;
    case 10: launch_nc_fp<10, FPM>(P, grid, block, pl.xu, pl.depth, pl.lds, s); break;
    case 12: launch_nc_fp<12, FPM>(P, grid, block, pl.xu, pl.depth, pl.lds, s); break;
    case 14: launch_nc_fp<14, FPM>(P, grid, block, pl.xu, pl.depth, pl.lds, s); break;
    default: launch_nc_fp<16, FPM>(P, grid, block, pl.xu, pl.depth, pl.lds, s); break;
  }
}

}  // namespace

// Dense one-row nvfp4 (fpm 0) / mxfp4 (fpm 1) decode; K-split plans finish with the shared
// fixed-order reduce.
hipError_t launch_qmv1_fp(const QmvParams& P, const Qmv1Plan& pl, int fpm, hipStream_t s) {
  if (P.M != 1 || P.n_pairs != 1 || P.items || P.lhs || P.rhs || (fpm != 0 && fpm != 1))
    return hipErrorInvalidValue;
  if (fpm == 0) launch_fp<0>(P, pl, s);
  else launch_fp<1>(P, pl, s);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess || P.ks == 1) return e;
  return launch_reduce_splits(P, s);
}

}  // namespace mi
