// Instances of the one-row decode kernel for the bias-less modes (nvfp4, mxfp4, mxfp8):
// dense calls of one activation row, the same plan as the affine group-size-64 instances
// (the odd widths' instances are in qmv1_odd.hip).
#include "qmv1_kernel.h"

namespace mi {

hipError_t launch_qmv1_odd(const QmvParams& P, const Qmv1Plan& pl, int fpm, hipStream_t s);

// Dense one-row nvfp4 (fpm 0) / mxfp4 (fpm 1) / mxfp8 (fpm 2) and affine 2/3/5/6-bit (fpm 100 + bits, group
// size 64) decode; K-split plans finish with the shared fixed-order reduce.
hipError_t launch_qmv1_fp(const QmvParams& P, const Qmv1Plan& pl, int fpm, hipStream_t s) {
  if (P.M != 1 || P.n_pairs != 1 || P.items || P.lhs || P.rhs) return hipErrorInvalidValue;
  if (fpm == 0) qmv1_detail::launch_fmt<0>(P, pl, s);
  else if (fpm == 1) qmv1_detail::launch_fmt<1>(P, pl, s);
  else if (fpm == 2) qmv1_detail::launch_fmt<2>(P, pl, s);
  else if (hipError_t e = launch_qmv1_odd(P, pl, fpm, s); e != hipSuccess) return e;
  hipError_t e = hipGetLastError();
  if (e != hipSuccess || P.ks == 1) return e;
  return launch_reduce_splits(P, s);
}

}  // namespace mi
