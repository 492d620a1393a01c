// Instances of the one-row decode kernel for affine 2/3/5/6/8-bit weights at group size 64:
// dense calls of one activation row, the same plan as the 4-bit instances.
#include "qmv1_kernel.h"

namespace mi {

hipError_t launch_qmv1_odd(const QmvParams& P, const Qmv1Plan& pl, int fpm, hipStream_t s) {
  switch (fpm) {
    case 102: qmv1_detail::launch_fmt<102>(P, pl, s); break;
    case 103: qmv1_detail::launch_fmt<103>(P, pl, s); break;
    case 105: qmv1_detail::launch_fmt<105>(P, pl, s); break;
    case 106: qmv1_detail::launch_fmt<106>(P, pl, s); break;
    case 108: qmv1_detail::launch_fmt<108>(P, pl, s); break;
    default: return hipErrorInvalidValue;
  }
  return hipSuccess;
}

}  // namespace mi
