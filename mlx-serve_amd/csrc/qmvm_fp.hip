// Dense instances of the few-row decode kernel (qmvm_kernel.h) for the bias-less fp
// modes (nvfp4, mxfp4, mxfp8).
#include "qmvm_kernel.h"

namespace mi {
namespace qmvm_detail {
template void launch_family<4, 16, false, false, 0>(const QmvmParams&, const QmvParams&,
                                                    const QmvmPlan&, dim3, hipStream_t);
template void launch_family<4, 32, false, false, 0>(const QmvmParams&, const QmvParams&,
                                                    const QmvmPlan&, dim3, hipStream_t);
template void launch_family<4, 16, false, false, 1>(const QmvmParams&, const QmvParams&,
                                                    const QmvmPlan&, dim3, hipStream_t);
template void launch_family<4, 32, false, false, 1>(const QmvmParams&, const QmvParams&,
                                                    const QmvmPlan&, dim3, hipStream_t);
template void launch_family<8, 16, false, false, 2>(const QmvmParams&, const QmvParams&,
                                                    const QmvmPlan&, dim3, hipStream_t);
template void launch_family<8, 32, false, false, 2>(const QmvmParams&, const QmvParams&,
                                                    const QmvmPlan&, dim3, hipStream_t);
}  // namespace qmvm_detail
}  // namespace mi
