// Gather instances of the few-row decode kernel (qmvm_kernel.h) for the bias-less fp
// modes (nvfp4, mxfp4, mxfp8).
#include "qmvm_kernel.h"

namespace mi {
namespace qmvm_detail {
template void launch_family<4, 16, false, true, 0>(const QmvmParams&, const QmvParams&,
                                                    const QmvmPlan&, dim3, hipStream_t);
template void launch_family<4, 32, false, true, 0>(const QmvmParams&, const QmvParams&,
                                                    const QmvmPlan&, dim3, hipStream_t);
template void launch_family<4, 16, false, true, 1>(const QmvmParams&, const QmvParams&,
                                                    const QmvmPlan&, dim3, hipStream_t);
template void launch_family<4, 32, false, true, 1>(const QmvmParams&, const QmvParams&,
                                                    const QmvmPlan&, dim3, hipStream_t);
template void launch_family<8, 16, false, true, 2>(const QmvmParams&, const QmvParams&,
                                                    const QmvmPlan&, dim3, hipStream_t);
template void launch_family<8, 32, false, true, 2>(const QmvmParams&, const QmvParams&,
                                                    const QmvmPlan&, dim3, hipStream_t);
}  // namespace qmvm_detail
}  // namespace mi
