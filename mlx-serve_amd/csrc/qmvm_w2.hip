// 2-bit affine instances (dense and gathers) of the few-row decode kernel (qmvm_kernel.h).
#include "qmvm_kernel.h"

namespace mi {
namespace qmvm_detail {
template void launch_family<4, 16, false, false, 102>(const QmvmParams&, const QmvParams&,
                                                     const QmvmPlan&, dim3, hipStream_t);
template void launch_family<4, 32, false, false, 102>(const QmvmParams&, const QmvParams&,
                                                     const QmvmPlan&, dim3, hipStream_t);
template void launch_family<4, 16, false, true, 102>(const QmvmParams&, const QmvParams&,
                                                    const QmvmPlan&, dim3, hipStream_t);
template void launch_family<4, 32, false, true, 102>(const QmvmParams&, const QmvParams&,
                                                    const QmvmPlan&, dim3, hipStream_t);
}  // namespace qmvm_detail
}  // namespace mi
