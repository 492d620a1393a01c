// 8-bit dense instances of the few-row decode kernel (qmvm_kernel.h).
#include "qmvm_kernel.h"

namespace mi {
namespace qmvm_detail {
template void launch_family<8, 16, true, false>(const QmvmParams&, const QmvParams&,
                                                const QmvmPlan&, dim3, hipStream_t);
template void launch_family<8, 16, false, false>(const QmvmParams&, const QmvParams&,
                                                 const QmvmPlan&, dim3, hipStream_t);
template void launch_family<8, 32, false, false>(const QmvmParams&, const QmvParams&,
                                                 const QmvmPlan&, dim3, hipStream_t);
}  // namespace qmvm_detail
}  // namespace mi
