// Gather instances of the few-row decode kernel (qmvm_kernel.h): sorted expert runs and
// unsorted pairs of 2..32 rows.
#include "qmvm_kernel.h"

namespace mi {
namespace qmvm_detail {
template void launch_family<4, 16, true, true>(const QmvmParams&, const QmvParams&, const QmvmPlan&,
                                            dim3, hipStream_t);
template void launch_family<4, 16, false, true>(const QmvmParams&, const QmvParams&,
                                             const QmvmPlan&, dim3, hipStream_t);
template void launch_family<4, 32, false, true>(const QmvmParams&, const QmvParams&,
                                             const QmvmPlan&, dim3, hipStream_t);
}  // namespace qmvm_detail
}  // namespace mi
