// Few-row decode GEMM instances for 33..64 activation rows (two 32-row passes), dense 4-
// and 8-bit (gather work items stay at <= 32 rows). Kernel in qmvm_kernel.h; plan and dispatch in qmvm.hip.
#include "qmvm_kernel.h"

namespace mi {
namespace qmvm_detail {
template void launch_family<4, 64, false, false>(const QmvmParams&, const QmvParams&,
                                              const QmvmPlan&, dim3, hipStream_t);
template void launch_family<8, 64, false, false>(const QmvmParams&, const QmvParams&,
                                              const QmvmPlan&, dim3, hipStream_t);
}  // namespace qmvm_detail
}  // namespace mi
