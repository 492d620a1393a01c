// Instances of the one-row decode kernel for group size 128.
#include "qmv1_kernel.h"

namespace mi {
template hipError_t launch_qmv1_gs<128>(const QmvParams&, dim3, int, int, int, size_t, hipStream_t);
}  // namespace mi
