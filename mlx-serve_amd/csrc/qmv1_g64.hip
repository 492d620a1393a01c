// Instances of the one-row decode kernel for group size 64 (the common MLX layout).
#include "qmv1_kernel.h"

namespace mi {
template hipError_t launch_qmv1_gs<64>(const QmvParams&, dim3, int, int, int, size_t, hipStream_t);
}  // namespace mi
