// Prefill (large-M) quantized GEMM. Placeholder until the MFMA GEMM lands: every
// shape is declined here and served by the small-M kernel in row chunks.
#include "mi_internal.h"

namespace mi {
bool qmm_supported(int, int, int, int, int) { return false; }
hipError_t launch_qmm(const QmmParams&, hipStream_t) { return hipErrorNotSupported; }
}  // namespace mi
