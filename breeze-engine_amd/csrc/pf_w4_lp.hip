// Prefill GEMM kernels for INT4 weights, INT8 activations.
#include "prefill_kernel.h"

namespace bq {
template hipError_t launch_pf<4, false>(bool*, const PfArgs&, int, int, int, dim3, hipStream_t);
}  // namespace bq
