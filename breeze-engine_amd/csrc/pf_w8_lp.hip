// Prefill GEMM kernels for INT8 weights, INT8 activations.
#include "prefill_kernel.h"

namespace bq {
template hipError_t launch_pf<8, false>(bool*, const PfArgs&, int, int, int, dim3, hipStream_t);
}  // namespace bq
