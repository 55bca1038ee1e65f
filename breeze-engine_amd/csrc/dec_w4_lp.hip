// Decode kernels for INT4 weights, INT8 activations.
#include "dec8_kernel.h"
#include "dec_kernel.h"

namespace bq {
template hipError_t launch_dec_bits<4, false>(bool*, const GemvArgs&, int, int, int, bool, bool, bool,
                                                    hipStream_t);
template hipError_t launch_dec8<4, false>(bool*, const GemvArgs&, const uint4*, int, int, int, bool, bool,
                                          hipStream_t);
}  // namespace bq
