// Decode kernels for INT8 weights, two-pass INT16 activations.
#include "dec8_kernel.h"
#include "dec_kernel.h"

namespace bq {
template hipError_t launch_dec_bits<8, true>(bool*, const GemvArgs&, int, int, int, bool, bool, bool,
                                                    hipStream_t);
template hipError_t launch_dec8<8, true>(bool*, const GemvArgs&, const uint4*, int, int, int, bool, bool,
                                          hipStream_t);
}  // namespace bq
