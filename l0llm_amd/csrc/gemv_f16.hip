// Instantiations of the weight-streaming GEMV for L0H_F16 weights (see gemv_kernel.h).
#include "gemv_kernel.h"

namespace l0h {
int gemv_dispatch_f16(hipStream_t s, const GemvParams& p, int mr) { return dispatch_wt<L0H_F16>(s, p, mr); }
}  // namespace l0h
