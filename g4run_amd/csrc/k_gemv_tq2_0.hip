// k_gemv_tq2_0.hip -- GEMV instantiations for tq2_0 weights (see gemv.h).
#include "gemv.h"

namespace g4 {
hipError_t launch_gemv_tq2_0(const g4h_tensor &W, const uint8_t *act, size_t stride, const float *x, float *Y, int nb, hipStream_t s,
                             int lpr, int upl, const GemvOut &out) {
    return gemv_format<FTQ2_0>(W, act, stride, x, Y, nb, s, lpr, upl, out);
}
}  // namespace g4
