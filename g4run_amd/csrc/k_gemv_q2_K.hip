// k_gemv_q2_K.hip -- GEMV instantiations for q2_K weights (see gemv.h).
#include "gemv.h"

namespace g4 {
hipError_t launch_gemv_q2_K(const g4h_tensor &W, const uint8_t *act, size_t stride, const float *x, float *Y, int nb, hipStream_t s, int lpr,
                          int upl, const GemvOut &out) {
    return gemv_format<FQ2_K>(W, act, stride, x, Y, nb, s, lpr, upl, out);
}
}  // namespace g4
