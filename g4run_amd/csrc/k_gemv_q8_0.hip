// k_gemv_q8_0.hip -- GEMV instantiations for q8_0 weights (see gemv.h).
#include "gemv.h"

namespace g4 {
hipError_t launch_gemv_q8_0(const g4h_tensor &W, const uint8_t *act, size_t stride, float *Y, int nb, hipStream_t s, int lpr,
                          int upl) {
    return gemv_format<FQ8_0>(W, act, stride, Y, nb, s, lpr, upl);
}
}  // namespace g4
