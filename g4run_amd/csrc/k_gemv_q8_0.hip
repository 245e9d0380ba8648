// k_gemv_q8_0.hip -- GEMV instantiations for q8_0 weights (see gemv.h).
#include "gemv.h"
#include "gemv_p.h"

namespace g4 {
hipError_t launch_gemv_q8_0(const g4h_tensor &W, const uint8_t *act, size_t stride, const float *x, float *Y, int nb, hipStream_t s, int lpr,
                          int upl, const GemvOut &out) {
    return gemv_format<FQ8_0>(W, act, stride, x, Y, nb, s, lpr, upl, out);
}
hipError_t launch_gemv_p_q8_0(const g4h_tensor &W, const uint8_t *act, float *Y, const GemvPro &pro, const GemvEpi &epi,
                             hipStream_t s, int lpr, int upl, int grid) {
    return gemv_p_format<FQ8_0>(W, act, Y, pro, epi, s, lpr, upl, grid);
}
}  // namespace g4
