// k_gemv_f16.hip -- GEMV over f16 / bf16 weight rows (matmul_b's G4_F16 and
// G4_BF16 cases, model.c:238-239, over g4_dot_f16 / g4_dot_bf16,
// quants.c:1319-1347) and the activation conversions of prep_act's AC_F16 /
// AC_BF16 classes (model.c:163-180).
//
// Floating-point weights carry no block scales and no integer sums: each lane
// widens 8 weights (one 16-byte load) and 8 activations to fp32 and fma's them
// into one accumulator per token, lanes stride the row, and the wave sums its
// lanes.  The fp32 order differs from the CPU's 8-lane AVX2 order (within the
// path's fp32 tolerance) but does not depend on the token count, so a batch
// gives every token the single-token bits.
#include "common.h"
#include "kernels.h"

namespace g4 {

// g4_fp32_to_bf16 (g4run.h:64-68): a NaN keeps its high half with the quiet
// bit set; everything else rounds to nearest even by the header's add-and-shift.
__device__ __forceinline__ uint16_t f2bf(float f) {
    const uint32_t x = __float_as_uint(f);
    if ((x & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((x >> 16) | 64u);
    return (uint16_t)((x + (0x7fffu + ((x >> 16) & 1u))) >> 16);
}

// x fp32 [nb][ncols] (row stride xs floats) -> f16 rows (AC_F16) or bf16-rounded
// fp32 rows (AC_BF16) at `os` bytes per token
__global__ __launch_bounds__(256) void k_act_float(int wtype, const float *__restrict__ x, size_t xs, int64_t ncols,
                                                   uint8_t *__restrict__ out, size_t os) {
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    const int b = blockIdx.y;
    if (i >= ncols) return;
    const float v = x[(size_t)b * xs + i];
    if (wtype == F16) ((uint16_t *)(out + (size_t)b * os))[i] = f2h(v);
    else ((float *)(out + (size_t)b * os))[i] = __uint_as_float((uint32_t)f2bf(v) << 16);
}

template <int WT>
__device__ __forceinline__ void widen8(const uint4 w, float (&f)[8]) {
    const uint32_t u[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
    for (int k = 0; k < 4; k++) {
        if constexpr (WT == F16) {
            f[2 * k] = h2f((uint16_t)(u[k] & 0xffff));
            f[2 * k + 1] = h2f((uint16_t)(u[k] >> 16));
        } else {                                            // bf16 -> fp32: the high half of a word
            f[2 * k] = __uint_as_float(u[k] << 16);
            f[2 * k + 1] = __uint_as_float(u[k] & 0xffff0000u);
        }
    }
}

// One wave per row.  W rows at `ws` bytes, activations of NB tokens at `as`
// bytes (f16 for F16 weights, fp32 for BF16), 16-byte aligned, ncols % 8 == 0.
// XF: `act` holds the tokens as fp32 rows instead, converted on load with
// k_act_float's arithmetic (f16 round-to-nearest-even, or bf16 rounding), so
// the sums are those of converting first -- one launch instead of two.
template <int WT, int NB, bool XF, bool OUT>
__global__ __launch_bounds__(256) void k_gemv_float(const uint8_t *__restrict__ W, size_t ws, int64_t nrows, int64_t ncols,
                                                    const uint8_t *__restrict__ act, size_t as, float *__restrict__ Y,
                                                    size_t ys, GemvOut out) {
    const int lane = threadIdx.x & 63;
    const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    if (row >= nrows) return;                                       // wave-uniform
    const uint8_t *wr = W + (size_t)row * ws;
    const int64_t ng = ncols / 8;
    float acc[NB];
#pragma unroll
    for (int t = 0; t < NB; t++) acc[t] = 0.0f;
#pragma unroll 4
    for (int64_t g = lane; g < ng; g += 64) {
        float wf[8];
        widen8<WT>(*(const uint4 *)(wr + 16 * g), wf);
#pragma unroll
        for (int t = 0; t < NB; t++) {
            float af[8];
            if constexpr (XF) {
                const float4 a0 = *(const float4 *)(act + (size_t)t * as + 32 * g);
                const float4 a1 = *(const float4 *)(act + (size_t)t * as + 32 * g + 16);
                const float xr[8] = {a0.x, a0.y, a0.z, a0.w, a1.x, a1.y, a1.z, a1.w};
#pragma unroll
                for (int e = 0; e < 8; e++)
                    af[e] = WT == F16 ? h2f(f2h(xr[e])) : __uint_as_float((uint32_t)f2bf(xr[e]) << 16);
            } else if constexpr (WT == F16) {
                widen8<F16>(*(const uint4 *)(act + (size_t)t * as + 16 * g), af);
            } else {
                const float4 a0 = *(const float4 *)(act + (size_t)t * as + 32 * g);
                const float4 a1 = *(const float4 *)(act + (size_t)t * as + 32 * g + 16);
                af[0] = a0.x; af[1] = a0.y; af[2] = a0.z; af[3] = a0.w;
                af[4] = a1.x; af[5] = a1.y; af[6] = a1.z; af[7] = a1.w;
            }
#pragma unroll
            for (int e = 0; e < 8; e++) acc[t] = __builtin_fmaf(wf[e], af[e], acc[t]);
        }
    }
#pragma unroll
    for (int t = 0; t < NB; t++) {
        const float s = group_sum<64>(acc[t]);
        if (lane == 0) Y[(size_t)t * ys + row] = OUT ? gemv_out_value(out, row, s) : s;
    }
}

template <int WT, bool XF>
static hipError_t gf_go(const uint8_t *W, size_t ws, int64_t nrows, int64_t ncols, const uint8_t *act, size_t as, float *Y,
                        size_t ys, int nb, hipStream_t s, const GemvOut &out) {
    if (out.mode != OUT_STORE && nb != 1) return hipErrorInvalidValue;
    const dim3 grid((unsigned)((nrows + 3) / 4));
    if (out.mode != OUT_STORE) {
        hipLaunchKernelGGL((k_gemv_float<WT, 1, XF, true>), grid, dim3(256), 0, s, W, ws, nrows, ncols, act, as, Y, ys, out);
        return hipGetLastError();
    }
    switch (nb) {
    case 1: hipLaunchKernelGGL((k_gemv_float<WT, 1, XF, false>), grid, dim3(256), 0, s, W, ws, nrows, ncols, act, as, Y, ys, out); break;
    case 2: hipLaunchKernelGGL((k_gemv_float<WT, 2, XF, false>), grid, dim3(256), 0, s, W, ws, nrows, ncols, act, as, Y, ys, out); break;
    case 4: hipLaunchKernelGGL((k_gemv_float<WT, 4, XF, false>), grid, dim3(256), 0, s, W, ws, nrows, ncols, act, as, Y, ys, out); break;
    case 8: hipLaunchKernelGGL((k_gemv_float<WT, 8, XF, false>), grid, dim3(256), 0, s, W, ws, nrows, ncols, act, as, Y, ys, out); break;
    default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

hipError_t launch_gemv_float(int wtype, const uint8_t *W, size_t ws, int64_t nrows, int64_t ncols, const uint8_t *act, size_t as,
                             float *Y, size_t ys, int nb, hipStream_t s, const GemvOut &out) {
    if (ncols % 8 || ws % 16 || as % 16 || (uintptr_t)W % 16 || (uintptr_t)act % 16) return hipErrorInvalidValue;
    return wtype == F16 ? gf_go<F16, false>(W, ws, nrows, ncols, act, as, Y, ys, nb, s, out)
         : wtype == BF16 ? gf_go<BF16, false>(W, ws, nrows, ncols, act, as, Y, ys, nb, s, out)
                         : hipErrorInvalidValue;
}

// the same from fp32 tokens x (row stride xs floats), converted on load
hipError_t launch_gemv_float_x(int wtype, const uint8_t *W, size_t ws, int64_t nrows, int64_t ncols, const float *x, size_t xs,
                               float *Y, size_t ys, int nb, hipStream_t s, const GemvOut &out) {
    if (ncols % 8 || ws % 16 || xs % 4 || (uintptr_t)W % 16 || (uintptr_t)x % 16) return hipErrorInvalidValue;
    const uint8_t *a = (const uint8_t *)x;
    return wtype == F16 ? gf_go<F16, true>(W, ws, nrows, ncols, a, xs * 4, Y, ys, nb, s, out)
         : wtype == BF16 ? gf_go<BF16, true>(W, ws, nrows, ncols, a, xs * 4, Y, ys, nb, s, out)
                         : hipErrorInvalidValue;
}

hipError_t launch_act_float(int wtype, const float *x, size_t xs, int64_t ncols, int nb, uint8_t *out, size_t os, hipStream_t s) {
    hipLaunchKernelGGL(k_act_float, dim3((unsigned)((ncols + 255) / 256), (unsigned)nb), dim3(256), 0, s, wtype, x, xs, ncols, out, os);
    return hipGetLastError();
}

}  // namespace g4
