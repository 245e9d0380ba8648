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
#include <type_traits>

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

// Prompt batches on the matrix cores (g4h_matmul path 2): Y[t][r] = sum_k
// W[r][k] a[t][k] for 32-token x 32-row tiles, one v_mfma_f32_32x32x16_f16 /
// _bf16 per 16 columns.  The operands are the GEMV family's: f16 weights
// against f16-rounded activations, bf16 weights against bf16-rounded ones
// (prep_act's AC_F16 / AC_BF16, model.c:163-180), so every product is exact
// in fp32 (11 x 11 or 8 x 8 significant bits) and only the fp32 order of the
// sums differs from the CPU's and from the GEMV family's (within the path's
// tolerance).  The MMF_W waves of a workgroup split the 16-column steps (wave
// w takes steps w, w + MMF_W, ..., each chained into its accumulator in
// increasing order) and the waves' tiles are added in wave order through
// LDS: a token's result does not depend on the batch size.  Operand layout:
// lane l holds A[l % 32][8 (l / 32) .. + 7] and B[l % 32][8 (l / 32) .. + 7];
// C[i][j] with j = l % 32 (weight row), i = 8 (r / 4) + 4 (l / 32) + r % 4.
typedef _Float16 mf_v8h __attribute__((ext_vector_type(8)));
typedef __bf16 mf_v8bf __attribute__((ext_vector_type(8)));
typedef float mf_v16f __attribute__((ext_vector_type(16)));

constexpr int MMF_W = 8;              // waves per workgroup

// XF: fp32 token rows (row stride `as` bytes) rounded on load with
// k_act_float's arithmetic; else prepared rows (f16 for F16, bf16-rounded
// fp32 for BF16)
template <int WT, bool XF>
__global__ __launch_bounds__(64 * MMF_W) void k_mm_float(const uint8_t *__restrict__ W, size_t ws, int64_t nrows, int64_t ncols,
                                                         const uint8_t *__restrict__ act, size_t as, int M, float *__restrict__ Y) {
    __shared__ float part[MMF_W - 1][16][64];
    constexpr bool A32 = XF || WT == BF16;                          // activation rows of fp32
    const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x) >> 6;
    const int li = lane & 31, kh = lane >> 5;
    const int64_t n0 = (int64_t)blockIdx.x * 32;
    const int m0 = (int)blockIdx.y * 32;
    const int64_t row = min(n0 + li, nrows - 1);
    const int tok = min(m0 + li, M - 1);
    const uint8_t *wr = W + (size_t)row * ws + 16 * kh;
    const uint8_t *ar = act + (size_t)tok * as + (A32 ? 32 : 16) * kh;
    const int nk = (int)(ncols >> 4);
    const int nj = (nk - wave + MMF_W - 1) / MMF_W;                 // this wave's steps (uniform)
    struct Op {
        uint4 w, a0, a1;
    };
    auto load = [&](int j) __attribute__((always_inline)) -> Op {
        const size_t sk = (size_t)(wave + MMF_W * j);
        Op o;
        o.w = *(const uint4 *)(wr + 32 * sk);
        o.a0 = *(const uint4 *)(ar + (A32 ? 64 : 32) * sk);
        if constexpr (A32) o.a1 = *(const uint4 *)(ar + 64 * sk + 16);
        return o;
    };
    mf_v16f acc = {};
    auto mac = [&](const Op &o) __attribute__((always_inline)) {
        uint32_t ab[4];
        if constexpr (A32) {
            const float v[8] = {__uint_as_float(o.a0.x), __uint_as_float(o.a0.y), __uint_as_float(o.a0.z), __uint_as_float(o.a0.w),
                                __uint_as_float(o.a1.x), __uint_as_float(o.a1.y), __uint_as_float(o.a1.z), __uint_as_float(o.a1.w)};
#pragma unroll
            for (int k = 0; k < 4; k++) {
                uint32_t lo, hi;
                if constexpr (WT == F16) {
                    lo = f2h(v[2 * k]), hi = f2h(v[2 * k + 1]);
                } else if constexpr (XF) {
                    lo = f2bf(v[2 * k]), hi = f2bf(v[2 * k + 1]);
                } else {                                            // already bf16-rounded: the high halves
                    lo = __float_as_uint(v[2 * k]) >> 16, hi = __float_as_uint(v[2 * k + 1]) >> 16;
                }
                ab[k] = lo | (hi << 16);
            }
        } else {
            ab[0] = o.a0.x, ab[1] = o.a0.y, ab[2] = o.a0.z, ab[3] = o.a0.w;
        }
        const uint4 av = make_uint4(ab[0], ab[1], ab[2], ab[3]);
        if constexpr (WT == F16)
            acc = __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(mf_v8h, av), __builtin_bit_cast(mf_v8h, o.w), acc, 0, 0, 0);
        else
            acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(mf_v8bf, av), __builtin_bit_cast(mf_v8bf, o.w), acc, 0, 0,
                                                          0);
    };
    // straight-line chunks of steps whose loads all go out first
    auto chunk = [&](auto Cc, int j0) __attribute__((always_inline)) {
        constexpr int C = decltype(Cc)::value;
        Op ops[C];
#pragma unroll
        for (int k = 0; k < C; k++) ops[k] = load(j0 + k);
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int k = 0; k < C; k++) mac(ops[k]);
    };
    int j0 = 0;
    for (; j0 + 4 <= nj; j0 += 4) chunk(std::integral_constant<int, 4>{}, j0);
    if (nj - j0 >= 2) chunk(std::integral_constant<int, 2>{}, j0), j0 += 2;
    if (nj - j0 >= 1) chunk(std::integral_constant<int, 1>{}, j0);

    if (wave > 0) {
#pragma unroll
        for (int r = 0; r < 16; r++) part[wave - 1][r][lane] = acc[r];
    }
    __syncthreads();
    if (wave > 0) return;
    const int64_t n = n0 + li;
#pragma unroll
    for (int r = 0; r < 16; r++) {
        float o = acc[r];
#pragma unroll
        for (int w = 1; w < MMF_W; w++) o += part[w - 1][r][lane];
        const int m = m0 + 8 * (r >> 2) + 4 * kh + (r & 3);
        if (m < M && n < nrows) Y[(size_t)m * nrows + n] = o;
    }
}

// M tokens of f16 / bf16 weight rows (ws bytes apart, ncols % 16 == 0) on the
// matrix cores: x fp32 rows (xs floats apart) or prepared activation rows at
// `as` bytes (exactly one of x, act)
hipError_t launch_mm_float(int wtype, const uint8_t *W, size_t ws, int64_t nrows, int64_t ncols, const float *x, size_t xs,
                           const uint8_t *act, size_t as, int M, float *Y, hipStream_t s) {
    if ((wtype != F16 && wtype != BF16) || ncols % 16 || ws % 16 || (uintptr_t)W % 16 || M < 1 || (x == nullptr) == (act == nullptr))
        return hipErrorInvalidValue;
    if (x ? ((uintptr_t)x % 16 || xs % 4) : ((uintptr_t)act % 16 || as % 16)) return hipErrorInvalidValue;
    const dim3 grid((unsigned)((nrows + 31) / 32), (unsigned)((M + 31) / 32));
    const uint8_t *a = x ? (const uint8_t *)x : act;
    const size_t ab = x ? xs * 4 : as;
    if (wtype == F16) {
        if (x) hipLaunchKernelGGL((k_mm_float<F16, true>), grid, dim3(64 * MMF_W), 0, s, W, ws, nrows, ncols, a, ab, M, Y);
        else hipLaunchKernelGGL((k_mm_float<F16, false>), grid, dim3(64 * MMF_W), 0, s, W, ws, nrows, ncols, a, ab, M, Y);
    } else {
        if (x) hipLaunchKernelGGL((k_mm_float<BF16, true>), grid, dim3(64 * MMF_W), 0, s, W, ws, nrows, ncols, a, ab, M, Y);
        else hipLaunchKernelGGL((k_mm_float<BF16, false>), grid, dim3(64 * MMF_W), 0, s, W, ws, nrows, ncols, a, ab, M, Y);
    }
    return hipGetLastError();
}

hipError_t launch_act_float(int wtype, const float *x, size_t xs, int64_t ncols, int nb, uint8_t *out, size_t os, hipStream_t s) {
    hipLaunchKernelGGL(k_act_float, dim3((unsigned)((ncols + 255) / 256), (unsigned)nb), dim3(256), 0, s, wtype, x, xs, ncols, out, os);
    return hipGetLastError();
}

}  // namespace g4
