// k_gemv.hip -- decode GEMV / small-batch matmul over resident quantized
// weights (the GPU form of matmul_b + mm_kernel, model.c:191-270).
//
// One workgroup = 4 waves.  A wave covers 64/LPR rows at a time; the LPR lanes
// of a row split its units (blocks or quarter-superblocks) round-robin, each
// lane holding up to UPL units of weight bytes in registers.  Every weight
// byte is read from HBM exactly once with aligned 128-bit loads, issued before
// the workgroup waits for its activation staging so the stream is in flight
// while the activation lands in LDS.  The NB token activations of the call are
// staged once per workgroup; the per-token fp32 accumulation order depends on
// LPR only (chosen from the row length), never on NB, so token b's result is
// bit-identical for any batch size (the x4 contract of g4run.h:148-157).
#include "formats.h"
#include "kernels.h"

namespace g4 {

template <class F, int NB, int LPR, int UPL>
__global__ __launch_bounds__(256) void k_gemv(g4h_tensor W, const uint8_t *__restrict__ act, size_t act_stride,
                                              float *__restrict__ Y, int units) {
    extern __shared__ __align__(16) uint8_t lds[];
    using Act = typename F::Act;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int g = lane % LPR, rg = lane / LPR;
    constexpr int RPW = 64 / LPR;
    const int64_t row0 = (int64_t)blockIdx.x * 4 * RPW + wave * RPW + rg;
    const bool row_ok = row0 < W.nrows;
    const int64_t row = row_ok ? row0 : W.nrows - 1;

    typename F::Frag fr[UPL];
#pragma unroll
    for (int k = 0; k < UPL; k++) {
        const int u = g + k * LPR;
        if (u < units) F::load(fr[k], W, row, u);
    }
    if constexpr (F::type == Q4_0 || F::type == Q8_0) stage_q8_0<NB>(lds, act, act_stride, (int)W.nb);
    else stage_q8_K<NB>(lds, act, act_stride, (int)W.nb);
    __syncthreads();

    float acc[NB];
#pragma unroll
    for (int t = 0; t < NB; t++) acc[t] = 0.0f;
#pragma unroll
    for (int k = 0; k < UPL; k++) {
        const int u = g + k * LPR;
        if (u < units) {
#pragma unroll
            for (int t = 0; t < NB; t++) acc[t] = F::accum(fr[k], Act(lds, (int)W.nb, t), u, acc[t]);
        }
    }
    // units beyond LPR*UPL (very long rows): further passes in the same order
    for (int base = LPR * UPL; base < units; base += LPR * UPL) {
#pragma unroll
        for (int k = 0; k < UPL; k++) {
            const int u = base + g + k * LPR;
            if (u < units) F::load(fr[k], W, row, u);
        }
#pragma unroll
        for (int k = 0; k < UPL; k++) {
            const int u = base + g + k * LPR;
            if (u < units) {
#pragma unroll
                for (int t = 0; t < NB; t++) acc[t] = F::accum(fr[k], Act(lds, (int)W.nb, t), u, acc[t]);
            }
        }
    }
#pragma unroll
    for (int t = 0; t < NB; t++) acc[t] = group_sum<LPR>(acc[t]);
    if (g == 0 && row_ok) {
#pragma unroll
        for (int t = 0; t < NB; t++) Y[(size_t)t * W.nrows + row] = acc[t];
    }
}

// Exact per-block integer sums of every row against token `tok`: one thread
// per (row, block); the parts of a superblock are added as integers.
template <class F>
__global__ __launch_bounds__(256) void k_block_sums(g4h_tensor W, const uint8_t *__restrict__ act, size_t act_stride,
                                                    int tok, int32_t *__restrict__ out) {
    extern __shared__ __align__(16) uint8_t lds[];
    using Act = typename F::Act;
    if constexpr (F::type == Q4_0 || F::type == Q8_0) stage_q8_0<1>(lds, act + (size_t)tok * act_stride, act_stride, (int)W.nb);
    else stage_q8_K<1>(lds, act + (size_t)tok * act_stride, act_stride, (int)W.nb);
    __syncthreads();
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= W.nrows * W.nb) return;
    const int64_t row = i / W.nb;
    const int j = (int)(i - row * W.nb);
    int tot[F::nsums] = {};
    for (int p = 0; p < F::units_per_block; p++) {
        typename F::Frag f;
        const int u = j * F::units_per_block + p;
        F::load(f, W, row, u);
        int s[F::nsums];
        F::sums(f, Act(lds, (int)W.nb, 0), u, s);
        for (int k = 0; k < F::nsums; k++) tot[k] += s[k];
    }
    for (int k = 0; k < F::nsums; k++) out[i * F::nsums + k] = tot[k];
}

// ------------------------------------------------------------- dispatch ----
template <class F>
size_t act_lds_bytes(int nb_tokens, int64_t nblk) { return (size_t)nb_tokens * F::Act::bytes_per_token((int)nblk); }

template <class F, int NB, int LPR, int UPL>
static hipError_t go(const g4h_tensor &W, const uint8_t *act, size_t stride, float *Y, int units, hipStream_t s) {
    constexpr int rows_per_wg = 4 * (64 / LPR);
    const unsigned grid = (unsigned)((W.nrows + rows_per_wg - 1) / rows_per_wg);
    const size_t lds = act_lds_bytes<F>(NB, W.nb);
    hipLaunchKernelGGL((k_gemv<F, NB, LPR, UPL>), dim3(grid), dim3(256), lds, s, W, act, stride, Y, units);
    return hipGetLastError();
}

template <class F, int NB>
static hipError_t pick(const g4h_tensor &W, const uint8_t *act, size_t stride, float *Y, hipStream_t s, int lpr, int upl) {
    const int units = (int)(W.nb * F::units_per_block);
#define G4_CASE(L, U) if (lpr == L && upl == U) return go<F, NB, L, U>(W, act, stride, Y, units, s)
    G4_CASE(16, 4); G4_CASE(16, 8); G4_CASE(32, 4); G4_CASE(32, 8); G4_CASE(64, 4); G4_CASE(64, 8);
#undef G4_CASE
    return hipErrorInvalidValue;
}

// Lanes per row from the row length only (so the fp32 order never depends on
// the batch size): the fewest lanes that keep each lane at <= 8 units.
void gemv_shape(int type, int64_t nblk, int *lpr, int *upl) {
    const int units = (int)(nblk * (blck(type) == 256 ? 4 : 1));
    int L = units <= 16 * 8 ? 16 : units <= 32 * 8 ? 32 : 64;
    const int per = (units + L - 1) / L;
    *lpr = L;
    *upl = per <= 4 ? 4 : 8;
}

size_t gemv_lds_bytes(int type, int nb_tokens, int64_t nblk) {
    return (type == Q4_0 || type == Q8_0) ? act_lds_bytes<FQ8_0>(nb_tokens, nblk) : act_lds_bytes<FQ4_K>(nb_tokens, nblk);
}

hipError_t launch_gemv(const g4h_tensor &W, const uint8_t *act, size_t stride, float *Y, int nb, hipStream_t s) {
    int lpr, upl;
    gemv_shape(W.type, W.nb, &lpr, &upl);
#define G4_NB(N)                                                                             \
    if (nb == N) {                                                                           \
        switch (W.type) {                                                                    \
        case Q8_0: return pick<FQ8_0, N>(W, act, stride, Y, s, lpr, upl);                    \
        case Q4_0: return pick<FQ4_0, N>(W, act, stride, Y, s, lpr, upl);                    \
        case Q4_K: return pick<FQ4_K, N>(W, act, stride, Y, s, lpr, upl);                    \
        case Q3_K: return pick<FQ3_K, N>(W, act, stride, Y, s, lpr, upl);                    \
        case Q2_K: return pick<FQ2_K, N>(W, act, stride, Y, s, lpr, upl);                    \
        default: return hipErrorInvalidValue;                                                \
        }                                                                                    \
    }
    G4_NB(1) G4_NB(2) G4_NB(4) G4_NB(8)
#undef G4_NB
    return hipErrorInvalidValue;
}

template <class F>
static hipError_t bs_go(const g4h_tensor &W, const uint8_t *act, size_t stride, int tok, int32_t *out, hipStream_t s) {
    const int64_t n = W.nrows * W.nb;
    hipLaunchKernelGGL(k_block_sums<F>, dim3((unsigned)((n + 255) / 256)), dim3(256), act_lds_bytes<F>(1, W.nb), s,
                       W, act, stride, tok, out);
    return hipGetLastError();
}

hipError_t launch_block_sums(const g4h_tensor &W, const uint8_t *act, size_t stride, int tok, int32_t *out, hipStream_t s) {
    switch (W.type) {
    case Q8_0: return bs_go<FQ8_0>(W, act, stride, tok, out, s);
    case Q4_0: return bs_go<FQ4_0>(W, act, stride, tok, out, s);
    case Q4_K: return bs_go<FQ4_K>(W, act, stride, tok, out, s);
    case Q3_K: return bs_go<FQ3_K>(W, act, stride, tok, out, s);
    case Q2_K: return bs_go<FQ2_K>(W, act, stride, tok, out, s);
    default: return hipErrorInvalidValue;
    }
}

int block_sums_per_block(int type) { return (type == Q2_K || type == Q4_K) ? 2 : 1; }

}  // namespace g4
