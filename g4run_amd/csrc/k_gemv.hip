// k_gemv.hip -- GEMV dispatch (kernel family in gemv.h, one instantiation unit
// per weight format) and the per-block integer-sum instrument.
#include <algorithm>

#include "gemv.h"
#include "gemv_p.h"

namespace g4 {

hipError_t launch_gemv_q8_0(const g4h_tensor &, const uint8_t *, size_t, const float *, float *, int, hipStream_t, int, int, const GemvOut &);
hipError_t launch_gemv_q4_0(const g4h_tensor &, const uint8_t *, size_t, const float *, float *, int, hipStream_t, int, int, const GemvOut &);
hipError_t launch_gemv_q4_K(const g4h_tensor &, const uint8_t *, size_t, const float *, float *, int, hipStream_t, int, int, const GemvOut &);
hipError_t launch_gemv_q3_K(const g4h_tensor &, const uint8_t *, size_t, const float *, float *, int, hipStream_t, int, int, const GemvOut &);
hipError_t launch_gemv_q5_K(const g4h_tensor &, const uint8_t *, size_t, const float *, float *, int, hipStream_t, int, int, const GemvOut &);
hipError_t launch_gemv_q6_K(const g4h_tensor &, const uint8_t *, size_t, const float *, float *, int, hipStream_t, int, int, const GemvOut &);
hipError_t launch_gemv_q2_K(const g4h_tensor &, const uint8_t *, size_t, const float *, float *, int, hipStream_t, int, int, const GemvOut &);
hipError_t launch_gemv_tq2_0(const g4h_tensor &, const uint8_t *, size_t, const float *, float *, int, hipStream_t, int, int, const GemvOut &);

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

// About 64 weight bytes per lane per pass (2 q8_0 blocks, 4 q4_0 blocks, 2
// K-quant quarter-superblocks): enough loads in flight per lane, enough waves
// in flight per CU (measured best on the BASELINE shapes).
void gemv_shape(int type, int64_t nblk, int *lpr, int *upl) {
    const int units = (int)(nblk * (blck(type) == 256 ? 4 : 1));
    const int target = type == Q4_0 ? 4 : 2;
    const int want = (units + target - 1) / target;
    int L = want <= 16 ? 16 : want <= 32 ? 32 : 64;
    if (const char *e = getenv("G4H_GEMV_LPR")) L = atoi(e);
    const int per = (units + L - 1) / L;
    *lpr = L;
    *upl = per <= 2 ? 2 : per <= 4 ? 4 : 8;
}

void gemv_launch_shape(const g4h_tensor &W, int *lpr, int *upl, int *wpg, int64_t *grid, int nb, bool xq) {
    gemv_shape(W.type, W.nb, lpr, upl);
    const int rpw = 64 / *lpr;
    *wpg = gemv_pick_waves(W, nb, rpw, xq, gemv_lds_bytes(W.type, nb, W.nb));
    const int64_t waves = (W.nrows + rpw - 1) / rpw;
    *grid = (waves + *wpg - 1) / *wpg;
}

size_t gemv_lds_bytes(int type, int nb_tokens, int64_t nblk) {
    return (type == Q4_0 || type == Q8_0) ? act_lds_bytes<FQ8_0>(nb_tokens, nblk) : act_lds_bytes<FQ4_K>(nb_tokens, nblk);
}

static hipError_t gemv_dispatch(const g4h_tensor &W, const uint8_t *act, size_t stride, const float *x, float *Y, int nb,
                                hipStream_t s, const GemvOut &out) {
    int lpr, upl;
    gemv_shape(W.type, W.nb, &lpr, &upl);
    switch (W.type) {
    case Q8_0: return launch_gemv_q8_0(W, act, stride, x, Y, nb, s, lpr, upl, out);
    case Q4_0: return launch_gemv_q4_0(W, act, stride, x, Y, nb, s, lpr, upl, out);
    case Q4_K: return launch_gemv_q4_K(W, act, stride, x, Y, nb, s, lpr, upl, out);
    case Q3_K: return launch_gemv_q3_K(W, act, stride, x, Y, nb, s, lpr, upl, out);
    case Q5_K: return launch_gemv_q5_K(W, act, stride, x, Y, nb, s, lpr, upl, out);
    case Q6_K: return launch_gemv_q6_K(W, act, stride, x, Y, nb, s, lpr, upl, out);
    case Q2_K: return launch_gemv_q2_K(W, act, stride, x, Y, nb, s, lpr, upl, out);
    case TQ2_0: return launch_gemv_tq2_0(W, act, stride, x, Y, nb, s, lpr, upl, out);
    default: return hipErrorInvalidValue;
    }
}

hipError_t launch_gemv(const g4h_tensor &W, const uint8_t *act, size_t stride, float *Y, int nb, hipStream_t s, const GemvOut &out) {
    return gemv_dispatch(W, act, stride, nullptr, Y, nb, s, out);
}

// The fused-quantizer variant exists for q8_0 / q4_0 weights when every
// thread of the launch holds at most 2 groups of 4 inputs, or 4 for one token
// (gemv_xq_shape).
bool gemv_fused_fits(const g4h_tensor &W, int nb) {
    const bool kq = blck(W.type) == 256 && W.type != Q8_K;          // K-quants: q8_K activations, one token
    if (W.type != Q8_0 && W.type != Q4_0 && !(kq && nb == 1)) return false;
    if (nb != 1 && nb != 2 && nb != 4 && nb != 8) return false;
    int lpr, upl, wpg, xwpg;
    int64_t grid;
    gemv_launch_shape(W, &lpr, &upl, &wpg, &grid, nb, true);
    const int64_t waves = (W.nrows + 64 / lpr - 1) / (64 / lpr);
    return gemv_xq_shape(W.ncols, nb, waves, wpg, &xwpg) != 0;
}

hipError_t launch_gemv_x(const g4h_tensor &W, const float *x, float *Y, int nb, hipStream_t s, const GemvOut &out) {
    if (!gemv_fused_fits(W, nb) || !x) return hipErrorInvalidValue;
    return gemv_dispatch(W, nullptr, 0, x, Y, nb, s, out);
}

hipError_t launch_gemv_p_q8_0(const g4h_tensor &, const uint8_t *, float *, const GemvPro &, const GemvEpi &, hipStream_t, int,
                              int, int);
hipError_t launch_gemv_p_q4_0(const g4h_tensor &, const uint8_t *, float *, const GemvPro &, const GemvEpi &, hipStream_t, int,
                              int, int);

// Persistent family: the one-shot kernel's LPR/UPL (identical results), a
// single pass over each row (units <= LPR*UPL), prologue inputs <= 16384 wide.
// The GELU epilogue pairs rows inside a wave, so it takes only shapes whose
// one-shot LPR is at most 32: any other LPR would sum each row in another
// order than the one-shot kernel (e.g. q8_0 rows of 2560, LPR 64), and the
// decode step runs GELU as its own step there.
static bool gemv_p_shape(const g4h_tensor &W, const GemvEpi &epi, int *lpr, int *upl) {
    gemv_shape(W.type, W.nb, lpr, upl);
    if (epi.kind == EPI_GELU && *lpr > 32) return false;
    return W.nb <= (int64_t)(*lpr) * (*upl);
}

bool gemv_p_fits(const g4h_tensor &W, const GemvPro &pro, const GemvEpi &epi) {
    int lpr, upl;
    if (W.type != Q4_0 && W.type != Q8_0) return false;
    if (!gemv_p_shape(W, epi, &lpr, &upl)) return false;
    if (pro.kind != PRO_ACT && (W.ncols > 16384 || W.ncols % 32 || pro.n != W.ncols)) return false;
    if (epi.kind == EPI_GELU && W.nrows % 2) return false;
    return true;
}

// workgroups: a fixed count per CU (G4H_GEMV_P_OCC overrides the default of 2)
int gemv_p_grid_size() {
    static const int occ = [] {
        const char *e = getenv("G4H_GEMV_P_OCC");
        const int v = e ? atoi(e) : 2;
        return v < 1 ? 1 : v > 4 ? 4 : v;
    }();
    return 256 * occ;
}

hipError_t launch_gemv_p(const g4h_tensor &W, const uint8_t *act, float *Y, const GemvPro &pro, const GemvEpi &epi,
                         hipStream_t s) {
    if (!gemv_p_fits(W, pro, epi)) return hipErrorInvalidValue;
    if (pro.kind == PRO_ACT && !act) return hipErrorInvalidValue;
    if (pro.kind != PRO_ACT && !pro.x) return hipErrorInvalidValue;
    if (pro.kind == PRO_NORM && (!pro.w_pre || !pro.x_out || (pro.delta && !pro.w_post))) return hipErrorInvalidValue;
    if (epi.kind == EPI_GELU ? (!epi.h || !epi.gelu) : !Y) return hipErrorInvalidValue;
    int lpr, upl;
    gemv_p_shape(W, epi, &lpr, &upl);
    // no more workgroups than row groups to give each wave one (a wave without
    // a row group would still stream a clamped duplicate of the last row)
    const int64_t groups = (W.nrows + 64 / lpr - 1) / (64 / lpr);
    const int grid = (int)std::min<int64_t>(gemv_p_grid_size(), (groups + GP_WAVES - 1) / GP_WAVES);
    return W.type == Q8_0 ? launch_gemv_p_q8_0(W, act, Y, pro, epi, s, lpr, upl, grid)
                          : launch_gemv_p_q4_0(W, act, Y, pro, epi, s, lpr, upl, grid);
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
    case Q5_K: return bs_go<FQ5_K>(W, act, stride, tok, out, s);
    case Q6_K: return bs_go<FQ6_K>(W, act, stride, tok, out, s);
    case Q2_K: return bs_go<FQ2_K>(W, act, stride, tok, out, s);
    case TQ2_0: return bs_go<FTQ2_0>(W, act, stride, tok, out, s);
    default: return hipErrorInvalidValue;
    }
}

int block_sums_per_block(int type) { return (type == Q2_K || type == Q4_K || type == Q5_K) ? 2 : 1; }

}  // namespace g4
