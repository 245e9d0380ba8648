// gemv.h -- decode GEMV / small-batch matmul over resident quantized
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
#pragma once
#include <algorithm>
#include <cstdint>
#include <cstdlib>

#include "formats.h"
#include "kernels.h"

namespace g4 {

template <class F>
size_t act_lds_bytes(int nb_tokens, int64_t nblk) { return (size_t)nb_tokens * F::Act::bytes_per_token((int)nblk) + kStageDump; }


// XQ = 0: the NB activations are GGUF q8_0 / q8_K rows (act, act_stride).
// XQ > 0: x holds the NB tokens as fp32 rows of ncols (contiguous) and every
// workgroup quantizes them to q8_0 (q4_0 / q8_0 weights) or q8_K (K-quant
// weights: a superblock per 16 or 32 threads) itself, in LDS (q8_lds4 / q8K_rows: the
// arithmetic of the standalone quantizers, so results equal quantize-then-GEMV
// bit for bit);
// XQ is the number of 4-float groups per thread (NB*ncols/4 <= XQ*blockDim).
// The x loads go out before the weight stream and the quantization runs while
// the weights are in flight; an LDS-only barrier hands the activation over
// without waiting for the stream.
// Eight pre-quantized tokens over q8_0 / q4_0 weights may stage more than
// 64 KB of activations (rows of 10240 and more): that variant takes up to 16
// waves (gemv_big_stage below).
template <class F>
constexpr bool gemv_qk() { return F::type == Q4_0 || F::type == Q8_0; }
template <class F, int NB, int XQ>
constexpr int gemv_max_threads() { return XQ == 4 || (NB == 8 && XQ == 0 && gemv_qk<F>()) ? 1024 : 512; }

template <class F, int NB, int LPR, int UPL, int XQ>
__global__ __launch_bounds__((gemv_max_threads<F, NB, XQ>())) void k_gemv(g4h_tensor W, const uint8_t *__restrict__ act, size_t act_stride,
                                               const float *__restrict__ x, float *__restrict__ Y, int units) {
    extern __shared__ __align__(16) uint8_t lds[];
    using Act = typename F::Act;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, wpg = blockDim.x >> 6;
    const int g = lane % LPR, rg = lane / LPR;
    constexpr int RPW = 64 / LPR;
    const int64_t row0 = ((int64_t)blockIdx.x * wpg + wave) * RPW + rg;
    const bool row_ok = row0 < W.nrows;
    const int64_t row = row_ok ? row0 : W.nrows - 1;
    constexpr bool QK = F::type == Q4_0 || F::type == Q8_0;

    // activation loads first, then the weight stream (see formats.h); one
    // K-quant token needs about two q8_K items per thread, both issued here
    constexpr int KS = (!QK && NB == 1) ? 2 : 1;
    typename StageOf<F::type>::S stg[KS];
    float xv[XQ > 0 ? XQ : 1][4];
    const int gpt = (int)(W.ncols >> 2);                            // 4-float groups per token
    if constexpr (XQ > 0) {
        // q8_0: groups t, t + blockDim, ..; K-quants (one token): the XQ
        // consecutive groups XQ t .. (a superblock per 64 / XQ threads)
#pragma unroll
        for (int s = 0; s < XQ; s++) {                                   // clamped, unconditional
            const int gi = QK ? min((int)(threadIdx.x + s * blockDim.x), NB * gpt - 1) : min((int)(XQ * threadIdx.x) + s, gpt - 1);
            const float4 v = *(const float4 *)(x + 4 * (size_t)gi);
            xv[s][0] = v.x; xv[s][1] = v.y; xv[s][2] = v.z; xv[s][3] = v.w;
        }
    } else if constexpr (QK) {
        stage_q8_0_load<NB>(stg[0], threadIdx.x, act, act_stride, (int)W.nb);
    } else {
#pragma unroll
        for (int s = 0; s < KS; s++) stage_q8_K_load<NB>(stg[s], threadIdx.x + s * blockDim.x, act, act_stride, (int)W.nb);
    }

    issue_barrier();
    // branch-free stream: lanes past the row's last unit reload that unit and
    // leave it out of the sums (a load under a branch would make the compiler
    // wait for the whole stream before the prologue below)
    typename F::Frag fr[UPL];
#pragma unroll
    for (int k = 0; k < UPL; k++) F::load(fr[k], W, row, min(g + k * LPR, units - 1));
    issue_order();                                                   // the whole stream goes out before any wait
    if constexpr (XQ > 0 && QK) {
#pragma unroll
        for (int s = 0; s < XQ; s++) {                                   // no branch: keeps the x loads up front
            const int gi = threadIdx.x + s * blockDim.x;
            const int t = gi / gpt;
            q8_lds4(xv[s], gi - t * gpt, gi < NB * gpt, lds, (int)W.nb, t);
        }
    } else if constexpr (XQ > 0) {
        // a superblock per row of 64 / XQ threads (one token: gemv_fused_fits,
        // whose shapes give every superblock a row); rows past the last one
        // skip it
        static_assert(NB == 1, "K-quant weights quantize one fp32 token in-kernel");
        q8K_rows<XQ>(xv, (int)threadIdx.x / (64 / XQ), (int)(W.ncols >> 8), lds, (int)W.nb);
    } else if constexpr (QK) {
        stage_q8_0_store(stg[0], lds, (int)W.nb, stage_dump<ActQ8_0>(lds, NB, (int)W.nb));
        stage_q8_0_rest<NB>(lds, act, act_stride, (int)W.nb);
    } else {
#pragma unroll
        for (int s = 0; s < KS; s++) stage_q8_K_store(stg[s], lds, (int)W.nb, stage_dump<ActQ8_K>(lds, NB, (int)W.nb));
        stage_q8_K_rest<NB>(lds, act, act_stride, (int)W.nb, KS);
    }
    lds_barrier();

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

// Waves per workgroup chosen so the grid is (close to) a multiple of the 256
// CUs with equal rows per workgroup: every CU streams the same bytes.
// `stage` is the cost of one workgroup's activation staging in units of one
// wave's rows: 0 for one token (measured: its staging hides under the weight
// stream), half a row per restaged token row otherwise (gemv_stage_cost).
static inline int gemv_waves_per_group(int64_t nrows, int rpw, double stage = 0.0) {
    const int64_t waves = (nrows + rpw - 1) / rpw;
    if (const char *e = getenv("G4H_GEMV_WPG")) return atoi(e) < 1 ? 1 : atoi(e) > 8 ? 8 : atoi(e);
    // minimise the busiest CU's work, ceil(grid/256) * (wpg + stage),
    // preferring larger groups (fewer activation stagings) on ties
    int best = 1;
    double best_cost = 1e300;
    for (int w = 1; w <= 8; w++) {
        const int64_t grid = (waves + w - 1) / w;
        const double cost = (double)((grid + 255) / 256) * (w + stage);
        if (cost <= best_cost) { best_cost = cost; best = w; }
    }
    return best;
}

// Staging cost of nb > 1 tokens for gemv_waves_per_group: each token's
// activation row (q8_0 for q8_0 / q4_0 weights, q8_K for K-quants) against
// the rpw weight rows of one wave, at half the cost of a streamed weight byte
// (the activations come from L2).  Without it 8 tokens of q8_0 11008x4096
// ran one-row workgroups that each staged all 8 rows: 82.6 us against 29.6 us
// for the 4096x11008 transpose.
static inline double gemv_stage_cost(int type, int64_t nblk, int nb, int rpw) {
    if (nb <= 1) return 0.0;
    const bool kq = blck(type) == 256;
    const double act = kq ? 292.0 * nblk : 34.0 * nblk;               // q8_K / q8_0 bytes per token row
    return 0.5 * nb * act / ((double)rpw * (double)bsize(type) * (double)nblk);
}

// LDS of one CU, and the staging size from which fewer than three
// workgroups fit on it.
constexpr size_t kCuLds = 160 * 1024;
constexpr size_t kLdsSmall = 64 * 1024;
// Eight pre-quantized tokens over q8_0 / q4_0 rows whose activations take
// more than 64 KB of LDS (8 x 10240 inputs: 105 KB) leave room for one
// workgroup per CU.  The waves per workgroup then go up to 16 and the choice
// counts rounds of resident workgroups: 2560 rows of 10240 run as 256
// workgroups of 10 waves in one round, where 8 waves would need 320
// workgroups, a second round for 64 of them.
static inline bool gemv_big_stage(int type, int nb, bool xq, size_t lds) {
    return nb == 8 && !xq && (type == Q4_0 || type == Q8_0) && lds > kLdsSmall;
}
static inline int gemv_waves_big(int64_t nrows, int rpw, double stage, size_t lds) {
    const int64_t waves = (nrows + rpw - 1) / rpw;
    const int64_t res = std::max<int64_t>(1, (int64_t)(kCuLds / lds));  // workgroups a CU holds
    int best = 1;
    double best_cost = 1e300;
    for (int w = 1; w <= 16; w++) {
        const int64_t n = ((waves + w - 1) / w + 255) / 256;           // workgroups per CU
        const int64_t rounds = (n + res - 1) / res;
        const double cost = (double)rounds * (double)std::min(n, res) * (w + stage);
        if (cost <= best_cost) { best_cost = cost; best = w; }
    }
    return best;
}
static inline int gemv_pick_waves(const g4h_tensor &W, int nb, int rpw, bool xq, size_t lds) {
    const double stage = gemv_stage_cost(W.type, W.nb, nb, rpw);
    return gemv_big_stage(W.type, nb, xq, lds) ? gemv_waves_big(W.nrows, rpw, stage, lds)
                                               : gemv_waves_per_group(W.nrows, rpw, stage);
}

// 4-float groups per thread the fused quantizer needs (0 = no fused variant).
// Every workgroup reads and quantizes all of x, so the fused form pays only
// while x is small next to the workgroup's weights: up to two groups per
// thread (q4_0 10240x2560: 5.5 us fused against 7.3 us for quantize + GEMV;
// with eight groups, 2560x10240 took 8.8 us against 7.9 us).
// One token with a wider input (the 10240-wide down projection) takes up to
// four groups per thread instead, in workgroups of up to 16 waves chosen as
// gemv_waves_per_group does: 2560x10240 runs 256 workgroups of 10 waves, one
// per CU, so each CU reads and quantizes x once.  Past two such workgroups per
// CU a separate quantizer launch is cheaper (q4_0 32768x10240: 49.3 us fused
// against 29.9 us for the GEMV on a quantized input).  Returns 0, 2 or 4 and
// the waves per workgroup of that launch.
static inline int gemv_xq_shape(int64_t ncols, int nb, int64_t waves, int wpg, int *xwpg) {
    const int64_t ng = (int64_t)nb * (ncols / 4);
    *xwpg = wpg;
    if (ng <= 2 * 64 * (int64_t)wpg) return 2;
    static const bool wide = [] {
        const char *e = getenv("G4H_GEMV_XQ4");
        return !e || atoi(e) != 0;
    }();
    if (nb != 1 || !wide) return 0;
    int best = 0;
    int64_t best_cost = INT64_MAX;
    for (int w = 1; w <= 16; w++) {
        if (ng > 4 * 64 * (int64_t)w) continue;
        const int64_t grid = (waves + w - 1) / w;
        const int64_t cost = (grid + 255) / 256 * w;
        if (cost < best_cost) { best_cost = cost; best = w; }
    }
    if (!best || best_cost > 2 * 16) return 0;                      // more than two 16-wave workgroups per CU
    *xwpg = best;
    return 4;
}

template <class F, int NB, int LPR, int UPL>
static hipError_t go(const g4h_tensor &W, const uint8_t *act, size_t stride, const float *x, float *Y, int units, hipStream_t s) {
    constexpr int RPW = 64 / LPR;
    const size_t lds = act_lds_bytes<F>(NB, W.nb);
    const int wpg = gemv_pick_waves(W, NB, RPW, x != nullptr, lds);
    const int64_t waves = (W.nrows + RPW - 1) / RPW;
    const unsigned grid = (unsigned)((waves + wpg - 1) / wpg);
    if (!x) {
        if (64 * wpg > gemv_max_threads<F, NB, 0>()) return hipErrorInvalidValue;
        hipLaunchKernelGGL((k_gemv<F, NB, LPR, UPL, 0>), dim3(grid), dim3(64 * wpg), lds, s, W, act, stride, x, Y, units);
        return hipGetLastError();
    }
    constexpr bool QK = F::type == Q4_0 || F::type == Q8_0;
    if constexpr (!QK && NB != 1) {
        return hipErrorInvalidValue;                                 // K-quants: one fused token (gemv_fused_fits)
    } else {
        int xwpg;
        const int xq = gemv_xq_shape(W.ncols, NB, waves, wpg, &xwpg);
        if (xq == 2) {
            hipLaunchKernelGGL((k_gemv<F, NB, LPR, UPL, 2>), dim3(grid), dim3(64 * wpg), lds, s, W, act, stride, x, Y, units);
        } else if constexpr (NB == 1) {
            if (xq != 4) return hipErrorInvalidValue;
            const unsigned grid4 = (unsigned)((waves + xwpg - 1) / xwpg);
            hipLaunchKernelGGL((k_gemv<F, 1, LPR, UPL, 4>), dim3(grid4), dim3(64 * xwpg), lds, s, W, act, stride, x, Y, units);
        } else {
            return hipErrorInvalidValue;
        }
        return hipGetLastError();
    }
}

template <class F, int NB>
static hipError_t pick(const g4h_tensor &W, const uint8_t *act, size_t stride, const float *x, float *Y, hipStream_t s, int lpr,
                       int upl) {
    const int units = (int)(W.nb * F::units_per_block);
#define G4_CASE(L, U) if (lpr == L && upl == U) return go<F, NB, L, U>(W, act, stride, x, Y, units, s)
    upl = gemv_upl_final(W.type, W.nb, NB, lpr, upl);
    if constexpr (NB == 1) {
        G4_CASE(16, 1); G4_CASE(16, 2); G4_CASE(16, 3); G4_CASE(16, 4); G4_CASE(16, 5); G4_CASE(16, 6); G4_CASE(16, 7);
        G4_CASE(16, 8); G4_CASE(32, 1); G4_CASE(32, 2); G4_CASE(32, 3); G4_CASE(32, 4); G4_CASE(32, 5); G4_CASE(32, 6);
        G4_CASE(32, 7); G4_CASE(32, 8); G4_CASE(64, 1); G4_CASE(64, 2); G4_CASE(64, 3); G4_CASE(64, 4); G4_CASE(64, 5);
        G4_CASE(64, 6); G4_CASE(64, 7); G4_CASE(64, 8);
    } else {
        G4_CASE(16, 2); G4_CASE(16, 4); G4_CASE(16, 8); G4_CASE(32, 2); G4_CASE(32, 4); G4_CASE(32, 8);
        G4_CASE(64, 2); G4_CASE(64, 4); G4_CASE(64, 8);
    }
#undef G4_CASE
    return hipErrorInvalidValue;
}

// one translation unit per format instantiates these
// x != nullptr: fp32 tokens quantized inside the kernel (q8_0 / q4_0 weights;
// the caller checks gemv_fused_fits)
template <class F>
hipError_t gemv_format(const g4h_tensor &W, const uint8_t *act, size_t stride, const float *x, float *Y, int nb, hipStream_t s,
                       int lpr, int upl) {
    switch (nb) {
    case 1: return pick<F, 1>(W, act, stride, x, Y, s, lpr, upl);
    case 2: return pick<F, 2>(W, act, stride, x, Y, s, lpr, upl);
    case 4: return pick<F, 4>(W, act, stride, x, Y, s, lpr, upl);
    case 8: return pick<F, 8>(W, act, stride, x, Y, s, lpr, upl);
    default: return hipErrorInvalidValue;
    }
}

}  // namespace g4
