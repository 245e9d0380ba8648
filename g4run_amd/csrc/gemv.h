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
#define G4_GEMV_STORE(v) (v)
#include "gemv_body.inc"
#undef G4_GEMV_STORE
}

// one token whose store is `out` (a GELU product, GemvOut): a kernel of its
// own, so the plain store carries neither the argument nor the branch
template <class F, int LPR, int UPL, int XQ>
__global__ __launch_bounds__((gemv_max_threads<F, 1, XQ>())) void k_gemv_out(g4h_tensor W, const uint8_t *__restrict__ act, size_t act_stride,
                                               const float *__restrict__ x, float *__restrict__ Y, int units, GemvOut out) {
    constexpr int NB = 1;
#define G4_GEMV_STORE(v) gemv_out_value(out, row, (v))
#include "gemv_body.inc"
#undef G4_GEMV_STORE
}

template <class F, int NB, int LPR, int UPL, int XQ>
static void gemv_launch(dim3 grid, dim3 block, size_t lds, hipStream_t s, const g4h_tensor &W, const uint8_t *act, size_t stride,
                        const float *x, float *Y, int units, const GemvOut &out) {
    if constexpr (NB == 1) {
        if (out.mode != OUT_STORE) {
            hipLaunchKernelGGL((k_gemv_out<F, LPR, UPL, XQ>), grid, block, lds, s, W, act, stride, x, Y, units, out);
            return;
        }
    }
    hipLaunchKernelGGL((k_gemv<F, NB, LPR, UPL, XQ>), grid, block, lds, s, W, act, stride, x, Y, units);
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
static hipError_t go(const g4h_tensor &W, const uint8_t *act, size_t stride, const float *x, float *Y, int units, hipStream_t s,
                     const GemvOut &out) {
    constexpr int RPW = 64 / LPR;
    const size_t lds = act_lds_bytes<F>(NB, W.nb);
    const int wpg = gemv_pick_waves(W, NB, RPW, x != nullptr, lds);
    const int64_t waves = (W.nrows + RPW - 1) / RPW;
    const unsigned grid = (unsigned)((waves + wpg - 1) / wpg);
    if (!x) {
        if (64 * wpg > gemv_max_threads<F, NB, 0>()) return hipErrorInvalidValue;
        gemv_launch<F, NB, LPR, UPL, 0>(dim3(grid), dim3(64 * wpg), lds, s, W, act, stride, x, Y, units, out);
        return hipGetLastError();
    }
    constexpr bool QK = F::type == Q4_0 || F::type == Q8_0;
    if constexpr (!QK && NB != 1) {
        return hipErrorInvalidValue;                                 // K-quants: one fused token (gemv_fused_fits)
    } else {
        int xwpg;
        const int xq = gemv_xq_shape(W.ncols, NB, waves, wpg, &xwpg);
        if (xq == 2) {
            gemv_launch<F, NB, LPR, UPL, 2>(dim3(grid), dim3(64 * wpg), lds, s, W, act, stride, x, Y, units, out);
        } else if constexpr (NB == 1) {
            if (xq != 4) return hipErrorInvalidValue;
            const unsigned grid4 = (unsigned)((waves + xwpg - 1) / xwpg);
            gemv_launch<F, 1, LPR, UPL, 4>(dim3(grid4), dim3(64 * xwpg), lds, s, W, act, stride, x, Y, units, out);
        } else {
            return hipErrorInvalidValue;
        }
        return hipGetLastError();
    }
}

template <class F, int NB>
static hipError_t pick(const g4h_tensor &W, const uint8_t *act, size_t stride, const float *x, float *Y, hipStream_t s, int lpr,
                       int upl, const GemvOut &out) {
    const int units = (int)(W.nb * F::units_per_block);
#define G4_CASE(L, U) if (lpr == L && upl == U) return go<F, NB, L, U>(W, act, stride, x, Y, units, s, out)
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
                       int lpr, int upl, const GemvOut &out) {
    if (out.mode != OUT_STORE && nb != 1) return hipErrorInvalidValue;
    switch (nb) {
    case 1: return pick<F, 1>(W, act, stride, x, Y, s, lpr, upl, out);
    case 2: return pick<F, 2>(W, act, stride, x, Y, s, lpr, upl, out);
    case 4: return pick<F, 4>(W, act, stride, x, Y, s, lpr, upl, out);
    case 8: return pick<F, 8>(W, act, stride, x, Y, s, lpr, upl, out);
    default: return hipErrorInvalidValue;
    }
}

}  // namespace g4
