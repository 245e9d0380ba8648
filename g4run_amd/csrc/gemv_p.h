// gemv_p.h -- persistent single-token GEMV with fused activation prologues
// and an optional GELU epilogue (decode form of matmul_b, model.c:191-270).
//
// The grid is a fixed number of workgroups per CU.  Each wave walks row
// groups gw, gw + NW, gw + 2 NW, ... (NW = all waves) with two register sets:
// the next group's weight loads are in flight while the current group is
// multiplied.  A row's units, lanes and reduction are exactly those of k_gemv
// (gemv.h) with the same LPR/UPL, so every output is bit-identical to the
// one-shot kernel's.
//
// The activation is produced once per workgroup, in LDS, by the prologue:
//   PRO_ACT    GGUF q8_0 rows staged from global memory;
//   PRO_QUANT  fp32 x quantized to q8_0 (prep_act, model.c:144-153; the
//              arithmetic of quants.c:74-109);
//   PRO_NORM   the residual update and RMSNorm in front of a projection
//              (model.c:338-345, 711-722): if delta, x' = x + rms(delta)*w_post
//              (workgroup 0 stores x' to x_out), then q8_0(rms(x')*w_pre).
// Its loads are issued before the first weight loads and its arithmetic runs
// while those are in flight.  Epilogue EPI_GELU: rows come as (gate, up) pairs
// in one wave and h = gelu(gate)*up (fp16 table, g4run.h:73-77) replaces Y.
#pragma once
#include <cstdint>

#include "formats.h"
#include "kernels.h"
#include "steps.h"

namespace g4 {

constexpr int GP_WAVES = 8;                      // waves per workgroup
constexpr int GP_MAXS = 8;                       // prologue groups of 4 per thread

struct ProLoads {
    float v[GP_MAXS][4], d[GP_MAXS][4], wp[GP_MAXS][4], wq[GP_MAXS][4];
};

// The prologue's threads are the first bd of the workgroup (bd a multiple of
// 64; every thread by default): thread t takes the groups of 4 inputs t,
// t + bd, ...  A larger workgroup that runs it with the persistent family's
// bd keeps its sums, and so its bits.  load_delta = false leaves r.d at zero
// for the caller to fill (a delta handed over inside the launch).
template <int PRO, int S>
__device__ __forceinline__ void pro_issue(ProLoads &r, const GemvPro &p, int bd = blockDim.x, bool load_delta = true) {
    const int ng = p.n >> 2, t = threadIdx.x;
    const bool act = t < bd;
    const float4 z = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
    for (int s = 0; s < S; s++) {
        const int gi = t + s * bd;
        const bool own = act && gi < ng;
        f4(own ? ldf4(p.x + 4 * gi) : z, r.v[s]);
        if constexpr (PRO == PRO_NORM) {
            f4(own && p.delta && load_delta ? ldf4(p.delta + 4 * gi) : z, r.d[s]);
            f4(own && p.delta ? ldf4(p.w_post + 4 * gi) : z, r.wp[s]);
            f4(own ? ldf4(p.w_pre + 4 * gi) : z, r.wq[s]);
        }
    }
}

template <int PRO, int S>
__device__ void pro_finish(ProLoads &r, const GemvPro &p, uint8_t *lds, int nb, bool first = blockIdx.x == 0,
                           int bd = blockDim.x) {
    __shared__ double red[16];
    const int ng = p.n >> 2, t = threadIdx.x;
    const bool act = t < bd;                                         // uniform over each wave
    if constexpr (PRO == PRO_NORM) {
        if (p.delta) {
            double ss = 0.0;
#pragma unroll
            for (int s = 0; s < S; s++)
#pragma unroll
                for (int k = 0; k < 4; k++) ss += (double)r.d[s][k] * r.d[s][k];
            const float sc = rms_scale(wg_sum_double(ss, red), p.n, p.eps);
#pragma unroll
            for (int s = 0; s < S; s++)
#pragma unroll
                for (int k = 0; k < 4; k++) r.v[s][k] = r.v[s][k] + r.d[s][k] * sc * r.wp[s][k];
        }
        if (first) {                                                 // one workgroup stores x
#pragma unroll
            for (int s = 0; s < S; s++) {
                const int gi = t + s * bd;
                if (act && gi < ng) *(float4 *)(p.x_out + 4 * gi) = make_float4(r.v[s][0], r.v[s][1], r.v[s][2], r.v[s][3]);
            }
        }
        double ss = 0.0;
#pragma unroll
        for (int s = 0; s < S; s++)
#pragma unroll
            for (int k = 0; k < 4; k++) ss += (double)r.v[s][k] * r.v[s][k];
        const float sc = rms_scale(wg_sum_double(ss, red), p.n, p.eps);
#pragma unroll
        for (int s = 0; s < S; s++)
#pragma unroll
            for (int k = 0; k < 4; k++) r.v[s][k] = r.v[s][k] * sc * r.wq[s][k];
    }
#pragma unroll
    for (int s = 0; s < S; s++) {
        if (s * bd >= ng) break;                                     // uniform
        const int gi = t + s * bd;
        if (act) q8_lds4(r.v[s], gi, gi < ng, lds, nb, 0);
    }
}

template <class F, int LPR, int UPL, int PRO, int EPI, int S>
__global__ __launch_bounds__(64 * GP_WAVES) void k_gemv_p(g4h_tensor W, const uint8_t *__restrict__ act, float *__restrict__ Y,
                                                           int units, GemvPro pro, GemvEpi epi) {
    extern __shared__ __align__(16) uint8_t lds[];
    using Act = typename F::Act;
    constexpr int RPW = 64 / LPR;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int g = lane % LPR, rg = lane / LPR;
    const int64_t NW = (int64_t)gridDim.x * GP_WAVES;
    const int64_t ngroups = (W.nrows + RPW - 1) / RPW;
    int64_t grp = (int64_t)blockIdx.x * GP_WAVES + wave;
    const int nb = (int)W.nb;

    auto row_of = [&](int64_t gq) { return min(gq * RPW + rg, W.nrows - 1); };
    // branch-free loads (clamped to the last row / unit; the extras are not
    // summed): a load under a branch makes the compiler wait for every load in
    // flight before the prologue arithmetic
    auto load = [&](typename F::Frag (&fr)[UPL], int64_t gq) {
        const int64_t row = row_of(gq);
#pragma unroll
        for (int k = 0; k < UPL; k++) F::load(fr[k], W, row, min(g + k * LPR, units - 1));
    };
    // GELU epilogue, one row group behind: the table entry of a group's gate
    // is loaded (every lane, unconditionally, behind the next group's weights)
    // and used once the next group is done, so its latency is not waited for
    // on its own.  gelu(x) = 0 for x <= -10, x for x >= 10, else the fp16
    // table (g4run.h:73-77).
    float p_gate = 0.0f, p_up = 0.0f;
    uint16_t p_tab = 0;
    int64_t p_row = -1;
    auto gelu_flush = [&]() {
        if (p_row >= 0 && g == 0 && (rg & 1) == 0 && p_row < W.nrows) {
            const float gl = p_gate <= -10.0f ? 0.0f : p_gate >= 10.0f ? p_gate : h2f(p_tab);
            epi.h[p_row >> 1] = gl * p_up;
        }
    };
    auto finish = [&](const typename F::Frag (&fr)[UPL], int64_t gq) {
        float acc = 0.0f;
        const Act A(lds, nb, 0);
#pragma unroll
        for (int k = 0; k < UPL; k++) {
            const int u = g + k * LPR;
            if (u < units) acc = F::accum(fr[k], A, u, acc);
        }
        acc = group_sum<LPR>(acc);
        const int64_t row0 = gq * RPW + rg;
        if constexpr (EPI == EPI_GELU) {
            const float up = partner<LPR>(acc);                     // row 2i+1: lane ^ LPR (LPR 16 or 32)
            const uint16_t tab = epi.gelu[f2h(acc)];
            issue_order();
            gelu_flush();                                            // the previous group's output
            p_gate = acc; p_up = up; p_tab = tab; p_row = row0;
        } else {
            if (g == 0 && row0 < W.nrows) Y[row0] = acc;
        }
    };

    // prologue loads, then the first weight set, then the prologue arithmetic
    typename StageOf<F::type>::S stg;
    ProLoads pr;
    if constexpr (PRO == PRO_ACT) stage_q8_0_load<1>(stg, threadIdx.x, act, 0, nb);
    else pro_issue<PRO, S>(pr, pro);
    typename F::Frag fa[UPL], fb[UPL];
    issue_barrier();
    load(fa, grp);
    issue_order();
    if constexpr (PRO == PRO_ACT) {
        stage_q8_0_store(stg, lds, nb, stage_dump<ActQ8_0>(lds, 1, nb));
        stage_q8_0_rest<1>(lds, act, 0, nb);
    } else {
        pro_finish<PRO, S>(pr, pro, lds, nb);
    }
    lds_barrier();                                                   // the first weight set stays in flight

    for (; grp < ngroups; grp += 2 * NW) {                            // wave-uniform
        const int64_t g2 = grp + NW, g3 = grp + 2 * NW;
        if (g2 < ngroups) load(fb, g2);
        finish(fa, grp);
        if (g2 >= ngroups) break;
        if (g3 < ngroups) load(fa, g3);
        finish(fb, g2);
    }
    if constexpr (EPI == EPI_GELU) gelu_flush();
}

template <class F, int LPR, int UPL, int PRO, int EPI>
static hipError_t gp_go(const g4h_tensor &W, const uint8_t *act, float *Y, const GemvPro &pro, const GemvEpi &epi,
                        hipStream_t s, int grid) {
    const int units = (int)(W.nb * F::units_per_block);
    const size_t lds = (size_t)F::Act::bytes_per_token((int)W.nb) + kStageDump;
    const int slots = (int)((W.ncols / 4 + 64 * GP_WAVES - 1) / (64 * GP_WAVES));
#define G4_GP(S_)                                                                                                \
    hipLaunchKernelGGL((k_gemv_p<F, LPR, UPL, PRO, EPI, S_>), dim3(grid), dim3(64 * GP_WAVES), lds, s, W, act, Y, \
                       units, pro, epi)
    if constexpr (PRO == PRO_ACT) {
        G4_GP(1);
    } else {
        if (slots <= 2) G4_GP(2);
        else if (slots <= 4) G4_GP(4);
        else G4_GP(GP_MAXS);
    }
#undef G4_GP
    return hipGetLastError();
}

template <class F, int LPR, int UPL>
static hipError_t gp_mode(const g4h_tensor &W, const uint8_t *act, float *Y, const GemvPro &pro, const GemvEpi &epi,
                          hipStream_t s, int grid) {
    if (epi.kind == EPI_GELU) {
        if constexpr (LPR <= 32) {
            if (pro.kind == PRO_NORM) return gp_go<F, LPR, UPL, PRO_NORM, EPI_GELU>(W, act, Y, pro, epi, s, grid);
        }
        return hipErrorInvalidValue;
    }
    switch (pro.kind) {
    case PRO_ACT: return gp_go<F, LPR, UPL, PRO_ACT, EPI_STORE>(W, act, Y, pro, epi, s, grid);
    case PRO_QUANT: return gp_go<F, LPR, UPL, PRO_QUANT, EPI_STORE>(W, act, Y, pro, epi, s, grid);
    case PRO_NORM: return gp_go<F, LPR, UPL, PRO_NORM, EPI_STORE>(W, act, Y, pro, epi, s, grid);
    default: return hipErrorInvalidValue;
    }
}

template <class F>
hipError_t gemv_p_format(const g4h_tensor &W, const uint8_t *act, float *Y, const GemvPro &pro, const GemvEpi &epi,
                         hipStream_t s, int lpr, int upl, int grid) {
#define G4_GPC(L, U) if (lpr == L && upl == U) return gp_mode<F, L, U>(W, act, Y, pro, epi, s, grid)
    G4_GPC(16, 2); G4_GPC(16, 4); G4_GPC(16, 8); G4_GPC(32, 2); G4_GPC(32, 4); G4_GPC(32, 8);
    G4_GPC(64, 2); G4_GPC(64, 4); G4_GPC(64, 8);
#undef G4_GPC
    return hipErrorInvalidValue;
}

}  // namespace g4
