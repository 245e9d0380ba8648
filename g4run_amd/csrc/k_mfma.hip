// k_mfma.hip -- batched-prefill matmul on the int8 matrix cores (the
// many-token form of matmul_b, model.c:191-270, for q8_0 / q4_0 weights
// against q8_0 activations).
//
// One v_mfma_i32_32x32x32_i8 covers exactly one 32-element block for a 32
// token x 32 row tile, so every per-block integer sum is exact (the integers
// of quants.c:535-562).  The block's fp32 scale d_w*d_a is the outer product
// of the two fp16 scale vectors, formed exactly by one v_mfma_f32_32x32x16_f16
// whose only non-zero k carries (d_a, d_w) -- an fp16 x fp16 product is exact
// in fp32 -- and lands in the same accumulator layout.  The VALU then does
// one convert and one fma per output per block:
//   acc[t][r] = fma(float(isum_b[t][r]), d_a[t][b] * d_w[r][b], acc[t][r]),
// blocks in increasing order (a different fp32 order from the GEMV family,
// within the path's fp32 tolerance).  q4_0 nibbles are unpacked to q-8 in
// registers.  Each output keeps four fp32 partial sums (residue pair
// b / 2 mod 4 of block b) added in a fixed order, so a token's result does not
// depend on the batch size or on the kernel variant (the x4 contract of
// g4run.h:148-157 within this family).
//
// Activations are first laid out planar (qa [M][nb][32] int8, da [M][nb] fp16)
// so every operand load is an aligned 16-byte load.  Kernels: k_mm_few, 16-row
// strips that read each weight byte once for up to 64 tokens (their own
// tile-major activation layout); k_mm_mfma, one 32 x 32 tile per workgroup
// whose residue pairs are split over 4 waves and added in wave order through
// LDS; and k_mm_lds, 64 x 128 tiles staged through LDS in 8-block stages
// shared by 8 waves (many tokens: 1/8 of the operand traffic per output).
#include <algorithm>
#include <cstdio>
#include <type_traits>

#include "formats.h"
#include "kernels.h"
#include "steps.h"

namespace g4 {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));
typedef _Float16 v8h __attribute__((ext_vector_type(8)));
typedef float v16f __attribute__((ext_vector_type(16)));
typedef float v32f __attribute__((ext_vector_type(32)));
typedef float v4f __attribute__((ext_vector_type(4)));
typedef _Float16 v4h __attribute__((ext_vector_type(4)));

constexpr int MM_KB_SMALL = 8;       // blocks per operand set, one-tile workgroups


// q4_0 half-block: nibbles of 16 bytes -> 16 int8 values q - 8 (low nibbles
// are elements 0..15, high nibbles 16..31, quants.c:542-545)
__device__ __forceinline__ v4i q4_half(v4i w, int kh) {
    v4i r;
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const uint32_t n = ((uint32_t)w[i] >> (4 * kh)) & 0x0F0F0F0Fu;
        r[i] = (int)((n + 0x78787878u) ^ 0x80808080u);          // per byte: n - 8, no carries (n + 0x78 <= 0x87)
    }
    return r;
}

template <int WT, int WM, int WN, int KB>
__global__ __launch_bounds__(256) void k_mm_mfma(g4h_tensor W, const int8_t *__restrict__ qa,
                                                  const uint16_t *__restrict__ da, int M, float *__restrict__ Y) {
    // Four partial sums per output, one per residue pair (the blocks b with
    // b / 2 mod 4 = r), each over its blocks in increasing order, then
    // ((p0 + p1) + p2) + p3.  Wave ks of the four on a tile holds residue
    // pair ks: blocks 8 j + 2 ks and 8 j + 2 ks + 1 for j = 0, 1, ...
    constexpr int KS = 4;
    static_assert(KB % 2 == 0, "a set is whole pair steps");
    __shared__ float red[(KS - 1) * 64 * 16];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int wm = wave % WM, wn = (wave / WM) % WN, ks = wave / (WM * WN);
    const int m0 = (blockIdx.y * WM + wm) * 32, n0 = (blockIdx.x * WN + wn) * 32;
    const int li = lane & 31, kh = lane >> 5;
    const int nb = (int)W.nb;
    const int tok = min(m0 + li, M - 1);
    const int64_t row = min((int64_t)(n0 + li), W.nrows - 1);
    const int8_t *pa = qa + (size_t)tok * nb * 32 + 16 * kh;
    const uint16_t *pda = da + (size_t)tok * nb;
    // q8_0: lane half kh reads its half-block plane (common.h); 16 bytes per block either way
    const uint8_t *pw = (WT == Q8_0 && kh ? W.ex : W.qs) + (size_t)row * nb * 16;
    const uint16_t *pdw = (const uint16_t *)W.sc + (size_t)row * nb;

    v16f acc;
#pragma unroll
    for (int r = 0; r < 16; r++) acc[r] = 0.0f;
    const v16i zi = {};
    const v16f zf = {};
    // operands of KB blocks (KB / 2 pair steps); two sets alternate so the
    // next set's loads are in flight while the current one is multiplied
    struct Ops {
        v4i a[KB], w[KB];
        uint16_t sa[KB], sw[KB];
    };
    // block k of the set that starts at pair step j0
    auto blk = [&](int j0, int k) { return 8 * (j0 + (k >> 1)) + 2 * ks + (k & 1); };
    auto load = [&](Ops &o, int j0) {
#pragma unroll
        for (int k = 0; k < KB; k++) {
            const int b = min(blk(j0, k), nb - 1);
            o.a[k] = *(const v4i *)(pa + (size_t)b * 32);
            o.w[k] = *(const v4i *)(pw + (size_t)b * 16);
            o.sa[k] = pda[b];
            o.sw[k] = pdw[b];
        }
    };
    auto mul = [&](const Ops &o, int j0) {
#pragma unroll
        for (int k = 0; k < KB; k++) {
            if (blk(j0, k) < nb) {                                   // uniform
                const v4i wv = WT == Q8_0 ? o.w[k] : q4_half(o.w[k], kh);
                const v16i is = __builtin_amdgcn_mfma_i32_32x32x32_i8(o.a[k], wv, zi, 0, 0, 0);
                // selects, not a lane-divergent branch (which splits the loop
                // into exec-masked blocks)
                const _Float16 zh = (_Float16)0.0f;
                const v8h ha = {kh == 0 ? __builtin_bit_cast(_Float16, o.sa[k]) : zh, zh, zh, zh, zh, zh, zh, zh};
                const v8h hw = {kh == 0 ? __builtin_bit_cast(_Float16, o.sw[k]) : zh, zh, zh, zh, zh, zh, zh, zh};
                const v16f sc = __builtin_amdgcn_mfma_f32_32x32x16_f16(ha, hw, zf, 0, 0, 0);
#pragma unroll
                for (int r = 0; r < 16; r++) acc[r] = __builtin_fmaf((float)is[r], sc[r], acc[r]);
            }
        }
    };
    constexpr int STEP = KB / 2;
    Ops o0, o1;
    load(o0, 0);
    for (int j0 = 0;;) {
        if (blk(j0 + STEP, 0) < nb) load(o1, j0 + STEP);
        mul(o0, j0);
        j0 += STEP;
        if (blk(j0, 0) >= nb) break;
        if (blk(j0 + STEP, 0) < nb) load(o0, j0 + STEP);
        mul(o1, j0);
        j0 += STEP;
        if (blk(j0, 0) >= nb) break;
    }
    // partials of waves 1..3 through LDS, added to wave 0's in wave order
    v16f out = acc;
    if (ks > 0) {
#pragma unroll
        for (int r = 0; r < 16; r++) red[((ks - 1) * 16 + r) * 64 + lane] = out[r];
    }
    __syncthreads();
    if (ks > 0) return;
#pragma unroll
    for (int q = 1; q < KS; q++)
#pragma unroll
        for (int r = 0; r < 16; r++) out[r] += red[((q - 1) * 16 + r) * 64 + lane];
    // C[i][j]: j = lane % 32 (weight row), i = 8*(r/4) + 4*(lane/32) + r%4 (token)
    const int64_t n = n0 + li;
    if (n < W.nrows) {
#pragma unroll
        for (int r = 0; r < 16; r++) {
            const int m = m0 + 8 * (r >> 2) + 4 * kh + (r & 3);
            if (m < M) Y[(size_t)m * W.nrows + n] = out[r];
        }
    }
}

// LDS-staged tiles for many tokens (nb a multiple of KB).  A workgroup of
// TM x TN waves owns a (32 TM) token x (32 TN) row output tile; wave (im, in)
// its 32 x 32 subtile.  The K loop runs over stages of KB blocks: every thread
// loads a share of the stage's activation and weight bytes into registers
// (threads 0..BM+BN-1 also one 16-byte run of KB fp16 scales) while the waves
// multiply the previous stage from LDS, then writes them to the other LDS
// buffer, q4_0 nibbles unpacked to q - 8 and the scales widened to fp32 on the
// way.  Per block and subtile the arithmetic is that of k_mm_mfma: one int8
// MFMA for the exact block sums, the exact scale outer product d_a * d_w (here
// two blocks' from one v_mfma_f32_32x32x1_2b_f32, lanes 0..31 block k and
// 32..63 block k + 1: an fp16 x fp16 product is exact in fp32 either way), an
// fma into the accumulator of the block's residue pair, and at the end
// ((p0 + p1) + p2) + p3 -- so every output is bit-identical to k_mm_mfma's.
constexpr int MML_KB = 8;                                           // blocks per stage

template <int WT, int TM, int TN, int KB, int RST>
__global__ __launch_bounds__(64 * TM * TN, 2) void k_mm_lds(g4h_tensor W, const int8_t *__restrict__ qa,
                                                         const uint16_t *__restrict__ da, int M, float *__restrict__ Y) {
    constexpr int BM = 32 * TM, BN = 32 * TN, NT = 64 * TM * TN;
    constexpr int WB = WT == Q8_0 ? 32 : 16;                        // weight bytes per block in memory
    constexpr int RS = KB * 32 + 16;                                // padded LDS row stride (bytes), A and B
    constexpr int ACH = 2 * KB, BCH = KB * WB / 16;                 // 16-byte chunks per row and stage
    constexpr int APT = BM * ACH / NT, BPT = BN * BCH / NT;
    static_assert(BM * ACH % NT == 0 && BN * BCH % NT == 0 && NT % ACH == 0 && NT % BCH == 0, "tile shape");
    static_assert(BM + BN <= NT && KB == 8, "one 16-byte scale run per thread");
    constexpr int ZR = BM + BN;                                     // scale columns: tokens, then weight rows
    __shared__ __align__(16) int8_t As[2][BM * RS];
    __shared__ __align__(16) int8_t Bs[2][BN * RS];
    __shared__ __align__(16) float Sd[2][KB * ZR];                  // [block][token | row]: lanes read along a row
    const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
    const int im = wave % TM, in = wave / TM;
    const int li = lane & 31, kh = lane >> 5;
    const int nb = (int)W.nb, nst = nb / KB;
    const int m0 = blockIdx.y * BM;
    const int64_t n0 = (int64_t)blockIdx.x * BN;

    // per-thread load offsets (bytes from the stage's base); chunk c = t + i NT
    uint32_t aoff[APT], boff[BPT];
#pragma unroll
    for (int i = 0; i < APT; i++) {
        const int c = t + i * NT, r = c / ACH, q = c % ACH;
        aoff[i] = (uint32_t)(((size_t)min(m0 + r, M - 1) * nb) * 32 + 16 * q);
    }
    // q8_0 chunk q of a row's stage: half q & 1 of block q / 2, from that
    // half's plane (common.h); q4_0 chunk q: block q
    const uint32_t hoff = (uint32_t)(W.ex - W.qs);
#pragma unroll
    for (int i = 0; i < BPT; i++) {
        const int c = t + i * NT, r = c / BCH, q = c % BCH;
        const size_t rb = (size_t)min(n0 + r, W.nrows - 1) * nb * 16;
        boff[i] = WT == Q8_0 ? (uint32_t)(rb + 16 * (q >> 1)) + ((q & 1) ? hoff : 0u) : (uint32_t)(rb + 16 * q);
    }
    // threads past the scale rows load a weight row's run too and keep it
    const uint16_t *psc = t < BM ? da + (size_t)min(m0 + t, M - 1) * nb
                                 : (const uint16_t *)W.sc + (size_t)min(n0 + min(t - BM, BN - 1), W.nrows - 1) * nb;

    struct Stage {
        v4i a[APT], b[BPT], s;
    };
    auto load = [&](Stage &S, int s) {
        const int8_t *ab = qa + (size_t)s * KB * 32;
        const uint8_t *bb = W.qs + (size_t)s * KB * 16;
#pragma unroll
        for (int i = 0; i < APT; i++) S.a[i] = *(const v4i *)(ab + aoff[i]);
#pragma unroll
        for (int i = 0; i < BPT; i++) S.b[i] = *(const v4i *)(bb + boff[i]);
        S.s = *(const v4i *)(psc + (size_t)s * KB);
    };
    auto store = [&](const Stage &S, int buf) {
#pragma unroll
        for (int i = 0; i < APT; i++) {
            const int c = t + i * NT;
            *(v4i *)&As[buf][(c / ACH) * RS + 16 * (c % ACH)] = S.a[i];
        }
#pragma unroll
        for (int i = 0; i < BPT; i++) {
            const int c = t + i * NT, r = c / BCH, q = c % BCH;
            if constexpr (WT == Q8_0) {
                *(v4i *)&Bs[buf][r * RS + 16 * q] = S.b[i];
            } else {                                                    // block q: elements 0..15, 16..31
                *(v4i *)&Bs[buf][r * RS + 32 * q] = q4_half(S.b[i], 0);
                *(v4i *)&Bs[buf][r * RS + 32 * q + 16] = q4_half(S.b[i], 1);
            }
        }
        if (t < ZR) {
#pragma unroll
            for (int j = 0; j < KB; j++) Sd[buf][j * ZR + t] = h2f((uint16_t)((uint32_t)S.s[j / 2] >> (16 * (j & 1))));
        }
    };

    v16f acc[4];
#pragma unroll
    for (int q = 0; q < 4; q++)
#pragma unroll
        for (int r = 0; r < 16; r++) acc[q][r] = 0.0f;
    const v16i zi = {};
    const int arow = (32 * im + li) * RS + 16 * kh, brow = (32 * in + li) * RS + 16 * kh;
    const int sacol = kh * ZR + 32 * im + li, sbcol = kh * ZR + BM + 32 * in + li;
    const v32f zf32 = {};
    // block k's operands, and its exact integer sums
    struct Opnd {
        v4i a, w;
    };
    auto opnd = [&](int cur, int k) {
        return Opnd{*(const v4i *)&As[cur][arow + 32 * k], *(const v4i *)&Bs[cur][brow + 32 * k]};
    };
    auto isum = [&](const Opnd &o) { return __builtin_amdgcn_mfma_i32_32x32x32_i8(o.a, o.w, zi, 0, 0, 0); };
    // scale outer products of blocks k, k + 1 (k even) from the operands read
    // at (cur, k): registers 0..15, 16..31
    struct Sop {
        float a, b;
    };
    auto sop = [&](int cur, int k) { return Sop{Sd[cur][k * ZR + sacol], Sd[cur][k * ZR + sbcol]}; };
    auto scales = [&](const Sop &o) { return __builtin_amdgcn_mfma_f32_32x32x1f32(o.a, o.b, zf32, 0, 0, 0); };
    // the empty asm pins the block's fmas here: left alone the compiler sinks
    // every epilogue of the stage below the LDS stores, which keeps all the
    // stage's MFMA results live at once
    auto epi = [&](int k, const v16i &is, const v32f &sc, int r0 = 0, int r1 = 16) {
        v16f &p = acc[(k >> 1) & 3];                                // KB % 8 == 0: residue pair of the block
        const int o = 16 * (k & 1);
#pragma unroll
        for (int r = r0; r < r1; r++) {
            p[r] = __builtin_fmaf((float)is[r], sc[o + r], p[r]);
            asm volatile("" : "+v"(p[r]));
        }
    };
    // software-pipelined over the stage's blocks: block k + 1's integer MFMA
    // and the next pair's scale MFMA are issued before block k's epilogue, so
    // the VALU work of one block runs while the matrix cores work ahead of it;
    // every LDS operand is read one epilogue before its MFMA.  The scheduling
    // barriers keep the compiler from hoisting every MFMA of the stage (which
    // would need more registers than a wave has).
    auto compute = [&](int s) {
        const int cur = s & 1;
        Opnd o0 = opnd(cur, 0), o1 = opnd(cur, 1);
        Sop so = sop(cur, 0);
        v16i is0 = isum(o0), is1;
        v32f sc[2];
        sc[0] = scales(so);
        if (KB > 2) so = sop(cur, 2);
#pragma unroll
        for (int k = 0; k < KB; k += 2) {
            const int p = k >> 1;
            is1 = isum(o1);
            if (k + 2 < KB) o0 = opnd(cur, k + 2);
            epi(k, is0, sc[p & 1], 0, 8);                            // the matrix core runs is1 meanwhile
            __builtin_amdgcn_sched_barrier(0);
            if (k + 2 < KB) sc[(p + 1) & 1] = scales(so);
            epi(k, is0, sc[p & 1], 8, 16);
            __builtin_amdgcn_sched_barrier(0);
            if (k + 2 < KB) {
                is0 = isum(o0);
                o1 = opnd(cur, k + 3);
                if (k + 4 < KB) so = sop(cur, k + 4);
            }
            epi(k + 1, is1, sc[p & 1]);
            __builtin_amdgcn_sched_barrier(0);
        }
    };
    // RST = 2: two stages of loads in flight: while stage s is multiplied
    // from LDS, the registers hold stage s + 1 (loaded one stage earlier,
    // stored to LDS after the multiply) and receive stage s + 2.  RST = 1: the
    // registers receive stage s + 1 only (fewer registers).  Every load is
    // issued on every pass (past the end it repeats the last stage) and every
    // store made, so the memory counter waits before a store cover only the
    // stage stored, not the one just issued.
    if constexpr (RST == 2) {
        Stage S0, S1;
        load(S0, 0);
        load(S1, min(1, nst - 1));
        store(S0, 0);
        __syncthreads();
        for (int s = 0;; s += 2) {                                  // uniform
            load(S0, min(s + 2, nst - 1));
            compute(s);
            store(S1, 1);
            __syncthreads();
            if (s + 1 >= nst) break;
            load(S1, min(s + 3, nst - 1));
            compute(s + 1);
            store(S0, 0);
            __syncthreads();
            if (s + 2 >= nst) break;
        }
    } else {
        Stage S0;
        load(S0, 0);
        store(S0, 0);
        __syncthreads();
        for (int s = 0;; s++) {                                     // uniform
            load(S0, min(s + 1, nst - 1));
            compute(s);
            store(S0, (s + 1) & 1);
            __syncthreads();
            if (s + 1 >= nst) break;
        }
    }
    v16f out = acc[0];
#pragma unroll
    for (int q = 1; q < 4; q++)
#pragma unroll
        for (int r = 0; r < 16; r++) out[r] += acc[q][r];
    // C[i][j]: j = lane % 32 (weight row), i = 8*(r/4) + 4*(lane/32) + r%4 (token)
    const int64_t n = n0 + 32 * in + li;
    if (n < W.nrows) {
#pragma unroll
        for (int r = 0; r < 16; r++) {
            const int m = m0 + 32 * im + 8 * (r >> 2) + 4 * kh + (r & 3);
            if (m < M) Y[(size_t)m * W.nrows + n] = out[r];
        }
    }
}

// Few tokens (M <= 64): 16-row strips.  A workgroup of 4 waves owns 16 weight
// rows and every token, so each weight byte is read from HBM once per call;
// there is no LDS staging and no barrier until the final sum.  Wave w takes
// the blocks of residue pair w (blocks 8 j + 2 w, 8 j + 2 w + 1: a "pair
// step").  Per pair step and lane: one 16-byte weight load (q8_0; 8 bytes of
// nibbles for q4_0) covering both blocks of its row (lane groups 0, 1 block
// 2 p, groups 2, 3 block 2 p + 1), one 2-byte weight scale, one 16-byte
// activation load per 16-token tile and one 8-byte load of four tiles'
// activation scales.  A wave keeps the loads of FEW_AHEAD pair steps in
// flight: step k + FEW_AHEAD's loads go out before step k multiplies.
// One v_permlane32_swap per dword pair turns the loaded halves into the
// operands of the two blocks' int8 MFMAs (lane group g then holds slice
// sigma(g) of the block: (0, 2, 1, 3) for q8_0, g for q4_0), and the
// activations are laid out so that each lane's 16 bytes are its slice of both
// blocks (k_quantize_few).  Per block and 16 x 16 tile: one
// v_mfma_i32_16x16x32_i8 for the exact block sums, one v_mfma_f32_16x16x16_f16
// for the exact scale product d_a * d_w (one non-zero k per lane group picks
// the block and tile), and an fma into the tile's accumulator -- the
// arithmetic of k_mm_mfma and k_mm_lds, so every output is the same bits.
//
// Activation layout for M <= 64 (MT 16-token tiles, np = ceil(nb / 2) block
// pairs, padding tokens and the padding block zero):
//   qa [np][MT][16 tok][4 slices][2 blocks][8 bytes]
//   da [np][16 tok][2 blocks][4 tiles] fp16 (tile slots past MT zero)
constexpr int MMF_MAXM = 64;


typedef long v1l;
typedef int v2i __attribute__((ext_vector_type(2)));

// f(integral_constant<int, I>) for I = 0 .. N-1 as straight-line code (every
// array index a constant from the start, so the arrays stay in registers)
template <int I, int N, class F>
__device__ __forceinline__ void static_for(F &&f) {
    if constexpr (I < N) {
        f(std::integral_constant<int, I>{});
        static_for<I + 1, N>(f);
    }
}

size_t mm_few_bytes(int M, int64_t ncols) {
    const int64_t np = (ncols / 32 + 1) / 2, mt = (M + 15) / 16;
    return (((size_t)np * mt * 1024 + 255) & ~(size_t)255) + (size_t)np * 256;
}

// The pair steps run as straight-line chunks of FEW_CHUNK steps (then one
// chunk each of 8, 4, 2, 1 for the rest, so no step is wasted), FEW_AHEAD
// steps of loads in flight (MT + 3 loads per step, within the 63 the memory
// counter tracks).  Straight-line code keeps the compiler's memory-counter
// waits exact: a register ring carried around a loop is undone (InstCombine
// folds the phi of loads into one load at the loop head, buffer loads sink to
// the latch) and every iteration drains.  Measured against whole segments of
// loads issued before their multiplies (x quantized in the call, us):
// q8_0 4096x4096 at 32 / 64 tokens 12.95 -> 11.79 / 16.36 -> 14.89; q4_0
// 2560x10240 at 1 token 22.4 -> 18.4; q4_0 20480x2560 at 32 tokens 35.0 ->
// 25.1; q8_0 2048x2048 at 1 token 9.86 -> 7.58.  A window of 8 steps was
// slower at 64 tokens (16.0 us).
constexpr int FEW_CHUNK = 16, FEW_AHEAD = 4;

template <int WT, int MT>
__global__ __launch_bounds__(256) void k_mm_few(g4h_tensor W, const int8_t *__restrict__ qa,
                                                const uint16_t *__restrict__ da, int M, float *__restrict__ Y) {
    using WV = std::conditional_t<WT == Q8_0, v4i, v2i>;
    __shared__ float red[3 * MT * 4 * 64];
    // the wave index in a scalar register: the first lane's thread index / 64
    // (the compiler folds a readfirstlane of threadIdx.x / 64 itself away and
    // then keeps the value in a vector register).  Every per-step branch and
    // address part below is then scalar, with no exec-masked flow blocks.
    const int t = threadIdx.x, lane = t & 63;
    const int wave = __builtin_amdgcn_readfirstlane(t) >> 6;
    const int li = lane & 15, kg = lane >> 4;
    const int nb = (int)W.nb, np = (nb + 1) >> 1;
    const int nj = (np - wave + 3) >> 2;                                    // this wave's pair steps
    const int64_t row = min((int64_t)blockIdx.x * 16 + li, W.nrows - 1);
    // the slice of a block this lane group feeds the int8 MFMA after the swap
    const int sl = WT == Q8_0 ? ((kg & 1) << 1) | (kg >> 1) : kg;
    // per-lane 32-bit byte offsets, fixed over the loop; the per-step part is
    // uniform (the launch keeps the weight planes under 4 GB).  q8_0: lane
    // group kg takes half kg & 1 of block 2 p + kg / 2 from that half's plane
    // (common.h); q4_0: bytes 8 kg .. 8 kg + 7 of the pair's 32 nibble bytes.
    // The weight bytes of an odd last pair's missing block are the next row's
    // (or, past the last row, the next plane's): loaded, never used.  Its
    // scale index is clamped to the row.
    const uint32_t wlane = WT == Q8_0 ? (uint32_t)((uint64_t)row * nb * 16) + 16 * (kg >> 1) + ((kg & 1) ? (uint32_t)(W.ex - W.qs) : 0u)
                                      : (uint32_t)((uint64_t)row * nb * 16) + 8 * kg;
    const uint32_t slane1 = (uint32_t)((uint64_t)row * nb * 2) + 2 * (kg & 1), slane0 = slane1 - 2 * (kg & 1);
    const uint32_t alane = li * 64 + 16 * sl, dlane = 8 * (2 * li + (kg & 1));

    struct Op {
        WV w;
        v4i a[MT];
        uint64_t d;
        uint32_t s;
    };
    // pair step j of this wave: pair 4 j + wave, clamped to the last pair
    auto load = [&](int j) __attribute__((always_inline)) -> Op {
        const int p = min(4 * j + wave, np - 1);
        Op o;
        o.w = *(const WV *)(W.qs + (size_t)p * 32 + wlane);
        o.s = *(const uint16_t *)(W.sc + (size_t)p * 4 + (2 * p + 1 < nb ? slane1 : slane0));
        // a step past the wave's last, or the missing block of an odd last
        // pair, gets weight scale 0: its products add +0 to the accumulator,
        // which never holds -0, so the sums keep their bits
        const bool live = j < nj, live1 = live && 2 * p + 1 < nb;            // uniform
        if (!((kg & 1) ? live1 : live)) o.s = 0;
        static_for<0, MT>([&](auto I) { o.a[I.value] = *(const v4i *)(qa + ((size_t)p * MT + I.value) * 1024 + alane); });
        o.d = *(const uint64_t *)((const uint8_t *)da + (size_t)p * 256 + dlane);
        return o;
    };
    v4f acc[MT];
#pragma unroll
    for (int tt = 0; tt < MT; tt++) acc[tt] = v4f{0.0f, 0.0f, 0.0f, 0.0f};
    const v4i zi = {};
    const v4f zf = {};
    auto mac = [&](const Op &o) __attribute__((always_inline)) {
        uint32_t x0, x1, y0, y1;
        if constexpr (WT == Q8_0) {
            x0 = (uint32_t)o.w[0], x1 = (uint32_t)o.w[1], y0 = (uint32_t)o.w[2], y1 = (uint32_t)o.w[3];
        } else {
            // bytes 8 (kg & 1) .. + 7 of a block: low nibbles are slice kg & 1,
            // high nibbles slice 2 + (kg & 1) (quants.c:542-545), each as q - 8
            const uint32_t u0 = (uint32_t)o.w[0], u1 = (uint32_t)o.w[1];
            x0 = ((u0 & 0x0F0F0F0Fu) + 0x78787878u) ^ 0x80808080u;
            x1 = ((u1 & 0x0F0F0F0Fu) + 0x78787878u) ^ 0x80808080u;
            y0 = (((u0 >> 4) & 0x0F0F0F0Fu) + 0x78787878u) ^ 0x80808080u;
            y1 = (((u1 >> 4) & 0x0F0F0F0Fu) + 0x78787878u) ^ 0x80808080u;
        }
        // lanes 32..63 of x trade with lanes 0..31 of y: x becomes block 2 p
        // in all four lane groups, y block 2 p + 1
        const auto s0 = __builtin_amdgcn_permlane32_swap(x0, y0, false, false);
        const auto s1 = __builtin_amdgcn_permlane32_swap(x1, y1, false, false);
        const v1l bx = (v1l)(((uint64_t)s1[0] << 32) | s0[0]), by = (v1l)(((uint64_t)s1[1] << 32) | s0[1]);
        // scale operands: lane group 0 holds d_w of block 2 p, group 1 that of
        // 2 p + 1; hw[h][e] has it at k = 4 h + e, where the activation
        // operand holds d_a of block h for tile 2 (tt / 2) + e
        // (selects, not branches: lane-divergent ifs here split the loop into
        // exec-masked blocks, across which the compiler kept every step's
        // MFMA results live -- 256 registers and more instead of 84 to 166)
        const _Float16 sw = __builtin_bit_cast(_Float16, (uint16_t)o.s), zh = (_Float16)0.0f;
        const _Float16 sw0 = kg == 0 ? sw : zh, sw1 = kg == 1 ? sw : zh;
        const v4h hw[2][2] = {{v4h{sw0, zh, zh, zh}, v4h{zh, sw0, zh, zh}}, {v4h{sw1, zh, zh, zh}, v4h{zh, sw1, zh, zh}}};
#pragma unroll
        for (int tt = 0; tt < MT; tt++) {
            const v2i dv = {(int)(uint32_t)(o.d >> (32 * (tt >> 1))), 0};
            const v4h ha = __builtin_bit_cast(v4h, dv);
            const v1l a0 = (v1l)(((uint64_t)(uint32_t)o.a[tt][1] << 32) | (uint32_t)o.a[tt][0]);
            const v1l a1 = (v1l)(((uint64_t)(uint32_t)o.a[tt][3] << 32) | (uint32_t)o.a[tt][2]);
            const v4i i0 = __builtin_amdgcn_mfma_i32_16x16x32_i8(a0, bx, zi, 0, 0, 0);
            const v4f c0 = __builtin_amdgcn_mfma_f32_16x16x16f16(ha, hw[0][tt & 1], zf, 0, 0, 0);
#pragma unroll
            for (int r = 0; r < 4; r++) acc[tt][r] = __builtin_fmaf((float)i0[r], c0[r], acc[tt][r]);
            const v4i i1 = __builtin_amdgcn_mfma_i32_16x16x32_i8(a1, by, zi, 0, 0, 0);
            const v4f c1 = __builtin_amdgcn_mfma_f32_16x16x16f16(ha, hw[1][tt & 1], zf, 0, 0, 0);
#pragma unroll
            for (int r = 0; r < 4; r++) acc[tt][r] = __builtin_fmaf((float)i1[r], c1[r], acc[tt][r]);
        }
    };

    // a chunk of C pair steps from j0; scheduling barriers keep each step's
    // loads where they are issued and one step's multiplies at a time (left
    // alone the compiler hoists the chunk's MFMAs and runs out of registers)
    auto chunk = [&](auto Cc, int j0) __attribute__((always_inline)) {
        constexpr int C = decltype(Cc)::value, A = FEW_AHEAD < C ? FEW_AHEAD : C;
        Op ops[C];
        static_for<0, A>([&](auto I) { ops[I.value] = load(j0 + I.value); });
        __builtin_amdgcn_sched_barrier(0);
        static_for<0, C>([&](auto I) {
            constexpr int k = I.value;
            if constexpr (k + A < C) ops[k + A] = load(j0 + k + A);
            __builtin_amdgcn_sched_barrier(0);
            mac(ops[k]);
            __builtin_amdgcn_sched_barrier(0);
        });
    };
    int j0 = 0;
    for (; j0 + FEW_CHUNK <= nj; j0 += FEW_CHUNK) chunk(std::integral_constant<int, FEW_CHUNK>{}, j0);
    const int rest = nj - j0;                                                // uniform in the wave
    static_assert(FEW_CHUNK == 16, "the rest is taken as 8 + 4 + 2 + 1");
    if (rest & 8) chunk(std::integral_constant<int, 8>{}, j0), j0 += 8;
    if (rest & 4) chunk(std::integral_constant<int, 4>{}, j0), j0 += 4;
    if (rest & 2) chunk(std::integral_constant<int, 2>{}, j0), j0 += 2;
    if (rest & 1) chunk(std::integral_constant<int, 1>{}, j0);

    // ((p0 + p1) + p2) + p3 through LDS; C[i][j]: i = 4 kg + r (token), j = li (row)
    if (wave > 0) {
#pragma unroll
        for (int tt = 0; tt < MT; tt++)
#pragma unroll
            for (int r = 0; r < 4; r++) red[(((wave - 1) * MT + tt) * 4 + r) * 64 + lane] = acc[tt][r];
    }
    __syncthreads();
    if (wave > 0) return;
    const int64_t orow = (int64_t)blockIdx.x * 16 + li;
#pragma unroll
    for (int tt = 0; tt < MT; tt++) {
#pragma unroll
        for (int r = 0; r < 4; r++) {
            float o = acc[tt][r];
#pragma unroll
            for (int q = 1; q < 4; q++) o += red[(((q - 1) * MT + tt) * 4 + r) * 64 + lane];
            const int m = tt * 16 + 4 * kg + r;
            if (m < M && orow < W.nrows) Y[(size_t)m * W.nrows + orow] = o;
        }
    }
}

// x fp32 [M][ncols] (row stride xs floats) -> q8_0 codes and fp16 scales with
// the quantizer arithmetic of quants.c:74-109 (8 lanes per block), laid out
// token-major (qa [M][nb][32], da [M][nb]) or, FEW, in k_mm_few's layout of
// mt tiles: there grid.y also covers the padding tokens up to an even tile
// count and grid.x the padding block of an odd nb, which get zero codes and
// scales.  A thread quantizes QP groups of 4 inputs, 256 groups apart, all
// loads issued first.
constexpr int QP = 4;
template <bool FEW>
__global__ __launch_bounds__(256) void k_quantize_planar(const float *__restrict__ x, size_t xs, int64_t ncols, int M, int mt,
                                                         int8_t *__restrict__ qa, uint16_t *__restrict__ da) {
    const int64_t ng = ncols / 4, nb = ncols / 32;
    const int64_t ngo = FEW ? ((nb + 1) & ~(int64_t)1) * 8 : ng;     // groups written per token
    const int m = blockIdx.y;
    float v[QP][4];
#pragma unroll
    for (int j = 0; j < QP; j++) {
        const int64_t gi = (int64_t)blockIdx.x * 256 * QP + j * 256 + threadIdx.x;
        if (m < M && gi < ng) f4(ldf4(x + (size_t)m * xs + 4 * gi), v[j]);
        else v[j][0] = v[j][1] = v[j][2] = v[j][3] = 0.0f;
    }
#pragma unroll
    for (int j = 0; j < QP; j++) {
        const int64_t gi = (int64_t)blockIdx.x * 256 * QP + j * 256 + threadIdx.x;
        float am = fmaxf(fmaxf(fabsf(v[j][0]), fabsf(v[j][1])), fmaxf(fabsf(v[j][2]), fabsf(v[j][3])));
        am = group_max<8>(am);
        const float id = am != 0.0f ? 127.0f / am : 0.0f;
        uint32_t pk = 0;
#pragma unroll
        for (int e = 0; e < 4; e++) pk |= ((uint32_t)(int)__builtin_rintf(v[j][e] * id) & 0xffu) << (8 * e);
        if (gi < ngo) {
            const uint16_t d = f2h(am * (1.0f / 127.0f));
            if constexpr (FEW) {
                const int64_t b = gi >> 3;
                const int g = (int)(gi & 7);
                if ((m >> 4) < mt) *(uint32_t *)(qa + few_q(b, m, mt, 4 * g)) = pk;
                if (g == 0) da[few_d(b, m)] = d;
            } else {
                *(uint32_t *)(qa + ((size_t)m * nb) * 32 + 4 * gi) = pk;
                if ((gi & 7) == 0) da[(size_t)m * nb + gi / 8] = d;
            }
        }
    }
}

// GGUF q8_0 activation rows (stride bytes) -> token-major or (FEW) few-token
// layout, padding as k_quantize_planar's
template <bool FEW>
__global__ __launch_bounds__(256) void k_act_planar(const uint8_t *__restrict__ act, size_t stride, int64_t nb, int M, int mt,
                                                    int8_t *__restrict__ qa, uint16_t *__restrict__ da) {
    const int64_t nbo = FEW ? (nb + 1) & ~(int64_t)1 : nb;
    const int mo = FEW ? 16 * ((mt + 1) & ~1) : M;
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;    // (token, block, quarter)
    if (i >= (int64_t)mo * nbo * 4) return;
    const int64_t m = i / (nbo * 4), r = i - m * nbo * 4, b = r >> 2, q = r & 3;
    uint32_t w[2] = {0, 0};
    uint16_t d = 0;
    if (m < M && b < nb) {
        const uint8_t *blk = act + (size_t)m * stride + (size_t)b * 34;
#pragma unroll
        for (int k = 0; k < 2; k++) {
            const uint8_t *p = blk + 2 + 8 * q + 4 * k;
            w[k] = (uint32_t)p[0] | ((uint32_t)p[1] << 8) | ((uint32_t)p[2] << 16) | ((uint32_t)p[3] << 24);
        }
        d = (uint16_t)(blk[0] | (blk[1] << 8));
    }
    if constexpr (FEW) {
        if ((m >> 4) < mt) *(uint2 *)(qa + few_q(b, (int)m, mt, 8 * (int)q)) = make_uint2(w[0], w[1]);
        if (q == 0) da[few_d(b, (int)m)] = d;
    } else {
        *(uint2 *)(qa + ((size_t)m * nb + b) * 32 + 8 * q) = make_uint2(w[0], w[1]);
        if (q == 0) da[(size_t)m * nb + b] = d;
    }
}

// k_mm_few for up to 64 tokens while its 32-bit weight offsets reach every row
static bool mm_few(const g4h_tensor &W, int M) {
    if (const char *e = getenv("G4H_MM_FEW"))
        if (atoi(e) == 0) return false;
    return M <= MMF_MAXM && (uint64_t)W.nrows * W.nb * (W.type == Q8_0 ? 32 : 16) < (1ull << 32) - 256;
}

size_t mm_planar_bytes(int M, int64_t ncols) {
    const int64_t nb = ncols / 32;
    const size_t planar = (((size_t)M * nb * 32 + 255) & ~(size_t)255) + (size_t)M * nb * 2;
    return M <= MMF_MAXM ? std::max(planar, mm_few_bytes(M, ncols)) : planar;
}

// One 32 x 32 tile per workgroup with the blocks split over 4 waves while
// that gives at most one workgroup per CU, LDS-staged tiles beyond (those need
// nb % 8 == 0 and 32-bit operand offsets; other shapes stay on the one-tile
// kernel, whose outputs are the same bits).  Measured (x quantized in the
// call, us one-tile / staged): q8_0 4096 x 4096 at 72 tokens 33.0 / 25.3, 128
// tokens 39.7 / 25.7, 192 tokens 54.7 / 26.0; q4_0 2560 x 2048 at 96 tokens
// (240 tiles) 14.3 / 15.0, 128 tokens 21.5 / 15.0; q4_0 2560 x 10240 at 96
// tokens 51.2 / 54.0, 128 tokens 79.5 / 54.5, 256 tokens 120.9 / 56.3.
static bool mm_small(const g4h_tensor &W, int M) {
    const int64_t tiles = ((W.nrows + 31) / 32) * ((M + 31) / 32);
    const uint64_t wb = W.type == Q8_0 ? 32 : 16;
    int64_t most = 256;                                              // G4H_MM_SMALL_TILES overrides (measurement)
    if (const char *e = getenv("G4H_MM_SMALL_TILES")) most = atoll(e);
    return tiles <= most || W.nb % MML_KB != 0 || (uint64_t)M * W.nb * 32 >= (1ull << 32) ||
           (uint64_t)W.nrows * W.nb * wb >= (1ull << 32) - 512;     // q8_0: the second half-plane starts 256-B aligned
}

// Staged tile shape: 64 x 128 (8 waves, two register stages) when that still
// gives every CU a workgroup, else 64 x 64 (4 waves, one register stage).
// Measured on q8_0 4096 x 4096: 256 tokens 26.4 us as 64 x 64 / 35.7 us as
// 64 x 128; 512 tokens 41.7 / 40.4 us.  Both give the same bits.
static bool mm_wide(const g4h_tensor &W, int M) { return ((W.nrows + 127) / 128) * ((M + 63) / 64) >= 256; }

void mm_describe(const g4h_tensor &W, int M, char *buf, size_t len) {
    const char *tn = W.type == Q8_0 ? "q8_0" : "q4_0";
    if (mm_few(W, M)) {
        snprintf(buf, len, "k_mm_few<%s,mt=%d> grid=%lld block=256", tn, (M + 15) / 16, (long long)((W.nrows + 15) / 16));
    } else if (mm_small(W, M)) {
        snprintf(buf, len, "k_mm_mfma<%s,wm=1,wn=1,kb=%d> grid=%lldx%d block=256", tn, MM_KB_SMALL,
                 (long long)((W.nrows + 31) / 32), (M + 31) / 32);
    } else if (mm_wide(W, M)) {
        snprintf(buf, len, "k_mm_lds<%s,tm=2,tn=4,kb=%d,rst=2> grid=%lldx%d block=512", tn, MML_KB,
                 (long long)((W.nrows + 127) / 128), (M + 63) / 64);
    } else {
        snprintf(buf, len, "k_mm_lds<%s,tm=2,tn=2,kb=%d,rst=1> grid=%lldx%d block=256", tn, MML_KB,
                 (long long)((W.nrows + 63) / 64), (M + 63) / 64);
    }
}

bool mm_few_ready(const g4h_tensor &W, int M) { return (W.type == Q8_0 || W.type == Q4_0) && W.nb % 2 == 0 && mm_few(W, M); }

size_t few_act_bytes(int64_t ncols, int M, size_t *da_off) {
    const size_t np = (size_t)(ncols / 32 + 1) / 2, mt = (M + 15) / 16;
    *da_off = (np * mt * 1024 + 255) & ~(size_t)255;
    return mm_few_bytes(M, ncols);
}

__global__ __launch_bounds__(256) void k_clear(uint4 *p, size_t n) {
    const size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
    if (i < n) p[i] = make_uint4(0, 0, 0, 0);
}
hipError_t launch_few_clear(uint8_t *buf, size_t bytes, hipStream_t s) {
    if ((uintptr_t)buf % 16 || bytes % 16) return hipErrorInvalidValue;
    const size_t n = bytes / 16;
    if (n) hipLaunchKernelGGL(k_clear, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, (uint4 *)buf, n);
    return hipGetLastError();
}

static hipError_t few_go(const g4h_tensor &W, const int8_t *qa, const uint16_t *da, int M, float *Y, hipStream_t s) {
    const int mt = (M + 15) / 16;
    const dim3 grid((unsigned)((W.nrows + 15) / 16));
#define G4_MF(T)                                                                                                    \
    if (mt == T) {                                                                                                  \
        if (W.type == Q8_0) hipLaunchKernelGGL((k_mm_few<Q8_0, T>), grid, dim3(256), 0, s, W, qa, da, M, Y);       \
        else hipLaunchKernelGGL((k_mm_few<Q4_0, T>), grid, dim3(256), 0, s, W, qa, da, M, Y);                    \
        return hipGetLastError();                                                                                   \
    }
    G4_MF(1) G4_MF(2) G4_MF(3) G4_MF(4)
#undef G4_MF
    return hipErrorInvalidValue;
}

hipError_t launch_quantize_few(const float *x, size_t xs, int64_t ncols, int M, const FewAct &a, hipStream_t s) {
    if (!x || !a.qa || !a.da || M <= 0 || M > MMF_MAXM || a.mt != (M + 15) / 16 || ncols % 32 || (uintptr_t)x % 16 || xs % 4)
        return hipErrorInvalidValue;
    const int mte = (a.mt + 1) & ~1;
    const int64_t np = (ncols / 32 + 1) / 2;
    hipLaunchKernelGGL(k_quantize_planar<true>, dim3((unsigned)((np * 16 + 256 * QP - 1) / (256 * QP)), 16 * mte), dim3(256), 0, s, x,
                       xs, ncols, M, a.mt, a.qa, a.da);
    return hipGetLastError();
}

hipError_t launch_mm_few_ready(const g4h_tensor &W, const FewAct &a, int M, float *Y, hipStream_t s) {
    if (M <= 0 || !mm_few_ready(W, M) || !a.qa || !a.da || a.mt != (M + 15) / 16) return hipErrorInvalidValue;
    return few_go(W, a.qa, a.da, M, Y, s);
}

template <int WT, int WM, int WN, int KB>
static hipError_t mm_go(const g4h_tensor &W, const int8_t *qa, const uint16_t *da, int M, float *Y, hipStream_t s) {
    const dim3 grid((unsigned)((W.nrows + 32 * WN - 1) / (32 * WN)), (unsigned)((M + 32 * WM - 1) / (32 * WM)));
    hipLaunchKernelGGL((k_mm_mfma<WT, WM, WN, KB>), grid, dim3(256 * WM * WN), 0, s, W, qa, da, M, Y);
    return hipGetLastError();
}

// Y[M][nrows] = W * act^T on the matrix cores.  `act` is GGUF q8_0 rows at
// `stride` (x == nullptr) or x fp32 rows (x_stride floats); `ws` holds the
// re-laid activations (mm_planar_bytes).
hipError_t launch_matmul_mfma(const g4h_tensor &W, const float *x, size_t x_stride, const uint8_t *act, size_t stride, int M,
                              float *Y, uint8_t *ws, hipStream_t s) {
    if ((W.type != Q8_0 && W.type != Q4_0) || M <= 0 || W.ncols % 32) return hipErrorInvalidValue;
    const int64_t nb = W.nb;
    int8_t *qa = (int8_t *)ws;
    if (mm_few(W, M)) {
        const int mt = (M + 15) / 16, mte = (mt + 1) & ~1;
        const int64_t np = (nb + 1) / 2;
        uint16_t *da = (uint16_t *)(ws + (((size_t)np * mt * 1024 + 255) & ~(size_t)255));
        if (x) {
            hipLaunchKernelGGL(k_quantize_planar<true>, dim3((unsigned)((np * 16 + 256 * QP - 1) / (256 * QP)), 16 * mte), dim3(256), 0,
                               s, x, x_stride, W.ncols, M, mt, qa, da);
        } else {
            const int64_t n = (int64_t)16 * mte * np * 2 * 4;
            hipLaunchKernelGGL(k_act_planar<true>, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, act, stride, nb, M, mt, qa, da);
        }
        if (hipError_t e = hipGetLastError()) return e;
        return few_go(W, qa, da, M, Y, s);
    }
    uint16_t *da = (uint16_t *)(ws + (((size_t)M * nb * 32 + 255) & ~(size_t)255));
    if (x) {
        hipLaunchKernelGGL(k_quantize_planar<false>, dim3((unsigned)((W.ncols / 4 + 256 * QP - 1) / (256 * QP)), M), dim3(256), 0, s,
                           x, x_stride, W.ncols, M, 0, qa, da);
    } else {
        const int64_t n = (int64_t)M * nb * 4;
        hipLaunchKernelGGL(k_act_planar<false>, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, act, stride, nb, M, 0, qa, da);
    }
    if (hipError_t e = hipGetLastError()) return e;
    const bool small = mm_small(W, M);
    if (small) {
        if (W.type == Q8_0) return mm_go<Q8_0, 1, 1, MM_KB_SMALL>(W, qa, da, M, Y, s);
        return mm_go<Q4_0, 1, 1, MM_KB_SMALL>(W, qa, da, M, Y, s);
    }
    if (mm_wide(W, M)) {
        const dim3 grid((unsigned)((W.nrows + 127) / 128), (unsigned)((M + 63) / 64));
        if (W.type == Q8_0) hipLaunchKernelGGL((k_mm_lds<Q8_0, 2, 4, MML_KB, 2>), grid, dim3(512), 0, s, W, qa, da, M, Y);
        else hipLaunchKernelGGL((k_mm_lds<Q4_0, 2, 4, MML_KB, 2>), grid, dim3(512), 0, s, W, qa, da, M, Y);
    } else {
        const dim3 grid((unsigned)((W.nrows + 63) / 64), (unsigned)((M + 63) / 64));
        if (W.type == Q8_0) hipLaunchKernelGGL((k_mm_lds<Q8_0, 2, 2, MML_KB, 1>), grid, dim3(256), 0, s, W, qa, da, M, Y);
        else hipLaunchKernelGGL((k_mm_lds<Q4_0, 2, 2, MML_KB, 1>), grid, dim3(256), 0, s, W, qa, da, M, Y);
    }
    return hipGetLastError();
}

}  // namespace g4
