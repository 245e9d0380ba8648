// k_mfma_k.hip -- batched-prefill matmul on the int8 matrix cores for K-quant
// weights (q4_K, q6_K) against q8_K activations: the many-token form of
// matmul_b (model.c:191-270) for the formats real gemma GGUFs carry, whose
// batched dots are x1 dots four times (quants.c:1535-1547).
//
// A workgroup owns a 32-token x 32-row output tile; its MMK_NW waves split
// the row's superblocks (wave w takes s = w, w + MMK_NW, ...), two
// superblocks' operands loaded at a time, and their partial tiles are summed
// through LDS in wave order.
// Per superblock every integer the reference forms is exact:
//   q4_K (quants.c:713-762): isum = sum_j sc_j * sum_32 q4 * q8 over the 8
//     sub-blocks j of 32 -- one v_mfma_i32_32x32x32_i8 per sub-block, each
//     tile scaled by the lane's row's 6-bit sc_j on the VALU (a 24-bit
//     multiply-add); summ = sum_g m_{g/2} * bsum_g over the q8_K row's 16
//     sums of 16 -- one v_mfma_f32_32x32x16_f16 whose operands (|bsum| <=
//     2048, m <= 63) and partial sums (< 2^24) are integers fp16 and fp32
//     hold exactly.  y += (d_a * d) * isum - (d_a * dmin) * summ.
//   q6_K (quants.c:582-622): per 16-element sub-block s, sum (q6 - 32) * q8 *
//     sc_s = sc_s * sum q6u * q8 - 32 * sc_s * bsum_s with q6u = q6 + 32 in
//     0..63: each sub-block is one v_mfma_i32_32x32x16_i8, scaled by sc_s on
//     the VALU; the correction sum_s sc_s * bsum_s (|.| < 2^23) is one exact
//     f16 MFMA.  y += (d_a * d) * (isum - 32 * corr).
// The fp32 products d_a * d (and d_a * dmin) of a superblock come from one
// fp32 MFMA whose only nonzero k term is each product (rounded once), in the
// integer tiles' layout.  Each wave accumulates its
// superblocks in increasing order and the waves' tiles are added in wave
// order, so a token's result does not depend on the batch size (the x4
// contract of g4run.h:148-157 within this family); the fp32 order differs
// from the CPU dots' within the path's tolerance.
//
// Activations are the GGUF q8_K rows themselves (d f32 | 256 int8 | 16 int16
// bsums, 292 bytes a superblock): a lane's 16-byte operand slices are
// 4-byte-aligned loads.
#include <algorithm>
#include <cstdio>

#include "formats.h"
#include "kernels.h"

namespace g4 {

typedef int mk_v2i __attribute__((ext_vector_type(2)));
typedef int mk_v4i __attribute__((ext_vector_type(4)));
typedef int mk_v16i __attribute__((ext_vector_type(16)));
typedef float mk_v16f __attribute__((ext_vector_type(16)));
typedef float mk_v32f __attribute__((ext_vector_type(32)));
typedef _Float16 mk_v8h __attribute__((ext_vector_type(8)));

constexpr int MMK_NW = 8;             // waves per workgroup, splitting the superblocks of one 32 x 32 tile

__device__ __forceinline__ mk_v4i mk_ld(const uint8_t *p) { return *(const mk_v4i *)p; }
__device__ __forceinline__ mk_v16i mk_mma(mk_v4i a, mk_v4i b, mk_v16i c) { return __builtin_amdgcn_mfma_i32_32x32x32_i8(a, b, c, 0, 0, 0); }
__device__ __forceinline__ mk_v16i mk_mma16(mk_v2i a, mk_v2i b, mk_v16i c) {
    return __builtin_amdgcn_mfma_i32_32x32x16_i8(__builtin_bit_cast(long, a), __builtin_bit_cast(long, b), c, 0, 0, 0);
}
__device__ __forceinline__ mk_v16f mk_mma_h(mk_v8h a, mk_v8h b) {
    const mk_v16f z = {};
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, z, 0, 0, 0);
}

// the lane's slice of one q8_K superblock of its token: quants 32 j + 16 kh
// .. + 15 of every sub-block j, bsums 8 kh .. 8 kh + 7, and d
struct MkAct {
    mk_v4i q[8], bs;
    float d;
};
__device__ __forceinline__ void mk_load_act(MkAct &a, const uint8_t *ab, int kh) {
#pragma unroll
    for (int j = 0; j < 8; j++) a.q[j] = mk_ld(ab + 4 + 32 * j + 16 * kh);
    a.bs = mk_ld(ab + 260 + 16 * kh);
    a.d = *(const float *)ab;
}
// the 8 int16 bsums as fp16 (exact: |bsum| <= 16 * 128)
__device__ __forceinline__ mk_v8h mk_bsums(const mk_v4i &bs) {
    mk_v8h h;
#pragma unroll
    for (int k = 0; k < 4; k++) {
        h[2 * k] = (_Float16)(short)(bs[k] & 0xffff);
        h[2 * k + 1] = (_Float16)(short)((uint32_t)bs[k] >> 16);
    }
    return h;
}

// one q4_K superblock: exact isum tile, exact summ tile, and the scale
// products (P[0..15] = d_a d, P[16..31] = d_a dmin)
struct Q4KSb {
    static constexpr int T = Q4_K, SEG = 2;                              // superblocks whose loads go out together
    // the lane's row: 16-byte header (d | dmin | 12 scale bytes) and its
    // k-half of the 4 nibble rows of 32 bytes
    struct W {
        mk_v4i hdr, q[4];
    };
    static __device__ __forceinline__ void load(W &w, const g4h_tensor &Wt, int64_t row, int s, int kh) {
        const uint8_t *b = Wt.qs + ((size_t)row * Wt.nb + s) * 144;
        w.hdr = mk_ld(b);
#pragma unroll
        for (int p = 0; p < 4; p++) w.q[p] = mk_ld(b + 16 + 32 * p + 16 * kh);
    }
    // 6-bit scale and min of sub-block j (quants.c:417-423, get_scale_min_k4)
    static __device__ __forceinline__ void scale_min(const mk_v4i &hdr, int j, int &sc, int &m) {
        const uint32_t w0 = (uint32_t)hdr.y, w1 = (uint32_t)hdr.z, w2 = (uint32_t)hdr.w;   // scale bytes 0..11
        auto byte = [&](int i) -> int { return (int)(((i < 4 ? w0 : i < 8 ? w1 : w2) >> (8 * (i & 3))) & 0xff); };
        if (j < 4) {
            sc = byte(j) & 63;
            m = byte(j + 4) & 63;
        } else {
            sc = (byte(j + 4) & 0xF) | ((byte(j - 4) >> 6) << 4);
            m = (byte(j + 4) >> 4) | ((byte(j) >> 6) << 4);
        }
    }
    static __device__ __forceinline__ void load_act(MkAct &a, const uint8_t *ab, int kh) { mk_load_act(a, ab, kh); }
    static __device__ __forceinline__ void mul(const W &w, const MkAct &a, int kh, mk_v16f &acc) {
        const mk_v16i z = {};
        mk_v16i isum = {};
        int mn[8];
#pragma unroll
        for (int p = 0; p < 4; p++) {
            const mk_v4i lo = w.q[p] & 0x0F0F0F0F, hi = (w.q[p] >> 4) & 0x0F0F0F0F;
            int sc0, sc1;
            scale_min(w.hdr, 2 * p, sc0, mn[2 * p]);
            scale_min(w.hdr, 2 * p + 1, sc1, mn[2 * p + 1]);
            const mk_v16i i0 = mk_mma(a.q[2 * p], lo, z), i1 = mk_mma(a.q[2 * p + 1], hi, z);
#pragma unroll
            for (int r = 0; r < 16; r++) isum[r] = __mul24(sc1, i1[r]) + (__mul24(sc0, i0[r]) + isum[r]);
        }
        // weight operand of summ: m of bsums 8 kh .. 8 kh + 7, sub-blocks 4 kh .. 4 kh + 3
        mk_v8h mh;
#pragma unroll
        for (int t = 0; t < 4; t++) mh[2 * t] = mh[2 * t + 1] = (_Float16)(kh ? mn[4 + t] : mn[t]);
        const mk_v16f summ = mk_mma_h(mk_bsums(a.bs), mh);
        const float dw = h2f((uint16_t)((uint32_t)w.hdr.x & 0xffff)), dm = h2f((uint16_t)((uint32_t)w.hdr.x >> 16));
        const mk_v32f zf = {};
        const mk_v32f P = __builtin_amdgcn_mfma_f32_32x32x1f32(a.d, kh ? dm : dw, zf, 0, 0, 0);
#pragma unroll
        for (int r = 0; r < 16; r++) {
            acc[r] = __builtin_fmaf(P[r], (float)isum[r], acc[r]);
            acc[r] = __builtin_fmaf(-P[16 + r], summ[r], acc[r]);
        }
    }
};

// one q6_K superblock: ql [128], qh [64], int8 scales [16], fp16 d in the
// resident planes.  Group (h, j) of 32 elements 128 h + 32 j + e takes
// ql[64 h + 32 (j & 1) + e] (low nibble for j < 2, high for j >= 2) and bits
// 2 j, 2 j + 1 of qh[32 h + e]; its sub-blocks of 16 are 8 h + 2 j and
// 8 h + 2 j + 1 (quants.c:582-622).  Lane half kh holds elements 8 kh .. + 7
// and 16 + 8 kh .. + 7 of every group, activations and weights alike, so
// each sub-block is one v_mfma_i32_32x32x16_i8 on 8 bytes of each operand.
struct Q6KSb {
    static constexpr int T = Q6_K, SEG = 1;
    struct W {
        mk_v4i l0[2], l1[2], hb[2], sc;
        uint16_t d;
    };
    static __device__ __forceinline__ mk_v4i ld_split(const uint8_t *p) {
        const mk_v2i a = *(const mk_v2i *)p, b = *(const mk_v2i *)(p + 16);
        return mk_v4i{a.x, a.y, b.x, b.y};
    }
    static __device__ __forceinline__ void load(W &w, const g4h_tensor &Wt, int64_t row, int s, int kh) {
        const size_t j = (size_t)row * Wt.nb + s;
#pragma unroll
        for (int h = 0; h < 2; h++) {
            const uint8_t *ql = Wt.qs + j * 128 + 64 * h + 8 * kh;
            w.l0[h] = ld_split(ql);
            w.l1[h] = ld_split(ql + 32);
            w.hb[h] = ld_split(Wt.ex + j * 64 + 32 * h + 8 * kh);
        }
        w.sc = mk_ld(Wt.sc + j * 16);
        w.d = ((const uint16_t *)Wt.dd)[j];
    }
    static __device__ __forceinline__ void load_act(MkAct &a, const uint8_t *ab, int kh) {
#pragma unroll
        for (int g = 0; g < 8; g++) a.q[g] = ld_split(ab + 4 + 32 * g + 8 * kh);
        a.bs = mk_ld(ab + 260 + 16 * kh);
        a.d = *(const float *)ab;
    }
    static __device__ __forceinline__ void mul(const W &w, const MkAct &a, int kh, mk_v16f &acc) {
        const mk_v16i z = {};
        auto scb = [&](int s) { return (int)(int8_t)(((uint32_t)w.sc[s >> 2] >> (8 * (s & 3))) & 0xff); };
        mk_v16i isum = {};
#pragma unroll
        for (int h = 0; h < 2; h++) {
#pragma unroll
            for (int j = 0; j < 4; j++) {
                const mk_v4i &L = (j & 1) ? w.l1[h] : w.l0[h];
                mk_v4i q = ((L >> (j >= 2 ? 4 : 0)) & 0x0F0F0F0F) | (((w.hb[h] >> (2 * j)) & 0x03030303) << 4);
                const int s0 = 8 * h + 2 * j;
                const int c0 = scb(s0), c1 = scb(s0 + 1);
                const mk_v4i &x = a.q[4 * h + j];
                // the group's weight operand waits for the previous group's
                // multiply-adds: the compiler would otherwise issue all 16
                // MFMAs first and hold 256 result registers
                asm volatile("" : "+v"(q) : "v"(isum[15]));
                const mk_v16i i0 = mk_mma16(x.xy, q.xy, z), i1 = mk_mma16(x.zw, q.zw, z);
#pragma unroll
                for (int r = 0; r < 16; r++) isum[r] = __mul24(c1, i1[r]) + (__mul24(c0, i0[r]) + isum[r]);
            }
        }
        // weight operand of the correction: sc of bsums (= sub-blocks) 8 kh .. 8 kh + 7
        mk_v8h ch;
#pragma unroll
        for (int t = 0; t < 8; t++) ch[t] = (_Float16)(kh ? scb(8 + t) : scb(t));
        const mk_v16f corr = mk_mma_h(mk_bsums(a.bs), ch);
        // d_a * d in the tiles' layout: one k term of two, the other zero
        const mk_v16f zf = {};
        const mk_v16f P = __builtin_amdgcn_mfma_f32_32x32x2f32(kh ? 0.0f : a.d, h2f(w.d), zf, 0, 0, 0);
#pragma unroll
        for (int r = 0; r < 16; r++) acc[r] = __builtin_fmaf(P[r], (float)(isum[r] - 32 * (int)corr[r]), acc[r]);
    }
};

// One workgroup per (row tile, token tile) of 32 x 32.  Workgroup b runs on
// XCD b % 8: row tiles r with r % 8 == b % 8 go there, the token tiles of a
// row tile consecutively, so they find its weights in that XCD's L2.  The
// grid is padded to whole groups of 8 row tiles; padding workgroups return.
template <class S>
__global__ __launch_bounds__(64 * MMK_NW) void k_mmk(g4h_tensor W, const uint8_t *__restrict__ act, size_t stride, int M,
                                                     float *__restrict__ Y, int ntok) {
    __shared__ float part[MMK_NW][32][33];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int li = lane & 31, kh = lane >> 5;
    const int x = blockIdx.x & 7, l = blockIdx.x >> 3;
    const int64_t rt = (int64_t)(l / ntok) * 8 + x;
    const int m0 = (l % ntok) * 32;
    if (rt * 32 >= W.nrows) return;                                      // uniform over the workgroup
    const int64_t n0 = rt * 32;
    const int64_t row = std::min<int64_t>(n0 + li, W.nrows - 1);
    const uint8_t *arow = act + (size_t)std::min(m0 + li, M - 1) * stride;
    const int nb = (int)W.nb;
    mk_v16f acc = {};
    // the wave's superblocks s = wave, wave + MMK_NW, .. two at a time: both
    // superblocks' operands are loaded before the first multiply, in
    // straight-line code (a register ring carried around the loop was undone
    // by the compiler: its loads sank to their uses, several round trips per
    // superblock)
    // q4_K: a lone last superblock is loaded twice; its second multiply gets the
    // activation scale 0, so its products add +0 to an accumulator that never
    // holds -0 (no branch: the compiler would sink that superblock's loads
    // into it).
    for (int s0 = wave; s0 < nb; s0 += S::SEG * MMK_NW) {               // uniform over the wave
        if constexpr (S::SEG == 2) {
            const bool two = s0 + MMK_NW < nb;
            const int s1 = two ? s0 + MMK_NW : s0;
            typename S::W w0, w1;
            MkAct a0, a1;
            S::load(w0, W, row, s0, kh);
            S::load_act(a0, arow + (size_t)s0 * 292, kh);
            S::load(w1, W, row, s1, kh);
            S::load_act(a1, arow + (size_t)s1 * 292, kh);
            if (!two) a1.d = 0.0f;
            __builtin_amdgcn_sched_barrier(0);
            S::mul(w0, a0, kh, acc);
            __builtin_amdgcn_sched_barrier(0);
            S::mul(w1, a1, kh, acc);
        } else {                                                          // q6_K: two superblocks' operands spill
            typename S::W w0;
            MkAct a0;
            S::load(w0, W, row, s0, kh);
            S::load_act(a0, arow + (size_t)s0 * 292, kh);
            S::mul(w0, a0, kh, acc);
        }
    }
    // C[i][j]: j = lane % 32 (weight row), i = 8 (r / 4) + 4 kh + r % 4 (token)
#pragma unroll
    for (int r = 0; r < 16; r++) part[wave][8 * (r >> 2) + 4 * kh + (r & 3)][li] = acc[r];
    __syncthreads();
#pragma unroll
    for (int h = 0; h < 32 * 32 / (64 * MMK_NW); h++) {
        const int o = threadIdx.x + 64 * MMK_NW * h, i = o >> 5, j = o & 31;
        float v = part[0][i][j];
#pragma unroll
        for (int w = 1; w < MMK_NW; w++) v += part[w][i][j];
        const int m = m0 + i;
        const int64_t n = n0 + j;
        if (m < M && n < W.nrows) Y[(size_t)m * W.nrows + n] = v;
    }
}

bool mmk_capable(int type) { return type == Q4_K || type == Q6_K; }

static void mmk_grid(const g4h_tensor &W, int M, int64_t &grid, int &ntok) {
    ntok = (M + 31) / 32;
    grid = (W.nrows + 255) / 256 * 8 * ntok;
}

hipError_t launch_matmul_mfma_k(const g4h_tensor &W, const uint8_t *act, size_t stride, int M, float *Y, hipStream_t s) {
    if (!mmk_capable(W.type) || M < 1 || !act || !Y || stride % 4 || stride < (size_t)W.nb * 292) return hipErrorInvalidValue;
    int64_t grid;
    int ntok;
    mmk_grid(W, M, grid, ntok);
    if (grid > 0x7fffffff) return hipErrorInvalidValue;
    if (W.type == Q4_K) hipLaunchKernelGGL(k_mmk<Q4KSb>, dim3((unsigned)grid), dim3(64 * MMK_NW), 0, s, W, act, stride, M, Y, ntok);
    else hipLaunchKernelGGL(k_mmk<Q6KSb>, dim3((unsigned)grid), dim3(64 * MMK_NW), 0, s, W, act, stride, M, Y, ntok);
    return hipGetLastError();
}

void mmk_describe(const g4h_tensor &W, int M, char *buf, size_t len) {
    int64_t grid;
    int ntok;
    mmk_grid(W, M, grid, ntok);
    snprintf(buf, len, "k_mmk<%s> grid=%lld block=%d (int8 MFMA, 32x32 tiles, %d waves split the superblocks)",
             W.type == Q4_K ? "q4_K" : "q6_K", (long long)grid, 64 * MMK_NW, MMK_NW);
}

}  // namespace g4
