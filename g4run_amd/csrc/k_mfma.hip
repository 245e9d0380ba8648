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
// registers.  Each output keeps four fp32 partial sums (block residue mod 4)
// added in a fixed order, so a token's result does not depend on the batch
// size or on the tile variant (the x4 contract of g4run.h:148-157 within this
// family).
//
// Activations are first laid out planar (qa [M][nb][32] int8, da [M][nb] fp16)
// so every operand load is an aligned 16-byte load.  Kernels: k_mm_mfma, one
// 32 x 32 tile per workgroup whose blocks are split over 4 waves and added in
// wave order through LDS (fewer tokens: enough waves in flight to stream the
// weights), and k_mm_lds, 64 x 128 tiles staged through LDS in 8-block stages
// shared by 8 waves (many tokens: 1/8 of the operand traffic per output).
#include <cstdio>

#include "formats.h"
#include "kernels.h"
#include "steps.h"

namespace g4 {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));
typedef _Float16 v8h __attribute__((ext_vector_type(8)));
typedef float v16f __attribute__((ext_vector_type(16)));

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

template <int WT, int WM, int WN, int KS, int KB>
__global__ __launch_bounds__(256) void k_mm_mfma(g4h_tensor W, const int8_t *__restrict__ qa,
                                                  const uint16_t *__restrict__ da, int M, float *__restrict__ Y) {
    // Four partial sums per output, one per block residue mod 4, each over its
    // blocks in increasing order, then ((p0 + p1) + p2) + p3: the same fp32
    // arithmetic whether one wave holds all four (KS = 1) or KS waves split them.
    constexpr int NR = 4 / KS;                                  // residues per wave
    static_assert(KB % NR == 0 && 4 % KS == 0, "tile shape");
    __shared__ float red[KS > 1 ? (KS - 1) * 64 * 16 : 1];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int wm = wave % WM, wn = (wave / WM) % WN, ks = wave / (WM * WN);
    const int m0 = (blockIdx.y * WM + wm) * 32, n0 = (blockIdx.x * WN + wn) * 32;
    const int li = lane & 31, kh = lane >> 5;
    const int nb = (int)W.nb;
    const int tok = min(m0 + li, M - 1);
    const int64_t row = min((int64_t)(n0 + li), W.nrows - 1);
    const int8_t *pa = qa + (size_t)tok * nb * 32 + 16 * kh;
    const uint16_t *pda = da + (size_t)tok * nb;
    const uint8_t *pw = WT == Q8_0 ? W.qs + (size_t)row * nb * 32 + 16 * kh : W.qs + (size_t)row * nb * 16;
    const uint16_t *pdw = (const uint16_t *)W.sc + (size_t)row * nb;

    v16f acc[NR];
#pragma unroll
    for (int q = 0; q < NR; q++)
#pragma unroll
        for (int r = 0; r < 16; r++) acc[q][r] = 0.0f;
    const v16i zi = {};
    const v16f zf = {};
    // operands of KB blocks; two sets alternate so the next set's loads are in
    // flight while the current one is multiplied
    struct Ops {
        v4i a[KB], w[KB];
        uint16_t sa[KB], sw[KB];
    };
    auto load = [&](Ops &o, int b0) {
#pragma unroll
        for (int k = 0; k < KB; k++) {
            const int b = min(b0 + k * KS, nb - 1);
            o.a[k] = *(const v4i *)(pa + (size_t)b * 32);
            o.w[k] = *(const v4i *)(pw + (size_t)b * (WT == Q8_0 ? 32 : 16));
            o.sa[k] = pda[b];
            o.sw[k] = pdw[b];
        }
    };
    // wave ks takes blocks ks, ks + KS, ...; block b0 + k*KS has residue (ks + k*KS) % 4
    auto mul = [&](const Ops &o, int b0) {
#pragma unroll
        for (int k = 0; k < KB; k++) {
            if (b0 + k * KS < nb) {                                  // uniform
                const v4i wv = WT == Q8_0 ? o.w[k] : q4_half(o.w[k], kh);
                const v16i is = __builtin_amdgcn_mfma_i32_32x32x32_i8(o.a[k], wv, zi, 0, 0, 0);
                v8h ha = {}, hw = {};
                if (kh == 0) {
                    ha[0] = __builtin_bit_cast(_Float16, o.sa[k]);
                    hw[0] = __builtin_bit_cast(_Float16, o.sw[k]);
                }
                const v16f sc = __builtin_amdgcn_mfma_f32_32x32x16_f16(ha, hw, zf, 0, 0, 0);
                v16f &p = acc[k % NR];
#pragma unroll
                for (int r = 0; r < 16; r++) p[r] = __builtin_fmaf((float)is[r], sc[r], p[r]);
            }
        }
    };
    constexpr int STEP = KS * KB;
    Ops o0, o1;
    load(o0, ks);
    for (int b0 = ks;;) {
        if (b0 + STEP < nb) load(o1, b0 + STEP);
        mul(o0, b0);
        b0 += STEP;
        if (b0 >= nb) break;
        if (b0 + STEP < nb) load(o0, b0 + STEP);
        mul(o1, b0);
        b0 += STEP;
        if (b0 >= nb) break;
    }
    v16f out = acc[0];
    if constexpr (KS == 1) {
#pragma unroll
        for (int q = 1; q < 4; q++)
#pragma unroll
            for (int r = 0; r < 16; r++) out[r] += acc[q][r];
    } else {
        // partials of waves 1..KS-1 through LDS, added to wave 0's in wave order
        static_assert(KS == 4, "KS is 1 or 4");
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
    }
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

// LDS-staged tiles for many tokens.  A workgroup of TM x TN waves owns a
// (32 TM) token x (32 TN) row output tile; wave (im, in) its 32 x 32 subtile.
// The K loop runs over stages of KB blocks: every thread loads a share of the
// stage's activation and weight bytes (and fp16 scales) into registers while
// the waves multiply the previous stage from LDS, then writes them to the other
// LDS buffer.  Per block and subtile the arithmetic is that of k_mm_mfma: one
// int8 MFMA for the exact block sums, one f16 MFMA for the scale outer product,
// an fma into the accumulator of the block's residue mod 4, and at the end
// ((p0 + p1) + p2) + p3 -- so every output is bit-identical to k_mm_mfma's.
constexpr int MML_KB = 8;                                           // blocks per stage

template <int WT, int TM, int TN, int KB>
__global__ __launch_bounds__(64 * TM * TN) void k_mm_lds(g4h_tensor W, const int8_t *__restrict__ qa,
                                                         const uint16_t *__restrict__ da, int M, float *__restrict__ Y) {
    constexpr int BM = 32 * TM, BN = 32 * TN, NT = 64 * TM * TN;
    constexpr int WB = WT == Q8_0 ? 32 : 16;                        // weight bytes per block
    constexpr int AS = KB * 32 + 16, BS = KB * WB + 16;             // padded LDS row strides (bytes)
    constexpr int AC = BM * KB * 2, BC = BN * KB * WB / 16;         // 16-byte chunks per stage
    constexpr int APT = (AC + NT - 1) / NT, BPT = (BC + NT - 1) / NT;
    __shared__ __align__(16) int8_t As[2][BM * AS];
    __shared__ __align__(16) uint8_t Bs[2][BN * BS];
    __shared__ __align__(16) uint16_t Ad[2][BM * KB], Bd[2][BN * KB];
    const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
    const int im = wave % TM, in = wave / TM;
    const int li = lane & 31, kh = lane >> 5;
    const int nb = (int)W.nb, nst = (nb + KB - 1) / KB;
    const int m0 = blockIdx.y * BM;
    const int64_t n0 = (int64_t)blockIdx.x * BN;

    struct Stage {
        v4i a[APT], b[BPT];
        uint16_t sa[KB], sb[KB];                                    // kept as loaded: no wait at load time
    };
    // chunk c of the A stage: token row c / (2 KB), 16 bytes (c % (2 KB)) of its KB blocks
    auto load = [&](Stage &S, int s) {
#pragma unroll
        for (int i = 0; i < APT; i++) {
            const int c = min(t + i * NT, AC - 1), r = c / (2 * KB), q = c % (2 * KB);
            const int m = min(m0 + r, M - 1), b = min(s * KB + q / 2, nb - 1);
            S.a[i] = *(const v4i *)(qa + ((size_t)m * nb + b) * 32 + 16 * (q & 1));
        }
#pragma unroll
        for (int i = 0; i < BPT; i++) {
            const int c = min(t + i * NT, BC - 1), r = c / (KB * WB / 16), q = c % (KB * WB / 16);
            const int64_t n = min(n0 + r, W.nrows - 1);
            const int b = min(s * KB + q * 16 / WB, nb - 1);
            S.b[i] = *(const v4i *)(W.qs + ((size_t)n * nb + b) * WB + (WT == Q8_0 ? 16 * (q & 1) : 0));
        }
        // scales: thread r < BM loads token r's KB fp16 scales, r < BN row r's
        const int ra = min(t, BM - 1), rb = min(t, BN - 1);
        const int ma = min(m0 + ra, M - 1);
        const int64_t nr = min(n0 + rb, W.nrows - 1);
#pragma unroll
        for (int k = 0; k < KB; k++) {
            const int b = min(s * KB + k, nb - 1);
            S.sa[k] = da[(size_t)ma * nb + b];
            S.sb[k] = ((const uint16_t *)W.sc)[(size_t)nr * nb + b];
        }
    };
    auto store = [&](const Stage &S, int buf) {
#pragma unroll
        for (int i = 0; i < APT; i++) {
            const int c = t + i * NT;
            if (c < AC) *(v4i *)&As[buf][(c / (2 * KB)) * AS + 16 * (c % (2 * KB))] = S.a[i];
        }
#pragma unroll
        for (int i = 0; i < BPT; i++) {
            const int c = t + i * NT;
            if (c < BC) *(v4i *)&Bs[buf][(c / (KB * WB / 16)) * BS + 16 * (c % (KB * WB / 16))] = S.b[i];
        }
        if (t < BM) {
#pragma unroll
            for (int k = 0; k < KB; k++) Ad[buf][t * KB + k] = S.sa[k];
        }
        if (t < BN) {
#pragma unroll
            for (int k = 0; k < KB; k++) Bd[buf][t * KB + k] = S.sb[k];
        }
    };

    v16f acc[4];
#pragma unroll
    for (int q = 0; q < 4; q++)
#pragma unroll
        for (int r = 0; r < 16; r++) acc[q][r] = 0.0f;
    const v16i zi = {};
    const v16f zf = {};
    // one block's two MFMAs (exact integer sums; the scale outer product)
    auto mfmas = [&](int cur, int k, v16i &is, v16f &sc) {
        const int8_t *arow = &As[cur][(32 * im + li) * AS + 16 * kh];
        const uint8_t *brow = &Bs[cur][(32 * in + li) * BS + (WT == Q8_0 ? 16 * kh : 0)];
        const v4i av = *(const v4i *)(arow + 32 * k);
        const v4i wraw = *(const v4i *)(brow + WB * k);
        const v4i wv = WT == Q8_0 ? wraw : q4_half(wraw, kh);
        is = __builtin_amdgcn_mfma_i32_32x32x32_i8(av, wv, zi, 0, 0, 0);
        v8h ha = {}, hw = {};
        if (kh == 0) {
            ha[0] = __builtin_bit_cast(_Float16, Ad[cur][(32 * im + li) * KB + k]);
            hw[0] = __builtin_bit_cast(_Float16, Bd[cur][(32 * in + li) * KB + k]);
        }
        sc = __builtin_amdgcn_mfma_f32_32x32x16_f16(ha, hw, zf, 0, 0, 0);
    };
    auto epi = [&](int b, const v16i &is, const v16f &sc) {
        v16f &p = acc[b & 3];
#pragma unroll
        for (int r = 0; r < 16; r++) p[r] = __builtin_fmaf((float)is[r], sc[r], p[r]);
    };
    // software-pipelined over the stage's blocks: block k + 1's MFMAs are
    // issued before block k's epilogue, so the VALU work of one block runs
    // while the matrix cores work on the next
    auto compute = [&](int s) {
        const int cur = s & 1;
        const int kn = min(KB, nb - s * KB);                         // blocks in this stage (uniform)
        v16i is0, is1;
        v16f sc0, sc1;
        mfmas(cur, 0, is0, sc0);
#pragma unroll
        for (int k = 0; k < KB; k += 2) {
            if (k + 1 < kn) mfmas(cur, k + 1, is1, sc1);
            if (k < kn) epi(s * KB + k, is0, sc0);
            if (k + 2 < kn) mfmas(cur, k + 2, is0, sc0);
            if (k + 1 < kn) epi(s * KB + k + 1, is1, sc1);
        }
    };
    // two stages of loads in flight: while stage s is multiplied from LDS, the
    // registers hold stage s + 1 (loaded one stage earlier, stored to LDS after
    // the multiply) and receive stage s + 2
    Stage S0, S1;
    load(S0, 0);
    if (nst > 1) load(S1, 1);
    store(S0, 0);
    __syncthreads();
    for (int s = 0; s < nst; s += 2) {
        if (s + 2 < nst) load(S0, s + 2);
        compute(s);
        if (s + 1 < nst) store(S1, 1);
        __syncthreads();
        if (s + 1 >= nst) break;
        if (s + 3 < nst) load(S1, s + 3);
        compute(s + 1);
        if (s + 2 < nst) store(S0, 0);
        __syncthreads();
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

// x fp32 [M][ncols] (row stride xs floats) -> planar q8_0 with the quantizer
// arithmetic of quants.c:74-109 (8 lanes per block).
__global__ __launch_bounds__(256) void k_quantize_planar(const float *__restrict__ x, size_t xs, int64_t ncols, int M,
                                                         int8_t *__restrict__ qa, uint16_t *__restrict__ da) {
    const int64_t ng = ncols / 4;
    const int64_t gi = (int64_t)blockIdx.x * 256 + threadIdx.x;
    const int m = blockIdx.y;
    const bool own = gi < ng;
    float v[4] = {0.f, 0.f, 0.f, 0.f};
    if (own) f4(ldf4(x + (size_t)m * xs + 4 * gi), v);
    float am = fmaxf(fmaxf(fabsf(v[0]), fabsf(v[1])), fmaxf(fabsf(v[2]), fabsf(v[3])));
    am = group_max<8>(am);
    if (!own) return;
    const float id = am != 0.0f ? 127.0f / am : 0.0f;
    uint32_t pk = 0;
#pragma unroll
    for (int j = 0; j < 4; j++) pk |= ((uint32_t)(int)__builtin_rintf(v[j] * id) & 0xffu) << (8 * j);
    const int64_t nb = ncols / 32;
    *(uint32_t *)(qa + ((size_t)m * nb) * 32 + 4 * gi) = pk;
    if ((gi & 7) == 0) da[(size_t)m * nb + gi / 8] = f2h(am * (1.0f / 127.0f));
}

// GGUF q8_0 activation rows (stride bytes) -> planar
__global__ __launch_bounds__(256) void k_act_planar(const uint8_t *__restrict__ act, size_t stride, int64_t nb, int M,
                                                    int8_t *__restrict__ qa, uint16_t *__restrict__ da) {
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;    // (token, block, quarter)
    if (i >= (int64_t)M * nb * 4) return;
    const int64_t m = i / (nb * 4), r = i - m * nb * 4, b = r >> 2, q = r & 3;
    const uint8_t *blk = act + (size_t)m * stride + (size_t)b * 34;
    uint32_t w[2];
#pragma unroll
    for (int k = 0; k < 2; k++) {
        const uint8_t *p = blk + 2 + 8 * q + 4 * k;
        w[k] = (uint32_t)p[0] | ((uint32_t)p[1] << 8) | ((uint32_t)p[2] << 16) | ((uint32_t)p[3] << 24);
    }
    *(uint2 *)(qa + ((size_t)m * nb + b) * 32 + 8 * q) = make_uint2(w[0], w[1]);
    if (q == 0) da[(size_t)m * nb + b] = (uint16_t)(blk[0] | (blk[1] << 8));
}

size_t mm_planar_bytes(int M, int64_t ncols) {
    const int64_t nb = ncols / 32;
    return (((size_t)M * nb * 32 + 255) & ~(size_t)255) + (size_t)M * nb * 2;
}

// One 32 x 32 tile per workgroup with the blocks split over 4 waves while
// that gives at most 3 workgroups per CU, LDS-staged 64 x 128 tiles beyond.
// Measured on q8_0 4096 x 4096: 128 tokens 39 us split / 58 us staged, 256
// tokens 68 / 58 us, 512 tokens 128 / 61 us (the staged kernel runs at about
// the same time for any token count: its per-workgroup latency, not the
// memory system, bounds it).
static bool mm_small(const g4h_tensor &W, int M) {
    const int64_t tiles = ((W.nrows + 31) / 32) * ((M + 31) / 32);
    return tiles <= 3 * 256;
}

void mm_describe(const g4h_tensor &W, int M, char *buf, size_t len) {
    if (mm_small(W, M)) {
        snprintf(buf, len, "k_mm_mfma<%s,wm=1,wn=1,ks=4,kb=%d> grid=%lldx%d block=256", W.type == Q8_0 ? "q8_0" : "q4_0",
                 MM_KB_SMALL, (long long)((W.nrows + 31) / 32), (M + 31) / 32);
        return;
    }
    snprintf(buf, len, "k_mm_lds<%s,tm=2,tn=4,kb=%d> grid=%lldx%d block=512", W.type == Q8_0 ? "q8_0" : "q4_0", MML_KB,
             (long long)((W.nrows + 127) / 128), (M + 63) / 64);
}

template <int WT, int WM, int WN, int KS, int KB>
static hipError_t mm_go(const g4h_tensor &W, const int8_t *qa, const uint16_t *da, int M, float *Y, hipStream_t s) {
    const dim3 grid((unsigned)((W.nrows + 32 * WN - 1) / (32 * WN)), (unsigned)((M + 32 * WM - 1) / (32 * WM)));
    hipLaunchKernelGGL((k_mm_mfma<WT, WM, WN, KS, KB>), grid, dim3(64 * WM * WN * KS), 0, s, W, qa, da, M, Y);
    return hipGetLastError();
}

// Y[M][nrows] = W * act^T on the matrix cores.  `act` is GGUF q8_0 rows at
// `stride` (x == nullptr) or x fp32 rows (x_stride floats); `ws` holds the
// planar activations (mm_planar_bytes).
hipError_t launch_matmul_mfma(const g4h_tensor &W, const float *x, size_t x_stride, const uint8_t *act, size_t stride, int M,
                              float *Y, uint8_t *ws, hipStream_t s) {
    if ((W.type != Q8_0 && W.type != Q4_0) || M <= 0 || W.ncols % 32) return hipErrorInvalidValue;
    const int64_t nb = W.nb;
    int8_t *qa = (int8_t *)ws;
    uint16_t *da = (uint16_t *)(ws + (((size_t)M * nb * 32 + 255) & ~(size_t)255));
    if (x) {
        hipLaunchKernelGGL(k_quantize_planar, dim3((unsigned)((W.ncols / 4 + 255) / 256), M), dim3(256), 0, s, x, x_stride,
                           W.ncols, M, qa, da);
    } else {
        const int64_t n = (int64_t)M * nb * 4;
        hipLaunchKernelGGL(k_act_planar, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, act, stride, nb, M, qa, da);
    }
    if (hipError_t e = hipGetLastError()) return e;
    const bool small = mm_small(W, M);
    if (small) {
        if (W.type == Q8_0) return mm_go<Q8_0, 1, 1, 4, MM_KB_SMALL>(W, qa, da, M, Y, s);
        return mm_go<Q4_0, 1, 1, 4, MM_KB_SMALL>(W, qa, da, M, Y, s);
    }
    const dim3 grid((unsigned)((W.nrows + 127) / 128), (unsigned)((M + 63) / 64));
    if (W.type == Q8_0) hipLaunchKernelGGL((k_mm_lds<Q8_0, 2, 4, MML_KB>), grid, dim3(512), 0, s, W, qa, da, M, Y);
    else hipLaunchKernelGGL((k_mm_lds<Q4_0, 2, 4, MML_KB>), grid, dim3(512), 0, s, W, qa, da, M, Y);
    return hipGetLastError();
    return hipGetLastError();
}

}  // namespace g4
