// k_attn.hip -- decode attention over an f16 or q8_0 KV cache (the GPU form of
// attn_kernel + kv_store, model.c:509-589), as a split-K pass over positions.
//
// Cache layout: [slot][n_kv][hd] rows (one row = one head's K or V for one
// position), f16 or q8_0 blocks.  Query heads map to KV heads h / (n_head/n_kv)
// (model.c:1099).  Numerics follow the reference step by step:
//   1. scores: q rounded to the K cache's activation form (fp16, or q8_0
//      blocks) and dotted with each cached K row in the shipped dot's order --
//      eight fp32 lanes of fused products and the same horizontal-sum tree
//      (quants.c:1319-1331 / 984-999) -- one GPU lane per position, so the
//      scores are bit-identical to the CPU's; no 1/sqrt(d) factor (model.c:538);
//   2. softmax: global max, e_j = expf(s_j - max) (computed as exp in double
//      rounded to float), sum in double, inv = (float)(1/sum) (model.c:547-549);
//   3. weights: fp16(e_j * inv) for an f16 V cache, e_j * inv for q8_0
//      (model.c:555, 573);
//   4. o = sum_j w_j V_j in fp32, as chunk partials added in a fixed order
//      (the only step whose rounding differs from the CPU's sequential loop).
#include <type_traits>

#include "formats.h"
#include "kernels.h"
#include "steps.h"

namespace g4 {

constexpr int ATT_CHUNK = 128;       // positions per score / V workgroup (one chunk maximum, one partial)
constexpr int ATT_SCHUNK = 256;      // positions per softmax workgroup

__device__ __forceinline__ int npos_of(int npos, const int *npos_dev) { return npos_dev ? *npos_dev : npos; }

__device__ __forceinline__ float wave_max(float v) {
    for (int k = 32; k >= 1; k >>= 1) v = fmaxf(v, shfl_xor(v, k));
    return v;
}
__device__ __forceinline__ double wave_sum_d(double v) {
    for (int k = 32; k >= 1; k >>= 1) v += __shfl_xor(v, k, 64);
    return v;
}

// Chunk maximum over the workgroup's positions: per wave, then the waves in
// LDS; the first GRP threads store Mc[h][c].
template <int GRP, int NW>
__device__ __forceinline__ void store_chunk_max(const float (&m)[GRP], float (*wm)[GRP], float *Mc, int h0, int nchunk_max, int c) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
#pragma unroll
    for (int g = 0; g < GRP; g++) {
        const float w = wave_max(m[g]);
        if (lane == 0) wm[wave][g] = w;
    }
    __syncthreads();
    if (threadIdx.x < GRP) {
        float r = wm[0][threadIdx.x];
        for (int w = 1; w < NW; w++) r = fmaxf(r, wm[w][threadIdx.x]);
        Mc[(size_t)(h0 + threadIdx.x) * nchunk_max + c] = r;
    }
}

// ---------------------------------------------------------------- scores --
// f16 cache.  grid (n_kv, chunks), 256 threads; a lane pair per position (32
// per wave): the even lane keeps the four fp32 accumulators of elements
// 8k..8k+3, the odd lane those of 8k+4..8k+7, i.e. the eight lanes of the
// shipped dot split in two; the horizontal sum then combines the pair with the
// same tree.  Every K load of the lane (hd/8 of 8 B) is issued before any use.
template <int GRP>
__global__ __launch_bounds__(256) void k_attn_scores_f16(const float *__restrict__ q, const uint8_t *__restrict__ kc, int n_kv,
                                                         int hd, int npos_arg, const int *npos_dev, float *__restrict__ S,
                                                         float *__restrict__ Mc, int nchunk_max) {
    __shared__ __align__(16) float4 qf[GRP][64];             // fp16-rounded query
    __shared__ float wm[4][GRP];
    const int npos = npos_of(npos_arg, npos_dev);
    const int kvh = blockIdx.x, c = blockIdx.y, t = threadIdx.x;
    const int lane = t & 63, wave = t >> 6, hf = lane & 1;
    const int h0 = kvh * GRP;
    if (c * ATT_CHUNK >= npos) {
        if (t < GRP) Mc[(size_t)(h0 + t) * nchunk_max + c] = -INFINITY;
        return;
    }
    const int j = c * ATT_CHUNK + wave * 32 + (lane >> 1);
    const bool ok = j < npos;
    // query loads first (global loads complete in issue order), then every K load
    constexpr int QPT = (GRP * 256 + 255) / 256;             // query elements per thread (hd <= 256)
    float qv[QPT];
#pragma unroll
    for (int k = 0; k < QPT; k++) {
        const int i = t + 256 * k;
        qv[k] = i < GRP * hd ? q[(size_t)h0 * hd + i] : 0.0f;
    }
    const uint2 *row = (const uint2 *)(kc + ((size_t)(ok ? j : npos - 1) * n_kv + kvh) * hd * 2) + hf;
    const int nk = hd >> 3;
    uint2 kv[32];
#pragma unroll
    for (int k = 0; k < 32; k++)
        if (k < nk) kv[k] = row[2 * k];
#pragma unroll
    for (int k = 0; k < QPT; k++) {
        const int i = t + 256 * k;
        if (i < GRP * hd) {
            const int g = i / hd, e = i - g * hd;
            ((float *)qf[g])[e] = h2f(f2h(qv[k]));
        }
    }
    __syncthreads();
    float acc[GRP][4];
#pragma unroll
    for (int g = 0; g < GRP; g++)
#pragma unroll
        for (int i = 0; i < 4; i++) acc[g][i] = 0.0f;
#pragma unroll
    for (int k = 0; k < 32; k++) {
        if (k < nk) {
            const float kf[4] = {h2f((uint16_t)(kv[k].x & 0xffff)), h2f((uint16_t)(kv[k].x >> 16)),
                                 h2f((uint16_t)(kv[k].y & 0xffff)), h2f((uint16_t)(kv[k].y >> 16))};
#pragma unroll
            for (int g = 0; g < GRP; g++) {
                const float4 qv = qf[g][2 * k + hf];
                acc[g][0] = __builtin_fmaf(kf[0], qv.x, acc[g][0]);
                acc[g][1] = __builtin_fmaf(kf[1], qv.y, acc[g][1]);
                acc[g][2] = __builtin_fmaf(kf[2], qv.z, acc[g][2]);
                acc[g][3] = __builtin_fmaf(kf[3], qv.w, acc[g][3]);
            }
        }
    }
    float m[GRP];
#pragma unroll
    for (int g = 0; g < GRP; g++) {
        // lane l of the eight is acc[l & 3] of the pair member l >> 2; r_i = v[i+4] + v[i]
        float r[4];
#pragma unroll
        for (int i = 0; i < 4; i++) r[i] = acc[g][i] + shfl_xor(acc[g][i], 1);
        const float sc = (r[0] + r[2]) + (r[1] + r[3]);
        if (ok && hf == 0) S[(size_t)(h0 + g) * npos + j] = sc;
        m[g] = ok ? sc : -INFINITY;
    }
    store_chunk_max<GRP, 4>(m, wm, Mc, h0, nchunk_max, c);
}

// q8_0 cache.  grid (n_kv, chunks), 128 threads, one lane per position; the
// query is q8_0-quantized per block (model.c:533) and each block pair of the
// row is dotted in the AVX2 order of quants.c:984-999.
template <int GRP>
__global__ __launch_bounds__(128) void k_attn_scores_q8(const float *__restrict__ q, const uint8_t *__restrict__ kc, int n_kv,
                                                        int hd, int npos_arg, const int *npos_dev, float *__restrict__ S,
                                                        float *__restrict__ Mc, int nchunk_max) {
    __shared__ __align__(16) int4 qq[GRP][8][2];
    __shared__ float qd[GRP][8];
    __shared__ float wm[2][GRP];
    const int npos = npos_of(npos_arg, npos_dev);
    const int kvh = blockIdx.x, c = blockIdx.y, t = threadIdx.x;
    const int h0 = kvh * GRP;
    if (c * ATT_CHUNK >= npos) {
        if (t < GRP) Mc[(size_t)(h0 + t) * nchunk_max + c] = -INFINITY;
        return;
    }
    for (int i = t; i < GRP * hd / 4; i += 128) {          // 8 lanes per block; hd/4 is a multiple of 8
        const int g = i / (hd / 4), e4 = i - g * (hd / 4);
        const float *src = q + (size_t)(h0 + g) * hd + 4 * e4;
        float v[4] = {src[0], src[1], src[2], src[3]};
        float am = fmaxf(fmaxf(fabsf(v[0]), fabsf(v[1])), fmaxf(fabsf(v[2]), fabsf(v[3])));
        am = fmaxf(am, shfl_xor(am, 1)); am = fmaxf(am, shfl_xor(am, 2)); am = fmaxf(am, shfl_xor(am, 4));
        const float id = am != 0.0f ? 127.0f / am : 0.0f;
        uint32_t pk = 0;
        for (int k = 0; k < 4; k++) pk |= ((uint32_t)(int)__builtin_rintf(v[k] * id) & 0xffu) << (8 * k);
        const int b = e4 >> 3, w = e4 & 7;
        ((uint32_t *)&qq[g][b][0])[w] = pk;
        if (w == 0) qd[g][b] = h2f(f2h(am * (1.0f / 127.0f)));
    }
    __syncthreads();
    const int j = c * ATT_CHUNK + t;
    const bool ok = j < npos;
    const uint8_t *row = kc + ((size_t)(ok ? j : npos - 1) * n_kv + kvh) * (hd / 32) * 34;
    float acc[GRP][8];
#pragma unroll
    for (int g = 0; g < GRP; g++)
#pragma unroll
        for (int l = 0; l < 8; l++) acc[g][l] = 0.0f;
    for (int b = 0; b < hd / 32; b += 2) {
        uint32_t v[17];
        const uint32_t *src = (const uint32_t *)(row + (size_t)b * 34);
#pragma unroll
        for (int k = 0; k < 17; k++) v[k] = src[k];
        uint32_t w0[8], w1[8];
#pragma unroll
        for (int k = 0; k < 8; k++) { w0[k] = __builtin_amdgcn_alignbyte(v[k + 1], v[k], 2); w1[k] = v[9 + k]; }
        const float d0 = h2f((uint16_t)(v[0] & 0xffff)), d1 = h2f((uint16_t)(v[8] >> 16));
#pragma unroll
        for (int g = 0; g < GRP; g++) {
            const int4 a0 = qq[g][b][0], a1 = qq[g][b][1], c0 = qq[g][b + 1][0], c1 = qq[g][b + 1][1];
            const int aw[8] = {a0.x, a0.y, a0.z, a0.w, a1.x, a1.y, a1.z, a1.w};
            const int cw[8] = {c0.x, c0.y, c0.z, c0.w, c1.x, c1.y, c1.z, c1.w};
            const float da = d0 * qd[g][b], db = d1 * qd[g][b + 1];
#pragma unroll
            for (int l = 0; l < 8; l++) acc[g][l] = __builtin_fmaf(da, (float)dot4(w0[l], aw[l], 0), acc[g][l]);
#pragma unroll
            for (int l = 0; l < 8; l++) acc[g][l] = __builtin_fmaf(db, (float)dot4(w1[l], cw[l], 0), acc[g][l]);
        }
    }
    float m[GRP];
#pragma unroll
    for (int g = 0; g < GRP; g++) {
        const float *a = acc[g];
        const float r0 = a[4] + a[0], r1 = a[5] + a[1], r2 = a[6] + a[2], r3 = a[7] + a[3];
        const float sc = (r0 + r2) + (r1 + r3);
        if (ok) S[(size_t)(h0 + g) * npos + j] = sc;
        m[g] = ok ? sc : -INFINITY;
    }
    store_chunk_max<GRP, 2>(m, wm, Mc, h0, nchunk_max, c);
}

// --------------------------------------------------------------- softmax --
// grid (n_head, chunks of 256 positions): global max over the chunk maxima,
// e_j = (float)exp(s_j - max) written in place, and the chunk's double sum
// Ps[h][c] (wave butterflies, then the four waves in order).
__global__ __launch_bounds__(256) void k_attn_softmax(float *__restrict__ S, const float *__restrict__ Mc, int nchunk_max,
                                                      double *__restrict__ Ps, int nschunk_max, int npos_arg, const int *npos_dev) {
    __shared__ float wm[4];
    __shared__ double ws[4];
    const int npos = npos_of(npos_arg, npos_dev);
    const int h = blockIdx.x, c = blockIdx.y, t = threadIdx.x, lane = t & 63, wave = t >> 6;
    if (c * ATT_SCHUNK >= npos) return;
    const int j = c * ATT_SCHUNK + t;
    float *sp = S + (size_t)h * npos + j;
    const float sv = j < npos ? *sp : 0.0f;
    const int nchunk = (npos + ATT_CHUNK - 1) / ATT_CHUNK;
    float m = -INFINITY;
    for (int i = t; i < nchunk; i += 256) m = fmaxf(m, Mc[(size_t)h * nchunk_max + i]);
    m = wave_max(m);
    if (lane == 0) wm[wave] = m;
    __syncthreads();
    const float mx = fmaxf(fmaxf(wm[0], wm[1]), fmaxf(wm[2], wm[3]));
    double e = 0.0;
    if (j < npos) {
        const float ef = (float)exp((double)(sv - mx));
        *sp = ef;
        e = ef;
    }
    e = wave_sum_d(e);
    if (lane == 0) ws[wave] = e;
    __syncthreads();
    if (t == 0) Ps[(size_t)h * nschunk_max + c] = ((ws[0] + ws[1]) + ws[2]) + ws[3];
}

// ------------------------------------------------------------ V partials --
// grid (n_kv, chunks of 128), 256 threads.  inv = (float)(1 / sum of the chunk
// sums); the chunk's weights w_j = fp16(e_j*inv) (f16 cache) or e_j*inv (q8_0)
// go to LDS once; each wave then accumulates w_j * V_j over its 32 positions
// (all V loads of the lane issued up front), lane owning 4 consecutive
// elements; the waves add in order into the partial P[h][c][hd].
template <int KV, int GRP>
__global__ __launch_bounds__(256) void k_attn_v(const float *__restrict__ E, const double *__restrict__ Ps, int nschunk_max,
                                                const uint8_t *__restrict__ vc, int n_kv, int hd, int npos_arg,
                                                const int *npos_dev, float *__restrict__ P, int nvchunk_max) {
    __shared__ float part[4][GRP][256];
    __shared__ float wl[GRP][ATT_CHUNK];
    __shared__ float inv_s[GRP];
    const int npos = npos_of(npos_arg, npos_dev);
    const int kvh = blockIdx.x, c = blockIdx.y, t = threadIdx.x, lane = t & 63, wave = t >> 6;
    const int h0 = kvh * GRP;
    if (c * ATT_CHUNK >= npos) return;
    const int j0 = c * ATT_CHUNK + wave * 32;
    const int ns = (npos + ATT_SCHUNK - 1) / ATT_SCHUNK;
    // 1. the small loads: chunk sums (wave w reduces heads w, w+4), e_j of the chunk
    constexpr int HPW = (GRP + 3) / 4;                         // heads per wave
    double ps[HPW];
#pragma unroll
    for (int q = 0; q < HPW; q++) {
        const int g = wave + 4 * q;
        ps[q] = g < GRP && lane < ns ? Ps[(size_t)(h0 + g) * nschunk_max + lane] : 0.0;
    }
    constexpr int EPT = (GRP * ATT_CHUNK + 255) / 256;        // weights per thread
    float ev[EPT];
#pragma unroll
    for (int k = 0; k < EPT; k++) {
        const int i = t + 256 * k, g = i / ATT_CHUNK, jw = c * ATT_CHUNK + (i - g * ATT_CHUNK);
        ev[k] = i < GRP * ATT_CHUNK && jw < npos ? E[(size_t)(h0 + g) * npos + jw] : 0.0f;
    }
    // 2. the V rows: lane owns elements 4*lane .. 4*lane+3 (lanes beyond hd/4 idle)
    const bool lane_ok = 4 * lane < hd;
    uint2 vv[32];
    if constexpr (KV == F16) {
#pragma unroll
        for (int k = 0; k < 32; k++) {
            const int j = min(j0 + k, npos - 1);
            if (lane_ok) vv[k] = *((const uint2 *)(vc + ((size_t)j * n_kv + kvh) * hd * 2) + lane);
        }
    }
    // 3. inv = (float)(1 / sum of the chunk sums), chunks beyond 64 added in further passes
#pragma unroll
    for (int q = 0; q < HPW; q++) {
        const int g = wave + 4 * q;
        if (g < GRP) {                                         // uniform over the wave
            double sum = wave_sum_d(ps[q]);
            for (int c0 = 64; c0 < ns; c0 += 64)
                sum += wave_sum_d(c0 + lane < ns ? Ps[(size_t)(h0 + g) * nschunk_max + c0 + lane] : 0.0);
            if (lane == 0) inv_s[g] = (float)(1.0 / sum);
        }
    }
    __syncthreads();
#pragma unroll
    for (int k = 0; k < EPT; k++) {
        const int i = t + 256 * k;
        if (i < GRP * ATT_CHUNK) {
            const int g = i / ATT_CHUNK, p = i - g * ATT_CHUNK;
            const float w = ev[k] * inv_s[g];
            wl[g][p] = KV == F16 ? h2f(f2h(w)) : w;
        }
    }
    __syncthreads();
    float o[GRP][4];
#pragma unroll
    for (int g = 0; g < GRP; g++)
#pragma unroll
        for (int e = 0; e < 4; e++) o[g][e] = 0.0f;
    if constexpr (KV == F16) {
#pragma unroll
        for (int k = 0; k < 32; k++) {
            if (j0 + k < npos) {
                const float v[4] = {h2f((uint16_t)(vv[k].x & 0xffff)), h2f((uint16_t)(vv[k].x >> 16)),
                                    h2f((uint16_t)(vv[k].y & 0xffff)), h2f((uint16_t)(vv[k].y >> 16))};
#pragma unroll
                for (int g = 0; g < GRP; g++) {
                    const float w = wl[g][wave * 32 + k];
#pragma unroll
                    for (int e = 0; e < 4; e++) o[g][e] = __builtin_fmaf(w, v[e], o[g][e]);
                }
            }
        }
    } else {
        for (int k = 0; k < 32; k++) {
            const int j = j0 + k;
            if (j >= npos) break;
            if (lane_ok) {
                const uint8_t *blk = vc + ((size_t)j * n_kv + kvh) * (hd / 32) * 34 + (lane >> 3) * 34;
                const float d = h2f((uint16_t)(blk[0] | (blk[1] << 8)));
                float v[4];
#pragma unroll
                for (int e = 0; e < 4; e++) v[e] = (float)(int8_t)blk[2 + 4 * (lane & 7) + e] * d;
#pragma unroll
                for (int g = 0; g < GRP; g++) {
                    const float w = wl[g][wave * 32 + k];
#pragma unroll
                    for (int e = 0; e < 4; e++) o[g][e] = __builtin_fmaf(w, v[e], o[g][e]);
                }
            }
        }
    }
    if (lane_ok) {
#pragma unroll
        for (int g = 0; g < GRP; g++)
            *(float4 *)&part[wave][g][4 * lane] = make_float4(o[g][0], o[g][1], o[g][2], o[g][3]);
    }
    __syncthreads();
    for (int i = t; i < GRP * hd; i += 256) {
        const int g = i / hd, e = i - g * hd;
        const float r = ((part[0][g][e] + part[1][g][e]) + part[2][g][e]) + part[3][g][e];
        P[((size_t)(h0 + g) * nvchunk_max + c) * hd + e] = r;
    }
}

// -------------------------------------------------------------- combine --
// out[h][e] = sum over chunks in order (all loads of a thread issued before the
// adds); when q8out is given, each head row is also quantized to q8_0 (the
// activation of the following Wo projection, quants.c:74-109 arithmetic).
// grid n_head, hd threads.
__global__ __launch_bounds__(256) void k_attn_combine(const float *__restrict__ P, int nvchunk_max, int hd, int npos_arg,
                                                      const int *npos_dev, float *__restrict__ out, uint8_t *__restrict__ q8out) {
    __shared__ float row[256];
    const int npos = npos_of(npos_arg, npos_dev);
    const int h = blockIdx.x, e = threadIdx.x;
    const int nvc = (npos + ATT_CHUNK - 1) / ATT_CHUNK;
    if (e < hd) {
        const float *p = P + (size_t)h * nvchunk_max * hd + e;
        float r = 0.0f;
        int c = 0;
        for (; c + 32 <= nvc; c += 32) {
            float v[32];
#pragma unroll
            for (int k = 0; k < 32; k++) v[k] = p[(size_t)(c + k) * hd];
#pragma unroll
            for (int k = 0; k < 32; k++) r += v[k];
        }
        for (; c < nvc; c++) r += p[(size_t)c * hd];
        out[(size_t)h * hd + e] = r;
        row[e] = r;
    }
    if (!q8out) return;
    __syncthreads();
    const int gi = e;
    const bool own = gi < hd / 4;
    float v[4] = {0.f, 0.f, 0.f, 0.f};
    if (own)
        for (int k = 0; k < 4; k++) v[k] = row[4 * gi + k];
    if (gi < 64) q8_store4(v, gi, own, q8out + (size_t)h * (hd / 32) * 34);
}

// ------------------------------------------------------------- KV store --
// model.c:583-589: an f16 row (RNE) or q8_0 blocks per head row.
__global__ __launch_bounds__(256) void k_kv_store_f16(const float *__restrict__ src, uint16_t *__restrict__ dst, int n) {
    const int i = blockIdx.x * 256 + threadIdx.x;
    if (i < n) dst[i] = f2h(src[i]);
}

// ------------------------------------------------------------ launchers --
// Workspace: S [n_head][npos] f32 scores/exps, Mc [n_head][nc] f32 chunk
// maxima, Ps [n_head][nsc] f64 chunk sums, P [n_head][nc][hd] f32 partials.
static size_t al256(size_t v) { return (v + 255) & ~(size_t)255; }
size_t attn_workspace_bytes(int n_head, int hd, int npos_max) {
    const size_t nc = (npos_max + ATT_CHUNK - 1) / ATT_CHUNK, nsc = (npos_max + ATT_SCHUNK - 1) / ATT_SCHUNK;
    return al256((size_t)n_head * npos_max * 4) + al256((size_t)n_head * nc * 4) + al256((size_t)n_head * nsc * 8) +
           al256((size_t)n_head * nc * hd * 4);
}

template <int KV, int GRP>
static hipError_t attn_go(const float *q, const uint8_t *kc, const uint8_t *vc, int n_head, int n_kv, int hd, int npos,
                          const int *npos_dev, int npos_max, float *out, uint8_t *q8out, uint8_t *ws, hipStream_t s) {
    const int nc = (npos_max + ATT_CHUNK - 1) / ATT_CHUNK, nsc = (npos_max + ATT_SCHUNK - 1) / ATT_SCHUNK;
    float *S = (float *)ws;
    float *Mc = (float *)(ws + al256((size_t)n_head * npos_max * 4));
    double *Ps = (double *)((uint8_t *)Mc + al256((size_t)n_head * nc * 4));
    float *P = (float *)((uint8_t *)Ps + al256((size_t)n_head * nsc * 8));
    if constexpr (KV == F16)
        hipLaunchKernelGGL((k_attn_scores_f16<GRP>), dim3(n_kv, nc), dim3(256), 0, s, q, kc, n_kv, hd, npos, npos_dev, S, Mc, nc);
    else
        hipLaunchKernelGGL((k_attn_scores_q8<GRP>), dim3(n_kv, nc), dim3(128), 0, s, q, kc, n_kv, hd, npos, npos_dev, S, Mc, nc);
    hipLaunchKernelGGL(k_attn_softmax, dim3(n_head, nsc), dim3(256), 0, s, S, Mc, nc, Ps, nsc, npos, npos_dev);
    hipLaunchKernelGGL((k_attn_v<KV, GRP>), dim3(n_kv, nc), dim3(256), 0, s, S, Ps, nsc, vc, n_kv, hd, npos, npos_dev, P, nc);
    hipLaunchKernelGGL(k_attn_combine, dim3(n_head), dim3(256), 0, s, P, nc, hd, npos, npos_dev, out, q8out);
    return hipGetLastError();
}

hipError_t launch_attn_decode(const float *q, const uint8_t *kc, const uint8_t *vc, int kv_type, int n_head, int n_kv, int hd,
                              int npos, const int *npos_dev, int npos_max, float *out, uint8_t *q8out, uint8_t *ws,
                              hipStream_t s) {
    const int grp = n_head / n_kv;
#define G4_ATT(KV, G) \
    if (kv_type == KV && grp == G) return attn_go<KV, G>(q, kc, vc, n_head, n_kv, hd, npos, npos_dev, npos_max, out, q8out, ws, s)
    G4_ATT(F16, 1); G4_ATT(F16, 2); G4_ATT(F16, 4); G4_ATT(F16, 8);
    G4_ATT(Q8_0, 1); G4_ATT(Q8_0, 2); G4_ATT(Q8_0, 4); G4_ATT(Q8_0, 8);
#undef G4_ATT
    return hipErrorInvalidValue;
}

hipError_t launch_kv_store(int kv_type, const float *src, uint8_t *dst, int hd, int rows, size_t dst_stride, hipStream_t s) {
    if (kv_type == F16) {
        if (dst_stride == (size_t)hd * 2) {
            hipLaunchKernelGGL(k_kv_store_f16, dim3((rows * hd + 255) / 256), dim3(256), 0, s, src, (uint16_t *)dst, rows * hd);
            return hipGetLastError();
        }
        for (int r = 0; r < rows; r++) {
            hipLaunchKernelGGL(k_kv_store_f16, dim3((hd + 255) / 256), dim3(256), 0, s, src + (size_t)r * hd,
                               (uint16_t *)(dst + r * dst_stride), hd);
        }
        return hipGetLastError();
    }
    if (kv_type == Q8_0) return launch_quantize_q8_0(src, hd, dst, dst_stride, hd, rows, s);
    if (kv_type == Q4_0) return launch_quantize_q4_0(src, hd, dst, dst_stride, hd, rows, s);
    return hipErrorInvalidValue;
}

}  // namespace g4
