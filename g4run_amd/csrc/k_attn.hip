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

namespace g4 {

constexpr int ATT_CHUNK = 64;        // positions per score workgroup (one per lane)
constexpr int ATT_VCHUNK = 128;      // positions per V workgroup

__device__ __forceinline__ float hsum8(const float *v) {
    const float r0 = v[4] + v[0], r1 = v[5] + v[1], r2 = v[6] + v[2], r3 = v[7] + v[3];
    return (r0 + r2) + (r1 + r3);
}

__device__ __forceinline__ int npos_of(int npos, const int *npos_dev) { return npos_dev ? *npos_dev : npos; }

// ---------------------------------------------------------------- scores --
// grid (n_kv, chunks), 64 threads: lane = position.  Writes S[h][j] and the
// chunk maximum Mc[h][c] for every query head h of the group.
template <int KV, int GRP>
__global__ __launch_bounds__(64) void k_attn_scores(const float *__restrict__ q, const uint8_t *__restrict__ kc, int n_kv,
                                                    int hd, int npos_arg, const int *npos_dev, float *__restrict__ S,
                                                    float *__restrict__ Mc, int nchunk_max) {
    __shared__ __align__(16) float qf[GRP][256];            // fp16-rounded query (f16 cache)
    __shared__ __align__(16) int4 qq[GRP][8][2];            // q8_0 query blocks (q8_0 cache)
    __shared__ float qd[GRP][8];
    const int npos = npos_of(npos_arg, npos_dev);
    const int kvh = blockIdx.x, c = blockIdx.y, lane = threadIdx.x;
    const int h0 = kvh * GRP;
    const int n_head = n_kv * GRP;
    if (c * ATT_CHUNK >= npos) {                            // chunk past the context: mark empty
        if (lane < GRP) Mc[(size_t)(h0 + lane) * nchunk_max + c] = -INFINITY;
        return;
    }
    if constexpr (KV == F16) {
        for (int i = lane; i < GRP * hd; i += 64) {
            const int g = i / hd, e = i - g * hd;
            qf[g][e] = h2f(f2h(q[(size_t)(h0 + g) * hd + e]));
        }
    } else {
        // q8_0 query blocks (model.c:533): wave-cooperative quantizer, 8 lanes per block
        for (int i = lane; i < GRP * hd / 4; i += 64) {
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
    }
    __syncthreads();
    const int j = c * ATT_CHUNK + lane;
    const bool ok = j < npos;
    float s[GRP];
    if (ok) {
        if constexpr (KV == F16) {
            const uint8_t *row = kc + ((size_t)j * n_kv + kvh) * hd * 2;
            float acc[GRP][8];
#pragma unroll
            for (int g = 0; g < GRP; g++)
#pragma unroll
                for (int l = 0; l < 8; l++) acc[g][l] = 0.0f;
            // 128 elements (16 loads in flight) per step, then a 64-element tail
            auto step = [&](int e0, auto nload) {
                constexpr int NL = decltype(nload)::value;
                int4 kv[NL];
#pragma unroll
                for (int k = 0; k < NL; k++) kv[k] = ld4(row + 2 * e0 + 16 * k);
#pragma unroll
                for (int k = 0; k < NL; k++) {
                    const uint32_t w[4] = {(uint32_t)kv[k].x, (uint32_t)kv[k].y, (uint32_t)kv[k].z, (uint32_t)kv[k].w};
#pragma unroll
                    for (int l = 0; l < 8; l++) {
                        const float kf = h2f((uint16_t)(w[l >> 1] >> (16 * (l & 1))));
#pragma unroll
                        for (int g = 0; g < GRP; g++) acc[g][l] = __builtin_fmaf(kf, qf[g][e0 + 8 * k + l], acc[g][l]);
                    }
                }
            };
            int e0 = 0;
            for (; e0 + 128 <= hd; e0 += 128) step(e0, std::integral_constant<int, 16>{});
            if (e0 < hd) step(e0, std::integral_constant<int, 8>{});
#pragma unroll
            for (int g = 0; g < GRP; g++) s[g] = hsum8(acc[g]);
        } else {
            // q8_0 rows: hd/32 blocks of 34 B; AVX2 order of quants.c:984-999
            const uint8_t *row = kc + ((size_t)j * n_kv + kvh) * (hd / 32) * 34;
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
#pragma unroll
            for (int g = 0; g < GRP; g++) s[g] = hsum8(acc[g]);
        }
    }
#pragma unroll
    for (int g = 0; g < GRP; g++) {
        float m = ok ? s[g] : -INFINITY;
        if (ok) S[(size_t)(h0 + g) * npos + j] = s[g];
        for (int k = 32; k >= 1; k >>= 1) m = fmaxf(m, shfl_xor(m, k));
        if (lane == 0) Mc[(size_t)(h0 + g) * nchunk_max + c] = m;
    }
    (void)n_head;
}

// --------------------------------------------------------------- softmax --
// grid (n_head, chunks of 256 positions): global max over the chunk maxima,
// e_j = (float)exp(s_j - max) written in place, and the chunk's double sum
// Ps[h][c] (wave butterflies, then the four waves in order).
constexpr int ATT_SCHUNK = 256;

__device__ __forceinline__ float wave_max(float v) {
    for (int k = 32; k >= 1; k >>= 1) v = fmaxf(v, shfl_xor(v, k));
    return v;
}
__device__ __forceinline__ double wave_sum_d(double v) {
    for (int k = 32; k >= 1; k >>= 1) v += __shfl_xor(v, k, 64);
    return v;
}

__global__ __launch_bounds__(256) void k_attn_softmax(float *__restrict__ S, const float *__restrict__ Mc, int nchunk_max,
                                                      double *__restrict__ Ps, int nschunk_max, int npos_arg, const int *npos_dev) {
    __shared__ float wm[4];
    __shared__ double ws[4];
    const int npos = npos_of(npos_arg, npos_dev);
    const int h = blockIdx.x, c = blockIdx.y, t = threadIdx.x, lane = t & 63, wave = t >> 6;
    if (c * ATT_SCHUNK >= npos) return;
    const int nchunk = (npos + ATT_CHUNK - 1) / ATT_CHUNK;
    float m = -INFINITY;
    for (int i = t; i < nchunk; i += 256) m = fmaxf(m, Mc[(size_t)h * nchunk_max + i]);
    m = wave_max(m);
    if (lane == 0) wm[wave] = m;
    __syncthreads();
    const float mx = fmaxf(fmaxf(wm[0], wm[1]), fmaxf(wm[2], wm[3]));
    const int j = c * ATT_SCHUNK + t;
    double e = 0.0;
    if (j < npos) {
        float *sp = S + (size_t)h * npos + j;
        const float ef = (float)exp((double)(*sp - mx));
        *sp = ef;
        e = ef;
    }
    e = wave_sum_d(e);
    if (lane == 0) ws[wave] = e;
    __syncthreads();
    if (t == 0) Ps[(size_t)h * nschunk_max + c] = ((ws[0] + ws[1]) + ws[2]) + ws[3];
}

// ------------------------------------------------------------ V partials --
// grid (n_kv, vchunks), 256 threads: inv = (float)(1/sum of the chunk sums in
// order); each of the 4 waves takes 32 positions, issues all their V loads,
// then accumulates w_j * V_j (w_j = fp16(e_j*inv) for an f16 cache); lane owns
// hd/64 elements; partials P[h][c][hd] add the waves in order.
template <int KV, int GRP>
__global__ __launch_bounds__(256) void k_attn_v(const float *__restrict__ E, const double *__restrict__ Ps, int nschunk_max,
                                                const uint8_t *__restrict__ vc, int n_kv, int hd, int npos_arg,
                                                const int *npos_dev, float *__restrict__ P, int nvchunk_max) {
    __shared__ float part[4][GRP][256];
    __shared__ float inv_s[GRP];
    const int npos = npos_of(npos_arg, npos_dev);
    const int kvh = blockIdx.x, c = blockIdx.y, lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int h0 = kvh * GRP;
    if (c * ATT_VCHUNK >= npos) return;
    if (threadIdx.x < GRP) {
        const int ns = (npos + ATT_SCHUNK - 1) / ATT_SCHUNK;
        double sum = 0.0;
        for (int i = 0; i < ns; i++) sum += Ps[(size_t)(h0 + threadIdx.x) * nschunk_max + i];
        inv_s[threadIdx.x] = (float)(1.0 / sum);
    }
    __syncthreads();
    const int epl = hd / 64;                                   // elements per lane (<= 4)
    constexpr int PW = ATT_VCHUNK / 4;                         // positions per wave
    const int j0 = c * ATT_VCHUNK + wave * PW;
    float o[GRP][4];
#pragma unroll
    for (int g = 0; g < GRP; g++)
#pragma unroll
        for (int e = 0; e < 4; e++) o[g][e] = 0.0f;
    if constexpr (KV == F16) {
        uint2 vv[PW];
#pragma unroll
        for (int k = 0; k < PW; k++) {
            const int j = min(j0 + k, npos - 1);
            const uint16_t *row = (const uint16_t *)(vc + ((size_t)j * n_kv + kvh) * hd * 2) + lane * epl;
            if (epl == 4) vv[k] = *(const uint2 *)row;
            else vv[k] = make_uint2(epl > 0 ? row[0] | (epl > 1 ? (uint32_t)row[1] << 16 : 0u) : 0u,
                                    epl > 2 ? row[2] | (epl > 3 ? (uint32_t)row[3] << 16 : 0u) : 0u);
        }
#pragma unroll
        for (int k = 0; k < PW; k++) {
            const int j = j0 + k;
            if (j >= npos) break;
            const float v[4] = {h2f((uint16_t)(vv[k].x & 0xffff)), h2f((uint16_t)(vv[k].x >> 16)),
                                h2f((uint16_t)(vv[k].y & 0xffff)), h2f((uint16_t)(vv[k].y >> 16))};
#pragma unroll
            for (int g = 0; g < GRP; g++) {
                const float w = h2f(f2h(E[(size_t)(h0 + g) * npos + j] * inv_s[g]));
#pragma unroll
                for (int e = 0; e < 4; e++)
                    if (e < epl) o[g][e] = __builtin_fmaf(w, v[e], o[g][e]);
            }
        }
    } else {
        for (int k = 0; k < PW; k++) {
            const int j = j0 + k;
            if (j >= npos) break;
            const uint8_t *row = vc + ((size_t)j * n_kv + kvh) * (hd / 32) * 34;
            float v[4];
            for (int e = 0; e < epl; e++) {
                const int i = lane * epl + e;
                const uint8_t *blk = row + (i >> 5) * 34;
                v[e] = (float)(int8_t)blk[2 + (i & 31)] * h2f((uint16_t)(blk[0] | (blk[1] << 8)));
            }
#pragma unroll
            for (int g = 0; g < GRP; g++) {
                const float w = E[(size_t)(h0 + g) * npos + j] * inv_s[g];
                for (int e = 0; e < epl; e++) o[g][e] = __builtin_fmaf(w, v[e], o[g][e]);
            }
        }
    }
#pragma unroll
    for (int g = 0; g < GRP; g++)
        for (int e = 0; e < epl; e++) part[wave][g][lane * epl + e] = o[g][e];
    __syncthreads();
    for (int i = threadIdx.x; i < GRP * hd; i += 256) {
        const int g = i / hd, e = i - g * hd;
        const float r = ((part[0][g][e] + part[1][g][e]) + part[2][g][e]) + part[3][g][e];
        P[((size_t)(h0 + g) * nvchunk_max + c) * hd + e] = r;
    }
}

// -------------------------------------------------------------- combine --
// out[h][e] = sum over chunks in order (loads issued 16 at a time); when
// q8out is given, each head row is also quantized to q8_0 blocks (the
// activation of the following Wo projection, quants.c:74-109 arithmetic).
__global__ __launch_bounds__(256) void k_attn_combine(const float *__restrict__ P, int nvchunk_max, int hd, int npos_arg,
                                                      const int *npos_dev, float *__restrict__ out, uint8_t *__restrict__ q8out) {
    __shared__ float row[256];
    const int npos = npos_of(npos_arg, npos_dev);
    const int h = blockIdx.x, e = threadIdx.x;
    const int nvc = (npos + ATT_VCHUNK - 1) / ATT_VCHUNK;
    if (e < hd) {
        const float *p = P + (size_t)h * nvchunk_max * hd + e;
        float r = 0.0f;
        int c = 0;
        for (; c + 16 <= nvc; c += 16) {
            float v[16];
#pragma unroll
            for (int k = 0; k < 16; k++) v[k] = p[(size_t)(c + k) * hd];
#pragma unroll
            for (int k = 0; k < 16; k++) r += v[k];
        }
        for (; c < nvc; c++) r += p[(size_t)c * hd];
        out[(size_t)h * hd + e] = r;
        row[e] = r;
    }
    if (!q8out) return;
    __syncthreads();
    if (e < hd / 4) {
        const int b = e >> 3, k = e & 7;
        float v[4] = {row[4 * e], row[4 * e + 1], row[4 * e + 2], row[4 * e + 3]};
        float am = fmaxf(fmaxf(fabsf(v[0]), fabsf(v[1])), fmaxf(fabsf(v[2]), fabsf(v[3])));
        am = fmaxf(am, shfl_xor(am, 1)); am = fmaxf(am, shfl_xor(am, 2)); am = fmaxf(am, shfl_xor(am, 4));
        const float id = am != 0.0f ? 127.0f / am : 0.0f;
        uint32_t pk = 0;
#pragma unroll
        for (int j = 0; j < 4; j++) pk |= ((uint32_t)(int)__builtin_rintf(v[j] * id) & 0xffu) << (8 * j);
        uint8_t *blk = q8out + ((size_t)h * (hd / 32) + b) * 34;
        uint16_t *p16 = (uint16_t *)(blk + 2 + 4 * k);
        p16[0] = (uint16_t)(pk & 0xffff);
        p16[1] = (uint16_t)(pk >> 16);
        if (k == 0) *(uint16_t *)blk = f2h(am * (1.0f / 127.0f));
    }
}

// ------------------------------------------------------------- KV store --
// model.c:583-589: an f16 row (RNE) or q8_0 blocks per head row.
__global__ __launch_bounds__(256) void k_kv_store_f16(const float *__restrict__ src, uint16_t *__restrict__ dst, int n) {
    const int i = blockIdx.x * 256 + threadIdx.x;
    if (i < n) dst[i] = f2h(src[i]);
}

// ------------------------------------------------------------ launchers --
size_t attn_workspace_bytes(int n_head, int hd, int npos_max) {
    const size_t nc = (npos_max + ATT_CHUNK - 1) / ATT_CHUNK, nvc = (npos_max + ATT_VCHUNK - 1) / ATT_VCHUNK,
                 nsc = (npos_max + ATT_SCHUNK - 1) / ATT_SCHUNK;
    auto al = [](size_t v) { return (v + 255) & ~(size_t)255; };
    return al((size_t)n_head * npos_max * 4) + al((size_t)n_head * nc * 4) + al((size_t)n_head * nsc * 8) +
           al((size_t)n_head * nvc * hd * 4);
}

template <int KV, int GRP>
static hipError_t attn_go(const float *q, const uint8_t *kc, const uint8_t *vc, int n_head, int n_kv, int hd, int npos,
                          const int *npos_dev, int npos_max, float *out, uint8_t *q8out, uint8_t *ws, hipStream_t s) {
    const int nc = (npos_max + ATT_CHUNK - 1) / ATT_CHUNK, nvc = (npos_max + ATT_VCHUNK - 1) / ATT_VCHUNK,
              nsc = (npos_max + ATT_SCHUNK - 1) / ATT_SCHUNK;
    auto al = [](size_t v) { return (v + 255) & ~(size_t)255; };
    float *S = (float *)ws;
    float *Mc = (float *)(ws + al((size_t)n_head * npos_max * 4));
    double *Ps = (double *)((uint8_t *)Mc + al((size_t)n_head * nc * 4));
    float *P = (float *)((uint8_t *)Ps + al((size_t)n_head * nsc * 8));
    hipLaunchKernelGGL((k_attn_scores<KV, GRP>), dim3(n_kv, nc), dim3(64), 0, s, q, kc, n_kv, hd, npos, npos_dev, S, Mc, nc);
    hipLaunchKernelGGL(k_attn_softmax, dim3(n_head, nsc), dim3(256), 0, s, S, Mc, nc, Ps, nsc, npos, npos_dev);
    hipLaunchKernelGGL((k_attn_v<KV, GRP>), dim3(n_kv, nvc), dim3(256), 0, s, S, Ps, nsc, vc, n_kv, hd, npos, npos_dev, P, nvc);
    hipLaunchKernelGGL(k_attn_combine, dim3(n_head), dim3(256), 0, s, P, nvc, hd, npos, npos_dev, out, q8out);
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
