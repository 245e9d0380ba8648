// k_attn.hip -- decode attention over an f16 or q8_0 KV cache (the GPU form of
// attn_kernel + kv_store, model.c:509-589, with the q/k/v head preparation of
// model.c:664-687 folded in), as three passes over 128-position chunks.
//
// Cache layout: [slot][n_kv][hd] rows (one row = one head's K or V for one
// position), f16 or q8_0 blocks.  Query heads map to KV heads h / (n_head/n_kv)
// (model.c:1099).
//
//   scores   grid (KV head, chunk).  Optionally prepares the rows first: the
//            group's query heads (RMSNorm * q_norm, NeoX RoPE) and -- in the
//            chunk holding the current position -- the new key (RMSNorm *
//            k_norm, RoPE) and value (RMSNorm) rows, stored into the caches at
//            that position.  q is rounded to the K cache's activation form
//            (fp16, or q8_0 blocks, model.c:530-533) and dotted with each K
//            row in the shipped dot's order: eight fp32 lanes of fused
//            products and the same horizontal-sum tree (quants.c:1319-1331 /
//            984-999), so scores equal the CPU's bit for bit; no 1/sqrt(d)
//            (model.c:538).  Per chunk it also stores the maximum m_c and
//            l_c = sum exp(s_j - m_c) in double.
//   V        grid (KV head, chunk).  M = max_c m_c is the global maximum, so
//            e_j = (float)exp(s_j - M) is the reference's expf(s_j - max)
//            (model.c:547); the normaliser sum_c l_c exp(m_c - M) equals the
//            reference's double sum up to the grouping of that sum, and
//            inv = (float)(1/sum) (model.c:549).  Weights fp16(e_j*inv) for an
//            f16 V cache, e_j*inv for q8_0 (model.c:555, 573); each wave
//            accumulates w_j V_j over 32 positions into chunk partials.
//   combine  grid n_head: the chunk partials in order, and q8_0 of each head
//            row for the output projection (quants.c:74-109).
// Only the fp32 order of the value sum and the double grouping of the
// normaliser differ from the CPU's sequential loops.
#include "formats.h"
#include "kernels.h"
#include "steps.h"

namespace g4 {

constexpr int ATT_CHUNK = 128;       // positions per score / V workgroup

__device__ __forceinline__ float wave_max(float v) {
    for (int k = 32; k >= 1; k >>= 1) v = fmaxf(v, shfl_xor(v, k));
    return v;
}
__device__ __forceinline__ double wave_sum_d(double v) {
    for (int k = 32; k >= 1; k >>= 1) v += __shfl_xor(v, k, 64);
    return v;
}

// ------------------------------------------------------- row preparation --
// One projection row handled by one wave, lane holding hd/64 consecutive
// elements (<= 4): the loads are issued by prep_load, the arithmetic by
// prep_finish (RMSNorm in double, weight, NeoX rotation of (i, i + hd/2) whose
// partner is 32 lanes away), as in model.c:338-367.
struct PrepRow {
    float v[4], w[4];
};
__device__ __forceinline__ void prep_load(PrepRow &r, const float *src, const float *w, int hd) {
    const int lane = threadIdx.x & 63, epl = hd >> 6;
#pragma unroll
    for (int e = 0; e < 4; e++) {
        r.v[e] = e < epl ? src[lane * epl + e] : 0.0f;
        r.w[e] = e < epl && w ? w[lane * epl + e] : 1.0f;
    }
}
__device__ __forceinline__ void rope_load(float cs[4], float sn[4], const float *rope, int p, int hd) {
    const int lane = threadIdx.x & 63, epl = hd >> 6, half = hd >> 1;
#pragma unroll
    for (int e = 0; e < 4; e++) {
        const int t = lane * epl + e, i = t < half ? t : t - half;
        cs[e] = e < epl ? rope[(size_t)p * hd + 2 * i] : 1.0f;
        sn[e] = e < epl ? rope[(size_t)p * hd + 2 * i + 1] : 0.0f;
    }
}
__device__ __forceinline__ void prep_finish(const PrepRow &r, bool weighted, bool rotate, const float cs[4], const float sn[4],
                                            int hd, float eps, float y[4]) {
    const int lane = threadIdx.x & 63, epl = hd >> 6;
    double ss = 0.0;
#pragma unroll
    for (int e = 0; e < 4; e++) ss += (double)r.v[e] * r.v[e];
    const float sc = rms_scale(wave_sum_dd(ss), hd, eps);
#pragma unroll
    for (int e = 0; e < 4; e++) y[e] = weighted ? r.v[e] * sc * r.w[e] : r.v[e] * sc;
    if (rotate) {
        const bool lo = lane < 32;
#pragma unroll
        for (int e = 0; e < 4; e++) {
            if (e < epl) {                                           // uniform over the wave
                const float other = __shfl_xor(y[e], 32, 64);
                const float a = lo ? y[e] : other, b = lo ? other : y[e];
                y[e] = lo ? a * cs[e] - b * sn[e] : a * sn[e] + b * cs[e];
            }
        }
    }
}
// a prepared row into a cache slot (f16 RNE, or q8_0 blocks via an LDS row of
// 256 floats for this wave); the whole wave calls it
__device__ __forceinline__ void cache_store(const float y[4], int kv_type, uint8_t *dst, int hd, float *wb) {
    const int lane = threadIdx.x & 63, epl = hd >> 6;
    if (kv_type == F16) {
#pragma unroll
        for (int e = 0; e < 4; e++)
            if (e < epl) ((uint16_t *)dst)[lane * epl + e] = f2h(y[e]);
        return;
    }
#pragma unroll
    for (int e = 0; e < 4; e++)
        if (e < epl) wb[lane * epl + e] = y[e];
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    const bool own = lane < hd / 4;
    float o[4] = {0.f, 0.f, 0.f, 0.f};
    if (own)
        for (int k = 0; k < 4; k++) o[k] = wb[4 * lane + k];
    q8_store4(o, lane, own, dst);
    __builtin_amdgcn_wave_barrier();
}

struct AttnCtx {
    const float *q;          // prepared queries [n_head][hd] (when qkv is null)
    const float *qkv;        // or the raw fused projection output q|k|v to prepare here
    QkvArgs a;               // n_head, n_kv, hd, kv_type, norms, rope, caches, eps
    int npos;                // positions attended (when npos_dev is null)
    const int *npos_dev;     // device position count (graph replay); current position = npos - 1
    float *S;                // [n_head][npos] scores
    float *Mc;               // [n_head][nc] chunk maxima
    double *Lc;              // [n_head][nc] chunk sums of exp(s - m_c)
    float *P;                // [n_head][nc][hd] partial outputs
    int nc;                  // chunk stride of the workspace
    float *out;              // [n_head][hd]
    uint8_t *q8out;          // optional q8_0 rows of out
};

__device__ __forceinline__ int npos_of(const AttnCtx &c) { return c.npos_dev ? *c.npos_dev : c.npos; }

// chunk statistics of GRP heads from per-thread scores: m_c over the valid
// lanes (wave max + LDS), then l_c = sum exp((double)(s - m_c)) over the lanes
// that own a position (`once`: one lane of a pair), waves in order
template <int GRP, int NW>
__device__ void chunk_stats(const float (&s)[GRP], bool ok, bool once, const AttnCtx &c, int h0, int ch, float (*wm)[GRP],
                            double (*wl)[GRP]) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
#pragma unroll
    for (int g = 0; g < GRP; g++) {
        const float m = wave_max(ok ? s[g] : -INFINITY);
        if (lane == 0) wm[wave][g] = m;
    }
    __syncthreads();
    float mc[GRP];
#pragma unroll
    for (int g = 0; g < GRP; g++) {
        mc[g] = wm[0][g];
        for (int w = 1; w < NW; w++) mc[g] = fmaxf(mc[g], wm[w][g]);
        const double e = ok && once ? exp((double)(s[g] - mc[g])) : 0.0;
        const double l = wave_sum_d(e);
        if (lane == 0) wl[wave][g] = l;
    }
    __syncthreads();
    if (threadIdx.x < GRP) {
        const int g = threadIdx.x;
        double l = 0.0;
        for (int w = 0; w < NW; w++) l += wl[w][g];
        c.Mc[(size_t)(h0 + g) * c.nc + ch] = mc[g];
        c.Lc[(size_t)(h0 + g) * c.nc + ch] = l;
    }
}

// ---------------------------------------------------------------- scores --
// f16 cache.  256 threads; a lane pair per position (32 per wave): the even
// lane keeps the fp32 accumulators of elements 8k..8k+3, the odd lane those of
// 8k+4..8k+7 (the shipped dot's eight lanes split in two), combined with the
// same horizontal-sum tree.  Every K load of a lane is issued before any use;
// the lane pair of the current position then takes the new key from LDS.
template <int GRP>
__global__ __launch_bounds__(256) void k_attn_scores_f16(AttnCtx c) {
    __shared__ __align__(16) float4 qf[GRP][64];              // fp16-rounded query
    __shared__ __align__(16) uint16_t kpos[256];              // the new key row (fp16 bits)
    __shared__ float wm[4][GRP];
    __shared__ double wl[4][GRP];
    const int npos = npos_of(c);
    const int kvh = blockIdx.x, ch = blockIdx.y, t = threadIdx.x;
    const int lane = t & 63, wave = t >> 6, hf = lane & 1;
    const int hd = c.a.hd, n_kv = c.a.n_kv, h0 = kvh * GRP, p = npos - 1;
    if (ch * ATT_CHUNK >= npos) return;
    const bool pos_chunk = c.qkv && ch == p / ATT_CHUNK;
    // 1. preparation loads: rows r = 0..GRP-1 (queries), then key and value in
    //    the position's chunk; row r on wave r % 4, slot r / 4
    constexpr int SL = (GRP + 2 + 3) / 4;
    const int nrow = c.qkv ? GRP + (pos_chunk ? 2 : 0) : 0;
    PrepRow pr[SL];
    float cs[4], sn[4];
    constexpr int QPT = GRP;                                   // ready queries: GRP*hd <= GRP*256 elements
    float qv[QPT];
    if (c.qkv) {
        rope_load(cs, sn, c.a.rope, p, hd);
#pragma unroll
        for (int sl = 0; sl < SL; sl++) {
            const int r = wave + 4 * sl;
            if (r < nrow) {
                const int src_row = r < GRP ? h0 + r : r == GRP ? c.a.n_head + kvh : c.a.n_head + n_kv + kvh;
                const float *w = r < GRP ? c.a.q_norm : r == GRP ? c.a.k_norm : nullptr;
                prep_load(pr[sl], c.qkv + (size_t)src_row * hd, w, hd);
            }
        }
    } else {
#pragma unroll
        for (int k = 0; k < QPT; k++) {
            const int i = t + 256 * k;
            qv[k] = i < GRP * hd ? c.q[(size_t)h0 * hd + i] : 0.0f;
        }
    }
    // 2. every K load of the lane
    const int j = ch * ATT_CHUNK + wave * 32 + (lane >> 1);
    const bool ok = j < npos;
    const uint2 *row = (const uint2 *)(c.a.kc + ((size_t)(ok ? j : npos - 1) * n_kv + kvh) * hd * 2) + hf;
    const int nk = hd >> 3;
    uint2 kv[32];
#pragma unroll
    for (int k = 0; k < 32; k++)
        if (k < nk) kv[k] = row[2 * k];
    // 3. preparation arithmetic: queries to LDS; key / value rows to the caches
    if (c.qkv) {
        const int epl = hd >> 6;
#pragma unroll
        for (int sl = 0; sl < SL; sl++) {
            const int r = wave + 4 * sl;
            if (r < nrow) {                                          // uniform over the wave
                float y[4];
                prep_finish(pr[sl], r <= GRP, r <= GRP, cs, sn, hd, c.a.eps, y);
                if (r < GRP) {
#pragma unroll
                    for (int e = 0; e < 4; e++)
                        if (e < epl) ((float *)qf[r])[lane * epl + e] = h2f(f2h(y[e]));
                } else {
                    uint8_t *cache = r == GRP ? c.a.kc : c.a.vc;
                    cache_store(y, F16, cache + ((size_t)p * n_kv + kvh) * hd * 2, hd, nullptr);
                    if (r == GRP) {
#pragma unroll
                        for (int e = 0; e < 4; e++)
                            if (e < epl) kpos[lane * epl + e] = f2h(y[e]);
                    }
                }
            }
        }
    } else {
#pragma unroll
        for (int k = 0; k < QPT; k++) {
            const int i = t + 256 * k;
            if (i < GRP * hd) ((float *)qf[i / hd])[i % hd] = h2f(f2h(qv[k]));
        }
    }
    __syncthreads();
    if (pos_chunk && j == p) {                                       // the new key, not the stale cache row
#pragma unroll
        for (int k = 0; k < 32; k++)
            if (k < nk) kv[k] = ((const uint2 *)kpos)[2 * k + hf];
    }
    // 4. scores
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
                const float4 qq = qf[g][2 * k + hf];
                acc[g][0] = __builtin_fmaf(kf[0], qq.x, acc[g][0]);
                acc[g][1] = __builtin_fmaf(kf[1], qq.y, acc[g][1]);
                acc[g][2] = __builtin_fmaf(kf[2], qq.z, acc[g][2]);
                acc[g][3] = __builtin_fmaf(kf[3], qq.w, acc[g][3]);
            }
        }
    }
    float s[GRP];
#pragma unroll
    for (int g = 0; g < GRP; g++) {
        // lane l of the eight is acc[l & 3] of the pair member l >> 2; r_i = v[i+4] + v[i]
        float r[4];
#pragma unroll
        for (int i = 0; i < 4; i++) r[i] = acc[g][i] + shfl_xor(acc[g][i], 1);
        s[g] = (r[0] + r[2]) + (r[1] + r[3]);
        if (ok && hf == 0) c.S[(size_t)(h0 + g) * npos + j] = s[g];
    }
    chunk_stats<GRP, 4>(s, ok, hf == 0, c, h0, ch, wm, wl);
}

// q8_0 cache.  128 threads, one lane per position; the query is q8_0-quantized
// per block (model.c:533) and each block pair of the row is dotted in the AVX2
// order of quants.c:984-999.
template <int GRP>
__global__ __launch_bounds__(128) void k_attn_scores_q8(AttnCtx c) {
    __shared__ __align__(16) int4 qq[GRP][8][2];
    __shared__ float qd[GRP][8];
    __shared__ __align__(16) uint8_t kpos[8 * 34 + 4];         // the new key row (q8_0 blocks)
    __shared__ float wbuf[2][256];
    __shared__ float qrow[GRP][256];
    __shared__ float wm[2][GRP];
    __shared__ double wl[2][GRP];
    const int npos = npos_of(c);
    const int kvh = blockIdx.x, ch = blockIdx.y, t = threadIdx.x, lane = t & 63, wave = t >> 6;
    const int hd = c.a.hd, n_kv = c.a.n_kv, h0 = kvh * GRP, p = npos - 1;
    if (ch * ATT_CHUNK >= npos) return;
    const bool pos_chunk = c.qkv && ch == p / ATT_CHUNK;
    // queries (prepared here or given) as fp32 rows in LDS; new key/value to the caches
    if (c.qkv) {
        float cs[4], sn[4];
        rope_load(cs, sn, c.a.rope, p, hd);
        const int nrow = GRP + (pos_chunk ? 2 : 0);
        for (int r = wave; r < nrow; r += 2) {                         // uniform over the wave
            const int src_row = r < GRP ? h0 + r : r == GRP ? c.a.n_head + kvh : c.a.n_head + n_kv + kvh;
            PrepRow pr;
            prep_load(pr, c.qkv + (size_t)src_row * hd, r < GRP ? c.a.q_norm : r == GRP ? c.a.k_norm : nullptr, hd);
            float y[4];
            prep_finish(pr, r <= GRP, r <= GRP, cs, sn, hd, c.a.eps, y);
            const int epl = hd >> 6;
            if (r < GRP) {
                for (int e = 0; e < epl; e++) qrow[r][lane * epl + e] = y[e];
            } else {
                uint8_t *dst = (r == GRP ? c.a.kc : c.a.vc) + ((size_t)p * n_kv + kvh) * (hd / 32) * 34;
                cache_store(y, Q8_0, dst, hd, wbuf[wave]);
                if (r == GRP) cache_store(y, Q8_0, kpos, hd, wbuf[wave]);
            }
        }
    } else {
        for (int i = t; i < GRP * hd; i += 128) qrow[i / hd][i % hd] = c.q[(size_t)h0 * hd + i];
    }
    __syncthreads();
    for (int i = t; i < GRP * hd / 4; i += 128) {              // 8 lanes per block; hd/4 is a multiple of 8
        const int g = i / (hd / 4), e4 = i - g * (hd / 4);
        const float v[4] = {qrow[g][4 * e4], qrow[g][4 * e4 + 1], qrow[g][4 * e4 + 2], qrow[g][4 * e4 + 3]};
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
    const int j = ch * ATT_CHUNK + t;
    const bool ok = j < npos;
    const uint8_t *row = pos_chunk && j == p ? kpos : c.a.kc + ((size_t)(ok ? j : npos - 1) * n_kv + kvh) * (hd / 32) * 34;
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
    float s[GRP];
#pragma unroll
    for (int g = 0; g < GRP; g++) {
        const float *a = acc[g];
        const float r0 = a[4] + a[0], r1 = a[5] + a[1], r2 = a[6] + a[2], r3 = a[7] + a[3];
        s[g] = (r0 + r2) + (r1 + r3);
        if (ok) c.S[(size_t)(h0 + g) * npos + j] = s[g];
    }
    chunk_stats<GRP, 2>(s, ok, true, c, h0, ch, wm, wl);
}

// ------------------------------------------------------------ V partials --
// grid (n_kv, chunks of 128), 256 threads.  M and the normaliser from the
// chunk statistics; the chunk's weights go to LDS once; each wave then
// accumulates w_j * V_j over its 32 positions (all V loads of the lane issued
// up front), lane owning 4 consecutive elements; the waves add in order into
// the partial P[h][c][hd].
template <int KV, int GRP>
__global__ __launch_bounds__(256) void k_attn_v(AttnCtx c) {
    __shared__ float part[4][GRP][256];
    __shared__ float wl[GRP][ATT_CHUNK];
    __shared__ float inv_s[GRP], max_s[GRP];
    const int npos = npos_of(c);
    const int kvh = blockIdx.x, ch = blockIdx.y, t = threadIdx.x, lane = t & 63, wave = t >> 6;
    const int hd = c.a.hd, n_kv = c.a.n_kv, h0 = kvh * GRP;
    if (ch * ATT_CHUNK >= npos) return;
    const int j0 = ch * ATT_CHUNK + wave * 32;
    const int nch = (npos + ATT_CHUNK - 1) / ATT_CHUNK;
    // 1. the small loads: chunk statistics (wave w reduces heads w, w+4), the chunk's scores
    constexpr int HPW = (GRP + 3) / 4;
    float mcv[HPW];
    double lcv[HPW];
#pragma unroll
    for (int q = 0; q < HPW; q++) {
        const int g = wave + 4 * q;
        const bool on = g < GRP && lane < nch;
        mcv[q] = on ? c.Mc[(size_t)(h0 + g) * c.nc + lane] : -INFINITY;
        lcv[q] = on ? c.Lc[(size_t)(h0 + g) * c.nc + lane] : 0.0;
    }
    constexpr int EPT = (GRP * ATT_CHUNK + 255) / 256;
    float sv[EPT];
#pragma unroll
    for (int k = 0; k < EPT; k++) {
        const int i = t + 256 * k, g = i / ATT_CHUNK, jw = ch * ATT_CHUNK + (i - g * ATT_CHUNK);
        sv[k] = i < GRP * ATT_CHUNK && jw < npos ? c.S[(size_t)(h0 + g) * npos + jw] : 0.0f;
    }
    // 2. the V rows: lane owns elements 4*lane .. 4*lane+3 (lanes beyond hd/4 idle)
    const bool lane_ok = 4 * lane < hd;
    uint2 vv[32];
    if constexpr (KV == F16) {
#pragma unroll
        for (int k = 0; k < 32; k++) {
            const int j = min(j0 + k, npos - 1);
            if (lane_ok) vv[k] = *((const uint2 *)(c.a.vc + ((size_t)j * n_kv + kvh) * hd * 2) + lane);
        }
    }
    // 3. global max and normaliser (chunks beyond 64 in further passes)
#pragma unroll
    for (int q = 0; q < HPW; q++) {
        const int g = wave + 4 * q;
        if (g < GRP) {                                               // uniform over the wave
            float m = wave_max(mcv[q]);
            for (int c0 = 64; c0 < nch; c0 += 64)
                m = fmaxf(m, wave_max(c0 + lane < nch ? c.Mc[(size_t)(h0 + g) * c.nc + c0 + lane] : -INFINITY));
            double sum = wave_sum_d(lane < nch ? lcv[q] * exp((double)mcv[q] - (double)m) : 0.0);
            for (int c0 = 64; c0 < nch; c0 += 64) {
                const bool on = c0 + lane < nch;
                const float mc = on ? c.Mc[(size_t)(h0 + g) * c.nc + c0 + lane] : 0.0f;
                const double lc = on ? c.Lc[(size_t)(h0 + g) * c.nc + c0 + lane] : 0.0;
                sum += wave_sum_d(on ? lc * exp((double)mc - (double)m) : 0.0);
            }
            if (lane == 0) {
                inv_s[g] = (float)(1.0 / sum);
                max_s[g] = m;
            }
        }
    }
    __syncthreads();
#pragma unroll
    for (int k = 0; k < EPT; k++) {
        const int i = t + 256 * k;
        if (i < GRP * ATT_CHUNK) {
            const int g = i / ATT_CHUNK, pp = i - g * ATT_CHUNK;
            const float e = (float)exp((double)(sv[k] - max_s[g]));
            const float w = e * inv_s[g];
            wl[g][pp] = KV == F16 ? h2f(f2h(w)) : w;
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
                const uint8_t *blk = c.a.vc + ((size_t)j * n_kv + kvh) * (hd / 32) * 34 + (lane >> 3) * 34;
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
        c.P[((size_t)(h0 + g) * c.nc + ch) * hd + e] = r;
    }
}

// -------------------------------------------------------------- combine --
// out[h][e] = sum over chunks in order (32 loads of a thread issued before the
// adds); with q8out, each head row is also quantized to q8_0.  grid n_head.
__global__ __launch_bounds__(256) void k_attn_combine(AttnCtx c) {
    __shared__ float row[256];
    const int npos = npos_of(c);
    const int h = blockIdx.x, e = threadIdx.x, hd = c.a.hd;
    const int nch = (npos + ATT_CHUNK - 1) / ATT_CHUNK;
    if (e < hd) {
        const float *p = c.P + (size_t)h * c.nc * hd + e;
        float r = 0.0f;
        int k0 = 0;
        for (; k0 + 32 <= nch; k0 += 32) {
            float v[32];
#pragma unroll
            for (int k = 0; k < 32; k++) v[k] = p[(size_t)(k0 + k) * hd];
#pragma unroll
            for (int k = 0; k < 32; k++) r += v[k];
        }
        for (; k0 < nch; k0++) r += p[(size_t)k0 * hd];
        c.out[(size_t)h * hd + e] = r;
        row[e] = r;
    }
    if (!c.q8out) return;
    __syncthreads();
    const bool own = e < hd / 4;
    float v[4] = {0.f, 0.f, 0.f, 0.f};
    if (own)
        for (int k = 0; k < 4; k++) v[k] = row[4 * e + k];
    if (e < 64) q8_store4(v, e, own, c.q8out + (size_t)h * (hd / 32) * 34);
}

// ------------------------------------------------------------- KV store --
// model.c:583-589: an f16 row (RNE) or q8_0 blocks per head row.
__global__ __launch_bounds__(256) void k_kv_store_f16(const float *__restrict__ src, uint16_t *__restrict__ dst, int n) {
    const int i = blockIdx.x * 256 + threadIdx.x;
    if (i < n) dst[i] = f2h(src[i]);
}

// ------------------------------------------------------------ launchers --
// Workspace: S [n_head][npos] f32 scores, Mc [n_head][nc] f32 chunk maxima,
// Lc [n_head][nc] f64 chunk sums, P [n_head][nc][hd] f32 partials.
static size_t al256(size_t v) { return (v + 255) & ~(size_t)255; }
size_t attn_workspace_bytes(int n_head, int hd, int npos_max) {
    const size_t nc = (npos_max + ATT_CHUNK - 1) / ATT_CHUNK;
    return al256((size_t)n_head * npos_max * 4) + al256((size_t)n_head * nc * 4) + al256((size_t)n_head * nc * 8) +
           al256((size_t)n_head * nc * hd * 4);
}

template <int KV, int GRP>
static hipError_t attn_go(AttnCtx c, int n_head, int n_kv, int npos_max, uint8_t *ws, hipStream_t s) {
    const int nc = (npos_max + ATT_CHUNK - 1) / ATT_CHUNK;
    c.nc = nc;
    c.S = (float *)ws;
    c.Mc = (float *)(ws + al256((size_t)n_head * npos_max * 4));
    c.Lc = (double *)((uint8_t *)c.Mc + al256((size_t)n_head * nc * 4));
    c.P = (float *)((uint8_t *)c.Lc + al256((size_t)n_head * nc * 8));
    if constexpr (KV == F16) hipLaunchKernelGGL((k_attn_scores_f16<GRP>), dim3(n_kv, nc), dim3(256), 0, s, c);
    else hipLaunchKernelGGL((k_attn_scores_q8<GRP>), dim3(n_kv, nc), dim3(128), 0, s, c);
    hipLaunchKernelGGL((k_attn_v<KV, GRP>), dim3(n_kv, nc), dim3(256), 0, s, c);
    hipLaunchKernelGGL(k_attn_combine, dim3(n_head), dim3(256), 0, s, c);
    return hipGetLastError();
}

// q: prepared queries, or nullptr with `qkv` the raw q|k|v projection output
// to prepare (its k/v rows go into the caches at position npos - 1).
hipError_t launch_attn_decode(const float *q, const float *qkv, const QkvArgs &a, int npos, const int *npos_dev, int npos_max,
                              float *out, uint8_t *q8out, uint8_t *ws, hipStream_t s) {
    if (a.hd % 64 || a.hd > 256 || a.n_kv <= 0 || a.n_head % a.n_kv) return hipErrorInvalidValue;
    if (qkv && (!a.rope || !a.q_norm || !a.k_norm)) return hipErrorInvalidValue;
    AttnCtx c{};
    c.q = q;
    c.qkv = qkv;
    c.a = a;
    c.npos = npos;
    c.npos_dev = npos_dev;
    c.out = out;
    c.q8out = q8out;
    const int grp = a.n_head / a.n_kv;
#define G4_ATT(KV, G) \
    if (a.kv_type == KV && grp == G) return attn_go<KV, G>(c, a.n_head, a.n_kv, npos_max, ws, s)
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
