// k_attn.hip -- decode attention over an f16 or q8_0 KV cache (the GPU form of
// attn_kernel + kv_store, model.c:509-589, with the q/k/v head preparation of
// model.c:664-687 folded in) over 128-position chunks.
//
// Cache layout: [slot][n_kv][hd] rows (one row = one head's K or V for one
// position), f16, q8_0 or q4_0 blocks.  Query heads map to KV heads h / (n_head/n_kv)
// (model.c:1099).
//
// Steps (one launch, k_attn_fused_f16, for f16 caches whose chunks the device
// holds resident at once; otherwise three launches through global memory):
//   preparation  optionally the group's query heads (RMSNorm * q_norm, NeoX
//                RoPE) and -- in the chunk holding the current position -- the
//                new key (RMSNorm * k_norm, RoPE) and value (RMSNorm) rows,
//                stored into the caches at that position; q is rounded to the
//                K cache's activation form (fp16, or q8_0 blocks for a q8_0 /
//                q4_0 cache, model.c:530-533).
//   scores       s_j = K_j . q, no 1/sqrt(d) (model.c:538).  f16: each lane's 8
//                products in element order, then a butterfly over the row's
//                lanes -- a fixed order that differs from the CPU's 8-lane f16
//                dot (quants.c:1319-1331) only in the fp32 rounding of the sum.
//                q8_0 / q4_0: one lane per position in the AVX2 q8_0 / q4_0 dot's order
//                (quants.c:984-999), equal to the CPU's bit for bit.  Per chunk
//                the maximum m_c and l_c = sum exp(s_j - m_c) in double.
//   weights      M = max_c m_c is the global maximum, so e_j = (float)exp(s_j - M)
//                is the reference's expf(s_j - max) (model.c:547); the
//                normaliser sum_c l_c exp(m_c - M) equals the reference's
//                double sum up to the grouping of that sum, and inv =
//                (float)(1/sum) (model.c:549).  Weights fp16(e_j*inv) for an f16
//                V cache, e_j*inv for q8_0 / q4_0 (model.c:555, 573).
//   V / combine  chunk partials of sum w_j V_j, added in chunk order, and q8_0
//                of each head row for the output projection (quants.c:74-109).
// Beyond the f16 score sum, only the fp32 order of the value sum and the
// double grouping of the normaliser differ from the CPU's sequential loops;
// the one-launch and three-launch forms give identical bits.
#include <algorithm>
#include <map>
#include <mutex>
#include <type_traits>

#include "formats.h"
#include "gemv_p.h"
#include "handoff.h"
#include "kernels.h"
#include "steps.h"

namespace g4 {

constexpr int ATT_CHUNK = 128;       // positions per score / V workgroup
constexpr int ATT_WIDE = 512;        // gemma4's full-attention head width (one KV head), run as two halves
constexpr int ATT_HALF = 256;
constexpr int ATT_CSUM = 8;          // chunks per group in the combine's two-level sum
// one-launch form: V loads per lane issued while K is scored; the rest are
// issued after the statistics hand-off
#ifndef ATT_V_EARLY
#define ATT_V_EARLY 16
#endif
#ifndef ATT_QKV_WAIT
#define ATT_QKV_WAIT 1
#endif
#ifndef ATT_QKV_KLATE
#define ATT_QKV_KLATE 0
#endif
#ifndef ATT_QKV_VFIRST
#define ATT_QKV_VFIRST 0
#endif

__device__ __forceinline__ float wave_max(float v) { return group_max<64>(v); }
__device__ __forceinline__ double wave_sum_d(double v) { return group_sum_t<64>(v); }

// ------------------------------------------------------- row preparation --
// One projection row handled by one wave, lane holding hd/64 consecutive
// elements (<= N: 4 for rows up to 256, 8 for the 512-wide heads): the loads
// are issued by prep_load, the arithmetic by prep_finish (RMSNorm in double,
// weight, NeoX rotation of (i, i + hd/2) whose partner is 32 lanes away), as in
// model.c:338-367.
template <int N>
struct PrepRowN {
    float v[N], w[N];
};
using PrepRow = PrepRowN<4>;
template <int N>
__device__ __forceinline__ void prep_load(PrepRowN<N> &r, const float *src, const float *w, int hd) {
    const int lane = threadIdx.x & 63, epl = hd >> 6;
#pragma unroll
    for (int e = 0; e < N; e++) {
        r.v[e] = e < epl ? src[lane * epl + e] : 0.0f;
        r.w[e] = e < epl && w ? w[lane * epl + e] : 1.0f;
    }
}
template <int N>
__device__ __forceinline__ void rope_load(float (&cs)[N], float (&sn)[N], const float *rope, int p, int hd) {
    const int lane = threadIdx.x & 63, epl = hd >> 6, half = hd >> 1;
#pragma unroll
    for (int e = 0; e < N; e++) {
        const int t = lane * epl + e, i = t < half ? t : t - half;
        cs[e] = e < epl ? rope[(size_t)p * hd + 2 * i] : 1.0f;
        sn[e] = e < epl ? rope[(size_t)p * hd + 2 * i + 1] : 0.0f;
    }
}
template <int N>
__device__ __forceinline__ void prep_finish(const PrepRowN<N> &r, bool weighted, bool rotate, const float (&cs)[N],
                                            const float (&sn)[N], int hd, float eps, float (&y)[N]) {
    const int lane = threadIdx.x & 63, epl = hd >> 6;
    double ss = 0.0;
#pragma unroll
    for (int e = 0; e < N; e++) ss += (double)r.v[e] * r.v[e];
    const float sc = rms_scale(wave_sum_dd(ss), hd, eps);
#pragma unroll
    for (int e = 0; e < N; e++) y[e] = weighted ? r.v[e] * sc * r.w[e] : r.v[e] * sc;
    if (rotate) {
        const bool lo = lane < 32;
#pragma unroll
        for (int e = 0; e < N; e++) {
            if (e < epl) {                                           // uniform over the wave
                const float other = partner<32>(y[e]);
                const float a = lo ? y[e] : other, b = lo ? other : y[e];
                y[e] = lo ? a * cs[e] - b * sn[e] : a * sn[e] + b * cs[e];
            }
        }
    }
}
// a prepared row into a cache slot (f16 RNE, or q8_0 / q4_0 blocks via an LDS
// row of 64 N floats for this wave); the whole wave calls it
template <int N>
__device__ __forceinline__ void cache_store(const float (&y)[N], int kv_type, uint8_t *dst, int hd, float *wb) {
    const int lane = threadIdx.x & 63, epl = hd >> 6;
    if (kv_type == F16) {
#pragma unroll
        for (int e = 0; e < N; e++)
            if (e < epl) ((uint16_t *)dst)[lane * epl + e] = f2h(y[e]);
        return;
    }
#pragma unroll
    for (int e = 0; e < N; e++)
        if (e < epl) wb[lane * epl + e] = y[e];
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
#pragma unroll
    for (int k = 0; k < N / 4; k++) {                                // groups of 4 elements: lane + 64 k
        const int gi = lane + 64 * k;
        const bool own = gi < hd / 4;
        float o[4] = {0.f, 0.f, 0.f, 0.f};
        if (own)
            for (int i = 0; i < 4; i++) o[i] = wb[4 * gi + i];
        if (kv_type == Q4_0) q4_store4(o, gi, own, dst);
        else q8_store4(o, gi, own, dst);
    }
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
    // fused launch: tagged statistics T [n_head][nc][ATT_TW] (3 words used) and partials
    // PT [n_head][nc][hd]; this launch's tag is *epoch * tag_mul + tag_add + 1
    uint64_t *T, *PT;
    const unsigned *epoch;
    unsigned tag_mul, tag_add;
    // self-advancing epoch (calls without an external epoch): every workgroup
    // stores a tagged word in SW [grid] once it has this launch's tag; the
    // last workgroup polls them all and then stores the tag into *adv, so the
    // next launch on the workspace gets the next tag
    unsigned *adv;
    uint64_t *SW;
    unsigned *err;           // set when a poll gives up
    unsigned spin;           // polls give up after this many retries
    uint32_t poll_xor;       // nonzero (test hook only): polls wait for a tag no store carries
    // one launch with the q|k|v projection folded in (decode step): every
    // workgroup computes qrows projection rows of W from the RMSNorm prologue
    // `pro` and publishes them as tagged words QT [rows] (one 128-byte line
    // per workgroup); the attention rows are then taken from QT
    g4h_tensor W;
    GemvPro pro;
    uint64_t *QT;
    int qrows;
    int pabs, mirror;        // set by attn_view
    // a batch of ntok > 1 tokens on grid.z (the three passes only): token b
    // attends npos + b positions with query / output rows b, its q8_0 output
    // row q8_tok bytes further and its own workspace block ws_tok bytes further
    int ntok;
    size_t ws_tok, q8_tok;
    // the output projection folded into the one-launch form (decode step):
    // the head rows' q8_0 blocks go out as tagged words QO [block][16] (one
    // 128-byte line each, 9 words used) and every workgroup then computes Wo
    // row groups into wo_out with the GEMV family's arithmetic
    g4h_tensor Wo;
    float *wo_out;
    uint64_t *QO;
};

__device__ __forceinline__ int npos_of(const AttnCtx &c) { return c.npos_dev ? *c.npos_dev : c.npos; }

// token blockIdx.z of a batch (causal prefill, model.c:514-521: token b at
// position pos0 + b attends positions 0 .. pos0 + b): its rows, its
// positions and its workspace block; every three-pass kernel starts here
__device__ __forceinline__ void attn_token(AttnCtx &c) {
    if (c.ntok <= 1) return;
    const int b = blockIdx.z;
    const size_t rows = (size_t)b * c.a.n_head * c.a.hd;
    c.q += rows;
    c.out += rows;
    if (c.q8out) c.q8out += b * c.q8_tok;
    c.npos += b;
    const size_t sh = b * c.ws_tok;
    c.S = (float *)((uint8_t *)c.S + sh);
    c.Mc = (float *)((uint8_t *)c.Mc + sh);
    c.Lc = (double *)((uint8_t *)c.Lc + sh);
    c.P = (float *)((uint8_t *)c.P + sh);
}

// The rows a launch attends as a linear cache (every kernel starts here):
// positions j0 .. npos-1 with j0 = max(0, npos - window) (a sliding window,
// model.c:517-519; window 0: all positions).  On a ring of `ring` slots each
// row is stored twice, at slot s and s + ring (s = position % ring), so any
// window of at most `ring` positions is contiguous from slot j0 % ring: the
// cache pointers are moved there and the caller sees rows 0 .. nv-1.  Sets
// c.pabs (the current position, the RoPE row) and c.mirror (the row index of
// the current row's second copy, relative to the moved pointers, or INT_MIN).
__device__ __forceinline__ int attn_view(AttnCtx &c) {
    const int npos = npos_of(c);
    c.pabs = npos - 1;
    c.mirror = INT_MIN;
    if (!c.a.window) return npos;
    const int j0 = npos > c.a.window ? npos - c.a.window : 0;
    const int base = c.a.ring ? j0 % c.a.ring : j0;
    const size_t row = c.a.kv_type == F16 ? (size_t)c.a.hd * 2 : (size_t)(c.a.hd / 32) * (c.a.kv_type == Q4_0 ? 18 : 34);
    const size_t slot = (size_t)c.a.n_kv * row;
    c.a.kc += (size_t)base * slot;
    c.a.vc += (size_t)base * slot;
    const int nv = npos - j0;
    if (c.a.ring) {
        const int s = base + nv - 1;                               // slot of the current row's first copy
        c.mirror = (s < c.a.ring ? s + c.a.ring : s - c.a.ring) - base;
    }
    return nv;
}


// chunk statistics of GRP heads from per-thread scores: m_c over the valid
// lanes (wave max + LDS), then l_c = sum exp((double)(s - m_c)) over the lanes
// that own a position (`once`: one lane of a pair), waves in order
template <int GRP, int NW, bool AG>
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
        if constexpr (AG) {
            st_ag(&c.Mc[(size_t)(h0 + g) * c.nc + ch], mc[g]);
            st_ag(&c.Lc[(size_t)(h0 + g) * c.nc + ch], l);
        } else {
            c.Mc[(size_t)(h0 + g) * c.nc + ch] = mc[g];
            c.Lc[(size_t)(h0 + g) * c.nc + ch] = l;
        }
    }
}

// ---------------------------------------------------------------- scores --
// f16 cache.  256 threads; a lane pair per position (32 per wave): the even
// lane keeps the fp32 accumulators of elements 8k..8k+3, the odd lane those of
// 8k+4..8k+7 (the shipped dot's eight lanes split in two), combined with the
// same horizontal-sum tree.  Every K load of a lane is issued before any use;
// the lane pair of the current position then takes the new key from LDS.

// preparation state: rows r = 0..GRP-1 (queries), then key and value in the
// chunk of the current position; row r on wave r % 4, slot r / 4
template <int GRP>
struct PrepF16 {
    static constexpr int SL = (GRP + 2 + 3) / 4;
    PrepRow pr[SL];
    float cs[4], sn[4];
    float qv[GRP];                   // given queries: GRP*hd <= 256*GRP elements
    int nrow;
};

// decode step with the projection folded in: the rows' norm weights and RoPE
// row here; their values come later from the projection's tagged words
template <int GRP, int HD>
__device__ __forceinline__ void prep_f16_issue_w(PrepF16<GRP> &st, const AttnCtx &c, int kvh, int p, bool pos_chunk) {
    constexpr int hd = HD, epl = hd >> 6;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    st.nrow = GRP + (pos_chunk ? 2 : 0);
    rope_load(st.cs, st.sn, c.a.rope, c.pabs, hd);
#pragma unroll
    for (int sl = 0; sl < PrepF16<GRP>::SL; sl++) {
        const int r = wave + 4 * sl;
        if (r < st.nrow) {
            const float *w = r < GRP ? c.a.q_norm : r == GRP ? c.a.k_norm : nullptr;
#pragma unroll
            for (int e = 0; e < 4; e++) st.pr[sl].w[e] = e < epl && w ? w[lane * epl + e] : 1.0f;
        }
    }
}

template <int GRP, int HD>
__device__ __forceinline__ void prep_f16_issue(PrepF16<GRP> &st, const AttnCtx &c, int kvh, int p, bool pos_chunk) {
    constexpr int hd = HD;
    const int t = threadIdx.x, wave = t >> 6, h0 = kvh * GRP;
    st.nrow = c.qkv ? GRP + (pos_chunk ? 2 : 0) : 0;
    if (c.qkv) {
        rope_load(st.cs, st.sn, c.a.rope, c.pabs, hd);
#pragma unroll
        for (int sl = 0; sl < PrepF16<GRP>::SL; sl++) {
            const int r = wave + 4 * sl;
            if (r < st.nrow) {
                const int src_row = r < GRP ? h0 + r : r == GRP ? c.a.n_head + kvh : c.a.n_head + c.a.n_kv + kvh;
                const float *w = r < GRP ? c.a.q_norm : r == GRP ? c.a.k_norm : nullptr;
                prep_load(st.pr[sl], c.qkv + (size_t)src_row * hd, w, hd);
            }
        }
    } else {
#pragma unroll
        for (int k = 0; k < GRP; k++) {
            const int i = t + 256 * k;
            st.qv[k] = i < GRP * hd ? c.q[(size_t)h0 * hd + i] : 0.0f;
        }
    }
}

// queries (fp16-rounded) into LDS; the key / value rows of the current
// position into the caches and, as fp16 bits, into kpos / vpos (vpos optional)
template <int GRP, int HD>
__device__ __forceinline__ void prep_f16_finish(const PrepF16<GRP> &st, const AttnCtx &c, int kvh, int p, float4 (*qf)[64],
                                                uint16_t *kpos, uint16_t *vpos) {
    constexpr int hd = HD, epl = hd >> 6;
    const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
    if (st.nrow > 0) {                                                  // rows to prepare (projection output)
#pragma unroll
        for (int sl = 0; sl < PrepF16<GRP>::SL; sl++) {
            const int r = wave + 4 * sl;
            if (r < st.nrow) {                                          // uniform over the wave
                float y[4];
                prep_finish(st.pr[sl], r <= GRP, r <= GRP, st.cs, st.sn, hd, c.a.eps, y);
                if (r < GRP) {
#pragma unroll
                    for (int e = 0; e < 4; e++)
                        if (e < epl) ((float *)qf[r])[lane * epl + e] = h2f(f2h(y[e]));
                } else {
                    uint8_t *cache = r == GRP ? c.a.kc : c.a.vc;
                    cache_store(y, F16, cache + ((size_t)p * c.a.n_kv + kvh) * hd * 2, hd, nullptr);
                    if (c.mirror != INT_MIN)                               // the ring's second copy
                        cache_store(y, F16, cache + ((ptrdiff_t)c.mirror * c.a.n_kv + kvh) * hd * 2, hd, nullptr);
                    uint16_t *keep = r == GRP ? kpos : vpos;
                    if (keep) {
#pragma unroll
                        for (int e = 0; e < 4; e++)
                            if (e < epl) keep[lane * epl + e] = f2h(y[e]);
                    }
                }
            }
        }
    } else {
#pragma unroll
        for (int k = 0; k < GRP; k++) {
            const int i = t + 256 * k;
            if (i < GRP * hd) ((float *)qf[i / hd])[i % hd] = h2f(f2h(st.qv[k]));
        }
    }
}

// K and V rows of a wave's 32 positions as 16-byte non-temporal loads (the
// cache is read once per step; measured 12.9 against 17.8 us for the whole
// one-launch attention at 8192 positions with plain loads), coalesced: a row is
// HD/8 slots of 8 elements; lane l = r * VS + q takes slot q of rows r, r + VR,
// r + 2 VR, ... (VS = HD/8 rounded up to a power of two lanes per row, VR =
// 64 / VS rows per load; lanes with q >= HD/8 load slot HD/8 - 1 again and
// stay out of the sums).  Rows past the last position are the last row again.
template <int HD>
struct VGeo {
    static constexpr int NS = HD / 8;                                // 8-element slots per row
    static constexpr int VS = NS <= 8 ? 8 : NS <= 16 ? 16 : 32;
    static constexpr int VR = 64 / VS;
    static constexpr int NV = 32 / VR;                               // loads per lane
};
// load i of the lane: slot q of row j0 + i * VR + r
template <int HD>
__device__ __forceinline__ uint4 row_load(const uint8_t *cache, int n_kv, int kvh, int j0, int i, int npos) {
    using G = VGeo<HD>;
    const int lane = threadIdx.x & 63, r = lane / G::VS, q = min(lane % G::VS, G::NS - 1);
    const int j = min(j0 + i * G::VR + r, npos - 1);
    const int4 w = ld4s((const uint4 *)(cache + ((size_t)j * n_kv + kvh) * HD * 2) + q);
    return make_uint4(w.x, w.y, w.z, w.w);
}
template <int HD>
__device__ __forceinline__ void rows_load(uint4 (&rq)[16], const uint8_t *cache, int n_kv, int kvh, int j0, int npos) {
#pragma unroll
    for (int i = 0; i < 16; i++)
        if (i < VGeo<HD>::NV) rq[i] = row_load<HD>(cache, n_kv, kvh, j0, i, npos);
}
// the row of position p (in the wave's rows j0 ..) from an LDS copy (fp16
// bits); p < 0: none.  A select, not a branch (a branch here would make the
// compiler wait for all of the rows' loads at once).
template <int HD>
__device__ __forceinline__ uint4 new_row_slot(const uint16_t *row) {
    using G = VGeo<HD>;
    return ((const uint4 *)row)[min((int)(threadIdx.x & 63) % G::VS, G::NS - 1)];
}
template <int HD>
__device__ __forceinline__ void new_row1(uint4 &rq, const uint4 &nr, int j0, int i, int p) {
    using G = VGeo<HD>;
    const bool hit = j0 + i * G::VR + (int)(threadIdx.x & 63) / G::VS == p;
    rq.x = hit ? nr.x : rq.x;
    rq.y = hit ? nr.y : rq.y;
    rq.z = hit ? nr.z : rq.z;
    rq.w = hit ? nr.w : rq.w;
}
template <int HD>
__device__ __forceinline__ void new_row(uint4 (&rq)[16], const uint16_t *row, int j0, int p) {
    const uint4 nr = new_row_slot<HD>(row);
#pragma unroll
    for (int i = 0; i < VGeo<HD>::NV; i++) new_row1<HD>(rq[i], nr, j0, i, p);
}
__device__ __forceinline__ void h8(const uint4 &w, float (&v)[8]) {
    const uint32_t u[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
    for (int e = 0; e < 4; e++) {
        v[2 * e] = h2f((uint16_t)(u[e] & 0xffff));
        v[2 * e + 1] = h2f((uint16_t)(u[e] >> 16));
    }
}
// the lane's 8 query elements of each head (fp16-rounded queries in LDS)
template <int GRP, int HD>
__device__ __forceinline__ void q_slot(const float4 (*qf)[64], float (&qv)[GRP][8]) {
    using G = VGeo<HD>;
    const int q = min((int)(threadIdx.x & 63) % G::VS, G::NS - 1);
#pragma unroll
    for (int g = 0; g < GRP; g++) {
        const float4 a = qf[g][2 * q], b = qf[g][2 * q + 1];
        qv[g][0] = a.x; qv[g][1] = a.y; qv[g][2] = a.z; qv[g][3] = a.w;
        qv[g][4] = b.x; qv[g][5] = b.y; qv[g][6] = b.z; qv[g][7] = b.w;
    }
}
// Scores s_j = K_j . q (no 1/sqrt(d), model.c:538) of the wave's 32 positions
// into sc[g][wave*32 + k]: each lane's 8 products in element order, then the
// row's lanes summed by a butterfly (xor VS/2, ..., 1).  A fixed order, the
// same in the three-pass and the one-launch forms; it differs from the CPU's
// 8-lane accumulation only in the fp32 rounding of the sum.
template <int GRP, int HD>
__device__ __forceinline__ void score_row(const uint4 &kq, const float (&qv)[GRP][8], float (*sc)[ATT_CHUNK], int i) {
    using G = VGeo<HD>;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, r = lane / G::VS, q = lane % G::VS;
    const bool act = q < G::NS;
    float kf[8];
    h8(kq, kf);
#pragma unroll
    for (int g = 0; g < GRP; g++) {
        float acc = 0.0f;
#pragma unroll
        for (int e = 0; e < 8; e++) acc = __builtin_fmaf(kf[e], qv[g][e], acc);
        acc = act ? acc : 0.0f;
        acc = group_sum<G::VS>(acc);
        if (q == 0) sc[g][wave * 32 + i * G::VR + r] = acc;
    }
}
template <int GRP, int HD>
__device__ __forceinline__ void scores_rows(const uint4 (&kq)[16], const float (&qv)[GRP][8], float (*sc)[ATT_CHUNK]) {
#pragma unroll
    for (int i = 0; i < VGeo<HD>::NV; i++) score_row<GRP, HD>(kq[i], qv, sc, i);
}

// grid (n_kv, chunks of 128), 256 threads: wave w scores positions
// ch*128 + 32w .. +31; lane l < 32 of the wave then owns position 32w + l for
// the chunk statistics.  The chunk of the current position takes the new key
// row from LDS in place of the stale cache row.
template <int GRP, int HD>
__global__ __launch_bounds__(256) void k_attn_scores_f16(AttnCtx c) {
    __shared__ __align__(16) float4 qf[GRP][64];              // fp16-rounded query
    __shared__ __align__(16) uint16_t kpos[256];              // the new key row (fp16 bits)
    __shared__ float sc[GRP][ATT_CHUNK];
    __shared__ float wm[4][GRP];
    __shared__ double wl[4][GRP];
    attn_token(c);
    const int npos = attn_view(c);
    const int kvh = blockIdx.x, ch = blockIdx.y, t = threadIdx.x;
    const int lane = t & 63, wave = t >> 6;
    const int h0 = kvh * GRP, p = npos - 1;
    if (ch * ATT_CHUNK >= npos) return;
    const bool pos_chunk = c.qkv && ch == p / ATT_CHUNK;
    const int j0 = ch * ATT_CHUNK + wave * 32;
    PrepF16<GRP> st;
    prep_f16_issue<GRP, HD>(st, c, kvh, p, pos_chunk);
    wait_loads();
    uint4 kq[16];
    rows_load<HD>(kq, c.a.kc, c.a.n_kv, kvh, j0, npos);
    issue_order();
    prep_f16_finish<GRP, HD>(st, c, kvh, p, qf, kpos, nullptr);
    lds_barrier();
    new_row<HD>(kq, kpos, j0, pos_chunk ? p : -1);
    float qv[GRP][8];
    q_slot<GRP, HD>(qf, qv);
    scores_rows<GRP, HD>(kq, qv, sc);
    lds_barrier();
    const int j = j0 + lane;
    const bool ok = lane < 32 && j < npos;
    float s[GRP];
#pragma unroll
    for (int g = 0; g < GRP; g++) {
        s[g] = lane < 32 ? sc[g][wave * 32 + lane] : 0.0f;
        if (ok) c.S[(size_t)(h0 + g) * npos + j] = s[g];
    }
    chunk_stats<GRP, 4, false>(s, ok, lane < 32, c, h0, ch, wm, wl);
}

// q8_0 / q4_0 cache.  128 threads, one lane per position; the query is
// q8_0-quantized per block (model.c:533) and each block pair of the row is
// dotted in the AVX2 order of quants.c:984-999 (q8_0) / 964-982 (q4_0): eight
// int32 lanes of 4 elements, one fma per lane and block, then hsum_float_8.
template <int KV, int GRP, int HD>
__global__ __launch_bounds__(128) void k_attn_scores_q8(AttnCtx c) {
    constexpr int BS = KV == Q4_0 ? 18 : 34;                      // bytes per 32-element block
    __shared__ __align__(16) int4 qq[GRP][8][2];
    __shared__ float qd[GRP][8];
    __shared__ __align__(16) uint8_t kpos[8 * 34 + 4];         // the new key row (q8_0 / q4_0 blocks)
    __shared__ float wbuf[2][256];
    __shared__ float qrow[GRP][256];
    __shared__ float wm[2][GRP];
    __shared__ double wl[2][GRP];
    attn_token(c);
    const int npos = attn_view(c);
    const int kvh = blockIdx.x, ch = blockIdx.y, t = threadIdx.x, lane = t & 63, wave = t >> 6;
    constexpr int hd = HD;
    const int n_kv = c.a.n_kv, h0 = kvh * GRP, p = npos - 1;
    if (ch * ATT_CHUNK >= npos) return;
    const bool pos_chunk = c.qkv && ch == p / ATT_CHUNK;
    // queries (prepared here or given) as fp32 rows in LDS; new key/value to the caches
    if (c.qkv) {
        float cs[4], sn[4];
        rope_load(cs, sn, c.a.rope, c.pabs, hd);
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
                uint8_t *dst = (r == GRP ? c.a.kc : c.a.vc) + ((size_t)p * n_kv + kvh) * (hd / 32) * BS;
                cache_store(y, KV, dst, hd, wbuf[wave]);
                if (c.mirror != INT_MIN)                                   // the ring's second copy
                    cache_store(y, KV, (r == GRP ? c.a.kc : c.a.vc) + ((ptrdiff_t)c.mirror * n_kv + kvh) * (hd / 32) * BS, hd,
                                wbuf[wave]);
                if (r == GRP) cache_store(y, KV, kpos, hd, wbuf[wave]);
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
        am = group_max<8>(am);
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
    const uint8_t *row = pos_chunk && j == p ? kpos : c.a.kc + ((size_t)(ok ? j : npos - 1) * n_kv + kvh) * (hd / 32) * BS;
    float acc[GRP][8];
#pragma unroll
    for (int g = 0; g < GRP; g++)
#pragma unroll
        for (int l = 0; l < 8; l++) acc[g][l] = 0.0f;
    for (int b = 0; b < hd / 32; b += 2) {
        // the two blocks' 32 signed quants as 8 words each (lane l = elements 4l..4l+3)
        uint32_t w0[8], w1[8];
        float d0, d1;
        if constexpr (KV == Q4_0) {
            uint32_t v[9];
            const uint32_t *src = (const uint32_t *)(row + (size_t)b * 18);
#pragma unroll
            for (int k = 0; k < 9; k++) v[k] = src[k];
            uint32_t n0[4], n1[4];
#pragma unroll
            for (int k = 0; k < 4; k++) { n0[k] = __builtin_amdgcn_alignbyte(v[k + 1], v[k], 2); n1[k] = v[5 + k]; }
            // nibble n -> n - 8 as a signed byte, carry-free: (n + 0x78) ^ 0x80
#pragma unroll
            for (int k = 0; k < 4; k++) {
                w0[k] = ((n0[k] & 0x0F0F0F0Fu) + 0x78787878u) ^ 0x80808080u;
                w0[k + 4] = (((n0[k] >> 4) & 0x0F0F0F0Fu) + 0x78787878u) ^ 0x80808080u;
                w1[k] = ((n1[k] & 0x0F0F0F0Fu) + 0x78787878u) ^ 0x80808080u;
                w1[k + 4] = (((n1[k] >> 4) & 0x0F0F0F0Fu) + 0x78787878u) ^ 0x80808080u;
            }
            d0 = h2f((uint16_t)(v[0] & 0xffff));
            d1 = h2f((uint16_t)(v[4] >> 16));
        } else {
            uint32_t v[17];
            const uint32_t *src = (const uint32_t *)(row + (size_t)b * 34);
#pragma unroll
            for (int k = 0; k < 17; k++) v[k] = src[k];
#pragma unroll
            for (int k = 0; k < 8; k++) { w0[k] = __builtin_amdgcn_alignbyte(v[k + 1], v[k], 2); w1[k] = v[9 + k]; }
            d0 = h2f((uint16_t)(v[0] & 0xffff));
            d1 = h2f((uint16_t)(v[8] >> 16));
        }
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
    chunk_stats<GRP, 2, false>(s, ok, true, c, h0, ch, wm, wl);
}

// ------------------------------------------------------------ V partials --
// o[g][e] (elements 8q .. 8q+7, on lanes with r = 0) = sum over the wave's 32
// positions of w_j * V_j: each lane sums its rows in order, then the VR row
// classes are added in order (r = 0, 1, ...).  Positions past the last one
// carry weight 0 (their rows are the last row again).
template <int GRP, int HD>
__device__ __forceinline__ void v_accum_f16(const uint4 (&vq)[16], const float (*wts)[ATT_CHUNK], float (&o)[GRP][8],
                                            uint4 nr = uint4{}, int j0 = 0, int p = -1) {
    using G = VGeo<HD>;
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63, r = lane / G::VS;
#pragma unroll
    for (int g = 0; g < GRP; g++)
#pragma unroll
        for (int e = 0; e < 8; e++) o[g][e] = 0.0f;
#pragma unroll
    for (int i = 0; i < G::NV; i++) {
        uint4 row = vq[i];
        new_row1<HD>(row, nr, j0, i, p);                             // p >= 0: the new value row of position p
        const uint32_t w32[4] = {row.x, row.y, row.z, row.w};
        float v[8];
#pragma unroll
        for (int e = 0; e < 4; e++) {
            v[2 * e] = h2f((uint16_t)(w32[e] & 0xffff));
            v[2 * e + 1] = h2f((uint16_t)(w32[e] >> 16));
        }
#pragma unroll
        for (int g = 0; g < GRP; g++) {
            const float w = wts[g][wave * 32 + i * G::VR + r];
#pragma unroll
            for (int e = 0; e < 8; e++) o[g][e] = __builtin_fmaf(w, v[e], o[g][e]);
        }
    }
    // the VR row classes (lanes VS apart, same slot) by a butterfly over them;
    // the exchanges are exact lane ^ 8 / 16 / 32, since the lanes of a class
    // hold different elements
#pragma unroll
    for (int g = 0; g < GRP; g++)
#pragma unroll
        for (int e = 0; e < 8; e++) {
            float sum = o[g][e];
            if constexpr (G::VS <= 8) sum += xor8(sum);
            if constexpr (G::VS <= 16) sum += partner<16>(sum);
            sum += partner<32>(sum);
            o[g][e] = sum;
        }
}

// the four waves' partials added in order into P[h][ch][hd]
template <int GRP, int HD, bool AG>
__device__ __forceinline__ void v_partial_store(const float (&o)[GRP][8], float (*part)[GRP][256], const AttnCtx &c, int h0,
                                                int ch) {
    using G = VGeo<HD>;
    constexpr int hd = HD;
    const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
    if (lane < G::NS) {
#pragma unroll
        for (int g = 0; g < GRP; g++) {
            *(float4 *)&part[wave][g][8 * lane] = make_float4(o[g][0], o[g][1], o[g][2], o[g][3]);
            *(float4 *)&part[wave][g][8 * lane + 4] = make_float4(o[g][4], o[g][5], o[g][6], o[g][7]);
        }
    }
    __syncthreads();
    for (int i = t; i < GRP * hd; i += 256) {
        const int g = i / hd, e = i - g * hd;
        const float r = ((part[0][g][e] + part[1][g][e]) + part[2][g][e]) + part[3][g][e];
        float *dst = &c.P[((size_t)(h0 + g) * c.nc + ch) * hd + e];
        if constexpr (AG) st_ag(dst, r);
        else *dst = r;
    }
}

// q8_0 / q4_0 V path: lane owns elements 4*lane .. 4*lane+3; the four waves'
// partials added in order into P[h][ch][hd]
template <int GRP, int HD>
__device__ __forceinline__ void v_partial_store4(const float (&o)[GRP][4], float (*part)[GRP][256], const AttnCtx &c, int h0,
                                                 int ch) {
    constexpr int hd = HD;
    const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
    if (4 * lane < hd) {
#pragma unroll
        for (int g = 0; g < GRP; g++)
            *(float4 *)&part[wave][g][4 * lane] = make_float4(o[g][0], o[g][1], o[g][2], o[g][3]);
    }
    __syncthreads();
    for (int i = t; i < GRP * hd; i += 256) {
        const int g = i / hd, e = i - g * hd;
        c.P[((size_t)(h0 + g) * c.nc + ch) * hd + e] = ((part[0][g][e] + part[1][g][e]) + part[2][g][e]) + part[3][g][e];
    }
}

// grid (n_kv, chunks of 128), 256 threads.  M and the normaliser from the
// chunk statistics; the chunk's weights go to LDS once; each wave then
// accumulates w_j * V_j over its 32 positions (all V loads of the lane issued
// up front), lane owning 4 consecutive elements; the waves add in order into
// the partial P[h][c][hd].
template <int KV, int GRP, int HD>
__global__ __launch_bounds__(256) void k_attn_v(AttnCtx c) {
    __shared__ float part[4][GRP][256];
    __shared__ __align__(16) float wl[GRP][ATT_CHUNK];
    __shared__ float inv_s[GRP], max_s[GRP];
    attn_token(c);
    const int npos = attn_view(c);
    const int kvh = blockIdx.x, ch = blockIdx.y, t = threadIdx.x, lane = t & 63, wave = t >> 6;
    constexpr int hd = HD;
    const int n_kv = c.a.n_kv, h0 = kvh * GRP;
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
    // 2. the V rows (f16: 16-byte loads, see v_rows_load; q8_0 / q4_0: below, lane
    // owning elements 4*lane .. 4*lane+3, lanes beyond hd/4 idle)
    const bool lane_ok = 4 * lane < hd;
    uint4 vq[16];
    if constexpr (KV == F16) rows_load<HD>(vq, c.a.vc, n_kv, kvh, j0, npos);
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
            wl[g][pp] = ch * ATT_CHUNK + pp >= npos ? 0.0f : KV == F16 ? h2f(f2h(w)) : w;
        }
    }
    __syncthreads();
    if constexpr (KV == F16) {
        float o[GRP][8];
        v_accum_f16<GRP, HD>(vq, wl, o);
        v_partial_store<GRP, HD, false>(o, part, c, h0, ch);
    } else {
        float o[GRP][4];
#pragma unroll
        for (int g = 0; g < GRP; g++)
#pragma unroll
            for (int e = 0; e < 4; e++) o[g][e] = 0.0f;
        for (int k = 0; k < 32; k++) {
            const int j = j0 + k;
            if (j >= npos) break;
            if (lane_ok) {
                // the lane's 4 elements, dequantized as g4_dequant_row does (quants.c:364-378)
                constexpr int BS = KV == Q4_0 ? 18 : 34;
                const uint8_t *blk = c.a.vc + ((size_t)j * n_kv + kvh) * (hd / 32) * BS + (lane >> 3) * BS;
                const float d = h2f((uint16_t)(blk[0] | (blk[1] << 8)));
                float v[4];
#pragma unroll
                for (int e = 0; e < 4; e++) {
                    const int jj = 4 * (lane & 7) + e;                       // element of the block
                    if constexpr (KV == Q4_0) {
                        const int nib = jj < 16 ? (blk[2 + jj] & 15) : (blk[2 + jj - 16] >> 4);
                        v[e] = (float)(nib - 8) * d;
                    } else {
                        v[e] = (float)(int8_t)blk[2 + jj] * d;
                    }
                }
#pragma unroll
                for (int g = 0; g < GRP; g++) {
                    const float w = wl[g][wave * 32 + k];
#pragma unroll
                    for (int e = 0; e < 4; e++) o[g][e] = __builtin_fmaf(w, v[e], o[g][e]);
                }
            }
        }
        v_partial_store4<GRP, HD>(o, part, c, h0, ch);
    }
}

// -------------------------------------------------------------- combine --
// out[h][e] = sum over chunks in order (32 loads of a thread issued before the
// adds); with q8out, the head row is also quantized to q8_0.  256 threads.
template <bool AG>
__device__ __forceinline__ void combine_head(const AttnCtx &c, int h, int nch, float *row) {
    const int e = threadIdx.x, hd = c.a.hd;
    if (e < hd) {
        const float *p = c.P + (size_t)h * c.nc * hd + e;
        // chunk order of the one-launch combine: groups of ATT_CSUM chunks,
        // each summed in order, then the group sums in order
        float r = 0.0f;
        for (int k0 = 0; k0 < nch; k0 += ATT_CSUM) {
            float v[ATT_CSUM];
#pragma unroll
            for (int k = 0; k < ATT_CSUM; k++) {
                const size_t kk = (size_t)min(k0 + k, nch - 1) * hd;
                const float x = AG ? ld_ag(p + kk) : p[kk];
                v[k] = k0 + k < nch ? x : 0.0f;
            }
            float sg = 0.0f;
#pragma unroll
            for (int k = 0; k < ATT_CSUM; k++) sg += v[k];
            r += sg;
        }
        c.out[(size_t)h * hd + e] = r;
        row[e] = r;
    }
    if (c.q8out) {                                                   // uniform
        __syncthreads();
        const bool own = e < hd / 4;
        float v[4] = {0.f, 0.f, 0.f, 0.f};
        if (own)
            for (int k = 0; k < 4; k++) v[k] = row[4 * e + k];
        if (e < 64) q8_store4(v, e, own, c.q8out + (size_t)h * (hd / 32) * 34);
        __syncthreads();                                             // row is reused for the next head
    }
}

// grid n_head (x tokens)
__global__ __launch_bounds__(256) void k_attn_combine(AttnCtx c) {
    __shared__ float row[256];
    attn_token(c);
    const int npos = attn_view(c);
    combine_head<false>(c, blockIdx.x, (npos + ATT_CHUNK - 1) / ATT_CHUNK, row);
}

// ------------------------------------------------------------ fused (f16) --
// The three passes in one launch for an f16 cache, on a grid (KV head, chunk)
// that the device holds resident all at once (the host checks occupancy).
// A workgroup loads its chunk's K rows, computes the scores and chunk
// statistics as the score pass does and publishes m_c and l_c; its V loads
// go out next, so they stream while the other chunks' statistics arrive.  It
// then reads every chunk's statistics of its heads, forms the weights and
// value partial as the V pass does and publishes the partial.  Finally all
// workgroups of the KV head (chunks past the last position included) share
// the combine: 32-element blocks of its output rows, each summed over the
// chunks in order and, with q8out, quantized to one q8_0 block.
//
// Hand-off without counters: every published value is a 64-bit word, the
// value's bits low and the launch's tag high, stored at agent scope (coherent
// across the XCDs' L2 caches).  A 64-bit store is single-copy atomic, so a
// reader that sees the current tag sees the value stored with it; readers poll
// until every word they need carries the tag.  Tags never repeat on one
// workspace (see AttnCtx::tag).  A poll gives up after AttnCtx::spin retries
// (ATT_SPIN_LIMIT): the workgroup writes NaN into the outputs it owns and sets
// the error word, so the launch always ends and the host sees the failure
// (g4h_attn_status, g4h_model_status).  A test hook makes every poll wait for
// a tag that no store carries, with a short limit, so the failure path runs
// deterministically while every kernel still ends.  Same arithmetic as the three passes: outputs are
// bit-identical to theirs.
constexpr unsigned ATT_SPIN_LIMIT = 1u << 20;
constexpr int ATT_FUSED_MAXC = 128;  // chunks per KV head (two per lane)
// words per (head, chunk) statistics record: its three tagged words alone in a
// 128-byte line.  Measured: 64 workgroups polling words that share lines with
// other writers see the last store about 2.0 us late, 0.75 us with one writer
// per line.
constexpr int ATT_TW = 16;

__device__ __forceinline__ uint32_t tag_of(const AttnCtx &c) { return *c.epoch * c.tag_mul + c.tag_add + 1u; }

// the attention rows (queries, and the new key / value in the chunk of the
// current position) from the projection's tagged words, for prep_f16_finish
template <int GRP, int HD>
__device__ __forceinline__ bool prep_f16_poll(PrepF16<GRP> &st, const AttnCtx &c, int kvh, uint32_t tag) {
    constexpr int hd = HD, epl = hd >> 6;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, h0 = kvh * GRP;
    bool ok = true;
#pragma unroll
    for (int sl = 0; sl < PrepF16<GRP>::SL; sl++) {
        const int r = wave + 4 * sl;
        if (r < st.nrow) {                                            // uniform over the wave
            const int src_row = r < GRP ? h0 + r : r == GRP ? c.a.n_head + kvh : c.a.n_head + c.a.n_kv + kvh;
            const uint64_t *src[4];
            bool need[4];
            uint32_t bits[4];
#pragma unroll
            for (int e = 0; e < 4; e++) {
                src[e] = c.QT + (size_t)src_row * hd + lane * epl + min(e, epl - 1);
                need[e] = e < epl;
            }
            ok &= poll_words<4>(src, need, tag ^ c.poll_xor, bits, c.spin);
#pragma unroll
            for (int e = 0; e < 4; e++) st.pr[sl].v[e] = e < epl ? __uint_as_float(bits[e]) : 0.0f;
        }
    }
    return ok;
}

// The projection rows of this workgroup (QKV launches): rows L*qrows .. of W,
// in passes of 4 waves x 64/LPR rows; a row's lanes, units and reduction are
// those of k_gemv / k_gemv_p with the same LPR, so each row is bit-identical to
// theirs.  The first two passes' weights are issued by qkv_issue (before the
// K stream), later passes (small models only) after it.
template <class FQ, int LPR, int UPL>
struct QkvRows {
    static constexpr int RPW = 64 / LPR;
    typename FQ::Frag fa[UPL], fb[UPL];
    int units;
    __device__ __forceinline__ int64_t row_of(const AttnCtx &c, int L, int pass) const {
        const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
        return (int64_t)L * c.qrows + pass * 4 * RPW + wave * RPW + lane / LPR;
    }
    __device__ __forceinline__ void load(typename FQ::Frag (&fr)[UPL], const AttnCtx &c, int L, int pass) const {
        const int g = (threadIdx.x & 63) % LPR;
        const int64_t row = min(row_of(c, L, pass), c.W.nrows - 1);
#pragma unroll
        for (int k = 0; k < UPL; k++) FQ::load(fr[k], c.W, row, min(g + k * LPR, units - 1));
    }
    __device__ __forceinline__ void finish(const typename FQ::Frag (&fr)[UPL], const AttnCtx &c, int L, int pass,
                                           const uint8_t *act, uint32_t tag) const {
        const int g = (threadIdx.x & 63) % LPR;
        float acc = 0.0f;
        const typename FQ::Act A(const_cast<uint8_t *>(act), (int)c.W.nb, 0);
#pragma unroll
        for (int k = 0; k < UPL; k++) {
            const int u = g + k * LPR;
            if (u < units) acc = FQ::accum(fr[k], A, u, acc);
        }
        acc = group_sum<LPR>(acc);
        const int64_t row = row_of(c, L, pass);
        if (g == 0 && row < c.W.nrows && row < (int64_t)(L + 1) * c.qrows) st_tag(&c.QT[row], __float_as_uint(acc), tag);
    }
};

constexpr int ATT_WO_MAXB = 64;      // q8_0 blocks of the attention output the Wo fold takes (n_head * hd <= 2048)

template <int GRP, int HD, class FQ = void, int LPR = 32, int UPL = 4, class FO = void, int LPRO = 16, int UPLO = 4>
__global__ __launch_bounds__(256) void k_attn_fused_f16(AttnCtx c) {
    constexpr bool QKV = !std::is_void<FQ>::value;
    constexpr bool WO = !std::is_void<FO>::value;
    extern __shared__ __align__(16) uint8_t act_lds[];               // QKV: the projection's q8_0 activation
    __shared__ __align__(16) float4 qf[GRP][64];
    __shared__ __align__(16) uint16_t kpos[256], vpos[256];
    __shared__ float wm[4][GRP];
    __shared__ double wl[4][GRP];
    __shared__ __align__(16) float wts[GRP][ATT_CHUNK];
    __shared__ float sc[GRP][ATT_CHUNK];
    __shared__ float inv_s[GRP], max_s[GRP];
    __shared__ __align__(16) float part[4][GRP][256];
    __shared__ float vals[ATT_FUSED_MAXC * 32];                      // combine: [chunk][32]
    __shared__ float gsum[ATT_FUSED_MAXC / ATT_CSUM * 32];           // combine: [chunk group][32]
    __shared__ int bad;
    const int npos = attn_view(c);
    const uint32_t tag = tag_of(c);
    const int kvh = blockIdx.x, ch = blockIdx.y, t = threadIdx.x;
    const int lane = t & 63, wave = t >> 6;
    constexpr int hd = HD;
    const int h0 = kvh * GRP, p = npos - 1;
    const int nch = (npos + ATT_CHUNK - 1) / ATT_CHUNK;
    const bool live = ch < nch;                                      // uniform over the workgroup
    if (t == 0) bad = 0;
    // a launch on a workspace whose error word is still set (an earlier launch
    // gave up and no status call has cleared it) writes NaN: a workgroup of
    // that launch which started after its last workgroup advanced the epoch
    // took this launch's tag, and its words may be read as this launch's
    const bool stale = c.adv && ld_ag(c.err) != 0u;
    if (c.adv && t == 0) st_tag(c.SW + ((size_t)ch * gridDim.x + kvh), 0u, tag);
    const int j0 = ch * ATT_CHUNK + wave * 32, j = j0 + lane;      // lane < 32 owns position j
    const bool pos_chunk = (QKV || c.qkv) && ch == p / ATT_CHUNK;
    PrepF16<GRP> st;
    uint4 kq[16], vq[16];
    constexpr bool v_first = QKV && ATT_QKV_VFIRST;                   // V issued with K, before the projection poll
    if constexpr (QKV) {
        // the projection: prologue loads and the norm / RoPE rows, then its
        // weights, then the K stream; the prologue arithmetic and the rows
        // run while K streams, and the attention rows come back through QT
        // (that poll completes behind the K rows, which the scores need next)
        const int L = blockIdx.y * gridDim.x + blockIdx.x;
        constexpr int S = 4;                                          // prologue groups of 4 per thread
        ProLoads pr;
        QkvRows<FQ, LPR, UPL> qr;
        qr.units = (int)(c.W.nb * FQ::units_per_block);
        const int np = (c.qrows + 4 * qr.RPW - 1) / (4 * qr.RPW);
        if (live) prep_f16_issue_w<GRP, HD>(st, c, kvh, p, pos_chunk);
        pro_issue<PRO_NORM, S>(pr, c.pro);
        if (ATT_QKV_WAIT) wait_loads();                               // landed before the streams queue up
        issue_barrier();
        qr.load(qr.fa, c, L, 0);
        qr.load(qr.fb, c, L, 1);                                      // unconditional: a load under a branch is waited for there
        issue_order();
        if (!ATT_QKV_KLATE) {
            if (live) rows_load<HD>(kq, c.a.kc, c.a.n_kv, kvh, j0, npos);
            if (v_first && live) rows_load<HD>(vq, c.a.vc, c.a.n_kv, kvh, j0, npos);
            issue_order();
        }
        pro_finish<PRO_NORM, S>(pr, c.pro, act_lds, (int)c.W.nb, L == 0);
        lds_barrier();
        if (ATT_QKV_KLATE) {                                          // K (and V) behind the prologue arithmetic
            if (live) rows_load<HD>(kq, c.a.kc, c.a.n_kv, kvh, j0, npos);
            if (v_first && live) rows_load<HD>(vq, c.a.vc, c.a.n_kv, kvh, j0, npos);
            issue_order();
        }
        qr.finish(qr.fa, c, L, 0, act_lds, tag);
        if (np > 1) qr.finish(qr.fb, c, L, 1, act_lds, tag);
        for (int pass = 2; pass < np; pass++) {                       // uniform; small models only
            qr.load(qr.fa, c, L, pass);
            qr.finish(qr.fa, c, L, pass, act_lds, tag);
        }
        if (live && !prep_f16_poll<GRP, HD>(st, c, kvh, tag)) bad = 1;
    } else if (live) {
        // the small loads first (landed before the streams start), then the
        // wave's K rows
        prep_f16_issue<GRP, HD>(st, c, kvh, p, pos_chunk);
        wait_loads();
        rows_load<HD>(kq, c.a.kc, c.a.n_kv, kvh, j0, npos);
        issue_order();
    }
    if (live) {
        const bool mine = lane < 32;
        float s[GRP];
        {
            // each V row is issued once the K row it follows has been scored,
            // so the scores start with the first K row and V streams behind K
            // while the statistics proceed
            prep_f16_finish<GRP, HD>(st, c, kvh, p, qf, kpos, vpos);
            lds_barrier();
            float qv[GRP][8];
            q_slot<GRP, HD>(qf, qv);
            const uint4 nk = new_row_slot<HD>(kpos);
#pragma unroll
            for (int i = 0; i < VGeo<HD>::NV; i++) {
                new_row1<HD>(kq[i], nk, j0, i, pos_chunk ? p : -1);  // the new key, not the stale cache row
                score_row<GRP, HD>(kq[i], qv, sc, i);
                if (!v_first && i < ATT_V_EARLY) vq[i] = row_load<HD>(c.a.vc, c.a.n_kv, kvh, j0, i, npos);
                issue_order();
            }
            lds_barrier();
#pragma unroll
            for (int g = 0; g < GRP; g++) s[g] = mine ? sc[g][wave * 32 + lane] : 0.0f;
        }
        // chunk statistics (as chunk_stats), published as tagged words
        const bool ok = mine && j < npos, once = mine;
#pragma unroll
        for (int g = 0; g < GRP; g++) {
            const float m = wave_max(ok ? s[g] : -INFINITY);
            if (lane == 0) wm[wave][g] = m;
        }
        lds_barrier();
#pragma unroll
        for (int g = 0; g < GRP; g++) {
            float mc = wm[0][g];
            for (int w = 1; w < 4; w++) mc = fmaxf(mc, wm[w][g]);
            const double e = ok && once ? exp((double)(s[g] - mc)) : 0.0;
            const double l = wave_sum_d(e);
            if (lane == 0) wl[wave][g] = l;
        }
        lds_barrier();
        if (t < GRP) {
            const int g = t;
            float mc = wm[0][g];
            for (int w = 1; w < 4; w++) mc = fmaxf(mc, wm[w][g]);
            double l = 0.0;
            for (int w = 0; w < 4; w++) l += wl[w][g];
            uint64_t *w3 = c.T + ((size_t)(h0 + g) * c.nc + ch) * ATT_TW;
            const uint64_t lb = (uint64_t)__double_as_longlong(l);
            st_tag(w3, __float_as_uint(mc), tag);
            st_tag(w3 + 1, (uint32_t)lb, tag);
            st_tag(w3 + 2, (uint32_t)(lb >> 32), tag);
        }
        // every chunk's statistics: global maximum and normaliser (as the V pass)
        constexpr int HPW = (GRP + 3) / 4;
#pragma unroll
        for (int q = 0; q < HPW; q++) {
            const int g = wave + 4 * q;
            if (g < GRP) {                                           // uniform over the wave
                const uint64_t *w3 = c.T + (size_t)(h0 + g) * c.nc * ATT_TW;
                const uint64_t *src[6];
                bool need[6];
                uint32_t bits[6];
#pragma unroll
                for (int r = 0; r < 2; r++)
#pragma unroll
                    for (int k = 0; k < 3; k++) {
                        const int ci = 64 * r + lane;
                        src[3 * r + k] = w3 + (size_t)min(ci, nch - 1) * ATT_TW + k;
                        need[3 * r + k] = ci < nch;
                    }
                if (!poll_words<6>(src, need, tag ^ c.poll_xor, bits, c.spin)) bad = 1;
                float mc[2];
                double lc[2];
#pragma unroll
                for (int r = 0; r < 2; r++) {
                    const bool on = 64 * r + lane < nch;
                    mc[r] = on ? __uint_as_float(bits[3 * r]) : -INFINITY;
                    lc[r] = on ? __longlong_as_double((long long)(((uint64_t)bits[3 * r + 2] << 32) | bits[3 * r + 1])) : 0.0;
                }
                float m = wave_max(mc[0]);
                if (nch > 64) m = fmaxf(m, wave_max(mc[1]));
                double sum = wave_sum_d(lane < nch ? lc[0] * exp((double)mc[0] - (double)m) : 0.0);
                if (nch > 64) sum += wave_sum_d(64 + lane < nch ? lc[1] * exp((double)mc[1] - (double)m) : 0.0);
                if (lane == 0) {
                    inv_s[g] = (float)(1.0 / sum);
                    max_s[g] = m;
                }
            }
        }
        lds_barrier();
        // the rest of V, behind the statistics hand-off (a CU returns loads in
        // issue order, so V rows issued before the poll would delay it); the
        // weights are formed while these rows land
#pragma unroll
        for (int i = ATT_V_EARLY; i < VGeo<HD>::NV; i++)
            if (!v_first) vq[i] = row_load<HD>(c.a.vc, c.a.n_kv, kvh, j0, i, npos);
        issue_order();
        if (mine) {
#pragma unroll
            for (int g = 0; g < GRP; g++) {
                const float e = (float)exp((double)((j < npos ? s[g] : 0.0f) - max_s[g]));
                wts[g][wave * 32 + lane] = j < npos ? h2f(f2h(e * inv_s[g])) : 0.0f;
            }
        }
        lds_barrier();
        // the chunk's value partial (as the V pass), published as tagged words
        float o[GRP][8];
        v_accum_f16<GRP, HD>(vq, wts, o, new_row_slot<HD>(vpos), j0, pos_chunk ? p : -1);
        if (lane < VGeo<HD>::NS) {
#pragma unroll
            for (int g = 0; g < GRP; g++) {
                *(float4 *)&part[wave][g][8 * lane] = make_float4(o[g][0], o[g][1], o[g][2], o[g][3]);
                *(float4 *)&part[wave][g][8 * lane + 4] = make_float4(o[g][4], o[g][5], o[g][6], o[g][7]);
            }
        }
        lds_barrier();
        for (int i = t; i < GRP * hd; i += 256) {
            const int g = i / hd, e = i - g * hd;
            const float r = ((part[0][g][e] + part[1][g][e]) + part[2][g][e]) + part[3][g][e];
            st_tag(&c.PT[((size_t)(h0 + g) * c.nc + ch) * hd + e], __float_as_uint(r), tag);
        }
    }
    // Wo fold: the wave's first row group of Wo goes out now, behind this
    // launch's K/V streams (their registers are free again), so it lands
    // during the hand-offs below; row groups gw, gw + NWV, ... of all waves
    using FW = std::conditional_t<WO, FO, FQ4_0>;                   // a frag type also when there is no fold
    constexpr int RPWO = 64 / LPRO;
    const int64_t gw = ((int64_t)blockIdx.y * gridDim.x + blockIdx.x) * 4 + wave;
    const int64_t NWV = (int64_t)gridDim.x * gridDim.y * 4;
    const int go = lane % LPRO, rgo = lane / LPRO;
    const int units_o = WO ? (int)(c.Wo.nb * FW::units_per_block) : 1;
    typename FW::Frag fo[UPLO];
    auto wo_load = [&](int64_t gq) __attribute__((always_inline)) {
        const int64_t row = min(gq * RPWO + rgo, c.Wo.nrows - 1);
#pragma unroll
        for (int k = 0; k < UPLO; k++) FW::load(fo[k], c.Wo, row, min(go + k * LPRO, units_o - 1));
    };
    if constexpr (WO) {
        wo_load(gw);
        issue_order();
    }
    // combine, shared by every workgroup of the KV head: blocks ch, ch + nwg, ...
    // of its GRP*hd outputs; thread (slot r = t / 32, element i = t % 32)
    // gathers chunks r, r + 8, ... into LDS, then 32 threads add them in chunk
    // order (as the combine pass)
    const int nblk = GRP * hd / 32, nwg = gridDim.y;
    for (int b = ch; b < nblk; b += nwg) {                           // uniform over the workgroup
        lds_barrier();
        const int g = (b * 32) / hd, e0 = b * 32 - g * hd, i = t & 31, r0 = t >> 5;
        const uint64_t *base = c.PT + (size_t)(h0 + g) * c.nc * hd + e0 + i;
        constexpr int PER = ATT_FUSED_MAXC / 8;                      // chunks per thread
        const uint64_t *src[PER];
        bool need[PER];
        uint32_t bits[PER];
#pragma unroll
        for (int q = 0; q < PER; q++) {
            const int k = r0 + 8 * q;
            src[q] = base + (size_t)min(k, nch - 1) * hd;
            need[q] = k < nch;
        }
        if (!poll_words<PER>(src, need, tag ^ c.poll_xor, bits, c.spin)) bad = 1;
#pragma unroll
        for (int q = 0; q < PER; q++)
            if (need[q]) vals[(r0 + 8 * q) * 32 + i] = __uint_as_float(bits[q]);
        lds_barrier();
        // groups of ATT_CSUM chunks summed in order by 8 thread rows (group
        // k of element i on thread row k % 8), then the group sums in order
        // by 32 threads.  Slots past the last chunk add +0, which leaves every
        // sum's bits unchanged (a sum of partials that start from +0 is never
        // -0); the reads are unconditional, since reads under a per-slot
        // condition each wait for LDS alone.
        const int ngrp = (nch + ATT_CSUM - 1) / ATT_CSUM;
        for (int gi = r0; gi < ngrp; gi += 8) {
            float v[ATT_CSUM];
#pragma unroll
            for (int q = 0; q < ATT_CSUM; q++) {
                const float x = vals[(gi * ATT_CSUM + q) * 32 + i];
                v[q] = gi * ATT_CSUM + q < nch ? x : 0.0f;
            }
            float sg = 0.0f;
#pragma unroll
            for (int q = 0; q < ATT_CSUM; q++) sg += v[q];
            gsum[gi * 32 + i] = sg;
        }
        lds_barrier();
        float r = 0.0f;
        if (t < 32) {
            for (int g0 = 0; g0 < ngrp; g0 += 8) {
                float v[8];
#pragma unroll
                for (int q = 0; q < 8; q++) {
                    const float x = gsum[min(g0 + q, ATT_FUSED_MAXC / ATT_CSUM - 1) * 32 + t];
                    v[q] = g0 + q < ngrp ? x : 0.0f;
                }
#pragma unroll
                for (int q = 0; q < 8; q++) r += v[q];
            }
            if (bad || stale) r = __builtin_nanf("");
            c.out[(size_t)(h0 + g) * hd + e0 + t] = r;
        }
        if (c.q8out || WO) {                                         // uniform
            lds_barrier();
            if (t < 32) vals[t] = r;
            lds_barrier();
            if (t < 8) {
                float v4[4];
#pragma unroll
                for (int k = 0; k < 4; k++) v4[k] = vals[4 * t + k];
                if constexpr (WO) {
                    // the block as tagged words: quant words 0..7, the fp16 scale in word 8
                    uint16_t d16;
                    const uint32_t pk = q8_pack4(v4, &d16);
                    uint64_t *qo = c.QO + ((size_t)(h0 + g) * (hd / 32) + e0 / 32) * 16;
                    st_tag(qo + t, pk, tag);
                    if (t == 0) st_tag(qo + 8, d16, tag);
                } else {
                    q8_store4(v4, t, true, c.q8out + (size_t)(h0 + g) * (hd / 32) * 34 + (size_t)(e0 / 32) * 34);
                }
            }
        }
    }
    if constexpr (WO) {
        // every workgroup: all blocks of the head rows (9 tagged words each)
        // into the GEMV family's q8_0 activation layout in LDS, then its waves'
        // Wo row groups (the lanes, units and reduction of k_gemv with this
        // LPR / UPL, so each row has the bits of the separate Wo launch)
        __shared__ uint32_t wo_raw[WO ? ATT_WO_MAXB * 9 : 1];
        __shared__ __align__(16) uint8_t wo_act[WO ? ATT_WO_MAXB * 40 : 16];
        const int nbo = (int)c.Wo.nb, nw = nbo * 9;
        for (int i0 = 0; i0 < nw; i0 += 4 * 256) {                    // uniform
            const uint64_t *src[4];
            bool need[4];
            uint32_t bits[4];
#pragma unroll
            for (int q = 0; q < 4; q++) {
                const int i = i0 + q * 256 + t, ic = min(i, nw - 1);
                src[q] = c.QO + (size_t)(ic / 9) * 16 + ic % 9;
                need[q] = i < nw;
            }
            if (!poll_words<4>(src, need, tag ^ c.poll_xor, bits, c.spin)) bad = 1;
#pragma unroll
            for (int q = 0; q < 4; q++)
                if (need[q]) wo_raw[i0 + q * 256 + t] = bits[q];
        }
        lds_barrier();
        const ActQ8_0 A(wo_act, nbo, 0);
        for (int k = t; k < nbo; k += 256) {
            const uint32_t *w9 = wo_raw + 9 * k;
            const int4 a0 = make_int4(w9[0], w9[1], w9[2], w9[3]), a1 = make_int4(w9[4], w9[5], w9[6], w9[7]);
            A.q0[k] = a0;
            A.q1[k] = a1;
            A.d[k] = h2f((uint16_t)(w9[8] & 0xffff));
            A.s[k] = sum_i8x16(a0) + sum_i8x16(a1);
        }
        lds_barrier();
        const int64_t ngo = (c.Wo.nrows + RPWO - 1) / RPWO;
        for (int64_t gq = gw; gq < ngo; gq += NWV) {                   // wave-uniform
            if (gq != gw) wo_load(gq);
            float acc = 0.0f;
#pragma unroll
            for (int k = 0; k < UPLO; k++) {
                const int u = go + k * LPRO;
                if (u < units_o) acc = FW::accum(fo[k], A, u, acc);
            }
            acc = group_sum<LPRO>(acc);
            const int64_t row = gq * RPWO + rgo;
            if (go == 0 && row < c.Wo.nrows) c.wo_out[row] = bad || stale ? __builtin_nanf("") : acc;
        }
    }
    if (c.adv && kvh == (int)gridDim.x - 1 && ch == (int)gridDim.y - 1) {   // uniform over the workgroup
        // every workgroup of the launch has read the epoch word: advance it
        // (also after a poll gave up, so that tags never repeat)
        const int nwg = (int)(gridDim.x * gridDim.y);
        for (int i0 = 0; i0 < nwg; i0 += 4 * 256) {                  // uniform
            const uint64_t *src[4];
            bool need[4];
            uint32_t bits[4];
#pragma unroll
            for (int q = 0; q < 4; q++) {
                const int i = i0 + q * 256 + t;
                src[q] = c.SW + min(i, nwg - 1);
                need[q] = i < nwg;
            }
            if (!poll_words<4>(src, need, tag ^ c.poll_xor, bits, c.spin)) bad = 1;
        }
        lds_barrier();
        if (t == 0) st_ag(c.adv, tag);                              // the epoch this launch's tag follows
    }
    // any poll of this workgroup that gave up (its partials or outputs are not
    // valid) is reported, whether or not it owned a combine block
    lds_barrier();
    if (t == 0 && bad) st_ag(c.err, 1u);
}

// ------------------------------------------------------------- KV store --
// model.c:583-589: an f16 row (RNE) or q8_0 / q4_0 blocks per head row.
__global__ __launch_bounds__(256) void k_kv_store_f16(const float *__restrict__ src, uint16_t *__restrict__ dst, int n) {
    const int i = blockIdx.x * 256 + threadIdx.x;
    if (i < n) dst[i] = f2h(src[i]);
}

// ------------------------------------------------------------ launchers --
// zero the tagged words and the epoch / error words (their first use)
__global__ void k_attn_clear(uint64_t *w, size_t n) {
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x) w[i] = 0;
}

// Workspace: the error word (offset 0, the same for every shape, sticky until
// g4h_attn_status reads it), S [n_head][npos] f32 scores, Mc [n_head][nc] f32
// chunk maxima, Lc [n_head][nc] f64 chunk sums, P [n_head][nc][hd] f32
// partials (three passes); then the fused launch's epoch word and its tagged
// words T [n_head][nc][ATT_TW] (3 used) and PT [n_head][nc][hd].
static size_t al256(size_t v) { return (v + 255) & ~(size_t)255; }
struct AttnWs {
    size_t err, S, Mc, Lc, P, epoch, T, PT, QO, SW, total;
};
static AttnWs attn_ws(int n_head, int hd, int npos_max) {
    const size_t nc = (npos_max + ATT_CHUNK - 1) / ATT_CHUNK;
    AttnWs w;
    w.err = 0;
    w.S = 256;
    w.Mc = w.S + al256((size_t)n_head * npos_max * 4);
    w.Lc = w.Mc + al256((size_t)n_head * nc * 4);
    w.P = w.Lc + al256((size_t)n_head * nc * 8);
    w.epoch = w.P + al256((size_t)n_head * nc * hd * 4);
    w.T = w.epoch + 256;
    w.PT = w.T + al256((size_t)n_head * nc * ATT_TW * 8);
    w.QO = w.PT + al256((size_t)n_head * nc * hd * 8);
    w.SW = w.QO + al256((size_t)n_head * hd / 32 * 128);
    w.total = w.SW + al256((size_t)n_head * nc * 8);
    return w;
}

size_t attn_batch_workspace_bytes(int n_head, int hd, int npos_max, int nb);
size_t attn_workspace_bytes(int n_head, int hd, int npos_max) {
    if (hd == ATT_WIDE) return attn_batch_workspace_bytes(n_head, hd, npos_max, 1);   // the wide form's layout
    return attn_ws(n_head, hd, npos_max).total;
}

// The epoch word of calls without an external epoch sits at a fixed offset of
// the workspace header, so that it survives changes of layout (the layout
// follows the position count): every tagged word ever stored in a workspace
// carries a tag drawn from that one counter, at most its current value, so a
// launch's new tag matches no stale word wherever the regions fall.
constexpr size_t ATT_EPOCH_OFF = 128;
// Workspaces known to hold only zeros and such tagged words ("clean"): the
// first call on a workspace clears all of it (ws_bytes when known), a launch
// that writes untagged data into it (the three passes, the batch form) makes
// it unclean, and g4h_free drops it.  A clear recorded into a graph capture
// does not count, since it runs only with the graph.
static std::mutex g_ws_mu;
static std::map<uintptr_t, bool> g_ws_clean;
enum WsState { WS_READY, WS_CLEAR_TAGS, WS_CLEAR_ALL };
static WsState attn_ws_ready(const uint8_t *ws, hipStream_t s) {
    hipStreamCaptureStatus st = hipStreamCaptureStatusNone;
    if (hipStreamIsCapturing(s, &st) != hipSuccess) st = hipStreamCaptureStatusNone;
    std::lock_guard<std::mutex> lk(g_ws_mu);
    const auto it = g_ws_clean.find((uintptr_t)ws);
    if (it != g_ws_clean.end() && it->second) return WS_READY;
    const WsState r = it == g_ws_clean.end() ? WS_CLEAR_ALL : WS_CLEAR_TAGS;   // a new workspace: its error word too
    g_ws_clean[(uintptr_t)ws] = st == hipStreamCaptureStatusNone;   // the caller clears it now, in stream order
    return r;
}
void attn_ws_forget(const void *p) {
    std::lock_guard<std::mutex> lk(g_ws_mu);
    g_ws_clean.erase((uintptr_t)p);
}
static void attn_ws_untagged(const uint8_t *ws) {
    std::lock_guard<std::mutex> lk(g_ws_mu);
    const auto it = g_ws_clean.find((uintptr_t)ws);
    if (it != g_ws_clean.end()) it->second = false;
}

static unsigned g_attn_spin = ATT_SPIN_LIMIT;
static uint32_t g_attn_poll_xor = 0;
void attn_force_timeout(bool on) {
    g_attn_spin = on ? 64u : ATT_SPIN_LIMIT;
    g_attn_poll_xor = on ? 0x80000000u : 0u;
}
unsigned attn_spin_limit() { return g_attn_spin; }
uint32_t attn_poll_xor() { return g_attn_poll_xor; }

// workgroups of 256 threads of one kernel instantiation, with `lds` bytes of
// dynamic LDS, that the device holds resident at once (cached per instantiation
// and LDS size)
static int resident_capacity(const void *kernel, size_t lds) {
    static std::mutex mu;
    static std::map<std::pair<const void *, size_t>, int> cache;
    std::lock_guard<std::mutex> lk(mu);
    const auto key = std::make_pair(kernel, lds);
    const auto it = cache.find(key);
    if (it != cache.end()) return it->second;
    int dev = 0, cus = 0, occ = 0;
    int cap = 0;
    if (hipGetDevice(&dev) == hipSuccess && hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess &&
        hipOccupancyMaxActiveBlocksPerMultiprocessor(&occ, kernel, 256, lds) == hipSuccess)
        cap = cus * occ;
    cache[key] = cap;
    return cap;
}

// workgroups of the plain fused kernel the device holds resident at once
template <int GRP, int HD>
static int fused_capacity() {
    return resident_capacity(reinterpret_cast<const void *>(k_attn_fused_f16<GRP, HD>), 0);
}

template <int HD>
static int fused_capacity(int grp) {
    return grp == 1 ? fused_capacity<1, HD>() : grp == 2 ? fused_capacity<2, HD>() : grp == 4 ? fused_capacity<4, HD>()
         : grp == 8 ? fused_capacity<8, HD>() : 0;
}

bool attn_fused_fits(int kv_type, int n_head, int n_kv, int hd, int npos_max) {
    if (kv_type != F16) return false;
    if (const char *e = getenv("G4H_ATTN_PASSES"))
        if (atoi(e) == 3) return false;
    const int nc = (npos_max + ATT_CHUNK - 1) / ATT_CHUNK, grp = n_head / n_kv;
    if (nc > ATT_FUSED_MAXC) return false;
    const int cap = hd == 64 ? fused_capacity<64>(grp) : hd == 128 ? fused_capacity<128>(grp) : hd == 192 ? fused_capacity<192>(grp)
                  : hd == 256 ? fused_capacity<256>(grp) : 0;
    return (int64_t)n_kv * nc <= cap;
}

// ------------------------------------------------------------- Wo fold --
// The (type, LPR, UPL) shapes of the output projection the one-launch form
// takes (gemv_shape's choice for Wo; q4_0 / q8_0 rows of 256 and 2048), for
// groups of 2 query heads of 64 or 256.
#define G4_WO_SHAPES(X) X(FQ4_0, 16, 2) X(FQ4_0, 16, 4) X(FQ8_0, 16, 2) X(FQ8_0, 32, 2)

template <int GRP, int HD>
static hipError_t attn_wo_go(AttnCtx c, int n_kv, int nc, uint8_t *qo, hipStream_t s) {
    if constexpr (GRP == 2 && (HD == 64 || HD == 256)) {
        c.QO = (uint64_t *)qo;
        int lpr, upl;
        gemv_shape(c.Wo.type, c.Wo.nb, &lpr, &upl);
#define G4_WOL(F, L, U)                                                                                    \
        if (c.Wo.type == F::type && lpr == L && upl == U) {                                                 \
            hipLaunchKernelGGL((k_attn_fused_f16<GRP, HD, void, 32, 4, F, L, U>), dim3(n_kv, nc), dim3(256), 0, s, c); \
            return hipGetLastError();                                                                      \
        }
        G4_WO_SHAPES(G4_WOL)
#undef G4_WOL
    }
    return hipErrorInvalidValue;
}

template <int GRP, int HD>
static int wo_capacity(int wtype, int lpr, int upl) {
    if constexpr (GRP == 2 && (HD == 64 || HD == 256)) {
#define G4_WOC(F, L, U)                                                                                     \
        if (wtype == F::type && lpr == L && upl == U)                                                       \
            return resident_capacity(reinterpret_cast<const void *>(k_attn_fused_f16<GRP, HD, void, 32, 4, F, L, U>), 0);
        G4_WO_SHAPES(G4_WOC)
#undef G4_WOC
    }
    return 0;
}

bool attn_wo_fits(const g4h_tensor &Wo, const QkvArgs &a, int npos_max) {
    if (a.kv_type != F16 || a.window || a.ring || !attn_fused_fits(F16, a.n_head, a.n_kv, a.hd, npos_max)) return false;
    if (a.n_head / a.n_kv != 2 || (a.hd != 64 && a.hd != 256)) return false;
    if ((Wo.type != Q4_0 && Wo.type != Q8_0) || Wo.ncols != (int64_t)a.n_head * a.hd || Wo.nb > ATT_WO_MAXB) return false;
    int lpr, upl;
    gemv_shape(Wo.type, Wo.nb, &lpr, &upl);
    if (Wo.nb > (int64_t)lpr * upl) return false;                     // one pass over each row
    const int nc = (npos_max + ATT_CHUNK - 1) / ATT_CHUNK;
    const int cap = a.hd == 64 ? wo_capacity<2, 64>(Wo.type, lpr, upl) : wo_capacity<2, 256>(Wo.type, lpr, upl);
    return (int64_t)a.n_kv * nc <= cap;
}

template <int KV, int GRP, int HD>
static hipError_t attn_go(AttnCtx c, int n_head, int n_kv, int npos_max, uint8_t *ws, const AttnTag *tg, hipStream_t s,
                          size_t ws_bytes) {
    const AttnWs w = attn_ws(n_head, c.a.hd, npos_max);
    const int nc = (npos_max + ATT_CHUNK - 1) / ATT_CHUNK;
    c.nc = nc;
    c.S = (float *)(ws + w.S);
    c.Mc = (float *)(ws + w.Mc);
    c.Lc = (double *)(ws + w.Lc);
    c.P = (float *)(ws + w.P);
    if constexpr (KV == F16) {
        if (attn_fused_fits(KV, n_head, n_kv, HD, npos_max)) {
            c.T = (uint64_t *)(ws + w.T);
            c.PT = (uint64_t *)(ws + w.PT);
            c.err = (unsigned *)(ws + w.err);
            c.spin = g_attn_spin;
            c.poll_xor = g_attn_poll_xor;
            if (tg) {
                c.epoch = tg->epoch;
                c.tag_mul = tg->mul;
                c.tag_add = tg->add;
            } else {
                // the workspace's own epoch word, advanced by each launch
                const WsState ready = attn_ws_ready(ws, s);
                if (ready != WS_READY) {
                    const size_t from = ready == WS_CLEAR_ALL ? w.err : ATT_EPOCH_OFF;   // the error word of a new one too
                    const size_t nw = ((ws_bytes ? ws_bytes : w.total) - from) / 8;
                    hipLaunchKernelGGL(k_attn_clear, dim3((unsigned)std::min<size_t>((nw + 255) / 256, 1024)), dim3(256), 0, s,
                                       (uint64_t *)(ws + from), nw);
                }
                c.epoch = (const unsigned *)(ws + ATT_EPOCH_OFF);
                c.tag_mul = 1;
                c.tag_add = 0;
                c.adv = (unsigned *)(ws + ATT_EPOCH_OFF);
                c.SW = (uint64_t *)(ws + w.SW);
            }
            if (c.wo_out) return attn_wo_go<GRP, HD>(c, n_kv, nc, ws + w.QO, s);
            hipLaunchKernelGGL((k_attn_fused_f16<GRP, HD>), dim3(n_kv, nc), dim3(256), 0, s, c);
            return hipGetLastError();
        }
    }
    if (c.wo_out) return hipErrorInvalidValue;                        // the fold exists in the one-launch form only
    attn_ws_untagged(ws);                                            // scores, statistics and partials
    if constexpr (KV == F16) hipLaunchKernelGGL((k_attn_scores_f16<GRP, HD>), dim3(n_kv, nc), dim3(256), 0, s, c);
    else hipLaunchKernelGGL((k_attn_scores_q8<KV, GRP, HD>), dim3(n_kv, nc), dim3(128), 0, s, c);
    hipLaunchKernelGGL((k_attn_v<KV, GRP, HD>), dim3(n_kv, nc), dim3(256), 0, s, c);
    hipLaunchKernelGGL(k_attn_combine, dim3(n_head), dim3(256), 0, s, c);
    return hipGetLastError();
}

// ------------------------------------------------ causal batch (prefill) --
// nb tokens whose first attends npos0 positions, the last npos0 + nb - 1: the
// three passes once over grid.z = nb, each token with its own block of
// scores S, chunk statistics Mc / Lc and partials P sized for npos0 + nb - 1
// positions; chunks past a token's last position return at once.  Per token
// the arithmetic of the three passes, which the one-launch form shares: every
// token's rows are bit-identical to a decode call at its position.
struct AttnBatchWs {
    size_t S, Mc, Lc, P, tok;
};
static AttnBatchWs attn_batch_ws(int n_head, int hd, int npos_max) {
    const size_t nc = (npos_max + ATT_CHUNK - 1) / ATT_CHUNK;
    AttnBatchWs w;
    w.S = 0;
    w.Mc = al256((size_t)n_head * npos_max * 4);
    w.Lc = w.Mc + al256((size_t)n_head * nc * 4);
    w.P = w.Lc + al256((size_t)n_head * nc * 8);
    w.tok = w.P + al256((size_t)n_head * nc * hd * 4);
    return w;
}
// The batch blocks start after the decode layout's 256-byte header, so the
// error word (offset 0) and the epoch word (offset 128) of a workspace shared
// with the decode form keep their values.
constexpr size_t ATT_BATCH_OFF = 256;
// 512-wide heads run as twice the heads of 256 (attn_wide_go), plus the
// half-major query and output rows
static size_t wide_rows_bytes(int n_head, int nb) { return al256((size_t)nb * n_head * ATT_WIDE * 4); }
size_t attn_batch_workspace_bytes(int n_head, int hd, int npos_max, int nb) {
    if (hd == ATT_WIDE)
        return std::max(ATT_BATCH_OFF + (size_t)nb * attn_batch_ws(2 * n_head, ATT_HALF, npos_max).tok + 2 * wide_rows_bytes(n_head, nb),
                        attn_batch_mm_workspace_bytes(n_head, hd, npos_max, nb));
    return std::max(ATT_BATCH_OFF + (size_t)nb * attn_batch_ws(n_head, hd, npos_max).tok,
                    attn_batch_mm_workspace_bytes(n_head, hd, npos_max, nb));   // either form
}

template <int KV, int GRP, int HD>
static hipError_t attn_batch_go(AttnCtx c, int n_head, int n_kv, int npos0, int nb, uint8_t *ws, hipStream_t s) {
    // rows any token attends: all positions, or at most the window
    const int npos_max = c.a.window ? std::min(c.a.window, npos0 + nb - 1) : npos0 + nb - 1;
    const AttnBatchWs w = attn_batch_ws(n_head, c.a.hd, npos_max);
    const int nc = (npos_max + ATT_CHUNK - 1) / ATT_CHUNK;
    c.nc = nc;
    ws += ATT_BATCH_OFF;
    c.S = (float *)(ws + w.S);
    c.Mc = (float *)(ws + w.Mc);
    c.Lc = (double *)(ws + w.Lc);
    c.P = (float *)(ws + w.P);
    c.ntok = nb;
    c.ws_tok = w.tok;
    if (!c.q8_tok) c.q8_tok = (size_t)n_head * (c.a.hd / 32) * 34;
    const dim3 grid(n_kv, nc, nb);
    if constexpr (KV == F16) hipLaunchKernelGGL((k_attn_scores_f16<GRP, HD>), grid, dim3(256), 0, s, c);
    else hipLaunchKernelGGL((k_attn_scores_q8<KV, GRP, HD>), grid, dim3(128), 0, s, c);
    hipLaunchKernelGGL((k_attn_v<KV, GRP, HD>), grid, dim3(256), 0, s, c);
    hipLaunchKernelGGL(k_attn_combine, dim3(n_head, 1, nb), dim3(256), 0, s, c);
    return hipGetLastError();
}

// The rows of nb tokens prepared as the decode kernels prepare them
// (model.c:664-687, the preparation steps of k_attn_scores_* / the fused
// kernel): grid (token, KV head), one wave per row -- the group's queries
// (RMSNorm x q_norm, NeoX RoPE at pos0 + b) into q rows of qout, the key
// (RMSNorm x k_norm, RoPE) and value (RMSNorm) into the caches at pos0 + b.
// Runs before the batch attends, so every token finds the earlier tokens'
// rows in the caches.  On a ring (a.ring > 0) a row goes to slot p % ring and
// again to p % ring + ring, the two copies the decode kernels store; with a
// window and no ring, to slot p.  Within a batch of at most ring - window + 1
// tokens no token's store overwrites a row an earlier token of the batch
// still attends.
constexpr int PREP_MAXW = 10;                                        // one wave per row: GQA-8 groups + K + V
template <int HD>
__global__ __launch_bounds__(64 * PREP_MAXW) void k_attn_prep_rows(QkvArgs a, const float *__restrict__ qkv, int pos0,
                                                                   float *__restrict__ qout, const int *pos_dev) {
    if (pos_dev) pos0 = *pos_dev;
    constexpr int N = HD > 256 ? 8 : 4;                              // elements per lane held
    __shared__ float wb[PREP_MAXW][64 * N];                          // q8_0 / q4_0 stores
    constexpr int epl = HD >> 6;
    const int b = blockIdx.x, kvh = blockIdx.y, wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int grp = a.n_head / a.n_kv, h0 = kvh * grp, p = pos0 + b;
    const float *src = qkv + (size_t)b * (a.n_head + 2 * a.n_kv) * HD;
    const size_t rb = a.kv_type == F16 ? (size_t)HD * 2 : (size_t)(HD / 32) * (a.kv_type == Q4_0 ? 18 : 34);
    float cs[N], sn[N];
    rope_load(cs, sn, a.rope, p, HD);
    for (int r = wave; r < grp + 2; r += (int)(blockDim.x >> 6)) {   // uniform over the wave
        const int src_row = r < grp ? h0 + r : r == grp ? a.n_head + kvh : a.n_head + a.n_kv + kvh;
        const float *w = r < grp ? a.q_norm : r == grp ? a.k_norm : nullptr;
        PrepRowN<N> pr;
        prep_load(pr, src + (size_t)src_row * HD, w, HD);
        float y[N];
        prep_finish(pr, r <= grp, r <= grp, cs, sn, HD, a.eps, y);
        if (r < grp) {
#pragma unroll
            for (int e = 0; e < N; e++)
                if (e < epl) qout[((size_t)b * a.n_head + h0 + r) * HD + lane * epl + e] = y[e];
        } else {
            uint8_t *cache = r == grp ? a.kc : a.vc;
            const int slot = a.ring ? p % a.ring : p;
            cache_store(y, a.kv_type, cache + ((size_t)slot * a.n_kv + kvh) * rb, HD, wb[wave]);
            if (a.ring) cache_store(y, a.kv_type, cache + ((size_t)(slot + a.ring) * a.n_kv + kvh) * rb, HD, wb[wave]);
        }
    }
}

hipError_t launch_attn_prep_rows(const float *qkv, const QkvArgs &a, int pos0, int nb, float *qout, hipStream_t s,
                                 const int *pos_dev) {
    if (a.hd % 64 || (a.hd > 256 && a.hd != 512) || a.n_kv <= 0 || a.n_head % a.n_kv || nb < 1 || nb > 65535)
        return hipErrorInvalidValue;
    if (a.ring && (a.window <= 0 || a.window > a.ring || nb > a.ring - a.window + 1)) return hipErrorInvalidValue;
    if (!a.rope || !a.q_norm || !a.k_norm) return hipErrorInvalidValue;
    const dim3 grid(nb, a.n_kv), block(64 * std::min(a.n_head / a.n_kv + 2, PREP_MAXW));   // a wave per row
    if (a.hd == 64) hipLaunchKernelGGL(k_attn_prep_rows<64>, grid, block, 0, s, a, qkv, pos0, qout, pos_dev);
    else if (a.hd == 128) hipLaunchKernelGGL(k_attn_prep_rows<128>, grid, block, 0, s, a, qkv, pos0, qout, pos_dev);
    else if (a.hd == 192) hipLaunchKernelGGL(k_attn_prep_rows<192>, grid, block, 0, s, a, qkv, pos0, qout, pos_dev);
    else if (a.hd == 256) hipLaunchKernelGGL(k_attn_prep_rows<256>, grid, block, 0, s, a, qkv, pos0, qout, pos_dev);
    else hipLaunchKernelGGL(k_attn_prep_rows<512>, grid, block, 0, s, a, qkv, pos0, qout, pos_dev);
    return hipGetLastError();
}

static hipError_t attn_wide(const AttnCtx &c, int npos_max, int nb, uint8_t *ws, hipStream_t s);

hipError_t launch_attn_batch(const float *q, const QkvArgs &a, int npos0, int nb, float *out, uint8_t *q8out, uint8_t *ws,
                             hipStream_t s, size_t q8_stride) {
    if (a.hd % 64 || (a.hd > 256 && a.hd != ATT_WIDE) || a.n_kv <= 0 || a.n_head % a.n_kv || nb < 1 || npos0 < 1 || nb > 65535)
        return hipErrorInvalidValue;
    attn_ws_untagged(ws);                                            // blocks per token of untagged data
    AttnCtx c{};
    c.q = q;
    c.a = a;
    c.npos = npos0;
    c.out = out;
    c.q8out = q8out;
    c.q8_tok = q8_stride;
    if (a.hd == ATT_WIDE) return attn_wide(c, a.window ? std::min(a.window, npos0 + nb - 1) : npos0 + nb - 1, nb, ws, s);
    const int grp = a.n_head / a.n_kv;
#define G4_ATT(KV, G)                                                                        \
    if (a.kv_type == KV && grp == G) {                                                       \
        if (a.hd == 64) return attn_batch_go<KV, G, 64>(c, a.n_head, a.n_kv, npos0, nb, ws, s);   \
        if (a.hd == 128) return attn_batch_go<KV, G, 128>(c, a.n_head, a.n_kv, npos0, nb, ws, s); \
        if (a.hd == 192) return attn_batch_go<KV, G, 192>(c, a.n_head, a.n_kv, npos0, nb, ws, s); \
        if (a.hd == 256) return attn_batch_go<KV, G, 256>(c, a.n_head, a.n_kv, npos0, nb, ws, s); \
    }
    G4_ATT(F16, 1); G4_ATT(F16, 2); G4_ATT(F16, 4); G4_ATT(F16, 8);
    G4_ATT(Q8_0, 1); G4_ATT(Q8_0, 2); G4_ATT(Q8_0, 4); G4_ATT(Q8_0, 8);
    G4_ATT(Q4_0, 1); G4_ATT(Q4_0, 2); G4_ATT(Q4_0, 4); G4_ATT(Q4_0, 8);
#undef G4_ATT
    return hipErrorInvalidValue;
}

// ---------------------------------------------------- 512-wide heads --
// gemma4's full-attention heads are 512 wide over one KV head (g4run.h:283-292,
// model.c:530, 571).  They run on the 256-wide three passes as two halves:
// the cache rows [slot][512] are read as [slot][2][256], i.e. as two KV heads
// of 256, and the query rows are laid out half-major, [2][n_head][256], so the
// queries of half k fall on KV head k.  The score pass forms each half's
// partial dot; k_attn_wide_join adds the two (s = s_lo + s_hi: the f16 dot's
// fp32 order, which differs from the CPU's 8-lane order in rounding only) into
// the score rows of both halves and forms the chunk statistics of the sums
// (chunk_stats, as the score pass would), so the value passes of both halves
// take the same softmax weights, every output element's sum being that of a
// 256-wide head.  The outputs come back to [n_head][512].
__global__ __launch_bounds__(128) void k_attn_wide_rows(const float *__restrict__ src, float *__restrict__ dst, int n_head,
                                                        int to_halves) {
    // grid (n_head, nb): one 512-float row, a float4 per thread
    const int h = blockIdx.x, b = blockIdx.y, t = threadIdx.x, half = t >> 6, e = 4 * (t & 63);
    const size_t row = ((size_t)b * n_head + h) * ATT_WIDE + half * ATT_HALF + e;            // [b][h][half][e]
    const size_t hm = (((size_t)b * 2 + half) * n_head + h) * ATT_HALF + e;                  // [b][half][h][e]
    if (to_halves) *(float4 *)(dst + hm) = *(const float4 *)(src + row);
    else *(float4 *)(dst + row) = *(const float4 *)(src + hm);
}

template <int GRP>
__global__ __launch_bounds__(256) void k_attn_wide_join(AttnCtx c) {
    __shared__ float wm[4][GRP];
    __shared__ double wl[4][GRP];
    attn_token(c);
    const int npos = attn_view(c);
    const int ch = blockIdx.y, lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    if (ch * ATT_CHUNK >= npos) return;
    // lane l < 32 of wave w holds position ch * 128 + 32 w + l, as in the score pass
    const int j = ch * ATT_CHUNK + wave * 32 + lane;
    const bool ok = lane < 32 && j < npos;
    float s[GRP];
#pragma unroll
    for (int g = 0; g < GRP; g++) {
        float *lo = c.S + (size_t)g * npos + j, *hi = c.S + (size_t)(GRP + g) * npos + j;
        s[g] = ok ? *lo + *hi : 0.0f;
        if (ok) *lo = *hi = s[g];
    }
    chunk_stats<GRP, 4, false>(s, ok, lane < 32, c, 0, ch, wm, wl);
    chunk_stats<GRP, 4, false>(s, ok, lane < 32, c, GRP, ch, wm, wl);
}

// heads of 512 over one KV head: q rows prepared (no preparation, projection
// or Wo fold in this form), nb tokens as a batch (token b attends npos0 + b
// positions) or one token with a device position count (npos_dev)
template <int KV, int GRP>
static hipError_t attn_wide_go(AttnCtx c, int npos_max, int nb, uint8_t *ws, hipStream_t s) {
    const int H = c.a.n_head;
    const AttnBatchWs w = attn_batch_ws(2 * H, ATT_HALF, npos_max);
    const int nc = (npos_max + ATT_CHUNK - 1) / ATT_CHUNK;
    uint8_t *base = ws + ATT_BATCH_OFF;
    float *qh = (float *)(base + (size_t)nb * w.tok), *oh = (float *)((uint8_t *)qh + wide_rows_bytes(H, nb));
    float *out = c.out;
    c.nc = nc;
    c.S = (float *)(base + w.S);
    c.Mc = (float *)(base + w.Mc);
    c.Lc = (double *)(base + w.Lc);
    c.P = (float *)(base + w.P);
    c.ntok = nb;
    c.ws_tok = w.tok;
    c.a.n_head = 2 * H;
    c.a.n_kv = 2;
    c.a.hd = ATT_HALF;
    attn_ws_untagged(ws);
    hipLaunchKernelGGL(k_attn_wide_rows, dim3(H, nb), dim3(128), 0, s, c.q, qh, H, 1);
    c.q = qh;
    c.out = oh;
    const dim3 grid(2, nc, nb);
    if constexpr (KV == F16) hipLaunchKernelGGL((k_attn_scores_f16<GRP, ATT_HALF>), grid, dim3(256), 0, s, c);
    else hipLaunchKernelGGL((k_attn_scores_q8<KV, GRP, ATT_HALF>), grid, dim3(128), 0, s, c);
    hipLaunchKernelGGL((k_attn_wide_join<GRP>), dim3(1, nc, nb), dim3(256), 0, s, c);
    hipLaunchKernelGGL((k_attn_v<KV, GRP, ATT_HALF>), grid, dim3(256), 0, s, c);
    hipLaunchKernelGGL(k_attn_combine, dim3(2 * H, 1, nb), dim3(256), 0, s, c);
    hipLaunchKernelGGL(k_attn_wide_rows, dim3(H, nb), dim3(128), 0, s, oh, out, H, 0);
    return hipGetLastError();
}

static hipError_t attn_wide(const AttnCtx &c, int npos_max, int nb, uint8_t *ws, hipStream_t s) {
    const QkvArgs &a = c.a;
    if (a.n_kv != 1 || !c.q || c.qkv || c.q8out || c.wo_out) return hipErrorInvalidValue;
    const int grp = a.n_head;
#define G4_AW(KV, G) \
    if (a.kv_type == KV && grp == G) return attn_wide_go<KV, G>(c, npos_max, nb, ws, s)
    G4_AW(F16, 1); G4_AW(F16, 2); G4_AW(F16, 4); G4_AW(F16, 8);
    G4_AW(Q8_0, 1); G4_AW(Q8_0, 2); G4_AW(Q8_0, 4); G4_AW(Q8_0, 8);
    G4_AW(Q4_0, 1); G4_AW(Q4_0, 2); G4_AW(Q4_0, 4); G4_AW(Q4_0, 8);
#undef G4_AW
    return hipErrorInvalidValue;
}

// ------------------------------------------- projection + attention launch --
template <int GRP, int HD, class FQ, int LPR, int UPL>
static hipError_t attn_qkv_go(AttnCtx c, int npos_max, uint8_t *ws, hipStream_t s) {
    const AttnWs w = attn_ws(c.a.n_head, HD, npos_max);
    const int nc = (npos_max + ATT_CHUNK - 1) / ATT_CHUNK;
    const int nwg = c.a.n_kv * nc;
    c.nc = nc;
    c.T = (uint64_t *)(ws + w.T);
    c.PT = (uint64_t *)(ws + w.PT);
    c.err = (unsigned *)(ws + w.err);
    c.spin = g_attn_spin;
    c.poll_xor = g_attn_poll_xor;
    // rows per workgroup: a multiple of 16, so each workgroup's words fill whole 128-byte lines
    c.qrows = (int)(((c.W.nrows + nwg - 1) / nwg + 15) / 16 * 16);
    const size_t lds = ActQ8_0::bytes_per_token((int)c.W.nb) + kStageDump;
    hipLaunchKernelGGL((k_attn_fused_f16<GRP, HD, FQ, LPR, UPL>), dim3(c.a.n_kv, nc), dim3(256), lds, s, c);
    return hipGetLastError();
}

template <int GRP, int HD>
static hipError_t attn_qkv_fmt(const AttnCtx &c, int lpr, int upl, int npos_max, uint8_t *ws, hipStream_t s) {
#define G4_AQ(F, L, U) \
    if (lpr == L && upl == U) return attn_qkv_go<GRP, HD, F, L, U>(c, npos_max, ws, s)
    if (c.W.type == Q4_0) { G4_AQ(FQ4_0, 16, 2); G4_AQ(FQ4_0, 32, 4); G4_AQ(FQ4_0, 64, 2); }
    if (c.W.type == Q8_0) { G4_AQ(FQ8_0, 16, 2); G4_AQ(FQ8_0, 32, 4); G4_AQ(FQ8_0, 64, 2); }
#undef G4_AQ
    return hipErrorInvalidValue;
}

// resident capacity of the exact projection-in-attention instantiation that
// launch_attn_qkv would launch, with its dynamic LDS (its register use differs
// from the plain kernel's, so the plain kernel's capacity does not bound it)
template <int GRP, int HD>
static int qkv_capacity(int wtype, int lpr, int upl, size_t lds) {
#define G4_AC(F, L, U)      \
    if (lpr == L && upl == U) return resident_capacity(reinterpret_cast<const void *>(k_attn_fused_f16<GRP, HD, F, L, U>), lds)
    if (wtype == Q4_0) { G4_AC(FQ4_0, 16, 2); G4_AC(FQ4_0, 32, 4); G4_AC(FQ4_0, 64, 2); }
    if (wtype == Q8_0) { G4_AC(FQ8_0, 16, 2); G4_AC(FQ8_0, 32, 4); G4_AC(FQ8_0, 64, 2); }
#undef G4_AC
    return 0;
}

bool attn_qkv_fits(const g4h_tensor &W, const QkvArgs &a, int npos_max) {
    if (a.kv_type != F16 || !attn_fused_fits(F16, a.n_head, a.n_kv, a.hd, npos_max)) return false;
    if (W.type != Q4_0 && W.type != Q8_0) return false;
    if (W.ncols % 32 || W.ncols > 4 * 4 * 256 || W.nrows != (int64_t)(a.n_head + 2 * a.n_kv) * a.hd) return false;
    const int grp = a.n_head / a.n_kv;
    if (grp != 2 || (a.hd != 64 && a.hd != 256)) return false;
    int lpr, upl;
    gemv_shape(W.type, W.nb, &lpr, &upl);
    const bool shape = (lpr == 16 && upl == 2) || (lpr == 32 && upl == 4) || (lpr == 64 && upl == 2);
    if (!shape || W.nb * blck(W.type) / 32 > (int64_t)lpr * upl) return false;
    const size_t lds = ActQ8_0::bytes_per_token((int)W.nb) + kStageDump;
    const int cap = a.hd == 256 ? qkv_capacity<2, 256>(W.type, lpr, upl, lds) : qkv_capacity<2, 64>(W.type, lpr, upl, lds);
    const int nc = (npos_max + ATT_CHUNK - 1) / ATT_CHUNK;
    return (int64_t)a.n_kv * nc <= cap;
}

hipError_t launch_attn_qkv(const g4h_tensor &W, const GemvPro &pro, const QkvArgs &a, const int *npos_dev, int npos_max,
                           float *out, uint8_t *q8out, uint8_t *ws, uint64_t *qt, hipStream_t s, const AttnTag &tag) {
    if (!attn_qkv_fits(W, a, npos_max) || pro.kind != PRO_NORM || pro.n != W.ncols || !qt) return hipErrorInvalidValue;
    AttnCtx c{};
    c.a = a;
    c.npos_dev = npos_dev;
    c.out = out;
    c.q8out = q8out;
    c.epoch = tag.epoch;
    c.tag_mul = tag.mul;
    c.tag_add = tag.add;
    c.W = W;
    c.pro = pro;
    c.QT = qt;
    int lpr, upl;
    gemv_shape(W.type, W.nb, &lpr, &upl);
    if (a.hd == 256) return attn_qkv_fmt<2, 256>(c, lpr, upl, npos_max, ws, s);
    return attn_qkv_fmt<2, 64>(c, lpr, upl, npos_max, ws, s);
}

// q: prepared queries, or nullptr with `qkv` the raw q|k|v projection output
// to prepare (its k/v rows go into the caches at position npos - 1).
hipError_t launch_attn_decode(const float *q, const float *qkv, const QkvArgs &a, int npos, const int *npos_dev, int npos_max,
                              float *out, uint8_t *q8out, uint8_t *ws, hipStream_t s, const AttnTag *tag, const g4h_tensor *Wo,
                              float *wo_out, size_t ws_bytes) {
    if (a.hd % 64 || (a.hd > 256 && a.hd != ATT_WIDE) || a.n_kv <= 0 || a.n_head % a.n_kv) return hipErrorInvalidValue;
    if (qkv && (!a.rope || !a.q_norm || !a.k_norm)) return hipErrorInvalidValue;
    if (Wo && (!wo_out || !attn_wo_fits(*Wo, a, npos_max))) return hipErrorInvalidValue;
    AttnCtx c{};
    c.q = q;
    c.qkv = qkv;
    c.a = a;
    c.npos = npos;
    c.npos_dev = npos_dev;
    c.out = out;
    c.q8out = q8out;
    if (Wo) {
        c.Wo = *Wo;
        c.wo_out = wo_out;
    }
    if (a.hd == ATT_WIDE) return tag ? hipErrorInvalidValue : attn_wide(c, npos_max, 1, ws, s);
    const int grp = a.n_head / a.n_kv;
#define G4_ATT(KV, G)                                                                                 \
    if (a.kv_type == KV && grp == G) {                                                                \
        if (a.hd == 64) return attn_go<KV, G, 64>(c, a.n_head, a.n_kv, npos_max, ws, tag, s, ws_bytes);       \
        if (a.hd == 128) return attn_go<KV, G, 128>(c, a.n_head, a.n_kv, npos_max, ws, tag, s, ws_bytes);     \
        if (a.hd == 192) return attn_go<KV, G, 192>(c, a.n_head, a.n_kv, npos_max, ws, tag, s, ws_bytes);     \
        if (a.hd == 256) return attn_go<KV, G, 256>(c, a.n_head, a.n_kv, npos_max, ws, tag, s, ws_bytes);     \
    }
    G4_ATT(F16, 1); G4_ATT(F16, 2); G4_ATT(F16, 4); G4_ATT(F16, 8);
    G4_ATT(Q8_0, 1); G4_ATT(Q8_0, 2); G4_ATT(Q8_0, 4); G4_ATT(Q8_0, 8);
    G4_ATT(Q4_0, 1); G4_ATT(Q4_0, 2); G4_ATT(Q4_0, 4); G4_ATT(Q4_0, 8);
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
