// k_attn_mm.hip -- causal attention of a prompt batch on the matrix cores:
// attn_kernel (model.c:509-545) for nb new tokens over an f16 KV cache (head
// dims 64 to 512, gemma4's full layers included), the
// tokens of a tile sharing every K and V row they read.
//
// Rows of a tile are (token, query head) pairs of one KV head: 32 / GRP
// tokens x GRP heads = 32 rows.  Token b sits at position p0 + b and attends
// positions j0(b) .. p0 + b, j0 = max(0, p + 1 - window) with a window (else
// 0); on a ring, position j's row is at slot j % ring.  The batch's positions
// are cut at multiples of 128 (score chunks) and 256 (value spans) counted
// from 0, so every sum a row takes -- its scores, its chunk statistics, the
// normaliser over its own chunks (lane k = its k-th chunk), each span's
// weighted values and the spans added in order -- has the same operands in
// the same order whatever other tokens share the batch: a token's row has
// the same bits in any batch, alone included.
//   scores   grid (KV head x tile, 128-position chunk), 4 waves x 32
//            positions: S = fp16(q) . K_j (model.c:530-538, no 1/sqrt(d)) as
//            one v_mfma_f32_32x32x16_f16 per 16 head elements (exact
//            products, fp32 sums); per row and chunk the maximum m_c and
//            l_c = sum expf(s - m_c) over the row's positions, summed in
//            double.
//   values   grid (KV head x tile, 256-position span): per row the global
//            maximum M and normaliser (sum_c l_c exp(m_c - M) in double) as in
//            the decode kernels, the weights fp16(expf(s - M) * inv)
//            (model.c:547-555) into LDS (0 outside a row's positions), then
//            sum_j w_j V_j on v_mfma_f32_32x32x16_f16 with the positions as
//            the contraction: lane (c, half) loads V[j][2c], V[j][2c + 1] of
//            its 8 positions, the even and the odd columns of a 64-column
//            group being two 32-column tiles.
//   combine  per (token, head) its spans' partials added in order.
// With a device position (decode steps replayed from a graph) the grids are
// sized for the most positions a call can span and the workgroups past the
// call's last position return at once.
// Differences from the per-token kernels are the fp32 orders of the score and
// value sums, the grouping of the double normaliser and the exponentials of
// the scores and weights taken in fp32 (expf, about 1 ulp; the reference
// rounds exp in double to float: the weights' fp16 rounding can differ by
// one step where a product lands within ~1e-7 of a rounding boundary):
// within the attention's tolerance of the CPU, not bit-identical to them.  A non-finite
// V row (an f16 overflow) reaches the earlier rows of its tile as 0 * inf.
#include <algorithm>
#include <cmath>

#include "formats.h"
#include "kernels.h"
#include "steps.h"

namespace g4 {

typedef _Float16 am_v8h __attribute__((ext_vector_type(8)));
typedef float am_v16f __attribute__((ext_vector_type(16)));

constexpr int AMM_CH = 128;          // positions per score workgroup
constexpr int AMM_NP = 256;          // positions per value workgroup
constexpr size_t AMM_OFF = 256;      // the decode layout's header (error and epoch words) stays untouched

struct AmmArgs {
    const float *q;                  // [nb][n_head][hd] prepared queries
    float *out;                      // [nb][n_head][hd]
    uint8_t *q8out;                  // optional q8_0 rows of out, q8_stride bytes per token
    size_t q8_stride;
    FewAct few;                      // or (few.qa set) out as q8_0 in k_mm_few's layout
    const uint8_t *kc, *vc;
    int n_head, n_kv, window, ring;
    int p0, nb;                      // token 0's position (or *pos_dev) and the token count
    const int *pos_dev;
    int nch, nchv, ntt;              // the grid: chunks, spans (the strides of Mc / Lc and P), token tiles
    int jb, span;                    // set on the device by amm_view: first position (a multiple of AMM_NP) and count
    float *S;                        // [nb * n_head][nch * AMM_CH]
    float *Mc;                       // [nb * n_head][nch]
    double *Lc;                      // [nb * n_head][nch]
    float *P;                        // [nb * n_head][nchv][hd]
};

static size_t amm_al(size_t v) { return (v + 255) & ~(size_t)255; }
struct AmmWs {
    size_t S, Mc, Lc, P, total;
};
// most positions a batch spans: its last token's window (or all of its
// positions) plus the earlier tokens, from a multiple of AMM_NP
static int amm_span_max(int npos_max, int nb) { return npos_max + nb - 1 + AMM_NP - 1; }
static AmmWs amm_ws(int n_head, int hd, int nb, int span) {
    const size_t R = (size_t)nb * n_head, nch = (span + AMM_CH - 1) / AMM_CH, nchv = (span + AMM_NP - 1) / AMM_NP;
    AmmWs w;
    w.S = AMM_OFF;
    w.Mc = w.S + amm_al(R * nch * AMM_CH * 4);
    w.Lc = w.Mc + amm_al(R * nch * 4);
    w.P = w.Lc + amm_al(R * nch * 8);
    w.total = w.P + amm_al(R * nchv * hd * 4);
    return w;
}
size_t attn_batch_mm_workspace_bytes(int n_head, int hd, int npos_max, int nb) {
    return amm_ws(n_head, hd, nb, amm_span_max(npos_max, nb)).total;
}

// the call's positions: token 0's position, the first position any token
// attends rounded down to a multiple of AMM_NP, and the count from there
__device__ __forceinline__ void amm_view(AmmArgs &c) {
    if (c.pos_dev) c.p0 = *c.pos_dev;
    const int j0 = c.window ? max(0, c.p0 + 1 - c.window) : 0;
    c.jb = j0 / AMM_NP * AMM_NP;
    c.span = c.p0 + c.nb - c.jb;
}

__device__ __forceinline__ am_v8h amm_ld8(const void *p) { return *(const am_v8h *)p; }
__device__ __forceinline__ am_v16f amm_mma(am_v8h a, am_v8h b, am_v16f c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
}
__device__ __forceinline__ const uint8_t *amm_row(const AmmArgs &c, const uint8_t *cache, int j, int kvh, int hd) {
    const int slot = c.ring ? j % c.ring : j;
    return cache + ((size_t)slot * c.n_kv + kvh) * hd * 2;
}
// tile row i: token b and head h; the row's positions j0 .. p
template <int GRP>
__device__ __forceinline__ void amm_rowinfo(const AmmArgs &c, int kvh, int tt, int i, int &b, int &h, int &j0, int &p) {
    constexpr int T = 32 / GRP;
    b = tt * T + i / GRP;
    h = kvh * GRP + i % GRP;
    p = c.p0 + b;
    j0 = c.window ? std::max(0, p + 1 - c.window) : 0;
}

template <int HD, int GRP>
__global__ __launch_bounds__(256) void k_amm_scores(AmmArgs c) {
    constexpr int T = 32 / GRP, QS = HD + 8;
    __shared__ __align__(16) uint16_t qs[32][QS];                   // fp16 queries of the tile
    __shared__ float wm[4][32];
    __shared__ double wl[4][32];
    amm_view(c);
    const int kvh = blockIdx.x / c.ntt, tt = blockIdx.x % c.ntt, ch = blockIdx.y;
    if (ch * AMM_CH >= c.span) return;                               // past the call's last position
    const int t = threadIdx.x, lane = t & 63, wave = t >> 6, li = lane & 31, kh = lane >> 5;
    const int jl = ch * AMM_CH + wave * 32 + li, j = c.jb + jl;    // the lane's position (MFMA column)
    const int jfirst = c.window ? max(0, c.p0 + 1 - c.window) : 0;
    const uint8_t *krow = amm_row(c, c.kc, std::min(std::max(j, jfirst), c.jb + c.span - 1), kvh, HD);
    am_v8h kb[HD / 16];
#pragma unroll
    for (int s = 0; s < HD / 16; s++) kb[s] = amm_ld8(krow + (16 * s + 8 * kh) * 2);
    // the tile's queries: all of a thread's loads issued before any conversion
    constexpr int NQ = 32 * HD / 4 / 256;                           // float4 per thread
    float4 qv[NQ];
#pragma unroll
    for (int k = 0; k < NQ; k++) {
        const int x = t + 256 * k, i = x / (HD / 4), e4 = x % (HD / 4), b = tt * T + i / GRP, h = kvh * GRP + i % GRP;
        qv[k] = b < c.nb ? *(const float4 *)(c.q + ((size_t)b * c.n_head + h) * HD + 4 * e4) : make_float4(0.f, 0.f, 0.f, 0.f);
    }
#pragma unroll
    for (int k = 0; k < NQ; k++) {
        const int x = t + 256 * k, i = x / (HD / 4), e4 = x % (HD / 4);
        const uint32_t lo = f2h(qv[k].x) | ((uint32_t)f2h(qv[k].y) << 16), hi = f2h(qv[k].z) | ((uint32_t)f2h(qv[k].w) << 16);
        *(uint2 *)&qs[i][4 * e4] = make_uint2(lo, hi);
    }
    __syncthreads();
    am_v16f acc = {};
#pragma unroll
    for (int s = 0; s < HD / 16; s++) acc = amm_mma(amm_ld8(&qs[li][16 * s + 8 * kh]), kb[s], acc);
    // C[i][li]: rows i = 8 (r / 4) + 4 kh + r % 4
    bool ok[16];
#pragma unroll
    for (int r = 0; r < 16; r++) {
        const int i = 8 * (r >> 2) + 4 * kh + (r & 3);
        int b, h, j0, p;
        amm_rowinfo<GRP>(c, kvh, tt, i, b, h, j0, p);
        ok[r] = b < c.nb && jl < c.span && j >= j0 && j <= p;
        if (ok[r]) c.S[((size_t)b * c.n_head + h) * c.nch * AMM_CH + jl] = acc[r];
        const float m = group_max<32>(ok[r] ? acc[r] : -INFINITY);
        if (li == 0) wm[wave][i] = m;
    }
    __syncthreads();
#pragma unroll
    for (int r = 0; r < 16; r++) {
        const int i = 8 * (r >> 2) + 4 * kh + (r & 3);
        // rows 8 (r / 4) .. 8 (r / 4) + 7 hold tokens from (8 (r / 4)) / GRP
        // on: none of them in the batch (a decode step's later rows) skips
        // the exps for the whole wave
        if (tt * T + 8 * (r >> 2) / GRP >= c.nb) continue;           // uniform
        const float mc = fmaxf(fmaxf(wm[0][i], wm[1][i]), fmaxf(wm[2][i], wm[3][i]));
        const double l = group_sum_t<32>(ok[r] ? (double)expf(acc[r] - mc) : 0.0);
        if (li == 0) wl[wave][i] = l;
    }
    __syncthreads();
    if (t < 32) {
        int b, h, j0, p;
        amm_rowinfo<GRP>(c, kvh, tt, t, b, h, j0, p);
        if (b < c.nb) {
            const size_t R = (size_t)b * c.n_head + h;
            c.Mc[R * c.nch + ch] = fmaxf(fmaxf(wm[0][t], wm[1][t]), fmaxf(wm[2][t], wm[3][t]));
            c.Lc[R * c.nch + ch] = ((wl[0][t] + wl[1][t]) + wl[2][t]) + wl[3][t];
        }
    }
}

// PF: steps of V loads in flight per wave in the value sums: 8, or for calls
// of one row tile (decode steps and short verify batches, whose few
// workgroups are bound by that chain's round trips) 16 at heads up to 256
// wide, the whole span loaded at the start; the MFMAs and their order are
// the same either way.  Measured on the 64-token prompt chunk of 26 layers
// (8 q / 4 KV heads of 256 at position 4096): 3.58 ms with 4 steps, 3.50 with
// 8, 3.76 with 16.
template <int HD, int GRP, int PF>
__global__ __launch_bounds__(256) void k_amm_v(AmmArgs c) {
    constexpr int WS = AMM_NP + 8;
    __shared__ __align__(16) uint16_t wsh[32][WS];                  // fp16 weights of the span
    __shared__ float mx[32], iv[32];
    amm_view(c);
    const int kvh = blockIdx.x / c.ntt, tt = blockIdx.x % c.ntt, cv = blockIdx.y;
    if (cv * AMM_NP >= c.span) return;                               // past the call's last position
    const int t = threadIdx.x, lane = t & 63, wave = t >> 6, li = lane & 31, kh = lane >> 5;
    const int jl0 = cv * AMM_NP;
    const int jfirst = c.window ? max(0, c.p0 + 1 - c.window) : 0, jlast = c.jb + c.span - 1;
    // the attended positions jfirst .. jlast are at most `ring` apart, so on
    // a ring (rows stored at j % ring and again at j % ring + ring) they are
    // one contiguous run of slots from jfirst % ring: one modulo per thread
    // instead of one per row loaded
    const uint8_t *vbase = c.vc + ((size_t)(c.ring ? jfirst % c.ring : jfirst) * c.n_kv + kvh) * HD * 2;
    // lane (c, half)'s V words of step st in column group g (columns 2c,
    // 2c + 1 of its 8 positions): rows clamped to the positions the batch
    // attends, so every row loaded holds a stored value
    auto vword = [&](int g, int st, int k) __attribute__((always_inline)) {
        const int jb8 = c.jb + jl0 + 16 * st + 8 * kh;
        return *(const uint32_t *)(vbase + (size_t)(std::min(std::max(jb8 + k, jfirst), jlast) - jfirst) * c.n_kv * HD * 2 +
                                   (64 * g + 2 * li) * 2);
    };
    // one row tile with one column group per wave: every load of the kernel
    // (this wave's V words, this thread's scores) goes out first, so the
    // three phases below wait on one round trip instead of three
    constexpr bool EARLY = PF == 16 && HD <= 256;
    uint32_t xe[EARLY ? 16 : 1][8];
    float se[EARLY ? 32 : 1];
    if constexpr (EARLY) {
        if (wave < HD / 64) {                                        // uniform
#pragma unroll
            for (int q = 0; q < 16; q++)
#pragma unroll
                for (int k = 0; k < 8; k++) xe[q][k] = vword(wave, q, k);
        }
        const int jl = jl0 + t, j = c.jb + jl;
#pragma unroll
        for (int i = 0; i < 32; i++) {
            int b, h, j0, p;
            amm_rowinfo<GRP>(c, kvh, tt, i, b, h, j0, p);
            const bool ok = b < c.nb && jl < c.span && j >= j0 && j <= p;
            se[i] = ok ? c.S[((size_t)b * c.n_head + h) * c.nch * AMM_CH + jl] : 0.0f;
        }
    }
    // 1. per row the global maximum and normaliser over the row's own chunks
    // (wave w: rows 8 w .. 8 w + 7; lane k: the row's k-th chunk, 64 per
    // round), the eight rows' loads of a round issued together
    {
        const int nca = (c.span + AMM_CH - 1) / AMM_CH;              // >= any row's chunk count
        int clo[8], nrc[8];
        size_t base[8];
        bool rv[8];
#pragma unroll
        for (int k = 0; k < 8; k++) {
            int b, h, j0, p;
            amm_rowinfo<GRP>(c, kvh, tt, wave * 8 + k, b, h, j0, p);
            rv[k] = b < c.nb;
            clo[k] = rv[k] ? (j0 - c.jb) / AMM_CH : 0;
            nrc[k] = rv[k] ? (p - c.jb) / AMM_CH - clo[k] + 1 : 0;
            base[k] = ((size_t)(rv[k] ? b : 0) * c.n_head + h) * c.nch + clo[k];
        }
        float mcv[8], m[8];
        double lcv[8], sum[8];
        bool on[8];
#pragma unroll
        for (int k = 0; k < 8; k++) {
            on[k] = lane < nrc[k];
            mcv[k] = on[k] ? c.Mc[base[k] + lane] : -INFINITY;
            lcv[k] = on[k] ? c.Lc[base[k] + lane] : 0.0;
        }
#pragma unroll
        for (int k = 0; k < 8; k++) m[k] = group_max<64>(mcv[k]);
        for (int c1 = 64; c1 < nca; c1 += 64)
#pragma unroll
            for (int k = 0; k < 8; k++) m[k] = fmaxf(m[k], group_max<64>(c1 + lane < nrc[k] ? c.Mc[base[k] + c1 + lane] : -INFINITY));
#pragma unroll
        for (int k = 0; k < 8; k++)                                  // rows outside the batch (uniform) skip the exp
            sum[k] = rv[k] ? group_sum_t<64>(on[k] ? lcv[k] * exp((double)mcv[k] - (double)m[k]) : 0.0) : 1.0;
        for (int c1 = 64; c1 < nca; c1 += 64)
#pragma unroll
            for (int k = 0; k < 8; k++) {
                const bool o = c1 + lane < nrc[k];
                const float mc = o ? c.Mc[base[k] + c1 + lane] : 0.0f;
                const double lc = o ? c.Lc[base[k] + c1 + lane] : 0.0;
                sum[k] += group_sum_t<64>(o ? lc * exp((double)mc - (double)m[k]) : 0.0);
            }
        if (lane == 0)
#pragma unroll
            for (int k = 0; k < 8; k++) {
                mx[wave * 8 + k] = m[k];
                iv[wave * 8 + k] = (float)(1.0 / sum[k]);
            }
    }
    __syncthreads();
    // 2. the weights (0 outside a row's positions): thread t owns position t
    // of the span in every row, its score loads issued 16 rows at a time
    static_assert(AMM_NP == 256, "one position per thread");
#pragma unroll
    for (int i0 = 0; i0 < 32; i0 += 16) {
        const int jl = jl0 + t, j = c.jb + jl;
        float sv[16];
        bool ok[16];
#pragma unroll
        for (int i = 0; i < 16; i++) {
            int b, h, j0, p;
            amm_rowinfo<GRP>(c, kvh, tt, i0 + i, b, h, j0, p);
            ok[i] = b < c.nb && jl < c.span && j >= j0 && j <= p;
            if constexpr (EARLY) sv[i] = se[i0 + i];
            else sv[i] = ok[i] ? c.S[((size_t)b * c.n_head + h) * c.nch * AMM_CH + jl] : 0.0f;
        }
#pragma unroll
        for (int i = 0; i < 16; i++) {
            int b, h, j0, p;
            amm_rowinfo<GRP>(c, kvh, tt, i0 + i, b, h, j0, p);
            // a row outside the batch (uniform: a decode step's rows past
            // its GRP heads) takes weight 0 without the exp
            wsh[i0 + i][t] = b < c.nb ? f2h(ok[i] ? expf(sv[i] - mx[i0 + i]) * iv[i0 + i] : 0.0f) : (uint16_t)0;
        }
    }
    __syncthreads();
    // 3. sum_j w_j V_j over the span's 16 steps of 16 positions, in step
    // order (the MFMA's accumulation): wave w takes the 64-column groups w,
    // w + 4, ..; lane (c, half) loads columns 2c, 2c + 1 of its 8 positions
    // per step (the even and the odd columns two 32-column tiles)
#pragma unroll 1
    for (int g = wave; g < HD / 64; g += 4) {
        const int col = 64 * g + 2 * li;
        am_v16f ae = {}, ao = {};
        for (int st0 = 0; st0 < AMM_NP / 16; st0 += PF) {
            uint32_t x[PF][8];
#pragma unroll
            for (int q = 0; q < PF; q++)
#pragma unroll
                for (int k = 0; k < 8; k++) {
                    if constexpr (EARLY) x[q][k] = xe[q][k];                  // loaded at the start (g == wave)
                    else x[q][k] = vword(g, st0 + q, k);
                }
#pragma unroll
            for (int q = 0; q < PF; q++) {
                am_v8h be, bo;
#pragma unroll
                for (int k = 0; k < 8; k++) {
                    be[k] = __builtin_bit_cast(_Float16, (uint16_t)(x[q][k] & 0xffff));
                    bo[k] = __builtin_bit_cast(_Float16, (uint16_t)(x[q][k] >> 16));
                }
                const am_v8h a = amm_ld8(&wsh[li][16 * (st0 + q) + 8 * kh]);
                ae = amm_mma(a, be, ae);
                ao = amm_mma(a, bo, ao);
            }
        }
#pragma unroll
        for (int r = 0; r < 16; r++) {
            const int i = 8 * (r >> 2) + 4 * kh + (r & 3);
            int b, h, j0, p;
            amm_rowinfo<GRP>(c, kvh, tt, i, b, h, j0, p);
            if (b < c.nb) {
                float *dst = c.P + (((size_t)b * c.n_head + h) * c.nchv + cv) * HD;
                *(float2 *)(dst + col) = make_float2(ae[r], ao[r]);
            }
        }
    }
}

// grid (n_head, nb), 256 threads (elements e and e + 256): the spans'
// partials in order; with q8out (or few), the head row as q8_0 blocks too
// (quants.c:74-109)
template <int HD>
__global__ __launch_bounds__(256) void k_amm_combine(AmmArgs c) {
    constexpr int EP = (HD + 255) / 256;                             // elements per thread
    __shared__ float row[HD];
    amm_view(c);
    const int h = blockIdx.x, b = blockIdx.y, t = threadIdx.x;
    const size_t R = (size_t)b * c.n_head + h;
    const int p = c.p0 + b, j0 = c.window ? max(0, p + 1 - c.window) : 0;
    const int first = (j0 - c.jb) / AMM_NP, last = (p - c.jb) / AMM_NP;   // the token's spans
#pragma unroll
    for (int q = 0; q < EP; q++) {
        const int e = t + 256 * q;
        if (e < HD) {
            const float *src = c.P + R * c.nchv * HD + e;
            float r = 0.0f;
            for (int c0 = first; c0 <= last; c0 += 8) {              // eight loads in flight, added in order
                float v[8];
#pragma unroll
                for (int k = 0; k < 8; k++) v[k] = c0 + k <= last ? src[(size_t)(c0 + k) * HD] : 0.0f;
#pragma unroll
                for (int k = 0; k < 8; k++)
                    if (c0 + k <= last) r += v[k];
            }
            c.out[R * HD + e] = r;
            row[e] = r;
        }
    }
    if (c.q8out || c.few.qa) {
        __syncthreads();
        const bool own = t < HD / 4;
        float v[4] = {0.f, 0.f, 0.f, 0.f};
        if (own)
            for (int k = 0; k < 4; k++) v[k] = row[4 * t + k];
        if (t < (HD / 4 + 63) / 64 * 64) {
            if (c.few.qa) q8_store4_few(v, h * (HD / 4) + t, own, c.few, b);
            else q8_store4(v, t, own, c.q8out + (size_t)b * c.q8_stride + (size_t)h * (HD / 32) * 34);
        }
    }
}

bool attn_batch_mm_ok(const QkvArgs &a) {
    const int grp = a.n_kv > 0 ? a.n_head / a.n_kv : 0;
    return a.kv_type == F16 && (a.hd == 64 || a.hd == 128 || a.hd == 256 || a.hd == 512) && a.n_kv > 0 && a.n_head % a.n_kv == 0 &&
           (grp == 1 || grp == 2 || grp == 4 || grp == 8);
}

template <int HD, int GRP>
static void amm_go(const AmmArgs &c, hipStream_t s) {
    hipLaunchKernelGGL((k_amm_scores<HD, GRP>), dim3(c.n_kv * c.ntt, c.nch), dim3(256), 0, s, c);
    constexpr int PF1 = HD == 512 ? 8 : 16;                          // 16 steps of 512-wide rows spill
    if (c.ntt == 1) hipLaunchKernelGGL((k_amm_v<HD, GRP, PF1>), dim3(c.n_kv * c.ntt, c.nchv), dim3(256), 0, s, c);
    else hipLaunchKernelGGL((k_amm_v<HD, GRP, 8>), dim3(c.n_kv * c.ntt, c.nchv), dim3(256), 0, s, c);
    hipLaunchKernelGGL(k_amm_combine<HD>, dim3(c.n_head, c.nb), dim3(256), 0, s, c);
}

hipError_t launch_attn_batch_mm(const float *q, const QkvArgs &a, int npos0, int nb, float *out, uint8_t *q8out, uint8_t *ws,
                                size_t ws_bytes, hipStream_t s, size_t q8_stride, const int *pos_dev, int npos_max,
                                const FewAct &few) {
    if (!attn_batch_mm_ok(a) || !q || !out || !ws || nb < 1 || nb > 65535 || (!pos_dev && npos0 < 1) || (pos_dev && npos_max < 1) ||
        (few.qa && nb > 16 * few.mt))
        return hipErrorInvalidValue;
    if (a.ring && (a.window <= 0 || a.window > a.ring || nb > a.ring - a.window + 1)) return hipErrorInvalidValue;
    AmmArgs c{};
    c.q = q;
    c.out = out;
    c.q8out = q8out;
    c.q8_stride = q8_stride ? q8_stride : (size_t)a.n_head * (a.hd / 32) * 34;
    c.few = few;
    c.kc = a.kc;
    c.vc = a.vc;
    c.n_head = a.n_head;
    c.n_kv = a.n_kv;
    c.window = a.window;
    c.ring = a.ring;
    c.p0 = npos0 - 1;
    c.nb = nb;
    c.pos_dev = pos_dev;
    // the grid: this call's positions, or with a device position the most a
    // call can span (npos_max positions attended by its last token)
    int span;
    if (pos_dev) {
        span = amm_span_max(a.window ? std::min(a.window, npos_max) : npos_max, nb);
    } else {
        const int j0 = a.window ? std::max(0, c.p0 + 1 - a.window) : 0;
        span = c.p0 + nb - j0 / AMM_NP * AMM_NP;
    }
    c.nch = (span + AMM_CH - 1) / AMM_CH;
    c.nchv = (span + AMM_NP - 1) / AMM_NP;
    const int grp = a.n_head / a.n_kv;
    c.ntt = (nb + 32 / grp - 1) / (32 / grp);
    const AmmWs w = amm_ws(a.n_head, a.hd, nb, span);
    if (ws_bytes < w.total || (size_t)c.n_kv * c.ntt > 0x7fffffff) return hipErrorInvalidValue;
    c.S = (float *)(ws + w.S);
    c.Mc = (float *)(ws + w.Mc);
    c.Lc = (double *)(ws + w.Lc);
    c.P = (float *)(ws + w.P);
#define G4_AMM(HD_, G_) \
    if (a.hd == HD_ && grp == G_) amm_go<HD_, G_>(c, s);
    G4_AMM(64, 1) G4_AMM(64, 2) G4_AMM(64, 4) G4_AMM(64, 8)
    G4_AMM(128, 1) G4_AMM(128, 2) G4_AMM(128, 4) G4_AMM(128, 8)
    G4_AMM(256, 1) G4_AMM(256, 2) G4_AMM(256, 4) G4_AMM(256, 8)
    G4_AMM(512, 1) G4_AMM(512, 2) G4_AMM(512, 4) G4_AMM(512, 8)
#undef G4_AMM
    return hipGetLastError();
}

}  // namespace g4
