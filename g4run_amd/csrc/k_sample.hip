// k_sample.hip -- the sampling chain of sampler.c:74-210 on the GPU: one
// workgroup of 1024 threads draws one id from a logits row resident in HBM,
// so a decode step can sample without a host round trip.
//
// Stages, in the reference's order, with its arithmetic:
//   bans -> -inf, no-repeat-ngram hits -> -inf           (sampler.c:78-101)
//   repeat / frequency / presence penalties, each distinct id of the window
//   once; the window is sorted in LDS so a run gives the count (104-137)
//   greedy: first index of the maximum                     (140-144)
//   top-k (k = top_k in 1..511, else 512, at most n_vocab)  (147-176)
//   top-p over the fp32 softmax, double sums               (179-194)
//   temperature softmax in double and the draw             (197-209)
//
// Top-k.  The reference keeps a bounded min-heap over the ids in order and
// insertion-sorts the heap array.  When the k+1 largest values are pairwise
// different (float compare, so -0 == +0 counts as a tie) and no logit is NaN,
// its result is fixed by the values alone: the k largest, in descending order.
// The fast path finds them with a 16-ary search over the order-preserving
// 32-bit keys for a threshold with between k+1 and 1024 elements at or above
// it (the row held in registers when it has at most 32 values per thread,
// else read in batches of 8 per thread), gathers those, bitonic-sorts them one
// per thread (lane shuffles within a wave, LDS across waves) and checks the
// condition.
// Otherwise (ties, NaN, or more than 4096 elements sharing the boundary key)
// wave 0 replays the reference's heap exactly, skipping 64 ids at a time
// whose values cannot enter it, and the heap array is ordered as the
// insertion sort orders it (a stable sort by value; the literal insertion
// sort when NaNs are present).
//
// exp: expf(x) is computed as (float)exp((double)x), exp in double is the
// device exp; both agree with the host libm except in rare last-ulp cases,
// which can only move a top-p cut whose cumulative sum lands within ~1e-7 of
// top_p or a draw within ~1e-16 of a bucket edge.  No contraction anywhere
// (the penalty and softmax arithmetic is the C text's, rounded per operation).
#include "kernels.h"
#include "steps.h"

#pragma clang fp contract(off)

namespace g4 {

namespace {

constexpr int NT = 1024;            // threads per workgroup
constexpr int NW = NT / 64;         // waves
constexpr int CAP = 4096;           // LDS key array (penalty window, sorts)
constexpr int GT = 1024;            // gathered candidates of the fast path: one per thread
constexpr int RPT = 32;             // row values per thread held in registers (n_vocab <= RPT * NT)
constexpr int KMAX = SAMPLER_TOPK_MAX;

// order-preserving key: larger float <=> larger key (-0 < +0; NaNs at the ends)
__device__ __forceinline__ uint32_t okey(float v) {
    const uint32_t u = __float_as_uint(v);
    return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}
__device__ __forceinline__ float okey_val(uint32_t k) {
    return __uint_as_float((k & 0x80000000u) ? (k & 0x7fffffffu) : ~k);
}

// bitonic sort of a[0..n) in LDS (n a power of two <= 4096), descending if
// DESC; every thread of the workgroup calls it
template <typename T, bool DESC>
__device__ void lds_bitonic(T *a, int n) {
    for (int k = 2; k <= n; k <<= 1)
        for (int j = k >> 1; j > 0; j >>= 1) {
            for (int i = threadIdx.x; i < n; i += NT) {
                const int p = i ^ j;
                if (p > i) {
                    const T x = a[i], y = a[p];
                    const bool asc = ((i & k) == 0) != DESC;
                    if (asc ? (x > y) : (x < y)) {
                        a[i] = y;
                        a[p] = x;
                    }
                }
            }
            __syncthreads();
        }
}

// descending bitonic sort of a[0..n) (n a power of two <= NT, distinct keys
// apart from zero padding), one key per thread: exchanges within a wave are
// lane shuffles, wider ones go through a[] in LDS.  The same compare-exchange
// network as lds_bitonic<uint64_t, true>; every thread calls it.
__device__ void reg_bitonic_desc(uint64_t *a, int n) {
    const int t = threadIdx.x;
    uint64_t x = t < n ? a[t] : 0;
    for (int k = 2; k <= n; k <<= 1)
        for (int j = k >> 1; j > 0; j >>= 1) {
            uint64_t y;
            if (j >= 64) {                                           // uniform
                __syncthreads();
                if (t < n) a[t] = x;
                __syncthreads();
                y = t < n ? a[t ^ j] : 0;
            } else {
                const uint32_t lo = (uint32_t)__shfl_xor((int)(uint32_t)x, j, 64);
                const uint32_t hi = (uint32_t)__shfl_xor((int)(uint32_t)(x >> 32), j, 64);
                y = ((uint64_t)hi << 32) | lo;
            }
            const bool lower = (t & j) == 0, asc = (t & k) != 0;     // descending overall
            x = (lower == asc) ? (x < y ? x : y) : (x < y ? y : x);
        }
    __syncthreads();
    if (t < n) a[t] = x;
    __syncthreads();
}

__device__ __forceinline__ int wave_isum(int v) {
    for (int m = 32; m >= 1; m >>= 1) v += __shfl_xor(v, m, 64);
    return v;
}

// splitmix64 seeding of all-zero state, then the xoshiro256+ step
// (sampler.c:51-70); one thread
__device__ uint64_t rng_next(SamplerDev *S) {
    uint64_t w[4] = {S->rng[0], S->rng[1], S->rng[2], S->rng[3]};
    if ((w[0] | w[1] | w[2] | w[3]) == 0) {
        uint64_t z = S->seed + 0x9e3779b97f4a7c15ull;
        for (int i = 0; i < 4; i++) {
            z += 0x9e3779b97f4a7c15ull;
            uint64_t v = z;
            v = (v ^ (v >> 30)) * 0xbf58476d1ce4e5b9ull;
            v = (v ^ (v >> 27)) * 0x94d049bb133111ebull;
            w[i] = v ^ (v >> 31);
        }
    }
    const uint64_t out = w[0] + w[3];
    const uint64_t sh = w[1] << 17;
    w[2] ^= w[0];
    w[3] ^= w[1];
    w[1] ^= w[2];
    w[0] ^= w[3];
    w[2] ^= sh;
    w[3] = (w[3] << 45) | (w[3] >> 19);
    for (int i = 0; i < 4; i++) S->rng[i] = w[i];
    return out;
}

__device__ __forceinline__ int ring_at(const SamplerDev *S, int i) {
    return S->recent[(S->recent_head + i) % SAMPLER_RING];
}

// The ring push of sampler.c:37-48 (one thread).
__device__ __forceinline__ void ring_push(SamplerDev *S, int id) {
    if (S->recent_n == SAMPLER_RING) {
        S->recent[S->recent_head] = id;
        S->recent_head = (S->recent_head + 1) % SAMPLER_RING;
    } else {
        S->recent[(S->recent_head + S->recent_n) % SAMPLER_RING] = id;
        S->recent_n++;
    }
}

struct Lds {
    union {
        uint64_t keys[CAP];               // gathered (key << 32 | ~id)
        int win[CAP];                     // penalty window, sorted
    };
    float cv[KMAX];                       // candidates, descending
    int ci[KMAX];
    float pf[KMAX];                       // top-p weights (fp32)
    double pd[KMAX];                      // temperature weights (double)
    float hv[KMAX];                       // exact heap (slow path)
    int hi[KMAX];
    int red[NW][16];
    int cred[2][NW][16];                  // per-round wave counts of the threshold search
    int cnt[16];
    float bv[NW];
    int bi[NW];
    int suf[64];
    int flag, n_keep, gathered, id;
    double dsum;
};

// Workgroup totals of 15 per-thread counts (wave sums by lane exchanges, the
// waves' sums through LDS; buf alternates between calls so one barrier does)
__device__ __forceinline__ void wg_counts15(int c[15], Lds &sh, int buf) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    int (*cr)[16] = sh.cred[buf & 1];
#pragma unroll
    for (int j = 0; j < 15; j++) {
        const int v = group_isum<64>(c[j]);
        if (lane == j) cr[wave][j] = v;
    }
    __syncthreads();
#pragma unroll
    for (int j = 0; j < 15; j++) {
        int v = 0;
        for (int w = 0; w < NW; w++) v += cr[w][j];
        c[j] = v;
    }
}

// The reference's heap over ids 0..nv-1 (sampler.c:149-168) on wave 0;
// lane 0 writes the heap, every lane reads it.  Ids whose value cannot enter
// (the heap is full and the value is not above its root, which only grows)
// are skipped 64 at a time.
__device__ void heap_replay(const float *L, int nv, int k, Lds &sh) {
    const int lane = threadIdx.x & 63;
    int hn = 0;
    float root = 0.0f;
    for (int base = 0; base < nv; base += 64) {
        const int i = base + lane;
        const float l = i < nv ? L[i] : 0.0f;
        uint64_t m = __ballot(i < nv && (hn < k || l > root));
        while (m) {
            const int j = __builtin_ctzll(m);
            m &= m - 1;
            const float v = __shfl(l, j, 64);
            const int id = base + j;
            if (hn < k) {
                int p = hn++;
                if (lane == 0) { sh.hv[p] = v; sh.hi[p] = id; }
                while (p > 0) {
                    const int up = (p - 1) / 2;
                    const float a = sh.hv[p], b = sh.hv[up];
                    if (!(a < b)) break;
                    const int ia = sh.hi[p], ib = sh.hi[up];
                    if (lane == 0) { sh.hv[up] = a; sh.hi[up] = ia; sh.hv[p] = b; sh.hi[p] = ib; }
                    p = up;
                }
            } else if (v > sh.hv[0]) {
                if (lane == 0) { sh.hv[0] = v; sh.hi[0] = id; }
                int p = 0;
                for (;;) {
                    const int a = 2 * p + 1, b = 2 * p + 2;
                    int lo = p;
                    if (a < k && sh.hv[a] < sh.hv[lo]) lo = a;
                    if (b < k && sh.hv[b] < sh.hv[lo]) lo = b;
                    if (lo == p) break;
                    const float x = sh.hv[lo], y = sh.hv[p];
                    const int ix = sh.hi[lo], iy = sh.hi[p];
                    if (lane == 0) { sh.hv[lo] = y; sh.hi[lo] = iy; sh.hv[p] = x; sh.hi[p] = ix; }
                    p = lo;
                }
            }
            root = sh.hv[0];
        }
    }
}

template <int REG>
__global__ __launch_bounds__(NT) void k_sample(SamplerDev *S, float *L, int *out, int accept, int *state, int n_ctx) {
    __shared__ Lds sh;
    const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
    const int nv = S->n_vocab, rn = S->recent_n;
    const float temp = S->temp, top_p = S->top_p, rp = S->repeat_penalty, fp = S->freq_penalty,
                pp = S->presence_penalty;
    const int rln = S->repeat_last_n, ngram = S->no_repeat_ngram;

    // ---- bans and no-repeat-ngram (sampler.c:78-101) ----
    const int *ban = sampler_bans(S);
    for (int j = t; j < S->n_ban; j += NT) L[ban[j]] = -INFINITY;
    if (ngram >= 2 && rn >= ngram) {
        const int m = ngram - 1 < 64 ? ngram - 1 : 64;
        if (t < m) sh.suf[t] = ring_at(S, rn - m + t);
        __syncthreads();
        for (int p = t; p + m < rn; p += NT) {
            bool hit = true;
            for (int j = 0; j < m && hit; j++) hit = ring_at(S, p + j) == sh.suf[j];
            if (hit) L[ring_at(S, p + m)] = -INFINITY;
        }
    }
    __syncthreads();

    // ---- penalties over the newest min(repeat_last_n, recent_n) ids (104-137) ----
    if ((rp != 1.0f || fp != 0 || pp != 0) && rln > 0 && rn > 0) {
        const int win = rln < rn ? rln : rn;
        int P = 1;
        while (P < win) P <<= 1;
        for (int i = t; i < P; i += NT) sh.win[i] = i < win ? ring_at(S, rn - 1 - i) : 0x7fffffff;
        __syncthreads();
        lds_bitonic<int, false>(sh.win, P);
        for (int i = t; i < win; i += NT) {
            const int id = sh.win[i];
            if (i > 0 && sh.win[i - 1] == id) continue;
            int lo = i + 1, hi = win;                  // end of the run of id
            while (lo < hi) {
                const int mid = (lo + hi) >> 1;
                if (sh.win[mid] == id) lo = mid + 1;
                else hi = mid;
            }
            const int count = lo - i;
            float l = L[id];
            if (rp != 1.0f) l = l <= 0 ? l * rp : l / rp;
            const float fterm = (float)count * fp;
            l -= fterm + (count > 0 ? pp : 0.0f);
            L[id] = l;
        }
        __syncthreads();
    }

    // ---- greedy (140-144) ----
    if (temp <= 0.0f) {
        const int id = wg_first_argmax(L, nv, sh.bv, sh.bi);
        if (t == 0) {
            if (out) *out = id;
            if (accept) ring_push(S, id);
            if (state) state_advance(state, id, n_ctx);
        }
        return;
    }

    // ---- top-k (147-176) ----
    int k = S->top_k > 0 && S->top_k < KMAX ? S->top_k : KMAX;
    if (k > nv) k = nv;
    const int K1 = k < nv ? k + 1 : k;     // the k largest plus the next one, to see a tie at the edge

    // the row after bans and penalties: in registers (REG per thread), or read
    // again per pass in batches of 8 per thread (their loads in flight together)
    float lv[REG > 0 ? REG : 1];
    if constexpr (REG > 0) {
#pragma unroll
        for (int r = 0; r < REG; r++) {
            const int i = t + r * NT;
            lv[r] = i < nv ? L[i] : 0.0f;
        }
    }
    auto each = [&](auto &&f) {
        if constexpr (REG > 0) {
#pragma unroll
            for (int r = 0; r < REG; r++) {
                const int i = t + r * NT;
                if (i < nv) f(i, lv[r]);
            }
        } else {
            for (int i0 = t; i0 < nv; i0 += 8 * NT) {
                float b[8];
#pragma unroll
                for (int q = 0; q < 8; q++) {
                    const int i = i0 + q * NT;
                    b[q] = i < nv ? L[i] : 0.0f;
                }
#pragma unroll
                for (int q = 0; q < 8; q++) {
                    const int i = i0 + q * NT;
                    if (i < nv) f(i, b[q]);
                }
            }
        }
    };

    // NaN scan, the largest and the smallest key (wave maxima by lane
    // exchanges, the NaN flag by a ballot)
    uint32_t kmax = 0, kmin_c = 0;                 // kmin_c: complement of the smallest key
    int nan = 0;
    each([&](int, float v) {
        nan |= __builtin_isnan(v);
        const uint32_t kk = okey(v);
        kmax = kk > kmax ? kk : kmax;
        kmin_c = ~kk > kmin_c ? ~kk : kmin_c;
    });
    kmax = wave_umax(kmax);
    kmin_c = wave_umax(kmin_c);
    const bool wnan = __ballot(nan != 0) != 0;
    if (lane == 0) { sh.red[wave][0] = (int)kmax; sh.red[wave][1] = wnan; sh.red[wave][2] = (int)kmin_c; }
    if (t == 0) { sh.gathered = 0; sh.flag = 0; }
    __syncthreads();
    kmax = 0;
    kmin_c = 0;
    nan = 0;
    for (int w = 0; w < NW; w++) {
        kmax = max(kmax, (uint32_t)sh.red[w][0]);
        kmin_c = max(kmin_c, (uint32_t)sh.red[w][2]);
        nan |= sh.red[w][1];
    }
    __syncthreads();

    bool slow = nan != 0;
    uint32_t lo = ~kmin_c;                 // count(key >= lo) >= K1: every element
    if (!slow) {
        uint64_t hi = (uint64_t)kmax + 1;  // count(key >= hi) < K1
        int c_lo = nv, buf = 0;
        // the 15 counts of keys >= p[j] over the row
        auto row_counts = [&](const uint32_t p[15], int c[15]) {
#pragma unroll
            for (int j = 0; j < 15; j++) c[j] = 0;
            each([&](int, float v) {
                const uint32_t k = okey(v);
#pragma unroll
                for (int j = 0; j < 15; j++) c[j] += k >= p[j];
            });
            wg_counts15(c, sh, buf++);
        };
        for (int round = 0; c_lo > GT; round++) {
            const uint64_t span = hi - lo;
            if (span <= 1) { slow = true; break; }       // > GT elements share the boundary key: ties
            uint32_t p[15];
            int c[15];
            // the first round's thresholds close in on the largest key
            // geometrically (hi - span / 2^m, m = 15 .. 1: the k largest of a
            // row of logits sit in a narrow band of keys at its top), later
            // rounds split the bracket evenly
#pragma unroll
            for (int j = 0; j < 15; j++)
                p[j] = round == 0 ? (uint32_t)(hi - (span >> (j + 1))) : (uint32_t)(lo + (span * (uint64_t)(j + 1)) / 16);
            row_counts(p, c);
            int jbest = -1;
#pragma unroll
            for (int j = 0; j < 15; j++)
                if (c[j] >= K1) jbest = j;
            if (jbest >= 0) {
                if (p[jbest] > lo) { lo = p[jbest]; c_lo = c[jbest]; }
                hi = jbest < 14 ? p[jbest + 1] : hi;
            } else {
                hi = p[0];
            }
        }
    }

    if (!slow) {
        // gather every element with key >= lo (at most GT) by wave-ballot compaction
        auto gather = [&](int i, float v) {                          // every lane of the wave, each step
            const uint32_t kk = i < nv ? okey(v) : 0u;
            const bool keep = i < nv && kk >= lo;
            const uint64_t m = __ballot(keep);
            int base = 0;
            if (lane == 0 && m) base = atomicAdd(&sh.gathered, __builtin_popcountll(m));
            base = __shfl(base, 0, 64);
            if (keep) {
                const int slot = base + __builtin_popcountll(m & ((1ull << lane) - 1));
                sh.keys[slot] = ((uint64_t)kk << 32) | (uint32_t)~(uint32_t)i;
            }
        };
        if constexpr (REG > 0) {
#pragma unroll
            for (int r = 0; r < REG; r++) gather(t + r * NT, lv[r]);
        } else {
            for (int i0 = 0; i0 < nv; i0 += NT) gather(i0 + t, i0 + t < nv ? L[i0 + t] : 0.0f);
        }
        __syncthreads();
        const int G = sh.gathered;
        int P = 1;
        while (P < G) P <<= 1;
        for (int i = G + t; i < P; i += NT) sh.keys[i] = 0;
        __syncthreads();
        reg_bitonic_desc(sh.keys, P);
        // the k largest must be strictly decreasing and the (k+1)-th strictly smaller
        for (int i = t; i + 1 < K1; i += NT)
            if (okey_val((uint32_t)(sh.keys[i] >> 32)) == okey_val((uint32_t)(sh.keys[i + 1] >> 32))) sh.flag = 1;
        __syncthreads();
        slow = sh.flag != 0;
        if (!slow)
            for (int i = t; i < k; i += NT) {
                sh.cv[i] = okey_val((uint32_t)(sh.keys[i] >> 32));
                sh.ci[i] = (int)~(uint32_t)sh.keys[i];
            }
        __syncthreads();
    }

    if (slow) {
        if (wave == 0) heap_replay(L, nv, k, sh);
        __syncthreads();
        if (!nan) {
            // stable descending sort of the heap array: (value, -0 as +0) desc, heap slot asc
            int P = 1;
            while (P < k) P <<= 1;
            for (int i = t; i < P; i += NT) {
                const float v = sh.hv[i < k ? i : 0];
                sh.keys[i] = i < k ? ((uint64_t)okey(v == 0.0f ? 0.0f : v) << 32) | (uint32_t)(0xffffffffu - i) : 0;
            }
            __syncthreads();
            reg_bitonic_desc(sh.keys, P);
            for (int i = t; i < k; i += NT) {
                const int slot = (int)(0xffffffffu - (uint32_t)sh.keys[i]);
                sh.cv[i] = sh.hv[slot];
                sh.ci[i] = sh.hi[slot];
            }
        } else if (t == 0) {
            // the reference's insertion sort, literally (its order with NaNs is not a sort order)
            for (int i = 0; i < k; i++) { sh.cv[i] = sh.hv[i]; sh.ci[i] = sh.hi[i]; }
            for (int i = 1; i < k; i++) {
                const float v = sh.cv[i];
                const int vi = sh.ci[i];
                int j = i - 1;
                while (j >= 0 && sh.cv[j] < v) {
                    sh.cv[j + 1] = sh.cv[j];
                    sh.ci[j + 1] = sh.ci[j];
                    j--;
                }
                sh.cv[j + 1] = v;
                sh.ci[j + 1] = vi;
            }
        }
        if (t == 0) S->slow_draws += 1;
        __syncthreads();
    }

    // ---- top-p (179-194) ----
    // The sums and running sums are one thread's, in index order as in the
    // reference; it reads the LDS terms 8 at a time so their latencies overlap
    // and runs each batch without branches (terms past the end are +0, which
    // leaves a sum of non-negative terms unchanged; a running sum past its
    // cut no longer matters), and the quotients pf[i] / sum come from all
    // threads.
    for (int i = t; i < k; i += NT) sh.pf[i] = (float)exp((double)(sh.cv[i] - sh.cv[0]));
    __syncthreads();
    const bool cut = top_p < 1.0f && top_p > 0.0f;
    if (t == 0 && cut) {                                             // the sum serves the cut only
        double sum = 0;
        for (int i0 = 0; i0 < k; i0 += 8) {
            float b[8];
#pragma unroll
            for (int q = 0; q < 8; q++) b[q] = i0 + q < k ? sh.pf[i0 + q] : 0.0f;
#pragma unroll
            for (int q = 0; q < 8; q++) sum += b[q];
        }
        sh.dsum = sum;
    }
    if (t == 0) sh.n_keep = k;
    __syncthreads();
    if (cut) {
        const double sum = sh.dsum;
        for (int i = t; i < k; i += NT) sh.pd[i] = sh.pf[i] / sum;
        __syncthreads();
        if (t == 0) {
            double cum = 0;
            int n = k;
            for (int i0 = 0; i0 < k && n == k; i0 += 8) {
                double b[8];
#pragma unroll
                for (int q = 0; q < 8; q++) b[q] = i0 + q < k ? sh.pd[i0 + q] : 0.0;
#pragma unroll
                for (int q = 0; q < 8; q++) {
                    cum += b[q];
                    n = (n == k && i0 + q < k && cum >= top_p) ? i0 + q + 1 : n;
                }
            }
            sh.n_keep = n;
        }
        __syncthreads();
    }
    const int n = sh.n_keep;

    // ---- temperature and the draw (197-209) ----
    const float shift = sh.cv[0] / temp;
    for (int i = t; i < n; i += NT) sh.pd[i] = exp((double)sh.cv[i] / temp - shift);
    __syncthreads();
    if (t == 0) {
        double sum = 0;
        for (int i0 = 0; i0 < n; i0 += 8) {
            double b[8];
#pragma unroll
            for (int q = 0; q < 8; q++) b[q] = i0 + q < n ? sh.pd[i0 + q] : 0.0;
#pragma unroll
            for (int q = 0; q < 8; q++) sum += b[q];
        }
        const double r = (double)(rng_next(S) >> 11) / 9007199254740992.0 * sum;
        double cum = 0;
        int id = sh.ci[n - 1], hit = -1;
        for (int i0 = 0; i0 < n && hit < 0; i0 += 8) {
            double b[8];
#pragma unroll
            for (int q = 0; q < 8; q++) b[q] = i0 + q < n ? sh.pd[i0 + q] : 0.0;
#pragma unroll
            for (int q = 0; q < 8; q++) {
                cum += b[q];
                hit = (hit < 0 && i0 + q < n && r < cum) ? i0 + q : hit;
            }
        }
        if (hit >= 0) id = sh.ci[hit];
        if (out) *out = id;
        if (accept) ring_push(S, id);
        if (state) state_advance(state, id, n_ctx);
    }
}

__global__ __launch_bounds__(64) void k_sampler_push(SamplerDev *S, const int *ids, int n) {
    if (threadIdx.x == 0)
        for (int i = 0; i < n; i++) ring_push(S, ids[i]);
}

}  // namespace

hipError_t launch_sample(SamplerDev *S, int n_vocab, float *logits, int *out, int accept, int *state, int n_ctx,
                         hipStream_t s) {
    if (!S || !logits || n_vocab <= 0 || ((uintptr_t)logits & 15)) return hipErrorInvalidValue;
    if (n_vocab <= RPT * NT) hipLaunchKernelGGL(k_sample<RPT>, dim3(1), dim3(NT), 0, s, S, logits, out, accept, state, n_ctx);
    else hipLaunchKernelGGL(k_sample<0>, dim3(1), dim3(NT), 0, s, S, logits, out, accept, state, n_ctx);
    return hipGetLastError();
}

hipError_t launch_sampler_push(SamplerDev *S, const int *ids, int n, hipStream_t s) {
    if (!S || (n > 0 && !ids) || n < 0) return hipErrorInvalidValue;
    if (n == 0) return hipSuccess;
    hipLaunchKernelGGL(k_sampler_push, dim3(1), dim3(64), 0, s, S, ids, n);
    return hipGetLastError();
}

}  // namespace g4
