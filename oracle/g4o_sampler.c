/*
 * g4o_sampler.c -- CPU restatement of the reference's sampling chain
 * (src/sampler.c): bans -> no-repeat-ngram -> repeat/freq/presence penalties
 * -> greedy | top-k (bounded min-heap) -> top-p -> temperature -> draw.
 *
 * TEST INFRASTRUCTURE ONLY (see g4o.h).  The struct is laid out as the
 * reference's g4_sampler (g4run.h:464-482) so that one ctypes structure drives
 * both this file and the reference build in oracle/_ref.
 *
 * The arithmetic is the C text's, evaluated in IEEE order with no contraction
 * (this file is built with -ffp-contract=off -fno-fast-math): the oracle/_ref
 * build of sampler.c uses the same flags, and the tests compare both bit for
 * bit (returned ids, the logits the call rewrites and the RNG words).
 */
#include "g4o.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

#define G4O_SAMPLER_RING 4096       /* sampler.c:10 */
#define G4O_TOPK_MAX 512            /* sampler.c:147 */

void g4o_sampler_init(g4o_sampler *s, int n_vocab) {       /* sampler.c:5-14 */
    memset(s, 0, sizeof *s);
    s->temp = 1.0f;
    s->top_k = 64;
    s->top_p = 0.95f;
    s->repeat_penalty = 1.0f;
    s->repeat_last_n = 128;
    s->n_vocab = n_vocab;
    s->recent_cap = G4O_SAMPLER_RING;
    s->recent = (int *)malloc((size_t)s->recent_cap * sizeof(int));
    s->cnt = (int *)calloc((size_t)n_vocab, sizeof(int));
    s->seed = 0xdeadbeefull;
}

void g4o_sampler_reset(g4o_sampler *s) {                   /* sampler.c:16-20 */
    s->recent_n = 0;
    s->recent_head = 0;
    if (s->cnt) memset(s->cnt, 0, (size_t)s->n_vocab * sizeof(int));
}

void g4o_sampler_free(g4o_sampler *s) {                    /* sampler.c:22-25 */
    free(s->recent);
    free(s->cnt);
    free(s->ban_ids);
    memset(s, 0, sizeof *s);
}

void g4o_sampler_ban(g4o_sampler *s, int id) {             /* sampler.c:27-35 */
    if (id < 0 || id >= s->n_vocab) return;
    for (int i = 0; i < s->n_ban; i++)
        if (s->ban_ids[i] == id) return;
    if (s->n_ban == s->ban_cap) {
        s->ban_cap = s->ban_cap ? 2 * s->ban_cap : 16;
        s->ban_ids = (int *)realloc(s->ban_ids, (size_t)s->ban_cap * sizeof(int));
    }
    s->ban_ids[s->n_ban++] = id;
}

/* The ring keeps the last recent_cap ids, oldest at recent_head
 * (sampler.c:37-48). */
void g4o_sampler_accept(g4o_sampler *s, int id) {
    const int cap = s->recent_cap;
    if (s->recent_n == cap) {
        const int old = s->recent[s->recent_head];
        if (s->cnt[old] > 0) s->cnt[old]--;
        s->recent[s->recent_head] = id;
        s->recent_head = (s->recent_head + 1) % cap;
    } else {
        s->recent[(s->recent_head + s->recent_n) % cap] = id;
        s->recent_n++;
    }
    s->cnt[id]++;
}

/* i-th oldest id of the ring */
static int ring_at(const g4o_sampler *s, int i) { return s->recent[(s->recent_head + i) % s->recent_cap]; }

/* splitmix64 seeding of all-zero state, then the xoshiro256+ step
 * (sampler.c:51-70) */
uint64_t g4o_sampler_rng_next(g4o_sampler *s) {
    uint64_t *w = s->rng;
    if ((w[0] | w[1] | w[2] | w[3]) == 0) {
        uint64_t z = s->seed + 0x9e3779b97f4a7c15ull;
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
    return out;
}

typedef struct { float v; int id; } cand;

/* Rewrites `logits` as the reference does (bans and n-gram hits to -inf,
 * penalised ids), then returns the drawn id. */
int g4o_sample(g4o_sampler *s, float *logits) {
    const int nv = s->n_vocab;

    /* hard bans (sampler.c:78) */
    for (int j = 0; j < s->n_ban; j++) logits[s->ban_ids[j]] = -INFINITY;

    /* no-repeat-ngram (sampler.c:82-101): every earlier occurrence of the
     * newest m = min(N-1, 64) ids bans the id that followed it */
    if (s->no_repeat_ngram >= 2 && s->recent_n >= s->no_repeat_ngram) {
        const int m = s->no_repeat_ngram - 1 < 64 ? s->no_repeat_ngram - 1 : 64;
        const int n = s->recent_n;
        for (int p = 0; p + m < n; p++) {
            int hit = 1;
            for (int j = 0; j < m && hit; j++) hit = ring_at(s, p + j) == ring_at(s, n - m + j);
            if (hit) logits[ring_at(s, p + m)] = -INFINITY;
        }
    }

    /* penalties over the newest min(repeat_last_n, recent_n) ids
     * (sampler.c:104-137): each distinct id once, with its count in the window */
    if ((s->repeat_penalty != 1.0f || s->freq_penalty != 0 || s->presence_penalty != 0) && s->repeat_last_n > 0 &&
        s->recent_n > 0) {
        const int win = s->repeat_last_n < s->recent_n ? s->repeat_last_n : s->recent_n;
        const int newest = s->recent_n - 1;
        for (int i = 0; i < win; i++) {
            const int id = ring_at(s, newest - i);
            int first = 1, count = 0;
            for (int j = 0; j < i && first; j++) first = ring_at(s, newest - j) != id;
            if (!first) continue;
            for (int j = 0; j < win; j++) count += ring_at(s, newest - j) == id;
            float l = logits[id];
            if (s->repeat_penalty != 1.0f) l = l <= 0 ? l * s->repeat_penalty : l / s->repeat_penalty;
            const float fterm = (float)count * s->freq_penalty;
            l -= fterm + (count > 0 ? s->presence_penalty : 0.0f);
            logits[id] = l;
        }
    }

    /* greedy: first index of the maximum (sampler.c:140-144) */
    if (s->temp <= 0.0f) return g4o_argmax(logits, nv);

    /* top-k through a bounded min-heap over the ids in order (sampler.c:147-168) */
    int k = s->top_k > 0 && s->top_k < G4O_TOPK_MAX ? s->top_k : G4O_TOPK_MAX;
    if (k > nv) k = nv;
    cand heap[G4O_TOPK_MAX];
    int hn = 0;
    for (int i = 0; i < nv; i++) {
        const float l = logits[i];
        if (hn < k) {
            int j = hn++;
            heap[j].v = l;
            heap[j].id = i;
            while (j > 0) {
                const int up = (j - 1) / 2;
                if (!(heap[j].v < heap[up].v)) break;
                const cand t = heap[up];
                heap[up] = heap[j];
                heap[j] = t;
                j = up;
            }
        } else if (l > heap[0].v) {
            heap[0].v = l;
            heap[0].id = i;
            int j = 0;
            for (;;) {
                const int a = 2 * j + 1, b = 2 * j + 2;
                int lo = j;
                if (a < k && heap[a].v < heap[lo].v) lo = a;
                if (b < k && heap[b].v < heap[lo].v) lo = b;
                if (lo == j) break;
                const cand t = heap[lo];
                heap[lo] = heap[j];
                heap[j] = t;
                j = lo;
            }
        }
    }
    /* descending insertion sort of the heap array (sampler.c:170-176) */
    cand c[G4O_TOPK_MAX];
    memcpy(c, heap, (size_t)hn * sizeof(cand));
    for (int i = 1; i < hn; i++) {
        const cand v = c[i];
        int j = i - 1;
        while (j >= 0 && c[j].v < v.v) {
            c[j + 1] = c[j];
            j--;
        }
        c[j + 1] = v;
    }

    /* top-p over the fp32 softmax of the candidates, double sums
     * (sampler.c:179-194) */
    int n = hn;
    {
        float pf[G4O_TOPK_MAX];
        double sum = 0;
        for (int i = 0; i < n; i++) {
            pf[i] = expf(c[i].v - c[0].v);
            sum += pf[i];
        }
        if (s->top_p < 1.0f && s->top_p > 0.0f) {
            double cum = 0;
            int keep = n;
            for (int i = 0; i < n; i++) {
                cum += pf[i] / sum;
                if (cum >= s->top_p) {
                    keep = i + 1;
                    break;
                }
            }
            n = keep;
        }
    }

    /* temperature softmax in double and the draw (sampler.c:197-209); the
     * shift is the fp32 quotient c[0]/temp */
    const float shift = c[0].v / s->temp;
    double pd[G4O_TOPK_MAX], sum = 0;
    for (int i = 0; i < n; i++) {
        pd[i] = exp((double)c[i].v / s->temp - shift);
        sum += pd[i];
    }
    const double r = (double)(g4o_sampler_rng_next(s) >> 11) / 9007199254740992.0 * sum;
    double cum = 0;
    for (int i = 0; i < n; i++) {
        cum += pd[i];
        if (r < cum) return c[i].id;
    }
    return c[n - 1].id;
}
