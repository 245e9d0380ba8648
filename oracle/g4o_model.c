/*
 * g4o_model.c -- CPU oracle: activation prep, the row-parallel matmul driver,
 * its thread pool, norms, RoPE, GELU, decode attention and the synthetic
 * gemma-style decode step, restated from the reference's src/model.c.
 *
 * TEST INFRASTRUCTURE ONLY (see g4o.h).  The reference's model.c does not
 * compile on Linux (it includes windows.h), so this is a restatement from the
 * source text; the pool uses pthreads and a sense-reversing generation
 * counter instead of WaitOnAddress.
 */
#include "g4o.h"

#include <math.h>
#include <pthread.h>
#if defined(__F16C__) && defined(__FMA__)
#include <immintrin.h>
#endif
#include <stdlib.h>
#include <string.h>

/* ------------------------------------------------------------ dot table -- */
static float dot_q8_0(const void *w, const void *a, int64_t n) { return g4o_dot(G4O_Q8_0, w, a, n); }
static float dot_q4_0(const void *w, const void *a, int64_t n) { return g4o_dot(G4O_Q4_0, w, a, n); }
static float dot_q2_K(const void *w, const void *a, int64_t n) { return g4o_dot(G4O_Q2_K, w, a, n); }
static float dot_q3_K(const void *w, const void *a, int64_t n) { return g4o_dot(G4O_Q3_K, w, a, n); }
static float dot_q5_K(const void *w, const void *a, int64_t n) { return g4o_dot(G4O_Q5_K, w, a, n); }
static float dot_q6_K(const void *w, const void *a, int64_t n) { return g4o_dot(G4O_Q6_K, w, a, n); }
static float dot_tq2_0(const void *w, const void *a, int64_t n) { return g4o_dot(G4O_TQ2_0, w, a, n); }
static float dot_f16w(const void *w, const void *a, int64_t n) { return g4o_dot_f16(w, a, n); }
static float dot_bf16w(const void *w, const void *a, int64_t n) { return g4o_dot_bf16(w, a, n); }
static float dot_q4_K(const void *w, const void *a, int64_t n) { return g4o_dot(G4O_Q4_K, w, a, n); }

static g4o_dot_fn dot_override[64];

static g4o_dot_fn dot_for(int wtype) {
    if (wtype >= 0 && wtype < 64 && dot_override[wtype]) return dot_override[wtype];
    switch (wtype) {
    case G4O_Q8_0: return dot_q8_0;
    case G4O_Q4_0: return dot_q4_0;
    case G4O_Q2_K: return dot_q2_K;
    case G4O_Q3_K: return dot_q3_K;
    case G4O_Q5_K: return dot_q5_K;
    case G4O_Q6_K: return dot_q6_K;
    case G4O_TQ2_0: return dot_tq2_0;
    case G4O_F16: return dot_f16w;
    case G4O_BF16: return dot_bf16w;
    case G4O_Q4_K: return dot_q4_K;
    default: return NULL;
    }
}
void g4o_set_dot_fn(int wtype, g4o_dot_fn fn) {
    if (wtype >= 0 && wtype < 64) dot_override[wtype] = fn;
}
static g4o_dot_f16_fn dot_f16_override;
void g4o_set_dot_f16_fn(g4o_dot_f16_fn fn) { dot_f16_override = fn; }
static float dot_f16(const uint16_t *w, const uint16_t *a, int64_t n) {
    return dot_f16_override ? dot_f16_override(w, a, n) : g4o_dot_f16(w, a, n);
}

/* ---------------------------------------------------------- thread pool -- */
/* model.c:42-125: a fixed pool; each parallel_for splits [0,total) into
 * nth contiguous chunks of ceil(total/nth); the caller runs chunk 0; runs
 * serially when total < 4. */
static struct {
    pthread_mutex_t mu;
    pthread_cond_t go, done_cv;
    pthread_t th[256];
    int nth, running, quit;
    unsigned gen;
    int done;
    g4o_pf_fn fn;
    void *ud;
    int64_t total;
} P = { .mu = PTHREAD_MUTEX_INITIALIZER, .go = PTHREAD_COND_INITIALIZER, .done_cv = PTHREAD_COND_INITIALIZER };

static void pool_chunk(int idx) {
    int64_t per = (P.total + P.nth - 1) / P.nth;
    int64_t r0 = per * idx, r1 = r0 + per;
    if (r1 > P.total) r1 = P.total;
    if (r0 < r1) P.fn(r0, r1, P.ud, idx);
}

static void *pool_worker(void *arg) {
    int idx = (int)(intptr_t)arg;
    unsigned seen = 0;
    pthread_mutex_lock(&P.mu);
    for (;;) {
        while (P.gen == seen && !P.quit) pthread_cond_wait(&P.go, &P.mu);
        if (P.quit) break;
        seen = P.gen;
        pthread_mutex_unlock(&P.mu);
        pool_chunk(idx);
        pthread_mutex_lock(&P.mu);
        if (++P.done == P.nth - 1) pthread_cond_signal(&P.done_cv);
    }
    pthread_mutex_unlock(&P.mu);
    return NULL;
}

void g4o_pool_start(int n) {
    if (P.running) g4o_pool_stop();
    if (n < 1) n = 1;
    if (n > 256) n = 256;
    P.nth = n; P.quit = 0; P.gen = 0;
    for (int i = 1; i < n; i++) pthread_create(&P.th[i], NULL, pool_worker, (void *)(intptr_t)i);
    P.running = 1;
}

void g4o_pool_stop(void) {
    if (!P.running) return;
    pthread_mutex_lock(&P.mu);
    P.quit = 1;
    pthread_cond_broadcast(&P.go);
    pthread_mutex_unlock(&P.mu);
    for (int i = 1; i < P.nth; i++) pthread_join(P.th[i], NULL);
    P.running = 0; P.nth = 1;
}

void g4o_parallel_for(int64_t total, g4o_pf_fn fn, void *ud) {
    if (!P.running || P.nth <= 1 || total < 4) { fn(0, total, ud, 0); return; }
    pthread_mutex_lock(&P.mu);
    P.fn = fn; P.ud = ud; P.total = total; P.done = 0; P.gen++;
    pthread_cond_broadcast(&P.go);
    pthread_mutex_unlock(&P.mu);
    pool_chunk(0);
    pthread_mutex_lock(&P.mu);
    while (P.done != P.nth - 1) pthread_cond_wait(&P.done_cv, &P.mu);
    pthread_mutex_unlock(&P.mu);
}

/* ------------------------------------------------------- act prep/matmul -- */
/* model.c:132-141 (the formats on this path only). */
int g4o_act_type(int wtype) {
    switch (wtype) {
    case G4O_Q4_0: case G4O_Q8_0: return G4O_Q8_0;
    case G4O_Q2_K: case G4O_Q3_K: case G4O_Q4_K: case G4O_Q5_K: case G4O_Q6_K: case G4O_TQ2_0: return G4O_Q8_K;
    case G4O_F16: return G4O_F16;                     /* AC_F16 (model.c:163-170) */
    case G4O_BF16: return G4O_F32;                    /* AC_BF16: bf16-rounded fp32 (model.c:172-180) */
    default: return -1;
    }
}
/* model.c:148-149, 156-157: per-token stride rounded up to 64 bytes. */
size_t g4o_act_stride(int wtype, int64_t ncols) {
    size_t st = g4o_row_size(g4o_act_type(wtype), ncols);
    return (st + 63) & ~(size_t)63;
}
void g4o_prep_act(int wtype, const float *x, int64_t ncols, int nb, void *qa) {
    size_t st = g4o_act_stride(wtype, ncols);
    for (int b = 0; b < nb; b++) {
        uint8_t *dst = (uint8_t *)qa + (size_t)b * st;
        const float *src = x + (size_t)b * ncols;
        if (wtype == G4O_F16) {
            for (int64_t i = 0; i < ncols; i++) ((uint16_t *)dst)[i] = g4o_fp32_to_fp16(src[i]);
        } else if (wtype == G4O_BF16) {
            for (int64_t i = 0; i < ncols; i++) {
                uint32_t u = (uint32_t)g4o_fp32_to_bf16(src[i]) << 16;
                memcpy((float *)dst + i, &u, 4);
            }
        } else if (g4o_act_type(wtype) == G4O_Q8_0) {
            g4o_quantize_q8_0(src, (g4o_q8_0 *)dst, ncols);
        } else {
            g4o_quantize_q8_K(src, (g4o_q8_K *)dst, ncols);
        }
    }
}

typedef struct {
    g4o_dot_fn dot;
    const uint8_t *W; size_t row_bytes;
    const uint8_t *act; size_t act_stride;
    float *Y; int64_t ncols, nrows; int nb;
} mm_job;

/* model.c:202-254: weight row outer, tokens inner, so the row stays in cache
 * across the batch.  The x4 dots are bit-identical to x1 (g4run.h:148-157),
 * so the token loop calls the x1 dot for every token. */
static void mm_rows(int64_t r0, int64_t r1, void *p, int tid) {
    (void)tid;
    const mm_job *u = p;
    for (int64_t r = r0; r < r1; r++) {
        const void *row = u->W + (size_t)r * u->row_bytes;
        for (int b = 0; b < u->nb; b++)
            u->Y[(size_t)b * u->nrows + r] = u->dot(row, u->act + (size_t)b * u->act_stride, u->ncols);
    }
}

void g4o_matmul(int wtype, const void *W, const void *act, size_t act_stride,
                float *Y, int64_t ncols, int64_t nrows, int nb, int nthreads) {
    mm_job u = { dot_for(wtype), W, g4o_row_size(wtype, ncols), act, act_stride, Y, ncols, nrows, nb };
    if (!u.dot) return;
    if (nthreads > 1) g4o_parallel_for(nrows, mm_rows, &u);
    else mm_rows(0, nrows, &u, 0);
}

/* --------------------------------------------------------- norms / rope -- */
/* model.c:338-345: sum of squares in double, fp32 scale 1/sqrt(mean+eps). */
void g4o_rms_norm(const float *x, const float *w, float *y, int n, float eps) {
    double s = 0.0;
    for (int i = 0; i < n; i++) s += (double)x[i] * x[i];
    const float mean = (float)(s / n);
    const float scale = 1.0f / sqrtf(mean + eps);
    for (int i = 0; i < n; i++) y[i] = w ? x[i] * scale * w[i] : x[i] * scale;
}

/* model.c:349-358: theta_i = pos * base^(-2i/n), accumulated by repeated
 * multiplication as the reference does. */
void g4o_rope_cache(float *cs, int n_dims, int pos, float freq_base) { g4o_rope_cache_ff(cs, n_dims, pos, freq_base, NULL); }

/* with per-pair frequency factors ff (model.c:352-353: theta / ff[i]) */
void g4o_rope_cache_ff(float *cs, int n_dims, int pos, float freq_base, const float *ff) {
    const float theta_scale = powf(freq_base, -2.0f / n_dims);
    float theta = (float)pos;
    for (int i = 0; i < n_dims / 2; i++) {
        const float t = ff ? theta / ff[i] : theta;
        cs[2 * i] = cosf(t);
        cs[2 * i + 1] = sinf(t);
        theta *= theta_scale;
    }
}
/* model.c:359-367: NeoX rotation of the pair (i, i + n/2). */
void g4o_rope_apply(float *x, const float *cs, int n_dims) {
    const int h = n_dims / 2;
    for (int i = 0; i < h; i++) {
        const float c = cs[2 * i], s = cs[2 * i + 1];
        const float a = x[i], b = x[i + h];
        x[i] = a * c - b * s;
        x[i + h] = a * s + b * c;
    }
}

/* quants.c:49-58 and g4run.h:73-77: GELU (tanh form) tabulated per fp16 code. */
uint16_t g4o_gelu_table_entry(uint16_t h) {
    const float x = g4o_fp16_to_fp32(h);
    const float g = 0.5f * x * (1.0f + tanhf(0.79788456080286535587989211986876f * x * (1.0f + 0.044715f * x * x)));
    return g4o_fp32_to_fp16(g);
}
static uint16_t *gelu_tab;
static pthread_once_t gelu_once = PTHREAD_ONCE_INIT;
static void gelu_init(void) {
    gelu_tab = malloc(65536 * sizeof(uint16_t));
    for (uint32_t i = 0; i < 65536; i++) gelu_tab[i] = g4o_gelu_table_entry((uint16_t)i);
}
float g4o_gelu(float x) {
    if (x <= -10.0f) return 0.0f;
    if (x >= 10.0f) return x;
    pthread_once(&gelu_once, gelu_init);
    return g4o_fp16_to_fp32(gelu_tab[g4o_fp32_to_fp16(x)]);
}

/* sampler.c:139-144: first index of the maximum. */
int g4o_argmax(const float *v, int n) {
    int best = 0; float bv = v[0];
    for (int i = 1; i < n; i++) if (v[i] > bv) { bv = v[i]; best = i; }
    return best;
}

/* ------------------------------------------------------------ attention -- */
/* model.c:583-589 */
void g4o_kv_store(int kv_type, void *dst, const float *src, int hd) {
    if (kv_type == G4O_Q8_0) g4o_quantize_q8_0(src, dst, hd);
    else if (kv_type == G4O_Q4_0) g4o_quantize_q4_0(src, dst, hd);
    else { uint16_t *d = dst; for (int i = 0; i < hd; i++) d[i] = g4o_fp32_to_fp16(src[i]); }
}

typedef struct {
    const float *q; const uint8_t *kc, *vc; int kv_type;
    int n_head, n_kv, hd, pos; float *out;
    size_t row_bytes;
    int j0, slots;           /* first attended position; positions live in slot j % slots */
} attn_job;

/* model.c:509-580 for one decode token, one query head per work item.
 * Query rounded to the K cache's activation form; scores without a 1/sqrt(d)
 * factor; softmax with the sum in double; an f16 V cache is weighted by the
 * fp16-rounded probability, a quantized V cache by the fp32 one. */
static void attn_heads(int64_t h0, int64_t h1, void *p, int tid) {
    (void)tid;
    const attn_job *u = p;
    const int hd = u->hd, nv = u->pos - u->j0 + 1, grp = u->n_head / u->n_kv;
    float *att = malloc((size_t)nv * sizeof(float));
    float *vtmp = malloc((size_t)hd * sizeof(float));
    uint16_t *q16 = malloc((size_t)hd * 2);
    g4o_q8_0 *q8 = malloc((size_t)(hd / 32) * sizeof(g4o_q8_0));
    for (int64_t h = h0; h < h1; h++) {
        const int kvh = (int)h / grp;
        const float *qh = u->q + (size_t)h * hd;
        float *o = u->out + (size_t)h * hd;
        if (u->kv_type == G4O_F16) for (int i = 0; i < hd; i++) q16[i] = g4o_fp32_to_fp16(qh[i]);
        else g4o_quantize_q8_0(qh, q8, hd);
        float mx = -INFINITY;
        for (int j = 0; j < nv; j++) {
            const uint8_t *krow = u->kc + ((size_t)((u->j0 + j) % u->slots) * u->n_kv + kvh) * u->row_bytes;
            float s;
            if (u->kv_type == G4O_F16) s = dot_f16((const uint16_t *)krow, q16, hd);
            else s = dot_for(u->kv_type)(krow, q8, hd);
            att[j] = s;
            if (s > mx) mx = s;
        }
        double sum = 0.0;
        for (int j = 0; j < nv; j++) { float e = expf(att[j] - mx); att[j] = e; sum += e; }
        const float inv = (float)(1.0 / sum);
        for (int i = 0; i < hd; i++) o[i] = 0.0f;
        for (int j = 0; j < nv; j++) {
            const uint8_t *vrow = u->vc + ((size_t)((u->j0 + j) % u->slots) * u->n_kv + kvh) * u->row_bytes;
            if (u->kv_type == G4O_F16) {
                const float wj = g4o_fp16_to_fp32(g4o_fp32_to_fp16(att[j] * inv));
                const uint16_t *v = (const uint16_t *)vrow;
#if defined(__F16C__) && defined(__FMA__)
                /* model.c:553-562: 8 elements per step, F16C widening + FMA
                 * (element-wise identical to the scalar form below) */
                const __m256 wv = _mm256_set1_ps(wj);
                for (int i = 0; i < hd; i += 8) {
                    const __m256 vf = _mm256_cvtph_ps(_mm_loadu_si128((const __m128i *)(v + i)));
                    _mm256_storeu_ps(o + i, _mm256_fmadd_ps(wv, vf, _mm256_loadu_ps(o + i)));
                }
#else
                for (int i = 0; i < hd; i++) o[i] = fmaf(wj, g4o_fp16_to_fp32(v[i]), o[i]);
#endif
            } else {
                const float wj = att[j] * inv;
                g4o_dequant_row(u->kv_type, vrow, vtmp, hd);
                for (int i = 0; i < hd; i++) o[i] = fmaf(wj, vtmp[i], o[i]);
            }
        }
    }
    free(att); free(vtmp); free(q16); free(q8);
}

void g4o_attn_window(const float *q, const void *kc, const void *vc, int kv_type, int n_head, int n_kv, int hd,
                     int pos, int j0, int slots, float *out, int nthreads) {
    attn_job u = { q, kc, vc, kv_type, n_head, n_kv, hd, pos, out,
                   kv_type == G4O_F16 ? (size_t)hd * 2 : g4o_row_size(kv_type, hd), j0, slots };
    if (pos < j0) {                                   /* nothing to attend (model.c:523) */
        for (int64_t i = 0; i < (int64_t)n_head * hd; i++) out[i] = 0.0f;
        return;
    }
    if (nthreads > 1) g4o_parallel_for(n_head, attn_heads, &u);
    else attn_heads(0, n_head, &u, 0);
}

void g4o_attn_decode(const float *q, const void *kc, const void *vc, int kv_type,
                     int n_head, int n_kv, int hd, int pos, float *out, int nthreads) {
    g4o_attn_window(q, kc, vc, kv_type, n_head, n_kv, hd, pos, 0, pos + 1, out, nthreads);
}

/* ---------------------------------------------------------- decode step -- */
typedef struct {
    float *x, *xb, *qkv, *att, *ff, *rc;
    uint8_t *qa;
} scratch_t;

static size_t align64(size_t v) { return (v + 63) & ~(size_t)63; }

size_t g4o_model_scratch_bytes(const g4o_model *m) {
    const int qkv = (m->n_head + 2 * m->n_kv) * m->hd;
    int wide = m->n_ff > m->n_embd ? m->n_ff : m->n_embd;
    if (m->n_head * m->hd > wide) wide = m->n_head * m->hd;
    size_t s = 0;
    s += align64((size_t)m->n_embd * 4) * 2;
    s += align64((size_t)qkv * 4);
    s += align64((size_t)m->n_head * m->hd * 4);
    s += align64((size_t)2 * m->n_ff * 4);
    s += align64((size_t)m->hd * 4);
    s += align64(g4o_act_stride(m->wtype, wide) + g4o_act_stride(m->head_type, m->n_embd));
    return s;
}

static scratch_t carve(const g4o_model *m, void *base) {
    const int qkv = (m->n_head + 2 * m->n_kv) * m->hd;
    uint8_t *p = base;
    scratch_t s;
    s.x = (float *)p;   p += align64((size_t)m->n_embd * 4);
    s.xb = (float *)p;  p += align64((size_t)m->n_embd * 4);
    s.qkv = (float *)p; p += align64((size_t)qkv * 4);
    s.att = (float *)p; p += align64((size_t)m->n_head * m->hd * 4);
    s.ff = (float *)p;  p += align64((size_t)2 * m->n_ff * 4);
    s.rc = (float *)p;  p += align64((size_t)m->hd * 4);
    s.qa = p;
    return s;
}

static void mm(const g4o_model *m, int wtype, const void *W, const float *x, int64_t ncols,
               int64_t nrows, float *y, uint8_t *qa, int nthreads) {
    g4o_prep_act(wtype, x, ncols, 1, qa);
    g4o_matmul(wtype, W, qa, g4o_act_stride(wtype, ncols), y, ncols, nrows, 1, nthreads);
    (void)m;
}

/* The layer order of model.c:647-736 without the gemma4-only parts
 * (per-layer embeddings, SWA ring, shared KV, softcap), in three parts:
 *   qkv   xb = rms(x)*attn_norm; q|k|v = Wqkv xb
 *   attn  q,k <- rms-norm per head with q_norm/k_norm then RoPE; v <- rms-norm
 *         without weight (model.c:684); store k,v at pos; attention
 *   post  xb = Wo att; x += rms(xb)*post_attn_norm; xb = rms(x)*ffn_norm;
 *         g|u = Wgu xb; h = gelu(g)*u; xb = Wdown h; x += rms(xb)*post_ffw_norm */
void g4o_model_qkv(const g4o_model *m, int il, const float *x, float *qkv, void *scratch, int nthreads) {
    scratch_t s = carve(m, scratch);
    const int E = m->n_embd, rows = (m->n_head + 2 * m->n_kv) * m->hd;
    g4o_rms_norm(x, m->attn_norm[il], s.xb, E, m->eps);
    mm(m, m->wtype, m->wqkv[il], s.xb, E, rows, qkv, s.qa, nthreads);
}

void g4o_model_attn(const g4o_model *m, int il, int pos, float *qkv, float *att, void *scratch, int nthreads) {
    scratch_t s = carve(m, scratch);
    const int hd = m->hd, H = m->n_head, KV = m->n_kv;
    const int qrows = H * hd, kvrows = KV * hd;
    const size_t kv_row = m->kv_type == G4O_F16 ? (size_t)hd * 2 : g4o_row_size(m->kv_type, hd);
    g4o_rope_cache(s.rc, hd, pos, m->rope_base);
    float *q = qkv, *k = qkv + qrows, *v = qkv + qrows + kvrows;
    for (int h = 0; h < H; h++) {
        g4o_rms_norm(q + h * hd, m->q_norm[il], q + h * hd, hd, m->eps);
        g4o_rope_apply(q + h * hd, s.rc, hd);
    }
    for (int h = 0; h < KV; h++) {
        g4o_rms_norm(k + h * hd, m->k_norm[il], k + h * hd, hd, m->eps);
        g4o_rope_apply(k + h * hd, s.rc, hd);
        g4o_rms_norm(v + h * hd, NULL, v + h * hd, hd, m->eps);
        g4o_kv_store(m->kv_type, (uint8_t *)m->kc[il] + ((size_t)pos * KV + h) * kv_row, k + h * hd, hd);
        g4o_kv_store(m->kv_type, (uint8_t *)m->vc[il] + ((size_t)pos * KV + h) * kv_row, v + h * hd, hd);
    }
    g4o_attn_decode(q, m->kc[il], m->vc[il], m->kv_type, H, KV, hd, pos, att, nthreads);
}

void g4o_model_post(const g4o_model *m, int il, float *x, const float *att, void *scratch, int nthreads) {
    scratch_t s = carve(m, scratch);
    const int E = m->n_embd, F = m->n_ff;
    mm(m, m->wtype, m->wo[il], att, m->n_head * m->hd, E, s.xb, s.qa, nthreads);
    g4o_rms_norm(s.xb, m->post_attn_norm[il], s.xb, E, m->eps);
    for (int i = 0; i < E; i++) x[i] += s.xb[i];

    g4o_rms_norm(x, m->ffn_norm[il], s.xb, E, m->eps);
    mm(m, m->wtype, m->wgu[il], s.xb, E, 2 * F, s.ff, s.qa, nthreads);
    for (int i = 0; i < F; i++) s.ff[i] = g4o_gelu(s.ff[i]) * s.ff[F + i];
    mm(m, m->wtype, m->wdown[il], s.ff, F, E, s.xb, s.qa, nthreads);
    g4o_rms_norm(s.xb, m->post_ffw_norm[il], s.xb, E, m->eps);
    for (int i = 0; i < E; i++) x[i] += s.xb[i];
}

/* One layer, in place on x[n_embd]. */
void g4o_model_layer(const g4o_model *m, int il, int pos, float *x, void *scratch, int nthreads) {
    scratch_t s = carve(m, scratch);
    g4o_model_qkv(m, il, x, s.qkv, scratch, nthreads);
    g4o_model_attn(m, il, pos, s.qkv, s.att, scratch, nthreads);
    g4o_model_post(m, il, x, s.att, scratch, nthreads);
}

/* Embedding: dequantized head row times sqrt(n_embd) (model.c:605-612). */
void g4o_model_embed(const g4o_model *m, int token, float *x) {
    const int E = m->n_embd;
    g4o_dequant_row(m->head_type, (const uint8_t *)m->head + (size_t)token * g4o_row_size(m->head_type, E), x, E);
    const float es = sqrtf((float)E);
    for (int i = 0; i < E; i++) x[i] *= es;
}

/* Head: rms(x)*output_norm, logits = head x (model.c:767-769), greedy argmax
 * (sampler.c:139-144). */
int g4o_model_head(const g4o_model *m, const float *x, float *logits, void *scratch, int nthreads) {
    scratch_t s = carve(m, scratch);
    g4o_rms_norm(x, m->output_norm, s.xb, m->n_embd, m->eps);
    mm(m, m->head_type, m->head, s.xb, m->n_embd, m->n_vocab, logits, s.qa, nthreads);
    return g4o_argmax(logits, m->n_vocab);
}

int g4o_model_decode(const g4o_model *m, int token, int pos, float *logits, void *scratch, int nthreads) {
    scratch_t s = carve(m, scratch);
    g4o_model_embed(m, token, s.x);
    for (int il = 0; il < m->n_layer; il++) g4o_model_layer(m, il, pos, s.x, scratch, nthreads);
    return g4o_model_head(m, s.x, logits, scratch, nthreads);
}
