/*
 * g4o.h -- CPU oracle for the quantized weight x activation path.
 *
 * TEST INFRASTRUCTURE ONLY.  Nothing in the product (the g4run_amd package,
 * its HIP library or its C ABI) links, loads or calls this code.  Only
 * tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg use it, and
 * only as the checker or the timed CPU baseline.
 *
 * It restates g4run's CPU arithmetic (src/g4run.h, src/quants.c, src/model.c,
 * src/sampler.c of the reference) in plain C.  Each function cites the lines
 * it follows.  Pinning status of every function (what checks it against
 * something other than its own formula) is listed at the end of this header.
 */
#ifndef G4O_H
#define G4O_H

#include <stdint.h>
#include <stddef.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ggml type ids, g4run.h:80-94 (values are a file-format contract). */
enum {
    G4O_F32 = 0, G4O_F16 = 1, G4O_Q4_0 = 2, G4O_Q8_0 = 8,
    G4O_Q2_K = 10, G4O_Q3_K = 11, G4O_Q4_K = 12, G4O_Q5_K = 13, G4O_Q6_K = 14, G4O_Q8_K = 15,
    G4O_BF16 = 30, G4O_TQ2_0 = 35
};

/* Packed block layouts, g4run.h:107-118.  Byte-for-byte the GGUF formats. */
#pragma pack(push, 1)
typedef struct { uint16_t d; uint8_t qs[16]; }  g4o_q4_0;                      /* 18 B  */
typedef struct { uint16_t d; int8_t  qs[32]; }  g4o_q8_0;                      /* 34 B  */
typedef struct { float d; int8_t qs[256]; int16_t bsums[16]; } g4o_q8_K;       /* 292 B */
typedef struct { uint8_t scales[16]; uint8_t qs[64]; uint16_t d, dmin; } g4o_q2_K;        /* 84 B */
typedef struct { uint8_t hmask[32]; uint8_t qs[64]; uint8_t scales[12]; uint16_t d; } g4o_q3_K; /* 110 B */
typedef struct { uint16_t d, dmin; uint8_t scales[12]; uint8_t qs[128]; } g4o_q4_K;       /* 144 B */
typedef struct { uint16_t d, dmin; uint8_t scales[12]; uint8_t qh[32]; uint8_t qs[128]; } g4o_q5_K; /* 176 B */
typedef struct { uint8_t ql[128]; uint8_t qh[64]; int8_t scales[16]; uint16_t d; } g4o_q6_K; /* 210 B */
typedef struct { uint8_t qs[64]; uint16_t d; } g4o_tq2_0;                                    /* 66 B */
#pragma pack(pop)

/* ---- type table (gguf.c:11-46) ---- */
int    g4o_type_blck(int type);
size_t g4o_type_size(int type);
size_t g4o_row_size(int type, int64_t n);       /* 0 when n % blck != 0 (gguf.c:42-46) */

/* ---- fp16 (g4run.h:37-59, quants.c:27-46) ---- */
float    g4o_fp16_to_fp32(uint16_t h);
uint16_t g4o_fp32_to_fp16(float f);
int      g4o_nearest_int(float f);              /* quants.c:63-67 */
void     g4o_fp16_to_fp32_n(const uint16_t *h, float *f, int64_t n);
void     g4o_fp32_to_fp16_n(const float *f, uint16_t *h, int64_t n);

/* ---- activation / KV quantizers (quants.c:71-175) ---- */
void g4o_quantize_q8_0(const float *x, g4o_q8_0 *y, int64_t n);   /* AVX2 semantics, quants.c:74-109 */
void g4o_quantize_q8_K(const float *x, g4o_q8_K *y, int64_t n);   /* quants.c:146-175 */
void g4o_quantize_q4_0(const float *x, g4o_q4_0 *y, int64_t n);   /* quants.c:125-144 */

/* ---- dequant (quants.c:364-531) ---- */
int  g4o_dequant_row(int type, const void *x, float *y, int64_t n);  /* returns -1 on unknown type */

/* ---- per-block integer sums ----
 * q8_0 / q4_0: one int32 per 32-block: sum_j w_j * a_j (q4_0 elements are q-8).
 * q2_K / q4_K / q5_K: two int32 per superblock: isum (scale-weighted quant sum) and
 *              msum (min-weighted bsums), so that the superblock value is
 *              d_a*(d_w*isum - dmin_w*msum)   (quants.c:633-652, 743-758).
 * q3_K: one int32 per superblock, isum = sum_s (scale_s-32) * sum q3*q8.
 * q6_K: one int32 per superblock, isum = sum_s scale_s * sum (q6-32)*q8
 *       (quants.c:582-622).
 * tq2_0: one int32 per superblock, sum (trit-1)*q8 (quants.c:564-580).       */
void g4o_block_sums(int type, const void *w, const void *a, int64_t n, int32_t *out);

/* ---- scalar reference dots (quants.c:535-762), sequential fp32 order ---- */
float g4o_dot_ref(int type, const void *w, const void *a, int64_t n);

/* ---- shipped AVX2-order dots: same integer lanes, the same fused
 *      multiply-adds and the same horizontal-sum tree as quants.c:820-1259,
 *      written in portable C.  Results are bit-identical to the reference's
 *      AVX2 build. ---- */
float g4o_dot(int type, const void *w, const void *a, int64_t n);
float g4o_dot_f16(const uint16_t *w, const uint16_t *a, int64_t n);   /* quants.c:1319-1331 */
float g4o_dot_bf16(const uint16_t *w, const float *a, int64_t n);     /* quants.c:1333-1347 */
uint16_t g4o_fp32_to_bf16(float f);                                   /* g4run.h:64-68 */

/* ---- activation class + prep, matmul driver (model.c:132-270) ---- */
int    g4o_act_type(int wtype);                 /* G4O_Q8_0 or G4O_Q8_K, -1 otherwise */
size_t g4o_act_stride(int wtype, int64_t ncols);/* 64-B padded per-token stride (model.c:148-149) */
void   g4o_prep_act(int wtype, const float *x, int64_t ncols, int nb, void *qa);
/* Y[b][r] = dot(W[r,:], act[b]); token-major like model.c:197.  nthreads<=1: serial. */
void   g4o_matmul(int wtype, const void *W, const void *act, size_t act_stride,
                  float *Y, int64_t ncols, int64_t nrows, int nb, int nthreads);

/* ---- thread pool: static contiguous split, caller runs chunk 0
 *      (model.c:59-65, 117-125), pthreads instead of Win32 ---- */
typedef void (*g4o_pf_fn)(int64_t r0, int64_t r1, void *ud, int tid);
void g4o_pool_start(int nthreads);
void g4o_pool_stop(void);
void g4o_parallel_for(int64_t total, g4o_pf_fn fn, void *ud);

/* ---- dot-function table used by the matmul driver; lets the same driver time
 *      either this restatement or the reference's compiled kernels ---- */
typedef float (*g4o_dot_fn)(const void *w, const void *a, int64_t n);
void g4o_set_dot_fn(int wtype, g4o_dot_fn fn);  /* NULL restores the restatement */
typedef float (*g4o_dot_f16_fn)(const void *w, const uint16_t *a, int64_t n);
void g4o_set_dot_f16_fn(g4o_dot_f16_fn fn);      /* attention's f16 score dot */

/* ---- norms, rope, gelu, argmax (model.c:338-367, g4run.h:73-77, quants.c:49-58,
 *      sampler.c:139-144) ---- */
void     g4o_rms_norm(const float *x, const float *w, float *y, int n, float eps);
void     g4o_rope_cache(float *cs, int n_dims, int pos, float freq_base);
void     g4o_rope_cache_ff(float *cs, int n_dims, int pos, float freq_base, const float *ff);
void     g4o_rope_apply(float *x, const float *cs, int n_dims);
uint16_t g4o_gelu_table_entry(uint16_t h);      /* fp16(gelu_tanh(fp32(h))) */
float    g4o_gelu(float x);
int      g4o_argmax(const float *v, int n);

/* ---- decode attention over one KV head group (model.c:509-580), GQA mapping
 *      kvh = h / (n_head/n_kv) as model.c:1099.  KV rows: [slot][n_kv][hd] in
 *      kv_type (G4O_F16 or G4O_Q8_0).  q: [n_head][hd] fp32, out: [n_head][hd].
 *      Attends positions 0..pos (no ring wrap; slots >= pos+1). ---- */
void g4o_attn_decode(const float *q, const void *kc, const void *vc, int kv_type,
                     int n_head, int n_kv, int hd, int pos, float *out, int nthreads);
/* The same over positions j0..pos held in slot j % slots (the sliding window
 * and KV ring of model.c:517-537); out is zero when pos < j0. */
void g4o_attn_window(const float *q, const void *kc, const void *vc, int kv_type, int n_head, int n_kv, int hd,
                     int pos, int j0, int slots, float *out, int nthreads);
/* kv_store (model.c:583-589) */
void g4o_kv_store(int kv_type, void *dst, const float *src, int hd);

/* ---- synthetic gemma-style decoder (layer order of model.c:647-736,
 *      head model.c:766-769), weights supplied by the caller ---- */
typedef struct {
    int n_layer, n_embd, n_head, n_kv, hd, n_ff, n_vocab, n_ctx;
    float rope_base, eps;
    int kv_type;                     /* G4O_F16 or G4O_Q8_0 */
    /* per-layer weights, q4_0 rows (or any supported type in wtype) */
    int wtype;
    const void **wqkv;               /* [n_layer] fused rows: q (n_head*hd) | k (n_kv*hd) | v (n_kv*hd) */
    const void **wo;                 /* [n_layer] n_embd rows x n_head*hd cols */
    const void **wgu;                /* [n_layer] fused rows: gate (n_ff) | up (n_ff) */
    const void **wdown;              /* [n_layer] n_embd rows x n_ff cols */
    const float **attn_norm, **q_norm, **k_norm, **post_attn_norm, **ffn_norm, **post_ffw_norm;
    const float *output_norm;
    int head_type;                   /* G4O_Q8_0 */
    const void *head;                /* n_vocab rows x n_embd (tied with the input embedding) */
    void **kc, **vc;                 /* [n_layer] caches: n_ctx slots x n_kv x hd */
} g4o_model;

/* One decode step for `token` at `pos`.  Writes logits[n_vocab], returns argmax.
 * scratch must hold g4o_model_scratch_bytes(m) bytes. */
size_t g4o_model_scratch_bytes(const g4o_model *m);
int    g4o_model_decode(const g4o_model *m, int token, int pos, float *logits,
                        void *scratch, int nthreads);
/* The step's parts: the embedding x = dequant(head row) * sqrt(n_embd), one
 * layer in place on x (its K/V rows stored at pos), and the head (returns the
 * argmax).  g4o_model_decode is embed, every layer, head. */
void   g4o_model_embed(const g4o_model *m, int token, float *x);
void   g4o_model_layer(const g4o_model *m, int il, int pos, float *x, void *scratch, int nthreads);
/* The layer's parts (g4o_model_layer = qkv, attn, post): the Wqkv projection
 * of x into qkv[(n_head + 2 n_kv) hd]; the q/k/v preparation, K/V store at pos
 * and attention from qkv (prepared in place) into att[n_head hd]; and Wo, the
 * residual adds and the FFN from att onto x in place. */
void   g4o_model_qkv(const g4o_model *m, int il, const float *x, float *qkv, void *scratch, int nthreads);
void   g4o_model_attn(const g4o_model *m, int il, int pos, float *qkv, float *att, void *scratch, int nthreads);
void   g4o_model_post(const g4o_model *m, int il, float *x, const float *att, void *scratch, int nthreads);
int    g4o_model_head(const g4o_model *m, const float *x, float *logits, void *scratch, int nthreads);

/* ---- the gemma4 forward (model.c:592-799) ----
 * One KV head; sliding-window layers (is_swa) use head dim hd_swa, RoPE base
 * rope_base_swa and a ring of 576 slots (G4_SWA_RING, g4run.h:24-26); full
 * layers hd_full, rope_base_full with frequency factors rope_freqs and n_ctx
 * slots.  Layers >= n_layer_kv have no K/V projection and attend the cache of
 * layer n_layer_kv-2 (sliding) or n_layer_kv-1 (full).  RoPE covers the whole
 * head (n_rot == head dim). */
typedef struct { const void *data; int type; int64_t ncols, nrows; } g4o_mat;   /* GGUF rows */
typedef struct {
    g4o_mat wq, wk, wv, wo, gate, up, down, inp_gate, proj;     /* wv.data NULL: V = K */
    const float *attn_norm, *q_norm, *k_norm, *post_attn_norm, *ffn_norm, *post_ffw_norm, *post_norm;
    float out_scale;
} g4o_gemma_layer;
typedef struct {
    int n_layer, n_layer_kv, n_embd, n_head, n_vocab, n_embd_per_layer, hd_full, hd_swa, n_swa, n_ctx;
    float rope_base_full, rope_base_swa, eps, softcap;
    const uint8_t *is_swa;
    const int *n_ff;
    int kv_type;                         /* G4O_F16, G4O_Q8_0 or G4O_Q4_0 */
    g4o_mat tok_embd, per_layer_tok_embd, per_layer_model_proj;
    const float *per_layer_proj_norm, *output_norm, *rope_freqs;
    const g4o_gemma_layer *layers;
    void **kc, **vc;                     /* [n_layer_kv] caches, g4o_gemma_cache_bytes each */
} g4o_gemma;
size_t g4o_gemma_cache_bytes(const g4o_gemma *g, int il);
/* tokens[0..nb) at positions pos0..: logits [nb][n_vocab] of every position
 * and, if hnext, the head's input rms(x)*output_norm [nb][n_embd] */
void   g4o_gemma_forward(const g4o_gemma *g, const int *tokens, int nb, int pos0, float *logits, float *hnext,
                         int nthreads);

/* ---- sampling chain (sampler.c), laid out as g4run.h:464-482's g4_sampler
 *      so one structure drives this restatement and the reference build ---- */
typedef struct {
    float temp;                      /* <= 0: greedy */
    int   top_k;
    float top_p;
    float repeat_penalty;
    int   repeat_last_n;
    float freq_penalty;
    float presence_penalty;
    int   no_repeat_ngram;           /* 0/1 off, else the n-gram length */
    uint64_t seed;
    uint64_t rng[4];                 /* all zero: seeded from `seed` on first use */
    int  *recent;                    /* ring of the last recent_cap accepted ids */
    int   recent_cap, recent_n, recent_head;
    int  *cnt;                       /* per-id counts kept by accept */
    int  *ban_ids;
    int   n_ban, ban_cap;
    int   n_vocab;
} g4o_sampler;
void     g4o_sampler_init(g4o_sampler *s, int n_vocab);   /* sampler.c:5-14 */
void     g4o_sampler_reset(g4o_sampler *s);               /* sampler.c:16-20 */
void     g4o_sampler_free(g4o_sampler *s);                /* sampler.c:22-25 */
void     g4o_sampler_ban(g4o_sampler *s, int id);         /* sampler.c:27-35 */
void     g4o_sampler_accept(g4o_sampler *s, int id);      /* sampler.c:37-48 */
uint64_t g4o_sampler_rng_next(g4o_sampler *s);            /* sampler.c:51-70 */
int      g4o_sample(g4o_sampler *s, float *logits);       /* sampler.c:74-210 */

/*
 * Pinning (checks that are not a retyping of the function's own formula):
 *   fp16 both ways        exhaustive 65536-code round trip; RNE on ties and
 *                         subnormals vs numpy float16 casts (tests)
 *   quantize_q8_0/q8_K    bit-exact vs the reference build oracle/_ref and the
 *                         committed fixtures; closed-form special cases
 *   quantize_q4_0         bit-exact vs oracle/_ref
 *   dequant               bit-exact vs oracle/_ref on random blocks and the
 *                         committed fixtures (q8_0 .. q6_K, tq2_0, f16, bf16)
 *   block_sums            brute-force dequant identity in exact integer math,
 *                         and unit-scale calls of the reference _ref dots
 *   dot_ref               within the reference selftest's tolerance (1e-3,
 *                         quants.c:1583) of the reference build's scalar _ref
 *                         dots: the README build vectorises those under
 *                         -Ofast, so their bits are not the C text's
 *   dot (AVX2 order)      bit-exact vs the reference's AVX2 dots (oracle/_ref)
 *   dot_f16 / dot_bf16    bit-exact vs the reference's g4_dot_f16 / g4_dot_bf16
 *                         (fixtures with a scalar tail, n = 2053)
 *   tq2_0 (dequant, sums, dots)
 *                         bit-exact vs the reference's fixtures and live build,
 *                         sums also by the brute-force dequant identity
 *   fp32_to_bf16          float64 nearest-even selection over random and
 *                         special bit patterns (NaN, overflow, subnormals)
 *   matmul                row loop of dot(); x4 == x1 invariant
 *   rms_norm, rope, attention, decode graph
 *                         model.c does not compile here (windows.h), so these
 *                         are checked by invariants (softmax of a one-hot,
 *                         rope as a rotation, attention of identical keys,
 *                         float64 recomputation) -- see tests/test_oracle_model.py
 *   attention, q8_0/q4_0 caches
 *                         identical keys give exactly the fp32 weight
 *                         (float)(1/n) (an fp16-rounded weight fails at n = 3),
 *                         a one-hot key, and a float64 recomputation from the
 *                         dequantized K/V and the q8_0-quantized query that
 *                         rejects an fp16 query or fp16 weights by 10x
 *   gelu table            against math.tanh-based float64 recomputation
 *   sampler               bit-exact vs the reference's sampler.c built in place
 *                         with the same IEEE flags (oracle/_ref): drawn ids,
 *                         rewritten logits and RNG words over seeded runs with
 *                         bans, n-gram blocks, penalties, ties, NaN and -inf;
 *                         without that build, by closed forms (greedy = first
 *                         argmax, top_k = 1, the splitmix/xoshiro words of a
 *                         published seed, draw frequencies of a two-token
 *                         softmax)
 */

#ifdef __cplusplus
}
#endif
#endif
