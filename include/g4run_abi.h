/*
 * g4run_abi.h -- g4run.h's quantized-kernel entry points, exported by
 * libg4hip.so under their reference names and signatures, so that a C caller
 * written against g4run.h (model.c-style code, its self-tests, tools) links
 * -lg4hip in place of quants.c for these symbols.
 *
 * Every function here runs on the GPU: the host buffers of one call are
 * staged to device memory (per host thread), the library's gfx950 kernel
 * runs, and the result is copied back before the call returns.  They are
 * therefore synchronous and carry a per-call latency of a few tens of
 * microseconds; a caller that streams weights every token uses the resident
 * path of g4hip.h (g4h_tensor_load + g4h_matmul) instead, as
 * tests/c/g4gpu.c shows.
 *
 * Semantics kept from the reference:
 *   - names, argument types, block layouts and type ids (g4run.h:28-169);
 *   - the dots, quantizers and dequant are pure and re-entrant, callable from
 *     many host threads at once (each thread has its own staging buffers and
 *     stream);
 *   - the x4 dots give, for each of the 4 activations, exactly the 1-token dot
 *     (g4run.h:148-149);
 *   - a row length that is not a multiple of the block size is truncated to
 *     whole blocks, as the reference's loops do (e.g. quants.c:966).
 * Results: the quantizers and the dequant are bit-identical to the reference
 * build of quants.c (README flags); the integer block sums inside every dot
 * are exact and the fp32 result is within 1e-3 relative / 1e-5 absolute of
 * the reference's AVX2 dot (the GPU adds in its own order).
 * Differences (the reference has no error channel and exits on an unknown
 * type, quants.c:529): a call that cannot run (no device, unknown type, a
 * HIP error) never exits the process; dots return NaN, dequant writes NaN,
 * quantizers leave the output untouched, and g4h_last_error() (g4hip.h)
 * holds the message.
 * The sampler entry points (g4run.h:464-489) are exported too; see below.
 * Not exported: the scalar _ref twins and g4_selftest_quants (the
 * reference's own CPU self-test oracle, g4run.h:159-169) and the JIT requant
 * quantizers g4_quantize_q2_K / q3_K (g4run.h:124-125, a load-time
 * conversion outside the decode hot path).
 */
#ifndef G4RUN_ABI_H
#define G4RUN_ABI_H

#include <stdbool.h>
#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* g4run.h:28-29 */
typedef uint16_t g4_fp16;
typedef uint16_t g4_bf16;

/* g4run.h:32-33: filled by g4_init_tables (the inline fp16 helpers of g4run.h
 * read them) */
extern float   g4_fp16_to_fp32_table[65536];
extern g4_fp16 g4_gelu_fp16_table[65536];

/* g4run.h:70: builds both tables on the host and initialises the device
 * (g4h_init on device $G4H_DEVICE, default 0).  Call it first, as main.c:1222
 * does. */
void g4_init_tables(void);

/* g4run.h:96-99 (gguf.c:27-46): the ggml type table of the formats above. */
const char *g4_type_name(int t);
int         g4_type_blck(int t);
size_t      g4_type_size(int t);
size_t      g4_row_size(int t, int64_t n);

/* g4run.h:107-118: packed GGUF blocks (file-format contract). */
#pragma pack(push, 1)
typedef struct { g4_fp16 d; uint8_t qs[16]; } block_q4_0;
typedef struct { g4_fp16 d; int8_t qs[32]; } block_q8_0;
typedef struct { uint8_t ql[128]; uint8_t qh[64]; int8_t scales[16]; g4_fp16 d; } block_q6_K;
typedef struct { uint8_t qs[64]; g4_fp16 d; } block_tq2_0;
typedef struct { float d; int8_t qs[256]; int16_t bsums[16]; } block_q8_K;
typedef struct { uint8_t scales[16]; uint8_t qs[64]; g4_fp16 d; g4_fp16 dmin; } block_q2_K;
typedef struct { uint8_t hmask[32]; uint8_t qs[64]; uint8_t scales[12]; g4_fp16 d; } block_q3_K;
typedef struct { g4_fp16 d; g4_fp16 dmin; uint8_t scales[12]; uint8_t qs[128]; } block_q4_K;
typedef struct { g4_fp16 d; g4_fp16 dmin; uint8_t scales[12]; uint8_t qh[32]; uint8_t qs[128]; } block_q5_K;
#pragma pack(pop)

/* g4run.h:121-123: activation / KV quantizers (n elements). */
void g4_quantize_q8_0(const float *x, block_q8_0 *y, int64_t n);
void g4_quantize_q8_K(const float *x, block_q8_K *y, int64_t n);
void g4_quantize_q4_0(const float *x, block_q4_0 *y, int64_t n);

/* g4run.h:128: one row of any weight format above (and f16, bf16, f32). */
void g4_dequant_row(int type, const void *x, float *y, int64_t n);

/* g4run.h:131-134: the CPU's AVX-512 toggle has no meaning on this path; the
 * flag stays 0 and the setter only records the request. */
extern int g4_avx512;
void g4_set_avx512(int on);
int  g4_avx512_available(void);

/* g4run.h:136-145: one weight row (n elements) against one activation. */
float g4_dot_q4_0_q8_0(const void *w, const void *a, int64_t n);
float g4_dot_q8_0_q8_0(const void *w, const void *a, int64_t n);
float g4_dot_q6_K_q8_K(const void *w, const void *a, int64_t n);
float g4_dot_tq2_0_q8_K(const void *w, const void *a, int64_t n);
float g4_dot_q2_K_q8_K(const void *w, const void *a, int64_t n);
float g4_dot_q3_K_q8_K(const void *w, const void *a, int64_t n);
float g4_dot_q4_K_q8_K(const void *w, const void *a, int64_t n);
float g4_dot_q5_K_q8_K(const void *w, const void *a, int64_t n);
float g4_dot_f16(const void *w, const g4_fp16 *a, int64_t n);
float g4_dot_bf16(const void *w, const float *a, int64_t n);

/* g4run.h:148-157: one weight row against 4 activations; out[i] equals the
 * 1-token dot of a[i] bit for bit. */
void g4_dot_q4_0_q8_0_x4(const void *w, const void *const a[4], int64_t n, float out[4]);
void g4_dot_q8_0_q8_0_x4(const void *w, const void *const a[4], int64_t n, float out[4]);
void g4_dot_q6_K_q8_K_x4(const void *w, const void *const a[4], int64_t n, float out[4]);
void g4_dot_tq2_0_q8_K_x4(const void *w, const void *const a[4], int64_t n, float out[4]);
void g4_dot_q2_K_q8_K_x4(const void *w, const void *const a[4], int64_t n, float out[4]);
void g4_dot_q3_K_q8_K_x4(const void *w, const void *const a[4], int64_t n, float out[4]);
void g4_dot_q4_K_q8_K_x4(const void *w, const void *const a[4], int64_t n, float out[4]);
void g4_dot_q5_K_q8_K_x4(const void *w, const void *const a[4], int64_t n, float out[4]);

/* g4run.h:176-184: a GGUF tensor descriptor (what the loader hands model.c);
 * the resident path uploads tensor->data once (tests/c/g4gpu.c). */
typedef struct {
    char        name[80];
    int         type;
    int         ndim;
    int64_t     ne[4];
    uint64_t    offset;
    const void *data;
} g4_tensor;

/* g4run.h:172-246: the GGUF model file.  g4_gguf_open maps the file (a
 * read-only private mmap; the reference uses a Win32 view, gguf.c:124-160)
 * and parses GGUF v2/v3 as gguf.c:162-404 does: the same metadata keys and
 * defaults, tensor table, alignment, data offsets and bounds checks, and the
 * same architecture checks (gemma4, gemma4-assistant, qwen35).  Tensor data
 * pointers point into the mapping.  g4_gguf_write (a pruning export) and
 * g4_gguf_dump (a debug print) are not exported. */
#define G4_MAX_LAYERS 64                     /* g4run.h:22 */
typedef struct {
    const char *ptr;                         /* into the mapping, not NUL-terminated */
    uint32_t    len;
} g4_str;

typedef struct {
    void    *map_base;
    uint64_t map_size;
    void    *h_file, *h_map;                 /* unused here (NULL) */
    uint32_t version;
    uint64_t n_tensors, n_kv;
    uint64_t data_start;
    uint64_t kv_end;
    uint64_t ff_len_off;
    int      ff_len_vt;
    uint32_t alignment;
    g4_tensor *tensors;
    char  arch[32];
    int   n_layer, n_embd, n_vocab, n_head, n_head_kv;
    int   n_embd_per_layer;
    int   n_ff[G4_MAX_LAYERS];
    int   head_dim_full, head_dim_swa;
    int   n_rot_full, n_rot_swa;
    float rope_base_full, rope_base_swa;
    float rms_eps;
    float final_softcap;
    int   n_swa;
    int   n_kv_shared;
    int   n_layer_kv;
    uint8_t is_swa[G4_MAX_LAYERS];
    int   n_ctx_train;
    bool  is_assistant;
    int   n_embd_out;
    int   n_nextn;
    bool  is_qwen35;
    int   n_embd_head_k, n_embd_head_v;
    int   ssm_d_conv, ssm_d_inner, ssm_d_state, ssm_dt_rank, ssm_n_group;
    int   full_attn_interval;
    int   rope_sections[4];
    uint8_t is_recr[G4_MAX_LAYERS];
    int   tok_pre;
    int      tok_n;
    g4_str  *tok_text;
    const int32_t *tok_type;
    int      merges_n;
    g4_str  *merges;
    int   bos_id, eos_id, eot_id, unk_id, pad_id;
    bool  add_bos;
    float meta_temp, meta_top_p;
    int   meta_top_k;
    g4_str chat_template;
} g4_model_file;

int  g4_gguf_open(g4_model_file *mf, const char *path, bool verbose);
void g4_gguf_close(g4_model_file *mf);
const g4_tensor *g4_find_tensor(const g4_model_file *mf, const char *name);

/* g4run.h:464-489: the sampling chain, with the reference's struct.  The
 * state-keeping calls are host bookkeeping with sampler.c's semantics
 * (sampler.c:5-48: defaults, the 4096-id ring, per-id counts, deduplicated
 * bans); g4_sample stages the logits and the state to the device, runs the
 * chain on the GPU (the kernel of g4h_sample) and copies back the rewritten
 * logits and the RNG words, so the draw, the logits and s->rng are the
 * reference's bit for bit.  g4_sample returns -1 (g4h_last_error() says why)
 * when it cannot run: no device, or a recent_cap other than
 * g4_sampler_init's 4096. */
typedef struct {
    float temp;
    int   top_k;
    float top_p;
    float repeat_penalty;
    int   repeat_last_n;
    float freq_penalty;
    float presence_penalty;
    int   no_repeat_ngram;
    uint64_t seed;
    uint64_t rng[4];
    int  *recent;
    int   recent_cap, recent_n, recent_head;
    int  *cnt;
    int  *ban_ids;
    int   n_ban, ban_cap;
    int   n_vocab;
} g4_sampler;

void g4_sampler_init(g4_sampler *s, int n_vocab);
void g4_sampler_reset(g4_sampler *s);
void g4_sampler_ban(g4_sampler *s, int id);
void g4_sampler_free(g4_sampler *s);
void g4_sampler_accept(g4_sampler *s, int id);
int  g4_sample(g4_sampler *s, float *logits);

#ifdef __cplusplus
}
#endif
#endif
