/*
 * g4hip.h -- C ABI of the MI355X (gfx950) quantized weight x activation path.
 *
 * This is the drop-in boundary for the hot path of the reference's g4run
 * (a GGUF CPU inference engine).  Every entry point below names the reference
 * interface it replaces.  Conventions:
 *   - plain C, opaque handles, pointers and sizes only; `stream` is a
 *     hipStream_t passed as void* (NULL = the null stream);
 *   - all tensors/activations named *_dev live in device memory;
 *   - every call returns an int status (G4H_OK == 0) and never exits the
 *     process (the reference's g4_dequant_row calls exit(1), quants.c:529);
 *     g4h_last_error() gives a message for the calling thread;
 *   - calls are stream-ordered and asynchronous unless stated otherwise;
 *   - block types and ids are the GGUF/ggml ones of g4run.h:80-118.
 */
#ifndef G4HIP_H
#define G4HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Type ids: identical to enum g4_type, g4run.h:80-94 (Q8_K is ggml's id 15,
 * used by the reference only as the K-quant activation format). */
enum {
    G4H_F32 = 0, G4H_F16 = 1, G4H_Q4_0 = 2, G4H_Q8_0 = 8,
    G4H_Q2_K = 10, G4H_Q3_K = 11, G4H_Q4_K = 12, G4H_Q5_K = 13, G4H_Q6_K = 14, G4H_Q8_K = 15,
    G4H_BF16 = 30, G4H_TQ2_0 = 35
};

enum {
    G4H_OK = 0,
    G4H_ERR_ARG = 1,      /* null pointer, bad size, bad stride           */
    G4H_ERR_TYPE = 2,     /* type not supported on this path              */
    G4H_ERR_SHAPE = 3,    /* n not a multiple of the block size (the reference
                             silently truncates, e.g. quants.c:966)        */
    G4H_ERR_NOMEM = 4,    /* device allocation failed                     */
    G4H_ERR_DEVICE = 5,   /* no gfx950 device / not initialised           */
    G4H_ERR_HIP = 6,      /* a HIP runtime call failed                    */
    G4H_ERR_TIMEOUT = 7   /* a bounded device-side wait gave up (the
                             one-launch attention's hand-off); the outputs
                             it owned are NaN                             */
};

/* ------------------------------------------------------------ runtime ---- */
/* Replaces g4_init_tables() (g4run.h:70, main.c:1222): selects `device`,
 * checks it is gfx950, uploads the fp16 GELU table. */
int         g4h_init(int device);
const char *g4h_last_error(void);
const char *g4h_status_str(int status);
/* Test hook: make the next `n` device allocations fail with G4H_ERR_NOMEM
 * (lets host code exercise the failure path without a real OOM). */
void        g4h_debug_fail_alloc(int n);
/* Test hook: with on != 0, the one-launch attention's hand-off polls wait for
 * a tag that no store carries and give up after 64 retries (instead of 2^20),
 * so every such wait fails while every kernel still runs to its end and the
 * failure path (g4h_attn_status, g4h_model_status, G4H_ERR_TIMEOUT) can be
 * tested deterministically.  0 restores normal operation. */
void        g4h_debug_attn_timeout(int on);

/* Plumbing (thin wrappers over HIP so that callers need no HIP headers). */
int g4h_malloc(void **ptr, size_t bytes);
int g4h_free(void *ptr);
int g4h_memcpy_h2d(void *dst_dev, const void *src, size_t bytes, void *stream);
int g4h_memcpy_d2h(void *dst, const void *src_dev, size_t bytes, void *stream);
int g4h_memcpy_d2d(void *dst_dev, const void *src_dev, size_t bytes, void *stream);
int g4h_memset(void *dst_dev, int value, size_t bytes, void *stream);
int g4h_stream_create(void **stream);
int g4h_stream_destroy(void *stream);
int g4h_stream_synchronize(void *stream);
int g4h_event_create(void **event);
int g4h_event_destroy(void *event);
int g4h_event_record(void *event, void *stream);
int g4h_event_elapsed_ms(float *ms, void *start, void *stop);   /* synchronizes on stop */
int g4h_graph_begin(void *stream);                              /* hipStreamBeginCapture */
int g4h_graph_end(void *stream, void **graph_exec);             /* capture -> instantiated graph */
int g4h_graph_launch(void *graph_exec, void *stream);
int g4h_graph_destroy(void *graph_exec);

/* ----------------------------------------------------- sizes / classes ---- */
/* g4_row_size (g4run.h:99, gguf.c:42-46): 0 when n is not a multiple of the
 * block size or the type is unknown. */
size_t g4h_row_size(int type, int64_t n);
/* act_class (model.c:132-141): activation format a weight type dots against
 * (G4H_Q8_0 for q4_0/q8_0, G4H_Q8_K for q2_K/q3_K/q4_K/q5_K/q6_K/tq2_0, G4H_F16
 * for f16, G4H_F32 -- bf16-rounded fp32 rows -- for bf16), -1 otherwise. */
int    g4h_act_type(int wtype);
/* prep_act stride (model.c:148-149,156-157): per-token bytes, 64-B padded. */
size_t g4h_act_stride(int wtype, int64_t ncols);

/* ---------------------------------------------------------- quantizers ---- */
/* g4_quantize_q8_0 / g4_quantize_q8_K / g4_quantize_q4_0 (g4run.h:121-123),
 * applied to `rows` rows of n floats (x row stride x_stride floats) writing
 * GGUF blocks at y_stride bytes per row.  Bit-identical to the reference
 * build (README flags) of quants.c:71-175. */
int g4h_quantize_q8_0(const float *x_dev, size_t x_stride, void *y_dev, size_t y_stride,
                      int64_t n, int rows, void *stream);
int g4h_quantize_q8_K(const float *x_dev, size_t x_stride, void *y_dev, size_t y_stride,
                      int64_t n, int rows, void *stream);
int g4h_quantize_q4_0(const float *x_dev, size_t x_stride, void *y_dev, size_t y_stride,
                      int64_t n, int rows, void *stream);

/* g4_dequant_row (g4run.h:128) for `rows` GGUF rows of n elements. */
int g4h_dequant_rows(int type, const void *x_dev, size_t x_stride, float *y_dev, size_t y_stride,
                     int64_t n, int rows, void *stream);

/* g4_dot_<fmt> (g4run.h:137-143) applied to `rows` raw GGUF weight rows at
 * w_stride bytes against one quantized activation row:
 *   out[r] = g4_dot_<wtype>(w + r*w_stride, a, n). */
int g4h_vec_dot(int wtype, const void *w_dev, size_t w_stride, const void *a_dev, int64_t n,
                int rows, float *out_dev, void *stream);

/* --------------------------------------------------- resident weights ---- */
/* A weight matrix resident in HBM in the layout the kernels stream (scales
 * split from quants so every quant load is an aligned 128-bit load).  This is
 * what replaces a g4_tensor's `data` pointer (g4run.h:177-184) on the GPU. */
typedef struct g4h_tensor g4h_tensor;

int    g4h_tensor_create(int type, int64_t ncols, int64_t nrows, g4h_tensor **out);
/* Load GGUF rows (nrows x g4h_row_size(type,ncols) bytes, contiguous) from host
 * memory (src_is_device == 0) or device memory, repacking on the device. */
int    g4h_tensor_load(g4h_tensor *t, const void *rows, int src_is_device, void *stream);
/* Write the tensor back as contiguous GGUF rows (device destination). */
int    g4h_tensor_store(const g4h_tensor *t, void *rows_dev, void *stream);
int    g4h_tensor_free(g4h_tensor *t);
size_t g4h_tensor_bytes(const g4h_tensor *t);     /* resident bytes */
int    g4h_tensor_info(const g4h_tensor *t, int *type, int64_t *ncols, int64_t *nrows);

/* ------------------------------------------------------------- matmul ---- */
/* matmul_b (model.c:257-270) with prep_act (model.c:144-187) fused ahead:
 *   Y[b][r] = dot(W[r,:], act[b]),  b < nb,  r < nrows, Y token-major.
 * Either x_dev (nb x ncols floats, quantized here to W's activation format) or
 * pre_dev (already-quantized activations, nb rows at pre_stride bytes) is
 * given; the other is NULL.  Token b's outputs are bit-identical for any nb
 * within one kernel family (g4run.h:148-157 contract); families switch at
 * nb thresholds given by g4h_matmul_path(). */
int g4h_matmul(const g4h_tensor *W, const float *x_dev, const void *pre_dev, size_t pre_stride,
               float *Y_dev, int nb, void *stream);
/* Same with an explicit kernel family: 0 = auto (g4h_matmul_path), 1 = the
 * GEMV family (token chunks of <= 8 staged per workgroup), 2 = matrix-core
 * tiles: int8 for q8_0 / q4_0 / q4_K / q6_K weights (every per-block or
 * per-superblock integer sum exact, fp32 scaling in a fixed order), f16 / bf16
 * for f16 / bf16 rows of whole 16-column steps (exact products, fp32 sums);
 * token rows independent of nb.  g4h_matmul_path returns the family auto
 * picks: 2 for those weights from 9 tokens on, else 1. */
int g4h_matmul_ex(const g4h_tensor *W, const float *x_dev, const void *pre_dev, size_t pre_stride,
                  float *Y_dev, int nb, int path, void *stream);
int g4h_matmul_path(const g4h_tensor *W, int nb);
/* g4h_matmul_ex without any device allocation -- no counterpart in the
 * reference; for callers that cannot allocate (code under HIP graph capture,
 * serving loops, harnesses that forbid hipMalloc).  Where g4h_matmul_ex takes
 * its scratch (the activations quantized from x_dev, the matrix-core path's
 * planar copy) from a per-stream pool it may grow, this call uses a fixed
 * scratch array of g4h_matmul_noalloc_max_bytes() (4 MiB) per device, set up by
 * g4h_init; a call that needs more fails with G4H_ERR_ARG.  The caller still
 * passes W, x_dev / pre_dev and Y_dev.  Results equal g4h_matmul_ex's bit for
 * bit.  Every call on one device shares that array: calls that overlap on one
 * device (different streams, different host threads) race; nothing in the
 * array needs to start at zero. */
int    g4h_matmul_noalloc(const g4h_tensor *W, const float *x_dev, const void *pre_dev, size_t pre_stride,
                          float *Y_dev, int nb, int path, void *stream);
size_t g4h_matmul_noalloc_max_bytes(void);
/* Diagnostic (no reference counterpart): the kernel instantiation and launch
 * shape g4h_matmul_ex would use, e.g. "k_gemv<q4_0,nb=1,lpr=32,upl=4> grid=256
 * block=512", written NUL-terminated into buf (at most len bytes).  Profiles
 * and benchmarks name the kernel they time with it. */
int g4h_matmul_describe(const g4h_tensor *W, int nb, int path, char *buf, size_t len);
/* Diagnostic (no reference counterpart): the read floor.  One launch reads
 * `bytes` (a multiple of 16, src 16-byte aligned) once with the GEMV's 128-bit
 * non-temporal loads -- workgroups of `threads` (64..1024, a multiple of 64),
 * `loads` (1..8) loads per thread -- and writes ny floats of y (0 to skip), the
 * one output per row a GEMV writes.  It computes nothing: benchmarks time it
 * beside a GEMV over the same bytes to show what the memory system gives one
 * launch of that size. */
int g4h_read_floor(const void *src, size_t bytes, float *y, int64_t ny, int threads, int loads, void *stream);

/* Per-block integer sums of every row of W against token `tok` of pre_dev:
 * q8_0/q4_0 one int32 per 32-block, q3_K/q6_K/tq2_0 one per superblock, q2_K/q4_K/q5_K
 * two per superblock (scale-weighted quant sum, min-weighted bsum), i.e. the
 * integers the reference's dots scale (quants.c:535-818).
 * sums_dev: nrows x count. */
int g4h_block_sums(const g4h_tensor *W, const void *pre_dev, size_t pre_stride, int tok,
                   int32_t *sums_dev, void *stream);

/* ---------------------------------------------------------- attention ---- */
/* Decode attention (attn_kernel, model.c:509-580) for one token: n_head query
 * heads (q_dev: n_head x hd fp32) over cached positions 0..n_pos-1.  Cache
 * rows [slot][n_kv][hd] in kv_type (G4H_F16, G4H_Q8_0 or G4H_Q4_0) for K and V; query
 * head h reads KV head h/(n_head/n_kv) (model.c:1099); no 1/sqrt(hd) factor
 * (model.c:538).  hd in {64,128,192,256}; n_head/n_kv in {1,2,4,8}.
 * ws_dev: g4h_attn_workspace_bytes() bytes of caller-owned scratch (the
 * reference's attbuf, model.c:465).  out_dev: n_head x hd fp32.
 * The workspace carries state from call to call for the one-launch form (an
 * epoch word each launch advances on the device, and hand-off words tagged
 * with it): the first call on a workspace clears it (ws_bytes of it), later
 * calls of any position count (graph replays included) do not, until a
 * three-pass or batch call stores untagged data there (past its first 256
 * bytes, which hold the error and epoch words).  Memory that held
 * anything else since must have been freed with g4h_free, or be zeroed before
 * it is used as a workspace again.  Calls that overlap on one workspace race. */
size_t g4h_attn_workspace_bytes(int n_head, int hd, int n_pos);
/* Diagnostic (no reference counterpart): *passes = the launches
 * g4h_attn_decode makes for this shape, 1 when the f16 cache runs as one fused
 * launch (its grid of n_kv x ceil(n_pos/128) workgroups fits on the device at
 * once), else 3 (score, value and combine passes).  Both give the same bits;
 * G4H_ATTN_PASSES=3 in the environment forces the three passes. */
int g4h_attn_passes(int kv_type, int n_head, int n_kv, int hd, int n_pos, int *passes);
int g4h_attn_decode(const float *q_dev, const void *kc_dev, const void *vc_dev, int kv_type,
                    int n_head, int n_kv, int hd, int n_pos, float *out_dev,
                    void *ws_dev, size_t ws_bytes, void *stream);
/* Whether any attention call on ws_dev since the last query had a hand-off wait
 * give up (*failed = 1; its outputs hold NaN), else *failed = 0.  The
 * attention calls are asynchronous (and may be graph-replayed), so they cannot
 * return this status themselves; this call synchronizes `stream`, reads the
 * workspace's error word and clears it; after a failure the next call on
 * ws_dev clears the whole workspace first (a workgroup that started late may
 * have left words under the next launch's tag).  No reference counterpart:
 * the CPU attention (model.c:509-580) has no cross-thread wait. */
int g4h_attn_status(void *ws_dev, int *failed, void *stream);
/* The same with the sliding window and KV ring of model.c:517-537: the
 * current position is n_pos-1 and it attends positions max(0, n_pos -
 * window) .. n_pos-1 (window 0: all).  ring > 0 (then 0 < window <= ring):
 * the caches are a ring in which position j's row sits at slot j % ring and
 * again at slot j % ring + ring (2*ring slots), so every window is one
 * contiguous run -- the reference keeps one copy in G4_SWA_RING slots.
 * ws_bytes must cover g4h_attn_workspace_bytes(n_head, hd, min(window, n_pos)). */
int g4h_attn_decode_window(const float *q_dev, const void *kc_dev, const void *vc_dev, int kv_type, int n_head, int n_kv,
                           int hd, int n_pos, int window, int ring, float *out_dev, void *ws_dev, size_t ws_bytes,
                           void *stream);
/* attn_kernel over a batch of nb new tokens (model.c:509-545 with nb > 1):
 * token b sits at position pos0 + b and attends cached positions
 * [0, pos0 + b] -- causal, the batch's own rows already stored in kc/vc.
 * q_dev / out_dev: nb x n_head x hd fp32.  With ws_bytes covering
 * g4h_attn_prefill_workspace_bytes(n_head, hd, pos0, nb) all tokens run in
 * one set of three launches (scores, values, combine; a token grid
 * dimension); with at least g4h_attn_workspace_bytes(n_head, hd, pos0 + nb)
 * they run as stream-ordered decode-attention launches on ws.  Either way
 * every token's row has the bits of g4h_attn_decode at its position. */
int g4h_attn_prefill(const float *q_dev, const void *kc_dev, const void *vc_dev, int kv_type,
                     int n_head, int n_kv, int hd, int pos0, int nb, float *out_dev,
                     void *ws_dev, size_t ws_bytes, void *stream);
/* The same batch on the matrix cores, for prompt prefill: f16 caches, head
 * dims 64 / 128 / 256 / 512, 1 / 2 / 4 / 8 query heads per KV head, with the
 * sliding window and ring of g4h_attn_decode_window (window 0: all positions;
 * on a ring nb <= ring - window + 1).  Tiles of 32 (token, head) rows share
 * every K and V row: scores and weighted value sums on f16 MFMA (exact
 * products, fp32 sums), the softmax statistics and the fp16 weights of the
 * decode kernels.  Rows are within the attention's tolerance of
 * g4h_attn_prefill's, not bit-identical to them, and a token's row has the
 * same bits in any batch (positions cut at fixed multiples of 128 / 256);
 * a non-finite V row reaches the earlier rows of its tile.  ws_bytes >= g4h_attn_prefill_workspace_bytes
 * (n_head, hd, pos0, nb).  Asynchronous.  No counterpart in the reference. */
int g4h_attn_prefill_mm(const float *q_dev, const void *kc_dev, const void *vc_dev, int kv_type, int n_head, int n_kv,
                        int hd, int pos0, int nb, int window, int ring, float *out_dev, void *ws_dev, size_t ws_bytes,
                        void *stream);
/* workspace bytes of g4h_attn_prefill's one-set form (a block of scores,
 * chunk statistics and partials per token); 0 for a bad argument.  No
 * counterpart in the reference, which attends on the CPU. */
size_t g4h_attn_prefill_workspace_bytes(int n_head, int hd, int pos0, int nb);
/* kv_store (model.c:583-589): `rows` rows of hd floats into cache rows
 * dst_stride bytes apart (0 = packed rows), as f16 (RNE) or q8_0 / q4_0
 * blocks. */
int g4h_kv_store(int kv_type, const float *src_dev, void *dst_dev, int hd, int rows,
                 size_t dst_stride, void *stream);

/* -------------------------------------------------------- decode step ---- */
/* A gemma-style decoder resident on the device (the model behind
 * g4_ctx_init / g4_forward, g4run.h:303-311): layer order of model.c:647-736
 * (RMSNorm, fused QKV projection, q/k RMSNorm + NeoX RoPE, KV store, attention,
 * Wo, post-attention norm + residual, fused gate/up, GELU(gate)*up, down,
 * post-FFN norm + residual), a tied q8_0 embedding / output head
 * (model.c:605-612, 766-769) and greedy argmax (sampler.c:139-144).  Weights
 * are random-initialised on the device: N(0, 0.02) quantized with the q4_0 /
 * q8_0 quantizers, norm weights N(1, 0.05). */
typedef struct {
    int n_layer, n_embd, n_head, n_kv, head_dim, n_ff, n_vocab, n_ctx;
    float rope_base, rms_eps;
    int wtype;       /* layer weights: G4H_Q4_0 or G4H_Q8_0 */
    int head_type;   /* G4H_Q8_0 */
    int kv_type;     /* G4H_F16, G4H_Q8_0 or G4H_Q4_0 */
} g4h_model_config;
typedef struct g4h_model g4h_model;

enum { G4H_W_QKV = 0, G4H_W_O = 1, G4H_W_GU = 2, G4H_W_DOWN = 3, G4H_W_HEAD = 4 };
enum { G4H_N_ATTN = 0, G4H_N_Q = 1, G4H_N_K = 2, G4H_N_POST_ATTN = 3, G4H_N_FFN = 4,
       G4H_N_POST_FFW = 5, G4H_N_OUTPUT = 6 };

int  g4h_model_create(const g4h_model_config *cfg, uint64_t seed, g4h_model **out);
int  g4h_model_free(g4h_model *m);
/* Fill every KV slot of every layer with N(0,1) values (stored as kv_type). */
int  g4h_model_fill_kv(g4h_model *m, uint64_t seed, void *stream);
/* g4_forward (g4run.h:309-311): one decode step for `token` at `pos`
 * (synchronous); logits stay on the device (g4h_model_logits), the next token
 * (greedy argmax, or the draw of the sampler set by g4h_model_set_sampler) is
 * returned in *next_token. */
int  g4h_forward(g4h_model *m, int token, int pos, int *next_token, void *stream);
/* The same step reading token/pos from device state and advancing it
 * (token <- argmax or the sampler's draw, pos <- pos+1): asynchronous,
 * capturable in a graph. */
int  g4h_forward_state(g4h_model *m, void *stream);
int  g4h_model_set_state(g4h_model *m, int token, int pos, void *stream);
int  g4h_model_get_state(g4h_model *m, int *token, int *pos, void *stream);
/* Device-side conditions of the state-driven steps since the last set_state
 * (synchronizes `stream`): G4H_STATUS_CTX_FULL -- a step ran at the last
 * position n_ctx-1, so pos did not advance (the reference's full-attention
 * cache has n_ctx slots, model.c:442; a further step re-decodes n_ctx-1 and
 * never indexes past the cache); G4H_STATUS_ATTN_TIMEOUT -- an attention
 * hand-off wait gave up and the logits are NaN (reported once, then cleared).
 * g4h_forward returns G4H_ERR_TIMEOUT in the second case. */
enum { G4H_STATUS_CTX_FULL = 1, G4H_STATUS_ATTN_TIMEOUT = 2 };
int  g4h_model_status(g4h_model *m, int *flags, void *stream);
const float *g4h_model_logits(const g4h_model *m);
/* Diagnostic (no reference counterpart): with trace_dev non-NULL, every later
 * step also copies its intermediate vectors into trace_dev (device memory, fp32):
 * per layer l a record of 4 n_embd + (n_head + 2 n_kv) head_dim + n_head head_dim
 * + n_ff floats -- x (the layer's input; layer 0: the scaled embedding), q|k|v
 * (the projection output; not written when the projection runs inside the
 * attention launch, G4H_DECODE_FUSE bit 16), att (attention output), wo (Wo
 * output), xmid (x after the attention residual), h (gelu(gate)*up; not written
 * without G4H_DECODE_FUSE bit 2) and down (Wdown output) -- then n_embd floats,
 * the x the head normalises.  A CPU implementation can then
 * check each part of each layer on the GPU's own inputs: the whole stack is
 * chaotic at the ulp level (the fp16 rounding of q ahead of the unscaled
 * softmax, model.c:530-538, turns a last-bit difference of the projection into
 * a visible change of the attention output), so only such part-by-part checks
 * hold a per-element tolerance.  The batched forwards write one such step
 * trace per token (token b's at b times a step's size, so trace_dev must hold
 * nb of them; g4h_forward_batch writes the final x of its last token only).
 * NULL turns it off. */
int g4h_model_trace(g4h_model *m, float *trace_dev);
/* The model's fp16 GELU table (65536 codes, device memory): entry h =
 * fp16(gelu_tanh(fp32(h))) as quants.c:48-58 builds g4_gelu_table. */
const uint16_t *g4h_model_gelu_table(const g4h_model *m);
/* Parameter access (for checking against a CPU implementation).  The
 * G4H_W_GU matrix holds its 2*n_ff rows interleaved: row 2i is gate row i,
 * row 2i+1 is up row i (the reference's w_gate_up is [gate | up]). */
g4h_tensor *g4h_model_matrix(g4h_model *m, int layer, int which);
float      *g4h_model_norm(g4h_model *m, int layer, int which);
int         g4h_model_kv(g4h_model *m, int layer, void **k_dev, void **v_dev, size_t *bytes);
size_t      g4h_model_weight_bytes(const g4h_model *m);

/* ---------------------------------------------------- batched forward ---- */
/* g4_forward_batch (g4run.h:312-313, model.c:758-776): the layers for nb
 * tokens (host ids, 1 <= nb <= 64 = G4_BATCH_MAX) at positions pos0 ..
 * pos0+nb-1 (< n_ctx), their K/V rows stored; with want_logits the last
 * token's logits go to g4h_model_logits.  Synchronous.  A prompt chunk:
 * attention and the row steps take the decode step's arithmetic, and the
 * projections the kernel family g4h_matmul_path picks for nb tokens -- from 9
 * tokens on q8_0 / q4_0 weights stream once through the int8 matrix cores, so
 * rows agree with decoding the tokens one by one within the fp32 tolerance
 * (below 9, bit for bit).  The decode state (g4h_model_set_state) is not
 * touched. */
int g4h_forward_batch(g4h_model *m, const int *tokens, int nb, int pos0, int want_logits, void *stream);
/* g4_forward_batch_heads (model.c:780-799), the speculative-decoding verify
 * batch (main.c:383-397): the same layers with every projection on the decode
 * step's GEMV family, so row b's logits equal those of decoding tokens[0..b]
 * one by one, bit for bit; then every position's head: logits_dev
 * [nb][n_vocab] and, if hnext_dev, the head's input feature
 * rms(x)*output_norm [nb][n_embd] (device, 16-byte aligned).  Synchronous. */
int g4h_forward_batch_heads(g4h_model *m, const int *tokens, int nb, int pos0, float *logits_dev, float *hnext_dev,
                            void *stream);
/* The greedy choice of every row (main.c:348-349's ARGMAX): out_dev[b] = the
 * first index of the maximum of logits_dev[b][0..n) (rows 16-byte aligned,
 * n % 4 == 0 when nb > 1).  Asynchronous. */
int g4h_argmax_rows(const float *logits_dev, int n, int nb, int *out_dev, void *stream);

/* ------------------------------------------------------------- gemma4 ---- */
/* A gemma4 GGUF model resident on the device: g4_ctx_init (g4run.h:302-303,
 * model.c:373-477) for the model file parsed by g4_gguf_open (model_file is a
 * `const g4_model_file *`, include/g4run_abi.h), or straight from a GGUF path
 * (g4h_gemma_open maps, uploads and unmaps).  Every weight matrix is uploaded
 * and repacked once; the KV caches (kv_type G4H_F16, G4H_Q8_0 or G4H_Q4_0)
 * hold n_ctx positions for full layers and a ring of 576 (G4_SWA_RING) for
 * sliding-window layers.  Limits of this path: head dims 64/128/192/256/512
 * with RoPE over the whole head, 1/2/4/8 query heads per KV head, a window of
 * at most 512 (G4_SWA_WINDOW_MAX), per-layer width <= 1024; the layers past
 * n_layer_kv must be of the kind of the layer whose cache they read.
 * Synchronous. */
typedef struct g4h_gemma g4h_gemma;
int g4h_gemma_create(const void *model_file, int n_ctx, int kv_type, g4h_gemma **out);
int g4h_gemma_open(const char *path, int n_ctx, int kv_type, g4h_gemma **out);
int g4h_gemma_free(g4h_gemma *g);
int g4h_gemma_info(const g4h_gemma *g, int *n_vocab, int *n_embd, int *n_layer, int *n_ctx);
/* g4_forward_batch_heads (model.c:780-799) of the gemma4 forward: nb (1..64)
 * host token ids at positions pos0.. (K/V stored): every position's logits
 * [nb][n_vocab] (soft-capped) into logits_dev and, if hnext_dev, the head
 * input rms(x)*output_norm [nb][n_embd].  nb = 1 is g4_forward (g4run.h:309-311).
 * Row b equals the same forward run one token at a time, bit for bit.
 * Synchronous; G4H_ERR_TIMEOUT if a one-launch attention wait gave up (the
 * logits are then NaN). */
int g4h_gemma_forward(g4h_gemma *g, const int *tokens, int nb, int pos0, float *logits_dev, float *hnext_dev, void *stream);
/* g4_forward_batch (model.c:757-776), the prompt prefill of the gemma4 forward:
 * nb (1..64) host token ids at positions pos0.. (K/V stored); then, if
 * logits_dev, the last position's logits [n_vocab] (soft-capped).  The
 * projections take g4h_matmul's automatic path, so from 9 tokens the q8_0,
 * q4_0, q4_K and q6_K weights run on the int8 matrix cores and f16 / bf16
 * rows on the f16 / bf16 ones, each weight matrix streamed once per batch;
 * rows then differ from g4h_gemma_forward's within the matrix-core path's
 * tolerance.  Synchronous; G4H_ERR_TIMEOUT as
 * g4h_gemma_forward. */
int g4h_gemma_prefill(g4h_gemma *g, const int *tokens, int nb, int pos0, float *logits_dev, void *stream);
/* The decode step of the gemma4 model driven from device state (g4_forward,
 * g4run.h:309-311, as the synthetic model's g4h_forward_state): set_state puts
 * (token, pos) on the device; each g4h_gemma_step runs the forward of that
 * token at that position, its logits into g4h_gemma_logits, then token <- the
 * first maximum of the logits and pos += 1 (at pos == n_ctx - 1 pos stays and
 * g4h_gemma_status reports G4H_STATUS_CTX_FULL).  The step only enqueues work
 * (no host synchronisation, no host-side token or position), so a stream
 * capture of it is replayed once per token; run one step before capturing so
 * the attention workspaces are set up outside the capture.  Its logits equal
 * those of g4h_gemma_forward of the same token at the same position, bit for
 * bit.  status also reports an attention wait that gave up
 * (G4H_STATUS_ATTN_TIMEOUT). */
int g4h_gemma_set_state(g4h_gemma *g, int token, int pos, void *stream);
int g4h_gemma_step(g4h_gemma *g, void *stream);
int g4h_gemma_get_state(g4h_gemma *g, int *token, int *pos, void *stream);
int g4h_gemma_status(g4h_gemma *g, int *flags, void *stream);
const float *g4h_gemma_logits(const g4h_gemma *g);
/* Diagnostic (no reference counterpart): with trace_dev non-NULL, every later
 * g4h_gemma_forward copies each token's intermediate vectors into trace_dev
 * (fp32, *floats_per_token floats per token, token b's at b times that): the
 * per-layer inputs (n_layer * n_embd_per_layer, after their projection and
 * norm, model.c:617-635), then per layer x (the layer's input) | q | k | v (the
 * raw projections, before their norms and RoPE; k and v not written on
 * shared-KV layers, v not without attn_v) | att | wo (Wo output) | xmid (x
 * after the attention residual) | g | u (gate and up outputs) | h
 * (gelu(g) * u) | down | xffn (x after the FFN residual) | plg (inp_gate
 * output) | plh (gelu(plg) * per-layer input) | proj | -- q and att
 * n_head * hd_max floats, k and v hd_max, g, u and h the widest FFN, plg and
 * plh n_embd_per_layer, the rest n_embd, each part's leading elements written
 * -- then the final x.  A CPU implementation can then check each part of each
 * layer on the GPU's own inputs.  NULL turns it off. */
int g4h_gemma_trace(g4h_gemma *g, float *trace_dev, size_t *floats_per_token);
/* Diagnostic: layer `layer`'s K and V caches (device) and their bytes; rows of
 * one KV head, n_ctx slots for full layers, a ring of 576 slots stored twice
 * (slot p % 576 and p % 576 + 576) for sliding-window layers.  Layers past
 * n_layer_kv have no cache of their own. */
int g4h_gemma_kv(g4h_gemma *g, int layer, void **k_dev, void **v_dev, size_t *bytes);

/* ------------------------------------------------------------ sampler ---- */
/* The sampling chain of sampler.c (g4run.h:464-489) with its settings, RNG,
 * ring of recent ids and ban list resident on the device, so a decode step
 * draws its next token without a host round trip.  Draws are the reference's
 * bit for bit: the same ids, the same rewritten logits (bans and n-gram hits
 * at -inf, penalised ids) and the same RNG words, for the same settings,
 * history and logits.  The ring holds the last 4096 ids (sampler.c:10); the
 * per-id counts g4_sampler_accept keeps are not kept (g4_sample never reads
 * them). */
typedef struct g4h_sampler g4h_sampler;
typedef struct {                  /* the settings of g4_sampler, g4run.h:465-473 */
    float temp;                   /* <= 0: greedy (first index of the maximum) */
    int   top_k;                  /* 1..511, else 512 (sampler.c:147) */
    float top_p;
    float repeat_penalty;
    int   repeat_last_n;
    float freq_penalty;
    float presence_penalty;
    int   no_repeat_ngram;        /* 0/1 off, else the n-gram length */
    uint64_t seed;                /* seeds the RNG while its state is all zero */
} g4h_sampler_params;
/* g4_sampler_init's defaults (sampler.c:5-14): temp 1, top_k 64, top_p 0.95,
 * repeat_penalty 1, repeat_last_n 128, seed 0xdeadbeef, the rest 0. */
void g4h_sampler_default_params(g4h_sampler_params *p);
/* g4_sampler_init (sampler.c:5-14); p NULL: the defaults.  Synchronous. */
int  g4h_sampler_create(int n_vocab, const g4h_sampler_params *p, g4h_sampler **out);
/* g4_sampler_free (sampler.c:22-25) */
int  g4h_sampler_free(g4h_sampler *s);
/* Assigning g4_sampler's setting fields: the RNG state is kept (as in the
 * reference, a new seed only matters while the state is all zero). */
int  g4h_sampler_set_params(g4h_sampler *s, const g4h_sampler_params *p, void *stream);
/* The xoshiro256+ state words (sampler.c:51-70); all zero re-seeds from seed
 * on the next draw. */
int  g4h_sampler_set_rng(g4h_sampler *s, const uint64_t rng[4], void *stream);
/* g4_sampler_reset (sampler.c:16-20): empties the ring; bans stay. */
int  g4h_sampler_reset(g4h_sampler *s, void *stream);
/* g4_sampler_ban (sampler.c:27-35): ids outside [0, n_vocab) and repeats are
 * ignored. */
int  g4h_sampler_ban(g4h_sampler *s, int id, void *stream);
/* g4_sampler_accept (sampler.c:37-48) for n host ids, in order (synchronous). */
int  g4h_sampler_accept(g4h_sampler *s, const int *ids, int n, void *stream);
/* g4_sample (sampler.c:74-210) on logits_dev[n_vocab] (device, 16-byte
 * aligned, rewritten in place as the reference rewrites its argument): the
 * drawn id goes to *out_dev (device, may be NULL); accept != 0 also pushes it
 * into the ring, as main.c:265-277 follows each g4_sample with
 * g4_sampler_accept.  Asynchronous, capturable in a graph. */
int  g4h_sample(g4h_sampler *s, float *logits_dev, int *out_dev, int accept, void *stream);
/* Read back (synchronous): the RNG words, the ring oldest first into
 * recent[4096] (either may be NULL), its length, and how many draws so far
 * took the exact heap replay of top-k (ties among the k+1 largest logits or a
 * NaN; the other draws take the sort-based path). */
int  g4h_sampler_get_state(g4h_sampler *s, uint64_t rng[4], int *recent, int *recent_n, int *slow_draws,
                           void *stream);
/* The model's decode steps draw with s (accepting each id) instead of the
 * greedy argmax; NULL restores the argmax.  s must have the model's n_vocab
 * and outlive its use. */
int  g4h_model_set_sampler(g4h_model *m, g4h_sampler *s);

#ifdef __cplusplus
}
#endif
#endif
