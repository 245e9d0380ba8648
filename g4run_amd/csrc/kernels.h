// kernels.h -- host-side launchers of the gfx950 kernels (internal).
#pragma once

#include "common.h"

namespace g4 {

// k_quant.hip
hipError_t launch_quantize_q8_0(const float *x, size_t xs, uint8_t *y, size_t ys, int64_t n, int rows, hipStream_t s);
hipError_t launch_quantize_q8_K(const float *x, size_t xs, uint8_t *y, size_t ys, int64_t n, int rows, hipStream_t s);
hipError_t launch_quantize_q4_0(const float *x, size_t xs, uint8_t *y, size_t ys, int64_t n, int rows, hipStream_t s);
// ridx (optional, device): output row r dequantizes source row ridx[r] (an
// embedding gather whose token ids live on the device)
hipError_t launch_dequant(int type, const uint8_t *x, size_t xs, float *y, size_t ys, int64_t n, int rows, hipStream_t s,
                          const int *ridx = nullptr);
hipError_t launch_repack(const g4h_tensor &t, const uint8_t *rows, hipStream_t s);
hipError_t launch_unpack(const g4h_tensor &t, uint8_t *rows, hipStream_t s);
hipError_t launch_vec_dot_raw(int wtype, const uint8_t *w, size_t ws, const uint8_t *a, int64_t n, int rows, float *out,
                              hipStream_t s);

// k_stream.hip: one launch reading bytes (a 16-byte multiple) once with
// 128-bit non-temporal loads, workgroups of `threads`, `loads` per thread, and
// writing ny floats of y (the read floor a GEMV launch is measured against)
hipError_t launch_read_floor(const uint8_t *p, size_t bytes, float *y, int64_t ny, int threads, int loads, hipStream_t s);

// k_gemv.hip

void gemv_shape(int type, int64_t nblk, int *lpr, int *upl);
// The units per lane a launch of nb_tokens tokens finally uses: one token takes
// exactly as many as the row needs (1..8, so no load is spare); eight K-quant
// tokens cap it at 2 (register file).  A lane visits its units in the same
// order for any UPL, so results do not depend on it.
inline int gemv_upl_final(int type, int64_t nblk, int nb_tokens, int lpr, int upl) {
    const int upb = blck(type) == 256 ? 4 : 1;
    if (nb_tokens == 1) {
        const int per = (int)((nblk * upb + lpr - 1) / lpr);
        return per < 1 ? 1 : per > 8 ? 8 : per;
    }
    return (upb == 4 && nb_tokens == 8 && upl > 2) ? 2 : upl;
}
size_t gemv_lds_bytes(int type, int nb_tokens, int64_t nblk);
void gemv_launch_shape(const g4h_tensor &W, int *lpr, int *upl, int *wpg, int64_t *grid, int nb = 1, bool xq = false);

// The store of the one-shot GEMVs for one token: Y[row] = acc (OUT_STORE),
// or a GELU product folded in with k_gelu_mul's arithmetic, so the bits of the
// two launches it replaces: gelu(e[row]) * acc (OUT_GELU_E; Y may be e) or
// gelu(acc) * e[row] (OUT_GELU_ACC), through the fp16 table `gelu`.
enum { OUT_STORE = 0, OUT_GELU_E = 1, OUT_GELU_ACC = 2 };
struct GemvOut {
    int mode = OUT_STORE;
    const float *e = nullptr;
    const uint16_t *gelu = nullptr;
};
__device__ __forceinline__ float gemv_out_value(const GemvOut &o, int64_t row, float acc) {
    if (o.mode == OUT_GELU_E) return gelu_lut(o.gelu, o.e[row]) * acc;
    if (o.mode == OUT_GELU_ACC) return gelu_lut(o.gelu, acc) * o.e[row];
    return acc;
}

// A producer's q8_0 activation written straight into k_mm_few's operand
// layout (k_mfma.hip) for mt 16-token tiles instead of GGUF rows (qa ==
// nullptr: rows).  Codes and scales of the padding tokens are never written:
// the buffers hold zeros there (launch_few_clear).
struct FewAct {
    int8_t *qa = nullptr;
    uint16_t *da = nullptr;
    int mt = 0;
};

// g4h_matmul_ex on the GEMV family with the store `out` (api.cpp); fp32 x
int matmul_out(const g4h_tensor *W, const float *x, float *Y, int nb, void *stream, const GemvOut &out);
// whether g4h_matmul_ex(W, nb tokens of GGUF rows, path) runs k_mm_few on
// whole block pairs, so that its producer may write the FewAct layout, and
// that matmul on activations already in it
bool matmul_few_ready(const g4h_tensor *W, int nb, int path);
// whether the batched forwards hand k_mm_few its layout directly (G4H_FEW_DIRECT=0:
// GGUF rows or fp32 rows quantized per projection, for measurement and the
// check that both give the same bits)
bool few_direct();
int matmul_few(const g4h_tensor *W, const FewAct &a, float *Y, int nb, void *stream);

// Persistent single-token GEMV (gemv_p.h) over q4_0 / q8_0 rows with a fused
// activation prologue and an optional GELU epilogue.
enum { PRO_ACT = 0, PRO_QUANT = 1, PRO_NORM = 2 };
enum { EPI_STORE = 0, EPI_GELU = 1 };
struct GemvPro {
    int kind = PRO_ACT;
    const float *x = nullptr;        // PRO_QUANT / PRO_NORM: fp32 input (n = W.ncols)
    float *x_out = nullptr;          // PRO_NORM: the updated residual (written by workgroup 0)
    const float *delta = nullptr;    // PRO_NORM: branch output added after its RMSNorm, or null
    const float *w_post = nullptr;   // PRO_NORM: weight of that RMSNorm
    const float *w_pre = nullptr;    // PRO_NORM: weight of the RMSNorm in front of the matmul
    float eps = 0.0f;
    int n = 0;
};
struct GemvEpi {
    int kind = EPI_STORE;
    const uint16_t *gelu = nullptr;  // EPI_GELU: fp16 GELU table
    float *h = nullptr;              // EPI_GELU: nrows/2 outputs gelu(row 2i) * row 2i+1
};
// false when the shape is outside the persistent family (then use launch_gemv)
bool gemv_p_fits(const g4h_tensor &W, const GemvPro &pro, const GemvEpi &epi);
int gemv_p_grid_size();
hipError_t launch_gemv_p(const g4h_tensor &W, const uint8_t *act, float *Y, const GemvPro &pro, const GemvEpi &epi,
                         hipStream_t s);
// out: one token only (nb == 1 unless out.mode == OUT_STORE)
hipError_t launch_gemv(const g4h_tensor &W, const uint8_t *act, size_t stride, float *Y, int nb, hipStream_t s,
                       const GemvOut &out = GemvOut());
// fp32 tokens x [nb][ncols] quantized inside the GEMV when gemv_fused_fits:
// to q8_0 for q8_0 / q4_0 weights (nb in {1, 2, 4, 8}), to q8_K for one
// token of K-quant weights; bit-identical to the standalone quantizer
// followed by launch_gemv
bool gemv_fused_fits(const g4h_tensor &W, int nb);
hipError_t launch_gemv_x(const g4h_tensor &W, const float *x, float *Y, int nb, hipStream_t s, const GemvOut &out = GemvOut());
// k_gemv_f16.hip: f16 / bf16 weight rows (W at ws bytes per row, 16-byte
// aligned, ncols % 8 == 0) against nb in {1, 2, 4, 8} prepared activation rows
// (f16 for F16, bf16-rounded fp32 for BF16) at `as` bytes; Y rows at ys floats
hipError_t launch_gemv_float(int wtype, const uint8_t *W, size_t ws, int64_t nrows, int64_t ncols, const uint8_t *act, size_t as,
                             float *Y, size_t ys, int nb, hipStream_t s, const GemvOut &out = GemvOut());
hipError_t launch_act_float(int wtype, const float *x, size_t xs, int64_t ncols, int nb, uint8_t *out, size_t os, hipStream_t s);
// M tokens of f16 / bf16 weights on the matrix cores (ncols % 16 == 0): x fp32
// rows (xs floats apart, 16-byte aligned) or prepared activation rows at `as`
// bytes; a token's row has the same bits in any batch
hipError_t launch_mm_float(int wtype, const uint8_t *W, size_t ws, int64_t nrows, int64_t ncols, const float *x, size_t xs,
                           const uint8_t *act, size_t as, int M, float *Y, hipStream_t s);
// the float GEMV straight from fp32 tokens (x 16-byte aligned, row stride xs
// floats a multiple of 4), with launch_act_float's conversion on load
hipError_t launch_gemv_float_x(int wtype, const uint8_t *W, size_t ws, int64_t nrows, int64_t ncols, const float *x, size_t xs,
                               float *Y, size_t ys, int nb, hipStream_t s, const GemvOut &out = GemvOut());
hipError_t launch_block_sums(const g4h_tensor &W, const uint8_t *act, size_t stride, int tok, int32_t *out, hipStream_t s);
int block_sums_per_block(int type);

// The decode step's q/k/v head preparation (folded into the attention score
// pass) and k_model.hip's single-workgroup steps (steps.h).
struct QkvArgs {
    int n_head = 0, n_kv = 0, hd = 0, kv_type = 0;
    const float *q_norm = nullptr, *k_norm = nullptr, *rope = nullptr;
    uint8_t *kc = nullptr, *vc = nullptr;
    float eps = 0.0f;
    // sliding window: attend the last `window` positions (0: all); on a ring
    // cache of `ring` slots every row is stored at slot pos % ring and again
    // at that slot + ring (the caches hold 2 * ring slots), so a window of at
    // most ring positions reads as one contiguous run (model.c:517-537)
    int window = 0, ring = 0;
};
hipError_t launch_rand_normal(float *y, int64_t n, uint64_t seed, float mean, float std, hipStream_t s);
// The row forms (nb tokens): x / delta / y rows of n floats, gu rows of 2 n_ff
// floats, act rows at ast bytes; token[b] feeds row b.
// With few.qa set the activations go to that layout (token b as token b of
// the tiles) and act is not written.
hipError_t launch_embed_norm(const g4h_tensor &head, const int *token, float *x, float es, const float *w_pre, float eps,
                             uint8_t *act, hipStream_t s, int nb = 1, size_t ast = 0, const FewAct &few = FewAct());
hipError_t launch_norm_quant(float *x, const float *delta, const float *w_post, const float *w_pre, float eps, int n,
                             uint8_t *act, hipStream_t s, int nb = 1, size_t ast = 0, float *y = nullptr,
                             const FewAct &few = FewAct());
// hout (optional): the h rows themselves, hs floats apart (16-byte aligned)
hipError_t launch_gelu_quant(const float *gu, int n_ff, const uint16_t *tab, uint8_t *act, hipStream_t s, int nb = 1,
                             size_t ast = 0, float *hout = nullptr, size_t hs = 0, const FewAct &few = FewAct());
// out[b] = first index of the maximum of row b of logits [nb][n] (16-byte
// aligned rows)
hipError_t launch_argmax_rows(const float *logits, int n, int nb, int *out, hipStream_t s);
// state: token, pos, npos = pos + 1, steps taken, flags.  Advances pos unless
// pos + 1 == n_ctx: then pos stays and flags |= STATE_CTX_FULL (no later step can
// index past the cache).
constexpr int STATE_CTX_FULL = 1;
hipError_t launch_argmax_advance(const float *logits, int n, int *state, int n_ctx, hipStream_t s);

// k_sample.hip: the sampling chain of sampler.c:74-210 on one workgroup.
// Device image of a sampler: g4_sampler's settings and state (g4run.h:464-482)
// with a fixed ring of SAMPLER_RING ids (the reference's recent_cap,
// sampler.c:10) and the ban list after the struct (n_vocab ints).  The
// per-id counts the reference keeps in accept are not kept: g4_sample never
// reads them.
constexpr int SAMPLER_RING = 4096;
constexpr int SAMPLER_TOPK_MAX = 512;     // sampler.c:147
struct SamplerDev {
    float temp;
    int top_k;
    float top_p;
    float repeat_penalty;
    int repeat_last_n;
    float freq_penalty;
    float presence_penalty;
    int no_repeat_ngram;
    uint64_t seed;
    uint64_t rng[4];
    int n_vocab, recent_n, recent_head, n_ban;
    int slow_draws;                       // draws that took the exact heap emulation (ties / NaN)
    int pad_[3];
    int recent[SAMPLER_RING];
};
inline size_t sampler_dev_bytes(int n_vocab) { return sizeof(SamplerDev) + (size_t)n_vocab * sizeof(int); }
__host__ __device__ inline int *sampler_bans(SamplerDev *S) { return reinterpret_cast<int *>(S + 1); }
// Draws one id from logits[n_vocab] (rewritten in place as sampler.c does),
// writes it to *out if out, pushes it into the ring if accept, and if state is
// given (the model's token, pos, npos, steps, flags) stores it there and
// advances the position as launch_argmax_advance does.
hipError_t launch_sample(SamplerDev *S, int n_vocab, float *logits, int *out, int accept, int *state, int n_ctx,
                         hipStream_t s);
// Pushes n ids into the ring in order (sampler.c:37-48).
hipError_t launch_sampler_push(SamplerDev *S, const int *ids, int n, hipStream_t s);

// k_gemma.hip: the gemma4 forward's row steps (nb token rows each)
hipError_t launch_rms_rows(const float *x, const float *w, float *y, int n, int nb, float eps, hipStream_t s);
// x = (x + rms(d) * w) * os; with w2 and y also y = rms(x) * w2 (the next
// RMSNorm, y may be d)
hipError_t launch_resid(float *x, const float *d, const float *w, int n, int nb, float eps, float os, hipStream_t s,
                        const float *w2 = nullptr, float *y = nullptr);
hipError_t launch_scale(float *y, int64_t n, float sc, hipStream_t s);
hipError_t launch_ple_prep(const float *plp, float *pl, const float *w, int pe, int n_layer, int nb, float ps, float is2,
                           float eps, hipStream_t s);
hipError_t launch_gelu_mul(float *g, size_t gs, const float *u, size_t us, int n, int nb, const uint16_t *tab, hipStream_t s);
// pos_dev (optional, device): the first row's position instead of pos0
hipError_t launch_head_prep(float *q, int n_head, int hd, int nb, const float *w, const float *rope, int pos0, float eps,
                            hipStream_t s, const int *pos_dev = nullptr);
hipError_t launch_pack_qkv(const float *q, const float *k, const float *v, float *qkv, int nq, int hd, int nb, hipStream_t s);
hipError_t launch_softcap(float *l, int64_t n, float cap, hipStream_t s);

// k_mfma.hip: many-token matmul on the int8 matrix cores (q8_0 / q4_0 weights)
size_t mm_planar_bytes(int M, int64_t ncols);
void mm_describe(const g4h_tensor &W, int M, char *buf, size_t len);
hipError_t launch_matmul_mfma(const g4h_tensor &W, const float *x, size_t x_stride, const uint8_t *act, size_t stride, int M,
                              float *Y, uint8_t *ws, hipStream_t s);
// k_mm_few on activations a producer wrote in its layout (FewAct, mt = (M +
// 15) / 16): mm_few_ready says whether launch_matmul_mfma would take k_mm_few
// for W at M tokens and W has whole block pairs (no padding block);
// few_act_bytes sizes the buffers for rows of up to ncols columns (the scales
// at *da_off); launch_few_clear zeroes them for a new token count.
bool mm_few_ready(const g4h_tensor &W, int M);
size_t few_act_bytes(int64_t ncols, int M, size_t *da_off);
hipError_t launch_few_clear(uint8_t *buf, size_t bytes, hipStream_t s);
// x fp32 rows (xs floats apart) quantized to q8_0 into that layout, padding
// tokens and block included (launch_matmul_mfma's own quantizer launch)
hipError_t launch_quantize_few(const float *x, size_t xs, int64_t ncols, int M, const FewAct &a, hipStream_t s);
hipError_t launch_mm_few_ready(const g4h_tensor &W, const FewAct &a, int M, float *Y, hipStream_t s);

// k_mfma_k.hip: many-token matmul on the int8 matrix cores for q4_K / q6_K
// weights against GGUF q8_K activation rows at `stride` bytes
bool mmk_capable(int type);
void mmk_describe(const g4h_tensor &W, int M, char *buf, size_t len);
hipError_t launch_matmul_mfma_k(const g4h_tensor &W, const uint8_t *act, size_t stride, int M, float *Y, hipStream_t s);

// k_attn.hip
size_t attn_workspace_bytes(int n_head, int hd, int npos_max);
// drop a workspace from the cleared-workspace registry (its memory is freed)
void attn_ws_forget(const void *p);
// The one-launch form's bounded polls give up after a fixed retry count; a
// workgroup that gives up writes NaN and sets the workspace's error word at
// offset 0 (ATTN_ERR_OFFSET), which stays set until the host clears it.  Test
// hook: with `on`, every poll waits for a tag no store carries and gives up
// after 64 retries, so the failure path runs deterministically.
void attn_force_timeout(bool on);
constexpr size_t ATTN_ERR_OFFSET = 0;
// f16 caches run as one fused launch when its grid fits on the device at once
// (attn_fused_fits).  Its hand-off words in ws carry a tag that must differ
// from every earlier launch on that ws: *epoch * mul + add + 1 when `tag` is
// given (a caller-kept counter, with ws zeroed before first use), else the
// launch clears its words first and starts the tags over.
struct AttnTag {
    const unsigned *epoch;
    unsigned mul, add;
};
bool attn_fused_fits(int kv_type, int n_head, int n_kv, int hd, int npos_max);
// causal attention of nb tokens over one cache (the first attends npos0
// positions, token b npos0 + b; with a.window, the last window of them),
// three passes with a token grid dimension; ws of
// attn_batch_workspace_bytes(n_head, hd, rows, nb), rows = npos0 + nb - 1 or,
// with a window, at most the window
size_t attn_batch_workspace_bytes(int n_head, int hd, int npos_max, int nb);
// q8out (optional): q8_0 rows of each token's output, q8_stride bytes apart
// (0: packed rows)
hipError_t launch_attn_batch(const float *q, const QkvArgs &a, int npos0, int nb, float *out, uint8_t *q8out, uint8_t *ws,
                             hipStream_t s, size_t q8_stride = 0);
// The same causal batch on the matrix cores (f16 caches, hd 64 / 128 / 256,
// 1 / 2 / 4 / 8 query heads per KV head; attn_batch_mm_ok): tiles of 32
// (token, head) rows share every K and V row they read; within the
// attention's tolerance of launch_attn_batch, not bit-identical to it, and a
// token's row has the same bits in any batch.  ws of
// attn_batch_workspace_bytes (which covers both forms), ws_bytes its size.
// With pos_dev, token 0's position is read on the device (npos0 unused) and
// the grid covers a last token attending up to npos_max positions.
bool attn_batch_mm_ok(const QkvArgs &a);
// prompt batches of at least this many tokens take the matrix-core kernels
// (g4h_matmul_path, the batched forwards' attention)
constexpr int kMmMinTokens = 9;
size_t attn_batch_mm_workspace_bytes(int n_head, int hd, int npos_max, int nb);
hipError_t launch_attn_batch_mm(const float *q, const QkvArgs &a, int npos0, int nb, float *out, uint8_t *q8out, uint8_t *ws,
                                size_t ws_bytes, hipStream_t s, size_t q8_stride = 0, const int *pos_dev = nullptr,
                                int npos_max = 0, const FewAct &few = FewAct());
// the query / key / value rows of nb tokens from the fused projection output
// (rows of (n_head + 2 n_kv) hd floats) prepared as the decode kernels do:
// queries into qout [nb][n_head][hd], key and value rows into the caches at
// pos0 .. pos0 + nb - 1 (on a ring both copies; at most ring - window + 1
// tokens)
hipError_t launch_attn_prep_rows(const float *qkv, const QkvArgs &a, int pos0, int nb, float *qout, hipStream_t s,
                                 const int *pos_dev = nullptr);
// Wo (optional, with wo_out): the output projection folded into the
// one-launch form (attn_wo_fits), its rows into wo_out instead of a separate
// GEMV on q8out's rows, with the same bits
hipError_t launch_attn_decode(const float *q, const float *qkv, const QkvArgs &a, int npos, const int *npos_dev, int npos_max,
                              float *out, uint8_t *q8out, uint8_t *ws, hipStream_t s, const AttnTag *tag = nullptr,
                              const g4h_tensor *Wo = nullptr, float *wo_out = nullptr, size_t ws_bytes = 0);
bool attn_wo_fits(const g4h_tensor &Wo, const QkvArgs &a, int npos_max);
hipError_t launch_kv_store(int kv_type, const float *src, uint8_t *dst, int hd, int rows, size_t dst_stride, hipStream_t s);
// The decode step's q|k|v projection W (q4_0 / q8_0) with its PRO_NORM
// prologue computed inside the one-launch attention: every workgroup computes
// a slice of the projection rows while its K stream is in flight and hands
// them over as tagged words in qt ((n_head + 2 n_kv) * hd words, zeroed once,
// 128-byte aligned).  Bit-identical to launch_gemv_p(W, PRO_NORM) followed by
// launch_attn_decode on its output.
bool attn_qkv_fits(const g4h_tensor &W, const QkvArgs &a, int npos_max);
// the bounded-wait settings every hand-off poll uses (attn_force_timeout)
unsigned attn_spin_limit();
uint32_t attn_poll_xor();
hipError_t launch_attn_qkv(const g4h_tensor &W, const GemvPro &pro, const QkvArgs &a, const int *npos_dev, int npos_max,
                           float *out, uint8_t *q8out, uint8_t *ws, uint64_t *qt, hipStream_t s, const AttnTag &tag);

}  // namespace g4
