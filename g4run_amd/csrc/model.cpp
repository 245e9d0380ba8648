// model.cpp -- a synthetic gemma-style decoder resident on one MI355X and its
// decode step (the GPU form of g4_forward / forward_layers, g4run.h:309-311,
// model.c:593-775), built from this library's kernels.
//
// Per layer (model.c:647-736 without the gemma4-only per-layer embeddings,
// sliding-window ring, shared KV and softcap):
//   a  = q8_0(rms(x)*attn_norm), x <- x + rms(prev)*post_ffw_norm first    k_norm_quant
//   qkv = Wqkv a                                                            GEMV
//   q,k <- rms(.)*q_norm/k_norm, RoPE; v <- rms(v); k,v stored at pos
//   o  = attention(q, K[0..pos], V[0..pos])     scores (+ the q/k/v preparation), V, combine (+ q8_0(o))
//   y  = Wo q8_0(o)                                                         GEMV
//   x <- x + rms(y)*post_attn_norm; a = q8_0(rms(x)*ffn_norm)               k_norm_quant
//   g|u = Wgu a;  a = q8_0(gelu(g)*u)                                 GEMV, k_gelu_quant
//   y  = Wdown a                                                            GEMV
// then x <- x + rms(y)*post_ffw_norm, a = q8_0(rms(x)*output_norm),
// logits = Head a (tied q8_0 embedding), token = argmax.  The embedding
// kernel also produces the first layer's a.
#include "../../include/g4hip.h"

#include <algorithm>
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <vector>

#include "host_fp16.h"
#include "kernels.h"

using namespace g4;


extern "C" int g4h_internal_fail(int status, const char *msg);
extern "C" int g4h_internal_attn_error(void *ws, void *stream, const char *fn);
// sampler.cpp
int sampler_n_vocab(const g4h_sampler *s);
SamplerDev *sampler_device(g4h_sampler *s);


struct g4h_model {
    g4h_model_config c;
    std::vector<g4h_tensor *> wqkv, wo, wgu, wdown;
    g4h_tensor *head = nullptr;
    float *norms = nullptr;          // [n_layer][6][n_embd-or-hd] + output norm
    size_t norm_stride = 0;          // floats per (layer, which) slot
    uint8_t *kv = nullptr;           // all caches
    size_t kv_layer_bytes = 0;       // one of K or V for one layer
    float *rope = nullptr;           // [n_ctx][hd] cos/sin pairs
    uint16_t *gelu = nullptr;        // 65536 fp16 codes
    int *state = nullptr;            // token, pos, npos, steps taken, flags (STATE_*)
    float *x = nullptr, *x2 = nullptr, *xb = nullptr, *qkv = nullptr, *q = nullptr, *att = nullptr, *ff = nullptr, *logits = nullptr;
    uint8_t *act = nullptr, *ws = nullptr;
    uint64_t *qt = nullptr;          // FUSE_QATT: tagged q|k|v projection rows
    size_t act_bytes = 0, ws_bytes = 0;
    std::vector<void *> allocs;
    int fuse = 0;                    // FUSE_* steps folded into the GEMVs
    float *trace = nullptr;          // optional per-layer x | qkv | att rows, then the final x (g4h_model_trace)
    g4h_sampler *sampler = nullptr;  // draws the next token (g4h_model_set_sampler); null: greedy argmax
    // rows of the batched forward (g4h_forward_batch*), for up to kBatchMax
    // tokens, allocated by its first call; bws is its own attention workspace
    // (per-token form), bbw the batch attention's (a block per token), bq the
    // prepared query rows
    float *bx = nullptr, *bxb = nullptr, *bqkv = nullptr, *batt = nullptr, *bff = nullptr, *bhn = nullptr, *bq = nullptr;
    uint8_t *bact = nullptr, *bws = nullptr, *bbw = nullptr;
    int *btok = nullptr;
    // a prompt batch's activations in k_mm_few's layout (FewAct) for rows of
    // up to few_cols columns; zeroed for few_nb tokens
    uint8_t *bfew = nullptr;
    int64_t few_cols = 0;
    int few_nb = 0;
};

static constexpr int kBatchMax = 64;   // G4_BATCH_MAX, g4run.h:23

// Steps of the chain folded into the persistent GEMV family (gemv_p.h) or
// into the attention launch:
//   FUSE_QKV   residual + attention RMSNorm + q8_0 in front of Wqkv
//   FUSE_GU    residual + FFN RMSNorm + q8_0 in front of Wgu, GELU(gate)*up after it
//   FUSE_DOWN  q8_0 of h in front of Wdown (with FUSE_GU)
//   FUSE_HEAD  residual + output RMSNorm + q8_0 in front of the head
//   FUSE_QATT  the Wqkv GEMV with its norm prologue inside the one-launch
//              attention, its rows computed while the K stream is in flight
//   FUSE_WO    the Wo GEMV inside the one-launch attention, after a hand-off
//              of the q8_0 head rows (its weights prefetched during the
//              attention's own hand-offs)
enum { FUSE_QKV = 1, FUSE_GU = 2, FUSE_DOWN = 4, FUSE_HEAD = 8, FUSE_QATT = 16, FUSE_WO = 32 };
// measured on the BASELINE decode step (tok/s, 128 steps at ctx 8192): none
// 842, QKV 856, GU 928, QKV|GU 955, QKV|GU|QATT 929; QKV|GU 968 against
// QKV|GU|WO 991 (two runs each, after later kernel work).  In the QATT launch
// a wave that has queued its K stream cannot run the projection until the
// stream drains far enough to accept its loads, so the rows come out ~5.6 us
// into the launch and the attention starts later than after a separate GEMV.
// The WO hand-off costs most of the Wo launch it replaces (~0.9 us net per
// layer).  (Wdown and the next layer's Wqkv in one launch, Wdown's rows handed
// over as tagged words, measured 896 against 962 and was taken out: gathering
// those rows in every workgroup waits for poll round trips behind the other
// CUs' streams.)
// QKV|GU|WO|HEAD 965-970 against QKV|GU|WO 960-966 (six alternating pairs,
// HEAD ahead in each); QKV|GU|WO|DOWN 887.
static constexpr int kDefaultFuse = FUSE_QKV | FUSE_GU | FUSE_WO | FUSE_HEAD;

static int model_alloc(g4h_model *m, void **p, size_t bytes) {
    if (int rc = g4h_malloc(p, bytes)) return rc;
    m->allocs.push_back(*p);
    return G4H_OK;
}

#define M_HIP(call)                                                                \
    do {                                                                           \
        hipError_t e_ = (call);                                                    \
        if (e_ != hipSuccess) return g4h_internal_fail(G4H_ERR_HIP, hipGetErrorString(e_)); \
    } while (0)
#define M_RC(call)                  \
    do {                            \
        int rc_ = (call);           \
        if (rc_) return rc_;        \
    } while (0)

// random matrix: N(0, std) fp32 -> quantized GGUF rows -> resident tensor.
// With `interleave` the random rows [A (rows/2) | B (rows/2)] are stored in
// the order A0 B0 A1 B1 ... (the gate/up layout of Wgu).
static int init_matrix(int type, int64_t rows, int64_t cols, uint64_t seed, float *tmp_f, uint8_t *tmp_q, bool interleave,
                       g4h_tensor **out, hipStream_t s) {
    if (type != Q8_0 && type != Q4_0) return g4h_internal_fail(G4H_ERR_TYPE, "g4h_model_create: weights must be q4_0 or q8_0");
    M_RC(g4h_tensor_create(type, cols, rows, out));
    const size_t rb = g4h_row_size(type, cols);
    auto quant = [&](const float *x, uint8_t *y, size_t ys, int64_t nr) {
        return type == Q8_0 ? launch_quantize_q8_0(x, cols, y, ys, cols, (int)nr, s)
                            : launch_quantize_q4_0(x, cols, y, ys, cols, (int)nr, s);
    };
    hipError_t e = launch_rand_normal(tmp_f, rows * cols, seed, 0.0f, 0.02f, s);
    if (e == hipSuccess && interleave) {
        e = quant(tmp_f, tmp_q, 2 * rb, rows / 2);
        if (e == hipSuccess) e = quant(tmp_f + (size_t)(rows / 2) * cols, tmp_q + rb, 2 * rb, rows / 2);
    } else if (e == hipSuccess) {
        e = quant(tmp_f, tmp_q, rb, rows);
    }
    int rc = e == hipSuccess ? G4H_OK : g4h_internal_fail(G4H_ERR_HIP, hipGetErrorString(e));
    if (!rc) rc = g4h_tensor_load(*out, tmp_q, 1, s);
    if (rc) { g4h_tensor_free(*out); *out = nullptr; }
    return rc;
}

extern "C" int g4h_model_create(const g4h_model_config *cfg, uint64_t seed, g4h_model **out) {
    if (!cfg || !out) return g4h_internal_fail(G4H_ERR_ARG, "g4h_model_create: null argument");
    *out = nullptr;
    const g4h_model_config &c = *cfg;
    if (c.n_layer <= 0 || c.n_embd <= 0 || c.n_head <= 0 || c.n_kv <= 0 || c.n_ff <= 0 || c.n_vocab <= 0 || c.n_ctx <= 0)
        return g4h_internal_fail(G4H_ERR_ARG, "g4h_model_create: non-positive dimension");
    if (c.n_embd % 32 || c.n_ff % 256 || c.head_dim % 64 || c.head_dim > 256 || c.n_head % c.n_kv || c.n_embd > 8192 ||
        c.n_ff % 32)
        return g4h_internal_fail(G4H_ERR_SHAPE, "g4h_model_create: n_embd%32 (<=8192), n_ff%256, head_dim%64 (<=256), n_head%n_kv");
    if ((c.wtype != Q4_0 && c.wtype != Q8_0) || c.head_type != Q8_0 || (c.kv_type != F16 && c.kv_type != Q8_0 && c.kv_type != Q4_0))
        return g4h_internal_fail(G4H_ERR_TYPE, "g4h_model_create: wtype q4_0|q8_0, head q8_0, kv f16|q8_0|q4_0");
    g4h_model *m = new g4h_model();
    m->c = c;
    m->fuse = kDefaultFuse;
    if (const char *e = getenv("G4H_DECODE_FUSE")) m->fuse = atoi(e) & 63;
    const int E = c.n_embd, H = c.n_head, KV = c.n_kv, hd = c.head_dim, F = c.n_ff;
    const int qkv_rows = (H + 2 * KV) * hd, qd = H * hd;
    hipStream_t s = nullptr;
    int rc = G4H_OK;
    auto bail = [&](int r) { g4h_model_free(m); return r; };

    // scratch for init: the largest matrix as fp32 and as GGUF rows
    int64_t big = (int64_t)c.n_vocab * E;
    big = std::max(big, (int64_t)2 * F * E);
    big = std::max(big, (int64_t)qkv_rows * E);
    big = std::max(big, (int64_t)E * F);
    float *tmp_f = nullptr;
    uint8_t *tmp_q = nullptr;
    if ((rc = g4h_malloc((void **)&tmp_f, big * 4))) return bail(rc);
    if ((rc = g4h_malloc((void **)&tmp_q, big * 2))) { g4h_free(tmp_f); return bail(rc); }
    uint64_t k = seed * 0x100000001b3ull + 17;
    for (int l = 0; l < c.n_layer && !rc; l++) {
        g4h_tensor *t;
        if ((rc = init_matrix(c.wtype, qkv_rows, E, k++, tmp_f, tmp_q, false, &t, s))) break;
        m->wqkv.push_back(t);
        if ((rc = init_matrix(c.wtype, E, qd, k++, tmp_f, tmp_q, false, &t, s))) break;
        m->wo.push_back(t);
        if ((rc = init_matrix(c.wtype, 2 * F, E, k++, tmp_f, tmp_q, true, &t, s))) break;
        m->wgu.push_back(t);
        if ((rc = init_matrix(c.wtype, E, F, k++, tmp_f, tmp_q, false, &t, s))) break;
        m->wdown.push_back(t);
    }
    if (!rc) rc = init_matrix(c.head_type, c.n_vocab, E, k++, tmp_f, tmp_q, false, &m->head, s);
    const hipError_t init_err = hipStreamSynchronize(s);
    g4h_free(tmp_f);
    g4h_free(tmp_q);
    if (rc) return bail(rc);
    if (init_err != hipSuccess) return bail(g4h_internal_fail(G4H_ERR_HIP, hipGetErrorString(init_err)));

    // norm weights ~ N(1, 0.05): [layer][6] slots of max(E, hd) floats + output norm
    m->norm_stride = (size_t)std::max(E, hd);
    const size_t n_norm = ((size_t)c.n_layer * 6 + 1) * m->norm_stride;
    if ((rc = model_alloc(m, (void **)&m->norms, n_norm * 4))) return bail(rc);
    if (launch_rand_normal(m->norms, (int64_t)n_norm, k++, 1.0f, 0.05f, s) != hipSuccess) return bail(G4H_ERR_HIP);

    // KV caches: [layer][K|V][n_ctx][n_kv][row]
    const size_t row = c.kv_type == F16 ? (size_t)hd * 2 : g4h_row_size(c.kv_type, hd);
    m->kv_layer_bytes = (size_t)c.n_ctx * KV * row;
    if ((rc = model_alloc(m, (void **)&m->kv, m->kv_layer_bytes * 2 * c.n_layer))) return bail(rc);
    if (hipMemsetAsync(m->kv, 0, m->kv_layer_bytes * 2 * c.n_layer, s) != hipSuccess) return bail(G4H_ERR_HIP);

    // RoPE table, built as rope_cache (model.c:349-358) for every position
    std::vector<float> rope((size_t)c.n_ctx * hd);
    const float theta_scale = powf(c.rope_base, -2.0f / hd);
    for (int p = 0; p < c.n_ctx; p++) {
        float theta = (float)p;
        for (int i = 0; i < hd / 2; i++) {
            rope[(size_t)p * hd + 2 * i] = cosf(theta);
            rope[(size_t)p * hd + 2 * i + 1] = sinf(theta);
            theta *= theta_scale;
        }
    }
    if ((rc = model_alloc(m, (void **)&m->rope, rope.size() * 4))) return bail(rc);
    if (hipMemcpy(m->rope, rope.data(), rope.size() * 4, hipMemcpyHostToDevice) != hipSuccess) return bail(G4H_ERR_HIP);

    // GELU fp16 table (quants.c:48-58)
    std::vector<uint16_t> gt(65536);
    for (uint32_t h = 0; h < 65536; h++) gt[h] = gelu_table_entry((uint16_t)h);
    if ((rc = model_alloc(m, (void **)&m->gelu, 65536 * 2))) return bail(rc);
    if (hipMemcpy(m->gelu, gt.data(), 65536 * 2, hipMemcpyHostToDevice) != hipSuccess) return bail(G4H_ERR_HIP);

    // activations and state
    const int wide = std::max(std::max(E, 2 * F), std::max(qkv_rows, c.n_vocab));
    if ((rc = model_alloc(m, (void **)&m->state, 64))) return bail(rc);
    if ((rc = model_alloc(m, (void **)&m->x, E * 4))) return bail(rc);
    if ((rc = model_alloc(m, (void **)&m->x2, E * 4))) return bail(rc);
    if ((rc = model_alloc(m, (void **)&m->xb, E * 4))) return bail(rc);
    if ((rc = model_alloc(m, (void **)&m->qkv, qkv_rows * 4))) return bail(rc);
    if ((rc = model_alloc(m, (void **)&m->q, qd * 4))) return bail(rc);
    if ((rc = model_alloc(m, (void **)&m->att, qd * 4))) return bail(rc);
    if ((rc = model_alloc(m, (void **)&m->ff, 2 * F * 4))) return bail(rc);
    if ((rc = model_alloc(m, (void **)&m->logits, (size_t)c.n_vocab * 4))) return bail(rc);
    m->act_bytes = (g4h_row_size(Q8_0, std::max(E, std::max(F, qd))) + 63) & ~(size_t)63;
    if ((rc = model_alloc(m, (void **)&m->act, m->act_bytes))) return bail(rc);
    m->ws_bytes = g4h_attn_workspace_bytes(H, hd, c.n_ctx);
    if ((rc = model_alloc(m, (void **)&m->ws, m->ws_bytes))) return bail(rc);
    if ((rc = model_alloc(m, (void **)&m->qt, (size_t)qkv_rows * 8))) return bail(rc);
    if (hipMemset(m->qt, 0, (size_t)qkv_rows * 8) != hipSuccess) return bail(G4H_ERR_HIP);
    (void)wide;
    if (hipMemset(m->state, 0, 64) != hipSuccess) return bail(G4H_ERR_HIP);
    if (hipMemset(m->ws, 0, m->ws_bytes) != hipSuccess) return bail(G4H_ERR_HIP);   // no attention tag seen yet
    if (hipDeviceSynchronize() != hipSuccess) return bail(g4h_internal_fail(G4H_ERR_HIP, "g4h_model_create: init kernels failed"));
    *out = m;
    return G4H_OK;
}

extern "C" int g4h_model_free(g4h_model *m) {
    if (!m) return G4H_OK;
    for (auto *v : {&m->wqkv, &m->wo, &m->wgu, &m->wdown})
        for (g4h_tensor *t : *v) g4h_tensor_free(t);
    g4h_tensor_free(m->head);
    for (void *p : m->allocs) g4h_free(p);
    delete m;
    return G4H_OK;
}

extern "C" int g4h_model_fill_kv(g4h_model *m, uint64_t seed, void *stream) {
    if (!m) return g4h_internal_fail(G4H_ERR_ARG, "g4h_model_fill_kv: null model");
    const hipStream_t s = (hipStream_t)stream;
    const g4h_model_config &c = m->c;
    const int64_t n = (int64_t)c.n_ctx * c.n_kv * c.head_dim;
    float *tmp;
    M_RC(g4h_malloc((void **)&tmp, n * 4));
    const size_t row = c.kv_type == F16 ? (size_t)c.head_dim * 2 : g4h_row_size(c.kv_type, c.head_dim);
    hipError_t e = hipSuccess;
    for (int i = 0; i < 2 * c.n_layer && e == hipSuccess; i++) {
        e = launch_rand_normal(tmp, n, seed * 7919 + i, 0.0f, 1.0f, s);
        if (e == hipSuccess)
            e = launch_kv_store(c.kv_type, tmp, m->kv + (size_t)i * m->kv_layer_bytes, c.head_dim, (int)(n / c.head_dim), row, s);
    }
    const hipError_t e2 = hipStreamSynchronize(s);
    g4h_free(tmp);
    if (e != hipSuccess || e2 != hipSuccess)
        return g4h_internal_fail(G4H_ERR_HIP, hipGetErrorString(e != hipSuccess ? e : e2));
    return G4H_OK;
}

static float *norm_of(g4h_model *m, int layer, int which) {
    return m->norms + ((size_t)layer * 6 + which) * m->norm_stride;
}

// one decode step from the device state (token, pos); advances it
extern "C" int g4h_forward_state(g4h_model *m, void *stream) {
    if (!m) return g4h_internal_fail(G4H_ERR_ARG, "g4h_forward_state: null model");
    const hipStream_t s = (hipStream_t)stream;
    const g4h_model_config &c = m->c;
    const int E = c.n_embd, H = c.n_head, KV = c.n_kv, hd = c.head_dim, F = c.n_ff;
    const int qkv_rows = (H + 2 * KV) * hd;
    int *token = m->state, *npos = m->state + 2;    // state: token, pos, npos = pos + 1
    // trace record (g4h_model_trace): x | qkv | att | wo | xmid | h | down
    const size_t TR_X = 0, TR_QKV = E, TR_ATT = TR_QKV + qkv_rows, TR_WO = TR_ATT + (size_t)H * hd, TR_XMID = TR_WO + E,
                 TR_H = TR_XMID + E, TR_DOWN = TR_H + F, trace_rec = TR_DOWN + E;
    auto trace_copy = [&](float *rec, size_t off, const float *src, int n) -> int {
        if (!rec) return G4H_OK;
        M_HIP(hipMemcpyAsync(rec + off, src, (size_t)n * 4, hipMemcpyDeviceToDevice, s));
        return G4H_OK;
    };
    const size_t ast = m->act_bytes;
    const int fz = m->fuse;
    float *x = m->x, *xn = m->x2;    // residual; a norm prologue writes x' to xn and the two swap
    // GEMV over W with the residual update + RMSNorm + q8_0 in its prologue
    auto norm_gemv = [&](const g4h_tensor &W, const float *delta, const float *w_post, const float *w_pre, float *Y,
                         bool gelu) {
        GemvPro pro;
        pro.kind = PRO_NORM;
        pro.x = x;
        pro.x_out = xn;
        pro.delta = delta;
        pro.w_post = w_post;
        pro.w_pre = w_pre;
        pro.eps = c.rms_eps;
        pro.n = E;
        GemvEpi epi;
        if (gelu) {
            epi.kind = EPI_GELU;
            epi.gelu = m->gelu;
            epi.h = m->ff;
        }
        const hipError_t e = launch_gemv_p(W, nullptr, Y, pro, epi, s);
        std::swap(x, xn);
        return e;
    };
    const bool qkv_pro = fz & (FUSE_QKV | FUSE_QATT);     // the attention norm runs in a projection prologue
    // whether W takes the GELU epilogue (the persistent family sums its rows in
    // the one-shot kernel's order only where its LPR allows row pairs in a wave)
    auto gelu_fits = [&](const g4h_tensor &W) {
        GemvPro p;
        p.kind = PRO_NORM;
        p.n = (int)W.ncols;
        GemvEpi e;
        e.kind = EPI_GELU;
        return gemv_p_fits(W, p, e);
    };
    M_HIP(launch_embed_norm(*m->head, token, x, sqrtf((float)E), qkv_pro ? nullptr : norm_of(m, 0, G4H_N_ATTN),
                            c.rms_eps, m->act, s));
    for (int l = 0; l < c.n_layer; l++) {
        uint8_t *kc = m->kv + (size_t)(2 * l) * m->kv_layer_bytes, *vc = kc + m->kv_layer_bytes;
        const float *prev_post = l ? norm_of(m, l - 1, G4H_N_POST_FFW) : nullptr;
        QkvArgs qa;
        qa.n_head = H;
        qa.n_kv = KV;
        qa.hd = hd;
        qa.kv_type = c.kv_type;
        qa.q_norm = norm_of(m, l, G4H_N_Q);
        qa.k_norm = norm_of(m, l, G4H_N_K);
        qa.rope = m->rope;
        qa.kc = kc;
        qa.vc = vc;
        qa.eps = c.rms_eps;
        const AttnTag tag{(const unsigned *)(m->state + 3), (unsigned)c.n_layer, (unsigned)l};
        bool wo_done = false;                                         // Wo computed inside the attention launch
        if ((fz & FUSE_QATT) && attn_qkv_fits(*m->wqkv[l], qa, c.n_ctx)) {
            GemvPro pro;
            pro.kind = PRO_NORM;
            pro.x = x;
            pro.x_out = xn;
            pro.delta = l ? m->xb : nullptr;
            pro.w_post = prev_post;
            pro.w_pre = norm_of(m, l, G4H_N_ATTN);
            pro.eps = c.rms_eps;
            pro.n = E;
            M_HIP(launch_attn_qkv(*m->wqkv[l], pro, qa, npos, c.n_ctx, m->att, m->act, m->ws, m->qt, s, tag));
            std::swap(x, xn);
        } else {
            if (qkv_pro) {
                M_HIP(norm_gemv(*m->wqkv[l], l ? m->xb : nullptr, prev_post, norm_of(m, l, G4H_N_ATTN), m->qkv, false));
            } else {
                if (l) M_HIP(launch_norm_quant(x, m->xb, prev_post, norm_of(m, l, G4H_N_ATTN), c.rms_eps, E, m->act, s));
                M_HIP(launch_gemv(*m->wqkv[l], m->act, ast, m->qkv, 1, s));
            }
            wo_done = (fz & FUSE_WO) && attn_wo_fits(*m->wo[l], qa, c.n_ctx);
            M_HIP(launch_attn_decode(nullptr, m->qkv, qa, 0, npos, c.n_ctx, m->att, m->act, m->ws, s, &tag,
                                     wo_done ? m->wo[l] : nullptr, wo_done ? m->xb : nullptr));
        }
        float *tr = m->trace ? m->trace + (size_t)l * trace_rec : nullptr;
        // x holds this layer's input once its Wqkv launch is queued
        M_RC(trace_copy(tr, TR_X, x, E));
        M_RC(trace_copy(tr, TR_QKV, m->qkv, qkv_rows));
        M_RC(trace_copy(tr, TR_ATT, m->att, H * hd));
        if (!wo_done) M_HIP(launch_gemv(*m->wo[l], m->act, ast, m->xb, 1, s));
        M_RC(trace_copy(tr, TR_WO, m->xb, E));
        if ((fz & FUSE_GU) && !gelu_fits(*m->wgu[l])) {
            // the residual norm in the Wgu prologue, GELU * up as its own step
            M_HIP(norm_gemv(*m->wgu[l], m->xb, norm_of(m, l, G4H_N_POST_ATTN), norm_of(m, l, G4H_N_FFN), m->ff, false));
            M_RC(trace_copy(tr, TR_XMID, x, E));
            M_HIP(launch_gelu_quant(m->ff, F, m->gelu, m->act, s));
            M_HIP(launch_gemv(*m->wdown[l], m->act, ast, m->xb, 1, s));
        } else if (fz & FUSE_GU) {
            M_HIP(norm_gemv(*m->wgu[l], m->xb, norm_of(m, l, G4H_N_POST_ATTN), norm_of(m, l, G4H_N_FFN), nullptr, true));
            M_RC(trace_copy(tr, TR_XMID, x, E));
            M_RC(trace_copy(tr, TR_H, m->ff, F));
            if (fz & FUSE_DOWN) {
                GemvPro pro;
                pro.kind = PRO_QUANT;
                pro.x = m->ff;
                pro.n = F;
                M_HIP(launch_gemv_p(*m->wdown[l], nullptr, m->xb, pro, GemvEpi(), s));
            } else if (gemv_fused_fits(*m->wdown[l], 1) && (uintptr_t)m->ff % 16 == 0) {
                M_HIP(launch_gemv_x(*m->wdown[l], m->ff, m->xb, 1, s));      // h quantized in the GEMV
            } else {
                M_HIP(launch_quantize_q8_0(m->ff, F, m->act, ast, F, 1, s));
                M_HIP(launch_gemv(*m->wdown[l], m->act, ast, m->xb, 1, s));
            }
        } else {
            M_HIP(launch_norm_quant(x, m->xb, norm_of(m, l, G4H_N_POST_ATTN), norm_of(m, l, G4H_N_FFN), c.rms_eps, E, m->act, s));
            M_RC(trace_copy(tr, TR_XMID, x, E));
            M_HIP(launch_gemv(*m->wgu[l], m->act, ast, m->ff, 1, s));
            M_HIP(launch_gelu_quant(m->ff, F, m->gelu, m->act, s));
            M_HIP(launch_gemv(*m->wdown[l], m->act, ast, m->xb, 1, s));
        }
        M_RC(trace_copy(tr, TR_DOWN, m->xb, E));
    }
    const float *last_post = norm_of(m, c.n_layer - 1, G4H_N_POST_FFW), *out_norm = norm_of(m, c.n_layer, 0);
    if (fz & FUSE_HEAD) {
        M_HIP(norm_gemv(*m->head, m->xb, last_post, out_norm, m->logits, false));
    } else {
        M_HIP(launch_norm_quant(x, m->xb, last_post, out_norm, c.rms_eps, E, m->act, s));
        M_HIP(launch_gemv(*m->head, m->act, ast, m->logits, 1, s));
    }
    M_RC(trace_copy(m->trace ? m->trace + (size_t)c.n_layer * trace_rec : nullptr, TR_X, x, E));
    if (m->sampler)
        M_HIP(launch_sample(sampler_device(m->sampler), c.n_vocab, m->logits, nullptr, 1, m->state, c.n_ctx, s));
    else
        M_HIP(launch_argmax_advance(m->logits, c.n_vocab, m->state, c.n_ctx, s));
    return G4H_OK;
}

extern "C" int g4h_model_set_sampler(g4h_model *m, g4h_sampler *s) {
    if (!m) return g4h_internal_fail(G4H_ERR_ARG, "g4h_model_set_sampler: null model");
    if (s && sampler_n_vocab(s) != m->c.n_vocab)
        return g4h_internal_fail(G4H_ERR_SHAPE, "g4h_model_set_sampler: the sampler's n_vocab differs from the model's");
    m->sampler = s;
    return G4H_OK;
}

// ------------------------------------------------------- batched forward ----
// more than one token attends in one set of launches (G4H_BATCH_ATTN=0: one
// decode attention launch per token, the same bits).  Measured on the
// default model at position 4096: 8 tokens 2.35 against 4.62 ms per forward,
// 64 tokens 12.3 against 34.6 ms; one token keeps the one-launch form (1.30
// against 1.45 ms).
static bool batch_attn() {
    static const bool on = [] {
        const char *e = getenv("G4H_BATCH_ATTN");
        return !e || atoi(e) != 0;
    }();
    return on;
}

static int batch_alloc(g4h_model *m) {
    if (m->bx) return G4H_OK;
    const g4h_model_config &c = m->c;
    const size_t E = c.n_embd, R = (size_t)(c.n_head + 2 * c.n_kv) * c.head_dim, Q = (size_t)c.n_head * c.head_dim,
                 F = c.n_ff, B = kBatchMax;
    M_RC(model_alloc(m, (void **)&m->bx, B * E * 4));
    M_RC(model_alloc(m, (void **)&m->bxb, B * E * 4));
    M_RC(model_alloc(m, (void **)&m->bhn, B * E * 4));
    M_RC(model_alloc(m, (void **)&m->bqkv, B * R * 4));
    M_RC(model_alloc(m, (void **)&m->batt, B * Q * 4));
    M_RC(model_alloc(m, (void **)&m->bff, B * 2 * F * 4));
    M_RC(model_alloc(m, (void **)&m->bact, B * m->act_bytes));
    M_RC(model_alloc(m, (void **)&m->bws, m->ws_bytes));
    M_RC(model_alloc(m, (void **)&m->bq, B * Q * 4));
    M_RC(model_alloc(m, (void **)&m->bbw, attn_batch_workspace_bytes(c.n_head, c.head_dim, c.n_ctx, kBatchMax)));
    M_RC(model_alloc(m, (void **)&m->btok, B * sizeof(int)));
    size_t da_off;
    m->few_cols = std::max(E, std::max(Q, F));
    M_RC(model_alloc(m, (void **)&m->bfew, few_act_bytes(m->few_cols, kBatchMax, &da_off)));
    M_HIP(hipMemset(m->bws, 0, m->ws_bytes));
    return G4H_OK;
}

// floats of one step's trace record per layer, and of the whole step's trace
static size_t trace_rec_floats(const g4h_model_config &c) {
    return 4 * (size_t)c.n_embd + (size_t)(c.n_head + 2 * c.n_kv) * c.head_dim + (size_t)c.n_head * c.head_dim + c.n_ff;
}
static size_t trace_step_floats(const g4h_model_config &c) { return (size_t)c.n_layer * trace_rec_floats(c) + c.n_embd; }

// forward_layers (model.c:592-736) for nb tokens at positions pos0 .. pos0+nb-1.
// Attention and the row steps take the decode step's arithmetic (its q/k/v
// preparation for every token, K/V rows stored at pos0 .. pos0 + nb - 1
// before token b attends 0 .. pos0 + b).  The projections run on kernel family
// `path` of g4h_matmul_ex: 1, the GEMV family of the decode step, makes row b
// equal the decode step of tokens[b] at pos0 + b after tokens[0 .. b-1] bit
// for bit (what speculative verify compares); 0 lets a prompt chunk of 9 or
// more q8_0 / q4_0 tokens read each weight once on the int8 matrix cores, whose
// rows agree with the decode step within the fp32 tolerance instead.  With a
// trace (g4h_model_trace) each token's per-layer record and final x are copied
// out as the decode step's are, token b's at b times a step's trace size.
// Leaves the residual rows in bx and the last Wdown output in bxb.
static int forward_rows(g4h_model *m, const int *tokens, int nb, int pos0, hipStream_t s, int path) {
    const g4h_model_config &c = m->c;
    if (nb < 1 || nb > kBatchMax) return g4h_internal_fail(G4H_ERR_ARG, "g4h_forward_batch: nb must be 1..64 (G4_BATCH_MAX)");
    if (pos0 < 0 || pos0 + nb > c.n_ctx) return g4h_internal_fail(G4H_ERR_ARG, "g4h_forward_batch: positions outside the context");
    if (!tokens) return g4h_internal_fail(G4H_ERR_ARG, "g4h_forward_batch: null tokens");
    for (int b = 0; b < nb; b++)
        if (tokens[b] < 0 || tokens[b] >= c.n_vocab) return g4h_internal_fail(G4H_ERR_ARG, "g4h_forward_batch: token out of range");
    M_RC(batch_alloc(m));
    const int E = c.n_embd, H = c.n_head, KV = c.n_kv, hd = c.head_dim, F = c.n_ff;
    const int R = (H + 2 * KV) * hd, Q = H * hd;
    const size_t ast = m->act_bytes;
    // trace: the decode step's record (x | qkv | att | wo | xmid | h | down) per
    // layer, then the final x; token b's trace starts at b * tf floats
    const size_t TR_QKV = E, TR_ATT = TR_QKV + R, TR_WO = TR_ATT + Q, TR_XMID = TR_WO + E, TR_H = TR_XMID + E,
                 TR_DOWN = TR_H + F, rec = TR_DOWN + E, tf = trace_step_floats(c);
    auto trace_rows = [&](int l, size_t off, const float *src, size_t src_stride, int n) -> int {
        if (!m->trace) return G4H_OK;
        M_HIP(hipMemcpy2DAsync(m->trace + (size_t)l * rec + off, tf * 4, src, src_stride * 4, (size_t)n * 4, nb,
                               hipMemcpyDeviceToDevice, s));
        return G4H_OK;
    };
    // A prompt batch whose projections run k_mm_few: each activation's
    // producer writes that kernel's operand layout itself, sparing the
    // re-layout launch per projection (same codes and scales, so the same
    // bits).  One buffer serves every activation: a block pair's place does
    // not depend on the row length, and the padding tokens stay zero.
    FewAct fa;
    if (path != 1 && nb >= kMmMinTokens && few_direct()) {
        size_t da_off;
        const size_t bytes = few_act_bytes(m->few_cols, nb, &da_off);
        fa.qa = (int8_t *)m->bfew;
        fa.da = (uint16_t *)(m->bfew + da_off);
        fa.mt = (nb + 15) / 16;
        if (m->few_nb != nb) {
            M_HIP(launch_few_clear(m->bfew, bytes, s));
            m->few_nb = nb;
        }
    }
    auto dst = [&](const g4h_tensor *W) { return fa.qa && matmul_few_ready(W, nb, path) ? fa : FewAct(); };
    auto proj = [&](const g4h_tensor *W, const FewAct &f, float *Y) -> int {
        if (f.qa) return matmul_few(W, f, Y, nb, s);
        return g4h_matmul_ex(W, nullptr, m->bact, ast, Y, nb, path, s);
    };
    M_HIP(hipMemcpyAsync(m->btok, tokens, (size_t)nb * sizeof(int), hipMemcpyHostToDevice, s));
    FewAct f = dst(m->wqkv[0]);
    M_HIP(launch_embed_norm(*m->head, m->btok, m->bx, sqrtf((float)E), norm_of(m, 0, G4H_N_ATTN), c.rms_eps, m->bact, s, nb, ast,
                            f));
    for (int l = 0; l < c.n_layer; l++) {
        if (l) {
            f = dst(m->wqkv[l]);
            M_HIP(launch_norm_quant(m->bx, m->bxb, norm_of(m, l - 1, G4H_N_POST_FFW), norm_of(m, l, G4H_N_ATTN), c.rms_eps, E,
                                    m->bact, s, nb, ast, nullptr, f));
        }
        M_RC(trace_rows(l, 0, m->bx, E, E));
        M_RC(proj(m->wqkv[l], f, m->bqkv));
        M_RC(trace_rows(l, TR_QKV, m->bqkv, R, R));
        QkvArgs qa;
        qa.n_head = H;
        qa.n_kv = KV;
        qa.hd = hd;
        qa.kv_type = c.kv_type;
        qa.q_norm = norm_of(m, l, G4H_N_Q);
        qa.k_norm = norm_of(m, l, G4H_N_K);
        qa.rope = m->rope;
        qa.kc = m->kv + (size_t)(2 * l) * m->kv_layer_bytes;
        qa.vc = qa.kc + m->kv_layer_bytes;
        qa.eps = c.rms_eps;
        f = FewAct();
        if (nb > 1 && batch_attn()) {
            // every token's rows prepared and its key / value stored first, then
            // the batch attends in one set of launches
            M_HIP(launch_attn_prep_rows(m->bqkv, qa, pos0, nb, m->bq, s));
            if (path != 1 && nb >= kMmMinTokens && attn_batch_mm_ok(qa)) {  // a prompt batch: the matrix cores
                f = dst(m->wo[l]);
                M_HIP(launch_attn_batch_mm(m->bq, qa, pos0 + 1, nb, m->batt, m->bact, m->bbw,
                                           attn_batch_workspace_bytes(c.n_head, c.head_dim, c.n_ctx, kBatchMax), s, ast,
                                           nullptr, 0, f));
            } else {
                M_HIP(launch_attn_batch(m->bq, qa, pos0 + 1, nb, m->batt, m->bact, m->bbw, s, ast));
            }
        } else {
            for (int b = 0; b < nb; b++)
                M_HIP(launch_attn_decode(nullptr, m->bqkv + (size_t)b * R, qa, pos0 + b + 1, nullptr, c.n_ctx,
                                         m->batt + (size_t)b * Q, m->bact + (size_t)b * ast, m->bws, s));
        }
        M_RC(trace_rows(l, TR_ATT, m->batt, Q, Q));
        M_RC(proj(m->wo[l], f, m->bxb));
        M_RC(trace_rows(l, TR_WO, m->bxb, E, E));
        f = dst(m->wgu[l]);
        M_HIP(launch_norm_quant(m->bx, m->bxb, norm_of(m, l, G4H_N_POST_ATTN), norm_of(m, l, G4H_N_FFN), c.rms_eps, E, m->bact,
                                s, nb, ast, nullptr, f));
        M_RC(trace_rows(l, TR_XMID, m->bx, E, E));
        M_RC(proj(m->wgu[l], f, m->bff));
        f = dst(m->wdown[l]);
        M_HIP(launch_gelu_quant(m->bff, F, m->gelu, m->bact, s, nb, ast, m->trace ? m->trace + (size_t)l * rec + TR_H : nullptr,
                                tf, f));
        M_RC(proj(m->wdown[l], f, m->bxb));
        M_RC(trace_rows(l, TR_DOWN, m->bxb, E, E));
    }
    return G4H_OK;
}

extern "C" int g4h_forward_batch(g4h_model *m, const int *tokens, int nb, int pos0, int want_logits, void *stream) {
    if (!m) return g4h_internal_fail(G4H_ERR_ARG, "g4h_forward_batch: null model");
    const hipStream_t s = (hipStream_t)stream;
    const g4h_model_config &c = m->c;
    M_RC(forward_rows(m, tokens, nb, pos0, s, 0));
    if (want_logits) {
        // head of the last token only (model.c:760-769)
        const size_t E = c.n_embd, last = (size_t)(nb - 1) * E;
        M_HIP(launch_norm_quant(m->bx + last, m->bxb + last, norm_of(m, c.n_layer - 1, G4H_N_POST_FFW), norm_of(m, c.n_layer, 0),
                                c.rms_eps, c.n_embd, m->bact, s));
        if (m->trace)                                        // the last token's final x
            M_HIP(hipMemcpyAsync(m->trace + (size_t)(nb - 1) * trace_step_floats(c) + (size_t)c.n_layer * trace_rec_floats(c),
                                 m->bx + last, E * 4, hipMemcpyDeviceToDevice, s));
        M_RC(g4h_matmul_ex(m->head, nullptr, m->bact, m->act_bytes, m->logits, 1, 1, s));
    }
    M_HIP(hipStreamSynchronize(s));
    return g4h_internal_attn_error(m->bws, s, "g4h_forward_batch");           // per-token one-launch attention
}

extern "C" int g4h_forward_batch_heads(g4h_model *m, const int *tokens, int nb, int pos0, float *logits_dev, float *hnext_dev,
                                       void *stream) {
    if (!m || !logits_dev) return g4h_internal_fail(G4H_ERR_ARG, "g4h_forward_batch_heads: null argument");
    if ((uintptr_t)logits_dev % 16 || (hnext_dev && (uintptr_t)hnext_dev % 16))
        return g4h_internal_fail(G4H_ERR_ARG, "g4h_forward_batch_heads: outputs must be 16-byte aligned");
    const hipStream_t s = (hipStream_t)stream;
    const g4h_model_config &c = m->c;
    M_RC(forward_rows(m, tokens, nb, pos0, s, 1));
    // every position's head input feature and logits (model.c:790-793)
    M_HIP(launch_norm_quant(m->bx, m->bxb, norm_of(m, c.n_layer - 1, G4H_N_POST_FFW), norm_of(m, c.n_layer, 0), c.rms_eps,
                            c.n_embd, m->bact, s, nb, m->act_bytes, hnext_dev ? hnext_dev : m->bhn));
    if (m->trace)                                            // every token's final x
        M_HIP(hipMemcpy2DAsync(m->trace + (size_t)c.n_layer * trace_rec_floats(c), trace_step_floats(c) * 4, m->bx,
                               (size_t)c.n_embd * 4, (size_t)c.n_embd * 4, nb, hipMemcpyDeviceToDevice, s));
    M_RC(g4h_matmul_ex(m->head, nullptr, m->bact, m->act_bytes, logits_dev, nb, 1, s));
    M_HIP(hipStreamSynchronize(s));
    return g4h_internal_attn_error(m->bws, s, "g4h_forward_batch_heads");
}

extern "C" int g4h_argmax_rows(const float *logits_dev, int n, int nb, int *out_dev, void *stream) {
    if (!logits_dev || !out_dev || n < 1 || nb < 1) return g4h_internal_fail(G4H_ERR_ARG, "g4h_argmax_rows: bad argument");
    if ((uintptr_t)logits_dev % 16 || (nb > 1 && n % 4))
        return g4h_internal_fail(G4H_ERR_ARG, "g4h_argmax_rows: rows must be 16-byte aligned");
    M_HIP(launch_argmax_rows(logits_dev, n, nb, out_dev, (hipStream_t)stream));
    return G4H_OK;
}

extern "C" int g4h_model_trace(g4h_model *m, float *trace_dev) {
    if (!m) return g4h_internal_fail(G4H_ERR_ARG, "g4h_model_trace: null model");
    m->trace = trace_dev;
    return G4H_OK;
}

extern "C" int g4h_model_set_state(g4h_model *m, int token, int pos, void *stream) {
    if (!m) return g4h_internal_fail(G4H_ERR_ARG, "g4h_model_set_state: null model");
    if (pos < 0 || pos >= m->c.n_ctx) return g4h_internal_fail(G4H_ERR_ARG, "g4h_model_set_state: pos outside the context");
    if (token < 0 || token >= m->c.n_vocab) return g4h_internal_fail(G4H_ERR_ARG, "g4h_model_set_state: token out of range");
    const int st[3] = {token, pos, pos + 1};
    M_HIP(hipMemcpyAsync(m->state, st, sizeof st, hipMemcpyHostToDevice, (hipStream_t)stream));
    M_HIP(hipMemsetAsync(m->state + 4, 0, sizeof(int), (hipStream_t)stream));     // flags start clear
    M_HIP(hipStreamSynchronize((hipStream_t)stream));
    return G4H_OK;
}

extern "C" int g4h_model_status(g4h_model *m, int *flags, void *stream) {
    if (!m || !flags) return g4h_internal_fail(G4H_ERR_ARG, "g4h_model_status: null argument");
    const hipStream_t s = (hipStream_t)stream;
    int st[5];
    unsigned err = 0;
    M_HIP(hipMemcpyAsync(st, m->state, sizeof st, hipMemcpyDeviceToHost, s));
    M_HIP(hipMemcpyAsync(&err, m->ws + ATTN_ERR_OFFSET, sizeof err, hipMemcpyDeviceToHost, s));
    M_HIP(hipStreamSynchronize(s));
    *flags = ((st[4] & STATE_CTX_FULL) ? G4H_STATUS_CTX_FULL : 0) | (err ? G4H_STATUS_ATTN_TIMEOUT : 0);
    if (err) {                                               // reported once
        M_HIP(hipMemsetAsync(m->ws + ATTN_ERR_OFFSET, 0, sizeof err, s));
        M_HIP(hipStreamSynchronize(s));
    }
    return G4H_OK;
}

extern "C" int g4h_model_get_state(g4h_model *m, int *token, int *pos, void *stream) {
    if (!m) return g4h_internal_fail(G4H_ERR_ARG, "g4h_model_get_state: null model");
    int st[3];
    M_HIP(hipMemcpyAsync(st, m->state, sizeof st, hipMemcpyDeviceToHost, (hipStream_t)stream));
    M_HIP(hipStreamSynchronize((hipStream_t)stream));
    if (token) *token = st[0];
    if (pos) *pos = st[1];
    return G4H_OK;
}

extern "C" int g4h_forward(g4h_model *m, int token, int pos, int *next_token, void *stream) {
    M_RC(g4h_model_set_state(m, token, pos, stream));
    M_RC(g4h_forward_state(m, stream));
    if (next_token) M_RC(g4h_model_get_state(m, next_token, nullptr, stream));
    int flags = 0;
    M_RC(g4h_model_status(m, &flags, stream));
    if (flags & G4H_STATUS_ATTN_TIMEOUT)
        return g4h_internal_fail(G4H_ERR_TIMEOUT, "g4h_forward: an attention hand-off wait gave up; the logits are NaN");
    return G4H_OK;
}

extern "C" const uint16_t *g4h_model_gelu_table(const g4h_model *m) { return m ? m->gelu : nullptr; }

extern "C" const float *g4h_model_logits(const g4h_model *m) { return m ? m->logits : nullptr; }

extern "C" g4h_tensor *g4h_model_matrix(g4h_model *m, int layer, int which) {
    if (!m) return nullptr;
    if (which == G4H_W_HEAD) return m->head;
    if (layer < 0 || layer >= m->c.n_layer) return nullptr;
    switch (which) {
    case G4H_W_QKV: return m->wqkv[layer];
    case G4H_W_O: return m->wo[layer];
    case G4H_W_GU: return m->wgu[layer];
    case G4H_W_DOWN: return m->wdown[layer];
    default: return nullptr;
    }
}

extern "C" float *g4h_model_norm(g4h_model *m, int layer, int which) {
    if (!m) return nullptr;
    if (which == G4H_N_OUTPUT) return norm_of(m, m->c.n_layer, 0);
    if (layer < 0 || layer >= m->c.n_layer || which < 0 || which > 5) return nullptr;
    return norm_of(m, layer, which);
}

extern "C" int g4h_model_kv(g4h_model *m, int layer, void **k_dev, void **v_dev, size_t *bytes) {
    if (!m || layer < 0 || layer >= m->c.n_layer) return g4h_internal_fail(G4H_ERR_ARG, "g4h_model_kv: bad layer");
    if (k_dev) *k_dev = m->kv + (size_t)(2 * layer) * m->kv_layer_bytes;
    if (v_dev) *v_dev = m->kv + (size_t)(2 * layer + 1) * m->kv_layer_bytes;
    if (bytes) *bytes = m->kv_layer_bytes;
    return G4H_OK;
}

extern "C" size_t g4h_model_weight_bytes(const g4h_model *m) {
    if (!m) return 0;
    size_t b = 0;
    for (const auto *v : {&m->wqkv, &m->wo, &m->wgu, &m->wdown})
        for (const g4h_tensor *t : *v) b += (size_t)t->nrows * g4h_row_size(t->type, t->ncols);
    return b + (size_t)m->head->nrows * g4h_row_size(m->head->type, m->head->ncols);
}
