// gemma.cpp -- a gemma4 model from a GGUF file resident on one MI355X and its
// forward (the GPU form of g4_ctx_init + forward_layers / g4_forward_batch_heads,
// model.c:373-477 and 592-799).
//
// Every weight matrix of the file is uploaded once and repacked into the
// resident layout (g4h_tensor_load); token_embd (tied with the head) and
// per_layer_token_embd also stay as GGUF rows for the embedding gather.
// Per token, the forward runs model.c's steps with this library's kernels:
// the projections on the GEMV family (any weight format, the input prepared
// in the weight's activation class as matmul_b does), the decode attention
// with its q/k/v preparation and, for sliding-window layers, a window over a
// KV ring (rows stored twice so every window is one contiguous run), layers
// past n_layer_kv reading the cache of layer n_layer_kv-2 (sliding) or
// n_layer_kv-1 (full), the per-layer embedding injection and the soft-cap.
#include "../../include/g4hip.h"
#include "../../include/g4run_abi.h"

#include <algorithm>
#include <cmath>
#include <cstring>
#include <vector>

#include "host_fp16.h"
#include "kernels.h"

using namespace g4;

extern "C" int g4h_internal_fail(int status, const char *msg);
extern "C" int g4h_internal_attn_error(void *ws, void *stream, const char *fn);

namespace {
constexpr int kRows = 64;          // G4_BATCH_MAX (g4run.h:23)
constexpr int kRing = 576;         // G4_SWA_RING (g4run.h:24-26)
constexpr int kWindowMax = 512;    // G4_SWA_WINDOW_MAX

struct GLayer {
    g4h_tensor *wq = nullptr, *wk = nullptr, *wv = nullptr, *wo = nullptr, *gate = nullptr, *up = nullptr, *down = nullptr,
               *inp_gate = nullptr, *proj = nullptr;
    float *attn_norm = nullptr, *q_norm = nullptr, *k_norm = nullptr, *post_attn_norm = nullptr, *ffn_norm = nullptr,
          *post_ffw_norm = nullptr, *post_norm = nullptr;
    float out_scale = 1.0f;
    int swa = 0, hd = 0, n_ff = 0;
};
}  // namespace

struct g4h_gemma {
    int n_layer = 0, n_layer_kv = 0, E = 0, H = 0, V = 0, PE = 0, hd_full = 0, hd_swa = 0, n_swa = 0, n_ctx = 0, kv_type = 0,
        max_ff = 0, hd_max = 0;
    float eps = 0, softcap = 0;
    std::vector<GLayer> L;
    g4h_tensor *head = nullptr, *ple_proj = nullptr;
    uint8_t *tok_raw = nullptr, *ple_raw = nullptr;
    int tok_type = 0, ple_type = 0;
    size_t tok_rb = 0, ple_rb = 0;
    float *ple_norm = nullptr, *out_norm = nullptr, *rope_swa = nullptr, *rope_full = nullptr;
    std::vector<uint8_t *> kc, vc;
    float *x = nullptr, *xb = nullptr, *q = nullptr, *k = nullptr, *v = nullptr, *qkv = nullptr, *att = nullptr, *g = nullptr,
          *u = nullptr, *pl = nullptr, *plp = nullptr, *plg = nullptr, *hn = nullptr;
    uint8_t *ws = nullptr, *wsf = nullptr;     // one-token attention workspaces: sliding / full layers
    uint8_t *bws = nullptr;                    // batch attention workspace
    uint8_t *bfew = nullptr;                   // a prompt chunk's xb rows as q8_0 in k_mm_few's layout
    int *tok = nullptr;                        // device token ids of a call (kRows)
    int *state = nullptr;                      // decode state: token, pos, npos = pos + 1, steps, flags
    float *logits = nullptr;                   // the step's logits (n_vocab)
    uint16_t *gelu = nullptr;
    float *trace = nullptr;                    // optional per-token trace (g4h_gemma_trace)
    std::vector<void *> allocs;
    std::vector<g4h_tensor *> tensors;
};

#define G_HIP(call)                                                                \
    do {                                                                           \
        hipError_t e_ = (call);                                                    \
        if (e_ != hipSuccess) return g4h_internal_fail(G4H_ERR_HIP, hipGetErrorString(e_)); \
    } while (0)
#define G_RC(call)                  \
    do {                            \
        int rc_ = (call);           \
        if (rc_) return rc_;        \
    } while (0)

namespace {

int gfail(int status, const char *fmt, const char *a = "") {
    char msg[256];
    snprintf(msg, sizeof msg, fmt, a);
    return g4h_internal_fail(status, msg);
}

int galloc(g4h_gemma *m, void **p, size_t bytes) {
    G_RC(g4h_malloc(p, bytes));
    m->allocs.push_back(*p);
    return G4H_OK;
}

const g4_tensor *find(const g4_model_file *mf, const char *fmt, int il, bool need, int *rc) {
    char name[96];
    snprintf(name, sizeof name, fmt, il);
    const g4_tensor *t = g4_find_tensor(mf, name);
    if (!t && need) *rc = gfail(G4H_ERR_ARG, "g4h_gemma_create: missing tensor %s", name);
    return t;
}

// a 2-D weight matrix, uploaded and repacked
int up_matrix(g4h_gemma *m, const g4_tensor *t, g4h_tensor **out) {
    if (t->ndim > 2 || t->ne[2] != 1 || t->ne[3] != 1) return gfail(G4H_ERR_SHAPE, "g4h_gemma_create: %s is not a matrix", t->name);
    G_RC(g4h_tensor_create(t->type, t->ne[0], t->ne[1], out));
    m->tensors.push_back(*out);
    return g4h_tensor_load(*out, t->data, 0, nullptr);
}

// an f32 vector of n values
int up_vec(g4h_gemma *m, const g4_tensor *t, int64_t n, float **out) {
    if (t->type != G4H_F32 || t->ne[0] * t->ne[1] * t->ne[2] * t->ne[3] != n)
        return gfail(G4H_ERR_SHAPE, "g4h_gemma_create: %s must be an f32 vector of the model's width", t->name);
    G_RC(galloc(m, (void **)out, (size_t)n * 4));
    G_HIP(hipMemcpy(*out, t->data, (size_t)n * 4, hipMemcpyHostToDevice));
    return G4H_OK;
}

// rope_cache (model.c:349-357) for every position: [n_ctx][hd] (cos, sin) pairs
std::vector<float> rope_table(int n_ctx, int hd, float base, const float *ff) {
    std::vector<float> t((size_t)n_ctx * hd);
    const float theta_scale = powf(base, -2.0f / hd);
    for (int p = 0; p < n_ctx; p++) {
        float theta = (float)p;
        for (int i = 0; i < hd / 2; i++) {
            const float a = ff ? theta / ff[i] : theta;
            t[(size_t)p * hd + 2 * i] = cosf(a);
            t[(size_t)p * hd + 2 * i + 1] = sinf(a);
            theta *= theta_scale;
        }
    }
    return t;
}

bool attn_hd(int hd) { return hd == 64 || hd == 128 || hd == 192 || hd == 256 || hd == 512; }

int create(const g4_model_file *mf, int n_ctx, int kv_type, g4h_gemma *m) {
    if (std::strcmp(mf->arch, "gemma4") != 0) return gfail(G4H_ERR_TYPE, "g4h_gemma_create: architecture %s is not gemma4", mf->arch);
    if (kv_type != G4H_F16 && kv_type != G4H_Q8_0 && kv_type != G4H_Q4_0)
        return gfail(G4H_ERR_TYPE, "g4h_gemma_create: KV type must be f16, q8_0 or q4_0");
    m->n_layer = mf->n_layer;
    m->n_layer_kv = mf->n_layer_kv;
    m->E = mf->n_embd;
    m->H = mf->n_head;
    m->V = mf->n_vocab;
    m->PE = mf->n_embd_per_layer;
    m->hd_full = mf->head_dim_full;
    m->hd_swa = mf->head_dim_swa;
    m->n_swa = mf->n_swa;
    m->n_ctx = n_ctx;
    m->kv_type = kv_type;
    m->eps = mf->rms_eps;
    m->softcap = mf->final_softcap;
    if (m->n_layer < 1 || m->n_layer_kv < 2 || m->E <= 0 || m->V <= 0 || m->PE <= 0 || n_ctx <= 0)
        return gfail(G4H_ERR_SHAPE, "g4h_gemma_create: bad dimensions");
    if (!attn_hd(m->hd_full) || !attn_hd(m->hd_swa))
        return gfail(G4H_ERR_SHAPE, "g4h_gemma_create: head dims must be 64, 128, 192, 256 or 512 (the attention kernels' rows)");
    if (mf->n_rot_full != m->hd_full || mf->n_rot_swa != m->hd_swa)
        return gfail(G4H_ERR_SHAPE, "g4h_gemma_create: RoPE must cover the whole head (n_rot == head dim)");
    if (m->H != 1 && m->H != 2 && m->H != 4 && m->H != 8)
        return gfail(G4H_ERR_SHAPE, "g4h_gemma_create: 1, 2, 4 or 8 query heads per KV head");
    if (m->n_swa < 1 || m->n_swa > kWindowMax) return gfail(G4H_ERR_SHAPE, "g4h_gemma_create: sliding window must be 1..512");
    if (m->PE > 1024 || m->PE % 4 || m->E % 4) return gfail(G4H_ERR_SHAPE, "g4h_gemma_create: per-layer width <= 1024, widths % 4");
    int rc = G4H_OK;
    const g4_tensor *t_tok = find(mf, "token_embd.weight", 0, true, &rc), *t_ple = find(mf, "per_layer_token_embd.weight", 0, true, &rc),
                    *t_pproj = find(mf, "per_layer_model_proj.weight", 0, true, &rc),
                    *t_pnorm = find(mf, "per_layer_proj_norm.weight", 0, true, &rc),
                    *t_onorm = find(mf, "output_norm.weight", 0, true, &rc), *t_rf = find(mf, "rope_freqs.weight", 0, true, &rc);
    if (rc) return rc;
    const int NPL = m->n_layer * m->PE;
    if (t_tok->ne[0] != m->E || t_tok->ne[1] != m->V || t_ple->ne[0] != NPL || t_ple->ne[1] < m->V)
        return gfail(G4H_ERR_SHAPE, "g4h_gemma_create: embedding shapes");
    G_RC(up_matrix(m, t_tok, &m->head));
    G_RC(up_matrix(m, t_pproj, &m->ple_proj));
    m->tok_type = t_tok->type;
    m->ple_type = t_ple->type;
    m->tok_rb = g4h_row_size(t_tok->type, m->E);
    m->ple_rb = g4h_row_size(t_ple->type, NPL);
    G_RC(galloc(m, (void **)&m->tok_raw, m->tok_rb * m->V));
    G_RC(galloc(m, (void **)&m->ple_raw, m->ple_rb * m->V));
    G_HIP(hipMemcpy(m->tok_raw, t_tok->data, m->tok_rb * m->V, hipMemcpyHostToDevice));
    G_HIP(hipMemcpy(m->ple_raw, t_ple->data, m->ple_rb * m->V, hipMemcpyHostToDevice));
    G_RC(up_vec(m, t_pnorm, m->PE, &m->ple_norm));
    G_RC(up_vec(m, t_onorm, m->E, &m->out_norm));
    if (t_rf->type != G4H_F32 || t_rf->ne[0] < m->hd_full / 2) return gfail(G4H_ERR_SHAPE, "g4h_gemma_create: rope_freqs");
    {
        const std::vector<float> rs = rope_table(n_ctx, m->hd_swa, mf->rope_base_swa, nullptr);
        const std::vector<float> rf = rope_table(n_ctx, m->hd_full, mf->rope_base_full, (const float *)t_rf->data);
        G_RC(galloc(m, (void **)&m->rope_swa, rs.size() * 4));
        G_RC(galloc(m, (void **)&m->rope_full, rf.size() * 4));
        G_HIP(hipMemcpy(m->rope_swa, rs.data(), rs.size() * 4, hipMemcpyHostToDevice));
        G_HIP(hipMemcpy(m->rope_full, rf.data(), rf.size() * 4, hipMemcpyHostToDevice));
    }
    m->L.resize(m->n_layer);
    for (int il = 0; il < m->n_layer; il++) {
        GLayer &L = m->L[il];
        L.swa = mf->is_swa[il] != 0;
        L.hd = L.swa ? m->hd_swa : m->hd_full;
        L.n_ff = mf->n_ff[il];
        m->max_ff = std::max(m->max_ff, L.n_ff);
        const bool kv = il < m->n_layer_kv;
        struct { const char *name; g4h_tensor **dst; bool need; } mats[] = {
            {"blk.%d.attn_q.weight", &L.wq, true},     {"blk.%d.attn_k.weight", &L.wk, kv},
            {"blk.%d.attn_v.weight", &L.wv, false},    {"blk.%d.attn_output.weight", &L.wo, true},
            {"blk.%d.ffn_gate.weight", &L.gate, true}, {"blk.%d.ffn_up.weight", &L.up, true},
            {"blk.%d.ffn_down.weight", &L.down, true}, {"blk.%d.inp_gate.weight", &L.inp_gate, true},
            {"blk.%d.proj.weight", &L.proj, true}};
        for (auto &mm : mats) {
            if (!kv && (mm.dst == &L.wk || mm.dst == &L.wv)) continue;
            const g4_tensor *t = find(mf, mm.name, il, mm.need, &rc);
            if (rc) return rc;
            if (t) G_RC(up_matrix(m, t, mm.dst));
        }
        struct { const char *name; float **dst; int64_t n; bool need; } vecs[] = {
            {"blk.%d.attn_norm.weight", &L.attn_norm, m->E, true},
            {"blk.%d.attn_q_norm.weight", &L.q_norm, L.hd, true},
            {"blk.%d.attn_k_norm.weight", &L.k_norm, L.hd, kv},
            {"blk.%d.post_attention_norm.weight", &L.post_attn_norm, m->E, true},
            {"blk.%d.ffn_norm.weight", &L.ffn_norm, m->E, true},
            {"blk.%d.post_ffw_norm.weight", &L.post_ffw_norm, m->E, true},
            {"blk.%d.post_norm.weight", &L.post_norm, m->E, true}};
        for (auto &vv : vecs) {
            if (!kv && vv.dst == &L.k_norm) continue;
            const g4_tensor *t = find(mf, vv.name, il, vv.need, &rc);
            if (rc) return rc;
            if (t) G_RC(up_vec(m, t, vv.n, vv.dst));
        }
        if (const g4_tensor *t = find(mf, "blk.%d.layer_output_scale.weight", il, false, &rc)) {
            if (t->type != G4H_F32) return gfail(G4H_ERR_TYPE, "g4h_gemma_create: %s must be f32", t->name);
            L.out_scale = *(const float *)t->data;
        }
        // shapes the forward relies on (model.c:421-433)
        const int64_t qrows = (int64_t)m->H * L.hd;
        if (L.wq->nrows != qrows || L.wq->ncols != m->E || L.wo->ncols != qrows || L.wo->nrows != m->E ||
            (kv && (L.wk->nrows != L.hd || (L.wv && L.wv->nrows != L.hd))) || L.gate->nrows != L.n_ff || L.up->nrows != L.n_ff ||
            L.down->ncols != L.n_ff || L.inp_gate->nrows != m->PE || L.proj->ncols != m->PE || L.proj->nrows != m->E)
            return gfail(G4H_ERR_SHAPE, "g4h_gemma_create: layer shapes differ from the hparams");
        if (L.n_ff % 4) return gfail(G4H_ERR_SHAPE, "g4h_gemma_create: FFN width % 4");
    }
    m->hd_max = std::max(m->hd_full, m->hd_swa);
    // layers past n_layer_kv read the cache of layer n_layer_kv - 2 (sliding) or
    // n_layer_kv - 1 (full) (model.c:692): that layer must be of the same kind,
    // so its cache holds rows of the width and the slot count the reader assumes
    for (int il = m->n_layer_kv; il < m->n_layer; il++) {
        const GLayer &L = m->L[il];
        const int cil = L.swa ? m->n_layer_kv - 2 : m->n_layer_kv - 1;
        if (cil < 0 || m->L[cil].swa != L.swa || m->L[cil].hd != L.hd) {
            char msg[160];
            snprintf(msg, sizeof msg, "g4h_gemma_create: shared-KV layer %d would read layer %d's cache of another kind", il, cil);
            return g4h_internal_fail(G4H_ERR_SHAPE, msg);
        }
    }
    // KV caches: sliding layers a ring of kRing slots stored twice, full layers n_ctx slots
    for (int il = 0; il < m->n_layer_kv; il++) {
        const GLayer &L = m->L[il];
        const size_t row = kv_type == G4H_F16 ? (size_t)L.hd * 2 : g4h_row_size(kv_type, L.hd);
        const size_t bytes = row * (L.swa ? 2 * kRing : (size_t)n_ctx);
        uint8_t *k, *v;
        G_RC(galloc(m, (void **)&k, bytes));
        G_RC(galloc(m, (void **)&v, bytes));
        G_HIP(hipMemset(k, 0, bytes));
        G_HIP(hipMemset(v, 0, bytes));
        m->kc.push_back(k);
        m->vc.push_back(v);
    }
    const size_t B = kRows, E = m->E, Q = (size_t)m->H * m->hd_max;
    G_RC(galloc(m, (void **)&m->x, B * E * 4));
    G_RC(galloc(m, (void **)&m->xb, B * E * 4));
    G_RC(galloc(m, (void **)&m->hn, B * E * 4));
    G_RC(galloc(m, (void **)&m->q, B * Q * 4));
    G_RC(galloc(m, (void **)&m->k, B * m->hd_max * 4));
    G_RC(galloc(m, (void **)&m->v, B * m->hd_max * 4));
    G_RC(galloc(m, (void **)&m->qkv, B * (Q + 2 * m->hd_max) * 4));
    G_RC(galloc(m, (void **)&m->att, B * Q * 4));
    G_RC(galloc(m, (void **)&m->g, B * m->max_ff * 4));
    G_RC(galloc(m, (void **)&m->u, B * m->max_ff * 4));
    G_RC(galloc(m, (void **)&m->pl, B * NPL * 4));
    G_RC(galloc(m, (void **)&m->plp, B * NPL * 4));
    G_RC(galloc(m, (void **)&m->plg, B * m->PE * 4));
    size_t da_off;
    G_RC(galloc(m, (void **)&m->bfew, few_act_bytes(E, kRows, &da_off)));
    // one workspace per layer kind (the 512-wide heads' three passes leave
    // untagged words that the one-launch form of the other kind would clear)
    const size_t wss = g4h_attn_workspace_bytes(m->H, m->hd_swa, std::min(n_ctx, m->n_swa)),
                 wsf = g4h_attn_workspace_bytes(m->H, m->hd_full, n_ctx);
    G_RC(galloc(m, (void **)&m->ws, wss));
    G_RC(galloc(m, (void **)&m->wsf, wsf));
    G_HIP(hipMemset(m->ws, 0, wss));
    G_HIP(hipMemset(m->wsf, 0, wsf));
    G_RC(galloc(m, (void **)&m->tok, kRows * sizeof(int)));
    G_RC(galloc(m, (void **)&m->state, 8 * sizeof(int)));
    G_RC(galloc(m, (void **)&m->logits, (size_t)m->V * 4));
    G_HIP(hipMemset(m->state, 0, 8 * sizeof(int)));
    G_RC(galloc(m, (void **)&m->bws, std::max(attn_batch_workspace_bytes(m->H, m->hd_full, n_ctx, kRows),
                                              attn_batch_workspace_bytes(m->H, m->hd_swa, n_ctx, kRows))));
    std::vector<uint16_t> gt(65536);
    for (uint32_t h = 0; h < 65536; h++) gt[h] = gelu_table_entry((uint16_t)h);
    G_RC(galloc(m, (void **)&m->gelu, 65536 * 2));
    G_HIP(hipMemcpy(m->gelu, gt.data(), 65536 * 2, hipMemcpyHostToDevice));
    G_HIP(hipDeviceSynchronize());
    return G4H_OK;
}

// Y[b] = W x[b], x rows of W->ncols floats prepared in W's activation class;
// `path` of g4h_matmul_ex: 1, the GEMV family (token rows bit-identical for any
// count), or 0 (prompt prefill: the int8 matrix cores from 9 tokens)
int mm(const g4h_tensor *W, const float *x, float *Y, int nb, int path, hipStream_t s) {
    return g4h_matmul_ex(W, x, nullptr, 0, Y, nb, path, s);
}

// floats of one token's trace: the per-layer inputs, n_layer records of
// x | q | k | v | att | wo | xmid | g | u | h | down | xffn | plg | plh | proj
// (q and att H * hd_max, k and v hd_max, g | u | h the widest FFN, plg | plh the
// per-layer width, the rest n_embd), then the final x
size_t gemma_trace_floats(const g4h_gemma *m) {
    const size_t E = m->E, Qm = (size_t)m->H * m->hd_max, Fm = m->max_ff, PE = m->PE;
    const size_t rec = 6 * E + 2 * Qm + 2 * (size_t)m->hd_max + 3 * Fm + 2 * PE;
    return (size_t)m->n_layer * PE + (size_t)m->n_layer * rec + E;
}

}  // namespace

extern "C" int g4h_gemma_trace(g4h_gemma *m, float *trace_dev, size_t *floats_per_token) {
    if (!m) return g4h_internal_fail(G4H_ERR_ARG, "g4h_gemma_trace: null model");
    m->trace = trace_dev;
    if (floats_per_token) *floats_per_token = gemma_trace_floats(m);
    return G4H_OK;
}

extern "C" int g4h_gemma_kv(g4h_gemma *m, int layer, void **k_dev, void **v_dev, size_t *bytes) {
    if (!m || layer < 0 || layer >= m->n_layer_kv) return g4h_internal_fail(G4H_ERR_ARG, "g4h_gemma_kv: bad layer");
    const GLayer &L = m->L[layer];
    const size_t row = m->kv_type == G4H_F16 ? (size_t)L.hd * 2 : g4h_row_size(m->kv_type, L.hd);
    if (k_dev) *k_dev = m->kc[layer];
    if (v_dev) *v_dev = m->vc[layer];
    if (bytes) *bytes = row * (L.swa ? 2 * kRing : (size_t)m->n_ctx);
    return G4H_OK;
}

extern "C" int g4h_gemma_free(g4h_gemma *m) {
    if (!m) return G4H_OK;
    for (g4h_tensor *t : m->tensors) g4h_tensor_free(t);
    for (void *p : m->allocs) g4h_free(p);
    delete m;
    return G4H_OK;
}

extern "C" int g4h_gemma_create(const void *model_file, int n_ctx, int kv_type, g4h_gemma **out) {
    if (!model_file || !out) return g4h_internal_fail(G4H_ERR_ARG, "g4h_gemma_create: null argument");
    *out = nullptr;
    g4h_gemma *m = new g4h_gemma();
    if (int rc = create((const g4_model_file *)model_file, n_ctx, kv_type, m)) {
        g4h_gemma_free(m);
        return rc;
    }
    *out = m;
    return G4H_OK;
}

extern "C" int g4h_gemma_open(const char *path, int n_ctx, int kv_type, g4h_gemma **out) {
    if (!path || !out) return g4h_internal_fail(G4H_ERR_ARG, "g4h_gemma_open: null argument");
    g4_model_file mf;
    if (g4_gguf_open(&mf, path, false) != 0) return gfail(G4H_ERR_ARG, "g4h_gemma_open: cannot read GGUF file %s", path);
    const int rc = g4h_gemma_create(&mf, n_ctx, kv_type, out);
    g4_gguf_close(&mf);                      // every tensor now lives on the device
    return rc;
}

extern "C" int g4h_gemma_info(const g4h_gemma *m, int *n_vocab, int *n_embd, int *n_layer, int *n_ctx) {
    if (!m) return g4h_internal_fail(G4H_ERR_ARG, "g4h_gemma_info: null model");
    if (n_vocab) *n_vocab = m->V;
    if (n_embd) *n_embd = m->E;
    if (n_layer) *n_layer = m->n_layer;
    if (n_ctx) *n_ctx = m->n_ctx;
    return G4H_OK;
}

// The attention of nb tokens over the cache of qa, the queries prepared in
// m->q: on the matrix cores where the layer allows (f16 cache, head dim up to
// 256), for every call -- a token's row has the same bits in any batch, so
// decode steps, verify batches and prompt batches agree --, else the
// per-token kernels' batch form.  pos_dev: token 0's position on the device
// (a decode step), then npos_max bounds the positions attended.
static int attend(g4h_gemma *m, const QkvArgs &qa, int pos0, int nb, const int *pos_dev, int npos_max, hipStream_t s) {
    if (attn_batch_mm_ok(qa)) {
        const size_t wsb = std::max(attn_batch_workspace_bytes(m->H, m->hd_full, m->n_ctx, kRows),
                                    attn_batch_workspace_bytes(m->H, m->hd_swa, m->n_ctx, kRows));
        G_HIP(launch_attn_batch_mm(m->q, qa, pos0 + 1, nb, m->att, nullptr, m->bws, wsb, s, 0, pos_dev, npos_max));
    } else {
        G_HIP(launch_attn_batch(m->q, qa, pos0 + 1, nb, m->att, nullptr, m->bws, s));
    }
    return G4H_OK;
}

// The forward of nb tokens whose ids are in tok_dev (device) at positions
// pos0 .. pos0 + nb - 1; with `st` (one token, the decode state token | pos |
// npos on the device) the position comes from st instead, and the call is
// stream-ordered only (graph-capturable).  With `last` false every position's
// logits go to logits_dev, the head inputs to hnext_dev if given; with `last`
// true only the last position's logits, if logits_dev (g4_forward_batch).
// `path` is the projections' matmul path (mm).
static int run(g4h_gemma *m, const int *tok_dev, int nb, int pos0, const int *st, float *logits_dev, float *hnext_dev,
               int path, bool last, hipStream_t s) {
    const int *pos_dev = st ? st + 1 : nullptr, *npos_dev = st ? st + 2 : nullptr;
    const int E = m->E, H = m->H, PE = m->PE, NPL = m->n_layer * PE;
    const float eps = m->eps;
    // per-token trace (g4h_gemma_trace): pl, then per layer the record below, then the final x
    const size_t Qm = (size_t)H * m->hd_max, Fm = m->max_ff;
    const size_t T_X = 0, T_Q = E, T_K = T_Q + Qm, T_V = T_K + m->hd_max, T_ATT = T_V + m->hd_max, T_WO = T_ATT + Qm,
                 T_XMID = T_WO + E, T_G = T_XMID + E, T_U = T_G + Fm, T_H = T_U + Fm, T_DOWN = T_H + Fm, T_XFFN = T_DOWN + E,
                 T_PLG = T_XFFN + E, T_PLH = T_PLG + PE, T_PROJ = T_PLH + PE, rec = T_PROJ + E;
    const size_t tf = gemma_trace_floats(m);
    auto tr = [&](size_t off, const float *src, size_t stride, size_t n) -> int {
        if (!m->trace) return G4H_OK;
        G_HIP(hipMemcpy2DAsync(m->trace + off, tf * 4, src, stride * 4, n * 4, nb, hipMemcpyDeviceToDevice, s));
        return G4H_OK;
    };
    auto trl = [&](int il, size_t off, const float *src, size_t stride, size_t n) {
        return tr((size_t)NPL + (size_t)il * rec + off, src, stride, n);
    };

    // A prompt chunk's projections of the xb rows that run k_mm_few (q / k /
    // v, gate / up) share one quantizer launch per group: the codes are those
    // each call would make, so the same bits.  fq_ok: fq holds the current xb.
    FewAct fq;
    bool fq_ok = false;
    if (path != 1 && nb >= kMmMinTokens && nb <= kRows && few_direct()) {
        size_t da_off;
        few_act_bytes(E, nb, &da_off);
        fq.qa = (int8_t *)m->bfew;
        fq.da = (uint16_t *)(m->bfew + da_off);
        fq.mt = (nb + 15) / 16;
    }
    auto mm_xb = [&](const g4h_tensor *W, float *Y) -> int {
        if (!fq.qa || W->ncols != E || !matmul_few_ready(W, nb, path)) return mm(W, m->xb, Y, nb, path, s);
        if (!fq_ok) {
            G_HIP(launch_quantize_few(m->xb, E, E, nb, fq, s));
            fq_ok = true;
        }
        return matmul_few(W, fq, Y, nb, s);
    };

    // embeddings and per-layer token rows (model.c:602-615), gathered on the device
    G_HIP(launch_dequant(m->tok_type, m->tok_raw, m->tok_rb, m->x, E, E, nb, s, tok_dev));
    G_HIP(launch_dequant(m->ple_type, m->ple_raw, m->ple_rb, m->pl, NPL, NPL, nb, s, tok_dev));
    G_HIP(launch_scale(m->x, (int64_t)nb * E, sqrtf((float)E), s));
    G_HIP(launch_scale(m->pl, (int64_t)nb * NPL, sqrtf((float)PE), s));
    // per-layer input projection (model.c:617-635)
    G_RC(mm(m->ple_proj, m->x, m->plp, nb, path, s));
    G_HIP(launch_ple_prep(m->plp, m->pl, m->ple_norm, PE, m->n_layer, nb, 1.0f / sqrtf((float)E), 1.0f / sqrtf(2.0f), eps, s));
    G_RC(tr(0, m->pl, NPL, NPL));

    for (int il = 0; il < m->n_layer; il++) {
        const GLayer &L = m->L[il];
        const int hd = L.hd, nq = H * hd, F = L.n_ff;
        const float *rope = L.swa ? m->rope_swa : m->rope_full;
        G_RC(trl(il, T_X, m->x, E, E));
        if (il == 0) G_HIP(launch_rms_rows(m->x, L.attn_norm, m->xb, E, nb, eps, s));   // later layers: the previous residual's launch
        fq_ok = false;                                                  // xb rewritten: q / k / v read it next
        // one token of a layer with its own K and V: the projections write the
        // attention's q | k | v row in place (no packing launch)
        const bool direct = nb == 1 && il < m->n_layer_kv && L.wv;
        float *qraw = direct ? m->qkv : m->q;
        G_RC(mm_xb(L.wq, qraw));
        G_RC(trl(il, T_Q, qraw, nq, nq));
        QkvArgs qa;
        qa.n_head = H;
        qa.n_kv = 1;
        qa.hd = hd;
        qa.kv_type = m->kv_type;
        qa.q_norm = L.q_norm;
        qa.k_norm = L.k_norm;
        qa.rope = rope;
        qa.eps = eps;
        qa.window = L.swa ? m->n_swa : 0;
        qa.ring = L.swa ? kRing : 0;
        const int npos_max = L.swa ? std::min(m->n_ctx, m->n_swa) : m->n_ctx;
        uint8_t *ws = L.swa ? m->ws : m->wsf;
        if (il < m->n_layer_kv) {
            // own K/V: q | k | v prepared, stored at the position and attended in one step (model.c:664-689)
            float *kraw = direct ? m->qkv + nq : m->k, *vraw = direct ? m->qkv + nq + hd : m->v;
            G_RC(mm_xb(L.wk, kraw));
            if (L.wv) G_RC(mm_xb(L.wv, vraw));
            G_RC(trl(il, T_K, kraw, hd, hd));
            if (L.wv) G_RC(trl(il, T_V, vraw, hd, hd));
            if (!direct) G_HIP(launch_pack_qkv(m->q, m->k, L.wv ? m->v : nullptr, m->qkv, nq, hd, nb, s));
            qa.kc = m->kc[il];
            qa.vc = m->vc[il];
            if (attn_batch_mm_ok(qa)) {                              // every row stored, then the matrix cores attend
                G_HIP(launch_attn_prep_rows(m->qkv, qa, pos0, nb, m->q, s, pos_dev));
                G_RC(attend(m, qa, pos0, nb, pos_dev, npos_max, s));
            } else if (nb > 1) {                                     // every row stored, then the batch attends
                G_HIP(launch_attn_prep_rows(m->qkv, qa, pos0, nb, m->q, s));
                G_RC(attend(m, qa, pos0, nb, nullptr, 0, s));
            } else if (hd == 512) {                                  // wide heads: rows prepared first, then the halves attend
                G_HIP(launch_attn_prep_rows(m->qkv, qa, pos0, 1, m->q, s, pos_dev));
                G_HIP(launch_attn_decode(m->q, nullptr, qa, pos0 + 1, npos_dev, npos_max, m->att, nullptr, ws, s));
            } else {
                G_HIP(launch_attn_decode(nullptr, m->qkv, qa, pos0 + 1, npos_dev, npos_max, m->att, nullptr, ws, s));
            }
        } else {
            // a shared cache: the queries are prepared here (model.c:666-672, 692)
            const int cil = L.swa ? m->n_layer_kv - 2 : m->n_layer_kv - 1;
            G_HIP(launch_head_prep(m->q, H, hd, nb, L.q_norm, rope, pos0, eps, s, pos_dev));
            qa.kc = m->kc[cil];
            qa.vc = m->vc[cil];
            if (nb > 1 || attn_batch_mm_ok(qa)) G_RC(attend(m, qa, pos0, nb, pos_dev, npos_max, s));
            else G_HIP(launch_attn_decode(m->q, nullptr, qa, pos0 + 1, npos_dev, npos_max, m->att, nullptr, ws, s));
        }
        G_RC(trl(il, T_ATT, m->att, nq, nq));
        G_RC(mm(L.wo, m->att, m->xb, nb, path, s));
        G_RC(trl(il, T_WO, m->xb, E, E));
        // the attention residual and the FFN's RMSNorm in one launch
        G_HIP(launch_resid(m->x, m->xb, L.post_attn_norm, E, nb, eps, 1.0f, s, L.ffn_norm, m->xb));
        G_RC(trl(il, T_XMID, m->x, E, E));
        // FFN (model.c:718-736); one untraced token: h = gelu(gate) * up in the
        // up projection's store (k_gelu_mul's arithmetic, one launch fewer)
        const bool fold = nb == 1 && !m->trace;
        fq_ok = false;                                                  // xb rewritten: gate / up read it next
        G_RC(mm_xb(L.gate, m->g));
        if (fold) {
            GemvOut o;
            o.mode = OUT_GELU_E;
            o.e = m->g;
            o.gelu = m->gelu;
            G_RC(matmul_out(L.up, m->xb, m->g, 1, s, o));
        } else {
            G_RC(mm_xb(L.up, m->u));
            G_RC(trl(il, T_G, m->g, F, F));
            G_RC(trl(il, T_U, m->u, F, F));
            G_HIP(launch_gelu_mul(m->g, F, m->u, F, F, nb, m->gelu, s));
        }
        G_RC(trl(il, T_H, m->g, F, F));
        G_RC(mm(L.down, m->g, m->xb, nb, path, s));
        G_RC(trl(il, T_DOWN, m->xb, E, E));
        G_HIP(launch_resid(m->x, m->xb, L.post_ffw_norm, E, nb, eps, 1.0f, s));
        G_RC(trl(il, T_XFFN, m->x, E, E));
        // per-layer embedding injection (model.c:738-752)
        if (fold) {                                                      // gelu(gate) * the layer's row, in the store
            GemvOut o;
            o.mode = OUT_GELU_ACC;
            o.e = m->pl + (size_t)il * PE;
            o.gelu = m->gelu;
            G_RC(matmul_out(L.inp_gate, m->x, m->plg, 1, s, o));
        } else {
            G_RC(mm(L.inp_gate, m->x, m->plg, nb, path, s));
            G_RC(trl(il, T_PLG, m->plg, PE, PE));
            G_HIP(launch_gelu_mul(m->plg, PE, m->pl + (size_t)il * PE, NPL, PE, nb, m->gelu, s));
        }
        G_RC(trl(il, T_PLH, m->plg, PE, PE));
        G_RC(mm(L.proj, m->plg, m->xb, nb, path, s));
        G_RC(trl(il, T_PROJ, m->xb, E, E));
        // the layer's last residual and the next layer's RMSNorm in one launch
        const float *next_norm = il + 1 < m->n_layer ? m->L[il + 1].attn_norm : nullptr;
        G_HIP(launch_resid(m->x, m->xb, L.post_norm, E, nb, eps, L.out_scale, s, next_norm, next_norm ? m->xb : nullptr));
    }
    G_RC(tr((size_t)NPL + (size_t)m->n_layer * rec, m->x, E, E));
    if (last) {
        // the last token's head (model.c:757-776)
        if (!logits_dev) return G4H_OK;
        G_HIP(launch_rms_rows(m->x + (size_t)(nb - 1) * E, m->out_norm, m->hn, E, 1, eps, s));
        G_RC(mm(m->head, m->hn, logits_dev, 1, 1, s));
        if (m->softcap > 0) G_HIP(launch_softcap(logits_dev, m->V, m->softcap, s));
        return G4H_OK;
    }
    // every position's head (model.c:790-798)
    float *hn = hnext_dev ? hnext_dev : m->hn;
    G_HIP(launch_rms_rows(m->x, m->out_norm, hn, E, nb, eps, s));
    G_RC(mm(m->head, hn, logits_dev, nb, path, s));
    if (m->softcap > 0) G_HIP(launch_softcap(logits_dev, (int64_t)nb * m->V, m->softcap, s));
    return G4H_OK;
}

// the host tokens checked and uploaded, the forward run, its attention waits checked
static int batch_call(g4h_gemma *m, const int *tokens, int nb, int pos0, float *logits_dev, float *hnext_dev, int path,
                      bool last, hipStream_t s, const char *fn) {
    if (nb < 1 || nb > kRows) return gfail(G4H_ERR_ARG, "%s: nb must be 1..64 (G4_BATCH_MAX)", fn);
    if (pos0 < 0 || pos0 + nb > m->n_ctx) return gfail(G4H_ERR_ARG, "%s: positions outside the context", fn);
    for (int b = 0; b < nb; b++)
        if (tokens[b] < 0 || tokens[b] >= m->V) return gfail(G4H_ERR_ARG, "%s: token out of range", fn);
    G_HIP(hipMemcpyAsync(m->tok, tokens, (size_t)nb * sizeof(int), hipMemcpyHostToDevice, s));
    G_RC(run(m, m->tok, nb, pos0, nullptr, logits_dev, hnext_dev, path, last, s));
    G_HIP(hipStreamSynchronize(s));
    const int e0 = g4h_internal_attn_error(m->ws, s, fn);                 // both read and cleared
    const int e1 = g4h_internal_attn_error(m->wsf, s, fn);
    return e0 ? e0 : e1;
}

extern "C" int g4h_gemma_forward(g4h_gemma *m, const int *tokens, int nb, int pos0, float *logits_dev, float *hnext_dev,
                                 void *stream) {
    if (!m || !tokens || !logits_dev) return g4h_internal_fail(G4H_ERR_ARG, "g4h_gemma_forward: null argument");
    return batch_call(m, tokens, nb, pos0, logits_dev, hnext_dev, 1, false, (hipStream_t)stream, "g4h_gemma_forward");
}

extern "C" int g4h_gemma_prefill(g4h_gemma *m, const int *tokens, int nb, int pos0, float *logits_dev, void *stream) {
    if (!m || !tokens) return g4h_internal_fail(G4H_ERR_ARG, "g4h_gemma_prefill: null argument");
    return batch_call(m, tokens, nb, pos0, logits_dev, nullptr, 0, true, (hipStream_t)stream, "g4h_gemma_prefill");
}

// ------------------------------------------------ device-driven decode --
extern "C" int g4h_gemma_set_state(g4h_gemma *m, int token, int pos, void *stream) {
    if (!m) return g4h_internal_fail(G4H_ERR_ARG, "g4h_gemma_set_state: null model");
    if (pos < 0 || pos >= m->n_ctx) return g4h_internal_fail(G4H_ERR_ARG, "g4h_gemma_set_state: pos outside the context");
    if (token < 0 || token >= m->V) return g4h_internal_fail(G4H_ERR_ARG, "g4h_gemma_set_state: token out of range");
    const int st[5] = {token, pos, pos + 1, 0, 0};
    G_HIP(hipMemcpyAsync(m->state, st, sizeof st, hipMemcpyHostToDevice, (hipStream_t)stream));
    G_HIP(hipStreamSynchronize((hipStream_t)stream));
    return G4H_OK;
}

extern "C" int g4h_gemma_step(g4h_gemma *m, void *stream) {
    if (!m) return g4h_internal_fail(G4H_ERR_ARG, "g4h_gemma_step: null model");
    const hipStream_t s = (hipStream_t)stream;
    G_RC(run(m, m->state, 1, 0, m->state, m->logits, nullptr, 1, false, s));
    G_HIP(launch_argmax_advance(m->logits, m->V, m->state, m->n_ctx, s));   // token <- first argmax, pos += 1
    return G4H_OK;
}

extern "C" int g4h_gemma_get_state(g4h_gemma *m, int *token, int *pos, void *stream) {
    if (!m) return g4h_internal_fail(G4H_ERR_ARG, "g4h_gemma_get_state: null model");
    int st[3];
    G_HIP(hipMemcpyAsync(st, m->state, sizeof st, hipMemcpyDeviceToHost, (hipStream_t)stream));
    G_HIP(hipStreamSynchronize((hipStream_t)stream));
    if (token) *token = st[0];
    if (pos) *pos = st[1];
    return G4H_OK;
}

extern "C" int g4h_gemma_status(g4h_gemma *m, int *flags, void *stream) {
    if (!m || !flags) return g4h_internal_fail(G4H_ERR_ARG, "g4h_gemma_status: null argument");
    const hipStream_t s = (hipStream_t)stream;
    int st[5];
    G_HIP(hipMemcpyAsync(st, m->state, sizeof st, hipMemcpyDeviceToHost, s));
    G_HIP(hipStreamSynchronize(s));
    const int t0 = g4h_internal_attn_error(m->ws, s, "g4h_gemma_status"), t1 = g4h_internal_attn_error(m->wsf, s, "g4h_gemma_status");
    if ((t0 && t0 != G4H_ERR_TIMEOUT) || (t1 && t1 != G4H_ERR_TIMEOUT)) return t0 ? t0 : t1;
    *flags = ((st[4] & STATE_CTX_FULL) ? G4H_STATUS_CTX_FULL : 0) | (t0 || t1 ? G4H_STATUS_ATTN_TIMEOUT : 0);
    return G4H_OK;
}

extern "C" const float *g4h_gemma_logits(const g4h_gemma *m) { return m ? m->logits : nullptr; }
