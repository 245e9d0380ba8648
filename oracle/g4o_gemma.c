/*
 * g4o_gemma.c -- CPU restatement of the reference's gemma4 forward
 * (model.c:592-799): per-layer token embeddings, sliding-window layers with a
 * KV ring, full layers with RoPE frequency factors, single-KV-head attention,
 * KV shared by the last layers, per-layer FFN widths, the per-layer embedding
 * injection and the final logit soft-cap.
 *
 * TEST INFRASTRUCTURE ONLY (see g4o.h).  Weights are raw GGUF rows of any
 * type the oracle's matmul takes; each projection's input is prepared in its
 * own activation class exactly as matmul_b does (model.c:257-270).
 */
#include "g4o.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

#define G4O_SWA_RING 576     /* g4run.h:24-26: window 512 + one batch of 64 */

/* Y[b] = W x[b] for nb rows of x (fp32), x prepared in W's activation class */
static void mm(const g4o_mat *W, const float *x, int nb, float *Y, int nthreads) {
    const size_t st = g4o_act_stride(W->type, W->ncols);
    void *qa = malloc(st * (size_t)nb + 64);
    g4o_prep_act(W->type, x, W->ncols, nb, qa);
    g4o_matmul(W->type, W->data, qa, st, Y, W->ncols, W->nrows, nb, nthreads);
    free(qa);
}

size_t g4o_gemma_cache_bytes(const g4o_gemma *g, int il) {
    const int hd = g->is_swa[il] ? g->hd_swa : g->hd_full;
    const int slots = g->is_swa[il] ? G4O_SWA_RING : g->n_ctx;
    const size_t row = g->kv_type == G4O_F16 ? (size_t)hd * 2 : g4o_row_size(g->kv_type, hd);
    return row * (size_t)slots;
}

void g4o_gemma_forward(const g4o_gemma *g, const int *tokens, int nb, int pos0, float *logits, float *hnext,
                       int nthreads) {
    const int E = g->n_embd, H = g->n_head, PE = g->n_embd_per_layer, NPL = g->n_layer * PE;
    const float eps = g->eps;
    int max_ff = 0, hd_max = g->hd_full > g->hd_swa ? g->hd_full : g->hd_swa;
    for (int l = 0; l < g->n_layer; l++) max_ff = g->n_ff[l] > max_ff ? g->n_ff[l] : max_ff;
    const int wide = max_ff > E ? max_ff : E;
    float *x = calloc((size_t)nb * E, 4), *xb = calloc((size_t)nb * E, 4);
    float *pl = calloc((size_t)nb * NPL, 4), *plp = calloc((size_t)nb * NPL, 4), *plg = calloc((size_t)nb * PE, 4);
    float *q = calloc((size_t)nb * H * hd_max, 4), *k = calloc((size_t)nb * hd_max, 4), *v = calloc((size_t)nb * hd_max, 4);
    float *att = calloc((size_t)nb * H * hd_max, 4), *ffh = calloc((size_t)nb * wide, 4), *ffh2 = calloc((size_t)nb * wide, 4);
    float *rc_full = calloc((size_t)nb * g->hd_full, 4), *rc_swa = calloc((size_t)nb * g->hd_swa, 4);
    float *row = calloc((size_t)(NPL > E ? NPL : E), 4);

    /* embeddings and per-layer token rows (model.c:602-615) */
    const float es = sqrtf((float)E), ts = sqrtf((float)PE);
    const size_t erb = g4o_row_size(g->tok_embd.type, E), prb = g4o_row_size(g->per_layer_tok_embd.type, NPL);
    for (int b = 0; b < nb; b++) {
        g4o_dequant_row(g->tok_embd.type, (const uint8_t *)g->tok_embd.data + (size_t)tokens[b] * erb, x + (size_t)b * E, E);
        for (int i = 0; i < E; i++) x[(size_t)b * E + i] *= es;
        g4o_dequant_row(g->per_layer_tok_embd.type, (const uint8_t *)g->per_layer_tok_embd.data + (size_t)tokens[b] * prb,
                        pl + (size_t)b * NPL, NPL);
        for (int i = 0; i < NPL; i++) pl[(size_t)b * NPL + i] *= ts;
    }
    /* per-layer input projection (model.c:617-635) */
    mm(&g->per_layer_model_proj, x, nb, plp, nthreads);
    const float ps = 1.0f / sqrtf((float)E), is2 = 1.0f / sqrtf(2.0f);
    for (int b = 0; b < nb; b++) {
        float *pp_b = plp + (size_t)b * NPL, *pt_b = pl + (size_t)b * NPL;
        for (int i = 0; i < NPL; i++) pp_b[i] *= ps;
        for (int l = 0; l < g->n_layer; l++) {
            float *pp = pp_b + (size_t)l * PE, *pt = pt_b + (size_t)l * PE;
            g4o_rms_norm(pp, g->per_layer_proj_norm, pp, PE, eps);
            for (int i = 0; i < PE; i++) pt[i] = (pp[i] + pt[i]) * is2;
        }
    }
    /* rope caches (model.c:638-642) */
    for (int b = 0; b < nb; b++) {
        g4o_rope_cache_ff(rc_swa + (size_t)b * g->hd_swa, g->hd_swa, pos0 + b, g->rope_base_swa, NULL);
        g4o_rope_cache_ff(rc_full + (size_t)b * g->hd_full, g->hd_full, pos0 + b, g->rope_base_full, g->rope_freqs);
    }

    for (int il = 0; il < g->n_layer; il++) {
        const g4o_gemma_layer *L = &g->layers[il];
        const int swa = g->is_swa[il] != 0, hd = swa ? g->hd_swa : g->hd_full, qrows = H * hd;
        const float *rc = swa ? rc_swa : rc_full;
        const int slots = swa ? G4O_SWA_RING : g->n_ctx;
        const size_t krb = g->kv_type == G4O_F16 ? (size_t)hd * 2 : g4o_row_size(g->kv_type, hd);

        for (int b = 0; b < nb; b++) g4o_rms_norm(x + (size_t)b * E, L->attn_norm, xb + (size_t)b * E, E, eps);
        mm(&L->wq, xb, nb, q, nthreads);
        for (int b = 0; b < nb; b++)
            for (int h = 0; h < H; h++) {
                float *qh = q + (size_t)b * qrows + (size_t)h * hd;
                g4o_rms_norm(qh, L->q_norm, qh, hd, eps);
                g4o_rope_apply(qh, rc + (size_t)b * hd, hd);
            }
        if (il < g->n_layer_kv) {
            mm(&L->wk, xb, nb, k, nthreads);
            if (L->wv.data) mm(&L->wv, xb, nb, v, nthreads);
            for (int b = 0; b < nb; b++) {
                float *kb = k + (size_t)b * hd, *vb = v + (size_t)b * hd;
                if (!L->wv.data) memcpy(vb, kb, (size_t)hd * 4);     /* V = K (raw projection) */
                g4o_rms_norm(kb, L->k_norm, kb, hd, eps);
                g4o_rope_apply(kb, rc + (size_t)b * hd, hd);
                g4o_rms_norm(vb, NULL, vb, hd, eps);
                g4o_kv_store(g->kv_type, (uint8_t *)g->kc[il] + (size_t)((pos0 + b) % slots) * krb, kb, hd);
                g4o_kv_store(g->kv_type, (uint8_t *)g->vc[il] + (size_t)((pos0 + b) % slots) * krb, vb, hd);
            }
        }
        /* attention over this layer's cache or the one it shares (model.c:691-707) */
        const int cil = il < g->n_layer_kv ? il : (swa ? g->n_layer_kv - 2 : g->n_layer_kv - 1);
        for (int b = 0; b < nb; b++) {
            const int pos = pos0 + b;
            const int j0 = swa && pos - (g->n_swa - 1) > 0 ? pos - (g->n_swa - 1) : 0;
            g4o_attn_window(q + (size_t)b * qrows, g->kc[cil], g->vc[cil], g->kv_type, H, 1, hd, pos, j0, slots,
                            att + (size_t)b * qrows, nthreads);
        }
        /* output projection + residual (model.c:710-716) */
        mm(&L->wo, att, nb, xb, nthreads);
        for (int b = 0; b < nb; b++) {
            float *xx = x + (size_t)b * E, *y = xb + (size_t)b * E;
            g4o_rms_norm(y, L->post_attn_norm, y, E, eps);
            for (int i = 0; i < E; i++) xx[i] += y[i];
        }
        /* FFN (model.c:718-736) */
        const int F = g->n_ff[il];
        for (int b = 0; b < nb; b++) g4o_rms_norm(x + (size_t)b * E, L->ffn_norm, xb + (size_t)b * E, E, eps);
        mm(&L->gate, xb, nb, ffh, nthreads);
        mm(&L->up, xb, nb, ffh2, nthreads);
        for (int b = 0; b < nb; b++)
            for (int i = 0; i < F; i++) ffh[(size_t)b * F + i] = g4o_gelu(ffh[(size_t)b * F + i]) * ffh2[(size_t)b * F + i];
        mm(&L->down, ffh, nb, xb, nthreads);
        for (int b = 0; b < nb; b++) {
            float *xx = x + (size_t)b * E, *y = xb + (size_t)b * E;
            g4o_rms_norm(y, L->post_ffw_norm, y, E, eps);
            for (int i = 0; i < E; i++) xx[i] += y[i];
        }
        /* per-layer embedding injection (model.c:738-752) */
        mm(&L->inp_gate, x, nb, plg, nthreads);
        for (int b = 0; b < nb; b++)
            for (int i = 0; i < PE; i++)
                plg[(size_t)b * PE + i] = g4o_gelu(plg[(size_t)b * PE + i]) * pl[(size_t)b * NPL + (size_t)il * PE + i];
        mm(&L->proj, plg, nb, xb, nthreads);
        for (int b = 0; b < nb; b++) {
            float *xx = x + (size_t)b * E, *y = xb + (size_t)b * E;
            g4o_rms_norm(y, L->post_norm, y, E, eps);
            for (int i = 0; i < E; i++) xx[i] = (xx[i] + y[i]) * L->out_scale;
        }
    }

    /* every position's head (model.c:790-798) */
    float *hn = hnext ? hnext : calloc((size_t)nb * E, 4);
    for (int b = 0; b < nb; b++) g4o_rms_norm(x + (size_t)b * E, g->output_norm, hn + (size_t)b * E, E, eps);
    mm(&g->tok_embd, hn, nb, logits, nthreads);
    if (g->softcap > 0) {
        const float cap = g->softcap;
        for (size_t i = 0; i < (size_t)nb * g->n_vocab; i++) logits[i] = cap * tanhf(logits[i] / cap);
    }
    if (!hnext) free(hn);
    free(x); free(xb); free(pl); free(plp); free(plg); free(q); free(k); free(v); free(att);
    free(ffh); free(ffh2); free(rc_full); free(rc_swa); free(row);
}
