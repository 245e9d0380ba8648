/* abi_driver.c -- a C caller written to g4run.h's prototypes (include/g4run_abi.h),
 * linked with -lg4hip and nothing of the reference, checked against the CPU
 * oracle (liboracle.so, test infrastructure):
 *   tables      g4_init_tables' fp16 and GELU tables, all 65536 codes, bit for bit
 *   quantizers  g4_quantize_q8_0 / q8_K / q4_0, bit for bit
 *   dequant     g4_dequant_row for every weight format, bit for bit
 *   dots        g4_dot_<fmt> within |gpu - cpu| <= 1e-5 + 1e-3 |cpu| of the
 *               oracle's shipped-order dot; g4_dot_<fmt>_x4 equal to the 1-token
 *               dots bit for bit
 *   matmul      g4gpu_matmul (tests/c/g4gpu.c, the INTEGRATION.md backend) on
 *               uploaded g4_tensor weights against the oracle's prep_act+matmul
 *   sampler     g4_sampler_init/ban/accept/free and g4_sample on the reference's
 *               struct against the oracle's chain: ids, rewritten logits, RNG
 *               words and ring bookkeeping bit for bit
 * Prints one line per check and exits non-zero on the first failure. */
#include <math.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "g4gpu.h"
#include "g4o.h"

static uint64_t rs = 0x9e3779b97f4a7c15ull;
static uint64_t next64(void) {                 /* splitmix64 */
    uint64_t z = (rs += 0x9e3779b97f4a7c15ull);
    z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ull;
    z = (z ^ (z >> 27)) * 0x94d049bb133111ebull;
    return z ^ (z >> 31);
}
static double unif(void) { return (double)(next64() >> 11) * (1.0 / 9007199254740992.0); }
static float gauss(void) {
    const double u = unif() + 1e-300, v = unif();
    return (float)(sqrt(-2.0 * log(u)) * cos(6.283185307179586 * v));
}

static int failures;
#define CHECK(cond, ...)                                  \
    do {                                                  \
        if (!(cond)) {                                    \
            printf("FAIL ");                              \
            printf(__VA_ARGS__);                          \
            printf("\n");                                 \
            fflush(stdout);                               \
            exit(1);                                      \
        }                                                 \
    } while (0)

/* random GGUF rows: every byte random, int8 quants in [-127, 127] for q8_0,
 * fp16 scale fields finite and small (their offsets: g4run.h:107-118) */
static void *rand_rows(int type, int64_t n, int rows) {
    const size_t rb = g4o_row_size(type, n), bs = g4o_type_size(type);
    uint8_t *w = malloc(rb * rows);
    for (size_t i = 0; i < rb * rows; i++) w[i] = (uint8_t)next64();
    int offs[2] = {-1, -1};
    float mul = 1e-4f;
    switch (type) {
    case G4O_Q8_0: offs[0] = 0; mul = 0.02f / 127; break;
    case G4O_Q4_0: offs[0] = 0; mul = 0.02f / 8; break;
    case G4O_Q2_K: offs[0] = 80; offs[1] = 82; break;
    case G4O_Q3_K: offs[0] = 108; break;
    case G4O_Q4_K: case G4O_Q5_K: offs[0] = 0; offs[1] = 2; break;
    case G4O_Q6_K: offs[0] = 208; mul = 1e-5f; break;
    case G4O_TQ2_0: offs[0] = 64; mul = 0.02f; break;
    }
    for (size_t b = 0; b < rb * rows / bs; b++) {
        uint8_t *blk = w + b * bs;
        if (type == G4O_Q8_0)
            for (int j = 0; j < 32; j++) blk[2 + j] = (uint8_t)(int8_t)((int)(next64() % 255) - 127);
        for (int k = 0; k < 2; k++)
            if (offs[k] >= 0) {
                const uint16_t h = g4o_fp32_to_fp16(fabsf(gauss()) * mul);
                memcpy(blk + offs[k], &h, 2);
            }
    }
    return w;
}

static float *rand_x(int64_t n) {
    float *x = malloc(n * sizeof(float));
    for (int64_t i = 0; i < n; i++) x[i] = gauss();
    return x;
}

static int close_enough(float got, float ref) {
    return fabs((double)got - (double)ref) <= 1e-5 + 1e-3 * fabs((double)ref);
}

static void check_tables(void) {
    g4_init_tables();
    for (uint32_t h = 0; h < 65536; h++) {
        const float r = g4o_fp16_to_fp32((uint16_t)h);
        CHECK(memcmp(&g4_fp16_to_fp32_table[h], &r, 4) == 0, "fp16 table code %u", h);
        CHECK(g4_gelu_fp16_table[h] == g4o_gelu_table_entry((uint16_t)h), "gelu table code %u", h);
    }
    CHECK(g4_row_size(2, 2560) == 1440 && g4_row_size(12, 11008) == 6192 && g4_row_size(2, 33) == 0, "g4_row_size");
    CHECK(g4_type_blck(8) == 32 && g4_type_size(14) == 210 && !strcmp(g4_type_name(12), "Q4_K"), "type table");
    printf("ok tables (65536 fp16 and GELU codes)\n");
}

static void check_quantizers(void) {
    const int64_t n = 11008;
    float *x = rand_x(n);
    for (int i = 0; i < 32; i++) x[64 + i] = 0.0f;          /* an all-zero block */
    x[5] = 63.5f;                                            /* one large value */
    uint8_t *a = malloc(g4o_row_size(G4O_Q8_K, n)), *b = malloc(g4o_row_size(G4O_Q8_K, n));
    g4_quantize_q8_0(x, (block_q8_0 *)a, n);
    g4o_quantize_q8_0(x, (g4o_q8_0 *)b, n);
    CHECK(!memcmp(a, b, g4o_row_size(G4O_Q8_0, n)), "g4_quantize_q8_0");
    g4_quantize_q8_K(x, (block_q8_K *)a, n);
    g4o_quantize_q8_K(x, (g4o_q8_K *)b, n);
    CHECK(!memcmp(a, b, g4o_row_size(G4O_Q8_K, n)), "g4_quantize_q8_K");
    g4_quantize_q4_0(x, (block_q4_0 *)a, n);
    g4o_quantize_q4_0(x, (g4o_q4_0 *)b, n);
    CHECK(!memcmp(a, b, g4o_row_size(G4O_Q4_0, n)), "g4_quantize_q4_0");
    free(x); free(a); free(b);
    printf("ok quantizers q8_0 q8_K q4_0 (n=%lld)\n", (long long)n);
}

static const int kFmts[] = {G4O_Q4_0, G4O_Q8_0, G4O_Q2_K, G4O_Q3_K, G4O_Q4_K, G4O_Q5_K, G4O_Q6_K, G4O_TQ2_0};
static const char *kNames[] = {"q4_0", "q8_0", "q2_K", "q3_K", "q4_K", "q5_K", "q6_K", "tq2_0"};

static float api_dot(int t, const void *w, const void *a, int64_t n) {
    switch (t) {
    case G4O_Q4_0: return g4_dot_q4_0_q8_0(w, a, n);
    case G4O_Q8_0: return g4_dot_q8_0_q8_0(w, a, n);
    case G4O_Q2_K: return g4_dot_q2_K_q8_K(w, a, n);
    case G4O_Q3_K: return g4_dot_q3_K_q8_K(w, a, n);
    case G4O_Q4_K: return g4_dot_q4_K_q8_K(w, a, n);
    case G4O_Q5_K: return g4_dot_q5_K_q8_K(w, a, n);
    case G4O_Q6_K: return g4_dot_q6_K_q8_K(w, a, n);
    default: return g4_dot_tq2_0_q8_K(w, a, n);
    }
}
static void api_dot4(int t, const void *w, const void *const a[4], int64_t n, float out[4]) {
    switch (t) {
    case G4O_Q4_0: g4_dot_q4_0_q8_0_x4(w, a, n, out); break;
    case G4O_Q8_0: g4_dot_q8_0_q8_0_x4(w, a, n, out); break;
    case G4O_Q2_K: g4_dot_q2_K_q8_K_x4(w, a, n, out); break;
    case G4O_Q3_K: g4_dot_q3_K_q8_K_x4(w, a, n, out); break;
    case G4O_Q4_K: g4_dot_q4_K_q8_K_x4(w, a, n, out); break;
    case G4O_Q5_K: g4_dot_q5_K_q8_K_x4(w, a, n, out); break;
    case G4O_Q6_K: g4_dot_q6_K_q8_K_x4(w, a, n, out); break;
    default: g4_dot_tq2_0_q8_K_x4(w, a, n, out); break;
    }
}

static void check_dequant_and_dots(void) {
    const int rows = 24;
    for (size_t f = 0; f < sizeof kFmts / sizeof kFmts[0]; f++) {
        const int t = kFmts[f];
        const int64_t n = (t == G4O_Q4_0 || t == G4O_Q8_0) ? 4096 : 2816;
        const size_t rb = g4o_row_size(t, n);
        uint8_t *w = rand_rows(t, n, rows);
        float *y0 = malloc(n * 4), *y1 = malloc(n * 4);
        g4_dequant_row(t, w, y0, n);
        g4o_dequant_row(t, w, y1, n);
        CHECK(!memcmp(y0, y1, n * 4), "g4_dequant_row %s", kNames[f]);
        /* 4 activations in the weight type's activation format */
        const int at = g4o_act_type(t);
        const size_t ab = g4o_row_size(at, n);
        uint8_t *acts[4];
        for (int k = 0; k < 4; k++) {
            float *x = rand_x(n);
            acts[k] = malloc(ab);
            if (at == G4O_Q8_0) g4_quantize_q8_0(x, (block_q8_0 *)acts[k], n);
            else g4_quantize_q8_K(x, (block_q8_K *)acts[k], n);
            free(x);
        }
        float worst = 0.0f;
        for (int r = 0; r < rows; r++) {
            const uint8_t *wr = w + r * rb;
            const void *aa[4] = {acts[0], acts[1], acts[2], acts[3]};
            float d4[4];
            api_dot4(t, wr, aa, n, d4);
            for (int k = 0; k < 4; k++) {
                const float d1 = api_dot(t, wr, acts[k], n), ref = g4o_dot(t, wr, acts[k], n);
                CHECK(memcmp(&d1, &d4[k], 4) == 0, "g4_dot_%s_x4 token %d differs from the 1-token dot", kNames[f], k);
                CHECK(close_enough(d1, ref), "g4_dot_%s row %d token %d: %.9g vs oracle %.9g", kNames[f], r, k, d1, ref);
                if (fabsf(d1 - ref) > worst) worst = fabsf(d1 - ref);
            }
        }
        /* a length that is not a whole number of blocks is truncated (quants.c:966) */
        const int b = g4o_type_blck(t);
        const float tr = api_dot(t, w, acts[0], n + b / 2), full = api_dot(t, w, acts[0], n);
        CHECK(memcmp(&tr, &full, 4) == 0, "g4_dot_%s does not truncate a partial block", kNames[f]);
        for (int k = 0; k < 4; k++) free(acts[k]);
        free(w); free(y0); free(y1);
        printf("ok %s: dequant bit-exact, %d rows x 4 tokens within 1e-3/1e-5 (worst %.3g), x4 == x1\n", kNames[f], rows,
               worst);
    }
}

static void check_float_dots(void) {
    const int64_t n = 2053;                    /* not a multiple of 8: the reference's scalar tail */
    uint16_t *w = malloc(n * 2), *a16 = malloc(n * 2), *wb = malloc(n * 2);
    float *a32 = malloc(n * 4), *y0 = malloc(n * 4), *y1 = malloc(n * 4);
    for (int64_t i = 0; i < n; i++) {
        w[i] = g4o_fp32_to_fp16(gauss() * 0.02f);
        wb[i] = g4o_fp32_to_bf16(gauss() * 0.02f);
        const float x = gauss();
        a16[i] = g4o_fp32_to_fp16(x);
        const uint16_t xb = g4o_fp32_to_bf16(x);
        const uint32_t u = (uint32_t)xb << 16;
        memcpy(&a32[i], &u, 4);
    }
    const float d16 = g4_dot_f16(w, a16, n), r16 = g4o_dot_f16(w, a16, n);
    CHECK(close_enough(d16, r16), "g4_dot_f16 %.9g vs %.9g", d16, r16);
    const float db = g4_dot_bf16(wb, a32, n), rbf = g4o_dot_bf16(wb, a32, n);
    CHECK(close_enough(db, rbf), "g4_dot_bf16 %.9g vs %.9g", db, rbf);
    g4_dequant_row(G4O_F16, w, y0, n);
    g4o_dequant_row(G4O_F16, w, y1, n);
    CHECK(!memcmp(y0, y1, n * 4), "g4_dequant_row f16");
    g4_dequant_row(G4O_BF16, wb, y0, n);
    g4o_dequant_row(G4O_BF16, wb, y1, n);
    CHECK(!memcmp(y0, y1, n * 4), "g4_dequant_row bf16");
    free(w); free(a16); free(wb); free(a32); free(y0); free(y1);
    printf("ok f16 / bf16 dots (n=%lld) and dequant\n", (long long)n);
}

static void check_matmul(void) {
    const struct { int type; int64_t ncols, nrows; } cases[] = {{G4O_Q4_0, 2560, 1024}, {G4O_Q4_K, 2816, 512},
                                                               {G4O_Q8_0, 4096, 256}};
    for (size_t c = 0; c < sizeof cases / sizeof cases[0]; c++) {
        const int t = cases[c].type;
        const int64_t nc = cases[c].ncols, nr = cases[c].nrows;
        g4_tensor tw;
        memset(&tw, 0, sizeof tw);
        snprintf(tw.name, sizeof tw.name, "blk.0.ffn_up.weight");
        tw.type = t;
        tw.ndim = 2;
        tw.ne[0] = nc;
        tw.ne[1] = nr;
        tw.ne[2] = tw.ne[3] = 1;
        tw.data = rand_rows(t, nc, (int)nr);
        g4gpu_weight W;
        CHECK(g4gpu_upload(&tw, &W) == 0, "g4gpu_upload type %d", t);
        for (int nb = 1; nb <= 3; nb += 2) {
            float *x = rand_x(nc * nb), *Y = malloc(nb * nr * 4), *R = malloc(nb * nr * 4);
            CHECK(g4gpu_matmul(&W, x, Y, nc, nr, nb) == 0, "g4gpu_matmul");
            const size_t st = g4o_act_stride(t, nc);
            void *qa = malloc(st * nb);
            g4o_prep_act(t, x, nc, nb, qa);
            g4o_matmul(t, tw.data, qa, st, R, nc, nr, nb, 1);
            for (int64_t i = 0; i < nb * nr; i++) CHECK(close_enough(Y[i], R[i]), "g4gpu_matmul type %d nb %d [%lld]", t, nb, (long long)i);
            free(x); free(Y); free(R); free(qa);
        }
        g4gpu_release(&W);
        free((void *)tw.data);
        printf("ok g4gpu_matmul type %d %lldx%lld (nb 1, 3)\n", t, (long long)nr, (long long)nc);
    }
}

static void check_sampler(void) {
    /* the reference's struct and calls against the oracle's restatement */
    const int nv = 32768;
    float *lg = malloc(nv * 4), *l1 = malloc(nv * 4), *l2 = malloc(nv * 4);
    for (int cfg = 0; cfg < 4; cfg++) {
        g4_sampler a;
        g4o_sampler b;
        g4_sampler_init(&a, nv);
        g4o_sampler_init(&b, nv);
        const float temps[4] = {0.8f, 0.0f, 1.3f, 1.0f};
        a.temp = b.temp = temps[cfg];
        a.top_k = b.top_k = cfg == 2 ? 600 : 40;
        a.repeat_penalty = b.repeat_penalty = 1.1f;
        a.freq_penalty = b.freq_penalty = cfg == 3 ? 0.2f : 0.0f;
        a.no_repeat_ngram = b.no_repeat_ngram = cfg == 1 ? 0 : 3;
        a.seed = b.seed = 1000 + (uint64_t)cfg;
        g4_sampler_ban(&a, 5);
        g4o_sampler_ban(&b, 5);
        for (int i = 0; i < 300; i++) {
            const int t = (int)(rand() % 40);
            g4_sampler_accept(&a, t);
            g4o_sampler_accept(&b, t);
        }
        for (int step = 0; step < 8; step++) {
            for (int i = 0; i < nv; i++) lg[i] = gauss() * 3.0f;
            if (cfg == 3)
                for (int i = 0; i < nv; i++) lg[i] = roundf(lg[i]);   /* ties: the exact heap replay */
            memcpy(l1, lg, nv * 4);
            memcpy(l2, lg, nv * 4);
            const int t1 = g4_sample(&a, l1), t2 = g4o_sample(&b, l2);
            CHECK(t1 == t2, "g4_sample cfg %d step %d: %d vs oracle %d", cfg, step, t1, t2);
            CHECK(!memcmp(l1, l2, nv * 4), "g4_sample cfg %d step %d: rewritten logits", cfg, step);
            CHECK(!memcmp(a.rng, b.rng, sizeof a.rng), "g4_sample cfg %d step %d: rng words", cfg, step);
            g4_sampler_accept(&a, t1);
            g4o_sampler_accept(&b, t2);
        }
        int same = a.recent_n == b.recent_n && a.recent_head == b.recent_head && !memcmp(a.cnt, b.cnt, sizeof(int) * (size_t)nv);
        for (int i = 0; same && i < a.recent_n; i++)      /* the filled part of the ring (malloc'd, not zeroed) */
            same = a.recent[(a.recent_head + i) % a.recent_cap] == b.recent[(b.recent_head + i) % b.recent_cap];
        CHECK(same, "g4_sampler bookkeeping cfg %d", cfg);
        g4_sampler_free(&a);
        g4o_sampler_free(&b);
    }
    free(lg); free(l1); free(l2);
    printf("ok g4_sampler_* / g4_sample (n_vocab %d, 4 settings, ties)\n", nv);
}

int main(void) {
    setvbuf(stdout, NULL, _IOLBF, 0);
    check_tables();
    CHECK(g4gpu_init(0) == 0, "g4gpu_init");
    check_quantizers();
    check_dequant_and_dots();
    check_float_dots();
    check_matmul();
    check_sampler();
    printf("PASS (%d failures)\n", failures);
    return 0;
}
