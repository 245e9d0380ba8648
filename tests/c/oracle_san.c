/* oracle_san.c -- drives the CPU oracle (oracle/*.c, test infrastructure)
 * through every function family for the sanitizer builds: AddressSanitizer +
 * UndefinedBehaviorSanitizer, and ThreadSanitizer for the pthread pool that
 * restates model.c's row-split thread pool.  Sizes are small; the point is
 * that no access leaves its buffer, no UB is reported and the pool has no
 * data race.  Prints "ok" and exits 0 when the sanitizers stay quiet. */
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "g4o.h"

static uint64_t s_rng = 88172645463325252ull;
static uint32_t rnd(void) {
    s_rng ^= s_rng << 13;
    s_rng ^= s_rng >> 7;
    s_rng ^= s_rng << 17;
    return (uint32_t)(s_rng >> 11);
}
static float gauss(void) {
    const float u1 = (rnd() + 1.0f) / 4294967296.0f, u2 = rnd() / 4294967296.0f;
    return sqrtf(-2.0f * logf(u1)) * cosf(6.2831853f * u2);
}

static void fill_blocks(uint8_t *p, size_t n) {
    for (size_t i = 0; i < n; i++) p[i] = (uint8_t)rnd();
}

/* keep fp16 scale fields finite: every 2-byte field at the listed offsets */
static void tame(int type, uint8_t *row, int64_t n) {
    const int bs = (int)g4o_type_size(type), nb = (int)(n / g4o_type_blck(type));
    for (int b = 0; b < nb; b++) {
        uint8_t *blk = row + (size_t)b * bs;
        int offs[2] = {-1, -1};
        switch (type) {
        case G4O_Q4_0: case G4O_Q8_0: offs[0] = 0; break;
        case G4O_Q2_K: offs[0] = 80; offs[1] = 82; break;
        case G4O_Q3_K: offs[0] = 108; break;
        case G4O_Q4_K: case G4O_Q5_K: offs[0] = 0; offs[1] = 2; break;
        case G4O_Q6_K: offs[0] = 208; break;
        case G4O_TQ2_0: offs[0] = 64; break;
        }
        for (int k = 0; k < 2; k++)
            if (offs[k] >= 0) {
                const uint16_t h = g4o_fp32_to_fp16(fabsf(gauss()) * 0.01f);
                memcpy(blk + offs[k], &h, 2);
            }
    }
}

int main(void) {
    const int64_t n = 512;
    const int types[] = {G4O_Q4_0, G4O_Q8_0, G4O_Q2_K, G4O_Q3_K, G4O_Q4_K, G4O_Q5_K, G4O_Q6_K, G4O_TQ2_0};
    float *x = malloc(n * 4 * 8), *y = malloc(n * 4);
    for (int64_t i = 0; i < n * 8; i++) x[i] = gauss();

    /* quantizers, dequant, block sums, both dot forms, x4 matmul through the pool */
    g4o_pool_start(4);
    for (size_t t = 0; t < sizeof types / sizeof types[0]; t++) {
        const int ty = types[t];
        const int rows = 37;
        const size_t rb = g4o_row_size(ty, n);
        uint8_t *w = malloc(rb * rows);
        fill_blocks(w, rb * rows);
        for (int r = 0; r < rows; r++) tame(ty, w + (size_t)r * rb, n);
        const size_t st = g4o_act_stride(ty, n);
        uint8_t *act = malloc(st * 4);
        g4o_prep_act(ty, x, n, 4, act);
        float *Y = malloc((size_t)rows * 4 * 4);
        g4o_matmul(ty, w, act, st, Y, n, rows, 4, 4);
        g4o_dequant_row(ty, w, y, n);
        int32_t sums[64];
        g4o_block_sums(ty, w, act, n, sums);
        volatile float d = g4o_dot(ty, w, act, n) + g4o_dot_ref(ty, w, act, n);
        (void)d;
        free(w); free(act); free(Y);
    }
    {   /* f16 / bf16 dots and conversions */
        uint16_t *w = malloc(n * 2), *a = malloc(n * 2);
        for (int64_t i = 0; i < n; i++) { w[i] = g4o_fp32_to_fp16(gauss()); a[i] = g4o_fp32_to_fp16(gauss()); }
        volatile float d = g4o_dot_f16(w, a, n) + g4o_dot_bf16(w, x, n);
        (void)d;
        free(w); free(a);
    }
    {   /* attention over a window of a ring, f16 and q8_0 caches, through the pool */
        const int H = 4, hd = 64, slots = 40, pos = 90;
        for (int kt = 0; kt < 2; kt++) {
            const int kv = kt ? G4O_Q8_0 : G4O_F16;
            const size_t rb = kv == G4O_F16 ? (size_t)hd * 2 : g4o_row_size(kv, hd);
            uint8_t *kc = malloc(rb * slots), *vc = malloc(rb * slots);
            for (int s = 0; s < slots; s++) {
                g4o_kv_store(kv, kc + s * rb, x + s % 8 * 64, hd);
                g4o_kv_store(kv, vc + s * rb, x + (s + 3) % 8 * 64, hd);
            }
            float out[4 * 64];
            g4o_attn_window(x, kc, vc, kv, H, 1, hd, pos, pos - 30, slots, out, 4);
            free(kc); free(vc);
        }
    }
    g4o_pool_stop();
    {   /* the sampling chain: bans, n-grams, penalties, heap top-k, top-p */
        g4o_sampler s;
        const int nv = 3000;
        g4o_sampler_init(&s, nv);
        s.no_repeat_ngram = 3;
        s.repeat_penalty = 1.2f;
        s.freq_penalty = 0.1f;
        s.top_k = 600;
        g4o_sampler_ban(&s, 7);
        float *lg = malloc(nv * 4);
        for (int step = 0; step < 5000; step++) {
            for (int i = 0; i < nv; i++) lg[i] = (step % 3) ? gauss() : roundf(gauss());
            g4o_sampler_accept(&s, g4o_sample(&s, lg));
        }
        free(lg);
        g4o_sampler_free(&s);
    }
    free(x); free(y);
    printf("ok\n");
    return 0;
}
