/*
 * g4o_quants.c -- CPU oracle: fp16, quantizers, dequant, per-block integer
 * sums and the two dot orders (scalar _ref and shipped AVX2) of the
 * reference's src/quants.c.
 *
 * TEST INFRASTRUCTURE ONLY (see g4o.h).  Compiled with -ffp-contract=off so
 * that every fused multiply-add below is the explicit fmaf() the reference's
 * AVX2 code performs and nothing else is fused.
 */
#include "g4o.h"

#include <math.h>
#include <string.h>

/* ------------------------------------------------------------ type table -- */
/* gguf.c:11-25: elements per block / bytes per block. */
int g4o_type_blck(int t) {
    switch (t) {
    case G4O_F32: case G4O_F16: case G4O_BF16: return 1;
    case G4O_Q4_0: case G4O_Q8_0: return 32;
    case G4O_Q2_K: case G4O_Q3_K: case G4O_Q4_K: case G4O_Q5_K: case G4O_Q6_K: case G4O_Q8_K: case G4O_TQ2_0: return 256;
    default: return 0;
    }
}
size_t g4o_type_size(int t) {
    switch (t) {
    case G4O_F32: return 4;
    case G4O_F16: case G4O_BF16: return 2;
    case G4O_Q4_0: return sizeof(g4o_q4_0);
    case G4O_Q8_0: return sizeof(g4o_q8_0);
    case G4O_Q2_K: return sizeof(g4o_q2_K);
    case G4O_Q3_K: return sizeof(g4o_q3_K);
    case G4O_Q5_K: return sizeof(g4o_q5_K);
    case G4O_Q6_K: return sizeof(g4o_q6_K);
    case G4O_TQ2_0: return sizeof(g4o_tq2_0);
    case G4O_Q4_K: return sizeof(g4o_q4_K);
    case G4O_Q8_K: return sizeof(g4o_q8_K);
    default: return 0;
    }
}
/* gguf.c:42-46 */
size_t g4o_row_size(int t, int64_t n) {
    int b = g4o_type_blck(t);
    if (b == 0 || n % b) return 0;
    return (size_t)(n / b) * g4o_type_size(t);
}

/* ------------------------------------------------------------------ fp16 -- */
static inline uint32_t f2u(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
static inline float u2f(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }

/* Half -> single, exact for every code (quants.c:27-46): subnormal halves are
 * normalised by shifting the significand up until its hidden bit appears.
 * Looked up in a table built once at load (as g4_init_tables does). */
static float fp16_compute(uint16_t h);
static float fp16_tab[65536];
__attribute__((constructor)) static void fp16_tab_init(void) {
    for (uint32_t i = 0; i < 65536; i++) fp16_tab[i] = fp16_compute((uint16_t)i);
}
float g4o_fp16_to_fp32(uint16_t h) { return fp16_tab[h]; }
static float fp16_compute(uint16_t h) {
    uint32_t sign = (uint32_t)(h >> 15) << 31;
    uint32_t e = (h >> 10) & 31u, m = h & 1023u;
    if (e == 31) return u2f(sign | 0x7f800000u | (m << 13));
    if (e == 0) {
        if (m == 0) return u2f(sign);
        int shift = 0;
        while (!(m & 1024u)) { m <<= 1; shift++; }
        /* value = m * 2^-24 with m normalised: exponent 2^(-14 - shift) */
        return u2f(sign | ((uint32_t)(127 - 14 - shift) << 23) | ((m & 1023u) << 13));
    }
    return u2f(sign | ((e + 112u) << 23) | (m << 13));
}

/* Single -> half with round-to-nearest-even, gradual underflow, overflow to
 * infinity and quiet NaN (g4run.h:37-59). */
uint16_t g4o_fp32_to_fp16(float f) {
    uint32_t u = f2u(f);
    uint16_t sign = (uint16_t)((u >> 16) & 0x8000u);
    uint32_t mag = u & 0x7fffffffu;
    if (mag > 0x7f800000u) {                         /* NaN: keep payload top bits, force quiet */
        uint32_t p = (mag >> 13) & 1023u;
        return (uint16_t)(sign | 0x7e00u | (p ? p : 1u));
    }
    if (mag >= 0x47800000u) return (uint16_t)(sign | 0x7c00u);   /* >= 65536: inf */
    if (mag < 0x38800000u) {                         /* below 2^-14: half subnormal or zero */
        if (mag < 0x33000000u) return sign;          /* below 2^-25: rounds to zero */
        uint32_t e = mag >> 23;                      /* 102..112 */
        uint32_t sig = (mag & 0x7fffffu) | 0x800000u;
        uint32_t sh = 126u - e;                      /* 14..24: value = sig * 2^(e-150), unit 2^-24 */
        uint32_t q = sig >> sh, r = sig & ((1u << sh) - 1u), half = 1u << (sh - 1u);
        if (r > half || (r == half && (q & 1u))) q++;
        return (uint16_t)(sign | q);
    }
    /* normal range: rebias and round the 13 dropped bits to nearest even */
    uint32_t r = mag + 0x0fffu + ((mag >> 13) & 1u);
    return (uint16_t)(sign | ((r - 0x38000000u) >> 13));
}

void g4o_fp16_to_fp32_n(const uint16_t *h, float *f, int64_t n) { for (int64_t i = 0; i < n; i++) f[i] = g4o_fp16_to_fp32(h[i]); }
void g4o_fp32_to_fp16_n(const float *f, uint16_t *h, int64_t n) { for (int64_t i = 0; i < n; i++) h[i] = g4o_fp32_to_fp16(f[i]); }

/* quants.c:63-67: adding 1.5*2^23 puts the integer part in the low mantissa
 * bits under the current (nearest-even) rounding mode; valid for |f| < 2^22. */
int g4o_nearest_int(float f) {
    float v = f + 12582912.0f;
    return (int)(f2u(v) & 0x007fffffu) - 0x00400000;
}

/* ------------------------------------------------------------ quantizers -- */
/* AVX2 q8_0 quantizer semantics (quants.c:74-109): amax over the block,
 * d = amax/127 stored as fp16, id = 127/amax (0 for an all-zero block),
 * q = round-half-even(x*id) -- _mm256_round_ps(TO_NEAREST) then a saturating
 * pack, and |x*id| <= 127 so the saturation never fires.
 * The README build (-Ofast, i.e. -freciprocal-math) compiles the constant
 * division amax/127.f at quants.c:91 as amax * fp32(1/127); 127.f/amax stays a
 * true division.  This oracle follows the shipped build. */
void g4o_quantize_q8_0(const float *x, g4o_q8_0 *y, int64_t n) {
    for (int64_t b = 0; b < n / 32; b++, x += 32) {
        float amax = 0.0f;
        for (int j = 0; j < 32; j++) { float a = fabsf(x[j]); if (a > amax) amax = a; }
        y[b].d = g4o_fp32_to_fp16(amax * (1.0f / 127.0f));
        const float id = amax != 0.0f ? 127.0f / amax : 0.0f;
        for (int j = 0; j < 32; j++) {
            float v = rintf(x[j] * id);
            if (v > 127.0f) v = 127.0f;
            if (v < -128.0f) v = -128.0f;
            y[b].qs[j] = (int8_t)(int)v;
        }
    }
}

/* quants.c:146-175: the signed value of largest magnitude sets the scale
 * (iscale = -127/max), q clipped at +127, bsums over 16-element groups,
 * d = 1/iscale in fp32.  An all-zero block stores zeros.
 * Under the README's -Ofast the reciprocal of the quotient at quants.c:172 is
 * folded to max * fp32(-1/127), which differs from 1/iscale by one ulp in about
 * a quarter of the blocks, and the rounding add of nearest_int is fused with
 * the product; this oracle follows the shipped build. */
void g4o_quantize_q8_K(const float *x, g4o_q8_K *y, int64_t n) {
    for (int64_t b = 0; b < n / 256; b++, x += 256) {
        float amax = 0.0f, smax = 0.0f;
        for (int j = 0; j < 256; j++) {
            float a = fabsf(x[j]);
            if (a > amax) { amax = a; smax = x[j]; }
        }
        if (amax == 0.0f) { memset(&y[b], 0, sizeof(y[b])); continue; }
        const float iscale = -127.0f / smax;
        for (int j = 0; j < 256; j++) {
            /* -ffp-contract=fast fuses nearest_int's magic add with the product
             * (quants.c:164 through 63-67): fma(iscale, x, 1.5*2^23), i.e. the
             * exact product rounded half-even once. */
            float t = fmaf(iscale, x[j], 12582912.0f);
            int v = (int)(f2u(t) & 0x007fffffu) - 0x00400000;
            y[b].qs[j] = (int8_t)(v < 127 ? v : 127);
        }
        for (int g = 0; g < 16; g++) {
            int s = 0;
            for (int k = 0; k < 16; k++) s += y[b].qs[16 * g + k];
            y[b].bsums[g] = (int16_t)s;
        }
        y[b].d = smax * (-1.0f / 127.0f);
    }
}

/* quants.c:125-144: signed max sets d = max/-8; q = min(15, trunc(x*id + 8.5))
 * with id = 1/d; low nibble holds element j, high nibble element j+16.  The
 * README build fuses x*id + 8.5 into one fma (-ffp-contract=fast); followed. */
void g4o_quantize_q4_0(const float *x, g4o_q4_0 *y, int64_t n) {
    for (int64_t b = 0; b < n / 32; b++, x += 32) {
        float amax = 0.0f, smax = 0.0f;
        for (int j = 0; j < 32; j++) {
            if (amax < fabsf(x[j])) { amax = fabsf(x[j]); smax = x[j]; }
        }
        const float d = smax / -8.0f;
        const float id = d != 0.0f ? 1.0f / d : 0.0f;
        y[b].d = g4o_fp32_to_fp16(d);
        for (int j = 0; j < 16; j++) {
            uint8_t lo = (uint8_t)fmaf(x[j], id, 8.5f);
            uint8_t hi = (uint8_t)fmaf(x[j + 16], id, 8.5f);
            if (lo > 15) lo = 15;
            if (hi > 15) hi = 15;
            y[b].qs[j] = (uint8_t)(lo | (hi << 4));
        }
    }
}

/* ----------------------------------------------------- K-quant unpacking -- */
/* q4_K 6-bit (scale, min) pairs from 12 bytes, quants.c:417-423. */
static void q4k_scale_min(const uint8_t *s, int j, int *sc, int *mn) {
    if (j < 4) { *sc = s[j] & 63; *mn = s[j + 4] & 63; }
    else {
        *sc = (s[j + 4] & 15) | ((s[j - 4] >> 6) << 4);
        *mn = (s[j + 4] >> 4) | ((s[j] >> 6) << 4);
    }
}
/* q3_K: 16 signed 6-bit scales (stored biased by 32), quants.c:447-461 /
 * 692-697: low 4 bits from scales[0..7] (low nibbles for sub-blocks 0-7,
 * high nibbles for 8-15), high 2 bits from scales[8..11]. */
static void q3k_scales(const uint8_t *s, int out[16]) {
    for (int i = 0; i < 16; i++) {
        int lo = i < 8 ? (s[i] & 15) : (s[i - 8] >> 4);
        int hi = (s[8 + (i & 3)] >> (2 * (i >> 2))) & 3;
        out[i] = (lo | (hi << 4)) - 32;
    }
}
/* element e of a q2_K superblock: quant value 0..3 and its 16-group index
 * (quants.c:425-445): e = 128h + 32j + l, byte qs[32h + l], shift 2j. */
static inline int q2k_q(const g4o_q2_K *b, int e) {
    int h = e >> 7, j = (e >> 5) & 3, l = e & 31;
    return (b->qs[32 * h + l] >> (2 * j)) & 3;
}
/* element e of a q3_K superblock: signed value -4..3 (quants.c:447-477). */
static inline int q3k_q(const g4o_q3_K *b, int e) {
    int h = e >> 7, j = (e >> 5) & 3, l = e & 31;
    int lo = (b->qs[32 * h + l] >> (2 * j)) & 3;
    int hb = (b->hmask[l] >> (4 * h + j)) & 1;
    return lo - (hb ? 0 : 4);
}
/* element e of a q5_K superblock: 0..31 and sub-block e/32 (quants.c:497-515):
 * chunk c = e/32, nibble of qs[32(c/2) + l] (low for even c) + 16 * bit c of
 * qh[l]. */
static inline int q5k_q(const g4o_q5_K *b, int e) {
    int c = e >> 5, l = e & 31;
    uint8_t byte = b->qs[32 * (c >> 1) + l];
    return ((c & 1) ? (byte >> 4) : (byte & 15)) + (((b->qh[l] >> c) & 1) << 4);
}
/* element e of a q6_K superblock: signed value -32..31 (quants.c:379-400):
 * e = 128h + 32j + l, low nibble of ql[64h + 32(j&1) + l] (high nibble for
 * j >= 2), high 2 bits (qh[32h + l] >> 2j) & 3; its scale is scales[e/16]. */
static inline int q6k_q(const g4o_q6_K *b, int e) {
    int h = e >> 7, j = (e >> 5) & 3, l = e & 31;
    uint8_t byte = b->ql[64 * h + 32 * (j & 1) + l];
    int lo = j >= 2 ? (byte >> 4) : (byte & 15);
    int hi = (b->qh[32 * h + l] >> (2 * j)) & 3;
    return (lo | (hi << 4)) - 32;
}
/* element e of a tq2_0 superblock: trit - 1 (quants.c:402-411): e = 128h + 32j
 * + m is (qs[32h + m] >> 2j) & 3. */
static inline int tq2_q(const g4o_tq2_0 *b, int e) {
    int h = e >> 7, j = (e >> 5) & 3, m = e & 31;
    return ((b->qs[32 * h + m] >> (2 * j)) & 3) - 1;
}
/* element e of a q4_K superblock: 0..15 and sub-block e/32 (quants.c:479-495). */
static inline int q4k_q(const g4o_q4_K *b, int e) {
    int p = e >> 6, hi = (e >> 5) & 1, l = e & 31;
    uint8_t byte = b->qs[32 * p + l];
    return hi ? (byte >> 4) : (byte & 15);
}

/* ---------------------------------------------------------------- dequant -- */
int g4o_dequant_row(int type, const void *vx, float *y, int64_t n) {
    switch (type) {
    case G4O_F32: memcpy(y, vx, (size_t)n * 4); return 0;
    case G4O_F16: { const uint16_t *h = vx; for (int64_t i = 0; i < n; i++) y[i] = g4o_fp16_to_fp32(h[i]); return 0; }
    case G4O_BF16: {                                       /* quants.c:520: the high half of an fp32 */
        const uint16_t *h = vx;
        for (int64_t i = 0; i < n; i++) { uint32_t u = (uint32_t)h[i] << 16; memcpy(&y[i], &u, 4); }
        return 0;
    }
    case G4O_Q8_0: {                                       /* quants.c:373-378 */
        const g4o_q8_0 *x = vx;
        for (int64_t b = 0; b < n / 32; b++) {
            float d = g4o_fp16_to_fp32(x[b].d);
            for (int j = 0; j < 32; j++) y[32 * b + j] = x[b].qs[j] * d;
        }
        return 0;
    }
    case G4O_Q4_0: {                                       /* quants.c:364-372 */
        const g4o_q4_0 *x = vx;
        for (int64_t b = 0; b < n / 32; b++) {
            float d = g4o_fp16_to_fp32(x[b].d);
            for (int j = 0; j < 16; j++) {
                y[32 * b + j] = ((int)(x[b].qs[j] & 15) - 8) * d;
                y[32 * b + j + 16] = ((int)(x[b].qs[j] >> 4) - 8) * d;
            }
        }
        return 0;
    }
    case G4O_Q2_K: {                                       /* quants.c:425-445 */
        const g4o_q2_K *x = vx;
        for (int64_t b = 0; b < n / 256; b++) {
            float d = g4o_fp16_to_fp32(x[b].d), dm = g4o_fp16_to_fp32(x[b].dmin);
            for (int e = 0; e < 256; e++) {
                uint8_t sc = x[b].scales[e >> 4];
                float dl = d * (sc & 15), ml = dm * (sc >> 4);
                y[256 * b + e] = dl * q2k_q(&x[b], e) - ml;
            }
        }
        return 0;
    }
    case G4O_Q3_K: {                                       /* quants.c:447-477 */
        const g4o_q3_K *x = vx;
        for (int64_t b = 0; b < n / 256; b++) {
            float d = g4o_fp16_to_fp32(x[b].d);
            int sc[16]; q3k_scales(x[b].scales, sc);
            for (int e = 0; e < 256; e++) {
                float dl = d * sc[e >> 4];
                y[256 * b + e] = dl * q3k_q(&x[b], e);
            }
        }
        return 0;
    }
    case G4O_Q4_K: {                                       /* quants.c:479-495 */
        const g4o_q4_K *x = vx;
        for (int64_t b = 0; b < n / 256; b++) {
            float d = g4o_fp16_to_fp32(x[b].d), dm = g4o_fp16_to_fp32(x[b].dmin);
            for (int e = 0; e < 256; e++) {
                int sc, mn; q4k_scale_min(x[b].scales, e >> 5, &sc, &mn);
                y[256 * b + e] = d * sc * q4k_q(&x[b], e) - dm * mn;
            }
        }
        return 0;
    }
    case G4O_Q5_K: {                                       /* quants.c:497-515: (d*sc)*q - dmin*m */
        const g4o_q5_K *x = vx;
        for (int64_t b = 0; b < n / 256; b++) {
            float d = g4o_fp16_to_fp32(x[b].d), dm = g4o_fp16_to_fp32(x[b].dmin);
            for (int e = 0; e < 256; e++) {
                int sc, mn; q4k_scale_min(x[b].scales, e >> 5, &sc, &mn);
                y[256 * b + e] = d * sc * q5k_q(&x[b], e) - dm * mn;
            }
        }
        return 0;
    }
    case G4O_Q6_K: {                                       /* quants.c:379-400: (d*sc)*q */
        const g4o_q6_K *x = vx;
        for (int64_t b = 0; b < n / 256; b++) {
            float d = g4o_fp16_to_fp32(x[b].d);
            for (int e = 0; e < 256; e++) y[256 * b + e] = d * x[b].scales[e >> 4] * q6k_q(&x[b], e);
        }
        return 0;
    }
    case G4O_TQ2_0: {                                      /* quants.c:402-411: (q-1)*d */
        const g4o_tq2_0 *x = vx;
        for (int64_t b = 0; b < n / 256; b++) {
            float d = g4o_fp16_to_fp32(x[b].d);
            for (int e = 0; e < 256; e++) y[256 * b + e] = (float)tq2_q(&x[b], e) * d;
        }
        return 0;
    }
    default: return -1;
    }
}

/* ------------------------------------------------------- integer sums -- */
static int32_t sum_q8_0(const g4o_q8_0 *w, const g4o_q8_0 *a) {
    int32_t s = 0;
    for (int j = 0; j < 32; j++) s += w->qs[j] * a->qs[j];
    return s;
}
static int32_t sum_q4_0(const g4o_q4_0 *w, const g4o_q8_0 *a) {
    int32_t s = 0;
    for (int j = 0; j < 16; j++) {
        s += ((w->qs[j] & 15) - 8) * a->qs[j];
        s += ((w->qs[j] >> 4) - 8) * a->qs[j + 16];
    }
    return s;
}
/* q2_K: isum = sum_e (sc_e & 15) * q2_e * a_e ; msum = sum_g bsums_g * (sc_g >> 4)
 * (quants.c:633-650). */
static void sums_q2_K(const g4o_q2_K *w, const g4o_q8_K *a, int32_t *isum, int32_t *msum) {
    int32_t is = 0, ms = 0;
    for (int e = 0; e < 256; e++) is += (w->scales[e >> 4] & 15) * q2k_q(w, e) * a->qs[e];
    for (int g = 0; g < 16; g++) ms += a->bsums[g] * (w->scales[g] >> 4);
    *isum = is; *msum = ms;
}
static int32_t sum_q3_K(const g4o_q3_K *w, const g4o_q8_K *a) {
    int sc[16]; q3k_scales(w->scales, sc);
    int32_t s = 0;
    for (int e = 0; e < 256; e++) s += sc[e >> 4] * q3k_q(w, e) * a->qs[e];
    return s;
}
/* q4_K: isum = sum_e sc_{e/32} * q4_e * a_e ; msum = sum_g bsums_g * m_{g/2}
 * (quants.c:743-754). */
static void sums_q4_K(const g4o_q4_K *w, const g4o_q8_K *a, int32_t *isum, int32_t *msum) {
    int sc[8], mn[8];
    for (int j = 0; j < 8; j++) q4k_scale_min(w->scales, j, &sc[j], &mn[j]);
    int32_t is = 0, ms = 0;
    for (int e = 0; e < 256; e++) is += sc[e >> 5] * q4k_q(w, e) * a->qs[e];
    for (int g = 0; g < 16; g++) ms += a->bsums[g] * mn[g >> 1];
    *isum = is; *msum = ms;
}

/* q5_K: as q4_K with 5-bit quants (quants.c:797-813). */
static void sums_q5_K(const g4o_q5_K *w, const g4o_q8_K *a, int32_t *isum, int32_t *msum) {
    int sc[8], mn[8];
    for (int j = 0; j < 8; j++) q4k_scale_min(w->scales, j, &sc[j], &mn[j]);
    int32_t is = 0, ms = 0;
    for (int e = 0; e < 256; e++) is += sc[e >> 5] * q5k_q(w, e) * a->qs[e];
    for (int g = 0; g < 16; g++) ms += a->bsums[g] * mn[g >> 1];
    *isum = is; *msum = ms;
}
static int32_t sum_q6_K(const g4o_q6_K *w, const g4o_q8_K *a) {
    int32_t s = 0;
    for (int e = 0; e < 256; e++) s += w->scales[e >> 4] * q6k_q(w, e) * a->qs[e];
    return s;
}
static int32_t sum_tq2_0(const g4o_tq2_0 *w, const g4o_q8_K *a) {
    int32_t s = 0;
    for (int e = 0; e < 256; e++) s += tq2_q(w, e) * a->qs[e];
    return s;
}

void g4o_block_sums(int type, const void *w, const void *a, int64_t n, int32_t *out) {
    switch (type) {
    case G4O_Q8_0: for (int64_t b = 0; b < n / 32; b++) out[b] = sum_q8_0((const g4o_q8_0 *)w + b, (const g4o_q8_0 *)a + b); break;
    case G4O_Q4_0: for (int64_t b = 0; b < n / 32; b++) out[b] = sum_q4_0((const g4o_q4_0 *)w + b, (const g4o_q8_0 *)a + b); break;
    case G4O_Q2_K: for (int64_t b = 0; b < n / 256; b++) sums_q2_K((const g4o_q2_K *)w + b, (const g4o_q8_K *)a + b, &out[2 * b], &out[2 * b + 1]); break;
    case G4O_Q3_K: for (int64_t b = 0; b < n / 256; b++) out[b] = sum_q3_K((const g4o_q3_K *)w + b, (const g4o_q8_K *)a + b); break;
    case G4O_Q5_K: for (int64_t b = 0; b < n / 256; b++) sums_q5_K((const g4o_q5_K *)w + b, (const g4o_q8_K *)a + b, &out[2 * b], &out[2 * b + 1]); break;
    case G4O_Q6_K: for (int64_t b = 0; b < n / 256; b++) out[b] = sum_q6_K((const g4o_q6_K *)w + b, (const g4o_q8_K *)a + b); break;
    case G4O_TQ2_0: for (int64_t b = 0; b < n / 256; b++) out[b] = sum_tq2_0((const g4o_tq2_0 *)w + b, (const g4o_q8_K *)a + b); break;
    case G4O_Q4_K: for (int64_t b = 0; b < n / 256; b++) sums_q4_K((const g4o_q4_K *)w + b, (const g4o_q8_K *)a + b, &out[2 * b], &out[2 * b + 1]); break;
    default: break;
    }
}

/* ------------------------------------------------------ scalar ref dots -- */
/* Sequential fp32 accumulation in the order of quants.c:535-762. */
float g4o_dot_ref(int type, const void *vw, const void *va, int64_t n) {
    float acc = 0.0f;
    switch (type) {
    case G4O_F16: {                                       /* quants.c:1509-1513 (non-AVX2 build) */
        const uint16_t *w = vw, *a = va;
        for (int64_t i = 0; i < n; i++) acc += g4o_fp16_to_fp32(w[i]) * g4o_fp16_to_fp32(a[i]);
        return acc;
    }
    case G4O_BF16: {                                      /* quants.c:1514-1518 */
        const uint16_t *w = vw; const float *a = va;
        for (int64_t i = 0; i < n; i++) { uint32_t u = (uint32_t)w[i] << 16; float f; memcpy(&f, &u, 4); acc += f * a[i]; }
        return acc;
    }
    case G4O_Q8_0: {                                      /* quants.c:552-562 */
        const g4o_q8_0 *w = vw, *a = va;
        for (int64_t b = 0; b < n / 32; b++)
            acc += sum_q8_0(&w[b], &a[b]) * (g4o_fp16_to_fp32(w[b].d) * g4o_fp16_to_fp32(a[b].d));
        return acc;
    }
    case G4O_Q4_0: {                                      /* quants.c:535-550: (sumi*dw)*da */
        const g4o_q4_0 *w = vw; const g4o_q8_0 *a = va;
        for (int64_t b = 0; b < n / 32; b++)
            acc += (float)sum_q4_0(&w[b], &a[b]) * g4o_fp16_to_fp32(w[b].d) * g4o_fp16_to_fp32(a[b].d);
        return acc;
    }
    case G4O_TQ2_0: {                                     /* quants.c:564-580 */
        const g4o_tq2_0 *w = vw; const g4o_q8_K *a = va;
        for (int64_t b = 0; b < n / 256; b++) acc += (float)sum_tq2_0(&w[b], &a[b]) * (a[b].d * g4o_fp16_to_fp32(w[b].d));
        return acc;
    }
    case G4O_Q2_K: {                                      /* quants.c:624-655 */
        const g4o_q2_K *w = vw; const g4o_q8_K *a = va;
        for (int64_t b = 0; b < n / 256; b++) {
            int32_t is, ms; sums_q2_K(&w[b], &a[b], &is, &ms);
            float dall = a[b].d * g4o_fp16_to_fp32(w[b].d);
            float dmin = a[b].d * g4o_fp16_to_fp32(w[b].dmin);
            acc += dall * is - dmin * ms;
        }
        return acc;
    }
    case G4O_Q3_K: case G4O_Q4_K: case G4O_Q5_K: case G4O_Q6_K: {
        /* quants.c:657-711 / 713-762 / 582-622: 8 int32 lanes (element e -> lane e%8)
         * carry the scale-weighted sums of one superblock; each lane is scaled
         * into an 8-float accumulator; the lanes are summed at the end. */
        float sums[8] = {0};
        float mins_acc = 0.0f;
        for (int64_t b = 0; b < n / 256; b++) {
            int32_t lane[8] = {0};
            float d;
            if (type == G4O_Q3_K) {
                const g4o_q3_K *w = (const g4o_q3_K *)vw + b; const g4o_q8_K *a = (const g4o_q8_K *)va + b;
                int sc[16]; q3k_scales(w->scales, sc);
                for (int e = 0; e < 256; e++) lane[e & 7] += sc[e >> 4] * (q3k_q(w, e) * a->qs[e]);
                d = g4o_fp16_to_fp32(w->d) * a->d;
            } else if (type == G4O_Q6_K) {
                const g4o_q6_K *w = (const g4o_q6_K *)vw + b; const g4o_q8_K *a = (const g4o_q8_K *)va + b;
                for (int e = 0; e < 256; e++) lane[e & 7] += w->scales[e >> 4] * (q6k_q(w, e) * a->qs[e]);
                d = g4o_fp16_to_fp32(w->d) * a->d;
            } else if (type == G4O_Q5_K) {                    /* quants.c:764-818 */
                const g4o_q5_K *w = (const g4o_q5_K *)vw + b; const g4o_q8_K *a = (const g4o_q8_K *)va + b;
                int32_t is, ms; sums_q5_K(w, a, &is, &ms);
                int sc[8], mn[8];
                for (int j = 0; j < 8; j++) q4k_scale_min(w->scales, j, &sc[j], &mn[j]);
                for (int e = 0; e < 256; e++) lane[e & 7] += sc[e >> 5] * (q5k_q(w, e) * a->qs[e]);
                d = g4o_fp16_to_fp32(w->d) * a->d;
                float dmin = g4o_fp16_to_fp32(w->dmin) * a->d;
                mins_acc -= dmin * ms;
            } else {
                const g4o_q4_K *w = (const g4o_q4_K *)vw + b; const g4o_q8_K *a = (const g4o_q8_K *)va + b;
                int32_t is, ms; sums_q4_K(w, a, &is, &ms);
                int sc[8], mn[8];
                for (int j = 0; j < 8; j++) q4k_scale_min(w->scales, j, &sc[j], &mn[j]);
                for (int e = 0; e < 256; e++) lane[e & 7] += sc[e >> 5] * (q4k_q(w, e) * a->qs[e]);
                d = g4o_fp16_to_fp32(w->d) * a->d;
                float dmin = g4o_fp16_to_fp32(w->dmin) * a->d;
                mins_acc -= dmin * ms;
            }
            for (int l = 0; l < 8; l++) sums[l] += d * lane[l];
        }
        float s = mins_acc;
        for (int l = 0; l < 8; l++) s += sums[l];
        return s;
    }
    default: return NAN;
    }
}

/* ---------------------------------------------------- AVX2-order dots -- */
/* hsum_float_8 (quants.c:823-829): fold the upper 128-bit half onto the lower,
 * then lanes 2,3 onto 0,1, then lane 1 onto lane 0. */
static float hsum8(const float v[8]) {
    float r0 = v[4] + v[0], r1 = v[5] + v[1], r2 = v[6] + v[2], r3 = v[7] + v[3];
    float s0 = r0 + r2, s1 = r1 + r3;
    return s0 + s1;
}

/* q8_0 / q4_0 (quants.c:964-999): per block, 8 int32 lanes with lane i the
 * sum of elements 4i..4i+3, then acc_i = fma(dw*da, float(lane_i), acc_i). */
static float dot_q8_0_avx2(const g4o_q8_0 *w, const g4o_q8_0 *a, int64_t nb) {
    float acc[8] = {0};
    for (int64_t b = 0; b < nb; b++) {
        const float d = g4o_fp16_to_fp32(w[b].d) * g4o_fp16_to_fp32(a[b].d);
        for (int i = 0; i < 8; i++) {
            int32_t s = 0;
            for (int k = 4 * i; k < 4 * i + 4; k++) s += w[b].qs[k] * a[b].qs[k];
            acc[i] = fmaf(d, (float)s, acc[i]);
        }
    }
    return hsum8(acc);
}
static float dot_q4_0_avx2(const g4o_q4_0 *w, const g4o_q8_0 *a, int64_t nb) {
    float acc[8] = {0};
    for (int64_t b = 0; b < nb; b++) {
        const float d = g4o_fp16_to_fp32(w[b].d) * g4o_fp16_to_fp32(a[b].d);
        int8_t e[32];
        for (int j = 0; j < 16; j++) { e[j] = (int8_t)((w[b].qs[j] & 15) - 8); e[j + 16] = (int8_t)((w[b].qs[j] >> 4) - 8); }
        for (int i = 0; i < 8; i++) {
            int32_t s = 0;
            for (int k = 4 * i; k < 4 * i + 4; k++) s += e[k] * a[b].qs[k];
            acc[i] = fmaf(d, (float)s, acc[i]);
        }
    }
    return hsum8(acc);
}
/* q2_K (quants.c:1098-1145).  Per superblock: 8 int32 "mins" lanes
 * (lane i = bsums pair 2i,2i+1 times their min nibbles) FMA'd with
 * dmin = -da*dmin_w, then 8 int32 lanes of scale-weighted products (lane i
 * = bytes 4i..4i+3 of every 32-byte chunk) FMA'd with d = da*d_w. */
static float dot_q2_K_avx2(const g4o_q2_K *w, const g4o_q8_K *a, int64_t nb) {
    float acc[8] = {0};
    for (int64_t b = 0; b < nb; b++) {
        const float d = a[b].d * g4o_fp16_to_fp32(w[b].d);
        const float dmin = -a[b].d * g4o_fp16_to_fp32(w[b].dmin);
        for (int i = 0; i < 8; i++) {
            int32_t p = (w[b].scales[2 * i] >> 4) * a[b].bsums[2 * i] + (w[b].scales[2 * i + 1] >> 4) * a[b].bsums[2 * i + 1];
            acc[i] = fmaf(dmin, (float)p, acc[i]);
        }
        int32_t lane[8] = {0};
        for (int e = 0; e < 256; e++) {
            int byte_in_chunk = e & 31;
            lane[byte_in_chunk >> 2] += (w[b].scales[e >> 4] & 15) * q2k_q(&w[b], e) * a[b].qs[e];
        }
        for (int i = 0; i < 8; i++) acc[i] = fmaf(d, (float)lane[i], acc[i]);
    }
    return hsum8(acc);
}
/* q3_K (quants.c:1147-1211): same chunk/lane structure, one FMA per superblock. */
static float dot_q3_K_avx2(const g4o_q3_K *w, const g4o_q8_K *a, int64_t nb) {
    float acc[8] = {0};
    for (int64_t b = 0; b < nb; b++) {
        const float d = a[b].d * g4o_fp16_to_fp32(w[b].d);
        int sc[16]; q3k_scales(w[b].scales, sc);
        int32_t lane[8] = {0};
        for (int e = 0; e < 256; e++) lane[(e & 31) >> 2] += sc[e >> 4] * q3k_q(&w[b], e) * a[b].qs[e];
        for (int i = 0; i < 8; i++) acc[i] = fmaf(d, (float)lane[i], acc[i]);
    }
    return hsum8(acc);
}
/* q6_K (quants.c:1028-1094): lane i = bytes 4i..4i+3 of every 32-element
 * chunk, scale-weighted (q6-32)*q8 sums, one FMA per superblock. */
static float dot_q6_K_avx2(const g4o_q6_K *w, const g4o_q8_K *a, int64_t nb) {
    float acc[8] = {0};
    for (int64_t b = 0; b < nb; b++) {
        const float d = a[b].d * g4o_fp16_to_fp32(w[b].d);
        int32_t lane[8] = {0};
        for (int e = 0; e < 256; e++) lane[(e & 31) >> 2] += w[b].scales[e >> 4] * q6k_q(&w[b], e) * a[b].qs[e];
        for (int i = 0; i < 8; i++) acc[i] = fmaf(d, (float)lane[i], acc[i]);
    }
    return hsum8(acc);
}
/* tq2_0 (quants.c:1001-1026): the integer sum of a superblock is exact
 * (trits 0..2 against q8 minus the bsums), and it is scaled into one scalar
 * accumulator; the shipped build contracts the multiply-add into one fma. */
static float dot_tq2_0_avx2(const g4o_tq2_0 *w, const g4o_q8_K *a, int64_t nb) {
    float acc = 0.0f;
    for (int64_t b = 0; b < nb; b++) acc = fmaf((float)sum_tq2_0(&w[b], &a[b]), a[b].d * g4o_fp16_to_fp32(w[b].d), acc);
    return acc;
}
/* q5_K (quants.c:1261-1313): the mins sum of a superblock goes to one scalar
 * accumulator, the scale-weighted products to 8 lanes as in q4_K; the result
 * is hsum_float_8(acc) + summs.  The shipped -Ofast build evaluates
 * summs += (-d_a*dmin_w) * msum as fma(-dmin_w, d_a*msum, summs) (the
 * reassociation its fast-math flags allow); that is the form that reproduces
 * the reference build's outputs bit for bit. */
static float dot_q5_K_avx2(const g4o_q5_K *w, const g4o_q8_K *a, int64_t nb) {
    float acc[8] = {0}, summs = 0.0f;
    for (int64_t b = 0; b < nb; b++) {
        const float d = a[b].d * g4o_fp16_to_fp32(w[b].d);
        int sc[8], mn[8];
        for (int j = 0; j < 8; j++) q4k_scale_min(w[b].scales, j, &sc[j], &mn[j]);
        int32_t msum = 0;
        for (int k = 0; k < 8; k++) msum += mn[k] * (a[b].bsums[2 * k] + a[b].bsums[2 * k + 1]);
        summs = fmaf(-g4o_fp16_to_fp32(w[b].dmin), a[b].d * (float)msum, summs);
        int32_t lane[8] = {0};
        for (int e = 0; e < 256; e++) lane[(e & 31) >> 2] += sc[e >> 5] * q5k_q(&w[b], e) * a[b].qs[e];
        for (int i = 0; i < 8; i++) acc[i] = fmaf(d, (float)lane[i], acc[i]);
    }
    return hsum8(acc) + summs;
}
/* q4_K (quants.c:1213-1259): mins go to a separate 4-lane accumulator
 * (lane i = mins 2i,2i+1 times bsum pairs), folded 0+2,1+3 then added. */
static float dot_q4_K_avx2(const g4o_q4_K *w, const g4o_q8_K *a, int64_t nb) {
    float acc[8] = {0}, accm[4] = {0};
    for (int64_t b = 0; b < nb; b++) {
        const float d = a[b].d * g4o_fp16_to_fp32(w[b].d);
        const float dmin = -a[b].d * g4o_fp16_to_fp32(w[b].dmin);
        int sc[8], mn[8];
        for (int j = 0; j < 8; j++) q4k_scale_min(w[b].scales, j, &sc[j], &mn[j]);
        int32_t pair[8];
        for (int k = 0; k < 8; k++) pair[k] = a[b].bsums[2 * k] + a[b].bsums[2 * k + 1];
        for (int i = 0; i < 4; i++) {
            int32_t p = mn[2 * i] * pair[2 * i] + mn[2 * i + 1] * pair[2 * i + 1];
            accm[i] = fmaf(dmin, (float)p, accm[i]);
        }
        int32_t lane[8] = {0};
        for (int e = 0; e < 256; e++) lane[(e & 31) >> 2] += sc[e >> 5] * q4k_q(&w[b], e) * a[b].qs[e];
        for (int i = 0; i < 8; i++) acc[i] = fmaf(d, (float)lane[i], acc[i]);
    }
    float m0 = accm[0] + accm[2], m1 = accm[1] + accm[3];
    return hsum8(acc) + (m0 + m1);
}

float g4o_dot(int type, const void *w, const void *a, int64_t n) {
    switch (type) {
    case G4O_Q8_0: return dot_q8_0_avx2(w, a, n / 32);
    case G4O_Q4_0: return dot_q4_0_avx2(w, a, n / 32);
    case G4O_Q2_K: return dot_q2_K_avx2(w, a, n / 256);
    case G4O_Q3_K: return dot_q3_K_avx2(w, a, n / 256);
    case G4O_Q4_K: return dot_q4_K_avx2(w, a, n / 256);
    case G4O_Q5_K: return dot_q5_K_avx2(w, a, n / 256);
    case G4O_Q6_K: return dot_q6_K_avx2(w, a, n / 256);
    case G4O_TQ2_0: return dot_tq2_0_avx2(w, a, n / 256);
    case G4O_F16: return g4o_dot_f16(w, a, n);
    case G4O_BF16: return g4o_dot_bf16(w, a, n);
    default: return NAN;
    }
}

/* g4run.h:64-68: a NaN keeps its high half with the quiet bit set; otherwise
 * round to nearest even by adding 0x7fff plus the kept lsb, then truncating. */
uint16_t g4o_fp32_to_bf16(float f) {
    uint32_t x; memcpy(&x, &f, 4);
    if ((x & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((x >> 16) | 64u);
    return (uint16_t)((x + (0x7fffu + ((x >> 16) & 1u))) >> 16);
}
/* quants.c:1333-1347: as g4_dot_f16 with the weights widened by a 16-bit shift
 * and fp32 activations. */
float g4o_dot_bf16(const uint16_t *w, const float *a, int64_t n) {
    float acc[8] = {0};
    int64_t i = 0;
    for (; i + 8 <= n; i += 8)
        for (int l = 0; l < 8; l++) {
            uint32_t u = (uint32_t)w[i + l] << 16; float f; memcpy(&f, &u, 4);
            acc[l] = fmaf(f, a[i + l], acc[l]);
        }
    float s = hsum8(acc);
    for (; i < n; i++) { uint32_t u = (uint32_t)w[i] << 16; float f; memcpy(&f, &u, 4); s += f * a[i]; }
    return s;
}
/* quants.c:1319-1331: 8 fp32 lanes of fused products, tree sum, scalar tail. */
float g4o_dot_f16(const uint16_t *w, const uint16_t *a, int64_t n) {
    float acc[8] = {0};
    int64_t i = 0;
    for (; i + 8 <= n; i += 8)
        for (int l = 0; l < 8; l++) acc[l] = fmaf(g4o_fp16_to_fp32(w[i + l]), g4o_fp16_to_fp32(a[i + l]), acc[l]);
    float s = hsum8(acc);
    for (; i < n; i++) s += g4o_fp16_to_fp32(w[i]) * g4o_fp16_to_fp32(a[i]);
    return s;
}
