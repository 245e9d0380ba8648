// g4run_abi.cpp -- g4run.h's quantized-kernel entry points (include/g4run_abi.h)
// under their reference names, each one a GPU batch call of the C ABI in
// include/g4hip.h on host buffers: the call's inputs are staged to device
// memory of the calling thread, the gfx950 kernel runs on that thread's
// stream, and the result is copied back before the call returns.
#include "../../include/g4run_abi.h"

#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <mutex>
#include <vector>

#include "../../include/g4hip.h"
#include "host_fp16.h"
#include "kernels.h"

using namespace g4;

extern "C" int g4h_internal_fail(int status, const char *msg);

float g4_fp16_to_fp32_table[65536];
g4_fp16 g4_gelu_fp16_table[65536];
int g4_avx512 = 0;

extern "C" void g4_set_avx512(int on) { (void)on; }     // no AVX-512 kernels here: the dots run on the GPU
extern "C" int g4_avx512_available(void) { return 0; }

static std::once_flag g_tables_once;
static int g_init_status = G4H_ERR_DEVICE;

extern "C" void g4_init_tables(void) {
    std::call_once(g_tables_once, [] {
        for (uint32_t h = 0; h < 65536; h++) {
            g4_fp16_to_fp32_table[h] = host_h2f((uint16_t)h);
            g4_gelu_fp16_table[h] = gelu_table_entry((uint16_t)h);
        }
        const char *d = getenv("G4H_DEVICE");
        g_init_status = g4h_init(d ? atoi(d) : 0);
        if (g_init_status)
            fprintf(stderr, "g4run_abi: g4_init_tables: no usable device (%s); the g4_* kernels will return NaN\n",
                    g4h_last_error());
    });
}


// -------------------------------------------------------------- staging ----
// Per host thread: one stream and one growing device buffer, kept until the
// process ends (pool threads call the dots concurrently, as model.c's do).
namespace {
struct Staging {
    void *stream = nullptr;
    uint8_t *buf = nullptr;
    size_t cap = 0;
};
thread_local Staging tl;

size_t al256(size_t v) { return (v + 255) & ~(size_t)255; }

// device memory of at least `bytes` on this thread's stream, or null
uint8_t *stage(size_t bytes) {
    g4_init_tables();
    if (g_init_status) return nullptr;
    if (!tl.stream && g4h_stream_create(&tl.stream)) return nullptr;
    if (tl.cap < bytes) {
        if (tl.buf) {
            g4h_stream_synchronize(tl.stream);
            g4h_free(tl.buf);
            tl.buf = nullptr;
            tl.cap = 0;
        }
        const size_t want = bytes < ((size_t)1 << 20) ? ((size_t)1 << 20) : al256(bytes);
        void *p = nullptr;
        if (g4h_malloc(&p, want)) return nullptr;
        tl.buf = (uint8_t *)p;
        tl.cap = want;
    }
    return tl.buf;
}

void report(const char *fn) {
    static std::once_flag once;
    std::call_once(once, [fn] { fprintf(stderr, "g4run_abi: %s failed: %s\n", fn, g4h_last_error()); });
}

// activation bytes one dot reads for n elements of weight type wt
size_t act_bytes(int wt, int64_t n) {
    if (wt == G4H_F16) return (size_t)n * 2;
    if (wt == G4H_BF16) return (size_t)n * 4;
    return g4h_row_size(g4h_act_type(wt), n);
}

// nt dots of one weight row against nt activations; out[i] for a[i].  Float
// rows are padded with zeros to a multiple of 8 elements (the GPU row unit),
// which adds only +0 products.
bool dots(int wt, const void *w, const void *const *a, int nt, int64_t n, float *out) {
    const int b = g4_type_blck(wt);
    n -= n % b;                                          // whole blocks, as the reference's loops
    if (n <= 0) {
        for (int i = 0; i < nt; i++) out[i] = 0.0f;
        return true;
    }
    const bool fl = wt == G4H_F16 || wt == G4H_BF16;
    const int64_t np = fl ? (n + 7) / 8 * 8 : n;
    const size_t wb = fl ? (size_t)n * 2 : g4h_row_size(wt, n), wbp = fl ? (size_t)np * 2 : wb;
    const size_t ab = act_bytes(wt, n), abp = act_bytes(wt, np);
    const size_t o_w = 0, o_a = al256(wbp), o_o = o_a + (size_t)nt * al256(abp), total = o_o + 256;
    uint8_t *d = stage(total);
    if (!d) return false;
    void *s = tl.stream;
    if (fl && np != n) {
        if (g4h_memset(d + o_w, 0, wbp, s)) return false;
        for (int i = 0; i < nt; i++)
            if (g4h_memset(d + o_a + (size_t)i * al256(abp), 0, abp, s)) return false;
    }
    if (g4h_memcpy_h2d(d + o_w, w, wb, s)) return false;
    for (int i = 0; i < nt; i++)
        if (g4h_memcpy_h2d(d + o_a + (size_t)i * al256(abp), a[i], ab, s)) return false;
    for (int i = 0; i < nt; i++)
        if (g4h_vec_dot(wt, d + o_w, wbp, d + o_a + (size_t)i * al256(abp), np, 1, (float *)(d + o_o) + i, s)) return false;
    return g4h_memcpy_d2h(out, d + o_o, (size_t)nt * 4, s) == G4H_OK;
}

float dot1(int wt, const void *w, const void *a, int64_t n, const char *fn) {
    float r;
    const void *aa[1] = {a};
    if (!dots(wt, w, aa, 1, n, &r)) {
        report(fn);
        return NAN;
    }
    return r;
}

void dot4(int wt, const void *w, const void *const a[4], int64_t n, float out[4], const char *fn) {
    if (!dots(wt, w, a, 4, n, out)) {
        report(fn);
        for (int i = 0; i < 4; i++) out[i] = NAN;
    }
}

typedef int (*QuantFn)(const float *, size_t, void *, size_t, int64_t, int, void *);

void quantize(QuantFn q, int qt, const float *x, void *y, int64_t n, const char *fn) {
    n -= n % (qt == G4H_Q8_K ? 256 : 32);                // whole blocks (q8_K is not in the tensor type table)
    if (n <= 0) return;
    const size_t xb = (size_t)n * 4, yb = g4h_row_size(qt, n);
    uint8_t *d = stage(al256(xb) + yb);
    void *s = tl.stream;
    if (!d || g4h_memcpy_h2d(d, x, xb, s) || q((const float *)d, (size_t)n, d + al256(xb), yb, n, 1, s) ||
        g4h_memcpy_d2h(y, d + al256(xb), yb, s))
        report(fn);
}
}  // namespace

// ------------------------------------------------------------ quantizers ----
extern "C" void g4_quantize_q8_0(const float *x, block_q8_0 *y, int64_t n) {
    quantize(g4h_quantize_q8_0, G4H_Q8_0, x, y, n, "g4_quantize_q8_0");
}
extern "C" void g4_quantize_q8_K(const float *x, block_q8_K *y, int64_t n) {
    quantize(g4h_quantize_q8_K, G4H_Q8_K, x, y, n, "g4_quantize_q8_K");
}
extern "C" void g4_quantize_q4_0(const float *x, block_q4_0 *y, int64_t n) {
    quantize(g4h_quantize_q4_0, G4H_Q4_0, x, y, n, "g4_quantize_q4_0");
}

// --------------------------------------------------------------- dequant ----
extern "C" void g4_dequant_row(int type, const void *x, float *y, int64_t n) {
    const int b = g4_type_blck(type);
    if (b) n -= n % b;                                   // whole blocks, as the reference's loops
    const size_t xb = b ? g4_row_size(type, n) : 0;
    bool ok = b != 0 && type != 24 && type != 25 && type != 26 && type != 27 && type != 28;
    if (ok && n > 0) {
        uint8_t *d = stage(al256(xb) + (size_t)n * 4);
        void *s = tl.stream;
        ok = d && !g4h_memcpy_h2d(d, x, xb, s) &&
             !g4h_dequant_rows(type, d, xb, (float *)(d + al256(xb)), (size_t)n, n, 1, s) &&
             !g4h_memcpy_d2h(y, d + al256(xb), (size_t)n * 4, s);
    } else if (!ok) {
        char msg[96];
        snprintf(msg, sizeof msg, "g4_dequant_row: type %d unsupported", type);
        g4h_internal_fail(G4H_ERR_TYPE, msg);
    }
    if (!ok) {
        report("g4_dequant_row");
        for (int64_t i = 0; i < n; i++) y[i] = NAN;
    }
}

// ------------------------------------------------------------------ dots ----
#define G4_DOT(NAME, WT)                                                                       \
    extern "C" float g4_dot_##NAME(const void *w, const void *a, int64_t n) {                 \
        return dot1(WT, w, a, n, "g4_dot_" #NAME);                                             \
    }                                                                                          \
    extern "C" void g4_dot_##NAME##_x4(const void *w, const void *const a[4], int64_t n, float out[4]) { \
        dot4(WT, w, a, n, out, "g4_dot_" #NAME "_x4");                                         \
    }
G4_DOT(q4_0_q8_0, G4H_Q4_0)
G4_DOT(q8_0_q8_0, G4H_Q8_0)
G4_DOT(q6_K_q8_K, G4H_Q6_K)
G4_DOT(tq2_0_q8_K, G4H_TQ2_0)
G4_DOT(q2_K_q8_K, G4H_Q2_K)
G4_DOT(q3_K_q8_K, G4H_Q3_K)
G4_DOT(q4_K_q8_K, G4H_Q4_K)
G4_DOT(q5_K_q8_K, G4H_Q5_K)
#undef G4_DOT

extern "C" float g4_dot_f16(const void *w, const g4_fp16 *a, int64_t n) { return dot1(G4H_F16, w, a, n, "g4_dot_f16"); }
extern "C" float g4_dot_bf16(const void *w, const float *a, int64_t n) { return dot1(G4H_BF16, w, a, n, "g4_dot_bf16"); }

// --------------------------------------------------------------- sampler ----
// Host bookkeeping of sampler.c:5-48 on the reference's struct; the draw runs
// on the GPU.
extern "C" void g4_sampler_init(g4_sampler *s, int n_vocab) {
    std::memset(s, 0, sizeof *s);
    s->temp = 1.0f;
    s->top_k = 64;
    s->top_p = 0.95f;
    s->repeat_penalty = 1.0f;
    s->repeat_last_n = 128;
    s->n_vocab = n_vocab;
    s->recent_cap = SAMPLER_RING;
    s->recent = (int *)std::malloc((size_t)s->recent_cap * sizeof(int));
    s->cnt = (int *)std::calloc((size_t)(n_vocab > 0 ? n_vocab : 1), sizeof(int));
    s->seed = 0xdeadbeefull;
}

extern "C" void g4_sampler_reset(g4_sampler *s) {
    s->recent_n = 0;
    s->recent_head = 0;
    if (s->cnt) std::memset(s->cnt, 0, (size_t)s->n_vocab * sizeof(int));
}

extern "C" void g4_sampler_free(g4_sampler *s) {
    std::free(s->recent);
    std::free(s->cnt);
    std::free(s->ban_ids);
    std::memset(s, 0, sizeof *s);
}

extern "C" void g4_sampler_ban(g4_sampler *s, int id) {
    if (id < 0 || id >= s->n_vocab) return;
    for (int i = 0; i < s->n_ban; i++)
        if (s->ban_ids[i] == id) return;
    if (s->n_ban == s->ban_cap) {
        const int cap = s->ban_cap ? 2 * s->ban_cap : 16;
        int *p = (int *)std::realloc(s->ban_ids, (size_t)cap * sizeof(int));
        if (!p) return;
        s->ban_ids = p;
        s->ban_cap = cap;
    }
    s->ban_ids[s->n_ban++] = id;
}

extern "C" void g4_sampler_accept(g4_sampler *s, int id) {
    const int cap = s->recent_cap;
    if (s->recent_n == cap) {
        const int old = s->recent[s->recent_head];
        if (s->cnt[old] > 0) s->cnt[old]--;
        s->recent[s->recent_head] = id;
        s->recent_head = (s->recent_head + 1) % cap;
    } else {
        s->recent[(s->recent_head + s->recent_n) % cap] = id;
        s->recent_n++;
    }
    s->cnt[id]++;
}

// The device image (settings, RNG words, the ring from its oldest id, bans)
// and the logits go up in one staged buffer; the kernel draws without
// accepting (g4_sample does not accept); logits, id and RNG words come back.
extern "C" int g4_sample(g4_sampler *s, float *logits) {
    if (s->recent_cap != SAMPLER_RING || s->n_vocab <= 0 || s->recent_n > SAMPLER_RING) {
        g4h_internal_fail(G4H_ERR_ARG, "g4_sample: the ring must be g4_sampler_init's (4096 ids)");
        report("g4_sample");
        return -1;
    }
    const int nv = s->n_vocab;
    const size_t img = al256(sampler_dev_bytes(0) + (size_t)s->n_ban * sizeof(int));
    const size_t o_l = img, o_o = o_l + al256((size_t)nv * 4);
    uint8_t *d = stage(o_o + 256);
    if (!d) {
        report("g4_sample");
        return -1;
    }
    void *st = tl.stream;
    std::vector<uint8_t> h(img, 0);
    SamplerDev *S = reinterpret_cast<SamplerDev *>(h.data());
    S->temp = s->temp;
    S->top_k = s->top_k;
    S->top_p = s->top_p;
    S->repeat_penalty = s->repeat_penalty;
    S->repeat_last_n = s->repeat_last_n;
    S->freq_penalty = s->freq_penalty;
    S->presence_penalty = s->presence_penalty;
    S->no_repeat_ngram = s->no_repeat_ngram;
    S->seed = s->seed;
    for (int i = 0; i < 4; i++) S->rng[i] = s->rng[i];
    S->n_vocab = nv;
    S->recent_n = s->recent_n;
    S->recent_head = 0;
    S->n_ban = s->n_ban;
    for (int i = 0; i < s->recent_n; i++) S->recent[i] = s->recent[(s->recent_head + i) % s->recent_cap];
    if (s->n_ban) std::memcpy(sampler_bans(S), s->ban_ids, (size_t)s->n_ban * sizeof(int));
    SamplerDev *dS = reinterpret_cast<SamplerDev *>(d);
    int id = -1;
    const bool ok = !g4h_memcpy_h2d(d, h.data(), img, st) && !g4h_memcpy_h2d(d + o_l, logits, (size_t)nv * 4, st) &&
                    launch_sample(dS, nv, (float *)(d + o_l), (int *)(d + o_o), 0, nullptr, 0, (hipStream_t)st) ==
                        hipSuccess &&
                    !g4h_memcpy_d2h(logits, d + o_l, (size_t)nv * 4, st) && !g4h_memcpy_d2h(&id, d + o_o, sizeof id, st) &&
                    !g4h_memcpy_d2h(s->rng, dS->rng, sizeof s->rng, st);
    if (!ok) {
        report("g4_sample");
        return -1;
    }
    return id;
}
