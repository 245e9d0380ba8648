// sampler.cpp -- host side of the device-resident sampler (include/g4hip.h,
// the GPU form of g4run.h:464-489 / sampler.c).  The settings, RNG words,
// ring of recent ids and ban list live in one device allocation laid out as
// g4::SamplerDev, followed by the ban list (n_vocab ints) and a staging area
// for the ids of g4h_sampler_accept.
#include "../../include/g4hip.h"

#include <cstring>
#include <vector>

#include "kernels.h"

using namespace g4;

extern "C" int g4h_internal_fail(int status, const char *msg);

namespace {
constexpr int kStage = 4096;      // ids per accept launch
}

struct g4h_sampler {
    int n_vocab = 0;
    SamplerDev *dev = nullptr;
    int *stage = nullptr;
    std::vector<int> bans;        // host copy, for the dedup of sampler.c:29
};

#define S_HIP(call)                                                                \
    do {                                                                           \
        hipError_t e_ = (call);                                                    \
        if (e_ != hipSuccess) return g4h_internal_fail(G4H_ERR_HIP, hipGetErrorString(e_)); \
    } while (0)

extern "C" void g4h_sampler_default_params(g4h_sampler_params *p) {
    if (!p) return;
    std::memset(p, 0, sizeof *p);
    p->temp = 1.0f;
    p->top_k = 64;
    p->top_p = 0.95f;
    p->repeat_penalty = 1.0f;
    p->repeat_last_n = 128;
    p->seed = 0xdeadbeefull;
}

static void put_params(SamplerDev &d, const g4h_sampler_params &p) {
    d.temp = p.temp;
    d.top_k = p.top_k;
    d.top_p = p.top_p;
    d.repeat_penalty = p.repeat_penalty;
    d.repeat_last_n = p.repeat_last_n;
    d.freq_penalty = p.freq_penalty;
    d.presence_penalty = p.presence_penalty;
    d.no_repeat_ngram = p.no_repeat_ngram;
    d.seed = p.seed;
}

extern "C" int g4h_sampler_create(int n_vocab, const g4h_sampler_params *p, g4h_sampler **out) {
    if (!out || n_vocab <= 0) return g4h_internal_fail(G4H_ERR_ARG, "g4h_sampler_create: bad argument");
    *out = nullptr;
    g4h_sampler_params def;
    g4h_sampler_default_params(&def);
    auto *s = new g4h_sampler();
    s->n_vocab = n_vocab;
    const size_t bytes = sampler_dev_bytes(n_vocab) + kStage * sizeof(int);
    if (int rc = g4h_malloc((void **)&s->dev, bytes)) {
        delete s;
        return rc;
    }
    s->stage = sampler_bans(s->dev) + n_vocab;
    SamplerDev img;
    std::memset(&img, 0, sizeof img);
    put_params(img, p ? *p : def);
    img.n_vocab = n_vocab;
    if (hipMemcpy(s->dev, &img, sizeof img, hipMemcpyHostToDevice) != hipSuccess) {
        g4h_free(s->dev);
        delete s;
        return g4h_internal_fail(G4H_ERR_HIP, "g4h_sampler_create: upload failed");
    }
    *out = s;
    return G4H_OK;
}

extern "C" int g4h_sampler_free(g4h_sampler *s) {
    if (!s) return G4H_OK;
    g4h_free(s->dev);
    delete s;
    return G4H_OK;
}

// Copies a host image of the settings block (temp .. seed, the leading fields
// of SamplerDev) to the device and waits, so `img` may go out of scope.
extern "C" int g4h_sampler_set_params(g4h_sampler *s, const g4h_sampler_params *p, void *stream) {
    if (!s || !p) return g4h_internal_fail(G4H_ERR_ARG, "g4h_sampler_set_params: null argument");
    SamplerDev img;
    put_params(img, *p);
    const hipStream_t st = (hipStream_t)stream;
    S_HIP(hipMemcpyAsync(s->dev, &img, offsetof(SamplerDev, rng), hipMemcpyHostToDevice, st));
    S_HIP(hipStreamSynchronize(st));
    return G4H_OK;
}

extern "C" int g4h_sampler_set_rng(g4h_sampler *s, const uint64_t rng[4], void *stream) {
    if (!s || !rng) return g4h_internal_fail(G4H_ERR_ARG, "g4h_sampler_set_rng: null argument");
    uint64_t w[4] = {rng[0], rng[1], rng[2], rng[3]};
    const hipStream_t st = (hipStream_t)stream;
    S_HIP(hipMemcpyAsync(s->dev->rng, w, sizeof w, hipMemcpyHostToDevice, st));
    S_HIP(hipStreamSynchronize(st));
    return G4H_OK;
}

extern "C" int g4h_sampler_reset(g4h_sampler *s, void *stream) {
    if (!s) return g4h_internal_fail(G4H_ERR_ARG, "g4h_sampler_reset: null sampler");
    const int z[2] = {0, 0};          // recent_n, recent_head
    const hipStream_t st = (hipStream_t)stream;
    S_HIP(hipMemcpyAsync(&s->dev->recent_n, z, sizeof z, hipMemcpyHostToDevice, st));
    S_HIP(hipStreamSynchronize(st));
    return G4H_OK;
}

extern "C" int g4h_sampler_ban(g4h_sampler *s, int id, void *stream) {
    if (!s) return g4h_internal_fail(G4H_ERR_ARG, "g4h_sampler_ban: null sampler");
    if (id < 0 || id >= s->n_vocab) return G4H_OK;
    for (int b : s->bans)
        if (b == id) return G4H_OK;
    const int slot = (int)s->bans.size(), n = slot + 1;
    const hipStream_t st = (hipStream_t)stream;
    S_HIP(hipMemcpyAsync(sampler_bans(s->dev) + slot, &id, sizeof id, hipMemcpyHostToDevice, st));
    S_HIP(hipMemcpyAsync(&s->dev->n_ban, &n, sizeof n, hipMemcpyHostToDevice, st));
    S_HIP(hipStreamSynchronize(st));
    s->bans.push_back(id);
    return G4H_OK;
}

extern "C" int g4h_sampler_accept(g4h_sampler *s, const int *ids, int n, void *stream) {
    if (!s || n < 0 || (n > 0 && !ids)) return g4h_internal_fail(G4H_ERR_ARG, "g4h_sampler_accept: bad argument");
    for (int i = 0; i < n; i++)
        if (ids[i] < 0 || ids[i] >= s->n_vocab) return g4h_internal_fail(G4H_ERR_ARG, "g4h_sampler_accept: id out of range");
    const hipStream_t st = (hipStream_t)stream;
    for (int i = 0; i < n; i += kStage) {
        const int c = n - i < kStage ? n - i : kStage;
        S_HIP(hipMemcpyAsync(s->stage, ids + i, (size_t)c * sizeof(int), hipMemcpyHostToDevice, st));
        S_HIP(launch_sampler_push(s->dev, s->stage, c, st));
        S_HIP(hipStreamSynchronize(st));
    }
    return G4H_OK;
}

extern "C" int g4h_sample(g4h_sampler *s, float *logits_dev, int *out_dev, int accept, void *stream) {
    if (!s || !logits_dev) return g4h_internal_fail(G4H_ERR_ARG, "g4h_sample: null argument");
    if ((uintptr_t)logits_dev % 16) return g4h_internal_fail(G4H_ERR_ARG, "g4h_sample: logits must be 16-byte aligned");
    S_HIP(launch_sample(s->dev, s->n_vocab, logits_dev, out_dev, accept, nullptr, 0, (hipStream_t)stream));
    return G4H_OK;
}

extern "C" int g4h_sampler_get_state(g4h_sampler *s, uint64_t rng[4], int *recent, int *recent_n, int *slow_draws,
                                     void *stream) {
    if (!s) return g4h_internal_fail(G4H_ERR_ARG, "g4h_sampler_get_state: null sampler");
    std::vector<uint8_t> buf(sizeof(SamplerDev));
    const hipStream_t st = (hipStream_t)stream;
    S_HIP(hipMemcpyAsync(buf.data(), s->dev, buf.size(), hipMemcpyDeviceToHost, st));
    S_HIP(hipStreamSynchronize(st));
    const SamplerDev *d = reinterpret_cast<const SamplerDev *>(buf.data());
    if (rng)
        for (int i = 0; i < 4; i++) rng[i] = d->rng[i];
    if (recent)
        for (int i = 0; i < d->recent_n; i++) recent[i] = d->recent[(d->recent_head + i) % SAMPLER_RING];
    if (recent_n) *recent_n = d->recent_n;
    if (slow_draws) *slow_draws = d->slow_draws;
    return G4H_OK;
}

// For the model's decode step (model.cpp).
int sampler_n_vocab(const g4h_sampler *s) { return s ? s->n_vocab : 0; }
SamplerDev *sampler_device(g4h_sampler *s) { return s ? s->dev : nullptr; }
