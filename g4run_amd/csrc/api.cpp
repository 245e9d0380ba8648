// api.cpp -- the C ABI declared in include/g4hip.h: validation, status codes,
// resident-tensor management and dispatch to the gfx950 kernels.
#include "../../include/g4hip.h"

#include <atomic>
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <mutex>
#include <unordered_map>

#include "kernels.h"

using namespace g4;

// ----------------------------------------------------------- errors ----
static thread_local char g_err[512] = "";

static int fail(int status, const char *fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_err, sizeof g_err, fmt, ap);
    va_end(ap);
    return status;
}
static int hip_fail(hipError_t e, const char *what) {
    return fail(G4H_ERR_HIP, "%s: %s", what, hipGetErrorString(e));
}
#define G4_HIP(call)                                          \
    do {                                                      \
        hipError_t e_ = (call);                               \
        if (e_ != hipSuccess) return hip_fail(e_, #call);     \
    } while (0)

static int g_device = -1;

// Fixed scratch of the allocation-free matmul (g4h_matmul_noalloc), 4 MiB: each
// device holds its own copy until the process ends.  Host code never uses the
// array's name as an address: g4h_init resolves it once per device with
// hipGetSymbolAddress, and calls pass that address to the kernels.
static constexpr size_t kNoAllocBytes = (size_t)4 << 20;
static __device__ __align__(256) uint8_t scratch[kNoAllocBytes];
static std::mutex g_noalloc_mu;
static std::unordered_map<int, void *> g_noalloc_ptr;     // device -> address of `scratch` there
static std::atomic<int> g_fail_alloc{0};

#define G4_NEED_INIT() \
    do { if (g_device < 0) return fail(G4H_ERR_DEVICE, "g4h_init() has not been called"); } while (0)

extern "C" const char *g4h_last_error(void) { return g_err; }
// status + message for the library's other host files (not part of the ABI)
extern "C" int g4h_internal_fail(int status, const char *msg) { return fail(status, "%s", msg); }
// After a synchronised call that ran one-launch attention on workspace ws: the
// error word a bounded hand-off wait sets when it gives up (the outputs are
// then NaN) is read, cleared and reported as G4H_ERR_TIMEOUT.  The workspace
// is then cleared before its next use: a workgroup that started after the
// launch's last one advanced the epoch took the next launch's tag, and its
// words must not be read as that launch's.
extern "C" int g4h_internal_attn_error(void *ws, void *stream, const char *fn) {
    const hipStream_t s = (hipStream_t)stream;
    unsigned err = 0;
    G4_HIP(hipMemcpyAsync(&err, (uint8_t *)ws + ATTN_ERR_OFFSET, sizeof err, hipMemcpyDeviceToHost, s));
    G4_HIP(hipStreamSynchronize(s));
    if (!err) return G4H_OK;
    G4_HIP(hipMemsetAsync((uint8_t *)ws + ATTN_ERR_OFFSET, 0, sizeof err, s));
    G4_HIP(hipStreamSynchronize(s));
    attn_ws_forget(ws);
    return fail(G4H_ERR_TIMEOUT, "%s: an attention hand-off wait gave up; the outputs are NaN", fn);
}

extern "C" const char *g4h_status_str(int s) {
    switch (s) {
    case G4H_OK: return "ok";
    case G4H_ERR_ARG: return "invalid argument";
    case G4H_ERR_TYPE: return "unsupported type";
    case G4H_ERR_SHAPE: return "invalid shape";
    case G4H_ERR_NOMEM: return "out of device memory";
    case G4H_ERR_DEVICE: return "no usable device";
    case G4H_ERR_HIP: return "HIP runtime error";
    case G4H_ERR_TIMEOUT: return "device-side wait gave up";
    default: return "unknown status";
    }
}

extern "C" void g4h_debug_fail_alloc(int n) { g_fail_alloc.store(n < 0 ? 0 : n); }
extern "C" void g4h_debug_attn_timeout(int on) { attn_force_timeout(on != 0); }

extern "C" int g4h_init(int device) {
    int n = 0;
    hipError_t e = hipGetDeviceCount(&n);
    if (e != hipSuccess || n == 0) return fail(G4H_ERR_DEVICE, "no HIP device (%s)", hipGetErrorString(e));
    if (device < 0 || device >= n) return fail(G4H_ERR_DEVICE, "device %d out of range (%d devices)", device, n);
    G4_HIP(hipSetDevice(device));
    hipDeviceProp_t p;
    G4_HIP(hipGetDeviceProperties(&p, device));
    if (strncmp(p.gcnArchName, "gfx950", 6) != 0)
        return fail(G4H_ERR_DEVICE, "device %d is %s; this library is built for gfx950 only", device, p.gcnArchName);
    // the allocation-free matmul's scratch: its address on this device, once
    {
        std::lock_guard<std::mutex> lk(g_noalloc_mu);
        if (!g_noalloc_ptr.count(device)) {
            void *ptr = nullptr;
            G4_HIP(hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch)));
            g_noalloc_ptr[device] = ptr;
        }
    }
    g_device = device;
    return G4H_OK;
}

// ------------------------------------------------------------ plumbing ----
static int dev_alloc(void **p, size_t bytes) {
    if (g_fail_alloc.load() > 0) {
        g_fail_alloc.fetch_sub(1);
        *p = nullptr;
        return fail(G4H_ERR_NOMEM, "device allocation of %zu bytes failed (injected)", bytes);
    }
    hipError_t e = hipMalloc(p, bytes ? bytes : 1);
    if (e != hipSuccess) {
        (void)hipGetLastError();
        *p = nullptr;
        return fail(G4H_ERR_NOMEM, "device allocation of %zu bytes failed: %s", bytes, hipGetErrorString(e));
    }
    return G4H_OK;
}

extern "C" int g4h_malloc(void **ptr, size_t bytes) {
    G4_NEED_INIT();
    if (!ptr) return fail(G4H_ERR_ARG, "g4h_malloc: null out pointer");
    return dev_alloc(ptr, bytes);
}
extern "C" int g4h_free(void *ptr) {
    if (!ptr) return G4H_OK;
    g4::attn_ws_forget(ptr);                                     // a later allocation there starts uncleared
    G4_HIP(hipFree(ptr));
    return G4H_OK;
}
extern "C" int g4h_memcpy_h2d(void *d, const void *s, size_t n, void *st) {
    G4_HIP(hipMemcpyAsync(d, s, n, hipMemcpyHostToDevice, (hipStream_t)st));
    return G4H_OK;
}
extern "C" int g4h_memcpy_d2h(void *d, const void *s, size_t n, void *st) {
    G4_HIP(hipMemcpyAsync(d, s, n, hipMemcpyDeviceToHost, (hipStream_t)st));
    G4_HIP(hipStreamSynchronize((hipStream_t)st));
    return G4H_OK;
}
extern "C" int g4h_memcpy_d2d(void *d, const void *s, size_t n, void *st) {
    G4_HIP(hipMemcpyAsync(d, s, n, hipMemcpyDeviceToDevice, (hipStream_t)st));
    return G4H_OK;
}
extern "C" int g4h_memset(void *d, int v, size_t n, void *st) {
    G4_HIP(hipMemsetAsync(d, v, n, (hipStream_t)st));
    return G4H_OK;
}
extern "C" int g4h_stream_create(void **s) {
    G4_NEED_INIT();
    G4_HIP(hipStreamCreateWithFlags((hipStream_t *)s, hipStreamNonBlocking));
    return G4H_OK;
}
extern "C" int g4h_stream_destroy(void *s) { G4_HIP(hipStreamDestroy((hipStream_t)s)); return G4H_OK; }
extern "C" int g4h_stream_synchronize(void *s) { G4_HIP(hipStreamSynchronize((hipStream_t)s)); return G4H_OK; }
extern "C" int g4h_event_create(void **e) { G4_HIP(hipEventCreate((hipEvent_t *)e)); return G4H_OK; }
extern "C" int g4h_event_destroy(void *e) { G4_HIP(hipEventDestroy((hipEvent_t)e)); return G4H_OK; }
extern "C" int g4h_event_record(void *e, void *s) { G4_HIP(hipEventRecord((hipEvent_t)e, (hipStream_t)s)); return G4H_OK; }
extern "C" int g4h_event_elapsed_ms(float *ms, void *a, void *b) {
    G4_HIP(hipEventSynchronize((hipEvent_t)b));
    G4_HIP(hipEventElapsedTime(ms, (hipEvent_t)a, (hipEvent_t)b));
    return G4H_OK;
}
extern "C" int g4h_graph_begin(void *s) {
    G4_HIP(hipStreamBeginCapture((hipStream_t)s, hipStreamCaptureModeThreadLocal));
    return G4H_OK;
}
extern "C" int g4h_graph_end(void *s, void **exec) {
    hipGraph_t g;
    G4_HIP(hipStreamEndCapture((hipStream_t)s, &g));
    hipError_t e = hipGraphInstantiate((hipGraphExec_t *)exec, g, nullptr, nullptr, 0);
    (void)hipGraphDestroy(g);
    if (e != hipSuccess) return hip_fail(e, "hipGraphInstantiate");
    return G4H_OK;
}
extern "C" int g4h_graph_launch(void *exec, void *s) { G4_HIP(hipGraphLaunch((hipGraphExec_t)exec, (hipStream_t)s)); return G4H_OK; }
extern "C" int g4h_graph_destroy(void *exec) { G4_HIP(hipGraphExecDestroy((hipGraphExec_t)exec)); return G4H_OK; }

// ------------------------------------------------------------- sizes ----
static bool supported(int t) {
    return t == Q4_0 || t == Q8_0 || t == Q2_K || t == Q3_K || t == Q4_K || t == Q5_K || t == Q6_K || t == TQ2_0;
}
// f16 / bf16 weights (matmul_b's G4_F16 / G4_BF16 rows, model.c:238-239)
static bool is_float(int t) { return t == F16 || t == BF16; }

extern "C" size_t g4h_row_size(int type, int64_t n) {
    const int b = blck(type);
    if (b == 0 || n <= 0 || n % b) return 0;
    return (size_t)(n / b) * bsize(type);
}
extern "C" int g4h_act_type(int wtype) {
    switch (wtype) {
    case Q4_0: case Q8_0: return Q8_0;
    case Q2_K: case Q3_K: case Q4_K: case Q5_K: case Q6_K: case TQ2_0: return Q8_K;
    case F16: return F16;                                   // AC_F16 (model.c:163-170)
    case BF16: return F32;                                  // AC_BF16: bf16-rounded fp32 (model.c:172-180)
    default: return -1;
    }
}
extern "C" size_t g4h_act_stride(int wtype, int64_t ncols) {
    const int at = g4h_act_type(wtype);
    if (at < 0) return 0;
    const size_t r = g4h_row_size(at, ncols);
    return (r + 63) & ~(size_t)63;
}

// Per-stream scratch for activations quantized inside g4h_matmul.  Growth
// synchronizes that stream first; calls on one stream are ordered, calls on
// different streams use different buffers.
static std::mutex g_scratch_mu;
static std::unordered_map<hipStream_t, std::pair<void *, size_t>> g_scratch;

static int scratch_for(hipStream_t s, size_t bytes, void **out) {
    std::lock_guard<std::mutex> lk(g_scratch_mu);
    auto &e = g_scratch[s];
    if (e.second < bytes) {
        if (e.first) {
            G4_HIP(hipStreamSynchronize(s));
            G4_HIP(hipFree(e.first));
            e.first = nullptr;
            e.second = 0;
        }
        const size_t want = bytes < (1u << 20) ? (1u << 20) : bytes;
        int rc = dev_alloc(&e.first, want);
        if (rc) return rc;
        e.second = want;
    }
    *out = e.first;
    return G4H_OK;
}

// --------------------------------------------------------- quantizers ----
static int check_q(const char *fn, int qt, const float *x, size_t xs, void *y, size_t ys, int64_t n, int rows) {
    G4_NEED_INIT();
    if (!x || !y) return fail(G4H_ERR_ARG, "%s: null pointer", fn);
    if (rows < 0 || n <= 0) return fail(G4H_ERR_ARG, "%s: bad size n=%lld rows=%d", fn, (long long)n, rows);
    if (n % blck(qt)) return fail(G4H_ERR_SHAPE, "%s: n=%lld is not a multiple of %d", fn, (long long)n, blck(qt));
    if (rows > 1 && (xs < (size_t)n || ys < g4h_row_size(qt, n)))
        return fail(G4H_ERR_ARG, "%s: row strides smaller than a row", fn);
    if ((uintptr_t)x % 4) return fail(G4H_ERR_ARG, "%s: x must be 4-byte aligned", fn);
    const size_t ya = qt == Q8_K ? 4 : 2;
    if ((uintptr_t)y % ya || ys % ya) return fail(G4H_ERR_ARG, "%s: y and y_stride must be %zu-byte aligned", fn, ya);
    return G4H_OK;
}

extern "C" int g4h_quantize_q8_0(const float *x, size_t xs, void *y, size_t ys, int64_t n, int rows, void *s) {
    if (int rc = check_q("g4h_quantize_q8_0", Q8_0, x, xs, y, ys, n, rows)) return rc;
    if (rows == 0) return G4H_OK;
    G4_HIP(launch_quantize_q8_0(x, xs, (uint8_t *)y, ys, n, rows, (hipStream_t)s));
    return G4H_OK;
}
extern "C" int g4h_quantize_q8_K(const float *x, size_t xs, void *y, size_t ys, int64_t n, int rows, void *s) {
    if (int rc = check_q("g4h_quantize_q8_K", Q8_K, x, xs, y, ys, n, rows)) return rc;
    if (rows == 0) return G4H_OK;
    G4_HIP(launch_quantize_q8_K(x, xs, (uint8_t *)y, ys, n, rows, (hipStream_t)s));
    return G4H_OK;
}
extern "C" int g4h_quantize_q4_0(const float *x, size_t xs, void *y, size_t ys, int64_t n, int rows, void *s) {
    if (int rc = check_q("g4h_quantize_q4_0", Q4_0, x, xs, y, ys, n, rows)) return rc;
    if (rows == 0) return G4H_OK;
    G4_HIP(launch_quantize_q4_0(x, xs, (uint8_t *)y, ys, n, rows, (hipStream_t)s));
    return G4H_OK;
}

extern "C" int g4h_dequant_rows(int type, const void *x, size_t xs, float *y, size_t ys, int64_t n, int rows, void *s) {
    G4_NEED_INIT();
    if (!x || !y || n <= 0 || rows < 0) return fail(G4H_ERR_ARG, "g4h_dequant_rows: bad argument");
    if (!supported(type) && !is_float(type) && type != F32) return fail(G4H_ERR_TYPE, "g4h_dequant_rows: type %d unsupported", type);
    if (n % blck(type)) return fail(G4H_ERR_SHAPE, "g4h_dequant_rows: n=%lld not a multiple of %d", (long long)n, blck(type));
    if (rows == 0) return G4H_OK;
    G4_HIP(launch_dequant(type, (const uint8_t *)x, xs, y, ys, n, rows, (hipStream_t)s));
    return G4H_OK;
}

extern "C" int g4h_vec_dot(int wtype, const void *w, size_t ws, const void *a, int64_t n, int rows, float *out, void *s) {
    G4_NEED_INIT();
    if (!w || !a || !out || n <= 0 || rows < 0) return fail(G4H_ERR_ARG, "g4h_vec_dot: bad argument");
    if (is_float(wtype)) {
        // g4_dot_f16 / g4_dot_bf16: f16 or fp32 activation, aligned rows
        if (n % 8 || (uintptr_t)w % 16 || (uintptr_t)a % 16 || (rows > 1 && ws % 16))
            return fail(G4H_ERR_ARG, "g4h_vec_dot: f16/bf16 rows need n %% 8 == 0 and 16-byte aligned rows and activation");
        if (rows > 1 && ws < g4h_row_size(wtype, n)) return fail(G4H_ERR_ARG, "g4h_vec_dot: row stride smaller than a row");
        if (rows == 0) return G4H_OK;
        G4_HIP(launch_gemv_float(wtype, (const uint8_t *)w, rows > 1 ? ws : 16 * ((g4h_row_size(wtype, n) + 15) / 16), rows, n,
                                 (const uint8_t *)a, 0, out, 0, 1, (hipStream_t)s));
        return G4H_OK;
    }
    if (!supported(wtype)) return fail(G4H_ERR_TYPE, "g4h_vec_dot: weight type %d unsupported", wtype);
    if (n % blck(wtype)) return fail(G4H_ERR_SHAPE, "g4h_vec_dot: n=%lld not a multiple of %d", (long long)n, blck(wtype));
    if ((uintptr_t)a % 4) return fail(G4H_ERR_ARG, "g4h_vec_dot: activation must be 4-byte aligned");
    if (rows > 1 && ws < g4h_row_size(wtype, n)) return fail(G4H_ERR_ARG, "g4h_vec_dot: row stride smaller than a row");
    if (gemv_lds_bytes(wtype, 1, n / blck(wtype)) > 65536) return fail(G4H_ERR_SHAPE, "g4h_vec_dot: row too long");
    if (rows == 0) return G4H_OK;
    G4_HIP(launch_vec_dot_raw(wtype, (const uint8_t *)w, ws, (const uint8_t *)a, n, rows, out, (hipStream_t)s));
    return G4H_OK;
}

// ------------------------------------------------------------ tensors ----
static size_t al256(size_t v) { return (v + 255) & ~(size_t)255; }

extern "C" int g4h_tensor_create(int type, int64_t ncols, int64_t nrows, g4h_tensor **out) {
    G4_NEED_INIT();
    if (!out) return fail(G4H_ERR_ARG, "g4h_tensor_create: null out");
    *out = nullptr;
    if (!supported(type) && !is_float(type)) return fail(G4H_ERR_TYPE, "g4h_tensor_create: type %d unsupported", type);
    if (is_float(type) && ncols % 8) return fail(G4H_ERR_SHAPE, "g4h_tensor_create: f16/bf16 rows need ncols %% 8 == 0");
    if (ncols <= 0 || nrows <= 0) return fail(G4H_ERR_ARG, "g4h_tensor_create: empty shape");
    if (ncols % blck(type)) return fail(G4H_ERR_SHAPE, "g4h_tensor_create: ncols=%lld not a multiple of %d", (long long)ncols, blck(type));
    const int64_t nb = ncols / blck(type);
    if (!is_float(type) && gemv_lds_bytes(type, 1, nb) > 65536)
        return fail(G4H_ERR_SHAPE, "g4h_tensor_create: ncols=%lld exceeds the supported row length", (long long)ncols);
    const size_t n = (size_t)(nrows * nb);
    size_t qs = 0, sc = 0, ex = 0, dd = 0;
    switch (type) {
    case Q8_0: qs = al256(n * 16) + n * 16; sc = n * 2; break;   // lo | hi halves (common.h)
    case Q4_0: qs = n * 16; sc = n * 2; break;
    case Q4_K: qs = n * 144; break;
    case Q5_K: qs = n * 176; break;
    case Q2_K: qs = n * 64; sc = n * 16; ex = n * 4; break;
    case Q3_K: qs = n * 64; ex = n * 32; sc = n * 12; dd = n * 2; break;
    case Q6_K: qs = n * 128; ex = n * 64; sc = n * 16; dd = n * 2; break;
    case TQ2_0: qs = n * 64; sc = n * 2; break;
    case F16: case BF16: qs = n * 2; break;
    }
    const size_t total = al256(qs) + al256(sc) + al256(ex) + al256(dd);
    g4h_tensor *t = new g4h_tensor();
    t->type = type; t->ncols = ncols; t->nrows = nrows; t->nb = nb;
    void *base = nullptr;
    if (int rc = dev_alloc(&base, total)) { delete t; return rc; }
    t->base = (uint8_t *)base;
    t->bytes = total;
    t->qs = t->base;
    t->sc = t->qs + al256(qs);
    t->ex = t->sc + al256(sc);
    t->dd = t->ex + al256(ex);
    if (type == Q8_0) t->ex = t->qs + al256(n * 16);            // bytes 16..31 of every block
    *out = t;
    return G4H_OK;
}

extern "C" int g4h_tensor_load(g4h_tensor *t, const void *rows, int src_is_device, void *s) {
    G4_NEED_INIT();
    if (!t || !rows) return fail(G4H_ERR_ARG, "g4h_tensor_load: null pointer");
    const size_t bytes = (size_t)t->nrows * g4h_row_size(t->type, t->ncols);
    const hipStream_t st = (hipStream_t)s;
    if (src_is_device) {
        G4_HIP(launch_repack(*t, (const uint8_t *)rows, st));
        return G4H_OK;
    }
    void *tmp = nullptr;
    if (int rc = dev_alloc(&tmp, bytes)) return rc;
    hipError_t e = hipMemcpyAsync(tmp, rows, bytes, hipMemcpyHostToDevice, st);
    if (e == hipSuccess) e = launch_repack(*t, (const uint8_t *)tmp, st);
    if (e == hipSuccess) e = hipStreamSynchronize(st);
    (void)hipFree(tmp);
    if (e != hipSuccess) return hip_fail(e, "g4h_tensor_load");
    return G4H_OK;
}

extern "C" int g4h_tensor_store(const g4h_tensor *t, void *rows_dev, void *s) {
    G4_NEED_INIT();
    if (!t || !rows_dev) return fail(G4H_ERR_ARG, "g4h_tensor_store: null pointer");
    G4_HIP(launch_unpack(*t, (uint8_t *)rows_dev, (hipStream_t)s));
    return G4H_OK;
}

extern "C" int g4h_tensor_free(g4h_tensor *t) {
    if (!t) return G4H_OK;
    hipError_t e = hipFree(t->base);
    delete t;
    if (e != hipSuccess) return hip_fail(e, "g4h_tensor_free");
    return G4H_OK;
}
extern "C" size_t g4h_tensor_bytes(const g4h_tensor *t) { return t ? t->bytes : 0; }
extern "C" int g4h_tensor_info(const g4h_tensor *t, int *type, int64_t *ncols, int64_t *nrows) {
    if (!t) return fail(G4H_ERR_ARG, "g4h_tensor_info: null tensor");
    if (type) *type = t->type;
    if (ncols) *ncols = t->ncols;
    if (nrows) *nrows = t->nrows;
    return G4H_OK;
}

// ------------------------------------------------------------- matmul ----
static constexpr size_t kMaxLds = 65536;

// fp32 inputs of the GEMV family are quantized inside the GEMV (one launch)
// unless G4H_GEMV_FUSED_QUANT=0 asks for the separate quantizer launch; the
// results are the same bit for bit either way.
static bool fused_quant_enabled() {
    static const bool on = [] {
        const char *e = getenv("G4H_GEMV_FUSED_QUANT");
        return !(e && atoi(e) == 0);
    }();
    return on;
}

// The LDS a GEMV launch over W may stage its activations in: 64 KB, or for
// eight q8_0 / q4_0 tokens what one workgroup may hold on this device (those
// launches take up to 16 waves per workgroup, one workgroup per CU).
static size_t gemv_lds_cap(const g4h_tensor &W, int chunk) {
    if (chunk != 8 || (W.type != Q4_0 && W.type != Q8_0)) return kMaxLds;
    static const size_t dev_max = [] {
        int dev = 0, v = 0;
        if (hipGetDevice(&dev) != hipSuccess ||
            hipDeviceGetAttribute(&v, hipDeviceAttributeMaxSharedMemoryPerBlock, dev) != hipSuccess || v <= 0)
            return kMaxLds;
        return (size_t)v;
    }();
    return dev_max > kMaxLds ? dev_max : kMaxLds;
}

// GEMV token chunks of 8/4/2/1 within the LDS budget: the chunk that starts at
// token `done` of nb
static int gemv_chunk_at(const g4h_tensor &W, int nb, int done) {
    int chunk = 8;
    while (chunk > nb - done || (chunk > 1 && gemv_lds_bytes(W.type, chunk, W.nb) > gemv_lds_cap(W, chunk))) chunk >>= 1;
    return chunk;
}

// whether an fp32-input call of nb tokens quantizes inside every GEMV chunk
// (16-byte aligned x assumed); otherwise a quantizer launch runs first
static bool x_fused(const g4h_tensor &W, int nb) {
    if (!fused_quant_enabled()) return false;
    for (int done = 0; done < nb;) {
        const int chunk = gemv_chunk_at(W, nb, done);
        if (!gemv_fused_fits(W, chunk)) return false;
        done += chunk;
    }
    return true;
}

// From kMmMinTokens tokens the matrix-core family replaces the GEMV family:
// the measured crossover on q8_0 4096x4096 (graph-timed calls, quantization
// included) lies between 8 tokens (GEMV 9.5 us, matrix cores 11.5 us) and 16
// (17.0 us vs 11.5 us), past 8 tokens the GEMV family taking a second launch;
// q4_K / q6_K 4096x11008 are already faster on the matrix cores at 8 tokens
// (23.0 / 31.1 us against 24.8 / 33.7 us).

// f16 / bf16 rows need whole 16-column steps (k_mm_float)
static bool mfma_capable(const g4h_tensor *W) {
    return W && (W->type == Q8_0 || W->type == Q4_0 || mmk_capable(W->type) || (is_float(W->type) && W->ncols % 16 == 0));
}

extern "C" int g4h_matmul_path(const g4h_tensor *W, int nb) {
    return mfma_capable(W) && nb >= kMmMinTokens ? 2 : 1;
}

static const char *type_name(int t) {
    switch (t) {
    case Q4_0: return "q4_0";
    case Q8_0: return "q8_0";
    case Q2_K: return "q2_K";
    case Q3_K: return "q3_K";
    case Q5_K: return "q5_K";
    case Q6_K: return "q6_K";
    case TQ2_0: return "tq2_0";
    case F16: return "f16";
    case BF16: return "bf16";
    case Q4_K: return "q4_K";
    default: return "?";
    }
}

extern "C" int g4h_matmul_describe(const g4h_tensor *W, int nb, int path, char *buf, size_t len) {
    if (!W || !buf || len == 0 || nb <= 0 || path < 0 || path > 2) return fail(G4H_ERR_ARG, "g4h_matmul_describe: bad argument");
    if (path == 0) path = g4h_matmul_path(W, nb);
    if (path == 2) {
        if (!mfma_capable(W)) return fail(G4H_ERR_TYPE, "g4h_matmul_describe: the matrix-core path takes q8_0 / q4_0 / q4_K / q6_K weights and f16 / bf16 rows of whole 16-column steps");
        if (mmk_capable(W->type)) mmk_describe(*W, nb, buf, len);
        else if (is_float(W->type))
            snprintf(buf, len, "k_mm_float<%s> grid=%lldx%d block=512 (matrix cores, 32x32 tiles, 8 waves split the columns)",
                     type_name(W->type), (long long)((W->nrows + 31) / 32), (nb + 31) / 32);
        else mm_describe(*W, nb, buf, len);
        return G4H_OK;
    }
    if (is_float(W->type)) {
        const int chunk = nb >= 8 ? 8 : nb >= 4 ? 4 : nb >= 2 ? 2 : 1;
        snprintf(buf, len, "k_gemv_float<%s,nb=%d> grid=%lld block=256 (x%d launches); fp32 x converted by a separate launch",
                 type_name(W->type), chunk, (long long)((W->nrows + 3) / 4), (nb + chunk - 1) / chunk);
        return G4H_OK;
    }
    int lpr, upl, wpg;
    int64_t grid;
    const int chunk = gemv_chunk_at(*W, nb, 0);
    int launches = 0;
    for (int done = 0; done < nb; launches++) done += gemv_chunk_at(*W, nb, done);
    const bool xq = x_fused(*W, nb);
    gemv_launch_shape(*W, &lpr, &upl, &wpg, &grid, chunk, xq);
    upl = gemv_upl_final(W->type, W->nb, chunk, lpr, upl);
    snprintf(buf, len, "k_gemv<%s,nb=%d,lpr=%d,upl=%d> grid=%lld block=%d (x%d launches); fp32 x %s", type_name(W->type), chunk,
             lpr, upl, (long long)grid, 64 * wpg, launches, xq ? "quantized in-kernel" : "quantized by a separate launch");
    return G4H_OK;
}

static int check_act(const char *fn, const g4h_tensor *W, const void *pre, size_t stride, int nb) {
    if ((uintptr_t)pre % 4 || stride % 4) return fail(G4H_ERR_ARG, "%s: activations must be 4-byte aligned with a 4-byte multiple stride", fn);
    if (nb > 1 && stride < g4h_row_size(g4h_act_type(W->type), W->ncols))
        return fail(G4H_ERR_ARG, "%s: activation stride %zu smaller than a row", fn, stride);
    return G4H_OK;
}


// where g4h_matmul_ex / g4h_matmul_noalloc take the scratch of one call from
struct ScratchSrc {
    void *fixed = nullptr;      // the device's `scratch` (no allocation), or null: the per-stream pool
    int get(hipStream_t s, size_t bytes, void **out) const {
        if (!fixed) return scratch_for(s, bytes, out);
        if (bytes > kNoAllocBytes)
            return fail(G4H_ERR_ARG, "g4h_matmul_noalloc: this call needs %zu bytes of scratch, more than the fixed %zu "
                                     "(use g4h_matmul)", bytes, kNoAllocBytes);
        *out = fixed;
        return G4H_OK;
    }
};

static int matmul_impl(const g4h_tensor *W, const float *x, const void *pre, size_t pre_stride, float *Y, int nb, int path,
                       void *stream, const ScratchSrc &scr, const GemvOut &out = GemvOut());

extern "C" int g4h_matmul_ex(const g4h_tensor *W, const float *x, const void *pre, size_t pre_stride, float *Y, int nb,
                             int path, void *stream) {
    return matmul_impl(W, x, pre, pre_stride, Y, nb, path, stream, ScratchSrc());
}

extern "C" size_t g4h_matmul_noalloc_max_bytes(void) { return kNoAllocBytes; }

extern "C" int g4h_matmul_noalloc(const g4h_tensor *W, const float *x, const void *pre, size_t pre_stride, float *Y, int nb,
                                  int path, void *stream) {
    G4_NEED_INIT();
    int dev = -1;
    G4_HIP(hipGetDevice(&dev));
    ScratchSrc scr;
    {
        std::lock_guard<std::mutex> lk(g_noalloc_mu);
        const auto it = g_noalloc_ptr.find(dev);
        if (it == g_noalloc_ptr.end())
            return fail(G4H_ERR_DEVICE, "g4h_matmul_noalloc: g4h_init(%d) has not been called for the current device", dev);
        scr.fixed = it->second;
    }
    return matmul_impl(W, x, pre, pre_stride, Y, nb, path, stream, scr);
}

static int matmul_impl(const g4h_tensor *W, const float *x, const void *pre, size_t pre_stride, float *Y, int nb, int path,
                       void *stream, const ScratchSrc &scr, const GemvOut &out) {
    G4_NEED_INIT();
    if (!W || !Y) return fail(G4H_ERR_ARG, "g4h_matmul: null tensor or output");
    if ((x == nullptr) == (pre == nullptr)) return fail(G4H_ERR_ARG, "g4h_matmul: pass exactly one of x_dev and pre_dev");
    if (nb < 0) return fail(G4H_ERR_ARG, "g4h_matmul: nb=%d", nb);
    if (path < 0 || path > 2) return fail(G4H_ERR_ARG, "g4h_matmul: path=%d", path);
    if (nb == 0) return G4H_OK;
    const hipStream_t s = (hipStream_t)stream;
    if (out.mode != OUT_STORE) {
        if (nb != 1 || path == 2) return fail(G4H_ERR_ARG, "g4h_matmul: a GELU-product store takes one token on the GEMV family");
        path = 1;
    }
    if (path == 0) path = g4h_matmul_path(W, nb);
    if (path == 2 && mfma_capable(W) && mmk_capable(W->type)) {
        // K-quants: q8_K activation rows (quantized here from x, or given), read as they are
        const uint8_t *act = (const uint8_t *)pre;
        size_t stride = pre_stride;
        if (x) {
            if ((uintptr_t)x % 4) return fail(G4H_ERR_ARG, "g4h_matmul: x must be 4-byte aligned");
            stride = g4h_act_stride(W->type, W->ncols);
            void *buf;
            if (int rc = scr.get(s, stride * nb, &buf)) return rc;
            const hipError_t e = launch_quantize_q8_K(x, W->ncols, (uint8_t *)buf, stride, W->ncols, nb, s);
            if (e != hipSuccess) return hip_fail(e, "g4h_matmul: quantize");
            act = (const uint8_t *)buf;
        } else {
            if (int rc = check_act("g4h_matmul", W, pre, pre_stride, nb)) return rc;
            if (nb == 1) stride = g4h_act_stride(W->type, W->ncols);
        }
        const hipError_t e = launch_matmul_mfma_k(*W, act, stride, nb, Y, s);
        if (e != hipSuccess) return hip_fail(e, "g4h_matmul: matrix-core launch");
        return G4H_OK;
    }
    if (path == 2 && is_float(W->type) && mfma_capable(W)) {
        // f16 / bf16 rows on the matrix cores: fp32 x rounded on load, or the
        // prepared rows (f16 / bf16-rounded fp32) as they are
        hipError_t e;
        if (x) {
            if ((uintptr_t)x % 16) return fail(G4H_ERR_ARG, "g4h_matmul: x must be 16-byte aligned on the matrix-core path");
            e = launch_mm_float(W->type, W->qs, (size_t)W->ncols * 2, W->nrows, W->ncols, x, W->ncols, nullptr, 0, nb, Y, s);
        } else {
            if (int rc = check_act("g4h_matmul", W, pre, pre_stride, nb)) return rc;
            const size_t stride = nb == 1 ? g4h_act_stride(W->type, W->ncols) : pre_stride;
            if ((uintptr_t)pre % 16 || stride % 16)
                return fail(G4H_ERR_ARG, "g4h_matmul: f16/bf16 activations must be 16-byte aligned with a 16-byte multiple stride");
            e = launch_mm_float(W->type, W->qs, (size_t)W->ncols * 2, W->nrows, W->ncols, nullptr, 0, (const uint8_t *)pre, stride, nb,
                                Y, s);
        }
        if (e != hipSuccess) return hip_fail(e, "g4h_matmul: matrix-core launch");
        return G4H_OK;
    }
    if (path == 2) {
        if (!mfma_capable(W)) return fail(G4H_ERR_TYPE, "g4h_matmul: the matrix-core path takes q8_0 / q4_0 / q4_K / q6_K weights and f16 / bf16 rows of whole 16-column steps");
        if (x && (uintptr_t)x % 16) return fail(G4H_ERR_ARG, "g4h_matmul: x must be 16-byte aligned on the matrix-core path");
        if (!x)
            if (int rc = check_act("g4h_matmul", W, pre, pre_stride, nb)) return rc;
        void *buf;
        if (int rc = scr.get(s, mm_planar_bytes(nb, W->ncols), &buf)) return rc;
        const hipError_t e = launch_matmul_mfma(*W, x, W->ncols, (const uint8_t *)pre, pre_stride, nb, Y, (uint8_t *)buf, s);
        if (e != hipSuccess) return hip_fail(e, "g4h_matmul: matrix-core launch");
        return G4H_OK;
    }
    if (is_float(W->type)) {
        // prep_act's conversion (model.c:163-180), then the float GEMV in token
        // chunks of 8/4/2/1
        const uint8_t *act = (const uint8_t *)pre;
        size_t stride = pre_stride;
        if (x && nb <= 2 && (uintptr_t)x % 16 == 0 && W->ncols % 8 == 0) {
            // one or two aligned fp32 tokens: converted inside the GEMV, same
            // bits, one launch (larger batches convert once up front: every
            // wave would reread and convert all of their tokens)
            for (int done = 0; done < nb;) {
                const int left = nb - done, chunk = left >= 8 ? 8 : left >= 4 ? 4 : left >= 2 ? 2 : 1;
                const hipError_t e = launch_gemv_float_x(W->type, W->qs, (size_t)W->ncols * 2, W->nrows, W->ncols,
                                                         x + (size_t)done * W->ncols, W->ncols, Y + (size_t)done * W->nrows,
                                                         W->nrows, chunk, s, out);
                if (e != hipSuccess) return hip_fail(e, "g4h_matmul: gemv launch");
                done += chunk;
            }
            return G4H_OK;
        }
        if (x) {
            if ((uintptr_t)x % 4) return fail(G4H_ERR_ARG, "g4h_matmul: x must be 4-byte aligned");
            stride = g4h_act_stride(W->type, W->ncols);
            void *buf;
            if (int rc = scr.get(s, stride * nb, &buf)) return rc;
            const hipError_t e = launch_act_float(W->type, x, W->ncols, W->ncols, nb, (uint8_t *)buf, stride, s);
            if (e != hipSuccess) return hip_fail(e, "g4h_matmul: activation conversion");
            act = (const uint8_t *)buf;
        } else {
            if (int rc = check_act("g4h_matmul", W, pre, pre_stride, nb)) return rc;
            if ((uintptr_t)pre % 16 || (nb > 1 && pre_stride % 16))
                return fail(G4H_ERR_ARG, "g4h_matmul: f16/bf16 activations must be 16-byte aligned with a 16-byte multiple stride");
            if (nb == 1) stride = 16;
        }
        for (int done = 0; done < nb;) {
            const int left = nb - done, chunk = left >= 8 ? 8 : left >= 4 ? 4 : left >= 2 ? 2 : 1;
            const hipError_t e = launch_gemv_float(W->type, W->qs, (size_t)W->ncols * 2, W->nrows, W->ncols, act + (size_t)done * stride,
                                                   stride, Y + (size_t)done * W->nrows, W->nrows, chunk, s, out);
            if (e != hipSuccess) return hip_fail(e, "g4h_matmul: gemv launch");
            done += chunk;
        }
        return G4H_OK;
    }
    const uint8_t *act = (const uint8_t *)pre;
    size_t stride = pre_stride;
    if (x && (uintptr_t)x % 16 == 0 && fused_quant_enabled()) {
        // q8_0 / q4_0 weights (and one K-quant token): every chunk quantizes its
        // fp32 tokens in the GEMV prologue
        if (x_fused(*W, nb)) {
            for (int done = 0; done < nb;) {
                const int chunk = gemv_chunk_at(*W, nb, done);
                const hipError_t e = launch_gemv_x(*W, x + (size_t)done * W->ncols, Y + (size_t)done * W->nrows, chunk, s, out);
                if (e != hipSuccess) return hip_fail(e, "g4h_matmul: gemv launch");
                done += chunk;
            }
            return G4H_OK;
        }
    }
    if (x) {
        if ((uintptr_t)x % 4) return fail(G4H_ERR_ARG, "g4h_matmul: x must be 4-byte aligned");
        stride = g4h_act_stride(W->type, W->ncols);
        void *buf;
        if (int rc = scr.get(s, stride * nb, &buf)) return rc;
        const hipError_t e = g4h_act_type(W->type) == Q8_0
                                 ? launch_quantize_q8_0(x, W->ncols, (uint8_t *)buf, stride, W->ncols, nb, s)
                                 : launch_quantize_q8_K(x, W->ncols, (uint8_t *)buf, stride, W->ncols, nb, s);
        if (e != hipSuccess) return hip_fail(e, "g4h_matmul: quantize");
        act = (const uint8_t *)buf;
    } else if (int rc = check_act("g4h_matmul", W, pre, pre_stride, nb)) {
        return rc;
    }
    // GEMV family in token chunks of 8/4/2/1 that fit the LDS budget
    int done = 0;
    while (done < nb) {
        const int chunk = gemv_chunk_at(*W, nb, done);
        const hipError_t e = launch_gemv(*W, act + (size_t)done * stride, stride, Y + (size_t)done * W->nrows, chunk, s, out);
        if (e != hipSuccess) return hip_fail(e, "g4h_matmul: gemv launch");
        done += chunk;
    }
    return G4H_OK;
}

extern "C" int g4h_matmul(const g4h_tensor *W, const float *x, const void *pre, size_t pre_stride, float *Y, int nb, void *s) {
    return g4h_matmul_ex(W, x, pre, pre_stride, Y, nb, 0, s);
}

namespace g4 {
int matmul_out(const g4h_tensor *W, const float *x, float *Y, int nb, void *stream, const GemvOut &out) {
    return matmul_impl(W, x, nullptr, 0, Y, nb, 1, stream, ScratchSrc(), out);
}
bool few_direct() {
    const char *e = getenv("G4H_FEW_DIRECT");
    return !e || atoi(e) != 0;
}
bool matmul_few_ready(const g4h_tensor *W, int nb, int path) {
    if (!W || nb < 1 || path == 1 || (path == 0 && g4h_matmul_path(W, nb) != 2)) return false;
    return mm_few_ready(*W, nb);
}
int matmul_few(const g4h_tensor *W, const FewAct &a, float *Y, int nb, void *stream) {
    if (!W || !Y) return fail(G4H_ERR_ARG, "g4h_matmul: null tensor or output");
    const hipError_t e = launch_mm_few_ready(*W, a, nb, Y, (hipStream_t)stream);
    if (e != hipSuccess) return hip_fail(e, "g4h_matmul: matrix-core launch");
    return G4H_OK;
}
}  // namespace g4

extern "C" int g4h_read_floor(const void *src, size_t bytes, float *y, int64_t ny, int threads, int loads, void *s) {
    G4_NEED_INIT();
    if (!src || bytes < 16 || bytes % 16 || (uintptr_t)src % 16 || threads < 64 || threads > 1024 || threads % 64 || loads < 1 ||
        loads > 8 || ny < 0 || (ny > 0 && !y))
        return fail(G4H_ERR_ARG, "g4h_read_floor: bad argument");
    G4_HIP(launch_read_floor((const uint8_t *)src, bytes, y, ny, threads, loads, (hipStream_t)s));
    return G4H_OK;
}

extern "C" int g4h_block_sums(const g4h_tensor *W, const void *pre, size_t pre_stride, int tok, int32_t *sums, void *s) {
    G4_NEED_INIT();
    if (!W || !pre || !sums || tok < 0) return fail(G4H_ERR_ARG, "g4h_block_sums: bad argument");
    if (is_float(W->type)) return fail(G4H_ERR_TYPE, "g4h_block_sums: f16/bf16 weights have no integer block sums");
    if (int rc = check_act("g4h_block_sums", W, pre, pre_stride, tok + 1)) return rc;
    G4_HIP(launch_block_sums(*W, (const uint8_t *)pre, pre_stride, tok, sums, (hipStream_t)s));
    return G4H_OK;
}

// ---------------------------------------------------------- attention ----
extern "C" size_t g4h_attn_workspace_bytes(int n_head, int hd, int n_pos) {
    if (n_head <= 0 || hd <= 0 || n_pos <= 0) return 0;
    return attn_workspace_bytes(n_head, hd, n_pos);
}

static int check_attn_shape(const char *fn, int kv_type, int n_head, int n_kv, int hd) {
    if (kv_type != F16 && kv_type != Q8_0 && kv_type != Q4_0)
        return fail(G4H_ERR_TYPE, "%s: KV type %d unsupported (f16, q8_0, q4_0)", fn, kv_type);
    if (n_kv <= 0 || n_head <= 0 || n_head % n_kv) return fail(G4H_ERR_SHAPE, "%s: n_head=%d not a multiple of n_kv=%d", fn, n_head, n_kv);
    const int grp = n_head / n_kv;
    if (grp != 1 && grp != 2 && grp != 4 && grp != 8) return fail(G4H_ERR_SHAPE, "%s: group size %d unsupported", fn, grp);
    if (hd == 512) {                         // gemma4's full-attention heads: one KV head (model.c:443-444)
        if (n_kv != 1) return fail(G4H_ERR_SHAPE, "%s: hd=512 takes one KV head (n_kv=%d)", fn, n_kv);
        return G4H_OK;
    }
    if (hd % 64 || hd > 256) return fail(G4H_ERR_SHAPE, "%s: hd=%d (must be a multiple of 64 up to 256, or 512)", fn, hd);
    return G4H_OK;
}

extern "C" int g4h_attn_passes(int kv_type, int n_head, int n_kv, int hd, int n_pos, int *passes) {
    G4_NEED_INIT();
    if (!passes) return fail(G4H_ERR_ARG, "g4h_attn_passes: null pointer");
    if (int rc = check_attn_shape("g4h_attn_passes", kv_type, n_head, n_kv, hd)) return rc;
    if (n_pos <= 0) return fail(G4H_ERR_ARG, "g4h_attn_passes: n_pos=%d", n_pos);
    *passes = hd == 512 ? 6 : attn_fused_fits(kv_type, n_head, n_kv, hd, n_pos) ? 1 : 3;   // 512: halves, joined
    return G4H_OK;
}

extern "C" int g4h_attn_decode(const float *q, const void *kc, const void *vc, int kv_type, int n_head, int n_kv, int hd,
                               int n_pos, float *out, void *ws, size_t ws_bytes, void *stream) {
    G4_NEED_INIT();
    if (!q || !kc || !vc || !out || !ws) return fail(G4H_ERR_ARG, "g4h_attn_decode: null pointer");
    if (int rc = check_attn_shape("g4h_attn_decode", kv_type, n_head, n_kv, hd)) return rc;
    if (n_pos <= 0) return fail(G4H_ERR_ARG, "g4h_attn_decode: n_pos=%d", n_pos);
    if (ws_bytes < attn_workspace_bytes(n_head, hd, n_pos))
        return fail(G4H_ERR_ARG, "g4h_attn_decode: workspace %zu < %zu bytes", ws_bytes, attn_workspace_bytes(n_head, hd, n_pos));
    const uintptr_t al = kv_type == F16 ? 8 : 4;
    if ((uintptr_t)kc % al || (uintptr_t)vc % al)
        return fail(G4H_ERR_ARG, "g4h_attn_decode: caches must be %zu-byte aligned", (size_t)al);
    QkvArgs a;
    a.n_head = n_head;
    a.n_kv = n_kv;
    a.hd = hd;
    a.kv_type = kv_type;
    a.kc = (uint8_t *)kc;          // read only: no preparation on this entry point
    a.vc = (uint8_t *)vc;
    G4_HIP(launch_attn_decode(q, nullptr, a, n_pos, nullptr, n_pos, out, nullptr, (uint8_t *)ws, (hipStream_t)stream, nullptr,
                              nullptr, nullptr, ws_bytes));
    return G4H_OK;
}

extern "C" int g4h_attn_decode_window(const float *q, const void *kc, const void *vc, int kv_type, int n_head, int n_kv, int hd,
                                      int n_pos, int window, int ring, float *out, void *ws, size_t ws_bytes, void *stream) {
    G4_NEED_INIT();
    if (!q || !kc || !vc || !out || !ws) return fail(G4H_ERR_ARG, "g4h_attn_decode_window: null pointer");
    if (int rc = check_attn_shape("g4h_attn_decode_window", kv_type, n_head, n_kv, hd)) return rc;
    if (n_pos <= 0 || window < 0 || ring < 0) return fail(G4H_ERR_ARG, "g4h_attn_decode_window: n_pos=%d window=%d ring=%d", n_pos, window, ring);
    if (ring && (!window || window > ring)) return fail(G4H_ERR_ARG, "g4h_attn_decode_window: a ring needs 0 < window <= ring");
    const int rows = window && window < n_pos ? window : n_pos;
    if (ws_bytes < attn_workspace_bytes(n_head, hd, rows))
        return fail(G4H_ERR_ARG, "g4h_attn_decode_window: workspace %zu < %zu bytes", ws_bytes, attn_workspace_bytes(n_head, hd, rows));
    const uintptr_t al = kv_type == F16 ? 8 : 4;
    if ((uintptr_t)kc % al || (uintptr_t)vc % al)
        return fail(G4H_ERR_ARG, "g4h_attn_decode_window: caches must be %zu-byte aligned", (size_t)al);
    QkvArgs a;
    a.n_head = n_head;
    a.n_kv = n_kv;
    a.hd = hd;
    a.kv_type = kv_type;
    a.kc = (uint8_t *)kc;          // read only: no preparation on this entry point
    a.vc = (uint8_t *)vc;
    a.window = window;
    a.ring = ring;
    G4_HIP(launch_attn_decode(q, nullptr, a, n_pos, nullptr, rows, out, nullptr, (uint8_t *)ws, (hipStream_t)stream, nullptr,
                              nullptr, nullptr, ws_bytes));
    return G4H_OK;
}

extern "C" int g4h_attn_status(void *ws, int *failed, void *stream) {
    G4_NEED_INIT();
    if (!ws || !failed) return fail(G4H_ERR_ARG, "g4h_attn_status: null pointer");
    const hipStream_t s = (hipStream_t)stream;
    unsigned err = 0;
    G4_HIP(hipMemcpyAsync(&err, (uint8_t *)ws + ATTN_ERR_OFFSET, sizeof err, hipMemcpyDeviceToHost, s));
    G4_HIP(hipStreamSynchronize(s));
    *failed = err ? 1 : 0;
    if (err) {
        G4_HIP(hipMemsetAsync((uint8_t *)ws + ATTN_ERR_OFFSET, 0, sizeof err, s));
        G4_HIP(hipStreamSynchronize(s));
        attn_ws_forget(ws);                  // cleared before its next use (g4h_internal_attn_error)
    }
    return G4H_OK;
}

extern "C" size_t g4h_attn_prefill_workspace_bytes(int n_head, int hd, int pos0, int nb) {
    if (n_head <= 0 || hd <= 0 || pos0 < 0 || nb <= 0) return 0;
    return attn_batch_workspace_bytes(n_head, hd, pos0 + nb, nb);
}

extern "C" int g4h_attn_prefill_mm(const float *q, const void *kc, const void *vc, int kv_type, int n_head, int n_kv, int hd,
                                   int pos0, int nb, int window, int ring, float *out, void *ws, size_t ws_bytes, void *s) {
    G4_NEED_INIT();
    if (!q || !out || !kc || !vc || !ws || nb < 1 || nb > 65535 || pos0 < 0 || window < 0 || ring < 0)
        return fail(G4H_ERR_ARG, "g4h_attn_prefill_mm: bad argument");
    if (int rc = check_attn_shape("g4h_attn_prefill_mm", kv_type, n_head, n_kv, hd)) return rc;
    QkvArgs a;
    a.n_head = n_head;
    a.n_kv = n_kv;
    a.hd = hd;
    a.kv_type = kv_type;
    a.kc = (uint8_t *)kc;
    a.vc = (uint8_t *)vc;
    a.window = window;
    a.ring = ring;
    if (!attn_batch_mm_ok(a)) return fail(G4H_ERR_TYPE, "g4h_attn_prefill_mm: takes f16 caches, head dims 64/128/256/512");
    if (ring && (!window || window > ring || nb > ring - window + 1))
        return fail(G4H_ERR_ARG, "g4h_attn_prefill_mm: a ring needs 0 < window <= ring and nb <= ring - window + 1");
    if ((uintptr_t)kc % 16 || (uintptr_t)vc % 16) return fail(G4H_ERR_ARG, "g4h_attn_prefill_mm: caches must be 16-byte aligned");
    const int rows = window ? std::min(window, pos0 + nb) : pos0 + nb;
    if (ws_bytes < attn_batch_mm_workspace_bytes(n_head, hd, rows, nb))
        return fail(G4H_ERR_ARG, "g4h_attn_prefill_mm: workspace smaller than g4h_attn_prefill_workspace_bytes");
    G4_HIP(launch_attn_batch_mm(q, a, pos0 + 1, nb, out, nullptr, (uint8_t *)ws, ws_bytes, (hipStream_t)s));
    return G4H_OK;
}

extern "C" int g4h_attn_prefill(const float *q, const void *kc, const void *vc, int kv_type, int n_head, int n_kv, int hd,
                                int pos0, int nb, float *out, void *ws, size_t ws_bytes, void *s) {
    G4_NEED_INIT();
    if (!q || !out || nb < 0 || pos0 < 0 || n_head <= 0 || hd <= 0) return fail(G4H_ERR_ARG, "g4h_attn_prefill: bad argument");
    if (nb == 0) return G4H_OK;
    if (!kc || !vc || !ws) return fail(G4H_ERR_ARG, "g4h_attn_prefill: null pointer");
    if (int rc = check_attn_shape("g4h_attn_prefill", kv_type, n_head, n_kv, hd)) return rc;
    if (nb <= 65535 && ws_bytes >= g4h_attn_prefill_workspace_bytes(n_head, hd, pos0, nb)) {
        // model.c:514-521, all tokens in one set of launches
        const uintptr_t al = kv_type == F16 ? 8 : 4;
        if ((uintptr_t)kc % al || (uintptr_t)vc % al)
            return fail(G4H_ERR_ARG, "g4h_attn_prefill: caches must be %zu-byte aligned", (size_t)al);
        QkvArgs a;
        a.n_head = n_head;
        a.n_kv = n_kv;
        a.hd = hd;
        a.kv_type = kv_type;
        a.kc = (uint8_t *)kc;
        a.vc = (uint8_t *)vc;
        G4_HIP(launch_attn_batch(q, a, pos0 + 1, nb, out, nullptr, (uint8_t *)ws, (hipStream_t)s));
        return G4H_OK;
    }
    if (ws_bytes < g4h_attn_workspace_bytes(n_head, hd, pos0 + nb))
        return fail(G4H_ERR_ARG, "g4h_attn_prefill: workspace smaller than g4h_attn_workspace_bytes(n_head, hd, pos0 + nb)");
    // a smaller workspace: one decode call per token (model.c:514-521: token b
    // at pos0 + b attends [0, pos0 + b])
    for (int b = 0; b < nb; b++) {
        const size_t off = (size_t)b * n_head * hd;
        if (int rc = g4h_attn_decode(q + off, kc, vc, kv_type, n_head, n_kv, hd, pos0 + b + 1, out + off, ws, ws_bytes, s)) return rc;
    }
    return G4H_OK;
}

extern "C" int g4h_kv_store(int kv_type, const float *src, void *dst, int hd, int rows, size_t dst_stride, void *stream) {
    G4_NEED_INIT();
    if (!src || !dst || hd <= 0 || rows < 0) return fail(G4H_ERR_ARG, "g4h_kv_store: bad argument");
    if (kv_type != F16 && kv_type != Q8_0 && kv_type != Q4_0) return fail(G4H_ERR_TYPE, "g4h_kv_store: type %d", kv_type);
    if (hd % blck(kv_type)) return fail(G4H_ERR_SHAPE, "g4h_kv_store: hd=%d", hd);
    const size_t rb = kv_type == F16 ? (size_t)hd * 2 : g4h_row_size(kv_type, hd);
    if (dst_stride == 0) dst_stride = rb;
    if (rows > 1 && dst_stride < rb) return fail(G4H_ERR_ARG, "g4h_kv_store: stride smaller than a row");
    if ((uintptr_t)dst % 2 || dst_stride % 2) return fail(G4H_ERR_ARG, "g4h_kv_store: destination must be 2-byte aligned");
    if (rows == 0) return G4H_OK;
    G4_HIP(launch_kv_store(kv_type, src, (uint8_t *)dst, hd, rows, dst_stride, (hipStream_t)stream));
    return G4H_OK;
}
