// k_model.hip -- the elementwise / reduction kernels of the decode step
// (model.c:593-775 for a gemma-style decoder) and device-side random init.
//
// Every kernel reads the position / token from device memory so that one
// decode step can be captured once and replayed.  Numerics follow the
// reference: RMSNorm sums squares in double and scales by 1/sqrt(mean+eps)
// (model.c:338-345); RoPE uses a host-computed cos/sin table built exactly as
// rope_cache does (model.c:349-358); GELU is the fp16 lookup table
// (g4run.h:73-77); argmax keeps the first maximum (sampler.c:139-144).
#include "formats.h"
#include "kernels.h"

namespace g4 {

// --------------------------------------------------------------- helpers --
__device__ __forceinline__ float rms_scale(double ss, int n, float eps) {
    const float mean = (float)(ss / n);
    return 1.0f / __builtin_sqrtf(mean + eps);
}

// q8_0-quantize n floats from LDS (n % 32 == 0) into GGUF blocks at dst, with
// the arithmetic of k_quantize_q8_0 (8 lanes per block).
__device__ void quantize_q8_0_lds(const float *x, int n, uint8_t *dst) {
    for (int i = threadIdx.x; i < n / 4; i += blockDim.x) {
        const int b = i >> 3, k = i & 7;
        float v[4] = {x[4 * i], x[4 * i + 1], x[4 * i + 2], x[4 * i + 3]};
        float am = fmaxf(fmaxf(fabsf(v[0]), fabsf(v[1])), fmaxf(fabsf(v[2]), fabsf(v[3])));
        am = fmaxf(am, shfl_xor(am, 1));
        am = fmaxf(am, shfl_xor(am, 2));
        am = fmaxf(am, shfl_xor(am, 4));
        const float id = am != 0.0f ? 127.0f / am : 0.0f;
        uint32_t pk = 0;
#pragma unroll
        for (int j = 0; j < 4; j++) pk |= ((uint32_t)(int)__builtin_rintf(v[j] * id) & 0xffu) << (8 * j);
        uint8_t *blk = dst + (size_t)b * 34;
        uint16_t *p16 = (uint16_t *)(blk + 2 + 4 * k);
        p16[0] = (uint16_t)(pk & 0xffff);
        p16[1] = (uint16_t)(pk >> 16);
        if (k == 0) *(uint16_t *)blk = f2h(am * (1.0f / 127.0f));
    }
}

// ---------------------------------------------------------- random init --
__device__ __forceinline__ uint64_t mix64(uint64_t z) {
    z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ull;
    z = (z ^ (z >> 27)) * 0x94d049bb133111ebull;
    return z ^ (z >> 31);
}
// y[i] = mean + std * N(0,1): Box-Muller on a counter-based splitmix64 stream
__global__ __launch_bounds__(256) void k_rand_normal(float *y, int64_t n, uint64_t seed, float mean, float std) {
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= n) return;
    const uint64_t r = mix64(seed + 0x9e3779b97f4a7c15ull * (uint64_t)(i + 1));
    const float u1 = ((uint32_t)(r >> 40) + 1) * (1.0f / 16777217.0f);      // (0, 1]
    const float u2 = (uint32_t)(r & 0xffffff) * (1.0f / 16777216.0f);
    y[i] = mean + std * __builtin_sqrtf(-2.0f * __logf(u1)) * __cosf(6.2831853f * u2);
}

// ------------------------------------------------------------- embedding --
// x = dequant(row `token` of the tied q8_0 head) * sqrt(n_embd)
// (model.c:605-612), read from the resident planes (qs [row][blk][32], d fp16).
__global__ __launch_bounds__(256) void k_embed_planes(const int8_t *qs, const uint16_t *sc, int64_t nb, const int *token,
                                                      float *x, int n, float es) {
    const int64_t r = *token;
    for (int i = threadIdx.x; i < n; i += blockDim.x) {
        const int64_t j = r * nb + (i >> 5);
        const float v = (float)qs[j * 32 + (i & 31)] * h2f(sc[j]);
        x[i] = v * es;
    }
}

// ------------------------------------------------------ norm + quantize --
// One workgroup of 1024 threads, thread t owning elements 4t..4t+3 (n <= 4096,
// n % 32 == 0).  If delta: x += rms(delta)*w_post (the post-norm residual of
// model.c:711-716 / 731-736).  Then q8_0(rms(x)*w_pre) into act (the next
// projection's activation, model.c:657-661 / 721-722).  Sums of squares are in
// double: wave butterflies, then the 16 wave partials in order.
__device__ __forceinline__ double wave_sum_dd(double v) {
    for (int k = 32; k >= 1; k >>= 1) v += __shfl_xor(v, k, 64);
    return v;
}
__device__ double block_sum_16w(double v, double *red) {
    v = wave_sum_dd(v);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
    __syncthreads();
    double r = 0.0;
    for (int w = 0; w < (int)(blockDim.x >> 6); w++) r += red[w];
    __syncthreads();
    return r;
}

__global__ __launch_bounds__(1024) void k_norm_quant(float *x, const float *delta, const float *w_post, const float *w_pre,
                                                     float eps, int n, uint8_t *act, float *xb_out) {
    __shared__ double red[16];
    const int t = threadIdx.x, i0 = 4 * t;
    const bool own = i0 < n;
    float v[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    if (own) {
        const float4 xv = *(const float4 *)(x + i0);
        v[0] = xv.x; v[1] = xv.y; v[2] = xv.z; v[3] = xv.w;
    }
    if (delta) {
        float d[4] = {0.0f, 0.0f, 0.0f, 0.0f};
        double ss = 0.0;
        if (own) {
            const float4 dv = *(const float4 *)(delta + i0);
            d[0] = dv.x; d[1] = dv.y; d[2] = dv.z; d[3] = dv.w;
            for (int k = 0; k < 4; k++) ss += (double)d[k] * d[k];
        }
        const float sc = rms_scale(block_sum_16w(ss, red), n, eps);
        if (own) {
            for (int k = 0; k < 4; k++) v[k] = v[k] + d[k] * sc * w_post[i0 + k];
            *(float4 *)(x + i0) = make_float4(v[0], v[1], v[2], v[3]);
        }
    }
    double ss = 0.0;
    for (int k = 0; k < 4; k++) ss += (double)v[k] * v[k];
    const float sc = rms_scale(block_sum_16w(ss, red), n, eps);
    if (own)
        for (int k = 0; k < 4; k++) v[k] = v[k] * sc * w_pre[i0 + k];
    if (xb_out && own) *(float4 *)(xb_out + i0) = make_float4(v[0], v[1], v[2], v[3]);
    // q8_0 blocks: 8 threads per 32 elements (quants.c:74-109 arithmetic)
    float am = fmaxf(fmaxf(fabsf(v[0]), fabsf(v[1])), fmaxf(fabsf(v[2]), fabsf(v[3])));
    am = fmaxf(am, shfl_xor(am, 1));
    am = fmaxf(am, shfl_xor(am, 2));
    am = fmaxf(am, shfl_xor(am, 4));
    if (!own) return;
    const float id = am != 0.0f ? 127.0f / am : 0.0f;
    uint32_t pk = 0;
#pragma unroll
    for (int j = 0; j < 4; j++) pk |= ((uint32_t)(int)__builtin_rintf(v[j] * id) & 0xffu) << (8 * j);
    const int b = t >> 3, k = t & 7;
    uint8_t *blk = act + (size_t)b * 34;
    uint16_t *p16 = (uint16_t *)(blk + 2 + 4 * k);
    p16[0] = (uint16_t)(pk & 0xffff);
    p16[1] = (uint16_t)(pk >> 16);
    if (k == 0) *(uint16_t *)blk = f2h(am * (1.0f / 127.0f));
}

// ------------------------------------------- q/k norm, RoPE, KV store --
// grid = n_head + 2*n_kv workgroups of hd threads over the fused q|k|v output:
// q heads: rms*q_norm, RoPE -> q_out; k heads: rms*k_norm, RoPE -> K cache slot
// pos; v heads: rms without weight -> V cache slot pos (model.c:664-687).
__global__ __launch_bounds__(256) void k_qkv_prep(const float *qkv, int n_head, int n_kv, int hd, const float *q_norm,
                                                  const float *k_norm, float eps, const float *rope, const int *pos,
                                                  float *q_out, uint8_t *kc, uint8_t *vc, int kv_type) {
    __shared__ double red[16];
    __shared__ float buf[256];
    const int h = blockIdx.x, t = threadIdx.x;
    const int p = *pos;
    const float *src = qkv + (size_t)h * hd;
    const float v = t < hd ? src[t] : 0.0f;
    const float sc = rms_scale(block_sum_16w(t < hd ? (double)v * v : 0.0, red), hd, eps);
    const bool is_q = h < n_head, is_k = !is_q && h < n_head + n_kv;
    const float *w = is_q ? q_norm : is_k ? k_norm : nullptr;
    if (t < hd) buf[t] = w ? v * sc * w[t] : v * sc;
    __syncthreads();
    float y = t < hd ? buf[t] : 0.0f;
    if ((is_q || is_k) && t < hd) {          // NeoX rotation of (i, i+hd/2) (model.c:359-367)
        const int half = hd / 2, i = t < half ? t : t - half;
        const float c = rope[(size_t)p * hd + 2 * i], s = rope[(size_t)p * hd + 2 * i + 1];
        const float a = buf[i], b = buf[i + half];
        y = t < half ? a * c - b * s : a * s + b * c;
    }
    __syncthreads();
    if (is_q) {
        if (t < hd) q_out[(size_t)h * hd + t] = y;
        return;
    }
    const int kvh = is_k ? h - n_head : h - n_head - n_kv;
    uint8_t *cache = is_k ? kc : vc;
    if (kv_type == F16) {
        if (t < hd) ((uint16_t *)cache)[((size_t)p * n_kv + kvh) * hd + t] = f2h(y);
    } else {
        if (t < hd) buf[t] = y;
        __syncthreads();
        quantize_q8_0_lds(buf, hd, cache + ((size_t)p * n_kv + kvh) * (hd / 32) * 34);
    }
}

// -------------------------------------------------------- gelu * up --
// h = gelu(g) * u with the fp16 GELU table (model.c:725-729, g4run.h:73-77),
// quantized to q8_0 for the down projection; one workgroup per 256 elements.
__global__ __launch_bounds__(256) void k_gelu_quant(const float *gu, int n_ff, const uint16_t *gelu_tab, uint8_t *act) {
    __shared__ float buf[256];
    const int i0 = blockIdx.x * 256, t = threadIdx.x;
    const int i = i0 + t;
    if (i < n_ff) {
        const float g = gu[i], u = gu[n_ff + i];
        float gg;
        if (g <= -10.0f) gg = 0.0f;
        else if (g >= 10.0f) gg = g;
        else gg = h2f(gelu_tab[f2h(g)]);
        buf[t] = gg * u;
    }
    __syncthreads();
    quantize_q8_0_lds(buf, min(256, n_ff - i0), act + (size_t)(i0 / 32) * 34);
}

// ---------------------------------------------------- argmax + advance --
// First index of the maximum (sampler.c:139-144); then token <- argmax,
// pos <- pos + 1, npos <- pos + 2 for the next step.
__global__ __launch_bounds__(1024) void k_argmax_advance(const float *logits, int n, int *token, int *pos, int *npos,
                                                         int advance) {
    __shared__ float bv[1024];
    __shared__ int bi[1024];
    const int t = threadIdx.x;
    float best = -INFINITY;
    int idx = 0x7fffffff;
    for (int i = t; i < n; i += blockDim.x) {
        const float v = logits[i];
        if (v > best) { best = v; idx = i; }
    }
    bv[t] = best; bi[t] = idx;
    __syncthreads();
    for (int k = blockDim.x >> 1; k >= 1; k >>= 1) {
        if (t < k) {
            const float ov = bv[t + k];
            const int oi = bi[t + k];
            if (ov > bv[t] || (ov == bv[t] && oi < bi[t])) { bv[t] = ov; bi[t] = oi; }
        }
        __syncthreads();
    }
    if (t == 0) {
        *token = bi[0] == 0x7fffffff ? 0 : bi[0];
        if (advance) { *pos += 1; *npos = *pos + 1; }
    }
}

// ------------------------------------------------------------ launchers --
hipError_t launch_rand_normal(float *y, int64_t n, uint64_t seed, float mean, float std, hipStream_t s) {
    hipLaunchKernelGGL(k_rand_normal, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, y, n, seed, mean, std);
    return hipGetLastError();
}
hipError_t launch_embed_planes(const g4h_tensor &head, const int *token, float *x, float es, hipStream_t s) {
    if (head.type != Q8_0) return hipErrorInvalidValue;
    hipLaunchKernelGGL(k_embed_planes, dim3(1), dim3(256), 0, s, (const int8_t *)head.qs, (const uint16_t *)head.sc, head.nb,
                       token, x, (int)head.ncols, es);
    return hipGetLastError();
}
hipError_t launch_norm_quant(float *x, const float *delta, const float *w_post, const float *w_pre, float eps, int n,
                             uint8_t *act, float *xb_out, hipStream_t s) {
    if (n % 32 || n > 4096) return hipErrorInvalidValue;
    const int threads = ((n / 4 + 63) / 64) * 64;
    hipLaunchKernelGGL(k_norm_quant, dim3(1), dim3(threads), 0, s, x, delta, w_post, w_pre, eps, n, act, xb_out);
    return hipGetLastError();
}
hipError_t launch_qkv_prep(const float *qkv, int n_head, int n_kv, int hd, const float *q_norm, const float *k_norm, float eps,
                           const float *rope, const int *pos, float *q_out, uint8_t *kc, uint8_t *vc, int kv_type, hipStream_t s) {
    hipLaunchKernelGGL(k_qkv_prep, dim3(n_head + 2 * n_kv), dim3(256), 0, s, qkv, n_head, n_kv, hd, q_norm, k_norm, eps, rope,
                       pos, q_out, kc, vc, kv_type);
    return hipGetLastError();
}
hipError_t launch_gelu_quant(const float *gu, int n_ff, const uint16_t *tab, uint8_t *act, hipStream_t s) {
    hipLaunchKernelGGL(k_gelu_quant, dim3((n_ff + 255) / 256), dim3(256), 0, s, gu, n_ff, tab, act);
    return hipGetLastError();
}
hipError_t launch_argmax_advance(const float *logits, int n, int *token, int *pos, int *npos, int advance, hipStream_t s) {
    hipLaunchKernelGGL(k_argmax_advance, dim3(1), dim3(1024), 0, s, logits, n, token, pos, npos, advance);
    return hipGetLastError();
}

}  // namespace g4
