// k_gemma.hip -- the elementwise and per-row steps of the gemma4 forward
// (model.c:592-799) between its matmuls: RMSNorm rows and residual adds, the
// per-layer embedding preparation and injection, the query preparation of
// layers that read a shared KV cache, GELU * up, the packing of separate
// q / k / v projections and the final soft-cap.  One token row per
// workgroup (grid.y or grid.x = token); the arithmetic is model.c's:
// rms_norm with the sum of squares in double, scale = 1/sqrtf(mean + eps)
// with the mean rounded to float, y = x*scale*w left to right
// (model.c:337-345); RoPE as rope_apply (model.c:359-367) from a table of the
// rope_cache values (model.c:349-357).
#include "kernels.h"
#include "steps.h"

namespace g4 {

namespace {

// scale = 1/sqrt(mean(x^2) + eps) of one row of n floats (256 threads),
// eight loads in flight per thread
__device__ float row_rms_scale(const float *x, int n, float eps, double *red) {
    double ss = 0.0;
#pragma unroll 8
    for (int i = threadIdx.x; i < n; i += blockDim.x) ss += (double)x[i] * x[i];
    return rms_scale(wg_sum_double(ss, red), n, eps);
}

// y = rms(x) * w (w may be null); rows at stride n (blockIdx.x = token).
// K > 0: row elements t + 256 k (k < K) held in registers, every load issued
// first (n <= 256 K); K = 0: any n.
template <int K>
__global__ __launch_bounds__(256) void k_rms_rows(const float *x, const float *w, float *y, int n, float eps) {
    __shared__ double red[4];
    const size_t b = blockIdx.x;
    x += b * n;
    y += b * n;
    if constexpr (K == 0) {
        const float sc = row_rms_scale(x, n, eps, red);
#pragma unroll 8
        for (int i = threadIdx.x; i < n; i += blockDim.x) y[i] = w ? x[i] * sc * w[i] : x[i] * sc;
    } else {
        float xv[K], wv[K];
        double ss = 0.0;
#pragma unroll
        for (int k = 0; k < K; k++) {
            const int i = threadIdx.x + 256 * k;
            xv[k] = i < n ? x[i] : 0.0f;
            wv[k] = i < n && w ? w[i] : 1.0f;
        }
#pragma unroll
        for (int k = 0; k < K; k++) ss += (double)xv[k] * xv[k];
        const float sc = rms_scale(wg_sum_double(ss, red), n, eps);
#pragma unroll
        for (int k = 0; k < K; k++) {
            const int i = threadIdx.x + 256 * k;
            if (i < n) y[i] = w ? xv[k] * sc * wv[k] : xv[k] * sc;
        }
    }
}

// x = (x + rms(d) * w) * os (model.c:711-716, 731-736 with os = 1; 748-751);
// then, with w2 (the next RMSNorm, model.c:695, 718), y = rms(x) * w2 -- the
// arithmetic of k_resid followed by k_rms_rows, in one launch.  y may be d.
template <int K>
__global__ __launch_bounds__(256) void k_resid(float *x, const float *d, const float *w, int n, float eps, float os,
                                               const float *w2, float *y) {
    __shared__ double red[4];
    const size_t b = blockIdx.x;
    x += b * n;
    d += b * n;
    if constexpr (K == 0) {
        const float sc = row_rms_scale(d, n, eps, red);
#pragma unroll 8
        for (int i = threadIdx.x; i < n; i += blockDim.x) x[i] = (x[i] + d[i] * sc * w[i]) * os;
    } else {
        float xv[K], dv[K], wv[K], w2v[K];
#pragma unroll
        for (int k = 0; k < K; k++) {
            const int i = threadIdx.x + 256 * k;
            const bool in = i < n;
            dv[k] = in ? d[i] : 0.0f;
            xv[k] = in ? x[i] : 0.0f;
            wv[k] = in ? w[i] : 0.0f;
            w2v[k] = in && w2 ? w2[i] : 1.0f;
        }
        double ss = 0.0;
#pragma unroll
        for (int k = 0; k < K; k++) ss += (double)dv[k] * dv[k];
        const float sc = rms_scale(wg_sum_double(ss, red), n, eps);
        double s2 = 0.0;
#pragma unroll
        for (int k = 0; k < K; k++) {
            const int i = threadIdx.x + 256 * k;
            if (i < n) {
                xv[k] = (xv[k] + dv[k] * sc * wv[k]) * os;
                x[i] = xv[k];
            }
            s2 += (double)xv[k] * xv[k];                               // 0 past n
        }
        if (y) {                                                       // uniform
            const float sc2 = rms_scale(wg_sum_double(s2, red), n, eps);
            y += b * n;
#pragma unroll
            for (int k = 0; k < K; k++) {
                const int i = threadIdx.x + 256 * k;
                if (i < n) y[i] = xv[k] * sc2 * w2v[k];
            }
        }
    }
}

// y = y * s over nb rows of n (the embedding scales, model.c:609-614)
__global__ __launch_bounds__(256) void k_scale(float *y, int64_t n, float s) {
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (i < n) y[i] = y[i] * s;
}

// per-layer inputs (model.c:617-635): pp = plp * ps, pp = rms(pp) * w,
// pl = (pp + pl) * is2, for layer blockIdx.x of token blockIdx.y; rows of
// n_layer * pe floats
__global__ __launch_bounds__(256) void k_ple_prep(const float *plp, float *pl, const float *w, int pe, int n_layer, float ps,
                                                  float is2, float eps) {
    __shared__ double red[4];
    __shared__ float pp[1024];
    const size_t off = ((size_t)blockIdx.y * n_layer + blockIdx.x) * pe;
    for (int i = threadIdx.x; i < pe; i += blockDim.x) pp[i] = plp[off + i] * ps;
    __syncthreads();
    const float sc = row_rms_scale(pp, pe, eps, red);
    for (int i = threadIdx.x; i < pe; i += blockDim.x) pl[off + i] = (pp[i] * sc * w[i] + pl[off + i]) * is2;
}

// g = gelu(g) * u (model.c:725-729, 740-744: the fp16 GELU table); rows of n
// at stride gs (g) / us (u) floats, grid.y = token
__global__ __launch_bounds__(256) void k_gelu_mul(float *g, size_t gs, const float *u, size_t us, int n, const uint16_t *tab) {
    const int i = blockIdx.x * 256 + threadIdx.x;
    if (i >= n) return;
    g += blockIdx.y * gs;
    u += blockIdx.y * us;
    g[i] = gelu_lut(tab, g[i]) * u[i];
}

// queries of a layer without its own K/V (model.c:666-672): every head of
// token blockIdx.y (blockIdx.x = head): q = rope(rms(q) * w) at position
// pos0 + token, in place; rows of n_head * hd floats; rope table rows of hd
// (cos, sin pairs)
__global__ __launch_bounds__(256) void k_head_prep(float *q, int n_head, int hd, const float *w, const float *rope, int pos0,
                                                   float eps, const int *pos_dev) {
    if (pos_dev) pos0 = *pos_dev;
    __shared__ double red[4];
    __shared__ float y[512];
    float *x = q + ((size_t)blockIdx.y * n_head + blockIdx.x) * hd;
    const float sc = row_rms_scale(x, hd, eps, red);
    for (int i = threadIdx.x; i < hd; i += blockDim.x) y[i] = x[i] * sc * w[i];
    __syncthreads();
    const float *cs = rope + (size_t)(pos0 + blockIdx.y) * hd;
    const int h = hd / 2;
    for (int i = threadIdx.x; i < h; i += blockDim.x) {
        const float c = cs[2 * i], s = cs[2 * i + 1], a = y[i], bb = y[i + h];
        x[i] = a * c - bb * s;
        x[i + h] = a * s + bb * c;
    }
}

// one row q | k | v of the attention's fused input per token from separate
// projections (v = k when vsrc is null: model.c:678, V = K before its norm)
__global__ __launch_bounds__(256) void k_pack_qkv(const float *q, const float *k, const float *v, float *qkv, int nq, int hd) {
    const size_t b = blockIdx.x;
    float *dst = qkv + b * (nq + 2 * hd);
    for (int i = threadIdx.x; i < nq; i += blockDim.x) dst[i] = q[b * nq + i];
    for (int i = threadIdx.x; i < hd; i += blockDim.x) {
        dst[nq + i] = k[b * hd + i];
        dst[nq + hd + i] = v ? v[b * hd + i] : k[b * hd + i];
    }
}

// logits = cap * tanh(logits / cap) (model.c:794-797)
__global__ __launch_bounds__(256) void k_softcap(float *l, int64_t n, float cap) {
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (i < n) l[i] = cap * tanhf(l[i] / cap);
}

unsigned blocks(int64_t n) { return (unsigned)((n + 255) / 256); }

}  // namespace

// elements per thread held in registers for a row of n (0: the loop form)
static int row_regs(int n) { return n <= 512 ? 2 : n <= 1024 ? 4 : n <= 2048 ? 8 : n <= 4096 ? 16 : n <= 6144 ? 24 : 0; }
hipError_t launch_rms_rows(const float *x, const float *w, float *y, int n, int nb, float eps, hipStream_t s) {
    switch (row_regs(n)) {
    case 2: hipLaunchKernelGGL(k_rms_rows<2>, dim3(nb), dim3(256), 0, s, x, w, y, n, eps); break;
    case 4: hipLaunchKernelGGL(k_rms_rows<4>, dim3(nb), dim3(256), 0, s, x, w, y, n, eps); break;
    case 8: hipLaunchKernelGGL(k_rms_rows<8>, dim3(nb), dim3(256), 0, s, x, w, y, n, eps); break;
    case 16: hipLaunchKernelGGL(k_rms_rows<16>, dim3(nb), dim3(256), 0, s, x, w, y, n, eps); break;
    case 24: hipLaunchKernelGGL(k_rms_rows<24>, dim3(nb), dim3(256), 0, s, x, w, y, n, eps); break;
    default: hipLaunchKernelGGL(k_rms_rows<0>, dim3(nb), dim3(256), 0, s, x, w, y, n, eps); break;
    }
    return hipGetLastError();
}
hipError_t launch_resid(float *x, const float *d, const float *w, int n, int nb, float eps, float os, hipStream_t s,
                        const float *w2, float *y) {
    if ((w2 == nullptr) != (y == nullptr)) return hipErrorInvalidValue;
    switch (row_regs(n)) {
    case 2: hipLaunchKernelGGL(k_resid<2>, dim3(nb), dim3(256), 0, s, x, d, w, n, eps, os, w2, y); break;
    case 4: hipLaunchKernelGGL(k_resid<4>, dim3(nb), dim3(256), 0, s, x, d, w, n, eps, os, w2, y); break;
    case 8: hipLaunchKernelGGL(k_resid<8>, dim3(nb), dim3(256), 0, s, x, d, w, n, eps, os, w2, y); break;
    case 16: hipLaunchKernelGGL(k_resid<16>, dim3(nb), dim3(256), 0, s, x, d, w, n, eps, os, w2, y); break;
    case 24: hipLaunchKernelGGL(k_resid<24>, dim3(nb), dim3(256), 0, s, x, d, w, n, eps, os, w2, y); break;
    default:                                                           // two launches
        hipLaunchKernelGGL(k_resid<0>, dim3(nb), dim3(256), 0, s, x, d, w, n, eps, os, nullptr, nullptr);
        if (y) hipLaunchKernelGGL(k_rms_rows<0>, dim3(nb), dim3(256), 0, s, x, w2, y, n, eps);
        break;
    }
    return hipGetLastError();
}
hipError_t launch_scale(float *y, int64_t n, float sc, hipStream_t s) {
    hipLaunchKernelGGL(k_scale, dim3(blocks(n)), dim3(256), 0, s, y, n, sc);
    return hipGetLastError();
}
hipError_t launch_ple_prep(const float *plp, float *pl, const float *w, int pe, int n_layer, int nb, float ps, float is2,
                           float eps, hipStream_t s) {
    if (pe > 1024) return hipErrorInvalidValue;
    hipLaunchKernelGGL(k_ple_prep, dim3(n_layer, nb), dim3(256), 0, s, plp, pl, w, pe, n_layer, ps, is2, eps);
    return hipGetLastError();
}
hipError_t launch_gelu_mul(float *g, size_t gs, const float *u, size_t us, int n, int nb, const uint16_t *tab, hipStream_t s) {
    hipLaunchKernelGGL(k_gelu_mul, dim3(blocks(n), nb), dim3(256), 0, s, g, gs, u, us, n, tab);
    return hipGetLastError();
}
hipError_t launch_head_prep(float *q, int n_head, int hd, int nb, const float *w, const float *rope, int pos0, float eps,
                            hipStream_t s, const int *pos_dev) {
    if (hd > 512 || hd % 2) return hipErrorInvalidValue;
    hipLaunchKernelGGL(k_head_prep, dim3(n_head, nb), dim3(256), 0, s, q, n_head, hd, w, rope, pos0, eps, pos_dev);
    return hipGetLastError();
}
hipError_t launch_pack_qkv(const float *q, const float *k, const float *v, float *qkv, int nq, int hd, int nb, hipStream_t s) {
    hipLaunchKernelGGL(k_pack_qkv, dim3(nb), dim3(256), 0, s, q, k, v, qkv, nq, hd);
    return hipGetLastError();
}
hipError_t launch_softcap(float *l, int64_t n, float cap, hipStream_t s) {
    hipLaunchKernelGGL(k_softcap, dim3(blocks(n)), dim3(256), 0, s, l, n, cap);
    return hipGetLastError();
}

}  // namespace g4
