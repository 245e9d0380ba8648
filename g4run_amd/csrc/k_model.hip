// k_model.hip -- the decode step's kernels between the GEMVs (model.c:593-775
// for a gemma-style decoder) and device-side random init.  The arithmetic of
// the norm / RoPE / quantizer steps is in steps.h.
//
// Every kernel reads the position / token from device memory so that one
// decode step can be captured once and replayed.  GELU is the fp16 lookup
// table (g4run.h:73-77); argmax keeps the first maximum (sampler.c:139-144).
#include "kernels.h"
#include "steps.h"

namespace g4 {

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
// x = dequant(row `token` of the tied q8_0 head) * sqrt(n_embd) (model.c:605-612),
// read from the resident planes (quants 0..15 of each block in lo, 16..31 in
// hi, d fp16); then
// act = q8_0(rms(x)*w_pre), the first layer's attention-norm activation
// (skipped without w_pre, when that norm runs in the Wqkv GEMV).  512 threads,
// n <= 8192; workgroup b takes token[b] into x + b*n and act + b*ast.
__global__ __launch_bounds__(512) void k_embed_norm(const int8_t *lo, const int8_t *hi, const uint16_t *sc, int64_t nb, const int *token,
                                                    float *x, int n, float es, const float *w_pre, float eps, uint8_t *act,
                                                    size_t ast, FewAct few) {
    const int b = blockIdx.x;
    const int64_t r = token[b];
    x += (size_t)b * n;
    for (int i = threadIdx.x; i < n; i += blockDim.x) {
        const int64_t j = r * nb + (i >> 5);
        const int e = i & 31;
        const float v = (float)(e < 16 ? lo : hi)[j * 16 + (e & 15)] * h2f(sc[j]);
        x[i] = v * es;
    }
    __syncthreads();
    if (w_pre) wg_norm_quant<4>(x, nullptr, nullptr, w_pre, eps, n, act + (size_t)b * ast, nullptr, few, b);
}

// ------------------------------------------------------ norm + quantize --
// One workgroup of 512 threads per token row b (n <= 8192, n % 32 == 0): if
// delta, x += rms(delta)*w_post (the post-norm residual, model.c:711-716 /
// 731-736); then act = q8_0(rms(x)*w_pre), the next projection's activation
// (model.c:657-661 / 721-722), and y = rms(x)*w_pre in fp32 if y is given
// (the head's input feature, model.c:791-793).  Rows at n floats; act rows at
// ast bytes.
__global__ __launch_bounds__(512) void k_norm_quant(float *x, const float *delta, const float *w_post, const float *w_pre,
                                                    float eps, int n, uint8_t *act, size_t ast, float *y, FewAct few) {
    const size_t b = blockIdx.x;
    wg_norm_quant<4>(x + b * n, delta ? delta + b * n : nullptr, w_post, w_pre, eps, n, act + b * ast, y ? y + b * n : nullptr,
                     few, (int)b);
}

// -------------------------------------------------------- gelu * up --
// h = gelu(g) * u with the fp16 GELU table (model.c:725-729), quantized to
// q8_0 for the down projection; gu holds the (gate, up) pairs interleaved,
// as the Wgu rows are stored.  256 threads, 4 elements each; grid.y token
// rows (gu rows of 2 n_ff floats, act rows at ast bytes, or few's layout).
__global__ __launch_bounds__(256) void k_gelu_quant(const float *gu, int n_ff, const uint16_t *tab, uint8_t *act, size_t ast,
                                                    float *hout, size_t hs, FewAct few) {
    const int gi = blockIdx.x * 256 + threadIdx.x;
    gu += (size_t)blockIdx.y * 2 * n_ff;             // token row blockIdx.y
    act += (size_t)blockIdx.y * ast;
    const bool own = 4 * gi < n_ff;
    float g[4] = {0.f, 0.f, 0.f, 0.f}, u[4] = {0.f, 0.f, 0.f, 0.f}, h[4];
    if (own) {
        float a[4], b[4];
        f4(ldf4(gu + 8 * gi), a);
        f4(ldf4(gu + 8 * gi + 4), b);
        g[0] = a[0]; u[0] = a[1]; g[1] = a[2]; u[1] = a[3];
        g[2] = b[0]; u[2] = b[1]; g[3] = b[2]; u[3] = b[3];
    }
#pragma unroll
    for (int k = 0; k < 4; k++) {
        float gg;
        if (g[k] <= -10.0f) gg = 0.0f;
        else if (g[k] >= 10.0f) gg = g[k];
        else gg = h2f(tab[f2h(g[k])]);
        h[k] = gg * u[k];
    }
    if (hout && own) *(float4 *)(hout + (size_t)blockIdx.y * hs + 4 * gi) = make_float4(h[0], h[1], h[2], h[3]);
    act_store4(h, gi, own, act, few, blockIdx.y);
}

// ---------------------------------------------------- argmax + advance --
// token <- the first index of the maximum (wg_first_argmax), then the
// position advances (state_advance).
__global__ __launch_bounds__(1024) void k_argmax_advance(const float *logits, int n, int *state, int n_ctx) {
    __shared__ float bv[16];
    __shared__ int bi[16];
    const int id = wg_first_argmax(logits, n, bv, bi);
    if (threadIdx.x == 0) state_advance(state, id, n_ctx);
}

// out[b] = the first index of the maximum of row b (main.c:348-349's ARGMAX
// over each verified position); one workgroup per row of n floats.
__global__ __launch_bounds__(1024) void k_argmax_rows(const float *logits, int n, int *out) {
    __shared__ float bv[16];
    __shared__ int bi[16];
    const int id = wg_first_argmax(logits + (size_t)blockIdx.x * n, n, bv, bi);
    if (threadIdx.x == 0) out[blockIdx.x] = id;
}

// ------------------------------------------------------------ launchers --
hipError_t launch_rand_normal(float *y, int64_t n, uint64_t seed, float mean, float std, hipStream_t s) {
    hipLaunchKernelGGL(k_rand_normal, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, y, n, seed, mean, std);
    return hipGetLastError();
}
hipError_t launch_embed_norm(const g4h_tensor &head, const int *token, float *x, float es, const float *w_pre, float eps,
                             uint8_t *act, hipStream_t s, int nb, size_t ast, const FewAct &few) {
    if (head.type != Q8_0 || head.ncols % 32 || head.ncols > 8192 || nb < 1 || (few.qa && nb > 16 * few.mt))
        return hipErrorInvalidValue;
    hipLaunchKernelGGL(k_embed_norm, dim3(nb), dim3(512), 0, s, (const int8_t *)head.qs, (const int8_t *)head.ex,
                       (const uint16_t *)head.sc, head.nb,
                       token, x, (int)head.ncols, es, w_pre, eps, act, ast, few);
    return hipGetLastError();
}
hipError_t launch_norm_quant(float *x, const float *delta, const float *w_post, const float *w_pre, float eps, int n,
                             uint8_t *act, hipStream_t s, int nb, size_t ast, float *y, const FewAct &few) {
    if (n % 32 || n > 8192 || nb < 1 || (few.qa && nb > 16 * few.mt)) return hipErrorInvalidValue;
    hipLaunchKernelGGL(k_norm_quant, dim3(nb), dim3(512), 0, s, x, delta, w_post, w_pre, eps, n, act, ast, y, few);
    return hipGetLastError();
}
hipError_t launch_gelu_quant(const float *gu, int n_ff, const uint16_t *tab, uint8_t *act, hipStream_t s, int nb, size_t ast,
                             float *hout, size_t hs, const FewAct &few) {
    if (n_ff % 32 || nb < 1 || (hout && ((uintptr_t)hout % 16 || hs % 4)) || (few.qa && nb > 16 * few.mt))
        return hipErrorInvalidValue;
    hipLaunchKernelGGL(k_gelu_quant, dim3((n_ff / 4 + 255) / 256, nb), dim3(256), 0, s, gu, n_ff, tab, act, ast, hout, hs, few);
    return hipGetLastError();
}
hipError_t launch_argmax_rows(const float *logits, int n, int nb, int *out, hipStream_t s) {
    if (n < 1 || nb < 1 || ((uintptr_t)logits & 15) || (nb > 1 && n % 4)) return hipErrorInvalidValue;
    hipLaunchKernelGGL(k_argmax_rows, dim3(nb), dim3(1024), 0, s, logits, n, out);
    return hipGetLastError();
}
hipError_t launch_argmax_advance(const float *logits, int n, int *state, int n_ctx, hipStream_t s) {
    hipLaunchKernelGGL(k_argmax_advance, dim3(1), dim3(1024), 0, s, logits, n, state, n_ctx);
    return hipGetLastError();
}

}  // namespace g4
