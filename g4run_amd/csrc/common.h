// common.h -- device helpers and the resident-tensor description shared by the
// gfx950 kernels of the quantized weight x activation path.
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

namespace g4 {

enum : int { F32 = 0, F16 = 1, Q4_0 = 2, Q8_0 = 8, Q2_K = 10, Q3_K = 11, Q4_K = 12, Q8_K = 15 };

constexpr int WAVE = 64;

// GGUF block geometry (g4run.h:107-118, gguf.c:11-25)
__host__ __device__ constexpr int blck(int t) {
    return (t == Q4_0 || t == Q8_0) ? 32 : (t == Q2_K || t == Q3_K || t == Q4_K || t == Q8_K) ? 256 : (t == F32 || t == F16) ? 1 : 0;
}
__host__ __device__ constexpr int bsize(int t) {
    return t == Q4_0 ? 18 : t == Q8_0 ? 34 : t == Q2_K ? 84 : t == Q3_K ? 110 : t == Q4_K ? 144 : t == Q8_K ? 292 : t == F16 ? 2 : t == F32 ? 4 : 0;
}

// ---------------------------------------------------------------- fp16 ----
// v_cvt_f32_f16 / v_cvt_f16_f32: exact widening and round-to-nearest-even
// narrowing; fp16 denormals are kept (gfx9 default FP16 denorm mode), which
// matters because about 30% of the synthetic q8_0 weight scales are subnormal.
// The fp32 operand is made opaque first: otherwise the backend folds a
// preceding multiply into v_fma_mix*_f16, which rounds the exact product to
// fp16 once instead of rounding to fp32 and then to fp16 as the reference's
// g4_fp32_to_fp16(x*y) does (and differs from it at fp16 rounding ties).
__device__ __forceinline__ float opaque(float f) {
    asm volatile("" : "+v"(f));
    return f;
}
__device__ __forceinline__ float h2f(uint16_t h) { return (float)__builtin_bit_cast(_Float16, h); }
__device__ __forceinline__ uint16_t f2h(float f) { return __builtin_bit_cast(uint16_t, (_Float16)opaque(f)); }

__device__ __forceinline__ int dot4(int a, int b, int c) { return __builtin_amdgcn_sdot4(a, b, c, false); }

// Round-half-even of the exact product a*b (valid for |a*b| < 2^22): the fused
// form the reference build gives nearest_int(a*b) (quants.c:63-67,164).
__device__ __forceinline__ int rne_prod(float a, float b) {
    float t = __builtin_fmaf(a, b, 12582912.0f);
    return (int)(__builtin_bit_cast(uint32_t, t) & 0x007fffffu) - 0x00400000;
}

template <typename T>
__device__ __forceinline__ T shfl_xor(T v, int m) { return __shfl_xor(v, m, WAVE); }

// wave-wide sum over groups of G lanes (G a power of two <= 64), fixed order
template <int G>
__device__ __forceinline__ float group_sum(float v) {
#pragma unroll
    for (int m = G / 2; m >= 1; m >>= 1) v += shfl_xor(v, m);
    return v;
}
template <int G>
__device__ __forceinline__ int group_isum(int v) {
#pragma unroll
    for (int m = G / 2; m >= 1; m >>= 1) v += shfl_xor(v, m);
    return v;
}

__device__ __forceinline__ int4 ld4(const void *p) { return *reinterpret_cast<const int4 *>(p); }

// 128-bit load of a stream that is read once per call (weight quants): the
// non-temporal hint keeps those lines from displacing reused data (activations,
// scales) in the caches.  -DG4_LD_PLAIN builds the plain form for comparison.
typedef int g4_v4i __attribute__((ext_vector_type(4)));
__device__ __forceinline__ int4 ld4s(const void *p) {
#ifdef G4_LD_PLAIN
    return ld4(p);
#else
    const g4_v4i v = __builtin_nontemporal_load(reinterpret_cast<const g4_v4i *>(p));
    return make_int4(v.x, v.y, v.z, v.w);
#endif
}

// Workgroup barrier for LDS hand-offs only.  __syncthreads() also waits for
// every outstanding global load of the calling wave (vmcnt(0)); a wave whose
// weight stream is in flight would stall there until the whole stream has
// landed.  This one waits for the wave's LDS and scalar traffic (lgkmcnt) and
// meets the other waves, so global loads stay in flight across it.  Only LDS
// data may be handed between waves through it.
__device__ __forceinline__ void lds_barrier() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }

// Keeps the loads issued before it ahead of those after it: global loads
// complete in issue order, so a small load that must be waited for early
// (activations) has to be issued before the weight stream.
__device__ __forceinline__ void issue_order() {
    asm volatile("" ::: "memory");
    __builtin_amdgcn_sched_barrier(0);
}

}  // namespace g4

// Resident weight matrix (the object behind the C ABI's g4h_tensor).
// Layout per type, per row r and per (super)block j, with nb blocks per row:
//   q8_0: qs plane  [r][j][32] int8          sc plane [r][j] fp16 d
//   q4_0: qs plane  [r][j][16] nibbles       sc plane [r][j] fp16 d
//   q4_K: qs plane  [r][j][144] the GGUF block unchanged (16-B header + qs)
//   q2_K: qs plane  [r][j][64] 2-bit quants  sc plane [r][j][16] scale|min
//         ex plane  [r][j] {fp16 d, fp16 dmin}
//   q3_K: qs plane  [r][j][64] low bits + [r][j][32] hmask in ex plane,
//         sc plane  [r][j][12] packed 6-bit scales, d plane [r][j] fp16
// Every plane starts 256-B aligned; quant rows are 16-B multiples so every
// quant load is an aligned 128-bit load.
struct g4h_tensor {
    int type;
    int64_t ncols, nrows, nb;   // nb = (super)blocks per row
    uint8_t *base;              // single allocation
    size_t bytes;
    uint8_t *qs;                // quant plane
    uint8_t *sc;                // scale plane (q8_0/q4_0: fp16 d; q2_K/q3_K: packed scales)
    uint8_t *ex;                // q2_K: {d,dmin}; q3_K: hmask
    uint8_t *dd;                // q3_K: fp16 d
};
