// common.h -- device helpers and the resident-tensor description shared by the
// gfx950 kernels of the quantized weight x activation path.
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

namespace g4 {

enum : int { F32 = 0, F16 = 1, Q4_0 = 2, Q8_0 = 8, Q2_K = 10, Q3_K = 11, Q4_K = 12, Q5_K = 13, Q6_K = 14, Q8_K = 15, BF16 = 30, TQ2_0 = 35 };

constexpr int WAVE = 64;

// GGUF block geometry (g4run.h:107-118, gguf.c:11-25)
__host__ __device__ constexpr int blck(int t) {
    return (t == Q4_0 || t == Q8_0) ? 32 : (t == Q2_K || t == Q3_K || t == Q4_K || t == Q5_K || t == Q6_K || t == Q8_K || t == TQ2_0) ? 256
         : (t == F32 || t == F16 || t == BF16) ? 1 : 0;
}
__host__ __device__ constexpr int bsize(int t) {
    return t == Q4_0 ? 18 : t == Q8_0 ? 34 : t == Q2_K ? 84 : t == Q3_K ? 110 : t == Q4_K ? 144 : t == Q5_K ? 176 : t == Q6_K ? 210 : t == Q8_K ? 292 : t == TQ2_0 ? 66
         : (t == F16 || t == BF16) ? 2 : t == F32 ? 4 : 0;
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

// gelu(x) through the fp16 table of quants.c:49-58 (g4run.h:73-77): 0 for
// x <= -10, x for x >= 10, else the table entry of fp16(x)
__device__ __forceinline__ float gelu_lut(const uint16_t *tab, float x) {
    if (x <= -10.0f) return 0.0f;
    if (x >= 10.0f) return x;
    return h2f(tab[f2h(x)]);
}

__device__ __forceinline__ int dot4(int a, int b, int c) { return __builtin_amdgcn_sdot4(a, b, c, false); }

// Round-half-even of the exact product a*b (valid for |a*b| < 2^22): the fused
// form the reference build gives nearest_int(a*b) (quants.c:63-67,164).
__device__ __forceinline__ int rne_prod(float a, float b) {
    float t = __builtin_fmaf(a, b, 12582912.0f);
    return (int)(__builtin_bit_cast(uint32_t, t) & 0x007fffffu) - 0x00400000;
}

template <typename T>
__device__ __forceinline__ T shfl_xor(T v, int m) { return __shfl_xor(v, m, WAVE); }

// ------------------------------------------------------ lane exchanges ----
// partner<M>(v): the value of a lane in the other half of the caller's
// aligned group of 2M lanes, on the VALU (no LDS round trip): M = 1, 2 are
// quad_perm DPP (lane ^ M), M = 4, 8 the row half-mirror / mirror DPP (lane i
// of an 8- or 16-lane group meets lane 7 - i / 15 - i), M = 16, 32 gfx950's
// v_permlane16_swap / v_permlane32_swap (lane ^ M).  A butterfly over
// M = 1, 2, 4, ... therefore adds, at every step, the sums of the same two
// aligned lane groups as the xor butterfly, and every lane of a group ends
// with the same bits.
template <int M>
__device__ __forceinline__ uint32_t partner_u32(uint32_t v) {
    if constexpr (M == 1) return (uint32_t)__builtin_amdgcn_mov_dpp((int)v, 0xB1, 0xF, 0xF, false);
    else if constexpr (M == 2) return (uint32_t)__builtin_amdgcn_mov_dpp((int)v, 0x4E, 0xF, 0xF, false);
    else if constexpr (M == 4) return (uint32_t)__builtin_amdgcn_mov_dpp((int)v, 0x141, 0xF, 0xF, false);
    else if constexpr (M == 8) return (uint32_t)__builtin_amdgcn_mov_dpp((int)v, 0x140, 0xF, 0xF, false);
    else if constexpr (M == 16) {
        const auto r = __builtin_amdgcn_permlane16_swap(v, v, false, false);
        return ((threadIdx.x >> 4) & 1) ? r[0] : r[1];
    } else {
        static_assert(M == 32, "partner<M>: M is a power of two up to 32");
        const auto r = __builtin_amdgcn_permlane32_swap(v, v, false, false);
        return (threadIdx.x & 32) ? r[0] : r[1];
    }
}
// Unsigned maximum over the wave, returned as a wave-uniform value: four
// exchanges within each 16-lane row, then the broadcasts of lane 15 into rows
// 1 and 3 and of lane 31 into rows 2 and 3, after which lane 63 holds the
// maximum.  For non-negative floats the bit patterns order as the values, so
// this is also their maximum (no NaN canonicalisation per step).
__device__ __forceinline__ uint32_t wave_umax(uint32_t u) {
    u = max(u, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)u, 0xB1, 0xF, 0xF, false));    // quad_perm [1,0,3,2]
    u = max(u, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)u, 0x4E, 0xF, 0xF, false));    // quad_perm [2,3,0,1]
    u = max(u, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)u, 0x141, 0xF, 0xF, false));   // row_half_mirror
    u = max(u, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)u, 0x140, 0xF, 0xF, false));   // row_mirror
    u = max(u, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)u, 0x142, 0xA, 0xF, false));   // row_bcast:15
    u = max(u, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)u, 0x143, 0xC, 0xF, false));   // row_bcast:31
    return (uint32_t)__builtin_amdgcn_readlane((int)u, 63);
}

// exactly lane ^ 8 (DPP row_ror:8), for exchanges between lanes that hold
// different quantities (partner<8> pairs lane i with 15 - i)
__device__ __forceinline__ float xor8(float v) {
    return __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), 0x128, 0xF, 0xF, false));
}
template <int M>
__device__ __forceinline__ float partner(float v) { return __builtin_bit_cast(float, partner_u32<M>(__builtin_bit_cast(uint32_t, v))); }
template <int M>
__device__ __forceinline__ int partner(int v) { return (int)partner_u32<M>((uint32_t)v); }
template <int M>
__device__ __forceinline__ uint32_t partner(uint32_t v) { return partner_u32<M>(v); }
template <int M>
__device__ __forceinline__ double partner(double v) {
    const uint64_t u = __builtin_bit_cast(uint64_t, v);
    const uint64_t lo = partner_u32<M>((uint32_t)u), hi = partner_u32<M>((uint32_t)(u >> 32));
    return __builtin_bit_cast(double, lo | (hi << 32));
}

// sums / maxima over aligned groups of G lanes (G a power of two <= 64),
// in the fixed butterfly order M = 1, 2, 4, ...; every lane gets the result
template <int G, typename T>
__device__ __forceinline__ T group_sum_t(T v) {
    if constexpr (G >= 2) v += partner<1>(v);
    if constexpr (G >= 4) v += partner<2>(v);
    if constexpr (G >= 8) v += partner<4>(v);
    if constexpr (G >= 16) v += partner<8>(v);
    if constexpr (G >= 32) v += partner<16>(v);
    if constexpr (G >= 64) v += partner<32>(v);
    return v;
}
template <int G>
__device__ __forceinline__ float group_sum(float v) { return group_sum_t<G>(v); }
template <int G>
__device__ __forceinline__ int group_isum(int v) { return group_sum_t<G>(v); }
template <int G>
__device__ __forceinline__ float group_max(float v) {
    if constexpr (G >= 2) v = fmaxf(v, partner<1>(v));
    if constexpr (G >= 4) v = fmaxf(v, partner<2>(v));
    if constexpr (G >= 8) v = fmaxf(v, partner<4>(v));
    if constexpr (G >= 16) v = fmaxf(v, partner<8>(v));
    if constexpr (G >= 32) v = fmaxf(v, partner<16>(v));
    if constexpr (G >= 64) v = fmaxf(v, partner<32>(v));
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

// Meets the other waves of the workgroup without waiting for memory: loads
// that any wave issued before it are queued ahead of loads any wave issues
// after it.  Measured: a CU returns its waves' loads in issue order, so a
// small load queued behind another wave's weight stream waits for that stream;
// kernels issue their small loads, meet here, then start the streams.
__device__ __forceinline__ void issue_barrier() {
    asm volatile("s_barrier" ::: "memory");
    __builtin_amdgcn_sched_barrier(0);
}

// Waits for every load this wave has in flight (s_waitcnt vmcnt(0)).  A kernel
// whose first small loads miss the caches calls it before starting its
// streams: once the whole device's streams are queued at the memory
// controllers, a miss issued just before them is served in the controllers'
// order, not first (measured: 0.8 us alone, 6-10 us behind the streams).
__device__ __forceinline__ void wait_loads() { __builtin_amdgcn_s_waitcnt(0x0F70); }

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
//   q8_0: qs plane  [r][j][16] int8 quants 0..15 of each block, then (at
//         ex = qs + the first half's 256-B aligned size) [r][j][16] quants
//         16..31; sc plane [r][j] fp16 d.  Lane l's 16-byte load of a row's
//         block l then sits next to lane l+1's: every wave load of a half is
//         one contiguous run (two 16-byte loads 32 bytes apart per block
//         streamed 16 % slower at 178 MB).
//   q4_0: qs plane  [r][j][16] nibbles       sc plane [r][j] fp16 d
//   q4_K: qs plane  [r][j][144] the GGUF block unchanged (16-B header + qs)
//   q5_K: qs plane  [r][j][176] the GGUF block unchanged (16-B header, qh, qs)
//   q2_K: qs plane  [r][j][64] 2-bit quants  sc plane [r][j][16] scale|min
//         ex plane  [r][j] {fp16 d, fp16 dmin}
//   q3_K: qs plane  [r][j][64] low bits + [r][j][32] hmask in ex plane,
//         sc plane  [r][j][12] packed 6-bit scales, d plane [r][j] fp16
//   q6_K: qs plane  [r][j][128] low nibbles (ql), ex plane [r][j][64] high
//         bits (qh), sc plane [r][j][16] int8 scales, d plane [r][j] fp16
//  tq2_0: qs plane  [r][j][64] 2-bit trits  sc plane [r][j] fp16 d
//  f16 / bf16: qs plane [r][ncols] the 16-bit values (ncols % 8 == 0)
// Every plane starts 256-B aligned; quant rows are 16-B multiples so every
// quant load is an aligned 128-bit load.
struct g4h_tensor {
    int type;
    int64_t ncols, nrows, nb;   // nb = (super)blocks per row
    uint8_t *base;              // single allocation
    size_t bytes;
    uint8_t *qs;                // quant plane
    uint8_t *sc;                // scale plane (q8_0/q4_0/tq2_0: fp16 d; q2_K/q3_K: packed scales)
    uint8_t *ex;                // q8_0: quants 16..31; q2_K: {d,dmin}; q3_K: hmask; q6_K: qh
    uint8_t *dd;                // q3_K / q6_K: fp16 d
};
