// formats.h -- per-format "unit" arithmetic of the quantized dots.
//
// A unit is the piece of one weight row a single lane handles:
//   q8_0 / q4_0 : one 32-element block;
//   q2_K / q3_K / q4_K : a quarter of a 256-element superblock (64 elements).
// Each format provides
//   Frag              registers holding one unit's weight bytes,
//   load(...)         the unit's global loads from the resident layout,
//   isums(...)        the exact integer sums of the unit against one token's
//                     activation held in LDS (the integers the reference
//                     scales, quants.c:535-762),
//   accum(...)        acc + those sums times their scales (fp32).
// The GEMV, the block-sum instrument and the raw-row vec_dot all go through
// these functions, so the integers checked bit-exactly by the tests are the
// ones the fast path scales.
#pragma once

#include "common.h"

namespace g4 {

// ---------------------------------------------------------------- LDS act --
// Activation of NB tokens staged in LDS.
// q8_0 act (blocks of 32): per token t: Q0[nb] int4 (qs 0..15), Q1[nb] int4
// (qs 16..31), D[nb] float (fp16 d widened), S[nb] int (sum of qs).
// q8_K act (superblocks of 256): per token t and superblock, 304 bytes: the
// GGUF block (d, 256 quants, 16 bsums: 292 bytes) shifted 12 bytes up, so d
// sits at byte 12, the quants at 16..271 (16-byte aligned) and the bsums at
// 272..303; the staging then moves whole 16-byte slots.
struct ActQ8_0 {
    static __host__ __device__ size_t bytes_per_token(int nb) { return ((size_t)nb * 40 + 15) & ~(size_t)15; }
    int4 *q0, *q1; float *d; int *s;
    __device__ ActQ8_0(uint8_t *base, int nb, int t) {
        uint8_t *p = base + (size_t)t * bytes_per_token(nb);
        q0 = (int4 *)p; q1 = q0 + nb; d = (float *)(q1 + nb); s = (int *)(d + nb);
    }
};
struct ActQ8_K {
    static constexpr int SB = 304;
    static __host__ __device__ size_t bytes_per_token(int nb) { return (size_t)nb * SB; }
    uint8_t *p;
    __device__ ActQ8_K(uint8_t *base, int nb, int t) : p(base + (size_t)t * bytes_per_token(nb)) {}
    __device__ const int8_t *q(int sb) const { return (const int8_t *)(p + (size_t)sb * SB + 16); }
    __device__ float d(int sb) const { return *(const float *)(p + (size_t)sb * SB + 12); }
    __device__ const int16_t *bs(int sb) const { return (const int16_t *)(p + (size_t)sb * SB + 272); }
};

// Staging.  A kernel issues the (small, mostly L2-resident) activation loads
// before its weight stream and writes LDS while the weights are in flight:
// global loads complete in issue order, so waiting for activations issued
// first never waits for the weights.  Loads and stores are branch-free: a load
// whose only use sits under a per-thread branch is sunk by the compiler below
// later loads (and its wait then covers them), and a branch join makes it wait
// early.  So a thread without an item reads a pad in device memory (one
// address for the whole wave: one request) and writes its own slot of a dump
// area placed after the staged tokens (kStageDump bytes, included in the LDS
// sizes; one slot per lane, so these writes do not collide in one bank).
constexpr size_t kStageDump = 64 * 80;
template <class Act>
__device__ __forceinline__ uint8_t *stage_dump(uint8_t *lds, int ntok, int nb) { return lds + (size_t)ntok * Act::bytes_per_token(nb); }
static __device__ uint32_t g_stage_pad[17];

// q8_0: one item = a pair of 34-B blocks = 17 aligned dwords.
struct StageQ8_0 {
    uint32_t v[17];
    int t, pr;
    bool ok;
};
template <int NB>
__device__ __forceinline__ void stage_q8_0_load(StageQ8_0 &S, int item, const uint8_t *act, size_t stride, int nb) {
    const int npair = nb >> 1;
    S.ok = item < NB * npair;
    S.t = (NB == 1 || !S.ok) ? 0 : item / npair;                     // one token: no division ahead of the stream
    S.pr = S.ok ? item - S.t * npair : 0;
    const uint32_t *src = S.ok ? (const uint32_t *)(act + (size_t)S.t * stride + (size_t)S.pr * 68) : g_stage_pad;
#pragma unroll
    for (int k = 0; k < 17; k++) S.v[k] = src[k];
}
__device__ __forceinline__ int sum_i8x16(int4 a) {
    int s = dot4(a.x, 0x01010101, 0);
    s = dot4(a.y, 0x01010101, s); s = dot4(a.z, 0x01010101, s); return dot4(a.w, 0x01010101, s);
}
__device__ __forceinline__ void stage_q8_0_store(const StageQ8_0 &S, uint8_t *lds, int nb, uint8_t *dump) {
    // the dump slot: a two-block layout (80 B) per lane
    ActQ8_0 A(S.ok ? lds : dump + 80 * (threadIdx.x & 63), S.ok ? nb : 2, S.t);
    const uint32_t *v = S.v;
    const int b = 2 * S.pr;
    int4 a0, a1;
    a0.x = __builtin_amdgcn_alignbyte(v[1], v[0], 2); a0.y = __builtin_amdgcn_alignbyte(v[2], v[1], 2);
    a0.z = __builtin_amdgcn_alignbyte(v[3], v[2], 2); a0.w = __builtin_amdgcn_alignbyte(v[4], v[3], 2);
    a1.x = __builtin_amdgcn_alignbyte(v[5], v[4], 2); a1.y = __builtin_amdgcn_alignbyte(v[6], v[5], 2);
    a1.z = __builtin_amdgcn_alignbyte(v[7], v[6], 2); a1.w = __builtin_amdgcn_alignbyte(v[8], v[7], 2);
    A.q0[b] = a0; A.q1[b] = a1; A.d[b] = h2f((uint16_t)(v[0] & 0xffff));
    A.s[b] = sum_i8x16(a0) + sum_i8x16(a1);
    const int4 c0 = make_int4(v[9], v[10], v[11], v[12]), c1 = make_int4(v[13], v[14], v[15], v[16]);
    A.q0[b + 1] = c0; A.q1[b + 1] = c1; A.d[b + 1] = h2f((uint16_t)(v[8] >> 16));
    A.s[b + 1] = sum_i8x16(c0) + sum_i8x16(c1);
}
// remaining items (rows longer than two blocks per thread) and an odd last block
template <int NB>
__device__ void stage_q8_0_rest(uint8_t *lds, const uint8_t *act, size_t stride, int nb) {
    for (int i = threadIdx.x + blockDim.x; i < NB * (nb >> 1); i += blockDim.x) {
        StageQ8_0 S;
        stage_q8_0_load<NB>(S, i, act, stride, nb);
        stage_q8_0_store(S, lds, nb, stage_dump<ActQ8_0>(lds, NB, nb));
    }
    if (nb & 1) {   // last block with 16-bit loads
        for (int t = threadIdx.x; t < NB; t += blockDim.x) {
            const uint16_t *src = (const uint16_t *)(act + (size_t)t * stride + (size_t)(nb - 1) * 34);
            uint32_t w[8];
#pragma unroll
            for (int k = 0; k < 8; k++) w[k] = (uint32_t)src[1 + 2 * k] | ((uint32_t)src[2 + 2 * k] << 16);
            ActQ8_0 A(lds, nb, t);
            const int4 a0 = make_int4(w[0], w[1], w[2], w[3]), a1 = make_int4(w[4], w[5], w[6], w[7]);
            A.q0[nb - 1] = a0; A.q1[nb - 1] = a1; A.d[nb - 1] = h2f(src[0]);
            A.s[nb - 1] = sum_i8x16(a0) + sum_i8x16(a1);
        }
    }
}
// q8_0 quantization of fp32 activations straight into the LDS layout: the
// arithmetic of the standalone quantizer (k_quant.hip, quants.c:74-109), so
// the staged token is bit-identical to quantizing first.  Four consecutive
// values v of token t, group j (elements 4j..4j+3); the 8 consecutive lanes of
// a 32-element block call it together (all lanes of the wave call it: the
// block maximum is a lane shuffle), and only lanes with `own` write.
__device__ __forceinline__ void q8_lds4(const float v[4], int j, bool own, uint8_t *lds, int nb, int t) {
    const float am = group_max<8>(fmaxf(fmaxf(fabsf(v[0]), fabsf(v[1])), fmaxf(fabsf(v[2]), fabsf(v[3]))));
    const float id = am != 0.0f ? 127.0f / am : 0.0f;
    uint32_t pk = 0;
#pragma unroll
    for (int i = 0; i < 4; i++) pk |= ((uint32_t)(int)__builtin_rintf(v[i] * id) & 0xffu) << (8 * i);
    const int sum = group_isum<8>(dot4((int)pk, 0x01010101, 0));
    if (!own) return;
    ActQ8_0 A(lds, nb, t);
    const int b = j >> 3, k = j & 7;
    ((uint32_t *)(k < 4 ? &A.q0[b] : &A.q1[b]))[k & 3] = pk;
    if (k == 0) {
        A.d[b] = h2f(f2h(am * (1.0f / 127.0f)));
        A.s[b] = sum;
    }
}

// q8_K arithmetic of one 256-element superblock held by one wave (lane l:
// elements 4l..4l+3; quants.c:146-175), shared by the standalone quantizer and
// the GEMV's in-kernel one, so both give the same bits.  The whole wave calls
// it.  pk: the lane's four quants; s16: the sum of the 16 quants of lanes
// 4k..4k+3; d: the superblock scale (max * fp32(-1/127), the shipped build's
// folding of 1/iscale).
struct Q8KLane {
    uint32_t pk;
    int s16;
    float d;
};
__device__ __forceinline__ Q8KLane q8K_wave(const float v[4]) {
    // value of largest magnitude, first occurrence on ties (quants.c:150-154):
    // the wave maximum of |x| (unsigned lane exchanges of the bit patterns),
    // then the lowest element index that reaches it (ballots), then that
    // element's signed value.  NaN elements are passed over, as the reference's
    // `ax > amax` passes them; an all-NaN superblock quantizes as all-zero.
    const float lm = fmaxf(fmaxf(fmaxf(fabsf(v[0]), fabsf(v[1])), 0.0f), fmaxf(fabsf(v[2]), fabsf(v[3])));
    const float am = __builtin_bit_cast(float, wave_umax(__builtin_bit_cast(uint32_t, lm)));
    int first = 255;
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const uint64_t m = __ballot(fabsf(v[i]) == am);
        if (m) first = min(first, 4 * __builtin_ctzll(m) + i);
    }
    const int fi = first & 3;
    const float mine = fi == 0 ? v[0] : fi == 1 ? v[1] : fi == 2 ? v[2] : v[3];
    const float bv = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, mine), first >> 2));
    Q8KLane r{0u, 0, 0.0f};
    if (am != 0.0f) {
        const float iscale = -127.0f / bv;
#pragma unroll
        for (int i = 0; i < 4; i++) {
            int q = rne_prod(iscale, v[i]);
            q = q < 127 ? q : 127;
            r.pk |= ((uint32_t)q & 0xffu) << (8 * i);
            r.s16 += q;
        }
        r.d = bv * (-1.0f / 127.0f);
    }
    r.s16 = group_isum<4>(r.s16);
    return r;
}

// q8_K quantization of one fp32 token straight into the LDS layout, a
// superblock per row of L = 64 / XQ lanes (16 or 32): lane i of row sb holds
// its elements 4 XQ i .. 4 XQ i + 4 XQ - 1 (XQ groups of 4).  The arithmetic
// is q8K_wave's, so the staged token is bit-identical to quantizing first:
// the row maximum of |x| (NaN passed over), the lowest element index that
// reaches it (a row minimum of 2 index + sign), -127 / that value as iscale,
// the same rounded products, their 16-element sums and d.  Rows are
// independent (every exchange stays inside its 16 or 32 lanes), so a row past
// the token's superblocks just skips it; the wave need not be uniform.
template <int XQ>
__device__ __forceinline__ void q8K_rows(const float (&v)[XQ][4], int sb, int nsb, uint8_t *lds, int nb) {
    static_assert(XQ == 2 || XQ == 4, "16 or 32 lanes per superblock");
    constexpr int L = 64 / XQ, E = 4 * XQ;                           // lanes per superblock, elements per lane
    if (sb >= nsb) return;
    const int i = threadIdx.x & (L - 1);
    float lm = 0.0f;
#pragma unroll
    for (int s = 0; s < XQ; s++)
#pragma unroll
        for (int k = 0; k < 4; k++) lm = fmaxf(lm, fabsf(v[s][k]));
    uint32_t u = __builtin_bit_cast(uint32_t, lm);                   // non-negative: bits order as values
    u = max(u, partner_u32<1>(u));
    u = max(u, partner_u32<2>(u));
    u = max(u, partner_u32<4>(u));
    u = max(u, partner_u32<8>(u));
    if constexpr (L == 32) u = max(u, partner_u32<16>(u));
    const float am = __builtin_bit_cast(float, u);
    uint32_t key = 0xffffffffu;
#pragma unroll
    for (int s = XQ - 1; s >= 0; s--)
#pragma unroll
        for (int k = 3; k >= 0; k--)
            if (fabsf(v[s][k]) == am) key = 2u * (uint32_t)(E * i + 4 * s + k) + (__builtin_bit_cast(uint32_t, v[s][k]) >> 31);
    key = min(key, partner_u32<1>(key));
    key = min(key, partner_u32<2>(key));
    key = min(key, partner_u32<4>(key));
    key = min(key, partner_u32<8>(key));
    if constexpr (L == 32) key = min(key, partner_u32<16>(key));
    uint32_t pk[XQ] = {};
    int sum = 0;
    float d = 0.0f;
    if (am != 0.0f) {
        const float bv = (key & 1u) ? -am : am;                      // the element itself: |x| == am
        const float iscale = -127.0f / bv;
#pragma unroll
        for (int s = 0; s < XQ; s++)
#pragma unroll
            for (int k = 0; k < 4; k++) {
                int q = rne_prod(iscale, v[s][k]);
                q = q < 127 ? q : 127;
                pk[s] |= ((uint32_t)q & 0xffu) << (8 * k);
                sum += q;
            }
        d = bv * (-1.0f / 127.0f);
    }
    if constexpr (L == 32) sum += partner<1>(sum);                   // lanes 2 g, 2 g + 1: bsums group g
    uint8_t *p = lds + (size_t)sb * ActQ8_K::SB;
    if constexpr (XQ == 4) {
        *(uint4 *)(p + 16 + 16 * i) = make_uint4(pk[0], pk[1], pk[2], pk[3]);
        ((int16_t *)(p + 272))[i] = (int16_t)sum;
    } else {
        *(uint2 *)(p + 16 + 8 * i) = make_uint2(pk[0], pk[1]);
        if ((i & 1) == 0) ((int16_t *)(p + 272))[i >> 1] = (int16_t)sum;
    }
    if (i == 0) *(float *)(p + 12) = d;
}

template <int NB>
__device__ void stage_q8_0(uint8_t *lds, const uint8_t *act, size_t stride, int nb) {
    StageQ8_0 S;
    stage_q8_0_load<NB>(S, threadIdx.x, act, stride, nb);
    stage_q8_0_store(S, lds, nb, stage_dump<ActQ8_0>(lds, NB, nb));
    stage_q8_0_rest<NB>(lds, act, stride, nb);
}

// q8_K: one item = one 16-byte slot s (0..18) of a staged superblock, i.e.
// dwords 4s-3 .. 4s of the GGUF block (slot 0 carries d in its last dword;
// its first three are padding).
struct StageQ8_K {
    uint32_t v[4];
    int t, sb, s;
    bool ok;
};
template <int NB>
__device__ __forceinline__ void stage_q8_K_load(StageQ8_K &S, int item, const uint8_t *act, size_t stride, int nb) {
    const int per = nb * 19;
    S.ok = item < NB * per;
    const int it = S.ok ? item : 0;
    S.t = NB == 1 ? 0 : it / per;                                    // one token: no division ahead of the stream
    const int r = it - S.t * per;
    S.sb = r / 19;
    S.s = r - S.sb * 19;
    const uint32_t *src = S.ok ? (const uint32_t *)(act + (size_t)S.t * stride) + (size_t)S.sb * 73 + max(4 * S.s - 3, 0)
                               : g_stage_pad;
#pragma unroll
    for (int k = 0; k < 4; k++) S.v[k] = src[k];
}
__device__ __forceinline__ void stage_q8_K_store(const StageQ8_K &S, uint8_t *lds, int nb, uint8_t *dump) {
    uint8_t *dst = S.ok ? lds + (size_t)S.t * ActQ8_K::bytes_per_token(nb) + (size_t)S.sb * ActQ8_K::SB + 16 * S.s
                        : dump + 16 * (threadIdx.x & 63);
    const bool first = S.s == 0;                                     // d goes to the slot's last dword
    *(int4 *)dst = make_int4(S.v[0], S.v[1], S.v[2], first ? S.v[0] : S.v[3]);
}
// items from `first` on (threads step by blockDim)
template <int NB>
__device__ void stage_q8_K_rest(uint8_t *lds, const uint8_t *act, size_t stride, int nb, int first = 1) {
    for (int i = threadIdx.x + first * blockDim.x; i < NB * nb * 19; i += blockDim.x) {
        StageQ8_K S;
        stage_q8_K_load<NB>(S, i, act, stride, nb);
        stage_q8_K_store(S, lds, nb, stage_dump<ActQ8_K>(lds, NB, nb));
    }
}
template <int NB>
__device__ void stage_q8_K(uint8_t *lds, const uint8_t *act, size_t stride, int nb) {
    StageQ8_K S;
    stage_q8_K_load<NB>(S, threadIdx.x, act, stride, nb);
    stage_q8_K_store(S, lds, nb, stage_dump<ActQ8_K>(lds, NB, nb));
    stage_q8_K_rest<NB>(lds, act, stride, nb);
}

// Format -> staging helpers
template <int T> struct StageOf;
template <> struct StageOf<Q8_0> { using S = StageQ8_0; };
template <> struct StageOf<Q4_0> { using S = StageQ8_0; };
template <> struct StageOf<Q2_K> { using S = StageQ8_K; };
template <> struct StageOf<Q3_K> { using S = StageQ8_K; };
template <> struct StageOf<Q4_K> { using S = StageQ8_K; };
template <> struct StageOf<Q5_K> { using S = StageQ8_K; };
template <> struct StageOf<Q6_K> { using S = StageQ8_K; };
template <> struct StageOf<TQ2_0> { using S = StageQ8_K; };

// ------------------------------------------------------------------ q8_0 --
struct FQ8_0 {
    static constexpr int type = Q8_0;
    using Act = ActQ8_0;
    static constexpr int units_per_block = 1;
    struct Frag { int4 w0, w1; uint16_t d; };
    static __device__ __forceinline__ void load(Frag &f, const g4h_tensor &W, int64_t row, int u) {
        const size_t j = (size_t)row * W.nb + u;
        f.w0 = ld4s(W.qs + j * 16); f.w1 = ld4s(W.ex + j * 16);      // the two half-block planes
        f.d = ((const uint16_t *)W.sc)[j];
    }
    static __device__ __forceinline__ int isum(const Frag &f, const Act &A, int u) {
        const int4 a0 = A.q0[u], a1 = A.q1[u];
        int s = dot4(f.w0.x, a0.x, 0);
        s = dot4(f.w0.y, a0.y, s); s = dot4(f.w0.z, a0.z, s); s = dot4(f.w0.w, a0.w, s);
        s = dot4(f.w1.x, a1.x, s); s = dot4(f.w1.y, a1.y, s); s = dot4(f.w1.z, a1.z, s); s = dot4(f.w1.w, a1.w, s);
        return s;
    }
    // block value: float(sumi) * (d_w * d_a), accumulated with one fma as the
    // reference's per-block step (quants.c:992,996)
    static __device__ __forceinline__ float accum(const Frag &f, const Act &A, int u, float acc) {
        return __builtin_fmaf(h2f(f.d) * A.d[u], (float)isum(f, A, u), acc);
    }
    static constexpr int nsums = 1;
    static __device__ __forceinline__ void sums(const Frag &f, const Act &A, int u, int *out) { out[0] = isum(f, A, u); }
};

// ------------------------------------------------------------------ q4_0 --
// Elements j<16 are the low nibbles of qs[j], j>=16 the high nibbles of
// qs[j-16] (quants.c:364-371); value q-8.  sum (q-8)*a = sum q*a - 8*sum a.
struct FQ4_0 {
    static constexpr int type = Q4_0;
    using Act = ActQ8_0;
    static constexpr int units_per_block = 1;
    struct Frag { int4 w; uint16_t d; };
    static __device__ __forceinline__ void load(Frag &f, const g4h_tensor &W, int64_t row, int u) {
        const size_t j = (size_t)row * W.nb + u;
        f.w = ld4s(W.qs + j * 16);
        f.d = ((const uint16_t *)W.sc)[j];
    }
    static __device__ __forceinline__ int isum(const Frag &f, const Act &A, int u) {
        const int m = 0x0F0F0F0F;
        const int4 a0 = A.q0[u], a1 = A.q1[u];
        const uint32_t x = f.w.x, y = f.w.y, z = f.w.z, w = f.w.w;
        int s = dot4(x & m, a0.x, 0);
        s = dot4(y & m, a0.y, s); s = dot4(z & m, a0.z, s); s = dot4(w & m, a0.w, s);
        s = dot4((x >> 4) & m, a1.x, s); s = dot4((y >> 4) & m, a1.y, s);
        s = dot4((z >> 4) & m, a1.z, s); s = dot4((w >> 4) & m, a1.w, s);
        return s - 8 * A.s[u];
    }
    static __device__ __forceinline__ float accum(const Frag &f, const Act &A, int u, float acc) {
        return __builtin_fmaf(h2f(f.d) * A.d[u], (float)isum(f, A, u), acc);
    }
    static constexpr int nsums = 1;
    static __device__ __forceinline__ void sums(const Frag &f, const Act &A, int u, int *out) { out[0] = isum(f, A, u); }
};

// ------------------------------------------------------------------ q4_K --
// Part p of a superblock covers elements 64p..64p+63: low nibbles of
// qs[32p..32p+31] (sub-block 2p) and their high nibbles (sub-block 2p+1)
// (quants.c:479-495).  6-bit (scale,min) pairs per quants.c:417-423.
struct FQ4_K {
    static constexpr int type = Q4_K;
    using Act = ActQ8_K;
    static constexpr int units_per_block = 4;
    struct Frag { int4 h, q0, q1; };
    static __device__ __forceinline__ void load(Frag &f, const g4h_tensor &W, int64_t row, int u) {
        const uint8_t *b = W.qs + ((size_t)row * W.nb + (u >> 2)) * 144;
        const int p = u & 3;
        f.h = ld4(b);
        f.q0 = ld4(b + 16 + 32 * p); f.q1 = ld4(b + 32 + 32 * p);   // plain: the header shares these lines
    }
    // 6-bit scale and min of sub-blocks 2p and 2p+1 (quants.c get_scale_min_k4:
    // j < 4 from the low six bits of scales[j] / scales[j+4]; j >= 4 from the
    // nibbles of scales[j+4] and the top two bits of scales[j-4] / scales[j]),
    // built four sub-blocks at a time in one register and without a branch on
    // p: the lanes of a wave hold different parts.
    static __device__ __forceinline__ void scale_min_pair(const Frag &f, int p, int &sc0, int &m0, int &sc1, int &m1) {
        const uint32_t y = (uint32_t)f.h.y, z = (uint32_t)f.h.z, w = (uint32_t)f.h.w;
        const bool hi = p >= 2;
        const uint32_t sc = hi ? (w & 0x0f0f0f0fu) | ((y >> 2) & 0x30303030u) : y & 0x3f3f3f3fu;
        const uint32_t mn = hi ? ((w >> 4) & 0x0f0f0f0fu) | ((z >> 2) & 0x30303030u) : z & 0x3f3f3f3fu;
        const int sh = 16 * (p & 1);
        sc0 = (int)((sc >> sh) & 0xff);
        sc1 = (int)((sc >> (sh + 8)) & 0xff);
        m0 = (int)((mn >> sh) & 0xff);
        m1 = (int)((mn >> (sh + 8)) & 0xff);
    }
    static __device__ __forceinline__ void isums(const Frag &f, const Act &A, int u, int &is, int &ms) {
        const int sb = u >> 2, p = u & 3, m = 0x0F0F0F0F;
        const int4 *a = (const int4 *)(A.q(sb) + 64 * p);
        const int4 l0 = a[0], l1 = a[1], h0 = a[2], h1 = a[3];
        const uint32_t w[8] = {(uint32_t)f.q0.x, (uint32_t)f.q0.y, (uint32_t)f.q0.z, (uint32_t)f.q0.w,
                               (uint32_t)f.q1.x, (uint32_t)f.q1.y, (uint32_t)f.q1.z, (uint32_t)f.q1.w};
        int sl = dot4(w[0] & m, l0.x, 0);
        sl = dot4(w[1] & m, l0.y, sl); sl = dot4(w[2] & m, l0.z, sl); sl = dot4(w[3] & m, l0.w, sl);
        sl = dot4(w[4] & m, l1.x, sl); sl = dot4(w[5] & m, l1.y, sl); sl = dot4(w[6] & m, l1.z, sl); sl = dot4(w[7] & m, l1.w, sl);
        int sh = dot4((w[0] >> 4) & m, h0.x, 0);
        sh = dot4((w[1] >> 4) & m, h0.y, sh); sh = dot4((w[2] >> 4) & m, h0.z, sh); sh = dot4((w[3] >> 4) & m, h0.w, sh);
        sh = dot4((w[4] >> 4) & m, h1.x, sh); sh = dot4((w[5] >> 4) & m, h1.y, sh); sh = dot4((w[6] >> 4) & m, h1.z, sh); sh = dot4((w[7] >> 4) & m, h1.w, sh);
        int sc0, m0, sc1, m1;
        scale_min_pair(f, p, sc0, m0, sc1, m1);
        const int16_t *bs = A.bs(sb) + 4 * p;
        // 24-bit products: |sl|, |sh| <= 32*15*128 and |bs[i] + bs[i+1]| <= 4096
        is = __mul24(sc0, sl) + __mul24(sc1, sh);
        ms = __mul24(m0, bs[0] + bs[1]) + __mul24(m1, bs[2] + bs[3]);
    }
    // superblock value d_a*(d_w*isum - dmin_w*msum) (quants.c:744-758), spread
    // over the four parts
    static __device__ __forceinline__ float accum(const Frag &f, const Act &A, int u, float acc) {
        int is, ms; isums(f, A, u, is, ms);
        const float da = A.d(u >> 2);
        const uint32_t dd = (uint32_t)f.h.x;
        acc = __builtin_fmaf(da * h2f((uint16_t)(dd & 0xffff)), (float)is, acc);
        return __builtin_fmaf(-da * h2f((uint16_t)(dd >> 16)), (float)ms, acc);
    }
    static constexpr int nsums = 2;
    static __device__ __forceinline__ void sums(const Frag &f, const Act &A, int u, int *out) { isums(f, A, u, out[0], out[1]); }
};

// ------------------------------------------------------------------ q5_K --
// The q4_K block with a fifth bit per element (quants.c:497-515, 764-818):
// 16-byte header (d, dmin, packed 6-bit scales / mins), qh[32] at 16, qs[128]
// at 48.  Element e = 32c + l (chunk c = 0..7): nibble of qs[32(c/2) + l]
// (low for even c) plus 16 * bit c of qh[l]; scale / min of sub-block c.
// Part p covers chunks 2p, 2p+1 (the 32 qs bytes 32p..32p+31 and all 32 qh
// bytes, which the four parts of a superblock share).
struct FQ5_K {
    static constexpr int type = Q5_K;
    using Act = ActQ8_K;
    static constexpr int units_per_block = 4;
    struct Frag { int4 h, q0, q1, hb0, hb1; };
    static __device__ __forceinline__ void load(Frag &f, const g4h_tensor &W, int64_t row, int u) {
        const uint8_t *b = W.qs + ((size_t)row * W.nb + (u >> 2)) * 176;
        const int p = u & 3;
        f.h = ld4(b);
        f.hb0 = ld4(b + 16); f.hb1 = ld4(b + 32);
        f.q0 = ld4(b + 48 + 32 * p); f.q1 = ld4(b + 64 + 32 * p);
    }
    static __device__ __forceinline__ void isums(const Frag &f, const Act &A, int u, int &is, int &ms) {
        const int sb = u >> 2, p = u & 3, m = 0x0F0F0F0F;
        const int4 *a = (const int4 *)(A.q(sb) + 64 * p);
        const int4 l0 = a[0], l1 = a[1], h0 = a[2], h1 = a[3];
        const uint32_t w[8] = {(uint32_t)f.q0.x, (uint32_t)f.q0.y, (uint32_t)f.q0.z, (uint32_t)f.q0.w,
                               (uint32_t)f.q1.x, (uint32_t)f.q1.y, (uint32_t)f.q1.z, (uint32_t)f.q1.w};
        const uint32_t hb[8] = {(uint32_t)f.hb0.x, (uint32_t)f.hb0.y, (uint32_t)f.hb0.z, (uint32_t)f.hb0.w,
                                (uint32_t)f.hb1.x, (uint32_t)f.hb1.y, (uint32_t)f.hb1.z, (uint32_t)f.hb1.w};
        const int c0 = 2 * p, c1 = 2 * p + 1;
        int lo[8], hi[8];
#pragma unroll
        for (int i = 0; i < 8; i++) {
            lo[i] = (int)((w[i] & m) | (((hb[i] >> c0) & 0x01010101) << 4));
            hi[i] = (int)(((w[i] >> 4) & m) | (((hb[i] >> c1) & 0x01010101) << 4));
        }
        int sl = dot4(lo[0], l0.x, 0);
        sl = dot4(lo[1], l0.y, sl); sl = dot4(lo[2], l0.z, sl); sl = dot4(lo[3], l0.w, sl);
        sl = dot4(lo[4], l1.x, sl); sl = dot4(lo[5], l1.y, sl); sl = dot4(lo[6], l1.z, sl); sl = dot4(lo[7], l1.w, sl);
        int sh = dot4(hi[0], h0.x, 0);
        sh = dot4(hi[1], h0.y, sh); sh = dot4(hi[2], h0.z, sh); sh = dot4(hi[3], h0.w, sh);
        sh = dot4(hi[4], h1.x, sh); sh = dot4(hi[5], h1.y, sh); sh = dot4(hi[6], h1.z, sh); sh = dot4(hi[7], h1.w, sh);
        FQ4_K::Frag hf;
        hf.h = f.h;
        int sc0, m0, sc1, m1;
        FQ4_K::scale_min_pair(hf, p, sc0, m0, sc1, m1);
        const int16_t *bs = A.bs(sb) + 4 * p;
        // 24-bit products: |sl|, |sh| <= 32*31*128 and |bs[i] + bs[i+1]| <= 4096
        is = __mul24(sc0, sl) + __mul24(sc1, sh);
        ms = __mul24(m0, bs[0] + bs[1]) + __mul24(m1, bs[2] + bs[3]);
    }
    // superblock value d_a*(d_w*isum - dmin_w*msum), spread over the four parts
    static __device__ __forceinline__ float accum(const Frag &f, const Act &A, int u, float acc) {
        int is, ms; isums(f, A, u, is, ms);
        const float da = A.d(u >> 2);
        const uint32_t dd = (uint32_t)f.h.x;
        acc = __builtin_fmaf(da * h2f((uint16_t)(dd & 0xffff)), (float)is, acc);
        return __builtin_fmaf(-da * h2f((uint16_t)(dd >> 16)), (float)ms, acc);
    }
    static constexpr int nsums = 2;
    static __device__ __forceinline__ void sums(const Frag &f, const Act &A, int u, int *out) { isums(f, A, u, out[0], out[1]); }
};

// ------------------------------------------------------------------ q2_K --
// Element e = 128h + 32j + 16k + l sits in byte qs[32h + 16k + l] at shift 2j,
// scale byte scales[8h + 2j + k] (low nibble scale, high nibble min)
// (quants.c:425-445).  Part p = 2h + k holds 16 quant bytes covering four
// 16-element groups j = 0..3.
struct FQ2_K {
    static constexpr int type = Q2_K;
    using Act = ActQ8_K;
    static constexpr int units_per_block = 4;
    struct Frag { int4 q, s; uint32_t dd; };
    static __device__ __forceinline__ void load(Frag &f, const g4h_tensor &W, int64_t row, int u) {
        const size_t j = (size_t)row * W.nb + (u >> 2);
        f.q = ld4s(W.qs + j * 64 + 16 * (u & 3));
        f.s = ld4(W.sc + j * 16);
        f.dd = ((const uint32_t *)W.ex)[j];
    }
    static __device__ __forceinline__ void isums(const Frag &f, const Act &A, int u, int &is, int &ms) {
        const int sb = u >> 2, p = u & 3, h = p >> 1, k = p & 1;
        const uint32_t w[4] = {(uint32_t)f.q.x, (uint32_t)f.q.y, (uint32_t)f.q.z, (uint32_t)f.q.w};
        const uint32_t sw[4] = {(uint32_t)f.s.x, (uint32_t)f.s.y, (uint32_t)f.s.z, (uint32_t)f.s.w};
        const int8_t *aq = A.q(sb) + 128 * h + 16 * k;
        const int16_t *bs = A.bs(sb);
        int isum = 0, msum = 0;
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const int4 a = *(const int4 *)(aq + 32 * j);
            int s = dot4((w[0] >> (2 * j)) & 0x03030303, a.x, 0);
            s = dot4((w[1] >> (2 * j)) & 0x03030303, a.y, s);
            s = dot4((w[2] >> (2 * j)) & 0x03030303, a.z, s);
            s = dot4((w[3] >> (2 * j)) & 0x03030303, a.w, s);
            const int g = 8 * h + 2 * j + k;                       // 16-element group / scale index
            const int sc = (sw[g >> 2] >> (8 * (g & 3))) & 0xff;
            isum += __mul24(sc & 15, s);                           // |s| <= 16*3*128, |bs| <= 2048
            msum += __mul24(sc >> 4, (int)bs[g]);
        }
        is = isum; ms = msum;
    }
    static __device__ __forceinline__ float accum(const Frag &f, const Act &A, int u, float acc) {
        int is, ms; isums(f, A, u, is, ms);
        const float da = A.d(u >> 2);
        acc = __builtin_fmaf(da * h2f((uint16_t)(f.dd & 0xffff)), (float)is, acc);
        return __builtin_fmaf(-da * h2f((uint16_t)(f.dd >> 16)), (float)ms, acc);
    }
    static constexpr int nsums = 2;
    static __device__ __forceinline__ void sums(const Frag &f, const Act &A, int u, int *out) { isums(f, A, u, out[0], out[1]); }
};

// ------------------------------------------------------------------ q3_K --
// Element e = 128h + 32j + 16k + l: low bits (qs[32h+16k+l] >> 2j) & 3, high
// bit hmask[16k+l] bit (4h+j); value low - 4 when the high bit is clear
// (quants.c:447-477).  6-bit scales biased by 32: low nibbles from
// scales[0..7], high 2 bits from scales[8..11] (quants.c:456-461).
// q3 = (low | hbit<<2) - 4, so sum q3*a = sum t*a - 4*bsum of the group.
struct FQ3_K {
    static constexpr int type = Q3_K;
    using Act = ActQ8_K;
    static constexpr int units_per_block = 4;
    struct Frag { int4 q, hm; uint32_t s0, s1, s2; uint16_t d; };
    static __device__ __forceinline__ void load(Frag &f, const g4h_tensor &W, int64_t row, int u) {
        const size_t j = (size_t)row * W.nb + (u >> 2);
        const int p = u & 3;
        f.q = ld4s(W.qs + j * 64 + 16 * p);
        f.hm = ld4(W.ex + j * 32 + 16 * (p & 1));
        const uint32_t *s = (const uint32_t *)(W.sc + j * 12);
        f.s0 = s[0]; f.s1 = s[1]; f.s2 = s[2];
        f.d = ((const uint16_t *)W.dd)[j];
    }
    static __device__ __forceinline__ int scale(const Frag &f, int i) {   // signed 6-bit scale i < 16
        const uint32_t lo_w = (i & 7) < 4 ? f.s0 : f.s1;
        const int lo = (lo_w >> (8 * (i & 3) + (i >= 8 ? 4 : 0))) & 15;
        const int hi = (f.s2 >> (8 * (i & 3) + 2 * (i >> 2))) & 3;
        return (lo | (hi << 4)) - 32;
    }
    static __device__ __forceinline__ int isum(const Frag &f, const Act &A, int u) {
        const int sb = u >> 2, p = u & 3, h = p >> 1, k = p & 1;
        const uint32_t w[4] = {(uint32_t)f.q.x, (uint32_t)f.q.y, (uint32_t)f.q.z, (uint32_t)f.q.w};
        const uint32_t hb[4] = {(uint32_t)f.hm.x, (uint32_t)f.hm.y, (uint32_t)f.hm.z, (uint32_t)f.hm.w};
        // hmask bit 4h+j of each byte brought to bit 2+j once per unit, so that
        // (hh >> j) & 4 is the high bit in place: h = 1 shifts right by 2,
        // h = 0 left by 2 (the bits that spill into the next byte land at bits
        // 0-1 there, below any bit read)
        uint32_t hh[4];
#pragma unroll
        for (int d = 0; d < 4; d++) hh[d] = h ? hb[d] >> 2 : hb[d] << 2;
        const int8_t *aq = A.q(sb) + 128 * h + 16 * k;
        const int16_t *bs = A.bs(sb);
        int total = 0;
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const int4 a = *(const int4 *)(aq + 32 * j);
            int s = 0;
            s = dot4(((w[0] >> (2 * j)) & 0x03030303) | ((hh[0] >> j) & 0x04040404), a.x, s);
            s = dot4(((w[1] >> (2 * j)) & 0x03030303) | ((hh[1] >> j) & 0x04040404), a.y, s);
            s = dot4(((w[2] >> (2 * j)) & 0x03030303) | ((hh[2] >> j) & 0x04040404), a.z, s);
            s = dot4(((w[3] >> (2 * j)) & 0x03030303) | ((hh[3] >> j) & 0x04040404), a.w, s);
            const int g = 8 * h + 2 * j + k;
            total += __mul24(scale(f, g), s - 4 * bs[g]);                // |s - 4 bs| <= 16*7*128 + 4*2048
        }
        return total;
    }
    static __device__ __forceinline__ float accum(const Frag &f, const Act &A, int u, float acc) {
        return __builtin_fmaf(A.d(u >> 2) * h2f(f.d), (float)isum(f, A, u), acc);
    }
    static constexpr int nsums = 1;
    static __device__ __forceinline__ void sums(const Frag &f, const Act &A, int u, int *out) { out[0] = isum(f, A, u); }
};

// ------------------------------------------------------------------ q6_K --
// Element e = 128h + 32j + l of a superblock (quants.c:379-400): low nibble of
// ql[64h + 32(j&1) + l] (the high nibble for j >= 2), high 2 bits
// (qh[32h + l] >> 2j) & 3, value (nibble | high<<4) - 32, int8 scale
// scales[e/16].  Part p = 2h + k holds the 16 elements l = 16k..16k+15 of each
// 32-element chunk j: 16 bytes of each ql half and 16 qh bytes, scales
// 8h + k + 2j.  sum (q-32)*a = sum q*a - 32*bsum of the 16-element group.
struct FQ6_K {
    static constexpr int type = Q6_K;
    using Act = ActQ8_K;
    static constexpr int units_per_block = 4;
    struct Frag { int4 l0, l1, hb; uint2 s; uint16_t d; };
    static __device__ __forceinline__ void load(Frag &f, const g4h_tensor &W, int64_t row, int u) {
        const size_t j = (size_t)row * W.nb + (u >> 2);
        const int p = u & 3, h = p >> 1, k = p & 1;
        const uint8_t *ql = W.qs + j * 128 + 64 * h + 16 * k;
        f.l0 = ld4s(ql);
        f.l1 = ld4s(ql + 32);
        f.hb = ld4s(W.ex + j * 64 + 32 * h + 16 * k);
        f.s = *(const uint2 *)(W.sc + j * 16 + 8 * h);
        f.d = ((const uint16_t *)W.dd)[j];
    }
    static __device__ __forceinline__ int isum(const Frag &f, const Act &A, int u) {
        const int sb = u >> 2, p = u & 3, h = p >> 1, k = p & 1;
        const uint32_t L0[4] = {(uint32_t)f.l0.x, (uint32_t)f.l0.y, (uint32_t)f.l0.z, (uint32_t)f.l0.w};
        const uint32_t L1[4] = {(uint32_t)f.l1.x, (uint32_t)f.l1.y, (uint32_t)f.l1.z, (uint32_t)f.l1.w};
        const uint32_t H[4] = {(uint32_t)f.hb.x, (uint32_t)f.hb.y, (uint32_t)f.hb.z, (uint32_t)f.hb.w};
        const int8_t *aq = A.q(sb) + 128 * h + 16 * k;
        const int16_t *bs = A.bs(sb);
        int total = 0;
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const int4 a = *(const int4 *)(aq + 32 * j);
            const int lo = j >= 2 ? 4 : 0;
            int q[4];
#pragma unroll
            for (int i = 0; i < 4; i++)
                q[i] = (int)((((j & 1) ? L1[i] : L0[i]) >> lo) & 0x0F0F0F0F) | (int)(((H[i] >> (2 * j)) & 0x03030303) << 4);
            int s = dot4(q[0], a.x, 0);
            s = dot4(q[1], a.y, s);
            s = dot4(q[2], a.z, s);
            s = dot4(q[3], a.w, s);
            const int sbyte = k + 2 * j;                               // scales[8h + k + 2j]
            const int sc = (int)(int8_t)(((sbyte < 4 ? f.s.x : f.s.y) >> (8 * (sbyte & 3))) & 0xff);
            total += __mul24(sc, s - 32 * bs[8 * h + 2 * j + k]);       // |s - 32 bs| <= 16*63*128 + 32*2048
        }
        return total;
    }
    static __device__ __forceinline__ float accum(const Frag &f, const Act &A, int u, float acc) {
        return __builtin_fmaf(A.d(u >> 2) * h2f(f.d), (float)isum(f, A, u), acc);
    }
    static constexpr int nsums = 1;
    static __device__ __forceinline__ void sums(const Frag &f, const Act &A, int u, int *out) { out[0] = isum(f, A, u); }
};

// ----------------------------------------------------------------- tq2_0 --
// 66-byte superblock: 64 bytes of trits and an fp16 d (g4run.h:111).  Element
// e = 128h + 32j + 16k + l is (qs[32h + 16k + l] >> 2j) & 3, value trit - 1
// (quants.c:402-411, 564-580): q2_K's quant layout without its scales.  So
// sum (t - 1) a = sum t a - the unit's four 16-element activation group sums.
struct FTQ2_0 {
    static constexpr int type = TQ2_0;
    using Act = ActQ8_K;
    static constexpr int units_per_block = 4;
    struct Frag { int4 q; uint16_t d; };
    static __device__ __forceinline__ void load(Frag &f, const g4h_tensor &W, int64_t row, int u) {
        const size_t j = (size_t)row * W.nb + (u >> 2);
        f.q = ld4s(W.qs + j * 64 + 16 * (u & 3));
        f.d = ((const uint16_t *)W.sc)[j];
    }
    static __device__ __forceinline__ int isum(const Frag &f, const Act &A, int u) {
        const int sb = u >> 2, p = u & 3, h = p >> 1, k = p & 1;
        const uint32_t w[4] = {(uint32_t)f.q.x, (uint32_t)f.q.y, (uint32_t)f.q.z, (uint32_t)f.q.w};
        const int8_t *aq = A.q(sb) + 128 * h + 16 * k;
        const int16_t *bs = A.bs(sb);
        int s = 0, b = 0;
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const int4 a = *(const int4 *)(aq + 32 * j);
            s = dot4((w[0] >> (2 * j)) & 0x03030303, a.x, s);
            s = dot4((w[1] >> (2 * j)) & 0x03030303, a.y, s);
            s = dot4((w[2] >> (2 * j)) & 0x03030303, a.z, s);
            s = dot4((w[3] >> (2 * j)) & 0x03030303, a.w, s);
            b += bs[8 * h + 2 * j + k];
        }
        return s - b;
    }
    static __device__ __forceinline__ float accum(const Frag &f, const Act &A, int u, float acc) {
        return __builtin_fmaf(A.d(u >> 2) * h2f(f.d), (float)isum(f, A, u), acc);
    }
    static constexpr int nsums = 1;
    static __device__ __forceinline__ void sums(const Frag &f, const Act &A, int u, int *out) { out[0] = isum(f, A, u); }
};

}  // namespace g4
