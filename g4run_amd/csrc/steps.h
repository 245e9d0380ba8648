// steps.h -- the single-workgroup steps of the decode chain between the
// GEMVs (residual + RMSNorm + q8_0) and the q8_0 helper they share with the
// attention and GELU kernels.
//
// Arithmetic (model.c:338-345 rms_norm, 359-367 rope, 711-736 residuals,
// quants.c:74-109 q8_0): sums of squares in double, scale = 1/sqrtf(mean +
// eps) with the mean rounded to float, products left to right; q8_0 with
// d = fp16(amax * (1/127)), quants rint(x * 127/amax).  Every load a step
// needs is issued before its first reduction, so a step costs one memory
// round trip plus its reductions.
#pragma once

#include "kernels.h"

namespace g4 {

__device__ __forceinline__ float rms_scale(double ss, int n, float eps) {
    const float mean = (float)(ss / n);
    return 1.0f / __builtin_sqrtf(mean + eps);
}

__device__ __forceinline__ double wave_sum_dd(double v) { return group_sum_t<64>(v); }
// Workgroup sum of doubles: wave butterflies, then the wave partials in order.
// LDS-only barriers: global loads the caller has in flight stay in flight.
__device__ __forceinline__ double wg_sum_double(double v, double *red) {
    v = wave_sum_dd(v);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
    lds_barrier();
    double r = 0.0;
    for (int w = 0; w < (int)(blockDim.x >> 6); w++) r += red[w];
    lds_barrier();
    return r;
}

// q8_0 of four consecutive values (quants.c:74-109): lane k's 4 quant bytes
// (elements 4k..4k+3 of the block) and the block's fp16 scale; the 8 lanes of
// a block call it together
__device__ __forceinline__ uint32_t q8_pack4(const float v[4], uint16_t *d16) {
    float am = fmaxf(fmaxf(fabsf(v[0]), fabsf(v[1])), fmaxf(fabsf(v[2]), fabsf(v[3])));
    am = group_max<8>(am);
    const float id = am != 0.0f ? 127.0f / am : 0.0f;
    uint32_t pk = 0;
#pragma unroll
    for (int j = 0; j < 4; j++) pk |= ((uint32_t)(int)__builtin_rintf(v[j] * id) & 0xffu) << (8 * j);
    *d16 = f2h(am * (1.0f / 127.0f));
    return pk;
}
// the same into GGUF blocks: the 8 consecutive lanes of a 32-element block all
// call this (the block is owned by all of them or none).  Group gi writes
// quants 4*(gi%8).. of block gi/8 of dst; its first lane the scale.
__device__ __forceinline__ void q8_store4(const float v[4], int gi, bool own, uint8_t *dst) {
    uint16_t d16;
    const uint32_t pk = q8_pack4(v, &d16);
    if (!own) return;
    const int b = gi >> 3, k = gi & 7;
    uint8_t *blk = dst + (size_t)b * 34;
    uint16_t *p16 = (uint16_t *)(blk + 2 + 4 * k);
    p16[0] = (uint16_t)(pk & 0xffff);
    p16[1] = (uint16_t)(pk >> 16);
    if (k == 0) *(uint16_t *)blk = d16;
}

// k_mm_few's operand layout: the byte offset of codes e .. of (block b, token
// m) with mt 16-token tiles, and the fp16 index of its scale.  Block pairs
// outermost, then tiles, then the 16 tokens of a tile, each token's 64 bytes
// holding codes 0-7 of the even block, 0-7 of the odd one, then 8-15, and so
// on; the scales in 4 tile slots per (pair, token, block).
__device__ __forceinline__ size_t few_q(int64_t b, int m, int mt, int e) {
    return ((((size_t)(b >> 1) * mt + (m >> 4)) * 16 + (m & 15)) * 64) + 16 * (e >> 3) + 8 * (b & 1) + (e & 7);
}
__device__ __forceinline__ size_t few_d(int64_t b, int m) { return ((((size_t)(b >> 1) * 16 + (m & 15)) * 2 + (b & 1)) * 4) + (m >> 4); }
// q8_store4 of token m's row into that layout
__device__ __forceinline__ void q8_store4_few(const float v[4], int gi, bool own, const FewAct &f, int m) {
    uint16_t d16;
    const uint32_t pk = q8_pack4(v, &d16);
    if (!own) return;
    const int b = gi >> 3, k = gi & 7;
    *(uint32_t *)(f.qa + few_q(b, m, f.mt, 4 * k)) = pk;
    if (k == 0) f.da[few_d(b, m)] = d16;
}
// either form: token m's row at `row`, or the layout when f.qa is set
__device__ __forceinline__ void act_store4(const float v[4], int gi, bool own, uint8_t *row, const FewAct &f, int m) {
    if (f.qa) q8_store4_few(v, gi, own, f, m);
    else q8_store4(v, gi, own, row);
}

// q4_0 of four consecutive values (quants.c:125-144 as the reference build
// computes it): the 8 consecutive lanes of a 32-element block all call this
// (the block is owned by all of them or none).  max = the element of largest
// |x| (first on ties), d = max * -0.125, id = 1/d, q = min(15,
// trunc(fma(x, id, 8.5))); lane k < 4 of a block writes bytes 4k..4k+3
// (elements 4k.. low nibbles, 16+4k.. high), its first lane the scale.
__device__ __forceinline__ void q4_store4(const float v[4], int gi, bool own, uint8_t *dst) {
    const int k = gi & 7;
    float ba = fabsf(v[0]), bv = v[0];
    int bi = 4 * k;
#pragma unroll
    for (int i = 1; i < 4; i++)
        if (fabsf(v[i]) > ba) { ba = fabsf(v[i]); bv = v[i]; bi = 4 * k + i; }
#pragma unroll
    for (int m = 1; m < 8; m <<= 1) {
        const float oa = shfl_xor(ba, m), ov = shfl_xor(bv, m);
        const int oi = shfl_xor(bi, m);
        if (oa > ba || (oa == ba && oi < bi)) { ba = oa; bv = ov; bi = oi; }
    }
    const float d = bv * -0.125f;
    const float id = d != 0.0f ? 1.0f / d : 0.0f;
    uint32_t q4 = 0;
#pragma unroll
    for (int i = 0; i < 4; i++) {
        int q = (int)__builtin_fmaf(v[i], id, 8.5f);
        q = q > 15 ? 15 : q;
        q4 |= (uint32_t)q << (8 * i);
    }
    const uint32_t hi = shfl_xor(q4, 4);
    if (own && k < 4) {
        uint8_t *blk = dst + (size_t)(gi >> 3) * 18;
        const uint32_t packed = q4 | (hi << 4);
        uint16_t *p16 = (uint16_t *)(blk + 2 + 4 * k);
        p16[0] = (uint16_t)(packed & 0xffff);
        p16[1] = (uint16_t)(packed >> 16);
        if (k == 0) *(uint16_t *)blk = f2h(d);
    }
}

__device__ __forceinline__ float4 ldf4(const float *p) { return *(const float4 *)p; }
__device__ __forceinline__ void f4(const float4 a, float o[4]) { o[0] = a.x; o[1] = a.y; o[2] = a.z; o[3] = a.w; }

// If delta: x <- x + rms(delta)*w_post (stored back).  Then act <- q8_0(rms(x)*w_pre)
// (or, with few.qa set, token m of few's layout), and y (if given) <-
// rms(x)*w_pre in fp32.
// n % 32 == 0 and n/4 <= S * blockDim.x; all threads of the workgroup call it.
template <int S>
__device__ void wg_norm_quant(float *x, const float *delta, const float *w_post, const float *w_pre, float eps, int n,
                              uint8_t *act, float *y = nullptr, const FewAct &few = FewAct(), int m = 0) {
    __shared__ double red[16];
    const int ng = n >> 2, bd = blockDim.x, t = threadIdx.x;
    float v[S][4], d[S][4], wp[S][4], wq[S][4];
    const float4 z = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
    for (int s = 0; s < S; s++) {
        const int gi = t + s * bd;
        const bool own = gi < ng;
        f4(own ? ldf4(x + 4 * gi) : z, v[s]);
        f4(own && delta ? ldf4(delta + 4 * gi) : z, d[s]);
        f4(own && delta ? ldf4(w_post + 4 * gi) : z, wp[s]);
        f4(own ? ldf4(w_pre + 4 * gi) : z, wq[s]);
    }
    if (delta) {
        double ss = 0.0;
#pragma unroll
        for (int s = 0; s < S; s++)
#pragma unroll
            for (int k = 0; k < 4; k++) ss += (double)d[s][k] * d[s][k];
        const float sc = rms_scale(wg_sum_double(ss, red), n, eps);
#pragma unroll
        for (int s = 0; s < S; s++) {
            const int gi = t + s * bd;
#pragma unroll
            for (int k = 0; k < 4; k++) v[s][k] = v[s][k] + d[s][k] * sc * wp[s][k];
            if (gi < ng) *(float4 *)(x + 4 * gi) = make_float4(v[s][0], v[s][1], v[s][2], v[s][3]);
        }
    }
    double ss = 0.0;
#pragma unroll
    for (int s = 0; s < S; s++)
#pragma unroll
        for (int k = 0; k < 4; k++) ss += (double)v[s][k] * v[s][k];
    const float sc = rms_scale(wg_sum_double(ss, red), n, eps);
#pragma unroll
    for (int s = 0; s < S; s++) {
        if (s * bd >= ng) break;                      // uniform
        const int gi = t + s * bd;
        float o[4];
#pragma unroll
        for (int k = 0; k < 4; k++) o[k] = v[s][k] * sc * wq[s][k];
        if (y && gi < ng) *(float4 *)(y + 4 * gi) = make_float4(o[0], o[1], o[2], o[3]);
        act_store4(o, gi, gi < ng, act, few, m);
    }
}

// The decode state after a step drew `id` (state: token, pos, npos, steps
// taken, flags): token <- id, pos <- pos + 1 and npos <- pos + 1 unless the
// cache is full (pos + 1 == n_ctx: pos stays, flags |= STATE_CTX_FULL), and
// the step count (the attention hand-off tags) + 1.  One thread.
__device__ __forceinline__ void state_advance(int *state, int id, int n_ctx) {
    state[0] = id;
    if (state[1] + 1 < n_ctx) {
        state[1] += 1;
        state[2] = state[1] + 1;
    } else {
        state[4] |= STATE_CTX_FULL;
    }
    state[3] += 1;
}

// First index of the maximum of logits[0..n) (sampler.c:140-144: the best
// starts at index 0 and later values must be strictly larger, so NaNs never
// win and a NaN at index 0 keeps index 0).  All threads of the workgroup
// (a multiple of 64, at most 1024) call it; bv / bi hold one slot per wave.
// Returns the index in thread 0 (other threads: their wave's partial).
__device__ __forceinline__ void argmax_merge(float &v, int &i, float v2, int i2) {
    if (v2 > v || (v2 == v && i2 < i)) { v = v2; i = i2; }
}
__device__ __forceinline__ int wg_first_argmax(const float *logits, int n, float *bv, int *bi) {
    const int t = threadIdx.x, nt = blockDim.x, lane = t & 63, wave = t >> 6;
    float best = -INFINITY;
    int idx = 0x7fffffff;
    const int ng = n >> 2;
    for (int base = 0; base < ng; base += 8 * nt) {
        float4 v[8];
#pragma unroll
        for (int k = 0; k < 8; k++) {
            const int gi = base + k * nt + t;
            v[k] = gi < ng ? ldf4(logits + 4 * gi) : make_float4(-INFINITY, -INFINITY, -INFINITY, -INFINITY);
        }
#pragma unroll
        for (int k = 0; k < 8; k++) {
            const int gi = base + k * nt + t;
            const float e[4] = {v[k].x, v[k].y, v[k].z, v[k].w};
#pragma unroll
            for (int j = 0; j < 4; j++)
                if (e[j] > best) { best = e[j]; idx = 4 * gi + j; }
        }
    }
    for (int i = 4 * ng + t; i < n; i += nt)
        if (logits[i] > best) { best = logits[i]; idx = i; }
    for (int k = 32; k >= 1; k >>= 1) argmax_merge(best, idx, __shfl_xor(best, k, 64), __shfl_xor(idx, k, 64));
    if (lane == 0) { bv[wave] = best; bi[wave] = idx; }
    __syncthreads();
    if (t == 0) {
        for (int w = 1; w < (nt >> 6); w++) argmax_merge(best, idx, bv[w], bi[w]);
        idx = (idx == 0x7fffffff || __builtin_isnan(logits[0])) ? 0 : idx;
    }
    return idx;
}

}  // namespace g4
