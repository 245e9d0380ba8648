// k_quant.hip -- activation quantizers (q8_0, q8_K, q4_0), dequantization,
// GGUF-row <-> resident-layout repacking and a raw-row vec_dot.
//
// The quantizers reproduce the reference build bit for bit (quants.c:71-175
// compiled with the README's -Ofast -ffp-contract=fast):
//   q8_0: d = fp16(amax * fp32(1/127)), id = 127/amax (correctly rounded
//         division), q = rint(x*id);
//   q8_K: q = rne(exact iscale*x) via one fma, d = max * fp32(-1/127);
//   q4_0: d = max * -0.125, id = 1/d, q = min(15, trunc(fma(x, id, 8.5))).
#include "formats.h"
#include "kernels.h"

namespace g4 {

// ------------------------------------------------------------------ q8_0 --
// 8 lanes per 32-element block, 4 elements per lane.
template <bool VEC>
__global__ __launch_bounds__(256) void k_quantize_q8_0(const float *__restrict__ x, size_t xs, uint8_t *__restrict__ y,
                                                       size_t ys, int nb, int rows) {
    const int64_t gid = (int64_t)blockIdx.x * 256 + threadIdx.x;
    const int64_t total = (int64_t)rows * nb;
    const int64_t blk = gid >> 3;
    const int k = (int)(gid & 7);
    const bool ok = blk < total;
    const int64_t bb = ok ? blk : total - 1;
    const int64_t r = bb / nb;
    const int b = (int)(bb - r * nb);
    const float *src = x + r * xs + (size_t)b * 32 + 4 * k;
    float v[4];
    if constexpr (VEC) {
        const float4 f = *(const float4 *)src;
        v[0] = f.x; v[1] = f.y; v[2] = f.z; v[3] = f.w;
    } else {
        for (int i = 0; i < 4; i++) v[i] = src[i];
    }
    float am = fmaxf(fmaxf(fabsf(v[0]), fabsf(v[1])), fmaxf(fabsf(v[2]), fabsf(v[3])));
    am = group_max<8>(am);
    const float id = am != 0.0f ? 127.0f / am : 0.0f;
    uint32_t packed = 0;
#pragma unroll
    for (int i = 0; i < 4; i++) packed |= ((uint32_t)(int)__builtin_rintf(v[i] * id) & 0xffu) << (8 * i);
    if (ok) {
        uint8_t *blkp = y + r * ys + (size_t)b * 34;
        uint16_t *p16 = (uint16_t *)(blkp + 2 + 4 * k);
        p16[0] = (uint16_t)(packed & 0xffff);
        p16[1] = (uint16_t)(packed >> 16);
        if (k == 0) *(uint16_t *)blkp = f2h(am * (1.0f / 127.0f));
    }
}

// ------------------------------------------------------------------ q8_K --
// One wave per 256-element superblock, 4 consecutive elements per lane.
__global__ __launch_bounds__(256) void k_quantize_q8_K(const float *__restrict__ x, size_t xs, uint8_t *__restrict__ y,
                                                       size_t ys, int nb, int rows) {
    const int64_t w = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    const int l = threadIdx.x & 63;
    const int64_t total = (int64_t)rows * nb;
    const bool ok = w < total;
    const int64_t ww = ok ? w : total - 1;
    const int64_t r = ww / nb;
    const int sb = (int)(ww - r * nb);
    const float *src = x + r * xs + (size_t)sb * 256 + 4 * l;
    float v[4];
    for (int i = 0; i < 4; i++) v[i] = src[i];
    const Q8KLane q = q8K_wave(v);
    if (ok) {
        uint8_t *blk = y + r * ys + (size_t)sb * 292;
        ((uint32_t *)(blk + 4))[l] = q.pk;
        if ((l & 3) == 0) ((int16_t *)(blk + 260))[l >> 2] = (int16_t)q.s16;
        if (l == 0) *(float *)blk = q.d;
    }
}

// ------------------------------------------------------------------ q4_0 --
// 8 lanes per block; lane k < 4 packs elements 4k..4k+3 with 16+4k..16+4k+3.
__global__ __launch_bounds__(256) void k_quantize_q4_0(const float *__restrict__ x, size_t xs, uint8_t *__restrict__ y,
                                                       size_t ys, int nb, int rows) {
    const int64_t gid = (int64_t)blockIdx.x * 256 + threadIdx.x;
    const int64_t total = (int64_t)rows * nb;
    const int64_t blk = gid >> 3;
    const int k = (int)(gid & 7);
    const bool ok = blk < total;
    const int64_t bb = ok ? blk : total - 1;
    const int64_t r = bb / nb;
    const int b = (int)(bb - r * nb);
    const float *src = x + r * xs + (size_t)b * 32 + 4 * k;
    float v[4];
    for (int i = 0; i < 4; i++) v[i] = src[i];
    float ba = fabsf(v[0]), bv = v[0];
    int bi = 4 * k;
    for (int i = 1; i < 4; i++)
        if (fabsf(v[i]) > ba) { ba = fabsf(v[i]); bv = v[i]; bi = 4 * k + i; }
    for (int m = 1; m < 8; m <<= 1) {
        const float oa = shfl_xor(ba, m), ov = shfl_xor(bv, m);
        const int oi = shfl_xor(bi, m);
        if (oa > ba || (oa == ba && oi < bi)) { ba = oa; bv = ov; bi = oi; }
    }
    const float d = bv * -0.125f;
    const float id = d != 0.0f ? 1.0f / d : 0.0f;
    uint32_t q4 = 0;
    for (int i = 0; i < 4; i++) {
        int q = (int)__builtin_fmaf(v[i], id, 8.5f);
        q = q > 15 ? 15 : q;
        q4 |= (uint32_t)q << (8 * i);
    }
    const uint32_t hi = shfl_xor(q4, 4);
    if (ok && k < 4) {
        uint8_t *blkp = y + r * ys + (size_t)b * 18;
        const uint32_t packed = q4 | (hi << 4);
        uint16_t *p16 = (uint16_t *)(blkp + 2 + 4 * k);
        p16[0] = (uint16_t)(packed & 0xffff);
        p16[1] = (uint16_t)(packed >> 16);
        if (k == 0) *(uint16_t *)blkp = f2h(d);
    }
}

// -------------------------------------------------------------- dequant --
__device__ __forceinline__ uint16_t ld16(const uint8_t *p) { return (uint16_t)(p[0] | (p[1] << 8)); }

// q4_K (scale, min) pair j of the 12 packed bytes (quants.c:417-423)
__device__ __forceinline__ void q4k_sm(const uint8_t *s, int j, int &sc, int &mn) {
    if (j < 4) { sc = s[j] & 63; mn = s[j + 4] & 63; }
    else { sc = (s[j + 4] & 15) | ((s[j - 4] >> 6) << 4); mn = (s[j + 4] >> 4) | ((s[j] >> 6) << 4); }
}

// One thread per element; every product below is exact in fp32, so only the
// final subtraction rounds (as in quants.c:364-495).
__global__ __launch_bounds__(256) void k_dequant(int type, const uint8_t *__restrict__ x, size_t xs, float *__restrict__ y,
                                                 size_t ys, int64_t n, int rows, const int *__restrict__ ridx) {
    const int64_t gid = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (gid >= n * rows) return;
    const int64_t r = gid / n, e = gid - r * n;
    const uint8_t *row = x + (ridx ? (int64_t)ridx[r] : r) * xs;       // ridx: source rows chosen on the device
    float out;
    switch (type) {
    case Q8_0: {
        const uint8_t *b = row + (e >> 5) * 34;
        out = (float)(int8_t)b[2 + (e & 31)] * h2f(ld16(b));
    } break;
    case Q4_0: {
        const uint8_t *b = row + (e >> 5) * 18;
        const int j = (int)(e & 31);
        const int q = j < 16 ? (b[2 + j] & 15) : (b[2 + j - 16] >> 4);
        out = (float)(q - 8) * h2f(ld16(b));
    } break;
    case Q2_K: {
        const uint8_t *b = row + (e >> 8) * 84;
        const int ee = (int)(e & 255), h = ee >> 7, j = (ee >> 5) & 3, k = (ee >> 4) & 1, l = ee & 15;
        const int q = (b[16 + 32 * h + 16 * k + l] >> (2 * j)) & 3;
        const int sc = b[ee >> 4];
        out = h2f(ld16(b + 80)) * (float)(sc & 15) * (float)q - h2f(ld16(b + 82)) * (float)(sc >> 4);
    } break;
    case Q3_K: {
        const uint8_t *b = row + (e >> 8) * 110;
        const int ee = (int)(e & 255), h = ee >> 7, j = (ee >> 5) & 3, l = ee & 31;
        const int lo = (b[32 + 32 * h + l] >> (2 * j)) & 3;
        const int hb = (b[l] >> (4 * h + j)) & 1;
        const int i = ee >> 4;
        const int s4 = i < 8 ? (b[96 + i] & 15) : (b[96 + i - 8] >> 4);
        const int s2 = (b[96 + 8 + (i & 3)] >> (2 * (i >> 2))) & 3;
        out = h2f(ld16(b + 108)) * (float)((s4 | (s2 << 4)) - 32) * (float)(lo - (hb ? 0 : 4));
    } break;
    case Q4_K: {
        const uint8_t *b = row + (e >> 8) * 144;
        const int ee = (int)(e & 255), p = ee >> 6, hi = (ee >> 5) & 1, l = ee & 31;
        const int byte = b[16 + 32 * p + l];
        const int q = hi ? (byte >> 4) : (byte & 15);
        int sc, mn;
        q4k_sm(b + 4, ee >> 5, sc, mn);
        out = h2f(ld16(b)) * (float)sc * (float)q - h2f(ld16(b + 2)) * (float)mn;
    } break;
    case Q5_K: {                                                   // quants.c:497-515
        const uint8_t *b = row + (e >> 8) * 176;
        const int ee = (int)(e & 255), c = ee >> 5, l = ee & 31;
        const int byte = b[48 + 32 * (c >> 1) + l];
        const int q = ((c & 1) ? byte >> 4 : byte & 15) + (((b[16 + l] >> c) & 1) << 4);
        int sc, mn;
        q4k_sm(b + 4, c, sc, mn);
        out = h2f(ld16(b)) * (float)sc * (float)q - h2f(ld16(b + 2)) * (float)mn;
    } break;
    case Q6_K: {                                                   // quants.c:379-400
        const uint8_t *b = row + (e >> 8) * 210;
        const int ee = (int)(e & 255), h = ee >> 7, j = (ee >> 5) & 3, l = ee & 31;
        const int byte = b[64 * h + 32 * (j & 1) + l];
        const int q = ((j >= 2 ? byte >> 4 : byte & 15) | (((b[128 + 32 * h + l] >> (2 * j)) & 3) << 4)) - 32;
        out = h2f(ld16(b + 208)) * (float)(int8_t)b[192 + (ee >> 4)] * (float)q;
    } break;
    case TQ2_0: {                                                  // quants.c:402-411
        const uint8_t *b = row + (e >> 8) * 66;
        const int ee = (int)(e & 255), h = ee >> 7, j = (ee >> 5) & 3, k = (ee >> 4) & 1, l = ee & 15;
        const int q = (b[32 * h + 16 * k + l] >> (2 * j)) & 3;
        out = (float)(q - 1) * h2f(ld16(b + 64));
    } break;
    case F16: out = h2f(ld16(row + 2 * e)); break;
    case BF16: out = __uint_as_float((uint32_t)ld16(row + 2 * e) << 16); break;      // quants.c:520
    default: out = ((const float *)row)[e]; break;
    }
    y[r * ys + e] = out;
}

// ------------------------------------------------------------- repacking --
// One thread per (row, block): GGUF block bytes <-> resident planes.
template <bool TO_PLANES>
__global__ __launch_bounds__(256) void k_repack(g4h_tensor t, uint8_t *__restrict__ rows) {
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= t.nrows * t.nb) return;
    const int bs = bsize(t.type);
    uint8_t *g = rows + i * bs;   // rows are contiguous, so block i of the flat row-major stream
    auto mv = [&](uint8_t *plane, int off, int len) {
        for (int k = 0; k < len; k++) {
            if (TO_PLANES) plane[k] = g[off + k];
            else g[off + k] = plane[k];
        }
    };
    switch (t.type) {
    case Q8_0: mv(t.sc + i * 2, 0, 2); mv(t.qs + i * 16, 2, 16); mv(t.ex + i * 16, 18, 16); break;
    case Q4_0: mv(t.sc + i * 2, 0, 2); mv(t.qs + i * 16, 2, 16); break;
    case Q4_K: mv(t.qs + i * 144, 0, 144); break;
    case Q5_K: mv(t.qs + i * 176, 0, 176); break;
    case Q2_K: mv(t.sc + i * 16, 0, 16); mv(t.qs + i * 64, 16, 64); mv(t.ex + i * 4, 80, 4); break;
    case Q3_K: mv(t.ex + i * 32, 0, 32); mv(t.qs + i * 64, 32, 64); mv(t.sc + i * 12, 96, 12); mv(t.dd + i * 2, 108, 2); break;
    case Q6_K: mv(t.qs + i * 128, 0, 128); mv(t.ex + i * 64, 128, 64); mv(t.sc + i * 16, 192, 16); mv(t.dd + i * 2, 208, 2); break;
    case TQ2_0: mv(t.qs + i * 64, 0, 64); mv(t.sc + i * 2, 64, 2); break;
    case F16: case BF16: mv(t.qs + i * 2, 0, 2); break;
    default: break;
    }
}

// -------------------------------------------------------- raw-row vec_dot --
// g4_dot_<fmt> over raw (unaligned) GGUF rows: the row's blocks are gathered
// into the resident planes' register form with byte loads, one wave per row,
// then the same unit arithmetic as the GEMV.
template <class F>
__device__ void raw_frag(typename F::Frag &f, const uint8_t *row, int u);

__device__ __forceinline__ int ldu32(const uint8_t *p) { return (int)(p[0] | (p[1] << 8) | (p[2] << 16) | ((uint32_t)p[3] << 24)); }
__device__ __forceinline__ int4 ldu128(const uint8_t *p) { return make_int4(ldu32(p), ldu32(p + 4), ldu32(p + 8), ldu32(p + 12)); }

template <> __device__ void raw_frag<FQ8_0>(FQ8_0::Frag &f, const uint8_t *row, int u) {
    const uint8_t *b = row + (size_t)u * 34;
    f.d = ld16(b); f.w0 = ldu128(b + 2); f.w1 = ldu128(b + 18);
}
template <> __device__ void raw_frag<FQ4_0>(FQ4_0::Frag &f, const uint8_t *row, int u) {
    const uint8_t *b = row + (size_t)u * 18;
    f.d = ld16(b); f.w = ldu128(b + 2);
}
template <> __device__ void raw_frag<FQ4_K>(FQ4_K::Frag &f, const uint8_t *row, int u) {
    const uint8_t *b = row + (size_t)(u >> 2) * 144;
    const int p = u & 3;
    f.h = ldu128(b); f.q0 = ldu128(b + 16 + 32 * p); f.q1 = ldu128(b + 32 + 32 * p);
}
template <> __device__ void raw_frag<FQ2_K>(FQ2_K::Frag &f, const uint8_t *row, int u) {
    const uint8_t *b = row + (size_t)(u >> 2) * 84;
    f.s = ldu128(b); f.q = ldu128(b + 16 + 16 * (u & 3)); f.dd = (uint32_t)ldu32(b + 80);
}
template <> __device__ void raw_frag<FQ3_K>(FQ3_K::Frag &f, const uint8_t *row, int u) {
    const uint8_t *b = row + (size_t)(u >> 2) * 110;
    const int p = u & 3;
    f.hm = ldu128(b + 16 * (p & 1)); f.q = ldu128(b + 32 + 16 * p);
    f.s0 = ldu32(b + 96); f.s1 = ldu32(b + 100); f.s2 = ldu32(b + 104); f.d = ld16(b + 108);
}

template <> __device__ void raw_frag<FQ5_K>(FQ5_K::Frag &f, const uint8_t *row, int u) {
    const uint8_t *b = row + (size_t)(u >> 2) * 176;
    const int p = u & 3;
    f.h = ldu128(b); f.hb0 = ldu128(b + 16); f.hb1 = ldu128(b + 32);
    f.q0 = ldu128(b + 48 + 32 * p); f.q1 = ldu128(b + 64 + 32 * p);
}
template <> __device__ void raw_frag<FQ6_K>(FQ6_K::Frag &f, const uint8_t *row, int u) {
    const uint8_t *b = row + (size_t)(u >> 2) * 210;
    const int p = u & 3, h = p >> 1, k = p & 1;
    f.l0 = ldu128(b + 64 * h + 16 * k); f.l1 = ldu128(b + 64 * h + 32 + 16 * k); f.hb = ldu128(b + 128 + 32 * h + 16 * k);
    f.s = make_uint2((uint32_t)ldu32(b + 192 + 8 * h), (uint32_t)ldu32(b + 196 + 8 * h)); f.d = ld16(b + 208);
}

template <> __device__ void raw_frag<FTQ2_0>(FTQ2_0::Frag &f, const uint8_t *row, int u) {
    const uint8_t *b = row + (size_t)(u >> 2) * 66;
    f.q = ldu128(b + 16 * (u & 3)); f.d = ld16(b + 64);
}

template <class F>
__global__ __launch_bounds__(256) void k_vec_dot_raw(const uint8_t *__restrict__ w, size_t ws, const uint8_t *__restrict__ a,
                                                     int nblk, int rows, float *__restrict__ out) {
    extern __shared__ __align__(16) uint8_t lds[];
    if constexpr (F::type == Q4_0 || F::type == Q8_0) stage_q8_0<1>(lds, a, 0, nblk);
    else stage_q8_K<1>(lds, a, 0, nblk);
    __syncthreads();
    const int64_t r = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    const int64_t rr = r < rows ? r : rows - 1;
    const int units = nblk * F::units_per_block;
    float acc = 0.0f;
    for (int u = lane; u < units; u += 64) {
        typename F::Frag f;
        raw_frag<F>(f, w + rr * ws, u);
        acc = F::accum(f, typename F::Act(lds, nblk, 0), u, acc);
    }
    acc = group_sum<64>(acc);
    if (lane == 0 && r < rows) out[r] = acc;
}

// ------------------------------------------------------------- launchers --
static unsigned nblocks(int64_t threads) { return (unsigned)((threads + 255) / 256); }

hipError_t launch_quantize_q8_0(const float *x, size_t xs, uint8_t *y, size_t ys, int64_t n, int rows, hipStream_t s) {
    const int nb = (int)(n / 32);
    const bool vec = ((uintptr_t)x % 16 == 0) && (xs % 4 == 0);
    if (vec) hipLaunchKernelGGL(k_quantize_q8_0<true>, dim3(nblocks((int64_t)rows * nb * 8)), dim3(256), 0, s, x, xs, y, ys, nb, rows);
    else hipLaunchKernelGGL(k_quantize_q8_0<false>, dim3(nblocks((int64_t)rows * nb * 8)), dim3(256), 0, s, x, xs, y, ys, nb, rows);
    return hipGetLastError();
}
hipError_t launch_quantize_q8_K(const float *x, size_t xs, uint8_t *y, size_t ys, int64_t n, int rows, hipStream_t s) {
    const int nb = (int)(n / 256);
    hipLaunchKernelGGL(k_quantize_q8_K, dim3((unsigned)(((int64_t)rows * nb + 3) / 4)), dim3(256), 0, s, x, xs, y, ys, nb, rows);
    return hipGetLastError();
}
hipError_t launch_quantize_q4_0(const float *x, size_t xs, uint8_t *y, size_t ys, int64_t n, int rows, hipStream_t s) {
    const int nb = (int)(n / 32);
    hipLaunchKernelGGL(k_quantize_q4_0, dim3(nblocks((int64_t)rows * nb * 8)), dim3(256), 0, s, x, xs, y, ys, nb, rows);
    return hipGetLastError();
}
hipError_t launch_dequant(int type, const uint8_t *x, size_t xs, float *y, size_t ys, int64_t n, int rows, hipStream_t s,
                          const int *ridx) {
    hipLaunchKernelGGL(k_dequant, dim3(nblocks(n * rows)), dim3(256), 0, s, type, x, xs, y, ys, n, rows, ridx);
    return hipGetLastError();
}
hipError_t launch_repack(const g4h_tensor &t, const uint8_t *rows, hipStream_t s) {
    hipLaunchKernelGGL(k_repack<true>, dim3(nblocks(t.nrows * t.nb)), dim3(256), 0, s, t, const_cast<uint8_t *>(rows));
    return hipGetLastError();
}
hipError_t launch_unpack(const g4h_tensor &t, uint8_t *rows, hipStream_t s) {
    hipLaunchKernelGGL(k_repack<false>, dim3(nblocks(t.nrows * t.nb)), dim3(256), 0, s, t, rows);
    return hipGetLastError();
}

template <class F>
static hipError_t vd_go(const uint8_t *w, size_t ws, const uint8_t *a, int64_t n, int rows, float *out, hipStream_t s) {
    const int nblk = (int)(n / blck(F::type));
    hipLaunchKernelGGL(k_vec_dot_raw<F>, dim3((unsigned)((rows + 3) / 4)), dim3(256), F::Act::bytes_per_token(nblk) + kStageDump, s,
                       w, ws, a, nblk, rows, out);
    return hipGetLastError();
}
hipError_t launch_vec_dot_raw(int wtype, const uint8_t *w, size_t ws, const uint8_t *a, int64_t n, int rows, float *out,
                              hipStream_t s) {
    switch (wtype) {
    case Q8_0: return vd_go<FQ8_0>(w, ws, a, n, rows, out, s);
    case Q4_0: return vd_go<FQ4_0>(w, ws, a, n, rows, out, s);
    case Q4_K: return vd_go<FQ4_K>(w, ws, a, n, rows, out, s);
    case Q3_K: return vd_go<FQ3_K>(w, ws, a, n, rows, out, s);
    case Q2_K: return vd_go<FQ2_K>(w, ws, a, n, rows, out, s);
    case Q5_K: return vd_go<FQ5_K>(w, ws, a, n, rows, out, s);
    case Q6_K: return vd_go<FQ6_K>(w, ws, a, n, rows, out, s);
    case TQ2_0: return vd_go<FTQ2_0>(w, ws, a, n, rows, out, s);
    default: return hipErrorInvalidValue;
    }
}

}  // namespace g4
