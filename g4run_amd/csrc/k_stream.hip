// k_stream.hip -- the read floor: one launch that reads a byte range once with
// the GEMV's 128-bit non-temporal loads and does nothing else.  It is the
// yardstick the GEMV launches are measured against (what the memory system
// gives one launch of that many bytes, ramp and drain included); nothing on the
// path calls it.
#include <algorithm>

#include "kernels.h"

namespace g4 {

// Workgroup g's thread t loads 16-byte chunks g*T*L + k*T + t, k < L (clamped
// to the last chunk), XORs them and, for i = g*T + t < ny, writes one float of
// y (the per-row output a GEMV writes).  The XOR is compared with a constant
// (a match writes y[0]) so the compiler cannot drop the loads.
template <int L>
__global__ __launch_bounds__(1024) void k_read_floor(const int4 *__restrict__ p, int64_t n16, float *__restrict__ y, int64_t ny) {
    const int64_t T = blockDim.x;
    const int64_t base = (int64_t)blockIdx.x * T * L + threadIdx.x;
    int4 v[L];
#pragma unroll
    for (int k = 0; k < L; k++) v[k] = ld4s(p + min(base + k * T, n16 - 1));
    int x = 0;
#pragma unroll
    for (int k = 0; k < L; k++) x ^= v[k].x ^ v[k].y ^ v[k].z ^ v[k].w;
    const int64_t i = (int64_t)blockIdx.x * T + threadIdx.x;
    if (i < ny) y[i] = (float)(x & 1);
    else if (x == 0x5eed1e55 && y) y[0] = 1.0f;
}

hipError_t launch_read_floor(const uint8_t *p, size_t bytes, float *y, int64_t ny, int threads, int loads, hipStream_t s) {
    if (!p || bytes < 16 || bytes % 16 || threads < 64 || threads > 1024 || threads % 64 || loads < 1 || loads > 8 ||
        ny < 0 || (ny > 0 && !y))
        return hipErrorInvalidValue;
    const int64_t n16 = (int64_t)(bytes / 16), per = (int64_t)threads * loads;
    const int64_t grid = std::max((n16 + per - 1) / per, (ny + threads - 1) / threads);
    if (grid > 0x7fffffff) return hipErrorInvalidValue;
#define G4_RF(L_)                                                                                                   \
    case L_: hipLaunchKernelGGL(k_read_floor<L_>, dim3((unsigned)grid), dim3(threads), 0, s, (const int4 *)p, n16, y, ny); break
    switch (loads) {
        G4_RF(1); G4_RF(2); G4_RF(3); G4_RF(4); G4_RF(5); G4_RF(6); G4_RF(7); G4_RF(8);
    }
#undef G4_RF
    return hipGetLastError();
}

}  // namespace g4
