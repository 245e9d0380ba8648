// handoff.h -- values handed from workgroup to workgroup inside one launch.
//
// Every published value is a 64-bit word, the value's bits low and the
// launch's tag high, stored at agent scope (coherent across the XCDs' L2
// caches).  A 64-bit store is single-copy atomic, so a reader that sees the
// current tag sees the value stored with it; readers poll until every word
// they need carries the tag, and give up after a bounded number of retries
// (the caller then writes NaN and sets an error word), so a launch always
// ends.
#pragma once
#include <hip/hip_runtime.h>
#include <cstdint>

#ifndef ATT_POLL_SLEEP
#define ATT_POLL_SLEEP 1
#endif

namespace g4 {

// loads and stores of data shared between the workgroups of one launch:
// agent scope, coherent across the XCDs' L2 caches
template <class T>
__device__ __forceinline__ T ld_ag(const T *p) {
    return __hip_atomic_load(const_cast<T *>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
template <class T>
__device__ __forceinline__ void st_ag(T *p, T v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

__device__ __forceinline__ void st_tag(uint64_t *p, uint32_t bits, uint32_t tag) { st_ag(p, ((uint64_t)tag << 32) | bits); }

// N tagged words: all loads issued together; while any tag is not yet
// current, the stale words are reloaded together
template <int N>
__device__ __forceinline__ bool poll_words(const uint64_t *const (&src)[N], const bool (&need)[N], uint32_t tag,
                                           uint32_t (&bits)[N], unsigned spin) {
    uint64_t w[N];
#pragma unroll
    for (int k = 0; k < N; k++) w[k] = need[k] ? ld_ag(src[k]) : ((uint64_t)tag << 32);
    for (unsigned it = 0;; it++) {
        bool all = true;
#pragma unroll
        for (int k = 0; k < N; k++) all &= (uint32_t)(w[k] >> 32) == tag;
        if (all) break;
        if (it >= spin) return false;
        __builtin_amdgcn_s_sleep(ATT_POLL_SLEEP);
#pragma unroll
        for (int k = 0; k < N; k++)
            if ((uint32_t)(w[k] >> 32) != tag) w[k] = ld_ag(src[k]);
    }
#pragma unroll
    for (int k = 0; k < N; k++) bits[k] = (uint32_t)w[k];
    return true;
}

}  // namespace g4
