// host_fp16.h -- host-side fp16 conversions and the fp16 GELU table, shared by
// the decode-step model and the g4run.h-compatible entry points (internal).
#pragma once
#include <cmath>
#include <cstdint>
#include <cstring>

namespace g4 {

// IEEE-754 binary16 -> binary32, exact (subnormals normalised, NaN payloads kept).
inline float host_h2f(uint16_t h) {
    const uint32_t sign = (uint32_t)(h >> 15) << 31, e = (h >> 10) & 31u, m = h & 1023u;
    uint32_t u;
    if (e == 31) u = sign | 0x7f800000u | (m << 13);
    else if (e == 0) {
        if (m == 0) u = sign;
        else {
            float f = std::ldexp((float)m, -24);
            std::memcpy(&u, &f, 4);
            u |= sign;
        }
    } else u = sign | ((e + 112u) << 23) | (m << 13);
    float f;
    std::memcpy(&f, &u, 4);
    return f;
}

// binary32 -> binary16, round to nearest even with gradual underflow; NaN
// stays a quiet NaN with its top payload bits, overflow goes to infinity.
inline uint16_t host_f2h(float f) {
    uint32_t u;
    std::memcpy(&u, &f, 4);
    const uint16_t sign = (uint16_t)((u >> 16) & 0x8000u);
    const uint32_t mag = u & 0x7fffffffu;
    if (mag > 0x7f800000u) return (uint16_t)(sign | 0x7e00u | ((mag >> 13) & 1023u ? (mag >> 13) & 1023u : 1u));
    if (mag >= 0x47800000u) return (uint16_t)(sign | 0x7c00u);
    if (mag < 0x38800000u) {
        // subnormal result: value / 2^-24 rounded half-even
        const float scaled = std::fabs(f) * 16777216.0f;           // exact (power-of-two scaling)
        return (uint16_t)(sign | (uint16_t)std::nearbyint(scaled));
    }
    const uint32_t r = mag + 0x0fffu + ((mag >> 13) & 1u);
    return (uint16_t)(sign | ((r - 0x38000000u) >> 13));
}

// The fp16 GELU table (quants.c:48-58): entry h = fp16(gelu_tanh(fp32(h))).
inline uint16_t gelu_table_entry(uint16_t h) {
    const float x = host_h2f(h);
    const float g = 0.5f * x * (1.0f + tanhf(0.79788456080286535587989211986876f * x * (1.0f + 0.044715f * x * x)));
    return host_f2h(g);
}

}  // namespace g4
