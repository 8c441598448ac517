// Host input generators for the harness workloads. Built with
// -ffp-contract=off: every expression rounds exactly as written, as in the
// reference's Rust source (Rust never fuses a*b+c).
#include <cmath>
#include <cstddef>
#include <cstdint>

#include "jade_runtime_hip.h"

namespace {
inline uint32_t xorshift32(uint32_t state) {
    state ^= state << 13;
    state ^= state >> 17;
    state ^= state << 5;
    return state;
}
}  // namespace

// src/runtime/workloads.rs:17-27.
extern "C" int jr_fill_values(float *out, size_t len, uint32_t seed, float scale) {
    if (!out && len) return 1;
    uint32_t state = seed;
    for (size_t i = 0; i < len; ++i) {
        state = xorshift32(state);
        const float unit = static_cast<float>(state >> 8) / 16777216.0f * 2.0f - 1.0f;
        out[i] = unit * scale;
    }
    return 0;
}

// Box-Muller over the xorshift32 stream (two draws per value).
extern "C" int jr_fill_normal(float *out, size_t len, uint32_t seed, float mean, float sigma) {
    if (!out && len) return 1;
    const double two_pi = 6.283185307179586476925286766559;
    uint32_t state = seed;
    for (size_t i = 0; i < len; ++i) {
        state = xorshift32(state);
        const double u1 = (static_cast<double>(state >> 8) + 1.0) / 16777216.0;
        state = xorshift32(state);
        const double u2 = static_cast<double>(state >> 8) / 16777216.0;
        const double z = std::sqrt(-2.0 * std::log(u1)) * std::cos(two_pi * u2);
        out[i] = static_cast<float>(static_cast<double>(mean) + static_cast<double>(sigma) * z);
    }
    return 0;
}
