#pragma once
// Deterministic synthetic data: counter-based normal draws, so any element can be made on
// any thread (or on the device) without replaying a sequential generator.
//
//   key(seed, stream)   = mix(mix(seed) ^ (stream * 0xD1B54A32D192ED03))
//   u_j                 = mix(key + j)                 (mix = splitmix64 finaliser)
//   normal(seed,stream,i) = sqrt(-2 ln(((u_2i >> 11) + 1) 2^-53)) * cos(2 pi (u_2i+1 >> 11) 2^-53)
//
// The same formulas run in the device fill kernels (rounding of the double-precision
// log / cos may differ in the last bit between host libm and device libm).
#include <cstdint>
#include <cmath>

namespace q35synth {

inline uint64_t mix64(uint64_t x) {
    x += 0x9E3779B97F4A7C15ULL;
    x = (x ^ (x >> 30)) * 0xBF58476D1CE4E5B9ULL;
    x = (x ^ (x >> 27)) * 0x94D049BB133111EBULL;
    return x ^ (x >> 31);
}

inline uint64_t stream_key(uint64_t seed, uint64_t stream) {
    return mix64(mix64(seed) ^ (stream * 0xD1B54A32D192ED03ULL));
}

inline double normal_at(uint64_t key, uint64_t i) {
    const uint64_t a = mix64(key + 2 * i), b = mix64(key + 2 * i + 1);
    const double u1 = (static_cast<double>(a >> 11) + 1.0) * (1.0 / 9007199254740992.0);
    const double u2 = static_cast<double>(b >> 11) * (1.0 / 9007199254740992.0);
    return std::sqrt(-2.0 * std::log(u1)) * std::cos(6.283185307179586 * u2);
}

// FNV-1a of a tensor name: the stream id of that tensor's values.
inline uint64_t name_stream(const char* s) {
    uint64_t h = 0xcbf29ce484222325ULL;
    for (; *s; ++s) {
        h ^= static_cast<unsigned char>(*s);
        h *= 0x100000001b3ULL;
    }
    return h;
}

// fp32 -> bf16, round to nearest even.
inline uint16_t f32_to_bf16(float f) {
    uint32_t u;
    __builtin_memcpy(&u, &f, 4);
    if ((u & 0x7fffffffu) > 0x7f800000u) return static_cast<uint16_t>((u >> 16) | 0x40);
    u += 0x7fffu + ((u >> 16) & 1u);
    return static_cast<uint16_t>(u >> 16);
}

}  // namespace q35synth
