// Seeded generators (reference: src/random.cpp:6-33 for fill_uniform).

#include "minicompiler/random.hpp"

#include <cmath>

namespace minicompiler {

namespace {

// splitmix64 (Steele, Lea, Flood, "Fast splittable pseudorandom number
// generators", OOPSLA 2014): add the golden-ratio increment, then a
// xor-shift / multiply finaliser.
inline std::uint64_t next_splitmix64(std::uint64_t& state) {
    state += 0x9E3779B97F4A7C15ull;
    std::uint64_t z = state;
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

}  // namespace

void fill_uniform(float* out, std::size_t count, std::uint64_t seed, float lo, float hi) {
    std::uint64_t state = seed;
    const float width = hi - lo;
    for (std::size_t i = 0; i < count; ++i) {
        // 24 random bits scaled by 2^-24: an exact float in [0, 1).
        const float u = static_cast<float>(next_splitmix64(state) >> 40) * (1.0f / 16777216.0f);
        // Two separately rounded steps; volatile stops the compiler from
        // contracting them into one fused multiply-add.
        volatile float scaled = width * u;
        out[i] = lo + scaled;
    }
}

std::vector<float> uniform_values(std::size_t count, std::uint64_t seed, float lo, float hi) {
    std::vector<float> v(count);
    fill_uniform(v.data(), count, seed, lo, hi);
    return v;
}

void fill_normal(float* out, std::size_t count, std::uint64_t seed, double mean, double stddev) {
    std::uint64_t state = seed;
    const double two_pi = 6.283185307179586476925286766559;
    for (std::size_t i = 0; i < count; i += 2) {
        // 53-bit uniforms: u1 in (0, 1] keeps the logarithm finite.
        const double u1 = static_cast<double>((next_splitmix64(state) >> 11) + 1) * 0x1p-53;
        const double u2 = static_cast<double>(next_splitmix64(state) >> 11) * 0x1p-53;
        const double r = std::sqrt(-2.0 * std::log(u1));
        out[i] = static_cast<float>(mean + stddev * (r * std::cos(two_pi * u2)));
        if (i + 1 < count) out[i + 1] = static_cast<float>(mean + stddev * (r * std::sin(two_pi * u2)));
    }
}

std::vector<float> normal_values(std::size_t count, std::uint64_t seed, double mean, double stddev) {
    std::vector<float> v(count);
    fill_normal(v.data(), count, seed, mean, stddev);
    return v;
}

}  // namespace minicompiler
