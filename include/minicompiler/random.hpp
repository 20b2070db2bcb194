#pragma once

// Seeded initialisation. fill_uniform keeps the reference's contract
// (include/minicompiler/random.hpp:15-16, src/random.cpp:6-26): splitmix64,
// the top 24 bits of each draw as an exact float u in [0,1), and
// lo + (hi - lo) * u with the multiply and the add rounded separately.
//
// fill_normal is an addition of this backend (the reference has no normal
// generator, but the BatchNorm workload asks for normal(0,1) data): each
// pair of outputs comes from two consecutive splitmix64 draws u1, u2 (53-bit
// doubles in (0,1] and [0,1)) through Box-Muller in double precision,
// z0 = r cos(2 pi u2), z1 = r sin(2 pi u2), r = sqrt(-2 ln u1), and
// mean + stddev * z rounded once to float.

#include <cstddef>
#include <cstdint>
#include <vector>

namespace minicompiler {

void fill_uniform(float* out, std::size_t count, std::uint64_t seed, float lo, float hi);
std::vector<float> uniform_values(std::size_t count, std::uint64_t seed, float lo, float hi);

void fill_normal(float* out, std::size_t count, std::uint64_t seed, double mean, double stddev);
std::vector<float> normal_values(std::size_t count, std::uint64_t seed, double mean, double stddev);

}  // namespace minicompiler
