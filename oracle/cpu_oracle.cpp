// CPU oracle: fp32 restatement of the reference's Eigen CPU backend
// (src/cpu/kernels.cpp:19-277) and its seeded generator (src/random.cpp:6-26).
// TEST INFRASTRUCTURE ONLY (see oracle.h): never linked into the product.

#include "oracle.h"

#include <algorithm>
#include <cmath>
#include <cstring>
#include <thread>
#include <vector>

namespace {

int g_threads = 1;

// Runs body(begin, end) over [0, count) split into g_threads contiguous
// chunks whose boundaries are multiples of `grain`.
template <typename F>
void parallel_chunks(size_t count, size_t grain, F body) {
    const size_t units = (count + grain - 1) / grain;
    const size_t t = std::max<size_t>(1, std::min<size_t>(static_cast<size_t>(g_threads), units));
    if (t == 1) {
        body(size_t{0}, count);
        return;
    }
    std::vector<std::thread> pool;
    for (size_t w = 0; w < t; ++w) {
        const size_t b = std::min(count, units * w / t * grain);
        const size_t e = std::min(count, units * (w + 1) / t * grain);
        if (b < e) pool.emplace_back(body, b, e);
    }
    for (auto& th : pool) th.join();
}

uint64_t splitmix_next(uint64_t* s) {
    uint64_t z = (*s += 0x9E3779B97F4A7C15ull);
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

bool valid_unary(int op) { return op >= 2 && op <= 8; }
bool valid_binary(int op) { return op >= 9 && op <= 12; }

float f_unary(int op, float x) {
    switch (op) {
        case 2: return -x;
        case 3: return expf(x);
        case 4: return logf(x);
        case 5: return sqrtf(x);
        case 6: return x > 0.0f ? x : 0.0f;
        case 7: {
            const float e = expf(-x);
            const float d = 1.0f + e;
            return 1.0f / d;
        }
        case 8: return tanhf(x);
    }
    return NAN;
}

float f_binary(int op, float a, float b) {
    switch (op) {
        case 9: return a + b;
        case 10: return a - b;
        case 11: return a * b;
        case 12: return a / b;
    }
    return NAN;
}

size_t count_of(const int64_t* shape, int rank) {
    size_t n = 1;
    for (int i = 0; i < rank; ++i) n *= static_cast<size_t>(shape[i]);
    return n;
}

// Strides of `in` read at the coordinates of `out` (0 where broadcast).
std::vector<int64_t> bstrides(const int64_t* in, int in_rank, int out_rank) {
    std::vector<int64_t> s(static_cast<size_t>(out_rank), 0);
    int64_t step = 1;
    for (int r = 0; r < in_rank; ++r) {
        const int64_t d = in[in_rank - 1 - r];
        if (d != 1) s[static_cast<size_t>(out_rank - 1 - r)] = step;
        step *= d;
    }
    return s;
}

int64_t offset_of(size_t i, const int64_t* out, int out_rank, const std::vector<int64_t>& strides) {
    int64_t off = 0;
    for (int d = out_rank - 1; d >= 0; --d) {
        const auto dim = static_cast<size_t>(out[d]);
        off += static_cast<int64_t>(i % dim) * strides[static_cast<size_t>(d)];
        i /= dim;
    }
    return off;
}

// How a fused program reads one input (kernels.cpp:88-108).
struct Plan {
    enum Kind { Contiguous, Scalar, Periodic, General } kind = Contiguous;
    size_t period = 0;
    std::vector<int64_t> strides;
};

Plan plan_of(const int64_t* in, int in_rank, const int64_t* out, int out_rank) {
    Plan p;
    const size_t n_in = count_of(in, in_rank);
    if (n_in == 1) {
        p.kind = Plan::Scalar;
        return p;
    }
    if (n_in == count_of(out, out_rank)) return p;
    int lead = 0;
    while (lead < in_rank && in[lead] == 1) ++lead;
    const int rest = in_rank - lead;
    bool suffix = rest <= out_rank;
    for (int i = 0; suffix && i < rest; ++i) suffix = in[lead + i] == out[out_rank - rest + i];
    if (suffix) {
        p.kind = Plan::Periodic;
        p.period = n_in;
        return p;
    }
    p.kind = Plan::General;
    p.strides = bstrides(in, in_rank, out_rank);
    return p;
}

constexpr size_t kBlock = 512;  // kernels.hpp:18

}  // namespace

extern "C" {

void orc_set_threads(int threads) { g_threads = std::max(1, threads); }
int orc_get_threads(void) { return g_threads; }

void orc_fill_uniform(float* out, size_t count, uint64_t seed, float lo, float hi) {
    uint64_t s = seed;
    const float range = hi - lo;
    for (size_t i = 0; i < count; ++i) {
        const float u = static_cast<float>(splitmix_next(&s) >> 40) * 5.9604644775390625e-8f;  // 2^-24
        volatile float scaled = range * u;  // rounded on its own: no contraction
        out[i] = lo + scaled;
    }
}

void orc_fill_normal(float* out, size_t count, uint64_t seed, double mean, double stddev) {
    uint64_t s = seed;
    for (size_t i = 0; i < count; i += 2) {
        const double u1 = static_cast<double>((splitmix_next(&s) >> 11) + 1) / 9007199254740992.0;  // (0,1]
        const double u2 = static_cast<double>(splitmix_next(&s) >> 11) / 9007199254740992.0;        // [0,1)
        const double radius = std::sqrt(-2.0 * std::log(u1));
        const double angle = 2.0 * M_PI * u2;
        out[i] = static_cast<float>(mean + stddev * (radius * std::cos(angle)));
        if (i + 1 < count) out[i + 1] = static_cast<float>(mean + stddev * (radius * std::sin(angle)));
    }
}

int orc_unary(int op, const float* x, float* y, size_t n) {
    if (!valid_unary(op)) return 1;
    parallel_chunks(n, 4096, [&](size_t b, size_t e) {
        for (size_t i = b; i < e; ++i) y[i] = f_unary(op, x[i]);
    });
    return 0;
}

// kernels.cpp:148-190: full/full, full/scalar and scalar/full directly;
// otherwise one output row (last dimension) at a time, each operand either
// advancing along the row or repeating one element.
int orc_binary(int op, const float* a, const int64_t* as, int ar, const float* b, const int64_t* bs, int br,
               float* out, const int64_t* os, int orank) {
    if (!valid_binary(op)) return 1;
    const size_t n = count_of(os, orank);
    const size_t na = count_of(as, ar), nb = count_of(bs, br);
    if (na == n && nb == n) {
        parallel_chunks(n, 4096, [&](size_t s, size_t e) {
            for (size_t i = s; i < e; ++i) out[i] = f_binary(op, a[i], b[i]);
        });
        return 0;
    }
    if (na == n && nb == 1) {
        for (size_t i = 0; i < n; ++i) out[i] = f_binary(op, a[i], b[0]);
        return 0;
    }
    if (na == 1 && nb == n) {
        for (size_t i = 0; i < n; ++i) out[i] = f_binary(op, a[0], b[i]);
        return 0;
    }
    if (orank == 0) {
        out[0] = f_binary(op, a[0], b[0]);
        return 0;
    }
    const std::vector<int64_t> sa = bstrides(as, ar, orank), sb = bstrides(bs, br, orank);
    const auto inner = static_cast<size_t>(os[orank - 1]);
    const bool a_moves = sa[static_cast<size_t>(orank - 1)] != 0, b_moves = sb[static_cast<size_t>(orank - 1)] != 0;
    for (size_t row = 0; row < n; row += inner) {
        const int64_t oa = offset_of(row, os, orank, sa), ob = offset_of(row, os, orank, sb);
        for (size_t j = 0; j < inner; ++j) {
            out[row + j] = f_binary(op, a[oa + (a_moves ? static_cast<int64_t>(j) : 0)],
                                    b[ob + (b_moves ? static_cast<int64_t>(j) : 0)]);
        }
    }
    return 0;
}

int orc_fused(int num_instrs, const int32_t* kind, const int32_t* op, const int32_t* ra, const int32_t* rb,
              const float* imm, int num_inputs, const float* const* inputs, const int64_t* shapes,
              const int32_t* ranks, float* out, const int64_t* os, int orank) {
    if (num_instrs < 1) return 1;
    std::vector<Plan> plans;
    {
        const int64_t* s = shapes;
        for (int j = 0; j < num_inputs; ++j) {
            plans.push_back(plan_of(s, ranks[j], os, orank));
            s += ranks[j];
        }
    }
    for (int r = 0; r < num_instrs; ++r) {
        if (kind[r] == 0 && (ra[r] < 0 || ra[r] >= num_inputs)) return 1;
        if (kind[r] == 2 && (!valid_unary(op[r]) || ra[r] < 0 || ra[r] >= r)) return 1;
        if (kind[r] == 3 && (!valid_binary(op[r]) || ra[r] < 0 || ra[r] >= r || rb[r] < 0 || rb[r] >= r)) return 1;
        if (kind[r] < 0 || kind[r] > 3) return 1;
    }
    const size_t n = count_of(os, orank);
    const size_t R = static_cast<size_t>(num_instrs);
    // One thread per contiguous run of blocks, each with its own register buffers.
    parallel_chunks(n, kBlock, [&](size_t begin, size_t end) {
        std::vector<float> scratch(R * kBlock);
        struct Reg {
            const float* vec;
            float scalar;
        };
        std::vector<Reg> regs(R);
        for (size_t start = begin; start < end; start += kBlock) {
            const size_t len = std::min(kBlock, end - start);
            for (size_t r = 0; r < R; ++r) {
                float* dst = r + 1 == R ? out + start : scratch.data() + r * kBlock;
                switch (kind[r]) {
                    case 0: {
                        const Plan& p = plans[static_cast<size_t>(ra[r])];
                        const float* in = inputs[ra[r]];
                        if (p.kind == Plan::Contiguous) {
                            regs[r] = {in + start, 0.0f};
                        } else if (p.kind == Plan::Scalar) {
                            regs[r] = {nullptr, in[0]};
                        } else if (p.kind == Plan::Periodic) {
                            size_t pos = start % p.period;
                            for (size_t j = 0; j < len;) {
                                const size_t chunk = std::min(len - j, p.period - pos);
                                std::memcpy(dst + j, in + pos, chunk * sizeof(float));
                                j += chunk;
                                pos = 0;
                            }
                            regs[r] = {dst, 0.0f};
                        } else {
                            for (size_t j = 0; j < len; ++j) dst[j] = in[offset_of(start + j, os, orank, p.strides)];
                            regs[r] = {dst, 0.0f};
                        }
                        break;
                    }
                    case 1: regs[r] = {nullptr, imm[r]}; break;
                    case 2: {
                        const Reg x = regs[static_cast<size_t>(ra[r])];
                        if (!x.vec) {
                            regs[r] = {nullptr, f_unary(op[r], x.scalar)};
                        } else {
                            for (size_t j = 0; j < len; ++j) dst[j] = f_unary(op[r], x.vec[j]);
                            regs[r] = {dst, 0.0f};
                        }
                        break;
                    }
                    case 3: {
                        const Reg x = regs[static_cast<size_t>(ra[r])], y = regs[static_cast<size_t>(rb[r])];
                        if (!x.vec && !y.vec) {
                            regs[r] = {nullptr, f_binary(op[r], x.scalar, y.scalar)};
                            break;
                        }
                        for (size_t j = 0; j < len; ++j) {
                            dst[j] = f_binary(op[r], x.vec ? x.vec[j] : x.scalar, y.vec ? y.vec[j] : y.scalar);
                        }
                        regs[r] = {dst, 0.0f};
                        break;
                    }
                }
            }
            const Reg res = regs[R - 1];
            if (!res.vec) {
                std::fill(out + start, out + start + len, res.scalar);
            } else if (res.vec != out + start) {
                std::memmove(out + start, res.vec, len * sizeof(float));
            }
        }
    });
    return 0;
}

// Reference doubles (tests/test_util.cpp:87-159)

static double d_unary(int op, double x) {
    switch (op) {
        case 2: return -x;
        case 3: return std::exp(x);
        case 4: return std::log(x);
        case 5: return std::sqrt(x);
        case 6: return x > 0.0 ? x : 0.0;
        case 7: return 1.0 / (1.0 + std::exp(-x));
        case 8: return std::tanh(x);
    }
    return NAN;
}

static double d_binary(int op, double a, double b) {
    switch (op) {
        case 9: return a + b;
        case 10: return a - b;
        case 11: return a * b;
        case 12: return a / b;
    }
    return NAN;
}

int orc_ref_unary(int op, const float* x, float* y, size_t n) {
    if (!valid_unary(op)) return 1;
    for (size_t i = 0; i < n; ++i) y[i] = static_cast<float>(d_unary(op, x[i]));
    return 0;
}

int orc_ref_binary(int op, const float* a, const int64_t* as, int ar, const float* b, const int64_t* bs, int br,
                   float* out, const int64_t* os, int orank) {
    if (!valid_binary(op)) return 1;
    const std::vector<int64_t> sa = bstrides(as, ar, orank), sb = bstrides(bs, br, orank);
    const size_t n = count_of(os, orank);
    for (size_t i = 0; i < n; ++i) {
        out[i] = static_cast<float>(d_binary(op, a[offset_of(i, os, orank, sa)], b[offset_of(i, os, orank, sb)]));
    }
    return 0;
}

int orc_ref_matmul(const float* a, const float* b, float* c, int64_t m, int64_t k, int64_t n) {
    for (int64_t r = 0; r < m; ++r) {
        for (int64_t col = 0; col < n; ++col) {
            double acc = 0.0;
            for (int64_t t = 0; t < k; ++t) acc += static_cast<double>(a[r * k + t]) * b[t * n + col];
            c[r * n + col] = static_cast<float>(acc);
        }
    }
    return 0;
}

int orc_ref_fused(int num_instrs, const int32_t* kind, const int32_t* op, const int32_t* ra, const int32_t* rb,
                  const float* imm, int num_inputs, const float* const* inputs, const int64_t* shapes,
                  const int32_t* ranks, float* out, const int64_t* os, int orank) {
    std::vector<std::vector<int64_t>> strides;
    const int64_t* s = shapes;
    for (int j = 0; j < num_inputs; ++j) {
        strides.push_back(bstrides(s, ranks[j], orank));
        s += ranks[j];
    }
    const size_t n = count_of(os, orank);
    std::vector<double> regs(static_cast<size_t>(num_instrs));
    for (size_t e = 0; e < n; ++e) {
        for (int r = 0; r < num_instrs; ++r) {
            double x = 0.0;
            switch (kind[r]) {
                case 0: x = inputs[ra[r]][offset_of(e, os, orank, strides[static_cast<size_t>(ra[r])])]; break;
                case 1: x = imm[r]; break;
                case 2: x = d_unary(op[r], regs[static_cast<size_t>(ra[r])]); break;
                case 3: x = d_binary(op[r], regs[static_cast<size_t>(ra[r])], regs[static_cast<size_t>(rb[r])]); break;
                default: return 1;
            }
            regs[static_cast<size_t>(r)] = static_cast<float>(x);  // float registers, as in the kernels
        }
        out[e] = static_cast<float>(regs.back());
    }
    return 0;
}

int orc_gemm_f64(const float* a, const float* b, double* exact, double* absdot, int64_t m, int64_t k, int64_t n) {
    parallel_chunks(static_cast<size_t>(m), 1, [&](size_t r0, size_t r1) {
        for (size_t r = r0; r < r1; ++r) {
            double* ex = exact + r * static_cast<size_t>(n);
            double* ab = absdot + r * static_cast<size_t>(n);
            std::fill(ex, ex + n, 0.0);
            std::fill(ab, ab + n, 0.0);
            for (int64_t t = 0; t < k; ++t) {
                const double av = a[static_cast<int64_t>(r) * k + t];
                const float* brow = b + t * n;
                for (int64_t c = 0; c < n; ++c) {
                    const double p = av * brow[c];
                    ex[c] += p;
                    ab[c] += std::fabs(p);
                }
            }
        }
    });
    return 0;
}

int orc_gemm_f64_sampled(const float* a, const float* b, const int64_t* rows, const int64_t* cols, int64_t count,
                         double* exact, double* absdot, int64_t k, int64_t n) {
    parallel_chunks(static_cast<size_t>(count), 1, [&](size_t i0, size_t i1) {
        for (size_t i = i0; i < i1; ++i) {
            double ex = 0.0, ab = 0.0;
            for (int64_t t = 0; t < k; ++t) {
                const double p = static_cast<double>(a[rows[i] * k + t]) * b[t * n + cols[i]];
                ex += p;
                ab += std::fabs(p);
            }
            exact[i] = ex;
            absdot[i] = ab;
        }
    });
    return 0;
}

}  // extern "C"
