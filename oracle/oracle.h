/* CPU oracle for the minicompiler HIP backend - TEST INFRASTRUCTURE ONLY.
 *
 * Only the tests (tests/), __graft_entry__.smoke() and bench.py's
 * cpu_baseline leg load this library, and only as the checker or the timed
 * CPU baseline. The product (libminicompiler_hip.so) never links, loads or
 * calls it, and has no CPU fallback.
 *
 * What it restates (file:line in the reference, kartsen03/minicompiler):
 *   orc_fill_uniform      src/random.cpp:6-26 (splitmix64, 24-bit u, two roundings)
 *   orc_unary/_binary/_matmul/_fused
 *                         src/cpu/kernels.cpp:19-277, the Eigen CPU backend's
 *                         per-node semantics: fp32 per op, NumPy broadcasting
 *                         row by row, fused programs in 512-element blocks
 *                         with Contiguous/Scalar/Periodic/General loads and
 *                         scalar registers for element-independent values.
 *   orc_ref_*             tests/test_util.cpp:87-159, the double-precision
 *                         evaluator: double math, every node result and every
 *                         fused register rounded to float.
 *   orc_gemm_f64*         the float64 dot products behind the GEMM error
 *                         bounds (tests/test_cuda_backend.cpp:147-159,
 *                         bench/bench_cuda.cpp:386-413).
 * The normal generator restates this library's own documented Box-Muller
 * (include/minicompiler/random.hpp), which the reference does not have.
 *
 * Eigen 3.4 itself (the reference's third-party arithmetic) is not available:
 * transcendental functions here use the C library (expf, logf, tanhf,
 * sqrtf) instead of Eigen's SIMD polynomials, so parity with Eigen's exact
 * bits is unpinned; parity is pinned to the reference's tolerances through
 * the double-precision evaluator.
 *
 * Op codes are the numeric values of minicompiler::OpKind: neg 2, exp 3,
 * log 4, sqrt 5, relu 6, sigmoid 7, tanh 8, add 9, sub 10, mul 11, div 12.
 * Fused instruction kinds: load 0, immediate 1, unary 2, binary 3.
 * Functions return 0, or 1 on a bad argument. */
#ifndef MINICOMPILER_ORACLE_H
#define MINICOMPILER_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

void orc_set_threads(int threads);
int orc_get_threads(void);

void orc_fill_uniform(float* out, size_t count, uint64_t seed, float lo, float hi);
void orc_fill_normal(float* out, size_t count, uint64_t seed, double mean, double stddev);

/* fp32, CPU backend semantics */
int orc_unary(int op, const float* x, float* y, size_t n);
int orc_binary(int op, const float* a, const int64_t* a_shape, int a_rank, const float* b, const int64_t* b_shape,
               int b_rank, float* out, const int64_t* out_shape, int out_rank);
int orc_matmul(const float* a, const float* b, float* c, int64_t m, int64_t k, int64_t n);
/* Program arrays of length num_instrs; inputs[j] has shape
 * shapes[offsets[j] .. offsets[j] + ranks[j]). */
int orc_fused(int num_instrs, const int32_t* kind, const int32_t* op, const int32_t* ra, const int32_t* rb,
              const float* imm, int num_inputs, const float* const* inputs, const int64_t* shapes,
              const int32_t* ranks, float* out, const int64_t* out_shape, int out_rank);

/* double-precision reference evaluator */
int orc_ref_unary(int op, const float* x, float* y, size_t n);
int orc_ref_binary(int op, const float* a, const int64_t* a_shape, int a_rank, const float* b,
                   const int64_t* b_shape, int b_rank, float* out, const int64_t* out_shape, int out_rank);
int orc_ref_matmul(const float* a, const float* b, float* c, int64_t m, int64_t k, int64_t n);
int orc_ref_fused(int num_instrs, const int32_t* kind, const int32_t* op, const int32_t* ra, const int32_t* rb,
                  const float* imm, int num_inputs, const float* const* inputs, const int64_t* shapes,
                  const int32_t* ranks, float* out, const int64_t* out_shape, int out_rank);

/* exact[i] = sum_t a[r,t] b[t,c] and absdot[i] = sum_t |a[r,t] b[t,c]| in
 * double, for all (r, c) or for `count` sampled (rows[i], cols[i]). */
int orc_gemm_f64(const float* a, const float* b, double* exact, double* absdot, int64_t m, int64_t k, int64_t n);
int orc_gemm_f64_sampled(const float* a, const float* b, const int64_t* rows, const int64_t* cols, int64_t count,
                         double* exact, double* absdot, int64_t k, int64_t n);

#ifdef __cplusplus
}
#endif

#endif
