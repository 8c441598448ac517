/*
 * Jade FP64 CPU oracle — TEST INFRASTRUCTURE ONLY.
 *
 * A plain-C restatement of the reference's independent FP64 CPU references
 * and input generators for the FP32 GEMM / attention / RMSNorm / Softmax /
 * SwiGLU / residual-MLP path. Only tests/, __graft_entry__.smoke() and the
 * cpu_baseline leg of bench.py may load this library, and only as the checker
 * or as the timed CPU baseline. The product (libjade_runtime_hip.so) never
 * links, loads or calls it, and has no CPU fallback.
 *
 * The reference is Rust (no Rust toolchain is present), so it cannot be built
 * into oracle/_ref; every function below cites the reference file:line it
 * restates. Parity pins for each function live in tests/test_oracle.py:
 * textbook known answers, the reference's own unit-test vectors, closed
 * forms, and brute-force agreement with numpy float64 library routines.
 */
#ifndef JADE_ORACLE_H
#define JADE_ORACLE_H
#include <stddef.h>
#include <stdint.h>
#ifdef __cplusplus
extern "C" {
#endif

/* Marsaglia xorshift32 (13, 17, 5): src/runtime/workloads.rs:21-23. */
uint32_t or_xorshift32(uint32_t state);

/* workloads::values, src/runtime/workloads.rs:17-27:
 * ((s >> 8) / 2^24 * 2 - 1) * scale, all FP32, after each xorshift step. */
void or_values(float *out, size_t len, uint32_t seed, float scale);

/* validation::inputs fill, src/validation.rs:8-17 (same map, no scale). */
void or_fill(float *out, size_t len, uint32_t seed);

/* Documented addition (the reference has no normal generator): Box-Muller
 * over the xorshift32 stream. Two draws per value: u1 = ((s1>>8)+1)/2^24 in
 * (0,1], u2 = (s2>>8)/2^24 in [0,1); z = sqrt(-2 ln u1) cos(2 pi u2) in FP64,
 * out = (float)(mean + sigma * z). */
void or_normal(float *out, size_t len, uint32_t seed, float mean, float sigma);

/* metal_lab::gemm_reference, src/runtime/metal_lab.rs:18-31: FP64, i-p-j
 * order. Rows [row0, row1) only; `threads` > 1 splits rows with OpenMP. */
void or_gemm_reference(uint32_t m, uint32_t n, uint32_t k, const float *a,
                       const float *b, double *out, uint32_t row0,
                       uint32_t row1, int threads);

/* workloads::dot, src/runtime/workloads.rs:28-32: FP64 operands, output
 * element i = sum_p a[i/n*k+p] * b[p*n+i%n], summed in p order. */
void or_dot(size_t m, size_t n, size_t k, const double *a, const double *b,
            double *out, int threads);

/* metal_lab::attention_reference, src/runtime/metal_lab.rs:33-73:
 * materialised FP64 rows, score = sum_d q*k / sqrt(dim), max-subtracted exp,
 * out = sum_col p/denom * v. Query rows [row0, row1) of every head.
 * Returns 0, or 1 when a thread's score buffer cannot be allocated. */
int or_attention_reference(uint32_t heads, uint32_t seq, uint32_t dim,
                            int causal, const float *q, const float *k,
                            const float *v, double *out, uint32_t row0,
                            uint32_t row1, int threads);

/* workloads::sigmoid, src/runtime/workloads.rs:36-43. */
double or_sigmoid(double x);

/* workloads::normalize (RMSNorm), src/runtime/workloads.rs:44-55. */
void or_normalize(size_t rows, size_t cols, const double *x,
                  const double *weight, double eps, double *out, int threads);

/* Softmax expectation, src/runtime/workloads.rs:134-142: row max taken in
 * FP32 then widened, exp(x - max) / sum in FP64. */
void or_softmax(size_t rows, size_t cols, const float *x, double *out,
                int threads);

/* SwiGLU expectation, src/runtime/workloads.rs:96-100: g * sigmoid(g) * u. */
void or_swiglu(size_t len, const float *gate, const float *up, double *out);

/* Residual MLP chain, src/runtime/workloads.rs:466-479 (FP64 throughout).
 * Returns 0, or 1 when the FP64 intermediates cannot be allocated. */
int or_mlp(size_t batch, size_t width, size_t hidden, const float *x,
           const float *norm, const float *wg, const float *wu,
           const float *wd, double eps, double *out, int threads);

/* workloads::compare, src/runtime/workloads.rs:224-243. */
typedef struct or_check {
    size_t elements;
    double max_abs_error;
    double max_relative_error;
    int status;        /* 0 pass, 1 nonfinite, 2 mismatch */
    size_t first_bad;  /* index of the failing element when status != 0 */
} or_check;
void or_compare(const float *actual, const double *expected, size_t len,
                double atol, double rtol, or_check *result);

/* validation::check, src/validation.rs:35-91: evenly spaced samples
 * including both ends, tolerance 2e-5 + max(2 K eps32, 2e-6) * sum|a b|
 * (0.0012 * sum|a b| for the FP16-input mode). status 0 pass, 1 nonfinite
 * output, 2 out of tolerance, 3 invalid budget. */
typedef struct or_validation {
    size_t checked_elements;
    double max_abs_error;
    double max_scaled_error;
    int status;
    size_t first_bad;
} or_validation;
void or_check_gemm(uint32_t m, uint32_t n, uint32_t k, const float *a,
                   const float *b, const float *out, size_t budget, int fp16,
                   or_validation *result);

#ifdef __cplusplus
}
#endif
#endif
