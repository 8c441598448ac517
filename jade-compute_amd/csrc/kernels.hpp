// Host-side launchers for the hand-written gfx950 kernels. Every launcher
// checks nothing about buffer ownership: the runtime has already validated
// binding counts, exact lengths and aliasing before any launch.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

#include "spec.hpp"

namespace jade {
namespace hipk {

struct LaunchShape {
    const char *kernel;
    uint32_t grid[3];
    uint32_t block[3];
    uint32_t lds_bytes;
    // GEMM K-group tiles over unaligned rows: the last k (1 or 2) that add in
    // the epilogue rather than in a stage of their own (0 otherwise).
    uint32_t epilogue_k = 0;
};

// jr_gemm_f32_noalloc's set-up on `device` (current): looks up and keeps the
// device address of its static scratch array. Throws dev::Refusal on failure.
void noalloc_prepare(int device);

// C[m,n] = A[m,k] * B[k,n], packed row-major FP32, FP32 MFMA accumulate.
// Small output grids split K; they need `gemm_f32_workspace_bytes` of device
// workspace (0 when the shape does not split), passed as `workspace`.
LaunchShape gemm_f32_shape(uint32_t m, uint32_t n, uint32_t k);
size_t gemm_f32_workspace_bytes(uint32_t m, uint32_t n, uint32_t k);
hipError_t gemm_f32(hipStream_t stream, const float *a, const float *b, float *c, uint32_t m, uint32_t n,
                    uint32_t k, float *workspace);
// `batch` independent products of one shape, product z at a + z*sa, b + z*sb,
// c + z*sc (elements), on direct-load 32x32 tiles with four waves splitting K.
// Needs k % 4 == 0 and 16-byte aligned rows of a (a and sa). For attention's
// materialised P.V per head.
hipError_t gemm_f32_batched_direct(hipStream_t stream, const float *a, const float *b, float *c, uint32_t m,
                                   uint32_t n, uint32_t k, uint32_t batch, size_t sa, size_t sb, size_t sc);
// The residual MLP's gate/up pair with SwiGLU fused: g = a bg, u = a bu and
// act = swiglu(g, u) in one launch, each output bit-identical to the paired
// GEMM launch followed by swiglu_f32. Only where gemm_f32_dual_swiglu_fits
// (shapes whose plan is whole 128x64 tiles) and a, bg, bu are 16-byte
// aligned; otherwise returns hipErrorInvalidValue without launching.
bool gemm_f32_dual_swiglu_fits(uint32_t m, uint32_t n, uint32_t k);
hipError_t gemm_f32_dual_swiglu(hipStream_t stream, const float *a, const float *bg, const float *bu, float *g,
                                float *u, float *act, uint32_t m, uint32_t n, uint32_t k);
// C = A B and, in the same epilogue, sum = C + residual (all [m, n]): the
// residual MLP's down projection and residual Add (src/runtime/workloads.rs:
// 440-465) in one launch, both outputs bit-identical to gemm_f32 followed by
// add_f32. Only where gemm_f32_residual_fits (plans of the four-wave tile
// kernel without split K); otherwise returns hipErrorInvalidValue without
// launching. `sum` must not alias a or b.
bool gemm_f32_residual_fits(uint32_t m, uint32_t n, uint32_t k);
hipError_t gemm_f32_residual(hipStream_t stream, const float *a, const float *b, float *c, const float *residual,
                             float *sum, uint32_t m, uint32_t n, uint32_t k);
// Two independent products of one shape (c0 = a0 b0, c1 = a1 b1) in one
// launch, for shapes whose plan needs no workspace and no 256x256 tile
// (gemm_f32_pairable); each output is bit-identical to its own gemm_f32.
bool gemm_f32_pairable(uint32_t m, uint32_t n, uint32_t k);
hipError_t gemm_f32_pair(hipStream_t stream, const float *a0, const float *b0, float *c0, const float *a1,
                         const float *b1, float *c1, uint32_t m, uint32_t n, uint32_t k);

// Flash-style online softmax(Q K^T / sqrt(dim)) V, [heads, seq, dim] contiguous.
// Grids smaller than the chip split the keys; they need
// `attention_online_workspace_bytes` of device workspace (0 when the shape
// does not split), passed as `workspace`.
LaunchShape attention_online_shape(uint32_t heads, uint32_t seq, uint32_t dim, bool causal);
size_t attention_online_workspace_bytes(uint32_t heads, uint32_t seq, uint32_t dim, bool causal);
hipError_t attention_online_f32(hipStream_t stream, const float *q, const float *k, const float *v, float *out,
                                uint32_t heads, uint32_t seq, uint32_t dim, bool causal, float *workspace);

// Materialised comparator: scaled scores [heads, seq, seq] (-inf above the
// causal diagonal) and probabilities x V.
LaunchShape attention_scores_shape(uint32_t heads, uint32_t seq, uint32_t dim, bool causal);
hipError_t attention_scores_f32(hipStream_t stream, const float *q, const float *k, float *scores, uint32_t heads,
                                uint32_t seq, uint32_t dim, bool causal);
LaunchShape attention_apply_shape(uint32_t heads, uint32_t seq, uint32_t dim);
hipError_t attention_apply_f32(hipStream_t stream, const float *p, const float *v, float *out, uint32_t heads,
                               uint32_t seq, uint32_t dim);

// Row kernels: one row per 64-lane wavefront.
LaunchShape rms_norm_shape(uint32_t rows, uint32_t cols);
hipError_t rms_norm_f32(hipStream_t stream, const float *x, const float *weight, float *out, uint32_t rows,
                        uint32_t cols, float epsilon);
LaunchShape softmax_shape(uint32_t rows, uint32_t cols);
hipError_t softmax_f32(hipStream_t stream, const float *x, float *out, uint32_t rows, uint32_t cols);

// Streaming elementwise kernels.
LaunchShape stream_shape(uint32_t len);
hipError_t swiglu_f32(hipStream_t stream, const float *gate, const float *up, float *out, uint32_t len);
hipError_t add_f32(hipStream_t stream, const float *a, const float *b, float *out, uint32_t len);
hipError_t axpy_f32(hipStream_t stream, float alpha, const float *a, const float *b, float *out, uint32_t len);
hipError_t copy_f32(hipStream_t stream, const float *in, float *out, uint32_t len);

// Postfix-expression interpreter over <= 8 inputs; `program` is device memory.
LaunchShape elementwise_shape(uint32_t len);
hipError_t elementwise_f32(hipStream_t stream, const float *const *inputs, uint32_t input_count, float *out,
                           uint32_t len, const Instr *program, uint32_t program_len);

}  // namespace hipk
}  // namespace jade
