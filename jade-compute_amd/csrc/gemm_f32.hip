// FP32 GEMM on CDNA4 matrix cores: C[M,N] = A[M,K] * B[K,N], packed row-major.
// Semantics follow the reference's Gemm/GemmSimd ops (src/runtime/ir.rs:21-32,
// 524-557; src/runtime/metal_simd.rs:29-110): no alpha/beta, no transposes,
// ragged edges read as zero and masked on store.
//
// Design (gfx950, wave64):
//  * 256-thread workgroup computes a 128x128 tile; each wave owns 64x64 as
//    2x2 blocks of v_mfma_f32_32x32x2_f32 (16 accumulators per lane each).
//  * K advances 32 per stage. A and B stages are double-buffered in LDS with a
//    register prefetch of the next stage, one barrier per stage.
//  * The MFMA K=2 operand split is permuted: lanes 0-31 take k in [0,16) and
//    lanes 32-63 take k in [16,32) of a stage, so an A operand run is 16
//    contiguous floats per lane (ds_read_b128) while B stays ds_read_b32 with
//    consecutive lanes on consecutive columns. A and B share the permutation,
//    so every product is still summed exactly once.
//  * Workgroup ids are remapped so each of the 8 XCDs (dispatched round-robin)
//    owns a contiguous range of tiles in grouped order, keeping A rows and B
//    columns hot in that XCD's private L2.
//  * Two-level accumulation: each 32-deep K stage is summed by the matrix
//    cores into zeroed accumulators and then added to the running sums with
//    round-to-nearest VALU adds. A single chained MFMA accumulation over
//    K = 4096 drifted by ~3.6e-4 absolute on unit-scale inputs, outside the
//    1e-4 gate; the stage split keeps the long recurrence to K/32 adds.
#include "kernels.hpp"

namespace jade {
namespace hipk {
namespace {

typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

constexpr int kBM = 128, kBN = 128, kBK = 32;
constexpr int kThreads = 256;
constexpr int kLDA = kBK + 4;  // LDS row stride of an A stage (floats)
constexpr int kLDB = kBN + 4;  // LDS row stride of a B stage (floats)
constexpr int kGroupM = 8;
constexpr int kAStage = kBM * kLDA;
constexpr int kBStage = kBK * kLDB;
constexpr int kStage = kAStage + kBStage;
constexpr uint32_t kLdsBytes = 2u * kStage * sizeof(float);

__device__ inline void tile_coords(int tiles_m, int tiles_n, int &tm, int &tn) {
    const int total = tiles_m * tiles_n;
    const int bid = blockIdx.x;
    const int per = total / 8, rem = total % 8;
    const int xcd = bid % 8, idx = bid / 8;
    const int logical = xcd * per + min(xcd, rem) + idx;
    const int group_span = kGroupM * tiles_n;
    const int group = logical / group_span;
    const int first_m = group * kGroupM;
    const int group_rows = min(tiles_m - first_m, kGroupM);
    const int in_group = logical - group * group_span;
    tm = first_m + in_group % group_rows;
    tn = in_group / group_rows;
}

// Stage loads: A tile 128x32 and B tile 32x128, four float4 per thread each.
template <bool VEC>
__device__ inline void load_stage(const float *__restrict__ A, const float *__restrict__ B, int M, int N, int K,
                                  int m0, int n0, int k0, f32x4 (&ra)[4], f32x4 (&rb)[4]) {
    const int t = threadIdx.x;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int f = t + i * kThreads;
        const int row = f >> 3, col = (f & 7) << 2;
        const int gr = m0 + row, gc = k0 + col;
        if (VEC) {
            ra[i] = (gr < M && gc < K) ? *reinterpret_cast<const f32x4 *>(A + (size_t)gr * K + gc)
                                       : f32x4{0.f, 0.f, 0.f, 0.f};
        } else {
            f32x4 v;
#pragma unroll
            for (int e = 0; e < 4; ++e) v[e] = (gr < M && gc + e < K) ? A[(size_t)gr * K + gc + e] : 0.f;
            ra[i] = v;
        }
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int f = t + i * kThreads;
        const int row = f >> 5, col = (f & 31) << 2;
        const int gr = k0 + row, gc = n0 + col;
        if (VEC) {
            rb[i] = (gr < K && gc < N) ? *reinterpret_cast<const f32x4 *>(B + (size_t)gr * N + gc)
                                       : f32x4{0.f, 0.f, 0.f, 0.f};
        } else {
            f32x4 v;
#pragma unroll
            for (int e = 0; e < 4; ++e) v[e] = (gr < K && gc + e < N) ? B[(size_t)gr * N + gc + e] : 0.f;
            rb[i] = v;
        }
    }
}

__device__ inline void store_stage(float *stage, const f32x4 (&ra)[4], const f32x4 (&rb)[4]) {
    const int t = threadIdx.x;
    float *as = stage, *bs = stage + kAStage;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int f = t + i * kThreads;
        *reinterpret_cast<f32x4 *>(as + (f >> 3) * kLDA + ((f & 7) << 2)) = ra[i];
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int f = t + i * kThreads;
        *reinterpret_cast<f32x4 *>(bs + (f >> 5) * kLDB + ((f & 31) << 2)) = rb[i];
    }
}

// One K stage into fresh accumulators; the caller adds the stage sums into the
// running totals with VALU adds, so the long K recurrence is 1 add per 32 k
// instead of 16 chained matrix-core accumulations per 32 k.
__device__ inline void mma_stage(const float *stage, int wm, int wn, int lane, f32x16 (&acc)[2][2]) {
    const int h = lane >> 5, c = lane & 31;
    const float *a0p = stage + (wm * 64 + c) * kLDA + 16 * h;
    const float *a1p = a0p + 32 * kLDA;
    const float *bp = stage + kAStage + (16 * h) * kLDB + wn * 64 + c;
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
            for (int v = 0; v < 16; ++v) acc[i][j][v] = 0.f;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        const f32x4 a0 = *reinterpret_cast<const f32x4 *>(a0p + 4 * q);
        const f32x4 a1 = *reinterpret_cast<const f32x4 *>(a1p + 4 * q);
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const int s = 4 * q + e;
            const float b0 = bp[s * kLDB];
            const float b1 = bp[s * kLDB + 32];
            acc[0][0] = __builtin_amdgcn_mfma_f32_32x32x2f32(a0[e], b0, acc[0][0], 0, 0, 0);
            acc[0][1] = __builtin_amdgcn_mfma_f32_32x32x2f32(a0[e], b1, acc[0][1], 0, 0, 0);
            acc[1][0] = __builtin_amdgcn_mfma_f32_32x32x2f32(a1[e], b0, acc[1][0], 0, 0, 0);
            acc[1][1] = __builtin_amdgcn_mfma_f32_32x32x2f32(a1[e], b1, acc[1][1], 0, 0, 0);
        }
    }
}

// Two waves per SIMD (LDS allows two 70.6 KB workgroups per CU); the register
// budget is capped to match so stage and running accumulators both fit.
template <bool VEC>
__global__ __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(2, 2))) void gemm_f32_mfma(
    const float *__restrict__ A, const float *__restrict__ B, float *__restrict__ C, int M, int N, int K,
    int tiles_m, int tiles_n) {
    __shared__ float smem[2 * kStage];
    int tm, tn;
    tile_coords(tiles_m, tiles_n, tm, tn);
    const int m0 = tm * kBM, n0 = tn * kBN;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int wm = wave >> 1, wn = wave & 1;

    f32x16 acc[2][2];
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
            for (int v = 0; v < 16; ++v) acc[i][j][v] = 0.f;

    f32x4 ra[4], rb[4];
    const int nk = (K + kBK - 1) / kBK;
    load_stage<VEC>(A, B, M, N, K, m0, n0, 0, ra, rb);
    store_stage(smem, ra, rb);
    __syncthreads();
    for (int kt = 0; kt < nk; ++kt) {
        const float *cur = smem + (kt & 1) * kStage;
        float *nxt = smem + ((kt + 1) & 1) * kStage;
        const bool more = kt + 1 < nk;
        if (more) load_stage<VEC>(A, B, M, N, K, m0, n0, (kt + 1) * kBK, ra, rb);
        f32x16 part[2][2];
        mma_stage(cur, wm, wn, lane, part);
#pragma unroll
        for (int i = 0; i < 2; ++i)
#pragma unroll
            for (int j = 0; j < 2; ++j) acc[i][j] += part[i][j];
        if (more) store_stage(nxt, ra, rb);
        __syncthreads();
    }

    const int h = lane >> 5, c = lane & 31;
#pragma unroll
    for (int i = 0; i < 2; ++i) {
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            const int col = n0 + wn * 64 + j * 32 + c;
#pragma unroll
            for (int v = 0; v < 16; ++v) {
                const int row = m0 + wm * 64 + i * 32 + 8 * (v >> 2) + 4 * h + (v & 3);
                if (row < M && col < N) C[(size_t)row * N + col] = acc[i][j][v];
            }
        }
    }
}

}  // namespace

LaunchShape gemm_f32_shape(uint32_t m, uint32_t n, uint32_t) {
    const uint32_t tiles = ((m + kBM - 1) / kBM) * ((n + kBN - 1) / kBN);
    return {"gemm_f32_mfma_128x128x32", {tiles, 1, 1}, {kThreads, 1, 1}, kLdsBytes};
}

hipError_t gemm_f32(hipStream_t stream, const float *a, const float *b, float *c, uint32_t m, uint32_t n,
                    uint32_t k) {
    const int tiles_m = int((m + kBM - 1) / kBM), tiles_n = int((n + kBN - 1) / kBN);
    const bool aligned = ((reinterpret_cast<uintptr_t>(a) | reinterpret_cast<uintptr_t>(b)) & 15u) == 0;
    const bool vec = aligned && (k % 4 == 0) && (n % 4 == 0);
    const dim3 grid(unsigned(tiles_m) * unsigned(tiles_n)), block(kThreads);
    if (vec)
        hipLaunchKernelGGL(gemm_f32_mfma<true>, grid, block, 0, stream, a, b, c, int(m), int(n), int(k), tiles_m,
                           tiles_n);
    else
        hipLaunchKernelGGL(gemm_f32_mfma<false>, grid, block, 0, stream, a, b, c, int(m), int(n), int(k), tiles_m,
                           tiles_n);
    return hipGetLastError();
}

}  // namespace hipk
}  // namespace jade
