// Row kernels, one row per 64-lane wavefront (four rows per 256-thread block),
// or for Softmax over rows of 1024..16384 floats, one row per block.
// RMSNorm follows src/runtime/ir.rs:488-500: inv = rsqrt(sum(x^2)/cols + eps),
// out = x * inv * w. Softmax follows ir.rs:501-523: max, sum(exp(x - max)),
// exp(x - max) / sum. When a row fits in registers (cols % 4 == 0 and
// cols <= 4096) it is read from HBM exactly once and written once; the
// reductions are wavefront butterflies with no LDS and no barrier. Output rows
// go out as non-temporal vector stores (no L2 allocation for a stream that is
// not re-read here), and the cached kernels read their rows through
// non-temporal loads as well (RMSNorm 4096x1024 streamed from HBM: 6.42 ->
// 5.96 us); the weight row, shared by every row, keeps ordinary loads.
#include "kernels.hpp"

#include <cmath>

namespace jade {
namespace hipk {
namespace {

typedef float f32x4 __attribute__((ext_vector_type(4)));

constexpr int kThreads = 256;
constexpr int kRowsPerBlock = kThreads / 64;
constexpr float kLog2e = 1.44269504088896340736f;

__device__ inline float wave_sum(float v) {
#pragma unroll
    for (int offset = 32; offset > 0; offset >>= 1) v += __shfl_xor(v, offset);
    return v;
}
__device__ inline float wave_max(float v) {
#pragma unroll
    for (int offset = 32; offset > 0; offset >>= 1) v = fmaxf(v, __shfl_xor(v, offset));
    return v;
}
__device__ inline float exp_f32(float x) { return __builtin_amdgcn_exp2f(x * kLog2e); }

template <int C4>
__global__ __launch_bounds__(kThreads) void rms_norm_cached(const float *__restrict__ x,
                                                            const float *__restrict__ w,
                                                            float *__restrict__ out, int rows, int cols,
                                                            float eps) {
    const int lane = threadIdx.x & 63;
    const int row = int(blockIdx.x) * kRowsPerBlock + (threadIdx.x >> 6);
    if (row >= rows) return;
    const int n4 = cols >> 2;
    const f32x4 *xr = reinterpret_cast<const f32x4 *>(x + size_t(row) * cols);
    f32x4 v[C4];
    float sum = 0.f;
#pragma unroll
    for (int i = 0; i < C4; ++i) {
        const int idx = lane + 64 * i;
        v[i] = idx < n4 ? __builtin_nontemporal_load(xr + idx) : f32x4{0.f, 0.f, 0.f, 0.f};
        sum = fmaf(v[i].x, v[i].x, sum);
        sum = fmaf(v[i].y, v[i].y, sum);
        sum = fmaf(v[i].z, v[i].z, sum);
        sum = fmaf(v[i].w, v[i].w, sum);
    }
    sum = wave_sum(sum);
    const float inv = rsqrtf(sum / float(cols) + eps);
    const f32x4 *w4 = reinterpret_cast<const f32x4 *>(w);
    f32x4 *o4 = reinterpret_cast<f32x4 *>(out + size_t(row) * cols);
#pragma unroll
    for (int i = 0; i < C4; ++i) {
        const int idx = lane + 64 * i;
        if (idx < n4) __builtin_nontemporal_store(v[i] * inv * w4[idx], o4 + idx);
    }
}

__global__ __launch_bounds__(kThreads) void rms_norm_rows(const float *__restrict__ x, const float *__restrict__ w,
                                                          float *__restrict__ out, int rows, int cols, float eps) {
    const int lane = threadIdx.x & 63;
    const int row = int(blockIdx.x) * kRowsPerBlock + (threadIdx.x >> 6);
    if (row >= rows) return;
    const float *xr = x + size_t(row) * cols;
    float sum = 0.f;
    for (int c = lane; c < cols; c += 64) sum = fmaf(xr[c], xr[c], sum);
    sum = wave_sum(sum);
    const float inv = rsqrtf(sum / float(cols) + eps);
    float *orow = out + size_t(row) * cols;
    for (int c = lane; c < cols; c += 64) orow[c] = xr[c] * inv * w[c];
}

template <int C4>
__global__ __launch_bounds__(kThreads) void softmax_cached(const float *__restrict__ x, float *__restrict__ out,
                                                           int rows, int cols) {
    const int lane = threadIdx.x & 63;
    const int row = int(blockIdx.x) * kRowsPerBlock + (threadIdx.x >> 6);
    if (row >= rows) return;
    const int n4 = cols >> 2;
    const f32x4 *xr = reinterpret_cast<const f32x4 *>(x + size_t(row) * cols);
    f32x4 v[C4];
    float m = -INFINITY;
#pragma unroll
    for (int i = 0; i < C4; ++i) {
        const int idx = lane + 64 * i;
        v[i] = idx < n4 ? __builtin_nontemporal_load(xr + idx) : f32x4{-INFINITY, -INFINITY, -INFINITY, -INFINITY};
        m = fmaxf(m, fmaxf(fmaxf(v[i].x, v[i].y), fmaxf(v[i].z, v[i].w)));
    }
    m = wave_max(m);
    float sum = 0.f;
#pragma unroll
    for (int i = 0; i < C4; ++i) {
        v[i].x = exp_f32(v[i].x - m);
        v[i].y = exp_f32(v[i].y - m);
        v[i].z = exp_f32(v[i].z - m);
        v[i].w = exp_f32(v[i].w - m);
        sum += (v[i].x + v[i].y) + (v[i].z + v[i].w);
    }
    sum = wave_sum(sum);
    const float inv = 1.0f / sum;
    f32x4 *o4 = reinterpret_cast<f32x4 *>(out + size_t(row) * cols);
#pragma unroll
    for (int i = 0; i < C4; ++i) {
        const int idx = lane + 64 * i;
        if (idx < n4) __builtin_nontemporal_store(v[i] * inv, o4 + idx);
    }
}

// Rows of 1024..16384 floats (cols % 4 == 0): one row per block of T threads
// (256 below 2048 columns, else 512), V float4 per lane, cross-wave
// reductions through LDS. Spreading a row over several waves keeps each
// wave's burst small: a 16 KiB burst per wave (the wave-per-row kernel at 4096
// columns) capped the stream at ~5.5 TB/s. At 32768x4096 (1 GiB moved) 256
// threads per row ran at 6.35 TB/s and 512 at 6.58, against 6.34 TB/s for a
// plain non-temporal copy of the same 512 MiB; 1024 threads ran at 5.97.
template <int T, int V>
__global__ __launch_bounds__(T) void softmax_block(const float *__restrict__ x, float *__restrict__ out, int cols) {
    constexpr int W = T / 64;
    __shared__ float partial[2][W];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int n4 = cols >> 2;
    const f32x4 *xr = reinterpret_cast<const f32x4 *>(x + size_t(blockIdx.x) * cols);
    f32x4 v[V];
    float m = -INFINITY;
#pragma unroll
    for (int i = 0; i < V; ++i) {
        const int idx = int(threadIdx.x) + T * i;
        v[i] = idx < n4 ? __builtin_nontemporal_load(xr + idx) : f32x4{-INFINITY, -INFINITY, -INFINITY, -INFINITY};
        m = fmaxf(m, fmaxf(fmaxf(v[i].x, v[i].y), fmaxf(v[i].z, v[i].w)));
    }
    m = wave_max(m);
    if (lane == 0) partial[0][wave] = m;
    __syncthreads();
    m = partial[0][0];
#pragma unroll
    for (int w = 1; w < W; ++w) m = fmaxf(m, partial[0][w]);
    float sum = 0.f;
#pragma unroll
    for (int i = 0; i < V; ++i) {
        v[i].x = exp_f32(v[i].x - m);
        v[i].y = exp_f32(v[i].y - m);
        v[i].z = exp_f32(v[i].z - m);
        v[i].w = exp_f32(v[i].w - m);
        sum += (v[i].x + v[i].y) + (v[i].z + v[i].w);
    }
    sum = wave_sum(sum);
    if (lane == 0) partial[1][wave] = sum;
    __syncthreads();
    float total = partial[1][0];
#pragma unroll
    for (int w = 1; w < W; ++w) total += partial[1][w];
    const float inv = 1.0f / total;
    f32x4 *o4 = reinterpret_cast<f32x4 *>(out + size_t(blockIdx.x) * cols);
#pragma unroll
    for (int i = 0; i < V; ++i) {
        const int idx = int(threadIdx.x) + T * i;
        if (idx < n4) __builtin_nontemporal_store(v[i] * inv, o4 + idx);
    }
}

// Any width: one online (max, sum) pass, then one normalising pass.
__global__ __launch_bounds__(kThreads) void softmax_rows(const float *__restrict__ x, float *__restrict__ out,
                                                         int rows, int cols) {
    const int lane = threadIdx.x & 63;
    const int row = int(blockIdx.x) * kRowsPerBlock + (threadIdx.x >> 6);
    if (row >= rows) return;
    const float *xr = x + size_t(row) * cols;
    float m = -INFINITY, s = 0.f;
    for (int c = lane; c < cols; c += 64) {
        const float v = xr[c];
        if (v > m) {
            s = s * exp_f32(m - v) + 1.0f;
            m = v;
        } else if (m != -INFINITY) {  // -inf entries (causal scores) add nothing
            s += exp_f32(v - m);
        }
    }
    const float row_max = wave_max(m);
    const float sum = wave_sum(m == -INFINITY ? 0.f : s * exp_f32(m - row_max));
    const float inv = 1.0f / sum;
    float *orow = out + size_t(row) * cols;
    for (int c = lane; c < cols; c += 64) orow[c] = exp_f32(xr[c] - row_max) * inv;
}

int cache_slots(uint32_t cols) {
    if (cols % 4 != 0) return 0;
    const uint32_t per_lane = (cols / 4 + 63) / 64;
    if (per_lane <= 1) return 1;
    if (per_lane <= 2) return 2;
    if (per_lane <= 4) return 4;
    if (per_lane <= 8) return 8;
    if (per_lane <= 16) return 16;
    return 0;
}

// softmax_block's threads per row for 1024 <= cols <= 16384, cols % 4 == 0
// (0 selects the wave-per-row kernels), and its float4 per lane.
int block_threads(uint32_t cols) {
    if (cols % 4 != 0 || cols < 1024 || cols > 16384) return 0;
    return cols < 2048 ? 256 : 512;
}
int block_slots(uint32_t cols) {
    const int t = block_threads(cols);
    if (!t) return 0;
    const uint32_t per_lane = (cols / 4 + t - 1) / t;
    return per_lane <= 1 ? 1 : per_lane <= 2 ? 2 : per_lane <= 4 ? 4 : 8;
}

bool aligned16(const void *a, const void *b, const void *c) {
    return ((reinterpret_cast<uintptr_t>(a) | reinterpret_cast<uintptr_t>(b) | reinterpret_cast<uintptr_t>(c)) &
            15u) == 0;
}

}  // namespace

LaunchShape rms_norm_shape(uint32_t rows, uint32_t cols) {
    const int c4 = cache_slots(cols);
    return {c4 ? "rms_norm_cached" : "rms_norm_rows", {(rows + kRowsPerBlock - 1) / kRowsPerBlock, 1, 1},
            {kThreads, 1, 1}, 0};
}

hipError_t rms_norm_f32(hipStream_t stream, const float *x, const float *weight, float *out, uint32_t rows,
                        uint32_t cols, float epsilon) {
    const dim3 grid((rows + kRowsPerBlock - 1) / kRowsPerBlock), block(kThreads);
    const int c4 = aligned16(x, weight, out) ? cache_slots(cols) : 0;
    switch (c4) {
        case 1: hipLaunchKernelGGL(rms_norm_cached<1>, grid, block, 0, stream, x, weight, out, int(rows), int(cols), epsilon); break;
        case 2: hipLaunchKernelGGL(rms_norm_cached<2>, grid, block, 0, stream, x, weight, out, int(rows), int(cols), epsilon); break;
        case 4: hipLaunchKernelGGL(rms_norm_cached<4>, grid, block, 0, stream, x, weight, out, int(rows), int(cols), epsilon); break;
        case 8: hipLaunchKernelGGL(rms_norm_cached<8>, grid, block, 0, stream, x, weight, out, int(rows), int(cols), epsilon); break;
        case 16: hipLaunchKernelGGL(rms_norm_cached<16>, grid, block, 0, stream, x, weight, out, int(rows), int(cols), epsilon); break;
        default: hipLaunchKernelGGL(rms_norm_rows, grid, block, 0, stream, x, weight, out, int(rows), int(cols), epsilon); break;
    }
    return hipGetLastError();
}

LaunchShape softmax_shape(uint32_t rows, uint32_t cols) {
    if (const int t = block_threads(cols))
        return {"softmax_block", {rows, 1, 1}, {uint32_t(t), 1, 1}, uint32_t(2 * (t / 64) * sizeof(float))};
    const int c4 = cache_slots(cols);
    return {c4 ? "softmax_cached" : "softmax_rows", {(rows + kRowsPerBlock - 1) / kRowsPerBlock, 1, 1},
            {kThreads, 1, 1}, 0};
}

hipError_t softmax_f32(hipStream_t stream, const float *x, float *out, uint32_t rows, uint32_t cols) {
    const bool aligned = aligned16(x, out, out);
    const int bt = aligned ? block_threads(cols) : 0;
    if (bt == 256) {
        switch (block_slots(cols)) {
            case 1: hipLaunchKernelGGL((softmax_block<256, 1>), dim3(rows), dim3(256), 0, stream, x, out, int(cols)); break;
            default: hipLaunchKernelGGL((softmax_block<256, 2>), dim3(rows), dim3(256), 0, stream, x, out, int(cols)); break;
        }
        return hipGetLastError();
    }
    if (bt == 512) {
        switch (block_slots(cols)) {
            case 1: hipLaunchKernelGGL((softmax_block<512, 1>), dim3(rows), dim3(512), 0, stream, x, out, int(cols)); break;
            case 2: hipLaunchKernelGGL((softmax_block<512, 2>), dim3(rows), dim3(512), 0, stream, x, out, int(cols)); break;
            case 4: hipLaunchKernelGGL((softmax_block<512, 4>), dim3(rows), dim3(512), 0, stream, x, out, int(cols)); break;
            default: hipLaunchKernelGGL((softmax_block<512, 8>), dim3(rows), dim3(512), 0, stream, x, out, int(cols)); break;
        }
        return hipGetLastError();
    }
    const dim3 grid((rows + kRowsPerBlock - 1) / kRowsPerBlock), block(kThreads);
    const int c4 = aligned ? cache_slots(cols) : 0;
    switch (c4) {
        case 1: hipLaunchKernelGGL(softmax_cached<1>, grid, block, 0, stream, x, out, int(rows), int(cols)); break;
        case 2: hipLaunchKernelGGL(softmax_cached<2>, grid, block, 0, stream, x, out, int(rows), int(cols)); break;
        case 4: hipLaunchKernelGGL(softmax_cached<4>, grid, block, 0, stream, x, out, int(rows), int(cols)); break;
        case 8: hipLaunchKernelGGL(softmax_cached<8>, grid, block, 0, stream, x, out, int(rows), int(cols)); break;
        case 16: hipLaunchKernelGGL(softmax_cached<16>, grid, block, 0, stream, x, out, int(rows), int(cols)); break;
        default: hipLaunchKernelGGL(softmax_rows, grid, block, 0, stream, x, out, int(rows), int(cols)); break;
    }
    return hipGetLastError();
}

}  // namespace hipk
}  // namespace jade
