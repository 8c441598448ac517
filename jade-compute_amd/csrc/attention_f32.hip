// FP32 self-attention for [heads, seq, dim] tensors, following the reference's
// contract (src/runtime/metal_attention.rs:1-8, 64-137; src/runtime/ir.rs:51-56):
// O = softmax(Q K^T / sqrt(dim)) V, scale 1/sqrt(float(dim)) in FP32, causal rows
// keep keys <= query (diagonal included), online max/normaliser recurrence.
//
// Flash-style kernel for CDNA4. One wave owns 32 queries; a 256-thread block
// owns 128 queries of one head and streams K/V through LDS in 32-key tiles.
// Both products run on v_mfma_f32_32x32x2_f32 in transposed form:
//   S^T[key, q] = sum_d K[key, d] Q[q, d]        (A = K from LDS, B = Q^T in registers)
//   O^T[d, q]  += sum_key V^T[d, key] P^T[key, q] (A = V^T from LDS, B = P^T in registers)
// The S^T accumulator leaves lane l holding query l%32 for 16 keys, and exactly
// those 16 values are the B operand the P.V product needs from lane l, so the
// probabilities never leave registers. Row max and row sum over a tile are a
// 16-value local reduction plus one exchange with lane l^32. Scores are kept in
// log2 units (Q pre-scaled by scale*log2(e)) so each probability is one v_exp_f32.
#include "kernels.hpp"

#include <cmath>

namespace jade {
namespace hipk {
namespace {

typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

constexpr int kThreads = 256;
constexpr int kBQ = 128;   // queries per block (4 waves x 32)
constexpr int kBKV = 32;   // keys per LDS tile
constexpr float kLog2e = 1.44269504088896340736f;  // log2(e)

template <int DP, bool CAUSAL, bool VEC>
__global__ __launch_bounds__(kThreads) void attention_online_mfma(const float *__restrict__ Q,
                                                                  const float *__restrict__ K,
                                                                  const float *__restrict__ V,
                                                                  float *__restrict__ O, int seq, int dim,
                                                                  float qscale, int q_blocks) {
    constexpr int LD = DP + 4;  // LDS row stride (floats); keeps float4 alignment
    constexpr int HALF = DP / 2;
    __shared__ float ks[kBKV * LD];
    __shared__ float vs[kBKV * LD];

    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int h = lane >> 5, c = lane & 31;
    const int qb = q_blocks - 1 - int(blockIdx.x);  // longest causal rows first
    const size_t base = size_t(blockIdx.y) * size_t(seq) * size_t(dim);
    const int q0 = qb * kBQ + wave * 32;
    const int qi = q0 + c;

    // Q^T operand: lane half h holds dims [h*HALF, h*HALF + HALF) of query qi.
    float qreg[HALF];
#pragma unroll
    for (int s = 0; s < HALF; ++s) {
        const int d = h * HALF + s;
        qreg[s] = (qi < seq && d < dim) ? Q[base + size_t(qi) * dim + d] * qscale : 0.f;
    }

    f32x16 acc[DP / 32];
#pragma unroll
    for (int b = 0; b < DP / 32; ++b)
#pragma unroll
        for (int v = 0; v < 16; ++v) acc[b][v] = 0.f;
    float row_max = -INFINITY, row_sum = 0.f;

    const int kv_end = CAUSAL ? min(seq, qb * kBQ + kBQ) : seq;
    for (int kt = 0; kt < kv_end; kt += kBKV) {
        __syncthreads();
        // Stage K and V rows [kt, kt+32) into LDS, zero-padded past seq and dim.
        for (int idx = threadIdx.x; idx < kBKV * DP / 4; idx += kThreads) {
            const int r = idx / (DP / 4), c4 = (idx % (DP / 4)) * 4;
            const int key = kt + r;
            f32x4 kv4 = {0.f, 0.f, 0.f, 0.f}, vv4 = {0.f, 0.f, 0.f, 0.f};
            if (key < seq) {
                const size_t off = base + size_t(key) * dim + c4;
                if (VEC) {
                    if (c4 < dim) {
                        kv4 = *reinterpret_cast<const f32x4 *>(K + off);
                        vv4 = *reinterpret_cast<const f32x4 *>(V + off);
                    }
                } else {
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        if (c4 + e < dim) {
                            kv4[e] = K[off + e];
                            vv4[e] = V[off + e];
                        }
                    }
                }
            }
            *reinterpret_cast<f32x4 *>(ks + r * LD + c4) = kv4;
            *reinterpret_cast<f32x4 *>(vs + r * LD + c4) = vv4;
        }
        __syncthreads();
        if (CAUSAL && kt > q0 + 31) continue;  // every query of this wave precedes the tile

        // S^T tile: 32 keys x 32 queries.
        f32x16 st;
#pragma unroll
        for (int v = 0; v < 16; ++v) st[v] = 0.f;
        const float *krow = ks + c * LD + h * HALF;
#pragma unroll
        for (int s4 = 0; s4 < HALF / 4; ++s4) {
            const f32x4 a = *reinterpret_cast<const f32x4 *>(krow + 4 * s4);
#pragma unroll
            for (int e = 0; e < 4; ++e) st = __builtin_amdgcn_mfma_f32_32x32x2f32(a[e], qreg[4 * s4 + e], st, 0, 0, 0);
        }

        // Mask, then the online max / normaliser update (log2 domain).
        float tile_max = -INFINITY;
#pragma unroll
        for (int v = 0; v < 16; ++v) {
            const int key = kt + 8 * (v >> 2) + 4 * h + (v & 3);
            const bool live = key < seq && (!CAUSAL || key <= qi);
            st[v] = live ? st[v] : -INFINITY;
            tile_max = fmaxf(tile_max, st[v]);
        }
        tile_max = fmaxf(tile_max, __shfl_xor(tile_max, 32));
        const float next_max = fmaxf(row_max, tile_max);
        const float old_weight = __builtin_amdgcn_exp2f(row_max - next_max);
        float tile_sum = 0.f;
#pragma unroll
        for (int v = 0; v < 16; ++v) {
            st[v] = __builtin_amdgcn_exp2f(st[v] - next_max);
            tile_sum += st[v];
        }
        tile_sum += __shfl_xor(tile_sum, 32);
        row_sum = row_sum * old_weight + tile_sum;
        row_max = next_max;
#pragma unroll
        for (int b = 0; b < DP / 32; ++b) acc[b] *= old_weight;

        // O^T += V^T P^T over the tile's 32 keys.
#pragma unroll
        for (int v = 0; v < 16; ++v) {
            const int key = 8 * (v >> 2) + 4 * h + (v & 3);
            const float *vrow = vs + key * LD + c;
#pragma unroll
            for (int b = 0; b < DP / 32; ++b)
                acc[b] = __builtin_amdgcn_mfma_f32_32x32x2f32(vrow[32 * b], st[v], acc[b], 0, 0, 0);
        }
    }

    if (qi < seq) {
        const float inv = 1.0f / row_sum;
        float *orow = O + base + size_t(qi) * dim;
#pragma unroll
        for (int b = 0; b < DP / 32; ++b) {
#pragma unroll
            for (int g = 0; g < 4; ++g) {
                const int d = 32 * b + 8 * g + 4 * h;
                if (VEC) {
                    if (d < dim) {
                        const f32x4 out = {acc[b][4 * g] * inv, acc[b][4 * g + 1] * inv, acc[b][4 * g + 2] * inv,
                                           acc[b][4 * g + 3] * inv};
                        *reinterpret_cast<f32x4 *>(orow + d) = out;
                    }
                } else {
#pragma unroll
                    for (int e = 0; e < 4; ++e)
                        if (d + e < dim) orow[d + e] = acc[b][4 * g + e] * inv;
                }
            }
        }
    }
}

// Materialised comparator, src/runtime/metal_attention.rs:142-171: one thread
// per score, FP32 fma dot product over dim, divided by sqrt(float(dim)).
__global__ __launch_bounds__(256) void attention_scores_kernel(const float *__restrict__ Q, const float *__restrict__ K,
                                                               float *__restrict__ S, int seq, int dim, int causal) {
    const int key = blockIdx.x * 16 + threadIdx.x % 16;
    const int query = blockIdx.y * 16 + threadIdx.x / 16;
    const size_t head = blockIdx.z;
    if (key >= seq || query >= seq) return;
    const size_t index = (head * seq + query) * size_t(seq) + key;
    if (causal && key > query) {
        S[index] = -INFINITY;
        return;
    }
    const float *qrow = Q + (head * seq + query) * size_t(dim);
    const float *krow = K + (head * seq + key) * size_t(dim);
    float dot = 0.f;
    for (int d = 0; d < dim; ++d) dot = fmaf(qrow[d], krow[d], dot);
    S[index] = dot / sqrtf(float(dim));
}

// src/runtime/metal_attention.rs:174-198: one thread per output element.
__global__ __launch_bounds__(256) void attention_apply_kernel(const float *__restrict__ P, const float *__restrict__ V,
                                                              float *__restrict__ O, int seq, int dim) {
    const int channel = blockIdx.x * 16 + threadIdx.x % 16;
    const int query = blockIdx.y * 16 + threadIdx.x / 16;
    const size_t head = blockIdx.z;
    if (channel >= dim || query >= seq) return;
    const float *prow = P + (head * seq + query) * size_t(seq);
    const float *vcol = V + head * size_t(seq) * dim + channel;
    float sum = 0.f;
    for (int key = 0; key < seq; ++key) sum = fmaf(prow[key], vcol[size_t(key) * dim], sum);
    O[(head * seq + query) * size_t(dim) + channel] = sum;
}

template <int DP, bool CAUSAL>
hipError_t launch_online(hipStream_t stream, const float *q, const float *k, const float *v, float *out,
                         uint32_t heads, uint32_t seq, uint32_t dim, bool vec) {
    const int q_blocks = int((seq + kBQ - 1) / kBQ);
    const float qscale = (1.0f / sqrtf(float(dim))) * kLog2e;
    const dim3 grid(unsigned(q_blocks), heads), block(kThreads);
    if (vec)
        hipLaunchKernelGGL((attention_online_mfma<DP, CAUSAL, true>), grid, block, 0, stream, q, k, v, out, int(seq),
                           int(dim), qscale, q_blocks);
    else
        hipLaunchKernelGGL((attention_online_mfma<DP, CAUSAL, false>), grid, block, 0, stream, q, k, v, out,
                           int(seq), int(dim), qscale, q_blocks);
    return hipGetLastError();
}

int padded_dim(uint32_t dim) { return dim <= 32 ? 32 : dim <= 64 ? 64 : 128; }

}  // namespace

LaunchShape attention_online_shape(uint32_t heads, uint32_t seq, uint32_t dim, bool) {
    const int dp = padded_dim(dim);
    const uint32_t lds = 2u * kBKV * (dp + 4) * sizeof(float);
    return {dp == 32 ? "attention_online_mfma_d32" : dp == 64 ? "attention_online_mfma_d64" : "attention_online_mfma_d128",
            {(seq + kBQ - 1) / kBQ, heads, 1},
            {kThreads, 1, 1},
            lds};
}

hipError_t attention_online_f32(hipStream_t stream, const float *q, const float *k, const float *v, float *out,
                                uint32_t heads, uint32_t seq, uint32_t dim, bool causal) {
    const bool aligned =
        ((reinterpret_cast<uintptr_t>(q) | reinterpret_cast<uintptr_t>(k) | reinterpret_cast<uintptr_t>(v) |
          reinterpret_cast<uintptr_t>(out)) &
         15u) == 0;
    const bool vec = aligned && dim % 4 == 0;
    switch (padded_dim(dim)) {
        case 32:
            return causal ? launch_online<32, true>(stream, q, k, v, out, heads, seq, dim, vec)
                          : launch_online<32, false>(stream, q, k, v, out, heads, seq, dim, vec);
        case 64:
            return causal ? launch_online<64, true>(stream, q, k, v, out, heads, seq, dim, vec)
                          : launch_online<64, false>(stream, q, k, v, out, heads, seq, dim, vec);
        default:
            return causal ? launch_online<128, true>(stream, q, k, v, out, heads, seq, dim, vec)
                          : launch_online<128, false>(stream, q, k, v, out, heads, seq, dim, vec);
    }
}

LaunchShape attention_scores_shape(uint32_t heads, uint32_t seq, uint32_t, bool) {
    return {"attention_scores", {(seq + 15) / 16, (seq + 15) / 16, heads}, {256, 1, 1}, 0};
}

hipError_t attention_scores_f32(hipStream_t stream, const float *q, const float *k, float *scores, uint32_t heads,
                                uint32_t seq, uint32_t dim, bool causal) {
    const dim3 grid((seq + 15) / 16, (seq + 15) / 16, heads);
    hipLaunchKernelGGL(attention_scores_kernel, grid, dim3(256), 0, stream, q, k, scores, int(seq), int(dim),
                       causal ? 1 : 0);
    return hipGetLastError();
}

LaunchShape attention_apply_shape(uint32_t heads, uint32_t seq, uint32_t dim) {
    return {"attention_apply", {(dim + 15) / 16, (seq + 15) / 16, heads}, {256, 1, 1}, 0};
}

hipError_t attention_apply_f32(hipStream_t stream, const float *p, const float *v, float *out, uint32_t heads,
                               uint32_t seq, uint32_t dim) {
    const dim3 grid((dim + 15) / 16, (seq + 15) / 16, heads);
    hipLaunchKernelGGL(attention_apply_kernel, grid, dim3(256), 0, stream, p, v, out, int(seq), int(dim));
    return hipGetLastError();
}

}  // namespace hipk
}  // namespace jade
