// FP32 self-attention for [heads, seq, dim] tensors, following the reference's
// contract (src/runtime/metal_attention.rs:1-8, 64-137; src/runtime/ir.rs:51-56):
// O = softmax(Q K^T / sqrt(dim)) V, scale 1/sqrt(float(dim)) in FP32, causal rows
// keep keys <= query (diagonal included), online max/normaliser recurrence.
//
// Flash-style kernel for CDNA4. One wave owns 32 queries; a block of NW waves
// owns 32*NW queries of one head and streams K/V through LDS in 64-key tiles,
// double-buffered with a register prefetch of the next tile (one barrier per
// tile). Both products run on v_mfma_f32_32x32x2_f32 in transposed form:
//   S^T[key, q] = sum_d K[key, d] Q[q, d]        (A = K from LDS, B = Q^T in registers)
//   O^T[d, q]  += sum_key V^T[d, key] P^T[key, q] (A = V^T from LDS, B = P^T in registers)
// The S^T accumulator leaves lane l holding query l%32 for 16 keys, and exactly
// those 16 values are the B operand the P.V product needs from lane l, so the
// probabilities never leave registers. Row max and row sum over a tile are a
// local reduction plus one exchange with lane l^32. Scores are kept in log2
// units (Q pre-scaled by scale*log2(e)) so each probability is one v_exp_f32.
//
// Scheduling: grid = (heads, query blocks) with the query-block index reversed,
// so the longest causal rows of every head dispatch first, and all blocks of a
// head share one XCD (workgroups go round-robin over 8 XCDs by linear id). A
// wave skips 32-key sub-tiles that lie wholly above its causal diagonal.
//
// Grids too small to fill the chip (fewer blocks than CUs) split each block's
// key tiles into slices of `per` tiles, one block per live slice. A slice writes its
// unnormalised O, running max and normaliser to a workspace, and
// attention_combine merges the slices of each row:
// O = sum_z 2^(m_z - M) O_z / sum_z 2^(m_z - M) l_z with M = max_z m_z.
// Fixed-size slices give a causal grid's long rows more slices than its short
// ones, so every live slice costs about the same.
#include "kernels.hpp"

#include <algorithm>
#include <cmath>
#include <type_traits>

namespace jade {
namespace hipk {
namespace {

typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

constexpr int kBKV = 64;  // keys per LDS tile (two 32-key sub-tiles)
// Online softmax with a lazy reference maximum: the reference moves only when
// a tile's maximum exceeds it by more than kLazyMax (log2 units), so every
// weight exp2(s - reference) stays at most 2^kLazyMax and the accumulators
// take a rescale only when the reference moves.
constexpr float kLazyMax = 8.0f;
constexpr uint32_t kMaxSplits = 16;  // key slices per row of a split launch, at most
constexpr float kLog2e = 1.44269504088896340736f;  // log2(e)
constexpr uint32_t kRawBuffer = 0x00020000;  // buffer descriptor word 3: raw buffer, 32-bit data format
// A buffer-load offset past every head of at most 2 GiB: reads zero without
// touching memory.
constexpr uint32_t kDeadOffset = 0x80000000u;

// Max and sum over lanes l and l ^ 32 (the two halves of the wave hold the
// two key halves of a query's scores). v_permlane32_swap exchanges the halves
// in the VALU, without the LDS round trip of a cross-half shuffle.
__device__ inline float halves_max(float x) {
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ inline float halves_sum(float x) {
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

// NB adjacent floats of one LDS row, read as one vector (NB = 1, 2 or 4).
template <int NB>
struct alignas(4 * NB) VRow {
    float x[NB];
};

template <int DP, int NW>
struct AttnShape {
    static constexpr int kThreads = NW * 64;
    static constexpr int kBQ = NW * 32;
    static constexpr int kLD = DP + 4;             // LDS row stride (floats), float4-aligned
    static constexpr int kTile = kBKV * kLD;       // floats in one K (or V) tile
    static constexpr int kLoads = kBKV * DP / 4 / kThreads;  // float4 per thread per tensor
    static constexpr uint32_t kLdsBytes = 2u * 2u * kTile * sizeof(float);
    static_assert(kLoads >= 1 && kBKV * DP / 4 % kThreads == 0, "tile must split evenly over the block");
};

// Global -> registers for one tensor's rows [kt, kt+64) of a K/V tile (zero
// past seq/dim).
template <int DP, int NW, bool VEC>
__device__ inline void load_rows(const float *__restrict__ X, size_t base, int kt, int seq, int dim,
                                 f32x4 (&p)[AttnShape<DP, NW>::kLoads]) {
    using S = AttnShape<DP, NW>;
#pragma unroll
    for (int i = 0; i < S::kLoads; ++i) {
        const int idx = threadIdx.x + i * S::kThreads;
        const int r = idx / (DP / 4), c4 = (idx % (DP / 4)) * 4;
        const int key = kt + r;
        f32x4 x = {0.f, 0.f, 0.f, 0.f};
        if (key < seq) {
            const size_t off = base + size_t(key) * dim + c4;
            if (VEC) {
                if (c4 < dim) x = *reinterpret_cast<const f32x4 *>(X + off);
            } else {
#pragma unroll
                for (int e = 0; e < 4; ++e)
                    if (c4 + e < dim) x[e] = X[off + e];
            }
        }
        p[i] = x;
    }
}

// VEC: one tensor's rows of a tile through buffer loads over the head
// (rows past seq lie past the buffer's end and read zero; dims past dim are
// aimed at kDeadOffset). `lane_off` is the lane's fixed byte offset inside a
// tile, `tile` the tile's first row times the row bytes.
template <int DP, int NW>
__device__ inline void load_rows_buf(__amdgpu_buffer_rsrc_t rsrc, const uint32_t (&lane_off)[AttnShape<DP, NW>::kLoads],
                                     uint32_t tile, f32x4 (&p)[AttnShape<DP, NW>::kLoads]) {
#pragma unroll
    for (int i = 0; i < AttnShape<DP, NW>::kLoads; ++i) {
        const auto v = __builtin_amdgcn_raw_buffer_load_b128(rsrc, int(lane_off[i] + tile), 0, 0);
        p[i] = f32x4{__uint_as_float(v[0]), __uint_as_float(v[1]), __uint_as_float(v[2]), __uint_as_float(v[3])};
    }
}

// Both tensors' rows of a tile, K and V loads interleaved.
template <int DP, int NW, bool VEC>
__device__ inline void load_kv(const float *__restrict__ K, const float *__restrict__ V, size_t base, int kt,
                               int seq, int dim, f32x4 (&pk)[AttnShape<DP, NW>::kLoads],
                               f32x4 (&pv)[AttnShape<DP, NW>::kLoads]) {
    using S = AttnShape<DP, NW>;
#pragma unroll
    for (int i = 0; i < S::kLoads; ++i) {
        const int idx = threadIdx.x + i * S::kThreads;
        const int r = idx / (DP / 4), c4 = (idx % (DP / 4)) * 4;
        const int key = kt + r;
        f32x4 kv = {0.f, 0.f, 0.f, 0.f}, vv = {0.f, 0.f, 0.f, 0.f};
        if (key < seq) {
            const size_t off = base + size_t(key) * dim + c4;
            if (VEC) {
                if (c4 < dim) {
                    kv = *reinterpret_cast<const f32x4 *>(K + off);
                    vv = *reinterpret_cast<const f32x4 *>(V + off);
                }
            } else {
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    if (c4 + e < dim) {
                        kv[e] = K[off + e];
                        vv[e] = V[off + e];
                    }
                }
            }
        }
        pk[i] = kv;
        pv[i] = vv;
    }
}

template <int DP, int NW>
__device__ inline void store_kv(float *tile, const f32x4 (&pk)[AttnShape<DP, NW>::kLoads],
                                const f32x4 (&pv)[AttnShape<DP, NW>::kLoads]) {
    using S = AttnShape<DP, NW>;
#pragma unroll
    for (int i = 0; i < S::kLoads; ++i) {
        const int idx = threadIdx.x + i * S::kThreads;
        const int r = idx / (DP / 4), c4 = (idx % (DP / 4)) * 4;
        *reinterpret_cast<f32x4 *>(tile + r * S::kLD + c4) = pk[i];
        *reinterpret_cast<f32x4 *>(tile + S::kTile + r * S::kLD + c4) = pv[i];
    }
}

template <int DP, int NW>
__device__ inline void store_rows(float *tile, const f32x4 (&p)[AttnShape<DP, NW>::kLoads]) {
    using S = AttnShape<DP, NW>;
#pragma unroll
    for (int i = 0; i < S::kLoads; ++i) {
        const int idx = threadIdx.x + i * S::kThreads;
        const int r = idx / (DP / 4), c4 = (idx % (DP / 4)) * 4;
        *reinterpret_cast<f32x4 *>(tile + r * S::kLD + c4) = p[i];
    }
}

// SPLIT: the grid is one block per live slice, longest rows first: blockIdx.x
// walks query blocks from the last, each contributing heads * ceil(T/per)
// blocks (T = its key tiles), head fastest. Slice z covers key tiles
// [z*per, min(T, (z+1)*per)) and writes partial results: unnormalised O rows to
// `O + z*rows*dim` and (running max, normaliser) to `ml[z*rows + row]`, where
// rows = heads*seq. A query with no live key in its slice gets (-inf, 0) and a
// zero row.
template <int DP, int NW, bool CAUSAL, bool VEC, bool SPLIT>
__global__ __launch_bounds__(NW * 64) void attention_online_mfma(const float *__restrict__ Q,
                                                                 const float *__restrict__ K,
                                                                 const float *__restrict__ V,
                                                                 float *__restrict__ O, float2 *__restrict__ ml,
                                                                 int seq, int dim, float qscale, int per,
                                                                 int heads) {
    using S = AttnShape<DP, NW>;
    constexpr int HALF = DP / 2;
    constexpr int LD = S::kLD;
    __shared__ float lds[2 * 2 * S::kTile];

    // The wave index through readfirstlane: the compiler then knows every
    // per-wave condition below (causal sub-tiles, unmasked tiles) is uniform
    // and branches on scalars.
    const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(int(threadIdx.x) >> 6);
    const int h = lane >> 5, c = lane & 31;
    auto tiles_of = [&](int b) { return ((CAUSAL ? min(seq, b * S::kBQ + S::kBQ) : seq) + kBKV - 1) / kBKV; };
    int head = int(blockIdx.x), qb = int(gridDim.y) - 1 - int(blockIdx.y);  // longest causal rows first
    int z = 0;
    if (SPLIT) {  // decode (query block, slice, head) from the live-slice index
        int rest = int(blockIdx.x);
        qb = (seq + S::kBQ - 1) / S::kBQ - 1;
        for (;; --qb) {
            const int n = heads * ((tiles_of(qb) + per - 1) / per);
            if (rest < n || qb == 0) break;
            rest -= n;
        }
        head = rest % heads;
        z = rest / heads;
    }
    const size_t base = size_t(head) * size_t(seq) * size_t(dim);
    const int q0 = qb * S::kBQ + wave * 32;
    const int qi = q0 + c;

    const int tiles = tiles_of(qb);
    int t_begin = 0, t_end = tiles;
    if (SPLIT) {
        t_begin = z * per;
        t_end = min(tiles, t_begin + per);
    }

    // Q^T operand: lane half h holds dims [h*HALF, h*HALF + HALF) of query qi.
    float qreg[HALF];
    if (VEC) {
#pragma unroll
        for (int s4 = 0; s4 < HALF / 4; ++s4) {
            const int d = h * HALF + 4 * s4;
            f32x4 x = {0.f, 0.f, 0.f, 0.f};
            if (qi < seq && d < dim) x = *reinterpret_cast<const f32x4 *>(Q + base + size_t(qi) * dim + d);
#pragma unroll
            for (int e = 0; e < 4; ++e) qreg[4 * s4 + e] = x[e] * qscale;
        }
    } else {
#pragma unroll
        for (int s = 0; s < HALF; ++s) {
            const int d = h * HALF + s;
            qreg[s] = (qi < seq && d < dim) ? Q[base + size_t(qi) * dim + d] * qscale : 0.f;
        }
    }

    constexpr int NB = DP / 32;  // accumulator blocks of O^T
    constexpr bool kInterleaved = NB == 4;  // block b holds dims NB r + b (else 32 b + r)
    f32x16 acc[NB];
#pragma unroll
    for (int b = 0; b < NB; ++b)
#pragma unroll
        for (int v = 0; v < 16; ++v) acc[b][v] = 0.f;
    float row_max = -INFINITY, row_sum = 0.f;

    // Head dim 128: one tensor's share of the next tile in flight at a time,
    // K during the score product, then V in the same registers during the
    // softmax and P.V (22 fewer registers; LLM config +1.3%). Head dims of 64
    // and less load both at the tile's start (the split measured 2% slower).
    constexpr bool kSplitStage = DP == 128;
    f32x4 stage[S::kLoads], vstage[kSplitStage ? 1 : S::kLoads];
    // VEC: K and V rows through buffer loads over the head (below 2 GiB, which
    // the launcher checks): a fixed byte offset per lane and load plus the
    // tile's, no bounds branches. Otherwise guarded scalar loads.
    const uint32_t head_bytes = VEC ? uint32_t(seq) * uint32_t(dim) * 4u : 0u, row_bytes = uint32_t(dim) * 4u;
    const __amdgpu_buffer_rsrc_t rk =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<float *>(K + base), 0, int(head_bytes), int(kRawBuffer));
    const __amdgpu_buffer_rsrc_t rv =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<float *>(V + base), 0, int(head_bytes), int(kRawBuffer));
    uint32_t kv_off[S::kLoads];
#pragma unroll
    for (int i = 0; i < S::kLoads; ++i) {
        const int idx = int(threadIdx.x) + i * S::kThreads;
        const int r = idx / (DP / 4), c4 = (idx % (DP / 4)) * 4;
        kv_off[i] = c4 < dim ? (uint32_t(r) * uint32_t(dim) + uint32_t(c4)) * 4u : kDeadOffset;
    }
    auto fetch = [&](bool is_k, int kt, f32x4(&p)[S::kLoads]) {
        if constexpr (VEC)
            load_rows_buf<DP, NW>(is_k ? rk : rv, kv_off, uint32_t(kt) * row_bytes, p);
        else
            load_rows<DP, NW, VEC>(is_k ? K : V, base, kt, seq, dim, p);
    };
    auto fetch_both = [&](int kt, f32x4(&pk)[S::kLoads], f32x4(&pv)[S::kLoads]) {
        if constexpr (VEC) {
#pragma unroll
            for (int i = 0; i < S::kLoads; ++i) {
                const int off = int(kv_off[i] + uint32_t(kt) * row_bytes);
                const auto a = __builtin_amdgcn_raw_buffer_load_b128(rk, off, 0, 0);
                const auto b = __builtin_amdgcn_raw_buffer_load_b128(rv, off, 0, 0);
                pk[i] = f32x4{__uint_as_float(a[0]), __uint_as_float(a[1]), __uint_as_float(a[2]), __uint_as_float(a[3])};
                pv[i] = f32x4{__uint_as_float(b[0]), __uint_as_float(b[1]), __uint_as_float(b[2]), __uint_as_float(b[3])};
            }
        } else {
            load_kv<DP, NW, VEC>(K, V, base, kt, seq, dim, pk, pv);
        }
    };
    if (t_begin < t_end) {  // block-uniform
        if constexpr (kSplitStage) {
            fetch(true, t_begin * kBKV, stage);
            store_rows<DP, NW>(lds, stage);
            fetch(false, t_begin * kBKV, stage);
            store_rows<DP, NW>(lds + S::kTile, stage);
        } else {
            fetch_both(t_begin * kBKV, stage, vstage);
            store_kv<DP, NW>(lds, stage, vstage);
        }
    }
    __syncthreads();

    for (int t = t_begin; t < t_end; ++t) {
        const int kt = t * kBKV;
        const bool more = t + 1 < t_end;
        // The next tile's buffer: no wave reads it during this tile (its last
        // reads were before the previous barrier).
        float *next = lds + ((t + 1 - t_begin) & 1) * 2 * S::kTile;
        if (more) {
            if constexpr (kSplitStage)
                fetch(true, kt + kBKV, stage);
            else
                fetch_both(kt + kBKV, stage, vstage);
        }
        const float *ks = lds + ((t - t_begin) & 1) * 2 * S::kTile;
        const float *vs = ks + S::kTile;
        // Sub-tiles of this tile the wave needs: none above its causal diagonal
        // and none wholly past seq. Wave-uniform.
        int subs = (kt + 32 < seq) ? 2 : 1;
        if (CAUSAL) subs = kt > q0 + 31 ? 0 : (kt + 32 > q0 + 31 ? 1 : subs);
        f32x16 st[2];
        float tile_max = -INFINITY;
        if (subs > 0) {
            // A tile whose 64 keys are all inside seq and at or below every
            // query of the wave needs no mask (wave-uniform).
            const bool full = kt + kBKV <= seq && (!CAUSAL || kt + kBKV - 1 <= q0);
            if (full) {
#pragma unroll
                for (int sb = 0; sb < 2; ++sb) {
                    const float *krow = ks + (sb * 32 + c) * LD + h * HALF;
#pragma unroll
                    for (int v = 0; v < 16; ++v) st[sb][v] = 0.f;
#pragma unroll
                    for (int s4 = 0; s4 < HALF / 4; ++s4) {
                        const f32x4 a = *reinterpret_cast<const f32x4 *>(krow + 4 * s4);
#pragma unroll
                        for (int e = 0; e < 4; ++e)
                            st[sb] = __builtin_amdgcn_mfma_f32_32x32x2f32(a[e], qreg[4 * s4 + e], st[sb], 0, 0, 0);
                    }
#pragma unroll
                    for (int v = 0; v < 16; ++v) tile_max = fmaxf(tile_max, st[sb][v]);
                }
            } else {
#pragma unroll
                for (int sb = 0; sb < 2; ++sb) {
#pragma unroll
                    for (int v = 0; v < 16; ++v) st[sb][v] = sb < subs ? 0.f : -INFINITY;
                    if (sb < subs) {
                        const float *krow = ks + (sb * 32 + c) * LD + h * HALF;
#pragma unroll
                        for (int s4 = 0; s4 < HALF / 4; ++s4) {
                            const f32x4 a = *reinterpret_cast<const f32x4 *>(krow + 4 * s4);
#pragma unroll
                            for (int e = 0; e < 4; ++e)
                                st[sb] =
                                    __builtin_amdgcn_mfma_f32_32x32x2f32(a[e], qreg[4 * s4 + e], st[sb], 0, 0, 0);
                        }
                    }
                }
                // Mask keys past seq and above the causal diagonal.
#pragma unroll
                for (int sb = 0; sb < 2; ++sb) {
#pragma unroll
                    for (int v = 0; v < 16; ++v) {
                        const int key = kt + sb * 32 + 8 * (v >> 2) + 4 * h + (v & 3);
                        const bool live = key < seq && (!CAUSAL || key <= qi);
                        st[sb][v] = live ? st[sb][v] : -INFINITY;
                        tile_max = fmaxf(tile_max, st[sb][v]);
                    }
                }
            }
        }
        // Split staging: the next tile's K goes to its buffer and its V takes
        // the registers.
        if (kSplitStage && more) {
            store_rows<DP, NW>(next, stage);
            fetch(false, kt + kBKV, stage);
        }
        if (subs > 0) {
            // The online max / normaliser update (log2 domain). The running
            // maximum is a lazy reference (kLazyMax): it moves only
            // when a tile exceeds it by more than 2^8, so the rescale below is
            // rarely needed.
            tile_max = halves_max(tile_max);
            float next_max = tile_max > row_max + kLazyMax ? tile_max : row_max;
            // A slice that starts past key 0 can meet a query with no live key
            // yet; keep its max finite so the weights below are 0, not NaN.
            if (SPLIT && next_max == -INFINITY) next_max = 0.f;
            const float old_weight = __builtin_amdgcn_exp2f(row_max - next_max);
            float tile_sum = 0.f;
#pragma unroll
            for (int sb = 0; sb < 2; ++sb) {
#pragma unroll
                for (int v = 0; v < 16; ++v) {
                    st[sb][v] = __builtin_amdgcn_exp2f(st[sb][v] - next_max);
                    tile_sum += st[sb][v];
                }
            }
            tile_sum = halves_sum(tile_sum);
            row_sum = row_sum * old_weight + tile_sum;
            row_max = next_max;
            // Once the running maxima settle, old_weight is exactly 1 in every
            // lane and the rescale is the identity: skip it (wave-uniform).
            if (__any(old_weight != 1.0f)) {
#pragma unroll
                for (int b = 0; b < NB; ++b) acc[b] *= old_weight;
            }

            // O^T += V^T P^T over the live sub-tiles. At head dim 128 the dims
            // are interleaved over the four accumulator blocks (block b, row r
            // holds dim 4r + b), so a lane's V operands of one key step for all
            // blocks are four adjacent floats, one ds_read_b128 where blocks
            // of 32 dims took four reads: LLM config 132.0 -> 133.9 TFLOP/s,
            // H64 S2048 D128 noncausal 135.1 -> 137.6. At head dim 64 (two
            // blocks, ds_read_b64) it was 1.5% slower, so there block b keeps
            // dims [32b, 32b + 32).
#pragma unroll
            for (int sb = 0; sb < 2; ++sb) {
                if (sb < subs) {
#pragma unroll
                    for (int v = 0; v < 16; ++v) {
                        const int key = sb * 32 + 8 * (v >> 2) + 4 * h + (v & 3);
                        if constexpr (kInterleaved) {
                            const VRow<NB> vr = *reinterpret_cast<const VRow<NB> *>(vs + key * LD + NB * c);
#pragma unroll
                            for (int b = 0; b < NB; ++b)
                                acc[b] = __builtin_amdgcn_mfma_f32_32x32x2f32(vr.x[b], st[sb][v], acc[b], 0, 0, 0);
                        } else {
                            const float *vrow = vs + key * LD + c;
#pragma unroll
                            for (int b = 0; b < NB; ++b)
                                acc[b] =
                                    __builtin_amdgcn_mfma_f32_32x32x2f32(vrow[32 * b], st[sb][v], acc[b], 0, 0, 0);
                        }
                    }
                }
            }
        }
        if (more) {
            if constexpr (kSplitStage)
                store_rows<DP, NW>(next + S::kTile, stage);
            else
                store_kv<DP, NW>(next, stage, vstage);
        }
        __syncthreads();
    }

    if (qi < seq) {
        float inv = 1.0f / row_sum;
        float *orow = O + base + size_t(qi) * dim;
        if (SPLIT) {
            const size_t rows = size_t(heads) * size_t(seq);
            const size_t row = size_t(head) * size_t(seq) + size_t(qi);
            // row_sum >= 1 once any key is live (the max key contributes 2^0).
            if (h == 0) ml[z * rows + row] = make_float2(row_sum == 0.f ? -INFINITY : row_max, row_sum);
            orow += z * rows * size_t(dim);
            inv = 1.0f;
        }
        if constexpr (kInterleaved) {
            // Register v of block b holds dim 4 (8 (v >> 2) + 4h + (v & 3)) + b:
            // for each v the four blocks give four adjacent dims.
#pragma unroll
            for (int v = 0; v < 16; ++v) {
                const int d = NB * (8 * (v >> 2) + 4 * h + (v & 3));
                if (VEC) {
                    if (d < dim) {
                        const f32x4 out = {acc[0][v] * inv, acc[1][v] * inv, acc[2][v] * inv, acc[3][v] * inv};
                        *reinterpret_cast<f32x4 *>(orow + d) = out;
                    }
                } else {
#pragma unroll
                    for (int b = 0; b < NB; ++b)
                        if (d + b < dim) orow[d + b] = acc[b][v] * inv;
                }
            }
        } else {
#pragma unroll
            for (int b = 0; b < NB; ++b) {
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

// Materialised scores on the matrix cores, for dim % 4 == 0 and 16-byte
// aligned rows: S[h] = Q[h] K[h]^T / sqrt(float(dim)), -inf above the causal
// diagonal. One wave per 32x32 tile (32 queries x 32 keys), four waves per
// block along the keys. Both MFMA operands are rows: lane (c, hf) needs
// Q[query c][16hf, 16hf+16) and K[key c][16hf, 16hf+16) of each 32-deep slice
// of dim, four 16-byte loads each, clamped into the tensors (a clamped query
// or key only reaches scores that are never stored; dims past `dim` are zeroed
// in both operands). Each slice is a 16-step MFMA chain from zero added to the
// running sum, as in the GEMM.
__global__ __launch_bounds__(256) void attention_scores_mfma(const float *__restrict__ Q, const float *__restrict__ K,
                                                             float *__restrict__ S, int seq, int dim, int causal) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int c = lane & 31, hf = lane >> 5;
    const int q0 = int(blockIdx.y) * 32, k0 = (int(blockIdx.x) * 4 + wave) * 32;
    if (k0 >= seq) return;  // wave-uniform; no barrier follows
    const size_t head = blockIdx.z;
    const float *qrow = Q + (head * seq + size_t(min(q0 + c, seq - 1))) * dim;
    const float *krow = K + (head * seq + size_t(min(k0 + c, seq - 1))) * dim;
    f32x16 acc;
#pragma unroll
    for (int v = 0; v < 16; ++v) acc[v] = 0.f;
    // Tiles wholly above the diagonal hold only -inf: no products needed.
    if (!(causal && k0 > q0 + 31)) {
        for (int d0 = 0; d0 < dim; d0 += 32) {
            const int db = d0 + 16 * hf;
            f32x4 a[4], b[4];
#pragma unroll
            for (int qd = 0; qd < 4; ++qd) {
                const int d = min(db + 4 * qd, dim - 4);
                a[qd] = *reinterpret_cast<const f32x4 *>(qrow + d);
                b[qd] = *reinterpret_cast<const f32x4 *>(krow + d);
            }
            const int valid = dim - db;  // operand pairs at s >= valid lie past dim
            f32x16 part;
#pragma unroll
            for (int v = 0; v < 16; ++v) part[v] = 0.f;
#pragma unroll
            for (int s4 = 0; s4 < 16; ++s4) {
                const float x = s4 < valid ? a[s4 >> 2][s4 & 3] : 0.f, y = s4 < valid ? b[s4 >> 2][s4 & 3] : 0.f;
                part = __builtin_amdgcn_mfma_f32_32x32x2f32(x, y, part, 0, 0, 0);
            }
            acc += part;
        }
    }
    const float root = sqrtf(float(dim));
    const int key = k0 + c;
#pragma unroll
    for (int v = 0; v < 16; ++v) {
        const int query = q0 + 8 * (v >> 2) + 4 * hf + (v & 3);
        if (query < seq && key < seq)
            S[(head * seq + query) * size_t(seq) + key] = (causal && key > query) ? -INFINITY : acc[v] / root;
    }
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

// Merges the key slices of a split launch: one thread per 4 outputs (VEC) or
// per output. A row of query block qb has ceil(T(qb)/per) slices, T(qb) being
// that block's key tiles. Split launches have fewer than 256 blocks of 128
// queries, so below 2^15 rows of at most 128 floats, and 32-bit indices cover
// them.
template <bool VEC, int MAXZ>
__global__ __launch_bounds__(256) void attention_combine(const float *__restrict__ part,
                                                         const float2 *__restrict__ ml, float *__restrict__ O,
                                                         uint32_t rows, uint32_t seq, uint32_t dim, uint32_t bq,
                                                         uint32_t per, int causal) {
    constexpr uint32_t W = VEC ? 4 : 1;
    const uint32_t per_row = dim / W;
    const uint32_t idx = blockIdx.x * 256u + threadIdx.x;
    if (idx >= rows * per_row) return;
    const uint32_t row = idx / per_row;
    const uint32_t qb = (row % seq) / bq;
    const uint32_t kv_end = causal ? min(seq, (qb + 1) * bq) : seq;
    const uint32_t tiles = (kv_end + kBKV - 1) / kBKV;
    const int slices = int((tiles + per - 1) / per);  // 1 <= slices <= MAXZ
    const uint32_t total = rows * dim;
    // Every slice's loads are issued before any is used (a loop over a
    // run-time count would wait for each load in turn). Indices past this
    // row's slices re-read its last slice, in bounds, and get weight 0.
    float2 s[MAXZ];
    f32x4 x[MAXZ];
#pragma unroll
    for (int z = 0; z < MAXZ; ++z) {
        const uint32_t zz = uint32_t(min(z, slices - 1));
        s[z] = ml[zz * rows + row];
        if constexpr (VEC)
            x[z] = *reinterpret_cast<const f32x4 *>(part + zz * total + idx * 4);
        else
            x[z][0] = part[zz * total + idx];
    }
    float top = -INFINITY;
#pragma unroll
    for (int z = 0; z < MAXZ; ++z) top = fmaxf(top, s[z].x);
    f32x4 num = {0.f, 0.f, 0.f, 0.f};
    float den = 0.f;
#pragma unroll
    for (int z = 0; z < MAXZ; ++z) {
        const float w = z < slices ? __builtin_amdgcn_exp2f(s[z].x - top) : 0.f;
        den = fmaf(w, s[z].y, den);
#pragma unroll
        for (int e = 0; e < int(W); ++e) num[e] = fmaf(w, x[z][e], num[e]);
    }
    if constexpr (VEC) {
        const f32x4 out = {num[0] / den, num[1] / den, num[2] / den, num[3] / den};
        *reinterpret_cast<f32x4 *>(O + idx * 4) = out;
    } else {
        O[idx] = num[0] / den;
    }
}

template <bool VEC>
void launch_combine(hipStream_t stream, const float *part, const float2 *ml, float *out, uint32_t rows, uint32_t seq,
                    uint32_t dim, uint32_t bq, uint32_t per, uint32_t slices, bool causal) {
    const uint32_t threads = rows * (VEC ? dim / 4 : dim);
    const dim3 grid((threads + 255) / 256), block(256);
    const int c = causal ? 1 : 0;
    if (slices <= 2)
        hipLaunchKernelGGL((attention_combine<VEC, 2>), grid, block, 0, stream, part, ml, out, rows, seq, dim, bq, per, c);
    else if (slices <= 4)
        hipLaunchKernelGGL((attention_combine<VEC, 4>), grid, block, 0, stream, part, ml, out, rows, seq, dim, bq, per, c);
    else if (slices <= 8)
        hipLaunchKernelGGL((attention_combine<VEC, 8>), grid, block, 0, stream, part, ml, out, rows, seq, dim, bq, per, c);
    else
        hipLaunchKernelGGL((attention_combine<VEC, 16>), grid, block, 0, stream, part, ml, out, rows, seq, dim, bq, per,
                           c);
}

int padded_dim(uint32_t dim) { return dim <= 32 ? 32 : dim <= 64 ? 64 : 128; }

// Eight waves per block when that still gives at least two blocks per CU;
// four waves (128 queries) for small problems so more CUs get work.
int waves_for(uint32_t heads, uint32_t seq) {
    const uint64_t blocks8 = uint64_t(heads) * ((seq + 255) / 256);
    return blocks8 >= 512 ? 8 : 4;
}

constexpr uint32_t kCUs = 256;

struct SplitPlan {
    uint32_t per;     // key tiles per slice
    uint32_t slices;  // slices of the longest rows (1 = no split)
    uint32_t live;    // blocks of a split launch: live slices over all rows
};

// Grids with at least one block per CU run unsplit. Smaller grids take the
// shortest slices whose live count still fits one block per CU, so the whole
// launch is one round of equal-cost slices (at most 16 slices per row).
SplitPlan split_plan(uint32_t heads, uint32_t seq, bool causal) {
    const uint32_t bq = 32u * uint32_t(waves_for(heads, seq));
    const uint32_t q_blocks = (seq + bq - 1) / bq;
    const uint32_t max_tiles = (seq + kBKV - 1) / kBKV;
    if (uint64_t(heads) * q_blocks >= kCUs) return {max_tiles, 1, 0};
    for (uint32_t per = (max_tiles + kMaxSplits - 1) / kMaxSplits; per < max_tiles; ++per) {
        uint64_t live = 0;
        for (uint32_t qb = 0; qb < q_blocks; ++qb) {
            const uint32_t kv_end = causal ? std::min(seq, (qb + 1) * bq) : seq;
            live += ((kv_end + kBKV - 1) / kBKV + per - 1) / per;
        }
        if (live * heads <= kCUs) return {per, (max_tiles + per - 1) / per, uint32_t(live * heads)};
    }
    return {max_tiles, 1, 0};
}

// Workspace layout of a split launch: slices*rows*dim partial O floats, then
// (rounded to 16 bytes) slices*rows float2 (max, normaliser); rows = heads*seq.
size_t split_part_floats(uint32_t heads, uint32_t seq, uint32_t dim, uint32_t slices) {
    const size_t n = size_t(slices) * heads * seq * dim;
    return (n + 3) & ~size_t(3);
}

// ---- Small grids: 16-query waves splitting keys inside the block -----------
// For grids whose 128-query blocks cannot fill the chip. A block of NW waves
// (eight for head dim 64, four for 128) owns two 16-query blocks of one head,
// x and X-1-x (X = ceil(seq/16); one block where the two coincide), so every
// block does the same work under the causal mask: x+1 and X-x 16-key units,
// X+1 in all (2X without the mask). A unit that serves both query blocks
// costs two, one that serves only X-1-x costs one; the block's units are cut
// into NW runs of equal cost, one per wave. Each wave loads its own K and V
// rows from global memory (L2) straight into registers in MFMA operand order,
// ahead of use, so the K loop has no LDS staging and no barrier. At the end
// the waves merge their partial (O, max, normaliser) rows through LDS and
// store O: no second launch and no workspace.
//
// Products run on v_mfma_f32_16x16x4_f32 in transposed form; lane l = 16g + i:
//  - S^T[key, query] over dims: step s takes dim (DP/4)g + s, so lane l
//    supplies K[key 16u + i][(DP/4)g + s] (A) and Q[query i][(DP/4)g + s]
//    (B), DP/4 consecutive floats of one row each. The result leaves lane l
//    holding query i's scores for keys 16u + 4g + r, r = 0..3, which are the
//    lane's B operands of the P.V product as they stand.
//  - O^T[dim, query] += V^T[dim, key] P^T[key, query]: step r takes keys
//    16u + 4g + r for lane group g, and row i of dim block db is dim
//    NDB i + db (NDB = DP/16), so lane l's A operands over db are the NDB
//    consecutive floats V[16u + 4g + r][NDB i ...]: vector loads.
//  - The O^T accumulators leave lane l holding query i's dims
//    (DP/4)g + NDB r' + db: DP/4 consecutive floats.
// Scores are in log2 units (Q pre-scaled by scale * log2(e)), as in the
// flash kernel above.
namespace pairs {
// Waves per block and units per chunk by padded head dim. A head-dim-64 wave
// fits in 256 registers, so eight-wave blocks hold two waves per SIMD and one
// wave's softmax runs beside the other's MFMAs (a wave's own VALU work does
// not overlap its MFMAs); a head-dim-128 wave needs more and runs alone on
// its SIMD in a four-wave block.
template <int DP>
struct Config {
    static constexpr int kWaves = DP == 64 ? 8 : 4, kChunk = 1;
};
constexpr int kUnit = 16;  // keys per unit, queries per query block

template <int DP>
struct UnitKV {
    static constexpr int kK = DP / 16, kV = DP / 64;
    f32x4 k[kK];     // K[16u + i][(DP/4)g + 4t ...], t < DP/16
    f32x4 v[4][kV];  // V[16u + 4g + r][NDB i + 4e ...], e < NDB/4
};

// Max and sum over the four lanes of one query (l, l^16, l^32, l^48), in the
// VALU: v_permlane16_swap pairs rows of 16 lanes, then v_permlane32_swap
// (above) pairs the two halves of the wave.
__device__ inline float rows_max(float x) {
    const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ inline float rows_sum(float x) {
    const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
__device__ inline float lanes_max(float x) { return halves_max(rows_max(x)); }
__device__ inline float lanes_sum(float x) { return halves_sum(rows_sum(x)); }

// Unconditional loads with row and column indices clamped into the tensors,
// so the compiler waits for exactly the chunk it consumes. A clamped key row
// only reaches masked scores (and P = 0 for V); a clamped dim of K meets a
// zero in Q, and a clamped dim of V only reaches outputs that are not stored.
template <int DP>
__device__ inline void load_unit_k(const float *__restrict__ K, size_t base, int key0, int seq, int dim, int i,
                                   int g, UnitKV<DP> &kv) {
    const size_t krow = size_t(min(key0 + i, seq - 1)) * dim;
#pragma unroll
    for (int t = 0; t < UnitKV<DP>::kK; ++t) {
        const int d = min((DP / 4) * g + 4 * t, dim - 4);
        kv.k[t] = *reinterpret_cast<const f32x4 *>(K + base + krow + d);
    }
}
template <int DP>
__device__ inline void load_unit_v(const float *__restrict__ V, size_t base, int key0, int seq, int dim, int i,
                                   int g, UnitKV<DP> &kv) {
    constexpr int NDB = DP / 16;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
        const size_t vrow = size_t(min(key0 + 4 * g + r, seq - 1)) * dim;
#pragma unroll
        for (int e = 0; e < UnitKV<DP>::kV; ++e) {
            const int d = min(NDB * i + 4 * e, dim - 4);
            kv.v[r][e] = *reinterpret_cast<const f32x4 *>(V + base + vrow + d);
        }
    }
}
// Unconditional loads with row and column indices clamped into the tensors,
// so the compiler waits for exactly the chunk it consumes. A clamped key row
// only reaches masked scores (and P = 0 for V); a clamped dim of K meets a
// zero in Q, and a clamped dim of V only reaches outputs that are not stored.
template <int DP>
__device__ inline void load_unit(const float *__restrict__ K, const float *__restrict__ V, size_t base, int key0,
                                 int seq, int dim, int i, int g, UnitKV<DP> &kv) {
    load_unit_k<DP>(K, base, key0, seq, dim, i, g, kv);
    load_unit_v<DP>(V, base, key0, seq, dim, i, g, kv);
}
}  // namespace pairs

// Grid: heads * ceil(X / 2) blocks, block b = pair b / heads of head b % heads
// (with `singles`, heads * X blocks, block b = query block b / heads alone).
// Needs dim % 4 == 0 and 16-byte aligned tensors (vector loads), dim <= DP.
template <int DP, bool CAUSAL, int CH, int NW>
__global__ __launch_bounds__(NW * 64) void attention_pairs_mfma(const float *__restrict__ Q,
                                                                        const float *__restrict__ K,
                                                                        const float *__restrict__ V,
                                                                        float *__restrict__ O, int seq, int dim,
                                                                        float qscale, int heads, int singles) {
    using namespace pairs;
    using KV = UnitKV<DP>;
    constexpr int D4 = DP / 4, NDB = DP / 16;
    // DP floats per query row, rows padded by 16 bytes: the flush's lanes
    // (query i, group g) write rows 16i + ... apart, which unpadded would put
    // sixteen lanes on the same LDS banks.
    __shared__ f32x4 part[NW * 2][kUnit][D4 + 1];
    __shared__ float2 mls[NW * 2][kUnit];

    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(int(threadIdx.x) >> 6);  // uniform: scalar loop control
    const int i = lane & 15, g = lane >> 4;
    const int blocks_q = (seq + kUnit - 1) / kUnit;  // query blocks, and key units
    const int head = int(blockIdx.x) % heads, pair = int(blockIdx.x) / heads;
    // `singles`: one query block per workgroup (noncausal small grids).
    const int xa = pair, xb = singles ? pair : blocks_q - 1 - pair;  // xa <= xb
    const bool single = xa == xb;
    // Key units [0, uc) serve both query blocks, [uc, ub) only xb (xa's keys
    // are a prefix of xb's under the causal mask, and all of them without it).
    const int ub = CAUSAL ? xb + 1 : blocks_q;
    const int uc = single ? 0 : (CAUSAL ? xa + 1 : blocks_q);
    // A shared unit costs two units of work, an xb-only unit one. Wave w
    // takes the units between the w-th and (w+1)-th quarter of the cost.
    const int cost = 2 * uc + (ub - uc);
    auto unit_at = [&](int c) { return c <= 2 * uc ? (c + 1) / 2 : c - uc; };
    const int u0 = unit_at(cost * wave / NW), u1 = unit_at(cost * (wave + 1) / NW);
    const size_t base = size_t(head) * size_t(seq) * size_t(dim);
    const f32x4 zero4 = {0.f, 0.f, 0.f, 0.f};

    // A chunk is up to CH units that are all shared or all xb-only, inside
    // the range [.., seg_end) the chunk loop is working on.
    int seg_end = u1;
    auto chunk_end = [&](int t) { return min(seg_end, min(t + CH, t < uc ? uc : ub)); };
    // Every chunk loads CH units; positions past the chunk's end re-read its
    // last unit and are never used.
    auto load_chunk = [&](KV(&buf)[CH], int t) {
        const int e = chunk_end(t);
#pragma unroll
        for (int c = 0; c < CH; ++c)
            pairs::load_unit<DP>(K, V, base, min(t + c, e - 1) * kUnit, seq, dim, i, g, buf[c]);
    };

    // Both query blocks' Q rows, scaled; dims past `dim` are zero.
    float qa[D4], qb[D4];
    auto load_q = [&](int x, float(&dst)[D4]) {
        const size_t row = size_t(min(x * kUnit + i, seq - 1)) * dim;
#pragma unroll
        for (int s4 = 0; s4 < D4 / 4; ++s4) {
            const int d = D4 * g + 4 * s4;
            const f32x4 v = *reinterpret_cast<const f32x4 *>(Q + base + row + min(d, dim - 4));
#pragma unroll
            for (int e = 0; e < 4; ++e) dst[4 * s4 + e] = d < dim ? v[e] * qscale : 0.f;
        }
    };
    load_q(xa, qa);
    load_q(xb, qb);

    // Per query block: O^T accumulators, the query's reference maximum (equal
    // in its four lanes) and this lane's share of the normaliser (the sum
    // over the query's keys 16u + 4g + r held by lane 16g + i); the four
    // shares are added once, when the rows are merged.
    struct State {
        f32x4 acc[NDB];
        float row_max, row_sum;
    };
    State sa, sb;
#pragma unroll
    for (int b = 0; b < NDB; ++b) sa.acc[b] = sb.acc[b] = zero4;
    sa.row_max = sb.row_max = -INFINITY;
    sa.row_sum = sb.row_sum = 0.f;

    // One chunk of n units starting at unit t for the 16 queries of block x.
    auto attend = [&](const KV(&kv)[CH], int t, int n, int x, const float(&q)[D4], State &st) {
        const int query = x * kUnit + i;
        f32x4 s[CH];
        float tile_max = -INFINITY;
#pragma unroll
        for (int c = 0; c < CH; ++c) {
            s[c] = zero4;
            if (c < n) {
#pragma unroll
                for (int d = 0; d < D4; ++d)
                    s[c] = __builtin_amdgcn_mfma_f32_16x16x4f32(kv[c].k[d >> 2][d & 3], q[d], s[c], 0, 0, 0);
                const int key0 = (t + c) * kUnit;
                // Only a unit on the causal diagonal or past the end of seq
                // holds masked keys (wave-uniform).
                if ((CAUSAL && t + c == x) || key0 + kUnit > seq) {
#pragma unroll
                    for (int r = 0; r < 4; ++r) {
                        const int key = key0 + 4 * g + r;
                        if (!(key < seq && (!CAUSAL || key <= query))) s[c][r] = -INFINITY;
                    }
                }
#pragma unroll
                for (int r = 0; r < 4; ++r) tile_max = fmaxf(tile_max, s[c][r]);
            }
        }
        // Every query of a processed chunk has a live key (the first key of
        // each unit lies at or below the diagonal and inside seq), so the
        // running max is finite from the first chunk on.
        tile_max = pairs::lanes_max(tile_max);
        const float next_max = fmaxf(st.row_max, tile_max);
        const float old_weight = __builtin_amdgcn_exp2f(st.row_max - next_max);
        float tile_sum = 0.f;
#pragma unroll
        for (int c = 0; c < CH; ++c)
            if (c < n) {
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    s[c][r] = __builtin_amdgcn_exp2f(s[c][r] - next_max);
                    tile_sum += s[c][r];
                }
            }
        st.row_sum = st.row_sum * old_weight + tile_sum;
        st.row_max = next_max;
        if (__any(old_weight != 1.0f)) {
#pragma unroll
            for (int b = 0; b < NDB; ++b) st.acc[b] *= old_weight;
        }
#pragma unroll
        for (int c = 0; c < CH; ++c)
            if (c < n) {
#pragma unroll
                for (int r = 0; r < 4; ++r)
#pragma unroll
                    for (int b = 0; b < NDB; ++b)
                        st.acc[b] =
                            __builtin_amdgcn_mfma_f32_16x16x4f32(kv[c].v[r][b >> 2][b & 3], s[c][r], st.acc[b], 0, 0, 0);
            }
    };
    // Shared chunks: both query blocks' scores, the online softmax update and
    // the P.V product, as separate steps so the pipelined loop below can put
    // the next chunk's scores beside this chunk's softmax.
    auto scores2 = [&](const KV(&kv)[CH], f32x4(&s_a)[CH], f32x4(&s_b)[CH]) {
#pragma unroll
        for (int c = 0; c < CH; ++c) {
            s_a[c] = zero4;
            s_b[c] = zero4;
#pragma unroll
            for (int d = 0; d < D4; ++d) {
                s_a[c] = __builtin_amdgcn_mfma_f32_16x16x4f32(kv[c].k[d >> 2][d & 3], qa[d], s_a[c], 0, 0, 0);
                s_b[c] = __builtin_amdgcn_mfma_f32_16x16x4f32(kv[c].k[d >> 2][d & 3], qb[d], s_b[c], 0, 0, 0);
            }
        }
    };
    // The online softmax of one chunk for both query blocks (TWO) or xb
    // alone, in place on the scores. Masks are selects on a wave-uniform flag
    // (MASK false: the caller knows no key of the chunk is masked). The
    // reference maximum is lazy (kLazyMax): a wave vote asks whether any
    // lane's own scores exceed its query's reference by more than kLazyMax;
    // only then (the first chunk, and rare jumps) do the queries take their
    // exact maxima across their four lanes, and the normaliser shares and
    // accumulators their rescale. Otherwise no cross-lane work is needed: the
    // weights exp2(s - reference) stay at most 2^kLazyMax. Softmax is exact
    // for any reference, so this differs from a tight maximum by rounding only.
    auto softmax2 = [&](f32x4(&s_a)[CH], f32x4(&s_b)[CH], int t, auto two, auto mask) {
        constexpr bool TWO = decltype(two)::value, MASK = decltype(mask)::value;
        auto lane_max = [&](f32x4(&s)[CH], int x) {
            const int query = x * kUnit + i;
            float m = -INFINITY;
#pragma unroll
            for (int c = 0; c < CH; ++c) {
                const int key0 = (t + c) * kUnit;
                // Only a unit on the causal diagonal or past the end of seq
                // holds masked keys (wave-uniform, rare).
                if (MASK && ((CAUSAL && t + c == x) || key0 + kUnit > seq)) {
#pragma unroll
                    for (int r = 0; r < 4; ++r) {
                        const int key = key0 + 4 * g + r;
                        if (!(key < seq && (!CAUSAL || key <= query))) s[c][r] = -INFINITY;
                    }
                }
#pragma unroll
                for (int r = 0; r < 4; ++r) m = fmaxf(m, s[c][r]);
            }
            return m;
        };
        const float ma = TWO ? lane_max(s_a, xa) : -INFINITY, mb = lane_max(s_b, xb);
        if (__any(ma > sa.row_max + kLazyMax || mb > sb.row_max + kLazyMax)) {
            // Every query of a processed chunk has a live key, so the new
            // maxima are finite. Exact maxima: weights at most 1 for this chunk.
            auto move = [&](float m, State &st) {
                const float next = fmaxf(st.row_max, pairs::lanes_max(m));
                const float w = __builtin_amdgcn_exp2f(st.row_max - next);
                st.row_max = next;
                st.row_sum *= w;
#pragma unroll
                for (int b = 0; b < NDB; ++b) st.acc[b] *= w;
            };
            if constexpr (TWO) move(ma, sa);
            move(mb, sb);
        }
        auto weigh = [&](f32x4(&s)[CH], State &st) {
            float sum = 0.f;
#pragma unroll
            for (int c = 0; c < CH; ++c)
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    s[c][r] = __builtin_amdgcn_exp2f(s[c][r] - st.row_max);
                    sum += s[c][r];
                }
            st.row_sum += sum;
        };
        if constexpr (TWO) weigh(s_a, sa);
        weigh(s_b, sb);
    };
    auto pv = [&](const KV(&kv)[CH], const f32x4(&s)[CH], State &st) {
#pragma unroll
        for (int c = 0; c < CH; ++c)
#pragma unroll
            for (int r = 0; r < 4; ++r)
#pragma unroll
                for (int b = 0; b < NDB; ++b)
                    st.acc[b] =
                        __builtin_amdgcn_mfma_f32_16x16x4f32(kv[c].v[r][b >> 2][b & 3], s[c][r], st.acc[b], 0, 0, 0);
    };
    // A whole shared chunk in one branch-free basic block for both query
    // blocks, so the scheduler can overlap one block's softmax with the
    // other's MFMAs.
    auto both_full = [&](const KV(&kv)[CH], int t) {
        f32x4 s_a[CH], s_b[CH];
        scores2(kv, s_a, s_b);
        softmax2(s_a, s_b, t, std::true_type{}, std::true_type{});
        pv(kv, s_a, sa);
        pv(kv, s_b, sb);
    };
    auto process = [&](const KV(&kv)[CH], int t) {
        const int n = chunk_end(t) - t;
        if (t < uc && n == CH) {
            both_full(kv, t);
            return;
        }
        if (t < uc) attend(kv, t, n, xa, qa, sa);
        attend(kv, t, n, xb, qb, sb);
    };

    // A wave's units run as a software pipeline of whole chunks: chunk c's
    // scores are computed in step c-1, so in step c the MFMAs of chunk c+1's
    // scores sit beside chunk c's softmax, then chunk c's P.V follows. K runs
    // two chunks ahead of use, V one; each has two buffers. The step's
    // exponentials, loads and score MFMAs share one basic block with an
    // explicit interleave; a unit holding masked keys (a diagonal unit, the
    // ragged last unit) takes its masks behind a wave-uniform branch. Two runs:
    // the shared units [u0, uc) (both query blocks) and the xb-only units
    // [uc, u1) (xb alone). What a run leaves over (less than a chunk) takes
    // the chunk loop further down.
    // The pipeline's loads are buffer loads: a per-lane byte offset fixed for
    // the kernel plus the unit's row offset as a scalar, so a load costs no
    // address arithmetic (a head's K and V must fit 2 GiB each); rows past
    // seq read zero.
    const bool offsets_fit = size_t(seq) * size_t(dim) * 4u < (size_t(1) << 31);
    auto steps_in = [&](int lo, int hi) { return offsets_fit && hi - lo >= CH ? (hi - lo) / CH : 0; };
    // Noncausal runs stop at the last whole unit (their only masked unit is
    // the ragged last one), so their steps compile without the mask branch.
    const int end = CAUSAL ? u1 : min(u1, seq / kUnit);
    const int n_two = steps_in(u0, min(end, uc));  // wave-uniform
    const int up = u0 + n_two * CH;
    const int b_lo = max(u0, uc);
    const int n_one = steps_in(b_lo, min(end, ub));  // wave-uniform
    const int bp = b_lo + n_one * CH;

    const uint32_t head_bytes = uint32_t(seq) * uint32_t(dim) * 4u, unit_bytes = kUnit * uint32_t(dim) * 4u;
    const __amdgpu_buffer_rsrc_t rk =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<float *>(K + base), 0, int(head_bytes), int(kRawBuffer));
    const __amdgpu_buffer_rsrc_t rv =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<float *>(V + base), 0, int(head_bytes), int(kRawBuffer));
    // Lane offsets inside a unit: K row i, dims (DP/4) g + 4 s; V rows
    // 4 g + r, dims NDB i + 4 e (dims clamped as in load_unit).
    uint32_t ok[KV::kK], ov[4][KV::kV];
#pragma unroll
    for (int s4 = 0; s4 < KV::kK; ++s4)
        ok[s4] = (uint32_t(i) * uint32_t(dim) + uint32_t(min((DP / 4) * g + 4 * s4, dim - 4))) * 4u;
#pragma unroll
    for (int r = 0; r < 4; ++r)
#pragma unroll
        for (int e = 0; e < KV::kV; ++e)
            ov[r][e] = (uint32_t(4 * g + r) * uint32_t(dim) + uint32_t(min(NDB * i + 4 * e, dim - 4))) * 4u;
    auto load4 = [](__amdgpu_buffer_rsrc_t rsrc, uint32_t lane_offset, uint32_t unit_offset) {
        const auto v = __builtin_amdgcn_raw_buffer_load_b128(rsrc, int(lane_offset), int(unit_offset), 0);
        return f32x4{__uint_as_float(v[0]), __uint_as_float(v[1]), __uint_as_float(v[2]), __uint_as_float(v[3])};
    };
    auto load_k = [&](KV(&buf)[CH], int t) {
#pragma unroll
        for (int c = 0; c < CH; ++c)
#pragma unroll
            for (int s4 = 0; s4 < KV::kK; ++s4) buf[c].k[s4] = load4(rk, ok[s4], uint32_t(t + c) * unit_bytes);
    };
    auto load_v = [&](KV(&buf)[CH], int t) {
#pragma unroll
        for (int c = 0; c < CH; ++c)
#pragma unroll
            for (int r = 0; r < 4; ++r)
#pragma unroll
                for (int e = 0; e < KV::kV; ++e) buf[c].v[r][e] = load4(rv, ov[r][e], uint32_t(t + c) * unit_bytes);
    };
    // xb's scores alone, the chunk's units interleaved so that two MFMA
    // chains alternate.
    // Four-wave blocks (one wave per SIMD, no second wave to cover a
    // dependent MFMA) with one unit per chunk: the two halves of the head dim
    // run as two MFMA chains, added at the end. Measured: H4 S1024 D128
    // noncausal 26.5 -> 24.9 us, H16 S512 D128 causal 19.8 -> 19.3; with two
    // waves per SIMD (head dim 64) it cost 0.5-1%.
    auto scores1 = [&](const KV(&kv)[CH], f32x4(&s_b)[CH]) {
        if constexpr (CH == 1 && NW == 4) {
            f32x4 lo = zero4, hi = zero4;
#pragma unroll
            for (int d = 0; d < D4 / 2; ++d) {
                lo = __builtin_amdgcn_mfma_f32_16x16x4f32(kv[0].k[d >> 2][d & 3], qb[d], lo, 0, 0, 0);
                const int e = d + D4 / 2;
                hi = __builtin_amdgcn_mfma_f32_16x16x4f32(kv[0].k[e >> 2][e & 3], qb[e], hi, 0, 0, 0);
            }
            s_b[0] = lo + hi;
        } else {
#pragma unroll
            for (int c = 0; c < CH; ++c) s_b[c] = zero4;
#pragma unroll
            for (int d = 0; d < D4; ++d)
#pragma unroll
                for (int c = 0; c < CH; ++c)
                    s_b[c] = __builtin_amdgcn_mfma_f32_16x16x4f32(kv[c].k[d >> 2][d & 3], qb[d], s_b[c], 0, 0, 0);
        }
    };
    // `steps` chunks from unit p0, for both query blocks (TWO) or xb alone.
    auto pipeline = [&](int p0, int steps, auto two) {
        constexpr bool TWO = decltype(two)::value;
        const int last = p0 + (steps - 1) * CH;  // first unit of the last chunk
        auto scores = [&](const KV(&kv)[CH], f32x4(&s_a)[CH], f32x4(&s_b)[CH]) {
            if constexpr (TWO)
                scores2(kv, s_a, s_b);
            else
                scores1(kv, s_b);
        };
        // Chunk t's softmax and P.V from its scores (s_a, s_b) and V.
        auto consume = [&](int t, const KV(&vcur)[CH], f32x4(&s_a)[CH], f32x4(&s_b)[CH]) {
            softmax2(s_a, s_b, t, two, std::bool_constant<CAUSAL>{});
            if constexpr (TWO) pv(vcur, s_a, sa);
            pv(vcur, s_b, sb);
        };
        KV kb0[CH], kb1[CH], vb0[CH], vb1[CH];
        f32x4 sa0[CH], sb0[CH], sa1[CH], sb1[CH];
        load_k(kb0, p0);
        load_k(kb1, min(p0 + CH, last));
        load_v(vb0, p0);
        scores(kb0, sa0, sb0);
        // Step for chunk t, not the last: scores in (s_a, s_b), V in vcur; the
        // next chunk's K in knext, its scores into (n_a, n_b); kfree takes the
        // K two chunks ahead and vnext the next chunk's V. Positions past the
        // run re-read its last chunk and are never used.
        auto step = [&](int t, KV(&kfree)[CH], const KV(&knext)[CH], const KV(&vcur)[CH], KV(&vnext)[CH],
                        f32x4(&s_a)[CH], f32x4(&s_b)[CH], f32x4(&n_a)[CH], f32x4(&n_b)[CH]) {
            // The softmax's rare rescale branch comes first, so that its
            // exponentials, the loads and the next chunk's score MFMAs share
            // one basic block.
            softmax2(s_a, s_b, t, two, std::bool_constant<CAUSAL>{});
            load_k(kfree, min(t + 2 * CH, last));
            load_v(vnext, min(t + CH, last));
            scores(knext, n_a, n_b);
            // CH D4 score MFMAs per query block and CH DP/8 vector loads; the
            // softmax fills the MFMA shadow.
            constexpr int kMfma = (TWO ? 2 : 1) * CH * D4, kLoads = CH * DP / 8;
#pragma unroll
            for (int j = 0; j < kLoads; ++j) {
                __builtin_amdgcn_sched_group_barrier(0x020, 1, 0);  // one load
                __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // one MFMA
                __builtin_amdgcn_sched_group_barrier(0x002, 4, 0);  // VALU
            }
#pragma unroll
            for (int j = kLoads; j < kMfma; ++j) {
                __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
                __builtin_amdgcn_sched_group_barrier(0x002, 3, 0);
            }
            __builtin_amdgcn_sched_barrier(0);
            if constexpr (TWO) pv(vcur, s_a, sa);
            pv(vcur, s_b, sb);
            // Nothing crosses into the next step: its scores wait on this
            // step's loads.
            __builtin_amdgcn_sched_barrier(0);
        };
        // Two steps per iteration with no branch between them: a step's
        // prefetch is consumed by the next step, and a block boundary there
        // lets the compiler sink the loads to their use.
        int t = p0, n = steps - 1;  // steps before the last
        for (; n >= 2; n -= 2, t += 2 * CH) {
            step(t, kb0, kb1, vb0, vb1, sa0, sb0, sa1, sb1);
            step(t + CH, kb1, kb0, vb1, vb0, sa1, sb1, sa0, sb0);
        }
        if (n) {
            step(t, kb0, kb1, vb0, vb1, sa0, sb0, sa1, sb1);
            consume(t + CH, vb1, sa1, sb1);
        } else {
            consume(t, vb0, sa0, sb0);
        }
    };
    if (n_two) pipeline(u0, n_two, std::true_type{});
    if (n_one) pipeline(b_lo, n_one, std::false_type{});

    // The rest: [up, b_lo) and [bp, u1) when the xb-only run was taken,
    // [up, u1) otherwise. Two chunk buffers: the next chunk's loads are in
    // flight while the current one is consumed (the last prefetch re-reads
    // the last chunk).
    KV buf0[CH], buf1[CH];
    for (int part = 0; part < 2; ++part) {
        const int lo = part == 0 ? up : (n_one ? bp : u1);
        seg_end = part == 0 && n_one ? b_lo : u1;
        if (lo >= seg_end) continue;
        int t = lo;
        load_chunk(buf0, t);
        for (;;) {
            int e = chunk_end(t);
            load_chunk(buf1, e < seg_end ? e : t);
            process(buf0, t);
            t = e;
            if (t >= seg_end) break;
            e = chunk_end(t);
            load_chunk(buf0, e < seg_end ? e : t);
            process(buf1, t);
            t = e;
            if (t >= seg_end) break;
        }
    }

    // Partial rows to LDS: slot (wave, 0) for xa, (wave, 1) for xb. A block
    // this wave did not touch leaves (max -inf, sum 0, zero row): weight 0 in
    // the merge.
    auto flush = [&](const State &st, int slot) {
#pragma unroll
        for (int r = 0; r < 4; ++r)
#pragma unroll
            for (int e = 0; e < NDB / 4; ++e) {
                const f32x4 o = {st.acc[4 * e][r], st.acc[4 * e + 1][r], st.acc[4 * e + 2][r], st.acc[4 * e + 3][r]};
                part[slot][i][(D4 * g + NDB * r) / 4 + e] = o;
            }
        const float row_sum = pairs::lanes_sum(st.row_sum);  // the query's four shares
        if (g == 0) mls[slot][i] = make_float2(st.row_max, row_sum);
    };
    flush(sa, wave * 2);
    flush(sb, wave * 2 + 1);
    __syncthreads();

    // Merge: thread -> (query block, query, 4 dims). With a single query
    // block, slot 1 of every wave holds it.
    for (int o = int(threadIdx.x); o < 2 * kUnit * D4; o += NW * 64) {
        const int seg = o / (kUnit * D4), rest = o % (kUnit * D4);
        const int qi = rest / D4, d4 = rest % D4;
        if (seg == 0 && single) continue;
        const int q = (seg ? xb : xa) * kUnit + qi, d = 4 * d4;
        if (q >= seq || d >= dim) continue;
        float top = -INFINITY;
#pragma unroll
        for (int w = 0; w < NW; ++w) top = fmaxf(top, mls[w * 2 + seg][qi].x);
        f32x4 num = zero4;
        float den = 0.f;
#pragma unroll
        for (int w = 0; w < NW; ++w) {
            const float2 ml = mls[w * 2 + seg][qi];
            const float wt = __builtin_amdgcn_exp2f(ml.x - top);
            den = fmaf(wt, ml.y, den);
            num += wt * part[w * 2 + seg][qi][d4];
        }
        const float inv = 1.0f / den;
        *reinterpret_cast<f32x4 *>(O + base + size_t(q) * dim + d) = num * inv;
    }
}

template <int DP, int NW, bool CAUSAL, bool SPLIT>
hipError_t launch_online(hipStream_t stream, const float *q, const float *k, const float *v, float *out,
                         float2 *ml, uint32_t heads, uint32_t seq, uint32_t dim, SplitPlan plan, bool vec) {
    using S = AttnShape<DP, NW>;
    const unsigned q_blocks = (seq + S::kBQ - 1) / S::kBQ;
    const float qscale = (1.0f / sqrtf(float(dim))) * kLog2e;
    const dim3 grid = SPLIT ? dim3(plan.live) : dim3(heads, q_blocks), block(S::kThreads);
    // The vector kernel reads K and V through buffer loads over one head.
    if (vec && uint64_t(seq) * uint64_t(dim) * 4u < (uint64_t(1) << 31))
        hipLaunchKernelGGL((attention_online_mfma<DP, NW, CAUSAL, true, SPLIT>), grid, block, 0, stream, q, k, v,
                           out, ml, int(seq), int(dim), qscale, int(plan.per), int(heads));
    else
        hipLaunchKernelGGL((attention_online_mfma<DP, NW, CAUSAL, false, SPLIT>), grid, block, 0, stream, q, k, v,
                           out, ml, int(seq), int(dim), qscale, int(plan.per), int(heads));
    return hipGetLastError();
}


// Blocks of the paired 16-query launch: heads x ceil(X / 2), X = ceil(seq / 16).
// How a grid that would otherwise split keys across blocks runs the 16-query
// kernel: not at all, on pairs of query blocks, or on single query blocks.
enum class PairMode { None, Pairs, Singles };

uint32_t query_units(uint32_t seq) { return (seq + 15) / 16; }
uint32_t pair_blocks(uint32_t heads, uint32_t seq) { return heads * ((query_units(seq) + 1) / 2); }

// Paired blocks run when the rows take vector loads (dim % 4 == 0), the head
// dim pads to 64 or 128, and the launch has at least kPairsMinBlocks blocks,
// or each wave has little work: at most kPairsSmallWork key units per wave (a
// shared unit counts twice, a head-dim-128 unit twice). Other small grids
// keep the split launch, which spreads any grid over every CU at the cost of a
// second, merging launch. Measured on MI355X, split against paired (us): H4
// S512 D64 causal 13.2 / 11.7 and H4 S256 D64 noncausal 11.3 / 10.1 (4 units
// per wave); H4 S512 D64 noncausal 13.3 / 14.8 (8); H2 S1024 D64 causal 16.4 /
// 16.5 (8); H2 S1024 D64 noncausal 17.5 / 23.7 and H1 S2048 D64 causal 22.0 /
// 25.3 (16).
//
// Noncausal rows need no pairing for balance: where one query block per
// workgroup still fits one round of the CUs, it halves each wave's work (at
// the price of loading each K/V unit for 16 queries instead of 32). Taken
// with at least kSinglesFullBlocks workgroups and at most kSinglesMaxWork
// units per wave, or with at most kSinglesSmallWork units per wave. Measured
// (us), split or paired against singles: H1 S4096 D64 49.7 / 42.6 (256
// workgroups, 32 units per wave), H2 S2048 D64 30.3 / 24.3, H3 S1024 D64
// 19.3 / 15.5 (192), H4 S1024 D64 23.8 (paired) / 15.5, H8 S512 D128 26.7 /
// 20.3, H4 S1024 D128 35.7 / 32.3 (32 units); H2 S1024 D64 17.5 / 15.5 (128
// workgroups, 8 units); against them H2 S2048 D128 54.5 / 55.8 (64 units) and
// H1 S2048 D64 22.6 / 24.2 (128 workgroups, 16 units).
constexpr uint32_t kPairsMinBlocks = 128, kPairsSmallWork = 6;
constexpr uint32_t kSinglesMaxBlocks = 256, kSinglesFullBlocks = 192, kSinglesMaxWork = 32, kSinglesSmallWork = 8;
PairMode pair_mode(uint32_t heads, uint32_t seq, uint32_t dim, bool causal) {
    if (split_plan(heads, seq, causal).slices <= 1 || dim % 4 != 0 || padded_dim(dim) < 64) return PairMode::None;
    const int dp = padded_dim(dim);
    const uint32_t x = query_units(seq), scale = uint32_t(dp / 64);
    const uint32_t waves = dp == 64 ? pairs::Config<64>::kWaves : pairs::Config<128>::kWaves;
    const uint64_t singles = uint64_t(heads) * x;
    const uint32_t single_work = x * scale;  // per workgroup; per wave after dividing by `waves`
    if (!causal && singles <= kSinglesMaxBlocks &&
        ((singles >= kSinglesFullBlocks && single_work <= kSinglesMaxWork * waves) ||
         single_work <= kSinglesSmallWork * waves))
        return PairMode::Singles;
    if (pair_blocks(heads, seq) >= kPairsMinBlocks) return PairMode::Pairs;
    const uint32_t cost = causal ? x + 1 : 2 * x;
    return cost * scale <= kPairsSmallWork * waves ? PairMode::Pairs : PairMode::None;
}
uint32_t pair_mode_blocks(uint32_t heads, uint32_t seq, PairMode mode) {
    return mode == PairMode::Singles ? heads * query_units(seq) : pair_blocks(heads, seq);
}

template <int DP>
hipError_t launch_pairs(hipStream_t stream, const float *q, const float *k, const float *v, float *out,
                        uint32_t heads, uint32_t seq, uint32_t dim, bool causal, PairMode mode) {
    using C = pairs::Config<DP>;
    const float qscale = (1.0f / sqrtf(float(dim))) * kLog2e;
    const dim3 grid(pair_mode_blocks(heads, seq, mode)), block(C::kWaves * 64);
    const int singles = mode == PairMode::Singles ? 1 : 0;
    if (causal)
        hipLaunchKernelGGL((attention_pairs_mfma<DP, true, C::kChunk, C::kWaves>), grid, block, 0, stream, q, k, v,
                           out, int(seq), int(dim), qscale, int(heads), singles);
    else
        hipLaunchKernelGGL((attention_pairs_mfma<DP, false, C::kChunk, C::kWaves>), grid, block, 0, stream, q, k, v,
                           out, int(seq), int(dim), qscale, int(heads), singles);
    return hipGetLastError();
}

template <int DP>
hipError_t dispatch_dim(hipStream_t stream, const float *q, const float *k, const float *v, float *out,
                        float *workspace, uint32_t heads, uint32_t seq, uint32_t dim, bool causal, bool vec) {
    if constexpr (DP >= 64) {
        const PairMode mode = pair_mode(heads, seq, dim, causal);
        if (vec && mode != PairMode::None) return launch_pairs<DP>(stream, q, k, v, out, heads, seq, dim, causal, mode);
    }
    const SplitPlan plan = split_plan(heads, seq, causal);
    if (plan.slices > 1) {
        // Split grids are small grids, which always take four-wave blocks.
        if (waves_for(heads, seq) != 4 || workspace == nullptr) return hipErrorInvalidValue;
        float *part = workspace;
        float2 *ml = reinterpret_cast<float2 *>(workspace + split_part_floats(heads, seq, dim, plan.slices));
        const hipError_t status =
            causal ? launch_online<DP, 4, true, true>(stream, q, k, v, part, ml, heads, seq, dim, plan, vec)
                   : launch_online<DP, 4, false, true>(stream, q, k, v, part, ml, heads, seq, dim, plan, vec);
        if (status != hipSuccess) return status;
        const uint32_t bq = AttnShape<DP, 4>::kBQ;
        if (vec)
            launch_combine<true>(stream, part, ml, out, heads * seq, seq, dim, bq, plan.per, plan.slices, causal);
        else
            launch_combine<false>(stream, part, ml, out, heads * seq, seq, dim, bq, plan.per, plan.slices, causal);
        return hipGetLastError();
    }
    const SplitPlan whole{plan.per, 1, 0};
    if (waves_for(heads, seq) == 8)
        return causal ? launch_online<DP, 8, true, false>(stream, q, k, v, out, nullptr, heads, seq, dim, whole, vec)
                      : launch_online<DP, 8, false, false>(stream, q, k, v, out, nullptr, heads, seq, dim, whole, vec);
    return causal ? launch_online<DP, 4, true, false>(stream, q, k, v, out, nullptr, heads, seq, dim, whole, vec)
                  : launch_online<DP, 4, false, false>(stream, q, k, v, out, nullptr, heads, seq, dim, whole, vec);
}

int pairs_waves(int dp) { return dp == 64 ? pairs::Config<64>::kWaves : pairs::Config<128>::kWaves; }

template <int DP>
uint32_t lds_bytes(int nw) {
    return nw == 8 ? AttnShape<DP, 8>::kLdsBytes : AttnShape<DP, 4>::kLdsBytes;
}

}  // namespace

LaunchShape attention_online_shape(uint32_t heads, uint32_t seq, uint32_t dim, bool causal) {
    const int dp = padded_dim(dim);
    const PairMode mode = pair_mode(heads, seq, dim, causal);
    if (mode != PairMode::None) {
        static const char *const names[2][2] = {
            {"attention_online_mfma16_d64_pairs", "attention_online_mfma16_d128_pairs"},
            {"attention_online_mfma16_d64_singles", "attention_online_mfma16_d128_singles"}};
        return {names[mode == PairMode::Singles][dp == 64 ? 0 : 1],
                {pair_mode_blocks(heads, seq, mode), 1, 1},
                {uint32_t(pairs_waves(dp) * 64), 1, 1},
                uint32_t(pairs_waves(dp) * 2 * pairs::kUnit * ((dp + 4) * sizeof(float) + sizeof(float2)))};
    }
    const int nw = waves_for(heads, seq);
    const uint32_t bq = 32u * nw;
    const SplitPlan plan = split_plan(heads, seq, causal);
    const uint32_t splits = plan.slices;
    const uint32_t lds = dp == 32 ? lds_bytes<32>(nw) : dp == 64 ? lds_bytes<64>(nw) : lds_bytes<128>(nw);
    static const char *const names[2][3] = {
        {"attention_online_mfma_d32", "attention_online_mfma_d64", "attention_online_mfma_d128"},
        {"attention_online_mfma_d32_split", "attention_online_mfma_d64_split", "attention_online_mfma_d128_split"}};
    return {names[splits > 1][dp == 32 ? 0 : dp == 64 ? 1 : 2],
            {splits > 1 ? plan.live : heads, splits > 1 ? 1u : (seq + bq - 1) / bq, 1},
            {uint32_t(nw) * 64u, 1, 1},
            lds};
}

size_t attention_online_workspace_bytes(uint32_t heads, uint32_t seq, uint32_t dim, bool causal) {
    if (pair_mode(heads, seq, dim, causal) != PairMode::None) return 0;
    const uint32_t splits = split_plan(heads, seq, causal).slices;
    if (splits <= 1) return 0;
    return (split_part_floats(heads, seq, dim, splits) + 2 * size_t(splits) * heads * seq) * sizeof(float);
}

hipError_t attention_online_f32(hipStream_t stream, const float *q, const float *k, const float *v, float *out,
                                uint32_t heads, uint32_t seq, uint32_t dim, bool causal, float *workspace) {
    const bool aligned =
        ((reinterpret_cast<uintptr_t>(q) | reinterpret_cast<uintptr_t>(k) | reinterpret_cast<uintptr_t>(v) |
          reinterpret_cast<uintptr_t>(out)) &
         15u) == 0;
    const bool vec = aligned && dim % 4 == 0;
    switch (padded_dim(dim)) {
        case 32: return dispatch_dim<32>(stream, q, k, v, out, workspace, heads, seq, dim, causal, vec);
        case 64: return dispatch_dim<64>(stream, q, k, v, out, workspace, heads, seq, dim, causal, vec);
        default: return dispatch_dim<128>(stream, q, k, v, out, workspace, heads, seq, dim, causal, vec);
    }
}

// The materialised path runs on the matrix cores when rows are 16-byte
// aligned (dim % 4 == 0 for the scores, seq % 4 == 0 for P.V), else on the
// one-thread-per-output kernels. Measured at H4 S512 D64: the three launches
// took 0.18 ms with the scalar kernels.
bool scores_on_mfma(uint32_t dim, const void *q, const void *k) {
    return dim % 4 == 0 && ((reinterpret_cast<uintptr_t>(q) | reinterpret_cast<uintptr_t>(k)) & 15u) == 0;
}

LaunchShape attention_scores_shape(uint32_t heads, uint32_t seq, uint32_t dim, bool) {
    if (dim % 4 == 0) return {"attention_scores_mfma", {(seq + 127) / 128, (seq + 31) / 32, heads}, {256, 1, 1}, 0};
    return {"attention_scores", {(seq + 15) / 16, (seq + 15) / 16, heads}, {256, 1, 1}, 0};
}

hipError_t attention_scores_f32(hipStream_t stream, const float *q, const float *k, float *scores, uint32_t heads,
                                uint32_t seq, uint32_t dim, bool causal) {
    if (scores_on_mfma(dim, q, k)) {
        const dim3 grid((seq + 127) / 128, (seq + 31) / 32, heads);
        hipLaunchKernelGGL(attention_scores_mfma, grid, dim3(256), 0, stream, q, k, scores, int(seq), int(dim),
                           causal ? 1 : 0);
        return hipGetLastError();
    }
    const dim3 grid((seq + 15) / 16, (seq + 15) / 16, heads);
    hipLaunchKernelGGL(attention_scores_kernel, grid, dim3(256), 0, stream, q, k, scores, int(seq), int(dim),
                       causal ? 1 : 0);
    return hipGetLastError();
}

LaunchShape attention_apply_shape(uint32_t heads, uint32_t seq, uint32_t dim) {
    if (seq % 4 == 0)
        return {"attention_apply_mfma", {((seq + 31) / 32) * ((dim + 31) / 32), heads, 1}, {256, 1, 1}, 3 * 16 * 64 * 4};
    return {"attention_apply", {(dim + 15) / 16, (seq + 15) / 16, heads}, {256, 1, 1}, 0};
}

hipError_t attention_apply_f32(hipStream_t stream, const float *p, const float *v, float *out, uint32_t heads,
                               uint32_t seq, uint32_t dim) {
    // out[h] = P[h] (seq x seq) . V[h] (seq x dim): a batched GEMM over heads.
    if (seq % 4 == 0 && (reinterpret_cast<uintptr_t>(p) & 15u) == 0)
        return gemm_f32_batched_direct(stream, p, v, out, seq, dim, seq, heads, size_t(seq) * seq, size_t(seq) * dim,
                                       size_t(seq) * dim);
    const dim3 grid((dim + 15) / 16, (seq + 15) / 16, heads);
    hipLaunchKernelGGL(attention_apply_kernel, grid, dim3(256), 0, stream, p, v, out, int(seq), int(dim));
    return hipGetLastError();
}

}  // namespace hipk
}  // namespace jade
