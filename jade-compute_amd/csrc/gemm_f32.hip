// FP32 GEMM on CDNA4 matrix cores: C[M,N] = A[M,K] * B[K,N], packed row-major.
// Semantics follow the reference's Gemm/GemmSimd ops (src/runtime/ir.rs:21-32,
// 524-557; src/runtime/metal_simd.rs:29-110): no alpha/beta, no transposes,
// ragged edges read as zero and masked on store.
//
// Design (gfx950, wave64):
//  * A 256-thread workgroup is a 2x2 grid of waves; each wave owns TM x TN
//    blocks of v_mfma_f32_32x32x2_f32 (16 accumulators per lane per block), so
//    a workgroup tile is (64*TM) x (64*TN): 128x128, 128x64 or 64x64, two
//    workgroups per CU. Two independent products of one shape can share a
//    launch. Grids of at most one 64x64 tile per CU run two or four such
//    groups of four waves per workgroup (KG), each over a share of the tile's
//    K stages.
//  * Grids of at least 256 whole 256x256 tiles run as 128x128 tiles, or, when
//    that grid's last round would be under a quarter full, as whole rounds of
//    gemm_f32_mfma_256 (one 512-thread workgroup per CU, eight waves of
//    128x64) plus a partial round of 128x128 or 64x64 tiles.
//  * K advances 32 per stage. Stages are double-buffered in LDS and filled by
//    LDS-direct loads: global loads for interior tiles, range-checked buffer
//    loads for edge tiles, for unaligned rows over whole stages and, masked
//    past the K range, for K ranges with a partial stage (K of at least 256;
//    not unaligned K with two K groups). The rest, and operands too long for
//    32-bit offsets, take a register prefetch (unaligned 64x64 and 128x64
//    tiles keep two stages in registers, loaded through buffer
//    instructions). One barrier per stage.
//  * The MFMA K=2 operand split is permuted: lanes 0-31 take k in [0,16) and
//    lanes 32-63 take k in [16,32) of a stage, so an A operand run is 16
//    contiguous floats per lane (ds_read_b128) while B stays ds_read_b32 with
//    consecutive lanes on consecutive columns. A and B share the permutation,
//    so every product is still summed exactly once.
//  * Workgroup ids are remapped so each of the 8 XCDs (dispatched round-robin)
//    owns a contiguous range of tiles in grouped order, keeping A rows and B
//    columns hot in that XCD's private L2.
//  * Two-level accumulation: a run of one or two 32-deep K stages is summed by
//    the matrix cores into zeroed accumulators and then added to the running
//    sums with round-to-nearest VALU adds. A single chained MFMA accumulation
//    over K = 4096 drifted by ~3.6e-4 absolute on unit-scale inputs, outside
//    the 1e-4 gate; the split keeps the long recurrence to K/32 or K/64 adds.
//  * Small grids with aligned A rows and moderate K run gemm_f32_direct: 32x32
//    tiles whose waves split K, operands loaded straight into registers, one
//    launch (below).
//  * Other shapes with too few output tiles to fill 256 CUs split K over
//    gridDim.y: each slice writes a partial product to a workspace and a
//    reduction kernel sums the slices in slice order (deterministic, no atomics).
#include "gemm_tiles.hpp"
#include "kernels.hpp"
#include "ops.hpp"

#include <algorithm>
#include <type_traits>

namespace jade {
namespace hipk {
namespace {

constexpr int kThreads = 256;
// Last k of an unaligned K-group tile's range that may add in its epilogue
// (gemm_f32_mfma) rather than as a stage of their own.
constexpr int kMaxTail = 2;
constexpr int kLDA = kBK + 4;  // LDS row stride of an A stage (floats)
constexpr uint32_t kBufferWord3 = 0x00020000;  // raw buffer, 32-bit data format
// A buffer-load offset past every buffer these kernels read (each below
// 2 GiB): the range check returns zero without touching memory.
constexpr uint32_t kDeadOffset = 0x80000000u;

template <int TM, int TN>
struct Tile {
    static constexpr int kBM = 64 * TM, kBN = 64 * TN;
    static constexpr int kLDB = kBN + 4;  // LDS row stride of a B stage (floats)
    static constexpr int kAStage = kBM * kLDA;
    static constexpr int kBStage = kBK * kLDB;
    static constexpr int kStage = kAStage + kBStage;
    static constexpr int kALoads = kBM * kBK / 4 / kThreads;  // float4 per thread
    static constexpr int kBLoads = kBK * kBN / 4 / kThreads;
    // Unpadded, XOR-swizzled stage written by LDS-direct loads (interior tiles).
    static constexpr int kAStageS = kBM * kBK, kBStageS = kBK * kBN, kStageS = kAStageS + kBStageS;
    static constexpr int kAInst = kAStageS * 4 / 1024 / 4;  // 1 KB LDS-direct loads per wave
    static constexpr int kBInst = kBStageS * 4 / 1024 / 4;
    static_assert(kStageS <= kStage, "swizzled stage must fit in the padded stage allocation");
    static constexpr uint32_t kLdsBytes = 2u * kStage * sizeof(float);
};

// Tile column of lane c's outputs in MFMA block j of a wave in column wn.
// With two blocks per wave (TN = 2) the blocks interleave: block j holds the
// wave's columns 2c + j, so a lane's two B operands of a k row are adjacent
// and come in one 8-byte LDS read. One block: columns 32 wn + c.
template <int TN>
__device__ inline int tile_col(int wn, int j, int c) {
    return TN == 2 ? wn * 64 + 2 * c + j : wn * 32 * TN + j * 32 + c;
}

template <int TM, int TN>
__device__ inline void issue_stage_dma(const float *__restrict__ A, const float *__restrict__ B, int N, int K,
                                       int m0, int n0, int k0, uint32_t stage_lds, int t) {
    using T = Tile<TM, TN>;
    const int lane = t & 63, wave = t >> 6;
    const float *abase = A + size_t(m0) * K + k0;
    const float *bbase = B + size_t(k0) * N + n0;
    const uint32_t sb = stage_lds + T::kAStageS * 4;
#pragma unroll
    for (int i = 0; i < T::kAInst; ++i) {  // eight 128-byte A rows per 1 KB load
        const int inst = wave * T::kAInst + i;
        const int row = inst * 8 + (lane >> 3), j = (lane & 7) ^ swz_a(row);
        lds_dma16(abase, uint32_t((row * K + 4 * j) * 4), stage_lds + inst * 1024);
    }
    constexpr int kChunks = T::kBN / 4, kRowsPer = 64 / kChunks;
#pragma unroll
    for (int i = 0; i < T::kBInst; ++i) {  // BN*4-byte B rows, kRowsPer per 1 KB load
        const int inst = wave * T::kBInst + i;
        const int row = inst * kRowsPer + lane / kChunks, j = (lane % kChunks) ^ swz_b(row);
        lds_dma16(bbase, uint32_t((row * N + 4 * j) * 4), sb + inst * 1024);
    }
}

// Loads [p n / P, (p + 1) n / P) of the n = kAInst + kBInst that
// issue_stage_dma issues (A's first), for a stage spread over P parts.
template <int TM, int TN, int P>
__device__ inline void issue_stage_dma_part(const float *__restrict__ A, const float *__restrict__ B, int N, int K,
                                            int m0, int n0, int k0, uint32_t stage_lds, int t, int p) {
    using T = Tile<TM, TN>;
    constexpr int kN = T::kAInst + T::kBInst;
    const int lane = t & 63, wave = t >> 6;
    const float *abase = A + size_t(m0) * K + k0;
    const float *bbase = B + size_t(k0) * N + n0;
    const uint32_t sb = stage_lds + T::kAStageS * 4;
    constexpr int kChunks = T::kBN / 4, kRowsPer = 64 / kChunks;
#pragma unroll
    for (int x = 0; x < kN; ++x) {
        if (x < p * kN / P || x >= (p + 1) * kN / P) continue;  // p is a compile-time index
        if (x < T::kAInst) {
            const int inst = wave * T::kAInst + x;
            const int row = inst * 8 + (lane >> 3), j = (lane & 7) ^ swz_a(row);
            lds_dma16(abase, uint32_t((row * K + 4 * j) * 4), stage_lds + inst * 1024);
        } else {
            const int inst = wave * T::kBInst + (x - T::kAInst);
            const int row = inst * kRowsPer + lane / kChunks, j = (lane % kChunks) ^ swz_b(row);
            lds_dma16(bbase, uint32_t((row * N + 4 * j) * 4), sb + inst * 1024);
        }
    }
}

// Edge tiles of aligned shapes, and tiles of unaligned shapes: the same stage
// through 16-byte buffer loads into LDS (buffer_load_dwordx4 ... lds) at
// 4-byte-aligned offsets, whose range check returns zero past the end of A
// (rows past M) and of B, so no bounds branch is needed. B runs past N read
// the next row's first columns, which feed only unstored outputs. `ra` and
// `rb` cover A and B. MASK: k at or past `kend` (a partial last stage, or a
// stage past the K range) reads zero, its A runs and B rows aimed at
// kDeadOffset. With K % 4 == 0 an A run lies wholly below kend or wholly at
// or past it; otherwise a run that straddles kend is loaded whole and its k
// past kend zeroed in LDS afterwards (k_loop_dma). Without MASK the stage
// must lie below K.
template <int TM, int TN, bool MASK = false, int PART = -1>
__device__ inline void issue_stage_buf(__amdgpu_buffer_rsrc_t ra, __amdgpu_buffer_rsrc_t rb, int N, int K, int m0,
                                       int n0, int k0, float *stage, int t, int kend = 0) {
    using T = Tile<TM, TN>;
    const int lane = t & 63, wave = __builtin_amdgcn_readfirstlane(t >> 6);
#pragma unroll
    for (int i = 0; i < (PART == 1 ? 0 : T::kAInst); ++i) {
        const int inst = wave * T::kAInst + i;
        const int row = inst * 8 + (lane >> 3), j = (lane & 7) ^ swz_a(row);
        const uint32_t off =
            !MASK || k0 + 4 * j < kend ? (uint32_t(m0 + row) * uint32_t(K) + uint32_t(k0 + 4 * j)) * 4u : kDeadOffset;
        __builtin_amdgcn_raw_ptr_buffer_load_lds(ra, (__attribute__((address_space(3))) void *)(stage + inst * 256), 16,
                                                 int(off), 0, 0, 0);
    }
    constexpr int kChunks = T::kBN / 4, kRowsPer = 64 / kChunks;
    float *bstage = stage + T::kAStageS;
#pragma unroll
    for (int i = 0; i < (PART == 0 ? 0 : T::kBInst); ++i) {
        const int inst = wave * T::kBInst + i;
        const int row = inst * kRowsPer + lane / kChunks, j = (lane % kChunks) ^ swz_b(row);
        const uint32_t off =
            !MASK || k0 + row < kend ? (uint32_t(k0 + row) * uint32_t(N) + uint32_t(n0 + 4 * j)) * 4u : kDeadOffset;
        __builtin_amdgcn_raw_ptr_buffer_load_lds(rb, (__attribute__((address_space(3))) void *)(bstage + inst * 256),
                                                 16, int(off), 0, 0, 0);
    }
}

__device__ inline void tile_coords(int tiles_m, int tiles_n, int &tm, int &tn) {
    grouped_tile(xcd_order(int(blockIdx.x), tiles_m * tiles_n), tiles_m, tiles_n, tm, tn);
}

// Stage loads: A tile BMx32 (8 float4 per row) and B tile 32xBN; `kend` is
// the end of this workgroup's K range (K itself unless K is split). GUARD=false
// is only used for tiles that lie wholly inside A, B and C with a K range that
// is a whole number of stages, so every access is in bounds without a check.
template <int TM, int TN, bool VEC, bool GUARD>
__device__ inline void load_stage(const float *__restrict__ A, const float *__restrict__ B, int M, int N, int K,
                                  int kend, int m0, int n0, int k0, f32x4 (&ra)[Tile<TM, TN>::kALoads],
                                  f32x4 (&rb)[Tile<TM, TN>::kBLoads], int t) {
    using T = Tile<TM, TN>;
#pragma unroll
    for (int i = 0; i < T::kALoads; ++i) {
        const int f = t + i * kThreads;
        const int row = f >> 3, col = (f & 7) << 2;
        const int gr = m0 + row, gc = k0 + col;
        if (VEC && !GUARD) {
            ra[i] = *reinterpret_cast<const f32x4 *>(A + (size_t)gr * K + gc);
        } else if (VEC) {
            ra[i] = (gr < M && gc < kend) ? *reinterpret_cast<const f32x4 *>(A + (size_t)gr * K + gc)
                                          : f32x4{0.f, 0.f, 0.f, 0.f};
        } else {
            f32x4 v;
#pragma unroll
            for (int e = 0; e < 4; ++e) v[e] = (gr < M && gc + e < kend) ? A[(size_t)gr * K + gc + e] : 0.f;
            ra[i] = v;
        }
    }
    constexpr int kRowF4 = T::kBN / 4;  // float4 per B row
#pragma unroll
    for (int i = 0; i < T::kBLoads; ++i) {
        const int f = t + i * kThreads;
        const int row = f / kRowF4, col = (f % kRowF4) * 4;
        const int gr = k0 + row, gc = n0 + col;
        if (VEC && !GUARD) {
            rb[i] = *reinterpret_cast<const f32x4 *>(B + (size_t)gr * N + gc);
        } else if (VEC) {
            rb[i] = (gr < kend && gc < N) ? *reinterpret_cast<const f32x4 *>(B + (size_t)gr * N + gc)
                                          : f32x4{0.f, 0.f, 0.f, 0.f};
        } else {
            f32x4 v;
#pragma unroll
            for (int e = 0; e < 4; ++e) v[e] = (gr < kend && gc + e < N) ? B[(size_t)gr * N + gc + e] : 0.f;
            rb[i] = v;
        }
    }
}

template <int TM, int TN>
__device__ inline void store_stage(float *stage, const f32x4 (&ra)[Tile<TM, TN>::kALoads],
                                   const f32x4 (&rb)[Tile<TM, TN>::kBLoads], int t) {
    using T = Tile<TM, TN>;
    float *as = stage, *bs = stage + T::kAStage;
#pragma unroll
    for (int i = 0; i < T::kALoads; ++i) {
        const int f = t + i * kThreads;
        *reinterpret_cast<f32x4 *>(as + (f >> 3) * kLDA + ((f & 7) << 2)) = ra[i];
    }
    constexpr int kRowF4 = T::kBN / 4;
#pragma unroll
    for (int i = 0; i < T::kBLoads; ++i) {
        const int f = t + i * kThreads;
        *reinterpret_cast<f32x4 *>(bs + (f / kRowF4) * T::kLDB + (f % kRowF4) * 4) = rb[i];
    }
}

// One K stage into fresh accumulators; the caller adds the stage sums into the
// running totals with VALU adds, so the long K recurrence is 1 add per 32 k
// instead of 16 chained matrix-core accumulations per 32 k.
template <int TM, int TN, bool ZERO = true>
__device__ inline void mma_stage(const float *stage, int wm, int wn, int lane, f32x16 (&acc)[TM][TN]) {
    using T = Tile<TM, TN>;
    const int h = lane >> 5, c = lane & 31;
    const float *ap = stage + (wm * 32 * TM + c) * kLDA + 16 * h;
    const float *bp = stage + T::kAStage + (16 * h) * T::kLDB;
    if (ZERO) {
#pragma unroll
        for (int i = 0; i < TM; ++i)
#pragma unroll
            for (int j = 0; j < TN; ++j)
#pragma unroll
                for (int v = 0; v < 16; ++v) acc[i][j][v] = 0.f;
    }
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        f32x4 a[TM];
#pragma unroll
        for (int i = 0; i < TM; ++i) a[i] = *reinterpret_cast<const f32x4 *>(ap + i * 32 * kLDA + 4 * q);
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const int s = 4 * q + e;
            float b[TN];
#pragma unroll
            for (int j = 0; j < TN; ++j) b[j] = bp[s * T::kLDB + tile_col<TN>(wn, j, c)];
#pragma unroll
            for (int i = 0; i < TM; ++i)
#pragma unroll
                for (int j = 0; j < TN; ++j)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(a[i][e], b[j], acc[i][j], 0, 0, 0);
        }
    }
}

// mma_stage over the swizzled layout: A stage at `as`, B stage at `bs`.
// ZERO: start the sums at zero; otherwise add onto `acc`.
struct NoHook {
    __device__ void operator()(int) const {}
};
// `hook(q)` runs after quarter q's operand reads are issued (the LDS-direct
// loop issues a share of the next stage's loads there): before the quarter's
// MFMAs, or with LATE after its first two of four. The tile loops take LATE
// for 64x64 wave tiles (us, the same bits: 1024^3 19.53 -> 19.47, 2048x1024x512
// 20.45 -> 20.11, 1024x832x512 11.38 -> 11.33, 1000x776x548 14.74 -> 14.66,
// 768^3 15.40 -> 15.33, 1000x777x545 14.72 -> 14.77; after the first one of
// four 1024^3 took 19.73). The loop written for LATE also changed the larger
// tiles' schedule with the hook at the top (128x128 +0.6%, the fused gate/up
// kernel +0.8%), so they keep this one; LATE itself moved 128x64 tiles by
// 0.15% at most either way (five shapes).
template <int TM, int TN, bool ZERO = true, class Hook = NoHook, bool LATE = false>
__device__ inline void mma_stage_swz(const float *as, const float *bs, int wm, int wn, int lane,
                                     f32x16 (&acc)[TM][TN], Hook hook = {}) {
    using T = Tile<TM, TN>;
    const int h = lane >> 5, c = lane & 31;
    if (ZERO) {
#pragma unroll
        for (int i = 0; i < TM; ++i)
#pragma unroll
            for (int j = 0; j < TN; ++j)
#pragma unroll
                for (int v = 0; v < 16; ++v) acc[i][j][v] = 0.f;
    }
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        f32x4 a[TM];
#pragma unroll
        for (int i = 0; i < TM; ++i) {
            const int row = wm * 32 * TM + i * 32 + c, chunk = 4 * h + q;
            a[i] = *reinterpret_cast<const f32x4 *>(as + row * kBK + ((chunk ^ swz_a(row)) << 2));
        }
        float b[4][TN];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const int krow = 16 * h + 4 * q + e;
#pragma unroll
            for (int j = 0; j < TN; ++j) {
                const int col = tile_col<TN>(wn, j, c);
                b[e][j] = bs[krow * T::kBN + (((col >> 2) ^ swz_b(krow)) << 2) + (col & 3)];
            }
        }
        if constexpr (LATE) {
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                if (e == 2) hook(q);
#pragma unroll
                for (int i = 0; i < TM; ++i)
#pragma unroll
                    for (int j = 0; j < TN; ++j)
                        acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(a[i][e], b[e][j], acc[i][j], 0, 0, 0);
            }
        } else {
            hook(q);
#pragma unroll
            for (int e = 0; e < 4; ++e)
#pragma unroll
                for (int i = 0; i < TM; ++i)
#pragma unroll
                    for (int j = 0; j < TN; ++j)
                        acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(a[i][e], b[e][j], acc[i][j], 0, 0, 0);
        }
    }
}

// The K loop for interior tiles: LDS-direct loads of stage kt+1 run while the
// matrix cores consume stage kt; each wave drains its own loads, then one
// barrier publishes the stage and retires the buffer the next loads overwrite.
// The matrix cores sum kFoldStages stages into `part` before each fold into
// acc (four against two: 4096^3 139.0 -> 141.1 TFLOP/s, 2048^3 131.8 ->
// 133.9; the worst 4096^3 output then used 20% of the 1e-4 tolerance against
// 17.5%; eight timed the same as four here). The fold sits only at a run's
// last stage, and a last, shorter run folds after the loop: a fold guarded by
// "or this is the last stage" was if-converted into an add and a select after
// every stage, whose reads of `part` waited for each stage's last MFMA (the
// MFMA pipeline drained every stage, not every fourth): 1024x832x512 11.91 ->
// 11.42 us, 2000x3000x1024 116.8 -> 108.4, 3000x3001x3008 505.7 -> 462.1,
// the same bits. `nk` whole stages from kbegin; `t` is the thread's index in
// its 256-thread group (every group of a workgroup runs the same number of
// stages, so the barriers match).
// BUF: BQB < 0 issues the next stage whole at the top of the current one;
// else its A loads at the top (BQA < 0) or after quarter BQA's operand
// reads, and its B loads after quarter BQB's.
template <int TM, int TN, bool BUF = false, int QA = -1, int QB = 2, bool MASKED = false, int BQA = -1, int BQB = -1>
__device__ inline void k_loop_dma(const float *__restrict__ A, const float *__restrict__ B, float *smem, int N,
                                  int K, int kbegin, int nk, int m0, int n0, int wm, int wn, int lane, int t,
                                  f32x16 (&acc)[TM][TN], int M = 0, int kend = 0) {
    using T = Tile<TM, TN>;
    const uint32_t lds0 = lds_address(smem);
    // BUF: edge tiles, through range-checked buffer loads over A and B.
    const __amdgpu_buffer_rsrc_t ra = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<float *>(A), 0, BUF ? int(uint32_t(M) * uint32_t(K) * 4u) : 0, int(kBufferWord3));
    const __amdgpu_buffer_rsrc_t rb = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<float *>(B), 0, BUF ? int(uint32_t(K) * uint32_t(N) * 4u) : 0, int(kBufferWord3));
    auto issue = [&](int k0, int buf) {
        if constexpr (BUF)
            if (!MASKED || k0 + kBK <= kend)  // block-uniform: a whole stage inside the K range
                issue_stage_buf<TM, TN>(ra, rb, N, K, m0, n0, k0, smem + buf * T::kStageS, t);
            else
                issue_stage_buf<TM, TN, MASKED>(ra, rb, N, K, m0, n0, k0, smem + buf * T::kStageS, t, kend);
        else
            issue_stage_dma<TM, TN>(A, B, N, K, m0, n0, k0, lds0 + uint32_t(buf * T::kStageS * 4), t);
    };
    auto issue_buf_part = [&](int k0, int buf, auto part) {
        constexpr int kPart = decltype(part)::value;
        if (!MASKED || k0 + kBK <= kend)
            issue_stage_buf<TM, TN, false, kPart>(ra, rb, N, K, m0, n0, k0, smem + buf * T::kStageS, t);
        else
            issue_stage_buf<TM, TN, MASKED, kPart>(ra, rb, N, K, m0, n0, k0, smem + buf * T::kStageS, t, kend);
    };
    // MASKED with unaligned rows (K % 4 != 0): an A run that straddles kend
    // was loaded whole; once this wave's loads have landed it zeroes the
    // run's k at or past kend in LDS, before the barrier publishes the stage.
    auto fix = [&](int k0, int buf) {
        if constexpr (MASKED) {
            if (K % 4 != 0 && k0 + kBK > kend) {  // block-uniform
                float *stage = smem + buf * T::kStageS;
                const int wave = t >> 6;
#pragma unroll
                for (int i = 0; i < T::kAInst; ++i) {
                    const int inst = wave * T::kAInst + i;
                    const int row = inst * 8 + (lane >> 3), j = (lane & 7) ^ swz_a(row);
                    const int ka = k0 + 4 * j;
#pragma unroll
                    for (int e = 1; e < 4; ++e)
                        if (ka < kend && ka + e >= kend) stage[inst * 256 + lane * 4 + e] = 0.f;
                }
            }
        }
    };
    issue(kbegin, 0);
    drain_vmem();
    fix(kbegin, 0);
    __syncthreads();
    // Partial sums run over kFoldStages stages before each fold into acc.
    f32x16 part[TM][TN];
    for (int kt = 0; kt < nk; kt += kFoldStages) {
#pragma unroll
        for (int uu = 0; uu < kFoldStages; ++uu) {
            const int k = kt + uu, u = uu & 1;
            if (k < nk) {  // block-uniform
                const float *cur = smem + u * T::kStageS;
                const bool more = k + 1 < nk;  // block-uniform
                // Interior tiles: the next stage's A loads go out at the top
                // of this stage (QA < 0) or after quarter QA's operand reads,
                // its B loads after quarter QB's.
                auto spread = [&](int q) {
                    if constexpr (BUF) {
                        if (BQB >= 0 && more && q == BQA)
                            issue_buf_part(kbegin + (k + 1) * kBK, 1 - u, std::integral_constant<int, 0>{});
                        if (BQB >= 0 && more && q == BQB)
                            issue_buf_part(kbegin + (k + 1) * kBK, 1 - u, std::integral_constant<int, 1>{});
                        return;
                    }
                    if (more && q == QA)
                        issue_stage_dma_part<TM, TN, 2>(A, B, N, K, m0, n0, kbegin + (k + 1) * kBK,
                                                        lds0 + uint32_t((1 - u) * T::kStageS * 4), t, 0);
                    if (more && q == QB)
                        issue_stage_dma_part<TM, TN, 2>(A, B, N, K, m0, n0, kbegin + (k + 1) * kBK,
                                                        lds0 + uint32_t((1 - u) * T::kStageS * 4), t, 1);
                };
                if (BUF && BQB < 0 && more) issue(kbegin + (k + 1) * kBK, 1 - u);
                if (BUF && BQB >= 0 && BQA < 0 && more)
                    issue_buf_part(kbegin + (k + 1) * kBK, 1 - u, std::integral_constant<int, 0>{});
                if (!BUF && QA < 0 && more)
                    issue_stage_dma_part<TM, TN, 2>(A, B, N, K, m0, n0, kbegin + (k + 1) * kBK,
                                                    lds0 + uint32_t((1 - u) * T::kStageS * 4), t, 0);
                // Raised wave priority while this wave has matrix work, so the
                // SIMD's arbiter favours it over the co-resident workgroup's
                // loads and folds (measured +1-2% at 4096^3).
                __builtin_amdgcn_s_setprio(1);
                if constexpr (BUF && BQB < 0) {
                    if (uu == 0)
                        mma_stage_swz<TM, TN, true>(cur, cur + T::kAStageS, wm, wn, lane, part);
                    else
                        mma_stage_swz<TM, TN, false>(cur, cur + T::kAStageS, wm, wn, lane, part);
                } else {
                    constexpr bool kLate = TM * TN == 1;
                    if (uu == 0)
                        mma_stage_swz<TM, TN, true, decltype(spread), kLate>(cur, cur + T::kAStageS, wm, wn, lane, part, spread);
                    else
                        mma_stage_swz<TM, TN, false, decltype(spread), kLate>(cur, cur + T::kAStageS, wm, wn, lane, part, spread);
                }
                if (uu == kFoldStages - 1) {
#pragma unroll
                    for (int i = 0; i < TM; ++i)
#pragma unroll
                        for (int j = 0; j < TN; ++j) acc[i][j] += part[i][j];
                }
                __builtin_amdgcn_s_setprio(0);
                drain_vmem();
                if (more) fix(kbegin + (k + 1) * kBK, 1 - u);
                __syncthreads();
            }
        }
    }
    if (nk % kFoldStages != 0) {  // the last, shorter run
#pragma unroll
        for (int i = 0; i < TM; ++i)
#pragma unroll
            for (int j = 0; j < TN; ++j) acc[i][j] += part[i][j];
    }
}

// The K loop of one workgroup: prefetch stage kt+1 into registers while the
// matrix cores consume stage kt from LDS, then publish it with one barrier.
// `nk` stages from kbegin; loads at or past kend read zero.
template <int TM, int TN, bool VEC, bool GUARD>
__device__ inline void k_loop(const float *__restrict__ A, const float *__restrict__ B, float *smem, int M, int N,
                              int K, int kbegin, int kend, int nk, int m0, int n0, int wm, int wn, int lane, int t,
                              f32x16 (&acc)[TM][TN]) {
    using T = Tile<TM, TN>;
    f32x4 ra[T::kALoads], rb[T::kBLoads];
    load_stage<TM, TN, VEC, GUARD>(A, B, M, N, K, kend, m0, n0, kbegin, ra, rb, t);
    store_stage<TM, TN>(smem, ra, rb, t);
    __syncthreads();
    // Partial sums run over two stages (64 k) before each fold into acc,
    // except at 128x128, whose register-staged loop would then spill.
    constexpr bool kPairs = TM * TN <= 2;
    f32x16 part[TM][TN];
    for (int kt = 0; kt < nk; kt += 2) {
#pragma unroll
        for (int u = 0; u < 2; ++u) {
            const int k = kt + u;
            if (k < nk) {  // block-uniform
                const float *cur = smem + u * T::kStage;
                float *nxt = smem + (1 - u) * T::kStage;
                const bool more = k + 1 < nk;
                if (more)
                    load_stage<TM, TN, VEC, GUARD>(A, B, M, N, K, kend, m0, n0, kbegin + (k + 1) * kBK, ra, rb, t);
                if (u == 0 || !kPairs)
                    mma_stage<TM, TN, true>(cur, wm, wn, lane, part);
                else
                    mma_stage<TM, TN, false>(cur, wm, wn, lane, part);
                if (u == 1 || !kPairs) {
#pragma unroll
                    for (int i = 0; i < TM; ++i)
#pragma unroll
                        for (int j = 0; j < TN; ++j) acc[i][j] += part[i][j];
                }
                if (more) store_stage<TM, TN>(nxt, ra, rb, t);
                __syncthreads();
            }
        }
    }
    if (kPairs && nk % 2 != 0) {  // the last pair held one stage
#pragma unroll
        for (int i = 0; i < TM; ++i)
#pragma unroll
            for (int j = 0; j < TN; ++j) acc[i][j] += part[i][j];
    }
}

// ---- Unaligned shapes: two stages of register prefetch ----------------------
// Rows that are not 16-byte aligned (K or N not a multiple of 4) load one
// float at a time. With one stage in flight those loads bound the K loop
// (~2.4 us per stage at 1000x777x513 against 0.43 us of matrix work), so the
// unaligned loop keeps two stages in registers. The waits stay exact only if
// the loads are branch-free: indices are clamped into A and B and every load
// is issued; the k >= kend mask is applied when the stage is written to LDS,
// one iteration after its loads. Clamped rows of A (columns of B) reach only
// rows (columns) of the tile that are never stored, so they are not masked.
template <int TM, int TN>
struct Regs {
    // One stage: a[j] = A[m0 + (t + 256j) / 32][k0 + (t + 256j) % 32] and
    // b[j] = B[k0 + (t + 256j) / BN][n0 + (t + 256j) % BN]: consecutive lanes
    // read consecutive floats of a row, so each load instruction covers two
    // 128-byte rows of A or one 256-byte (BN = 64) row of B.
    float a[Tile<TM, TN>::kBM * kBK / kThreads], b[kBK * Tile<TM, TN>::kBN / kThreads];
};

template <int TM, int TN>
__device__ inline void load_stage_clamped(const float *__restrict__ A, const float *__restrict__ B, int M, int N,
                                          int K, int m0, int n0, int k0, Regs<TM, TN> &r, int t) {
    using T = Tile<TM, TN>;
#pragma unroll
    for (int j = 0; j < T::kBM * kBK / kThreads; ++j) {
        const int f = t + j * kThreads;
        r.a[j] = A[size_t(min(m0 + f / kBK, M - 1)) * K + min(k0 + f % kBK, K - 1)];
    }
#pragma unroll
    for (int j = 0; j < kBK * T::kBN / kThreads; ++j) {
        const int f = t + j * kThreads;
        r.b[j] = B[size_t(min(k0 + f / T::kBN, K - 1)) * N + min(n0 + f % T::kBN, N - 1)];
    }
}

// Writes a stage loaded by load_stage_clamped, zeroing k >= kend in A and B.
template <int TM, int TN>
__device__ inline void store_stage_masked(float *stage, const Regs<TM, TN> &r, int k0, int kend, int t) {
    using T = Tile<TM, TN>;
    float *as = stage, *bs = stage + T::kAStage;
#pragma unroll
    for (int j = 0; j < T::kBM * kBK / kThreads; ++j) {
        const int f = t + j * kThreads;
        as[(f / kBK) * kLDA + f % kBK] = k0 + f % kBK < kend ? r.a[j] : 0.f;
    }
#pragma unroll
    for (int j = 0; j < kBK * T::kBN / kThreads; ++j) {
        const int f = t + j * kThreads;
        bs[(f / T::kBN) * T::kLDB + f % T::kBN] = k0 + f / T::kBN < kend ? r.b[j] : 0.f;
    }
}

// Writes a whole stage (k0 + 32 <= kend): no masks.
template <int TM, int TN>
__device__ inline void store_stage_plain(float *stage, const Regs<TM, TN> &r, int t) {
    using T = Tile<TM, TN>;
    float *as = stage, *bs = stage + T::kAStage;
#pragma unroll
    for (int j = 0; j < T::kBM * kBK / kThreads; ++j) {
        const int f = t + j * kThreads;
        as[(f / kBK) * kLDA + f % kBK] = r.a[j];
    }
#pragma unroll
    for (int j = 0; j < kBK * T::kBN / kThreads; ++j) {
        const int f = t + j * kThreads;
        bs[(f / T::kBN) * T::kLDB + f % T::kBN] = r.b[j];
    }
}

// Buffer loads for unaligned operands below 2 GiB. Each lane loads the same
// 16-byte runs as the aligned register path (store_stage's layout: four
// consecutive k of an A row, four consecutive columns of a B row), but at
// 4-byte-aligned offsets, which buffer loads take. Each lane keeps one 32-bit
// byte offset per run of the stage at kbegin (rows of A past M clamped once),
// and a stage is that offset plus a uniform step. The buffer's range check
// returns zero for any part of a run past the operand's end, so no load is
// clamped along K or N: a run that crosses the end of a B row reads the next
// row's first floats into columns past N, which no output keeps, and k >=
// kend is zeroed when a group's partial last stage is written to LDS.
template <int TM, int TN>
struct BufOffsets {
    uint32_t a[Tile<TM, TN>::kALoads], b[Tile<TM, TN>::kBLoads];
};
template <int TM, int TN>
struct Regs4 {
    f32x4 a[Tile<TM, TN>::kALoads], b[Tile<TM, TN>::kBLoads];
};

template <int TM, int TN>
__device__ inline void buffer_offsets(int M, int N, int K, int m0, int n0, int kbegin, int t,
                                      BufOffsets<TM, TN> &o) {
    using T = Tile<TM, TN>;
    constexpr int kRowF4 = T::kBN / 4;
#pragma unroll
    for (int i = 0; i < T::kALoads; ++i) {
        const int f = t + i * kThreads;
        o.a[i] = (uint32_t(min(m0 + (f >> 3), M - 1)) * uint32_t(K) + uint32_t(kbegin + ((f & 7) << 2))) * 4u;
    }
#pragma unroll
    for (int i = 0; i < T::kBLoads; ++i) {
        const int f = t + i * kThreads;
        o.b[i] = (uint32_t(kbegin + f / kRowF4) * uint32_t(N) + uint32_t(n0 + (f % kRowF4) * 4)) * 4u;
    }
}

// Stage s of the range (k0 = kbegin + 32 s): A advances 128 bytes per stage,
// B 32 rows.
template <int TM, int TN>
__device__ inline void load_stage_buffer(__amdgpu_buffer_rsrc_t ra, __amdgpu_buffer_rsrc_t rb,
                                         const BufOffsets<TM, TN> &o, uint32_t astep, uint32_t bstep,
                                         Regs4<TM, TN> &r) {
    using T = Tile<TM, TN>;
#pragma unroll
    for (int i = 0; i < T::kALoads; ++i) {
        const auto v = __builtin_amdgcn_raw_buffer_load_b128(ra, int(o.a[i] + astep), 0, 0);
        r.a[i] = f32x4{__uint_as_float(v[0]), __uint_as_float(v[1]), __uint_as_float(v[2]), __uint_as_float(v[3])};
    }
#pragma unroll
    for (int i = 0; i < T::kBLoads; ++i) {
        const auto v = __builtin_amdgcn_raw_buffer_load_b128(rb, int(o.b[i] + bstep), 0, 0);
        r.b[i] = f32x4{__uint_as_float(v[0]), __uint_as_float(v[1]), __uint_as_float(v[2]), __uint_as_float(v[3])};
    }
}

// store_stage with k >= kend zeroed (a group's partial last stage).
template <int TM, int TN>
__device__ inline void store_stage4_masked(float *stage, const Regs4<TM, TN> &r, int k0, int kend, int t) {
    using T = Tile<TM, TN>;
    float *as = stage, *bs = stage + T::kAStage;
#pragma unroll
    for (int i = 0; i < T::kALoads; ++i) {
        const int f = t + i * kThreads, kk = k0 + ((f & 7) << 2);
        f32x4 v = r.a[i];
#pragma unroll
        for (int e = 0; e < 4; ++e) v[e] = kk + e < kend ? v[e] : 0.f;
        *reinterpret_cast<f32x4 *>(as + (f >> 3) * kLDA + ((f & 7) << 2)) = v;
    }
    constexpr int kRowF4 = T::kBN / 4;
#pragma unroll
    for (int i = 0; i < T::kBLoads; ++i) {
        const int f = t + i * kThreads;
        const f32x4 zero = {0.f, 0.f, 0.f, 0.f};
        *reinterpret_cast<f32x4 *>(bs + (f / kRowF4) * T::kLDB + (f % kRowF4) * 4) =
            k0 + f / kRowF4 < kend ? r.b[i] : zero;
    }
}

// A barrier that orders LDS only: this wave's LDS reads and writes complete
// before it, global loads stay in flight across it. __syncthreads() carries a
// workgroup release fence, for which the compiler also waits for every
// outstanding global load, which would drain the register prefetch each stage.
// The "memory" clobber keeps the compiler from moving memory accesses across.
__device__ inline void lds_barrier() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }

// An empty asm statement that reads the register stage `r`: a use of the
// loaded values on the loop's exit path. Without one, the compiler moves the
// loads of the first stage of the unrolled pair into the second stage's
// branch (their only user when the pair is cut short), past the MFMAs they
// should overlap, so the EARLY store right after waits for their full
// latency.
template <class R>
__device__ inline void keep_live(const R &r) {
    for (const auto &x : r.a) asm volatile("" ::"v"(x));
    for (const auto &x : r.b) asm volatile("" ::"v"(x));
}

// `nk` stages from kbegin; stage kt+2's loads are issued while stage kt is
// consumed and stage kt+1 (loaded an iteration earlier) is written to LDS.
// BUF: buffer loads (operands below 2 GiB); else clamped global loads.
// EARLY: stage k+1 is written to LDS before stage k's MFMAs instead of after
// them. Measured on two-K-group 64x64 tiles (one workgroup per CU): 1000x777x513
// 15.73 -> 15.33 us, 1000x777x100 6.57 -> 6.42, 200x8x999 (split K) 10.2 -> 9.9;
// on one-group tiles (two workgroups per CU) it exposes the loads' latency
// (3000x3000x3001 508 -> 558 us) and on four groups it was mixed.
// PAIRS: partial sums over two stages per fold (else one). Measured with two
// against one: 128x64 tiles 2048x2048x2047 152.5 -> 146.3 us, 2000x1554x1026
// 80.8 -> 77.3; two K groups 1000x777x513 14.08 -> 13.96; one-group and
// four-group 64x64 tiles 1.3% slower (3000x3000x3001, 1000x777x1024).
// PRIO: raised wave priority over each stage's MFMAs and fold, as in the
// LDS-direct loop: one-group 64x64 tiles 3000x3000x3001 548 -> 519 us,
// four groups 1000x777x1024 23.4 -> 22.95; 1-2% slower on two-group and
// 128x64 tiles.
template <int TM, int TN, bool BUF, bool EARLY = false, bool PAIRS = false, bool PRIO = false>
__device__ inline void k_loop_unaligned(const float *__restrict__ A, const float *__restrict__ B, float *smem,
                                        int M, int N, int K, int kbegin, int kend, int nk, int m0, int n0, int wm,
                                        int wn, int lane, int t, f32x16 (&acc)[TM][TN]) {
    using T = Tile<TM, TN>;
    using R = std::conditional_t<BUF, Regs4<TM, TN>, Regs<TM, TN>>;
    R r[2];
    BufOffsets<TM, TN> off;
    __amdgpu_buffer_rsrc_t ra, rb;
    if constexpr (BUF) {
        ra = __builtin_amdgcn_make_buffer_rsrc(const_cast<float *>(A), 0, int(uint32_t(M) * uint32_t(K) * 4u),
                                               int(kBufferWord3));
        rb = __builtin_amdgcn_make_buffer_rsrc(const_cast<float *>(B), 0, int(uint32_t(K) * uint32_t(N) * 4u),
                                               int(kBufferWord3));
        buffer_offsets<TM, TN>(M, N, K, m0, n0, kbegin, t, off);
    }
    const uint32_t bstage = uint32_t(kBK) * uint32_t(N) * 4u;
    auto load = [&](int s, R &dst) {
        if constexpr (BUF)
            load_stage_buffer<TM, TN>(ra, rb, off, uint32_t(s) * (kBK * 4u), uint32_t(s) * bstage, dst);
        else
            load_stage_clamped<TM, TN>(A, B, M, N, K, m0, n0, kbegin + s * kBK, dst, t);
    };
    auto store = [&](float *stage, const R &src, int k0) {
        if constexpr (BUF) {
            if (k0 + kBK <= kend)  // block-uniform
                store_stage<TM, TN>(stage, src.a, src.b, t);
            else
                store_stage4_masked<TM, TN>(stage, src, k0, kend, t);
        } else {
            if (k0 + kBK <= kend)
                store_stage_plain<TM, TN>(stage, src, t);
            else
                store_stage_masked<TM, TN>(stage, src, k0, kend, t);
        }
    };
    load(0, r[0]);
    __builtin_amdgcn_sched_barrier(0);
    load(1, r[1]);
    __builtin_amdgcn_sched_barrier(0);
    store(smem, r[0], kbegin);
    lds_barrier();
    // Unrolled by two so the register stage in use is a compile-time index.
    f32x16 part[TM][TN];
    for (int kt = 0; kt < nk; kt += 2) {
#pragma unroll
        for (int u = 0; u < 2; ++u) {
            const int k = kt + u;
            if (k < nk) {  // block-uniform
                const float *cur = smem + u * T::kStage;
                // EARLY: stage k+1 goes to the other buffer first (every
                // wave's reads of it ended before the last barrier), so the
                // LDS writes run beside this stage's MFMAs rather than between
                // them and the barrier.
                if (EARLY && k + 1 < nk) store(smem + (1 - u) * T::kStage, r[1 - u], kbegin + (k + 1) * kBK);
                // Unconditional, so every path into the loop has the same
                // loads in flight and the waits below stay exact; stages past
                // nk load in-bounds (or range-checked) data that is never stored.
                load(k + 2, r[u]);
                __builtin_amdgcn_sched_barrier(0);
                if (PRIO) __builtin_amdgcn_s_setprio(1);
                if (!PAIRS || u == 0)
                    mma_stage<TM, TN, true>(cur, wm, wn, lane, part);
                else
                    mma_stage<TM, TN, false>(cur, wm, wn, lane, part);
                if (!PAIRS || u == 1) {
#pragma unroll
                    for (int i = 0; i < TM; ++i)
#pragma unroll
                        for (int j = 0; j < TN; ++j) acc[i][j] += part[i][j];
                }
                if (PRIO) __builtin_amdgcn_s_setprio(0);
                if (!EARLY && k + 1 < nk) store(smem + (1 - u) * T::kStage, r[1 - u], kbegin + (k + 1) * kBK);
                lds_barrier();
            }
        }
    }
    if (PAIRS && nk % 2 != 0) {  // the last pair held one stage
#pragma unroll
        for (int i = 0; i < TM; ++i)
#pragma unroll
            for (int j = 0; j < TN; ++j) acc[i][j] += part[i][j];
    }
    keep_live(r[0]);
    keep_live(r[1]);
}

// Two waves per SIMD (LDS allows two workgroups per CU at the largest tile);
// the register budget is capped to match so stage and running accumulators fit.
// gridDim.y > 1 splits K into slices of `kchunk` (a multiple of 32); slice z
// writes C + z*M*N, which is then a workspace the reduction kernel consumes.
// PATH kDmaOnly: every tile of the launch is interior and 16-byte aligned, so
// only the LDS-direct loop is compiled in (fewer registers, tighter code).
// kRegOnly: register-staged loads (64-bit addresses) for every tile, for
// operands too long for the LDS-direct loads' 32-bit offsets.
// kUnalignedBuf: unaligned rows (no 16-byte-aligned loads) through buffer
// loads, for 64x64 and 128x64 tiles over operands below 2 GiB each: into LDS
// directly over whole stages, else staged in registers.
// kBufAll: K ranges with a partial stage (tile_path gives the rule; operands
// whose 32-bit offsets fit): every tile through the buffer-load LDS-direct
// loop, the partial and empty stages masked to zero.
enum Path { kMixed = 0, kDmaOnly = 1, kRegOnly = 2, kUnalignedBuf = 3, kBufAll = 4 };

// LDS-direct loads address each lane's 16 bytes as a 32-bit byte offset from
// a wave-uniform base, computed in int: (row * K + 4 * chunk) * 4 for A rows
// below bm, (row * N + 4 * chunk) * 4 for the 32 B rows of a stage, chunks
// below bn / 4. Those must stay below 2^31; longer rows take 64-bit loads.
constexpr bool dma_offsets_fit(uint32_t bm, uint32_t bn, uint32_t k, uint32_t n) {
    return (uint64_t(bm) * k + kBK) * 4 < (uint64_t(1) << 31) && (uint64_t(kBK) * n + bn) * 4 < (uint64_t(1) << 31);
}

// tail_base >= 0: the launch covers the 256x256 tiles [tail_base, tail_base +
// gridDim.x / P) of the grouped order over a tiles_m x tiles_n grid of 256x256
// tiles, P = (256 / BM) x (256 / BN) workgroups each (the remainder after the
// 256x256 kernel's whole rounds).
// pair: a second, independent product of the same shape in the same launch
// (pair.tiles > 0): positions [tiles, 2*tiles) of the XCD order compute
// pair.c = pair.a * pair.b.
// pair.sum (single products only): the epilogue also stores
// sum = C + residual elementwise (both [M, N]), the FP32 add of the stream
// kernel, so `sum` is bit-identical to an Add launched after the product.
struct PairArgs {
    const float *a;
    const float *b;
    float *c;
    int tiles;
    const float *residual;
    float *sum;
};

// KG > 1: KG groups of four waves share the workgroup's tile. Group g sums
// the g-th run of ceil(stages / KG) stages of the workgroup's K range (every
// group runs that many, so the barriers match; stages past the range read
// zero), each group with its own double-buffered stages in LDS. The groups
// then leave their sums in LDS and each adds up (in group order) and stores a
// 1/KG share of the tile.
// KG = 2 (4) puts two (four) waves on each SIMD where a grid of 64x64 tiles
// gives each CU one workgroup, so one wave's barrier and LDS waits overlap
// the others' matrix work. Not used with pair or tail launches.
template <int TM, int TN, bool VEC, int PATH, int KG = 1, bool KTAIL = false>
__global__ __launch_bounds__(kThreads * KG) __attribute__((amdgpu_waves_per_eu(KG > 2 ? KG : 2, KG > 2 ? KG : 2))) void gemm_f32_mfma(
    const float *__restrict__ A, const float *__restrict__ B, float *__restrict__ C, int M, int N, int K,
    int tiles_m, int tiles_n, int kchunk, int tail_base, PairArgs pair) {
    using T = Tile<TM, TN>;
    __shared__ float smem[KG * 2 * T::kStage];
    static_assert(KG == 1 || (KG * kThreads * TM * TN * 16 <= KG * 2 * T::kStage && 16 % KG == 0),
                  "group sums must fit in the stage buffers");
    int tm, tn;
    if (pair.tiles > 0) {
        int pos = xcd_order(int(blockIdx.x), int(gridDim.x));
        if (pos >= pair.tiles) {
            A = pair.a;
            B = pair.b;
            C = pair.c;
            pos -= pair.tiles;
        }
        grouped_tile(pos, tiles_m, tiles_n, tm, tn);
    } else if (tail_base >= 0) {
        constexpr int kSubM = 256 / T::kBM, kSubN = 256 / T::kBN;
        const int pos = xcd_order(int(blockIdx.x), int(gridDim.x));
        int bm, bn;
        grouped_tile(tail_base + pos / (kSubM * kSubN), tiles_m, tiles_n, bm, bn);
        const int sub = pos % (kSubM * kSubN);
        tm = kSubM * bm + sub / kSubN;
        tn = kSubN * bn + sub % kSubN;
    } else {
        tile_coords(tiles_m, tiles_n, tm, tn);
    }
    const int m0 = tm * T::kBM, n0 = tn * T::kBN;
    const int kfirst = int(blockIdx.y) * kchunk;
    const int klast = min(K, kfirst + kchunk);
    // KTAIL (unaligned K-group tiles): a K range of whole stages that the
    // groups split evenly, plus at most kMaxTail last k. Those k would take a
    // round of their own (a stage of MFMAs on mostly zeros, and its
    // barriers); they add in the epilogue instead, as rank-1 updates of each
    // thread's stored outputs from values loaded before the loop.
    // 1000x777x513 on two groups: 9 rounds per group -> 8. The host picks
    // KTAIL only when the last K slice has such a tail (ktail_fits).
    constexpr bool kTail = KTAIL;
    static_assert(!KTAIL || (KG > 1 && !VEC && TM * TN <= 2), "the tail is for unaligned K-group tiles");
    int ktail = 0;
    if constexpr (kTail) {
        const int whole = (klast - kfirst) / kBK, rest = (klast - kfirst) % kBK;
        if (whole > 0 && whole % KG == 0 && rest <= kMaxTail) ktail = rest;
    }
    const int kmain = klast - ktail;
    const int group = KG > 1 ? __builtin_amdgcn_readfirstlane(int(threadIdx.x) / kThreads) : 0;
    const int t = int(threadIdx.x) % kThreads;
    const int nk = ((kmain - kfirst + kBK - 1) / kBK + KG - 1) / KG;  // stages per group
    const int kbegin = kfirst + group * nk * kBK;
    const int kend = min(kmain, kbegin + nk * kBK);
    float *gsmem = smem + group * 2 * T::kStage;
    float *__restrict__ out = C + size_t(blockIdx.y) * size_t(M) * size_t(N);
    const int lane = t & 63, wave = t >> 6;
    const int wm = wave >> 1, wn = wave & 1;

    f32x16 acc[TM][TN];
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j)
#pragma unroll
            for (int v = 0; v < 16; ++v) acc[i][j][v] = 0.f;

    // The tail's A and B values for the outputs this thread stores (entries
    // [group * 16 / KG, (group + 1) * 16 / KG) of each block, see the K-group
    // epilogue), at indices clamped into A and B, issued ahead of the loop's
    // loads and unconditionally, so every path into the loop has the same
    // loads in flight.
    constexpr int kShareT = kTail ? 16 / KG : 1;
    float ta[kTail ? TM : 1][kShareT][kMaxTail], tb[kTail ? TN : 1][kMaxTail];
    if constexpr (kTail) {
        const int h = lane >> 5, c = lane & 31;
#pragma unroll
        for (int e = 0; e < kMaxTail; ++e) {
            const int kk = min(kmain + e, K - 1);
#pragma unroll
            for (int i = 0; i < TM; ++i)
#pragma unroll
                for (int s = 0; s < kShareT; ++s) {
                    const int v = group * kShareT + s;
                    const int row = min(m0 + wm * 32 * TM + i * 32 + 8 * (v >> 2) + 4 * h + (v & 3), M - 1);
                    ta[i][s][e] = A[size_t(row) * K + kk];
                }
#pragma unroll
            for (int j = 0; j < TN; ++j) tb[j][e] = B[size_t(kk) * N + min(n0 + tile_col<TN>(wn, j, c), N - 1)];
        }
    }

    // Interior tiles with 16-byte rows stream through LDS-direct loads; edge
    // tiles and unaligned shapes over whole stages take the same loop through
    // buffer loads; K ranges that are not KG x nk whole stages take the
    // masked form of that loop (PATH kBufAll, chosen by the host) or the
    // guarded, register-staged path.
    const bool whole = kmain - kfirst == KG * nk * kBK;
    const bool interior = m0 + T::kBM <= M && n0 + T::kBN <= N && whole;
    // Where the interior loop issues the next stage's two load parts (QA,
    // QB) was measured per tile and group count (A at the top, B after
    // quarter 2 before): two and four groups after quarters 1 and 2 (1024^3
    // 19.79 -> 19.49 us, 1024x1024x2048 37.0 -> 34.9, 1024x1024x4096 69.7 ->
    // 65.9, 768x768x1024 19.78 -> 19.26, 1024x832x512 11.47 -> 11.39); one
    // group of 64x64 tiles after quarters 0 and 1 (1536^3 83.2 -> 78.1,
    // 1536x2048x1024 65.2 -> 57.2, 3000x3000x3072 490 -> 450; grids of
    // exactly two tiles per CU 0.6-0.9% slower); 128x64 tiles after quarters
    // 1 and 2 as well (3072x2048x1024 128.9 -> 100.2, 2304^3 261.7 -> 216.3,
    // 1024x6144x512 67.5 -> 53.3, others within 0.5%); 128x128 tiles keep A
    // at the top and B after quarter 2 (each alternative tried was 0.2-0.4%
    // slower). The same MFMAs in the same order: the bits do not change.
    constexpr bool kOne64 = KG == 1 && TM * TN == 1, k128x64 = KG == 1 && TM * TN == 2;
    constexpr int kQA = KG > 1 || k128x64 ? 1 : (kOne64 ? 0 : -1);
    constexpr int kQB = KG > 1 || k128x64 ? 2 : (kOne64 ? 1 : 2);
    // The buffer-load loop (edge tiles, unaligned rows, partial stages)
    // issues the next stage whole at the top of the current one, except with
    // two K groups and for 128x128 tiles, where A at the top and B after
    // quarter 2 measured faster (1000x832x512 12.38 -> 12.26 us, 2500^3
    // 322.5 -> 314.7); elsewhere that split was 0.5-6% slower. With the 64x64
    // tiles' loads after half of each quarter's MFMAs, the four-group 64x64
    // tiles still lose with B after quarter 1, 2 or 3 (1000x777x513 12.89 ->
    // 12.93-13.22 us, 1000x777x1027 24.51 -> 25.00-25.87).
    constexpr int kBufQB = KG == 2 || TM * TN == 4 ? 2 : -1;
    if (PATH == kBufAll)
        k_loop_dma<TM, TN, true, -1, 2, true, -1, kBufQB>(A, B, gsmem, N, K, kbegin, nk, m0, n0, wm, wn, lane, t, acc, M, kend);
    else if (PATH == kDmaOnly || (PATH == kMixed && VEC && interior))
        k_loop_dma<TM, TN, false, kQA, kQB>(A, B, gsmem, N, K, kbegin, nk, m0, n0, wm, wn, lane, t, acc);
    // Edge tiles of aligned shapes, and every tile of an unaligned shape, with
    // whole stages: the same loop through range-checked buffer loads
    // (operands whose 32-bit offsets, with a tile of rows past M, stay below
    // 2 GiB). The 16-byte runs of unaligned rows start at 4-byte-aligned
    // offsets, which buffer loads into LDS take as they are; whole stages
    // keep every A run inside its row, and a B run past N reads the next
    // row's first columns (zero past the end of B), which feed only
    // outputs that are never stored. Against the register-staged loop
    // (us): 1000x777x513 13.78 -> 13.59, 1000x777x512 13.28 -> 12.86,
    // 1000x777x1025 23.22 -> 22.20, 2048x2047x2048 144.1 -> 135.5,
    // 3000x3001x3008 533.8 -> 506.4.
    else if (((PATH == kMixed && VEC) || PATH == kUnalignedBuf) && whole &&
             (uint64_t(M) + T::kBM) * uint64_t(K) * 4u < (uint64_t(1) << 31) &&
             (uint64_t(K) + 1) * uint64_t(N) * 4u + T::kBN * 4u < (uint64_t(1) << 31))
        k_loop_dma<TM, TN, true, -1, 2, false, -1, kBufQB>(A, B, gsmem, N, K, kbegin, nk, m0, n0, wm, wn, lane, t, acc, M);
    else if (!VEC && TM * TN <= 2)  // the 128x128 tile would spill with two register stages
        k_loop_unaligned<TM, TN, PATH == kUnalignedBuf, KG == 2, TM * TN == 2 || KG == 2, TM * TN == 1 && KG != 2>(
            A, B, gsmem, M, N, K, kbegin, kend, nk, m0, n0, wm, wn, lane, t, acc);
    else
        k_loop<TM, TN, VEC, true>(A, B, gsmem, M, N, K, kbegin, kend, nk, m0, n0, wm, wn, lane, t, acc);

    const int h = lane >> 5, c = lane & 31;
    if constexpr (KG > 1) {
        // Both loops end on a barrier, so the stage buffers are free: the
        // groups' sums meet there, and group g then adds and stores entries
        // [g * 16 / KG, (g + 1) * 16 / KG) of each block, the groups' sums in
        // group order.
#pragma unroll
        for (int i = 0; i < TM; ++i)
#pragma unroll
            for (int j = 0; j < TN; ++j)
#pragma unroll
                for (int v = 0; v < 16; ++v) smem[(((group * TM + i) * TN + j) * 16 + v) * kThreads + t] = acc[i][j][v];
        __syncthreads();
        constexpr int kShare = 16 / KG;
#pragma unroll
        for (int i = 0; i < TM; ++i) {
#pragma unroll
            for (int j = 0; j < TN; ++j) {
                const int col = n0 + tile_col<TN>(wn, j, c);
#pragma unroll
                for (int s = 0; s < kShare; ++s) {
                    const int v = group * kShare + s;
                    float x = smem[((i * TN + j) * 16 + v) * kThreads + t];
#pragma unroll
                    for (int w = 1; w < KG; ++w) x += smem[(((w * TM + i) * TN + j) * 16 + v) * kThreads + t];
                    if constexpr (kTail) {
#pragma unroll
                        for (int e = 0; e < kMaxTail; ++e)
                            if (e < ktail) x = fmaf(ta[i][s][e], tb[j][e], x);
                    }
                    const int row = m0 + wm * 32 * TM + i * 32 + 8 * (v >> 2) + 4 * h + (v & 3);
                    if (PATH == kDmaOnly || (row < M && col < N)) {
                        const size_t at = size_t(row) * N + col;
                        out[at] = x;
                        if (pair.sum) pair.sum[at] = x + pair.residual[at];
                    }
                }
            }
        }
        return;
    }
    // The two blocks hold adjacent columns (tile_col): one 8-byte store per
    // pair where C (and the residual and sum) start 8-byte aligned; with
    // N % 4 == 0 every pair then is. Otherwise the single stores below.
    if constexpr (TN == 2 && VEC) {
        const bool pairs = ((reinterpret_cast<uintptr_t>(out) | reinterpret_cast<uintptr_t>(pair.residual) |
                             reinterpret_cast<uintptr_t>(pair.sum)) & 7u) == 0;
        if (pairs) {  // block-uniform
            const int col = n0 + tile_col<TN>(wn, 0, c);
#pragma unroll
            for (int i = 0; i < TM; ++i) {
#pragma unroll
                for (int v = 0; v < 16; ++v) {
                    const int row = m0 + wm * 32 * TM + i * 32 + 8 * (v >> 2) + 4 * h + (v & 3);
                    const size_t at = size_t(row) * N + col;
                    if (PATH == kDmaOnly || (row < M && col + 1 < N)) {
                        *reinterpret_cast<float2 *>(out + at) = make_float2(acc[i][0][v], acc[i][1][v]);
                        if (pair.sum) {
                            const float2 r = *reinterpret_cast<const float2 *>(pair.residual + at);
                            *reinterpret_cast<float2 *>(pair.sum + at) =
                                make_float2(acc[i][0][v] + r.x, acc[i][1][v] + r.y);
                        }
                    } else if (row < M && col < N) {
                        out[at] = acc[i][0][v];
                        if (pair.sum) pair.sum[at] = acc[i][0][v] + pair.residual[at];
                    }
                }
            }
            return;
        }
    }
#pragma unroll
    for (int i = 0; i < TM; ++i) {
#pragma unroll
        for (int j = 0; j < TN; ++j) {
            const int col = n0 + tile_col<TN>(wn, j, c);
#pragma unroll
            for (int v = 0; v < 16; ++v) {
                const int row = m0 + wm * 32 * TM + i * 32 + 8 * (v >> 2) + 4 * h + (v & 3);
                if (PATH == kDmaOnly || (row < M && col < N)) {
                    const size_t at = size_t(row) * N + col;
                    out[at] = acc[i][j][v];
                    if (pair.sum) pair.sum[at] = acc[i][j][v] + pair.residual[at];
                }
            }
        }
    }
}

// ---- Gate/up pair with a fused SwiGLU ---------------------------------------
// G = A Bg, U = A Bu and Act = swiglu(G, U) for the residual MLP's gate and up
// projections (src/runtime/workloads.rs:422-465), in one launch over 128x64
// tiles: waves 0-3 compute the gate tile and waves 4-7 the up tile of the same
// (row, column) block, from one LDS copy of the A stage and one B stage each.
// Each output takes exactly the MFMA steps and folds of the 128x64 kernel, and
// SwiGLU is the stream kernel's function, so all three outputs are
// bit-identical to the two GEMM launches followed by the SwiGLU launch. The
// up waves store U and pass it to the gate waves through LDS; the gate waves
// store G and Act. Interior tiles only: M % 128 == 0, N % 64 == 0,
// K % 32 == 0, 16-byte aligned rows.
//
// A grid whose last round of 128x64 tiles would leave CUs idle can hand that
// round's tiles, as whole tile columns at the right edge, to 64x64 tiles
// (twice as many, half the work each, so every CU takes one): the 128x64
// tiles cover columns [0, 64 body_tn), the 64x64 tiles the rest, launched
// after them. A 64x64 tile runs the 64x64 kernel's schedule, which per output
// is the 128x64 one (the same MFMA chain over k, the same fold every two
// stages), so the bits do not depend on which tile an output falls in.
namespace dual {
using T = Tile<2, 1>;
constexpr int kWaves = 8, kThreads = 64 * kWaves;
template <int TM>
struct Shape {
    using Tl = Tile<TM, 1>;
    static constexpr int kStage = Tl::kAStageS + 2 * Tl::kBStageS;  // A, then B for G, then B for U
    static constexpr int kAInst = Tl::kAStageS * 4 / 1024 / kWaves, kBInst = Tl::kBStageS * 4 / 1024 / (kWaves / 2);
    static_assert(kAInst * kWaves * 1024 == Tl::kAStageS * 4 && kBInst * (kWaves / 2) * 1024 == Tl::kBStageS * 4,
                  "stage loads must split evenly over the waves");
};
constexpr int kStage = Shape<2>::kStage;  // the LDS stage of either tile fits this one

// Waves 0-3 load B for G, waves 4-7 B for U; all eight load A. PART 0 issues
// only the A loads, PART 1 only the B loads, -1 both.
template <int TM, int PART = -1>
__device__ inline void issue_stage(const float *__restrict__ A, const float *__restrict__ B, int N, int K, int m0,
                                   int n0, int k0, uint32_t stage_lds, int wave, int lane) {
    using S = Shape<TM>;
    const float *abase = A + size_t(m0) * K + k0;
#pragma unroll
    for (int i = 0; i < (PART == 1 ? 0 : S::kAInst); ++i) {  // eight 128-byte A rows per 1 KiB load
        const int inst = wave * S::kAInst + i;
        const int row = inst * 8 + (lane >> 3), j = (lane & 7) ^ swz_a(row);
        lds_dma16(abase, uint32_t((row * K + 4 * j) * 4), stage_lds + inst * 1024);
    }
    const float *bbase = B + size_t(k0) * N + n0;
    const uint32_t sb = stage_lds + (S::Tl::kAStageS + (wave >> 2) * S::Tl::kBStageS) * 4;
    constexpr int kChunks = S::Tl::kBN / 4, kRowsPer = 64 / kChunks;
#pragma unroll
    for (int i = 0; i < (PART == 0 ? 0 : S::kBInst); ++i) {  // four 256-byte B rows per 1 KiB load
        const int inst = (wave & 3) * S::kBInst + i;
        const int row = inst * kRowsPer + lane / kChunks, j = (lane % kChunks) ^ swz_b(row);
        lds_dma16(bbase, uint32_t((row * N + 4 * j) * 4), sb + inst * 1024);
    }
}

// One (64 TM) x 64 tile at (m0, n0): its gate product in waves 0-3, its up
// product in waves 4-7. FOLD: stages per run before each fold, that of the
// kernel each product would run on alone.
template <int TM, int FOLD>
__device__ inline void tile(const float *__restrict__ A, const float *__restrict__ Bg, const float *__restrict__ Bu,
                            float *__restrict__ G, float *__restrict__ U, float *__restrict__ Act, int N, int K,
                            int m0, int n0, float *smem) {
    using S = Shape<TM>;
    using Tl = typename S::Tl;
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(int(threadIdx.x) >> 6);
    const int group = wave >> 2, wl = wave & 3;  // group 0: G, group 1: U
    const int wm = wl >> 1, wn = wl & 1;
    const float *B = group ? Bu : Bg;
    const uint32_t lds0 = lds_address(smem);
    f32x16 acc[TM][1];
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int v = 0; v < 16; ++v) acc[i][0][v] = 0.f;
    const int nk = K / kBK;
    issue_stage<TM>(A, B, N, K, m0, n0, 0, lds0, wave, lane);
    drain_vmem();
    __syncthreads();
    // The LDS-direct loop's schedule: partial sums over FOLD stages, then a
    // fold.
    f32x16 part[TM][1];
    for (int kt = 0; kt < nk; kt += FOLD) {
#pragma unroll
        for (int uu = 0; uu < FOLD; ++uu) {
            const int k = kt + uu, u = uu & 1;
            if (k < nk) {
                const float *cur = smem + u * S::kStage;
                const bool more = k + 1 < nk;
                const uint32_t nxt = lds0 + uint32_t((1 - u) * S::kStage * 4);
                auto spread = [&](int q) {
                    if (more && q == 2) issue_stage<TM, 1>(A, B, N, K, m0, n0, (k + 1) * kBK, nxt, wave, lane);
                };
                // The next stage's A loads at the top of this stage, its B loads
                // after the third quarter's operand reads (against all of them
                // at the top: MLP block 520.4 -> 515.3 us; A after the second
                // quarter's reads 538.3, after the first 541.7, A and B after
                // the first and second 530.0, B after the fourth 517.7).
                if (more) issue_stage<TM, 0>(A, B, N, K, m0, n0, (k + 1) * kBK, nxt, wave, lane);
                __builtin_amdgcn_s_setprio(1);
                if (uu == 0)
                    mma_stage_swz<TM, 1, true>(cur, cur + Tl::kAStageS + group * Tl::kBStageS, wm, wn, lane, part, spread);
                else
                    mma_stage_swz<TM, 1, false>(cur, cur + Tl::kAStageS + group * Tl::kBStageS, wm, wn, lane, part, spread);
                if (uu == FOLD - 1) {
#pragma unroll
                    for (int i = 0; i < TM; ++i) acc[i][0] += part[i][0];
                }
                __builtin_amdgcn_s_setprio(0);
                drain_vmem();
                __syncthreads();
            }
        }
    }
    if (nk % FOLD != 0) {  // the last, shorter run
#pragma unroll
        for (int i = 0; i < TM; ++i) acc[i][0] += part[i][0];
    }
    // The loop ended on a barrier: the stage buffers are free for U.
    const int h = lane >> 5, c = lane & 31;
    const int col = n0 + wn * 32 + c;
    float *ushare = smem;  // [i][v][256 threads of the U group]
    if (group == 1) {
#pragma unroll
        for (int i = 0; i < TM; ++i)
#pragma unroll
            for (int v = 0; v < 16; ++v) {
                const int row = m0 + wm * 32 * TM + i * 32 + 8 * (v >> 2) + 4 * h + (v & 3);
                U[size_t(row) * N + col] = acc[i][0][v];
                ushare[(i * 16 + v) * 256 + wl * 64 + lane] = acc[i][0][v];
            }
    }
    __syncthreads();
    if (group == 1) return;
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int v = 0; v < 16; ++v) {
            const int row = m0 + wm * 32 * TM + i * 32 + 8 * (v >> 2) + 4 * h + (v & 3);
            const float g = acc[i][0][v], u = ushare[(i * 16 + v) * 256 + wl * 64 + lane];
            G[size_t(row) * N + col] = g;
            Act[size_t(row) * N + col] = swiglu(g, u);
        }
}
}  // namespace dual

// Workgroups [0, tiles_m body_tn) take the 128x64 tiles of columns
// [0, 64 body_tn) in the XCD-grouped order; the rest take the 64x64 tiles of
// the columns right of them, row-major.
template <int FOLD>
__global__ __launch_bounds__(dual::kThreads) void gemm_f32_dual_swiglu(
    const float *__restrict__ A, const float *__restrict__ Bg, const float *__restrict__ Bu, float *__restrict__ G,
    float *__restrict__ U, float *__restrict__ Act, int N, int K, int tiles_m, int tiles_n, int body_tn) {
    __shared__ float smem[2 * dual::kStage];
    const int body = tiles_m * body_tn;
    if (int(blockIdx.x) < body) {  // block-uniform
        const int pos = xcd_order(int(blockIdx.x), body);
        int tm, tn;
        grouped_tile(pos, tiles_m, body_tn, tm, tn);
        dual::tile<2, FOLD>(A, Bg, Bu, G, U, Act, N, K, tm * 128, tn * 64, smem);
    } else {
        const int pos = int(blockIdx.x) - body, edge_n = tiles_n - body_tn;
        dual::tile<1, FOLD>(A, Bg, Bu, G, U, Act, N, K, (pos / edge_n) * 64, (body_tn + pos % edge_n) * 64, smem);
    }
}

// ---- 256x256 tile, eight waves of 128x64 ---------------------------------
// Runs the whole rounds (256 tiles each) of a grid of 256x256 tiles; the
// remainder goes to the 128x128 kernel in tail mode. One 512-thread workgroup
// per CU (two 64 KiB stages), waves 2 (M) x 4 (N), each
// wave 4x2 MFMA blocks. A stage's B operands for both column blocks are read
// once (32 registers), then each row block runs two 16-deep MFMA chains into
// fresh accumulators and folds them into the running sums while the next
// block's chains run, so only two blocks' partial sums are live (a fold every
// stage, where the smaller LDS-direct tiles fold every two). Per stage each wave
// issues 128 MFMAs against 16 ds_read_b128 and 16 ds_read2_b32, against 64
// MFMAs per 8 + 16 for the 64x64 wave tile. Interior tiles only: M and N
// multiples of 256, K a multiple of 32, 16-byte aligned rows.
namespace big {
constexpr int kBM = 256, kBN = 256, kWaves = 8, kThreads = 64 * kWaves;
constexpr int kAStage = kBM * kBK, kBStage = kBK * kBN, kStage = kAStage + kBStage;  // floats
constexpr int kAInst = kAStage * 4 / 1024 / kWaves, kBInst = kBStage * 4 / 1024 / kWaves;
constexpr uint32_t kLdsBytes = 2u * kStage * sizeof(float);
static_assert(kAInst * kWaves * 8 == kBM && kBInst * kWaves == kBK, "stage must split evenly over the waves");

__device__ inline void issue_stage(const float *__restrict__ A, const float *__restrict__ B, int N, int K, int m0,
                                   int n0, int k0, uint32_t stage_lds) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const float *abase = A + size_t(m0) * K + k0;
    const float *bbase = B + size_t(k0) * N + n0;
#pragma unroll
    for (int i = 0; i < kAInst; ++i) {  // eight 128-byte A rows per 1 KiB load
        const int inst = wave * kAInst + i;
        const int row = inst * 8 + (lane >> 3), j = (lane & 7) ^ swz_a(row);
        lds_dma16(abase, uint32_t((row * K + 4 * j) * 4), stage_lds + inst * 1024);
    }
#pragma unroll
    for (int i = 0; i < kBInst; ++i) {  // one 1 KiB B row per load
        const int row = wave * kBInst + i, j = lane ^ swz_b(row);
        lds_dma16(bbase, uint32_t((row * N + 4 * j) * 4), stage_lds + kAStage * 4 + row * 1024);
    }
}
}  // namespace big

__global__ __launch_bounds__(big::kThreads) void gemm_f32_mfma_256(const float *__restrict__ A,
                                                                   const float *__restrict__ B,
                                                                   float *__restrict__ C, int M, int N, int K,
                                                                   int tiles_m, int tiles_n) {
    using namespace big;
    __shared__ float smem[2 * kStage];
    int tm, tn;  // the launch covers the first gridDim.x tiles of the grouped order
    grouped_tile(xcd_order(int(blockIdx.x), int(gridDim.x)), tiles_m, tiles_n, tm, tn);
    const int m0 = tm * kBM, n0 = tn * kBN;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int wm = wave >> 2, wn = wave & 3;  // wave tile: rows [wm*128, +128), columns [wn*64, +64)
    const int h = lane >> 5, c = lane & 31;
    const uint32_t lds0 = lds_address(smem);
    f32x16 acc[4][2];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
            for (int v = 0; v < 16; ++v) acc[i][j][v] = 0.f;
    const int nk = K / kBK;
    issue_stage(A, B, N, K, m0, n0, 0, lds0);
    drain_vmem();
    __syncthreads();
    for (int kt = 0; kt < nk; ++kt) {
        const float *stage = smem + (kt & 1) * kStage;
        if (kt + 1 < nk) issue_stage(A, B, N, K, m0, n0, (kt + 1) * kBK, lds0 + uint32_t(((kt + 1) & 1) * kStage * 4));
        float b[2][16];  // k-steps 16h + s of this lane's two columns
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            const int col = wn * 64 + j * 32 + c;
#pragma unroll
            for (int s = 0; s < 16; ++s) {
                const int krow = 16 * h + s;
                b[j][s] = stage[kAStage + krow * kBN + (((col >> 2) ^ swz_b(krow)) << 2) + (col & 3)];
            }
        }
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int row = wm * 128 + i * 32 + c;
            f32x4 a[4];
#pragma unroll
            for (int q = 0; q < 4; ++q)
                a[q] = *reinterpret_cast<const f32x4 *>(stage + row * kBK + (((4 * h + q) ^ swz_a(row)) << 2));
            f32x16 p0, p1;
#pragma unroll
            for (int v = 0; v < 16; ++v) {
                p0[v] = 0.f;
                p1[v] = 0.f;
            }
#pragma unroll
            for (int s = 0; s < 16; ++s) {
                p0 = __builtin_amdgcn_mfma_f32_32x32x2f32(a[s >> 2][s & 3], b[0][s], p0, 0, 0, 0);
                p1 = __builtin_amdgcn_mfma_f32_32x32x2f32(a[s >> 2][s & 3], b[1][s], p1, 0, 0, 0);
            }
            acc[i][0] += p0;
            acc[i][1] += p1;
        }
        drain_vmem();
        __syncthreads();
    }
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            const int col = n0 + wn * 64 + j * 32 + c;
#pragma unroll
            for (int v = 0; v < 16; ++v) {
                const int row = m0 + wm * 128 + i * 32 + 8 * (v >> 2) + 4 * h + (v & 3);
                C[size_t(row) * N + col] = acc[i][j][v];
            }
        }
}

// ---- Direct-load 32x32 tiles for small grids -------------------------------
// For products whose 64x64 grid cannot fill the chip, with 16-byte aligned A
// rows (K % 4 == 0). A workgroup of G waves computes one 32x32 tile of C; wave
// g sums the 32-deep K slices g, g+G, g+2G, ... Each lane loads its own MFMA
// operands straight from global memory (L2) into registers: lane (c, h) needs
// A[row c][16h, 16h+16) of a slice (four 16-byte loads) and B[16h, 16h+16)[col
// c] (sixteen loads, each coalesced over 32 lanes into one 128-byte row
// segment). There is no LDS staging and no barrier in the K loop, so three
// slices (60 loads, inside the 6-bit vmcnt) stay in flight per wave, and the
// whole product is one launch (the split-K plan needs a second, reducing one).
//
// Loads carry no bounds branches, so the compiler waits for exactly the slice
// it consumes: row, column and k indices are clamped into the matrices. A
// clamped row of A (or column of B) only reaches rows (columns) of the 32x32
// product that are never stored; k >= K is zeroed in both operands when the
// last, partial slice is consumed. At the end waves 1..G-1 leave their sums in
// LDS and wave 0 adds them in wave order: the result is deterministic. Per
// element: a wave's slices form one MFMA chain when the wave has at most six
// of them; longer K ranges sum each slice as a 16-step chain from zero and add
// it to the wave's running sum.
namespace direct {
constexpr int kDepth = 3;  // slices in flight per wave

struct Slice {
    f32x4 a[4];   // A[row c][k0 + 16h + 4q + e] at a[q][e]
    float b[16];  // B[k0 + 16h + s][col c] at b[s]
};

// BUFA (A below 2 GiB; required when K % 4 != 0): buffer loads at
// 4-byte-aligned offsets, unclamped: a run that crosses the end of its row
// reads the next row's first floats at k >= K (zeroed when consumed), and the
// buffer's range check returns zero past the end of A. Otherwise a 4-float
// run clamped to start at most at K - 4 stays inside its (aligned) row.
//
// BUFB (K*N*4 < 2^31): B through buffer loads at a 32-bit offset per lane, one
// add per load instead of a clamped 64-bit address; rows k >= K lie past the
// buffer's end and read as zero.
//
// `live` false (a prefetch past the wave's last slice): buffer loads go to an
// offset past any buffer of this kernel, which reads zero without touching
// memory, so the kernel does not end waiting on loads nobody consumes.
//
// WHOLE (K % 32 == 0, with BUFB): every row of every slice lies inside B, so
// a B row's step is the load's scalar offset and costs no VALU add.
template <bool BUFA, bool BUFB, bool WHOLE = false>
__device__ inline void load_slice(const float *__restrict__ A, __amdgpu_buffer_rsrc_t ra,
                                  const float *__restrict__ B, __amdgpu_buffer_rsrc_t rb, int K, int N, size_t arow,
                                  int lda, int bcol, int k0, bool live, int h, Slice &s) {
    const int kb = k0 + 16 * h;
    if constexpr (BUFA) {
        const uint32_t first = live ? (uint32_t(arow) * uint32_t(lda) + uint32_t(kb)) * 4u : kDeadOffset;
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const auto v = __builtin_amdgcn_raw_buffer_load_b128(ra, int(first + 16u * q), 0, 0);
            s.a[q] = f32x4{__uint_as_float(v[0]), __uint_as_float(v[1]), __uint_as_float(v[2]), __uint_as_float(v[3])};
        }
    } else {
        const float *ap = A + arow * lda;
#pragma unroll
        for (int q = 0; q < 4; ++q) s.a[q] = *reinterpret_cast<const f32x4 *>(ap + min(kb + 4 * q, K - 4));
    }
    if constexpr (BUFB) {
        const uint32_t first = live ? (uint32_t(kb) * uint32_t(N) + uint32_t(bcol)) * 4u : kDeadOffset;
        const uint32_t row = uint32_t(N) * 4u;
#pragma unroll
        for (int e = 0; e < 16; ++e) {
            if constexpr (WHOLE)
                s.b[e] = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(rb, int(first), int(uint32_t(e) * row), 0));
            else
                s.b[e] = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(rb, int(first + uint32_t(e) * row), 0, 0));
        }
    } else {
#pragma unroll
        for (int e = 0; e < 16; ++e) s.b[e] = B[size_t(min(kb + e, K - 1)) * N + bcol];
    }
}

// `valid` = K - (k0 + 16h): operand pairs at s >= valid lie past K. ZB: B is
// already zero there (buffer loads), so only A is masked. CHAIN: the slice's
// MFMAs accumulate straight into the wave's running sum (for waves of at most
// kChainSlices slices, 192 k); otherwise each slice is summed from zero and
// folded into the running sum with VALU adds, which bounds the length of the
// matrix cores' accumulation chains for long K ranges.
constexpr int kChainSlices = 6;
template <bool ZB, bool CHAIN, bool WHOLE = false>
__device__ inline void mma_slice(const Slice &s, int valid, f32x16 &acc) {
    f32x16 part;
#pragma unroll
    for (int v = 0; v < 16; ++v) part[v] = 0.f;
    f32x16 &sum = CHAIN ? acc : part;
#pragma unroll
    for (int q = 0; q < 4; ++q)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const int i = 4 * q + e;
            const float a = WHOLE || i < valid ? s.a[q][e] : 0.f, b = WHOLE || ZB || i < valid ? s.b[i] : 0.f;
            sum = __builtin_amdgcn_mfma_f32_32x32x2f32(a, b, sum, 0, 0, 0);
        }
    if (!CHAIN) acc += part;
}
}  // namespace direct

// gridDim.y > 1: a batch of independent products, product z at A + z*sa,
// B + z*sb, C + z*sc (attention's P.V per head, or the K slices of a split
// product: sa = K, sb = K*N with A rows lda apart).
// BUFA: A is read through buffer loads, which needs ((M-1)*lda + K)*4 < 2^31
// (per product of a batch); unaligned rows (K % 4 != 0) require it. BUFB: B
// is read through buffer loads (K*N*4 < 2^31; per product of a batch).
// WHOLE: K % 32 == 0 and BUFB (no slice runs past K: no masks).
template <int G, bool BUFA, bool BUFB, bool CHAIN, bool WHOLE = false>
__global__ __launch_bounds__(64 * G) void gemm_f32_direct(const float *__restrict__ A, const float *__restrict__ B,
                                                          float *__restrict__ C, int M, int N, int K, int lda,
                                                          int tiles_m, int tiles_n, size_t sa, size_t sb,
                                                          size_t sc) {
    using namespace direct;
    constexpr int D = kDepth;
    __shared__ float red[(G > 1 ? G : 1) * 16 * 64];
    A += blockIdx.y * sa;
    B += blockIdx.y * sb;
    C += blockIdx.y * sc;
    const __amdgpu_buffer_rsrc_t ra = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<float *>(A), 0, BUFA ? int((uint32_t(M - 1) * uint32_t(lda) + uint32_t(K)) * 4u) : 0,
        int(kBufferWord3));
    const __amdgpu_buffer_rsrc_t rb = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<float *>(B), 0, BUFB ? int(uint32_t(K) * uint32_t(N) * 4u) : 0, int(kBufferWord3));
    int tm, tn;
    tile_coords(tiles_m, tiles_n, tm, tn);
    const int lane = threadIdx.x & 63;
    const int g = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // wave index, uniform
    const int c = lane & 31, h = lane >> 5;
    const int row = tm * 32 + c, col = tn * 32 + c;
    const size_t arow = size_t(min(row, M - 1));
    const int bcol = min(col, N - 1);
    const int slices = (K + kBK - 1) / kBK;
    const int count = g < slices ? (slices - g + G - 1) / G : 0;  // this wave's slices g, g+G, ...
    // K offset of this wave's j-th slice, clamped to the last slice: loads past
    // the end (dead: buffer loads skip them) re-read an in-range slice and are
    // never consumed.
    auto slice_k = [&](int j) { return min(g + j * G, slices - 1) * kBK; };
    auto valid = [&](int j) { return K - slice_k(j) - 16 * h; };
    f32x16 acc;
#pragma unroll
    for (int v = 0; v < 16; ++v) acc[v] = 0.f;
    Slice buf[D];
    if (count > 0) {
#pragma unroll
        for (int d = 0; d < D; ++d) {
            load_slice<BUFA, BUFB, WHOLE>(A, ra, B, rb, K, N, arow, lda, bcol, slice_k(d), d < count, h, buf[d]);
            __builtin_amdgcn_sched_barrier(0);  // loads issued slice by slice
        }
        int i = 0;
        for (; i + D <= count; i += D) {
#pragma unroll
            for (int d = 0; d < D; ++d) {
                mma_slice<BUFB, CHAIN, WHOLE>(buf[d], valid(i + d), acc);
                load_slice<BUFA, BUFB, WHOLE>(A, ra, B, rb, K, N, arow, lda, bcol, slice_k(i + d + D),
                                              i + d + D < count, h, buf[d]);
                // Keep the slices in order: interleaving their independent
                // MFMA chains would make the first one wait for every load.
                __builtin_amdgcn_sched_barrier(0);
            }
        }
#pragma unroll
        for (int d = 0; d < D; ++d)
            if (i + d < count) mma_slice<BUFB, CHAIN, WHOLE>(buf[d], valid(i + d), acc);
    }
    // The G partial tiles meet in LDS; wave g then sums and stores the
    // accumulator entries v of its share (16/G of them), adding the waves'
    // partials in wave order.
    constexpr int kShare = 16 / G;
    if (G > 1) {
#pragma unroll
        for (int v = 0; v < 16; ++v) red[(g * 16 + v) * 64 + lane] = acc[v];
        __syncthreads();
#pragma unroll
        for (int j = 0; j < kShare; ++j) {
            const int v = g * kShare + j;
            float sum = red[v * 64 + lane];
#pragma unroll
            for (int w = 1; w < G; ++w) sum += red[(w * 16 + v) * 64 + lane];
            acc[j] = sum;
        }
    }
    const bool interior = tm * 32 + 32 <= M && tn * 32 + 32 <= N;  // wave-uniform
#pragma unroll
    for (int j = 0; j < kShare; ++j) {
        const int v = G > 1 ? g * kShare + j : j;
        const int crow = tm * 32 + 8 * (v >> 2) + 4 * h + (v & 3);
        if (interior || (crow < M && col < N)) C[size_t(crow) * N + col] = acc[j];
    }
}

// One direct launch of G waves per 32x32 tile; A and B through buffer loads
// when a product's operand is below 2 GiB (A always when `bufa`: unaligned
// rows, whose limit the caller checks).
template <int G, bool CHAIN>
void launch_direct_gc(hipStream_t stream, dim3 grid, bool bufa, bool bufb, const float *a, const float *b, float *c,
                      int m, int n, int k, int lda, int tiles_m, int tiles_n, size_t sa, size_t sb, size_t sc) {
    const dim3 block(64 * G);
    auto go = [&](auto kernel) {
        hipLaunchKernelGGL(kernel, grid, block, 0, stream, a, b, c, m, n, k, lda, tiles_m, tiles_n, sa, sb, sc);
    };
    if (bufb && k % kBK == 0)
        bufa ? go(gemm_f32_direct<G, true, true, CHAIN, true>) : go(gemm_f32_direct<G, false, true, CHAIN, true>);
    else if (bufa)
        bufb ? go(gemm_f32_direct<G, true, true, CHAIN>) : go(gemm_f32_direct<G, true, false, CHAIN>);
    else
        bufb ? go(gemm_f32_direct<G, false, true, CHAIN>) : go(gemm_f32_direct<G, false, false, CHAIN>);
}
template <int G>
void launch_direct_g(hipStream_t stream, dim3 grid, bool bufa, const float *a, const float *b, float *c, int m,
                     int n, int k, int lda, int tiles_m, int tiles_n, size_t sa, size_t sb, size_t sc) {
    const bool bufb = uint64_t(k) * uint64_t(n) * 4u < (uint64_t(1) << 31);
    bufa = bufa || (uint64_t(m - 1) * uint64_t(lda) + uint64_t(k)) * 4u < (uint64_t(1) << 31);
    // A wave sums the slices g, g + G, ...: at most ceil(slices / G).
    const bool chain = (k + kBK - 1) / kBK <= direct::kChainSlices * G;
    if (chain)
        launch_direct_gc<G, true>(stream, grid, bufa, bufb, a, b, c, m, n, k, lda, tiles_m, tiles_n, sa, sb, sc);
    else
        launch_direct_gc<G, false>(stream, grid, bufa, bufb, a, b, c, m, n, k, lda, tiles_m, tiles_n, sa, sb, sc);
}

// ---- Direct tiles staged through LDS ----------------------------------------
// The unsplit direct plan (32x32 tiles, wave g of G summing the K slices g,
// g + G, ...) for aligned rows, one workgroup per CU: each wave moves its
// slices into its own LDS region with 16-byte buffer loads into LDS (A 32x32
// and B 32x32 per slice, 8 KiB), up to four slices ahead in a ring of at most
// four slots, and reads its MFMA operands from there. The loads of a wave's
// first slices all go out at entry as one-KiB requests; the register-staged
// form issued 20 narrower loads per slice (B as single floats, one column per
// lane) and its slices arrived a memory round trip apart. No barrier: a wave
// reads only what its own loads wrote, counted by vmcnt.
// Every wave runs S = ceil(slices / G) slices, fully unrolled: a wave with
// one slice fewer runs a last slice of zeros (its loads aim past both
// buffers, which reads zero without touching memory), so slots, LDS offsets
// and wait counts are compile-time and the loop has no branch. Adding zero
// products leaves the sums' bits unchanged (a chain that starts at +0 never
// holds -0), and per output the MFMA steps, the chain and the reduction are
// the register-staged kernel's: the outputs are bit-identical to it.
// Measured at 512^3 (back to back, us): register-staged 5.87-6.14; this form
// with a run-time slice loop 5.53, with branches on the slice count 5.18,
// branch-free 4.78. Timestamps per wave (medians): the first slice consumed
// 1.76 -> 1.44 us after entry, the other three 2.24 -> 1.36 us (their 48
// MFMAs take 1.28 us at the peak rate).
// A slot: A rows of 128 bytes, chunk j of row r at j ^ swz_a(r) (as the tile
// kernels' A stages); then B rows of 128 bytes, row r in row slot
// r ^ ((r >> 4) & 1), so that rows s and 16 + s, which one B operand read
// takes for the two halves of the wave, sit on different banks.
namespace dlds {
constexpr uint32_t kSlotB = 8192;
constexpr int kLoads = 8;       // one-KiB loads per slice: four of A, four of B
constexpr int kMaxSlices = 6;   // per wave: direct::kChainSlices
__host__ __device__ constexpr int ring(int s) { return s < 4 ? s : 4; }
}  // namespace dlds

template <int N>
__device__ inline void wait_vmcnt() {
    static_assert(N >= 0 && N <= 24 && N % 8 == 0, "wait counts of whole slices");
    if constexpr (N == 0)
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    else if constexpr (N == 8)
        asm volatile("s_waitcnt vmcnt(8)" ::: "memory");
    else if constexpr (N == 16)
        asm volatile("s_waitcnt vmcnt(16)" ::: "memory");
    else
        asm volatile("s_waitcnt vmcnt(24)" ::: "memory");
}

template <int G, int S, bool WHOLE>
__global__ __launch_bounds__(64 * G) void gemm_f32_direct_lds(const float *__restrict__ A,
                                                              const float *__restrict__ B, float *__restrict__ C,
                                                              int M, int N, int K, int tiles_m, int tiles_n) {
    using namespace dlds;
    static_assert(S >= 1 && S <= kMaxSlices, "slices per wave");
    constexpr int kRing = ring(S);
    constexpr uint32_t kWaveB = kRing * kSlotB;
    __shared__ __attribute__((aligned(1024))) char lds[G * kWaveB];
    const __amdgpu_buffer_rsrc_t ra = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<float *>(A), 0, int(uint32_t(M) * uint32_t(K) * 4u), int(kBufferWord3));
    const __amdgpu_buffer_rsrc_t rb = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<float *>(B), 0, int(uint32_t(K) * uint32_t(N) * 4u), int(kBufferWord3));
    int tm, tn;
    tile_coords(tiles_m, tiles_n, tm, tn);
    const int lane = threadIdx.x & 63;
    const int g = __builtin_amdgcn_readfirstlane(int(threadIdx.x) >> 6);
    const int c = lane & 31, h = lane >> 5;
    const int slices = (K + kBK - 1) / kBK;
    char *region = lds + g * kWaveB;
    // Per-lane byte offsets of the four A and four B loads of a slice at k 0;
    // slice k0 adds 4 k0 (A) and 4 k0 N (B). Rows past M (and, through 32-bit
    // wrap, far past it) read zero or rows that feed only unstored outputs;
    // B runs past N read the next row's first columns, also unstored.
    uint32_t aoff[4], boff[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int r = 8 * i + (lane >> 3), lc = (lane & 7) ^ swz_a(r);
        aoff[i] = (uint32_t(tm * 32 + r) * uint32_t(K) + uint32_t(4 * lc)) * 4u;
        const int p = 8 * i + (lane >> 3), row = p ^ ((p >> 4) & 1);
        boff[i] = (uint32_t(row) * uint32_t(N) + uint32_t(tn * 32 + 4 * (lane & 7))) * 4u;
    }
    // Slice j of this wave into `slot`; a slice past K aims its loads past
    // both buffers.
    auto issue = [&](int j, int slot) {
        const int sl = g + j * G;
        const bool live = sl < slices;
        const uint32_t k0 = uint32_t(sl) * kBK;
        char *dst = region + slot * kSlotB;
#pragma unroll
        for (int i = 0; i < 4; ++i)
            __builtin_amdgcn_raw_ptr_buffer_load_lds(
                ra, (__attribute__((address_space(3))) void *)(dst + i * 1024), 16,
                int(live ? aoff[i] + 4u * k0 : kDeadOffset), 0, 0, 0);
#pragma unroll
        for (int i = 0; i < 4; ++i)
            __builtin_amdgcn_raw_ptr_buffer_load_lds(
                rb, (__attribute__((address_space(3))) void *)(dst + 4096 + i * 1024), 16,
                int(live ? boff[i] + 4u * k0 * uint32_t(N) : kDeadOffset), 0, 0, 0);
    };
#pragma unroll
    for (int j = 0; j < kRing; ++j) issue(j, j);
    f32x16 acc;
#pragma unroll
    for (int v = 0; v < 16; ++v) acc[v] = 0.f;
    auto slice = [&](auto jc) __attribute__((always_inline)) {
        constexpr int j = decltype(jc)::value;
        constexpr int later = S - 1 - j < 3 ? S - 1 - j : 3;  // slices in flight behind this one
        wait_vmcnt<kLoads * later>();
        const char *sa = region + (j % kRing) * kSlotB;
        const char *sb = sa + 4096;
        f32x4 a[4];
        float b[16];
#pragma unroll
        for (int q = 0; q < 4; ++q)
            a[q] = *reinterpret_cast<const f32x4 *>(sa + c * 128 + (((4 * h + q) ^ swz_a(c)) << 4));
#pragma unroll
        for (int x = 0; x < 16; ++x) b[x] = *reinterpret_cast<const float *>(sb + ((16 * h + x) ^ h) * 128 + c * 4);
        // Elements past K (the last slice of a ragged K): A is zeroed; B's rows
        // past K lie past its buffer and read zero. One MFMA chain over all of
        // the wave's slices, as the register-staged kernel runs the unsplit
        // plans.
        const int valid = K - (g + j * G) * kBK - 16 * h;
#pragma unroll
        for (int q = 0; q < 4; ++q)
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const int i = 4 * q + e;
                acc = __builtin_amdgcn_mfma_f32_32x32x2f32(WHOLE || i < valid ? a[q][e] : 0.f, b[i], acc, 0, 0, 0);
            }
        if constexpr (j + kRing < S) {
            __builtin_amdgcn_sched_barrier(0);
            issue(j + kRing, j % kRing);  // the slot's operands are in registers
            __builtin_amdgcn_sched_barrier(0);
        }
    };
    slice(std::integral_constant<int, 0>{});
    if constexpr (S > 1) slice(std::integral_constant<int, 1>{});
    if constexpr (S > 2) slice(std::integral_constant<int, 2>{});
    if constexpr (S > 3) slice(std::integral_constant<int, 3>{});
    if constexpr (S > 4) slice(std::integral_constant<int, 4>{});
    if constexpr (S > 5) slice(std::integral_constant<int, 5>{});
    // Every load has been waited for (the last slice waits for vmcnt 0): the
    // G partial tiles meet in LDS (wave w's at the start of its region) and
    // wave g then sums and stores entries v of its share, in wave order.
    constexpr int kShare = 16 / G;
    constexpr int kRegionF = int(kWaveB / 4);
    float *red = reinterpret_cast<float *>(lds);
    if (G > 1) {
#pragma unroll
        for (int v = 0; v < 16; ++v) red[g * kRegionF + v * 64 + lane] = acc[v];
        __syncthreads();
#pragma unroll
        for (int j = 0; j < kShare; ++j) {
            const int v = g * kShare + j;
            float total = red[v * 64 + lane];
#pragma unroll
            for (int w = 1; w < G; ++w) total += red[w * kRegionF + v * 64 + lane];
            acc[j] = total;
        }
    }
    const int col = tn * 32 + c;
    const bool interior = tm * 32 + 32 <= M && tn * 32 + 32 <= N;  // wave-uniform
#pragma unroll
    for (int j = 0; j < kShare; ++j) {
        const int v = G > 1 ? g * kShare + j : j;
        const int crow = tm * 32 + 8 * (v >> 2) + 4 * h + (v & 3);
        if (interior || (crow < M && col < N)) C[size_t(crow) * N + col] = acc[j];
    }
}

// LDS bytes of the LDS-staged direct kernel for G waves over `slices` K slices.
uint32_t direct_lds_bytes(int g, int slices) {
    return uint32_t(g) * uint32_t(dlds::ring((slices + g - 1) / g)) * dlds::kSlotB;
}

hipError_t launch_direct_lds(hipStream_t stream, int g, const float *a, const float *b, float *c, int m, int n,
                             int k, int tiles_m, int tiles_n) {
    const dim3 grid(unsigned(tiles_m * tiles_n)), block(unsigned(64 * g));
    const int slices = (k + kBK - 1) / kBK, per_wave = (slices + g - 1) / g;
    const bool whole = k % kBK == 0;
    hipError_t status = hipErrorInvalidValue;
    auto go = [&](auto kernel) {
        hipLaunchKernelGGL(kernel, grid, block, 0, stream, a, b, c, m, n, k, tiles_m, tiles_n);
        status = hipGetLastError();
    };
    auto with_s = [&](auto gc, auto wc) {
        constexpr int G = decltype(gc)::value;
        constexpr bool WH = decltype(wc)::value;
        switch (per_wave) {
            case 1: go(gemm_f32_direct_lds<G, 1, WH>); break;
            case 2: go(gemm_f32_direct_lds<G, 2, WH>); break;
            case 3: go(gemm_f32_direct_lds<G, 3, WH>); break;
            case 4: go(gemm_f32_direct_lds<G, 4, WH>); break;
            case 5: go(gemm_f32_direct_lds<G, 5, WH>); break;
            case 6: go(gemm_f32_direct_lds<G, 6, WH>); break;
            default: break;  // more slices per wave: not a direct plan
        }
    };
    auto with_g = [&](auto wc) {
        if (g == 4) with_s(std::integral_constant<int, 4>{}, wc);
        else if (g == 2) with_s(std::integral_constant<int, 2>{}, wc);
        else if (g == 1) with_s(std::integral_constant<int, 1>{}, wc);
    };
    if (whole)
        with_g(std::true_type{});
    else
        with_g(std::false_type{});
    return status;
}

hipError_t launch_direct(hipStream_t stream, dim3 grid, int g, bool bufa, const float *a, const float *b, float *c,
                         int m, int n, int k, int lda, int tiles_m, int tiles_n, size_t sa = 0, size_t sb = 0,
                         size_t sc = 0) {
    if (g == 4)
        launch_direct_g<4>(stream, grid, bufa, a, b, c, m, n, k, lda, tiles_m, tiles_n, sa, sb, sc);
    else if (g == 2)
        launch_direct_g<2>(stream, grid, bufa, a, b, c, m, n, k, lda, tiles_m, tiles_n, sa, sb, sc);
    else if (g == 1)
        launch_direct_g<1>(stream, grid, bufa, a, b, c, m, n, k, lda, tiles_m, tiles_n, sa, sb, sc);
    else
        return hipErrorInvalidValue;
    return hipGetLastError();
}

// C[i] = sum over slices z (in order) of W[z*MN + i]. 16-byte runs only
// where every run of W and of C is 16-byte aligned: mn % 4 == 0 and both
// bases aligned (W is a whole workspace; C may start at any 4-byte boundary,
// as the allocation-free entry accepts).
__global__ __launch_bounds__(256) void splitk_reduce(const float *__restrict__ W, float *__restrict__ C,
                                                     size_t mn, int slices) {
    const size_t i = (size_t(blockIdx.x) * 256 + threadIdx.x) * 4;
    if (i >= mn) return;
    const bool runs = mn % 4 == 0 && ((reinterpret_cast<uintptr_t>(W) | reinterpret_cast<uintptr_t>(C)) & 15u) == 0;
    if (i + 4 <= mn && runs) {
        f32x4 s = *reinterpret_cast<const f32x4 *>(W + i);
        for (int z = 1; z < slices; ++z) s += *reinterpret_cast<const f32x4 *>(W + size_t(z) * mn + i);
        *reinterpret_cast<f32x4 *>(C + i) = s;
    } else {
        for (size_t e = i; e < i + 4 && e < mn; ++e) {
            float s = W[e];
            for (int z = 1; z < slices; ++z) s += W[size_t(z) * mn + e];
            C[e] = s;
        }
    }
}

struct Plan {
    int tm, tn;     // waves' MFMA blocks: tile = (64*tm) x (64*tn)
    int slices;     // K slices (1 = no split)
    int kchunk;     // K per slice, a multiple of 32
    int tiles_m, tiles_n;
    bool big;       // 256x256 eight-wave tile (tiles_m/tiles_n count 256x256 tiles)
    int big_full;   // 256x256 tiles in whole rounds; the rest run as 128x128 tiles
    int direct;     // > 0: gemm_f32_direct with this many waves (tiles_m/tiles_n count 32x32 tiles)
    int kgroups;    // 2 or 4: 64x64 tiles with that many K groups of four waves (0 or 1: one group)
    int tail_tm, tail_tn;  // big plans: the partial last round's tile, (64*tail_tm) x (64*tail_tn)
    bool bufa;             // direct plans over unaligned A rows: A through buffer loads
    bool ring = false;     // persistent 128x128 tiles, one workgroup per CU (gemm_f32_ring)
};

constexpr int kSlots = 512;        // co-resident 256-thread workgroups: two per CU
constexpr int kMinGroups = 384;    // a tile shape needs ~1.5 workgroups per CU to be considered
constexpr int kCUs = 256;
constexpr int kSplitTarget = 256;  // split K into about one workgroup per CU
constexpr int kMinChunk = 128;
// Unsplit 64x64 grids of up to one tile per CU with K of at least this run
// four K groups (16 waves, four per SIMD) instead of two. Measured on MI355X:
// 1024^3 22.8 -> 22.1 us, 1024x1024x2048 42.7 -> 40.5, 1024x1024x4096 82.3 ->
// 77.4, 1000x1000x1024 25.6 -> 24.5, 768x768x1024 22.6 -> 21.8; K = 512 ties
// (12.9 / 12.8). Unaligned rows through buffer loads: 1000x777x1024 24.2 ->
// 22.8, 1023x1000x2049 46.2 -> 44.2, but 1000x777x513 15.8 -> 16.3. The
// clamped global-load loop (operands of 2 GiB or more) keeps two groups: it
// spills at four waves per SIMD.
constexpr int kFourGroupMinK = 768;

// Tile choice among 128x128, 128x64 and 64x64 (128x64 measured at or above
// 64x128 on the tall and wide shapes tried, so 64x128 is not chosen). Each
// candidate with at least kMinGroups workgroups scores fill x eff, where
// fill = groups / (kSlots x rounds) is the busy share of its rounds and eff =
// 1.00 / 0.97 / 0.90 its throughput on whole rounds. Measured on MI355X:
// 3072^3 runs 64x64 at 111 TFLOP/s (128x128, whose second round is 12% full:
// 94); 6144x1024x1024 64x64 109 (128x64: 93); 2500^3 128x128 88 (128x64: 82);
// 1024x4096x4096 128x64 124 (64x128: 117).
//
// Below kMinGroups, 64x64 tiles, chosen by the tile count t:
//  * 256 < t < 384: one K group (1536x1024x1024 40.4 us; two groups 43.7).
//  * 128 < t <= 256: one workgroup per CU with two K groups, so two waves
//    share each SIMD: 1024^3 25.7 -> 22.8 us, 768^3 19.7 -> 17.6,
//    1000x777x512 17.2 -> 14.6, 1024x1024x4096 94.5 -> 81.6.
//  * t <= 128: the direct-load 32x32 kernel when it applies (below), else K
//    split over about kSplitTarget workgroups of two K groups each, then an
//    ordered reduction: 1024x512x1024 25.2 us unsplit, 16.7 split in two;
//    512x1024x2048 48.3 -> 25.8. A K group needs two stages or more.

// Grids of at least 256 tiles of 256x256 run as 128x128 tiles (two
// workgroups per CU, each with its own barrier, folding every kFoldStages)
// unless that grid's last round would hold fewer than 128 of its 512
// workgroups. Measured on MI355X, 128x128 against the 256x256 kernel (plus a
// tail in smaller tiles): 4096^3 136.6 / 135.2 TFLOP/s, 8192x8192x2048 136.4 /
// 134.7, 4096x4096x16384 138.6 / 136.4, 4096x11008x4096 (5.4 rounds) 133.5 /
// 131.3, 6144x6144x2048 (4.5) 135.0 / 132.9; but 5120x5120x2048 (3.1 rounds)
// 120.4 / 126.3. There the 256x256 tile (one workgroup per CU) takes the whole
// rounds of 256 tiles and the rest of the grid (a partial round) runs as
// smaller tiles: a partial round costs about a whole one.
bool big_fits(uint32_t m, uint32_t n, uint32_t k) {
    if (m % big::kBM != 0 || n % big::kBN != 0 || k % kBK != 0 || k == 0) return false;
    if (!dma_offsets_fit(big::kBM, big::kBN, k, n)) return false;
    return uint64_t(m / big::kBM) * (n / big::kBN) >= uint64_t(kCUs);
}

// The LDS-staged direct kernel serves unsplit direct plans with 16-byte rows
// (K and N multiples of 4, A and B starting 16-byte aligned), at most one
// workgroup per CU (up to 32 KiB of LDS per wave, 128 KiB per workgroup),
// both operands below 2 GiB (32-bit buffer offsets) and at most six slices
// per wave (direct_waves gives four waves from four slices up to 24).
bool direct_lds_fits(uint32_t m, uint32_t n, uint32_t k, int tiles) {
    return k % 4 == 0 && n % 4 == 0 && tiles <= kCUs && (k + kBK - 1) / kBK <= 4u * dlds::kMaxSlices &&
           uint64_t(m) * k * 4u < (uint64_t(1) << 31) && uint64_t(k) * n * 4u < (uint64_t(1) << 31);
}

// Direct-load 32x32 tiles (one launch, K split over the four waves of a
// workgroup) for grids of at most 128 64x64 tiles, aligned A rows, at least
// 64 tiles of 32x32 and at most 6 slices of 32 k per wave (no more waves than
// slices). Measured on MI355X: 512^3 7.5 us against 9.6 split in four,
// 384^3 6.8 against 7.9, 700^3 15.0 against 18.8 for 64x64 tiles with two K
// groups. At 8 slices per wave the split plan wins (1024x512x1024 18.1
// against 16.7), and unaligned rows (K = 513) cost the direct loads more than
// the LDS-staged kernel.
int direct_waves(uint32_t m, uint32_t n, uint32_t k) {
    if (k % 4 != 0) return 0;
    const uint64_t t64 = uint64_t((m + 63) / 64) * ((n + 63) / 64);
    const uint64_t t32 = uint64_t((m + 31) / 32) * ((n + 31) / 32);
    if (t64 > uint64_t(kCUs / 2) || t32 < 64) return 0;
    const uint32_t slices = (k + kBK - 1) / kBK;
    if (slices > 4 * 6) return 0;
    int g = 4;
    while (g > 1 && uint32_t(g) > slices) g /= 2;
    return g;
}

// Products of at most 32 rows (one 32-row tile: decode-like shapes) that the
// unsplit direct plan does not take stream B through direct-load 32x32 tiles
// split over K: four waves per tile, the K slices a batch of products into the
// workspace, summed in slice order by the reduce. The slice count aims at
// ~1536 waves, divides K into runs of a multiple of 4 (one run length for the
// batch) of at least 128, and needs at least 1024 waves. Measured on MI355X
// against the 64x64 split or
// K-group tiles: 1x4096x4096 27.4 -> 20.4 us, 1x11008x4096 79.5 -> 45.7,
// 32x11008x4096 79.7 -> 48.3, 16x1024x2816 13.2 -> 11.6. From 64 rows the
// 32x32 tiles read B once per 32 rows and lose (64x4096x4096 28.1 -> 34.2).
// Returns the slice count, or 0 where the plan does not apply.
int skinny_slices(uint32_t m, uint32_t n, uint32_t k) {
    if (m > 32 || k % 4 != 0 || k < 128) return 0;
    const uint64_t t64 = uint64_t((n + 63) / 64);
    if (t64 > uint64_t(kCUs)) return 0;
    const uint32_t tiles = (n + 31) / 32;
    int s = int(std::min<uint32_t>(16, (1536 + 4 * tiles - 1) / (4 * tiles)));
    while (s > 1 && (k % uint32_t(s) != 0 || (k / uint32_t(s)) % 4 != 0 || k / uint32_t(s) < 128)) --s;
    // Below ~1024 waves the streams fall short (1x4096x4096 unsplit: 31.7 us).
    return uint64_t(tiles) * uint64_t(s) * 4 >= 1024 ? s : 0;
}

// The partial last round of a 256x256 grid (`tail` such tiles) runs as
// 128x128 tiles when those are at most one workgroup per CU, else as 64x64
// tiles. Measured with the whole rounds before it: 5120x5120x2048 (144 tail
// tiles) 933 / 874 / 872 us with 128x128 / 128x64 / 64x64; 6144x6144x1024 (64)
// 603 with 128x128 against 630 with 128x64. (A grid takes the 256x256 plan
// only when its 128x128 last round would be under a quarter full, so the
// tail is 1-31 or 129-159 tiles, where 64x64 tiles fill the rounds better
// than 128x64 ones by the fill x efficiency measure of the whole-grid choice.)
void tail_tile(int tail, int &tm, int &tn) {
    tm = tn = 4 * tail <= kCUs ? 2 : 1;
}

// The unaligned loop's buffer loads address each operand with 32-bit byte
// offsets checked against its size: both operands must be below 2 GiB.
bool unaligned_buffers_fit(uint32_t m, uint32_t n, uint32_t k) {
    return uint64_t(m) * k * 4 < (uint64_t(1) << 31) && uint64_t(k) * n * 4 < (uint64_t(1) << 31);
}

// A second look at grids of more than one 64x64 tile per CU, over the tile
// shapes (index into {128x128, 128x64, 64x64}) whose grid has no edge tile.
// Such a grid runs every tile on the LDS-direct loop; one edge tile puts the
// whole launch on the mixed-path kernel. Its cost is the busiest CU's work:
// ceil(tiles / 256) tiles x tile area / the tile's efficiency (1.00 / 0.97 /
// 0.87; 0.93 / 0.90 for 128x128 / 128x64 grids of at most one tile per CU,
// which run one wave per SIMD). The edge-free choice replaces the round-fill
// choice `old` when `old` has edge tiles, or when it is predicted at least 5%
// faster, except that K below 512 keeps the smaller tile. Measured on MI355X
// (TFLOP/s, round-fill -> edge-free): 3072x1024x4096 98.9 -> 113.4 (128x64 ->
// 64x64), 2048x1536x512 87.5 -> 100.4, 2048x3072x1024 114.1 -> 122.8 (64x64 ->
// 128x64), 6144x1024x1024 114.6 -> 123.5, 2304^3 100.4 -> 108.0, 3648^2x1024
// 102.3 -> 112.6 (128x128 with edge tiles -> 64x64); at K = 384 the larger
// tile lost (2048x3072x384 103.3 -> 92.5), and predicted gains under 5% were
// ties or losses (12288x1024x1024 128x64 127.5, 128x128 122.8).
int edge_free_choice(uint32_t m, uint32_t n, uint32_t k, int old) {
    const int shapes[3][2] = {{2, 2}, {2, 1}, {1, 1}};
    const double eff_shared[3] = {1.00, 0.97, 0.87}, eff_alone[3] = {0.93, 0.90, 0.87};
    auto edge_free = [&](int i) { return m % (64u * shapes[i][0]) == 0 && n % (64u * shapes[i][1]) == 0; };
    auto cost = [&](int i) {
        const uint64_t tiles = uint64_t((m + 64 * shapes[i][0] - 1) / (64 * shapes[i][0])) *
                               ((n + 64 * shapes[i][1] - 1) / (64 * shapes[i][1]));
        const double per_cu = double((tiles + kCUs - 1) / kCUs), area = shapes[i][0] * shapes[i][1];
        return per_cu * area / (tiles > uint64_t(kCUs) ? eff_shared[i] : eff_alone[i]);
    };
    int cand = -1;
    for (int i = 0; i < 3; ++i)
        if (edge_free(i) && (cand < 0 || cost(i) < cost(cand))) cand = i;
    if (cand < 0 || cand == old) return old;
    if (!edge_free(old)) return cand;
    const bool larger = shapes[cand][0] * shapes[cand][1] > shapes[old][0] * shapes[old][1];
    if (larger && k < 512) return old;
    return cost(old) > 1.05 * cost(cand) ? cand : old;
}

// Unaligned rows (K % 4 != 0) on grids of at most half the CUs' worth of
// 64x64 tiles run the direct-load 32x32 tiles too, with A through buffer
// loads, when K has at most 24 slices of 32 and the grid at least 64 tiles of
// 32x32 (the split-K 64x64 plans otherwise). Measured on MI355X against them:
// 500x777x513 17.9 -> 12.4 us, 100x777x513 10.2 -> 8.3. On larger grids the
// direct tiles lose to the LDS-staged 64x64 tiles with two K groups
// (1000x777x513: 15.6 us against 20.8 with 32x32 tiles and 20.1 with 32x64
// tiles whose waves share each A operand between two MFMA chains).
int direct_waves_unaligned(uint32_t m, uint32_t n, uint32_t k) {
    if (k % 4 == 0 || !unaligned_buffers_fit(m, n, k)) return 0;
    const uint64_t t64 = uint64_t((m + 63) / 64) * ((n + 63) / 64);
    const uint64_t t32 = uint64_t((m + 31) / 32) * ((n + 31) / 32);
    if (t64 > uint64_t(kCUs / 2) || t32 < 64) return 0;
    const uint32_t slices = (k + kBK - 1) / kBK;
    if (slices > 4 * 6) return 0;
    int g = 4;
    while (g > 1 && uint32_t(g) > slices) g /= 2;
    return g;
}

// Persistent 128x128 tiles (gemm_f32_ring): whole tiles, K in whole
// eight-stage iterations, at least one tile per CU, 32-bit load offsets
// (with the stores' row offsets inside a tile).
bool ring_fits(uint32_t m, uint32_t n, uint32_t k) {
    if (m % ring::kBM != 0 || n % ring::kBN != 0 || k % (kBK * ring::kUnroll) != 0 || k == 0) return false;
    if (!dma_offsets_fit(ring::kBM, ring::kBN, k, n)) return false;
    return uint64_t(m / ring::kBM) * (n / ring::kBN) >= uint64_t(kCUs);
}

Plan plan_tiles(uint32_t m, uint32_t n, uint32_t k);

// The persistent kernel replaces the tile plans where it fits and K is at
// least 512, when the plan it replaces uses 128x128 or 256x256 tiles (those
// share its tile and its imbalance), or when its grid keeps the CUs busy: the
// busiest CU holds ceil(t / 256) of the t tiles, at most 1/0.9 of the average.
// Measured on MI355X against the tile plans (TFLOP/s): 4096^3 141.6 -> 149.3,
// 4096x11008x4096 138.6 -> 146.4, 5120x5120x2048 127.5 -> 131.9 (256x256
// tiles and a tail before), 4352x4096x1024 110.4 -> 122.7, 2560^3 109.5 ->
// 114.6 (400 tiles), 4608^2x1024 117.2 -> 124.1; over 128x64 tiles 2048^3
// 131.0 -> 138.3 (256 tiles), 4096x1024x2816 131.4 -> 141.2, 4096x2816x1024
// (704) 120.8 -> 129.3, 12288x1024x1024 (768) 132.1 -> 140.6, 1024x4096x4096
// 135.7 -> 145.9. Grids of 384 and 576 tiles lost to the smaller tiles
// (6144x1024x1024 127.5 -> 104.8, 1536x4096x4096 133.3 -> 110.9, 3072^3 on
// 64x64 tiles 118.0 -> 111.7), as did K = 256 (one iteration per tile:
// 4096x4096x256 119.6 -> 118.0).
bool ring_takes(uint32_t m, uint32_t n, uint32_t k, const Plan &tiles) {
    if (!ring_fits(m, n, k) || k < 512) return false;
    if (tiles.big || (tiles.tm == 2 && tiles.tn == 2)) return true;
    const uint64_t t = uint64_t(m / ring::kBM) * (n / ring::kBN), rounds = (t + kCUs - 1) / kCUs;
    return 10 * t >= 9 * rounds * uint64_t(kCUs);
}

Plan plan_for(uint32_t m, uint32_t n, uint32_t k) {
    const Plan p = plan_tiles(m, n, k);
    if (!ring_takes(m, n, k, p)) return p;
    Plan r{2, 2, 1, int(k), int(m / ring::kBM), int(n / ring::kBN), false, 0, 0, 1, 0, 0};
    r.ring = true;
    return r;
}

// The plan among the non-persistent kernels.
Plan plan_tiles(uint32_t m, uint32_t n, uint32_t k) {
    if (big_fits(m, n, k)) {
        const int tiles = int((m / big::kBM) * (n / big::kBN));
        if ((4 * tiles) % kSlots == 0 || (4 * tiles) % kSlots >= kSlots / 4)
            return Plan{2, 2, 1, int(k), int(m / 128), int(n / 128), false, 0, 0, 1, 0, 0};
        Plan p{4, 4, 1, int(k), int(m / big::kBM), int(n / big::kBN), true, tiles / kCUs * kCUs, 0, 1, 2, 2};
        tail_tile(tiles - p.big_full, p.tail_tm, p.tail_tn);
        return p;
    }
    const int kchunk = int(((k + kBK - 1) / kBK) * kBK);
    auto grid = [&](int tm, int tn) {
        return Plan{tm, tn, 1, kchunk, int((m + 64 * tm - 1) / (64 * tm)), int((n + 64 * tn - 1) / (64 * tn)), false,
                    0, 0, 1, 0, 0};
    };
    const int shapes[3][2] = {{2, 2}, {2, 1}, {1, 1}};
    const double eff[3] = {1.00, 0.97, 0.90};
    int best = -1;
    double best_score = 0.0;
    for (int i = 0; i < 3; ++i) {
        const Plan p = grid(shapes[i][0], shapes[i][1]);
        const int groups = p.tiles_m * p.tiles_n;
        if (groups < kMinGroups) continue;
        const int rounds = (groups + kSlots - 1) / kSlots;
        const double score = eff[i] * double(groups) / double(kSlots * rounds);
        if (score > best_score) best = i, best_score = score;
    }
    Plan p = grid(1, 1);
    const int t = p.tiles_m * p.tiles_n;
    if (t > kCUs) {
        const int pick = edge_free_choice(m, n, k, best >= 0 ? best : 2);
        return grid(shapes[pick][0], shapes[pick][1]);
    }
    if (t <= kCUs / 2) {
        if (const int g = direct_waves(m, n, k))
            return {1, 1, 1, kchunk, int((m + 31) / 32), int((n + 31) / 32), false, 0, g, 1, 0, 0};
        if (const int g = direct_waves_unaligned(m, n, k))
            return {1, 1, 1, kchunk, int((m + 31) / 32), int((n + 31) / 32), false, 0, g, 1, 0, 0, true};
    }
    if (const int s = skinny_slices(m, n, k))
        return {1, 1, s, int(k / s), 1, int((n + 31) / 32), false, 0, 4, 1, 0, 0};
    if (t <= kCUs / 2) {
        const int want = (kSplitTarget + t - 1) / t;
        const int most = int(k / kMinChunk);
        p.slices = std::max(1, std::min(want, most));
        if (p.slices > 1) {
            const int chunk = int((k + p.slices - 1) / p.slices);
            p.kchunk = ((chunk + kBK - 1) / kBK) * kBK;
            p.slices = int((k + p.kchunk - 1) / p.kchunk);
        }
    }
    if (p.kchunk >= 2 * kBK) p.kgroups = 2;
    const bool rows16 = k % 4 == 0 && n % 4 == 0;
    // Unaligned rows whose K is whole stages that four groups split evenly
    // (plus at most kMaxTail last k, added in the epilogue) load straight
    // into LDS; there four groups beat two from K = 512 (1000x777x513 13.20
    // -> 12.88 us, 1000x1000x513 13.43 -> 13.09, 1000x777x512 12.40 ->
    // 12.31), while aligned rows keep two below kFourGroupMinK (1024x832x512
    // 11.43 against 11.70 with four).
    const bool whole4 = !rows16 && k >= 512 && (k / kBK) % 4 == 0 && k % kBK <= uint32_t(kMaxTail);
    if (p.slices == 1 && (p.kchunk >= kFourGroupMinK || whole4) && (rows16 || unaligned_buffers_fit(m, n, k)))
        p.kgroups = 4;
    return p;
}

// The 4-wave kernel's load path for a launch: LDS-direct for every tile when
// all are interior, aligned and within the 32-bit offsets; a per-tile choice
// when only some are interior; register-staged otherwise. K ranges with a
// partial stage (K at least kBufAllMinK, and no epilogue tail) take the
// masked buffer-load loop for every tile instead of the register-staged one.
// Measured against it (us): 3000^3 535.0 -> 484.3, 1000^3 23.37 -> 21.58,
// 2000x2000x1000 78.1 -> 73.1, 2500^3 338.5 -> 321.4, 1000x776x548 15.04 ->
// 14.25, 1000x1000x300 10.14 -> 9.77; at K = 100 it lost (6.05 -> 6.18).
// Unaligned K (a run straddling the range's end is zeroed past it in LDS):
// 3000x3000x3001 535.4 -> 503.6, 1000x777x1027 25.48 -> 24.47,
// 2048x2048x2047 145.5 -> 142.3, 4095x4097x4093 1300 -> 1273; with two K
// groups it lost (1000x777x700 16.23 -> 16.71, 1000x777x300 9.31 -> 9.53),
// so those keep the register-staged loop.
constexpr uint32_t kBufAllMinK = 256;
bool ktail_fits(const Plan &p, bool vec, int kg, uint32_t k);
Path tile_path(const Plan &p, bool vec, uint32_t m, uint32_t n, uint32_t k, int tm, int tn, int kg) {
    {
        const uint32_t chunk = uint32_t(p.kchunk), last = k - (uint32_t(p.slices) - 1) * chunk;
        const bool whole = chunk % (kBK * kg) == 0 && last % (kBK * kg) == 0;
        if (!whole && !ktail_fits(p, vec, kg, k) && k >= kBufAllMinK && (k % 4 == 0 || kg != 2) &&
            (uint64_t(m) + 64u * tm) * uint64_t(k) * 4u < (uint64_t(1) << 31) &&
            (uint64_t(k) + 1) * uint64_t(n) * 4u + 64u * tn * 4u < (uint64_t(1) << 31))
            return kBufAll;
    }
    if (!vec)  // unaligned: no tile takes the LDS-direct loads
        return unaligned_buffers_fit(m, n, k) && tm * tn <= 2 ? kUnalignedBuf : kMixed;
    if (!dma_offsets_fit(uint32_t(64 * tm), uint32_t(64 * tn), k, n)) return kRegOnly;
    // Every K slice (the last may be shorter) must be a multiple of KG whole stages.
    const uint32_t chunk = uint32_t(p.kchunk), last = k - (uint32_t(p.slices) - 1) * chunk;
    const bool all_interior = m % (64 * tm) == 0 && n % (64 * tn) == 0 && chunk % (kBK * kg) == 0 &&
                              last % (kBK * kg) == 0;
    return all_interior ? kDmaOnly : kMixed;
}

// Whether gemm_f32_mfma has an instantiation for a tile of tm x tn MFMA
// blocks per wave, kg K groups and a load path. The host instantiates
// 64x64, 128x64 and 128x128 tiles with one group and 64x64 tiles with two or
// four; the buffer-load unaligned loop exists for tiles of at most two blocks
// per wave, and the clamped unaligned loop for at most two K groups.
bool tile_instantiated(int tm, int tn, int kg, Path path, bool vec) {
    const bool shape = kg == 1 ? ((tm == 1 && tn == 1) || (tm == 2 && tn == 1) || (tm == 2 && tn == 2))
                               : (tm == 1 && tn == 1 && (kg == 2 || kg == 4));
    if (!shape) return false;
    switch (path) {
        case kDmaOnly:
        case kRegOnly: return vec;
        case kUnalignedBuf: return !vec && tm * tn <= 2;
        case kMixed: return vec || kg <= 2;
        case kBufAll: return true;
    }
    return false;
}

// The launch gemm_f32 makes for one product shape: its plan and, for the
// four-wave tile kernel, the K-group count and load path. gemm_f32 and
// gemm_f32_shape both take their decision from here, so the kernel a
// description names is the one that runs. `launchable` is false only where
// no instantiation fits; gemm_f32 then returns hipErrorInvalidValue instead
// of launching nothing.
struct Route {
    Plan plan;
    bool vec;              // rows of A and B are 16-byte runs (k % 4 == 0, n % 4 == 0)
    int kg;                // tile kernel: K groups
    Path path;             // tile kernel: load path
    bool launchable;
    bool needs_workspace;  // split-K partials go through the caller's workspace
    bool ktail;            // tile kernel: the last k add in the epilogue (ktail_fits)
};

// Unaligned K-group tiles (the register-staged loop, at most two blocks per
// wave) over an unsplit K: whether K is whole stages that the KG groups split
// evenly plus 1..kMaxTail k, which gemm_f32_mfma's KTAIL variant adds in its
// epilogue instead of in a round of its own. Split plans keep the partial
// stage in the loop: their last slice is never the longest, so the tail
// would not shorten the launch (200x8x1025 measured 9.9 -> 10.4 us with it).
bool ktail_fits(const Plan &p, bool vec, int kg, uint32_t k) {
    const uint32_t whole = k / kBK, rest = k % kBK;
    return !vec && kg > 1 && p.tm * p.tn <= 2 && p.slices == 1 && whole > 0 && whole % uint32_t(kg) == 0 &&
           rest > 0 && rest <= uint32_t(kMaxTail);
}

Route route_for(uint32_t m, uint32_t n, uint32_t k) {
    Route r{plan_for(m, n, k), k % 4 == 0 && n % 4 == 0, 1, kMixed, m > 0 && n > 0 && k > 0, false, false};
    const Plan &p = r.plan;
    r.needs_workspace = p.slices > 1;
    if (p.big || p.ring) {
        r.launchable = r.launchable && r.vec;  // big_fits / ring_fits imply n % 128 == 0 and k % 32 == 0
        return r;
    }
    if (p.direct) {
        r.launchable = r.launchable && (k % 4 == 0 ? (p.slices == 1 || p.direct == 4) : (p.bufa && p.slices == 1));
        return r;
    }
    // A four-group plan whose loads would take the clamped global loads
    // (operands of 2 GiB or more with unaligned rows) runs two groups.
    r.kg = p.kgroups == 4 && (r.vec || unaligned_buffers_fit(m, n, k)) ? 4 : p.kgroups >= 2 ? 2 : 1;
    r.path = tile_path(p, r.vec, m, n, k, p.tm, p.tn, r.kg);
    r.launchable = r.launchable && tile_instantiated(p.tm, p.tn, r.kg, r.path, r.vec);
    r.ktail = r.launchable && ktail_fits(p, r.vec, r.kg, k);
    return r;
}

template <int TM, int TN, int KG, Path PATH, bool VEC, bool KTAIL = false>
hipError_t launch_instance(hipStream_t stream, const Plan &p, dim3 grid, dim3 block, const float *a, const float *b,
                           float *out, uint32_t m, uint32_t n, uint32_t k, const PairArgs &pair) {
    hipLaunchKernelGGL((gemm_f32_mfma<TM, TN, VEC, PATH, KG, KTAIL>), grid, block, 0, stream, a, b, out, int(m),
                       int(n), int(k), p.tiles_m, p.tiles_n, p.kchunk, -1, pair);
    return hipGetLastError();
}

// Unaligned tiles with TM x TN blocks per wave and KG groups, with or without
// the epilogue tail.
template <int TM, int TN, int KG, Path PATH>
hipError_t launch_unaligned(hipStream_t stream, const Route &r, dim3 grid, dim3 block, const float *a, const float *b,
                            float *out, uint32_t m, uint32_t n, uint32_t k, const PairArgs &pair) {
    if constexpr (KG > 1 && TM * TN <= 2)
        if (r.ktail)
            return launch_instance<TM, TN, KG, PATH, false, true>(stream, r.plan, grid, block, a, b, out, m, n, k,
                                                                 pair);
    return launch_instance<TM, TN, KG, PATH, false>(stream, r.plan, grid, block, a, b, out, m, n, k, pair);
}

// Launches the four-wave tile kernel for the route's (path, vec) on a
// TM x TN x KG instantiation; hipErrorInvalidValue when that combination has
// no instantiation (tile_instantiated).
template <int TM, int TN, int KG = 1>
hipError_t launch_tile(hipStream_t stream, const Route &r, const float *a, const float *b, float *out, uint32_t m,
                       uint32_t n, uint32_t k, PairArgs pair = PairArgs{}) {
    const Plan &p = r.plan;
    if (!tile_instantiated(TM, TN, KG, r.path, r.vec)) return hipErrorInvalidValue;
    const unsigned groups = unsigned(p.tiles_m) * unsigned(p.tiles_n) * (pair.tiles > 0 ? 2u : 1u);
    const dim3 grid(groups, unsigned(p.slices)), block(kThreads * KG);
    switch (r.path) {
        case kDmaOnly: return launch_instance<TM, TN, KG, kDmaOnly, true>(stream, p, grid, block, a, b, out, m, n, k, pair);
        case kRegOnly: return launch_instance<TM, TN, KG, kRegOnly, true>(stream, p, grid, block, a, b, out, m, n, k, pair);
        case kUnalignedBuf:
            if constexpr (TM * TN <= 2)
                return launch_unaligned<TM, TN, KG, kUnalignedBuf>(stream, r, grid, block, a, b, out, m, n, k, pair);
            break;
        case kBufAll:
            if (r.vec) return launch_instance<TM, TN, KG, kBufAll, true>(stream, p, grid, block, a, b, out, m, n, k, pair);
            return launch_instance<TM, TN, KG, kBufAll, false>(stream, p, grid, block, a, b, out, m, n, k, pair);
        case kMixed:
            if (r.vec) return launch_instance<TM, TN, KG, kMixed, true>(stream, p, grid, block, a, b, out, m, n, k, pair);
            if constexpr (KG <= 2)
                return launch_unaligned<TM, TN, KG, kMixed>(stream, r, grid, block, a, b, out, m, n, k, pair);
            break;
    }
    return hipErrorInvalidValue;
}

// The tile kernel instantiation the route names (one group: 64x64, 128x64,
// 128x128; two or four groups: 64x64).
hipError_t launch_route_tiles(hipStream_t stream, const Route &r, const float *a, const float *b, float *out,
                              uint32_t m, uint32_t n, uint32_t k, PairArgs pair = PairArgs{}) {
    const Plan &p = r.plan;
    if (r.kg == 4) return launch_tile<1, 1, 4>(stream, r, a, b, out, m, n, k, pair);
    if (r.kg == 2) return launch_tile<1, 1, 2>(stream, r, a, b, out, m, n, k, pair);
    if (p.tm == 2 && p.tn == 2) return launch_tile<2, 2>(stream, r, a, b, out, m, n, k, pair);
    if (p.tm == 2 && p.tn == 1) return launch_tile<2, 1>(stream, r, a, b, out, m, n, k, pair);
    if (p.tm == 1 && p.tn == 1) return launch_tile<1, 1>(stream, r, a, b, out, m, n, k, pair);
    return hipErrorInvalidValue;
}

bool aligned16(const void *p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

}  // namespace

size_t gemm_f32_workspace_bytes(uint32_t m, uint32_t n, uint32_t k) {
    const Route r = route_for(m, n, k);
    return r.needs_workspace ? size_t(r.plan.slices) * m * n * sizeof(float) : 0;
}

LaunchShape gemm_f32_shape(uint32_t m, uint32_t n, uint32_t k) {
    const Route r = route_for(m, n, k);
    const Plan &p = r.plan;
    if (!r.launchable) return {nullptr, {0, 0, 0}, {0, 0, 0}, 0};
    if (p.ring)
        return {"gemm_f32_ring_128x128x32",
                {uint32_t(std::min(p.tiles_m * p.tiles_n, kCUs)), 1, 1},
                {ring::kThreads, 1, 1},
                ring::kLdsBytes};
    if (p.big) {  // the first launch; a partial last round follows as smaller tiles
        const char *name = "gemm_f32_mfma_256x256x32";
        if (p.big_full < p.tiles_m * p.tiles_n)
            name = p.tail_tm == 1 ? "gemm_f32_mfma_256x256x32_tail64x64" : "gemm_f32_mfma_256x256x32_tail128x128";
        return {name, {uint32_t(p.big_full), 1, 1}, {big::kThreads, 1, 1}, big::kLdsBytes};
    }
    if (p.direct) {
        static const char *names[3] = {"gemm_f32_direct_32x32x32_w1", "gemm_f32_direct_32x32x32_w2",
                                       "gemm_f32_direct_32x32x32_w4"};
        static const char *buf_names[3] = {"gemm_f32_direct_32x32x32_w1_buf", "gemm_f32_direct_32x32x32_w2_buf",
                                           "gemm_f32_direct_32x32x32_w4_buf"};
        static const char *lds_names[3] = {"gemm_f32_direct_lds_32x32x32_w1", "gemm_f32_direct_lds_32x32x32_w2",
                                           "gemm_f32_direct_lds_32x32x32_w4"};
        const int w = p.direct == 4 ? 2 : p.direct - 1;
        if (p.slices == 1 && !p.bufa && direct_lds_fits(m, n, k, p.tiles_m * p.tiles_n))
            return {lds_names[w], {uint32_t(p.tiles_m * p.tiles_n), 1, 1}, {uint32_t(64 * p.direct), 1, 1},
                    direct_lds_bytes(p.direct, int((k + kBK - 1) / kBK))};
        return {p.slices > 1 ? "gemm_f32_direct_32x32x32_w4_splitk" : p.bufa ? buf_names[w] : names[w],
                {uint32_t(p.tiles_m * p.tiles_n), uint32_t(p.slices), 1},
                {uint32_t(64 * p.direct), 1, 1},
                uint32_t((p.direct > 1 ? p.direct : 1) * 16 * 64 * sizeof(float))};  // gemm_f32_direct's red[]
    }
    // Otherwise 128x128, 128x64 or 64x64 tiles; only 64x64 tiles split K or
    // run K groups.
    const uint32_t epilogue_k = r.ktail ? k % kBK : 0;
    if (r.kg == 4)
        return {"gemm_f32_mfma_64x64x32_k4", {uint32_t(p.tiles_m * p.tiles_n), 1, 1}, {4 * kThreads, 1, 1},
                4 * Tile<1, 1>::kLdsBytes, epilogue_k};
    if (r.kg == 2)
        return {p.slices > 1 ? "gemm_f32_mfma_64x64x32_splitk_k2" : "gemm_f32_mfma_64x64x32_k2",
                {uint32_t(p.tiles_m * p.tiles_n), uint32_t(p.slices), 1},
                {2 * kThreads, 1, 1},
                2 * Tile<1, 1>::kLdsBytes,
                epilogue_k};
    const int shape = p.tm == 2 ? (p.tn == 2 ? 2 : 1) : 0;
    static const char *names[3][2] = {{"gemm_f32_mfma_64x64x32", "gemm_f32_mfma_64x64x32_splitk"},
                                      {"gemm_f32_mfma_128x64x32", "gemm_f32_mfma_128x64x32_splitk"},
                                      {"gemm_f32_mfma_128x128x32", "gemm_f32_mfma_128x128x32_splitk"}};
    static const uint32_t lds_bytes[3] = {Tile<1, 1>::kLdsBytes, Tile<2, 1>::kLdsBytes, Tile<2, 2>::kLdsBytes};
    const uint32_t lds = lds_bytes[shape];
    return {names[shape][p.slices > 1 ? 1 : 0],
            {uint32_t(p.tiles_m * p.tiles_n), uint32_t(p.slices), 1},
            {kThreads, 1, 1},
            lds};
}

bool gemm_f32_pairable(uint32_t m, uint32_t n, uint32_t k) {
    const Route r = route_for(m, n, k);
    return r.launchable && !r.plan.big && !r.plan.ring && !r.plan.direct && r.kg == 1 && r.plan.slices == 1;
}

hipError_t gemm_f32_pair(hipStream_t stream, const float *a0, const float *b0, float *c0, const float *a1,
                         const float *b1, float *c1, uint32_t m, uint32_t n, uint32_t k) {
    if (!gemm_f32_pairable(m, n, k)) return hipErrorInvalidValue;
    if (!aligned16(a0) || !aligned16(b0) || !aligned16(a1) || !aligned16(b1)) return hipErrorInvalidValue;
    const Route r = route_for(m, n, k);
    const PairArgs pair{a1, b1, c1, r.plan.tiles_m * r.plan.tiles_n, nullptr, nullptr};
    return launch_route_tiles(stream, r, a0, b0, c0, m, n, k, pair);
}

bool gemm_f32_residual_fits(uint32_t m, uint32_t n, uint32_t k) {
    const Route r = route_for(m, n, k);
    return r.launchable && !r.plan.big && !r.plan.direct && r.plan.slices == 1;
}

hipError_t gemm_f32_residual(hipStream_t stream, const float *a, const float *b, float *c, const float *residual,
                             float *sum, uint32_t m, uint32_t n, uint32_t k) {
    if (!gemm_f32_residual_fits(m, n, k) || !aligned16(a) || !aligned16(b) || !residual || !sum)
        return hipErrorInvalidValue;
    const Route r = route_for(m, n, k);
    if (r.plan.ring)
        return launch_gemm_ring(stream, a, b, c, n, k, r.plan.tiles_m, r.plan.tiles_n,
                                unsigned(std::min(r.plan.tiles_m * r.plan.tiles_n, kCUs)), residual, sum);
    PairArgs extra{};
    extra.residual = residual;
    extra.sum = sum;
    return launch_route_tiles(stream, r, a, b, c, m, n, k, extra);
}

bool gemm_f32_dual_swiglu_fits(uint32_t m, uint32_t n, uint32_t k) {
    // The plan each product would take alone must give the fused kernel's
    // bits: the 128x64 tile (paired), or the persistent kernel, whose outputs
    // take the same MFMA steps over k; the fused launch then folds as that
    // plan does (every kFoldStages or ring::kFoldRun stages).
    const Route r = route_for(m, n, k);
    const Plan &p = r.plan;
    const bool same_bits = r.launchable && (p.ring || (gemm_f32_pairable(m, n, k) && p.tm == 2 && p.tn == 1));
    return same_bits && m % dual::T::kBM == 0 && n % dual::T::kBN == 0 && k % kBK == 0 &&
           dma_offsets_fit(dual::T::kBM, dual::T::kBN, k, n);
}

// Tile columns at the right edge that the fused launch runs as 64x64 tiles:
// when a grid of more than one round of 128x64 tiles ends in a partial round
// of at most half the CUs' worth of tiles that fills whole tile columns, those
// columns' tiles run as twice as many 64x64 tiles, so the busiest CU holds
// floor(tiles / CUs) + 1/2 tiles of work instead of floor(tiles / CUs) + 1.
// The MLP's 4096x2816 outputs: 1408 tiles, 128 past five rounds, four
// columns of 32 tiles.
int dual_edge_columns(int tiles_m, int tiles_n) {
    const int tiles = tiles_m * tiles_n, rem = tiles % kCUs;
    if (tiles <= kCUs || rem == 0 || rem > kCUs / 2 || rem % tiles_m != 0) return 0;
    return rem / tiles_m;
}

hipError_t gemm_f32_dual_swiglu(hipStream_t stream, const float *a, const float *bg, const float *bu, float *g,
                                float *u, float *act, uint32_t m, uint32_t n, uint32_t k) {
    if (!gemm_f32_dual_swiglu_fits(m, n, k) || !aligned16(a) || !aligned16(bg) || !aligned16(bu))
        return hipErrorInvalidValue;
    const int tiles_m = int(m / dual::T::kBM), tiles_n = int(n / dual::T::kBN);
    const int edge_n = dual_edge_columns(tiles_m, tiles_n), body_tn = tiles_n - edge_n;
    const unsigned grid = unsigned(tiles_m * body_tn + 2 * tiles_m * edge_n);
    if (route_for(m, n, k).plan.ring)
        hipLaunchKernelGGL(gemm_f32_dual_swiglu<ring::kFoldRun>, dim3(grid), dim3(dual::kThreads), 0, stream, a, bg,
                           bu, g, u, act, int(n), int(k), tiles_m, tiles_n, body_tn);
    else
        hipLaunchKernelGGL(gemm_f32_dual_swiglu<kFoldStages>, dim3(grid), dim3(dual::kThreads), 0, stream, a, bg,
                           bu, g, u, act, int(n), int(k), tiles_m, tiles_n, body_tn);
    return hipGetLastError();
}

hipError_t gemm_f32_batched_direct(hipStream_t stream, const float *a, const float *b, float *c, uint32_t m,
                                   uint32_t n, uint32_t k, uint32_t batch, size_t sa, size_t sb, size_t sc) {
    if (k % 4 != 0 || ((reinterpret_cast<uintptr_t>(a) | sa * sizeof(float)) & 15u) != 0) return hipErrorInvalidValue;
    const int tiles_m = int((m + 31) / 32), tiles_n = int((n + 31) / 32);
    return launch_direct(stream, dim3(unsigned(tiles_m * tiles_n), batch), 4, false, a, b, c, int(m), int(n), int(k),
                         int(k), tiles_m, tiles_n, sa, sb, sc);
}

hipError_t gemm_f32(hipStream_t stream, const float *a, const float *b, float *c, uint32_t m, uint32_t n,
                    uint32_t k, float *workspace) {
    // Operands are whole device regions (256-byte aligned); the kernels'
    // 16-byte loads rely on the base alignment.
    if (!aligned16(a) || !aligned16(b)) return hipErrorInvalidValue;
    const Route r = route_for(m, n, k);
    if (!r.launchable || (r.needs_workspace && !workspace)) return hipErrorInvalidValue;
    const Plan &p = r.plan;
    if (p.ring) {
        return launch_gemm_ring(stream, a, b, c, n, k, p.tiles_m, p.tiles_n,
                                unsigned(std::min(p.tiles_m * p.tiles_n, kCUs)));
    }
    if (p.big) {
        hipLaunchKernelGGL(gemm_f32_mfma_256, dim3(unsigned(p.big_full)), dim3(big::kThreads), 0, stream, a, b, c,
                           int(m), int(n), int(k), p.tiles_m, p.tiles_n);
        const int tail = p.tiles_m * p.tiles_n - p.big_full;
        if (tail > 0) {
            const dim3 grid(unsigned(tail * (4 / p.tail_tm) * (4 / p.tail_tn)));
            if (p.tail_tm == 1)
                hipLaunchKernelGGL((gemm_f32_mfma<1, 1, true, kDmaOnly>), grid, dim3(kThreads), 0, stream, a, b, c,
                                   int(m), int(n), int(k), p.tiles_m, p.tiles_n, int(k), p.big_full, PairArgs{});
            else
                hipLaunchKernelGGL((gemm_f32_mfma<2, 2, true, kDmaOnly>), grid, dim3(kThreads), 0, stream, a, b, c,
                                   int(m), int(n), int(k), p.tiles_m, p.tiles_n, int(k), p.big_full, PairArgs{});
        }
        return hipGetLastError();
    }
    if (p.direct) {
        const dim3 grid(unsigned(p.tiles_m * p.tiles_n));
        if (p.slices > 1) {
            // K slices of p.kchunk (which divides K) as a batch of products
            // into the workspace, then the ordered reduce.
            const size_t mn = size_t(m) * n;
            const hipError_t status =
                launch_direct(stream, dim3(grid.x, unsigned(p.slices)), 4, false, a, b, workspace, int(m), int(n),
                              p.kchunk, int(k), p.tiles_m, p.tiles_n, size_t(p.kchunk), size_t(p.kchunk) * n, mn);
            if (status != hipSuccess) return status;
            hipLaunchKernelGGL(splitk_reduce, dim3(unsigned((mn + 1023) / 1024)), dim3(256), 0, stream, workspace, c, mn,
                               p.slices);
            return hipGetLastError();
        }
        if (!p.bufa && direct_lds_fits(m, n, k, p.tiles_m * p.tiles_n))
            return launch_direct_lds(stream, p.direct, a, b, c, int(m), int(n), int(k), p.tiles_m, p.tiles_n);
        return launch_direct(stream, grid, p.direct, p.bufa, a, b, c, int(m), int(n), int(k), int(k), p.tiles_m,
                             p.tiles_n);
    }
    float *out = p.slices > 1 ? workspace : c;
    const hipError_t status = launch_route_tiles(stream, r, a, b, out, m, n, k);
    if (status != hipSuccess || p.slices == 1) return status;
    const size_t mn = size_t(m) * n;
    const unsigned groups = unsigned((mn + 1023) / 1024);
    hipLaunchKernelGGL(splitk_reduce, dim3(groups), dim3(256), 0, stream, workspace, c, mn, p.slices);
    return hipGetLastError();
}

}  // namespace hipk
}  // namespace jade
