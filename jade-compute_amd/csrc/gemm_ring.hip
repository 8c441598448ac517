// FP32 GEMM on persistent 128x128 tiles for large products whose grid
// covers every CU: C[M,N] = A[M,K] * B[K,N], packed row-major, the same
// contract as gemm_f32.hip (src/runtime/ir.rs:21-32). Built as its own
// translation unit so that its MFMAs accumulate in architectural VGPRs
// (-mllvm -amdgpu-mfma-vgpr-form=1 in the Makefile): the fold of a run into
// the running sums then reads the accumulators directly instead of through
// v_accvgpr_read.
#include <type_traits>

#include "gemm_tiles.hpp"

namespace jade {
namespace hipk {
namespace {

// ---- Persistent 128x128 tiles: one workgroup per CU, a four-stage LDS ring ----
// A launch of at most one workgroup per CU; workgroup b takes the tiles
// pos(b), pos(b) + G, pos(b) + 2G, ... of the XCD-grouped order (G workgroups,
// pos the XCD-contiguous position), so each XCD's 32 workgroups work on a
// block of 8 tile rows x 4 tile columns at a time. The workgroup's stages form
// one sequence over all its tiles; stage g+3 is loaded (LDS-direct) into the
// ring while stage g is consumed, so loads run across tile boundaries and the
// epilogue of one tile overlaps the first stage of the next.
//
// Eight waves of 32x64 (two blocks of v_mfma_f32_32x32x2_f32 each, two waves
// per SIMD), 128 KiB of LDS: four 32-deep stages (A regions in the first 64
// KiB, B regions in the second). Per stage:
//  * one barrier, after this wave's loads of stage g+1 have landed: it
//    publishes stage g+1 and retires stage g-1's slot, which stage g+3's loads
//    fill while stage g is consumed, one load after every eight MFMAs;
//  * the operands of quarter q+1 (8 k) are read one after each of quarter q's
//    first MFMAs, and quarter 0 of stage g+1 during quarter 3 of stage g, so
//    no MFMA waits on an LDS read after the barrier;
//  * every LDS operand address is a per-lane constant plus an immediate (12
//    address registers), and the load offsets are per-lane constants plus a
//    uniform base, so the loop carries no VALU address arithmetic;
//  * no branch: every stage issues its loads (past the end of the sequence
//    they re-read the last tile into a slot nothing reads), the load cursor
//    advances by selects, and each tile's first iteration, which stores the
//    previous tile, is a separate instantiation of the eight-stage body.
// Accumulation is the LDS-direct loops' two-level scheme with their MFMA
// order and a longer run: runs of kFoldRun (eight) stages sum in MFMA
// accumulators and are folded into the running sums with VALU adds, where the
// tile loops fold every four stages. The fold of a block sits right before
// that block's first MFMA of the next run. The fused gate/up kernel takes the
// same run length where it stands in for this kernel, so its outputs stay
// bit-identical to this kernel's.
//
// Measured at 4096^3 (TFLOP/s, A/B on one box; the non-persistent 128x128
// kernel ran 141.6): first form, four waves of 64x64 with all of a stage's
// loads at its top, 133.1; loads spread one per eight MFMAs, 136.9; no branch
// in the steady state (the first form carried ~12 branches and ~84 scalar
// instructions per stage), 145.7; operand reads interleaved with the MFMAs
// instead of issued back to back (the waves then waited on the LDS pipe four
// times as long as the library's kernel), 147.4 with four waves and 149.3 with
// eight; runs of eight stages instead of four before each fold (kFoldRun),
// 149.4; each load after the seventh of its eight MFMAs instead of the last,
// 150.5 (identical bits; 4096x11008x4096 -0.7% time, 2048^3 -0.5%).
// Halving the barriers (a timing-only copy without the odd stages' barriers)
// and folding the two waves of a SIMD at different stages (so one
// wave's MFMAs cover the other's fold) were measured and changed nothing.
// Also measured and dropped: raised wave priority over each stage's matrix
// work (s_setprio; 4096^3 913.95 -> 915.15 us, 4096x11008x4096 -0.4%);
// sixteen waves of 32x32 (four per SIMD), 1%
// slower at every shape; 128x256 tiles of 16-deep stages (eight waves of
// 32x128: half the operand reads per MFMA), 4096^3 918.5 -> 929 us.
// Requires M, N multiples of 128, K a multiple of 256 (whole eight-stage
// iterations per tile), 16-byte aligned operands, 32-bit load offsets.
namespace ring_local {
using namespace ring;
static_assert(kUnroll % kFoldRun == 0 && kUnroll % kDepth == 0, "slot and run start are compile-time per stage");

// One quarter of a stage's operands for one lane: a[i] = A[row block i][k
// 16h + 4q + e] at a[i][e]; b[e] = B[k 16h + 4q + e][columns 2c, 2c + 1].
template <int TM>
struct Quarter {
    f32x4 a[TM];
    float2 b[4];
};

// s_waitcnt vmcnt(N), then the workgroup barrier.
template <int N>
__device__ inline void wait_loads_barrier() {
    static_assert(N == 0 || N == 4 || N == 8 || N == 16, "wait counts in use");
    if constexpr (N == 0)
        asm volatile("s_waitcnt vmcnt(0)\n\ts_barrier" ::: "memory");
    else if constexpr (N == 4)
        asm volatile("s_waitcnt vmcnt(4)\n\ts_barrier" ::: "memory");
    else if constexpr (N == 8)
        asm volatile("s_waitcnt vmcnt(8)\n\ts_barrier" ::: "memory");
    else
        asm volatile("s_waitcnt vmcnt(16)\n\ts_barrier" ::: "memory");
}

__device__ inline int uniform(int x) { return __builtin_amdgcn_readfirstlane(x); }
__device__ inline const float *uniform(const float *p) {
    const uint64_t v = reinterpret_cast<uint64_t>(p);
    const uint32_t lo = __builtin_amdgcn_readfirstlane(uint32_t(v)), hi = __builtin_amdgcn_readfirstlane(uint32_t(v >> 32));
    return reinterpret_cast<const float *>((uint64_t(hi) << 32) | lo);
}
}  // namespace ring_local

// TM: MFMA row blocks per wave. A wave computes (32 TM) x 64 of the tile; the
// workgroup has 8 / TM waves as (4 / TM) x 2 (TM = 2: four waves of 64x64,
// one per SIMD; TM = 1: eight waves of 32x64, two per SIMD).
// PAIRS: C is 8-byte aligned, so each lane's two adjacent outputs go out as
// one 8-byte store.
// sum != nullptr: the epilogue also stores sum = C + residual (both [M, N]),
// the stream kernel's FP32 add, so `sum` is bit-identical to an Add launched
// after the product.
template <int TM, bool PAIRS>
__global__ __launch_bounds__(512 / TM) __attribute__((amdgpu_waves_per_eu(3 - TM, 3 - TM))) void gemm_f32_ring(
    const float *__restrict__ A, const float *__restrict__ B, float *__restrict__ C, int N, int K, int tiles_m,
    int tiles_n, const float *__restrict__ residual, float *__restrict__ sum) {
    using namespace ring;
    using namespace ring_local;
    constexpr int kWaves = 8 / TM;
    constexpr int kLoads = 32 / kWaves;      // one-KiB loads per wave per stage (half A, half B)
    constexpr int kMfmas = 4 * TM * 2;       // MFMAs per wave per quarter
    static_assert(kMfmas % 8 == 0 && kLoads == 4 * (kMfmas / 8), "one load per eight MFMAs");
    __shared__ __attribute__((aligned(1024))) char lds[kLdsBytes];
    const int lane = int(threadIdx.x) & 63;
    const int wave = uniform(int(threadIdx.x) >> 6);
    const int h = lane >> 5, c = lane & 31, wm = wave >> 1, wn = wave & 1;
    const int nwg = int(gridDim.x), tiles = tiles_m * tiles_n;
    const int pos = xcd_order(int(blockIdx.x), nwg);
    const int mine = (tiles - pos + nwg - 1) / nwg;  // tiles pos, pos + nwg, ...
    const int nk = K / kBK;
    const uint32_t lds0 = lds_address(lds);

    // Load offsets. A: 16 one-KiB loads of eight 128-byte rows per stage; B:
    // 16 loads of two 512-byte rows; kLoads / 2 of each per wave. The chunk
    // swizzles are the LDS-direct tiles' (swz_a, swz_b).
    constexpr int kHalf = kLoads / 2;
    uint32_t voa[kHalf], vob[kHalf];
#pragma unroll
    for (int i = 0; i < kHalf; ++i) {
        const int inst = wave * kHalf + i;
        const int ra = inst * 8 + (lane >> 3), ja = (lane & 7) ^ swz_a(ra);
        voa[i] = uint32_t((ra * K + 4 * ja) * 4);
        const int rb = inst * 2 + (lane >> 5), jb = (lane & 31) ^ swz_b(rb);
        vob[i] = uint32_t((rb * N + 4 * jb) * 4);
    }
    // Operand addresses. A row 32 (TM wm + i) + c has swizzle ((c >> 1) & 7)
    // for every block, so block i is +4 KiB; quarter q reads logical chunk
    // 4h + q. B row 16h + 4q + e has swizzle 4(q & 1) + e; q >= 2 is +4 KiB.
    uint32_t aoff[4], boff[2][4];
#pragma unroll
    for (int q = 0; q < 4; ++q)
        aoff[q] = uint32_t((wm * 32 * TM + c) * 128 + (((4 * h + q) ^ ((c >> 1) & 7)) << 4));
#pragma unroll
    for (int p = 0; p < 2; ++p)
#pragma unroll
        for (int e = 0; e < 4; ++e)
            boff[p][e] = kBRegion + uint32_t((16 * h + 4 * p + e) * 512 + (((wn * 16 + (c >> 1)) ^ (4 * p + e)) << 4) +
                                             (c & 1) * 8);
    // This lane's first output (row 4h of the wave's rows, column 2c of its
    // columns) relative to a tile's origin; other outputs are rows apart.
    const uint32_t out_lane = uint32_t((wm * 32 * TM + 4 * h) * N + wn * 64 + 2 * c);

    // Block-uniform load cursor: stage dks of the tile whose A rows start at
    // da and B columns at db; nda, ndb are the next tile's (the current
    // one's on the last tile, so that loads issued past the sequence's end,
    // which nothing reads, stay inside A and B).
    int dks = 0;
    const float *da, *db, *nda, *ndb;
    auto tile_origin = [&](int j, int &m0, int &n0) {
        int tm, tn;
        grouped_tile(j * nwg + pos, tiles_m, tiles_n, tm, tn);
        m0 = uniform(tm * kBM);
        n0 = uniform(tn * kBN);
    };
    auto bases = [&](int j, const float *&pa, const float *&pb) {
        int m0, n0;
        tile_origin(j, m0, n0);
        pa = uniform(A + size_t(m0) * size_t(K));
        pb = uniform(B + n0);
    };
    // Load x (A loads first, then B) of the stage at the cursor, into
    // `slot`; the last one advances the cursor, without a branch. A stage's
    // loads are spread one per eight MFMAs through the stage that consumes
    // stage g: a wave that issued them all at once stalled on the memory pipe
    // while its matrix pipe ran dry.
    auto issue_part = [&](int slot, int x) {
        if (x < kHalf) {
            lds_dma16(da + dks * kBK, voa[x], lds0 + slot * kAStageB + uint32_t((wave * kHalf + x) * 1024));
        } else {
            lds_dma16(db + size_t(dks) * kBK * size_t(N), vob[x - kHalf],
                      lds0 + kBRegion + slot * kBStageB + uint32_t((wave * kHalf + x - kHalf) * 1024));
            if (x == kLoads - 1) {
                const bool wrap = dks + 1 == nk;
                dks = wrap ? 0 : dks + 1;
                da = wrap ? nda : da;
                db = wrap ? ndb : db;
            }
        }
    };
    auto issue_next = [&](int slot) {
#pragma unroll
        for (int x = 0; x < kLoads; ++x) issue_part(slot, x);
    };
    // Read r of a quarter's TM + 4 operand reads (A blocks, then B rows).
    auto read_part = [&](int slot, int q, int r, Quarter<TM> &o) {
        if (r < TM)
            o.a[r] = *reinterpret_cast<const f32x4 *>(lds + aoff[q] + r * 4096 + slot * kAStageB);
        else
            o.b[r - TM] =
                *reinterpret_cast<const float2 *>(lds + boff[q & 1][r - TM] + (q >> 1) * 4096 + slot * kBStageB);
    };
    auto read_quarter = [&](int slot, int q, Quarter<TM> &o) {
#pragma unroll
        for (int r = 0; r < TM + 4; ++r) read_part(slot, q, r, o);
    };

    f32x16 acc[TM][2], part[TM][2];
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
            for (int v = 0; v < 16; ++v) acc[i][j][v] = part[i][j][v] = 0.f;

    // The tile at (m0, n0): row 8(v >> 2) + (v & 3) + 32i of the lane's rows.
    // The origin passes through an empty asm so that no address is computed
    // ahead of the branch that stores (it would hold the addresses in
    // registers over the K loop).
    auto store = [&](int m0, int n0) {
        m0 = uniform(m0);
        n0 = uniform(n0);
        asm volatile("" : "+s"(m0), "+s"(n0));
        const size_t tile = size_t(m0) * size_t(N) + n0;
#pragma unroll
        for (int i = 0; i < TM; ++i)
#pragma unroll
            for (int v = 0; v < 16; ++v) {
                const size_t at = tile + size_t(i * 32 + 8 * (v >> 2) + (v & 3)) * size_t(N) + out_lane;
                const float x0 = acc[i][0][v], x1 = acc[i][1][v];
                if constexpr (PAIRS) {
                    *reinterpret_cast<float2 *>(C + at) = make_float2(x0, x1);
                    if (sum) {  // block-uniform
                        const float2 r = *reinterpret_cast<const float2 *>(residual + at);
                        *reinterpret_cast<float2 *>(sum + at) = make_float2(x0 + r.x, x1 + r.y);
                    }
                } else {
                    C[at] = x0;
                    C[at + 1] = x1;
                    if (sum) {
                        sum[at] = x0 + residual[at];
                        sum[at + 1] = x1 + residual[at + 1];
                    }
                }
            }
    };

    bases(0, da, db);
    bases(mine > 1 ? 1 : 0, nda, ndb);
    issue_next(0);
    issue_next(1);
    issue_next(2);
    wait_loads_barrier<2 * kLoads>();
    Quarter<TM> cur;
    read_quarter(0, 0, cur);
    int m0, n0, pm0 = 0, pn0 = 0;
    tile_origin(0, m0, n0);

    // One stage at position U of an eight-stage iteration. Every stage issues
    // kLoads loads (stage g + 3 of the sequence, or, past its end, data that
    // is never read), so the wait for stage g + 1 is always vmcnt(kLoads),
    // except after FIRST: the first iteration of a tile after another one
    // stores that tile at the end of its stage U = 0, and vmcnt counts those
    // stores too, so stage U = 1 waits for everything.
    auto stage = [&](auto uc, auto fc) __attribute__((always_inline)) {
        constexpr int U = decltype(uc)::value;
        constexpr bool FIRST = decltype(fc)::value;
        constexpr int slot = U % kDepth;
        constexpr bool run_start = U % kFoldRun == 0;
        wait_loads_barrier<(FIRST && U == 1) ? 0 : kLoads>();  // publishes stage g + 1
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            Quarter<TM> nxt;
            const int rslot = q < 3 ? slot : (slot + 1) % kDepth, rq = (q + 1) % 4;
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int e = 0; e < 4; ++e)
#pragma unroll
                for (int i = 0; i < TM; ++i)
#pragma unroll
                    for (int j = 0; j < 2; ++j) {
                        const int n = (e * TM + i) * 2 + j;  // MFMA index in the quarter
                        const float b = j ? cur.b[e].y : cur.b[e].x;
                        if (run_start && q == 0 && e == 0) {
                            // Fold the previous run's sums of this block, then
                            // restart it from zero.
                            acc[i][j] += part[i][j];
                            part[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(cur.a[i][e], b, f32x16{}, 0, 0, 0);
                            __builtin_amdgcn_sched_barrier(0);
                        } else {
                            part[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(cur.a[i][e], b, part[i][j], 0, 0, 0);
                        }
                        // The next quarter's reads go out one after each of
                        // this quarter's first MFMAs, pinned there (the
                        // scheduler would sink them to their use to save
                        // registers); issued back to back they waited on the
                        // LDS pipe beside the LDS-direct writes.
                        if (n < TM + 4) {
                            __builtin_amdgcn_sched_barrier(0);
                            read_part(rslot, rq, n, nxt);
                            __builtin_amdgcn_sched_barrier(0);
                        }
                        // A load goes out after MFMA 6 of each eight, one
                        // before the group's end: 4096^3 920.8 -> 913.5 us
                        // against the group's last MFMA (after MFMA 5 917.4,
                        // 4 917.8, 3 921.2, 0 919.5). Moving the operand
                        // reads instead (one MFMA later, spread over the
                        // quarter, or B rows first) changed nothing (0.2%).
                        if (n % 8 == 6) {
                            __builtin_amdgcn_sched_barrier(0);
                            issue_part((U + 3) % kDepth, q * (kMfmas / 8) + n / 8);
                            __builtin_amdgcn_sched_barrier(0);
                        }
                    }
            __builtin_amdgcn_sched_barrier(0);
            cur = nxt;
        }
        if constexpr (FIRST && U == 0) {
            store(pm0, pn0);
#pragma unroll
            for (int i = 0; i < TM; ++i)
#pragma unroll
                for (int j = 0; j < 2; ++j) acc[i][j] = f32x16{};
        }
    };
    auto iteration = [&](auto fc) __attribute__((always_inline)) {
        stage(std::integral_constant<int, 0>{}, fc);
        stage(std::integral_constant<int, 1>{}, fc);
        stage(std::integral_constant<int, 2>{}, fc);
        stage(std::integral_constant<int, 3>{}, fc);
        stage(std::integral_constant<int, 4>{}, fc);
        stage(std::integral_constant<int, 5>{}, fc);
        stage(std::integral_constant<int, 6>{}, fc);
        stage(std::integral_constant<int, 7>{}, fc);
    };

    for (int j = 0; j < mine; ++j) {
        if (j > 0) {
            pm0 = m0;
            pn0 = n0;
            tile_origin(j, m0, n0);
            // The cursor is in tile j now; its wrap goes to tile j + 1.
            bases(j + 1 < mine ? j + 1 : j, nda, ndb);
            iteration(std::true_type{});
        } else {
            iteration(std::false_type{});
        }
        for (int it = 1; it < nk / kUnroll; ++it) iteration(std::false_type{});
    }
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j) acc[i][j] += part[i][j];
    store(m0, n0);
    // Loads past the sequence's end are still in flight; LDS must not be
    // released under them.
    drain_vmem();
}

// Eight waves of 32x64 (two per SIMD) against four of 64x64: 149.3 against
// 147.4 TFLOP/s at 4096^3, 146.4 against 144.7 at 4096x11008x4096, with the
// interleaved operand reads (bit-identical outputs).
constexpr int kRingTM = 1;
static_assert(512 / kRingTM == ring::kThreads, "the launch's workgroup size");

}  // namespace

hipError_t launch_gemm_ring(hipStream_t stream, const float *a, const float *b, float *c, uint32_t n, uint32_t k,
                            int tiles_m, int tiles_n, unsigned grid, const float *residual, float *sum) {
    constexpr int TM = kRingTM;
    const dim3 block(512 / TM);
    const bool pairs = ((reinterpret_cast<uintptr_t>(c) | reinterpret_cast<uintptr_t>(residual) |
                         reinterpret_cast<uintptr_t>(sum)) & 7u) == 0;
    if (pairs)
        hipLaunchKernelGGL((gemm_f32_ring<TM, true>), dim3(grid), block, 0, stream, a, b, c, int(n), int(k), tiles_m,
                           tiles_n, residual, sum);
    else
        hipLaunchKernelGGL((gemm_f32_ring<TM, false>), dim3(grid), block, 0, stream, a, b, c, int(n), int(k), tiles_m,
                           tiles_n, residual, sum);
    return hipGetLastError();
}

}  // namespace hipk
}  // namespace jade
