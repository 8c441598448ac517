// Device helpers shared by the FP32 GEMM kernels (gemm_f32.hip, gemm_ring.hip)
// and the host interface of the persistent ring kernel.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

namespace jade {
namespace hipk {

// Persistent 128x128 tiles (gemm_ring.hip): shape limits the host planner
// checks before it routes a product there.
namespace ring {
constexpr int kBM = 128, kBN = 128;
constexpr int kDepth = 4;   // 32-deep stages resident in LDS
constexpr int kUnroll = 8;  // stages per loop iteration; K must be a multiple of 32 * kUnroll
constexpr int kThreads = 512;  // eight waves of 32x64
// Stages summed in MFMA accumulators before each fold: eight, where the tile
// loops fold every four. Against four: 4096^3 928 -> 920 us (+0.8%),
// 4096x11008x4096 2648 -> 2620, 4096x1024x2816 164.4 -> 162.9; the worst
// 4096^3 output then uses a third of the 1e-4 + 1e-4|e| tolerance (a fifth
// with four).
constexpr int kFoldRun = 8;
constexpr uint32_t kAStageB = kBM * 32 * 4, kBStageB = 32 * kBN * 4;  // 16 KiB each
constexpr uint32_t kBRegion = kDepth * kAStageB;                      // B stages from 64 KiB
constexpr uint32_t kLdsBytes = kDepth * (kAStageB + kBStageB);        // 128 KiB
}  // namespace ring

// C = A B on the persistent kernel: `grid` workgroups (at most one per CU)
// over a tiles_m x tiles_n grid of 128x128 tiles. With `sum` non-null the
// epilogue also stores sum = C + residual.
hipError_t launch_gemm_ring(hipStream_t stream, const float *a, const float *b, float *c, uint32_t n, uint32_t k,
                            int tiles_m, int tiles_n, unsigned grid, const float *residual = nullptr,
                            float *sum = nullptr);

namespace {

typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

constexpr int kBK = 32;
// Stages whose products the LDS-direct tile loops (and the fused gate/up
// kernel where it stands in for them, which must match them bit for bit) sum
// in MFMA accumulators before each fold into the running sums: 4 stages,
// 128 k. Eight measured 0.5-18% slower on these loops (6144x1024x1024 103.5
// -> 122 us, 3072^3 499 -> 505, 1024x1024x4096 73.2 -> 74.5); the persistent
// kernel folds every ring::kFoldRun stages.
constexpr int kFoldStages = 4;
constexpr int kGroupM = 8;

// ---- LDS-direct staging --------------------------------------------------
// global_load_lds_dwordx4 moves 16 bytes per lane straight from global memory
// into LDS at M0 + lane*16, with no staging registers and no ds_write. It is
// issued through inline asm with a zero immediate offset: the hardware adds
// the immediate to both the global and the LDS address. Both bases are
// wave-uniform and are moved to SGPRs explicitly. The loads are counted by
// vmcnt, which the caller drains before the barrier that publishes a stage.
__device__ inline void lds_dma16(const float *base, uint32_t voff, uint32_t lds_addr) {
    const uint64_t b = reinterpret_cast<uint64_t>(base);
    const uint32_t lo = __builtin_amdgcn_readfirstlane(uint32_t(b));
    const uint32_t hi = __builtin_amdgcn_readfirstlane(uint32_t(b >> 32));
    const float *ub = reinterpret_cast<const float *>((uint64_t(hi) << 32) | lo);
    const uint32_t ul = __builtin_amdgcn_readfirstlane(lds_addr);
    asm volatile("s_mov_b32 m0, %2\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, %1\n" ::"v"(voff), "s"(ub), "s"(ul)
                 : "memory");
}
__device__ inline void drain_vmem() { asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); }
__device__ inline uint32_t lds_address(const void *p) {
    return uint32_t(reinterpret_cast<uintptr_t>((__attribute__((address_space(3))) const void *)p));
}

// Swizzled stage layout: row r of a stage is unpadded and its 16-byte chunk j
// sits at chunk position j ^ swz(r). An A operand read (ds_read_b128) serves 16
// lanes per cycle from 256 bytes of banks; those lanes read 16 consecutive
// 128-byte rows at one logical chunk, and swz_a = (r >> 1) & 7 gives the eight
// even and the eight odd rows eight distinct 16-byte slots each. (r & 7) left
// rows r and r+8 on the same banks: SQ_LDS_BANK_CONFLICT counted 4 cycles per
// read.) B operand reads cover 32 consecutive columns of one row per half-wave,
// which the XOR keeps inside one 128-byte group. Neither read needs padding.
__device__ inline int swz_a(int row) { return (row >> 1) & 7; }
__device__ inline int swz_b(int row) { return row & 7; }

// Position of block `bid` among `count` when each XCD (blocks go round-robin
// over the 8 XCDs by id) owns a contiguous range of positions.
__device__ inline int xcd_order(int bid, int count) {
    const int per = count / 8, rem = count % 8;
    const int xcd = bid % 8, idx = bid / 8;
    return xcd * per + min(xcd, rem) + idx;
}

// Grouped tile order: kGroupM tile rows at a time, column-major inside a group.
__device__ inline void grouped_tile(int logical, int tiles_m, int tiles_n, int &tm, int &tn) {
    const int group_span = kGroupM * tiles_n;
    const int group = logical / group_span;
    const int first_m = group * kGroupM;
    const int group_rows = min(tiles_m - first_m, kGroupM);
    const int in_group = logical - group * group_span;
    tm = first_m + in_group % group_rows;
    tn = in_group / group_rows;
}

}  // namespace
}  // namespace hipk
}  // namespace jade
