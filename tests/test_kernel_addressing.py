"""CPU restatement of the fused gate/up/SwiGLU GEMM's addressing
(gemm_f32_dual_swiglu in jade-compute_amd/csrc/gemm_f32.hip) at the C4 MLP
shape (x[4096x1024], Wg/Wu [1024x2816]) and at the other shapes the fusion
rule admits: every global address the kernel reads or writes, every LDS byte
its LDS-direct loads write, every LDS float its MFMA operand reads and the
U hand-off touch, lies inside its buffer. The kernel's index formulas are
restated with numpy over all lanes, waves, instructions and stages, so a
launch that the fusion rule accepts cannot address memory outside the
bindings or the 64 KiB of LDS it declares."""
import numpy as np
import pytest

BK = 32                    # K per stage
BM, BN = 128, 64           # the gate and up tiles (Tile<2, 1>)
A_STAGE, B_STAGE = BM * BK, BK * BN   # floats per stage, unpadded
STAGE = A_STAGE + 2 * B_STAGE         # A, then B for the gate, then B for the up product
LDS_FLOATS = 2 * STAGE                # two stages: 64 KiB
WAVES, LANES = 8, 64
A_INST = A_STAGE * 4 // 1024 // WAVES          # 1 KiB LDS-direct loads per wave per stage
B_INST = B_STAGE * 4 // 1024 // (WAVES // 2)


def swz_a(row):
    return (row >> 1) & 7


def swz_b(row):
    return row & 7


def stage_loads():
    """(wave, lane, inst) -> global element offsets relative to the A and B
    stage bases, and LDS byte offsets relative to the stage base
    (dual::issue_stage)."""
    wave = np.arange(WAVES)[:, None, None]
    lane = np.arange(LANES)[None, :, None]
    i = np.arange(A_INST)[None, None, :]
    inst = wave * A_INST + i
    row = inst * 8 + (lane >> 3)
    j = (lane & 7) ^ swz_a(row)
    a_rows, a_cols = row, 4 * j                       # A[m0 + row][k0 + 4j .. +3]
    a_lds = inst * 1024 + lane * 16                   # 16 bytes per lane
    chunks = BN // 4
    rows_per = 64 // chunks
    i = np.arange(B_INST)[None, None, :]
    inst_b = (wave & 3) * B_INST + i
    row_b = inst_b * rows_per + lane // chunks
    j_b = (lane % chunks) ^ swz_b(row_b)
    b_rows, b_cols = row_b, 4 * j_b                   # B[k0 + row][n0 + 4j .. +3]
    b_lds = (A_STAGE + (wave >> 2) * B_STAGE) * 4 + inst_b * 1024 + lane * 16
    return (a_rows, a_cols, a_lds), (b_rows, b_cols, b_lds)


def fusable(m, n, k):
    # gemm_f32_dual_swiglu_fits: whole 128x64 tiles and whole stages.
    return m % BM == 0 and n % BN == 0 and k % BK == 0 and k > 0


@pytest.mark.parametrize("m,n,k", [(4096, 2816, 1024), (2048, 2048, 256), (128, 64, 32), (8192, 2816, 4096)])
def test_fused_gate_up_swiglu_stays_in_bounds(m, n, k):
    assert fusable(m, n, k)
    (a_rows, a_cols, a_lds), (b_rows, b_cols, b_lds) = stage_loads()
    # Every A row and every 16-byte A chunk of the 128x32 stage is loaded once;
    # likewise the 32x64 B stage for each product.
    a_cells = set(zip((a_rows).ravel().tolist(), (a_cols // 4).ravel().tolist()))
    assert len(a_cells) == BM * BK // 4 == a_rows.size
    b_cells = set(zip((b_rows).ravel().tolist(), (b_cols // 4).ravel().tolist()))
    assert len(b_cells) == BK * BN // 4 and b_rows.size == 2 * len(b_cells)  # both products
    # LDS writes: 16 bytes per lane inside the stage, both stages inside 64 KiB.
    for u in (0, 1):
        lo = u * STAGE * 4 + np.minimum(a_lds.min(), b_lds.min())
        hi = u * STAGE * 4 + np.maximum(a_lds.max(), b_lds.max()) + 16
        assert lo >= 0 and hi <= LDS_FLOATS * 4
    # Global reads over all tiles and stages: A[m0 + row][k0 + col .. col + 3]
    # and B[k0 + row][n0 + col .. col + 3].
    m0 = np.arange(0, m, BM)
    n0 = np.arange(0, n, BN)
    k0 = np.arange(0, k, BK)
    a_last = (m0.max() + a_rows.max()) * k + k0.max() + a_cols.max() + 3
    b_last = (k0.max() + b_rows.max()) * n + n0.max() + b_cols.max() + 3
    assert a_rows.min() >= 0 and a_cols.min() >= 0 and a_last < m * k
    assert b_rows.min() >= 0 and b_cols.min() >= 0 and b_last < k * n


def test_fused_operand_reads_and_hand_off_stay_in_lds():
    # mma_stage_swz<2, 1> reads of one stage: A rows wm*64 + i*32 + c, chunk
    # (4h + q) ^ swz_a(row); B row 16h + 4q + e, column wn*32 + c through the
    # swizzle; the B stage is the group's (gate or up) one.
    lane = np.arange(LANES)
    h, c = lane >> 5, lane & 31
    worst = 0
    for group in (0, 1):
        for wl in range(4):
            wm, wn = wl >> 1, wl & 1
            for q in range(4):
                for i in range(2):
                    row = wm * 64 + i * 32 + c
                    idx = row * BK + (((4 * h + q) ^ swz_a(row)) << 2)
                    assert idx.min() >= 0 and idx.max() + 4 <= A_STAGE
                for e in range(4):
                    krow = 16 * h + 4 * q + e
                    col = wn * 32 + c
                    idx = A_STAGE + group * B_STAGE + krow * BN + (((col >> 2) ^ swz_b(krow)) << 2) + (col & 3)
                    assert idx.min() >= A_STAGE + group * B_STAGE
                    assert idx.max() < A_STAGE + (group + 1) * B_STAGE
                    worst = max(worst, int(idx.max()) + STAGE)  # second stage buffer
    assert worst < LDS_FLOATS
    # U hand-off: ushare[(i*16 + v)*256 + wl*64 + lane] for the 256 threads of
    # the up group, then the stores G/U/Act[row][col] of each 128x64 tile.
    i = np.arange(2)[:, None, None, None]
    v = np.arange(16)[None, :, None, None]
    wl = np.arange(4)[None, None, :, None]
    ln = lane[None, None, None, :]
    share = (i * 16 + v) * 256 + wl * 64 + ln
    assert share.min() == 0 and share.max() < LDS_FLOATS and np.unique(share).size == share.size
    wm = wl >> 1
    rows = wm * 64 + i * 32 + 8 * (v >> 2) + 4 * (ln >> 5) + (v & 3)
    cols = (wl & 1) * 32 + (ln & 31) + 0 * i * v
    assert rows.min() == 0 and rows.max() == BM - 1 and cols.min() == 0 and cols.max() == BN - 1
    cells = set(zip(np.broadcast_to(rows, share.shape).ravel().tolist(),
                    np.broadcast_to(cols, share.shape).ravel().tolist()))
    assert len(cells) == BM * BN  # every output of the tile written exactly once per product
