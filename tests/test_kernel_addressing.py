"""CPU restatement of the fused gate/up/SwiGLU GEMM's addressing
(gemm_f32_dual_swiglu in jade-compute_amd/csrc/gemm_f32.hip) at the C4 MLP
shape (x[4096x1024], Wg/Wu [1024x2816]) and at the other shapes the fusion
rule admits: every global address the kernel reads or writes, every LDS byte
its LDS-direct loads write, every LDS float its MFMA operand reads and the
U hand-off touch, lies inside its buffer, for both of its tiles (128x64, and
64x64 for the edge columns of a partial last round). The workgroup-to-tile
map covers every output exactly once. The kernel's index formulas are
restated with numpy over all lanes, waves, instructions and stages, so a
launch that the fusion rule accepts cannot address memory outside the
bindings or the 64 KiB of LDS it declares. The tile kernel's buffer loads
into LDS over unaligned rows and over partial stages are checked the same
way: every run that feeds a stored output holds its own row's elements of
the K range, and k outside it reads zero."""
import numpy as np
import pytest

BK = 32                    # K per stage
BN = 64                    # both tiles are 64 columns wide
WAVES, LANES = 8, 64
CUS, GROUP_M = 256, 8
LDS_FLOATS = 2 * (128 * BK + 2 * BK * BN)   # two stages of the 128x64 tile: 64 KiB


def shape(tm):
    """Per-stage sizes of the (64 tm) x 64 tile (dual::Shape<TM>)."""
    bm = 64 * tm
    a_stage, b_stage = bm * BK, BK * BN
    return bm, a_stage, b_stage, a_stage + 2 * b_stage


def swz_a(row):
    return (row >> 1) & 7


def swz_b(row):
    return row & 7


def stage_loads(tm):
    """(wave, lane, inst) -> global element offsets relative to the A and B
    stage bases, and LDS byte offsets relative to the stage base
    (dual::issue_stage<TM>)."""
    bm, a_stage, b_stage, _ = shape(tm)
    a_inst = a_stage * 4 // 1024 // WAVES
    b_inst = b_stage * 4 // 1024 // (WAVES // 2)
    assert a_inst * WAVES * 1024 == a_stage * 4 and b_inst * (WAVES // 2) * 1024 == b_stage * 4
    wave = np.arange(WAVES)[:, None, None]
    lane = np.arange(LANES)[None, :, None]
    i = np.arange(a_inst)[None, None, :]
    inst = wave * a_inst + i
    row = inst * 8 + (lane >> 3)
    j = (lane & 7) ^ swz_a(row)
    a_rows, a_cols = row, 4 * j                       # A[m0 + row][k0 + 4j .. +3]
    a_lds = inst * 1024 + lane * 16                   # 16 bytes per lane
    chunks = BN // 4
    rows_per = 64 // chunks
    i = np.arange(b_inst)[None, None, :]
    inst_b = (wave & 3) * b_inst + i
    row_b = inst_b * rows_per + lane // chunks
    j_b = (lane % chunks) ^ swz_b(row_b)
    b_rows, b_cols = row_b, 4 * j_b                   # B[k0 + row][n0 + 4j .. +3]
    b_lds = (a_stage + (wave >> 2) * b_stage) * 4 + inst_b * 1024 + lane * 16
    return (a_rows, a_cols, a_lds), (b_rows, b_cols, b_lds)


def fusable(m, n, k):
    # gemm_f32_dual_swiglu_fits: whole 128x64 tiles and whole stages.
    return m % 128 == 0 and n % BN == 0 and k % BK == 0 and k > 0


def edge_columns(tiles_m, tiles_n):
    """dual_edge_columns: tile columns that run as 64x64 tiles."""
    tiles = tiles_m * tiles_n
    rem = tiles % CUS
    if tiles <= CUS or rem == 0 or rem > CUS // 2 or rem % tiles_m != 0:
        return 0
    return rem // tiles_m


def xcd_order(bid, count):
    per, rem = count // 8, count % 8
    xcd, idx = bid % 8, bid // 8
    return xcd * per + np.minimum(xcd, rem) + idx


def grouped_tile(logical, tiles_m, tiles_n):
    span = GROUP_M * tiles_n
    group = logical // span
    first = group * GROUP_M
    rows = np.minimum(tiles_m - first, GROUP_M)
    inside = logical - group * span
    return first + inside % rows, inside // rows


def tile_origins(m, n):
    """Workgroup -> (tile height, m0, n0) of the launch (the kernel's blockIdx
    split and the launcher's grid size)."""
    tiles_m, tiles_n = m // 128, n // BN
    edge = edge_columns(tiles_m, tiles_n)
    body_tn = tiles_n - edge
    body = tiles_m * body_tn
    grid = body + 2 * tiles_m * edge
    bid = np.arange(grid)
    out = []
    if body:
        tm, tn = grouped_tile(xcd_order(bid[:body], body), tiles_m, body_tn)
        out += [(2, int(a) * 128, int(b) * 64) for a, b in zip(tm, tn)]
    pos = bid[body:] - body
    if pos.size:
        out += [(1, int(a) * 64, int(b) * 64) for a, b in zip(pos // edge, body_tn + pos % edge)]
    return out, edge


@pytest.mark.parametrize("m,n,expect_edge", [(4096, 2816, 4), (2048, 2048, 0), (128, 64, 0), (8192, 2816, 0),
                                             (1024, 4160, 1), (2048, 2112, 1), (3200, 2816, 0),
                                             (1152, 2880, 0)])
def test_fused_tiles_cover_every_output_once(m, n, expect_edge):
    origins, edge = tile_origins(m, n)
    assert edge == expect_edge
    count = np.zeros((m // 64, n // 64), dtype=np.int64)
    for tm, m0, n0 in origins:
        assert m0 % 64 == 0 and n0 % 64 == 0 and m0 + 64 * tm <= m and n0 + BN <= n
        count[m0 // 64:m0 // 64 + tm, n0 // 64] += 1
    assert (count == 1).all()
    if edge:
        # The busiest CU's work drops from ceil(tiles / CUs) to floor + 1/2.
        tiles = (m // 128) * (n // BN)
        half = sum(1 for tm, _, _ in origins if tm == 1)
        assert half == 2 * (tiles % CUS) and half <= CUS


@pytest.mark.parametrize("tm", [2, 1])
@pytest.mark.parametrize("m,n,k", [(4096, 2816, 1024), (2048, 2048, 256), (128, 64, 32), (8192, 2816, 4096)])
def test_fused_gate_up_swiglu_stays_in_bounds(m, n, k, tm):
    assert fusable(m, n, k)
    bm, a_stage, b_stage, stage = shape(tm)
    (a_rows, a_cols, a_lds), (b_rows, b_cols, b_lds) = stage_loads(tm)
    # Every A row and every 16-byte A chunk of the stage is loaded once;
    # likewise the 32x64 B stage for each product.
    a_cells = set(zip((a_rows).ravel().tolist(), (a_cols // 4).ravel().tolist()))
    assert len(a_cells) == bm * BK // 4 == a_rows.size
    b_cells = set(zip((b_rows).ravel().tolist(), (b_cols // 4).ravel().tolist()))
    assert len(b_cells) == BK * BN // 4 and b_rows.size == 2 * len(b_cells)  # both products
    # LDS writes: 16 bytes per lane inside the stage, both stages inside 64 KiB.
    for u in (0, 1):
        lo = u * stage * 4 + np.minimum(a_lds.min(), b_lds.min())
        hi = u * stage * 4 + np.maximum(a_lds.max(), b_lds.max()) + 16
        assert lo >= 0 and hi <= (u + 1) * stage * 4 <= LDS_FLOATS * 4
    # Global reads over every tile origin of this height and all stages:
    # A[m0 + row][k0 + col .. col + 3] and B[k0 + row][n0 + col .. col + 3].
    origins, _ = tile_origins(m, n)
    m0 = np.array([o[1] for o in origins if o[0] == tm] or [0])
    n0 = np.array([o[2] for o in origins if o[0] == tm] or [0])
    k0 = np.arange(0, k, BK)
    a_last = (m0.max() + a_rows.max()) * k + k0.max() + a_cols.max() + 3
    b_last = (k0.max() + b_rows.max()) * n + n0.max() + b_cols.max() + 3
    assert a_rows.min() >= 0 and a_cols.min() >= 0 and a_last < m * k
    assert b_rows.min() >= 0 and b_cols.min() >= 0 and b_last < k * n


@pytest.mark.parametrize("tm", [2, 1])
def test_fused_operand_reads_and_hand_off_stay_in_lds(tm):
    # mma_stage_swz<TM, 1> reads of one stage: A rows wm*32*TM + i*32 + c,
    # chunk (4h + q) ^ swz_a(row); B row 16h + 4q + e, column wn*32 + c
    # through the swizzle; the B stage is the group's (gate or up) one.
    bm, a_stage, b_stage, stage = shape(tm)
    lane = np.arange(LANES)
    h, c = lane >> 5, lane & 31
    worst = 0
    for group in (0, 1):
        for wl in range(4):
            wm, wn = wl >> 1, wl & 1
            for q in range(4):
                for i in range(tm):
                    row = wm * 32 * tm + i * 32 + c
                    idx = row * BK + (((4 * h + q) ^ swz_a(row)) << 2)
                    assert idx.min() >= 0 and idx.max() + 4 <= a_stage
                for e in range(4):
                    krow = 16 * h + 4 * q + e
                    col = wn * 32 + c
                    idx = a_stage + group * b_stage + krow * BN + (((col >> 2) ^ swz_b(krow)) << 2) + (col & 3)
                    assert idx.min() >= a_stage + group * b_stage
                    assert idx.max() < a_stage + (group + 1) * b_stage
                    worst = max(worst, int(idx.max()) + stage)  # second stage buffer
    assert worst < LDS_FLOATS
    # U hand-off: ushare[(i*16 + v)*256 + wl*64 + lane] for the 256 threads of
    # the up group, then the stores G/U/Act[row][col] of each tile.
    i = np.arange(tm)[:, None, None, None]
    v = np.arange(16)[None, :, None, None]
    wl = np.arange(4)[None, None, :, None]
    ln = lane[None, None, None, :]
    share = (i * 16 + v) * 256 + wl * 64 + ln
    assert share.min() == 0 and share.max() < LDS_FLOATS and np.unique(share).size == share.size
    wm = wl >> 1
    rows = wm * 32 * tm + i * 32 + 8 * (v >> 2) + 4 * (ln >> 5) + (v & 3)
    cols = (wl & 1) * 32 + (ln & 31) + 0 * i * v
    assert rows.min() == 0 and rows.max() == bm - 1 and cols.min() == 0 and cols.max() == BN - 1
    cells = set(zip(np.broadcast_to(rows, share.shape).ravel().tolist(),
                    np.broadcast_to(cols, share.shape).ravel().tolist()))
    assert len(cells) == bm * BN  # every output of the tile written exactly once per product


def tile_col(tn, wn, j, c):
    """gemm_f32.hip tile_col<TN>: a lane's output column in block j."""
    return wn * 64 + 2 * c + j if tn == 2 else wn * 32 * tn + j * 32 + c


@pytest.mark.parametrize("tn", [1, 2])
def test_tile_columns_cover_the_tile_once(tn):
    # Every column of a (64 tn)-wide tile is one lane's output in one block of
    # one wave column, exactly once; with two blocks (the 128x128 tile) a
    # lane's two columns are adjacent and start at an even column, so its B
    # values of a k row are one aligned 8-byte LDS read and its outputs one
    # 8-byte store (N % 4 == 0).
    wn, j, c = np.meshgrid(np.arange(2), np.arange(tn), np.arange(32), indexing="ij")
    cols = tile_col(tn, wn, j, c)
    assert sorted(cols.ravel().tolist()) == list(range(64 * tn))
    if tn == 2:
        assert (cols[:, 1, :] == cols[:, 0, :] + 1).all() and (cols[:, 0, :] % 2 == 0).all()
        # The B read of row krow, column col sits at chunk (col >> 2) ^ swz_b(krow):
        # the 32 lanes of a row read 256 contiguous bytes of one 16-chunk group
        # (all 64 banks once), whatever the row's swizzle.
        for krow in range(32):
            for w in range(2):
                chunks = {((int(x) >> 2) ^ swz_b(krow)) for x in cols[w, 0, :]}
                assert len(chunks) == 16 and len({ch // 16 for ch in chunks}) == 1


# The four-wave tile kernel (gemm_f32_mfma) over unaligned rows: whole
# stages go through issue_stage_buf, 16-byte buffer loads into LDS at
# 4-byte-aligned byte offsets (m0 + row) * K + k0 + 4j for A and
# (k0 + row) * N + n0 + 4j for B, with a range check at M*K*4 and K*N*4.
TILE_WAVES = 4


def tile_buf_loads(tm, tn):
    """(row, first column) of every 16-byte run one 256-thread group loads
    into a stage of the (64 tm) x (64 tn) tile, for A and for B, and the LDS
    byte each run lands at (issue_stage_buf<TM, TN>)."""
    bm, bn = 64 * tm, 64 * tn
    a_inst, b_inst = bm * BK * 4 // 1024 // TILE_WAVES, BK * bn * 4 // 1024 // TILE_WAVES
    wave = np.arange(TILE_WAVES)[:, None, None]
    lane = np.arange(LANES)[None, :, None]
    inst = wave * a_inst + np.arange(a_inst)[None, None, :]
    row = inst * 8 + (lane >> 3)
    a = (row, 4 * ((lane & 7) ^ swz_a(row)), inst * 1024 + lane * 16)
    chunks = bn // 4
    inst = wave * b_inst + np.arange(b_inst)[None, None, :]
    row = inst * (64 // chunks) + lane // chunks
    b = (row, 4 * ((lane % chunks) ^ swz_b(row)), bm * BK * 4 + inst * 1024 + lane * 16)
    return a, b


@pytest.mark.parametrize("m,n,k", [(1000, 777, 513), (1000, 777, 512), (1000, 777, 1025), (777, 1000, 770),
                                   (1000, 1001, 1024), (2000, 1555, 1024), (2048, 2047, 2048),
                                   (3000, 3001, 3008)])
def test_unaligned_whole_stages_load_inside_their_rows(m, n, k):
    """Every run an unaligned whole-stage tile loads for an output that is
    stored holds exactly the A row's or B row's own elements of the group's
    K range; runs for rows past M lie past the end of A (the range check
    returns zero), and B runs past N feed only columns past N. The plan
    (tile, K groups, epilogue k) is the library's own launch description."""
    import jade_hip
    launch = jade_hip.spec_describe({"op": "gemm", "m": m, "n": n, "k": k, "tiled": True})["launch"]
    name = launch["kernel"]
    assert name.startswith("gemm_f32_mfma_") and launch["grid"][1] == 1, name
    dims = name.split("_")[3]
    bm, bn = int(dims.split("x")[0]), int(dims.split("x")[1])
    last = name.split("_")[-1]
    kg = int(last[1:]) if last.startswith("k") else 1
    assert launch["block"][0] == 256 * kg
    kmain = k - launch.get("epilogue_k", 0)
    nk = -(-(-(-kmain // BK)) // kg)
    # The kernel's condition for this loop: whole stages, 32-bit offsets.
    assert kmain == kg * nk * BK
    assert (m + bm) * k * 4 < 2 ** 31 and (k + 1) * n * 4 + bn * 4 < 2 ** 31
    (a_row, a_col, a_lds), (b_row, b_col, b_lds) = tile_buf_loads(bm // 64, bn // 64)
    # Each stage's LDS bytes are written once, A then B.
    lds = np.concatenate([a_lds.ravel(), b_lds.ravel()])
    assert np.array_equal(np.sort(lds), np.arange(0, (bm + bn) * BK * 4, 16))
    m0 = (np.arange(-(-m // bm)) * bm)[:, None, None, None]
    n0 = (np.arange(-(-n // bn)) * bn)[:, None, None, None]
    k0 = (np.arange(kg * nk) * BK)[None, :, None, None]    # every group's stages
    for e in range(4):
        # A: element (m0 + row, k0 + col + e) at float offset (m0 + row) K + k0 + col + e.
        rows, cols = np.broadcast_arrays(m0 + a_row.reshape(1, 1, -1, 1), k0 + a_col.reshape(1, 1, -1, 1) + e)
        off = rows * k + cols
        assert off.max() * 4 < 2 ** 32                      # no 32-bit wrap
        assert (cols[rows < m] < kmain).all()
        assert (off[rows >= m] >= m * k).all()
        # B: element (k0 + row, n0 + col + e) where that column is below N.
        rows, cols = np.broadcast_arrays(k0 + b_row.reshape(1, 1, -1, 1), n0 + b_col.reshape(1, 1, -1, 1) + e)
        off = rows * n + cols
        assert off.max() * 4 < 2 ** 32
        assert rows.max() < kmain
        assert (off[cols < n] < k * n).all()


DEAD = 0x80000000  # kDeadOffset: past every buffer these kernels read


@pytest.mark.parametrize("m,n,k", [(1000, 1000, 1000), (1000, 776, 548), (2000, 1554, 1028), (700, 1300, 292),
                                   (200, 8, 1000), (1024, 512, 1000), (3000, 3000, 3000), (2500, 2500, 2500),
                                   (3000, 3001, 3001), (1000, 777, 1027), (2048, 2048, 2047)])
def test_partial_stages_mask_every_k_outside_the_range(m, n, k):
    """K ranges with a partial stage run every tile through the masked
    buffer loads into LDS: per K slice and group, the live A elements of a
    tile row cover each k of the slice exactly once, every run that starts at
    or past the group's end is aimed past both buffers (kDeadOffset, zero
    from the range check), a run that straddles the end (unaligned K) has
    exactly its k past the end zeroed in LDS, and no live B row reaches past
    the slice, so a split product never reads the next slice's rows. Slices
    come from the library's own launch description."""
    import jade_hip
    launch = jade_hip.spec_describe({"op": "gemm", "m": m, "n": n, "k": k, "tiled": True})["launch"]
    name = launch["kernel"]
    assert name.startswith("gemm_f32_mfma_"), name
    dims = name.split("_")[3]
    bm, bn = int(dims.split("x")[0]), int(dims.split("x")[1])
    last = name.split("_")[-1]
    kg = int(last[1:]) if last.startswith("k") else 1
    slices = launch["grid"][1]
    kchunk = -(-(-(-k // slices)) // BK) * BK
    assert -(-k // kchunk) == slices
    assert (m + bm) * k * 4 < DEAD and (k + 1) * n * 4 + bn * 4 < DEAD
    (a_row, a_col, _), (b_row, b_col, _) = tile_buf_loads(bm // 64, bn // 64)
    a_row, a_col = a_row.ravel(), a_col.ravel()
    b_row, b_col = b_row.ravel(), b_col.ravel()
    partial = False
    for z in range(slices):
        kfirst, klast = z * kchunk, min(k, (z + 1) * kchunk)
        nk = -(-(-(-(klast - kfirst) // BK)) // kg)
        partial |= klast - kfirst != kg * nk * BK
        cover = np.zeros((bm, klast - kfirst), dtype=np.int64)
        for g in range(kg):
            kbegin = kfirst + g * nk * BK
            kend = min(klast, kbegin + nk * BK)
            for s in range(nk):
                k0 = kbegin + s * BK
                ka = k0 + a_col
                live = ka < kend
                # A: live runs start inside [kfirst, klast); their elements
                # below kend cover it once, the rest (a straddling run's tail,
                # K % 4 != 0 only) is what k_loop_dma zeroes in LDS.
                assert (ka[live] >= kfirst).all()
                straddle = live & (ka + 3 >= kend)
                assert k % 4 != 0 or not straddle.any()
                for r, c in zip(a_row[live], ka[live]):
                    hi = min(c + 4, kend)
                    cover[r, c - kfirst:hi - kfirst] += 1
                off = np.where(live, (a_row.astype(np.int64) * k + ka) * 4, DEAD)
                assert (off[~live] == DEAD).all() and off[live].max(initial=0) < DEAD
                # B: live rows below the slice's end, dead rows past both buffers.
                kb = k0 + b_row
                live_b = kb < kend
                assert (kb[live_b] < klast).all()
                offb = np.where(live_b, (kb.astype(np.int64) * n + b_col) * 4, DEAD)
                assert offb[live_b].max(initial=0) < DEAD and (offb[~live_b] == DEAD).all()
        assert (cover == 1).all()
    assert partial  # these shapes take the masked loop
