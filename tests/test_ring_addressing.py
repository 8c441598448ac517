"""CPU restatement of the persistent 128x128 GEMM's addressing
(gemm_f32_ring in jade-compute_amd/csrc/gemm_ring.hip): the workgroup-to-tile
map covers every tile once and gives every workgroup a run of whole tiles;
each stage's LDS-direct loads fill exactly the A and B regions of their ring
slot, each 16-byte chunk once, from the tile's A rows and B columns at that
stage's k; the MFMA operand reads of every quarter read back the values the
MFMA operand layout needs (A[row][16h + 4q + e], B[16h + 4q + e][2c + j])
from inside the 128 KiB the kernel declares; the epilogue's stores cover the
128x128 tile once. The kernel's index formulas are restated with numpy over
all waves, lanes, loads, quarters and slots."""
import numpy as np
import pytest

BK, BM, BN = 32, 128, 128
DEPTH = 4
A_STAGE_B = BM * BK * 4            # 16 KiB
B_STAGE_B = BK * BN * 4
B_REGION = DEPTH * A_STAGE_B       # B slots from 64 KiB
LDS_BYTES = DEPTH * (A_STAGE_B + B_STAGE_B)
CUS, GROUP_M = 256, 8
TM = 1                             # the launched form: eight waves of 32x64
WAVES, LANES = 8 // TM, 64
LOADS = 32 // WAVES                # one-KiB loads per wave per stage
HALF = LOADS // 2


def swz_a(row):
    return (row >> 1) & 7


def swz_b(row):
    return row & 7


def xcd_order(bid, count):
    per, rem = divmod(count, 8)
    xcd, idx = bid % 8, bid // 8
    return xcd * per + min(xcd, rem) + idx


def grouped_tile(logical, tiles_m, tiles_n):
    span = GROUP_M * tiles_n
    group, inside = divmod(logical, span)
    first = group * GROUP_M
    rows = min(tiles_m - first, GROUP_M)
    return first + inside % rows, inside // rows


@pytest.mark.parametrize("tiles_m,tiles_n", [(32, 32), (32, 86), (16, 16), (40, 40), (34, 32), (96, 8), (32, 22)])
def test_persistent_map_covers_every_tile_once(tiles_m, tiles_n):
    # Workgroup b takes tiles pos(b) + j * G of the grouped order, j < mine:
    # every tile once, and the runs differ in length by at most one tile.
    tiles = tiles_m * tiles_n
    nwg = min(tiles, CUS)
    count, runs = {}, []
    for b in range(nwg):
        pos = xcd_order(b, nwg)
        mine = (tiles - pos + nwg - 1) // nwg
        runs.append(mine)
        for j in range(mine):
            key = grouped_tile(j * nwg + pos, tiles_m, tiles_n)
            count[key] = count.get(key, 0) + 1
    assert len(count) == tiles and set(count.values()) == {1}
    assert max(runs) - min(runs) <= 1 and sum(runs) == tiles


def lane_grid():
    wave = np.arange(WAVES)[:, None, None]
    lane = np.arange(LANES)[None, :, None]
    return wave, lane


@pytest.mark.parametrize("n,k", [(4096, 4096), (11008, 4096), (1024, 2816), (128, 256)])
def test_stage_loads_fill_their_slot_once(n, k):
    # issue_part: A load x of wave w is instruction w * HALF + x (eight
    # 128-byte rows of one KiB), B load x instruction w * HALF + x (two
    # 512-byte rows); lane l writes LDS at M0 + 16 l.
    wave, lane = lane_grid()
    x = np.arange(HALF)[None, None, :]
    inst = wave * HALF + x
    ra = inst * 8 + (lane >> 3)
    ja = (lane & 7) ^ swz_a(ra)
    voa = (ra * k + 4 * ja) * 4                          # bytes from the stage's A base
    rb = inst * 2 + (lane >> 5)
    jb = (lane & 31) ^ swz_b(rb)
    vob = (rb * n + 4 * jb) * 4
    for slot in range(DEPTH):
        a_lds = slot * A_STAGE_B + inst * 1024 + lane * 16
        b_lds = B_REGION + slot * B_STAGE_B + inst * 1024 + lane * 16
        # Each region filled exactly once, 16 bytes per lane.
        assert sorted(a_lds.ravel().tolist()) == list(range(slot * A_STAGE_B, (slot + 1) * A_STAGE_B, 16))
        assert sorted(b_lds.ravel().tolist()) == list(range(B_REGION + slot * B_STAGE_B,
                                                            B_REGION + (slot + 1) * B_STAGE_B, 16))
    # Sources: rows [0, 128) x k [0, 32) of A, rows [0, 32) x columns [0, 128)
    # of B, relative to the stage's bases, each 16-byte chunk once; and the
    # 32-bit offsets stay below 2^31 (dma_offsets_fit).
    a_row, a_col = voa // 4 // k, voa // 4 % k
    assert a_row.min() == 0 and a_row.max() == BM - 1 and a_col.max() <= BK - 4
    assert len(set(zip(a_row.ravel().tolist(), a_col.ravel().tolist()))) == BM * BK // 4
    b_row, b_col = vob // 4 // n, vob // 4 % n
    assert b_row.max() == BK - 1 and b_col.max() <= BN - 4
    assert len(set(zip(b_row.ravel().tolist(), b_col.ravel().tolist()))) == BK * BN // 4
    assert voa.max() < 2 ** 31 and vob.max() < 2 ** 31
    # The physical chunk a lane writes holds logical chunk j ^ swz (A) and
    # j ^ swz (B) of its row: the layout the operand reads undo.
    phys_a = (inst * 1024 + lane * 16) % 128 // 16
    assert np.array_equal(phys_a ^ swz_a(ra), a_col // 4)
    phys_b = (inst * 1024 + lane * 16) % 512 // 16
    assert np.array_equal(phys_b ^ swz_b(rb), b_col // 4)


def test_operand_reads_return_the_mfma_layout():
    # Fill a model of one slot with (row, k) tags through the load layout,
    # then restate read_part: A block i of quarter q is the 16 bytes at
    # aoff[q] + 4096 i + slot * 16K, B row e at boff[q & 1][e] + 4096 (q >> 1)
    # + slot * 16K. Lane (h, c) of wave (wm, wn) must read A[32 (TM wm + i) +
    # c][16h + 4q + e] and B[16h + 4q + e][64 wn + 2c + j].
    lds = np.full(LDS_BYTES // 4, -1, np.int64)
    slot = 2
    for row in range(BM):                    # A: logical chunk j of row at j ^ swz_a(row)
        for kk in range(BK):
            phys = ((kk // 4) ^ swz_a(row)) * 4 + kk % 4
            lds[(slot * A_STAGE_B) // 4 + row * BK + phys] = 1_000_000 + row * 1000 + kk
    for kr in range(BK):                     # B: logical chunk j of row at j ^ swz_b(row)
        for col in range(BN):
            phys = ((col // 4) ^ swz_b(kr)) * 4 + col % 4
            lds[(B_REGION + slot * B_STAGE_B) // 4 + kr * BN + phys] = 2_000_000 + kr * 1000 + col
    for wave in range(WAVES):
        wm, wn = wave >> 1, wave & 1
        for lane in range(LANES):
            h, c = lane >> 5, lane & 31
            aoff = [(wm * 32 * TM + c) * 128 + (((4 * h + q) ^ ((c >> 1) & 7)) << 4) for q in range(4)]
            boff = [[B_REGION + (16 * h + 4 * p + e) * 512 + (((wn * 16 + (c >> 1)) ^ (4 * p + e)) << 4)
                     + (c & 1) * 8 for e in range(4)] for p in range(2)]
            for q in range(4):
                for i in range(TM):
                    at = aoff[q] + i * 4096 + slot * A_STAGE_B
                    assert 0 <= at and at + 16 <= B_REGION
                    got = lds[at // 4: at // 4 + 4]
                    row = 32 * (TM * wm + i) + c
                    assert got.tolist() == [1_000_000 + row * 1000 + 16 * h + 4 * q + e for e in range(4)]
                for e in range(4):
                    at = boff[q & 1][e] + (q >> 1) * 4096 + slot * B_STAGE_B
                    assert B_REGION <= at and at + 8 <= LDS_BYTES
                    got = lds[at // 4: at // 4 + 2]
                    kr = 16 * h + 4 * q + e
                    assert got.tolist() == [2_000_000 + kr * 1000 + 64 * wn + 2 * c + j for j in range(2)]


def test_epilogue_covers_the_tile_once():
    # store: lane (h, c) of wave (wm, wn) writes rows 32 (TM wm + i) + 8 (v >> 2)
    # + 4h + (v & 3), columns 64 wn + 2c + j of the tile.
    seen = {}
    for wave in range(WAVES):
        wm, wn = wave >> 1, wave & 1
        for lane in range(LANES):
            h, c = lane >> 5, lane & 31
            for i in range(TM):
                for v in range(16):
                    row = 32 * (TM * wm + i) + 8 * (v >> 2) + 4 * h + (v & 3)
                    for j in range(2):
                        key = (row, 64 * wn + 2 * c + j)
                        seen[key] = seen.get(key, 0) + 1
    assert len(seen) == BM * BN and set(seen.values()) == {1}


def test_ring_schedule_never_overwrites_a_live_slot():
    # Model of the issue order: the prologue loads stages 0-2, then iteration
    # g loads stage g + 3 into slot (g + 3) % 4, LOADS loads per stage. At the
    # top of iteration g the kernel waits until at most LOADS loads are
    # outstanding (vmcnt counts loads in issue order), then publishes stage
    # g + 1 with the barrier; iteration g reads slot g % 4 and, in its last
    # quarter, stage g + 1's first operands. So stage g + 1 must be complete
    # at that wait, and the slot loaded during iteration g must be neither of
    # the two read then. The prologue waits down to 2 LOADS: stage 0.
    issued = [s for s in range(3) for _ in range(LOADS)]
    assert set(issued[:len(issued) - 2 * LOADS]) == {0}
    for g in range(96):
        complete = issued[:len(issued) - LOADS]       # vmcnt(LOADS)
        assert complete.count(g + 1) == LOADS and (g + 2) not in complete
        loading = (g + 3) % DEPTH
        assert loading not in (g % DEPTH, (g + 1) % DEPTH)
        issued += [g + 3] * LOADS
