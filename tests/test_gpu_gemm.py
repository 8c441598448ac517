"""FP32 MFMA GEMM parity against the FP64 oracle.

Cases: the reference's metal-verify GEMM shapes (src/runtime/metal_lab.rs:
400-413, inputs at :135-136, tolerance 5e-5 at :173), the `jade-compute
verify` odd shapes (src/main.rs:250-258, validation::check), its precision
probes (metal_lab.rs:437-461), and the BASELINE configs: 512^3, the
1024/2048/4096 squares and the ragged (1000,777,513) and (4096,11008,4096)
shapes with validation::inputs, gated at |a-e| <= 1e-4 + 1e-4|e|.
"""
import numpy as np
import pytest

import jade_hip
import oracle_binding as orc

pytestmark = pytest.mark.gpu

NORTH_STAR_TOL = 1e-4


def run_gemm(runtime, m, n, k, a, b, spec_op="gemm", repeats=1):
    spec = {"op": spec_op, "m": m, "n": n, "k": k}
    if spec_op == "gemm":
        spec["tiled"] = True
    kernel = runtime.compile(spec)
    ag, bg, out = runtime.resident(a), runtime.resident(b), runtime.alloc(m * n)
    runtime.execute([(kernel, [ag, bg, out])], repeats)
    got = runtime.download(out)
    assert np.array_equal(runtime.download(ag), a, equal_nan=True) and np.array_equal(
        runtime.download(bg), b, equal_nan=True), "input modified"
    for x in (ag, bg, out):
        x.free()
    return got


LAB_SHAPES = [(1, 1, 1), (7, 9, 13), (8, 8, 8), (31, 47, 19), (32, 32, 33), (33, 31, 65), (65, 67, 63),
              (1, 129, 33), (64, 64, 64), (127, 65, 129), (256, 256, 65), (257, 263, 67)]


@pytest.mark.parametrize("m,n,k", LAB_SHAPES)
@pytest.mark.parametrize("op", ["gemm", "gemm_simd"])
def test_lab_gemm_shapes(runtime, m, n, k, op):
    a = orc.values(m * k, 0x1234, 1.0)
    b = orc.values(k * n, 0xABCD, np.float32(1.0) / np.sqrt(np.float32(k)))
    want = orc.gemm_reference(m, n, k, a, b)
    got = run_gemm(runtime, m, n, k, a, b, op, repeats=3)
    check = orc.compare(got, want, 5e-5, 5e-5)
    assert check.status == 0, (check.first_bad, got[check.first_bad], want[check.first_bad])


@pytest.mark.parametrize("m,n,k", [(1, 1, 1), (1, 17, 33), (17, 1, 35), (31, 47, 19), (64, 64, 64), (65, 33, 17),
                                   (3, 5, 257)])
def test_jade_compute_verify_shapes(runtime, m, n, k):
    a, b = orc.inputs(m, n, k)
    got = run_gemm(runtime, m, n, k, a, b)
    result = orc.check_gemm(m, n, k, a, b, got, 1 << 62)
    assert result.status == 0 and result.checked_elements == m * n
    assert orc.compare(got, orc.gemm_reference(m, n, k, a, b), NORTH_STAR_TOL, NORTH_STAR_TOL).status == 0


@pytest.mark.parametrize("a,b", [(1.0001, 1.0003), (70000.25, 1.0000312)])
def test_fp32_precision_probes(runtime, a, b):
    av, bv = np.array([a], np.float32), np.array([b], np.float32)
    for op in ("gemm_simd", "gemm"):
        got = run_gemm(runtime, 1, 1, 1, av, bv, op)
        assert orc.compare(got, [float(av[0]) * float(bv[0])], 1e-5, 1e-6).status == 0


def gate(got, m, n, k, a, b, rows=None, margin=None):
    """Every output (of `rows`) within the north-star tolerance of the FP64
    oracle; with `margin`, the worst output also within that share of it."""
    want = orc.gemm_reference(m, n, k, a, b, rows=rows)
    part = got if rows is None else got[rows[0] * n:rows[1] * n]
    check = orc.compare(part, want, NORTH_STAR_TOL, NORTH_STAR_TOL)
    assert check.status == 0, (check.first_bad, part[check.first_bad], want[check.first_bad])
    if margin is not None:
        e = np.asarray(want, np.float64)
        share = np.abs(np.asarray(part, np.float64) - e) / (NORTH_STAR_TOL + NORTH_STAR_TOL * np.abs(e))
        worst = int(np.argmax(share))
        print(f"worst output {worst}: {share[worst]:.3f} of the tolerance")
        assert share[worst] <= margin, (worst, share[worst])
    return check


@pytest.mark.parametrize("m,n,k", [(512, 512, 512), (1024, 1024, 1024), (2048, 2048, 2048), (1000, 777, 513)])
def test_config_gemm_full_oracle(runtime, m, n, k):
    a, b = orc.inputs(m, n, k)
    got = run_gemm(runtime, m, n, k, a, b)
    gate(got, m, n, k, a, b)
    assert orc.check_gemm(m, n, k, a, b, got, 4096).status == 0


def test_config_gemm_4096_cubed(runtime):
    m = n = k = 4096
    a, b = orc.inputs(m, n, k)
    got = run_gemm(runtime, m, n, k, a, b)
    check = gate(got, m, n, k, a, b, margin=0.5)  # every element, worst at most half the tolerance
    print(f"4096^3 max_abs {check.max_abs_error:.3e} max_rel {check.max_relative_error:.3e}")
    assert orc.check_gemm(m, n, k, a, b, got, 8192).status == 0


def test_config_gemm_llm_shape(runtime):
    m, n, k = 4096, 11008, 4096
    a, b = orc.inputs(m, n, k)
    got = run_gemm(runtime, m, n, k, a, b)
    for rows in ((0, 1024), (1024, 2048), (2048, 3072), (3072, 4096)):
        gate(got, m, n, k, a, b, rows, margin=0.5)
    assert orc.check_gemm(m, n, k, a, b, got, 8192).status == 0


@pytest.mark.parametrize("m,n,k", [(129, 130, 131), (255, 257, 4), (3, 4100, 7), (4100, 3, 9), (128, 128, 1),
                                   (200, 8, 1000), (100, 200, 1000), (100, 200, 999), (1, 1024, 4096),
                                   (4097, 65, 300), (65, 4097, 300), (300, 300, 8192), (4000, 4000, 100),
                                   (4100, 2800, 64), (4100, 2800, 63)])
def test_edge_masking_shapes(runtime, m, n, k):
    # Covers every tile shape (128x128, 128x64, 64x64) with ragged edges, the
    # unaligned (scalar-load) path and split K with ragged and unaligned K slices.
    a = orc.values(m * k, 0x55, 1.0)
    b = orc.values(k * n, 0x66, 1.0)
    got = run_gemm(runtime, m, n, k, a, b)
    gate(got, m, n, k, a, b)


@pytest.mark.parametrize("m,n,k,waves", [(300, 200, 100, 4), (384, 320, 768, 4), (130, 520, 388, 4),
                                          (257, 255, 36, 2), (64, 2048, 96, 2), (255, 257, 4, 1),
                                          (700, 700, 700, 4), (2047, 33, 164, 4), (512, 512, 512, 4),
                                          (256, 256, 20, 1), (500, 300, 740, 4), (33, 4096, 36, 2)])
def test_direct_tile_shapes(runtime, m, n, k, waves):
    # The direct-load 32x32 kernel: ragged M and N (clamped rows and columns that
    # are never stored), a partial last K slice (zeroed past K), one, two and
    # four waves per tile, and per-wave slice counts that leave 0, 1 or 2 slices
    # after the last whole round of three in flight.
    # Grids of at most one tile per CU with 16-byte rows stage each wave's
    # slices through LDS (a ring of four slots: K = 768 reuses two of them).
    kernel = runtime.compile({"op": "gemm", "m": m, "n": n, "k": k, "tiled": True})
    staged = ((m + 31) // 32) * ((n + 31) // 32) <= 256 and k % 4 == 0 and n % 4 == 0
    want = f"gemm_f32_direct_lds_32x32x32_w{waves}" if staged else f"gemm_f32_direct_32x32x32_w{waves}"
    assert kernel.launch["kernel"] == want, kernel.launch
    a = orc.values(m * k, 0x99, 1.0)
    b = orc.values(k * n, 0xAA, 1.0)
    got = run_gemm(runtime, m, n, k, a, b, repeats=2)
    gate(got, m, n, k, a, b)


@pytest.mark.parametrize("m,n,k,waves", [(500, 777, 513, 4), (100, 777, 513, 4), (333, 555, 101, 4),
                                          (777, 300, 255, 4), (250, 300, 35, 2), (300, 300, 1, 1), (4100, 3, 9, 1)])
def test_direct_tiles_over_unaligned_rows(runtime, m, n, k, waves):
    # Small grids with K % 4 != 0 run the direct-load 32x32 kernel with A read
    # through buffer loads at 4-byte-aligned offsets: a run crossing the end of
    # its row reads the next row (zeroed past K), the buffer's range check
    # zeroes runs past the end of A; ragged M and N as for aligned rows.
    kernel = runtime.compile({"op": "gemm", "m": m, "n": n, "k": k, "tiled": True})
    assert kernel.launch["kernel"] == f"gemm_f32_direct_32x32x32_w{waves}_buf", kernel.launch
    assert kernel.description["workspace_bytes"] == 0
    a = orc.values(m * k, 0x9B, 1.0)
    b = orc.values(k * n, 0xAB, 1.0)
    got = run_gemm(runtime, m, n, k, a, b, repeats=2)
    gate(got, m, n, k, a, b)


@pytest.mark.parametrize("m,n,k", [
    (1000, 777, 545),  # 64x64 tiles, two K groups, unaligned rows: the last stage runs 31 k past K
    (1000, 777, 1027),  # four K groups, masked LDS-direct stages: row 4's last run straddles K, zeroed in LDS
    (200, 8, 999),     # K split into slices of 160: a slice's last stage runs into the next slice
    (500, 777, 513),   # direct-load 32x32 tiles over unaligned rows
])
def test_unaligned_rows_keep_non_finite_values_in_place(runtime, m, n, k):
    # Unaligned loops load whole 32-k runs: past the end of a K range they
    # read the next A row's first floats or the next slice's B rows. Those
    # must enter as zeros, so an Inf or NaN there stays in the outputs it
    # belongs to: A[5][0] = Inf (row 4's run past K reads it), A[7][2] = NaN,
    # B[160][3] = Inf (the first row of the second K slice at (200, 8, 999)).
    a = orc.values(m * k, 0xD1, 1.0)
    b = orc.values(k * n, 0xD2, 1.0)
    a[5 * k] = np.inf
    a[7 * k + 2] = np.nan
    b[160 * n + 3] = np.inf
    got = run_gemm(runtime, m, n, k, a, b).reshape(m, n)
    want = orc.gemm_reference(m, n, k, a, b).reshape(m, n)
    rows = np.setdiff1d(np.arange(m), [5, 7])
    cols = np.setdiff1d(np.arange(n), [3])
    clean_got, clean_want = got[np.ix_(rows, cols)], want[np.ix_(rows, cols)]
    assert np.isfinite(clean_got).all()
    check = orc.compare(clean_got.reshape(-1), clean_want.reshape(-1), NORTH_STAR_TOL, NORTH_STAR_TOL)
    assert check.status == 0, check.first_bad
    assert not np.isfinite(got[5]).any() and np.isnan(got[7]).all() and not np.isfinite(got[:, 3]).any()


@pytest.mark.parametrize("m,n,k,kernel", [
    (1000, 777, 513, "gemm_f32_mfma_64x64x32_k4"),  # 16 whole stages, 4 per group; k = 512 in the epilogue
    (1000, 777, 514, "gemm_f32_mfma_64x64x32_k4"),  # two tail k
    (1000, 777, 545, "gemm_f32_mfma_64x64x32_k2"),  # 17 whole stages: the partial stage stays in the loop
    (1000, 777, 769, "gemm_f32_mfma_64x64x32_k4"),  # 24 whole stages over four groups, one tail k
    (1000, 777, 1027, "gemm_f32_mfma_64x64x32_k4"),  # three last k: more than the epilogue takes
    (1000, 777, 65, "gemm_f32_mfma_64x64x32_k2"),  # one whole stage per group, then one k
    (1000, 777, 130, "gemm_f32_mfma_64x64x32_k2"),  # two stages per group, then two k
    (777, 1000, 1025, "gemm_f32_mfma_64x64x32_k4"),  # eight stages per group of four, then one k
    (200, 8, 1025, "gemm_f32_mfma_64x64x32_splitk_k2"),  # split K: the last slice (65 k) keeps its partial stage
    (300, 300, 2049, "gemm_f32_mfma_64x64x32_splitk_k2"),  # last slice of 129 k
])
def test_unaligned_tail_k_in_the_epilogue(runtime, m, n, k, kernel):
    # Unsplit unaligned K-group tiles whose K is whole stages that the groups
    # split evenly plus one or two k add those k in the epilogue, from values
    # loaded before the loop; the other shapes here keep the partial stage in
    # the loop. Either way an Inf or NaN in the last k reaches its own row or
    # column only: A[9][K-1] = NaN, B[K-1][5] = Inf.
    launch = runtime.compile({"op": "gemm", "m": m, "n": n, "k": k, "tiled": True}).launch
    assert launch["kernel"] == kernel, launch
    a = orc.values(m * k, 0xE1, 1.0)
    b = orc.values(k * n, 0xE2, 1.0)
    a[9 * k + k - 1] = np.nan
    b[(k - 1) * n + 5] = np.inf
    got = run_gemm(runtime, m, n, k, a, b, repeats=2).reshape(m, n)
    want = orc.gemm_reference(m, n, k, a, b).reshape(m, n)
    rows = np.setdiff1d(np.arange(m), [9])
    cols = np.setdiff1d(np.arange(n), [5])
    clean_got, clean_want = got[np.ix_(rows, cols)], want[np.ix_(rows, cols)]
    assert np.isfinite(clean_got).all()
    check = orc.compare(clean_got.reshape(-1), clean_want.reshape(-1), NORTH_STAR_TOL, NORTH_STAR_TOL)
    assert check.status == 0, check.first_bad
    assert np.isnan(got[9]).all() and not np.isfinite(got[:, 5]).any()


@pytest.mark.parametrize("m,n,k,kernel", [
    (1000, 777, 512, "gemm_f32_mfma_64x64x32_k4"),  # the last B row's last run crosses the end of B
    (1000, 777, 257, "gemm_f32_mfma_64x64x32_k2"),  # 8 whole stages over two groups, k = 256 in the epilogue
    (1000, 1001, 1024, "gemm_f32_mfma_64x64x32_k4"),
    (2000, 1555, 1024, "gemm_f32_mfma_128x64x32"),
    (777, 1000, 770, "gemm_f32_mfma_64x64x32_k4"),  # K unaligned: 24 whole stages, two k in the epilogue
])
def test_unaligned_whole_stages_through_buffer_loads_into_lds(runtime, m, n, k, kernel):
    # Unaligned rows over whole stages load 16-byte runs at 4-byte-aligned
    # offsets straight into LDS (buffer_load_dwordx4 ... lds): A runs stay in
    # their row, a B run past N reads the next row's first columns (past the
    # end of B, zero from the range check), rows past M read zero.
    launch = runtime.compile({"op": "gemm", "m": m, "n": n, "k": k, "tiled": True}).launch
    assert launch["kernel"] == kernel, launch
    a = orc.values(m * k, 0xB7, 1.0)
    b = orc.values(k * n, 0xC7, 1.0)
    got = run_gemm(runtime, m, n, k, a, b, repeats=2)
    gate(got, m, n, k, a, b)


@pytest.mark.parametrize("m,n,k,kernel", [
    (1000, 1000, 1000, "gemm_f32_mfma_64x64x32_k4"),  # 31 stages and 8 k: the last group's last stage partial
    (1000, 776, 548, "gemm_f32_mfma_64x64x32_k2"),
    (2000, 1554, 1028, "gemm_f32_mfma_128x64x32"),  # N unaligned: B runs past N, K with 4 k in its last stage
    (700, 1300, 292, "gemm_f32_mfma_64x64x32_k2"),
    (3000, 3001, 3001, "gemm_f32_mfma_64x64x32"),  # unaligned K: the last stage's straddling runs zeroed past K
    (1000, 777, 1027, "gemm_f32_mfma_64x64x32_k4"),
    (200, 8, 1000, "gemm_f32_mfma_64x64x32_splitk_k2"),  # slices of 160 k: each slice's last group stage lies
                                                          # in the next slice, whose B rows must read as zero
    (1024, 512, 1000, "gemm_f32_mfma_64x64x32_splitk_k2"),
])
def test_partial_stages_through_masked_buffer_loads(runtime, m, n, k, kernel):
    # K ranges with a partial stage (K % 4 == 0, K >= 256) load every tile's
    # stages straight into LDS through buffer loads; k at or past the range's
    # end is aimed past the buffers and reads zero.
    launch = runtime.compile({"op": "gemm", "m": m, "n": n, "k": k, "tiled": True}).launch
    assert launch["kernel"] == kernel, launch
    a = orc.values(m * k, 0xB9, 1.0)
    b = orc.values(k * n, 0xC9, 1.0)
    got = run_gemm(runtime, m, n, k, a, b, repeats=2)
    rows = None if m * n * k <= 2e9 else (0, 256)
    gate(got, m, n, k, a, b, rows=rows)


@pytest.mark.parametrize("m,n,k,kernel", [
    (1024, 1024, 512, "gemm_f32_mfma_64x64x32_k2"),  # LDS-direct stages, 8 per group
    (1000, 777, 700, "gemm_f32_mfma_64x64x32_k2"),  # unaligned rows, K below the four-group threshold
    (130, 70, 100, "gemm_f32_mfma_64x64x32_k2"),  # 4 stages, the last one partial
    (65, 67, 63, "gemm_f32_mfma_64x64x32_k2"),  # one stage per group
    (100, 100, 40, "gemm_f32_mfma_64x64x32_k2"),  # group 1's stage lies mostly past K
    (1024, 512, 1024, "gemm_f32_mfma_64x64x32_splitk_k2"),
    (200, 8, 1000, "gemm_f32_mfma_64x64x32_splitk_k2"),  # ragged last slice
    (40, 1024, 4096, "gemm_f32_mfma_64x64x32_splitk_k2"),  # over 32 rows: not the skinny plan
])
def test_two_group_tile_shapes(runtime, m, n, k, kernel):
    # 64x64 tiles whose two K groups of four waves sum the two halves of each
    # workgroup's K range and meet in LDS.
    launch = runtime.compile({"op": "gemm", "m": m, "n": n, "k": k, "tiled": True}).launch
    assert launch["kernel"] == kernel, launch
    a = orc.values(m * k, 0xBB, 1.0)
    b = orc.values(k * n, 0xCC, 1.0)
    got = run_gemm(runtime, m, n, k, a, b, repeats=2)
    gate(got, m, n, k, a, b)


@pytest.mark.parametrize("m,n,k", [
    (1024, 1024, 1024),  # LDS-direct stages, 8 per group
    (768, 768, 768),  # 6 stages per group
    (1000, 1000, 1024),  # edge tiles through buffer loads into LDS (16-byte rows), interior LDS-direct
    (1000, 600, 1000),  # 32 stages, the last partial: every tile register-staged
    (768, 768, 2048),  # 16 stages per group
    (1000, 777, 1024),  # unaligned rows through buffer loads into LDS
    (1000, 777, 513),  # unaligned rows into LDS, 4 whole stages per group, k = 512 in the epilogue
    (1023, 1000, 2049),  # unaligned rows, the last group's last stage partial: register-staged
])
def test_four_group_tile_shapes(runtime, m, n, k):
    # 64x64 tiles whose four K groups of four waves each sum a quarter of the
    # workgroup's K range; groups 1-3 leave their sums in LDS and group 0 adds
    # them in group order.
    launch = runtime.compile({"op": "gemm", "m": m, "n": n, "k": k, "tiled": True}).launch
    assert launch["kernel"] == "gemm_f32_mfma_64x64x32_k4" and launch["block"] == [1024, 1, 1], launch
    a = orc.values(m * k, 0xBD, 1.0)
    b = orc.values(k * n, 0xCE, 1.0)
    got = run_gemm(runtime, m, n, k, a, b, repeats=2)
    gate(got, m, n, k, a, b)


@pytest.mark.parametrize("m,n,k,want", [
    (4096, 4096, 32, "gemm_f32_mfma_128x128x32"),  # one stage
    (4096, 4096, 96, "gemm_f32_mfma_128x128x32"),  # odd stage count: the last two-stage run holds one
    (8192, 8192, 256, "gemm_f32_mfma_128x128x32"),  # eight rounds
    (4096, 11008, 64, "gemm_f32_mfma_128x128x32"),  # 5.4 rounds
    (5120, 5120, 64, "gemm_f32_mfma_256x256x32_tail64x64"),
    (4352, 4096, 32, "gemm_f32_mfma_256x256x32_tail128x128"),
])
def test_large_grid_shapes(runtime, m, n, k, want):
    # Grids of at least 256 tiles of 256x256: whole rounds of 128x128 tiles,
    # or, where that grid's last round would be under a quarter full, the
    # 256x256 eight-wave kernel for whole rounds plus a tail in smaller tiles.
    kernel = runtime.compile({"op": "gemm", "m": m, "n": n, "k": k, "tiled": True})
    assert kernel.launch["kernel"] == want, kernel.launch
    a = orc.values(m * k, 0x77, 1.0)
    b = orc.values(k * n, 0x88, 1.0)
    got = run_gemm(runtime, m, n, k, a, b)
    gate(got, m, n, k, a, b)


@pytest.mark.parametrize("m,n,k,slices", [
    (1, 4096, 4096, 2),  # a single row
    (16, 1024, 2816, 11),  # 11 runs of 256
    (31, 3000, 1000, 5),  # ragged N and M, runs of 200
    (32, 8192, 2048, 2),
    (1, 1024, 4096, 8),
])
def test_skinny_direct_split_shapes(runtime, m, n, k, slices):
    # At most 32 rows: direct-load 32x32 tiles split over K into a batch of
    # products (A rows K apart), summed in slice order by the reduce.
    kernel = runtime.compile({"op": "gemm", "m": m, "n": n, "k": k, "tiled": True})
    assert kernel.launch["kernel"] == "gemm_f32_direct_32x32x32_w4_splitk", kernel.launch
    assert kernel.launch["grid"][1] == slices, kernel.launch
    a = orc.values(m * k, 0x5C, 1.0)
    b = orc.values(k * n, 0x6D, 1.0)
    got = run_gemm(runtime, m, n, k, a, b, repeats=2)
    gate(got, m, n, k, a, b)


@pytest.mark.parametrize("m,n,k,want", [
    (2048, 1536, 512, "gemm_f32_mfma_64x64x32"),  # round fill picked 128x64; three 64x64 tiles per CU
    (1024, 6144, 512, "gemm_f32_mfma_128x64x32"),  # round fill picked 64x64; K >= 512 takes the larger tile
    (1088, 1088, 512, "gemm_f32_mfma_64x64x32"),  # 128x64 would leave edge tiles
])
def test_edge_free_plan_shapes(runtime, m, n, k, want):
    # Grids of more than one 64x64 tile per CU whose plan the edge-free
    # second look changes, or would change but for its limits.
    kernel = runtime.compile({"op": "gemm", "m": m, "n": n, "k": k, "tiled": True})
    assert kernel.launch["kernel"] == want, kernel.launch
    a = orc.values(m * k, 0x7A, 1.0)
    b = orc.values(k * n, 0x8B, 1.0)
    got = run_gemm(runtime, m, n, k, a, b)
    gate(got, m, n, k, a, b, rows=(0, 256))
    gate(got, m, n, k, a, b, rows=(m - 256, m))


# A seeded sample (random.Random(20261201)) of shapes below 2e8 products,
# drawn so that every small- and mid-grid plan family appears: direct-load
# 32x32 tiles, 64x64 tiles with two K groups (whole or split K), 64x64,
# 128x64 and 128x128 tiles, aligned and unaligned rows.
RANDOM_SHAPES = [(511, 305, 479), (139, 175, 471), (79, 931, 359), (50, 156, 7406), (2255, 1803, 4),
                 (137, 160, 8826), (512, 512, 512), (628, 1002, 247), (128, 256, 1000), (1690, 3463, 30),
                 (768, 1024, 128), (64, 256, 32), (41, 271, 7183), (2048, 1024, 64), (122, 130, 1844),
                 (417, 246, 998), (184, 658, 690), (72, 96, 2942), (128, 64, 512), (162, 1832, 90),
                 (1766, 790, 56), (256, 256, 128), (753, 65, 540), (512, 1024, 256), (1147, 1675, 58),
                 (2548, 523, 9), (234, 1051, 23), (2174, 761, 69), (2068, 2198, 25), (256, 256, 512),
                 (729, 20, 93), (2492, 718, 26), (860, 290, 149), (3983, 1198, 21), (131, 164, 96),
                 (963, 3612, 35), (567, 360, 260), (256, 1024, 64), (128, 512, 256), (985, 362, 249),
                 (211, 506, 103), (1024, 512, 128), (1989, 3572, 21), (574, 1472, 34), (43, 906, 65),
                 (64, 512, 64), (653, 249, 224), (1945, 1817, 32), (850, 614, 158), (768, 256, 512),
                 (351, 694, 504), (1591, 2326, 22), (1933, 3173, 32), (1776, 1805, 47), (3303, 3252, 17),
                 (2794, 1426, 9), (2078, 1475, 40), (3706, 3196, 3), (1109, 3061, 12), (2638, 1237, 32)]


def test_random_shapes_across_plans(runtime):
    kernels = set()
    for i, (m, n, k) in enumerate(RANDOM_SHAPES):
        kernels.add(runtime.compile({"op": "gemm", "m": m, "n": n, "k": k, "tiled": True}).launch["kernel"])
        a = orc.values(m * k, 0x1000 + i, 1.0)
        b = orc.values(k * n, 0x2000 + i, 1.0)
        got = run_gemm(runtime, m, n, k, a, b)
        want = orc.gemm_reference(m, n, k, a, b)
        check = orc.compare(got, want, NORTH_STAR_TOL, NORTH_STAR_TOL)
        assert check.status == 0, ((m, n, k), check.first_bad, got[check.first_bad], want[check.first_bad])
    for family in ("direct_32x32x32_w4", "64x64x32_k2", "64x64x32_splitk_k2", "mfma_64x64x32", "128x64x32",
                   "128x128x32"):
        assert any(family in name for name in kernels), (family, sorted(kernels))


def test_long_k_takes_64_bit_loads(runtime):
    # K long enough that a 64x64 tile's LDS-direct byte offsets (row * K * 4,
    # a 32-bit offset from a wave-uniform base) would pass 2^31: the launch
    # must take the register-staged loads with 64-bit addresses. A and B are
    # 2.3 GB each; the oracle checks two rows (1.1e9 FP64 products).
    m, n, k = 64, 64, 8912896
    a = orc.values(m * k, 0x91, 1.0)
    b = orc.values(k * n, 0x92, 1.0)
    got = run_gemm(runtime, m, n, k, a, b)
    gate(got, m, n, k, a, b, rows=(0, 2))
    assert np.isfinite(got).all()


def test_unaligned_operand_above_2_gib_takes_global_loads(runtime):
    # Unaligned rows (K % 4 != 0) normally load through buffer instructions
    # with 32-bit offsets and the buffer's range check; an operand of 2 GiB or
    # more (A here: 64 x 8388609 floats) must take the clamped 64-bit global
    # loads instead. The oracle checks the last two rows.
    m, n, k = 64, 3, 8388609
    a = orc.values(m * k, 0x93, 1.0)
    b = orc.values(k * n, 0x94, 1.0)
    got = run_gemm(runtime, m, n, k, a, b)
    gate(got, m, n, k, a, b, rows=(62, 64))
    assert np.isfinite(got).all()


def test_gemm_plan_abi_bench_flow():
    # src/main.rs:281-310 driving src/corex.rs through native/jade_corex.h.
    m = n = k = 512
    a, b = orc.inputs(m, n, k)
    plan = jade_hip.GemmPlan(m, n, k)
    try:
        assert "gfx950" in plan.device_info()
        with pytest.raises(jade_hip.JadeError):
            plan.run(1)  # upload first
        with pytest.raises(jade_hip.JadeError):
            plan.download()
        with pytest.raises(jade_hip.JadeError):
            plan.upload(a[:-1], b)
        plan.upload(a, b)
        ms = plan.run(1)
        assert ms > 0
        out = plan.download()
        assert orc.check_gemm(m, n, k, a, b, out, 4096).status == 0
        assert orc.compare(out, orc.gemm_reference(m, n, k, a, b), NORTH_STAR_TOL, NORTH_STAR_TOL).status == 0
        assert plan.run(3) > 0
        with pytest.raises(jade_hip.JadeError):
            plan.run(0)  # rejected before touching state (native/jade_corex.cpp:216-217)
        np.testing.assert_array_equal(plan.download(), out)
    finally:
        plan.close()


def _gemm_batch(runtime, jobs_spec, arrays, repeats=1, launches=None):
    # jobs_spec: list of (m, n, k, [names of A, B, C]); arrays: name -> host array or element count;
    # launches: the launch plan the batch must take (jr_plan_dispatches).
    bufs = {}
    for name, value in arrays.items():
        bufs[name] = runtime.resident(value) if isinstance(value, np.ndarray) else runtime.alloc(value)
    jobs = [(runtime.compile({"op": "gemm", "m": m, "n": n, "k": k, "tiled": True}), [bufs[x] for x in names])
            for m, n, k, names in jobs_spec]
    if launches is not None:
        assert runtime.plan(jobs) == launches, runtime.plan(jobs)
    runtime.execute(jobs, repeats)
    out = {name: runtime.download(buf) for name, buf in bufs.items()}
    for buf in bufs.values():
        buf.free()
    return out


def test_paired_gemms_match_separate_launches(runtime):
    # Two independent GEMMs of one shape (the MLP's gate and up projections)
    # run as one paired launch (a shape whose plan is one-group 128x64 tiles;
    # K-group, split, direct and persistent plans do not pair); each output
    # must equal its own launch bit for bit.
    m, n, k = 2048, 2048, 1056
    a, b0, b1 = orc.values(m * k, 0x31, 1.0), orc.values(k * n, 0x32, 1.0), orc.values(k * n, 0x33, 1.0)
    both = _gemm_batch(runtime, [(m, n, k, ["a", "b0", "c0"]), (m, n, k, ["a", "b1", "c1"])],
                       {"a": a, "b0": b0, "b1": b1, "c0": m * n, "c1": m * n}, launches=[("pair", 0)])
    one = _gemm_batch(runtime, [(m, n, k, ["a", "b0", "c0"])], {"a": a, "b0": b0, "c0": m * n})
    two = _gemm_batch(runtime, [(m, n, k, ["a", "b1", "c1"])], {"a": a, "b1": b1, "c1": m * n})
    np.testing.assert_array_equal(both["c0"], one["c0"])
    np.testing.assert_array_equal(both["c1"], two["c1"])
    gate(both["c1"], m, n, k, a, b1, rows=(0, 256))
    gate(both["c0"], m, n, k, a, b0, rows=(m - 256, m))


def test_dependent_gemms_keep_order(runtime):
    # Read-after-write (c1 = c0 * b) and write-after-read (the second job
    # overwrites the first job's input) must not share a launch.
    m = n = k = 1024
    a, b = orc.values(m * k, 0x41, 1.0), orc.values(k * n, 0x42, 0.03)
    raw = _gemm_batch(runtime, [(m, n, k, ["a", "b", "c0"]), (m, n, k, ["c0", "b", "c1"])],
                      {"a": a, "b": b, "c0": m * n, "c1": m * n}, launches=[("single", 0), ("single", 1)])
    c0 = orc.gemm_reference(m, n, k, a, b).astype(np.float32)
    gate(raw["c0"], m, n, k, a, b)
    gate(raw["c1"], m, n, k, raw["c0"], b)
    # war: job 1 reads x, job 2 writes x = a * b; two repeats, so the second
    # repeat's first job reads the product.
    war = _gemm_batch(runtime, [(m, n, k, ["x", "b", "c0"]), (m, n, k, ["a", "b", "x"])],
                      {"x": a.copy(), "a": a, "b": b, "c0": m * n}, repeats=2)
    gate(war["x"], m, n, k, a, b)
    gate(war["c0"], m, n, k, war["x"], b)
    assert np.abs(c0 - war["x"]).max() < 1e-3


@pytest.mark.parametrize("m,n,k", [(2048, 4096, 64), (2500, 2500, 256)])
def test_output_not_8_byte_aligned_takes_single_stores(runtime, m, n, k):
    # 128x128 tiles store each lane's two adjacent outputs as one 8-byte write
    # when C starts 8-byte aligned (always for the runtime's allocations). The
    # allocation-free entry takes any device C: here C starts 4 bytes into an
    # allocation, which must take the single stores and give the same bits.
    import ctypes
    kernel = runtime.compile({"op": "gemm", "m": m, "n": n, "k": k, "tiled": True})
    assert kernel.launch["kernel"] == "gemm_f32_mfma_128x128x32", kernel.launch
    a = orc.values(m * k, 0xF1, 1.0)
    b = orc.values(k * n, 0xF2, 1.0)
    want = run_gemm(runtime, m, n, k, a, b)
    fn = runtime._lib.jr_gemm_f32_noalloc
    fn.restype = ctypes.c_int
    fn.argtypes = [ctypes.c_void_p] * 4 + [ctypes.c_uint32] * 3 + [ctypes.c_char_p, ctypes.c_size_t]
    ag, bg, out = runtime.resident(a), runtime.resident(b), runtime.alloc(m * n + 1)
    err = ctypes.create_string_buffer(1024)
    print(f"jr_gemm_f32_noalloc {m}x{n}x{k}, C at +4 bytes", flush=True)
    assert fn(None, ag.ptr, bg.ptr, out.ptr + 4, m, n, k, err, len(err)) == 0, err.value
    hip = ctypes.CDLL("libamdhip64.so")
    assert hip.hipDeviceSynchronize() == 0
    got = runtime.download(out)
    for x in (ag, bg, out):
        x.free()
    assert got[0] == 0.0  # the float before C is untouched (allocations start zeroed)
    np.testing.assert_array_equal(got[1:], want)


@pytest.mark.parametrize("m,n,k,rows", [
    (2048, 2048, 512, None),       # 256 tiles: one per workgroup, 16 stages
    (2560, 2560, 1024, None),      # 400 tiles: runs of one and two tiles
    (4096, 2816, 1024, None),      # 704 tiles: runs of two and three (the MLP gate/up shape)
    (4096, 1024, 2816, None),      # the MLP down projection: K of 11 iterations
    (3840, 3840, 2048, (1792, 2304)),  # 900 tiles: runs of three and four
    (4096, 4096, 512, (0, 640)),   # 1024 tiles: four per workgroup
    (12288, 1024, 1024, (11264, 12288)),
])
def test_persistent_ring_shapes(runtime, m, n, k, rows):
    # Persistent 128x128 tiles (gemm_ring.hip): every workgroup runs its tiles
    # as one sequence of stages, so tile boundaries, the stores of the
    # previous tile and runs of unequal length are all inside one launch.
    kernel = runtime.compile({"op": "gemm", "m": m, "n": n, "k": k, "tiled": True})
    assert kernel.launch["kernel"] == "gemm_f32_ring_128x128x32" and kernel.launch["grid"][0] == 256, kernel.launch
    a = orc.values(m * k, 0x9A, 1.0)
    b = orc.values(k * n, 0x9B, 1.0)
    print(f"ring {m}x{n}x{k}", flush=True)
    got = run_gemm(runtime, m, n, k, a, b, repeats=2)
    if rows is None:
        gate(got, m, n, k, a, b)
    else:
        gate(got, m, n, k, a, b, rows)
        gate(got, m, n, k, a, b, (0, 128))
        gate(got, m, n, k, a, b, (m - 128, m))


@pytest.mark.parametrize("m,n,k", [(2048, 2048, 512), (2560, 2560, 1024)])
def test_persistent_ring_output_not_8_byte_aligned(runtime, m, n, k):
    # The persistent kernel stores pairs of adjacent outputs as one 8-byte
    # write when C (and a residual) start 8-byte aligned; C at +4 bytes
    # through the allocation-free entry takes single stores, same bits.
    import ctypes
    kernel = runtime.compile({"op": "gemm", "m": m, "n": n, "k": k, "tiled": True})
    assert kernel.launch["kernel"] == "gemm_f32_ring_128x128x32", kernel.launch
    a = orc.values(m * k, 0xF3, 1.0)
    b = orc.values(k * n, 0xF4, 1.0)
    want = run_gemm(runtime, m, n, k, a, b)
    fn = runtime._lib.jr_gemm_f32_noalloc
    fn.restype = ctypes.c_int
    fn.argtypes = [ctypes.c_void_p] * 4 + [ctypes.c_uint32] * 3 + [ctypes.c_char_p, ctypes.c_size_t]
    ag, bg, out = runtime.resident(a), runtime.resident(b), runtime.alloc(m * n + 1)
    err = ctypes.create_string_buffer(1024)
    print(f"jr_gemm_f32_noalloc ring {m}x{n}x{k}, C at +4 bytes", flush=True)
    assert fn(None, ag.ptr, bg.ptr, out.ptr + 4, m, n, k, err, len(err)) == 0, err.value
    hip = ctypes.CDLL("libamdhip64.so")
    assert hip.hipDeviceSynchronize() == 0
    got = runtime.download(out)
    for x in (ag, bg, out):
        x.free()
    assert got[0] == 0.0
    np.testing.assert_array_equal(got[1:], want)
