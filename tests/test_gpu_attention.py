"""Online (flash-style) FP32 attention parity against the FP64 materialised
oracle (src/runtime/metal_lab.rs:33-73).

Cases: the reference's metal-verify attention configs (metal_lab.rs:419-431,
inputs at :276-286, tolerance 5e-5, or 5e-4 for amplitude > 1, at :333), its
oracle KAT (:472-484), the materialised scores -> softmax -> apply chain
(:295-324), config C3 (B1 H8 S1024 D64, N(0,1)) and the LLM config (B4 H32
S4096 D128 causal) on query-row windows, gated at |a-e| <= 2e-4 + 2e-4|e|.
"""
import math

import numpy as np
import pytest

import oracle_binding as orc

pytestmark = pytest.mark.gpu

NORTH_STAR_TOL = 2e-4


def run_online(runtime, h, s, d, causal, q, k, v, repeats=1):
    kernel = runtime.compile({"op": "attention_online", "heads": h, "seq": s, "dim": d, "causal": causal})
    qg, kg, vg = runtime.resident(q), runtime.resident(k), runtime.resident(v)
    out = runtime.alloc(h * s * d)
    runtime.execute([(kernel, [qg, kg, vg, out])], repeats)
    got = runtime.download(out)
    assert np.array_equal(runtime.download(qg), q) and np.array_equal(runtime.download(vg), v)
    for x in (qg, kg, vg, out):
        x.free()
    return got


def run_materialised(runtime, h, s, d, causal, q, k, v):
    scores = runtime.compile({"op": "attention_scores", "heads": h, "seq": s, "dim": d, "causal": causal})
    softmax = runtime.compile({"op": "softmax", "rows": h * s, "cols": s})
    apply = runtime.compile({"op": "attention_apply", "heads": h, "seq": s, "dim": d})
    qg, kg, vg = runtime.resident(q), runtime.resident(k), runtime.resident(v)
    sc, pr, out = runtime.alloc(h * s * s), runtime.alloc(h * s * s), runtime.alloc(h * s * d)
    runtime.execute([(scores, [qg, kg, sc]), (softmax, [sc, pr]), (apply, [pr, vg, out])], 1)
    return runtime.download(out)


LAB = [(1, 1, 1, False, 1.0, False), (1, 1, 128, True, 1.0, False), (2, 7, 17, False, 1.0, False),
       (2, 7, 17, True, 1.0, False), (2, 33, 64, False, 1.0, False), (2, 33, 64, True, 1.0, False),
       (1, 65, 128, True, 1.0, False), (3, 17, 33, False, 1.0, True), (2, 17, 31, True, 1.0, True),
       (2, 17, 64, False, 20.0, False), (2, 17, 64, True, 20.0, False)]


@pytest.mark.parametrize("h,s,d,causal,amp,zeros", LAB)
def test_lab_attention_configs(runtime, h, s, d, causal, amp, zeros):
    n = h * s * d
    q = np.zeros(n, np.float32) if zeros else orc.values(n, 0x1111, amp)
    k = np.zeros(n, np.float32) if zeros else orc.values(n, 0x2222, amp)
    v = orc.values(n, 0x3333, 1.0)
    want = orc.attention_reference(h, s, d, causal, q, k, v)
    tol = 5e-4 if amp > 1.0 else 5e-5
    for got in (run_online(runtime, h, s, d, causal, q, k, v, repeats=3),
                run_materialised(runtime, h, s, d, causal, q, k, v)):
        check = orc.compare(got, want, tol, tol)
        assert check.status == 0, (check.first_bad, got[check.first_bad], want[check.first_bad])


@pytest.mark.parametrize("h,s,d,causal", [(2, 64, 64, True), (1, 512, 64, False), (3, 100, 36, True),
                                          (2, 132, 128, True), (1, 8, 4, False), (4, 256, 20, False)])
def test_materialised_on_matrix_cores(runtime, h, s, d, causal):
    # Scores (dim % 4 == 0) and P.V (seq % 4 == 0) on the MFMA kernels: a
    # partial last dim slice (36, 20), ragged 32x32 score tiles (100, 132),
    # causal tiles wholly above the diagonal, and a dim below one slice (4).
    n = h * s * d
    q, k, v = orc.normal(n, 0x1212), orc.normal(n, 0x3434), orc.normal(n, 0x5656)
    for op in ("attention_scores", "attention_apply"):
        spec = {"op": op, "heads": h, "seq": s, "dim": d}
        if op == "attention_scores":
            spec["causal"] = causal
        assert runtime.compile(spec).launch["kernel"].endswith("_mfma")
    got = run_materialised(runtime, h, s, d, causal, q, k, v)
    want = orc.attention_reference(h, s, d, causal, q, k, v)
    check = orc.compare(got, want, NORTH_STAR_TOL, NORTH_STAR_TOL)
    assert check.status == 0, (check.first_bad, got[check.first_bad], want[check.first_bad])


def test_oracle_kat_on_device(runtime):
    q = np.zeros(6, np.float32)
    v = np.array([1, 2, 3, 4, 8, 9], np.float32)
    np.testing.assert_allclose(run_online(runtime, 1, 3, 2, False, q, q, v), [4, 5, 4, 5, 4, 5], rtol=1e-6)
    np.testing.assert_allclose(run_online(runtime, 1, 3, 2, True, q, q, v), [1, 2, 2, 3, 4, 5], rtol=1e-6)


@pytest.mark.parametrize("h,s,d", [(3, 129, 96), (1, 300, 40), (2, 257, 128), (4, 130, 3), (1, 1000, 64)])
@pytest.mark.parametrize("causal", [False, True])
def test_ragged_tiles_and_padded_head_dims(runtime, h, s, d, causal):
    n = h * s * d
    q, k, v = orc.normal(n, 0x1111), orc.normal(n, 0x2222), orc.normal(n, 0x3333)
    want = orc.attention_reference(h, s, d, causal, q, k, v)
    got = run_online(runtime, h, s, d, causal, q, k, v)
    check = orc.compare(got, want, NORTH_STAR_TOL, NORTH_STAR_TOL)
    assert check.status == 0, (check.first_bad, got[check.first_bad], want[check.first_bad])


@pytest.mark.parametrize("causal", [False, True])
def test_config_c3(runtime, causal):
    h, s, d = 8, 1024, 64
    n = h * s * d
    q, k, v = orc.normal(n, 0x1111), orc.normal(n, 0x2222), orc.normal(n, 0x3333)
    got = run_online(runtime, h, s, d, causal, q, k, v)
    want = orc.attention_reference(h, s, d, causal, q, k, v)
    check = orc.compare(got, want, NORTH_STAR_TOL, NORTH_STAR_TOL)
    assert check.status == 0, (check.first_bad, got[check.first_bad], want[check.first_bad])


def test_config_llm_causal_full_output(runtime):
    h, s, d = 4 * 32, 4096, 128
    n = h * s * d
    q, k, v = orc.normal(n, 0x1111), orc.normal(n, 0x2222), orc.normal(n, 0x3333)
    got = run_online(runtime, h, s, d, True, q, k, v).reshape(h, s, d)
    for r0, r1 in ((0, 1024), (1024, 2048), (2048, 3072), (3072, 4096)):
        want = orc.attention_reference(h, s, d, True, q, k, v, rows=(r0, r1)).reshape(h, r1 - r0, d)
        check = orc.compare(got[:, r0:r1].reshape(-1), want.reshape(-1), NORTH_STAR_TOL, NORTH_STAR_TOL)
        assert check.status == 0, (r0, check.first_bad)
        print(f"rows {r0}..{r1} max_abs {check.max_abs_error:.3e} max_rel {check.max_relative_error:.3e}")
    # Causal row 0 attends to key 0 only.
    np.testing.assert_array_equal(got[:, 0], v.reshape(h, s, d)[:, 0])
    assert np.isfinite(got).all()


def test_scale_is_one_over_sqrt_dim(runtime):
    # Two keys whose scores differ by exactly sqrt(d): weights e^1 : 1.
    h, s, d = 1, 2, 16
    q = np.zeros((s, d), np.float32)
    k = np.zeros((s, d), np.float32)
    q[1, 0] = 1.0
    k[1, 0] = math.sqrt(d)
    v = np.zeros((s, d), np.float32)
    v[0, 0], v[1, 0] = 0.0, 1.0
    got = run_online(runtime, h, s, d, False, q.reshape(-1), k.reshape(-1), v.reshape(-1)).reshape(s, d)
    assert got[1, 0] == pytest.approx(math.e / (1.0 + math.e), rel=2e-6)
    assert got[0, 0] == pytest.approx(0.5, rel=2e-6)


@pytest.mark.parametrize("h,s,d,causal", [(2, 1024, 64, True), (1, 700, 128, True), (2, 513, 32, False),
                                          (1, 2048, 64, True), (3, 200, 5, True)])
def test_split_key_grids(runtime, h, s, d, causal):
    # Grids smaller than the chip split the keys into slices (one block per
    # live slice) and merge them; a causal slice can hold no live key for some
    # of its queries.
    kernel = runtime.compile({"op": "attention_online", "heads": h, "seq": s, "dim": d, "causal": causal})
    launch = kernel.launch
    assert launch["kernel"].endswith("_split") and launch["grid"][0] > h and launch["grid"][1] == 1, launch
    n = h * s * d
    q, k, v = orc.normal(n, 0x4444), orc.normal(n, 0x5555), orc.normal(n, 0x6666)
    got = run_online(runtime, h, s, d, causal, q, k, v, repeats=2)
    want = orc.attention_reference(h, s, d, causal, q, k, v)
    check = orc.compare(got, want, NORTH_STAR_TOL, NORTH_STAR_TOL)
    assert check.status == 0, (check.first_bad, got[check.first_bad], want[check.first_bad])


@pytest.mark.parametrize("h,s,d,causal", [
    (8, 1024, 64, True), (8, 1024, 64, False),  # config C3: 256 blocks of two 16-query blocks
    (8, 1000, 64, True),  # odd count of 16-query blocks (the middle one alone), ragged last block and unit
    (12, 700, 48, False),  # head dim padded to 64
    (16, 512, 128, True), (32, 256, 100, True),  # head dims 128 and 100 (padded to 128)
    (1, 4096, 64, True),  # one head, 128 blocks
    # Noncausal odd block counts (the middle block alone runs the one-block
    # pipeline), ragged and whole; long rows; head dims 128 and 96.
    (8, 1000, 64, False), (6, 1008, 64, False), (8, 1008, 64, True), (2, 3000, 64, False),
    (8, 1024, 128, False), (5, 1100, 96, False),
    # Grids below 128 pair blocks whose waves hold little work (the reference's
    # lab configs H4 S512 causal and H4 S256; tiny and ragged grids).
    (4, 512, 64, True), (4, 256, 64, False), (4, 256, 64, True), (1, 256, 64, False), (1, 128, 64, True),
    (1, 100, 64, True), (3, 72, 48, True),
])
def test_paired_small_grids(runtime, h, s, d, causal):
    # Grids that would otherwise split keys across blocks run 16-query waves
    # that split each block's keys among themselves and merge in LDS: one
    # launch, no workspace.
    kernel = runtime.compile({"op": "attention_online", "heads": h, "seq": s, "dim": d, "causal": causal})
    assert kernel.launch["kernel"].endswith(("_pairs", "_singles")), kernel.launch
    assert kernel.description["workspace_bytes"] == 0
    n = h * s * d
    q, k, v = orc.normal(n, 0x4141), orc.normal(n, 0x4242), orc.normal(n, 0x4343)
    got = run_online(runtime, h, s, d, causal, q, k, v, repeats=2)
    want = orc.attention_reference(h, s, d, causal, q, k, v)
    check = orc.compare(got, want, NORTH_STAR_TOL, NORTH_STAR_TOL)
    assert check.status == 0, (check.first_bad, got[check.first_bad], want[check.first_bad])


@pytest.mark.parametrize("h,s,d", [(4, 512, 64), (2, 1024, 64), (4, 1024, 64), (2, 2048, 64), (3, 700, 48),
                                   (4, 1024, 128), (1, 100, 64), (16, 256, 64), (1, 4096, 64)])
def test_single_query_block_grids(runtime, h, s, d):
    # Noncausal grids of at most 256 16-query blocks that fill most of the
    # chip or hold little work per wave run one query block per workgroup
    # (every key unit serves that block alone).
    kernel = runtime.compile({"op": "attention_online", "heads": h, "seq": s, "dim": d, "causal": False})
    assert kernel.launch["kernel"].endswith("_singles"), kernel.launch
    assert kernel.launch["grid"][0] == h * ((s + 15) // 16) and kernel.description["workspace_bytes"] == 0
    n = h * s * d
    q, k, v = orc.normal(n, 0x5151), orc.normal(n, 0x5252), orc.normal(n, 0x5353)
    got = run_online(runtime, h, s, d, False, q, k, v, repeats=2)
    want = orc.attention_reference(h, s, d, False, q, k, v)
    check = orc.compare(got, want, NORTH_STAR_TOL, NORTH_STAR_TOL)
    assert check.status == 0, (check.first_bad, got[check.first_bad], want[check.first_bad])


# A seeded sample (random.Random(20261202)) of heads <= 12, seq <= 1500 and any
# head dim <= 128 below 3e8 score products: odd dims (padded to 32/64/128 with
# scalar loads), ragged query blocks and key tiles, split launches.
RANDOM_SHAPES = [(3, 1037, 61, False), (1, 618, 122, False), (9, 138, 86, True), (3, 715, 52, True),
                 (4, 162, 26, False), (5, 550, 110, True), (8, 311, 71, True), (1, 811, 51, True),
                 (12, 246, 29, False), (9, 661, 42, False), (4, 470, 104, True), (3, 872, 116, True),
                 (4, 846, 81, True), (2, 1171, 73, False), (3, 418, 19, True), (8, 900, 42, True),
                 (7, 551, 80, False), (9, 437, 2, False), (10, 548, 7, True), (7, 467, 115, False),
                 (3, 72, 88, True), (1, 211, 41, True), (7, 426, 77, True), (2, 1252, 16, True)]


def test_random_shapes(runtime):
    for i, (h, s, d, causal) in enumerate(RANDOM_SHAPES):
        n = h * s * d
        q, k, v = orc.normal(n, 0x100 + i), orc.normal(n, 0x200 + i), orc.normal(n, 0x300 + i)
        got = run_online(runtime, h, s, d, causal, q, k, v)
        want = orc.attention_reference(h, s, d, causal, q, k, v)
        check = orc.compare(got, want, NORTH_STAR_TOL, NORTH_STAR_TOL)
        assert check.status == 0, ((h, s, d, causal), check.first_bad, got[check.first_bad], want[check.first_bad])


@pytest.mark.parametrize("causal", [False, True])
def test_unsplit_grid_padded_dims_and_ragged_tile(runtime, causal):
    # The flash kernel's K/V buffer loads: head dim 96 runs in the 128-dim
    # kernel (the lanes of dims 96-127 read zero from an offset past the
    # buffer), and seq 1000 ends inside a 64-key tile (rows past seq lie past
    # the head's buffer and read zero).
    h, s, d = 32, 1000, 96
    kernel = runtime.compile({"op": "attention_online", "heads": h, "seq": s, "dim": d, "causal": causal})
    assert kernel.launch["kernel"].startswith("attention_online_mfma_d128"), kernel.launch
    assert "split" not in kernel.launch["kernel"] and kernel.description["workspace_bytes"] == 0, kernel.launch
    n = h * s * d
    q, k, v = orc.normal(n, 0x4141), orc.normal(n, 0x4242), orc.normal(n, 0x4343)
    got = run_online(runtime, h, s, d, causal, q, k, v)
    want = orc.attention_reference(h, s, d, causal, q, k, v)
    check = orc.compare(got, want, NORTH_STAR_TOL, NORTH_STAR_TOL)
    assert check.status == 0, (check.first_bad, got[check.first_bad], want[check.first_bad])


@pytest.mark.parametrize("causal", [False, True])
def test_unsplit_four_wave_grid(runtime, causal):
    h, s, d = 32, 1024, 64  # 256 blocks of 128 queries: no key split
    kernel = runtime.compile({"op": "attention_online", "heads": h, "seq": s, "dim": d, "causal": causal})
    assert kernel.launch["grid"] == [32, 8, 1] and kernel.launch["block"][0] == 256, kernel.launch
    n = h * s * d
    q, k, v = orc.normal(n, 0x7777), orc.normal(n, 0x8888), orc.normal(n, 0x9999)
    got = run_online(runtime, h, s, d, causal, q, k, v)
    want = orc.attention_reference(h, s, d, causal, q, k, v)
    check = orc.compare(got, want, NORTH_STAR_TOL, NORTH_STAR_TOL)
    assert check.status == 0, (check.first_bad, got[check.first_bad], want[check.first_bad])
