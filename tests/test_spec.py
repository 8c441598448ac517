"""KernelSpec parsing and validation (the reference's IR, src/runtime/ir.rs),
checked on the CPU through the context-free C entry points."""
import json
import os

import pytest

import jade_hip

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "spec_fixtures.json")
FIXTURES = json.load(open(GOLDEN))


def describe(spec):
    return jade_hip.spec_describe(spec)


def rejected(spec):
    with pytest.raises(jade_hip.JadeError) as info:
        describe(spec)
    assert info.value.code == 1
    return info.value.message


@pytest.mark.parametrize("case", FIXTURES["cases"], ids=lambda c: c["case"])
def test_verify_suite_specs_parse_with_reference_bindings(case):
    # Spec files and binding manifest written by the reference's emit-suite.
    d = describe(case["spec_file_text"])
    assert d["bindings"] == case["bindings"]
    assert d["reference_valid"] and d["hip_supported"]
    assert json.loads(json.dumps(d["spec"])) == d["spec"]
    again = describe(json.dumps(d["spec"]))  # canonical form round-trips
    assert again == d
    # Field values survive the round trip.
    for key, value in case["spec"].items():
        if key not in ("expression",):
            assert d["spec"][key] == pytest.approx(value) if isinstance(value, float) else d["spec"][key] == value


def test_example_specs():
    by_name = {e["file"]: e["text"] for e in FIXTURES["examples"]}
    relu = describe(by_name["fused_axpy_relu.json"])
    assert relu["name"] == "elementwise" and len(relu["bindings"]) == 3
    att = describe(by_name["attention_online.json"])
    assert att["name"] == "attention_online" and att["reference_valid"]
    assert [b["elements"] for b in att["bindings"]] == [4 * 256 * 64] * 4
    simd = describe(by_name["gemm_simd.json"])
    assert simd["name"] == "gemm_simdgroup_fp32" and simd["hip_supported"]
    mps = describe(by_name["gemm_mps.json"])
    assert not mps["hip_supported"] and mps["launch"] is None and "MPS" in mps["hip_error"]


@pytest.mark.parametrize("op", ["gemm_simd", "attention_online", "attention_scores", "attention_apply"])
def test_specific_ops_validate_bindings_and_reject_write_alias(op):
    # src/runtime/ir.rs:582-625.
    spec = {"gemm_simd": {"op": "gemm_simd", "m": 33, "n": 17, "k": 65},
            "attention_online": {"op": "attention_online", "heads": 2, "seq": 33, "dim": 17, "causal": True},
            "attention_scores": {"op": "attention_scores", "heads": 2, "seq": 33, "dim": 17, "causal": True},
            "attention_apply": {"op": "attention_apply", "heads": 2, "seq": 33, "dim": 17}}[op]
    lengths = [b["elements"] for b in describe(spec)["bindings"]]
    ids = list(range(len(lengths)))
    jade_hip.spec_validate_bindings(spec, lengths, ids)
    ids[-1] = 0
    with pytest.raises(jade_hip.JadeError):
        jade_hip.spec_validate_bindings(spec, lengths, ids)


U32_MAX = 4294967295


@pytest.mark.parametrize("heads,seq,dim", [(0, 1, 1), (33, 1, 1), (1, 0, 1), (1, 2049, 1), (1, 1, 0), (1, 1, 129),
                                           (U32_MAX, U32_MAX, U32_MAX)])
def test_attention_shape_limits(heads, seq, dim):
    # src/runtime/ir.rs:626-643 rejects all of these; the HIP rules lift only
    # the Metal-era heads <= 32 and seq <= 2048 caps.
    spec = {"op": "attention_online", "heads": heads, "seq": seq, "dim": dim, "causal": False}
    if (heads, seq, dim) in ((33, 1, 1), (1, 2049, 1)):
        d = describe(spec)
        assert not d["reference_valid"] and d["hip_supported"]
    else:
        rejected(spec)


def test_llm_attention_config_is_valid_on_hip_only():
    d = describe({"op": "attention_online", "heads": 128, "seq": 4096, "dim": 128, "causal": True})
    assert not d["reference_valid"] and "heads" in d["reference_error"]
    assert d["bindings"][0]["elements"] == 128 * 4096 * 128
    # The materialised score tensor would need heads*seq*seq > INT_MAX elements.
    rejected({"op": "attention_scores", "heads": 128, "seq": 4096, "dim": 128, "causal": True})


def test_gemm_and_invalid_semantics():
    # src/runtime/ir.rs:644-650, 676-702.
    rejected({"op": "gemm_simd", "m": U32_MAX, "n": U32_MAX, "k": U32_MAX})
    rejected({"op": "gemm", "m": U32_MAX, "n": 2, "k": 1, "tiled": True})
    assert "epsilon" in rejected({"op": "rms_norm", "rows": 1, "cols": 17, "epsilon": 0.0})
    assert "alpha" in rejected({"op": "axpy", "len": 1, "alpha": 1e39})  # overflows f32 to infinity
    spec = {"op": "add", "len": 17}
    with pytest.raises(jade_hip.JadeError):
        jade_hip.spec_validate_bindings(spec, [17, 17, 17], [1, 2, 1])
    with pytest.raises(jade_hip.JadeError):
        jade_hip.spec_validate_bindings(spec, [17, 16, 17], [1, 2, 3])
    jade_hip.spec_validate_bindings(spec, [17, 17, 17], [1, 1, 3])  # read/read aliasing is fine
    with pytest.raises(jade_hip.JadeError):
        jade_hip.spec_validate_bindings(spec, [17, 17], [1, 2])


def _negates(count):
    e = {"kind": "input", "binding": 0}
    for _ in range(count):
        e = {"kind": "negate", "value": e}
    return e


def test_expression_limits():
    # src/runtime/ir.rs:86-110, 653-674.
    rejected({"op": "elementwise", "len": 7, "inputs": 1, "expression": {"kind": "input", "binding": 1}})
    describe({"op": "elementwise", "len": 7, "inputs": 1, "expression": _negates(32)})
    assert "complexity" in rejected({"op": "elementwise", "len": 7, "inputs": 1, "expression": _negates(33)})
    rejected({"op": "elementwise", "len": 7, "inputs": 9, "expression": {"kind": "input", "binding": 0}})
    rejected({"op": "elementwise", "len": 7, "inputs": 0, "expression": {"kind": "input", "binding": 0}})

    def tree(depth):  # complete binary tree: 2^(depth+1)-1 nodes
        if depth == 0:
            return {"kind": "constant", "value": 1.0}
        return {"kind": "add", "left": tree(depth - 1), "right": tree(depth - 1)}

    describe({"op": "elementwise", "len": 3, "inputs": 1, "expression": tree(7)})  # 255 nodes
    big = {"kind": "add", "left": tree(7), "right": tree(7)}  # 511 nodes
    describe({"op": "elementwise", "len": 3, "inputs": 1, "expression": big})
    bigger = {"kind": "add", "left": big, "right": {"kind": "constant", "value": 2.0}}  # 513 nodes
    rejected({"op": "elementwise", "len": 3, "inputs": 1, "expression": bigger})


def test_serde_shape_rules():
    assert "missing field" in rejected({"op": "gemm", "m": 1, "n": 1, "k": 1})
    assert "unknown variant" in rejected({"op": "conv2d", "len": 1})
    rejected({"op": "add", "len": -1})
    rejected({"op": "add", "len": 1.5})
    rejected({"op": "add", "len": U32_MAX + 1})
    rejected({"op": "gemm", "m": 1, "n": 1, "k": 1, "tiled": 1})
    rejected('{"op": "add", "len": 3')
    rejected('{"op": "add", "len": 3, "len": 4}')
    d = describe({"op": "add", "len": 3, "comment": "unknown members are ignored"})
    assert d["spec"] == {"op": "add", "len": 3}
    rejected({"op": "add", "len": 0})
    rejected("x" * 70000)  # over the 64 KiB spec cap


def test_constant_bits_round_trip():
    for value in (2.5, 1e-5, -0.375, 3.4028234663852886e38, 1.17549435e-38):
        spec = {"op": "elementwise", "len": 1, "inputs": 1,
                "expression": {"kind": "constant", "value": value}}
        d = describe(spec)
        import numpy as np
        assert np.float32(d["spec"]["expression"]["value"]) == np.float32(value)


@pytest.mark.parametrize("m,n,k,kernel,grid", [
    (4096, 4096, 4096, "gemm_f32_ring_128x128x32", [256, 1, 1]),  # persistent 128x128 tiles, one workgroup per CU
    (8192, 8192, 256, "gemm_f32_mfma_128x128x32", [4096, 1, 1]),  # K < 512 keeps the tile kernel
    (4096, 4096, 4112, "gemm_f32_mfma_128x128x32", [1024, 1, 1]),  # K not a multiple of 32
    (2048, 2048, 2048, "gemm_f32_ring_128x128x32", [256, 1, 1]),  # one tile per CU
    (2048, 2048, 2080, "gemm_f32_mfma_128x64x32", [512, 1, 1]),  # K not a multiple of 256
    (1024, 1024, 1024, "gemm_f32_mfma_64x64x32_k4", [256, 1, 1]),  # <= 256 tiles, K >= 768: four K groups
    (1024, 1024, 512, "gemm_f32_mfma_64x64x32_k2", [256, 1, 1]),  # shorter K: two K groups
    (1000, 777, 1024, "gemm_f32_mfma_64x64x32_k4", [208, 1, 1]),  # unaligned rows through buffer loads: four too
    (1000, 777, 513, "gemm_f32_mfma_64x64x32_k4", [208, 1, 1]),  # unaligned, whole stages four groups split
    (1000, 777, 545, "gemm_f32_mfma_64x64x32_k2", [208, 1, 1]),  # unaligned, a partial stage: two groups
    (1536, 1024, 1024, "gemm_f32_mfma_64x64x32", [384, 1, 1]),  # 256 < tiles < 384: one group
    (512, 512, 512, "gemm_f32_direct_lds_32x32x32_w4", [256, 1, 1]),  # one launch, four waves split K via LDS
    (384, 384, 516, "gemm_f32_direct_lds_32x32x32_w4", [144, 1, 1]),  # ragged last slice
    (512, 510, 512, "gemm_f32_direct_32x32x32_w4", [256, 1, 1]),  # N % 4 != 0: register-staged
    (700, 700, 700, "gemm_f32_direct_32x32x32_w4", [484, 1, 1]),  # 6 slices per wave
    (768, 768, 768, "gemm_f32_mfma_64x64x32_k4", [144, 1, 1]),  # > 128 64x64 tiles: not direct
    (255, 257, 4, "gemm_f32_direct_32x32x32_w1", [72, 1, 1]),  # one slice: one wave
    (1, 4096, 4096, "gemm_f32_direct_32x32x32_w4_splitk", [128, 2, 1]),  # <= 32 rows: K split ~1536 waves
    (16, 1024, 2816, "gemm_f32_direct_32x32x32_w4_splitk", [32, 11, 1]),  # slices divide K
    (1, 16384, 4096, "gemm_f32_direct_32x32x32_w4", [512, 1, 1]),  # enough tiles unsplit
    (1, 4096, 4100, "gemm_f32_mfma_64x64x32_splitk_k2", [64, 4, 1]),  # no divisor of K gives 1024 waves
    (33, 4096, 4096, "gemm_f32_mfma_64x64x32_splitk_k2", [64, 4, 1]),  # over 32 rows
    (1024, 512, 1024, "gemm_f32_mfma_64x64x32_splitk_k2", [128, 2, 1]),  # 8 slices per wave: split K
    (512, 512, 4096, "gemm_f32_mfma_64x64x32_splitk_k2", [64, 4, 1]),
    (256, 256, 4096, "gemm_f32_mfma_64x64x32_splitk_k2", [16, 16, 1]),
    (4096, 11008, 4096, "gemm_f32_ring_128x128x32", [256, 1, 1]),  # 10.75 tiles per workgroup
    (4096, 11008, 4128, "gemm_f32_mfma_128x128x32", [2752, 1, 1]),  # 128x128 last round 192/512 full
    (5120, 5120, 2048, "gemm_f32_ring_128x128x32", [256, 1, 1]),  # replaces 256x256 + tail
    (5120, 5120, 2080, "gemm_f32_mfma_256x256x32_tail64x64", [256, 1, 1]),  # 128x128 last round 64/512: 256x256 + tail
    (4352, 4096, 1056, "gemm_f32_mfma_256x256x32_tail128x128", [256, 1, 1]),  # tail 16: one 128x128 per CU
    (6144, 6144, 1024, "gemm_f32_ring_128x128x32", [256, 1, 1]),
    (6144, 6144, 1056, "gemm_f32_mfma_128x128x32", [2304, 1, 1]),
    (3072, 3072, 3072, "gemm_f32_mfma_64x64x32", [2304, 1, 1]),  # 128x128 would fill 56% of two rounds
    (2500, 2500, 2500, "gemm_f32_mfma_128x128x32", [400, 1, 1]),
    (1024, 4096, 4096, "gemm_f32_ring_128x128x32", [256, 1, 1]),  # 256 tiles: balanced
    (1024, 4096, 4128, "gemm_f32_mfma_128x64x32", [512, 1, 1]),  # 128x64 also for wide C
    (6144, 1024, 1024, "gemm_f32_mfma_128x64x32", [768, 1, 1]),  # 384 persistent tiles: 1.5 per CU, kept
    (2048, 3072, 1024, "gemm_f32_mfma_128x64x32", [768, 1, 1]),
    (2048, 3072, 384, "gemm_f32_mfma_64x64x32", [1536, 1, 1]),  # K < 512 keeps the smaller tile
    (3072, 1024, 4096, "gemm_f32_mfma_64x64x32", [768, 1, 1]),  # 3 tiles per CU against 2 of twice the size
    (3648, 3648, 1024, "gemm_f32_mfma_64x64x32", [3249, 1, 1]),  # 128x128 would leave edge tiles
    (12288, 1024, 1024, "gemm_f32_ring_128x128x32", [256, 1, 1]),  # 768 persistent tiles: balanced
    (12288, 1024, 1056, "gemm_f32_mfma_128x64x32", [1536, 1, 1]),  # 128x128 predicted < 5% faster: kept
    (4096, 2816, 1024, "gemm_f32_ring_128x128x32", [256, 1, 1]),  # MLP gate/up alone (704 tiles)
    (4096, 1024, 2816, "gemm_f32_ring_128x128x32", [256, 1, 1]),  # MLP down projection
    (500, 777, 513, "gemm_f32_direct_32x32x32_w4_buf", [400, 1, 1]),  # unaligned, <= half the CUs: buffer loads
])
def test_gemm_launch_plans(m, n, k, kernel, grid):
    # Persistent 128x128 tiles (gemm_ring.hip) for whole 128x128 tiles, K a
    # multiple of 256 and at least 512, at least 256 tiles, in place of
    # 128x128/256x256 plans or where ceil(t/256) <= t/256/0.9. Otherwise:
    # grids of >= 256 tiles of 256x256 as 128x128 tiles, unless that grid's
    # last round would be under a quarter full: then 256x256 for the whole
    # rounds (the rest as 128x128, 128x64 or 64x64 tiles); else the best of
    # 128x128 / 128x64 / 64x64 by round fill x tile
    # efficiency among grids of >= 384 workgroups, replaced by the edge-free
    # tile whose busiest CU finishes first when that choice has edge tiles or
    # is predicted 5% slower (K < 512 keeps the smaller tile); with at most
    # one 64x64 tile per CU, products of at most 32 rows as direct-load 32x32
    # tiles split over K, else 64x64 tiles with
    # two K groups (four for K >= 768, and for unaligned rows from K = 512
    # when four groups split K's whole stages evenly, at most two k left),
    # and at most half the CUs' worth of
    # tiles either direct-load 32x32 tiles (aligned, moderate K) or split K.
    launch = describe({"op": "gemm", "m": m, "n": n, "k": k, "tiled": True})["launch"]
    assert launch["kernel"] == kernel and launch["grid"] == grid, launch


def test_descriptions_report_workspace_bytes():
    # Split launches own a workspace allocated at jr_compile; others none.
    assert describe({"op": "gemm", "m": 256, "n": 256, "k": 4096, "tiled": True})["workspace_bytes"] == 16 * 256 * 256 * 4
    assert describe({"op": "gemm", "m": 512, "n": 512, "k": 512, "tiled": True})["workspace_bytes"] == 0
    assert describe({"op": "gemm", "m": 4096, "n": 4096, "k": 4096, "tiled": True})["workspace_bytes"] == 0
    assert describe({"op": "attention_online", "heads": 2, "seq": 1024, "dim": 64, "causal": True})["workspace_bytes"] > 0
    # Config C3 runs the paired 16-query kernel: one launch, no workspace.
    c3 = describe({"op": "attention_online", "heads": 8, "seq": 1024, "dim": 64, "causal": True})
    assert c3["workspace_bytes"] == 0 and c3["launch"]["kernel"] == "attention_online_mfma16_d64_pairs"
    assert c3["launch"]["grid"] == [256, 1, 1]
    assert describe({"op": "attention_online", "heads": 128, "seq": 4096, "dim": 128, "causal": True})[
        "workspace_bytes"] == 0
    assert describe({"op": "softmax", "rows": 4, "cols": 4})["workspace_bytes"] == 0


@pytest.mark.parametrize("op,dim,seq,kernel", [
    ("attention_scores", 64, 512, "attention_scores_mfma"), ("attention_scores", 5, 512, "attention_scores"),
    ("attention_apply", 64, 512, "attention_apply_mfma"), ("attention_apply", 64, 513, "attention_apply"),
])
def test_materialised_attention_kernels(op, dim, seq, kernel):
    # Scores run on the matrix cores when dim % 4 == 0, P.V when seq % 4 == 0
    # (16-byte rows); other shapes take the one-thread-per-output kernels.
    spec = {"op": op, "heads": 2, "seq": seq, "dim": dim}
    if op == "attention_scores":
        spec["causal"] = True
    assert describe(spec)["launch"]["kernel"] == kernel


def _xcd_order(bid, count):
    # gemm_f32.hip xcd_order: blocks go round-robin over 8 XCDs by id; each
    # XCD owns a contiguous range of positions.
    per, rem = divmod(count, 8)
    xcd, idx = bid % 8, bid // 8
    return xcd * per + min(xcd, rem) + idx


def _grouped_tile(logical, tiles_m, tiles_n, group_m=8):
    # gemm_f32.hip grouped_tile: 8 tile rows at a time, column-major inside.
    span = group_m * tiles_n
    group, inside = divmod(logical, span)
    first = group * group_m
    rows = min(tiles_m - first, group_m)
    return first + inside % rows, inside // rows


@pytest.mark.parametrize("m,n,tail_tm,tail_tn", [(5120, 5120, 1, 1), (4352, 4096, 2, 2), (8448, 4608, 1, 1),
                                                 (6144, 6144, 2, 2)])
def test_big_plan_covers_every_tile_once(m, n, tail_tm, tail_tn):
    # The 256x256 launch's whole rounds plus the tail launch in smaller tiles
    # (the mapping of gemm_f32_mfma_256 and gemm_f32_mfma's tail mode) compute
    # every 64x64 block of C exactly once.
    tiles_m, tiles_n = m // 256, n // 256
    tiles = tiles_m * tiles_n
    full = tiles // 256 * 256
    count = {}
    for bid in range(full):
        tm, tn = _grouped_tile(_xcd_order(bid, full), tiles_m, tiles_n)
        for i in range(4):
            for j in range(4):
                key = (4 * tm + i, 4 * tn + j)
                count[key] = count.get(key, 0) + 1
    sub_m, sub_n = 4 // tail_tm, 4 // tail_tn  # 256 / (64 * tile) per side
    bm_, bn_ = 64 * tail_tm, 64 * tail_tn
    groups = (tiles - full) * sub_m * sub_n
    for bid in range(groups):
        pos = _xcd_order(bid, groups)
        bm, bn = _grouped_tile(full + pos // (sub_m * sub_n), tiles_m, tiles_n)
        sub = pos % (sub_m * sub_n)
        tm, tn = sub_m * bm + sub // sub_n, sub_n * bn + sub % sub_n
        for i in range(bm_ // 64):
            for j in range(bn_ // 64):
                key = (tm * bm_ // 64 + i, tn * bn_ // 64 + j)
                count[key] = count.get(key, 0) + 1
    assert len(count) == (m // 64) * (n // 64) and set(count.values()) == {1}


ROUTE_DIMS = (1, 3, 4, 31, 32, 33, 64, 100, 127, 128, 255, 256, 500, 512, 513, 777, 1000, 1024, 2048, 4096, 8192)


def test_every_gemm_shape_routes_to_a_launch():
    # gemm_f32 and its description take their decision from one route
    # (gemm_f32.hip route_for): a shape whose plan has no kernel
    # instantiation is described as unsupported and rejected by jr_compile,
    # never launched as nothing. Every shape of this grid (aligned and
    # unaligned rows, edge and interior tiles, every plan family) has one.
    seen = set()
    shapes = [(m, n, k) for m in ROUTE_DIMS for n in ROUTE_DIMS for k in ROUTE_DIMS]
    # Long K (register-staged 64-bit loads) and operands of 2 GiB or more
    # with unaligned rows (clamped loads, two K groups at most).
    shapes += [(64, 64, 8912896), (1000, 777, 2097153), (300, 700, 2097153), (8192, 8192, 8)]
    # 256x256 whole rounds with a 64x64 or 128x128 tail (K not a multiple of
    # 256), and the persistent kernel.
    shapes += [(5120, 5120, 2080), (4352, 4096, 1056), (4096, 4096, 4096)]
    for m, n, k in shapes:
        d = describe({"op": "gemm", "m": m, "n": n, "k": k, "tiled": True})
        assert d["hip_supported"] and d["launch"]["kernel"], (m, n, k, d["hip_error"])
        seen.add(d["launch"]["kernel"])
    families = {"gemm_f32_mfma_256x256x32_tail64x64", "gemm_f32_mfma_256x256x32_tail128x128",
                "gemm_f32_direct_32x32x32_w4_buf", "gemm_f32_mfma_128x128x32", "gemm_f32_mfma_128x64x32",
                "gemm_f32_mfma_64x64x32", "gemm_f32_mfma_64x64x32_k2", "gemm_f32_mfma_64x64x32_k4",
                "gemm_f32_mfma_64x64x32_splitk_k2", "gemm_f32_direct_32x32x32_w4", "gemm_f32_direct_lds_32x32x32_w4",
                "gemm_f32_direct_32x32x32_w4_splitk", "gemm_f32_ring_128x128x32"}
    assert families <= seen, families - seen


def test_online_attention_query_blocks_fit_the_grid():
    # The online kernel's query blocks (>= 128 queries each) sit on grid.y,
    # whose HIP limit is 65535 blocks.
    ok = describe({"op": "attention_online", "heads": 1, "seq": 65535 * 128, "dim": 1, "causal": False})
    assert ok["launch"]["grid"][1] <= 65535
    msg = rejected({"op": "attention_online", "heads": 1, "seq": 65535 * 128 + 1, "dim": 1, "causal": False})
    assert "8388480" in msg


def test_noalloc_scratch_covers_every_split_plan():
    # jr_gemm_f32_noalloc keeps split-K partials in an 8 MiB static device
    # array; every split plan of this shape grid fits it (the planner splits K
    # only for grids of at most half the CUs' worth of tiles).
    limit = 8 << 20
    dims = (1, 16, 32, 64, 96, 127, 128, 192, 256, 384, 500, 512, 640, 768, 1000, 1536, 3000, 4096, 6000, 16384)
    most = 0
    for m in dims:
        for n in dims:
            for k in (128, 513, 1024, 4096, 65536):
                if m * k >= 2 ** 31 or k * n >= 2 ** 31:
                    continue
                most = max(most, describe({"op": "gemm", "m": m, "n": n, "k": k, "tiled": True})["workspace_bytes"])
    assert 0 < most <= limit, most


@pytest.mark.parametrize("heads,seq,dim,causal,kernel,blocks", [
    # Grids that fill the chip with 128-query blocks: the flash kernel.
    (128, 4096, 128, True, "attention_online_mfma_d128", 128),
    (64, 2048, 128, True, "attention_online_mfma_d128", 64),
    (32, 2048, 64, True, "attention_online_mfma_d64", 32),
    (1, 64, 64, True, "attention_online_mfma_d64", 1),
    # Config C3: pairs of 16-query blocks, 256 workgroups.
    (8, 1024, 64, True, "attention_online_mfma16_d64_pairs", 256),
    (8, 1024, 64, False, "attention_online_mfma16_d64_pairs", 256),
    (2, 2048, 128, False, "attention_online_mfma16_d128_pairs", 128),
    # Small grids with little work per wave: pairs (causal) or single query
    # blocks (noncausal, at most 256 workgroups).
    (4, 512, 64, True, "attention_online_mfma16_d64_pairs", 64),
    (4, 512, 64, False, "attention_online_mfma16_d64_singles", 128),
    (4, 256, 64, False, "attention_online_mfma16_d64_singles", 64),
    (2, 1024, 64, False, "attention_online_mfma16_d64_singles", 128),
    (4, 1024, 64, False, "attention_online_mfma16_d64_singles", 256),
    # More work per wave on few workgroups, head dims of at most 32 and
    # unaligned rows: the split launch and its merge.
    (2, 1024, 64, True, "attention_online_mfma_d64_split", 144),
    (1, 2048, 64, False, "attention_online_mfma_d64_split", 256),
    (1, 2048, 64, True, "attention_online_mfma_d64_split", 136),
    (2, 1000, 128, False, "attention_online_mfma_d128_split", 256),
    (3, 200, 5, True, "attention_online_mfma_d32_split", 18),
    (2, 513, 32, False, "attention_online_mfma_d32_split", 90),
])
def test_attention_kernel_selection(heads, seq, dim, causal, kernel, blocks):
    # The online-attention planner's choice per grid (attention_f32.hip:
    # pair_mode, split_plan, waves_for); the 16-query kernels need no workspace.
    d = describe({"op": "attention_online", "heads": heads, "seq": seq, "dim": dim, "causal": causal})
    assert d["launch"]["kernel"] == kernel and d["launch"]["grid"][0] == blocks, d["launch"]
    assert (d["workspace_bytes"] > 0) == kernel.endswith("_split")


def test_gemm_epilogue_tail_rule():
    # Unaligned K-group tiles (two or four groups of four waves, unsplit K) add
    # the last one or two k in the epilogue when K is whole 32-k stages that
    # the groups split evenly plus those k; the description reports them as
    # epilogue_k. Every other plan (aligned rows, split K, other tiles, three
    # or more last k, stages the groups cannot split evenly) has none.
    seen = set()
    for m, n in [(1000, 777), (777, 1000), (200, 8), (1023, 1001), (500, 777), (3000, 3001)]:
        for k in [33, 65, 66, 67, 97, 129, 130, 257, 513, 514, 515, 545, 769, 770, 1025, 1027, 2049]:
            launch = describe({"op": "gemm", "m": m, "n": n, "k": k, "tiled": True})["launch"]
            groups = {512: 2, 1024: 4}.get(launch["block"][0], 1) if "_k" in launch["kernel"] else 1
            whole, rest = divmod(k, 32)
            unaligned = k % 4 != 0 or n % 4 != 0
            want = rest if (unaligned and groups > 1 and launch["grid"][1] == 1 and whole > 0
                            and whole % groups == 0 and 0 < rest <= 2) else 0
            assert launch.get("epilogue_k", 0) == want, (m, n, k, launch)
            seen.add(want)
    assert seen == {0, 1, 2}
