"""Six-op residual MLP (src/runtime/workloads.rs:366-525) as one ordered
execute of six jobs, against the FP64 chain oracle (workloads.rs:466-479)."""
import numpy as np
import pytest

import oracle_binding as orc

pytestmark = pytest.mark.gpu


def mlp_jobs(runtime, batch, width, hidden, x, norm, wg, wu, wd, eps):
    specs = [
        {"op": "rms_norm", "rows": batch, "cols": width, "epsilon": eps},
        {"op": "gemm", "m": batch, "n": hidden, "k": width, "tiled": True},
        {"op": "gemm", "m": batch, "n": hidden, "k": width, "tiled": True},
        {"op": "swi_glu", "len": batch * hidden},
        {"op": "gemm", "m": batch, "n": width, "k": hidden, "tiled": True},
        {"op": "add", "len": batch * width},
    ]
    k = [runtime.compile(s) for s in specs]
    xg, ng, wgg, wug, wdg = (runtime.resident(t) for t in (x, norm, wg, wu, wd))
    normalized, gate, up = runtime.alloc(batch * width), runtime.alloc(batch * hidden), runtime.alloc(batch * hidden)
    act, proj, out = runtime.alloc(batch * hidden), runtime.alloc(batch * width), runtime.alloc(batch * width)
    jobs = [(k[0], [xg, ng, normalized]), (k[1], [normalized, wgg, gate]), (k[2], [normalized, wug, up]),
            (k[3], [gate, up, act]), (k[4], [act, wdg, proj]), (k[5], [proj, xg, out])]
    return jobs, out


@pytest.mark.parametrize("batch,width,hidden", [(8, 128, 256), (3, 33, 65), (64, 512, 1024)])
def test_reference_mlp_workload(runtime, batch, width, hidden):
    # workloads::mlp_with_gemm inputs (389-394), eps 1e-5, tolerance 5e-5.
    x = orc.values(batch * width, 0x1234, 1.0)
    norm = np.ones(width, np.float32)
    wg = orc.values(width * hidden, 0x3333, np.float32(1.0) / np.sqrt(np.float32(width)))
    wu = orc.values(width * hidden, 0x4444, np.float32(1.0) / np.sqrt(np.float32(width)))
    wd = orc.values(hidden * width, 0x5555, np.float32(1.0) / np.sqrt(np.float32(hidden)))
    eps = float(np.float32(1e-5))
    jobs, out = mlp_jobs(runtime, batch, width, hidden, x, norm, wg, wu, wd, 1e-5)
    timing = runtime.execute(jobs, 3)
    assert timing.dispatches == 18
    want = orc.mlp(batch, width, hidden, x, norm, wg, wu, wd, eps)
    check = orc.compare(runtime.download(out), want, 5e-5, 5e-5)
    assert check.status == 0, check.first_bad


def test_config_c4_mlp(runtime):
    batch, width, hidden = 4096, 1024, 2816
    x = orc.normal(batch * width, 0x1234)
    gamma = orc.values(width, 0x7777, 0.5) + np.float32(1.0)
    wg = orc.normal(width * hidden, 0x3333, 0.0, 0.02)
    wu = orc.normal(width * hidden, 0x4444, 0.0, 0.02)
    wd = orc.normal(hidden * width, 0x5555, 0.0, 0.02)
    eps = 1e-6
    jobs, out = mlp_jobs(runtime, batch, width, hidden, x, gamma, wg, wu, wd, eps)
    runtime.execute(jobs, 1)
    got = runtime.download(out)
    # Every output against the FP64 chain, as the reference compares every
    # output of its MLP (src/runtime/workloads.rs:480-481,509).
    want = orc.mlp(batch, width, hidden, x, gamma, wg, wu, wd, float(np.float32(eps)))
    check = orc.compare(got, want, 1e-4, 1e-4)
    assert check.status == 0, check.first_bad
    print(f"C4 MLP all {batch * width} outputs: max_abs {check.max_abs_error:.3e}", flush=True)


def _run_jobs(runtime, specs, arrays, plan, repeats=1, one_at_a_time=False, launches=None):
    # specs: name -> spec; arrays: name -> host array or element count;
    # plan: list of (spec name, [buffer names]); launches: the launch plan
    # the batch must take (jr_plan_dispatches), checked before it runs.
    kernels = {name: runtime.compile(spec) for name, spec in specs.items()}
    bufs = {name: runtime.resident(v) if isinstance(v, np.ndarray) else runtime.alloc(v) for name, v in arrays.items()}
    jobs = [(kernels[s], [bufs[b] for b in names]) for s, names in plan]
    if launches is not None:
        assert runtime.plan(jobs) == launches, runtime.plan(jobs)
    if one_at_a_time:
        for _ in range(repeats):
            for job in jobs:
                runtime.execute([job], 1)
    else:
        runtime.execute(jobs, repeats)
    out = {name: runtime.download(b) for name, b in bufs.items()}
    for b in bufs.values():
        b.free()
    return out


@pytest.mark.parametrize("m,n,k", [
    (2048, 2048, 256),  # two whole rounds of 128x64 tiles
    (4096, 2816, 96),   # 1408 tiles: the last four tile columns run as 64x64 tiles; three stages (odd fold)
    (4096, 2816, 1024),  # the C4 shape: alone, each product runs on the persistent 128x128 kernel
])
def test_fused_gate_up_swiglu_is_bit_identical(runtime, m, n, k):
    # gemm(x, Wg -> G), gemm(x, Wu -> U), swi_glu(G, U -> D) on whole 128x64
    # tiles run as one fused launch; each of G, U and D must equal the three
    # jobs launched one at a time (on the 128x64 tile kernel or the persistent
    # kernel, which take the same MFMA steps per output), bit for bit.
    specs = {"gemm": {"op": "gemm", "m": m, "n": n, "k": k, "tiled": True}, "swiglu": {"op": "swi_glu", "len": m * n}}
    assert runtime.compile(specs["gemm"]).launch["kernel"] in ("gemm_f32_mfma_128x64x32", "gemm_f32_ring_128x128x32")
    arrays = {"x": orc.normal(m * k, 0x21), "wg": orc.normal(k * n, 0x22, 0.0, 0.1),
              "wu": orc.normal(k * n, 0x23, 0.0, 0.1), "g": m * n, "u": m * n, "d": m * n}
    plan = [("gemm", ["x", "wg", "g"]), ("gemm", ["x", "wu", "u"]), ("swiglu", ["g", "u", "d"])]
    fused = _run_jobs(runtime, specs, arrays, plan, repeats=2, launches=[("gate_up_swiglu", 0)])
    alone = _run_jobs(runtime, specs, arrays, plan, one_at_a_time=True)
    for name in ("g", "u", "d"):
        np.testing.assert_array_equal(fused[name], alone[name], err_msg=name)
    rows = (0, 64)
    for name, w in (("g", "wg"), ("u", "wu")):
        want = orc.gemm_reference(m, n, k, arrays["x"], arrays[w], rows=rows)
        assert orc.compare(fused[name][:64 * n], want, 1e-4, 1e-4).status == 0, name
    want = orc.swiglu(fused["g"][:64 * n], fused["u"][:64 * n])
    assert orc.compare(fused["d"][:64 * n], want, 3e-5, 3e-5).status == 0


def test_swiglu_writing_a_gemm_input_is_not_fused(runtime):
    # swi_glu writes the gate weights the GEMMs read (k == m so the lengths
    # match): fusing would overwrite Wg while other workgroups still read it,
    # so the batch keeps its order; two repeats make the second read the
    # overwritten weights. The shape plans whole 128x64 tiles, so only the
    # hazard keeps the jobs apart.
    m, n, k = 2048, 2048, 2048
    specs = {"gemm": {"op": "gemm", "m": m, "n": n, "k": k, "tiled": True}, "swiglu": {"op": "swi_glu", "len": m * n}}
    assert runtime.compile(specs["gemm"]).launch["kernel"] == "gemm_f32_ring_128x128x32"
    arrays = {"x": orc.normal(m * k, 0x31, 0.0, 0.05), "wg": orc.normal(k * n, 0x32, 0.0, 0.05),
              "wu": orc.normal(k * n, 0x33, 0.0, 0.05), "g": m * n, "u": m * n}
    plan = [("gemm", ["x", "wg", "g"]), ("gemm", ["x", "wu", "u"]), ("swiglu", ["g", "u", "wg"])]
    batched = _run_jobs(runtime, specs, arrays, plan, repeats=2, launches=[("single", 0), ("single", 1), ("single", 2)])
    ordered = _run_jobs(runtime, specs, arrays, plan, repeats=2, one_at_a_time=True)
    for name in ("g", "u", "wg"):
        np.testing.assert_array_equal(batched[name], ordered[name], err_msg=name)


@pytest.mark.parametrize("m,n,k,order", [
    (4096, 1024, 2816, "px"),  # the C4 down projection: persistent 128x128 tiles
    (4096, 1024, 2816, "xp"),  # add(X, P -> O): the other operand order
    (4096, 1024, 2848, "px"),  # K not a multiple of 256: 128x64 LDS-direct tiles
    (1000, 777, 513, "px"),  # unaligned rows: register-staged tiles with two K groups, edge masks
    (1024, 1024, 1024, "px"),  # 64x64 tiles with four K groups
    (4096, 4096, 256, "px"),  # 128x128 tiles
])
def test_fused_gemm_residual_is_bit_identical(runtime, m, n, k, order):
    # gemm(a, w -> p) then add(p, x -> o) run as one launch (the residual
    # MLP's down projection and residual add); p and o must equal the two
    # jobs launched one at a time, bit for bit.
    specs = {"gemm": {"op": "gemm", "m": m, "n": n, "k": k, "tiled": True}, "add": {"op": "add", "len": m * n}}
    arrays = {"a": orc.normal(m * k, 0x41, 0.0, 0.5), "w": orc.normal(k * n, 0x42, 0.0, 0.05),
              "x": orc.normal(m * n, 0x43), "p": m * n, "o": m * n}
    operands = ["p", "x"] if order == "px" else ["x", "p"]
    plan = [("gemm", ["a", "w", "p"]), ("add", operands + ["o"])]
    fused = _run_jobs(runtime, specs, arrays, plan, repeats=2, launches=[("gemm_residual", 0)])
    alone = _run_jobs(runtime, specs, arrays, plan, one_at_a_time=True)
    for name in ("p", "o"):
        np.testing.assert_array_equal(fused[name], alone[name], err_msg=name)
    want = orc.gemm_reference(m, n, k, arrays["a"], arrays["w"], rows=(m - 32, m))
    assert orc.compare(fused["p"][(m - 32) * n:], want, 1e-4, 1e-4).status == 0
    np.testing.assert_array_equal(fused["o"], fused["p"] + arrays["x"])


def test_add_writing_a_gemm_input_is_not_fused(runtime):
    # add(p, x -> a) overwrites the GEMM's own A (n == k so the lengths
    # match): fused, the epilogue would write A while other workgroups still
    # read it, so the batch keeps its order; two repeats make the second
    # product read the overwritten A.
    m, n, k = 2048, 1024, 1024
    specs = {"gemm": {"op": "gemm", "m": m, "n": n, "k": k, "tiled": True}, "add": {"op": "add", "len": m * n}}
    arrays = {"a": orc.normal(m * k, 0x51, 0.0, 0.05), "w": orc.normal(k * n, 0x52, 0.0, 0.05),
              "x": orc.normal(m * n, 0x53, 0.0, 0.05), "p": m * n}
    plan = [("gemm", ["a", "w", "p"]), ("add", ["p", "x", "a"])]
    batched = _run_jobs(runtime, specs, arrays, plan, repeats=2, launches=[("single", 0), ("single", 1)])
    ordered = _run_jobs(runtime, specs, arrays, plan, repeats=2, one_at_a_time=True)
    for name in ("a", "p"):
        np.testing.assert_array_equal(batched[name], ordered[name], err_msg=name)


def test_c4_block_fused_equals_ordered_launches(runtime):
    # The whole C4 block batched (gate/up/SwiGLU and down/Add each fused) is
    # bit-identical, in every one of its six outputs, to the six jobs launched
    # one at a time.
    batch, width, hidden = 4096, 1024, 2816
    specs = {"norm": {"op": "rms_norm", "rows": batch, "cols": width, "epsilon": 1e-6},
             "up": {"op": "gemm", "m": batch, "n": hidden, "k": width, "tiled": True},
             "swiglu": {"op": "swi_glu", "len": batch * hidden},
             "down": {"op": "gemm", "m": batch, "n": width, "k": hidden, "tiled": True},
             "add": {"op": "add", "len": batch * width}}
    arrays = {"x": orc.normal(batch * width, 0x1234), "gamma": orc.values(width, 0x7777, 0.5) + np.float32(1.0),
              "wg": orc.normal(width * hidden, 0x3333, 0.0, 0.02), "wu": orc.normal(width * hidden, 0x4444, 0.0, 0.02),
              "wd": orc.normal(hidden * width, 0x5555, 0.0, 0.02), "normalized": batch * width,
              "gate": batch * hidden, "upv": batch * hidden, "act": batch * hidden, "proj": batch * width,
              "out": batch * width}
    plan = [("norm", ["x", "gamma", "normalized"]), ("up", ["normalized", "wg", "gate"]),
            ("up", ["normalized", "wu", "upv"]), ("swiglu", ["gate", "upv", "act"]), ("down", ["act", "wd", "proj"]),
            ("add", ["proj", "x", "out"])]
    fused = _run_jobs(runtime, specs, arrays, plan, repeats=2,
                      launches=[("single", 0), ("gate_up_swiglu", 1), ("gemm_residual", 4)])
    alone = _run_jobs(runtime, specs, arrays, plan, one_at_a_time=True)
    for name in ("normalized", "gate", "upv", "act", "proj", "out"):
        np.testing.assert_array_equal(fused[name], alone[name], err_msg=name)
