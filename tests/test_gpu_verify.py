"""The reference's `verify` conformance suite (src/runtime/workloads.rs:56-320)
and its runtime-contract GPU tests (src/runtime/metal.rs:775-991), run through
the HIP C ABI. Every output is compared against the FP64 oracle."""
import ctypes
import math

import numpy as np
import pytest

import jade_hip
import oracle_binding as orc

pytestmark = pytest.mark.gpu


def values(n, seed, scale):
    return orc.values(n, seed, scale)


def verify_cases():
    """workloads::cases (src/runtime/workloads.rs:56-215)."""
    cases = []
    for n in (1, 257, 1025):
        a, b = values(n, 0x1234, 2.0), values(n, 0xABCD, 1.0)
        cases.append((f"axpy_{n}", {"op": "axpy", "len": n, "alpha": -0.375}, [a, b],
                      -0.375 * a.astype(np.float64) + b.astype(np.float64)))
    a, b = values(257, 0x1234, 2.0), values(257, 0xABCD, 1.0)
    cases.append(("add_257", {"op": "add", "len": 257}, [a, b], a.astype(np.float64) + b.astype(np.float64)))
    gate = np.array([-1000.0, -100.0, -20.0, -1.0, 0.0, 0.25, 1.0, 20.0, 100.0, 1000.0], np.float32)
    up = values(10, 0xAACC, 2.0)
    cases.append(("swiglu_extreme", {"op": "swi_glu", "len": 10}, [gate, up], orc.swiglu(gate, up)))
    for rows, cols in ((1, 1), (3, 17), (2, 257)):
        x, w = values(rows * cols, 0x1234, 2.0), values(cols, 0xABCD, 1.0)
        eps = np.float32(1e-5)
        cases.append((f"rmsnorm_{rows}_{cols}", {"op": "rms_norm", "rows": rows, "cols": cols, "epsilon": 1e-5},
                      [x, w], orc.normalize(rows, cols, x, w, float(eps))))
        xs = np.array([1000.0 if i // cols == 0 else (i % cols) * 0.25 - 10000.0 for i in range(rows * cols)],
                      np.float32)
        cases.append((f"softmax_{rows}_{cols}", {"op": "softmax", "rows": rows, "cols": cols}, [xs],
                      orc.softmax(rows, cols, xs)))
    for m, n, k in ((1, 1, 1), (31, 47, 19), (8, 33, 65)):
        for tiled in (False, True):
            a, b = values(m * k, 0x1234, 1.0), values(k * n, 0xABCD, 1.0)
            cases.append((f"gemm_{m}_{n}_{k}_tiled_{str(tiled).lower()}",
                          {"op": "gemm", "m": m, "n": n, "k": k, "tiled": tiled}, [a, b],
                          orc.gemm_reference(m, n, k, a, b)))
    relu = {"kind": "maximum",
            "left": {"kind": "add",
                     "left": {"kind": "multiply", "left": {"kind": "input", "binding": 0},
                              "right": {"kind": "constant", "value": 2.5}},
                     "right": {"kind": "input", "binding": 1}},
            "right": {"kind": "constant", "value": 0.0}}
    a, b = values(257, 0x1234, 1.0), values(257, 0xABCD, 1.0)
    cases.append(("custom_fused_axpy_relu", {"op": "elementwise", "len": 257, "inputs": 2, "expression": relu},
                  [a, b], np.maximum(a.astype(np.float64) * 2.5 + b.astype(np.float64), 0.0)))
    x = values(73, 0x9988, 1.0)
    cases.append(("custom_negate_exp",
                  {"op": "elementwise", "len": 73, "inputs": 1,
                   "expression": {"kind": "exp", "value": {"kind": "negate", "value": {"kind": "input",
                                                                                        "binding": 0}}}},
                  [x], np.exp(-x.astype(np.float64))))
    return cases


CASES = verify_cases()


@pytest.mark.parametrize("name,spec,inputs,expected", CASES, ids=[c[0] for c in CASES])
def test_verify_case(runtime, name, spec, inputs, expected):
    kernel = runtime.compile(spec)
    buffers = [runtime.resident(x) for x in inputs]
    out = runtime.alloc(expected.size)
    timing = runtime.execute([(kernel, buffers + [out])], 2)
    assert timing.dispatches == 2 and timing.repeats == 2
    check = orc.compare(runtime.download(out), expected, 3e-5, 3e-5)
    assert check.status == 0, (name, check.first_bad, check.max_abs_error)
    for b in buffers + [out]:
        b.free()


def test_verify_rejections(runtime):
    # src/runtime/workloads.rs:270-316: all rejected before any GPU work.
    kernel = runtime.compile({"op": "add", "len": 17})
    a, b, wrong = runtime.alloc(17), runtime.alloc(17), runtime.alloc(16)
    with pytest.raises(jade_hip.JadeError):
        runtime.upload(a, np.zeros(16, np.float32))
    with pytest.raises(jade_hip.JadeError):
        runtime.execute([(kernel, [a, b, a])], 1)
    with pytest.raises(jade_hip.JadeError):
        runtime.execute([(kernel, [a, b, wrong])], 1)
    with pytest.raises(jade_hip.JadeError):
        runtime.execute([], 1)
    with pytest.raises(jade_hip.JadeError):
        runtime.execute([(kernel, [a, b, wrong])], 0)


def test_same_rejections_at_the_c_boundary(runtime):
    """The C layer enforces the rules itself, not only the Python binding."""
    lib = runtime._lib
    kernel = runtime.compile({"op": "add", "len": 17})
    a, b, wrong = runtime.alloc(17), runtime.alloc(17), runtime.alloc(16)
    err = ctypes.create_string_buffer(1024)
    host = np.zeros(16, np.float32)
    assert lib.jr_upload(runtime._ctx, a.ptr, host.ctypes.data_as(ctypes.c_void_p), 64, err, 1024) == 1

    def run(buffers, repeats=1, count=None):
        arr = (ctypes.c_void_p * len(buffers))(*[x.ptr for x in buffers])
        job = (jade_hip._Dispatch * 1)()
        job[0].kernel = kernel.handle
        job[0].buffers = ctypes.cast(arr, ctypes.POINTER(ctypes.c_void_p))
        job[0].buffer_count = len(buffers) if count is None else count
        ms = ctypes.c_double()
        return lib.jr_execute_dispatches(runtime._ctx, job, 1, repeats, ctypes.byref(ms), err, 1024)

    assert run([a, b, a]) == 1 and b"alias" in err.value
    assert run([a, b, wrong]) == 1 and b"expected 17" in err.value
    assert run([a, b, b], repeats=0) == 1
    assert run([a, b]) == 1
    assert run([a, b, runtime.alloc(17)]) == 0


def test_ordering_ownership_and_alias_checks(runtime):
    # src/runtime/metal.rs:918-991.
    other = jade_hip.HipRuntime(0)
    try:
        a, b = runtime.alloc(5), runtime.alloc(5)
        intermediate, out = runtime.alloc(5), runtime.alloc(5)
        foreign = other.alloc(5)
        runtime.upload(a, [0.0, 1.0, -2.0, 3.0, 1.0])
        runtime.upload(b, [-1.0, 2.0, 3.0, -4.0, 7.0])
        with pytest.raises(jade_hip.JadeError):
            runtime.upload(a, [1.0])
        with pytest.raises(jade_hip.JadeError):
            runtime.upload(foreign, np.zeros(5))
        with pytest.raises(jade_hip.JadeError):
            runtime.download(foreign)
        spec = {"op": "add", "len": 5}
        add, foreign_add = runtime.compile(spec), other.compile(spec)
        with pytest.raises(jade_hip.JadeError):
            runtime.execute([(foreign_add, [a, b, out])], 1)
        with pytest.raises(jade_hip.JadeError):
            runtime.execute([(add, [a, b, a])], 1)
        with pytest.raises(jade_hip.JadeError):
            runtime.execute([(add, [a, b, intermediate]), (add, [intermediate, foreign, out])], 1)
        np.testing.assert_array_equal(runtime.download(intermediate), np.zeros(5))
        jobs = [(add, [a, b, intermediate]), (add, [intermediate, b, out])]
        with pytest.raises(jade_hip.JadeError):
            runtime.execute(jobs, 0)
        timing = runtime.execute(jobs, 3)
        assert timing.dispatches == 6 and timing.repeats == 3
        np.testing.assert_array_equal(runtime.download(out), [-2.0, 5.0, 4.0, -5.0, 15.0])
        assert math.isfinite(timing.host_ms) and timing.host_ms > 0
        assert timing.gpu_ms is None or (math.isfinite(timing.gpu_ms) and timing.gpu_ms > 0)
    finally:
        other.close()


def test_mixed_gemm_add_batch_ordering_and_rejection(runtime):
    # src/runtime/metal.rs:825-916 with this backend's GEMM in place of MPS.
    other = jade_hip.HipRuntime(0)
    try:
        a, b, bias = runtime.resident([1, 2, 3, 4]), runtime.resident([2, 0, 1, 2]), runtime.resident(
            [1, -1, 2, -2])
        ab, shifted, out = runtime.resident([11, 12, 13, 14]), runtime.alloc(4), runtime.alloc(4)
        foreign = other.alloc(4)
        spec = {"op": "gemm", "m": 2, "n": 2, "k": 2, "tiled": True}
        gemm, foreign_gemm = runtime.compile(spec), other.compile(spec)
        add = runtime.compile({"op": "add", "len": 4})
        with pytest.raises(jade_hip.JadeError):
            runtime.execute([(gemm, [a, b, ab]), (add, [ab, foreign, shifted])], 1)
        np.testing.assert_array_equal(runtime.download(ab), [11, 12, 13, 14])
        with pytest.raises(jade_hip.JadeError):
            runtime.execute([(gemm, [a, b, ab]), (foreign_gemm, [ab, b, out])], 1)
        np.testing.assert_array_equal(runtime.download(ab), [11, 12, 13, 14])
        with pytest.raises(jade_hip.JadeError):
            runtime.execute([(gemm, [a, b, a])], 1)
        jobs = [(gemm, [a, b, ab]), (add, [ab, bias, shifted]), (gemm, [shifted, b, out])]
        timing = runtime.execute(jobs, 3)
        assert timing.dispatches == 9 and timing.repeats == 3
        np.testing.assert_array_equal(runtime.download(ab), [4, 4, 10, 8])
        np.testing.assert_array_equal(runtime.download(shifted), [5, 3, 12, 6])
        np.testing.assert_array_equal(runtime.download(out), [13, 6, 30, 12])
        np.testing.assert_array_equal(runtime.download(a), [1, 2, 3, 4])
        np.testing.assert_array_equal(runtime.download(b), [2, 0, 1, 2])
    finally:
        other.close()


def test_gemm_packed_fp32_and_ownership(runtime):
    # src/runtime/metal.rs:775-823 with validation::inputs and validation::check.
    for m, n, k in ((1, 1, 1), (2, 3, 2), (17, 31, 19), (64, 64, 64)):
        av, bv = orc.inputs(m, n, k)
        a, b, out = runtime.resident(av), runtime.resident(bv), runtime.alloc(m * n)
        kernel = runtime.compile({"op": "gemm_simd", "m": m, "n": n, "k": k})
        timing = runtime.execute([(kernel, [a, b, out])], 3)
        assert timing.dispatches == 3 and timing.repeats == 3
        result = orc.check_gemm(m, n, k, av, bv, runtime.download(out), 1 << 62)
        assert result.status == 0 and result.checked_elements == m * n
    a, b, out, short = runtime.alloc(4), runtime.alloc(4), runtime.alloc(4), runtime.alloc(3)
    kernel = runtime.compile({"op": "gemm_simd", "m": 2, "n": 2, "k": 2})
    for buffers in ([a, b, a], [a, b, b], [short, b, out]):
        with pytest.raises(jade_hip.JadeError):
            runtime.execute([(kernel, buffers)], 1)
    with pytest.raises(jade_hip.JadeError):
        runtime.execute([(kernel, [a, b, out])], 0)
    np.testing.assert_array_equal(runtime.download(out), np.zeros(4))
    runtime.upload(a, [1, 2, 3, 4])
    runtime.execute([(kernel, [a, a, out])], 1)  # read/read aliasing is valid
    np.testing.assert_array_equal(runtime.download(out), [7, 10, 15, 22])
    with pytest.raises(jade_hip.JadeError):
        runtime.compile({"op": "gemm_mps", "m": 2, "n": 2, "k": 2})


def test_allocations_are_zeroed_and_pipelines_cached(runtime):
    buf = runtime.alloc(1000)
    np.testing.assert_array_equal(runtime.download(buf), np.zeros(1000))
    k1 = runtime.compile({"op": "softmax", "rows": 3, "cols": 17})
    k2 = runtime.compile('{"cols": 17, "rows": 3, "op": "softmax"}')
    assert k1.handle == k2.handle
    k2.release()
    out = runtime.alloc(51)
    runtime.execute([(k1, [runtime.resident(np.zeros(51)), out])], 1)  # still alive after one release
    np.testing.assert_allclose(runtime.download(out), np.full(51, 1.0 / 17), rtol=1e-6)


LAUNCH = ctypes.CFUNCTYPE(ctypes.c_int, ctypes.c_void_p, ctypes.POINTER(ctypes.c_void_p))


def test_raw_launcher_path(runtime):
    """ABI-1 jr_execute with caller launchers (jade_runtime_corex.cpp:148-189)."""
    lib = runtime._lib
    calls = []
    ok = LAUNCH(lambda stream, buffers: calls.append(1) or 0)
    bad = LAUNCH(lambda stream, buffers: 1)
    buf = runtime.alloc(4)
    ptrs = (ctypes.c_void_p * 1)(buf.ptr)
    jobs = (jade_hip._Job * 2)()
    for j, fn in enumerate((ok, ok)):
        jobs[j].launch = ctypes.cast(fn, ctypes.c_void_p)
        jobs[j].buffers = ctypes.cast(ptrs, ctypes.POINTER(ctypes.c_void_p))
        jobs[j].buffer_count = 1
    err = ctypes.create_string_buffer(1024)
    ms = ctypes.c_double()
    assert lib.jr_execute(runtime._ctx, jobs, 2, 3, ctypes.byref(ms), err, 1024) == 0
    assert len(calls) == 6 and ms.value >= 0
    jobs[1].launch = ctypes.cast(bad, ctypes.c_void_p)
    assert lib.jr_execute(runtime._ctx, jobs, 2, 1, ctypes.byref(ms), err, 1024) == 2
    assert lib.jr_execute(runtime._ctx, jobs, 0, 1, ctypes.byref(ms), err, 1024) == 1
