"""RMSNorm, Softmax, SwiGLU and Add at the BASELINE configs and at the edge
shapes of each kernel's fast/generic paths, against the FP64 oracle."""
import numpy as np
import pytest

import oracle_binding as orc

pytestmark = pytest.mark.gpu

TOL = 1e-4


def run(runtime, spec, inputs, out_len):
    kernel = runtime.compile(spec)
    bufs = [runtime.resident(x) for x in inputs]
    out = runtime.alloc(out_len)
    runtime.execute([(kernel, bufs + [out])], 2)
    got = runtime.download(out)
    for x in bufs + [out]:
        x.free()
    return got


def assert_close(got, want, tol=TOL):
    check = orc.compare(got, want, tol, tol)
    assert check.status == 0, (check.first_bad, got[check.first_bad], want[check.first_bad])


@pytest.mark.parametrize("rows,cols", [(4096, 1024), (5, 4096), (3, 4100), (7, 1021), (1, 1), (9, 12), (2, 8192)])
def test_rms_norm(runtime, rows, cols):
    x = orc.normal(rows * cols, 0x1234)
    gamma = orc.values(cols, 0x7777, 0.5) + np.float32(1.0)  # U[0.5, 1.5)
    eps = 1e-6
    got = run(runtime, {"op": "rms_norm", "rows": rows, "cols": cols, "epsilon": eps}, [x, gamma], rows * cols)
    assert_close(got, orc.normalize(rows, cols, x, gamma, float(np.float32(eps))))


def test_softmax_config_32768x4096(runtime):
    rows, cols = 32768, 4096
    x = orc.normal(rows * cols, 0x6666, 0.0, 2.0)  # N(0, 4): variance 4, sigma 2
    got = run(runtime, {"op": "softmax", "rows": rows, "cols": cols}, [x], rows * cols).reshape(rows, cols)
    # Every row against the FP64 oracle, as the reference checks every row
    # (src/runtime/workloads.rs:134-142); in windows of 4096 rows to bound
    # the FP64 copy.
    xr = x.reshape(rows, cols)
    for r0 in range(0, rows, 4096):
        want = orc.softmax(4096, cols, xr[r0:r0 + 4096])
        assert_close(got[r0:r0 + 4096].reshape(-1), want)
    sums = got.astype(np.float64).sum(axis=1)
    assert np.abs(sums - 1.0).max() < 1e-5
    assert (got >= 0).all()


@pytest.mark.parametrize("rows,cols", [(64, 4096), (3, 17), (2, 257), (5, 4100), (4, 6000), (1, 1), (33, 64),
                                       (3, 1024), (2, 1020), (2, 2052), (2, 16384), (1, 16388), (3, 1536),
                                       (2, 2048), (2, 3000), (2, 8192), (2, 12000)])
def test_softmax_shapes(runtime, rows, cols):
    x = orc.normal(rows * cols, 0x4321, 0.0, 2.0)
    got = run(runtime, {"op": "softmax", "rows": rows, "cols": cols}, [x], rows * cols)
    assert_close(got, orc.softmax(rows, cols, x))


def test_softmax_handles_minus_infinity_entries(runtime):
    # Causal score rows hold -inf above the diagonal (metal_attention.rs:139-146).
    for cols in (16, 17, 5000):
        x = orc.normal(3 * cols, 0x99).reshape(3, cols)
        x[:, cols // 2:] = -np.inf
        got = run(runtime, {"op": "softmax", "rows": 3, "cols": cols}, [x.reshape(-1)], 3 * cols)
        want = np.exp(x.astype(np.float64) - x.max(axis=1, keepdims=True))
        want /= want.sum(axis=1, keepdims=True)
        assert_close(got, want.reshape(-1))


@pytest.mark.parametrize("n", [4096 * 2816, 10, 4097, 1, 3, 1 << 20])
def test_swiglu(runtime, n):
    gate, up = orc.normal(n, 0x8888, 0.0, 3.0), orc.normal(n, 0x9999)
    if n == 10:
        gate = np.array([-1000.0, -100.0, -20.0, -1.0, 0.0, 0.25, 1.0, 20.0, 100.0, 1000.0], np.float32)
    got = run(runtime, {"op": "swi_glu", "len": n}, [gate, up], n)
    assert_close(got, orc.swiglu(gate, up))


@pytest.mark.parametrize("n", [4096 * 1024, 257, 1, 6])
def test_add_and_axpy(runtime, n):
    a, b = orc.normal(n, 0x1), orc.normal(n, 0x2)
    got = run(runtime, {"op": "add", "len": n}, [a, b], n)
    np.testing.assert_array_equal(got, a + b)  # one f32 rounding, same as the FP64 sum rounded
    got = run(runtime, {"op": "axpy", "len": n, "alpha": -0.375}, [a, b], n)
    assert_close(got, -0.375 * a.astype(np.float64) + b.astype(np.float64), 3e-5)


def test_copy_expression_fast_path(runtime):
    n = 1 << 20
    a = orc.normal(n, 0x5)
    spec = {"op": "elementwise", "len": n, "inputs": 1, "expression": {"kind": "input", "binding": 0}}
    np.testing.assert_array_equal(run(runtime, spec, [a], n), a)


def test_expression_interpreter_eight_inputs(runtime):
    n = 1000
    xs = [orc.normal(n, 100 + i) for i in range(8)]
    e = {"kind": "input", "binding": 0}
    for i in range(1, 8):
        op = ["add", "multiply", "maximum"][i % 3]
        e = {"kind": op, "left": e, "right": {"kind": "input", "binding": i}}
    e = {"kind": "exp", "value": {"kind": "negate", "value": {"kind": "multiply", "left": e,
                                                               "right": {"kind": "constant", "value": 0.125}}}}
    got = run(runtime, {"op": "elementwise", "len": n, "inputs": 8, "expression": e}, xs, n)
    acc = xs[0].astype(np.float64)
    for i in range(1, 8):
        x = xs[i].astype(np.float64)
        acc = [acc + x, acc * x, np.maximum(acc, x)][i % 3]
    assert_close(got, np.exp(-(acc * 0.125)), 3e-5)


@pytest.mark.parametrize("cols,kernel,threads", [(1020, "softmax_cached", 256), (1024, "softmax_block", 256),
                                                 (2048, "softmax_block", 512), (4096, "softmax_block", 512),
                                                 (16384, "softmax_block", 512), (16388, "softmax_rows", 256),
                                                 (1025, "softmax_rows", 256)])
def test_softmax_kernel_choice(runtime, cols, kernel, threads):
    # Rows of 1024..16384 floats take one block per row (512 threads from 2048
    # columns); others one wave per row.
    launch = runtime.compile({"op": "softmax", "rows": 8, "cols": cols}).launch
    assert launch["kernel"] == kernel and launch["block"][0] == threads, launch
