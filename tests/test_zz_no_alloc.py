"""The allocation-free GEMM entry point (jr_gemm_f32_noalloc) against the
runtime's own GEMM path (jr_compile + jr_execute_dispatches) on the same
inputs: the same kernels, so the outputs must match bit for bit. The
split-K plans run through the static scratch array; two calls in a row, the
second smaller, show that what the first call left there does not leak into
the second."""
import ctypes

import numpy as np
import pytest

import oracle_binding as orc

pytestmark = pytest.mark.gpu


def _entry(lib):
    fn = lib.jr_gemm_f32_noalloc
    fn.restype = ctypes.c_int
    fn.argtypes = [ctypes.c_void_p] * 4 + [ctypes.c_uint32] * 3 + [ctypes.c_char_p, ctypes.c_size_t]
    return fn


def _device_sync():
    hip = ctypes.CDLL("libamdhip64.so")
    hip.hipDeviceSynchronize.restype = ctypes.c_int
    return hip.hipDeviceSynchronize()


def _runtime_gemm(rt, m, n, k, a, b):
    kernel = rt.compile({"op": "gemm", "m": m, "n": n, "k": k, "tiled": True})
    bufs = [rt.resident(a), rt.resident(b), rt.alloc(m * n)]
    rt.execute([(kernel, bufs)], 1)
    out = rt.download(bufs[2])
    for x in bufs:
        x.free()
    return out, kernel.description["workspace_bytes"]


def _noalloc_gemm(rt, fn, m, n, k, a, b):
    bufs = [rt.resident(a), rt.resident(b), rt.alloc(m * n)]
    err = ctypes.create_string_buffer(1024)
    print(f"jr_gemm_f32_noalloc {m}x{n}x{k}", flush=True)
    rc = fn(None, bufs[0].ptr, bufs[1].ptr, bufs[2].ptr, m, n, k, err, len(err))
    assert rc == 0, err.value
    assert _device_sync() == 0
    out = rt.download(bufs[2])
    for x in bufs:
        x.free()
    return out


@pytest.mark.parametrize("shapes", [
    ((256, 256, 4096), (96, 80, 700)),  # 64x64 split-K tiles, 4 MiB then 150 KB of scratch
    ((1, 4096, 4096), (16, 1024, 2816)),  # direct-load tiles split over K (few rows)
    ((512, 512, 512), (1000, 777, 513)),  # plans without split K (no scratch)
])
def test_noalloc_gemm_matches_runtime_path(runtime, shapes):
    fn = _entry(runtime._lib)
    for m, n, k in shapes:
        a = orc.values(m * k, 0x12345678, 1.0)
        b = orc.values(k * n, 0x9ABCDEF1, 1.0)
        want, workspace = _runtime_gemm(runtime, m, n, k, a, b)
        got = _noalloc_gemm(runtime, fn, m, n, k, a, b)
        np.testing.assert_array_equal(got, want)
        rows = (max(0, m - 8), m)
        ref = orc.gemm_reference(m, n, k, a, b, rows=rows)
        assert orc.compare(got[rows[0] * n:], ref, 1e-4, 1e-4).status == 0, (m, n, k, workspace)


def test_noalloc_rejects_bad_arguments(runtime):
    fn = _entry(runtime._lib)
    err = ctypes.create_string_buffer(1024)
    assert fn(None, None, None, None, 4, 4, 4, err, len(err)) == 1 and b"device pointers" in err.value
    buf = runtime.alloc(64)
    assert fn(None, buf.ptr, buf.ptr, buf.ptr, 0, 4, 4, err, len(err)) == 1
    assert fn(None, buf.ptr + 4, buf.ptr, buf.ptr, 4, 4, 4, err, len(err)) == 1 and b"16-byte" in err.value
    buf.free()


@pytest.mark.parametrize("m,n,k", [(256, 256, 4096), (1, 4096, 4096), (2048, 2048, 512)])
def test_noalloc_output_at_4_bytes(runtime, m, n, k):
    # Any 4-byte-aligned C is accepted. Split-K plans reduce into C with
    # 16-byte runs only where C (and the scratch) start 16-byte aligned; at
    # +4 bytes the reduce stores single floats, and the persistent kernel
    # single floats instead of pairs: the same bits as the runtime path.
    fn = _entry(runtime._lib)
    a = orc.values(m * k, 0x2468, 1.0)
    b = orc.values(k * n, 0x1357, 1.0)
    want, _ = _runtime_gemm(runtime, m, n, k, a, b)
    bufs = [runtime.resident(a), runtime.resident(b), runtime.alloc(m * n + 1)]
    err = ctypes.create_string_buffer(1024)
    print(f"jr_gemm_f32_noalloc {m}x{n}x{k}, C at +4 bytes", flush=True)
    assert fn(None, bufs[0].ptr, bufs[1].ptr, bufs[2].ptr + 4, m, n, k, err, len(err)) == 0, err.value
    assert _device_sync() == 0
    got = runtime.download(bufs[2])
    for x in bufs:
        x.free()
    assert got[0] == 0.0  # the float before C is untouched
    np.testing.assert_array_equal(got[1:], want)


def test_noalloc_under_graph_capture(runtime):
    # Calls captured on a non-blocking stream into a HIP graph (the callers
    # this entry is for): a split-K product first, then one on the persistent
    # kernel. The scratch address was looked up when the context was created,
    # so the capture holds kernel launches only. The graph is replayed three
    # times with the process's own eager work (zeroing the outputs) between
    # replays, and every replay must give the runtime path's bits.
    hip = ctypes.CDLL("libamdhip64.so")
    for name in ("hipStreamCreateWithFlags", "hipStreamBeginCapture", "hipStreamEndCapture", "hipGraphInstantiate",
                 "hipGraphLaunch", "hipStreamSynchronize", "hipGraphExecDestroy", "hipGraphDestroy",
                 "hipStreamDestroy"):
        getattr(hip, name).restype = ctypes.c_int
    fn = _entry(runtime._lib)
    shapes = [(256, 256, 4096), (2048, 2048, 512)]
    data, want, bufs = [], [], []
    for i, (m, n, k) in enumerate(shapes):
        a = orc.values(m * k, 0x3000 + i, 1.0)
        b = orc.values(k * n, 0x4000 + i, 1.0)
        want.append(_runtime_gemm(runtime, m, n, k, a, b)[0])
        bufs.append([runtime.resident(a), runtime.resident(b), runtime.alloc(m * n)])
    stream, graph, exe = ctypes.c_void_p(), ctypes.c_void_p(), ctypes.c_void_p()
    assert hip.hipStreamCreateWithFlags(ctypes.byref(stream), ctypes.c_uint(1)) == 0  # hipStreamNonBlocking
    err = ctypes.create_string_buffer(1024)
    print("capturing jr_gemm_f32_noalloc 256x256x4096 (split K) and 2048x2048x512 (persistent)", flush=True)
    assert hip.hipStreamBeginCapture(stream, ctypes.c_int(0)) == 0  # hipStreamCaptureModeGlobal
    codes = [fn(stream, g[0].ptr, g[1].ptr, g[2].ptr, m, n, k, err, len(err)) for (m, n, k), g in zip(shapes, bufs)]
    assert hip.hipStreamEndCapture(stream, ctypes.byref(graph)) == 0
    assert codes == [0, 0], err.value
    assert hip.hipGraphInstantiate(ctypes.byref(exe), graph, None, None, ctypes.c_size_t(0)) == 0
    try:
        for replay in range(3):
            for (m, n, _), g in zip(shapes, bufs):
                runtime.upload(g[2], np.zeros(m * n, np.float32))
            print(f"graph replay {replay}", flush=True)
            assert hip.hipGraphLaunch(exe, stream) == 0
            assert hip.hipStreamSynchronize(stream) == 0
            for w, g in zip(want, bufs):
                np.testing.assert_array_equal(runtime.download(g[2]), w)
    finally:
        hip.hipGraphExecDestroy(exe)
        hip.hipGraphDestroy(graph)
        hip.hipStreamDestroy(stream)
        for g in bufs:
            for x in g:
                x.free()
