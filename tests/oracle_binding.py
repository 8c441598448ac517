"""ctypes binding of oracle/liboracle.so, the FP64 CPU oracle.

Test infrastructure only: loaded by tests/, __graft_entry__.smoke() and the
cpu_baseline leg of bench.py, always as the checker or the timed CPU
baseline, never on the product path.
"""
import ctypes as _c
import os

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
LIBRARY_PATH = os.path.join(ROOT, "oracle", "liboracle.so")
THREADS = max(1, min(16, os.cpu_count() or 1))

_vp = _c.c_void_p


class Check(_c.Structure):
    _fields_ = [("elements", _c.c_size_t), ("max_abs_error", _c.c_double), ("max_relative_error", _c.c_double),
                ("status", _c.c_int), ("first_bad", _c.c_size_t)]


class Validation(_c.Structure):
    _fields_ = [("checked_elements", _c.c_size_t), ("max_abs_error", _c.c_double),
                ("max_scaled_error", _c.c_double), ("status", _c.c_int), ("first_bad", _c.c_size_t)]


def _load():
    if not os.path.exists(LIBRARY_PATH):
        raise FileNotFoundError(f"{LIBRARY_PATH} missing; run make -C oracle")
    lib = _c.CDLL(LIBRARY_PATH)
    u32, sz, i32, f32, f64 = _c.c_uint32, _c.c_size_t, _c.c_int, _c.c_float, _c.c_double
    lib.or_xorshift32.restype = u32
    lib.or_xorshift32.argtypes = [u32]
    lib.or_values.argtypes = [_vp, sz, u32, f32]
    lib.or_fill.argtypes = [_vp, sz, u32]
    lib.or_normal.argtypes = [_vp, sz, u32, f32, f32]
    lib.or_gemm_reference.argtypes = [u32, u32, u32, _vp, _vp, _vp, u32, u32, i32]
    lib.or_dot.argtypes = [sz, sz, sz, _vp, _vp, _vp, i32]
    lib.or_attention_reference.restype = i32
    lib.or_attention_reference.argtypes = [u32, u32, u32, i32, _vp, _vp, _vp, _vp, u32, u32, i32]
    lib.or_sigmoid.restype = f64
    lib.or_sigmoid.argtypes = [f64]
    lib.or_normalize.argtypes = [sz, sz, _vp, _vp, f64, _vp, i32]
    lib.or_softmax.argtypes = [sz, sz, _vp, _vp, i32]
    lib.or_swiglu.argtypes = [sz, _vp, _vp, _vp]
    lib.or_mlp.restype = i32
    lib.or_mlp.argtypes = [sz, sz, sz, _vp, _vp, _vp, _vp, _vp, f64, _vp, i32]
    lib.or_compare.argtypes = [_vp, _vp, sz, f64, f64, _c.POINTER(Check)]
    lib.or_check_gemm.argtypes = [u32, u32, u32, _vp, _vp, _vp, sz, i32, _c.POINTER(Validation)]
    return lib


lib = _load()


def _p(a):
    return a.ctypes.data_as(_vp)


def _f32(a):
    return np.ascontiguousarray(a, dtype=np.float32).reshape(-1)


def _f64(a):
    return np.ascontiguousarray(a, dtype=np.float64).reshape(-1)


def xorshift32(state):
    return lib.or_xorshift32(state & 0xFFFFFFFF)


def values(length, seed, scale=1.0):
    out = np.empty(length, np.float32)
    lib.or_values(_p(out), length, seed & 0xFFFFFFFF, scale)
    return out


def fill(length, seed):
    out = np.empty(length, np.float32)
    lib.or_fill(_p(out), length, seed & 0xFFFFFFFF)
    return out


def inputs(m, n, k):
    """validation::inputs (src/validation.rs:6-21)."""
    return fill(m * k, 0x12345678), fill(k * n, 0x9ABCDEF1)


def normal(length, seed, mean=0.0, sigma=1.0):
    out = np.empty(length, np.float32)
    lib.or_normal(_p(out), length, seed & 0xFFFFFFFF, mean, sigma)
    return out


def gemm_reference(m, n, k, a, b, rows=None, threads=THREADS):
    a, b = _f32(a), _f32(b)
    r0, r1 = (0, m) if rows is None else rows
    out = np.empty((r1 - r0) * n, np.float64)
    lib.or_gemm_reference(m, n, k, _p(a), _p(b), _p(out), r0, r1, threads)
    return out


def dot(m, n, k, a, b, threads=THREADS):
    a, b = _f64(a), _f64(b)
    out = np.empty(m * n, np.float64)
    lib.or_dot(m, n, k, _p(a), _p(b), _p(out), threads)
    return out


def attention_reference(heads, seq, dim, causal, q, k, v, rows=None, threads=THREADS):
    q, k, v = _f32(q), _f32(k), _f32(v)
    r0, r1 = (0, seq) if rows is None else rows
    out = np.empty(heads * (r1 - r0) * dim, np.float64)
    if lib.or_attention_reference(heads, seq, dim, 1 if causal else 0, _p(q), _p(k), _p(v), _p(out), r0, r1,
                                  threads):
        raise MemoryError("or_attention_reference: score buffer allocation failed")
    return out


def sigmoid(x):
    return lib.or_sigmoid(float(x))


def normalize(rows, cols, x, weight, eps, threads=THREADS):
    x, weight = _f64(x), _f64(weight)
    out = np.empty(rows * cols, np.float64)
    lib.or_normalize(rows, cols, _p(x), _p(weight), eps, _p(out), threads)
    return out


def softmax(rows, cols, x, threads=THREADS):
    x = _f32(x)
    out = np.empty(rows * cols, np.float64)
    lib.or_softmax(rows, cols, _p(x), _p(out), threads)
    return out


def swiglu(gate, up):
    gate, up = _f32(gate), _f32(up)
    out = np.empty(gate.size, np.float64)
    lib.or_swiglu(gate.size, _p(gate), _p(up), _p(out))
    return out


def mlp(batch, width, hidden, x, norm, wg, wu, wd, eps, threads=THREADS):
    x, norm, wg, wu, wd = (_f32(t) for t in (x, norm, wg, wu, wd))
    out = np.empty(batch * width, np.float64)
    if lib.or_mlp(batch, width, hidden, _p(x), _p(norm), _p(wg), _p(wu), _p(wd), eps, _p(out), threads):
        raise MemoryError("or_mlp: FP64 intermediate allocation failed")
    return out


def compare(actual, expected, atol, rtol):
    """workloads::compare; returns the Check (status 0 = pass)."""
    actual, expected = _f32(actual), _f64(expected)
    assert actual.size == expected.size, "oracle length mismatch"
    result = Check()
    lib.or_compare(_p(actual), _p(expected), actual.size, atol, rtol, _c.byref(result))
    return result


def check_gemm(m, n, k, a, b, out, budget, fp16=False):
    """validation::check; returns the Validation (status 0 = pass)."""
    a, b, out = _f32(a), _f32(b), _f32(out)
    result = Validation()
    lib.or_check_gemm(m, n, k, _p(a), _p(b), _p(out), budget, 1 if fp16 else 0, _c.byref(result))
    return result
