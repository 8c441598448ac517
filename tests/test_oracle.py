"""Pins the FP64 CPU oracle (oracle/oracle.c) before any GPU result is judged
against it. Each check is a textbook known answer, a vector from the
reference's own unit tests, a closed form, or agreement with an independent
numpy float64 library routine, chosen so a dropped term, a wrong sign or
index, or a transposed operand fails.
"""
import math
from fractions import Fraction

import numpy as np
import pytest

import oracle_binding as orc


# ---- A1: xorshift32 and the value maps --------------------------------------

def test_xorshift32_textbook_sequence():
    # Marsaglia, "Xorshift RNGs", J. Stat. Softw. 8(14), 2003: xor32 with
    # y = 2463534242 and shifts (13, 17, 5) starts 723471715, 2497366906, 2064144800.
    s = 2463534242
    seen = []
    for _ in range(3):
        s = orc.xorshift32(s)
        seen.append(s)
    assert seen == [723471715, 2497366906, 2064144800]


def _exact_values(length, seed, scale):
    """(s>>8)/2^24*2-1 is exact in f32; only `* scale` rounds (checked with
    exact rationals, then one correctly rounded f32 product)."""
    s = seed
    out = []
    for _ in range(length):
        s = orc.xorshift32(s)
        unit = Fraction(s >> 8, 1 << 24) * 2 - 1
        unit32 = np.float32(float(unit))
        assert Fraction(float(unit32)) == unit  # representable exactly
        out.append(np.float32(unit32 * np.float32(scale)))
    return np.array(out, dtype=np.float32)


@pytest.mark.parametrize("seed,scale", [(0x1234, 1.0), (0xABCD, 2.0), (0x3333, 1.0 / math.sqrt(1024)),
                                        (0x9988, 1.0), (0xAACC, 2.0)])
def test_values_match_exact_rational_map(seed, scale):
    got = orc.values(257, seed, scale)
    np.testing.assert_array_equal(got, _exact_values(257, seed, scale))
    assert np.all(np.abs(got) <= abs(np.float32(scale)))


def test_values_first_elements():
    # Restated from src/runtime/workloads.rs:17-27 and src/validation.rs:6-21.
    np.testing.assert_allclose(orc.values(4, 0x1234, 1.0),
                               [-0.41732967, -0.48519719, 0.77535272, -0.34298933], rtol=0, atol=5e-8)
    np.testing.assert_allclose(orc.values(4, 0xABCD, 1.0),
                               [0.45584667, -0.17299449, -0.01073086, 0.73545587], rtol=0, atol=5e-8)
    a, b = orc.inputs(2, 2, 2)
    np.testing.assert_allclose(a, [0.05933690, -0.83315611, -0.43649435, 0.01329565], rtol=0, atol=5e-8)
    np.testing.assert_allclose(b, [-0.64656949, 0.91684008, -0.64630735, -0.93583941], rtol=0, atol=5e-8)


def test_fill_equals_values_with_unit_scale():
    # validation::inputs uses the same map without the scale factor.
    np.testing.assert_array_equal(orc.fill(1000, 0x12345678), orc.values(1000, 0x12345678, 1.0))


def test_values_are_uniform_on_unit_interval():
    v = orc.values(1 << 20, 0x1234, 1.0).astype(np.float64)
    assert v.min() >= -1.0 and v.max() < 1.0
    assert abs(v.mean()) < 3e-3 and abs(v.var() - 1.0 / 3.0) < 3e-3


def test_normal_generator_is_box_muller_over_xorshift():
    # Documented addition: recompute with Python's math library.
    s = 0x1111
    expected = []
    for _ in range(64):
        s = orc.xorshift32(s)
        u1 = ((s >> 8) + 1) / 16777216.0
        s = orc.xorshift32(s)
        u2 = (s >> 8) / 16777216.0
        expected.append(np.float32(0.5 + 2.0 * (math.sqrt(-2.0 * math.log(u1)) * math.cos(2.0 * math.pi * u2))))
    np.testing.assert_array_equal(orc.normal(64, 0x1111, 0.5, 2.0), np.array(expected, np.float32))
    z = orc.normal(1 << 20, 0x2222).astype(np.float64)
    assert abs(z.mean()) < 5e-3 and abs(z.std() - 1.0) < 5e-3
    assert abs(np.mean(z ** 4) - 3.0) < 0.05  # normal kurtosis


# ---- A12: GEMM / dot --------------------------------------------------------

def test_gemm_reference_unit_test_vectors():
    # src/validation.rs:101-112: A=[1,2,-3,4] (2x2), B=[1..6] (2x3).
    np.testing.assert_array_equal(orc.gemm_reference(2, 3, 2, [1, 2, -3, 4], [1, 2, 3, 4, 5, 6]),
                                  [9, 12, 15, 13, 14, 15])
    # src/runtime/metal.rs:818-822: read/read aliasing [1,2,3,4]^2.
    np.testing.assert_array_equal(orc.gemm_reference(2, 2, 2, [1, 2, 3, 4], [1, 2, 3, 4]), [7, 10, 15, 22])
    # src/runtime/metal.rs:893-914: ab, ab + bias, (ab + bias) b.
    a, b, bias = [1, 2, 3, 4], [2, 0, 1, 2], np.array([1, -1, 2, -2], np.float64)
    ab = orc.gemm_reference(2, 2, 2, a, b)
    np.testing.assert_array_equal(ab, [4, 4, 10, 8])
    np.testing.assert_array_equal(ab + bias, [5, 3, 12, 6])
    np.testing.assert_array_equal(orc.gemm_reference(2, 2, 2, ab + bias, b), [13, 6, 30, 12])


@pytest.mark.parametrize("m,n,k", [(1, 1, 1), (7, 9, 13), (31, 47, 19), (65, 33, 17), (3, 5, 257),
                                   (127, 65, 129)])
def test_gemm_reference_matches_numpy(m, n, k):
    a = orc.values(m * k, 0x1234, 1.0)
    b = orc.values(k * n, 0xABCD, 1.0)
    want = a.astype(np.float64).reshape(m, k) @ b.astype(np.float64).reshape(k, n)
    np.testing.assert_allclose(orc.gemm_reference(m, n, k, a, b), want.reshape(-1), rtol=1e-13, atol=1e-13)
    np.testing.assert_allclose(orc.dot(m, n, k, a, b), want.reshape(-1), rtol=1e-13, atol=1e-13)


def test_gemm_reference_row_window_and_threads_agree():
    m, n, k = 37, 29, 23
    a, b = orc.inputs(m, n, k)
    full = orc.gemm_reference(m, n, k, a, b, threads=1)
    np.testing.assert_array_equal(orc.gemm_reference(m, n, k, a, b, threads=4), full)
    np.testing.assert_array_equal(orc.gemm_reference(m, n, k, a, b, rows=(5, 17)), full[5 * n:17 * n])


# ---- A12: attention ---------------------------------------------------------

def test_attention_reference_unit_test_vector():
    # src/runtime/metal_lab.rs:472-484.
    q = np.zeros(6)
    v = [1.0, 2.0, 3.0, 4.0, 8.0, 9.0]
    np.testing.assert_array_equal(orc.attention_reference(1, 3, 2, False, q, q, v), [4, 5, 4, 5, 4, 5])
    np.testing.assert_array_equal(orc.attention_reference(1, 3, 2, True, q, q, v), [1, 2, 2, 3, 4, 5])


def _numpy_attention(h, s, d, causal, q, k, v):
    q = q.astype(np.float64).reshape(h, s, d)
    k = k.astype(np.float64).reshape(h, s, d)
    v = v.astype(np.float64).reshape(h, s, d)
    scores = q @ np.swapaxes(k, 1, 2) / math.sqrt(d)
    if causal:
        scores = np.where(np.tril(np.ones((s, s), bool)), scores, -np.inf)
    scores -= scores.max(axis=-1, keepdims=True)
    p = np.exp(scores)
    p /= p.sum(axis=-1, keepdims=True)
    return (p @ v).reshape(-1)


@pytest.mark.parametrize("h,s,d,causal,amp", [(1, 1, 1, False, 1.0), (2, 7, 17, False, 1.0), (2, 7, 17, True, 1.0),
                                              (2, 33, 64, True, 1.0), (2, 17, 64, True, 20.0)])
def test_attention_reference_matches_numpy(h, s, d, causal, amp):
    n = h * s * d
    q, k, v = orc.values(n, 0x1111, amp), orc.values(n, 0x2222, amp), orc.values(n, 0x3333, 1.0)
    want = _numpy_attention(h, s, d, causal, q, k, v)
    got = orc.attention_reference(h, s, d, causal, q, k, v)
    np.testing.assert_allclose(got, want, rtol=1e-11, atol=1e-12)
    window = orc.attention_reference(h, s, d, causal, q, k, v, rows=(2, 5) if s > 5 else (0, s))
    r0, r1 = (2, 5) if s > 5 else (0, s)
    np.testing.assert_allclose(window.reshape(h, r1 - r0, d), want.reshape(h, s, d)[:, r0:r1], rtol=1e-11,
                               atol=1e-12)


def test_attention_reference_invariants():
    h, s, d = 2, 9, 5
    q, k, v = orc.values(h * s * d, 7, 1.0), orc.values(h * s * d, 8, 1.0), orc.values(h * s * d, 9, 1.0)
    out = orc.attention_reference(h, s, d, True, q, k, v).reshape(h, s, d)
    vv = v.astype(np.float64).reshape(h, s, d)
    np.testing.assert_allclose(out[:, 0], vv[:, 0], rtol=0, atol=0)  # causal row 0 is V[0]
    lo, hi = vv.min(axis=1), vv.max(axis=1)  # convex combinations of V rows
    assert np.all(out >= lo[:, None, :] - 1e-12) and np.all(out <= hi[:, None, :] + 1e-12)


# ---- A5-A7: RMSNorm, Softmax, SwiGLU ----------------------------------------

def test_normalize_closed_forms():
    eps = 1e-5
    np.testing.assert_allclose(orc.normalize(1, 1, [3.0], [2.0], eps), [3.0 / math.sqrt(9.0 + eps) * 2.0],
                               rtol=1e-15)
    row = np.full(17, -1.5)
    w = orc.values(17, 0xABCD, 1.0).astype(np.float64)
    np.testing.assert_allclose(orc.normalize(1, 17, row, w, eps), -1.5 / math.sqrt(2.25 + eps) * w, rtol=1e-14)
    x = orc.values(3 * 17, 0x1234, 2.0).astype(np.float64).reshape(3, 17)
    want = x / np.sqrt((x * x).mean(axis=1, keepdims=True) + eps) * w
    np.testing.assert_allclose(orc.normalize(3, 17, x, w, eps), want.reshape(-1), rtol=1e-13)


@pytest.mark.parametrize("rows,cols", [(1, 1), (3, 17), (2, 257)])
def test_softmax_closed_forms(rows, cols):
    # src/runtime/workloads.rs:125-133: row 0 all 1000; rows >= 1 0.25*j - 10000.
    x = np.array([1000.0 if i // cols == 0 else (i % cols) * 0.25 - 10000.0 for i in range(rows * cols)],
                 np.float32)
    got = orc.softmax(rows, cols, x).reshape(rows, cols)
    np.testing.assert_allclose(got[0], np.full(cols, 1.0 / cols), rtol=1e-15)
    j = np.arange(cols, dtype=np.float64)
    ramp = np.exp(0.25 * (j - (cols - 1)))
    for r in range(1, rows):
        np.testing.assert_allclose(got[r], ramp / ramp.sum(), rtol=1e-12)
    np.testing.assert_allclose(got.sum(axis=1), 1.0, rtol=1e-14)


def test_sigmoid_and_swiglu():
    assert orc.sigmoid(0.0) == 0.5
    for x in [-30.0, -1.0, 0.25, 2.0, 30.0]:
        assert orc.sigmoid(x) == pytest.approx(1.0 / (1.0 + math.exp(-x)), rel=1e-15)
        assert orc.sigmoid(-x) == pytest.approx(1.0 - orc.sigmoid(x), abs=4e-16)
    gate = np.array([-1000.0, -100.0, -20.0, -1.0, 0.0, 0.25, 1.0, 20.0, 100.0, 1000.0], np.float32)
    up = orc.values(10, 0xAACC, 2.0)
    got = orc.swiglu(gate, up)
    assert got[0] == 0.0 and got[4] == 0.0  # saturated off and exact zero gate
    assert got[-1] == pytest.approx(1000.0 * float(up[-1]), rel=1e-15)
    assert got[-2] == pytest.approx(100.0 * float(up[-2]), rel=1e-15)
    assert abs(got[1]) < 1e-40
    assert got[6] == pytest.approx(1.0 / (1.0 + math.exp(-1.0)) * float(up[6]), rel=1e-15)


# ---- A9: residual MLP -------------------------------------------------------

def test_mlp_matches_numpy_composition():
    batch, width, hidden, eps = 5, 16, 24, 1e-6
    x = orc.normal(batch * width, 0x1234)
    norm = orc.values(width, 0x7777, 0.5) + np.float32(1.0)
    wg = orc.normal(width * hidden, 0x3333, 0.0, 0.02)
    wu = orc.normal(width * hidden, 0x4444, 0.0, 0.02)
    wd = orc.normal(hidden * width, 0x5555, 0.0, 0.02)
    X = x.astype(np.float64).reshape(batch, width)
    n = X / np.sqrt((X * X).mean(axis=1, keepdims=True) + eps) * norm.astype(np.float64)
    g = n @ wg.astype(np.float64).reshape(width, hidden)
    u = n @ wu.astype(np.float64).reshape(width, hidden)
    act = g / (1.0 + np.exp(-g)) * u
    want = act @ wd.astype(np.float64).reshape(hidden, width) + X
    got = orc.mlp(batch, width, hidden, x, norm, wg, wu, wd, eps)
    np.testing.assert_allclose(got, want.reshape(-1), rtol=1e-12, atol=1e-14)
    # Rows are independent: a row window of the batch equals the same rows.
    part = orc.mlp(2, width, hidden, x[width:3 * width], norm, wg, wu, wd, eps)
    np.testing.assert_array_equal(part, got[width:3 * width])


# ---- A11: comparators -------------------------------------------------------

def test_compare_unit_test_vectors():
    # src/runtime/workloads.rs:536-539.
    assert orc.compare([0.0], [1.0], 1e-5, 1e-5).status == 2
    assert orc.compare([np.nan], [0.0], 1e-5, 1e-5).status == 1
    ok = orc.compare([1.0, 2.0001], [1.0, 2.0], 1e-4, 1e-4)
    assert ok.status == 0
    assert ok.max_abs_error == float(np.float32(2.0001)) - 2.0
    assert ok.max_relative_error == pytest.approx(ok.max_abs_error / 2.0)
    # Near zero the relative measure is taken against max(|e|, atol).
    small = orc.compare([1e-6], [0.0], 1e-5, 1e-5)
    assert small.status == 0 and small.max_relative_error == pytest.approx(0.1, rel=1e-3)


def test_check_gemm_unit_test_vectors():
    # src/validation.rs:101-112.
    a, b = [1, 2, -3, 4], [1, 2, 3, 4, 5, 6]
    c = np.array([9, 12, 15, 13, 14, 15], np.float32)
    assert orc.check_gemm(2, 3, 2, a, b, c, 1 << 60).status == 0
    c[5] = 0.0
    assert orc.check_gemm(2, 3, 2, a, b, c, 1 << 60).status == 2
    c[5] = np.nan
    assert orc.check_gemm(2, 3, 2, a, b, c, 1).status == 1
    assert orc.check_gemm(2, 3, 2, a, b, c, 0).status == 3


def test_check_gemm_samples_both_ends():
    m, n, k = 9, 11, 7
    a, b = orc.inputs(m, n, k)
    good = orc.gemm_reference(m, n, k, a, b).astype(np.float32)
    for idx in (0, m * n - 1):
        bad = good.copy()
        bad[idx] += 1.0
        assert orc.check_gemm(m, n, k, a, b, bad, 2).status == 2
    assert orc.check_gemm(m, n, k, a, b, good, 2).checked_elements == 2
