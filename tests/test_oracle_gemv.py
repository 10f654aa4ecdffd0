"""Pins the oracle's decode GEMV (oracle_gemv_f16w) before it checks the HIP kernel.

  - the reference's golden vectors tests/golden/gemv_{a,b}_{w,x,y} (torch `w.float() @ x`, written
    by tools/export_kern_golden.py:41-47), under the reference's own gate (test_kern.cpp:96-120:
    max error / running peak <= 2e-5, cosine >= 1 - 1e-12), for the fp32-activation path; a wrong
    layout (transposed weights), a dropped tail and fp16-rounded activations all fail that gate;
  - exact small-integer products, where every partial sum is an integer below 2^24 so any summation
    order gives the exact integer result: both accumulation orders must equal the integer matmul;
  - the fp16-activation path equals the fp32 path applied to the fp16-rounded activations (the
    reference's gemv_fmlal rounds x with f32_to_f16 first, t2s_engine.cpp:696-700);
  - epilogue order: act(acc + bias) + residual, checked on values where other orders differ.
"""
import numpy as np
import pytest

from conftest import check_close, load_bin

import oracle as O

F32, F16 = O.F32, O.F16


@pytest.fixture(scope="module", autouse=True)
def _lib(oracle_lib):
    return oracle_lib


def golden(tag):
    w = load_bin(f"{tag}_w.f16")
    x = load_bin(f"{tag}_x.f32")
    y = load_bin(f"{tag}_y.f32")
    return w, x, y


@pytest.mark.parametrize("tag,shape", [("gemv_a", (128, 96)), ("gemv_b", (33, 131))])
def test_gemv_matches_reference_golden(tag, shape):
    w, x, y = golden(tag)
    assert w.shape == shape and x.shape == (shape[1],) and y.shape == (shape[0],)
    got = O.gemv_f16w(F32, x, w.view(np.uint16), F32, round_x=False)[0]
    ok, worst, cos = check_close(got, y, 2e-5, 1.0 - 1e-12)
    assert ok, (worst, cos)
    assert worst < 2e-6  # fp32 rounding level, far inside the gate


@pytest.mark.parametrize("tag", ["gemv_a", "gemv_b"])
def test_gemv_golden_gate_rejects_planted_mistakes(tag):
    w, x, y = golden(tag)
    w64, x64 = w.astype(np.float64), x.astype(np.float64)
    assert check_close(w64 @ x64, y, 2e-5, 1 - 1e-12)[0]
    mistakes = {
        "tail dropped": w64[:, :-3] @ x64[:-3],
        "x rounded to fp16": w64 @ x.astype(np.float16).astype(np.float64),
        "weights rolled by one column": np.roll(w64, 1, axis=1) @ x64,
    }
    if w.shape[0] == w.shape[1]:
        mistakes["transposed"] = w64.T @ x64
    for name, bad in mistakes.items():
        assert not check_close(bad, y, 2e-5, 1 - 1e-12)[0], name
    # and the oracle's fp16-activation mode is one of those: it must fail the fp32 golden gate
    got16 = O.gemv_f16w(F32, x, w.view(np.uint16), F32, round_x=True)[0]
    assert not check_close(got16, y, 2e-5, 1 - 1e-12)[0]


@pytest.mark.parametrize("rows,n_out,n_in", [(3, 17, 131), (2, 40, 512), (1, 1, 1), (5, 64, 7),
                                             (4, 9, 200)])
def test_gemv_exact_integer_products(rows, n_out, n_in):
    """Integer weights in [-8, 8] and activations in [-64, 64]: |partial sums| <= 512 n_in < 2^24,
    so every order of summation is exact; both oracle orders must equal the integer matmul."""
    r = np.random.default_rng(rows * 1000 + n_in)
    wi = r.integers(-8, 9, (n_out, n_in))
    xi = r.integers(-64, 65, (rows, n_in))
    w = wi.astype(np.float16).view(np.uint16)
    want = (xi @ wi.T).astype(np.float32)
    for round_x in (False, True):
        got = O.gemv_f16w(F32, xi.astype(np.float32), w, F32, round_x=round_x)
        assert np.array_equal(got, want), round_x
    got16 = O.gemv_f16w(F16, xi.astype(np.float16).view(np.uint16), w, F32)
    assert np.array_equal(got16, want)


def test_gemv_fp16_mode_is_fp32_mode_on_rounded_x():
    r = np.random.default_rng(7)
    x = r.standard_normal((4, 300)).astype(np.float32)
    w = (0.05 * r.standard_normal((50, 300))).astype(np.float16).view(np.uint16)
    xh = x.astype(np.float16)
    a = O.gemv_f16w(F32, x, w, F32, round_x=True)
    b = O.gemv_f16w(F16, xh.view(np.uint16), w, F32)
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32))
    # the rounded mode is the fmlal order, not the f32acc order on rounded values: the two agree
    # to fp32 accumulation noise only
    c = O.gemv_f16w(F32, xh.astype(np.float32), w, F32, round_x=False)
    assert np.max(np.abs(a - c)) <= 1e-5 * max(1.0, float(np.max(np.abs(c))))


def test_gemv_epilogue_order():
    """One weight column, K = 1: acc = x. bias, act and residual chosen so that other orders give
    other values: relu(acc + b) + res."""
    w = np.array([[1.0]], dtype=np.float16).view(np.uint16)
    x = np.array([[-3.0], [2.0], [-0.0]], dtype=np.float32)
    bias = np.array([1.0], dtype=np.float32)
    res = np.array([[5.0], [-1.0], [0.25]], dtype=np.float32)
    got = O.gemv_f16w(F32, x, w, F32, bias=bias, act=1, residual=res, round_x=False)
    # relu(-3 + 1) + 5 = 5 (relu after residual would give 3); relu(2 + 1) - 1 = 2; relu(1) + .25
    assert got.ravel().tolist() == [5.0, 2.0, 1.25]
    # no bias, no act: the sum itself (accumulators start at +0, so -0 products give +0)
    got = O.gemv_f16w(F32, x, w, F32, round_x=False)
    assert got.ravel().tolist() == [-3.0, 2.0, 0.0] and not np.signbit(got[2, 0])
    # LeakyReLU and fp16 storage of the result
    got = O.gemv_f16w(F32, x, w, F16, bias=bias, act=3, slope=0.1, round_x=False)
    assert O.to_f32(F16, got).ravel().tolist() == [np.float32(np.float16(-2.0 * np.float32(0.1))),
                                                   3.0, 1.0]
