"""Pins the CPU oracle before the GPU kernels are compared against it.

Every oracle function is checked against the reference's own golden vectors where they exist
(tests/golden/*.f32 are the reference's tests/kern_golden files, unmodified) and otherwise against
what the mathematics fixes: float64 closed forms, exact rational arithmetic, identities and
special cases. Some checks also plant a plausible mistake (in a numpy copy of the formula, on the
CPU) and assert that the same gate rejects it, so the gate is shown to have teeth.
"""
import math
from fractions import Fraction

import numpy as np
import pytest

from conftest import check_close, load_bin

import oracle as O


@pytest.fixture(scope="module", autouse=True)
def _lib(oracle_lib):
    return oracle_lib


# ---- a1: kern::layernorm against the reference golden (test_kern.cpp:207-216) -------------------

def test_layernorm_matches_reference_golden():
    x, g, b, y = (load_bin(f"ln_{k}.f32") for k in "xgby")
    assert x.shape == (5, 512)
    got = np.stack([O.layernorm_row(x[r], g, b, 1e-5) for r in range(x.shape[0])])
    ok, worst, cos = check_close(got, y, 1e-5, 1.0 - 1e-12)
    assert ok, (worst, cos)
    # the oracle is far tighter than the gate: fp32 rounding level
    assert worst < 2e-6


def test_layernorm_golden_gate_rejects_planted_mistakes():
    """The same gate fails for plausible wrong formulas (computed in numpy, float64)."""
    x, g, b, y = (load_bin(f"ln_{k}.f32") for k in "xgby")
    x64 = x.astype(np.float64)
    mu = x64.mean(1, keepdims=True)
    var_biased = ((x64 - mu) ** 2).mean(1, keepdims=True)
    good = (x64 - mu) / np.sqrt(var_biased + 1e-5) * g + b
    assert check_close(good, y, 1e-5, 1 - 1e-12)[0]
    var_unbiased = ((x64 - mu) ** 2).sum(1, keepdims=True) / (x.shape[1] - 1)
    mistakes = {
        "unbiased variance": (x64 - mu) / np.sqrt(var_unbiased + 1e-5) * g + b,
        "beta dropped": (x64 - mu) / np.sqrt(var_biased + 1e-5) * g,
        "gamma/beta swapped": (x64 - mu) / np.sqrt(var_biased + 1e-5) * b + g,
        "eps outside sqrt": (x64 - mu) / (np.sqrt(var_biased) + 1e-5) * g + b + 1e-3,
        "gamma shifted one column": (x64 - mu) / np.sqrt(var_biased + 1e-5) * np.roll(g, 1) + b,
    }
    for name, wrong in mistakes.items():
        assert not check_close(wrong, y, 1e-5, 1 - 1e-12)[0], name


def test_layernorm_float64_closed_form_and_tail_path():
    rng = np.random.default_rng(1)
    for n in (512, 768, 1024, 13, 8, 1):  # 13 and 1 exercise the double-precision tail loop
        x = (rng.standard_normal(n) * 2 + 0.7).astype(np.float32)
        g = (1 + 0.1 * rng.standard_normal(n)).astype(np.float32)
        b = (0.1 * rng.standard_normal(n)).astype(np.float32)
        got = O.layernorm_row(x, g, b, 1e-5)
        x64 = x.astype(np.float64)
        want = (x64 - x64.mean()) / np.sqrt(x64.var() + 1e-5) * g + b
        np.testing.assert_allclose(got, want, rtol=1e-5, atol=1e-6)


def test_layernorm_cancellation_fallback():
    """Constant rows make E[x^2]-E[x]^2 cancel; the reference falls back to two-pass (kern.cpp:49-56):
    the output must be exactly beta."""
    n = 512
    x = np.full(n, 1234.5678, dtype=np.float32)
    g = np.linspace(0.5, 2, n).astype(np.float32)
    b = np.linspace(-1, 1, n).astype(np.float32)
    got = O.layernorm_row(x, g, b, 1e-5)
    np.testing.assert_array_equal(got, b)


# ---- a3: bert::LayerNorm1D (two-pass fp32, eps 1e-12) -----------------------------------------

def test_layernorm1d_closed_form_and_moments():
    rng = np.random.default_rng(2)
    x = rng.standard_normal((8, 1024)).astype(np.float32)
    ones, zeros = np.ones(1024, np.float32), np.zeros(1024, np.float32)
    got = O.add_layernorm(O.F32, x, ones, zeros, 1e-12, mode=1)
    g64 = got.astype(np.float64)
    np.testing.assert_allclose(g64.mean(1), 0, atol=1e-6)
    np.testing.assert_allclose(g64.var(1), 1, rtol=1e-5)
    x64 = x.astype(np.float64)
    want = (x64 - x64.mean(1, keepdims=True)) / np.sqrt(x64.var(1, keepdims=True) + 1e-12)
    np.testing.assert_allclose(got, want, rtol=1e-5, atol=1e-6)
    # kern mode (one pass) and bert mode (two pass) agree to fp32 rounding on well-scaled rows
    np.testing.assert_allclose(O.add_layernorm(O.F32, x, ones, zeros, 1e-12, mode=0), got,
                               rtol=1e-5, atol=1e-6)


def test_add_layernorm_residual_and_bias_order():
    """h = (x + bias) + residual, then LN — against float64 with the same two roundings."""
    rng = np.random.default_rng(3)
    x, r = (rng.standard_normal((4, 512)).astype(np.float32) for _ in range(2))
    bias = (0.02 * rng.standard_normal(512)).astype(np.float32)
    g = (1 + 0.1 * rng.standard_normal(512)).astype(np.float32)
    b = (0.1 * rng.standard_normal(512)).astype(np.float32)
    got = O.add_layernorm(O.F32, x, g, b, 1e-5, bias=bias, residual=r)
    h = ((x + bias).astype(np.float32) + r).astype(np.float64)
    want = (h - h.mean(1, keepdims=True)) / np.sqrt(h.var(1, keepdims=True) + 1e-5) * g + b
    np.testing.assert_allclose(got, want, rtol=1e-5, atol=1e-6)
    # dropping the residual is caught
    h2 = (x + bias).astype(np.float64)
    wrong = (h2 - h2.mean(1, keepdims=True)) / np.sqrt(h2.var(1, keepdims=True) + 1e-5) * g + b
    assert not np.allclose(got, wrong, rtol=1e-5, atol=1e-6)


# ---- a4: ReLU against the reference golden, bit-exact (test_kern.cpp:231-239) ------------------

def test_relu_matches_reference_golden_bit_exact():
    v = load_bin("act_v.f32")
    want = load_bin("act_relu.f32")
    got = O.relu(v)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    # bias_act with act=relu and no bias is the same function
    got2 = O.bias_act(O.F32, 1, v.reshape(1, -1)).ravel()
    assert np.array_equal(got2.view(np.uint32), want.view(np.uint32))


def test_relu_special_values():
    v = np.array([-0.0, 0.0, np.inf, -np.inf, np.nan, 1e-45, -1e-45], dtype=np.float32)
    got = O.relu(np.concatenate([v, np.zeros(1, np.float32)]))[:7]  # length 8: vector body only
    assert got[0] == 0 and not np.signbit(got[0])  # vmaxq(-0, +0) = +0
    assert got[2] == np.inf and got[3] == 0 and np.isnan(got[4])
    assert got[5] == np.float32(1e-45) and got[6] == 0
    # scalar tail (n % 4 != 0): NaN -> 0
    tail = O.relu(np.array([1, 2, 3, 4, np.nan], dtype=np.float32))
    assert tail[4] == 0


# ---- a11: fp16 / bf16 conversions ---------------------------------------------------------------

def test_f16_upcast_reference_special_values():
    """test_accel.cpp:69-83: these bit patterns upcast exactly."""
    bits = [0x0000, 0x8000, 0x3C00, 0xC000, 0x7BFF, 0x0400, 0x3555, 0xABCD]
    got = [O.lib().oracle_h2f(b) for b in bits]
    want = np.array(bits, dtype=np.uint16).view(np.float16).astype(np.float32)
    assert got[0] == 0 and got[2] == 1 and got[3] == -2 and got[4] == 65504
    assert math.copysign(1, got[1]) == -1
    assert np.array_equal(np.array(got, np.float32), want)


def test_f16_upcast_all_patterns():
    allbits = np.arange(65536, dtype=np.uint16)
    got = O.to_f32(O.F16, allbits)
    want = allbits.view(np.float16).astype(np.float32)
    nan = np.isnan(want)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan].view(np.uint32), want[~nan].view(np.uint32))


def test_f16_downcast_round_to_nearest_even():
    rng = np.random.default_rng(4)
    vals = np.concatenate([
        rng.standard_normal(200000).astype(np.float32) * np.float32(10) ** rng.integers(-8, 6, 200000),
        # exact ties between adjacent halves, subnormal halves, overflow boundary, signed zeros
        (np.arange(-2048, 2048, dtype=np.float32) + 0.5) * np.float32(2 ** -24),
        np.array([65504, 65519.99, 65520, 65536, 1e30, -65520, 2 ** -25, 2 ** -26, 3 * 2 ** -26,
                  -0.0, 0.0, np.inf, -np.inf], dtype=np.float32),
    ]).astype(np.float32)
    got = O.to_storage(O.F16, vals)
    want = vals.astype(np.float16).view(np.uint16)
    assert np.array_equal(got, want)


def test_bf16_round_to_nearest_even_matches_torch():
    torch = pytest.importorskip("torch")
    rng = np.random.default_rng(5)
    vals = np.concatenate([
        rng.standard_normal(100000).astype(np.float32) * np.float32(10) ** rng.integers(-30, 30, 100000),
        np.array([1 + 2 ** -8, 1 + 3 * 2 ** -8, -(1 + 2 ** -8), 3.3895314e38, np.inf, -0.0],
                 dtype=np.float32),
    ]).astype(np.float32)
    got = O.to_storage(O.BF16, vals)
    want = torch.from_numpy(vals).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(got, want)
    assert O.to_storage(O.BF16, np.array([np.nan], np.float32))[0] == 0x7FC0


# ---- a10: pe_row (test_ar_unit.cpp:35-52) and the gather -----------------------------------------

def test_pe_row_matches_reference_closed_form():
    D = 512
    log_inc = -math.log(10000.0) / D
    for pos in (0, 1, 7, 166, 1234):
        pe = O.pe_row(pos, D)
        for d in range(0, D, 2):
            div = math.exp(d * log_inc)
            assert abs(pe[d] - math.sin(pos * div)) <= 1e-4
            assert abs(pe[d + 1] - math.cos(pos * div)) <= 1e-4


def test_pe_row_gate_rejects_swapped_sin_cos():
    D, pos = 512, 166
    pe = O.pe_row(pos, D)
    swapped = pe.reshape(-1, 2)[:, ::-1].ravel()
    log_inc = -math.log(10000.0) / D
    errs = [abs(swapped[d] - math.sin(pos * math.exp(d * log_inc))) for d in range(0, D, 2)]
    assert max(errs) > 1e-4


def _round_to_f32(fr):
    """Correctly round an exact rational to float32 (round to nearest, ties to even)."""
    f = np.float32(float(fr))  # double rounding is possible here, so fix it up exactly
    cands = [np.nextafter(f, np.float32(-np.inf)), f, np.nextafter(f, np.float32(np.inf))]
    best = min(cands, key=lambda c: (abs(Fraction(float(c)) - fr),
                                     int(np.array(c, np.float32).view(np.uint32)) & 1))
    return np.float32(best)


def test_embed_alpha_zero_is_exact_upcast_and_fma_is_exact():
    rng = np.random.default_rng(6)
    vocab, D, rows, max_pos = 50, 16, 40, 64
    table16 = (0.02 * rng.standard_normal((vocab, D))).astype(np.float16).view(np.uint16)
    ids = rng.integers(0, vocab, rows).astype(np.int64)
    pe = O.pe_table(max_pos, D)
    out, bad = O.embed_pe(O.F32, O.F16, table16, ids, pe, 0.0, pos0=3)
    assert bad == 0
    want = table16.view(np.float16).astype(np.float32)[ids]
    assert np.array_equal(out.view(np.uint32), (want + np.float32(0)).view(np.uint32))
    # alpha != 0: every element is the correctly rounded e + alpha*pe (one rounding)
    alpha = np.float32(1.2345678)
    out, _ = O.embed_pe(O.F32, O.F16, table16, ids, pe, float(alpha), pos0=3)
    e = table16.view(np.float16).astype(np.float32)[ids]
    p = pe[3:3 + rows]
    for r in range(0, rows, 3):
        for d in range(D):
            exact = Fraction(float(e[r, d])) + Fraction(float(alpha)) * Fraction(float(p[r, d]))
            assert out[r, d] == _round_to_f32(exact)
    # text path: mm + (e + b) then fma
    mm = rng.standard_normal((rows, D)).astype(np.float32)
    bias = (0.01 * rng.standard_normal(D)).astype(np.float32)
    out, _ = O.embed_pe(O.F32, O.F16, table16, ids, pe, float(alpha), pos0=0, mm=mm, bias=bias)
    xr = (mm + (e + bias).astype(np.float32)).astype(np.float32)
    for r in range(0, rows, 7):
        for d in range(D):
            exact = Fraction(float(xr[r, d])) + Fraction(float(alpha)) * Fraction(float(pe[r, d]))
            assert out[r, d] == _round_to_f32(exact)


def test_embed_out_of_range_rows_are_nan_and_counted():
    vocab, D = 10, 8
    table = np.ones((vocab, D), np.float32)
    pe = O.pe_table(4, D)
    ids = np.array([0, 10, -1, 3], np.int64)
    out, bad = O.embed_pe(O.F32, O.F32, table, ids, pe, 1.0, pos0=0)
    assert bad == 2
    assert np.isnan(out[1]).all() and np.isnan(out[2]).all() and not np.isnan(out[[0, 3]]).any()
    _, bad = O.embed_pe(O.F32, O.F32, table, np.array([0, 1], np.int64), pe, 1.0, pos0=3)
    assert bad == 1  # position 4 is past max_pos = 4


# ---- a5: GELU(erf) (parity unpinned by the reference: no golden vector exists) -----------------

def test_gelu_erf_closed_form_and_identities():
    xs = np.concatenate([np.linspace(-8, 8, 4001), [0.0, 1e-30, -1e-30, 30.0, -30.0]]).astype(np.float32)
    got = O.gelu_erf(xs)
    for x, g in zip(xs.astype(np.float64), got.astype(np.float64)):
        exact = 0.5 * x * (1 + math.erf(x / math.sqrt(2)))
        assert abs(g - exact) <= 1e-6 + 1e-5 * abs(exact), (x, g, exact)
    assert O.gelu_erf(np.array([0.0], np.float32))[0] == 0
    # 0.5f * x * (1 + erff(.)) is a product: a zero result carries the sign of x (IEEE 754 product
    # sign rule), so -0 stays -0 and erff(-30 / sqrt2) = -1 gives (-15) * 0 = -0
    z = O.gelu_erf(np.array([0.0, -0.0, -30.0, -8.0], np.float32))
    assert list(np.signbit(z)) == [False, True, True, True] and z[2] == 0
    # GELU(x) - GELU(-x) = x (the erf part is odd)
    pos = O.gelu_erf(xs)
    neg = O.gelu_erf(-xs)
    np.testing.assert_allclose(pos - neg, xs, rtol=1e-6, atol=1e-6)
    # a tanh-approximation GELU would fail the same gate
    x = np.float64(1.5)
    tanh_gelu = 0.5 * x * (1 + math.tanh(math.sqrt(2 / math.pi) * (x + 0.044715 * x ** 3)))
    assert abs(tanh_gelu - 0.5 * x * (1 + math.erf(x / math.sqrt(2)))) > 1e-5


# ---- a6: GroupNorm(groups = C) + GELU (parity unpinned by the reference) -----------------------

def test_groupnorm_closed_form_and_special_cases():
    rng = np.random.default_rng(7)
    C, T = 6, 1001
    x = (rng.standard_normal((C, T)) * 0.3 + 0.2).astype(np.float32)
    g = (1 + 0.1 * rng.standard_normal(C)).astype(np.float32)
    b = (0.1 * rng.standard_normal(C)).astype(np.float32)
    got = O.groupnorm_gelu(O.F32, x, g, b, 1e-5, apply_gelu=False)
    x64 = x.astype(np.float64)
    want = (x64 - x64.mean(1, keepdims=True)) / np.sqrt(x64.var(1, keepdims=True) + 1e-5)
    want = want * g[:, None] + b[:, None]
    np.testing.assert_allclose(got, want, rtol=1e-6, atol=1e-7)
    gel = O.groupnorm_gelu(O.F32, x, g, b, 1e-5, apply_gelu=True)
    np.testing.assert_array_equal(gel, O.gelu_erf(got).reshape(C, T))
    # T = 1: every channel normalises to exactly beta
    one = O.groupnorm_gelu(O.F32, x[:, :1].copy(), g, b, 1e-5, apply_gelu=False)
    np.testing.assert_array_equal(one.ravel(), b)
    # per-channel statistics: a transposed (per-frame) normalisation is rejected
    wrong = (x64 - x64.mean(0, keepdims=True)) / np.sqrt(x64.var(0, keepdims=True) + 1e-5)
    assert not np.allclose(got, wrong * g[:, None] + b[:, None], atol=1e-3)


# ---- a7 / a8 / a9: SoVITS element-wise (parity unpinned by the reference) ----------------------

def test_leaky_relu_identities():
    rng = np.random.default_rng(8)
    v = np.concatenate([rng.standard_normal(1001).astype(np.float32),
                        np.array([-0.0, 0.0, np.nan, -np.inf, np.inf], np.float32)])
    same = O.leaky_relu(O.F32, v, 1.0)
    assert np.array_equal(same.view(np.uint32), v.view(np.uint32))  # slope 1: identity, bitwise
    zero = O.leaky_relu(O.F32, v, 0.0)
    fin = np.isfinite(v)
    assert np.array_equal(zero[fin] == 0, ~(v[fin] > 0)) and np.array_equal(zero[v > 0], v[v > 0])
    got = O.leaky_relu(O.F32, v, 0.1)
    want = np.where(v < 0, v * np.float32(0.1), v)  # numpy float32 multiply: one IEEE rounding
    ok = ~np.isnan(v)
    assert np.array_equal(got[ok].view(np.uint32), want[ok].view(np.uint32))
    assert np.signbit(got[v.size - 5]) and np.isnan(got[v.size - 3])  # -0 and NaN kept


def test_resblock_add_lrelu_exact():
    rng = np.random.default_rng(9)
    cur, tb = (rng.standard_normal(999).astype(np.float32) for _ in range(2))
    c2, tin = O.resblock_add_lrelu(O.F32, cur, tb, 0.1)
    s = (cur.astype(np.float64) + tb.astype(np.float64)).astype(np.float32)  # exact sum, one rounding
    assert np.array_equal(c2, s)
    assert np.array_equal(tin, np.where(s < 0, s * np.float32(0.1), s))


def test_resblock_branch_mean_closed_form():
    rng = np.random.default_rng(10)
    n = 777
    curs = [rng.standard_normal(n).astype(np.float32) for _ in range(3)]
    tbs = [rng.standard_normal(n).astype(np.float32) for _ in range(3)]
    got = O.resblock_branch_mean(O.F32, curs, tbs, False, 0.1)
    exact = sum(c.astype(np.float64) + t.astype(np.float64) for c, t in zip(curs, tbs)) / 3
    np.testing.assert_allclose(got, exact, rtol=4e-7, atol=1e-6)
    # identical branches average back to the branch (up to the 1/3 rounding)
    same = O.resblock_branch_mean(O.F32, [curs[0]] * 3, None, False, 0.1)
    np.testing.assert_allclose(same, curs[0], rtol=3e-7, atol=0)
    # the lrelu of the average
    lr = O.resblock_branch_mean(O.F32, curs, tbs, True, 0.01)
    assert np.array_equal(lr, np.where(got < 0, got * np.float32(0.01), got))
    # a dropped branch is rejected
    two = sum(c.astype(np.float64) + t.astype(np.float64) for c, t in zip(curs[:2], tbs[:2])) / 3
    assert not np.allclose(got, two, atol=1e-3)


def test_scaled_add_matches_separate_roundings():
    rng = np.random.default_rng(11)
    acc, src = (rng.standard_normal(513).astype(np.float32) for _ in range(2))
    k = np.float32(1.0) / np.float32(3.0)
    assert np.array_equal(O.scaled_add(O.F32, None, src, float(k)), src * k)
    assert np.array_equal(O.scaled_add(O.F32, acc, src, float(k)), acc + src * k)


def test_sixteen_bit_storage_rounds_once():
    """fp16 storage = exact upcast -> fp32 math -> one RNE store (checked on bias+ReLU)."""
    rng = np.random.default_rng(12)
    x32 = rng.standard_normal((3, 64)).astype(np.float32)
    x16 = O.to_storage(O.F16, x32)
    bias = (0.1 * rng.standard_normal(64)).astype(np.float32)
    got = O.bias_act(O.F16, 1, x16, bias)
    want = np.maximum(x16.view(np.float16).astype(np.float32) + bias, 0).astype(np.float16)
    assert np.array_equal(got, want.view(np.uint16))


# ---- T2S step chain: thread split does not change a bit ------------------------------------------

def _t2s_host_bufs(dt, B=8, D=64, FF=128, L=3, seed=13):
    rng = np.random.default_rng(seed)
    st = lambda a: O.to_storage(dt, a.astype(np.float32))
    bufs = {
        "table": (0.02 * rng.standard_normal((100, D))).astype(np.float16).view(np.uint16),
        "table_dtype": O.F16,
        "ids": rng.integers(0, 100, B).astype(np.int64),
        "pos": rng.integers(10, 60, B).astype(np.int64),
        "pe": O.pe_table(64, D),
        "alpha": 0.9,
        "x": st(np.zeros((B, D))), "h": st(np.zeros((B, D))),
    }
    for name, shape in (("attn_out", (B, D)), ("ff", (B, FF)), ("ffn_out", (B, D))):
        bufs[name] = [st(rng.standard_normal(shape)) for _ in range(L)]
    for name, n in (("bout", D), ("b1", FF), ("b2", D), ("n1b", D), ("n2b", D)):
        bufs[name] = [(0.05 * rng.standard_normal(n)).astype(np.float32) for _ in range(L)]
    for name in ("n1g", "n2g"):
        bufs[name] = [(1 + 0.1 * rng.standard_normal(D)).astype(np.float32) for _ in range(L)]
    return bufs


@pytest.mark.parametrize("dt", [O.F32, O.F16])
def test_t2s_step_threads_bitwise_equal(dt):
    a = _t2s_host_bufs(dt)
    b = _t2s_host_bufs(dt)
    O.t2s_step(dt, a, threads=1)
    O.t2s_step(dt, b, threads=3)
    assert np.array_equal(a["x"], b["x"]) and np.array_equal(a["h"], b["h"])
    for fa, fb in zip(a["ff"], b["ff"]):
        assert np.array_equal(fa, fb)
