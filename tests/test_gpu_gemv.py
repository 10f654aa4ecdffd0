"""GPU parity of gsvk_gemv_f16w (batched decode GEMV, fp16 weights, fused epilogue) against the
oracle's restatement of kern::gemv_f16w_f32acc / kern::gemv_f16x_fmlal and the bias / act /
residual loops of block_decode_impl.

Tolerance: the sum is formed in another order than the reference's (matrix-core tiles and per-wave
partials), so results are compared with the reference's own rule between two summation orders
(test_kern.cpp:111-118): |got - want| <= 1e-5 * max(1, max |want| over the row). A 16-bit result
may in addition sit one rounding step away (a pre-rounding difference at the 1e-5 level can cross a
rounding boundary), and GELU adds its own fp32 tolerance (1e-6 + 1e-5 |v|). The golden vectors of
the reference are also checked with the reference's gate (max rel 2e-5, cosine 1 - 1e-12).
"""
import numpy as np
import pytest
import torch

import gsvk
import oracle as O
from conftest import check_close, load_bin
from gpu_util import BF16, F16, F32, dev, devf, host, say

pytestmark = pytest.mark.gpu


def rng(k):
    return np.random.default_rng(20250823 + 9000 + k)


def step16(dt, w):
    w = np.abs(w.astype(np.float64))
    if dt == F16:
        return np.spacing(np.minimum(w, 65504).astype(np.float16)).astype(np.float64)
    e = np.floor(np.log2(np.maximum(w, 2.0 ** -126)))
    return 2.0 ** (e - 7)


def assert_gemv_close(y_dt, got, want, act=gsvk.ACT_NONE, what=""):
    g = O.to_f32(y_dt, got).astype(np.float64)
    w = O.to_f32(y_dt, want).astype(np.float64)
    assert g.shape == w.shape
    assert np.array_equal(np.isnan(g), np.isnan(w)), f"{what}: NaN positions differ"
    peak = np.maximum(1.0, np.nanmax(np.abs(w), axis=1, keepdims=True))
    tol = 1e-5 * peak
    if y_dt != F32:
        tol = tol + step16(y_dt, w)
    if act == gsvk.ACT_GELU_ERF:
        tol = tol + 1e-6 + 1e-5 * np.abs(w)
    err = np.abs(g - w)
    err[np.isnan(w)] = 0
    bad = np.argwhere(err > tol)
    assert bad.size == 0, f"{what}: {len(bad)} outside tolerance, worst {np.max(err - tol):.3e} " \
                          f"at {bad[:3].tolist()}"
    return float(np.max(err / peak))


def weights(r, n_out, n_in, scale=0.05):
    return (scale * r.standard_normal((n_out, n_in))).astype(np.float16).view(np.uint16)


def run_case(rows, n_out, n_in, x_dt, round_x, y_dt, act=gsvk.ACT_NONE, use_bias=True,
             use_res=False, slope=0.1, seed=0):
    say(f"gemv rows={rows} out={n_out} in={n_in} x={x_dt} round={round_x} y={y_dt} act={act} "
        f"bias={use_bias} res={use_res}")
    r = rng(seed + rows * 7 + n_out * 3 + n_in)
    x32 = r.standard_normal((rows, n_in)).astype(np.float32)
    x = O.to_storage(x_dt, x32)
    w = weights(r, n_out, n_in)
    bias = (0.02 * r.standard_normal(n_out)).astype(np.float32) if use_bias else None
    res = O.to_storage(y_dt, r.standard_normal((rows, n_out)).astype(np.float32)) if use_res \
        else None
    want = O.gemv_f16w(x_dt, x, w, y_dt, bias=bias, act=act, slope=slope, residual=res,
                       round_x=round_x)
    X, W = dev(x, x_dt), dev(w, F16)
    Y = torch.empty((rows, n_out), dtype=dev(np.zeros(1, O.storage_dtype(y_dt)), y_dt).dtype,
                    device="cuda")
    R = dev(res, y_dt) if use_res else None
    gsvk.gemv_f16w(X, W, Y, bias=devf(bias) if use_bias else None, act=act, slope=slope,
                   residual=R, round_x=round_x)
    torch.cuda.synchronize()
    return host(Y, y_dt), want, (X, W, bias, R, Y)


# ---- the reference's golden vectors -------------------------------------------------------------

@pytest.mark.parametrize("tag", ["gemv_a", "gemv_b"])
def test_gemv_reference_golden(tag):
    w = load_bin(f"{tag}_w.f16").view(np.uint16)
    x = load_bin(f"{tag}_x.f32")
    y = load_bin(f"{tag}_y.f32")
    say(f"gemv golden {tag} {w.shape}")
    X = devf(x[None, :])
    Y = torch.empty((1, w.shape[0]), dtype=torch.float32, device="cuda")
    gsvk.gemv_f16w(X, dev(w, F16), Y, round_x=False)
    torch.cuda.synchronize()
    got = host(Y, F32)[0]
    ok, worst, cos = check_close(got, y, 2e-5, 1.0 - 1e-12)
    assert ok, (worst, cos)
    want = O.gemv_f16w(F32, x, w, F32, round_x=False)
    assert_gemv_close(F32, got[None, :], want, what=tag)


# ---- decode shapes (B = 64, d_model 512, ffn 2048, vocab 1025) -----------------------------------

DECODE = [
    # (name, out, in, act, bias, residual, y dtype)
    ("qkv", 1536, 512, gsvk.ACT_NONE, True, False, F32),
    ("out_proj", 512, 512, gsvk.ACT_NONE, True, True, F16),
    ("w1_relu", 2048, 512, gsvk.ACT_RELU, True, False, F16),
    ("w2", 512, 2048, gsvk.ACT_NONE, True, True, F16),
    ("logits", 1025, 512, gsvk.ACT_NONE, False, False, F32),
]


@pytest.mark.parametrize("name,n_out,n_in,act,use_bias,use_res,y_dt", DECODE)
@pytest.mark.parametrize("x_dt,round_x", [(F16, True), (F32, True), (F32, False)])
def test_gemv_decode_shapes(name, n_out, n_in, act, use_bias, use_res, y_dt, x_dt, round_x):
    got, want, _ = run_case(64, n_out, n_in, x_dt, round_x, y_dt, act, use_bias, use_res)
    assert_gemv_close(y_dt, got, want, act, name)


def test_gemv_split_mode_is_fp32_accurate():
    """round_x = 0 must track the fp32 activations, not their fp16 rounding: against a float64
    product it stays at fp32-accumulation level, ~100x below the fp16-rounding error."""
    r = rng(1)
    x = r.standard_normal((64, 512)).astype(np.float32)
    w = weights(r, 512, 512)
    exact = x.astype(np.float64) @ w.view(np.float16).astype(np.float64).T
    Y = torch.empty((64, 512), dtype=torch.float32, device="cuda")
    gsvk.gemv_f16w(devf(x), dev(w, F16), Y, round_x=False)
    torch.cuda.synchronize()
    err_split = np.max(np.abs(host(Y, F32) - exact))
    gsvk.gemv_f16w(devf(x), dev(w, F16), Y, round_x=True)
    torch.cuda.synchronize()
    err_round = np.max(np.abs(host(Y, F32) - exact))
    say(f"split err {err_split:.3e} round err {err_round:.3e}")
    assert err_split < 1e-5 and err_round > 30 * err_split


# ---- shapes off the tile grid, row counts off 64, all output types -------------------------------

@pytest.mark.parametrize("rows,n_out,n_in", [
    (1, 1, 1), (3, 8, 8), (64, 7, 7), (17, 17, 131),   # generic path (K % 8 != 0)
    (1, 512, 512), (5, 33, 40), (63, 100, 72), (65, 130, 264), (130, 257, 1000),
    (200, 48, 2056), (7, 3, 4096),
])
@pytest.mark.parametrize("y_dt", [F32, F16, BF16])
def test_gemv_ragged(rows, n_out, n_in, y_dt):
    got, want, _ = run_case(rows, n_out, n_in, F16, True, y_dt, gsvk.ACT_NONE, True, True,
                            seed=11)
    assert_gemv_close(y_dt, got, want, what=f"{rows}x{n_out}x{n_in}")


@pytest.mark.parametrize("act", [gsvk.ACT_GELU_ERF, gsvk.ACT_LEAKY_RELU, gsvk.ACT_RELU])
def test_gemv_activations(act):
    got, want, _ = run_case(64, 3072, 768, F16, True, F16, act, True, False, slope=0.01, seed=3)
    assert_gemv_close(F16, got, want, act, f"act {act}")


def test_gemv_many_column_tiles():
    """16 rows x 65,576 columns: 4,099 tiles of 16 x 16, below the long-stream threshold (16,384
    tiles), so the decode tiles run over many column blocks."""
    got, want, _ = run_case(16, 65536 + 40, 512, F16, True, F16, gsvk.ACT_RELU, True, False,
                            seed=5)
    assert_gemv_close(F16, got, want, gsvk.ACT_RELU, "wide")


# Long weight streams (>= 16,384 tiles of 16 x 16 at K = 512 or 1024, no activation or ReLU, aligned
# operands) run on the persistent streaming kernel: against the oracle at four shapes (a ragged last
# column batch, a ragged row group with bf16 output and residual, K = 1024, 100 rows in two row
# groups), and bit for bit against
# the 64-row tiled kernel at K = 512, which sums in the same order (k slices of 128 per wave, waves
# added in order): forced there by a bias that is not 16-byte aligned.
STREAM = [  # rows, n_out, n_in, x_dt, round_x, y_dt, act, use_bias, use_res
    (64, 65536 + 4, 512, F16, True, F32, gsvk.ACT_NONE, True, False),
    (50, 65536, 512, F32, True, BF16, gsvk.ACT_NONE, True, True),
    (64, 65536 + 32, 1024, F16, True, F16, gsvk.ACT_RELU, True, True),
    (100, 40000, 512, F32, True, F32, gsvk.ACT_RELU, True, True),  # two row groups, the second partial
]


@pytest.mark.parametrize("rows,n_out,n_in,x_dt,round_x,y_dt,act,use_bias,use_res", STREAM)
def test_gemv_long_stream(rows, n_out, n_in, x_dt, round_x, y_dt, act, use_bias, use_res):
    got, want, _ = run_case(rows, n_out, n_in, x_dt, round_x, y_dt, act, use_bias, use_res,
                            seed=11)
    assert_gemv_close(y_dt, got, want, act, f"stream {rows}x{n_out}x{n_in}")


@pytest.mark.parametrize("y_dt", [F32, F16, BF16])
@pytest.mark.parametrize("x_dt,round_x", [(F16, True), (F32, True), (F32, False)])
def test_gemv_long_stream_equals_tiled(x_dt, round_x, y_dt):
    rows, n_out, n_in = 64, 65536 + 36, 512
    say(f"stream vs tiled x={x_dt} round={round_x} y={y_dt}")
    r = rng(40 + 3 * x_dt + y_dt + int(round_x))
    x = O.to_storage(x_dt, r.standard_normal((rows, n_in)).astype(np.float32))
    w = weights(r, n_out, n_in)
    b = (0.02 * r.standard_normal(n_out)).astype(np.float32)
    res = O.to_storage(y_dt, r.standard_normal((rows, n_out)).astype(np.float32))
    X, W, R = dev(x, x_dt), dev(w, F16), dev(res, y_dt)
    aligned = devf(b)
    shifted = devf(np.concatenate([np.zeros(1, np.float32), b]))[1:]  # same values, 4 bytes off
    assert aligned.data_ptr() % 16 == 0 and shifted.data_ptr() % 16 == 4
    outs = []
    for bias in (aligned, shifted):
        Y = torch.empty_like(R)
        gsvk.gemv_f16w(X, W, Y, bias=bias, act=gsvk.ACT_RELU, residual=R, round_x=round_x)
        torch.cuda.synchronize()
        outs.append(host(Y, y_dt))
    g, t = O.to_f32(y_dt, outs[0]), O.to_f32(y_dt, outs[1])
    assert np.array_equal(np.isnan(g), np.isnan(t))
    assert np.array_equal(outs[0], outs[1]), \
        f"{np.count_nonzero(outs[0] != outs[1])} elements differ between the two kernels"


def test_gemv_long_stream_residual_in_place():
    r = rng(12)
    rows, n_out, n_in = 64, 65536 + 4, 512
    x = O.to_storage(F16, r.standard_normal((rows, n_in)).astype(np.float32))
    w = weights(r, n_out, n_in)
    bias = (0.02 * r.standard_normal(n_out)).astype(np.float32)
    h = O.to_storage(F16, r.standard_normal((rows, n_out)).astype(np.float32))
    want = O.gemv_f16w(F16, x, w, F16, bias=bias, residual=h)
    X, W, B = dev(x, F16), dev(w, F16), devf(bias)
    outs = []
    for _ in range(2):
        Y = dev(h, F16)
        gsvk.gemv_f16w(X, W, Y, bias=B, residual=Y)
        torch.cuda.synchronize()
        outs.append(host(Y, F16))
    assert_gemv_close(F16, outs[0], want, what="stream in place")
    assert np.array_equal(outs[0], outs[1])


def test_gemv_residual_in_place_and_deterministic():
    r = rng(9)
    rows, n_out, n_in = 64, 512, 2048
    x = O.to_storage(F16, r.standard_normal((rows, n_in)).astype(np.float32))
    w = weights(r, n_out, n_in)
    bias = (0.02 * r.standard_normal(n_out)).astype(np.float32)
    h = O.to_storage(F16, r.standard_normal((rows, n_out)).astype(np.float32))
    want = O.gemv_f16w(F16, x, w, F16, bias=bias, residual=h)
    X, W, B = dev(x, F16), dev(w, F16), devf(bias)
    outs = []
    for _ in range(3):
        Y = dev(h, F16)
        gsvk.gemv_f16w(X, W, Y, bias=B, residual=Y)
        torch.cuda.synchronize()
        outs.append(host(Y, F16))
    assert_gemv_close(F16, outs[0], want, what="in place")
    assert all(np.array_equal(outs[0], o) for o in outs[1:])


def test_gemv_rejects_bad_arguments():
    X = torch.zeros((4, 64), dtype=torch.float16, device="cuda")
    W = torch.zeros((32, 64), dtype=torch.float16, device="cuda")
    Y = torch.zeros((4, 32), dtype=torch.float32, device="cuda")
    L = gsvk.lib()
    assert L.gsvk_gemv_f16w(F16, 1, X.data_ptr(), 64, W.data_ptr(), None, 0, 0.0, None, F32,
                            Y.data_ptr(), 32, 4, 32, 0, None) == gsvk.E_SIZE
    assert L.gsvk_gemv_f16w(BF16, 1, X.data_ptr(), 64, W.data_ptr(), None, 0, 0.0, None, F32,
                            Y.data_ptr(), 32, 4, 32, 64, None) == gsvk.E_DTYPE
    assert L.gsvk_gemv_f16w(F16, 1, X.data_ptr(), 64, W.data_ptr(), None, 9, 0.0, None, F32,
                            Y.data_ptr(), 32, 4, 32, 64, None) == gsvk.E_DTYPE
    assert L.gsvk_gemv_f16w(F16, 1, X.data_ptr(), 64, W.data_ptr(), None, 0, 0.0, None, F32,
                            X.data_ptr(), 32, 4, 32, 64, None) == gsvk.E_ALIAS
    assert L.gsvk_gemv_f16w(F16, 1, X.data_ptr(), 32, W.data_ptr(), None, 0, 0.0, None, F32,
                            Y.data_ptr(), 32, 4, 32, 64, None) == gsvk.E_SIZE
    assert L.gsvk_gemv_f16w(F16, 1, None, 64, W.data_ptr(), None, 0, 0.0, None, F32,
                            Y.data_ptr(), 32, 4, 32, 64, None) == gsvk.E_NULL


# ---- LayerNorm folded into the GEMV (gsvk_gemv_f16w_ln) ------------------------------------------

LN_CASES = [
    # rows, out, in, x_dt, round_x, y_dt, act, residual, affine
    (64, 2048, 512, F16, True, F16, gsvk.ACT_RELU, False, True),    # norm1 -> W1, fp16 storage
    (64, 1536, 512, F16, True, F32, gsvk.ACT_NONE, False, True),    # norm2 -> next QKV
    (64, 1025, 512, F16, True, F32, gsvk.ACT_NONE, False, True),    # norm2 -> logits
    (64, 2048, 512, F32, True, F32, gsvk.ACT_RELU, False, True),    # fp32 storage, x rounded
    (37, 96, 472, F32, False, F32, gsvk.ACT_NONE, True, False),     # split mode, ragged, k tail
    (21, 80, 200, F16, True, F16, gsvk.ACT_NONE, False, True),      # 16-bit x, k tail
    (5, 24, 120, F32, True, F16, gsvk.ACT_NONE, False, True),       # two waves, k tail
    (8, 40, 264, F32, True, F32, gsvk.ACT_NONE, False, True),       # two launches (2 blocks/wave)
    (19, 64, 1024, F16, True, F16, gsvk.ACT_GELU_ERF, True, True),  # the largest fused K
    (130, 40, 512, F16, True, F32, gsvk.ACT_NONE, False, True),     # several row blocks
    (16, 48, 2048, F16, True, F32, gsvk.ACT_NONE, False, True),     # two launches (K > 1024)
    (8, 40, 520, F32, True, F32, gsvk.ACT_NONE, False, True),       # two launches (K > 512 fp32)
    (8, 40, 100, F32, True, F32, gsvk.ACT_NONE, False, True),       # two launches (K % 8 != 0)
]


def ln_fused(rows, n_out, n_in):
    """Whether gsvk_gemv_f16w_ln runs as one launch: K % 8 == 0 and a launch plan whose waves hold
    all their k blocks (the GEMV's thresholds: 64-wide blocks over 1, 2, 4, 4 or 8 waves)."""
    nkb = (n_in + 63) // 64
    if n_in % 8 or (n_out + 15) // 16 * ((rows + 15) // 16) >= 16384:
        return False
    wk, d = (8, 2) if nkb >= 16 else (4, 2) if nkb >= 8 else (4, 1) if nkb >= 4 else \
        (2, 1) if nkb >= 2 else (1, 1)
    return -(-nkb // wk) <= d


@pytest.mark.parametrize("rows,n_out,n_in,x_dt,round_x,y_dt,act,use_res,affine", LN_CASES)
def test_gemv_ln_equals_layernorm_then_gemv(rows, n_out, n_in, x_dt, round_x, y_dt, act, use_res,
                                            affine):
    """The fused launch against the oracle: h within the LayerNorm tolerance (its statistics are
    summed in another order than gsvk_add_layernorm's), y = the oracle GEMV of that h; two calls
    give the same bits. Every storage / rounding mode, ragged rows, a partial k block, absent
    gamma / beta, and shapes that take the two-launch form (then equal to the two launches)."""
    say(f"gemv_ln rows={rows} out={n_out} in={n_in} x={x_dt} round={round_x} y={y_dt} act={act}")
    r = rng(500 + rows + n_out + n_in)
    z = O.to_storage(x_dt, (3.0 * r.standard_normal((rows, n_in)) + 0.5).astype(np.float32))
    g = (1.0 + 0.1 * r.standard_normal(n_in)).astype(np.float32) if affine else None
    b = (0.1 * r.standard_normal(n_in)).astype(np.float32) if affine else None
    w = weights(r, n_out, n_in)
    bias = (0.02 * r.standard_normal(n_out)).astype(np.float32)
    res = O.to_storage(y_dt, r.standard_normal((rows, n_out)).astype(np.float32)) if use_res \
        else None
    Z, W = dev(z, x_dt), dev(w, F16)
    G, Bt = (devf(g), devf(b)) if affine else (None, None)
    Bi = devf(bias)
    ytype = dev(np.zeros(1, O.storage_dtype(y_dt)), y_dt).dtype
    H1, H2 = torch.full_like(Z, 7), torch.full_like(Z, 7)
    Y1 = torch.empty((rows, n_out), dtype=ytype, device="cuda")
    Y2 = torch.empty_like(Y1)
    R = dev(res, y_dt) if use_res else None
    gsvk.gemv_f16w_ln(Z, G, Bt, 1e-5, H1, W, Y1, bias=Bi, act=act, residual=R, round_x=round_x)
    gsvk.gemv_f16w_ln(Z, G, Bt, 1e-5, H2, W, Y2, bias=Bi, act=act, residual=R, round_x=round_x)
    torch.cuda.synchronize()
    h1, h2 = host(H1, x_dt), host(H2, x_dt)
    y1, y2 = host(Y1, y_dt), host(Y2, y_dt)
    assert np.array_equal(h1, h2) and np.array_equal(y1, y2), "two calls differ"
    if not ln_fused(rows, n_out, n_in):  # the two-launch form: the same bits
        gsvk.add_layernorm(Z, G, Bt, H2, 1e-5)
        gsvk.gemv_f16w(H2, W, Y2, bias=Bi, act=act, residual=R, round_x=round_x)
        torch.cuda.synchronize()
        assert np.array_equal(h1, host(H2, x_dt)) and np.array_equal(y1, host(Y2, y_dt))
    # and against the oracle: h within the LayerNorm tolerance, y = the oracle GEMV of that h
    ones, zeros = np.ones(n_in, np.float32), np.zeros(n_in, np.float32)
    want_h = O.to_f32(x_dt, O.add_layernorm(x_dt, z, g if affine else ones,
                                            b if affine else zeros, 1e-5)).astype(np.float64)
    got_h = O.to_f32(x_dt, h1).astype(np.float64)
    tol_h = 2e-3 if x_dt == F16 else 1e-6 + 1e-5 * np.abs(want_h)
    assert np.all(np.abs(got_h - want_h) <= tol_h), "h vs oracle LayerNorm"
    want = O.gemv_f16w(x_dt, h1, w, y_dt, bias=bias, act=act, residual=res, round_x=round_x)
    assert_gemv_close(y_dt, y1, want, act, "gemv_ln vs oracle GEMV")
