"""GPU parity: every HIP kernel, called through the C ABI (libgsvk.so), against the CPU oracle on the
same seeded inputs — at the configuration shapes (where the oracle finishes in seconds) and on the
edge cases the reference's code admits (odd widths, unaligned buffers, in-place calls, special
values, out-of-range ids). Tolerances: see gpu_util."""
import numpy as np
import pytest
import torch

import gsvk
import oracle as O
from gpu_util import (ALL_DT, BF16, F16, F32, TORCH_DT, assert_bitexact, assert_close, dev, devf,
                      host, say)

pytestmark = pytest.mark.gpu

SEED = 20250823


def rng(k):
    return np.random.default_rng(SEED + k)


def st(dt, a):
    return O.to_storage(dt, np.asarray(a, dtype=np.float32))


def sync():
    torch.cuda.synchronize()


# ---- residual + LayerNorm ------------------------------------------------------------------------

LN_CASES = [
    # (rows, n, dtype, eps, mode, bias, residual)  mode 0 = kern::layernorm, 1 = bert LayerNorm1D
    (256, 512, F32, 1e-5, 0, False, True),     # config 1
    (64, 512, F16, 1e-5, 0, True, True),       # config 2 decode LN
    (512, 1024, F16, 1e-12, 1, False, True),   # config 3 BERT LN
    (499, 768, F16, 1e-5, 0, True, True),      # config 4 HuBERT LN
    (37, 512, BF16, 1e-5, 0, True, True),
    (5, 2048, F32, 1e-5, 0, True, False),      # 8 chunks per lane
    (3, 4096, F16, 1e-5, 0, False, False),
    (7, 333, F32, 1e-5, 0, True, True),        # odd width: generic path
    (3, 5000, F32, 1e-5, 0, True, True),       # wider than the register path: generic
    (1, 8, F16, 1e-5, 0, False, False),
]


@pytest.mark.parametrize("rows,n,dt,eps,mode,use_bias,use_res", LN_CASES)
def test_add_layernorm_matches_oracle(rows, n, dt, eps, mode, use_bias, use_res):
    say(f"add_layernorm rows={rows} n={n} dt={dt}")
    r = rng(rows * 7 + n)
    x = st(dt, r.standard_normal((rows, n)))
    res = st(dt, r.standard_normal((rows, n))) if use_res else None
    bias = (0.02 * r.standard_normal(n)).astype(np.float32) if use_bias else None
    g = (1 + 0.1 * r.standard_normal(n)).astype(np.float32)
    b = (0.1 * r.standard_normal(n)).astype(np.float32)
    want = O.add_layernorm(dt, x, g, b, eps, bias=bias, residual=res, mode=mode)
    X, Y = dev(x, dt), torch.empty_like(dev(x, dt))
    gsvk.add_layernorm(X, devf(g), devf(b), Y, eps, bias=devf(bias) if use_bias else None,
                       residual=dev(res, dt) if use_res else None)
    sync()
    assert_close(dt, host(Y, dt), want, f"LN {rows}x{n}")


def test_golden_layernorm_on_gpu():
    """The reference's own LayerNorm golden (ln_*.f32, test_kern.cpp:207-216) through the HIP path."""
    from conftest import check_close, load_bin
    x, g, b, y = (load_bin(f"ln_{k}.f32") for k in "xgby")
    X = devf(x)
    gsvk.add_layernorm(X, devf(g), devf(b), X, 1e-5)  # in place, as t2s_engine.cpp:986 calls it
    sync()
    ok, worst, cos = check_close(host(X, F32), y, 1e-5, 1 - 1e-12)
    assert ok, (worst, cos)


@pytest.mark.parametrize("dt", ALL_DT)
def test_add_layernorm_in_place_and_unaligned(dt):
    r = rng(101)
    rows, n = 9, 512
    x = st(dt, 3 * r.standard_normal((rows, n)) - 0.5)
    res = st(dt, r.standard_normal((rows, n)))
    g = (1 + 0.1 * r.standard_normal(n)).astype(np.float32)
    b = (0.1 * r.standard_normal(n)).astype(np.float32)
    want = O.add_layernorm(dt, x, g, b, 1e-5, residual=res)
    # y == residual
    X, R = dev(x, dt), dev(res, dt)
    gsvk.add_layernorm(X, devf(g), devf(b), R, 1e-5, residual=R)
    sync()
    assert_close(dt, host(R, dt), want, "y == residual")
    # y == x on a buffer that starts one element past a 16-byte boundary, with row stride ld > n
    ld = n + 3
    big = torch.zeros(rows * ld + 1, dtype=dev(x, dt).dtype, device="cuda")
    view = big[1:1 + rows * ld].view(rows, ld)[:, :n]
    view.copy_(dev(x, dt))
    rbig = torch.zeros_like(big)
    rview = rbig[1:1 + rows * ld].view(rows, ld)[:, :n]
    rview.copy_(dev(res, dt))
    gsvk.add_layernorm(view, devf(g), devf(b), view, 1e-5, residual=rview)
    sync()
    assert_close(dt, host(view, dt), want, "unaligned in place")
    assert host(big[:1], dt)[0] == 0  # nothing written outside the view


def test_add_layernorm_constant_rows_give_beta():
    n = 512
    x = np.full((4, n), 7.25, np.float32)
    b = np.linspace(-1, 1, n).astype(np.float32)
    X = devf(x)
    gsvk.add_layernorm(X, devf(np.ones(n, np.float32)), devf(b), X, 1e-5)
    sync()
    assert np.array_equal(host(X, F32), np.broadcast_to(b, (4, n)))


def test_add_layernorm_deterministic():
    r = rng(102)
    x = r.standard_normal((1000, 1024)).astype(np.float32)
    g, b = np.ones(1024, np.float32), np.zeros(1024, np.float32)
    outs = []
    for _ in range(3):
        Y = torch.empty((1000, 1024), device="cuda")
        gsvk.add_layernorm(devf(x), devf(g), devf(b), Y, 1e-5)
        sync()
        outs.append(host(Y, F32))
    assert np.array_equal(outs[0], outs[1]) and np.array_equal(outs[0], outs[2])


# ---- bias + activation -----------------------------------------------------------------------------

BA_CASES = [
    (64, 2048, F16, gsvk.ACT_RELU),       # config 2 FFN
    (512, 4096, F16, gsvk.ACT_GELU_ERF),  # config 3 FFN
    (499, 3072, F16, gsvk.ACT_GELU_ERF),  # config 4 FFN
    (33, 2048, F32, gsvk.ACT_RELU),
    (33, 1000, F32, gsvk.ACT_GELU_ERF),
    (17, 1024, BF16, gsvk.ACT_GELU_ERF),
    (9, 777, F32, gsvk.ACT_LEAKY_RELU),   # odd width: generic path
    (9, 512, F16, gsvk.ACT_NONE),
]


@pytest.mark.parametrize("rows,n,dt,act", BA_CASES)
def test_bias_act_matches_oracle(rows, n, dt, act):
    say(f"bias_act rows={rows} n={n} dt={dt} act={act}")
    r = rng(rows + n + act)
    x = st(dt, r.standard_normal((rows, n)))
    bias = (0.02 * r.standard_normal(n)).astype(np.float32)
    want = O.bias_act(dt, act, x, bias, 0.1)
    X = dev(x, dt)
    gsvk.bias_act(act, X, X, bias=devf(bias), slope=0.1)  # in place, as the callers do
    sync()
    got = host(X, dt)
    if act == gsvk.ACT_GELU_ERF:
        assert_close(dt, got, want, "bias+gelu")
    else:
        assert_bitexact(dt, got, want, "bias+act")


def test_relu_golden_and_special_values_bit_exact():
    from conftest import load_bin
    v = load_bin("act_v.f32").reshape(1, -1)
    X = devf(v)
    gsvk.bias_act(gsvk.ACT_RELU, X, X)
    sync()
    assert_bitexact(F32, host(X, F32).ravel(), load_bin("act_relu.f32"), "relu golden")
    sp = np.array([[-0.0, 0.0, np.inf, -np.inf, np.nan, 1e-45, -1e-45, 3.0]], np.float32)
    X = devf(sp)
    gsvk.bias_act(gsvk.ACT_RELU, X, X)
    sync()
    got = host(X, F32)
    assert_bitexact(F32, got, O.bias_act(F32, 1, sp), "relu special")
    assert not np.signbit(got[0, 0])


def test_gelu_special_values():
    sp = np.array([[0.0, -0.0, 1e-30, -1e-30, 8.0, -8.0, 30.0, -30.0, np.inf, -np.inf, 1.0, -1.0]],
                  np.float32)
    X = devf(sp)
    gsvk.bias_act(gsvk.ACT_GELU_ERF, X, X)
    sync()
    got = host(X, F32)
    want = O.bias_act(F32, 2, sp)
    fin = np.isfinite(want)
    assert_close(F32, got[fin], want[fin], "gelu special")
    assert got[0, 0] == 0 and got[0, 6] == 30.0 and got[0, 7] == 0
    # the reference's 0.5f * x * (1 + erff) keeps the sign of x on zero results: -0 -> -0, -30 -> -0
    np.testing.assert_array_equal(np.signbit(got[fin]), np.signbit(want[fin]))
    assert np.signbit(got[0, 1]) and np.signbit(got[0, 7]) and not np.signbit(got[0, 0])
    assert got[0, 8] == np.inf and np.isnan(got[0, 9])  # 0.5f*x*(1+erff(x)) at +-inf


@pytest.mark.parametrize("dt", [F32, F16])
def test_gelu_dense_sweep(dt):
    """The device GELU (erfc form, see gsvk_common.hpp) against the oracle's libm erff on every
    value of a dense grid over [-14, 14] plus the tiny / subnormal range, at the stated tolerance."""
    grid = np.linspace(-14, 14, 2 ** 20 + 1).astype(np.float32)
    tiny = np.float32(10.0) ** -np.linspace(5, 40, 4096).astype(np.float32)
    x32 = np.concatenate([grid, tiny, -tiny]).astype(np.float32)
    x32 = np.concatenate([x32, np.zeros((-x32.size) % 4096, np.float32)]).reshape(-1, 4096)
    x = st(dt, x32)
    want = O.bias_act(dt, gsvk.ACT_GELU_ERF, x)
    X = dev(x, dt)
    gsvk.bias_act(gsvk.ACT_GELU_ERF, X, X)
    sync()
    got = host(X, dt)
    assert_close(dt, got, want, "gelu sweep")
    # signs agree everywhere, zeros included (x <= -5.5 rounds erff to -1: the reference gives -0)
    g32, w32 = O.to_f32(dt, got), O.to_f32(dt, want)
    np.testing.assert_array_equal(np.signbit(g32), np.signbit(w32))


# ---- GroupNorm + GELU --------------------------------------------------------------------------

def hubert_conv0(seed):
    """Config 4 input: conv k10 s5 (no bias) of 10 s of 16 kHz audio ~ N(0, 0.1), 512 channels,
    weights ~ N(0, 0.3) -> [512, 31999] fp32."""
    r = rng(seed)
    audio = (0.1 * r.standard_normal(160000)).astype(np.float32)
    w = (0.3 * r.standard_normal((512, 10))).astype(np.float32)
    frames = np.lib.stride_tricks.as_strided(audio, shape=(31999, 10), strides=(20, 4))
    return np.ascontiguousarray((frames @ w.T).T.astype(np.float32))


@pytest.mark.parametrize("dt", [F32, F16])
def test_groupnorm_gelu_config4_matches_oracle(dt):
    say(f"groupnorm config4 dt={dt}")
    x32 = hubert_conv0(4000)
    x = st(dt, x32)
    r = rng(4001)
    g = (1 + 0.1 * r.standard_normal(512)).astype(np.float32)
    b = (0.1 * r.standard_normal(512)).astype(np.float32)
    want = O.groupnorm_gelu(dt, x, g, b, 1e-5)
    X = dev(x, dt)
    Y = torch.empty_like(X)
    gsvk.groupnorm_gelu(X, devf(g), devf(b), Y, 1e-5)
    sync()
    assert_close(dt, host(Y, dt), want, "groupnorm+gelu")


@pytest.mark.parametrize("C,T,dt,gelu", [(7, 1, F32, True), (5, 3, F32, False), (3, 1000, BF16, True),
                                         (4, 65537, F32, True), (3, 100001, F16, True),
                                         (6, 4097, F16, False),
                                         # the shortest rows of the register path (two 128-byte
                                         # lines) and the longest that take the generic one
                                         (9, 64, F32, True), (5, 63, F32, True),
                                         (4, 128, F16, True), (3, 127, BF16, False)])
def test_groupnorm_edge_shapes(C, T, dt, gelu):
    say(f"groupnorm C={C} T={T} dt={dt}")
    r = rng(C * T)
    x = st(dt, r.standard_normal((C, T)) * 0.5 + 0.3)
    g = (1 + 0.1 * r.standard_normal(C)).astype(np.float32)
    b = (0.1 * r.standard_normal(C)).astype(np.float32)
    want = O.groupnorm_gelu(dt, x, g, b, 1e-5, apply_gelu=gelu)
    X = dev(x, dt)
    gsvk.groupnorm_gelu(X, devf(g), devf(b), X, 1e-5, apply_gelu=gelu)  # in place
    sync()
    assert_close(dt, host(X, dt), want, f"groupnorm {C}x{T}")


@pytest.mark.parametrize("C,T,dt,params", [
    (1031, 8000, F32, True),    # 4 channels per workgroup and a ragged tail: both register buffers
    (600, 31999, F32, False),   # config 4's rows, no gamma / beta (1 / 0)
    (777, 9000, F16, True),     # 16-bit rows, 4 chunks per thread
])
def test_groupnorm_many_channels_per_workgroup(C, T, dt, params):
    """More channels than workgroups: each workgroup walks its channels through the two register
    buffers and the LDS buffer, and ends on either buffer."""
    say(f"groupnorm pipeline C={C} T={T} dt={dt} params={params}")
    r = rng(C + T)
    x = st(dt, r.standard_normal((C, T)) * 0.7 - 0.2)
    g = (1 + 0.1 * r.standard_normal(C)).astype(np.float32) if params else None
    b = (0.1 * r.standard_normal(C)).astype(np.float32) if params else None
    want = O.groupnorm_gelu(dt, x, g, b, 1e-5)
    X = dev(x, dt)
    Y = torch.empty_like(X)
    gsvk.groupnorm_gelu(X, devf(g) if params else None, devf(b) if params else None, Y, 1e-5)
    sync()
    assert_close(dt, host(Y, dt), want, f"groupnorm {C}x{T}")


def test_groupnorm_out_of_phase_buffers_use_generic_path():
    r = rng(55)
    C, T = 4, 999
    x = r.standard_normal((C, T)).astype(np.float32)
    g = np.ones(C, np.float32)
    b = np.zeros(C, np.float32)
    want = O.groupnorm_gelu(F32, x, g, b, 1e-5)
    X = devf(x)
    ybig = torch.zeros(C * T + 1, device="cuda")
    Y = ybig[1:].view(C, T)  # y is 4 bytes out of phase with x
    gsvk.groupnorm_gelu(X, devf(g), devf(b), Y, 1e-5)
    sync()
    assert_close(F32, host(Y, F32), want, "generic groupnorm")


# ---- SoVITS element-wise -------------------------------------------------------------------------

# the reference geometry's first and last stages, configuration 5's literal geometry (512 channels
# halving per stage: its first and last stages, 256 x 5000 and 32 x 320000), and a ragged small one
SOVITS_SHAPES = [(384, 5000), (24, 320000), (256, 5000), (32, 320000), (3, 1001)]


@pytest.mark.parametrize("C,T", SOVITS_SHAPES)
@pytest.mark.parametrize("dt", [F32, F16])
def test_leaky_relu_bit_exact(C, T, dt):
    r = rng(C + T + 1)
    x = st(dt, r.standard_normal(C * T))
    for slope in (0.1, 0.01):
        X = dev(x, dt)
        Y = torch.empty_like(X)
        gsvk.leaky_relu(X, Y, slope)  # leaky_relu_write
        gsvk.leaky_relu(X, X, slope)  # leaky_relu_io
        sync()
        want = O.leaky_relu(dt, x, slope)
        assert_bitexact(dt, host(Y, dt), want, "lrelu write")
        assert_bitexact(dt, host(X, dt), want, "lrelu io")


@pytest.mark.parametrize("C,T", SOVITS_SHAPES)
@pytest.mark.parametrize("dt", [F32, F16])
def test_resblock_add_lrelu_bit_exact(C, T, dt):
    r = rng(C + T + 2)
    cur = st(dt, r.standard_normal(C * T))
    tb = st(dt, r.standard_normal(C * T))
    want_cur, want_tin = O.resblock_add_lrelu(dt, cur, tb, 0.1)
    CUR, TB = dev(cur, dt), dev(tb, dt)
    TIN = torch.empty_like(CUR)
    gsvk.resblock_add_lrelu(CUR, TB, TIN, 0.1)
    sync()
    assert_bitexact(dt, host(CUR, dt), want_cur, "cur")
    assert_bitexact(dt, host(TIN, dt), want_tin, "t_in")
    CUR = dev(cur, dt)
    gsvk.resblock_add_lrelu(CUR, TB, None, 0.1)  # plain add_inplace
    sync()
    assert_bitexact(dt, host(CUR, dt), want_cur, "add only")


@pytest.mark.parametrize("C,T", SOVITS_SHAPES)
@pytest.mark.parametrize("dt", [F32, F16])
def test_resblock_branch_mean_bit_exact(C, T, dt):
    r = rng(C + T + 3)
    n = C * T
    curs = [st(dt, r.standard_normal(n)) for _ in range(3)]
    tbs = [st(dt, r.standard_normal(n)) for _ in range(3)]
    for slope, use_tb in ((0.1, True), (0.01, False)):
        want = O.resblock_branch_mean(dt, curs, tbs if use_tb else None, True, slope)
        OUT = torch.empty(n, dtype=dev(curs[0], dt).dtype, device="cuda")
        gsvk.resblock_branch_mean([dev(c, dt) for c in curs],
                                  [dev(t, dt) for t in tbs] if use_tb else None, OUT, True, slope)
        sync()
        assert_bitexact(dt, host(OUT, dt), want, f"branch mean slope={slope}")


@pytest.mark.parametrize("nb", [1, 2, 4])
def test_resblock_branch_mean_other_counts_and_no_lrelu(nb):
    r = rng(60 + nb)
    n = 10007
    curs = [st(F32, r.standard_normal(n)) for _ in range(nb)]
    want = O.resblock_branch_mean(F32, curs, None, False, 0.1)
    OUT = torch.empty(n, device="cuda")
    gsvk.resblock_branch_mean([devf(c) for c in curs], None, OUT, False, 0.1)
    sync()
    assert_bitexact(F32, host(OUT, F32), want, "branch mean nb")


@pytest.mark.parametrize("dt", [F32, BF16])
def test_scaled_add_and_unaligned_elementwise(dt):
    r = rng(70)
    n = 4099
    acc, src = st(dt, r.standard_normal(n)), st(dt, r.standard_normal(n))
    k = float(np.float32(1) / np.float32(3))
    A, S = dev(acc, dt), dev(src, dt)
    OUT = torch.empty_like(S)
    gsvk.scaled_add(None, S, OUT, k)  # mul_write
    gsvk.scaled_add(A, S, A, k)       # add_scaled_inplace
    sync()
    assert_bitexact(dt, host(OUT, dt), O.scaled_add(dt, None, src, k), "mul_write")
    assert_bitexact(dt, host(A, dt), O.scaled_add(dt, acc, src, k), "add_scaled_inplace")
    # unaligned buffers take the scalar kernels
    big = torch.zeros(n + 1, dtype=S.dtype, device="cuda")
    big[1:].copy_(S)
    out = torch.zeros(n + 1, dtype=S.dtype, device="cuda")
    gsvk.leaky_relu(big[1:], out[1:], 0.1)
    sync()
    assert_bitexact(dt, host(out[1:], dt), O.leaky_relu(dt, src, 0.1), "unaligned lrelu")


# ---- embedding gather + alpha * PE ----------------------------------------------------------------

@pytest.fixture(scope="module")
def pe2048():
    return gsvk.pe_table(2048, 512)


@pytest.mark.parametrize("out_dt", ALL_DT)
def test_embed_config2_bit_exact(out_dt, pe2048):
    say(f"embed config2 out={out_dt}")
    r = rng(200)
    D = 512
    text_tab = (0.02 * r.standard_normal((732, D))).astype(np.float16).view(np.uint16)
    audio_tab = (0.02 * r.standard_normal((1025, D))).astype(np.float16).view(np.uint16)
    a_text, a_audio = (float(np.float32(v)) for v in r.uniform(0.5, 1.5, 2))
    phones = r.integers(0, 732, 512).astype(np.int64)
    prompt = r.integers(0, 1025, 512).astype(np.int64)
    mm = st(out_dt, r.standard_normal((512, D)))
    bert_b = (0.02 * r.standard_normal(D)).astype(np.float32)
    dec_ids = r.integers(0, 1025, 64).astype(np.int32)
    dec_pos = r.integers(512, 2048, 64).astype(np.int64)
    PE = devf(pe2048)
    # text rows: positions 0..T-1, x = mm; x += e + b; x += alpha*pe (t2s_engine.cpp:1774-1780)
    want, bad = O.embed_pe(out_dt, F16, text_tab, phones, pe2048, a_text, pos0=0, mm=mm, bias=bert_b)
    OUT = torch.empty((512, D), dtype=dev(mm, out_dt).dtype, device="cuda")
    gsvk.embed_pe(dev(text_tab, F16), torch.from_numpy(phones).cuda(), PE, a_text, OUT, pos0=0,
                  mm=dev(mm, out_dt), bias=devf(bert_b))
    sync()
    assert bad == 0
    assert_bitexact(out_dt, host(OUT, out_dt), want, "text rows")
    # prompt rows: positions 0..P-1, x = e + alpha*pe (1781-1786)
    want, _ = O.embed_pe(out_dt, F16, audio_tab, prompt, pe2048, a_audio, pos0=0)
    gsvk.embed_pe(dev(audio_tab, F16), torch.from_numpy(prompt).cuda(), PE, a_audio, OUT)
    sync()
    assert_bitexact(out_dt, host(OUT, out_dt), want, "prompt rows")
    # decode rows: int32 ids, per-row positions (1866-1869)
    want, _ = O.embed_pe(out_dt, F16, audio_tab, dec_ids, pe2048, a_audio, pos=dec_pos)
    OUT2 = OUT[:64]
    gsvk.embed_pe(dev(audio_tab, F16), torch.from_numpy(dec_ids).cuda(), PE, a_audio, OUT2,
                  pos=torch.from_numpy(dec_pos).cuda())
    sync()
    assert_bitexact(out_dt, host(OUT2, out_dt), want, "decode rows")


PREFILL_CASES = [
    # (out dtype, T, P, D, text rows with bert_proj rows mm in place / apart / none, bias, int32)
    (F16, 512, 512, 512, "inplace", True, False),   # configuration 2's prefill input
    (F32, 512, 512, 512, "apart", True, True),
    (BF16, 512, 512, 512, None, False, False),
    (F16, 300, 77, 512, "inplace", True, False),    # more text than prompt rows
    (F16, 5, 260, 256, "apart", False, True),       # more prompt rows, narrower model
    (F32, 33, 40, 1024, "inplace", True, False),    # two column blocks per lane
    (F16, 9000, 8500, 512, "inplace", True, False), # 9000 positions: four-wave workgroups
    (F16, 20, 10, 6, "apart", True, False),         # D % 8 != 0: two gather launches
]


@pytest.mark.parametrize("case", PREFILL_CASES, ids=lambda c: "-".join(map(str, c)))
def test_prefill_input_equals_two_gathers_bit_exact(case, pe2048):
    """gsvk_t2s_prefill_input: every text row and every prompt row has the bits of the oracle's
    gather of that row (the two reference loops, t2s_engine.cpp:1774-1786)."""
    out_dt, T, P, D, mm_kind, use_bias, i32 = case
    say(f"prefill input {case}")
    r = rng(220 + T + P + D)
    pe = pe2048 if D == 512 and max(T, P) <= 2048 else gsvk.pe_table(max(T, P), D)
    text_tab = (0.02 * r.standard_normal((732, D))).astype(np.float16).view(np.uint16)
    audio_tab = (0.02 * r.standard_normal((1025, D))).astype(np.float16).view(np.uint16)
    a_text, a_audio = (float(np.float32(v)) for v in r.uniform(0.5, 1.5, 2))
    idt = np.int32 if i32 else np.int64
    phones = r.integers(0, 732, T).astype(idt)
    prompt = r.integers(0, 1025, P).astype(idt)
    mm = st(out_dt, r.standard_normal((T, D))) if mm_kind else None
    bert_b = (0.02 * r.standard_normal(D)).astype(np.float32) if use_bias else None
    want_t, bad_t = O.embed_pe(out_dt, F16, text_tab, phones, pe, a_text, pos0=0, mm=mm,
                               bias=bert_b)
    want_a, bad_a = O.embed_pe(out_dt, F16, audio_tab, prompt, pe, a_audio, pos0=0)
    assert bad_t == 0 and bad_a == 0
    XY = torch.empty((T + P, D), dtype=TORCH_DT[out_dt], device="cuda")
    MM = None
    if mm_kind == "inplace":
        XY[:T].copy_(dev(mm, out_dt))
        MM = XY
    elif mm_kind == "apart":
        MM = dev(mm, out_dt)
    err = torch.zeros(1, dtype=torch.int32, device="cuda")
    gsvk.t2s_prefill_input(dev(text_tab, F16), torch.from_numpy(phones).cuda(), a_text,
                           dev(audio_tab, F16), torch.from_numpy(prompt).cuda(), a_audio,
                           devf(pe), XY, mm=MM, bias=None if bert_b is None else devf(bert_b),
                           err=err)
    sync()
    got = host(XY, out_dt)
    assert int(err.item()) == 0
    assert_bitexact(out_dt, got[:T], want_t, "text rows")
    assert_bitexact(out_dt, got[T:], want_a, "prompt rows")


def test_prefill_input_out_of_range_rows(pe2048):
    """Bad ids in either gather, and positions past the PE table, give NaN rows and the flag; the
    other rows keep their bits."""
    r = rng(230)
    D, T, P = 512, 40, 30
    pe = pe2048[:35]  # positions 35.. are outside the table
    text_tab = (0.02 * r.standard_normal((100, D))).astype(np.float16).view(np.uint16)
    audio_tab = (0.02 * r.standard_normal((100, D))).astype(np.float16).view(np.uint16)
    phones = r.integers(0, 100, T).astype(np.int64)
    prompt = r.integers(0, 100, P).astype(np.int64)
    phones[[3, 7]] = [100, -2]
    prompt[5] = 1000
    want_t, bad_t = O.embed_pe(F16, F16, text_tab, phones, pe, 0.7, pos0=0)
    want_a, bad_a = O.embed_pe(F16, F16, audio_tab, prompt, pe, 0.9, pos0=0)
    assert bad_t == 2 + (T - 35) and bad_a == 1
    XY = torch.empty((T + P, D), dtype=torch.float16, device="cuda")
    err = torch.zeros(1, dtype=torch.int32, device="cuda")
    gsvk.t2s_prefill_input(dev(text_tab, F16), torch.from_numpy(phones).cuda(), 0.7,
                           dev(audio_tab, F16), torch.from_numpy(prompt).cuda(), 0.9, devf(pe), XY,
                           err=err)
    sync()
    assert int(err.item()) == 1
    got = host(XY, F16)
    assert_bitexact(F16, got[:T], want_t, "text rows")
    assert_bitexact(F16, got[T:], want_a, "prompt rows")


def test_embed_out_of_range_sets_flag_and_nan_rows(pe2048):
    r = rng(201)
    D = 512
    tab = r.standard_normal((100, D)).astype(np.float32)
    ids = np.array([0, 99, 100, -5, 7], np.int64)
    pos = np.array([0, 2047, 3, 4, 2048], np.int64)
    want, bad = O.embed_pe(F32, F32, tab, ids, pe2048, 0.8, pos=pos)
    assert bad == 3
    ERR = torch.zeros(1, dtype=torch.int32, device="cuda")
    OUT = torch.empty((5, D), device="cuda")
    gsvk.embed_pe(devf(tab), torch.from_numpy(ids).cuda(), devf(pe2048), 0.8, OUT,
                  pos=torch.from_numpy(pos).cuda(), err=ERR)
    sync()
    assert int(ERR.item()) == 1
    assert_bitexact(F32, host(OUT, F32), want, "oob rows")


def test_embed_f32_table_odd_width_scalar_path():
    r = rng(202)
    D = 10  # not a multiple of 8: scalar path
    tab = r.standard_normal((20, D)).astype(np.float32)
    pe = gsvk.pe_table(64, D)
    ids = r.integers(0, 20, 33).astype(np.int64)
    want, _ = O.embed_pe(F16, F32, tab, ids, pe, 1.1, pos0=5)
    OUT = torch.empty((33, D), dtype=torch.float16, device="cuda")
    gsvk.embed_pe(devf(tab), torch.from_numpy(ids).cuda(), devf(pe), 1.1, OUT, pos0=5)
    sync()
    assert_bitexact(F16, host(OUT, F16), want, "scalar embed")


def test_f16_store_rounds_subnormal_ties_to_even():
    """Every half-subnormal midpoint (k + 1/2) * 2^-24, its fp32 neighbours and the overflow
    boundary, stored to fp16 by a kernel: must round to nearest, ties to even."""
    k = np.arange(0, 1025, dtype=np.float32)
    mids = (k + np.float32(0.5)) * np.float32(2.0 ** -24)
    vals = np.concatenate([mids, -mids, np.nextafter(mids, np.float32(0)),
                           np.nextafter(mids, np.float32(1)), k * np.float32(2.0 ** -24),
                           np.array([2.0 ** -14, 65504, 65519.99, 65520, 1e-30], np.float32)])
    vals = vals.astype(np.float32)
    want = vals.astype(np.float16).view(np.uint16)  # numpy: correctly rounded, ties to even
    # The embed kernel with alpha = 0 and a zero PE row computes fmaf(0, 0, e) = e exactly for a
    # fp32 table row e (no signed zeros in vals), then stores it once as fp16.
    D = vals.size + (-vals.size) % 8
    tab = np.zeros((1, D), np.float32)
    tab[0, :vals.size] = vals
    pe = np.zeros((1, D), np.float32)
    OUT = torch.empty((1, D), dtype=torch.float16, device="cuda")
    gsvk.embed_pe(devf(tab), torch.zeros(1, dtype=torch.int64, device="cuda"), devf(pe), 0.0, OUT)
    sync()
    got = host(OUT, F16)[0, :vals.size]
    bad = np.flatnonzero(got != want)
    assert bad.size == 0, (vals[bad[:5]], got[bad[:5]], want[bad[:5]])


@pytest.mark.parametrize("n,offset", [(1, 0), (7, 0), (8, 0), (1001, 0), (4099, 1), (1 << 20, 0)])
def test_f32_to_f16_bit_exact(n, offset):
    """gsvk_f32_to_f16 (kern::f32_to_f16, gemv_fmlal.cpp:23-35) against numpy's round-to-nearest-
    even cast, bit for bit: ties, subnormals, overflow to inf, infinities and NaN; vector body and
    tail, and an output off the 16-byte alignment (element path)."""
    r = rng(700 + n)
    x = (r.standard_normal(n) * 10.0 ** r.uniform(-9, 5, n)).astype(np.float32)
    special = np.array([0.0, -0.0, 65504.0, 65519.99, 65520.0, -70000.0, 2.0 ** -24, 2.0 ** -25,
                        3 * 2.0 ** -26, 1e-8, np.inf, -np.inf, np.nan, 1.0 + 2.0 ** -11,
                        1.0 + 3 * 2.0 ** -11, -(2.0 ** -14) * 0.75], dtype=np.float32)
    x[:min(n, special.size)] = special[:min(n, special.size)]
    want = x.astype(np.float16).view(np.uint16)
    xd = devf(x)
    buf = torch.zeros(n + offset, dtype=torch.float16, device="cuda")
    y = buf[offset:]
    gsvk.f32_to_f16(xd, y)
    sync()
    got = y.cpu().view(torch.int16).numpy().view(np.uint16)
    nan = np.isnan(x)
    assert np.array_equal(np.isnan(got.view(np.float16)), nan)
    assert np.array_equal(got[~nan], want[~nan])
