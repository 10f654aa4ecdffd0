"""GPU parity of gsvk_conv1d (SoVITS Conv1d on the matrix cores with the ResBlock epilogues fused)
against the oracle's restatement of Conv1d::forward (conv1d.hpp:109-194) and the passes after it
in Generator::forward (dec.hpp:322-326).

Tolerance: the sum is formed in another order than the reference's (matrix-core tiles over 32
channels x one tap), so results follow the reference's own rule between two summation orders
(test_kern.cpp:111-118): |got - want| <= 1e-5 * max(1, max_t |conv[o, t]|) per output row o, plus
one fp32 step of the result (the residual add after it), and one fp16 step for fp16 storage (a
difference at the 1e-5 level can cross a rounding boundary). NaN / inf positions must agree.

Full reference sizes (the decoder stages at 500 frames, T up to 320,000) are checked through
column windows: a same-padded convolution restricted to columns [a, b) only reads x columns
[a - pad, b - pad + halo), so the oracle run on x[:, a - halo : b + halo] (clipped to [0, T), where
the clip coincides with the zero padding) gives exactly those outputs.
"""
import numpy as np
import pytest
import torch

import gsvk
import oracle as O
from gpu_util import F16, F32, dev, devf, host, say

pytestmark = pytest.mark.gpu


def rng(k):
    return np.random.default_rng(20250823 + 17000 + k)


def step16(w):
    w = np.abs(w.astype(np.float64))
    return np.spacing(np.minimum(w, 65504).astype(np.float16)).astype(np.float64)


def assert_conv_close(dt, got, want, conv_ref, what=""):
    g = O.to_f32(dt, got).astype(np.float64)
    w = O.to_f32(dt, want).astype(np.float64)
    assert g.shape == w.shape
    gn, wn = ~np.isfinite(g), ~np.isfinite(w)
    assert np.array_equal(np.isnan(g), np.isnan(w)), f"{what}: NaN positions differ"
    assert np.array_equal(np.isinf(g), np.isinf(w)), f"{what}: inf positions differ"
    assert np.array_equal(g[np.isinf(w)], w[np.isinf(w)]), f"{what}: inf signs differ"
    c = np.abs(O.to_f32(F32 if conv_ref.dtype == np.float32 else dt, conv_ref).astype(np.float64))
    c[~np.isfinite(c)] = 0
    peak = np.maximum(1.0, c.max(axis=1, keepdims=True))
    tol = 1e-5 * peak + 2.0 ** -23 * np.abs(w)
    if dt == F16:
        tol = tol + step16(w)
    err = np.abs(g - w)
    err[wn] = 0
    bad = np.argwhere(err > tol)
    assert bad.size == 0, f"{what}: {len(bad)} outside tolerance, worst {np.max(err - tol):.3e} " \
                          f"at {bad[:3].tolist()}"
    return float(np.max(err / peak))


def make(r, cin, cout, T, k, dt=F32, wscale=None, xscale=1.0):
    wscale = wscale if wscale is not None else 1.0 / np.sqrt(cin * k)
    x = O.to_storage(dt, (xscale * r.standard_normal((cin, T))).astype(np.float32))
    w = (wscale * r.standard_normal((cout, cin, k))).astype(np.float16).view(np.uint16)
    b = (0.05 * r.standard_normal(cout)).astype(np.float32)
    cur = O.to_storage(dt, r.standard_normal((cout, T)).astype(np.float32))
    return x, w, b, cur


def run_gpu(dt, x, w, b, dil, epi, cur=None, round_x=False, slope=0.1, ld_pad=0, y_offset=0):
    cin, T = x.shape
    cout, _, k = w.shape
    xd = dev(np.pad(x, ((0, 0), (0, ld_pad))), dt)[:, :T] if ld_pad else dev(x, dt)
    conv = gsvk.Conv1d(dev(w, F16), devf(b) if b is not None else None, dil)
    if b is None:
        conv.b = None
    yd = None
    if epi != gsvk.CONV_EPI_RES:
        buf = torch.empty(cout * (T + ld_pad) + y_offset, dtype=xd.dtype, device="cuda")
        yd = buf[y_offset:].view(cout, T + ld_pad)[:, :T] if ld_pad else \
            buf[y_offset:].view(cout, T)
    cd = dev(cur, dt) if cur is not None else None
    conv.forward(xd, yd, epi=epi, slope=slope, cur=cd, round_x=round_x)
    torch.cuda.synchronize()
    y = host(yd, dt) if yd is not None else None
    c = host(cd, dt) if cd is not None else None
    return y, c


def check_case(dt, cin, cout, T, k, dil, epi=0, round_x=False, use_bias=True, seed=0, ld_pad=0,
               y_offset=0, what=""):
    r = rng(seed)
    x, w, b, cur = make(r, cin, cout, T, k, dt)
    b = b if use_bias else None
    xo = O.to_storage(F32, O.to_f32(F16, O.to_storage(F16, x))) if round_x else x
    ref0 = O.conv1d(dt, xo, w, b, dil)  # the plain convolution: the tolerance scale
    has_res = epi in (gsvk.CONV_EPI_RES_LRELU, gsvk.CONV_EPI_RES)
    want = O.conv1d(dt, xo, w, b, dil, epi=epi, slope=0.1, cur=cur if has_res else None)
    y, c = run_gpu(dt, x, w, b, dil, epi, cur=cur if has_res else None, round_x=round_x,
                   ld_pad=ld_pad, y_offset=y_offset)
    tag = f"{what} dt={dt} {cin}->{cout} T={T} k={k} dil={dil} epi={epi} rx={round_x}"
    if epi in (2, 3):
        want_y, want_c = want
        e = assert_conv_close(dt, c, want_c, ref0, tag + " cur")
        if epi == 2:
            e = max(e, assert_conv_close(dt, y, want_y, ref0, tag + " y"))
    else:
        e = assert_conv_close(dt, y, want, ref0, tag)
    say(f"{tag}: max err / peak {e:.2e}")


# The decoder's ResBlock convolutions (ResBlock1: k 3 / 7 / 11, conv1 dilations 1 / 3 / 5, conv2
# dilation 1) at the stage channel counts 384 .. 24, with T cut to oracle-friendly lengths.
STAGES = [(384, 600), (192, 1000), (96, 1500), (48, 2000), (24, 3000)]


@pytest.mark.parametrize("C,T", STAGES)
@pytest.mark.parametrize("k,dil", [(3, 1), (7, 3), (11, 5)])
def test_resblock_conv1_fp32(C, T, k, dil):
    check_case(F32, C, C, T, k, dil, epi=gsvk.CONV_EPI_LRELU, seed=C + k)


@pytest.mark.parametrize("C,T", STAGES[1::2])
@pytest.mark.parametrize("epi", [gsvk.CONV_EPI_BIAS, gsvk.CONV_EPI_RES_LRELU, gsvk.CONV_EPI_RES])
def test_resblock_conv2_epilogues_fp32(C, T, epi):
    check_case(F32, C, C, T, 7, 1, epi=epi, seed=C + 31 * epi)


@pytest.mark.parametrize("epi", [0, 1, 2, 3])
def test_fp16_storage(epi):
    check_case(F16, 96, 96, 700, 11, 5, epi=epi, seed=40 + epi)


@pytest.mark.parametrize("C,k,dil", [(192, 3, 1), (48, 11, 5)])
def test_round_x_mode(C, k, dil):
    """round_x = 1: x rounded to fp16 first (the reference's AMX panel packing)."""
    check_case(F32, C, C, 500, k, dil, epi=0, round_x=True, seed=50 + C)


@pytest.mark.parametrize("cin,cout,T,k,dil", [
    (20, 5, 37, 3, 1),      # C_in and C_out below one chunk / fragment
    (45, 33, 130, 5, 2),    # ragged chunks and fragments, odd T
    (64, 17, 1, 7, 1),      # a single column: every tap but the centre reads padding
    (32, 16, 3, 11, 5),     # the halo spans the whole sequence
    (70, 100, 257, 4, 3),   # even k: pad (k - 1) dil / 2 rounds down
    (50, 40, 300, 1, 1),    # k = 1: a matrix product
    (40, 24, 400, 11, 20),  # halo 200 > 64: the wide-halo tile
    (40, 36, 700, 5, 4),    # halo 16: the largest the 16-column halo slab takes
    (40, 36, 700, 3, 9),    # halo 18: the first past it (64-column halo block)
    (192, 768, 50, 7, 1),   # conv_pre (192 -> 768, k 7) at 50 frames
])
def test_shapes_and_edges(cin, cout, T, k, dil):
    check_case(F32, cin, cout, T, k, dil, epi=0, seed=cin + cout + T)


def test_conv_post_no_bias():
    """conv_post: 24 -> 1 channel, k 7, no bias (conv1d.hpp:82-88)."""
    check_case(F32, 24, 1, 5000, 7, 1, epi=0, use_bias=False, seed=60)


@pytest.mark.parametrize("dt", [F32, F16])
def test_strided_and_unaligned_rows(dt):
    """x and y rows with ld > T (x, y) and a y base off the vector alignment (scalar stores)."""
    check_case(dt, 48, 40, 301, 3, 1, epi=1, ld_pad=7, seed=70, what="ld")
    check_case(dt, 48, 40, 300, 3, 1, epi=1, y_offset=1, seed=71, what="offset")


def test_nonfinite_inputs():
    r = rng(80)
    cin, cout, T, k, dil = 40, 20, 200, 7, 3
    x, w, b, _ = make(r, cin, cout, T, k)
    x[3, 50] = np.inf
    x[7, 120] = np.nan
    x[12, 199] = -np.inf
    want = O.conv1d(F32, x, w, b, dil)
    y, _ = run_gpu(F32, x, w, b, dil, 0)
    assert_conv_close(F32, y, want, want, "non-finite")


@pytest.mark.parametrize("round_x", [False, True])
def test_nonfinite_inputs_in_the_halo_slab(round_x):
    """k 3: the 16-column halo slab stages the columns past each 128-column tile (here 127 .. 142 of
    the first tile, 255 .. 270 of the second): inf / NaN placed there, and at a tile's first column,
    must reach exactly the outputs the oracle's sums reach."""
    r = rng(85 + round_x)
    cin, cout, T, k, dil = 40, 20, 600, 3, 1
    x, w, b, _ = make(r, cin, cout, T, k)
    x[3, 128] = np.inf
    x[7, 129] = np.nan
    x[12, 255] = -np.inf
    x[33, 256] = np.inf
    x[39, 142] = -np.inf
    xo = O.to_storage(F32, O.to_f32(F16, O.to_storage(F16, x))) if round_x else x
    want = O.conv1d(F32, xo, w, b, dil)
    y, _ = run_gpu(F32, x, w, b, dil, 0, round_x=round_x)
    assert_conv_close(F32, y, want, want, f"non-finite slab rx={round_x}")


def test_deterministic():
    r = rng(90)
    x, w, b, _ = make(r, 96, 96, 3000, 11)
    y1, _ = run_gpu(F32, x, w, b, 5, 0)
    y2, _ = run_gpu(F32, x, w, b, 5, 0)
    assert np.array_equal(y1.view(np.uint32), y2.view(np.uint32))


# Full decoder stage sizes (reference geometry, 500 frames), windowed oracle.
FULL = [(384, 5000, 11, 5), (192, 40000, 7, 3), (96, 80000, 3, 1), (48, 160000, 11, 1),
        (24, 320000, 11, 5)]


@pytest.mark.parametrize("C,T,k,dil", FULL)
def test_full_stage_windows(C, T, k, dil):
    r = rng(100 + C)
    x, w, b, cur = make(r, C, C, T, k)
    halo = (k - 1) * dil
    xd, cd = dev(x, F32), dev(cur, F32)
    conv = gsvk.Conv1d(dev(w, F16), devf(b), dil)
    yd = torch.empty(C, T, dtype=torch.float32, device="cuda")
    conv.forward(xd, yd, epi=gsvk.CONV_EPI_RES_LRELU, slope=0.1, cur=cd)
    torch.cuda.synchronize()
    y, c = host(yd, F32), host(cd, F32)
    width = 96
    starts = [0, 250, T // 2 - 37, T - 300, T - width]
    for a in starts:
        bnd = a + width
        w0, w1 = max(0, a - halo), min(T, bnd + halo)
        ref0 = O.conv1d(F32, x[:, w0:w1], w, b, dil)[:, a - w0:bnd - w0]
        wy, wc = O.conv1d(F32, x[:, w0:w1], w, b, dil, epi=2, slope=0.1, cur=cur[:, w0:w1])
        assert_conv_close(F32, c[:, a:bnd], wc[:, a - w0:bnd - w0], ref0, f"cur[{a}:{bnd}]")
        assert_conv_close(F32, y[:, a:bnd], wy[:, a - w0:bnd - w0], ref0, f"y[{a}:{bnd}]")
    say(f"full stage C={C} T={T} k={k} dil={dil}: {len(starts)} windows ok")


# ---- ConvTranspose1d (the upsampler) ------------------------------------------------------------

def run_gpu_t(dt, x, w, b, u, epi=0, cur=None, round_x=False, ld_pad=0):
    cin, T = x.shape
    _, cout, k = w.shape
    xd = dev(x, dt)
    conv = gsvk.ConvT1d(dev(w, F16), devf(b) if b is not None else None, u)
    if b is None:
        conv.b = None
    yd = None
    if epi != gsvk.CONV_EPI_RES:
        buf = torch.empty(cout, T * u + ld_pad, dtype=xd.dtype, device="cuda")
        yd = buf[:, :T * u]
    cd = dev(cur, dt) if cur is not None else None
    conv.forward(xd, yd, epi=epi, slope=0.1, cur=cd, round_x=round_x)
    torch.cuda.synchronize()
    return (host(yd, dt) if yd is not None else None), (host(cd, dt) if cd is not None else None)


def check_t(dt, cin, cout, T, k, u, epi=0, round_x=False, use_bias=True, seed=0, ld_pad=0):
    r = rng(seed)
    x = O.to_storage(dt, r.standard_normal((cin, T)).astype(np.float32))
    w = (r.standard_normal((cin, cout, k)) / np.sqrt(cin * k / u)).astype(np.float16).view(np.uint16)
    b = (0.05 * r.standard_normal(cout)).astype(np.float32) if use_bias else None
    cur = O.to_storage(dt, r.standard_normal((cout, T * u)).astype(np.float32)) if epi >= 2 else None
    xo = O.to_storage(F32, O.to_f32(F16, O.to_storage(F16, x))) if round_x else x
    ref0 = O.convt1d(dt, xo, w, u, b)
    want = O.convt1d(dt, xo, w, u, b, epi=epi, slope=0.1, cur=cur)
    y, c = run_gpu_t(dt, x, w, b, u, epi=epi, cur=cur, round_x=round_x, ld_pad=ld_pad)
    tag = f"convT dt={dt} {cin}->{cout} T={T} k={k} u={u} epi={epi} rx={round_x}"
    if epi in (2, 3):
        e = assert_conv_close(dt, c, want[1], ref0, tag + " cur")
        if epi == 2:
            e = max(e, assert_conv_close(dt, y, want[0], ref0, tag + " y"))
    else:
        e = assert_conv_close(dt, y, want, ref0, tag)
    say(f"{tag}: max err / peak {e:.2e}")


# Generator.ups (dec.hpp:55-76): 768 -> 384 (k 20, u 10), 384 -> 192 (16, 8), 192 -> 96 (8, 2),
# 96 -> 48 (2, 2), 48 -> 24 (2, 2), with T cut to oracle-friendly lengths.
UPS = [(768, 384, 40, 20, 10), (384, 192, 150, 16, 8), (192, 96, 400, 8, 2), (96, 48, 900, 2, 2),
       (48, 24, 2000, 2, 2)]


@pytest.mark.parametrize("cin,cout,T,k,u", UPS)
def test_upsample_stages_fp32(cin, cout, T, k, u):
    check_t(F32, cin, cout, T, k, u, seed=cin + k)


@pytest.mark.parametrize("cin,cout,T,k,u", [
    (20, 5, 7, 5, 2),     # odd k - u: pad rounds down, phases of unequal length
    (33, 17, 1, 3, 3),    # k == u (no overlap), one input column
    (40, 70, 2, 7, 3),    # ragged taps per phase (3, 2, 2), two input columns
    (64, 16, 37, 16, 8),
    (45, 33, 60, 4, 1),   # stride 1: an ordinary convolution with flipped taps
])
def test_upsample_edges(cin, cout, T, k, u):
    check_t(F32, cin, cout, T, k, u, seed=cin * 3 + T)


@pytest.mark.parametrize("epi", [1, 2, 3])
def test_upsample_epilogues(epi):
    check_t(F32, 96, 48, 300, 8, 2, epi=epi, seed=200 + epi)


def test_upsample_fp16_round_x_and_strided():
    check_t(F16, 96, 48, 300, 8, 2, seed=210)
    check_t(F32, 96, 48, 300, 16, 8, round_x=True, seed=211)
    check_t(F32, 48, 24, 301, 2, 2, use_bias=False, ld_pad=5, seed=212)


FULL_UPS = [(768, 384, 500, 20, 10), (384, 192, 5000, 16, 8), (192, 96, 40000, 8, 2),
            (96, 48, 80000, 2, 2), (48, 24, 160000, 2, 2)]


@pytest.mark.parametrize("cin,cout,T,k,u", FULL_UPS)
def test_upsample_full_stage_windows(cin, cout, T, k, u):
    r = rng(300 + cin)
    x = r.standard_normal((cin, T)).astype(np.float32)
    w = (r.standard_normal((cin, cout, k)) / np.sqrt(cin * k / u)).astype(np.float16).view(np.uint16)
    b = (0.05 * r.standard_normal(cout)).astype(np.float32)
    y, _ = run_gpu_t(F32, x, w, b, u)
    M = -(-k // u) + 1  # input columns that reach past a window edge
    width = 24
    for ja in [0, T // 3, T - width]:
        jb = ja + width
        wa, wb = max(0, ja - M), min(T, jb + M)
        win = O.convt1d(F32, x[:, wa:wb], w, u, b)
        ga = 0 if ja == 0 else ja * u        # complete output columns of the window
        gb = T * u if jb == T else jb * u
        got, want = y[:, ga:gb], win[:, ga - wa * u:gb - wa * u]
        assert_conv_close(F32, got, want, want, f"convT full {cin}->{cout} T={T} cols [{ga}, {gb})")
    say(f"convT full stage {cin}->{cout} T={T} k={k} u={u}: windows ok")



# ---- fused-pass epilogues used by the Generator stage ---------------------------------------------

def test_dual_epilogue_and_res_input_are_bitwise_the_plain_paths():
    """CONV_EPI_DUAL equals the plain convolution and a separate LeakyReLU of it, bit for bit; a
    residual read from `res` equals the in-place form on a copy, bit for bit (same tiles, same
    sums); for the transposed convolution as well."""
    r = rng(400)
    C, T = 48, 700
    x, w, b, cur = make(r, C, C, T, 7)
    xd, wd = dev(x, F32), dev(w, F16)
    conv = gsvk.Conv1d(wd, devf(b), 3)
    y0 = conv.forward(xd)
    y4 = torch.empty_like(y0)
    l4 = torch.empty_like(y0)
    conv.forward(xd, y4, epi=gsvk.CONV_EPI_DUAL, slope=0.1, cur=l4)
    lr = torch.empty_like(y0)
    gsvk.leaky_relu(y0, lr, 0.1)
    torch.cuda.synchronize()
    assert torch.equal(y4.view(torch.int32), y0.view(torch.int32))
    assert torch.equal(l4.view(torch.int32), lr.view(torch.int32))
    res = dev(cur, F32)
    c_a = res.clone()
    y_a = torch.empty_like(y0)
    conv.forward(xd, y_a, epi=gsvk.CONV_EPI_RES_LRELU, slope=0.1, cur=c_a)       # in place
    c_b = torch.full_like(y0, float("nan"))
    y_b = torch.empty_like(y0)
    conv.forward(xd, y_b, epi=gsvk.CONV_EPI_RES_LRELU, slope=0.1, cur=c_b, res=res)
    c_c = torch.full_like(y0, float("nan"))
    conv.forward(xd, None, epi=gsvk.CONV_EPI_RES, cur=c_c, res=res)
    torch.cuda.synchronize()
    assert torch.equal(c_b.view(torch.int32), c_a.view(torch.int32))
    assert torch.equal(y_b.view(torch.int32), y_a.view(torch.int32))
    assert torch.equal(c_c.view(torch.int32), c_a.view(torch.int32))
    assert torch.equal(res, dev(cur, F32))  # the residual source is only read
    # transposed: dual epilogue
    wt = (r.standard_normal((C, 24, 8)) / np.sqrt(C * 4)).astype(np.float16).view(np.uint16)
    up = gsvk.ConvT1d(dev(wt, F16), devf(b[:24]), 2)
    u0 = up.forward(xd)
    u4, ul = torch.empty_like(u0), torch.empty_like(u0)
    up.forward(xd, u4, epi=gsvk.CONV_EPI_DUAL, slope=0.1, cur=ul)
    ulr = torch.empty_like(u0)
    gsvk.leaky_relu(u0, ulr, 0.1)
    torch.cuda.synchronize()
    assert torch.equal(u4.view(torch.int32), u0.view(torch.int32))
    assert torch.equal(ul.view(torch.int32), ulr.view(torch.int32))


@pytest.mark.parametrize("dt", [F32, F16])
def test_tanh_epilogue_conv_post(dt):
    """conv_post (24 -> 1, k 7, no bias) with tanh fused (dec.hpp:343-344) against the oracle's
    conv + tanhf; tolerance: the convolution's, since |tanh'| <= 1, plus one fp32 / fp16 step."""
    check_case(dt, 24, 1, 3000, 7, 1, epi=gsvk.CONV_EPI_TANH, use_bias=False, seed=410)


# ---- 32-wide fragments (v_mfma_f32_32x32x16_f16, 256 positions x 64 rows per workgroup) --------
# The launcher takes them when 64-row tiles pad at most a sixth of the rows, the halo is <= 64 and
# the grid holds >= 384 such workgroups: the shapes below are the smallest that do (columns
# 256-ragged, output rows whole or 64-ragged within the sixth).
@pytest.mark.parametrize("C,T,k,dil,epi", [
    (64, 98305, 11, 5, gsvk.CONV_EPI_LRELU),       # one row block, ragged columns
    (64, 98304, 3, 1, gsvk.CONV_EPI_RES_LRELU),    # whole tiles only; residual + next LeakyReLU
    (120, 51201, 7, 3, gsvk.CONV_EPI_RES),          # 120 of 128 rows: a ragged second block
    (64, 98305, 11, 1, gsvk.CONV_EPI_BIAS),
    (64, 98305, 5, 4, gsvk.CONV_EPI_LRELU),  # halo 16: the slab's limit
])
def test_wide_tiles_fp32(C, T, k, dil, epi):
    check_case(F32, C, C, T, k, dil, epi=epi, seed=500 + C + k, what="wide")


def test_wide_tiles_fp16_round_x_and_strided():
    check_case(F16, 64, 64, 98305, 7, 3, epi=gsvk.CONV_EPI_RES_LRELU, seed=520, what="wide")
    check_case(F32, 64, 64, 98305, 11, 5, round_x=True, seed=521, what="wide")
    check_case(F32, 64, 64, 98305, 3, 1, epi=gsvk.CONV_EPI_LRELU, ld_pad=5, seed=522,
               what="wide ld")


def test_wide_tiles_transposed():
    """An upsampler phase grid of >= 384 wide workgroups: 128 -> 64, k 16, u 8 (stage 2's
    geometry, narrowed)."""
    check_t(F32, 128, 64, 12289, 16, 8, seed=530)
    check_t(F32, 128, 64, 12289, 16, 8, epi=gsvk.CONV_EPI_RES_LRELU, seed=531)


@pytest.mark.parametrize("dt,round_x", [(F32, False), (F32, True), (F16, False)])
def test_partial_channel_groups_on_interior_tiles(dt, round_x):
    """C_in = 45 over 5003 columns: most time tiles lie inside the sequence, and the second 32-channel
    chunk holds 13 channels, one whole 8-channel group and one partial (and two empty). Staging takes
    its interior path for the whole groups and the zeroing path for the others in the same tile.
    Against the oracle with the residual epilogue, and, reading lrelu(x) as it loads, bit for bit
    the convolution of the materialised lrelu(x)."""
    check_case(dt, 45, 40, 5003, 5, 2, epi=gsvk.CONV_EPI_RES_LRELU, round_x=round_x,
               seed=640 + dt + 2 * round_x, what="partial groups")
    r = rng(650 + dt + 2 * round_x)
    x, w, b, _ = make(r, 45, 40, 5003, 5, dt)
    xd = dev(x, dt)
    conv = gsvk.Conv1d(dev(w, F16), devf(b), 2)
    ya = conv.forward(xd, epi=gsvk.CONV_EPI_LRELU | gsvk.CONV_X_LRELU, slope=0.1, round_x=round_x)
    xl = torch.empty_like(xd)
    gsvk.leaky_relu(xd, xl, 0.1)
    yb = conv.forward(xl, epi=gsvk.CONV_EPI_LRELU, slope=0.1, round_x=round_x)
    torch.cuda.synchronize()
    assert torch.equal(ya.view(torch.int16), yb.view(torch.int16))


@pytest.mark.parametrize("dt,round_x", [(F32, False), (F32, True), (F16, False)])
def test_x_lrelu_input_equals_materialized_lrelu(dt, round_x):
    """GSVK_CONV_X_LRELU reads lrelu(x, slope) as the convolution loads x: bit for bit the same as
    materialising lrelu(x) first (gsvk_leaky_relu, one rounding to the storage type) and convolving
    that, for the convolution (both tile shapes' grids) and the transposed convolution; x itself is
    left unchanged."""
    r = rng(600 + dt + 2 * round_x)
    for C, T, k, dil in ((48, 3000, 7, 3), (64, 98305, 3, 1)):
        x, w, b, _ = make(r, C, C, T, k, dt)
        xd = dev(x, dt)
        x0 = xd.clone()
        conv = gsvk.Conv1d(dev(w, F16), devf(b), dil)
        ya = conv.forward(xd, epi=gsvk.CONV_EPI_LRELU | gsvk.CONV_X_LRELU, slope=0.1,
                          round_x=round_x)
        xl = torch.empty_like(xd)
        gsvk.leaky_relu(xd, xl, 0.1)
        yb = conv.forward(xl, epi=gsvk.CONV_EPI_LRELU, slope=0.1, round_x=round_x)
        torch.cuda.synchronize()
        assert torch.equal(xd.view(torch.int16), x0.view(torch.int16))
        assert torch.equal(ya.view(torch.int16), yb.view(torch.int16)), f"{C}x{T}"
    cin, cout, T, k, u = 96, 48, 700, 8, 2
    x = O.to_storage(dt, r.standard_normal((cin, T)).astype(np.float32))
    w = (r.standard_normal((cin, cout, k)) / np.sqrt(cin * k / u)).astype(np.float16)
    xd = dev(x, dt)
    up = gsvk.ConvT1d(dev(w.view(np.uint16), F16), None, u)
    ya = up.forward(xd, epi=gsvk.CONV_EPI_BIAS | gsvk.CONV_X_LRELU, slope=0.1, round_x=round_x)
    xl = torch.empty_like(xd)
    gsvk.leaky_relu(xd, xl, 0.1)
    yb = up.forward(xl, round_x=round_x)
    torch.cuda.synchronize()
    assert torch.equal(ya.view(torch.int16), yb.view(torch.int16))


def split_values(r, n):
    """fp32 values over the whole range the hi / lo split covers: magnitudes 2^-40 .. 2^15 (many
    with an fp16-subnormal remainder, every one below 2^-3), the end of the fp16 range
    (65504 <= |x| < 65520 rounds hi to 65504), both zeros and both signs."""
    e = r.uniform(-40.0, 15.99, n)
    x = np.exp2(e) * np.where(r.random(n) < 0.5, -1.0, 1.0)
    x[: n // 64] = r.uniform(65504.0, 65519.99, n // 64) * np.where(r.random(n // 64) < 0.5, -1, 1)
    x[n // 64: n // 64 + 16] = 0.0
    x[n // 64 + 16: n // 64 + 32] = -0.0
    return r.permutation(x.astype(np.float32))


@pytest.mark.parametrize("C", [64, 45])
@pytest.mark.parametrize("dt,round_x,xact", [(F32, False, False), (F32, False, True),
                                             (F32, True, False), (F32, True, True),
                                             (F16, False, True)])
def test_staging_split_with_identity_weights(C, dt, round_x, xact):
    """Identity weights (k 1, w[o, i] = 1 if o == i else 0) make each output the staged value itself:
    in the exact mode hi + lo of v, hi = f16(v), lo = f16(v - hi), added in fp32 (exact: at most 22
    significant bits), v = x or, with the input LeakyReLU (slope 0.1), lrelu(x); in round_x mode
    f16(v); with fp16 storage f16(v). The expected values come from numpy's fp16 rounding, so this
    pins the split bit for bit, fp16-subnormal remainders included. Zeros are compared as numbers
    (the other channels' zero products decide a zero sum's sign). T leaves a partial last tile and
    C = 45 a partial channel group, so both staging paths run."""
    r = rng(700 + C + 10 * dt + 2 * round_x + xact)
    T = 4096 + 37
    x = split_values(r, C * T).reshape(C, T)
    if dt == F16:
        x = np.clip(x, -60000, 60000).astype(np.float16).view(np.uint16)
    w = np.zeros((C, C, 1), np.float16)
    w[np.arange(C), np.arange(C), 0] = 1.0
    xd = dev(x, dt)
    conv = gsvk.Conv1d(dev(w.view(np.uint16), F16), None, 1)
    conv.b = None
    epi = gsvk.CONV_EPI_BIAS | (gsvk.CONV_X_LRELU if xact else 0)
    y = host(conv.forward(xd, epi=epi, slope=0.1, round_x=round_x), dt)
    torch.cuda.synchronize()
    v = O.to_f32(dt, x)
    if xact:
        v = np.where(v < 0, v * np.float32(0.1), v).astype(np.float32)
    hi = v.astype(np.float16)
    if dt == F16:
        want = hi.astype(np.float32)
    elif round_x:
        want = hi.astype(np.float32)
    else:
        lo = (v - hi.astype(np.float32)).astype(np.float16)
        want = hi.astype(np.float32) + lo.astype(np.float32)
    got = O.to_f32(dt, y)
    bad = np.argwhere(got != want)
    assert bad.size == 0, f"{len(bad)} differ, first {bad[:3].tolist()}: " \
                          f"x {v[tuple(bad[0])]!r} got {got[tuple(bad[0])]!r} want {want[tuple(bad[0])]!r}"
    say(f"identity split C={C} dt={dt} round_x={round_x} xact={xact}: {C * T} values exact")
