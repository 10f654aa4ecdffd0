"""Pins the oracle's SoVITS Conv1d (oracle_conv1d). The reference holds no golden tensors for the
decoder convolutions (its SoVITS fixtures are exported from checkpoints that are not available), so the
restatement is pinned by mathematics:
  - a float64 closed form built another way (a strided im2col of the padded input and one einsum),
    which the padding, dilation, bias and tap-order mistakes below all fail;
  - k = 1 is a matrix product;
  - a delta input reproduces the taps at t = t* - kk * dilation + pad (cross-correlation, as torch);
  - the epilogues are the reference's separate passes: leaky_relu_io, add_inplace, leaky_relu_write.
"""
import numpy as np
import pytest

import oracle as O

F32, F16 = O.F32, O.F16


@pytest.fixture(scope="module", autouse=True)
def _lib(oracle_lib):
    return oracle_lib


def closed_form(x, w, b, dil, pad=None, flip=False):
    """float64 same-padding Conv1d: y[o,t] = b[o] + sum_{i,kk} w[o,i,kk] x[i, t + kk*dil - pad]."""
    cout, cin, k = w.shape
    T = x.shape[1]
    pad = (k - 1) * dil // 2 if pad is None else pad
    xp = np.zeros((cin, T + 2 * (k - 1) * dil))
    off = (k - 1) * dil  # xp[:, off + s] = x[:, s]
    xp[:, off:off + T] = x
    wk = w[:, :, ::-1] if flip else w
    cols = np.stack([xp[:, off - pad + kk * dil: off - pad + kk * dil + T] for kk in range(k)], 1)
    y = np.einsum("oik,ikt->ot", wk.astype(np.float64), cols.astype(np.float64))
    return y + (0 if b is None else b[:, None])


def rnd(r, *s, std=1.0):
    return (std * r.standard_normal(s)).astype(np.float32)


@pytest.mark.parametrize("cin,cout,T,k,dil", [(8, 5, 50, 3, 1), (16, 12, 200, 7, 3), (4, 3, 37, 11, 5),
                                              (6, 2, 9, 11, 1), (3, 4, 64, 1, 1), (5, 5, 40, 4, 2)])
def test_conv_closed_form_and_planted_mistakes(cin, cout, T, k, dil):
    r = np.random.default_rng(cin * 100 + k)
    x = rnd(r, cin, T)
    w = (0.1 * r.standard_normal((cout, cin, k))).astype(np.float16)
    b = rnd(r, cout, std=0.02)
    got = O.conv1d(F32, x, w.view(np.uint16), b, dil).astype(np.float64)
    want = closed_form(x, w.astype(np.float64), b.astype(np.float64), dil)
    scale = np.einsum("oik,ikt->ot", np.abs(w.astype(np.float64)),
                      np.abs(np.stack([x] * k, 1)).astype(np.float64)) + 1.0
    tol = 1e-6 * scale
    assert np.all(np.abs(got - want) <= tol)
    mistakes = {"no bias": closed_form(x, w.astype(np.float64), None, dil),
                "causal pad": closed_form(x, w.astype(np.float64), b, dil, pad=(k - 1) * dil)}
    if k > 1:
        mistakes["flipped taps (convolution)"] = closed_form(x, w.astype(np.float64), b, dil, flip=True)
    if dil > 1:
        mistakes["no dilation"] = closed_form(x, w.astype(np.float64), b, 1)
    for name, bad in mistakes.items():
        if name == "causal pad" and (k - 1) * dil == 0:
            continue
        assert np.max(np.abs(got - bad)) > 100 * np.max(tol), name


def test_conv_k1_is_matmul():
    r = np.random.default_rng(3)
    x = rnd(r, 24, 100)
    w = (0.1 * r.standard_normal((7, 24, 1))).astype(np.float16)
    got = O.conv1d(F32, x, w.view(np.uint16))
    want = w[:, :, 0].astype(np.float64) @ x.astype(np.float64)
    assert np.max(np.abs(got - want)) < 1e-5


def test_conv_delta_input_gives_taps():
    cin, cout, T, k, dil = 3, 2, 40, 7, 3
    r = np.random.default_rng(4)
    w = (0.1 * r.standard_normal((cout, cin, k))).astype(np.float16)
    x = np.zeros((cin, T), np.float32)
    i0, t0 = 1, 20
    x[i0, t0] = 1.0
    y = O.conv1d(F32, x, w.view(np.uint16), None, dil)
    pad = (k - 1) * dil // 2
    for kk in range(k):
        t = t0 - kk * dil + pad
        assert np.array_equal(y[:, t], w[:, i0, kk].astype(np.float32))
    touched = {t0 - kk * dil + pad for kk in range(k)}
    assert np.all(y[:, [t for t in range(T) if t not in touched]] == 0)


def test_conv_epilogues_are_the_reference_passes():
    """fp32 (the decoder's type in the reference): the fused epilogues equal the separate passes
    bit for bit."""
    dt = F32
    r = np.random.default_rng(5)
    cin, cout, T, k = 6, 4, 30, 3
    x = rnd(r, cin, T)
    w = (0.3 * r.standard_normal((cout, cin, k))).astype(np.float16).view(np.uint16)
    b = rnd(r, cout, std=0.1)
    cur = rnd(r, cout, T)
    y0 = O.conv1d(dt, x, w, b)
    y1 = O.conv1d(dt, x, w, b, epi=1, slope=0.1)
    assert np.array_equal(y1, O.leaky_relu(dt, y0, 0.1))
    y2, c2 = O.conv1d(dt, x, w, b, epi=2, slope=0.1, cur=cur)
    c_want, t_in = O.resblock_add_lrelu(dt, cur, y0, 0.1)
    assert np.array_equal(c2, c_want) and np.array_equal(y2, t_in)
    _, c3 = O.conv1d(dt, x, w, b, epi=3, cur=cur)
    assert np.array_equal(c3, c_want)


def test_conv_f16_storage_rounds_each_output_once():
    """fp16 storage (this library's option; the reference keeps the decoder in fp32): every output
    is the fp32 epilogue value rounded to fp16 once."""
    r = np.random.default_rng(6)
    cin, cout, T, k = 6, 4, 30, 3
    x16 = O.to_storage(F16, rnd(r, cin, T))
    w = (0.3 * r.standard_normal((cout, cin, k))).astype(np.float16).view(np.uint16)
    b = rnd(r, cout, std=0.1)
    cur16 = O.to_storage(F16, rnd(r, cout, T))
    x32, cur32 = O.to_f32(F16, x16), O.to_f32(F16, cur16)
    y32 = O.conv1d(F32, x32, w, b)
    lr = lambda v: np.where(v > 0, v, np.float32(0.1) * v).astype(np.float32)
    assert np.array_equal(O.conv1d(F16, x16, w, b), O.to_storage(F16, y32))
    assert np.array_equal(O.conv1d(F16, x16, w, b, epi=1, slope=0.1), O.to_storage(F16, lr(y32)))
    c32 = (cur32 + y32).astype(np.float32)
    y2, c2 = O.conv1d(F16, x16, w, b, epi=2, slope=0.1, cur=cur16)
    assert np.array_equal(c2, O.to_storage(F16, c32)) and np.array_equal(y2, O.to_storage(F16, lr(c32)))


# ---- ConvTranspose1d ------------------------------------------------------------------------------
# Pinned against torch's own conv_transpose1d definition (float64, CPU), which shares nothing with
# the oracle's per-tap GEMM + scatter, and against planted mistakes.

def torch_convt(x, w, u, b=None):
    import torch
    cin, cout, k = w.shape
    pad = (k - u) // 2
    y = torch.nn.functional.conv_transpose1d(torch.from_numpy(x.astype(np.float64))[None],
                                             torch.from_numpy(w.astype(np.float64)), stride=u,
                                             padding=pad)[0].numpy()
    y = y[:, :x.shape[1] * u]  # an odd k - u leaves torch one extra column past T u
    return y + (0 if b is None else b.astype(np.float64)[:, None])


@pytest.mark.parametrize("cin,cout,T,k,u", [(16, 8, 40, 20, 10), (12, 6, 50, 16, 8),
                                            (10, 5, 60, 8, 2), (8, 4, 33, 2, 2), (6, 3, 21, 5, 2),
                                            (5, 7, 13, 7, 3), (4, 4, 9, 3, 3), (9, 5, 11, 1, 1)])
def test_convt_matches_torch_and_rejects_mistakes(cin, cout, T, k, u):
    r = np.random.default_rng(100 + k * u)
    x = rnd(r, cin, T)
    w = (r.standard_normal((cin, cout, k)) / np.sqrt(cin)).astype(np.float16)
    b = rnd(r, cout, std=0.05)
    got = O.convt1d(F32, x, w.view(np.uint16), u, b).astype(np.float64)
    want = torch_convt(x, w.astype(np.float64), u, b)
    assert got.shape == want.shape == (cout, T * u)
    tol = 1e-6 * (np.abs(want).max() + 1)
    assert np.max(np.abs(got - want)) <= tol
    w64 = w.astype(np.float64)
    mistakes = {"no bias": torch_convt(x, w64, u)}
    if k > 1:
        mistakes["flipped taps"] = torch_convt(x, w64[:, :, ::-1], u, b)
    if k - u >= 2:
        import torch
        mistakes["pad 0"] = torch.nn.functional.conv_transpose1d(
            torch.from_numpy(x.astype(np.float64))[None], torch.from_numpy(w64), stride=u)[0] \
            .numpy()[:, :T * u] + b[:, None]
    if cin == cout:
        mistakes["[out, in] layout"] = torch_convt(x, w64.transpose(1, 0, 2), u, b)
    for name, bad in mistakes.items():
        assert np.max(np.abs(got - bad)) > 100 * tol, name


def test_convt_delta_input_gives_taps():
    cin, cout, T, k, u = 3, 4, 10, 16, 8
    r = np.random.default_rng(7)
    w = (r.standard_normal((cin, cout, k)) / 4).astype(np.float16)
    x = np.zeros((cin, T), np.float32)
    i0, j0 = 2, 5
    x[i0, j0] = 1.0
    y = O.convt1d(F32, x, w.view(np.uint16), u)
    pad = (k - u) // 2
    for d in range(k):
        assert np.array_equal(y[:, j0 * u + d - pad], w[i0, :, d].astype(np.float32))
    touched = {j0 * u + d - pad for d in range(k)}
    assert np.all(y[:, [t for t in range(T * u) if t not in touched]] == 0)


def test_convt_stride1_k1_is_matmul():
    r = np.random.default_rng(8)
    x = rnd(r, 24, 50)
    w = (0.2 * r.standard_normal((24, 9, 1))).astype(np.float16)
    got = O.convt1d(F32, x, w.view(np.uint16), 1)
    want = w[:, :, 0].astype(np.float64).T @ x.astype(np.float64)
    assert np.max(np.abs(got - want)) < 1e-5


def test_convt_epilogues():
    r = np.random.default_rng(9)
    cin, cout, T, k, u = 6, 4, 12, 8, 2
    x = rnd(r, cin, T)
    w = (0.3 * r.standard_normal((cin, cout, k))).astype(np.float16).view(np.uint16)
    b = rnd(r, cout, std=0.1)
    cur = rnd(r, cout, T * u)
    y0 = O.convt1d(F32, x, w, u, b)
    assert np.array_equal(O.convt1d(F32, x, w, u, b, epi=1, slope=0.1), O.leaky_relu(F32, y0, 0.1))
    y2, c2 = O.convt1d(F32, x, w, u, b, epi=2, slope=0.1, cur=cur)
    c_want, t_in = O.resblock_add_lrelu(F32, cur, y0, 0.1)
    assert np.array_equal(c2, c_want) and np.array_equal(y2, t_in)


def test_conv_dual_and_tanh_epilogues():
    """epi 4 writes y and lrelu(y) (the upsampler output and the first pair's input); epi 5 is
    conv_post's tanh, against numpy's tanh of the plain convolution (float64, 1 ulp band)."""
    r = np.random.default_rng(11)
    x = rnd(r, 6, 40)
    w = (0.3 * r.standard_normal((4, 6, 7))).astype(np.float16).view(np.uint16)
    b = rnd(r, 4, std=0.1)
    y0 = O.conv1d(F32, x, w, b)
    y4, c4 = O.conv1d(F32, x, w, b, epi=4, slope=0.1)
    assert np.array_equal(y4, y0) and np.array_equal(c4, O.leaky_relu(F32, y0, 0.1))
    y5 = O.conv1d(F32, x, w, b, epi=5).astype(np.float64)
    want = np.tanh(y0.astype(np.float64))
    assert np.all(np.abs(y5 - want) <= 2 * np.spacing(np.abs(want).astype(np.float32)) + 1e-30)
    assert np.max(np.abs(y5 - y0)) > 0.01  # tanh is applied
    yt, ct = O.convt1d(F32, x, w.reshape(6, 4, 7), 2, b, epi=4, slope=0.1)
    assert np.array_equal(yt, O.convt1d(F32, x, w.reshape(6, 4, 7), 2, b))
    assert np.array_equal(ct, O.leaky_relu(F32, yt, 0.1))
