"""The whole SoVITS decoder on the GPU (gsvk_sovits_decoder_*, include/gsvk_sovits.h) against the
oracle chained in Generator::forward's order (dec.hpp:264-345):
  x = conv_pre(z) + b_pre;  x += cond(ge)[:, 0] (broadcast over frames);
  per stage: x = lrelu(x, 0.1); y = ups(x); three ResBlock1 chains; x = mean of the branches;
  x = lrelu(x, 0.01); out = tanh(conv_post(x)).

Tolerance: |d| <= 1e-4 at the output (tanh values, |out| <= 1). Each convolution meets its own fp32
bound; the GPU folds the broadcast add into conv_pre's bias (one fp32 rounding in another place) and
the summation order of every convolution differs from the oracle's, noise that compounds through
the 5 stages to ~1e-6 here. round_x: the convolutions see fp16-rounded inputs on both sides; a
one-ulp fp32 difference upstream can move one of those roundings by an fp16 step (2^-11 relative),
so that case is compared at 1e-3. A wrong stage order, slope, dilation or a dropped branch moves
the output by O(0.1).

At the full 10 s shape (500 frames -> 320000 samples) the oracle is too slow; there the decoder is
compared bit for bit with the same launches issued one by one from Python (GeneratorStage), and the
recorded graph with the eager launches over several replays.
"""
import numpy as np
import pytest
import torch

import gsvk
import oracle as O
from gpu_util import F16, F32, dev, devf, host, say
from sovits_util import gpu_stage, make_stage, oracle_stage, round_f16

pytestmark = pytest.mark.gpu

UPS_U = (10, 8, 2, 2, 2)    # dec.hpp:55
UPS_K = (20, 16, 8, 2, 2)   # dec.hpp:56


def make_decoder(r, c_z, c0, g_in, n_stages=5):
    """Random weights of the reference's decoder geometry with c0 channels after conv_pre."""
    w = lambda co, ci, k: (r.standard_normal((co, ci, k)) / np.sqrt(ci * k)).astype(np.float16)
    m = {"pre": (w(c0, c_z, 7), (0.05 * r.standard_normal(c0)).astype(np.float32))}
    m["cond"] = (w(c0, g_in, 1), (0.05 * r.standard_normal(c0)).astype(np.float32)) if g_in else None
    stages, c = [], c0
    for s in range(n_stages):
        stages.append(make_stage(r, c, c // 2, UPS_K[s], UPS_U[s]))
        c //= 2
    m["stages"] = stages
    m["post"] = w(1, c, 7)
    return m


def oracle_decoder(m, z, ge, round_x=False):
    q = round_f16 if round_x else (lambda a: a)
    w_pre, b_pre = m["pre"]
    x = O.conv1d(F32, q(z), w_pre.view(np.uint16), b_pre, 1)
    if m["cond"] is not None:
        w_c, b_c = m["cond"]
        cv = O.conv1d(F32, q(ge[:, None]), w_c.view(np.uint16), b_c, 1)[:, 0]
        x = (x + cv[:, None]).astype(np.float32)
    x = O.leaky_relu(F32, x, 0.1)
    n = len(m["stages"])
    for s, (up, rbs) in enumerate(m["stages"]):
        x = oracle_stage(x, up, rbs, UPS_U[s], 0.1 if s + 1 < n else 0.01, round_x=round_x)
    return O.conv1d(F32, q(x), m["post"].view(np.uint16), None, 1, epi=gsvk.CONV_EPI_TANH)[0]


def oracle_decoder_f16(m, z, ge):
    """The oracle chain with fp16 storage at the GPU's rounding points: each launch rounds what it
    stores to fp16 once (its fused epilogue computed in fp32 first, as the oracle's fused conv
    epilogues do), cond and the folded bias stay fp32."""
    w_pre, b_pre = m["pre"]
    bias = b_pre
    if m["cond"] is not None:
        w_c, b_c = m["cond"]
        cv = O.conv1d(F32, ge[:, None], w_c.view(np.uint16), b_c, 1)[:, 0]
        bias = (b_pre + cv).astype(np.float32)
    x = O.conv1d(F16, O.to_storage(F16, z), w_pre.view(np.uint16), bias, 1,
                 epi=gsvk.CONV_EPI_LRELU, slope=0.1)
    n = len(m["stages"])
    for s, ((w_up, b_up), rbs) in enumerate(m["stages"]):
        y, t_in0 = O.convt1d(F16, x, w_up.view(np.uint16), UPS_U[s], b_up,
                             epi=gsvk.CONV_EPI_DUAL, slope=0.1)
        curs = []
        for w1, b1, w2, b2 in rbs:
            src, cur = t_in0, y
            for k in range(3):
                t_a = O.conv1d(F16, src, w1[k].view(np.uint16), b1[k], (1, 3, 5)[k],
                               epi=gsvk.CONV_EPI_LRELU, slope=0.1)
                epi = gsvk.CONV_EPI_RES if k == 2 else gsvk.CONV_EPI_RES_LRELU
                src, cur = O.conv1d(F16, t_a, w2[k].view(np.uint16), b2[k], 1, epi=epi,
                                    slope=0.1, cur=cur)
            curs.append(cur)
        x = O.resblock_branch_mean(F16, curs, None, True, 0.1 if s + 1 < n else 0.01)
    return O.conv1d(F16, x, m["post"].view(np.uint16), None, 1, epi=gsvk.CONV_EPI_TANH)[0]


class GpuDecoder:
    """Device objects of one decoder's weights (packed once)."""

    def __init__(self, m):
        w_pre, b_pre = m["pre"]
        self.pre = gsvk.Conv1d(dev(w_pre.view(np.uint16), F16), devf(b_pre))
        self.cond = None
        if m["cond"] is not None:  # cond is k = 1: its fp16 [c0, g_in] matrix, unpacked
            w_c, b_c = m["cond"]
            self.cond = (dev(w_c[:, :, 0].view(np.uint16), F16), devf(b_c))
        self.stages = [gpu_stage(up, rbs, UPS_U[s]) for s, (up, rbs) in enumerate(m["stages"])]
        self.post = gsvk.Conv1d(dev(m["post"].view(np.uint16), F16), None)

    def bind(self, z, ge, out, round_x=False, graph=True):
        return gsvk.SovitsDecoder(self.pre, self.cond, self.stages, self.post, z, ge, out,
                                  round_x=round_x, graph=graph)

    def python_chain(self, z, ge, out, round_x=False):
        """The same launches issued one by one from Python: cond as a GEMV with b_pre as its
        residual (the bias fold), conv_pre + lrelu, GeneratorStage.forward per stage, conv_post +
        tanh."""
        bias = self.pre.b
        if self.cond is not None:
            w_c, b_c = self.cond
            bias = torch.empty_like(self.pre.b)
            gsvk.gemv_f16w(ge.view(1, -1), w_c, bias.view(1, -1), bias=b_c,
                           residual=self.pre.b.view(1, -1), round_x=round_x)
        x = torch.empty(self.pre.out_c, z.shape[1], dtype=z.dtype, device=z.device)
        gsvk.conv1d(z, self.pre.wp, self.pre.out_c, self.pre.k, x, bias, 1, gsvk.CONV_EPI_LRELU,
                    0.1, round_x=round_x)
        n = len(self.stages)
        for s, st in enumerate(self.stages):
            nx = torch.empty(st.ups.out_c, x.shape[1] * st.ups.stride_u, dtype=x.dtype,
                             device=x.device)
            st.forward(x, nx, slope_next=0.1 if s + 1 < n else 0.01, round_x=round_x)
            x = nx
        gsvk.conv1d(x, self.post.wp, 1, self.post.k, out.view(1, -1), None, 1,
                    gsvk.CONV_EPI_TANH, 0.0, round_x=round_x)


@pytest.mark.parametrize("c_z,c0,g_in,frames,round_x", [
    (16, 64, 32, 12, False),     # narrowed channels (64 -> 2), 12 frames -> 7680 samples
    (192, 768, 1024, 3, False),  # the model's channels and cond (768 -> 24), 3 frames: all edges
    (16, 64, 0, 9, False),       # no conditioning (g_in 0): conv_pre's own bias
    (16, 64, 32, 12, True),      # fp16-rounded convolution inputs (the AMX numerics)
])
def test_decoder_matches_oracle_chain(c_z, c0, g_in, frames, round_x):
    r = np.random.default_rng(20250901 + c0 + frames + 7 * round_x)
    m = make_decoder(r, c_z, c0, g_in)
    z = r.standard_normal((c_z, frames)).astype(np.float32)
    ge = r.standard_normal(g_in).astype(np.float32) if g_in else None
    say(f"decoder c_z={c_z} c0={c0} g_in={g_in} frames={frames} round_x={round_x}: oracle")
    want = oracle_decoder(m, z, ge, round_x)
    g = GpuDecoder(m)
    zd = devf(z)
    ged = devf(ge) if g_in else None
    n_out = frames * int(np.prod(UPS_U))
    out = torch.full((n_out,), float("nan"), dtype=torch.float32, device="cuda")
    dec = g.bind(zd, ged, out, round_x=round_x)
    assert dec.launches == (1 if g_in else 0) + 1 + 5 * 20 + 1
    dec.run()
    torch.cuda.synchronize()
    got = host(out, F32)
    err = np.abs(got.astype(np.float64) - want.astype(np.float64))
    tol = 1e-3 if round_x else 1e-4
    say(f"  max |d| {err.max():.2e} (tol {tol:g}), peak |out| {np.abs(want).max():.3f}")
    assert np.isfinite(got).all()
    assert err.max() <= tol


def test_decoder_eager_on_a_caller_stream_equals_the_graph():
    """The eager form runs ResBlocks 1 and 2 of each stage on the library's own streams, forked
    after the work already on the caller's stream and joined back before the branch mean: issued
    on a non-default stream behind a fill of the output, three calls in a row give the graph's
    bits (a late fork would read a stale upsampler output, a missing join a partial branch)."""
    r = np.random.default_rng(20251202)
    m = make_decoder(r, 16, 64, 32)
    frames = 12
    z = r.standard_normal((16, frames)).astype(np.float32)
    ge = r.standard_normal(32).astype(np.float32)
    g = GpuDecoder(m)
    zd, ged = devf(z), devf(ge)
    n_out = frames * int(np.prod(UPS_U))
    out_g = torch.full((n_out,), float("nan"), dtype=torch.float32, device="cuda")
    out_e = torch.full((n_out,), float("nan"), dtype=torch.float32, device="cuda")
    say("decoder graph vs eager on a caller stream: graph")
    g.bind(zd, ged, out_g).run()
    torch.cuda.synchronize()
    ref = host(out_g, F32)
    assert np.isfinite(ref).all()
    eager = g.bind(zd, ged, out_e, graph=False)
    s = torch.cuda.Stream()
    with torch.cuda.stream(s):
        for i in range(3):
            say(f"  eager call {i} on a caller stream")
            out_e.fill_(float("nan"))
            eager.run(stream=s)
            got = out_e.clone()
            s.synchronize()
            assert np.array_equal(host(got, F32).view(np.uint32), ref.view(np.uint32)), f"call {i}"


def test_decoder_fp16_storage():
    """fp16 activations (every stored activation rounded to fp16, arithmetic in fp32; ge, cond and
    the folded bias in fp32) against the oracle chain with the same rounding points. The only
    difference left is the fp32 summation order inside each convolution, which can move an fp16
    rounding by one step (2^-11 relative) and carry it downstream: compared at |d| <= 4e-3 on the
    tanh output (8 fp16 steps at |out| ~ 1). Also reported: the distance to the fp32 chain."""
    r = np.random.default_rng(20250921)
    m = make_decoder(r, 16, 64, 32)
    frames = 12
    z = r.standard_normal((16, frames)).astype(np.float32)
    ge = r.standard_normal(32).astype(np.float32)
    say("decoder fp16: oracle chains")
    want = O.to_f32(F16, oracle_decoder_f16(m, z, ge)).astype(np.float64)
    want32 = oracle_decoder(m, z, ge).astype(np.float64)
    g = GpuDecoder(m)
    zd = dev(O.to_storage(F16, z), F16)
    out = torch.full((frames * 640,), float("nan"), dtype=torch.float16, device="cuda")
    dec = g.bind(zd, devf(ge), out)
    dec.run()
    torch.cuda.synchronize()
    got = O.to_f32(F16, host(out, F16)).astype(np.float64)
    err = np.abs(got - want).max()
    say(f"  max |d| vs fp16 chain {err:.2e}, vs fp32 chain {np.abs(got - want32).max():.2e}")
    assert np.isfinite(got).all()
    assert err <= 4e-3


def test_decoder_full_shape_graph_eager_and_python_chain_agree():
    """500 frames (10 s) at the model's channels: the recorded graph, the eager launches and the
    Python chain of the same launches give the same bits; replays interleaved with eager work on the
    same buffers keep giving them."""
    r = np.random.default_rng(20250911)
    m = make_decoder(r, 192, 768, 1024)
    frames = 500
    zd = devf(r.standard_normal((192, frames)).astype(np.float32))
    ged = devf(r.standard_normal(1024).astype(np.float32))
    g = GpuDecoder(m)
    n_out = frames * 640
    out_g = torch.empty(n_out, dtype=torch.float32, device="cuda")
    out_e = torch.empty_like(out_g)
    out_p = torch.empty_like(out_g)
    say("full decoder: eager")
    eager = g.bind(zd, ged, out_e, graph=False)
    eager.run()
    say("full decoder: python chain")
    g.python_chain(zd, ged, out_p)
    say("full decoder: graph replays")
    graph = g.bind(zd, ged, out_g)
    ref = None
    for i in range(3):
        out_g.fill_(float("nan"))
        graph.run()
        torch.cuda.synchronize()
        got = host(out_g, F32)
        if ref is None:
            ref = got
            e = host(out_e, F32)
            p = host(out_p, F32)
            assert np.isfinite(ref).all() and np.abs(ref).max() <= 1.0
            assert np.array_equal(e.view(np.uint32), p.view(np.uint32))
        assert np.array_equal(got.view(np.uint32), ref.view(np.uint32)), f"replay {i}"
        eager.run()  # eager work on the shared weights between replays
        torch.cuda.synchronize()
        assert np.array_equal(host(out_e, F32).view(np.uint32), ref.view(np.uint32))
    say(f"  full decoder ok, peak |out| {np.abs(ref).max():.3f}")
