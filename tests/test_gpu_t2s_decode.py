"""The whole T2S decode step on the GPU (gsvk_t2s_decode_*) against the oracle chained the same way:
embed_pe, then per layer GEMV (QKV, fp32) -> attention with KV append -> GEMV + bias + residual ->
LayerNorm -> GEMV + bias + ReLU -> GEMV + bias + residual -> LayerNorm, then the logits GEMV, with the
activations rounded to fp16 at the same points (t2s_engine.cpp:1035-1120, 1864-1885).

Each stage meets its own kernel's tolerance (its test file); chained, a stage's fp32-noise difference
can move a later fp16 rounding by one step, so the chain is compared with a few fp16 steps of slack:
|x_gpu - x_oracle| <= 4 steps(x) + 4e-3, logits within 1e-2 * max(1, |logit|), the appended cache
rows of the first layer within one fp16 step (later layers: the chain slack). Graph and eager runs
must agree bit for bit.
"""
import numpy as np
import pytest
import torch

import gsvk
import oracle as O
from gpu_util import F16, F32, dev, devf, host, say

pytestmark = pytest.mark.gpu


def rng(k):
    return np.random.default_rng(20250823 + 13000 + k)


def build(B=5, D=128, H=4, FF=256, L=2, V=50, max_len=64, seed=0):
    r = rng(seed)
    w = lambda n, k, s=0.05: (s * r.standard_normal((n, k))).astype(np.float16).view(np.uint16)
    vec = lambda n, s=0.02, m=0.0: (m + s * r.standard_normal(n)).astype(np.float32)
    layers = []
    for _ in range(L):
        layers.append(dict(
            wqkv=w(3 * D, D), bqkv=vec(3 * D), wout=w(D, D), bout=vec(D),
            n1g=vec(D, 0.1, 1.0), n1b=vec(D, 0.1), w1=w(FF, D), b1=vec(FF), w2=w(D, FF),
            b2=vec(D), n2g=vec(D, 0.1, 1.0), n2b=vec(D, 0.1),
            k_cache=O.to_storage(F16, r.standard_normal((B, max_len, D)).astype(np.float32)),
            v_cache=O.to_storage(F16, r.standard_normal((B, max_len, D)).astype(np.float32))))
    m = dict(table=(0.02 * r.standard_normal((V, D))).astype(np.float16).view(np.uint16),
             pe=gsvk.pe_table(256, D), alpha=np.float32(0.93), heads=H, layers=layers,
             w_logits=w(V, D))
    io = dict(ids=r.integers(0, V, B).astype(np.int64),
              pos=r.integers(0, 200, B).astype(np.int64),
              kv_pos=r.integers(0, max_len, B).astype(np.int64))
    return m, io


def oracle_step(m, io, eps=1e-5):
    """The chain on host arrays; the caches in m are updated in place."""
    H = m["heads"]
    x, bad = O.embed_pe(F16, F16, m["table"], io["ids"], m["pe"], float(m["alpha"]),
                        pos=io["pos"])
    assert bad == 0
    D = x.shape[1]
    for ly in m["layers"]:
        qkv = O.gemv_f16w(F16, x, ly["wqkv"], F32, bias=ly["bqkv"])
        a32 = O.decode_attention(F16, qkv, ly["k_cache"], ly["v_cache"], io["kv_pos"], H, D // H)
        attn = O.to_storage(F16, a32)
        z = O.gemv_f16w(F16, attn, ly["wout"], F16, bias=ly["bout"], residual=x)
        h = O.add_layernorm(F16, z, ly["n1g"], ly["n1b"], eps)
        ff = O.gemv_f16w(F16, h, ly["w1"], F16, bias=ly["b1"], act=1)
        z = O.gemv_f16w(F16, ff, ly["w2"], F16, bias=ly["b2"], residual=h)
        x = O.add_layernorm(F16, z, ly["n2g"], ly["n2b"], eps)
    logits = O.gemv_f16w(F16, x, m["w_logits"], F32)
    return x, logits


def to_device(m, io, FF):
    B = io["ids"].size
    D = m["table"].shape[1]
    md = dict(table=dev(m["table"], F16), pe=devf(m["pe"]), alpha=float(m["alpha"]),
              heads=m["heads"], w_logits=dev(m["w_logits"], F16), layers=[])
    for ly in m["layers"]:
        d = {}
        for k, v in ly.items():
            d[k] = dev(v, F16) if v.dtype == np.uint16 else devf(v)
        md["layers"].append(d)
    V = m["table"].shape[0]
    iod = dict(ids=torch.from_numpy(io["ids"]).cuda(), pos=torch.from_numpy(io["pos"]).cuda(),
               kv_pos=torch.from_numpy(io["kv_pos"]).cuda(),
               err=torch.zeros(1, dtype=torch.int32, device="cuda"),
               x=torch.empty(B, D, dtype=torch.float16, device="cuda"),
               h=torch.empty(B, D, dtype=torch.float16, device="cuda"),
               z=torch.empty(B, D, dtype=torch.float16, device="cuda"),
               attn=torch.empty(B, D, dtype=torch.float16, device="cuda"),
               ff=torch.empty(B, FF, dtype=torch.float16, device="cuda"),
               qkv=torch.empty(B, 3 * D, dtype=torch.float32, device="cuda"),
               logits=torch.empty(B, V, dtype=torch.float32, device="cuda"))
    return md, iod


def compare(x_gpu, lg_gpu, x_want, lg_want, what):
    xg = O.to_f32(F16, x_gpu).astype(np.float64)
    xw = O.to_f32(F16, x_want).astype(np.float64)
    step = np.spacing(np.abs(xw).astype(np.float16)).astype(np.float64)
    dx = np.abs(xg - xw)
    say(f"{what}: max |dx| {dx.max():.3e}, fp16 steps {np.max(dx / step):.1f}, "
        f"max |dlogit| {np.max(np.abs(lg_gpu - lg_want)):.3e}")
    assert np.all(dx <= 4 * step + 4e-3), what
    assert np.all(np.abs(lg_gpu - lg_want) <= 1e-2 * np.maximum(1.0, np.abs(lg_want))), what


@pytest.mark.parametrize("graph", [False, True])
@pytest.mark.parametrize("len_bound", [0, 40])
def test_decode_step_matches_oracle_chain(graph, len_bound):
    FF = 256
    m, io = build(seed=1)
    md, iod = to_device(m, io, FF)
    x_want, lg_want = oracle_step(m, io)
    step = gsvk.T2SDecode(md, iod, len_bound=len_bound, graph=graph)
    # gather, 2 layers x (QKV, attention (+ merge), out-proj, W1 with norm1, W2), logits with
    # the last norm2 (each norm2 / norm1 runs inside the GEMV after it)
    assert not graph or step.launches in (1 + 5 * 2 + 1, 1 + 6 * 2 + 1)
    step.run()
    torch.cuda.synchronize()
    assert int(iod["err"].item()) == 0
    compare(host(iod["x"], F16), host(iod["logits"], F32), x_want, lg_want, f"graph={graph}")
    # appended cache rows: layer 0 (same input as the oracle) within one fp16 step, later layers
    # (inputs already carrying the chain's differences) within the chain slack; other rows equal
    for li, (ly_d, ly_h) in enumerate(zip(md["layers"], m["layers"])):
        for name in ("k_cache", "v_cache"):
            g = O.to_f32(F16, host(ly_d[name], F16)).astype(np.float64)
            w = O.to_f32(F16, ly_h[name]).astype(np.float64)
            st = np.spacing(np.abs(w).astype(np.float16)).astype(np.float64)
            slack = st if li == 0 else 4 * st + 4e-3
            assert np.all(np.abs(g - w) <= slack), (li, name)


def test_decode_step_graph_equals_eager_over_steps():
    """Three steps, the inputs advanced on the device between them; graph replays and eager runs
    give the same bits."""
    FF = 256
    outs = []
    for graph in (False, True):
        m, io = build(seed=2)
        md, iod = to_device(m, io, FF)
        step = gsvk.T2SDecode(md, iod, len_bound=64, graph=graph)
        xs = []
        for t in range(3):
            step.run()
            torch.cuda.synchronize()
            xs.append((host(iod["x"], F16), host(iod["logits"], F32)))
            iod["ids"].copy_(torch.argmax(iod["logits"], 1))
            iod["pos"].add_(1)
            iod["kv_pos"].add_(1).clamp_(max=63)
        outs.append(xs)
    for (xa, la), (xb, lb) in zip(*outs):
        assert np.array_equal(xa, xb) and np.array_equal(la.view(np.uint32), lb.view(np.uint32))


def test_decode_step_t2s_shape_four_layers():
    """B = 64, D = 512, 16 heads, FF = 2048, four chained layers, 1025-token vocabulary, every
    sequence at 960-1023 cached keys: the real shapes, with the residual path carrying each layer's
    differences into the next."""
    FF = 2048
    m, io = build(B=64, D=512, H=16, FF=FF, L=4, V=1025, max_len=1024, seed=3)
    io["kv_pos"][:] = np.random.default_rng(96).integers(960, 1024, 64)
    md, iod = to_device(m, io, FF)
    x_want, lg_want = oracle_step(m, io)
    step = gsvk.T2SDecode(md, iod, len_bound=1024)
    step.run()
    torch.cuda.synchronize()
    compare(host(iod["x"], F16), host(iod["logits"], F32), x_want, lg_want, "T2S shape")


def test_decode_step_two_halves_equal_one_chain():
    """A batch of 32 or more runs as two halves on two graph branches when the workspace holds both
    halves' attention states. 37 sequences (halves of 18 and 19) with 200 cached keys: the
    attention's key chunks depend only on the length there, so the halves give exactly the bits of
    the one-chain step (split=False), graph and eager, and both match the oracle chain."""
    FF = 256
    m, io = build(B=37, D=128, H=4, FF=FF, L=2, V=50, max_len=256, seed=4)
    io["kv_pos"][:] = np.random.default_rng(99).integers(150, 200, 37)
    x_want, lg_want = oracle_step({**m, "layers": [dict(ly, k_cache=ly["k_cache"].copy(),
                                                        v_cache=ly["v_cache"].copy())
                                                   for ly in m["layers"]]}, io)
    outs = {}
    for split, graph in ((False, True), (True, True), (True, False)):
        md, iod = to_device(m, io, FF)
        step = gsvk.T2SDecode(md, iod, len_bound=200, graph=graph, split=split)
        if graph:
            # gather, 2 layers x (QKV, attention, merge, out-proj, W1, W2), logits: per chain
            assert step.launches == (2 if split else 1) * (1 + 6 * 2 + 1), step.launches
        step.run()
        torch.cuda.synchronize()
        assert int(iod["err"].item()) == 0
        outs[(split, graph)] = (host(iod["x"], F16), host(iod["logits"], F32),
                                [host(ly["k_cache"], F16) for ly in md["layers"]])
        step.close()
    ref = outs[(False, True)]
    compare(ref[0], ref[1], x_want, lg_want, "one chain")
    for key in ((True, True), (True, False)):
        x, lg, kc = outs[key]
        assert np.array_equal(x, ref[0]), key
        assert np.array_equal(lg.view(np.uint32), ref[1].view(np.uint32)), key
        for a, b in zip(kc, ref[2]):
            assert np.array_equal(a, b), key


def test_decode_step_t2s_shape_halves_match_oracle():
    """B = 64 at the real shapes with 1000 cached keys: the two halves (each attention call splits
    its keys into more chunks than the whole batch's would) against the oracle chain, and their
    graph replay against their eager run, bit for bit."""
    FF = 2048
    m, io = build(B=64, D=512, H=16, FF=FF, L=2, V=1025, max_len=1024, seed=5)
    io["kv_pos"][:] = np.random.default_rng(98).integers(900, 1000, 64)
    x_want, lg_want = oracle_step({**m, "layers": [dict(ly, k_cache=ly["k_cache"].copy(),
                                                        v_cache=ly["v_cache"].copy())
                                                   for ly in m["layers"]]}, io)
    got = []
    for graph in (True, False):
        md, iod = to_device(m, io, FF)
        step = gsvk.T2SDecode(md, iod, len_bound=1000, graph=graph)
        if graph:
            assert step.launches == 2 * (1 + 6 * 2 + 1), step.launches
        step.run()
        torch.cuda.synchronize()
        got.append((host(iod["x"], F16), host(iod["logits"], F32)))
        step.close()
    compare(got[0][0], got[0][1], x_want, lg_want, "halves, T2S shape")
    assert np.array_equal(got[0][0], got[1][0])
    assert np.array_equal(got[0][1].view(np.uint32), got[1][1].view(np.uint32))


def test_decode_step_two_halves_without_positions():
    """With no PE position array every row r takes position r; the second half's rows then start at
    position B / 2. Halves and one chain, graph and eager, give the same bits."""
    FF = 256
    m, io = build(B=40, D=128, H=4, FF=FF, L=1, V=50, max_len=256, seed=6)
    io["kv_pos"][:] = np.random.default_rng(97).integers(100, 200, 40)
    outs = []
    for split, graph in ((False, True), (True, True), (True, False)):
        md, iod = to_device(m, io, FF)
        iod["pos"] = None
        step = gsvk.T2SDecode(md, iod, len_bound=200, graph=graph, split=split)
        step.run()
        torch.cuda.synchronize()
        assert int(iod["err"].item()) == 0
        outs.append((host(iod["x"], F16), host(iod["logits"], F32)))
        step.close()
    for x, lg in outs[1:]:
        assert np.array_equal(x, outs[0][0])
        assert np.array_equal(lg.view(np.uint32), outs[0][1].view(np.uint32))
    # and the one chain against the oracle with positions 0..B-1
    x_want, lg_want = oracle_step({**m, "layers": [dict(ly, k_cache=ly["k_cache"].copy(),
                                                        v_cache=ly["v_cache"].copy())
                                                   for ly in m["layers"]]},
                                  dict(io, pos=np.arange(40, dtype=np.int64)))
    compare(outs[0][0], outs[0][1], x_want, lg_want, "no position array")
