"""The T2S decode-step epilogue chain (include/gsvk_t2s.h) on the GPU.

1. Graph replay == eager launches, bitwise, on every one of several replays with eager work and
   host synchronisations between them (the captured graph holds kernel nodes only).
2. The chain against the oracle's chain on the same inputs, for the 73-launch form and the one-launch
   form (gsvk_t2s_step_fused). Each op is held to its own tolerance in test_gpu_parity; here the
   layers compound, so the bound is the per-op bound times the layer count: fp32
   |d| <= layers * (1e-6 + 1e-5 |w|); 16-bit storage |d| <= 4 storage steps of w, or of 2 where
   w is smaller (8e-3 in fp16, 6.25e-2 in bf16), because a single one-step rounding flip in an
   early layer is carried forward by the residual path. gather + ReLU outputs that do not depend on the chain (ff) must be bit-exact.
3. The one-launch form at the config shape and at odd ones (5 rows, D 1024 = two chunks per lane,
   FF not a multiple of the 64-chunk column tile, one layer, the 32-layer limit, int32 ids, fp32 /
   bf16 tables), in f32 / f16 / bf16 storage: against the oracle chain as in 2, graph replays equal
   to its eager launch bit for bit, and out-of-range ids give NaN rows and the error flag as the
   per-op launches do. Its LayerNorm statistics are one-pass (kern::layernorm's algorithm, the
   oracle's), the per-op kernel's two-pass, so the two forms agree within the chain bound, not
   bit for bit.
4. Constant rows: the one-pass variance is the rounding error of c^2, negative for some c, which
   sends the row through the centred second pass; every such row comes out as beta exactly.
"""
import ctypes

import numpy as np
import pytest
import torch

import gsvk
import oracle as O
from gpu_util import BF16, F16, F32, dev, devf, host, say

pytestmark = pytest.mark.gpu


def host_bufs(dt, B, D, FF, L, seed, tab_dt=F16, ids32=False):
    r = np.random.default_rng(seed)
    st = lambda a: O.to_storage(dt, np.asarray(a, np.float32))
    hb = {
        "table": O.to_storage(tab_dt, (0.02 * r.standard_normal((1025, D))).astype(np.float32)),
        "table_dtype": tab_dt,
        "ids": r.integers(0, 1025, B).astype(np.int32 if ids32 else np.int64),
        "pos": r.integers(512, 2048, B).astype(np.int64),
        "pe": gsvk.pe_table(2048, D),
        "alpha": float(np.float32(r.uniform(0.5, 1.5))),
        "x": st(np.zeros((B, D))), "h": st(np.zeros((B, D))),
    }
    for name, shape in (("attn_out", (B, D)), ("ff", (B, FF)), ("ffn_out", (B, D))):
        hb[name] = [st(r.standard_normal(shape)) for _ in range(L)]
    for name, n in (("bout", D), ("b1", FF), ("b2", D), ("n1b", D), ("n2b", D)):
        hb[name] = [(0.05 * r.standard_normal(n)).astype(np.float32) for _ in range(L)]
    for name in ("n1g", "n2g"):
        hb[name] = [(1 + 0.1 * r.standard_normal(D)).astype(np.float32) for _ in range(L)]
    return hb


def to_dev(hb, dt):
    db = {}
    for k, v in hb.items():
        if k == "table":
            db[k] = dev(v, hb["table_dtype"])
        elif k in ("ids", "pos"):
            db[k] = torch.from_numpy(v).cuda()
        elif k == "pe":
            db[k] = devf(v)
        elif k in ("x", "h"):
            db[k] = dev(v, dt)
        elif k in ("attn_out", "ff", "ffn_out"):
            db[k] = [dev(a, dt) for a in v]
        elif isinstance(v, list):
            db[k] = [devf(a) for a in v]
        else:
            db[k] = v
    db["err"] = torch.zeros(1, dtype=torch.int32, device="cuda")
    return db


def snapshot(db, dt):
    return {"x": host(db["x"], dt), "h": host(db["h"], dt), "ff": [host(t, dt) for t in db["ff"]]}


def reset_ff(db, hb, dt):
    for t, a in zip(db["ff"], hb["ff"]):
        t.copy_(dev(a, dt))


@pytest.mark.parametrize("dt", [F32, F16])
def test_t2s_step_graph_equals_eager_every_replay(dt):
    say(f"t2s step graph vs eager dt={dt}")
    hb = host_bufs(dt, 64, 512, 2048, 24, 3000 + dt)
    db = to_dev(hb, dt)
    eager = gsvk.T2SStep(db, graph=False)
    eager.run()
    torch.cuda.synchronize()
    want = snapshot(db, dt)
    step = gsvk.T2SStep(db, graph=True)
    assert step.launches == 73
    for rep in range(4):
        reset_ff(db, hb, dt)
        db["x"].zero_()
        db["h"].fill_(1)
        junk = torch.randn(1 << 20, device="cuda") * 3  # unrelated eager work between replays
        torch.cuda.synchronize()
        step.run()
        torch.cuda.synchronize()
        got = snapshot(db, dt)
        assert np.array_equal(got["x"], want["x"]), f"replay {rep}: x"
        assert np.array_equal(got["h"], want["h"]), f"replay {rep}: h"
        for a, b in zip(got["ff"], want["ff"]):
            assert np.array_equal(a, b), f"replay {rep}: ff"
        del junk
    assert int(db["err"].item()) == 0
    step.close()


def chain_bound(dt, w, layers):
    """fp32: the per-op bound times the layer count. 16-bit storage: 4 storage steps of w, and at
    least 4 steps at |w| = 2 (8e-3 in fp16, 6.25e-2 in bf16): a rounding flip of a typical
    activation in an early layer is carried forward to every later layer's value of that element,
    whatever its size there."""
    w = np.abs(w.astype(np.float64))
    if dt == F32:
        return layers * (1e-6 + 1e-5 * w)
    floor = 8e-3 if dt == F16 else 4 * 2.0 ** -6
    return np.maximum(floor, 4 * tol_step(dt, w))


def tol_step(dt, w):
    """One storage step of |w| in fp16 / bf16."""
    if dt == F16:
        return np.spacing(np.minimum(w, 65504).astype(np.float16)).astype(np.float64)
    e = np.floor(np.log2(np.maximum(w, 2.0 ** -126)))
    return 2.0 ** (e - 7)


def check_chain(dt, got, hb, layers, what):
    """x / h against the oracle chain (in place on hb), ff bit-exact; returns the worst error in
    units of its bound."""
    for a, b in zip(got["ff"], hb["ff"]):
        assert np.array_equal(a, b), f"{what}: bias+ReLU outputs differ"
    worst = 0.0
    for name in ("x", "h"):
        g = O.to_f32(dt, got[name]).astype(np.float64)
        w = O.to_f32(dt, hb[name]).astype(np.float64)
        err = np.abs(g - w)
        bound = chain_bound(dt, w, layers)
        assert (err <= bound).all(), f"{what} {name}: worst {err.max():.3e}"
        worst = max(worst, float((err / bound).max()))
    return worst


def oracle_chain(dt, hb):
    o = dict(hb)
    o["ids"] = hb["ids"].astype(np.int64)
    o["x"], o["h"] = hb["x"].copy(), hb["h"].copy()
    o["ff"] = [a.copy() for a in hb["ff"]]
    O.t2s_step(dt, o, threads=4)
    return o


@pytest.mark.parametrize("fused", [False, True])
@pytest.mark.parametrize("dt", [F32, F16])
def test_t2s_step_matches_oracle_chain(dt, fused):
    say(f"t2s step vs oracle dt={dt} fused={fused}")
    B, D, FF, L = 64, 512, 2048, 24
    hb = host_bufs(dt, B, D, FF, L, 4000 + dt)
    db = to_dev(hb, dt)
    step = gsvk.T2SStep(db, graph=True, fused=fused)
    step.run()
    torch.cuda.synchronize()
    got = snapshot(db, dt)
    worst = check_chain(dt, got, oracle_chain(dt, hb), L, f"fused={fused}")
    say(f"  worst error / bound: {worst:.3f}")
    step.close()


FUSED_CASES = [
    # (dt, B, D, FF, L, table dtype, int32 ids)
    (F16, 64, 512, 2048, 24, F16, False),   # configuration 2
    (F32, 64, 512, 2048, 24, F16, False),
    (BF16, 64, 512, 2048, 24, F16, False),
    (F16, 5, 1024, 1000, 3, F32, True),     # two chunks per lane, partial ReLU column tile
    (F32, 3, 256, 64, 1, BF16, False),
    (BF16, 7, 1024, 2056, 2, F16, True),
    (F16, 1, 8, 8, 32, F16, False),         # the layer limit, one lane of one chunk
    # two chunks per lane with the second partly active (64 < D / VEC < 128): guarded stores and
    # zeroed tail chunks
    (F16, 5, 800, 1000, 4, F16, False),
    (F32, 6, 400, 520, 3, F32, True),
]


@pytest.mark.parametrize("case", FUSED_CASES, ids=lambda c: "-".join(map(str, c)))
def test_fused_step_matches_oracle_chain(case):
    dt, B, D, FF, L, tdt, i32 = case
    say(f"fused step vs oracle chain {case}")
    hb = host_bufs(dt, B, D, FF, L, 5000 + B + D + L, tab_dt=tdt, ids32=i32)
    db = to_dev(hb, dt)
    want = oracle_chain(dt, hb)
    first = None
    for graph in (False, True):
        step = gsvk.T2SStep(db, graph=graph, fused=True)
        assert step.launches == 1
        for rep in range(3 if graph else 1):
            reset_ff(db, hb, dt)
            db["x"].zero_()
            db["h"].fill_(1)
            junk = torch.randn(1 << 18, device="cuda") * 3
            torch.cuda.synchronize()
            step.run()
            torch.cuda.synchronize()
            got = snapshot(db, dt)
            if first is None:
                first = got
                worst = check_chain(dt, got, want, L, f"graph={graph} rep {rep}")
                say(f"  worst error / bound: {worst:.3f}")
            else:  # every replay the same bits as the eager launch
                for name in ("x", "h"):
                    assert np.array_equal(got[name], first[name]), f"graph={graph} rep {rep}: {name}"
                for li, (a, b) in enumerate(zip(got["ff"], first["ff"])):
                    assert np.array_equal(a, b), f"graph={graph} rep {rep}: ff[{li}]"
            del junk
        step.close()
    assert int(db["err"].item()) == 0


def test_fused_step_out_of_range_ids_match_per_op_launches():
    say("fused step with out-of-range ids / positions")
    dt, B, L = F16, 16, 4
    hb = host_bufs(dt, B, 512, 2048, L, 6100)
    hb["ids"][3] = 1025
    hb["ids"][9] = -1
    hb["pos"][12] = 2048
    db = to_dev(hb, dt)
    gsvk.T2SStep(db, graph=False).run()
    torch.cuda.synchronize()
    want = snapshot(db, dt)
    assert int(db["err"].item()) == 1
    db["err"].zero_()
    reset_ff(db, hb, dt)
    step = gsvk.T2SStep(db, graph=False, fused=True)
    step.run()
    torch.cuda.synchronize()
    got = snapshot(db, dt)
    assert int(db["err"].item()) == 1
    for a, b in zip(got["ff"], want["ff"]):
        assert np.array_equal(a, b)
    for name in ("x", "h"):
        gf, wf = O.to_f32(dt, got[name]), O.to_f32(dt, want[name])
        assert np.array_equal(np.isnan(gf), np.isnan(wf)), name
        assert np.isnan(gf[[3, 9, 12]]).all() and not np.isnan(np.delete(gf, [3, 9, 12], 0)).any()
        ok = ~np.isnan(wf)
        err = np.abs(gf[ok].astype(np.float64) - wf[ok])
        assert (err <= chain_bound(dt, wf[ok], L)).all(), f"{name}: worst {err.max():.3e}"


@pytest.mark.parametrize("dt", [F32, F16])
def test_fused_step_constant_rows(dt):
    """Rows whose LayerNorm input is one constant c: the true variance is 0 and the one-pass
    E[x^2] - mean^2 is the rounding error of c^2 (the balanced sums of equal values are exact), so
    for the fp32 values of c below whose square rounds down it is negative and the row takes the
    centred second pass (kern.cpp:49-56). Every such row must come out as beta exactly: x - mean
    is 0 in either pass. The other rows are checked against the oracle chain."""
    say(f"fused step, constant rows dt={dt}")
    B, D, FF, L = 16, 512, 64, 1
    hb = host_bufs(dt, B, D, FF, L, 6200 + dt)
    hb["alpha"] = 0.0                    # x0 = table row
    hb["table"][hb["ids"][:8]] = 0       # ... = 0 for the constant rows
    hb["bout"][0][:] = 0.0               # so LN1's input is attn_out itself
    consts = np.array([300.0, -1000.1, 1.1, 0.0, 7.3, 12345.678, -0.3, 1e-3], np.float32)
    if dt == F32:
        c64 = consts.astype(np.float64)
        rounds_down = (consts * consts).astype(np.float64) < c64 * c64
        assert rounds_down.sum() >= 2, "some rows must take the second pass"
    att = O.to_f32(dt, hb["attn_out"][0]).copy()
    att[:8] = consts[:, None]
    hb["attn_out"][0] = O.to_storage(dt, att.astype(np.float32))
    db = to_dev(hb, dt)
    step = gsvk.T2SStep(db, graph=False, fused=True)
    step.run()
    torch.cuda.synchronize()
    got = snapshot(db, dt)
    gh = O.to_f32(dt, got["h"])
    assert np.isfinite(gh).all()
    beta = O.to_f32(dt, O.to_storage(dt, hb["n1b"][0]))
    for r in range(8):
        assert np.array_equal(gh[r], beta), f"constant row {r} (c = {consts[r]})"
    want = oracle_chain(dt, hb)
    g = gh[8:].astype(np.float64)
    w = O.to_f32(dt, want["h"])[8:].astype(np.float64)
    assert (np.abs(g - w) <= chain_bound(dt, w, L)).all()


def test_fused_step_revalidates_a_changed_descriptor():
    """The launch keeps the arguments of the last descriptor it validated and reuses them only for
    an identical one: after a good call, the same descriptor with one pointer or one size changed
    is validated again (here rejected), and the good one runs again with the results of its first
    run."""
    say("fused step: descriptor changes after a validated call")
    dt, B, D, FF, L = F16, 8, 512, 256, 3
    hb = host_bufs(dt, B, D, FF, L, 6300)
    db = to_dev(hb, dt)
    step = gsvk.T2SStep(db, graph=False, fused=True)
    lib, d = gsvk.lib(), step.desc
    run = lambda: lib.gsvk_t2s_step_fused(ctypes.byref(d), None)
    assert run() == gsvk.OK
    torch.cuda.synchronize()
    first = snapshot(db, dt)
    h = d.h
    d.h = d.x + 64                                   # h over x
    assert run() == gsvk.E_ALIAS
    d.h = h
    arr = step._arrays["ff"]
    ff2 = arr[2]
    arr[2] = step._arrays["attn_out"][1]             # a layer's FFN buffer over another's input
    assert run() == gsvk.E_ALIAS
    arr[2] = ff2
    d.d_model = 516                                  # a size: rows of partial chunks
    assert run() == gsvk.E_ARG
    d.d_model = D
    reset_ff(db, hb, dt)
    assert run() == gsvk.OK
    torch.cuda.synchronize()
    again = snapshot(db, dt)
    for name in ("x", "h"):
        assert np.array_equal(again[name], first[name]), name
    for a, b in zip(again["ff"], first["ff"]):
        assert np.array_equal(a, b)
