"""The T2S decode-step epilogue chain (include/gsvk_t2s.h) on the GPU.

1. Graph replay == eager launches, bitwise, on every one of several replays with eager work and
   host synchronisations between them (the captured graph holds kernel nodes only).
2. The chain against the oracle's chain on the same inputs. Each op is held to its own tolerance in
   test_gpu_parity; here 24 layers compound, so the bound is the per-op bound times the layer
   count: fp32 |d| <= 24 * (1e-6 + 1e-5 |w|); fp16 |d| <= 4 fp16 steps of w (or 8e-3), because a
   single one-step rounding flip in an early layer is carried forward by the residual path.
   gather + ReLU outputs that do not depend on the chain (ff) must be bit-exact.
3. The one-launch form (gsvk_t2s_step_fused) against the per-op launches, bitwise: the same
   operations in the same order with the same lane partition, at the config shape and at odd ones
   (5 rows, D 1024 = two chunks per lane, FF not a multiple of the 64-chunk column tile, one
   layer, the 32-layer limit, int32 ids, fp32 / bf16 tables), in f32 / f16 / bf16 storage, graph
   replays included; out-of-range ids give the same NaN rows and error flag.
"""
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
    O.t2s_step(dt, hb, threads=4)
    for a, b in zip(got["ff"], hb["ff"]):
        assert np.array_equal(a, b), "bias+ReLU outputs differ"
    for name in ("x", "h"):
        g = O.to_f32(dt, got[name]).astype(np.float64)
        w = O.to_f32(dt, hb[name]).astype(np.float64)
        if dt == F32:
            bound = L * (1e-6 + 1e-5 * np.abs(w))
        else:
            bound = np.maximum(8e-3, 4 * np.spacing(np.abs(w).astype(np.float16)).astype(np.float64))
        err = np.abs(g - w)
        assert (err <= bound).all(), f"{name}: worst {err.max():.3e}"
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
]


@pytest.mark.parametrize("case", FUSED_CASES, ids=lambda c: "-".join(map(str, c)))
def test_fused_step_equals_per_op_launches(case):
    dt, B, D, FF, L, tdt, i32 = case
    say(f"fused step vs per-op launches {case}")
    hb = host_bufs(dt, B, D, FF, L, 5000 + B + D + L, tab_dt=tdt, ids32=i32)
    db = to_dev(hb, dt)
    eager = gsvk.T2SStep(db, graph=False)
    eager.run()
    torch.cuda.synchronize()
    want = snapshot(db, dt)
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
            assert np.array_equal(got["x"], want["x"]), f"graph={graph} rep {rep}: x"
            assert np.array_equal(got["h"], want["h"]), f"graph={graph} rep {rep}: h"
            for li, (a, b) in enumerate(zip(got["ff"], want["ff"])):
                assert np.array_equal(a, b), f"graph={graph} rep {rep}: ff[{li}]"
            del junk
        step.close()
    assert int(db["err"].item()) == 0


def test_fused_step_out_of_range_ids_match_per_op_launches():
    say("fused step with out-of-range ids / positions")
    dt, B = F16, 16
    hb = host_bufs(dt, B, 512, 2048, 4, 6100)
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
    for name in ("x", "h"):
        gf, wf = O.to_f32(dt, got[name]), O.to_f32(dt, want[name])
        assert np.array_equal(np.isnan(gf), np.isnan(wf)), name
        assert np.isnan(gf[[3, 9, 12]]).all() and not np.isnan(np.delete(gf, [3, 9, 12], 0)).any()
        ok = ~np.isnan(wf)
        assert np.array_equal(gf[ok], wf[ok]), name
