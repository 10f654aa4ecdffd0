"""GPU parity at the sizes the benchmark runs, on the code paths that only large calls take:
  - LayerNorm with >= 8192 rows (two rows per wave, four-wave workgroups);
  - every kernel with >= 256 MiB moved per call (non-temporal loads and stores);
  - bias + activation with more row groups than one launch holds (host-side split);
  - the gather with >= 8192 rows (four-wave workgroups) and >= 256 MiB of output.
Each is compared with the oracle on the whole tensor (bit-exact where the op is, otherwise at the
stated tolerance, tests/gpu_util.py). Inputs are seeded; the oracle is the C restatement."""
import numpy as np
import pytest
import torch

import gsvk
import oracle as O
from gpu_util import BF16, F16, F32, assert_bitexact, assert_close, dev, devf, host, say

pytestmark = pytest.mark.gpu

MiB = 1 << 20


def rng(k):
    return np.random.default_rng(20250823 + 7000 + k)


def st(dt, a):
    return O.to_storage(dt, np.asarray(a, dtype=np.float32))


def randn(r, shape, scale=1.0):
    return (r.standard_normal(shape, dtype=np.float32) * np.float32(scale)).astype(np.float32)


def sync():
    torch.cuda.synchronize()


@pytest.mark.parametrize("rows,n,dt,use_bias", [
    (8195, 512, F16, True),      # 1 chunk per lane, 2 rows per wave
    (8195, 768, F16, True),      # 2 chunks per lane, partial
    (8195, 1024, BF16, False),
    (8195, 1024, F32, True),     # 4 chunks per lane
    (8195, 2048, F32, True),     # 8 chunks per lane
    (90001, 512, F16, True),     # > 256 MiB moved: non-temporal path
])
def test_layernorm_many_rows(rows, n, dt, use_bias):
    say(f"large LN rows={rows} n={n} dt={dt}")
    r = rng(rows + n)
    x = st(dt, randn(r, (rows, n)))
    res = st(dt, randn(r, (rows, n)))
    bias = randn(r, n, 0.02) if use_bias else None
    g = (1 + randn(r, n, 0.1)).astype(np.float32)
    b = randn(r, n, 0.1)
    want = O.add_layernorm(dt, x, g, b, 1e-5, bias=bias, residual=res)
    X = dev(x, dt)
    Y = torch.empty_like(X)
    gsvk.add_layernorm(X, devf(g), devf(b), Y, 1e-5, bias=devf(bias) if use_bias else None,
                       residual=dev(res, dt))
    sync()
    assert_close(dt, host(Y, dt), want, f"LN {rows}x{n}")


@pytest.mark.parametrize("rows,n,dt,act", [
    (70001, 2048, F16, gsvk.ACT_RELU),     # 573 MB, non-temporal, 4 rows per thread
    (140001, 1024, F32, gsvk.ACT_RELU),    # 1.1 GB, 2 rows per thread, 2 launches (row groups)
    (140001, 512, F32, gsvk.ACT_LEAKY_RELU),  # 64-chunk rows: 4 slices per workgroup
    (33001, 4096, F16, gsvk.ACT_GELU_ERF),  # 540 MB GELU, tolerance
])
def test_bias_act_streaming(rows, n, dt, act):
    say(f"large bias_act rows={rows} n={n} dt={dt} act={act}")
    r = rng(rows + act)
    x = st(dt, randn(r, (rows, n)))
    bias = randn(r, n, 0.02)
    assert 2 * x.nbytes >= 256 * MiB
    want = O.bias_act(dt, act, x, bias, 0.1)
    X = dev(x, dt)
    del x
    gsvk.bias_act(act, X, X, bias=devf(bias), slope=0.1)
    sync()
    got = host(X, dt)
    del X
    if act == gsvk.ACT_GELU_ERF:
        assert_close(dt, got, want, "large bias+gelu")
    else:
        assert_bitexact(dt, got, want, "large bias+act")


def test_bias_act_row_groups_split_over_launches():
    """f16 rows of 64 (8 chunks): cached path, 4 rows per workgroup, 65535 row groups per launch,
    so 300000 rows take two launches."""
    r = rng(5)
    rows, n = 300000, 64
    x = st(F16, randn(r, (rows, n)))
    bias = randn(r, n, 0.02)
    want = O.bias_act(F16, gsvk.ACT_RELU, x, bias)
    X = dev(x, F16)
    gsvk.bias_act(gsvk.ACT_RELU, X, X, bias=devf(bias))
    sync()
    assert_bitexact(F16, host(X, F16), want, "split bias+relu")


@pytest.mark.parametrize("dt", [F32, F16])
def test_sovits_streaming_bit_exact(dt):
    n = 80_000_003 if dt == F32 else 96_000_005   # > 256 MiB per call, tail elements
    say(f"large sovits n={n} dt={dt}")
    r = rng(10 + dt)
    cur, tb = st(dt, randn(r, n)), st(dt, randn(r, n))
    # K1: leaky_relu_write
    X, Y = dev(cur, dt), None
    Y = torch.empty_like(X)
    gsvk.leaky_relu(X, Y, 0.1)
    sync()
    assert_bitexact(dt, host(Y, dt), O.leaky_relu(dt, cur, 0.1), "K1")
    del Y
    # K2: cur += t_b; t_in = lrelu(cur)
    TB = dev(tb, dt)
    TIN = torch.empty_like(X)
    gsvk.resblock_add_lrelu(X, TB, TIN, 0.1)
    sync()
    want_cur, want_tin = O.resblock_add_lrelu(dt, cur, tb, 0.1)
    assert_bitexact(dt, host(X, dt), want_cur, "K2 cur")
    assert_bitexact(dt, host(TIN, dt), want_tin, "K2 t_in")
    del X, TB, TIN


def test_sovits_branch_mean_streaming_bit_exact():
    n = 20_000_001  # f32: 7 operands x 80 MB
    r = rng(20)
    curs = [st(F32, randn(r, n)) for _ in range(3)]
    tbs = [st(F32, randn(r, n)) for _ in range(3)]
    want = O.resblock_branch_mean(F32, curs, tbs, True, 0.01)
    OUT = torch.empty(n, device="cuda")
    gsvk.resblock_branch_mean([devf(c) for c in curs], [devf(t) for t in tbs], OUT, True, 0.01)
    sync()
    assert_bitexact(F32, host(OUT, F32), want, "K3")


def test_groupnorm_streaming():
    C, T = 1100, 31999  # 282 MB moved: non-temporal path
    r = rng(30)
    x = randn(r, (C, T), 0.5)
    g = (1 + randn(r, C, 0.1)).astype(np.float32)
    b = randn(r, C, 0.1)
    want = O.groupnorm_gelu(F32, x, g, b, 1e-5)
    X = devf(x)
    gsvk.groupnorm_gelu(X, devf(g), devf(b), X, 1e-5)
    sync()
    assert_close(F32, host(X, F32), want, "large groupnorm")


@pytest.mark.parametrize("rows", [10001, 262147])  # four-wave workgroups; > 256 MiB of output
def test_embed_large_bit_exact(rows):
    r = rng(40)
    D = 512
    pe = gsvk.pe_table(2048, D)
    tab = (0.02 * randn(r, (1025, D))).astype(np.float16).view(np.uint16)
    ids = r.integers(0, 1025, rows).astype(np.int64)
    pos = r.integers(0, 2048, rows).astype(np.int64)
    out_dt = F16 if rows > 100000 else F32
    want, bad = O.embed_pe(out_dt, F16, tab, ids, pe, 0.9, pos=pos)
    assert bad == 0
    OUT = torch.empty((rows, D), dtype=torch.float16 if out_dt == F16 else torch.float32,
                      device="cuda")
    gsvk.embed_pe(dev(tab, F16), torch.from_numpy(ids).cuda(), devf(pe), 0.9, OUT,
                  pos=torch.from_numpy(pos).cuda())
    sync()
    assert_bitexact(out_dt, host(OUT, out_dt), want, "large embed")


def test_embed_many_rows_int32_ids_bf16_out_partial_lanes():
    """The many-rows-per-wave path (>= 8192 rows) with int32 ids, a bf16 output, an fp32 table and
    D = 200 (25 chunks: lanes past the row end idle), rows not a multiple of the 32 rows a wave
    owns, and invalid ids / positions inside a wave's group."""
    r = rng(43)
    D, rows = 200, 9001
    pe = gsvk.pe_table(2048, D)
    tab = randn(r, (1025, D), 0.02)
    ids = r.integers(0, 1025, rows).astype(np.int32)
    pos = r.integers(0, 2048, rows).astype(np.int64)
    ids[[0, 31, 8999]] = [1025, -7, 4000]
    pos[[32, 9000]] = [-1, 2048]
    want, bad = O.embed_pe(BF16, F32, tab, ids, pe, 1.3, pos=pos)
    assert bad == 5
    OUT = torch.empty((rows, D), dtype=torch.bfloat16, device="cuda")
    err = torch.zeros(1, dtype=torch.int32, device="cuda")
    gsvk.embed_pe(devf(tab), torch.from_numpy(ids).cuda(), devf(pe), 1.3, OUT,
                  pos=torch.from_numpy(pos).cuda(), err=err)
    sync()
    assert int(err.item()) == 1
    assert_bitexact(BF16, host(OUT, BF16), want, "many-rows embed, int32 ids")


def test_embed_long_call_rows_split_by_position():
    """Calls past 256 MiB of output (the non-temporal path): every row written once, bit for bit,
    including text rows (mm + bias), invalid ids / positions (NaN rows and the error flag) and
    implicit positions."""
    r = rng(41)
    D, rows = 512, 262147
    pe = gsvk.pe_table(2048, D)
    tab = (0.02 * randn(r, (732, D))).astype(np.float16).view(np.uint16)
    ids = r.integers(0, 732, rows).astype(np.int64)
    pos = r.integers(0, 2048, rows).astype(np.int64)
    ids[[5, 70000, rows - 1]] = [732, -1, 9999]        # out-of-range ids
    pos[[6, 131072, rows - 2]] = [2048, -3, 1 << 40]   # out-of-range positions
    mm = O.to_storage(F16, randn(r, (rows, D), 1.0))
    bias = randn(r, D, 0.02)
    want, bad = O.embed_pe(F16, F16, tab, ids, pe, 0.9, pos=pos, mm=mm, bias=bias)
    assert bad == 6
    OUT = torch.empty((rows, D), dtype=torch.float16, device="cuda")
    err = torch.zeros(1, dtype=torch.int32, device="cuda")
    gsvk.embed_pe(dev(tab, F16), torch.from_numpy(ids).cuda(), devf(pe), 0.9, OUT,
                  pos=torch.from_numpy(pos).cuda(), mm=dev(mm, F16), bias=devf(bias), err=err)
    sync()
    assert int(err.item()) == 1
    assert_bitexact(F16, host(OUT, F16), want, "long embed, text rows")
    del OUT, want, mm
    # implicit positions pos0 + r over 2^20 + 1 rows of 64 fp32 columns
    D, rows, pos0 = 64, (1 << 20) + 1, 3
    pe = gsvk.pe_table(rows + pos0, D)
    tab = (0.02 * randn(r, (1025, D))).astype(np.float16).view(np.uint16)
    ids = r.integers(0, 1025, rows).astype(np.int64)
    want, bad = O.embed_pe(F32, F16, tab, ids, pe, 0.7, pos0=pos0)
    assert bad == 0
    OUT = torch.empty((rows, D), dtype=torch.float32, device="cuda")
    gsvk.embed_pe(dev(tab, F16), torch.from_numpy(ids).cuda(), devf(pe), 0.7, OUT, pos0=pos0)
    sync()
    assert_bitexact(F32, host(OUT, F32), want, "long embed, implicit positions")
