"""GPU parity of gsvk_decode_attention (KV append + single-query attention per head, B sequences)
against the oracle's restatement of block_decode_impl (t2s_engine.cpp:1051-1087).

Tolerance: the softmax is formed online (running maxima, chunks merged afterwards) in another order
than the reference's two-pass form, so outputs agree within fp32 rounding:
|got - want| <= 1e-5 * max(1, max |V| of the sequence); a 16-bit output may in addition sit one
rounding step away. The append itself is bit-exact (the cache rows equal the oracle's).
"""
import numpy as np
import pytest
import torch

import gsvk
import oracle as O
from gpu_util import BF16, F16, F32, dev, host, say

pytestmark = pytest.mark.gpu

TD = {F32: torch.float32, F16: torch.float16, BF16: torch.bfloat16}


def rng(k):
    return np.random.default_rng(20250823 + 11000 + k)


def step16(dt, w):
    w = np.abs(w.astype(np.float64))
    if dt == F16:
        return np.spacing(np.minimum(w, 65504).astype(np.float16)).astype(np.float64)
    e = np.floor(np.log2(np.maximum(w, 2.0 ** -126)))
    return 2.0 ** (e - 7)


def oracle_kv(kv_dt):
    # the oracle restates the reference's fp32 / fp16 caches; a bf16 cache is checked through the
    # fp32 path on bf16-representable values (rounding happens at the append)
    return F32 if kv_dt == BF16 else kv_dt


def poison_rows(kc, pos, kv_dt):
    """Fill cache rows pos[b] .. max_len - 1 of every sequence with NaN / +Inf / -Inf bit patterns
    (rows the call may not read into its result: the appended row and everything after it)."""
    pats = ([0x7E00, 0x7C00, 0xFC00] if kv_dt == F16 else
            [0x7FC0, 0x7F80, 0xFF80] if kv_dt == BF16 else [0x7FC00000, 0x7F800000, 0xFF800000])
    bits = kc.view(np.uint16 if kv_dt != F32 else np.uint32)
    for b, p in enumerate(pos):
        n = bits.shape[1] - p
        bits[b, p:] = np.resize(np.asarray(pats, bits.dtype), (n, 1)).repeat(bits.shape[2], 1)


def case(B, H, HD, max_len, pos, kv_dt, out_dt, seed, len_bound=0, use_ws=True, poison=False):
    say(f"attention B={B} H={H} HD={HD} max_len={max_len} kv={kv_dt} out={out_dt} "
        f"len_bound={len_bound} ws={use_ws} poison={poison}")
    r = rng(seed)
    D = H * HD
    qkv = r.standard_normal((B, 3 * D)).astype(np.float32)
    k32 = r.standard_normal((B, max_len, D)).astype(np.float32)
    v32 = r.standard_normal((B, max_len, D)).astype(np.float32)
    if kv_dt == BF16:
        # bf16-exact inputs so the fp32 oracle sees the same values the bf16 cache holds
        for a in (k32, v32):
            a[:] = O.to_f32(BF16, O.to_storage(BF16, a))
        qkv[:, D:] = O.to_f32(BF16, O.to_storage(BF16, qkv[:, D:]))
    kc = O.to_storage(kv_dt, k32)
    vc = O.to_storage(kv_dt, v32)
    pos = np.asarray(pos, dtype=np.int64)
    if poison:
        for a in (kc, vc):
            poison_rows(a, pos, kv_dt)
    okv = oracle_kv(kv_dt)
    kc_o = kc if okv == kv_dt else O.to_f32(kv_dt, kc)
    vc_o = vc if okv == kv_dt else O.to_f32(kv_dt, vc)
    kc_o, vc_o = kc_o.copy(), vc_o.copy()
    want = O.decode_attention(okv, qkv, kc_o, vc_o, pos, H, HD)
    Q = torch.from_numpy(qkv).cuda()
    KC, VC = dev(kc, kv_dt), dev(vc, kv_dt)
    P = torch.from_numpy(pos).cuda()
    OUT = torch.empty((B, D), dtype=TD[out_dt], device="cuda")
    ERR = torch.zeros(1, dtype=torch.int32, device="cuda")
    gsvk.decode_attention(Q, KC, VC, P, OUT, H, len_bound=len_bound, err=ERR, use_workspace=use_ws)
    torch.cuda.synchronize()
    got = O.to_f32(out_dt, host(OUT, out_dt))
    vmax = np.array([np.abs(O.to_f32(kv_dt, vc[b, :p])).max() if p > 0 else 0.0
                     for b, p in enumerate(np.clip(pos, 0, max_len))])
    tol = 1e-5 * np.maximum(1.0, vmax)[:, None]
    if out_dt != F32:
        tol = tol + step16(out_dt, want)
        want_c = O.to_f32(out_dt, O.to_storage(out_dt, want))
    else:
        want_c = want
    nan_g, nan_w = np.isnan(got), np.isnan(want_c)
    assert np.array_equal(nan_g, nan_w), "NaN rows differ"
    err = np.abs(got - want_c)
    err[nan_w] = 0
    bad = np.argwhere(err > tol)
    assert bad.size == 0, f"{len(bad)} outside tolerance, worst {np.max(err - tol):.3e} at " \
                          f"{bad[:3].tolist()}"
    # the append is exact; other rows untouched
    kc_g, vc_g = host(KC, kv_dt), host(VC, kv_dt)
    u = lambda a: a.view(np.uint32) if a.dtype == np.float32 else a
    if okv == kv_dt:
        assert np.array_equal(u(kc_g), u(kc_o)) and np.array_equal(u(vc_g), u(vc_o)), \
            "cache rows differ"
    else:
        assert np.array_equal(u(O.to_f32(kv_dt, kc_g)), u(kc_o)) and \
            np.array_equal(u(O.to_f32(kv_dt, vc_g)), u(vc_o)), "cache rows differ"
    return got, int(ERR.item()), (Q, KC, VC, P, OUT)


@pytest.mark.parametrize("kv_dt", [F32, F16, BF16])
def test_attention_small(kv_dt):
    _, e, _ = case(3, 4, 32, 40, [0, 17, 39], kv_dt, F32, 1)
    assert e == 0


@pytest.mark.parametrize("kv_dt,out_dt", [(F16, F16), (F16, F32), (F32, F32), (F16, BF16)])
@pytest.mark.parametrize("len_bound,use_ws", [(0, True), (1100, True), (256, True), (0, False)])
def test_attention_decode_batch(kv_dt, out_dt, len_bound, use_ws):
    """B = 64 sequences of different lengths, 16 heads of 32 (the T2S decoder), chunked and not."""
    r = rng(2)
    pos = r.integers(0, 1100, 64)
    pos[:3] = [0, 1, 1099]
    _, e, _ = case(64, 16, 32, 1100, pos, kv_dt, out_dt, 3, len_bound, use_ws)
    assert e == 0


@pytest.mark.parametrize("H,HD", [(8, 64), (16, 16), (4, 128), (1, 8), (2, 256)])
def test_attention_head_shapes(H, HD):
    r = rng(H * HD)
    pos = r.integers(0, 300, 5)
    case(5, H, HD, 300, pos, F16, F32, 4, 300)


def test_attention_invalid_position_nan_and_flag():
    got, e, _ = case(4, 16, 32, 50, [3, -1, 50, 49], F16, F32, 5, 50)
    assert e == 1
    assert np.all(np.isnan(got[1])) and np.all(np.isnan(got[2]))
    assert not np.any(np.isnan(got[[0, 3]]))


def test_attention_deterministic():
    r = rng(6)
    pos = r.integers(500, 1000, 64)
    a, _, (Q, KC, VC, P, OUT) = case(64, 16, 32, 1000, pos, F16, F32, 7, 1000)
    # the appended rows are in place; attending again with the same pos gives the same bits
    gsvk.decode_attention(Q, KC, VC, P, OUT, 16, len_bound=1000)
    torch.cuda.synchronize()
    b = host(OUT, F32)
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32))


@pytest.mark.parametrize("kv_dt", [F16, F32, BF16])
@pytest.mark.parametrize("len_bound,use_ws", [(0, False), (1100, True)])
def test_attention_ignores_nonfinite_rows_past_pos(kv_dt, len_bound, use_ws):
    """Rows at and past pos hold NaN / +-Inf: only rows < pos and the appended k / v enter the
    result (a padded key slot of a wave re-reads the last row of its chunk, which for the chunk
    holding pos is that row). Lengths cover odd key counts per wave, one key, and chunk borders."""
    pos = [0, 1, 2, 3, 5, 7, 9, 17, 33, 64, 99, 130, 257, 513, 1023, 1099]
    _, e, _ = case(len(pos), 16, 32, 1100, pos, kv_dt, F32, 8, len_bound, use_ws, poison=True)
    assert e == 0


def test_attention_rejects_bad_arguments():
    L = gsvk.lib()
    Q = torch.zeros((2, 3 * 512), dtype=torch.float32, device="cuda")
    K = torch.zeros((2, 8, 512), dtype=torch.float16, device="cuda")
    V = torch.zeros((2, 8, 512), dtype=torch.float16, device="cuda")
    P = torch.zeros(2, dtype=torch.int64, device="cuda")
    Y = torch.zeros((2, 512), dtype=torch.float32, device="cuda")

    def call(kv=F16, out=F32, q=Q.data_ptr(), ldq=1536, k=K.data_ptr(), y=Y.data_ptr(), H=16,
             HD=32):
        return L.gsvk_decode_attention(kv, out, q, ldq, k, V.data_ptr(), 8, P.data_ptr(), y, 512,
                                       2, H, HD, 0, None, 0, None, None)
    assert call() == gsvk.OK
    torch.cuda.synchronize()
    assert call(kv=7) == gsvk.E_DTYPE
    assert call(q=None) == gsvk.E_NULL
    assert call(ldq=1000) == gsvk.E_SIZE
    assert call(H=32, HD=32) == gsvk.E_ARG        # D = 1024 > 512
    assert call(H=32, HD=12) == gsvk.E_ARG        # head_dim not a multiple of 8
    assert call(y=K.data_ptr()) == gsvk.E_ALIAS   # output over the cache
