"""Pins the oracle's decode attention (oracle_decode_attention) and its softmax step.

  - softmax against the reference's golden vectors tests/golden/sm_{x,y} (F.softmax, written by
    tools/export_kern_golden.py:71-75) under the reference's own gate (test_kern.cpp:218-229: max
    rel 1e-6, cosine 1 - 1e-12, rows summing to 1 within 1e-6);
  - one key (pos = 0): the output is exactly the appended value row (p = exp(0) / 1 = 1);
  - equal keys: uniform weights, the output is the mean of the value rows;
  - a float64 closed form of scaled dot-product attention on the same (rounded) cache, which a
    missing scale, a swapped head or a dropped newest key fails;
  - the append: position pos holds the rounded k / v, every other position is untouched, and a
    position outside the cache gives a NaN row.
"""
import numpy as np
import pytest

from conftest import check_close, load_bin

import oracle as O

F32, F16 = O.F32, O.F16


@pytest.fixture(scope="module", autouse=True)
def _lib(oracle_lib):
    return oracle_lib


def test_softmax_matches_reference_golden():
    x, y = load_bin("sm_x.f32"), load_bin("sm_y.f32")
    assert x.shape == (7, 257)
    got = np.stack([O.softmax(r) for r in x])
    ok, worst, cos = check_close(got, y, 1e-6, 1.0 - 1e-12)
    assert ok, (worst, cos)
    assert np.all(np.abs(got.astype(np.float64).sum(1) - 1.0) <= 1e-6)
    # planted: a missing exp, the wrong axis, and a base-2 exponential all fail the same gate
    x64 = x.astype(np.float64)
    e = np.exp(x64 - x64.max(1, keepdims=True))
    assert check_close(e / e.sum(1, keepdims=True), y, 1e-6, 1 - 1e-12)[0]
    e0 = np.exp(x64 - x64.max(0, keepdims=True))
    e2 = np.exp2(x64 - x64.max(1, keepdims=True))
    for bad in (x64 / x64.sum(1, keepdims=True), e0 / e0.sum(0, keepdims=True),
                e2 / e2.sum(1, keepdims=True)):
        assert not check_close(bad, y, 1e-6, 1 - 1e-12)[0]


def make(B, max_len, H, HD, kv_dt, seed, fill=None):
    r = np.random.default_rng(seed)
    D = H * HD
    qkv = r.standard_normal((B, 3 * D)).astype(np.float32)
    k32 = r.standard_normal((B, max_len, D)).astype(np.float32)
    v32 = r.standard_normal((B, max_len, D)).astype(np.float32)
    if fill is not None:
        fill(qkv, k32, v32)
    kc = O.to_storage(kv_dt, k32)
    vc = O.to_storage(kv_dt, v32)
    return qkv, kc, vc


def closed_form(kv_dt, qkv, kc, vc, pos, H, HD, scale=None, swap_head=False, drop_new=False):
    """float64 attention on the cache after the append (kc / vc already hold the new rows)."""
    B = qkv.shape[0]
    D = H * HD
    K = O.to_f32(kv_dt, kc).astype(np.float64)
    V = O.to_f32(kv_dt, vc).astype(np.float64)
    out = np.zeros((B, D))
    sc = 1.0 / np.sqrt(np.float32(HD)) if scale is None else scale
    for b in range(B):
        n = pos[b] + (0 if drop_new else 1)
        if n == 0:
            continue
        for h in range(H):
            hk = (h + 1) % H if swap_head else h
            q = qkv[b, h * HD:(h + 1) * HD].astype(np.float64)
            s = K[b, :n, hk * HD:(hk + 1) * HD] @ q * sc
            p = np.exp(s - s.max())
            p /= p.sum()
            out[b, h * HD:(h + 1) * HD] = p @ V[b, :n, h * HD:(h + 1) * HD]
    return out


@pytest.mark.parametrize("kv_dt", [F32, F16])
def test_attention_closed_form_and_planted_mistakes(kv_dt):
    H, HD, B, max_len = 4, 32, 3, 40
    qkv, kc, vc = make(B, max_len, H, HD, kv_dt, 1)
    pos = np.array([0, 17, 39], dtype=np.int64)
    got = O.decode_attention(kv_dt, qkv, kc, vc, pos, H, HD)
    want = closed_form(kv_dt, qkv, kc, vc, pos, H, HD)
    tol = 1e-5 * np.maximum(1.0, np.abs(O.to_f32(kv_dt, vc)).max())
    assert np.max(np.abs(got - want)) <= tol
    for bad in (dict(scale=1.0), dict(swap_head=True), dict(drop_new=True)):
        wrong = closed_form(kv_dt, qkv, kc, vc, pos, H, HD, **bad)
        assert np.max(np.abs(got[1:] - wrong[1:])) > 100 * tol, bad


@pytest.mark.parametrize("kv_dt", [F32, F16])
def test_attention_one_key_returns_value_row(kv_dt):
    H, HD = 16, 32
    qkv, kc, vc = make(2, 8, H, HD, kv_dt, 2)
    pos = np.array([0, 0], dtype=np.int64)
    got = O.decode_attention(kv_dt, qkv, kc, vc, pos, H, HD)
    D = H * HD
    v_rounded = O.to_f32(kv_dt, O.to_storage(kv_dt, qkv[:, 2 * D:]))
    assert np.array_equal(got, v_rounded)


def test_attention_equal_keys_average_values():
    H, HD, L = 2, 32, 9

    def fill(qkv, k, v):
        k[:] = k[:, :1, :]          # every cached key equal to the first
        qkv[:, H * HD:2 * H * HD] = k[:, 0, :]  # and the new key too
    qkv, kc, vc = make(1, L, H, HD, F32, 3, fill)
    pos = np.array([L - 1], dtype=np.int64)
    got = O.decode_attention(F32, qkv, kc, vc, pos, H, HD)
    V = vc.astype(np.float64)[0, :L]
    assert np.max(np.abs(got[0] - V.mean(0))) < 1e-6


@pytest.mark.parametrize("kv_dt", [F32, F16])
def test_attention_append_and_bad_position(kv_dt):
    H, HD, max_len = 4, 16, 12
    qkv, kc, vc = make(3, max_len, H, HD, kv_dt, 4)
    k0, v0 = kc.copy(), vc.copy()
    pos = np.array([5, -1, 12], dtype=np.int64)
    got = O.decode_attention(kv_dt, qkv, kc, vc, pos, H, HD)
    D = H * HD
    assert np.array_equal(kc[0, 5], O.to_storage(kv_dt, qkv[0, D:2 * D]))
    assert np.array_equal(vc[0, 5], O.to_storage(kv_dt, qkv[0, 2 * D:]))
    mask = np.ones(max_len, bool)
    mask[5] = False
    assert np.array_equal(kc[0, mask], k0[0, mask]) and np.array_equal(vc[1:], v0[1:])
    assert np.array_equal(kc[1:], k0[1:])
    assert np.all(np.isnan(got[1])) and np.all(np.isnan(got[2])) and not np.any(np.isnan(got[0]))
