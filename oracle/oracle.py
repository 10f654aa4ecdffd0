"""numpy/ctypes front of the CPU oracle (liboracle.so, oracle/gsvk_oracle.c).

TEST INFRASTRUCTURE ONLY: used by tests/, the smoke check and the CPU-baseline leg of bench.py as
the reference results the GPU kernels are compared with. The product (libgsvk.so) never imports
or calls it.

Arrays are host numpy arrays holding the *storage* representation: float32 for dtype F32, uint16
bit patterns for F16 / BF16 (F16 may also be given as numpy float16).
"""
import ctypes
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "liboracle.so")
# tests/sanitizers.sh points this at the AddressSanitizer / UBSan build (oracle/_san/)
LIB_PATH = os.environ.get("GSVK_ORACLE_LIB", LIB_PATH)
F32, F16, BF16 = 0, 1, 2

_vp, _sz, _i, _f, _d = ctypes.c_void_p, ctypes.c_size_t, ctypes.c_int, ctypes.c_float, ctypes.c_double
_SIG = {
    "oracle_h2f": (_f, [ctypes.c_uint16]),
    "oracle_f2h": (ctypes.c_uint16, [_f]),
    "oracle_bf2f": (_f, [ctypes.c_uint16]),
    "oracle_f2bf": (ctypes.c_uint16, [_f]),
    "oracle_to_f32": (None, [_i, _vp, _vp, _sz]),
    "oracle_from_f32": (None, [_i, _vp, _vp, _sz]),
    "oracle_layernorm_row": (None, [_vp, _vp, _vp, _vp, _sz, _d]),
    "oracle_layernorm1d_row": (None, [_vp, _vp, _vp, _sz, _f]),
    "oracle_add_layernorm": (_i, [_i, _vp, _vp, _vp, _vp, _vp, _vp, _sz, _sz, _sz, _d, _i]),
    "oracle_bias_act": (_i, [_i, _i, _vp, _vp, _vp, _sz, _sz, _sz, _f]),
    "oracle_relu": (None, [_vp, _vp, _sz]),
    "oracle_gelu_erf": (_f, [_f]),
    "oracle_groupnorm_gelu": (_i, [_i, _vp, _vp, _vp, _vp, _sz, _sz, _sz, _d, _i]),
    "oracle_leaky_relu": (_i, [_i, _vp, _vp, _sz, _f]),
    "oracle_resblock_add_lrelu": (_i, [_i, _vp, _vp, _vp, _sz, _f]),
    "oracle_resblock_branch_mean": (_i, [_i, ctypes.POINTER(_vp), ctypes.POINTER(_vp), _i, _vp, _sz,
                                         _i, _f]),
    "oracle_scaled_add": (_i, [_i, _vp, _vp, _vp, _sz, _f]),
    "oracle_gemv_f16w": (_i, [_i, _i, _vp, _sz, _vp, _vp, _i, _f, _vp, _i, _vp, _sz, _sz, _sz,
                              _sz]),
    "oracle_decode_attention": (_i, [_i, _vp, _sz, _vp, _vp, _sz, _vp, _vp, _sz, _sz, _sz, _sz]),
    "oracle_softmax": (None, [_vp, _vp, _sz]),
    "oracle_convt1d": (_i, [_i, _vp, _sz, _vp, _vp, _i, _f, _vp, _sz, _vp, _sz, _sz, _sz, _sz, _sz,
                            _sz]),
    "oracle_conv1d": (_i, [_i, _vp, _sz, _vp, _vp, _i, _f, _vp, _sz, _vp, _sz, _sz, _sz, _sz, _sz,
                           _sz]),
    "oracle_pe_row": (None, [_vp, _sz, _sz]),
    "oracle_embed_pe": (ctypes.c_long, [_i, _i, _i, _vp, _sz, _vp, _vp, ctypes.c_int64, _vp, _sz,
                                        _f, _vp, _vp, _vp, _sz, _sz]),
    "oracle_t2s_step": (_i, [_i, _sz, _sz, _sz, _sz, _d, _vp, _i, _sz, _vp, _vp, _vp, _sz, _f, _vp,
                             _vp] + [ctypes.POINTER(_vp)] * 10 + [_i]),
}

_LIB = None


def lib():
    global _LIB
    if _LIB is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"{LIB_PATH} is not built (make -C oracle)")
        L = ctypes.CDLL(LIB_PATH)
        for name, (res, args) in _SIG.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _LIB = L
    return _LIB


def _p(a):
    return None if a is None else a.ctypes.data


def storage_dtype(dt):
    return np.float32 if dt == F32 else np.uint16


def to_storage(dt, x32):
    """float32 array -> storage array (float32 or uint16 bits), rounding to nearest even."""
    x32 = np.ascontiguousarray(x32, dtype=np.float32)
    if dt == F32:
        return x32.copy()
    out = np.empty(x32.shape, dtype=np.uint16)
    lib().oracle_from_f32(dt, _p(x32), _p(out), x32.size)
    return out


def to_f32(dt, s):
    """storage array -> float32 (exact)."""
    s = np.ascontiguousarray(s)
    if dt == F32:
        return s.astype(np.float32, copy=True)
    if s.dtype == np.float16:
        s = s.view(np.uint16)
    out = np.empty(s.shape, dtype=np.float32)
    lib().oracle_to_f32(dt, _p(s), _p(out), s.size)
    return out


def _rows(x):
    if x.ndim == 1:
        return 1, x.shape[0], x.shape[0]
    return x.shape[0], x.shape[1], x.strides[0] // x.itemsize


def layernorm_row(x, g, b, eps):
    x = np.ascontiguousarray(x, dtype=np.float32)
    y = np.empty_like(x)
    lib().oracle_layernorm_row(_p(x), _p(g), _p(b), _p(y), x.size, eps)
    return y


def add_layernorm(dt, x, gamma, beta, eps, bias=None, residual=None, mode=0):
    rows, n, ld = _rows(x)
    y = np.empty_like(x)
    rc = lib().oracle_add_layernorm(dt, _p(x), _p(bias), _p(residual), _p(gamma), _p(beta), _p(y),
                                    rows, n, ld, eps, mode)
    assert rc == 0
    return y


def bias_act(dt, act, x, bias=None, slope=0.0):
    rows, n, ld = _rows(x)
    y = np.empty_like(x)
    assert lib().oracle_bias_act(dt, act, _p(x), _p(bias), _p(y), rows, n, ld, slope) == 0
    return y


def relu(x):
    x = np.ascontiguousarray(x, dtype=np.float32)
    y = np.empty_like(x)
    lib().oracle_relu(_p(x), _p(y), x.size)
    return y


def gelu_erf(v):
    return np.array([lib().oracle_gelu_erf(float(t)) for t in np.ravel(v)], dtype=np.float32)


def groupnorm_gelu(dt, x, gamma, beta, eps, apply_gelu=True):
    C, T, ld = _rows(x)
    y = np.empty_like(x)
    assert lib().oracle_groupnorm_gelu(dt, _p(x), _p(gamma), _p(beta), _p(y), C, T, ld, eps,
                                       int(apply_gelu)) == 0
    return y


def leaky_relu(dt, x, slope):
    y = np.empty_like(x)
    assert lib().oracle_leaky_relu(dt, _p(x), _p(y), x.size, slope) == 0
    return y


def resblock_add_lrelu(dt, cur, t_b, slope, write_tin=True):
    cur = cur.copy()
    t_in = np.empty_like(cur) if write_tin else None
    assert lib().oracle_resblock_add_lrelu(dt, _p(cur), _p(t_b), _p(t_in), cur.size, slope) == 0
    return cur, t_in


def resblock_branch_mean(dt, curs, tbs, apply_lrelu, slope):
    nb = len(curs)
    out = np.empty_like(curs[0])
    c_arr = (_vp * nb)(*[_p(c) for c in curs])
    t_arr = (_vp * nb)(*[_p(t) for t in tbs]) if tbs is not None else None
    assert lib().oracle_resblock_branch_mean(dt, c_arr, t_arr, nb, _p(out), out.size,
                                             int(apply_lrelu), slope) == 0
    return out


def scaled_add(dt, acc, src, scale):
    out = np.empty_like(src)
    assert lib().oracle_scaled_add(dt, _p(acc), _p(src), _p(out), src.size, scale) == 0
    return out


def gemv_f16w(x_dt, x, w, y_dt, bias=None, act=0, slope=0.0, residual=None, round_x=True):
    """y [rows, out] storage array = act(w @ x[r] + bias) (+ residual[r]) per row.
    x: [rows, in] storage of x_dt (F32 or F16); w: [out, in] uint16 fp16 bits."""
    x = np.ascontiguousarray(x)
    if x.ndim == 1:
        x = x[None, :]
    w = np.ascontiguousarray(w).view(np.uint16)
    rows, n_in = x.shape
    n_out = w.shape[0]
    assert w.shape[1] == n_in
    y = np.empty((rows, n_out), dtype=storage_dtype(y_dt))
    if residual is not None:
        residual = np.ascontiguousarray(residual).reshape(rows, n_out)
    rc = lib().oracle_gemv_f16w(x_dt, int(round_x), _p(x), n_in, _p(w), _p(bias), act, slope,
                                _p(residual), y_dt, _p(y), n_out, rows, n_out, n_in)
    assert rc == 0
    return y


def conv1d(dt, x, w, bias=None, dil=1, epi=0, slope=0.1, cur=None):
    """SoVITS Conv1d + epilogue. x [cin, T] storage of dt; w [cout, cin, k] uint16 fp16 bits.
    Returns y (and the updated cur for epi 2 / 3)."""
    x = np.ascontiguousarray(x)
    w = np.ascontiguousarray(w).view(np.uint16)
    cout, cin, k = w.shape
    T = x.shape[1]
    y = np.zeros((cout, T), dtype=storage_dtype(dt))
    c = None if cur is None else np.ascontiguousarray(cur).copy()
    if epi == 4:
        c = np.zeros((cout, T), dtype=storage_dtype(dt))
    rc = lib().oracle_conv1d(dt, _p(x), T, _p(w), _p(bias), epi, slope, _p(c), T, _p(y), T, cin,
                             cout, T, k, dil)
    assert rc == 0
    return (y, c) if epi in (2, 3, 4) else y


def convt1d(dt, x, w, u, bias=None, epi=0, slope=0.1, cur=None):
    """SoVITS ConvTranspose1d + epilogue. x [cin, T] storage of dt; w [cin, cout, k] uint16 fp16
    bits (torch layout); stride u. Returns y [cout, T u] (and the updated cur for epi 2 / 3)."""
    x = np.ascontiguousarray(x)
    w = np.ascontiguousarray(w).view(np.uint16)
    cin, cout, k = w.shape
    T = x.shape[1]
    y = np.zeros((cout, T * u), dtype=storage_dtype(dt))
    c = None if cur is None else np.ascontiguousarray(cur).copy()
    if epi == 4:
        c = np.zeros((cout, T * u), dtype=storage_dtype(dt))
    rc = lib().oracle_convt1d(dt, _p(x), T, _p(w), _p(bias), epi, slope, _p(c), T * u, _p(y),
                              T * u, cin, cout, T, k, u)
    assert rc == 0
    return (y, c) if epi in (2, 3, 4) else y


def softmax(x):
    x = np.ascontiguousarray(x, dtype=np.float32)
    y = np.empty_like(x)
    lib().oracle_softmax(_p(x), _p(y), x.size)
    return y


def decode_attention(kv_dt, qkv, kcache, vcache, pos, H, HD):
    """KV append + single-query attention. qkv [B, 3D] float32; kcache / vcache [B, max_len, D]
    storage arrays of kv_dt (F32 or F16), updated in place at pos; returns out [B, D] float32."""
    qkv = np.ascontiguousarray(qkv, dtype=np.float32)
    B = qkv.shape[0]
    D = H * HD
    assert kcache.flags.c_contiguous and vcache.flags.c_contiguous
    max_len = kcache.shape[1]
    pos = np.ascontiguousarray(pos, dtype=np.int64)
    out = np.empty((B, D), dtype=np.float32)
    rc = lib().oracle_decode_attention(kv_dt, _p(qkv), qkv.shape[1], _p(kcache), _p(vcache),
                                       max_len, _p(pos), _p(out), D, B, H, HD)
    assert rc == 0
    return out


def pe_row(pos, D):
    pe = np.empty(D, dtype=np.float32)
    lib().oracle_pe_row(_p(pe), pos, D)
    return pe


def pe_table(max_pos, D):
    return np.stack([pe_row(p, D) for p in range(max_pos)]) if max_pos else np.empty((0, D), np.float32)


def embed_pe(out_dt, table_dt, table, ids, pe, alpha, pos=None, pos0=0, mm=None, bias=None):
    """Returns (out storage array [rows, D], number of out-of-range rows)."""
    vocab, D = table.shape
    ids = np.ascontiguousarray(ids)
    itype = 1 if ids.dtype == np.int32 else 0
    rows = ids.size
    out = np.empty((rows, D), dtype=storage_dtype(out_dt))
    bad = lib().oracle_embed_pe(out_dt, table_dt, itype, _p(table), vocab, _p(ids), _p(pos), pos0,
                                _p(pe), pe.shape[0], alpha, _p(mm), _p(bias), _p(out), rows, D)
    return out, int(bad)


def t2s_step(dt, bufs, eps=1e-5, threads=1):
    """One decode step's epilogue chain on host buffers (dict of numpy arrays, in place on
    bufs['x'], bufs['h'], bufs['ff'][l])."""
    L = len(bufs["attn_out"])
    B, D = bufs["x"].shape
    FF = bufs["ff"][0].shape[1]

    def arr(name):
        return (_vp * L)(*[_p(a) for a in bufs[name]])

    names = ("attn_out", "bout", "n1g", "n1b", "ff", "b1", "ffn_out", "b2", "n2g", "n2b")
    arrays = [arr(n) for n in names]
    table = bufs["table"]
    rc = lib().oracle_t2s_step(dt, B, D, FF, L, eps, _p(table), bufs["table_dtype"], table.shape[0],
                               _p(bufs["ids"]), _p(bufs["pos"]), _p(bufs["pe"]), bufs["pe"].shape[0],
                               bufs["alpha"], _p(bufs["x"]), _p(bufs["h"]),
                               *[ctypes.cast(a, ctypes.POINTER(_vp)) for a in arrays], threads)
    assert rc == 0
