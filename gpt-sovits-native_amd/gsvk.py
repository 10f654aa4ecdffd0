"""ctypes binding of libgsvk.so, the C ABI declared in include/gsvk.h and include/gsvk_t2s.h.

The library is the product; this module only marshals arguments. Device buffers are passed as
torch tensors (for their data pointers and strides) or as raw integer addresses. Every call checks
the returned status and raises GsvkError on anything but GSVK_OK. There is no fallback: if
libgsvk.so is missing or cannot be loaded, `lib()` raises.
"""
import ctypes
import os

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libgsvk.so")

F32, F16, BF16 = 0, 1, 2
I64, I32 = 0, 1
ACT_NONE, ACT_RELU, ACT_GELU_ERF, ACT_LEAKY_RELU = 0, 1, 2, 3
OK, E_NULL, E_SIZE, E_DTYPE, E_ALIAS, E_ARG, E_HIP = 0, -1, -2, -3, -4, -5, -6

# Every exported symbol of the C ABI with (restype, argtypes).
_vp, _sz, _i, _f, _d = ctypes.c_void_p, ctypes.c_size_t, ctypes.c_int, ctypes.c_float, ctypes.c_double
_i64 = ctypes.c_int64
SIGNATURES = {
    "gsvk_version": (ctypes.c_char_p, []),
    "gsvk_status_string": (ctypes.c_char_p, [_i]),
    "gsvk_add_layernorm": (_i, [_i, _vp, _vp, _vp, _vp, _vp, _vp, _sz, _sz, _sz, _d, _vp]),
    "gsvk_bias_act": (_i, [_i, _i, _vp, _vp, _vp, _sz, _sz, _sz, _f, _vp]),
    "gsvk_gemv_f16w": (_i, [_i, _i, _vp, _sz, _vp, _vp, _i, _f, _vp, _i, _vp, _sz, _sz, _sz, _sz,
                            _vp]),
    "gsvk_decode_attention": (_i, [_i, _i, _vp, _sz, _vp, _vp, _sz, _vp, _vp, _sz, _sz, _sz, _sz,
                                   _sz, _vp, _sz, _vp, _vp]),
    "gsvk_decode_attention_workspace_bytes": (_sz, [_sz, _sz, _sz, _sz]),
    "gsvk_groupnorm_gelu": (_i, [_i, _vp, _vp, _vp, _vp, _sz, _sz, _sz, _d, _i, _vp]),
    "gsvk_leaky_relu": (_i, [_i, _vp, _vp, _sz, _f, _vp]),
    "gsvk_resblock_add_lrelu": (_i, [_i, _vp, _vp, _vp, _sz, _f, _vp]),
    "gsvk_resblock_branch_mean": (_i, [_i, ctypes.POINTER(_vp), ctypes.POINTER(_vp), _i, _vp, _sz,
                                       _i, _f, _vp]),
    "gsvk_scaled_add": (_i, [_i, _vp, _vp, _vp, _sz, _f, _vp]),
    "gsvk_embed_pe": (_i, [_i, _i, _i, _vp, _sz, _vp, _vp, _i64, _vp, _sz, _f, _vp, _vp, _vp, _sz,
                           _sz, _vp, _vp]),
    "gsvk_pe_table": (_i, [_vp, _sz, _sz]),
    "gsvk_t2s_step_eager": (_i, [_vp, _vp]),
    "gsvk_t2s_step_create": (_i, [_vp, ctypes.POINTER(_vp)]),
    "gsvk_t2s_step_run": (_i, [_vp, _vp]),
    "gsvk_t2s_step_launches": (_i, [_vp]),
    "gsvk_t2s_step_destroy": (None, [_vp]),
    "gsvk_t2s_decode_eager": (_i, [_vp, _vp]),
    "gsvk_t2s_decode_create": (_i, [_vp, ctypes.POINTER(_vp)]),
}


class GsvkError(RuntimeError):
    def __init__(self, fn, status):
        super().__init__(f"{fn}: status {status}")
        self.status = status


_LIB = None


def lib():
    """Load libgsvk.so once; raise if it is not built."""
    global _LIB
    if _LIB is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"{LIB_PATH} is not built (run __graft_entry__.build())")
        L = ctypes.CDLL(LIB_PATH)
        for name, (res, args) in SIGNATURES.items():
            f = getattr(L, name)
            f.restype = res
            f.argtypes = args
        _LIB = L
    return _LIB


def _ptr(t):
    """Device address of a torch tensor (or an int address / None)."""
    if t is None:
        return None
    if isinstance(t, int):
        return t
    return t.data_ptr()


def _stream(stream):
    if stream is None:
        import torch
        return torch.cuda.current_stream().cuda_stream
    return stream if isinstance(stream, int) else stream.cuda_stream


def _check(fn, rc):
    if rc != OK:
        raise GsvkError(fn, rc)
    return rc


def dtype_code(t):
    import torch
    return {torch.float32: F32, torch.float16: F16, torch.bfloat16: BF16}[t.dtype]


def _rows(t):
    """(rows, n, ld) of a 2-D row-major view (or a 1-D buffer as one row)."""
    if t.dim() == 1:
        return 1, t.shape[0], t.shape[0]
    assert t.dim() == 2 and (t.stride(1) == 1 or t.shape[1] == 1), "rows must be contiguous"
    # a single row has no meaningful row stride (numpy / torch may report 0 for it)
    return t.shape[0], t.shape[1], t.stride(0) if t.shape[0] > 1 else t.shape[1]


def add_layernorm(x, gamma, beta, y, eps, bias=None, residual=None, stream=None, check=True):
    rows, n, ld = _rows(x)
    rc = lib().gsvk_add_layernorm(dtype_code(x), _ptr(x), _ptr(bias), _ptr(residual), _ptr(gamma),
                                  _ptr(beta), _ptr(y), rows, n, ld, eps, _stream(stream))
    return _check("gsvk_add_layernorm", rc) if check else rc


def bias_act(act, x, y, bias=None, slope=0.0, stream=None):
    rows, n, ld = _rows(x)
    return _check("gsvk_bias_act", lib().gsvk_bias_act(dtype_code(x), act, _ptr(x), _ptr(bias),
                                                       _ptr(y), rows, n, ld, slope,
                                                       _stream(stream)))


def gemv_f16w(x, w, y, bias=None, act=ACT_NONE, slope=0.0, residual=None, round_x=True,
              stream=None):
    """y[r] = act(w @ x[r] + bias) (+ residual[r]); x [rows, in] f32/f16, w [out, in] f16,
    y / residual [rows, out] sharing y's row stride."""
    rows, n_in, ldx = _rows(x)
    n_out = w.shape[0]
    _, _, ldy = _rows(y)
    assert residual is None or residual.data_ptr() == y.data_ptr() or _rows(residual)[2] == ldy, \
        "residual shares y's row stride"
    return _check("gsvk_gemv_f16w",
                  lib().gsvk_gemv_f16w(dtype_code(x), int(round_x), _ptr(x), ldx, _ptr(w),
                                       _ptr(bias), act, slope, _ptr(residual), dtype_code(y),
                                       _ptr(y), ldy, rows, n_out, n_in, _stream(stream)))


_WS = {}


def workspace(device, nbytes):
    """A device scratch tensor of at least nbytes, kept per device for the process. Grow it before
    any graph capture (allocation is not allowed while capturing)."""
    import torch
    dev = torch.device(device)
    key = dev.index if dev.index is not None else torch.cuda.current_device()
    ws = _WS.get(key)
    if ws is None or ws.numel() < nbytes:
        ws = torch.empty(max(nbytes, 1 << 20), dtype=torch.uint8, device=torch.device("cuda", key))
        _WS[key] = ws
    return ws


def decode_attention(qkv, k_cache, v_cache, pos, out, heads, len_bound=0, err=None, stream=None,
                     use_workspace=True):
    """Append k / v at pos and attend. qkv [B, >=3D] fp32; caches [B, max_len, D]; pos [B] int64;
    out [B, D]."""
    B = qkv.shape[0]
    D = out.shape[-1]
    max_len = k_cache.shape[1]
    hd = D // heads
    ws, wsb = None, 0
    if use_workspace:
        need = lib().gsvk_decode_attention_workspace_bytes(B, heads, hd, len_bound or max_len)
        if need:
            w = workspace(out.device, need)
            ws, wsb = w.data_ptr(), w.numel()
    return _check("gsvk_decode_attention",
                  lib().gsvk_decode_attention(dtype_code(k_cache), dtype_code(out), _ptr(qkv),
                                              _rows(qkv)[2], _ptr(k_cache), _ptr(v_cache),
                                              max_len, _ptr(pos), _ptr(out), _rows(out)[2], B,
                                              heads, hd, len_bound, ws, wsb, _ptr(err),
                                              _stream(stream)))


def groupnorm_gelu(x, gamma, beta, y, eps, apply_gelu=True, stream=None):
    C, T, ld = _rows(x)
    return _check("gsvk_groupnorm_gelu",
                  lib().gsvk_groupnorm_gelu(dtype_code(x), _ptr(x), _ptr(gamma), _ptr(beta),
                                            _ptr(y), C, T, ld, eps, int(apply_gelu),
                                            _stream(stream)))


def leaky_relu(x, y, slope, stream=None):
    return _check("gsvk_leaky_relu", lib().gsvk_leaky_relu(dtype_code(x), _ptr(x), _ptr(y),
                                                           x.numel(), slope, _stream(stream)))


def resblock_add_lrelu(cur, t_b, t_in, slope, stream=None):
    return _check("gsvk_resblock_add_lrelu",
                  lib().gsvk_resblock_add_lrelu(dtype_code(cur), _ptr(cur), _ptr(t_b), _ptr(t_in),
                                                cur.numel(), slope, _stream(stream)))


def resblock_branch_mean(curs, tbs, out, apply_lrelu, slope, stream=None):
    nb = len(curs)
    c_arr = (_vp * nb)(*[_ptr(c) for c in curs])
    t_arr = (_vp * nb)(*[_ptr(t) for t in tbs]) if tbs is not None else None
    return _check("gsvk_resblock_branch_mean",
                  lib().gsvk_resblock_branch_mean(dtype_code(out), c_arr, t_arr, nb, _ptr(out),
                                                  out.numel(), int(apply_lrelu), slope,
                                                  _stream(stream)))


def scaled_add(acc, src, out, scale, stream=None):
    return _check("gsvk_scaled_add", lib().gsvk_scaled_add(dtype_code(out), _ptr(acc), _ptr(src),
                                                           _ptr(out), out.numel(), scale,
                                                           _stream(stream)))


def embed_pe(table, ids, pe, alpha, out, pos=None, pos0=0, mm=None, bias=None, err=None,
             stream=None):
    import torch
    vocab, D = table.shape
    max_pos = pe.shape[0]
    itype = I32 if ids.dtype == torch.int32 else I64
    return _check("gsvk_embed_pe",
                  lib().gsvk_embed_pe(dtype_code(out), dtype_code(table), itype, _ptr(table), vocab,
                                      _ptr(ids), _ptr(pos), pos0, _ptr(pe), max_pos, alpha,
                                      _ptr(mm), _ptr(bias), _ptr(out), ids.numel(), D, _ptr(err),
                                      _stream(stream)))


def pe_table(max_pos, D):
    """Host PE table [max_pos, D] float32 (numpy) from the library's builder."""
    import numpy as np
    out = np.empty((max_pos, D), dtype=np.float32)
    _check("gsvk_pe_table", lib().gsvk_pe_table(out.ctypes.data, max_pos, D))
    return out


# ---- T2S decode-step driver (include/gsvk_t2s.h) -----------------------------------------------

class T2SStepDesc(ctypes.Structure):
    _fields_ = [
        ("dtype", ctypes.c_int), ("batch", _sz), ("d_model", _sz), ("ffn", _sz), ("layers", _sz),
        ("eps", _d), ("audio_table", _vp), ("table_dtype", ctypes.c_int), ("vocab", _sz),
        ("ids", _vp), ("index_type", ctypes.c_int), ("pos", _vp), ("pe", _vp), ("max_pos", _sz),
        ("alpha", _f), ("err", _vp), ("x", _vp), ("h", _vp),
        ("attn_out", ctypes.POINTER(_vp)), ("bout", ctypes.POINTER(_vp)),
        ("n1g", ctypes.POINTER(_vp)), ("n1b", ctypes.POINTER(_vp)), ("ff", ctypes.POINTER(_vp)),
        ("b1", ctypes.POINTER(_vp)), ("ffn_out", ctypes.POINTER(_vp)), ("b2", ctypes.POINTER(_vp)),
        ("n2g", ctypes.POINTER(_vp)), ("n2b", ctypes.POINTER(_vp)),
    ]


class T2SStep:
    """Owns a gsvk_t2s_step (graph of one decode step's epilogue launches) over torch buffers."""

    def __init__(self, bufs, eps=1e-5, graph=True):
        import torch
        self.bufs = bufs  # keep tensors alive
        L = len(bufs["attn_out"])
        self._arrays = {}

        def arr(name):
            a = (_vp * L)(*[_ptr(t) for t in bufs[name]])
            self._arrays[name] = a
            return a

        d = T2SStepDesc()
        d.dtype = dtype_code(bufs["x"])
        d.batch, d.d_model = bufs["x"].shape
        d.ffn = bufs["ff"][0].shape[1]
        d.layers = L
        d.eps = eps
        d.audio_table = _ptr(bufs["table"])
        d.table_dtype = dtype_code(bufs["table"])
        d.vocab = bufs["table"].shape[0]
        d.ids = _ptr(bufs["ids"])
        d.index_type = I32 if bufs["ids"].dtype == torch.int32 else I64
        d.pos = _ptr(bufs["pos"])
        d.pe = _ptr(bufs["pe"])
        d.max_pos = bufs["pe"].shape[0]
        d.alpha = bufs["alpha"]
        d.err = _ptr(bufs.get("err"))
        d.x = _ptr(bufs["x"])
        d.h = _ptr(bufs["h"])
        for name in ("attn_out", "bout", "n1g", "n1b", "ff", "b1", "ffn_out", "b2", "n2g", "n2b"):
            setattr(d, name, ctypes.cast(arr(name), ctypes.POINTER(_vp)))
        self.desc = d
        self.handle = None
        if graph:
            h = _vp()
            _check("gsvk_t2s_step_create", lib().gsvk_t2s_step_create(ctypes.byref(d),
                                                                      ctypes.byref(h)))
            self.handle = h

    @property
    def launches(self):
        return lib().gsvk_t2s_step_launches(self.handle) if self.handle else 1 + 3 * self.desc.layers

    def run(self, stream=None):
        if self.handle:
            return _check("gsvk_t2s_step_run", lib().gsvk_t2s_step_run(self.handle,
                                                                       _stream(stream)))
        return _check("gsvk_t2s_step_eager", lib().gsvk_t2s_step_eager(ctypes.byref(self.desc),
                                                                       _stream(stream)))

    def close(self):
        if self.handle:
            lib().gsvk_t2s_step_destroy(self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


# ---- whole T2S decode step (gsvk_t2s_decode_*) -------------------------------------------------

class T2SLayer(ctypes.Structure):
    _fields_ = [(n, _vp) for n in ("wqkv", "bqkv", "wout", "bout", "n1g", "n1b", "w1", "b1", "w2",
                                   "b2", "n2g", "n2b", "k_cache", "v_cache")]


class T2SDecodeDesc(ctypes.Structure):
    _fields_ = [
        ("dtype", ctypes.c_int), ("kv_dtype", ctypes.c_int), ("batch", _sz), ("d_model", _sz),
        ("heads", _sz), ("ffn", _sz), ("layers", _sz), ("max_len", _sz), ("len_bound", _sz),
        ("eps", _d), ("audio_table", _vp), ("table_dtype", ctypes.c_int), ("vocab", _sz),
        ("ids", _vp), ("index_type", ctypes.c_int), ("pos", _vp), ("kv_pos", _vp), ("pe", _vp),
        ("max_pos", _sz), ("alpha", _f), ("err", _vp), ("layer", ctypes.POINTER(T2SLayer)),
        ("w_logits", _vp), ("logits", _vp), ("x", _vp), ("h", _vp), ("z", _vp), ("attn", _vp),
        ("ff", _vp), ("qkv", _vp), ("workspace", _vp), ("workspace_bytes", _sz),
    ]


class T2SDecode:
    """One whole decode step (embedding, every layer's GEMVs / attention / LayerNorms, logits)
    over torch buffers; recorded into a graph unless graph=False. `m` holds the model tensors:
    table, pe, alpha, heads, layers (list of dicts with the gsvk_t2s_layer names), w_logits (or
    None); `io` holds ids, pos, kv_pos, err and the activations x, h, z, attn, ff, qkv, logits."""

    def __init__(self, m, io, eps=1e-5, len_bound=0, graph=True):
        import torch
        self.m, self.io = m, io
        layers = m["layers"]
        L = len(layers)
        self._layers = (T2SLayer * L)()
        for i, ly in enumerate(layers):
            for name, _ in T2SLayer._fields_:
                setattr(self._layers[i], name, _ptr(ly.get(name)))
        B, D = io["x"].shape
        k0 = layers[0]["k_cache"]
        d = T2SDecodeDesc()
        d.dtype = dtype_code(io["x"])
        d.kv_dtype = dtype_code(k0)
        d.batch, d.d_model, d.heads, d.ffn, d.layers = B, D, m["heads"], io["ff"].shape[1], L
        d.max_len = k0.shape[1]
        d.len_bound = len_bound
        d.eps = eps
        d.audio_table = _ptr(m["table"])
        d.table_dtype = dtype_code(m["table"])
        d.vocab = m["table"].shape[0]
        d.ids = _ptr(io["ids"])
        d.index_type = I32 if io["ids"].dtype == torch.int32 else I64
        d.pos, d.kv_pos = _ptr(io["pos"]), _ptr(io["kv_pos"])
        d.pe, d.max_pos, d.alpha = _ptr(m["pe"]), m["pe"].shape[0], m["alpha"]
        d.err = _ptr(io.get("err"))
        d.layer = ctypes.cast(self._layers, ctypes.POINTER(T2SLayer))
        d.w_logits = _ptr(m.get("w_logits"))
        d.logits = _ptr(io.get("logits"))
        for name in ("x", "h", "z", "attn", "ff", "qkv"):
            setattr(d, name, _ptr(io[name]))
        need = lib().gsvk_decode_attention_workspace_bytes(B, m["heads"], D // m["heads"],
                                                           len_bound or d.max_len)
        if need:
            ws = workspace(io["x"].device, need)
            d.workspace, d.workspace_bytes = ws.data_ptr(), ws.numel()
        self.desc = d
        self.handle = None
        if graph:
            h = _vp()
            _check("gsvk_t2s_decode_create",
                   lib().gsvk_t2s_decode_create(ctypes.byref(d), ctypes.byref(h)))
            self.handle = h

    @property
    def launches(self):
        return lib().gsvk_t2s_step_launches(self.handle) if self.handle else 0

    def run(self, stream=None):
        if self.handle:
            return _check("gsvk_t2s_step_run", lib().gsvk_t2s_step_run(self.handle,
                                                                       _stream(stream)))
        return _check("gsvk_t2s_decode_eager",
                      lib().gsvk_t2s_decode_eager(ctypes.byref(self.desc), _stream(stream)))

    def close(self):
        if self.handle:
            lib().gsvk_t2s_step_destroy(self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass
