"""ctypes binding of libgsvk.so, the C ABI declared in include/gsvk.h, gsvk_t2s.h, gsvk_gsv.h and
gsvk_sovits.h.

The library is the product; this module only marshals arguments. Device buffers are passed as
torch tensors (for their data pointers and strides) or as raw integer addresses. Every call checks
the returned status and raises GsvkError on anything but GSVK_OK. There is no fallback: if
libgsvk.so is missing or cannot be loaded, `lib()` raises.
"""
import ctypes
import os

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libgsvk.so")
# tests/sanitizers.sh points this at the host-sanitizer build (gpt-sovits-native_amd/_san/)
LIB_PATH = os.environ.get("GSVK_LIB", LIB_PATH)

F32, F16, BF16 = 0, 1, 2
I64, I32 = 0, 1
ACT_NONE, ACT_RELU, ACT_GELU_ERF, ACT_LEAKY_RELU = 0, 1, 2, 3
OK, E_NULL, E_SIZE, E_DTYPE, E_ALIAS, E_ARG, E_HIP, E_FORMAT, E_IO = 0, -1, -2, -3, -4, -5, -6, -7, -8
CONV_EPI_BIAS, CONV_EPI_LRELU, CONV_EPI_RES_LRELU, CONV_EPI_RES, CONV_EPI_DUAL, CONV_EPI_TANH = \
    0, 1, 2, 3, 4, 5
CONV_X_LRELU = 0x100  # OR-ed into epi: the convolution reads lrelu(x, slope)

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
    "gsvk_gemv_f16w_ln": (_i, [_i, _i, _vp, _sz, _vp, _vp, _d, _vp, _sz, _vp, _vp, _i, _f, _vp, _i,
                               _vp, _sz, _sz, _sz, _sz, _vp]),
    "gsvk_decode_attention": (_i, [_i, _i, _vp, _sz, _vp, _vp, _sz, _vp, _vp, _sz, _sz, _sz, _sz,
                                   _sz, _vp, _sz, _vp, _vp]),
    "gsvk_decode_attention_workspace_bytes": (_sz, [_sz, _sz, _sz, _sz]),
    "gsvk_t2s_prefill_input": (_i, [_i, _i, _i, _vp, _sz, _vp, _sz, _vp, _vp, _f, _vp, _sz, _vp,
                                    _sz, _f, _vp, _sz, _vp, _sz, _vp, _vp]),
    "gsvk_decode_attention_noalloc": (_i, [_i, _i, _vp, _sz, _vp, _vp, _sz, _vp, _vp, _sz, _sz, _sz,
                                           _sz, _sz, _vp, _vp]),
    "gsvk_conv1d": (_i, [_i, _i, _vp, _sz, _vp, _vp, _i, _f, _vp, _vp, _sz, _vp, _sz, _sz, _sz, _sz,
                         _sz, _sz, _vp]),
    "gsvk_conv1d_packed_elems": (_sz, [_sz, _sz, _sz]),
    "gsvk_conv1d_pack": (_i, [_vp, _sz, _sz, _sz, _vp, _sz, _vp]),
    "gsvk_convt1d": (_i, [_i, _i, _vp, _sz, _vp, _vp, _i, _f, _vp, _vp, _sz, _vp, _sz, _sz, _sz, _sz,
                          _sz, _sz, _vp]),
    "gsvk_convt1d_packed_elems": (_sz, [_sz, _sz, _sz, _sz]),
    "gsvk_convt1d_pack": (_i, [_vp, _sz, _sz, _sz, _sz, _vp, _sz, _vp]),
    "gsvk_groupnorm_gelu": (_i, [_i, _vp, _vp, _vp, _vp, _sz, _sz, _sz, _d, _i, _vp]),
    "gsvk_leaky_relu": (_i, [_i, _vp, _vp, _sz, _f, _vp]),
    "gsvk_resblock_add_lrelu": (_i, [_i, _vp, _vp, _vp, _sz, _f, _vp]),
    "gsvk_resblock_branch_mean": (_i, [_i, ctypes.POINTER(_vp), ctypes.POINTER(_vp), _i, _vp, _sz,
                                       _i, _f, _vp]),
    "gsvk_scaled_add": (_i, [_i, _vp, _vp, _vp, _sz, _f, _vp]),
    "gsvk_f32_to_f16": (_i, [_vp, _vp, _sz, _vp]),
    "gsvk_embed_pe": (_i, [_i, _i, _i, _vp, _sz, _vp, _vp, _i64, _vp, _sz, _f, _vp, _vp, _vp, _sz,
                           _sz, _vp, _vp]),
    "gsvk_pe_table": (_i, [_vp, _sz, _sz]),
    "gsvk_pe_row": (_i, [_vp, _sz, _sz]),
    "gsvk_t2s_step_eager": (_i, [_vp, _vp]),
    "gsvk_t2s_step_create": (_i, [_vp, ctypes.POINTER(_vp)]),
    "gsvk_t2s_step_run": (_i, [_vp, _vp]),
    "gsvk_t2s_step_launches": (_i, [_vp]),
    "gsvk_t2s_step_destroy": (None, [_vp]),
    "gsvk_t2s_step_fused": (_i, [_vp, _vp]),
    "gsvk_t2s_step_create_fused": (_i, [_vp, ctypes.POINTER(_vp)]),
    "gsvk_t2s_decode_eager": (_i, [_vp, _vp]),
    "gsvk_gsv_open": (_i, [ctypes.c_char_p, ctypes.POINTER(_vp)]),
    "gsvk_gsv_open_memory": (_i, [_vp, _sz, ctypes.POINTER(_vp)]),
    "gsvk_gsv_close": (None, [_vp]),
    "gsvk_gsv_header": (_i, [_vp, ctypes.POINTER(ctypes.c_uint32), ctypes.POINTER(ctypes.c_uint32),
                             ctypes.POINTER(_vp), ctypes.POINTER(_sz), ctypes.POINTER(_vp),
                             ctypes.POINTER(_sz), ctypes.POINTER(ctypes.c_uint32)]),
    "gsvk_gsv_tensor_at": (_i, [_vp, _sz, _vp]),
    "gsvk_gsv_find": (ctypes.c_long, [_vp, ctypes.c_char_p]),
    "gsvk_gsv_arena": (_i, [_vp, _i, ctypes.POINTER(ctypes.c_uint64),
                            ctypes.POINTER(ctypes.c_uint64)]),
    "gsvk_gsv_upload": (_i, [_vp, _i, _vp, _sz, _vp]),
    "gsvk_gsv_device_ptr": (_vp, [_vp, _i, _vp, _sz]),
    "gsvk_t2s_decode_create": (_i, [_vp, ctypes.POINTER(_vp)]),
    "gsvk_t2s_decode_workspace_bytes": (_sz, [_sz, _sz, _sz, _sz]),
    "gsvk_sovits_decoder_workspace_bytes": (_sz, [_vp]),
    "gsvk_sovits_decoder_eager": (_i, [_vp, _vp]),
    "gsvk_sovits_decoder_create": (_i, [_vp, ctypes.POINTER(_vp)]),
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


def gemv_f16w_ln(z, gamma, beta, eps, h, w, y, bias=None, act=ACT_NONE, slope=0.0, residual=None,
                 round_x=True, stream=None):
    """h[r] = LN(z[r]) (gamma / beta may be None) and y[r] = act(w @ h[r] + bias) (+ residual[r]) in
    one launch; z, h [rows, in] of one dtype, y / residual [rows, out] sharing y's row stride."""
    rows, n_in, ldz = _rows(z)
    _, _, ldh = _rows(h)
    n_out = w.shape[0]
    _, _, ldy = _rows(y)
    assert residual is None or residual.data_ptr() == y.data_ptr() or _rows(residual)[2] == ldy, \
        "residual shares y's row stride"
    return _check("gsvk_gemv_f16w_ln",
                  lib().gsvk_gemv_f16w_ln(dtype_code(z), int(round_x), _ptr(z), ldz, _ptr(gamma),
                                          _ptr(beta), float(eps), _ptr(h), ldh, _ptr(w), _ptr(bias),
                                          act, slope, _ptr(residual), dtype_code(y), _ptr(y), ldy,
                                          rows, n_out, n_in, _stream(stream)))


def conv1d_pack(w, stream=None):
    """Pack a [c_out, c_in, k] fp16 filter bank on its device; returns the packed uint16 tensor."""
    import torch
    c_out, c_in, k = w.shape
    assert w.dtype in (torch.float16, torch.int16) and w.is_contiguous()
    n = lib().gsvk_conv1d_packed_elems(c_out, c_in, k)
    wp = torch.empty(n, dtype=torch.int16, device=w.device)
    _check("gsvk_conv1d_pack", lib().gsvk_conv1d_pack(_ptr(w), c_out, c_in, k, _ptr(wp), n,
                                                      _stream(stream)))
    return wp


def conv1d(x, wp, c_out, k, y=None, bias=None, dilation=1, epi=CONV_EPI_BIAS, slope=0.1, cur=None,
           round_x=False, stream=None, check=True, res=None):
    """SoVITS Conv1d on channel-major x [c_in, T] with packed weights (conv1d_pack) and a fused
    epilogue (CONV_EPI_*); y / cur / res [c_out, T] of x's dtype (res: the residual source of the
    RES epilogues when it is not cur itself; it shares cur's row stride)."""
    c_in, T, ldx = _rows(x)
    ldy = _rows(y)[2] if y is not None else 0
    ldc = _rows(cur)[2] if cur is not None else 0
    rc = lib().gsvk_conv1d(dtype_code(x), int(round_x), _ptr(x), ldx, _ptr(wp), _ptr(bias), epi,
                           slope, _ptr(cur), _ptr(res), ldc, _ptr(y), ldy, c_in, c_out, T, k,
                           dilation, _stream(stream))
    return _check("gsvk_conv1d", rc) if check else rc


class Conv1d:
    """Mirror of the reference's sovits::Conv1d (conv1d.hpp:56-203): out_c, in_c, k, dilation, the
    fp16 weights packed once at load, fp32 bias (zeros when absent), forward(x, y)."""

    def __init__(self, w16, bias=None, dilation=1, stream=None):
        import torch
        self.out_c, self.in_c, self.k = (int(d) for d in w16.shape)
        self.dilation = int(dilation)
        self.wp = conv1d_pack(w16.contiguous(), stream)
        self.b = bias if bias is not None else torch.zeros(self.out_c, dtype=torch.float32,
                                                           device=w16.device)

    def forward(self, x, y=None, epi=CONV_EPI_BIAS, slope=0.1, cur=None, round_x=False,
                stream=None, res=None):
        import torch
        if y is None and (epi & ~CONV_X_LRELU) != CONV_EPI_RES:
            y = torch.empty(self.out_c, x.shape[1], dtype=x.dtype, device=x.device)
        conv1d(x, self.wp, self.out_c, self.k, y, self.b, self.dilation, epi, slope, cur, round_x,
               stream, res=res)
        return y


def convt1d_pack(w, stride, stream=None):
    """Pack a [c_in, c_out, k] fp16 ConvTranspose1d filter bank; returns the packed tensor."""
    import torch
    c_in, c_out, k = w.shape
    assert w.dtype in (torch.float16, torch.int16) and w.is_contiguous()
    n = lib().gsvk_convt1d_packed_elems(c_out, c_in, k, stride)
    wp = torch.empty(max(n, 1), dtype=torch.int16, device=w.device)
    _check("gsvk_convt1d_pack", lib().gsvk_convt1d_pack(_ptr(w), c_out, c_in, k, stride, _ptr(wp),
                                                        n, _stream(stream)))
    return wp


def convt1d(x, wp, c_out, k, stride, y=None, bias=None, epi=CONV_EPI_BIAS, slope=0.1, cur=None,
            round_x=False, stream=None, check=True, res=None):
    """SoVITS ConvTranspose1d on x [c_in, T] with packed weights (convt1d_pack) and a fused
    epilogue; y / cur / res [c_out, T * stride]."""
    c_in, T, ldx = _rows(x)
    ldy = _rows(y)[2] if y is not None else 0
    ldc = _rows(cur)[2] if cur is not None else 0
    rc = lib().gsvk_convt1d(dtype_code(x), int(round_x), _ptr(x), ldx, _ptr(wp), _ptr(bias), epi,
                            slope, _ptr(cur), _ptr(res), ldc, _ptr(y), ldy, c_in, c_out, T, k,
                            stride, _stream(stream))
    return _check("gsvk_convt1d", rc) if check else rc


class ConvT1d:
    """Mirror of the reference's sovits::ConvT1d (conv1d.hpp:205-360): out_c, in_c, k, stride_u,
    the torch-layout [in, out, k] fp16 weights packed once per phase, fp32 bias (zeros when
    absent), forward(x, y) with y of length T * stride_u."""

    def __init__(self, w16, bias, stride, stream=None):
        import torch
        self.in_c, self.out_c, self.k = (int(d) for d in w16.shape)
        self.stride_u = int(stride)
        self.wp = convt1d_pack(w16.contiguous(), self.stride_u, stream)
        self.b = bias if bias is not None else torch.zeros(self.out_c, dtype=torch.float32,
                                                           device=w16.device)

    def forward(self, x, y=None, epi=CONV_EPI_BIAS, slope=0.1, cur=None, round_x=False,
                stream=None, res=None):
        import torch
        if y is None and (epi & ~CONV_X_LRELU) != CONV_EPI_RES:
            y = torch.empty(self.out_c, x.shape[1] * self.stride_u, dtype=x.dtype, device=x.device)
        convt1d(x, self.wp, self.out_c, self.k, self.stride_u, y, self.b, epi, slope, cur, round_x,
                stream, res=res)
        return y


class ResBlock1:
    """Mirror of the reference's sovits ResBlock1 (dec.hpp:18-43): convs1 with dilations 1 / 3 / 5
    and convs2 with dilation 1, all of kernel size k, as device Conv1d objects."""

    def __init__(self, w1, b1, w2, b2, dilations=(1, 3, 5)):
        self.convs1 = [Conv1d(w, b, d) for w, b, d in zip(w1, b1, dilations)]
        self.convs2 = [Conv1d(w, b, 1) for w, b in zip(w2, b2)]


class GeneratorStage:
    """One stage of the reference's Generator::forward (dec.hpp:283-336) on the GPU, with every
    element-wise pass fused into a neighbouring kernel:
      y = ups(x)                                  x arrives already LeakyReLU'd (the previous
                                                  stage's branch mean, dec.hpp:284)
      for each ResBlock j: cur_j = y; for each pair m:
          t_a = lrelu(convs1[m](lrelu(cur_j)))    leaky_relu_write (dec.hpp:322) applied as the
                                                  conv reads its input (CONV_X_LRELU), the
                                                  leaky_relu_io after it (dec.hpp:323-324) in its
                                                  store: no t_in tensor
          cur_j += convs2[m](t_a)                 conv + add_inplace (dec.hpp:325-326); the first
                                                  pair reads y as its residual and writes cur_j:
                                                  no copy of y
      out = lrelu(mean_j cur_j, slope_next)       mul_write / add_scaled_inplace + the next stage's
                                                  leaky_relu_io (dec.hpp:328-336, 284 or 342)
    Launches: 1 upsampler, 18 convolutions, 1 branch mean. ResBlocks after the first run on side
    streams of their own (each with its own t_a), forked after the upsampler and joined back before
    the branch mean, as in gsvk_sovits_decoder_*."""

    def __init__(self, ups, resblocks):
        self.ups = ups
        self.resblocks = resblocks
        self._buf = None
        self._side = None

    def _buffers(self, C, T, dtype, device):
        import torch
        key = (C, T, dtype, device)
        if self._buf is None or self._buf[0] != key:
            mk = lambda: torch.empty(C, T, dtype=dtype, device=device)
            self._buf = (key, mk(), [mk() for _ in self.resblocks], [mk() for _ in self.resblocks])
        return self._buf[1:]

    def _side_streams(self, device):
        import torch
        if self._side is None or self._side[0] != device:
            self._side = (device, [torch.cuda.Stream(device=device)
                                   for _ in self.resblocks[1:]])
        return self._side[1]

    def forward(self, x, out, slope_next=0.1, round_x=False, stream=None):
        import torch
        y, tas, curs = self._buffers(self.ups.out_c, x.shape[1] * self.ups.stride_u, x.dtype,
                                     x.device)
        main = stream if stream is not None else torch.cuda.current_stream(x.device)
        if isinstance(main, int):
            main = torch.cuda.ExternalStream(main, device=x.device)
        self.ups.forward(x, y, round_x=round_x, stream=main)
        sides = self._side_streams(x.device)
        for sd in sides:
            sd.wait_stream(main)  # the upsampler's y before any branch reads it
        for j, (rb, t_a, cur) in enumerate(zip(self.resblocks, tas, curs)):
            st = main if j == 0 else sides[j - 1]
            src, res = y, y
            for c1, c2 in zip(rb.convs1, rb.convs2):
                c1.forward(src, t_a, epi=CONV_EPI_LRELU | CONV_X_LRELU, slope=0.1, round_x=round_x,
                           stream=st)
                c2.forward(t_a, None, epi=CONV_EPI_RES, cur=cur, res=res, round_x=round_x,
                           stream=st)
                src, res = cur, None
        for sd in sides:
            main.wait_stream(sd)  # every branch before the mean
        resblock_branch_mean(curs, None, out, True, slope_next, stream=main)
        return out


class SovitsStage(ctypes.Structure):
    """gsvk_sovits_stage: one upsampler and its three ResBlock1s (packed weights, fp32 biases)."""
    _fields_ = [
        ("c_in", _sz), ("c_out", _sz), ("ups_k", _sz), ("ups_u", _sz), ("ups_w", _vp),
        ("ups_b", _vp), ("res_k", _sz * 3), ("res_dil", _sz * 3), ("w1", (_vp * 3) * 3),
        ("b1", (_vp * 3) * 3), ("w2", (_vp * 3) * 3), ("b2", (_vp * 3) * 3),
    ]


class SovitsDecoderDesc(ctypes.Structure):
    _fields_ = [
        ("dtype", ctypes.c_int), ("round_x", ctypes.c_int), ("frames", _sz), ("c_z", _sz),
        ("c0", _sz), ("pre_k", _sz), ("pre_w", _vp), ("pre_b", _vp), ("g_in", _sz),
        ("cond_w", _vp), ("cond_b", _vp), ("n_stages", _sz),
        ("stage", ctypes.POINTER(SovitsStage)), ("post_k", _sz), ("post_w", _vp), ("z", _vp),
        ("ge", _vp), ("out", _vp), ("workspace", _vp), ("workspace_bytes", _sz),
    ]


class SovitsDecoder:
    """The whole SoVITS decoder (Generator::forward, dec.hpp:264-345) over one set of device
    buffers: conv_pre (+ cond(ge) folded into its bias) and LeakyReLU, the GeneratorStages, the final
    LeakyReLU(0.01), conv_post and tanh, as gsvk_sovits_decoder_* launches (a HIP graph unless
    graph=False; either way each stage's three ResBlocks run concurrently: graph branches, or the
    library's two side streams joined back into the caller's). conv_pre / conv_post are Conv1d, stages GeneratorStage objects, cond a pair
    (w16 [c0, g_in] fp16, bias [c0] fp32) or None; z [c_z, frames] fp32 or fp16 (the activation
    dtype), ge [g_in] fp32 (one frame; None without cond), out [frames * prod(u)] of z's dtype.
    The workspace is this object's own device allocation."""

    def __init__(self, conv_pre, cond, stages, conv_post, z, ge, out, round_x=False, graph=True):
        import torch
        self._keep = (conv_pre, cond, stages, conv_post, z, ge, out)
        n = len(stages)
        self._stages = (SovitsStage * n)()
        for i, st in enumerate(stages):
            S = self._stages[i]
            S.c_in, S.c_out = st.ups.in_c, st.ups.out_c
            S.ups_k, S.ups_u = st.ups.k, st.ups.stride_u
            S.ups_w, S.ups_b = _ptr(st.ups.wp), _ptr(st.ups.b)
            for j, rb in enumerate(st.resblocks):
                S.res_k[j] = rb.convs1[0].k
                for m in range(3):
                    S.res_dil[m] = rb.convs1[m].dilation
                    S.w1[j][m], S.b1[j][m] = _ptr(rb.convs1[m].wp), _ptr(rb.convs1[m].b)
                    S.w2[j][m], S.b2[j][m] = _ptr(rb.convs2[m].wp), _ptr(rb.convs2[m].b)
        d = SovitsDecoderDesc()
        d.dtype, d.round_x = dtype_code(z), int(round_x)
        d.c_z, d.frames = z.shape
        d.c0, d.pre_k = conv_pre.out_c, conv_pre.k
        d.pre_w, d.pre_b = _ptr(conv_pre.wp), _ptr(conv_pre.b)
        if cond is not None:
            w_cond, b_cond = cond
            assert ge.dtype == torch.float32, "ge is fp32 for either activation dtype"
            assert w_cond.shape == (conv_pre.out_c, ge.numel()) and w_cond.is_contiguous()
            d.g_in, d.cond_w, d.cond_b = w_cond.shape[1], _ptr(w_cond), _ptr(b_cond)
            d.ge = _ptr(ge)
        d.n_stages = n
        d.stage = ctypes.cast(self._stages, ctypes.POINTER(SovitsStage))
        d.post_k, d.post_w = conv_post.k, _ptr(conv_post.wp)
        d.z, d.out = _ptr(z), _ptr(out)
        need = lib().gsvk_sovits_decoder_workspace_bytes(ctypes.byref(d))
        if need == 0:
            raise GsvkError("gsvk_sovits_decoder_workspace_bytes", E_SIZE)
        self.ws = torch.empty(need, dtype=torch.uint8, device=z.device)
        d.workspace, d.workspace_bytes = self.ws.data_ptr(), need
        self.desc = d
        self.handle = None
        if graph:
            h = _vp()
            _check("gsvk_sovits_decoder_create",
                   lib().gsvk_sovits_decoder_create(ctypes.byref(d), ctypes.byref(h)))
            self.handle = h

    @property
    def launches(self):
        return lib().gsvk_t2s_step_launches(self.handle) if self.handle else 0

    def run(self, stream=None):
        if self.handle:
            return _check("gsvk_t2s_step_run", lib().gsvk_t2s_step_run(self.handle,
                                                                       _stream(stream)))
        return _check("gsvk_sovits_decoder_eager",
                      lib().gsvk_sovits_decoder_eager(ctypes.byref(self.desc), _stream(stream)))

    def close(self):
        if self.handle:
            lib().gsvk_t2s_step_destroy(self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


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


def decode_attention_noalloc(qkv, k_cache, v_cache, pos, out, heads, len_bound=0, err=None,
                             stream=None):
    """decode_attention with the chunk states in the library's own device array (no workspace)."""
    B = qkv.shape[0]
    D = out.shape[-1]
    return _check("gsvk_decode_attention_noalloc",
                  lib().gsvk_decode_attention_noalloc(
                      dtype_code(k_cache), dtype_code(out), _ptr(qkv), _rows(qkv)[2],
                      _ptr(k_cache), _ptr(v_cache), k_cache.shape[1], _ptr(pos), _ptr(out),
                      _rows(out)[2], B, heads, D // heads, len_bound, _ptr(err), _stream(stream)))


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


def f32_to_f16(x, y=None, stream=None):
    """fp16 copy of an fp32 device tensor, round to nearest even (kern::f32_to_f16)."""
    import torch
    if y is None:
        y = torch.empty(x.shape, dtype=torch.float16, device=x.device)
    _check("gsvk_f32_to_f16", lib().gsvk_f32_to_f16(_ptr(x), _ptr(y), x.numel(), _stream(stream)))
    return y


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


def t2s_prefill_input(text_table, phones, alpha_text, audio_table, prompt, alpha_audio, pe, xy,
                      mm=None, bias=None, err=None, stream=None):
    """xy [T + P, D]: the text rows (phones, positions 0..T-1, optional bert_proj rows mm and bias)
    then the prompt rows (prompt ids, positions 0..P-1), one launch."""
    import torch
    T, P = phones.numel(), prompt.numel()
    D = xy.shape[1]
    assert xy.shape[0] == T + P and phones.dtype == prompt.dtype
    itype = I32 if phones.dtype == torch.int32 else I64
    return _check("gsvk_t2s_prefill_input",
                  lib().gsvk_t2s_prefill_input(
                      dtype_code(xy), dtype_code(text_table), itype, _ptr(text_table),
                      text_table.shape[0], _ptr(phones), T, _ptr(mm), _ptr(bias), alpha_text,
                      _ptr(audio_table), audio_table.shape[0], _ptr(prompt), P, alpha_audio,
                      _ptr(pe), pe.shape[0], _ptr(xy), D, _ptr(err), _stream(stream)))


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
    """Owns a gsvk_t2s_step (graph of one decode step's epilogue launches) over torch buffers.
    fused=True: the whole step as one kernel launch (gsvk_t2s_step_fused): the gather and ff
    bitwise the same, h and x within the LayerNorm tolerance (one-pass statistics)."""

    def __init__(self, bufs, eps=1e-5, graph=True, fused=False):
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
        self.fused = fused
        if graph:
            h = _vp()
            create = "gsvk_t2s_step_create_fused" if fused else "gsvk_t2s_step_create"
            _check(create, getattr(lib(), create)(ctypes.byref(d), ctypes.byref(h)))
            self.handle = h

    @property
    def launches(self):
        if self.handle:
            return lib().gsvk_t2s_step_launches(self.handle)
        return 1 if self.fused else 1 + 3 * self.desc.layers

    def run(self, stream=None):
        if self.handle:
            return _check("gsvk_t2s_step_run", lib().gsvk_t2s_step_run(self.handle,
                                                                       _stream(stream)))
        fn = "gsvk_t2s_step_fused" if self.fused else "gsvk_t2s_step_eager"
        return _check(fn, getattr(lib(), fn)(ctypes.byref(self.desc), _stream(stream)))

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
        ("parts", ctypes.c_int),
    ]


class T2SDecode:
    """One whole decode step (embedding, every layer's GEMVs / attention / LayerNorms, logits)
    over torch buffers; recorded into a graph unless graph=False. `m` holds the model tensors:
    table, pe, alpha, heads, layers (list of dicts with the gsvk_t2s_layer names), w_logits (or
    None); `io` holds ids, pos, kv_pos, err and the activations x, h, z, attn, ff, qkv, logits.
    split=False runs a batch of 32 or more as one chain of launches instead of two concurrent
    halves (desc.parts = 1)."""

    def __init__(self, m, io, eps=1e-5, len_bound=0, graph=True, split=True):
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
        d.parts = 0 if split else 1
        need = lib().gsvk_t2s_decode_workspace_bytes(B, m["heads"], D // m["heads"],
                                                     len_bound or d.max_len)
        self._ws = None
        if need:
            # A workspace of its own: the recorded graph keeps its address, and the shared scratch
            # of workspace() is replaced (freed) when a later call needs a larger one.
            self._ws = ws = torch.empty(need, dtype=torch.uint8, device=io["x"].device)
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


# ---- .gsv container (include/gsvk_gsv.h) ------------------------------------------------------

class GsvTensorInfo(ctypes.Structure):
    _fields_ = [("name", _vp), ("name_len", _sz), ("rank", ctypes.c_uint32),
                ("dims", ctypes.c_uint32 * 8), ("numel", ctypes.c_uint64),
                ("src_dtype", ctypes.c_int), ("f32_offset", ctypes.c_uint64),
                ("f32_nbytes", ctypes.c_uint64), ("f16_offset", ctypes.c_uint64),
                ("f16_nbytes", ctypes.c_uint64)]


class GsvFile:
    """A validated .gsv file (gsvk_gsv_open). `tensors` maps name -> info dict; `config` is the
    parsed JSON (a file whose JSON does not parse is rejected, as GsvFile's constructor does,
    gsv_loader.cpp:145-150); `upload(kind)` copies the fp16 (F16) or fp32 (F32) segments to one
    device arena and returns {name: tensor view} for the tensors that have that segment."""

    def __init__(self, path=None, data=None):
        import json
        h = _vp()
        if data is not None:
            self._buf = ctypes.create_string_buffer(bytes(data), len(data))
            rc = lib().gsvk_gsv_open_memory(ctypes.cast(self._buf, _vp), len(data), ctypes.byref(h))
        else:
            rc = lib().gsvk_gsv_open(os.fsencode(path), ctypes.byref(h))
        _check("gsvk_gsv_open", rc)
        self.handle = h
        ver, flags, n = ctypes.c_uint32(), ctypes.c_uint32(), ctypes.c_uint32()
        nm, nml, cf, cfl = _vp(), _sz(), _vp(), _sz()
        _check("gsvk_gsv_header", lib().gsvk_gsv_header(h, ctypes.byref(ver), ctypes.byref(flags),
                                                        ctypes.byref(nm), ctypes.byref(nml),
                                                        ctypes.byref(cf), ctypes.byref(cfl),
                                                        ctypes.byref(n)))
        self.version, self.flags, self.n_tensors = ver.value, flags.value, n.value
        self.name = ctypes.string_at(nm.value, nml.value).decode() if nml.value else ""
        raw = ctypes.string_at(cf.value, cfl.value) if cfl.value else b""
        try:
            self.config = json.loads(raw.decode()) if raw else None
        except ValueError as exc:
            self.close()
            raise GsvkError("gsvk_gsv_open: config JSON", E_FORMAT) from exc
        self.tensors = {}
        self._index = {}
        for i in range(self.n_tensors):
            t = GsvTensorInfo()
            _check("gsvk_gsv_tensor_at", lib().gsvk_gsv_tensor_at(h, i, ctypes.byref(t)))
            name = ctypes.string_at(t.name, t.name_len).decode()
            self.tensors[name] = dict(dims=tuple(t.dims[:t.rank]), numel=t.numel,
                                      src_dtype=t.src_dtype, f32_offset=t.f32_offset,
                                      f32_nbytes=t.f32_nbytes, f16_offset=t.f16_offset,
                                      f16_nbytes=t.f16_nbytes)
            self._index[name] = i

    def arena_bytes(self, kind):
        base, nb = ctypes.c_uint64(), ctypes.c_uint64()
        _check("gsvk_gsv_arena", lib().gsvk_gsv_arena(self.handle, kind, ctypes.byref(base),
                                                      ctypes.byref(nb)))
        return nb.value

    def upload(self, kind, device="cuda", stream=None):
        import torch
        nb = self.arena_bytes(kind)
        arena = torch.empty(max(nb, 1), dtype=torch.uint8, device=device)
        _check("gsvk_gsv_upload", lib().gsvk_gsv_upload(self.handle, kind, arena.data_ptr(),
                                                        arena.numel(), _stream(stream)))
        tdt = torch.float16 if kind == F16 else torch.float32
        esz = 2 if kind == F16 else 4
        views = {}
        for name, i in self._index.items():
            ptr = lib().gsvk_gsv_device_ptr(self.handle, kind, arena.data_ptr(), i)
            if not ptr:
                continue
            off = ptr - arena.data_ptr()
            n = self.tensors[name]["numel"]
            views[name] = arena[off:off + n * esz].view(tdt).view(*self.tensors[name]["dims"])
        return arena, views

    def close(self):
        if getattr(self, "handle", None):
            lib().gsvk_gsv_close(self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


def t2s_model_from_gsv(g, dev="cuda", stream=None):
    """The decode step's model tensors (T2SDecode's `m`) from an ar_s1 .gsv, by the names
    T2SEngine's loader reads (t2s_engine.cpp:575-627): fp16 copies for the GEMV weights and the
    audio embedding table, fp32 for biases, LayerNorm parameters and alpha. Caches are the
    caller's. Returns (m, arenas)."""
    a16, t16 = g.upload(F16, dev, stream)
    a32, t32 = g.upload(F32, dev, stream)
    mc = (g.config or {}).get("model_config") or {}
    mm = mc.get("model", {})
    n_layer, heads = int(mm["n_layer"]), int(mm["head"])
    layers = []
    for l in range(n_layer):
        p, ps = f"h.layers.{l}.", f"h.layers.{l}.self_attn."
        layers.append(dict(wqkv=t16[ps + "in_proj_weight"], bqkv=t32[ps + "in_proj_bias"],
                           wout=t16[ps + "out_proj.weight"], bout=t32[ps + "out_proj.bias"],
                           n1g=t32[p + "norm1.weight"], n1b=t32[p + "norm1.bias"],
                           w1=t16[p + "linear1.weight"], b1=t32[p + "linear1.bias"],
                           w2=t16[p + "linear2.weight"], b2=t32[p + "linear2.bias"],
                           n2g=t32[p + "norm2.weight"], n2b=t32[p + "norm2.bias"]))
    import torch
    alpha = float(t32["ar_audio_position.alpha"].reshape(-1)[0].item())
    m = dict(table=t16["ar_audio_embedding.word_embeddings.weight"], heads=heads, layers=layers,
             w_logits=t16["ar_predict_layer.weight"], alpha=alpha,
             dims=dict(d_model=int(mm["hidden_dim"]), ffn=int(mm["linear_units"]),
                       vocab=int(mm["vocab_size"]), n_layer=n_layer))
    return m, (a16, a32)


SOVITS_UPS_U = (10, 8, 2, 2, 2)    # Generator upsample rates (dec.hpp:55)
SOVITS_RES_K = (3, 7, 11)          # ResBlock1 kernel sizes (dec.hpp:67)
SOVITS_RES_DIL = (1, 3, 5)         # convs1 dilations (dec.hpp:57)


def sovits_decoder_from_gsv(g, z, ge, out, round_x=False, graph=True, dev="cuda", stream=None):
    """A SovitsDecoder over the Generator weights of a sovits .gsv, by the names Generator::load
    reads (dec.hpp:54-75): conv_pre, cond, ups.{i}, resblocks.{3 i + j}.convs{1,2}.{m}, conv_post.
    Each weight comes as load_tensor_f16 takes it (sovits_types.hpp:76-87): the tensor's fp16 copy
    when the file has one, else its fp32 values rounded to fp16 on the device (gsvk_f32_to_f16);
    biases are fp32 (absent: zeros, as for conv_post). Channel counts and kernel sizes come from
    the tensors' shapes, strides and dilations are the model's. Returns (decoder, arenas)."""
    a16, t16 = g.upload(F16, dev, stream)
    a32, t32 = g.upload(F32, dev, stream)

    def w16(name):
        if name in t16:
            return t16[name]
        if name not in t32:
            raise GsvkError(f"sovits_decoder_from_gsv: missing tensor {name}", E_FORMAT)
        return f32_to_f16(t32[name], stream=stream)

    def b32(name):
        return t32.get(name)

    pre = Conv1d(w16("dec.conv_pre.weight"), b32("dec.conv_pre.bias"))
    cond = None
    if "dec.cond.weight" in t16 or "dec.cond.weight" in t32:
        cw = w16("dec.cond.weight")
        cond = (cw.reshape(cw.shape[0], -1).contiguous(), b32("dec.cond.bias"))
    stages = []
    for i, u in enumerate(SOVITS_UPS_U):
        ups = ConvT1d(w16(f"dec.ups.{i}.weight"), b32(f"dec.ups.{i}.bias"), u)
        blocks = []
        for j in range(len(SOVITS_RES_K)):
            p = f"dec.resblocks.{3 * i + j}."
            blocks.append(ResBlock1([w16(f"{p}convs1.{m}.weight") for m in range(3)],
                                    [b32(f"{p}convs1.{m}.bias") for m in range(3)],
                                    [w16(f"{p}convs2.{m}.weight") for m in range(3)],
                                    [b32(f"{p}convs2.{m}.bias") for m in range(3)],
                                    SOVITS_RES_DIL))
        stages.append(GeneratorStage(ups, blocks))
    post = Conv1d(w16("dec.conv_post.weight"), b32("dec.conv_post.bias"))
    dec = SovitsDecoder(pre, cond, stages, post, z, ge, out, round_x=round_x, graph=graph)
    return dec, (a16, a32)
