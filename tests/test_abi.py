"""The C ABI on the CPU: libgsvk.so loads, exports every function include/*.h declares, host-only
helpers work, and argument validation rejects bad calls before anything reaches a GPU (every call
here fails validation or is host-only, so no device is needed)."""
import ctypes
import os
import re
import subprocess

import numpy as np
import pytest

from conftest import ROOT

import gsvk


def _declared_functions():
    names = []
    for h in ("gsvk.h", "gsvk_t2s.h", "gsvk_gsv.h", "gsvk_sovits.h"):
        text = open(os.path.join(ROOT, "include", h)).read()
        text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
        names += re.findall(r"^\s*(?:const\s+)?\w+\s*\**\s*(gsvk_\w+)\s*\(", text, flags=re.M)
    return sorted(set(names))


def test_library_exports_every_declared_symbol(gsvk_lib):
    declared = _declared_functions()
    assert len(declared) >= 16
    out = subprocess.run(["nm", "-D", "--defined-only", gsvk.LIB_PATH], capture_output=True,
                         text=True, check=True).stdout
    exported = set(re.findall(r" T (gsvk_\w+)", out))
    missing = [n for n in declared if n not in exported]
    assert not missing, missing
    assert set(declared) == set(gsvk.SIGNATURES), "binding table out of sync with the headers"


def test_version_and_status_strings(gsvk_lib):
    assert b"gfx950" in gsvk_lib.gsvk_version()
    for code in (0, -1, -2, -3, -4, -5, -6, -7, -8):
        assert gsvk_lib.gsvk_status_string(code)
    assert gsvk_lib.gsvk_status_string(-99) == b"unknown status"


def test_pe_table_host_builder_matches_oracle_bitwise(gsvk_lib):
    import oracle as O
    got = gsvk.pe_table(2048, 512)
    want = O.pe_table(2048, 512)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    # gsvk_pe_row (T2SEngine::pe_row's one-row form) gives the table's rows
    row = np.empty(512, np.float32)
    for p in (0, 1, 7, 166, 1234, 2047, 100000):
        assert gsvk_lib.gsvk_pe_row(row.ctypes.data, p, 512) == gsvk.OK
        assert np.array_equal(row.view(np.uint32), O.pe_row(p, 512).view(np.uint32)), p
    assert gsvk_lib.gsvk_pe_row(None, 3, 512) == gsvk.E_NULL
    assert gsvk_lib.gsvk_pe_row(row.ctypes.data, 3, 511) == gsvk.E_ARG
    assert gsvk_lib.gsvk_pe_row(row.ctypes.data, 3, 0) == gsvk.E_SIZE
    assert gsvk_lib.gsvk_pe_table(None, 4, 4) == gsvk.E_NULL
    buf = np.empty(12, np.float32)
    assert gsvk_lib.gsvk_pe_table(buf.ctypes.data, 4, 3) == gsvk.E_ARG  # odd D
    assert gsvk_lib.gsvk_pe_table(buf.ctypes.data, 0, 4) == gsvk.E_SIZE


# Fake, never-dereferenced addresses: validation must reject these calls before any launch.
A, B, C = 0x100000, 0x200000, 0x300000


def test_layernorm_validation(gsvk_lib):
    f = gsvk_lib.gsvk_add_layernorm
    assert f(7, A, None, None, None, None, B, 4, 8, 8, 1e-5, None) == gsvk.E_DTYPE
    assert f(0, None, None, None, None, None, B, 4, 8, 8, 1e-5, None) == gsvk.E_NULL
    assert f(0, A, None, None, None, None, None, 4, 8, 8, 1e-5, None) == gsvk.E_NULL
    assert f(0, A, None, None, None, None, B, 0, 8, 8, 1e-5, None) == gsvk.E_SIZE
    assert f(0, A, None, None, None, None, B, 4, 0, 8, 1e-5, None) == gsvk.E_SIZE
    assert f(0, A, None, None, None, None, B, 4, 8, 7, 1e-5, None) == gsvk.E_SIZE  # ld < n
    assert f(0, A, None, None, None, None, B, 4, 8, 8, -1.0, None) == gsvk.E_ARG
    assert f(0, A, None, None, None, None, B, 4, 8, 8, float("nan"), None) == gsvk.E_ARG
    # partial overlap of y with x (y == x is allowed, y == x + 4 bytes is not)
    assert f(0, A, None, None, None, None, A + 4, 4, 8, 8, 1e-5, None) == gsvk.E_ALIAS
    assert f(0, A, None, B, None, None, B + 16, 4, 8, 8, 1e-5, None) == gsvk.E_ALIAS
    assert f(0, A, None, None, C, None, C - 8, 4, 8, 8, 1e-5, None) == gsvk.E_ALIAS  # gamma


def test_epilogue_validation(gsvk_lib):
    L = gsvk_lib
    assert L.gsvk_bias_act(0, 9, A, None, B, 1, 8, 8, 0.0, None) == gsvk.E_DTYPE
    assert L.gsvk_bias_act(0, 1, A, None, A + 4, 1, 8, 8, 0.0, None) == gsvk.E_ALIAS
    assert L.gsvk_bias_act(1, 1, A + 1, None, B, 1, 8, 8, 0.0, None) == gsvk.E_ARG  # misaligned f16
    assert L.gsvk_leaky_relu(0, A, B, 0, 0.1, None) == gsvk.E_SIZE
    assert L.gsvk_leaky_relu(0, A, A + 8, 16, 0.1, None) == gsvk.E_ALIAS
    assert L.gsvk_resblock_add_lrelu(0, A, None, None, 8, 0.1, None) == gsvk.E_NULL
    assert L.gsvk_resblock_add_lrelu(0, A, A, None, 8, 0.1, None) == gsvk.E_ALIAS
    assert L.gsvk_resblock_add_lrelu(0, A, B, A + 4, 8, 0.1, None) == gsvk.E_ALIAS
    vp = ctypes.c_void_p
    curs = (vp * 3)(A, B, C)
    assert L.gsvk_resblock_branch_mean(0, curs, None, 0, 0x400000, 8, 1, 0.1, None) == gsvk.E_ARG
    assert L.gsvk_resblock_branch_mean(0, curs, None, 5, 0x400000, 8, 1, 0.1, None) == gsvk.E_ARG
    assert L.gsvk_resblock_branch_mean(0, curs, None, 3, B + 4, 8, 1, 0.1, None) == gsvk.E_ALIAS
    assert L.gsvk_resblock_branch_mean(0, None, None, 3, B, 8, 1, 0.1, None) == gsvk.E_NULL
    assert L.gsvk_scaled_add(0, None, A, A, 8, 0.5, None) == gsvk.E_ALIAS
    assert L.gsvk_scaled_add(0, B + 4, A, B, 8, 0.5, None) == gsvk.E_ALIAS
    assert L.gsvk_groupnorm_gelu(0, A, None, None, B, 0, 8, 8, 1e-5, 1, None) == gsvk.E_SIZE
    assert L.gsvk_groupnorm_gelu(0, A, None, None, A + 4, 2, 8, 8, 1e-5, 1, None) == gsvk.E_ALIAS


def test_gemv_validation(gsvk_lib):
    f = gsvk_lib.gsvk_gemv_f16w

    def call(xdt=1, rx=1, x=A, ldx=64, w=B, bias=None, act=0, res=None, ydt=0, y=C, ldy=32,
             rows=4, out=32, n_in=64):
        return f(xdt, rx, x, ldx, w, bias, act, 0.0, res, ydt, y, ldy, rows, out, n_in, None)

    assert call(xdt=2) == gsvk.E_DTYPE          # bf16 activations are not a reference input
    assert call(ydt=5) == gsvk.E_DTYPE
    assert call(act=4) == gsvk.E_DTYPE
    assert call(x=None) == gsvk.E_NULL
    assert call(w=None) == gsvk.E_NULL
    assert call(y=None) == gsvk.E_NULL
    assert call(rows=0) == gsvk.E_SIZE
    assert call(n_in=0) == gsvk.E_SIZE
    assert call(ldx=63) == gsvk.E_SIZE          # ldx < in
    assert call(ldy=31) == gsvk.E_SIZE          # ldy < out
    assert call(rows=65535 * 16 + 1) == gsvk.E_SIZE
    assert call(y=A + 64) == gsvk.E_ALIAS       # over x
    assert call(y=B + 128) == gsvk.E_ALIAS      # over the weights
    assert call(bias=C + 16) == gsvk.E_ALIAS    # bias inside y
    assert call(res=C + 4) == gsvk.E_ALIAS      # residual partly over y (res == y is allowed)


def test_gemv_ln_validation(gsvk_lib):
    f = gsvk_lib.gsvk_gemv_f16w_ln
    H = A + (1 << 24)  # h: a region of its own

    def call(xdt=1, rx=1, z=A, ldz=64, g=None, b=None, eps=1e-5, h=H, ldh=64, w=B, bias=None,
             act=0, res=None, ydt=0, y=C, ldy=32, rows=4, out=32, n_in=64):
        return f(xdt, rx, z, ldz, g, b, eps, h, ldh, w, bias, act, 0.0, res, ydt, y, ldy, rows, out,
                 n_in, None)

    assert call(xdt=2) == gsvk.E_DTYPE
    assert call(act=4) == gsvk.E_DTYPE
    assert call(z=None) == gsvk.E_NULL
    assert call(h=None) == gsvk.E_NULL          # the LayerNorm output is always written
    assert call(rows=0) == gsvk.E_SIZE
    assert call(ldh=63) == gsvk.E_SIZE
    assert call(eps=-1.0) == gsvk.E_ARG
    assert call(eps=float("nan")) == gsvk.E_ARG
    assert call(h=A + 32) == gsvk.E_ALIAS       # h over z (other workgroups still read z)
    assert call(h=B + 64) == gsvk.E_ALIAS       # h over the weights
    assert call(g=H + 8) == gsvk.E_ALIAS        # gamma inside h
    assert call(y=H + 16) == gsvk.E_ALIAS       # y over h
    assert call(y=A + 64) == gsvk.E_ALIAS       # y over z
    # two-launch form (in % 8 != 0) takes one row stride for z and h
    assert call(n_in=60, ldz=64, ldh=72) == gsvk.E_ARG


def test_attention_validation(gsvk_lib):
    f = gsvk_lib.gsvk_decode_attention

    def call(kv=1, out=0, q=A, ldq=1536, k=B, v=C, max_len=8, pos=0x700000, y=0x800000, ldo=512,
             batch=2, H=16, HD=32, ws=None, wsb=0):
        return f(kv, out, q, ldq, k, v, max_len, pos, y, ldo, batch, H, HD, 0, ws, wsb, None, None)

    assert call(kv=9) == gsvk.E_DTYPE
    assert call(out=9) == gsvk.E_DTYPE
    assert call(pos=None) == gsvk.E_NULL
    assert call(max_len=0) == gsvk.E_SIZE
    assert call(ldq=1535) == gsvk.E_SIZE
    assert call(ldo=511) == gsvk.E_SIZE
    assert call(H=16, HD=40) == gsvk.E_ARG       # head_dim / 8 not a power of two
    assert call(H=32, HD=32) == gsvk.E_ARG       # D > 512
    assert call(q=A + 4) == gsvk.E_ARG           # rows not 16-byte aligned
    assert call(y=B + 64) == gsvk.E_ALIAS        # output over the key cache
    assert call(v=B + 1024) == gsvk.E_ALIAS      # caches overlap
    ws = gsvk_lib.gsvk_decode_attention_workspace_bytes
    assert ws(64, 16, 32, 100) == 0
    assert ws(64, 16, 32, 1024) > 0
    # len_bound 0 sizes for any max_len: at least what every explicit bound needs, also where the
    # batch exceeds half the CUs (long contexts then take one chunk, short ones still two)
    for batch in (1, 64, 129, 200, 256, 700):
        need = max(ws(batch, 16, 32, lb) for lb in (1, 128, 129, 200, 256, 257, 1024, 1 << 20))
        assert ws(batch, 16, 32, 0) >= need, batch
    assert ws(200, 16, 32, 0) >= ws(200, 16, 32, 200) > 0


def test_t2s_decode_workspace_and_parts(gsvk_lib):
    att = gsvk_lib.gsvk_decode_attention_workspace_bytes
    dec = gsvk_lib.gsvk_t2s_decode_workspace_bytes
    assert dec(0, 16, 32, 1024) == 0
    # below 32 sequences one chain: the attention call's own workspace
    assert dec(31, 16, 32, 1024) == att(31, 16, 32, 1024)
    # two halves: each half's chunk states, the first slice rounded up to 256 bytes
    for B, lb in ((64, 1024), (64, 0), (37, 200), (33, 5000)):
        h0 = att(B // 2, 16, 32, lb)
        need = (h0 + 255) // 256 * 256 + att(B - B // 2, 16, 32, lb)
        assert dec(B, 16, 32, lb) == max(need, att(B, 16, 32, lb)), (B, lb)
    assert dec(64, 16, 32, 1024) > att(64, 16, 32, 1024)  # halves split their keys finer
    # parts outside {0, 1}: E_ARG before anything runs (fake, never dereferenced pointers)
    fake = 0x10000000
    lay = (gsvk.T2SLayer * 1)()
    for name, _ in gsvk.T2SLayer._fields_:
        setattr(lay[0], name, fake)
    d = gsvk.T2SDecodeDesc()
    d.dtype = d.kv_dtype = gsvk.F16
    d.batch, d.d_model, d.heads, d.ffn, d.layers, d.max_len = 64, 512, 16, 2048, 1, 64
    d.layer = ctypes.cast(lay, ctypes.POINTER(gsvk.T2SLayer))
    for name in ("x", "h", "z", "attn", "ff", "qkv", "kv_pos"):
        setattr(d, name, fake)
    d.parts = 2
    assert gsvk_lib.gsvk_t2s_decode_eager(ctypes.byref(d), None) == gsvk.E_ARG
    out = ctypes.c_void_p()
    assert gsvk_lib.gsvk_t2s_decode_create(ctypes.byref(d), ctypes.byref(out)) == gsvk.E_ARG
    assert not out.value


def test_conv_validation(gsvk_lib):
    f = gsvk_lib.gsvk_conv1d
    n = gsvk_lib.gsvk_conv1d_packed_elems(8, 16, 3)
    assert n == 1 * 3 * 64 * 32  # one 32-channel chunk, 3 taps, 8 outputs padded to 64
    assert gsvk_lib.gsvk_conv1d_packed_elems(0, 16, 3) == 0
    assert gsvk_lib.gsvk_conv1d_packed_elems(65, 33, 1) == 2 * 1 * 128 * 32

    def call(dt=0, x=A, ldx=100, w=B, bias=None, epi=0, cur=None, res=None, ldc=0, y=C, ldy=100,
             cin=16, cout=8, T=100, k=3, dil=1):
        return f(dt, 0, x, ldx, w, bias, epi, 0.1, cur, res, ldc, y, ldy, cin, cout, T, k, dil,
                 None)

    assert call(dt=2) == gsvk.E_DTYPE           # bf16 activations are not a reference input
    assert call(epi=6) == gsvk.E_DTYPE
    assert call(epi=0x200) == gsvk.E_DTYPE                      # unknown flag bit
    assert call(epi=gsvk.CONV_X_LRELU | 6) == gsvk.E_DTYPE
    assert call(epi=4, cur=None) == gsvk.E_NULL   # the dual epilogue writes cur too
    assert call(epi=2, cur=0x700000, ldc=100, res=0x700000 + 8) == gsvk.E_ALIAS  # res inside cur
    assert call(epi=2, cur=0x700000, ldc=100, res=C + 8) == gsvk.E_ALIAS          # res inside y
    assert call(epi=4, cur=C + 64, ldc=100) == gsvk.E_ALIAS                        # cur over y
    assert call(x=None) == gsvk.E_NULL
    assert call(w=None) == gsvk.E_NULL
    assert call(y=None) == gsvk.E_NULL
    assert call(epi=2, cur=None) == gsvk.E_NULL  # the residual modes need cur
    assert call(T=0) == gsvk.E_SIZE
    assert call(dil=0) == gsvk.E_SIZE
    assert call(ldx=99) == gsvk.E_SIZE
    assert call(ldy=99) == gsvk.E_SIZE
    assert call(epi=3, cur=0x700000, ldc=99, y=None) == gsvk.E_SIZE
    assert call(k=11, dil=26) == gsvk.E_ARG      # halo (k - 1) dil above 256
    assert call(w=B + 8) == gsvk.E_ARG           # packed weights not 16-byte aligned
    assert call(ldx=1 << 26, T=100) == gsvk.E_SIZE  # 32 rows beyond 32-bit offsets
    assert call(cin=16384, cout=16384, k=4) == gsvk.E_SIZE  # 2 GiB of packed weights
    assert call(y=A + 64) == gsvk.E_ALIAS        # output over x
    assert call(y=B + 64) == gsvk.E_ALIAS        # output over the weights
    assert call(bias=C + 16) == gsvk.E_ALIAS     # bias inside y
    assert call(epi=2, cur=C + 64, ldc=100) == gsvk.E_ALIAS  # cur over y
    assert call(epi=3, cur=A + 4, ldc=100, y=None) == gsvk.E_ALIAS  # cur over x
    p = gsvk_lib.gsvk_conv1d_pack
    assert p(None, 8, 16, 3, B, n, None) == gsvk.E_NULL
    assert p(A, 8, 16, 3, B, n - 1, None) == gsvk.E_SIZE
    assert p(A, 8, 16, 0, B, n, None) == gsvk.E_SIZE
    assert p(A, 8, 16, 3, A + 64, n, None) == gsvk.E_ALIAS


def test_convt_validation(gsvk_lib):
    f = gsvk_lib.gsvk_convt1d
    assert gsvk_lib.gsvk_convt1d_packed_elems(8, 16, 16, 8) == 1 * 16 * 64 * 32  # taps add up to k
    assert gsvk_lib.gsvk_convt1d_packed_elems(8, 16, 4, 8) == 0                  # k < stride

    def call(dt=0, x=A, ldx=100, w=B, epi=0, cur=None, ldc=0, y=C, ldy=800, cin=16, cout=8, T=100,
             k=16, u=8):
        return f(dt, 0, x, ldx, w, None, epi, 0.1, cur, None, ldc, y, ldy, cin, cout, T, k, u, None)

    assert call(dt=2) == gsvk.E_DTYPE
    assert call(x=None) == gsvk.E_NULL
    assert call(u=0) == gsvk.E_SIZE
    assert call(ldy=799) == gsvk.E_SIZE          # output rows hold T * stride columns
    assert call(k=4) == gsvk.E_ARG               # k < stride: the reference's pad is undefined
    assert call(k=200, u=2) == gsvk.E_ARG        # 100 taps per phase do not fit one tile
    assert call(w=B + 8) == gsvk.E_ARG
    assert call(y=A + 64) == gsvk.E_ALIAS
    p = gsvk_lib.gsvk_convt1d_pack
    n = gsvk_lib.gsvk_convt1d_packed_elems(8, 16, 16, 8)
    assert p(A, 8, 16, 16, 8, B, n - 1, None) == gsvk.E_SIZE
    assert p(A, 8, 16, 4, 8, B, n, None) == gsvk.E_ARG
    assert p(A, 8, 16, 16, 8, A + 64, n, None) == gsvk.E_ALIAS


def test_embed_validation(gsvk_lib):
    f = gsvk_lib.gsvk_embed_pe
    args = dict(out=0, tab=1, it=0, table=A, vocab=10, ids=B, pos=None, pos0=0, pe=C, max_pos=4,
                alpha=1.0, mm=None, bias=None, outp=0x900000, rows=2, D=8, err=None)

    def call(**kw):
        a = dict(args, **kw)
        return f(a["out"], a["tab"], a["it"], a["table"], a["vocab"], a["ids"], a["pos"],
                 a["pos0"], a["pe"], a["max_pos"], a["alpha"], a["mm"], a["bias"], a["outp"],
                 a["rows"], a["D"], a["err"], None)

    assert call(it=5) == gsvk.E_DTYPE
    assert call(table=None) == gsvk.E_NULL
    assert call(rows=0) == gsvk.E_SIZE
    assert call(D=7) == gsvk.E_ARG
    assert call(outp=A) == gsvk.E_ALIAS          # writes over the table
    assert call(outp=C + 16) == gsvk.E_ALIAS     # writes over the PE table


def test_prefill_input_validation(gsvk_lib):
    f = gsvk_lib.gsvk_t2s_prefill_input
    args = dict(out=1, tab=1, it=0, ttab=A, tv=10, ph=B, T=4, mm=None, bias=None, at=1.0,
                atab=A + 4096, av=10, pr=B + 64, P=4, aa=1.0, pe=C, max_pos=8, xy=0x900000,
                D=8, err=None)

    def call(**kw):
        a = dict(args, **kw)
        return f(a["out"], a["tab"], a["it"], a["ttab"], a["tv"], a["ph"], a["T"], a["mm"],
                 a["bias"], a["at"], a["atab"], a["av"], a["pr"], a["P"], a["aa"], a["pe"],
                 a["max_pos"], a["xy"], a["D"], a["err"], None)

    assert call(out=7) == gsvk.E_DTYPE
    assert call(it=2) == gsvk.E_DTYPE
    assert call(atab=None) == gsvk.E_NULL
    assert call(ph=None) == gsvk.E_NULL           # T > 0 needs phones
    assert call(T=0, P=0) == gsvk.E_SIZE
    assert call(max_pos=0) == gsvk.E_SIZE
    assert call(T=1 << 35) == gsvk.E_SIZE
    assert call(P=(1 << 24) + 1) == gsvk.E_SIZE   # one wave per position: under 2^32 work-items
    assert call(D=7) == gsvk.E_ARG
    assert call(xy=A) == gsvk.E_ALIAS             # over the text table
    assert call(xy=C + 16) == gsvk.E_ALIAS        # over the PE table
    assert call(mm=0x900000 + 64) == gsvk.E_ALIAS  # bert_proj rows partly over xy (not xy itself)


def test_f32_to_f16_validation(gsvk_lib):
    f = gsvk_lib.gsvk_f32_to_f16
    assert f(None, 0x1000, 8, None) == gsvk.E_NULL
    assert f(0x1000, None, 8, None) == gsvk.E_NULL
    assert f(0x1000, 0x8000, 0, None) == gsvk.E_SIZE
    assert f(0x1000, 0x1010, 8, None) == gsvk.E_ALIAS     # y inside x's 32 bytes
    assert f(0x1002, 0x8000, 8, None) == gsvk.E_ARG       # x not 4-byte aligned
    assert f(0x1000, 0x8001, 8, None) == gsvk.E_ARG       # y not 2-byte aligned


def test_t2s_step_validation(gsvk_lib):
    out = ctypes.c_void_p()
    assert gsvk_lib.gsvk_t2s_step_create(None, ctypes.byref(out)) == gsvk.E_NULL
    assert gsvk_lib.gsvk_t2s_step_eager(None, None) == gsvk.E_NULL
    assert gsvk_lib.gsvk_t2s_step_run(None, None) == gsvk.E_NULL
    assert gsvk_lib.gsvk_t2s_step_launches(None) == 0
    gsvk_lib.gsvk_t2s_step_destroy(None)
    assert gsvk_lib.gsvk_t2s_step_fused(None, None) == gsvk.E_NULL
    assert gsvk_lib.gsvk_t2s_step_create_fused(None, ctypes.byref(out)) == gsvk.E_NULL


def _step_desc(L=24, B=64, D=512, FF=2048, dt=gsvk.F16, base=0x10000000, gap=1 << 24):
    """A decode-step descriptor over fake, never dereferenced, disjoint 16-byte aligned device
    addresses (`gap` bytes apart): the fused entry point must reject every variant below in
    validation."""
    nxt = [base]

    def addr():
        nxt[0] += gap
        return nxt[0]
    keep = {}

    def arr(name):
        a = (ctypes.c_void_p * L)(*[addr() for _ in range(L)])
        keep[name] = a
        return ctypes.cast(a, ctypes.POINTER(ctypes.c_void_p))
    d = gsvk.T2SStepDesc()
    d.dtype, d.batch, d.d_model, d.ffn, d.layers, d.eps = dt, B, D, FF, L, 1e-5
    d.audio_table, d.table_dtype, d.vocab = addr(), gsvk.F16, 1025
    d.ids, d.index_type, d.pos, d.pe, d.max_pos, d.alpha = addr(), gsvk.I64, addr(), addr(), 2048, 0.9
    d.err, d.x, d.h = addr(), addr(), addr()
    for name in ("attn_out", "bout", "n1g", "n1b", "ff", "b1", "ffn_out", "b2", "n2g", "n2b"):
        setattr(d, name, arr(name))
    return d, keep


def test_t2s_step_fused_validation(gsvk_lib):
    f = lambda d: gsvk_lib.gsvk_t2s_step_fused(ctypes.byref(d), None)
    d, k = _step_desc(L=33)
    assert f(d) == gsvk.E_SIZE                       # more layers than the kernel arguments hold
    d, k = _step_desc(D=1032)
    assert f(d) == gsvk.E_ARG                        # 129 chunks: more than two per lane
    d, k = _step_desc(D=516)
    assert f(d) == gsvk.E_ARG                        # not whole 16-byte chunks
    d, k = _step_desc(D=1024, dt=gsvk.F32)
    assert f(d) == gsvk.E_ARG                        # f32 rows of more than 512
    d, k = _step_desc(FF=2044)
    assert f(d) == gsvk.E_ARG
    d, k = _step_desc()
    d.x = d.h + 64
    assert f(d) == gsvk.E_ALIAS                      # x overlaps h
    d, k = _step_desc()
    d.h = k["attn_out"][3]
    assert f(d) == gsvk.E_ALIAS                      # h is an input of layer 3
    d, k = _step_desc()
    k["ff"][5] = k["ff"][2] + 1024
    assert f(d) == gsvk.E_ALIAS                      # two layers' FFN buffers overlap
    # an FFN buffer over anything the chain waves read while the ReLU tiles write it
    for name, layer in (("bout", 7), ("n1g", 0), ("n2b", 23), ("b2", 5)):
        d, k = _step_desc()
        k["ff"][4] = k[name][layer] - 64
        assert f(d) == gsvk.E_ALIAS, name
    for field in ("pe", "audio_table", "ids", "pos", "err"):
        d, k = _step_desc()
        k["ff"][9] = getattr(d, field)
        assert f(d) == gsvk.E_ALIAS, field
    d, k = _step_desc()
    d.x = d.x + 8
    assert f(d) == gsvk.E_ARG                        # x not 16-byte aligned
    d, k = _step_desc()
    d.index_type = 7
    assert f(d) == gsvk.E_DTYPE
    d, k = _step_desc()
    d.eps = float("nan")
    assert f(d) == gsvk.E_ARG
    d, k = _step_desc()
    d.ids = None
    assert f(d) == gsvk.E_NULL
    # 65,536 sequences with an FFN of 2^20: 24 x 2^25 one-wave ReLU workgroups, past the 2^32
    # work-items of one launch (buffers 2^40 bytes apart, so no overlap is reported first)
    d, k = _step_desc(B=1 << 16, FF=1 << 20, gap=1 << 40)
    assert f(d) == gsvk.E_SIZE


def _decoder_desc(frames=500, c0=768, n_stages=5, fake=0x1000):
    """A decoder descriptor of the reference's geometry (dec.hpp:54-75) with fake, never
    dereferenced device addresses: every call below fails validation or is host-only."""
    ups_u, ups_k = (10, 8, 2, 2, 2), (20, 16, 8, 2, 2)
    stages = (gsvk.SovitsStage * n_stages)()
    c = c0
    for s in range(n_stages):
        S = stages[s]
        S.c_in, S.c_out, S.ups_k, S.ups_u = c, c // 2, ups_k[s], ups_u[s]
        S.ups_w = S.ups_b = fake
        for j, k in enumerate((3, 7, 11)):
            S.res_k[j] = k
            S.res_dil[j] = (1, 3, 5)[j]
            for m in range(3):
                S.w1[j][m] = S.b1[j][m] = S.w2[j][m] = S.b2[j][m] = fake
        c //= 2
    d = gsvk.SovitsDecoderDesc()
    d.dtype, d.frames, d.c_z, d.c0, d.pre_k = gsvk.F32, frames, 192, c0, 7
    d.pre_w = d.pre_b = d.cond_w = d.cond_b = d.post_w = d.z = d.ge = d.out = fake
    d.g_in, d.n_stages, d.post_k = 1024, n_stages, 7
    d.stage = ctypes.cast(stages, ctypes.POINTER(gsvk.SovitsStage))
    return d, stages


def test_sovits_decoder_workspace_and_validation(gsvk_lib):
    d, keep = _decoder_desc()
    # the folded bias (768 floats), 8 slots of the largest stage tensor (192 x 40000 = 7.68M)
    want = (768 + 8 * 7_680_000) * 4
    assert gsvk_lib.gsvk_sovits_decoder_workspace_bytes(ctypes.byref(d)) == want
    assert gsvk_lib.gsvk_sovits_decoder_workspace_bytes(None) == 0
    h = ctypes.c_void_p()
    assert gsvk_lib.gsvk_sovits_decoder_create(ctypes.byref(d), None) == gsvk.E_NULL
    assert gsvk_lib.gsvk_sovits_decoder_create(None, ctypes.byref(h)) == gsvk.E_NULL
    assert gsvk_lib.gsvk_sovits_decoder_eager(ctypes.byref(d), None) == gsvk.E_NULL  # workspace
    d.workspace, d.workspace_bytes = 0x10000, want - 4
    assert gsvk_lib.gsvk_sovits_decoder_eager(ctypes.byref(d), None) == gsvk.E_SIZE
    assert gsvk_lib.gsvk_sovits_decoder_create(ctypes.byref(d), ctypes.byref(h)) == gsvk.E_SIZE
    assert not h.value
    d.workspace, d.workspace_bytes = 0x10008, want  # not 16-byte aligned
    assert gsvk_lib.gsvk_sovits_decoder_eager(ctypes.byref(d), None) == gsvk.E_ARG
    d.workspace = 0x10000

    def bad(**kw):
        e, k2 = _decoder_desc()
        e.workspace, e.workspace_bytes = 0x10000, want
        for key, v in kw.items():
            if key.startswith("stage1_"):
                setattr(k2[1], key[7:], v)
            else:
                setattr(e, key, v)
        return gsvk_lib.gsvk_sovits_decoder_eager(ctypes.byref(e), None)

    assert bad(dtype=gsvk.BF16) == gsvk.E_DTYPE
    e, k2 = _decoder_desc()
    e.dtype = gsvk.F16  # fp16 activation slots (2 bytes); the folded bias stays fp32
    assert gsvk_lib.gsvk_sovits_decoder_workspace_bytes(ctypes.byref(e)) == 768 * 4 + \
        8 * 7_680_000 * 2
    assert bad(frames=0) == gsvk.E_SIZE
    assert bad(n_stages=0) == gsvk.E_SIZE
    assert bad(n_stages=9) == gsvk.E_SIZE
    assert bad(stage1_c_in=100) == gsvk.E_SIZE       # stage chain: c_in must be the previous c_out
    assert bad(stage1_ups_u=0) == gsvk.E_SIZE
    assert bad(stage1_ups_w=None) == gsvk.E_NULL
    assert bad(z=None) == gsvk.E_NULL
    assert bad(ge=None) == gsvk.E_NULL               # g_in > 0 needs ge
    assert bad(post_w=None) == gsvk.E_NULL
    e, k2 = _decoder_desc()
    k2[2].w2[1][2] = None
    e.workspace, e.workspace_bytes = 0x10000, want
    assert gsvk_lib.gsvk_sovits_decoder_eager(ctypes.byref(e), None) == gsvk.E_NULL
    # shapes alone size the workspace: NULL buffers still give the figure
    e, k2 = _decoder_desc(fake=0)
    assert gsvk_lib.gsvk_sovits_decoder_workspace_bytes(ctypes.byref(e)) == want


def test_host_mirror_header_compiles(tmp_path):
    """host/gsvk/kern.hpp (the reference-named C++ API) compiles against the C ABI, and a call
    site written like the reference's (kern.hpp:25, 33; nn_ops.hpp:48-105) compiles unchanged."""
    src = r'''
#include <gsvk/kern.hpp>
void engine_like(float* x, const float* g, const float* b, float* ff, float* cur, const float* tb,
                 float* tin, float* sum) {
  gsv::kern::layernorm(x, g, b, x, 512, 1e-5);
  gsv::kern::relu(ff, ff, 2048);
  gsv::sovits::leaky_relu_io(cur, 1000, 0.1f);
  gsv::sovits::leaky_relu_write(cur, tin, 1000, 0.1f);
  gsv::sovits::add_inplace(cur, tb, 1000);
  gsv::sovits::mul_write(sum, cur, 1000, 1.f / 3);
  gsv::sovits::add_scaled_inplace(sum, cur, 1000, 1.f / 3);
  gsv::bert::layernorm1d_forward(x, g, b, 4, 1024);
  gsv::encoder::groupnorm_gelu(x, g, b, 512, 31999, 1e-5);
  gsv::kern::gemv_f16w_f32acc(reinterpret_cast<const uint16_t*>(g), x, ff, 2048, 512);
  gsv::kern::gemv_f16x_fmlal(reinterpret_cast<const uint16_t*>(g),
                             reinterpret_cast<const uint16_t*>(b), ff, 2048, 512);
  gsv::kern::gemv_fmlal_rows(reinterpret_cast<const uint16_t*>(g), x, ff, 64, 2048, 512, b,
                             GSVK_ACT_RELU);
  gsv::kern::gemv_fmlal_rows(reinterpret_cast<const uint16_t*>(g), x, ff, 64, 2048, 512, b,
                             GSVK_ACT_RELU, x);
  gsv::kern::layernorm_gemv_fmlal_rows(x, g, b, 1e-5, cur, reinterpret_cast<const uint16_t*>(g), ff,
                                       64, 2048, 512, b, GSVK_ACT_RELU);
  gsv::sovits::Conv1d c1;
  c1.load(reinterpret_cast<const uint16_t*>(g), b, 192, 192, 11, 5);
  c1.forward(cur, tin, 40000, GSVK_CONV_EPI_LRELU, 0.1f);
  c1.forward(tin, sum, 40000, GSVK_CONV_EPI_RES_LRELU, 0.1f, cur);
  gsv::sovits::ConvT1d up;
  up.load(reinterpret_cast<const uint16_t*>(g), b, 384, 192, 16, 8);
  up.forward(x, cur, 5000);
}
'''
    path = str(tmp_path / "compat_probe.cpp")
    open(path, "w").write(src)
    inc = ["-I", os.path.join(ROOT, "include"), "-I", os.path.join(ROOT, "gpt-sovits-native_amd", "host"),
           "-I", "/opt/rocm/include"]
    r = subprocess.run(["/opt/rocm/bin/hipcc", "-std=c++17", "-fsyntax-only", "-x", "c++",
                        "-D__HIP_PLATFORM_AMD__", *inc, path], capture_output=True, text=True)
    if r.returncode != 0 and "No such file" in r.stderr and "hipcc" in r.stderr:
        pytest.skip("hipcc not available")
    assert r.returncode == 0, r.stderr[-2000:]


def test_sovits_run_example_usage():
    """The C++ mirror's example program is built and rejects a wrong command line before touching
    the GPU (exit status 2, usage on stderr)."""
    exe = os.path.join(ROOT, "gpt-sovits-native_amd", "sovits_run")
    if not os.path.exists(exe):
        pytest.skip("sovits_run not built")
    r = subprocess.run([exe], capture_output=True, text=True, timeout=60)
    assert r.returncode == 2 and "usage" in r.stderr
