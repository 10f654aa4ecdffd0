"""The .gsv loader on the CPU (open, header, directory, validation); the upload is in
test_gpu_gsv.py. Mirrors the reference's tests/test_gsv_header.cpp and test_gsv_loader.cpp with a
synthetic ar_s1-shaped file in place of weights/ar_s1v3.gsv (not available here), plus every
malformed-directory rule gsv_loader.cpp:46-108 enforces."""
import ctypes
import os
import struct

import numpy as np
import pytest

import gsvk
from gsv_writer import gsv_bytes, t2s_tensors


def open_bytes(b):
    return gsvk.GsvFile(data=b)


def rc_of(b):
    """Status of gsvk_gsv_open_memory on b (the handle is closed again when it opened)."""
    h = ctypes.c_void_p()
    buf = ctypes.create_string_buffer(bytes(b), len(b))
    rc = gsvk.lib().gsvk_gsv_open_memory(ctypes.cast(buf, ctypes.c_void_p), len(b), ctypes.byref(h))
    if rc == 0:
        gsvk.lib().gsvk_gsv_close(h)
    return rc


@pytest.fixture(scope="module")
def model():
    t, cfg = t2s_tensors()
    return t, cfg, gsv_bytes("ar_s1v3", t, cfg)


def test_header_and_config(model, tmp_path):
    t, cfg, b = model
    p = tmp_path / "m.gsv"
    p.write_bytes(b)
    g = gsvk.GsvFile(str(p))
    assert (g.version, g.name, g.n_tensors) == (1, "ar_s1v3", len(t))
    assert g.flags == 1  # has fp16 segments
    assert set(g.config) == {"meta", "model_config"}
    m = g.config["model_config"]["model"]
    assert (m["hidden_dim"], m["head"], m["n_layer"], m["vocab_size"], m["EOS"]) == (128, 4, 2, 50, 49)
    g.close()


def test_shapes_dtypes_and_fp16_rule(model):
    t, cfg, b = model
    g = open_bytes(b)
    for name, arr in t.items():
        info = g.tensors[name]
        assert info["dims"] == arr.shape and info["numel"] == arr.size
        assert info["src_dtype"] == 2  # fp16 source
        assert (info["f16_nbytes"] != 0) == (arr.size >= 4096), name
        assert info["f32_offset"] % 64 == 0 and (not info["f16_nbytes"] or info["f16_offset"] % 64 == 0)
        # fp16 copy equals the fp32 copy (exact upcast) element for element
        if info["f16_nbytes"]:
            h = np.frombuffer(b, np.float16, arr.size, info["f16_offset"])
            f = np.frombuffer(b, np.float32, arr.size, info["f32_offset"])
            assert np.array_equal(h.astype(np.float32), f)
    assert gsvk.lib().gsvk_gsv_find(g.handle, b"h.layers.1.linear2.weight") >= 0
    assert gsvk.lib().gsvk_gsv_find(g.handle, "不存在的张量".encode()) == -1


def test_rejects_bad_magic_and_truncation():
    assert rc_of(b"XSV1" + bytes(10)) == gsvk.E_FORMAT
    assert rc_of(bytes([ord("G"), ord("S"), ord("V"), ord("1"), 1, 0, 0, 0, 1, 0, 0])) == gsvk.E_FORMAT
    good = gsv_bytes("t", {"x": np.ones(3, np.float32)})
    assert rc_of(good) == 0
    assert rc_of(good[:40]) == gsvk.E_FORMAT                    # directory cut short
    assert rc_of(struct.pack("<4sI", b"GSV1", 2) + good[8:]) == gsvk.E_FORMAT  # version 2


def dir_entry_offset(b):
    """Offset of the first directory entry's dtype field (one tensor named 'x', rank 1)."""
    nl = struct.unpack_from("<H", b, 12)[0]
    off = 14 + nl
    cl = struct.unpack_from("<I", b, off)[0]
    off += 4 + cl + 4            # config, n_tensors
    off += 2 + 1 + 2 + 4         # name len, 'x', rank, dims[0]
    return off


def patch(b, off, fmt, val):
    b = bytearray(b)
    struct.pack_into(fmt, b, off, val)
    return bytes(b)


def test_rejects_malformed_directory():
    good = gsv_bytes("t", {"x": np.ones(3, np.float32)})
    o = dir_entry_offset(good)
    assert rc_of(good) == 0
    assert rc_of(patch(good, o, "<H", 3)) == gsvk.E_FORMAT            # unknown dtype enum
    f32_off = struct.unpack_from("<Q", good, o + 2)[0]
    assert rc_of(patch(good, o + 2, "<Q", f32_off + 4)) == gsvk.E_FORMAT   # not 64-byte aligned
    assert rc_of(patch(good, o + 10, "<Q", 8)) == gsvk.E_FORMAT       # f32 bytes != numel * 4
    assert rc_of(patch(good, o + 2, "<Q", 1 << 20)) == gsvk.E_FORMAT  # segment past the end
    assert rc_of(patch(good, 8, "<I", 1)) == gsvk.E_FORMAT            # flags claim fp16 segments
    # rank 9
    nl = struct.unpack_from("<H", good, 12)[0]
    cl = struct.unpack_from("<I", good, 14 + nl)[0]
    rank_off = 14 + nl + 4 + cl + 4 + 2 + 1
    assert rc_of(patch(good, rank_off, "<H", 9)) == gsvk.E_FORMAT


def test_rejects_dims_whose_product_wraps_64_bits():
    """dims [2^20, 2^20, 2^24]: the running product passes 2^40 exactly, then the next multiply
    would wrap 2^64 to 0 and a 0-byte segment would match. The bound is checked before the
    multiply, so the header is rejected like any other numel above 2^40."""
    good = gsv_bytes("t", {"x": np.ones((1, 1, 3), np.float32)})
    assert rc_of(good) == 0
    nl = struct.unpack_from("<H", good, 12)[0]
    cl = struct.unpack_from("<I", good, 14 + nl)[0]
    dims_off = 14 + nl + 4 + cl + 4 + 2 + 1 + 2
    assert struct.unpack_from("<3I", good, dims_off) == (1, 1, 3)
    b = bytearray(good)
    struct.pack_into("<3I", b, dims_off, 1 << 20, 1 << 20, 1 << 24)
    struct.pack_into("<Q", b, dims_off + 12 + 2 + 8, 0)      # f32 bytes 0 = the wrapped numel x 4
    assert rc_of(bytes(b)) == gsvk.E_FORMAT
    struct.pack_into("<3I", b, dims_off, 1 << 20, 1 << 20, 1)  # exactly 2^40 elements: the size
    assert rc_of(bytes(b)) == gsvk.E_FORMAT                    # check (0 bytes) still rejects it


def test_fp16_sizes_and_slim_files():
    big = {"w": np.ones((64, 64), np.float16), "b": np.ones(4, np.float32)}
    b = gsv_bytes("t", big)
    assert rc_of(b) == 0
    g = open_bytes(b)
    info = g.tensors["w"]
    assert info["f16_nbytes"] == 64 * 64 * 2
    # wrong fp16 size
    buf = bytearray(b)
    # find the 'w' entry: first entry; its f16 bytes field is the last u64 of the entry
    o = 14 + 1 + 4 + struct.unpack_from("<I", b, 15)[0] + 4 + 2 + 1 + 2 + 8
    assert struct.unpack_from("<Q", b, o + 26)[0] == 64 * 64 * 2
    struct.pack_into("<Q", buf, o + 26, 100)
    assert rc_of(bytes(buf)) == gsvk.E_FORMAT
    # slim: fp16 copy only (f32 bytes 0) is accepted, as the reference's loader allows
    s = gsv_bytes("t", {"w": np.ones((64, 64), np.float16)}, slim={"w"})
    g = open_bytes(s)
    assert g.tensors["w"]["f32_nbytes"] == 0 and g.tensors["w"]["f16_nbytes"] == 8192


def test_bad_config_json_and_missing_file(tmp_path):
    b = gsv_bytes("t", {"x": np.ones(3, np.float32)})
    cl_off = 14 + 1
    cl = struct.unpack_from("<I", b, cl_off)[0]
    bad = bytearray(b)
    bad[cl_off + 4] = ord("[")  # '{' -> '[' with the matching '}' left: not JSON
    bad[cl_off + 4 + cl - 1] = ord("x")
    with pytest.raises(gsvk.GsvkError):
        open_bytes(bytes(bad))
    with pytest.raises(gsvk.GsvkError) as e:
        gsvk.GsvFile(str(tmp_path / "missing.gsv"))
    assert e.value.status == gsvk.E_IO


# ---- a file the reference's converter wrote (tests/golden/make_gsv_fixture.py) ----------------

GOLDEN_GSV = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden",
                          "convert_gsv1_small.gsv")


def converter_inputs(seed=20261202):
    """The state dict make_gsv_fixture.py gave the converter, as numpy arrays (same seed and draw
    order), keyed by name after the converter's prefix stripping."""
    r = np.random.default_rng(seed)
    f32 = lambda *s: r.standard_normal(s).astype(np.float32)
    f16 = lambda *s: r.standard_normal(s).astype(np.float16)
    return {"enc.weight": f32(64, 64), "enc.bias": f32(64), "dec.lin.weight": f16(32, 160),
            "dec.lin.bias": f16(32), "dec.conv.weight_g": f16(16, 1, 1),
            "dec.conv.weight_v": f16(16, 8, 3), "big.weight_g": f32(64, 1, 1),
            "big.weight_v": f32(64, 16, 4), "enc.pos_conv_embed.conv.weight_g": f32(1, 1, 5),
            "enc.pos_conv_embed.conv.weight_v": f32(8, 4, 5)}


def converter_expected():
    """What the converter's rules (convert.py:58-100, 102-183) make of those inputs, restated:
    prefixes stripped; weight = g v / ||v|| over every dim but 0 (over dims 0 and 1 for
    pos_conv_embed.conv.), in float64 here; integer tensors dropped; an fp16 copy for every tensor of
    >= 4096 elements that is not a fused weight-norm product. name -> (fp32 values, src dtype,
    has fp16 copy)."""
    x = converter_inputs()

    def fuse(base, dims):
        g = x[base + "weight_g"].astype(np.float64)
        v = x[base + "weight_v"].astype(np.float64)
        return g * v / np.sqrt((v * v).sum(axis=dims, keepdims=True))

    exp = {}
    for name in ("enc.weight", "enc.bias", "dec.lin.weight", "dec.lin.bias"):
        a = x[name]
        exp[name] = (a.astype(np.float64), 1 if a.dtype == np.float32 else 2, a.size >= 4096)
    exp["dec.conv.weight"] = (fuse("dec.conv.", (1, 2)), 1, False)
    exp["big.weight"] = (fuse("big.", (1, 2)), 1, False)
    exp["enc.pos_conv_embed.conv.weight"] = (fuse("enc.pos_conv_embed.conv.", (0, 1)), 1, False)
    return exp


def test_reference_converter_file_directory():
    """The loader's view of a file written by the reference's convert.py: header, config, every
    directory field, and the converter's layout (64-byte aligned segments, all fp32 blocks in
    directory order before all fp16 blocks)."""
    g = gsvk.GsvFile(GOLDEN_GSV)
    exp = converter_expected()
    assert (g.version, g.name, g.n_tensors, g.flags) == (1, "fixture_small", len(exp), 1)
    meta = g.config["meta"]
    assert g.config["model_config"] is None
    assert (meta["model"], meta["converter"], meta["weight_norm_fused"]) == \
        ("fixture_small", "convert.py GSV1", 3)
    assert set(g.tensors) == set(exp)  # prefixes stripped, pairs fused, integer tensors dropped
    ends32, f16_starts = [], []
    for name, (vals, src, has16) in exp.items():
        info = g.tensors[name]
        assert info["dims"] == vals.shape and info["numel"] == vals.size, name
        assert info["src_dtype"] == src, name
        assert info["f32_nbytes"] == 4 * vals.size and info["f32_offset"] % 64 == 0, name
        assert (info["f16_nbytes"] == 2 * vals.size) if has16 else (info["f16_nbytes"] == 0), name
        ends32.append(info["f32_offset"] + info["f32_nbytes"])
        if has16:
            assert info["f16_offset"] % 64 == 0
            f16_starts.append(info["f16_offset"])
    assert min(f16_starts) >= max(ends32)
    offs = [g.tensors[n]["f32_offset"] for n in g.tensors]
    assert offs == sorted(offs)
    g.close()


def test_reference_converter_file_values():
    """Every tensor read at the loader's offsets: fp32 copies of the sources exactly, the fused
    weight-norm products within fp32 rounding of the float64 closed form (and the pos_conv tensor
    fused over dims 0 and 1: the default dims give values far from it), fp16 copies as the fp32
    sources rounded to nearest even."""
    raw = open(GOLDEN_GSV, "rb").read()
    g = gsvk.GsvFile(GOLDEN_GSV)
    x = converter_inputs()
    for name, (vals, src, has16) in converter_expected().items():
        info = g.tensors[name]
        got = np.frombuffer(raw, np.float32, vals.size, info["f32_offset"]).reshape(vals.shape)
        if name in x:
            np.testing.assert_array_equal(got, x[name].astype(np.float32))
        else:
            np.testing.assert_allclose(got, vals, rtol=2e-6, atol=1e-7, err_msg=name)
        if has16:
            h = np.frombuffer(raw, np.uint16, vals.size, info["f16_offset"])
            assert np.array_equal(h, x[name].astype(np.float16).view(np.uint16).ravel()), name
    v = x["enc.pos_conv_embed.conv.weight_v"].astype(np.float64)
    default = x["enc.pos_conv_embed.conv.weight_g"] * v / np.sqrt((v * v).sum(axis=(1, 2), keepdims=True))
    info = g.tensors["enc.pos_conv_embed.conv.weight"]
    got = np.frombuffer(raw, np.float32, v.size, info["f32_offset"]).reshape(v.shape)
    assert np.abs(got - default).max() > 0.1
    g.close()
