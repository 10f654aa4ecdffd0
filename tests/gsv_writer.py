"""Writes GSV1 containers for the loader tests, following the layout rules of the reference's
converter (tools/convert.py:4-22, 131-183): header, directory, then every fp32 segment followed by
every fp16 segment, each 64-byte aligned; an fp16 copy for tensors of >= 4096 elements; the config
JSON as {"meta": ..., "model_config": ...} with sorted keys. The reference's real weight files are
not available here, so the tests build their own."""
import json
import struct

import numpy as np

ALIGN = 64
FP16_MIN_ELEMS = 4096


def _up(n):
    return (n + ALIGN - 1) // ALIGN * ALIGN


def gsv_bytes(name, tensors, model_config=None, slim=(), no16=()):
    """tensors: dict name -> numpy array (float32 or float16 source). slim: names written with an
    fp16 copy only (f32 bytes 0). no16: names written without an fp16 copy whatever their size (the
    converter's weight-norm products, convert.py:75-82). Returns the file as bytes."""
    cfg = json.dumps({"meta": {"model": name, "converter": "convert.py GSV1"},
                      "model_config": model_config}, ensure_ascii=False, sort_keys=True).encode()
    nm = name.encode()
    fixed = 4 + 4 + 4 + 2 + len(nm) + 4 + len(cfg) + 4
    dir_size = sum(2 + len(k.encode()) + 2 + 4 * v.ndim + 2 + 32 for k, v in tensors.items())
    pos = _up(fixed + dir_size)
    layout = []
    for k, v in tensors.items():
        nb = 0 if k in slim else 4 * v.size
        layout.append([k, v, pos if nb else 0, nb, 0, 0])
        pos += _up(nb)
    has16 = False
    for e in layout:
        k, v = e[0], e[1]
        if (v.size >= FP16_MIN_ELEMS and k not in no16) or k in slim:
            e[4], e[5] = pos, 2 * v.size
            pos += _up(e[5])
            has16 = True
    buf = bytearray(struct.pack("<4sIIH", b"GSV1", 1, 1 if has16 else 0, len(nm)) + nm)
    buf += struct.pack("<I", len(cfg)) + cfg + struct.pack("<I", len(layout))
    for k, v, o32, nb32, o16, nb16 in layout:
        kb = k.encode()
        buf += struct.pack("<H", len(kb)) + kb
        buf += struct.pack("<H", v.ndim) + struct.pack(f"<{v.ndim}I", *v.shape)
        buf += struct.pack("<HQQQQ", 2 if v.dtype == np.float16 else 1, o32, nb32, o16, nb16)
    assert len(buf) == fixed + dir_size
    out = bytearray(pos)
    out[:len(buf)] = buf
    for k, v, o32, nb32, o16, nb16 in layout:
        if nb32:
            out[o32:o32 + nb32] = v.astype(np.float32).tobytes()
        if nb16:
            out[o16:o16 + nb16] = v.astype(np.float16).tobytes()
    return bytes(out)


def t2s_tensors(D=128, H=4, FF=256, L=2, V=50, PV=40, seed=0):
    """An ar_s1-shaped model with the tensor names T2SEngine reads (t2s_engine.cpp:575-627), fp16
    source weights like the released checkpoint."""
    r = np.random.default_rng(seed)
    f16 = lambda *s, std=0.05: (std * r.standard_normal(s)).astype(np.float16)
    t = {"ar_text_embedding.word_embeddings.weight": f16(PV, D, std=0.02),
         "ar_audio_embedding.word_embeddings.weight": f16(V, D, std=0.02),
         "ar_text_position.alpha": np.array([3.830078125], np.float16),
         "ar_audio_position.alpha": np.array([0.93017578125], np.float16),
         "ar_predict_layer.weight": f16(V, D), "bert_proj.weight": f16(D, 1024),
         "bert_proj.bias": f16(D, std=0.02)}
    for l in range(L):
        p, ps = f"h.layers.{l}.", f"h.layers.{l}.self_attn."
        t[ps + "in_proj_weight"] = f16(3 * D, D)
        t[ps + "in_proj_bias"] = f16(3 * D, std=0.02)
        t[ps + "out_proj.weight"] = f16(D, D)
        t[ps + "out_proj.bias"] = f16(D, std=0.02)
        t[p + "linear1.weight"] = f16(FF, D)
        t[p + "linear1.bias"] = f16(FF, std=0.02)
        t[p + "linear2.weight"] = f16(D, FF)
        t[p + "linear2.bias"] = f16(D, std=0.02)
        t[p + "norm1.weight"] = (1 + 0.1 * r.standard_normal(D)).astype(np.float16)
        t[p + "norm1.bias"] = f16(D, std=0.1)
        t[p + "norm2.weight"] = (1 + 0.1 * r.standard_normal(D)).astype(np.float16)
        t[p + "norm2.bias"] = f16(D, std=0.1)
    cfg = {"model": {"hidden_dim": D, "embedding_dim": D, "head": H, "n_layer": L,
                     "linear_units": FF, "vocab_size": V, "phoneme_vocab_size": PV, "EOS": V - 1}}
    return t, cfg


def sovits_dec_tensors(c_z=16, c0=64, g_in=32, seed=0):
    """A SoVITS decoder (Generator) with the tensor names Generator::load reads (dec.hpp:54-75), c0
    channels after conv_pre (the model's: 768), the model's strides, kernels and dilations; fp32
    weights whose fp16 copies the loader uses when present."""
    r = np.random.default_rng(seed)
    w = lambda co, ci, k: (r.standard_normal((co, ci, k)) / np.sqrt(ci * k)).astype(np.float32)
    b = lambda n: (0.05 * r.standard_normal(n)).astype(np.float32)
    t = {"dec.conv_pre.weight": w(c0, c_z, 7), "dec.conv_pre.bias": b(c0),
         "dec.cond.weight": w(c0, g_in, 1), "dec.cond.bias": b(c0)}
    c = c0
    for i, (u, k) in enumerate(zip((10, 8, 2, 2, 2), (20, 16, 8, 2, 2))):
        t[f"dec.ups.{i}.weight"] = (r.standard_normal((c, c // 2, k)) /
                                   np.sqrt(c * k / u)).astype(np.float32)
        t[f"dec.ups.{i}.bias"] = b(c // 2)
        c //= 2
        for j, kr in enumerate((3, 7, 11)):
            for m in range(3):
                for conv in ("convs1", "convs2"):
                    t[f"dec.resblocks.{3 * i + j}.{conv}.{m}.weight"] = w(c, c, kr)
                    t[f"dec.resblocks.{3 * i + j}.{conv}.{m}.bias"] = b(c)
    t["dec.conv_post.weight"] = w(1, c, 7)
    return t
