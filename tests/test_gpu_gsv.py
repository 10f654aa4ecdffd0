"""The .gsv upload on the GPU: both segment arenas arrive bit-exact, the per-tensor device views
equal the file's arrays, and a decode step built from a .gsv (t2s_model_from_gsv, the names
T2SEngine's loader reads) matches the oracle chain run on the same weights."""
import numpy as np
import pytest
import torch

import gsvk
import oracle as O
from gpu_util import F16, F32, host, say
from gsv_writer import gsv_bytes, sovits_dec_tensors, t2s_tensors
from test_gpu_t2s_decode import compare, oracle_step

pytestmark = pytest.mark.gpu


def test_upload_arenas_bit_exact(tmp_path):
    t, cfg = t2s_tensors(seed=4)
    p = tmp_path / "m.gsv"
    p.write_bytes(gsv_bytes("ar_s1v3", t, cfg))
    g = gsvk.GsvFile(str(p))
    a16, v16 = g.upload(gsvk.F16)
    a32, v32 = g.upload(gsvk.F32)
    torch.cuda.synchronize()
    say(f"gsv arenas: fp16 {a16.numel()} B, fp32 {a32.numel()} B")
    for name, arr in t.items():
        np.testing.assert_array_equal(v32[name].cpu().numpy(), arr.astype(np.float32))
        if arr.size >= 4096:
            assert np.array_equal(v16[name].cpu().numpy().view(np.uint16),
                                  arr.astype(np.float16).view(np.uint16))
        else:
            assert name not in v16


def test_upload_reference_converter_file_bit_exact():
    """The arenas of a file the reference's convert.py wrote (tests/golden/convert_gsv1_small.gsv)
    arrive bit for bit: every device view equals the file's bytes at the directory's offsets."""
    from test_gsv_loader import GOLDEN_GSV
    raw = open(GOLDEN_GSV, "rb").read()
    g = gsvk.GsvFile(GOLDEN_GSV)
    a16, v16 = g.upload(gsvk.F16)
    a32, v32 = g.upload(gsvk.F32)
    torch.cuda.synchronize()
    assert set(v32) == set(g.tensors) and set(v16) == {"enc.weight", "dec.lin.weight"}
    for name, info in g.tensors.items():
        want = np.frombuffer(raw, np.uint32, info["numel"], info["f32_offset"])
        assert np.array_equal(v32[name].cpu().numpy().view(np.uint32).ravel(), want), name
        if info["f16_nbytes"]:
            want = np.frombuffer(raw, np.uint16, info["numel"], info["f16_offset"])
            assert np.array_equal(v16[name].cpu().numpy().view(np.uint16).ravel(), want), name
    g.close()


def test_decode_step_from_gsv_matches_oracle(tmp_path):
    D, H, FF, L, V, B, max_len = 128, 4, 256, 2, 50, 5, 64
    t, cfg = t2s_tensors(D, H, FF, L, V, seed=5)
    p = tmp_path / "m.gsv"
    p.write_bytes(gsv_bytes("ar_s1v3", t, cfg))
    g = gsvk.GsvFile(str(p))
    m, arenas = gsvk.t2s_model_from_gsv(g)
    r = np.random.default_rng(6)
    caches = [(O.to_storage(F16, r.standard_normal((B, max_len, D)).astype(np.float32)),
               O.to_storage(F16, r.standard_normal((B, max_len, D)).astype(np.float32)))
              for _ in range(L)]
    for ly, (kc, vc) in zip(m["layers"], caches):
        ly["k_cache"] = torch.from_numpy(kc.view(np.int16)).view(torch.float16).cuda()
        ly["v_cache"] = torch.from_numpy(vc.view(np.int16)).view(torch.float16).cuda()
    m["pe"] = torch.from_numpy(gsvk.pe_table(256, D)).cuda()
    io_h = dict(ids=r.integers(0, V, B).astype(np.int64), pos=r.integers(0, 200, B).astype(np.int64),
                kv_pos=r.integers(0, max_len, B).astype(np.int64))
    iod = dict(ids=torch.from_numpy(io_h["ids"]).cuda(), pos=torch.from_numpy(io_h["pos"]).cuda(),
               kv_pos=torch.from_numpy(io_h["kv_pos"]).cuda(),
               err=torch.zeros(1, dtype=torch.int32, device="cuda"),
               x=torch.empty(B, D, dtype=torch.float16, device="cuda"),
               h=torch.empty(B, D, dtype=torch.float16, device="cuda"),
               z=torch.empty(B, D, dtype=torch.float16, device="cuda"),
               attn=torch.empty(B, D, dtype=torch.float16, device="cuda"),
               ff=torch.empty(B, FF, dtype=torch.float16, device="cuda"),
               qkv=torch.empty(B, 3 * D, dtype=torch.float32, device="cuda"),
               logits=torch.empty(B, V, dtype=torch.float32, device="cuda"))
    step = gsvk.T2SDecode(m, iod, len_bound=max_len)
    step.run()
    torch.cuda.synchronize()
    # the same model on the host, from the same arrays (fp16 weights; fp32 biases / norms / alpha)
    mh = dict(table=t["ar_audio_embedding.word_embeddings.weight"].view(np.uint16),
              pe=gsvk.pe_table(256, D), alpha=np.float32(t["ar_audio_position.alpha"][0]),
              heads=H, w_logits=t["ar_predict_layer.weight"].view(np.uint16), layers=[])
    for l in range(L):
        pfx, ps = f"h.layers.{l}.", f"h.layers.{l}.self_attn."
        f32 = lambda k: t[k].astype(np.float32)
        mh["layers"].append(dict(
            wqkv=t[ps + "in_proj_weight"].view(np.uint16), bqkv=f32(ps + "in_proj_bias"),
            wout=t[ps + "out_proj.weight"].view(np.uint16), bout=f32(ps + "out_proj.bias"),
            n1g=f32(pfx + "norm1.weight"), n1b=f32(pfx + "norm1.bias"),
            w1=t[pfx + "linear1.weight"].view(np.uint16), b1=f32(pfx + "linear1.bias"),
            w2=t[pfx + "linear2.weight"].view(np.uint16), b2=f32(pfx + "linear2.bias"),
            n2g=f32(pfx + "norm2.weight"), n2b=f32(pfx + "norm2.bias"),
            k_cache=caches[l][0].copy(), v_cache=caches[l][1].copy()))
    x_want, lg_want = oracle_step(mh, io_h)
    compare(host(iod["x"], F16), host(iod["logits"], F32), x_want, lg_want, "from .gsv")


def test_sovits_decoder_from_gsv_matches_oracle(tmp_path):
    """The decoder bound to a sovits .gsv by Generator::load's names (dec.hpp:54-75). The upsampler
    and ResBlock weights are written without an fp16 copy, as the converter writes weight-norm
    products (convert.py:75-82), so the loader rounds their fp32 values to fp16 on the device;
    conv_pre, cond and conv_post come from their fp16 copies. The oracle chain runs on the same
    fp16 weights (numpy's round to nearest even): within the decoder test's 1e-4."""
    from test_gpu_sovits_decoder import oracle_decoder
    c_z, c0, g_in, frames = 16, 64, 32, 8
    t = sovits_dec_tensors(c_z, c0, g_in, seed=11)
    no16 = [k for k in t if k.startswith(("dec.ups.", "dec.resblocks.")) and k.endswith(".weight")]
    p = tmp_path / "s2.gsv"
    p.write_bytes(gsv_bytes("sovits_v2ProPlus", t, None, no16=no16))
    g = gsvk.GsvFile(str(p))
    assert all(g.tensors[k]["f16_nbytes"] == 0 for k in no16)
    assert g.tensors["dec.conv_pre.weight"]["f16_nbytes"] > 0
    h16 = lambda k: t[k].astype(np.float16)
    m = {"pre": (h16("dec.conv_pre.weight"), t["dec.conv_pre.bias"]),
         "cond": (h16("dec.cond.weight"), t["dec.cond.bias"]), "post": h16("dec.conv_post.weight"),
         "stages": []}
    for i in range(5):
        rbs = []
        for j in range(3):
            q = f"dec.resblocks.{3 * i + j}."
            rbs.append(([h16(f"{q}convs1.{k}.weight") for k in range(3)],
                        [t[f"{q}convs1.{k}.bias"] for k in range(3)],
                        [h16(f"{q}convs2.{k}.weight") for k in range(3)],
                        [t[f"{q}convs2.{k}.bias"] for k in range(3)]))
        m["stages"].append(((h16(f"dec.ups.{i}.weight"), t[f"dec.ups.{i}.bias"]), rbs))
    r = np.random.default_rng(12)
    z = r.standard_normal((c_z, frames)).astype(np.float32)
    ge = r.standard_normal(g_in).astype(np.float32)
    want = oracle_decoder(m, z, ge)
    out = torch.full((frames * 640,), float("nan"), device="cuda")
    dec, arenas = gsvk.sovits_decoder_from_gsv(g, torch.from_numpy(z).cuda(),
                                               torch.from_numpy(ge).cuda(), out)
    dec.run()
    torch.cuda.synchronize()
    got = host(out, F32)
    err = np.abs(got.astype(np.float64) - want.astype(np.float64)).max()
    say(f"sovits decoder from .gsv: max |d| {err:.2e}")
    assert np.isfinite(got).all() and err <= 1e-4


def test_cpp_generator_mirror_matches_python_decoder(tmp_path):
    """The C++ host mirror (gsv::sovits::Generator in host/gsvk/sovits.hpp, driven by the
    sovits_run example in its own process) loads the same .gsv by Generator::load's names
    (dec.hpp:54-75) and runs the same launches as the Python binding's decoder: bit-identical."""
    import os
    import subprocess
    exe = os.path.join(os.path.dirname(gsvk.__file__), "sovits_run")
    assert os.path.exists(exe), "sovits_run not built (make -C gpt-sovits-native_amd)"
    c_z, c0, g_in, frames = 16, 64, 32, 9
    t = sovits_dec_tensors(c_z, c0, g_in, seed=21)
    no16 = [k for k in t if k.startswith("dec.resblocks.") and k.endswith(".weight")]
    p = tmp_path / "s2.gsv"
    p.write_bytes(gsv_bytes("sovits_v2ProPlus", t, None, no16=no16))
    r = np.random.default_rng(22)
    z = r.standard_normal((c_z, frames)).astype(np.float32)
    ge = r.standard_normal(g_in).astype(np.float32)
    z.tofile(tmp_path / "z.f32")
    ge.tofile(tmp_path / "ge.f32")
    say(f"sovits_run: c0 {c0} frames {frames}")
    res = subprocess.run([exe, str(p), str(tmp_path / "z.f32"), str(frames),
                          str(tmp_path / "ge.f32"), str(tmp_path / "out.f32")],
                         capture_output=True, text=True, timeout=120)
    assert res.returncode == 0, res.stderr[-2000:]
    got = np.fromfile(tmp_path / "out.f32", dtype=np.float32)
    assert got.shape == (frames * 640,)

    g = gsvk.GsvFile(str(p))
    out = torch.full((frames * 640,), float("nan"), device="cuda")
    dec, arenas = gsvk.sovits_decoder_from_gsv(g, torch.from_numpy(z).cuda(),
                                               torch.from_numpy(ge).cuda(), out, graph=False)
    dec.run()
    torch.cuda.synchronize()
    want = host(out, F32)
    assert np.isfinite(got).all()
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
