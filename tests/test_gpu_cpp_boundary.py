"""The reference-named C++ boundary (gpt-sovits-native_amd/host/gsvk/kern.hpp) executed on device
buffers: host/examples/kern_run calls gsv::kern::layernorm / layernorm_rows / relu,
gsv::sovits::leaky_relu_io / leaky_relu_write / add_inplace / add_scaled_inplace / mul_write,
gsv::bert::LayerNorm1D::forward(Matrix&), a Tensor2D-backed leaky_relu_io and
gsv::ar::PeRows::pe_row and gsv::ar::prefill_input exactly as the reference's engines call them (kern.hpp:25, 33;
nn_ops.hpp:48-105; bert_ops.hpp:261-286; sovits_types.hpp:21-36; t2s_engine.hpp:187), in its own
process. Every output is checked against the oracle: bit-exact for ReLU, LeakyReLU, the adds and
the PE rows; the LayerNorms within the fp32 tolerance (1e-6 + 1e-5 |want|)."""
import os
import subprocess

import numpy as np
import pytest

import gsvk
import oracle as O
from gpu_util import F16, F32, assert_bitexact, assert_close, say

pytestmark = pytest.mark.gpu

EXE = os.path.join(os.path.dirname(gsvk.LIB_PATH), "kern_run")


def test_cpp_kernel_layer_on_device_buffers(tmp_path):
    assert os.path.exists(EXE), "kern_run is not built (make -C gpt-sovits-native_amd)"
    R, N, M = 4, 512, 4101
    r = np.random.default_rng(20250823 + 77)
    x = (r.standard_normal((R, N)) * 1.5 + 0.25).astype(np.float32)
    g = (1 + 0.1 * r.standard_normal(N)).astype(np.float32)
    b = (0.1 * r.standard_normal(N)).astype(np.float32)
    v = r.standard_normal(M).astype(np.float32)
    v[:4] = [0.0, -0.0, 1e-40, -1e-40]
    w = r.standard_normal(M).astype(np.float32)
    slope, scale, eps = np.float32(0.1), np.float32(1.0 / 3.0), np.float32(1e-5)
    src = tmp_path / "in.f32"
    dst = tmp_path / "out.f32"
    np.concatenate([x.ravel(), g, b, v, w, [slope, scale, eps]]).astype(np.float32).tofile(src)
    say("kern_run on device buffers")
    res = subprocess.run([EXE, str(src), str(dst), str(R), str(N), str(M)], capture_output=True,
                         text=True, timeout=120)
    assert res.returncode == 0, res.stderr
    out = np.fromfile(dst, dtype=np.float32)
    sizes = [N, R * N, M, M, M, M, M, M, R * N, 3 * (M // 3), 6 * N, 4 * R * N]
    assert out.size == sum(sizes)
    parts = np.split(out, np.cumsum(sizes)[:-1])

    assert_close(F32, parts[0], O.add_layernorm(F32, x[:1].copy(), g, b, float(eps))[0],
                 "layernorm")
    assert_close(F32, parts[1].reshape(R, N), O.add_layernorm(F32, x, g, b, float(eps)),
                 "layernorm_rows")
    assert_bitexact(F32, parts[2], O.relu(v), "relu")
    assert_bitexact(F32, parts[3], O.leaky_relu(F32, v, float(slope)), "leaky_relu_io")
    assert_bitexact(F32, parts[4], O.leaky_relu(F32, v, float(slope)), "leaky_relu_write")
    add, _ = O.resblock_add_lrelu(F32, v, w, 0.0, write_tin=False)
    assert_bitexact(F32, parts[5], add, "add_inplace")
    assert_bitexact(F32, parts[6], O.scaled_add(F32, v, w, float(scale)), "add_scaled_inplace")
    assert_bitexact(F32, parts[7], O.scaled_add(F32, None, w, float(scale)), "mul_write")
    assert_close(F32, parts[8].reshape(R, N),
                 O.add_layernorm(F32, x, g, b, 1e-12, mode=1), "LayerNorm1D::forward")
    assert_bitexact(F32, parts[9], O.leaky_relu(F32, v[:3 * (M // 3)].copy(), 0.01),
                    "Tensor2D leaky_relu_io")
    pe = parts[10].reshape(6, N)
    table = O.pe_table(2048, N)
    for i, p in enumerate((0, 1, 7, 166, 1234, 2047)):
        assert np.array_equal(pe[i].view(np.uint32), table[p].view(np.uint32)), f"pe_row({p})"
    # prefill_input: text rows over the bert_proj rows in place, then prompt rows, bit-exact
    T = P = 2 * R
    tab16 = x.astype(np.float16).view(np.uint16)
    ph = (np.arange(T) % R).astype(np.int64)
    pr = (R - 1 - np.arange(P) % R).astype(np.int64)
    want_t, _ = O.embed_pe(F32, F16, tab16, ph, table, 0.75, pos0=0,
                           mm=w[:T * N].reshape(T, N).copy(), bias=b)
    want_a, _ = O.embed_pe(F32, F16, tab16, pr, table, 1.25, pos0=0)
    xy = parts[11].reshape(T + P, N)
    assert_bitexact(F32, xy[:T], want_t, "prefill_input text rows")
    assert_bitexact(F32, xy[T:], want_a, "prefill_input prompt rows")
