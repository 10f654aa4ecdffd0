"""A whole SoVITS Generator stage on the GPU (gsvk.GeneratorStage: upsampler, 3 ResBlocks x 3 fused
conv pairs, branch mean + next LeakyReLU) against the oracle chained in the reference's order
(Generator::forward, dec.hpp:283-336): ups, then per ResBlock cur = x and per pair t_in = lrelu(cur),
t_a = lrelu(conv1(t_in)), cur += conv2(t_a), then the 1/3-weighted sum and the next LeakyReLU.

Tolerance: each convolution meets its own bound (test_gpu_conv.py); chained through an upsampler and
six convolutions per branch, the fp32 noise of the summation order compounds, so the stage output is
compared at |d| <= 1e-4 * max(1, peak |want|) per channel. A wrong dilation, a dropped residual or a
missing activation moves outputs by O(peak), far outside it.
"""
import numpy as np
import pytest
import torch

import gsvk
import oracle as O
from gpu_util import F16, F32, dev, devf, host, say

pytestmark = pytest.mark.gpu

KERNELS = (3, 7, 11)
DILATIONS = (1, 3, 5)


def make_stage(r, cin_up, C, k_up, u):
    w_up = (r.standard_normal((cin_up, C, k_up)) / np.sqrt(cin_up * k_up / u)).astype(np.float16)
    b_up = (0.05 * r.standard_normal(C)).astype(np.float32)
    rbs = []
    for k in KERNELS:
        w1 = [(r.standard_normal((C, C, k)) / np.sqrt(C * k)).astype(np.float16) for _ in range(3)]
        w2 = [(r.standard_normal((C, C, k)) / np.sqrt(C * k)).astype(np.float16) for _ in range(3)]
        b1 = [(0.05 * r.standard_normal(C)).astype(np.float32) for _ in range(3)]
        b2 = [(0.05 * r.standard_normal(C)).astype(np.float32) for _ in range(3)]
        rbs.append((w1, b1, w2, b2))
    return (w_up, b_up), rbs


def oracle_stage(x, up, rbs, u, slope_next):
    w_up, b_up = up
    y = O.convt1d(F32, x, w_up.view(np.uint16), u, b_up)
    curs = []
    for w1, b1, w2, b2 in rbs:
        cur = y.copy()
        for m in range(3):
            t_in = O.leaky_relu(F32, cur, 0.1)
            t_a = O.conv1d(F32, t_in, w1[m].view(np.uint16), b1[m], DILATIONS[m], epi=1, slope=0.1)
            t_b = O.conv1d(F32, t_a, w2[m].view(np.uint16), b2[m], 1)
            cur, _ = O.resblock_add_lrelu(F32, cur, t_b, 0.1, write_tin=False)
        curs.append(cur)
    return O.resblock_branch_mean(F32, curs, None, True, slope_next)


def gpu_stage(up, rbs, u):
    w_up, b_up = up
    ups = gsvk.ConvT1d(dev(w_up.view(np.uint16), F16), devf(b_up), u)
    blocks = [gsvk.ResBlock1([dev(w.view(np.uint16), F16) for w in w1], [devf(b) for b in b1],
                             [dev(w.view(np.uint16), F16) for w in w2], [devf(b) for b in b2])
              for w1, b1, w2, b2 in rbs]
    return gsvk.GeneratorStage(ups, blocks)


@pytest.mark.parametrize("cin_up,C,T_in,k_up,u,slope_next", [
    (64, 32, 40, 16, 8, 0.1),    # a middle stage, narrowed (stage 2 of 5: 384 -> 192, k 16, u 8)
    (48, 24, 150, 2, 2, 0.01),   # the last stage's shape (48 -> 24, k 2, u 2), then lrelu(0.01)
    (96, 40, 30, 20, 10, 0.1),   # the first stage's upsampler (k 20, u 10), ragged channels
])
def test_generator_stage_matches_oracle_chain(cin_up, C, T_in, k_up, u, slope_next):
    r = np.random.default_rng(20250823 + 23000 + cin_up)
    x = r.standard_normal((cin_up, T_in)).astype(np.float32)
    up, rbs = make_stage(r, cin_up, C, k_up, u)
    want = oracle_stage(x, up, rbs, u, slope_next)
    stage = gpu_stage(up, rbs, u)
    out = torch.empty(C, T_in * u, dtype=torch.float32, device="cuda")
    stage.forward(devf(x), out, slope_next=slope_next)
    torch.cuda.synchronize()
    got = host(out, F32).astype(np.float64)
    w = want.astype(np.float64)
    peak = np.maximum(1.0, np.abs(w).max(axis=1, keepdims=True))
    err = np.abs(got - w) / peak
    say(f"stage {cin_up}->{C} T={T_in}x{u}: max |d| / peak {err.max():.2e}")
    assert err.max() <= 1e-4
    # the same stage twice gives the same bits
    out2 = torch.empty_like(out)
    stage.forward(devf(x), out2, slope_next=slope_next)
    torch.cuda.synchronize()
    assert np.array_equal(host(out2, F32).view(np.uint32), host(out, F32).view(np.uint32))
