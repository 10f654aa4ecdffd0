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

from gpu_util import F32, devf, host, say
from sovits_util import gpu_stage, make_stage, oracle_stage

pytestmark = pytest.mark.gpu

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
