"""Shared pieces of the SoVITS decoder GPU tests: random stage weights of the reference's geometry
(ResBlock1 kernels 3 / 7 / 11, conv1 dilations 1 / 3 / 5; dec.hpp:54-75), the oracle chained in
Generator::forward's order (dec.hpp:283-336) and the device objects built from the same weights.
"""
import numpy as np

import gsvk
import oracle as O
from gpu_util import F16, F32, dev, devf

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


def round_f16(a):
    """The convolutions' round_x input: fp32 activations rounded to fp16 (to nearest even)."""
    return O.to_f32(F16, O.to_storage(F16, a))


def oracle_stage(x, up, rbs, u, slope_next, round_x=False):
    """One Generator stage on the oracle: ups, three ResBlock1 chains, the branch mean and the next
    LeakyReLU. round_x: every convolution sees its input rounded to fp16 (residuals stay fp32)."""
    q = round_f16 if round_x else (lambda a: a)
    w_up, b_up = up
    y = O.convt1d(F32, q(x), w_up.view(np.uint16), u, b_up)
    curs = []
    for w1, b1, w2, b2 in rbs:
        cur = y.copy()
        for m in range(3):
            t_in = O.leaky_relu(F32, cur, 0.1)
            t_a = O.conv1d(F32, q(t_in), w1[m].view(np.uint16), b1[m], DILATIONS[m], epi=1,
                           slope=0.1)
            t_b = O.conv1d(F32, q(t_a), w2[m].view(np.uint16), b2[m], 1)
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
