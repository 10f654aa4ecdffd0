"""Writes tests/golden/convert_gsv1_small.gsv with the reference's own converter (tools/convert.py,
`convert`: prefix stripping, weight-norm fusion, non-float skipping, the fp32 / fp16 segments) from
a small seeded state dict, so that the .gsv loader is checked against a file the reference wrote
(tests/test_gsv_loader.py, tests/test_gpu_gsv.py). It imports the converter from the reference
tree, so it runs only where that tree is (the build container); the fixture it writes is committed.

    python3 tests/golden/make_gsv_fixture.py

The state dict covers each rule of the converter once:
  - keys with the "model." and "module." prefixes (stripped);
  - a weight-norm pair with the default norm dims (all but dim 0), one with the pos_conv override
    (dims 0 and 1), and one whose fused product has >= 4096 elements (fused products get no fp16
    copy whatever their size);
  - fp32 and fp16 sources above and below the 4096-element fp16 threshold;
  - integer tensors (skipped).
"""
import os
import sys

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
OUT = os.path.join(HERE, "convert_gsv1_small.gsv")
SRC = "/tmp/gsvk_convert_fixture_src.pth"  # a fixed path: the converter records it in the file
REF_TOOLS = "/root/reference/tools"
SEED = 20261202


def state_dict(seed=SEED):
    """The converter's input. Kept in step with tests/test_gsv_loader.py::converter_inputs."""
    r = np.random.default_rng(seed)

    def f32(*shape):
        return torch.from_numpy(r.standard_normal(shape).astype(np.float32))

    def f16(*shape):
        return torch.from_numpy(r.standard_normal(shape).astype(np.float16))

    sd = {}
    sd["model.enc.weight"] = f32(64, 64)              # fp32 source, 4096 elements: fp16 copy
    sd["model.enc.bias"] = f32(64)                    # fp32 source, small: fp32 only
    sd["module.dec.lin.weight"] = f16(32, 160)        # fp16 source, 5120 elements: fp16 copy
    sd["module.dec.lin.bias"] = f16(32)               # fp16 source, small
    sd["model.dec.conv.weight_g"] = f16(16, 1, 1)     # weight norm, default dims (1, 2)
    sd["model.dec.conv.weight_v"] = f16(16, 8, 3)
    sd["model.big.weight_g"] = f32(64, 1, 1)          # fused product of 4096 elements: fp32 only
    sd["model.big.weight_v"] = f32(64, 16, 4)
    sd["model.enc.pos_conv_embed.conv.weight_g"] = f32(1, 1, 5)  # the dims (0, 1) override
    sd["model.enc.pos_conv_embed.conv.weight_v"] = f32(8, 4, 5)
    sd["model.position_ids"] = torch.arange(10, dtype=torch.int64)  # skipped (not float)
    sd["model.bn.num_batches_tracked"] = torch.tensor(5, dtype=torch.int64)  # skipped
    return sd


def main():
    sys.path.insert(0, REF_TOOLS)
    import convert  # the reference's converter (tools/convert.py)

    torch.save(state_dict(), SRC)
    convert.convert(SRC, OUT, "fixture_small", None, verify=True)
    os.remove(SRC)
    print(f"wrote {OUT} ({os.path.getsize(OUT)} bytes)")


if __name__ == "__main__":
    main()
