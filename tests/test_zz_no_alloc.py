"""gsvk_decode_attention_noalloc (the entry point that allocates nothing) against
gsvk_decode_attention with a caller workspace, through the C ABI: the same kernels and the same
partition of the keys, so the outputs must be bitwise equal. Two calls in a row, the second with a
smaller batch and shorter contexts (the library's device array keeps the first call's chunk states;
the second must not depend on them), for fp16 and fp32 caches; both calls split keys into several
chunks, so the array is in use."""
import numpy as np
import pytest
import torch

import gsvk
from gpu_util import say

pytestmark = pytest.mark.gpu


def _case(B, L, kv, seed):
    g = torch.Generator(device="cuda").manual_seed(seed)
    D, H = 512, 16
    max_len = L + 16
    kc = torch.randn(B, max_len, D, device="cuda", generator=g).to(kv)
    vc = torch.randn(B, max_len, D, device="cuda", generator=g).to(kv)
    qkv = torch.randn(B, 3 * D, device="cuda", generator=g)
    pos = torch.randint(L // 2, L, (B,), device="cuda", generator=g)
    return kc, vc, qkv, pos, H, D


@pytest.mark.parametrize("kv", [torch.float16, torch.float32])
def test_noalloc_attention_equals_workspace_form(kv):
    for call, (B, L) in enumerate(((64, 1100), (8, 600))):
        say(f"noalloc attention call {call}: B={B} L={L} kv={kv}")
        kc, vc, qkv, pos, H, D = _case(B, L, kv, 900 + call)
        lb = L
        assert gsvk.lib().gsvk_decode_attention_workspace_bytes(B, H, D // H, lb) > 0
        kc2, vc2 = kc.clone(), vc.clone()
        want = torch.empty(B, D, dtype=torch.float16, device="cuda")
        got = torch.full((B, D), float("nan"), dtype=torch.float16, device="cuda")
        err = torch.zeros(1, dtype=torch.int32, device="cuda")
        gsvk.decode_attention(qkv, kc, vc, pos, want, H, len_bound=lb, err=err)
        gsvk.decode_attention_noalloc(qkv, kc2, vc2, pos, got, H, len_bound=lb, err=err)
        torch.cuda.synchronize()
        assert int(err.item()) == 0
        assert torch.equal(got.view(torch.int16), want.view(torch.int16)), f"call {call}: out"
        assert torch.equal(kc2, kc) and torch.equal(vc2, vc), f"call {call}: appended rows"
        assert np.isfinite(got.float().cpu().numpy()).all()


def test_noalloc_attention_rejects_states_past_the_array():
    """4 MiB holds 1365 chunk states of 3 KiB. 700 sequences at contexts of up to 200 keys take two
    chunks each (1400 states): refused with GSVK_E_SIZE before anything is launched, and the
    workspace form of the same call still runs. 682 sequences (1364 states) fit."""
    D, H, L = 512, 16, 200
    for B, fits in ((682, True), (700, False)):
        say(f"noalloc attention capacity: B={B} L={L} fits={fits}")
        need = gsvk.lib().gsvk_decode_attention_workspace_bytes(B, H, D // H, L)
        assert need == B * 2 * 3072
        assert (need <= 4 << 20) == fits
        kc, vc, qkv, pos, H, D = _case(B, L, torch.float16, 950 + B)
        out = torch.empty(B, D, dtype=torch.float16, device="cuda")
        if fits:
            want = torch.empty_like(out)
            kc2, vc2 = kc.clone(), vc.clone()
            gsvk.decode_attention(qkv, kc2, vc2, pos, want, H, len_bound=L)
            gsvk.decode_attention_noalloc(qkv, kc, vc, pos, out, H, len_bound=L)
            torch.cuda.synchronize()
            assert torch.equal(out.view(torch.int16), want.view(torch.int16))
        else:
            before = kc.clone()
            with pytest.raises(gsvk.GsvkError) as e:
                gsvk.decode_attention_noalloc(qkv, kc, vc, pos, out, H, len_bound=L)
            assert e.value.status == gsvk.E_SIZE
            torch.cuda.synchronize()
            assert torch.equal(kc, before)  # nothing appended: no launch
