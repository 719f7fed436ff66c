"""smhip_flash_attention_backward_noalloc against smhip_flash_attention_backward.

The allocation-free entry uses the same kernels with its scratch in a fixed per-device array,
so its dQ/dK/dV must equal the pooled entry's bit for bit.  Two calls in a row, the second on
a smaller problem (the array keeps the first call's contents), plus the size limit: a problem
whose scratch exceeds the array is refused with SMHIP_EINVAL before anything is launched.
"""
import ctypes

import numpy as np
import pytest
import torch

import sharpmind_amd

pytestmark = pytest.mark.gpu


def _case(dev, B, S, Hq, Hkv, D, seed):
    g = torch.Generator(device="cpu").manual_seed(seed)
    mk = lambda h: torch.randn(B, S, h, D, generator=g).to(dev).to(torch.bfloat16).contiguous()
    q, k, v, dO = mk(Hq), mk(Hkv), mk(Hkv), mk(Hq)
    o = torch.empty(B, S, Hq, D, device=dev, dtype=torch.bfloat16)
    lse = torch.empty(B, Hq, S, device=dev)
    L = sharpmind_amd.lib()
    s = torch.cuda.current_stream().cuda_stream
    qd, kvd = Hq * D, Hkv * D
    sharpmind_amd.check(L.smhip_flash_attention_forward(q.data_ptr(), k.data_ptr(), v.data_ptr(), o.data_ptr(),
                                                        lse.data_ptr(), B, S, Hq, Hkv, D, qd, kvd, kvd, qd, s))
    return q, k, v, o, dO, lse


def _backward(dev, fn, case, B, S, Hq, Hkv, D):
    q, k, v, o, dO, lse = case
    qd, kvd = Hq * D, Hkv * D
    dq = torch.full((B, S, Hq, D), float("nan"), device=dev)
    dk = torch.full((B, S, Hkv, D), float("nan"), device=dev)
    dv = torch.full((B, S, Hkv, D), float("nan"), device=dev)
    rc = fn(q.data_ptr(), k.data_ptr(), v.data_ptr(), o.data_ptr(), dO.data_ptr(), lse.data_ptr(), dq.data_ptr(),
            dk.data_ptr(), dv.data_ptr(), B, S, Hq, Hkv, D, qd, kvd, kvd, qd, qd, qd, kvd, kvd,
            torch.cuda.current_stream().cuda_stream)
    sharpmind_amd.check(rc)
    torch.cuda.synchronize()
    return dq, dk, dv


def test_noalloc_matches_pooled_entry(dev):
    L = sharpmind_amd.lib()
    for (B, S, Hq, Hkv, D), seed in (((2, 1024, 16, 8, 128), 1), ((1, 256, 4, 2, 64), 2)):
        print("noalloc case", B, S, Hq, Hkv, D, flush=True)
        case = _case(dev, B, S, Hq, Hkv, D, seed)
        ref = _backward(dev, L.smhip_flash_attention_backward, case, B, S, Hq, Hkv, D)
        got = _backward(dev, L.smhip_flash_attention_backward_noalloc, case, B, S, Hq, Hkv, D)
        for a, b in zip(got, ref):
            assert torch.isfinite(b).all()
            assert torch.equal(a, b)


def test_noalloc_rejects_oversize(dev):
    L = sharpmind_amd.lib()
    lim = ctypes.c_int64()
    sharpmind_amd.check(L.smhip_flash_attention_backward_noalloc_limit(ctypes.byref(lim)))
    assert lim.value == 80 << 20
    B, S, Hq, Hkv, D = 8, 1024, 16, 8, 128  # 8*16*1024*257*4 bytes > 80 MiB
    assert B * Hq * S * (2 * D + 1) * 4 > lim.value
    t = torch.zeros(16, device=dev)
    p = t.data_ptr()
    rc = L.smhip_flash_attention_backward_noalloc(p, p, p, p, p, p, p, p, p, B, S, Hq, Hkv, D, Hq * D, Hkv * D, Hkv * D,
                                                  Hq * D, Hq * D, Hq * D, Hkv * D, Hkv * D, None)
    assert rc == -1
    assert b"exceed" in L.smhip_last_error()
