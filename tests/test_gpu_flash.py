"""Flash attention (bf16 MFMA) against the oracle's materialised-probability attention.

Inputs are rounded to bf16 first, so the oracle sees the same q/k/v/dO as the
kernel; the remaining difference is the kernel's bf16 rounding of P and dS
(tolerance 2e-2 norm-wise, the bf16 bar).
"""
import ctypes

import numpy as np
import pytest
import torch

import sharpmind_amd
from sharpmind_amd import check

from conftest import rel_err

pytestmark = pytest.mark.gpu
TOL = 2e-2


def _bf16_round(a):
    return torch.from_numpy(a).to(torch.bfloat16).float().numpy()


def _oracle(orc, q, k, v, dO, B, S, Hq, Hkv, D):
    probs = np.zeros((B, Hq, S, S), np.float32)
    out = np.zeros((B, S, Hq * D), np.float32)
    orc.orc_attention_fwd(q, k, v, probs, out, B, S, Hq, Hkv, D)
    dq = np.zeros((B, S, Hq, D), np.float32)
    dk = np.zeros((B, S, Hkv, D), np.float32)
    dv = np.zeros((B, S, Hkv, D), np.float32)
    g = Hq // Hkv
    for b in range(B):
        for h in range(Hq):
            tq, tk, tv = (np.zeros((S, D), np.float32) for _ in range(3))
            orc.orc_grad_attention(np.ascontiguousarray(dO[b, :, h]), np.ascontiguousarray(q[b, :, h]),
                                   np.ascontiguousarray(k[b, :, h // g]), np.ascontiguousarray(v[b, :, h // g]),
                                   np.ascontiguousarray(probs[b, h]), tq, tk, tv, S, D, float(1 / np.sqrt(D)))
            dq[b, :, h] = tq
            dk[b, :, h // g] += tk
            dv[b, :, h // g] += tv
    return probs, out, dq, dk, dv


@pytest.mark.parametrize("B,S,Hq,Hkv,D", [(2, 256, 4, 2, 128), (1, 384, 2, 2, 64), (1, 128, 8, 1, 128), (1, 1024, 4, 2, 128),
                                         (1, 512, 2, 1, 64)])
def test_flash_forward_backward(orc, dev, B, S, Hq, Hkv, D):
    rng = np.random.default_rng(S + D + Hq)
    q = _bf16_round(rng.standard_normal((B, S, Hq, D)).astype(np.float32))
    k = _bf16_round(rng.standard_normal((B, S, Hkv, D)).astype(np.float32))
    v = _bf16_round(rng.standard_normal((B, S, Hkv, D)).astype(np.float32))
    dO = _bf16_round(rng.standard_normal((B, S, Hq, D)).astype(np.float32))
    probs, ro, rdq, rdk, rdv = _oracle(orc, q, k, v, dO, B, S, Hq, Hkv, D)
    L = sharpmind_amd.lib()
    tq, tk, tv, tdo = (torch.from_numpy(a).to(dev).to(torch.bfloat16).contiguous() for a in (q, k, v, dO))
    o = torch.empty(B, S, Hq, D, device=dev, dtype=torch.bfloat16)
    lse = torch.empty(B, Hq, S, device=dev)
    s = torch.cuda.current_stream().cuda_stream
    qd, kvd = Hq * D, Hkv * D
    check(L.smhip_flash_attention_forward(tq.data_ptr(), tk.data_ptr(), tv.data_ptr(), o.data_ptr(), lse.data_ptr(),
                                          B, S, Hq, Hkv, D, qd, kvd, kvd, qd, s))
    torch.cuda.synchronize()
    assert rel_err(o.float().cpu().numpy().reshape(B, S, qd), ro) <= TOL
    # lse in log2 units: log2 sum_j exp(s_ij) over the causal row
    sc = np.einsum("bihd,bjhd->bhij", q.astype(np.float64), np.repeat(k, Hq // Hkv, axis=2)) / np.sqrt(D)
    mask = np.triu(np.ones((S, S), bool), 1)
    sc = np.where(mask, -np.inf, sc)
    mx = sc.max(-1, keepdims=True)
    ref_lse = (np.log(np.exp(sc - mx).sum(-1)) + mx[..., 0]) / np.log(2)
    assert np.abs(lse.cpu().numpy() - ref_lse).max() < 1e-3
    dq = torch.empty(B, S, Hq, D, device=dev)
    dk = torch.empty(B, S, Hkv, D, device=dev)
    dv = torch.empty(B, S, Hkv, D, device=dev)
    check(L.smhip_flash_attention_backward(tq.data_ptr(), tk.data_ptr(), tv.data_ptr(), o.data_ptr(), tdo.data_ptr(),
                                           lse.data_ptr(), dq.data_ptr(), dk.data_ptr(), dv.data_ptr(), B, S, Hq, Hkv,
                                           D, qd, kvd, kvd, qd, qd, qd, kvd, kvd, s))
    torch.cuda.synchronize()
    assert rel_err(dq.cpu().numpy(), rdq) <= TOL
    assert rel_err(dk.cpu().numpy(), rdk) <= TOL
    assert rel_err(dv.cpu().numpy(), rdv) <= TOL
    # determinism: a second backward is bit-identical
    dq2 = torch.empty_like(dq)
    check(L.smhip_flash_attention_backward(tq.data_ptr(), tk.data_ptr(), tv.data_ptr(), o.data_ptr(), tdo.data_ptr(),
                                           lse.data_ptr(), dq2.data_ptr(), dk.data_ptr(), dv.data_ptr(), B, S, Hq, Hkv,
                                           D, qd, kvd, kvd, qd, qd, qd, kvd, kvd, s))
    torch.cuda.synchronize()
    assert torch.equal(dq, dq2)


def _run(L, dev, q, k, v, dO, B, S, Hq, Hkv, D, shift):
    """Forward + backward with q and k starting `shift` elements into their buffers."""
    s = torch.cuda.current_stream().cuda_stream
    qd, kvd = Hq * D, Hkv * D

    def place(a, off):
        buf = torch.zeros(a.size + 8, device=dev, dtype=torch.bfloat16)
        buf[off:off + a.size] = torch.from_numpy(a.ravel()).to(dev).to(torch.bfloat16)
        return buf, buf[off:].data_ptr()

    (bq, pq), (bk, pk) = place(q, shift), place(k, shift)
    (bv, pv), (bo, pdo) = place(v, 0), place(dO, 0)
    o = torch.zeros(B * S, qd, device=dev, dtype=torch.bfloat16)
    lse = torch.empty(B, Hq, S, device=dev)
    check(L.smhip_flash_attention_forward(pq, pk, pv, o.data_ptr(), lse.data_ptr(), B, S, Hq, Hkv, D, qd, kvd, kvd, qd, s))
    dq = torch.empty(B * S, qd, device=dev)
    dk = torch.empty(B * S, kvd, device=dev)
    dv = torch.empty(B * S, kvd, device=dev)
    check(L.smhip_flash_attention_backward(pq, pk, pv, o.data_ptr(), pdo, lse.data_ptr(), dq.data_ptr(), dk.data_ptr(),
                                           dv.data_ptr(), B, S, Hq, Hkv, D, qd, kvd, kvd, qd, qd, qd, kvd, kvd, s))
    torch.cuda.synchronize()
    return o, lse, dq, dk, dv


@pytest.mark.parametrize("S", [256, 384])
def test_flash_d128_dma_matches_register_staging(dev, S):
    """Head dim 128 with 16-byte aligned q/k/v/dO takes the DMA-staged kernels (tiles copied global
    -> LDS, transposed operands read with ds_read_b64_tr_b16); q and k 8 bytes off that alignment
    take the register-staged kernels.  Both compute in the same order: bit-identical."""
    B, Hq, Hkv, D = 2, 4, 2, 128
    rng = np.random.default_rng(S)
    q, dO = (_bf16_round(rng.standard_normal((B, S, Hq, D)).astype(np.float32)) for _ in range(2))
    k, v = (_bf16_round(rng.standard_normal((B, S, Hkv, D)).astype(np.float32)) for _ in range(2))
    L = sharpmind_amd.lib()
    a = _run(L, dev, q, k, v, dO, B, S, Hq, Hkv, D, 0)
    b = _run(L, dev, q, k, v, dO, B, S, Hq, Hkv, D, 4)
    for x, y in zip(a, b):
        assert torch.equal(x, y)
