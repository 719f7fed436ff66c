"""Tied LM head forward + cross-entropy backward (smhip_lm_head_ce_bf16) against float64.

The logits are the fp32 MFMA sums of bf16 products (1e-5 bar against float64 on the
bf16-rounded inputs and the bit-exact dequantised table); dLogits are bf16 (2e-2 bar)
and the mean loss is held to 1e-5 relative.  Shapes with at least four 128x128 output
tiles per CU take the persistent GEMM that also emits the softmax row statistics
(max and sum of exponentials per row and 64 columns), so the cross-entropy reads the
logits once; the small shape takes the two-pass cross-entropy.
"""
import numpy as np
import pytest
import torch

import sharpmind_amd
from sharpmind_amd import check

from conftest import rel_err
from test_gpu_gemm import _quant, _rnd

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("T,V,d,qtype", [(256, 4096, 512, 8), (1024, 16384, 256, 8), (1024, 16384, 256, 12),
                                         (2048, 8192, 512, 8)])
def test_lm_head_ce(orc, dev, T, V, d, qtype):
    rng = np.random.default_rng(T + V + d + qtype)
    raw, deq = _quant(orc, qtype, (rng.standard_normal(V * d) * 0.05).astype(np.float32))
    eb = torch.from_numpy(deq).to(torch.bfloat16).double().numpy().reshape(V, d)
    x = _rnd((T, d), rng)
    lab = rng.integers(0, V, T).astype(np.int32)
    lab[rng.random(T) < 0.1] = -100
    tx = torch.from_numpy(x).to(dev).to(torch.bfloat16)
    logits = torch.empty(T, V, device=dev)
    dlog = torch.empty(T, V, device=dev, dtype=torch.bfloat16)
    loss = torch.zeros(1, device=dev)
    s = torch.cuda.current_stream().cuda_stream
    check(sharpmind_amd.lib().smhip_lm_head_ce_bf16(qtype, T, V, d, tx.data_ptr(), torch.from_numpy(raw).to(dev).data_ptr(),
                                                    torch.from_numpy(lab).to(dev).data_ptr(), logits.data_ptr(),
                                                    dlog.data_ptr(), loss.data_ptr(), s))
    torch.cuda.synchronize()
    z = x.astype(np.float64) @ eb.T
    assert rel_err(logits.cpu().numpy(), z) <= 1e-5
    keep = lab != -100
    zm = z - z.max(1, keepdims=True)
    p = np.exp(zm) / np.exp(zm).sum(1, keepdims=True)
    rows = np.nonzero(keep)[0]
    ref_loss = -np.log(p[rows, lab[rows]]).mean()
    g = p.copy()
    g[rows, lab[rows]] -= 1.0
    g /= keep.sum()
    g[~keep] = 0.0
    assert abs(float(loss.cpu()[0]) - ref_loss) <= 1e-5 * abs(ref_loss)
    assert rel_err(dlog.float().cpu().numpy(), g) <= 2e-2
