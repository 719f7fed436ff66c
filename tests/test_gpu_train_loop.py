"""The engine driven the way TrainLoop.RunAsync drives the reference (TrainLoop.cs:104-135).

- Gradient accumulation: ZeroGrad only at the start of a GradAccumSteps window, then every
  micro-batch's gradients add up (TrainLoop.cs:108-120).  Checked against the oracle, whose
  gradient buffers accumulate the same way, and graph replay against eager launches.
- Per-step learning rate: _optimizer.LearningRate = scheduler.GetLr(step + 1) before each
  Update (TrainLoop.cs:122-123).
- Clipping actually triggered: Gradients.ClipGlobalNorm (Gradients.cs:92-116) scales every
  gradient by maxNorm / ||g|| when ||g|| > maxNorm, before AdamW.
"""
import numpy as np
import pytest
import torch

import oracle
from sharpmind_amd.engine import next_token_labels
from sharpmind_amd.model import PREC_BF16, QTYPE_Q8_0, ModelConfig, tensor_specs

from conftest import rel_err
from test_gpu_engine import _ocfg, build

pytestmark = pytest.mark.gpu


def _lora_cfg(precision=0):
    return ModelConfig(n_layers=2, d_model=256, n_heads=4, n_kv_heads=2, head_dim=64, ffn_dim=512, vocab=512, batch=2,
                       seq=128 if precision else 32, rope_theta=1e6, rope_neox=1, qk_norm=1, base_qtype=QTYPE_Q8_0,
                       lora_rank=4, lora_alpha=8.0, precision=precision)


def _batches(c, dev, n, seed):
    rng = np.random.default_rng(seed)
    out = []
    for _ in range(n):
        ids = torch.from_numpy(rng.integers(0, c.vocab, c.tokens).astype(np.int32)).to(dev)
        out.append((ids, next_token_labels(ids, c.seq)))
    return out


def test_grad_accumulation_matches_oracle(orc, dev):
    """Three micro-batches accumulated (fp32 mode) == the oracle's accumulated gradients (1e-5)."""
    c = _lora_cfg()
    eng, P, G = build(orc, c, 31)
    batches = _batches(c, dev, 3, 32)
    for i, (ids, lab) in enumerate(batches):
        eng.forward_backward(ids, lab, accumulate=i > 0)
        oracle.engine_step(_ocfg(c), P, G, ids.cpu().numpy(), lab.cpu().numpy())
    torch.cuda.synchronize()
    errs = {n: rel_err(eng.get(n, g.shape, grad=True), g) for n, g in G.items()}
    assert max(errs.values()) <= 1e-5, sorted(errs.items(), key=lambda kv: -kv[1])[:5]
    # a new window starts from zero again
    eng.forward_backward(*batches[0])
    G1 = {n: np.zeros_like(g) for n, g in G.items()}
    oracle.engine_step(_ocfg(c), P, G1, batches[0][0].cpu().numpy(), batches[0][1].cpu().numpy())
    errs = {n: rel_err(eng.get(n, g.shape, grad=True), g) for n, g in G1.items()}
    assert max(errs.values()) <= 1e-5


def test_grad_accumulation_graph_matches_eager(orc, dev):
    """bf16 graph mode: a window of two micro-batches replayed as graphs gives the eager window's bits."""
    c = _lora_cfg(PREC_BF16)
    eng, P, G = build(orc, c, 33, init="config")
    batches = _batches(c, dev, 2, 34)
    names = list(G)

    def window():
        for i, (ids, lab) in enumerate(batches):
            eng.forward_backward(ids, lab, accumulate=i > 0)
        torch.cuda.synchronize()
        return {n: eng.get(n, G[n].shape, grad=True) for n in names}

    ref = window()
    eng.use_graph(True)
    for _ in range(2):
        got = window()
        for n in names:
            assert np.array_equal(got[n], ref[n]), n


def test_set_lr_and_clip_match_reference(orc, dev):
    """max_grad_norm below ||g||: the step clips (ClipGlobalNorm) and AdamW uses the learning rate
    set for this step; the new parameters equal the reference AdamW applied to the clipped
    gradients, and the clipped gradients equal g * maxNorm / ||g||."""
    c = _lora_cfg()
    eng, P, G = build(orc, c, 35, max_grad_norm=1e-3)
    ids, lab = _batches(c, dev, 1, 36)[0]
    eng.forward_backward(ids, lab)
    oracle.engine_step(_ocfg(c), P, G, ids.cpu().numpy(), lab.cpu().numpy())
    torch.cuda.synchronize()
    names = list(G)
    shapes = {n: s for n, s, _ in tensor_specs(c)}
    g0 = {n: eng.get(n, shapes[n], grad=True) for n in names}
    before = {n: eng.get(n, shapes[n]) for n in names}
    norm_sq = sum(float(np.sum(g.astype(np.float64) ** 2)) for g in g0.values())
    ref_norm_sq = sum(float(np.sum(g.astype(np.float64) ** 2)) for g in G.values())
    assert abs(norm_sq - ref_norm_sq) <= 2e-5 * ref_norm_sq
    norm = np.float32(np.sqrt(norm_sq))
    assert norm > 1e-3, "the test needs a gradient norm above max_grad_norm"
    eng.lr = 3e-4
    assert eng.lr == np.float32(3e-4)
    gns = torch.zeros(1, device=dev)
    eng.optimizer_step(gns)
    torch.cuda.synchronize()
    assert abs(float(gns.cpu()[0]) - norm_sq) <= 1e-6 * norm_sq
    scale = np.float32(1e-3) / norm
    bc1 = float(np.float32(1) - np.float32(0.9))
    bc2 = float(np.float32(1) - np.float32(0.95))
    for n in names:
        clipped = eng.get(n, shapes[n], grad=True)
        assert rel_err(clipped, g0[n] * scale) <= 1e-6, n
        ref = before[n].copy().ravel()
        m, v = np.zeros_like(ref), np.zeros_like(ref)
        orc.orc_adamw(ref, np.ascontiguousarray(clipped.ravel()), m, v, ref.size, 0.9, 0.95, bc1, bc2, 3e-4, 1e-8, 0.1)
        assert np.array_equal(eng.get(n, shapes[n]).ravel(), ref), n
