"""The benchmark configurations 3, 4 and 5 on the GPU.

Real widths against the oracle: each configuration's exact layer geometry (d_model,
heads, head_dim, FFN width, LoRA rank, base format) and sequence length, with one
layer, batch 1 and a reduced vocabulary so that the CPU oracle (oracle/engine.c)
finishes in seconds; every gradient is compared (bf16 bar 2e-2, fp32 bar 1e-5).

Full size (28 layers, vocabulary 151 936, the configuration's batch): properties
that do not need the oracle -- finite loss near ln(V) at initialisation, graph
replay bit-identical to eager launches, B = 0 => every dA = 0, the loss falls over
three optimizer steps on one batch, and (fp32 mode, config 4) a central finite
difference of the loss along the gradient direction of a few adapters equals the
gradient's norm.
"""
import math

import numpy as np
import pytest
import torch

import oracle
from sharpmind_amd.engine import Engine, next_token_labels
from sharpmind_amd.model import (PREC_BF16, PREC_FP32, QTYPE_F32, QTYPE_Q4_K, QTYPE_Q8_0, qwen3_0_6b, qwen3_1_7b,
                                 tensor_specs)

from conftest import rel_err
from test_gpu_engine import _ocfg, build

pytestmark = pytest.mark.gpu

CFGS = {
    "config3_full_bf16": lambda **k: qwen3_0_6b(batch=8, seq=512, qtype=QTYPE_F32, rank=0, alpha=0.0, **k),
    "config4_lora_q8": lambda **k: qwen3_0_6b(batch=4, seq=1024, qtype=QTYPE_Q8_0, rank=16, alpha=32.0, **k),
    "config5_lora_q4k": lambda **k: qwen3_1_7b(batch=2, seq=2048, qtype=QTYPE_Q4_K, rank=32, alpha=64.0, **k),
}


def _ids(c, dev, seed):
    ids = torch.from_numpy(np.random.default_rng(seed).integers(0, c.vocab, c.tokens).astype(np.int32)).to(dev)
    return ids, next_token_labels(ids, c.seq)


def _real_widths(name, precision=PREC_BF16):
    c = CFGS[name](precision=precision, layers=1)
    c.batch, c.vocab = 1, 4096
    return c


def _compare(orc, dev, c, seed, tol):
    eng, P, G = build(orc, c, seed, init="config")
    ids, lab = _ids(c, dev, seed + 1)
    loss = torch.zeros(1, device=dev)
    eng.forward_backward(ids, lab, loss)
    torch.cuda.synchronize()
    ref_loss = oracle.engine_step(_ocfg(c), P, G, ids.cpu().numpy(), lab.cpu().numpy())
    errs = {"loss": abs(float(loss.cpu()[0]) - ref_loss) / abs(ref_loss)}
    for n, g in G.items():
        errs[n] = rel_err(eng.get(n, g.shape, grad=True), g)
    worst = sorted(errs.items(), key=lambda kv: -kv[1])[:4]
    print(f"{c.d_model=} {c.seq=} worst {worst}")
    assert worst[0][1] <= tol, worst
    eng.close()


@pytest.mark.parametrize("name", list(CFGS))
def test_real_widths_bf16_vs_oracle(orc, dev, name):
    _compare(orc, dev, _real_widths(name), 101, 2e-2)


def test_config4_real_widths_fp32_vs_oracle(orc, dev):
    """The exactness mode (fp32 MFMA, materialised probabilities) at config 4's widths and S = 1024."""
    _compare(orc, dev, _real_widths("config4_lora_q8", PREC_FP32), 103, 1e-5)


def _full(name, precision=PREC_BF16, lr=1e-3):
    c = CFGS[name](precision=precision)
    eng = Engine(c, lr=lr, max_grad_norm=1.0)
    eng.init_synthetic(7)
    return c, eng


def _grads(eng, c, kind):
    return {n: eng.get(n, s, grad=True) for n, s, k in tensor_specs(c) if k in kind}


@pytest.mark.parametrize("name", list(CFGS))
def test_full_size_properties(dev, name):
    c, eng = _full(name, lr=1e-4 if name.startswith("config3") else 1e-3)
    kinds = ("lora",) if c.lora_rank else ("norm",)
    ids, lab = _ids(c, dev, 5)
    loss = torch.zeros(1, device=dev)
    eng.forward_backward(ids, lab, loss)
    torch.cuda.synchronize()
    l0 = float(loss.cpu()[0])
    assert math.isfinite(l0) and abs(l0 - math.log(c.vocab)) < 1.0, l0
    ref = _grads(eng, c, kinds)
    assert all(np.isfinite(g).all() for g in ref.values())
    # graph replay == eager, twice, with eager work in between
    eng.use_graph(True)
    for _ in range(2):
        torch.randn(1 << 20, device=dev).mul_(3.0).sum().item()
        eng.forward_backward(ids, lab, loss)
        torch.cuda.synchronize()
        assert float(loss.cpu()[0]) == l0
        got = _grads(eng, c, kinds)
        for n in ref:
            assert np.array_equal(got[n], ref[n]), n
    # three optimizer steps on this batch: the loss falls each time
    losses = [l0]
    for _ in range(3):
        eng.optimizer_step()
        eng.forward_backward(ids, lab, loss)
        torch.cuda.synchronize()
        losses.append(float(loss.cpu()[0]))
    print(name, losses)
    assert all(b < a for a, b in zip(losses, losses[1:])), losses
    eng.close()


@pytest.mark.parametrize("name", ["config4_lora_q8", "config5_lora_q4k"])
def test_full_size_b_zero_gives_zero_da(dev, name):
    c, eng = _full(name)
    for n, s, k in tensor_specs(c):
        if k == "lora" and n.endswith(".B"):
            eng.set(n, np.zeros(s, np.float32))
    ids, lab = _ids(c, dev, 6)
    eng.forward_backward(ids, lab)
    torch.cuda.synchronize()
    nonzero_b = 0
    for n, s, k in tensor_specs(c):
        if k != "lora":
            continue
        g = eng.get(n, s, grad=True)
        if n.endswith(".A"):
            assert not g.any(), n
        else:
            nonzero_b += bool(g.any())
    assert nonzero_b == 7 * c.n_layers  # dB = s u^T dY is not zero
    eng.close()


def test_config4_full_size_fp32_directional_derivative(dev):
    """fp32 engine at full config-4 size: (L(t + h v) - L(t - h v)) / 2h == <g, v> = |g_S| for v = g_S / |g_S|,
    with S three adapters spread through the depth."""
    c, eng = _full("config4_lora_q8", precision=PREC_FP32)
    ids, lab = _ids(c, dev, 8)
    loss = torch.zeros(1, device=dev)
    eng.forward_backward(ids, lab, loss)
    torch.cuda.synchronize()
    shapes = {n: s for n, s, _ in tensor_specs(c)}
    sel = ["l27.lora.q.B", "l14.lora.up.A", "l0.lora.down.B"]
    g = {n: eng.get(n, shapes[n], grad=True).astype(np.float64) for n in sel}
    theta = {n: eng.get(n, shapes[n]) for n in sel}
    gn = math.sqrt(sum(float((x ** 2).sum()) for x in g.values()))
    assert gn > 0
    h = 1e-2 / gn

    def loss_at(sign):
        for n in sel:
            eng.set(n, (theta[n] + sign * h * g[n] / gn).astype(np.float32))
        eng.forward_backward(ids, lab, loss)
        torch.cuda.synchronize()
        return float(loss.cpu()[0])

    fd = (loss_at(1) - loss_at(-1)) / (2 * h)
    print("fd", fd, "|g|", gn)
    assert abs(fd - gn) <= 2e-2 * gn, (fd, gn)
    eng.close()
