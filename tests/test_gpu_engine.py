"""End-to-end parity of the resident training engine against the oracle's whole step.

The oracle (oracle/engine.c) restates BackpropEngine's forward/backward on
the CPU in fp32 and is itself pinned by float64 finite differences
(tests/test_oracle_engine.py).  Both sides get identical weights; for a
quantised base the oracle receives the reference-dequantised fp32 values of the
very bytes the engine holds.  Bar (norm-wise relative error per tensor):
fp32 mode 1e-5; bf16 mode 2e-2 (loss and every gradient).  The bf16 whole-step
bar compares a bf16 forward (weights, q/k/v and activations rounded to bf16, as
the MFMA path requires) with an all-fp32 reference run.  Those tests draw their
weights the way the benchmark configurations do (base N(0, 0.02), LoRA A
Kaiming-uniform, B N(0, 1e-3), norms N(1, 0.1)); each bf16 kernel on identical
inputs is held to 2e-2 (and measures ~2e-3) in test_gpu_slots.py and
test_gpu_flash.py.
"""
import numpy as np
import pytest
import torch

import oracle
from oracle import DotNetRandom
from sharpmind_amd.engine import Engine, next_token_labels
from sharpmind_amd.model import (LORA_TARGETS, PREC_BF16, PREC_FP32, QTYPE_F32, QTYPE_Q4_K, QTYPE_Q8_0, ModelConfig,
                                 tensor_specs, tiny_llama)

from conftest import rel_err

pytestmark = pytest.mark.gpu


def _quant(orc, w, qtype):
    flat = np.ascontiguousarray(w, np.float32).ravel()
    if qtype == QTYPE_Q8_0:
        raw = np.zeros(flat.size // 32 * 34, np.uint8)
        assert orc.orc_quantize_q8_0(flat, flat.size, raw) == 0
        deq = np.zeros_like(flat)
        orc.orc_dequant_q8_0(raw, deq, flat.size)
    else:
        raw = np.zeros(flat.size // 256 * 144, np.uint8)
        assert orc.orc_quantize_q4k(flat, flat.size, raw) == 0
        deq = np.zeros_like(flat)
        orc.orc_dequant_q4k(raw, deq, flat.size)
    return raw, deq.reshape(w.shape)


def _ocfg(c):
    return oracle.EngineCfg(L=c.n_layers, d=c.d_model, Hq=c.n_heads, Hkv=c.n_kv_heads, D=c.head_dim, F=c.ffn_dim,
                            V=c.vocab, B=c.batch, S=c.seq, eps=c.norm_eps, theta=c.rope_theta, neox=c.rope_neox,
                            qk_norm=c.qk_norm, lora_rank=c.lora_rank, lora_alpha=c.lora_alpha)


def build(orc, c, seed, params=None, init="wide", max_grad_norm=0.0):
    """Random weights loaded into a GPU engine and the matching oracle dicts.

    init "wide": every weight N(0, 0.05) (large activations, exercises the fp32 bar);
    init "config": the benchmark configurations' draws (base N(0, 0.02), LoRA A
    Kaiming-uniform U(+-1/sqrt(In)), LoRA B N(0, 1e-3))."""
    rng = np.random.default_rng(seed)
    eng = Engine(c, lr=1e-3, max_grad_norm=max_grad_norm)
    P, G = {}, {}
    for name, shape, kind in tensor_specs(c):
        if params is not None and name in params:
            w = params[name]
        elif kind == "norm":
            w = (1 + 0.1 * rng.standard_normal(shape)).astype(np.float32)
        elif kind == "bias":
            w = (0.05 * rng.standard_normal(shape)).astype(np.float32)
        elif kind == "lora" and init == "config":
            if name.endswith(".A"):
                w = (rng.uniform(-1, 1, shape) / np.sqrt(shape[0])).astype(np.float32)
            else:
                w = (1e-3 * rng.standard_normal(shape)).astype(np.float32)
        elif init == "config":
            w = (0.02 * rng.standard_normal(shape)).astype(np.float32)
        else:
            w = (0.05 * rng.standard_normal(shape)).astype(np.float32)
        if kind == "base" and c.base_qtype != QTYPE_F32:
            raw, deq = _quant(orc, w, c.base_qtype)
            eng.set(name, raw)
            P[name] = np.ascontiguousarray(deq)
        else:
            eng.set(name, w)
            P[name] = np.ascontiguousarray(w, np.float32)
        if (kind == "lora") if c.lora_rank else True:
            G[name] = np.zeros(shape, np.float32)
    return eng, P, G


def run_pair(orc, dev, c, seed=0, tol=1e-5, params=None, ids=None, loss_tol=None, init="wide"):
    eng, P, G = build(orc, c, seed, params, init=init)
    if ids is None:
        ids = torch.from_numpy(np.random.default_rng(seed + 1).integers(0, c.vocab, c.tokens).astype(np.int32)).to(dev)
    labels = next_token_labels(ids, c.seq)
    loss = torch.zeros(1, device=dev)
    eng.forward_backward(ids, labels, loss)
    torch.cuda.synchronize()
    ref_loss = oracle.engine_step(_ocfg(c), P, G, ids.cpu().numpy(), labels.cpu().numpy())
    got_loss = float(loss.cpu()[0])
    errs = {"loss": abs(got_loss - ref_loss) / abs(ref_loss)}
    for name, g in G.items():
        errs[name] = rel_err(eng.get(name, g.shape, grad=True), g)
    assert errs["loss"] <= (tol if loss_tol is None else loss_tol), errs["loss"]
    worst = max(errs.items(), key=lambda kv: kv[1])
    print(f"worst {worst}, loss gpu {got_loss} oracle {ref_loss}")
    bad = sorted(((k, v) for k, v in errs.items() if v > tol), key=lambda kv: -kv[1])
    assert not bad, bad[:12]
    return eng, P, G, ids, labels


def test_engine_full_fp32_bias(orc, dev):
    c = ModelConfig(n_layers=2, d_model=64, n_heads=4, n_kv_heads=4, head_dim=16, ffn_dim=96, vocab=128, batch=2,
                    seq=32, rope_theta=1e4, rope_neox=0, use_bias=1)
    run_pair(orc, dev, c)


def test_engine_full_fp32_qknorm_gqa(orc, dev):
    c = ModelConfig(n_layers=2, d_model=64, n_heads=4, n_kv_heads=2, head_dim=16, ffn_dim=96, vocab=128, batch=2,
                    seq=32, rope_theta=1e6, rope_neox=1, qk_norm=1)
    run_pair(orc, dev, c, seed=3)


@pytest.mark.parametrize("qtype", [QTYPE_Q8_0, QTYPE_Q4_K])
def test_engine_lora_fp32(orc, dev, qtype):
    c = ModelConfig(n_layers=2, d_model=256, n_heads=4, n_kv_heads=2, head_dim=64, ffn_dim=512, vocab=512, batch=2,
                    seq=32, rope_theta=1e6, rope_neox=1, qk_norm=1, base_qtype=qtype, lora_rank=4, lora_alpha=8.0)
    run_pair(orc, dev, c, seed=5)


@pytest.mark.parametrize("neox", [0, 1])
def test_engine_full_fp32_head128(orc, dev, neox):
    """head_dim 128 (the vectorised QK-norm/RoPE kernels) with both RoPE pairings and the
    q_norm / k_norm weight gradients, fp32 mode."""
    c = ModelConfig(n_layers=1, d_model=256, n_heads=2, n_kv_heads=1, head_dim=128, ffn_dim=256, vocab=256, batch=2,
                    seq=64, rope_theta=1e6, rope_neox=neox, qk_norm=1)
    run_pair(orc, dev, c, seed=11 + neox)


@pytest.mark.parametrize("base_ws", ["1", "0"])
@pytest.mark.parametrize("qtype", [QTYPE_Q8_0, QTYPE_Q4_K])
def test_engine_lora_bf16(orc, dev, qtype, base_ws, monkeypatch):
    """LoRA bf16 step with the frozen base decoded into the bf16 workspace each step (1) and
    with the fused-decode GEMM loaders reading the quantised planes directly (0)."""
    monkeypatch.setenv("SMHIP_BASE_WS", base_ws)
    c = ModelConfig(n_layers=2, d_model=256, n_heads=4, n_kv_heads=2, head_dim=64, ffn_dim=512, vocab=512, batch=2,
                    seq=128, rope_theta=1e6, rope_neox=1, qk_norm=1, base_qtype=qtype, lora_rank=8, lora_alpha=16.0,
                    precision=PREC_BF16)
    run_pair(orc, dev, c, seed=7, tol=2e-2, init="config")


def test_engine_lora_bf16_rank4(orc, dev):
    """Rank 4: the fused projections' rank extensions (12, 8, 4 columns) are not multiples of 8,
    so the Q8_0 fragment-plane GEMM stages them element-wise (its general instantiation)."""
    c = ModelConfig(n_layers=1, d_model=256, n_heads=4, n_kv_heads=2, head_dim=64, ffn_dim=512, vocab=512, batch=2,
                    seq=128, rope_theta=1e6, rope_neox=1, qk_norm=1, base_qtype=QTYPE_Q8_0, lora_rank=4,
                    lora_alpha=8.0, precision=PREC_BF16)
    run_pair(orc, dev, c, seed=17, tol=2e-2, init="config")


def test_engine_lora_bf16_large_vocab(orc, dev):
    """Vocabulary above the register-resident cross-entropy limit (the two-pass row kernel,
    bf16 output) in a LoRA bf16 step."""
    c = ModelConfig(n_layers=1, d_model=256, n_heads=4, n_kv_heads=2, head_dim=64, ffn_dim=256, vocab=40000, batch=1,
                    seq=128, rope_theta=1e6, rope_neox=1, qk_norm=1, base_qtype=QTYPE_Q8_0, lora_rank=8,
                    lora_alpha=16.0, precision=PREC_BF16)
    run_pair(orc, dev, c, seed=13, tol=2e-2, init="config")


def test_engine_full_bf16(orc, dev):
    c = ModelConfig(n_layers=2, d_model=256, n_heads=4, n_kv_heads=2, head_dim=64, ffn_dim=512, vocab=512, batch=2,
                    seq=128, rope_theta=1e6, rope_neox=1, qk_norm=1, precision=PREC_BF16)
    run_pair(orc, dev, c, seed=9, tol=2e-2, init="config")


def test_engine_config1_tiny_llama_exact(orc, dev):
    """Config 1 at full size with the reference's own initialisation: WeightInitializer.InitializeRandomly
    with .NET Random(0) (WeightInitializer.cs:23-45, FillNormal :98-106) over [In, Out]-stored weights in the
    order emb, then per block Wq, Wk, Wv, Wo, Wf1 (fused gate|up), Wf2; norms 1; biases 0."""
    c = tiny_llama()
    r = DotNetRandom(0)
    d, F, V, qd = c.d_model, c.ffn_dim, c.vocab, c.q_dim
    params = {"emb": r.normal(V * d, 0.02).reshape(V, d)}
    for l in range(c.n_layers):
        wq = r.normal(d * qd, 0.02).reshape(d, qd)          # [In, Out]
        wk = r.normal(d * c.kv_dim, 0.02).reshape(d, c.kv_dim)
        wv = r.normal(d * c.kv_dim, 0.02).reshape(d, c.kv_dim)
        wo = r.normal(qd * d, 0.02).reshape(qd, d)
        wf1 = r.normal(d * 2 * F, 0.02).reshape(d, 2 * F)
        wf2 = r.normal(F * d, 0.02).reshape(F, d)
        p = f"l{l}."
        params[p + "wqkv"] = np.ascontiguousarray(np.concatenate([wq, wk, wv], 1).T)
        params[p + "wo"] = np.ascontiguousarray(wo.T)
        params[p + "wgu"] = np.ascontiguousarray(wf1.T)
        params[p + "wd"] = np.ascontiguousarray(wf2.T)
        params[p + "norm1"] = np.ones(d, np.float32)
        params[p + "norm2"] = np.ones(d, np.float32)
        for b, n in (("bqkv", qd + 2 * c.kv_dim), ("bo", d), ("bgu", 2 * F), ("bd", d)):
            params[p + b] = np.zeros(n, np.float32)
    params["norm_f"] = np.ones(d, np.float32)
    run_pair(orc, dev, c, params=params)


def test_engine_optimizer_step_matches_adamw(orc, dev):
    """Clip off: new params = TrainingKernels AdamW on the engine's own grads, bit for bit."""
    c = ModelConfig(n_layers=1, d_model=256, n_heads=4, n_kv_heads=2, head_dim=64, ffn_dim=512, vocab=512, batch=1,
                    seq=128, rope_theta=1e6, rope_neox=1, qk_norm=1, base_qtype=QTYPE_Q8_0, lora_rank=4,
                    lora_alpha=8.0, precision=PREC_BF16)
    eng, P, G = build(orc, c, 11)
    ids = torch.from_numpy(np.random.default_rng(1).integers(0, c.vocab, c.tokens).astype(np.int32)).to(dev)
    labels = next_token_labels(ids, c.seq)
    eng.forward_backward(ids, labels)
    names = [n for n, _, k in tensor_specs(c) if k == "lora"]
    shapes = {n: s for n, s, _ in tensor_specs(c)}
    before = {n: eng.get(n, shapes[n]) for n in names}
    grads = {n: eng.get(n, shapes[n], grad=True) for n in names}
    eng.optimizer_step()
    for n in names:
        ref = before[n].copy().ravel()
        m = np.zeros_like(ref)
        v = np.zeros_like(ref)
        # bias corrections as AdamW.Update computes them in float: 1f - MathF.Pow(beta, step) (AdamW.cs:55-56)
        bc1 = float(np.float32(1) - np.float32(0.9))
        bc2 = float(np.float32(1) - np.float32(0.95))
        orc.orc_adamw(ref, np.ascontiguousarray(grads[n].ravel()), m, v, ref.size, 0.9, 0.95, bc1, bc2, 1e-3, 1e-8, 0.1)
        assert np.array_equal(eng.get(n, shapes[n]).ravel(), ref), n


def test_engine_lora_b_zero_invariant(orc, dev):
    """With B = 0 every dA is zero (the adapter contributes nothing and receives no A gradient)."""
    c = ModelConfig(n_layers=1, d_model=256, n_heads=4, n_kv_heads=2, head_dim=64, ffn_dim=512, vocab=512, batch=1,
                    seq=128, rope_neox=1, qk_norm=1, base_qtype=QTYPE_Q8_0, lora_rank=4, lora_alpha=8.0,
                    precision=PREC_BF16)
    zeros = {}
    for n, s, k in tensor_specs(c):
        if k == "lora" and n.endswith(".B"):
            zeros[n] = np.zeros(s, np.float32)
    eng, P, G = build(orc, c, 13, params=zeros)
    ids = torch.from_numpy(np.random.default_rng(2).integers(0, c.vocab, c.tokens).astype(np.int32)).to(dev)
    eng.forward_backward(ids, next_token_labels(ids, c.seq))
    for n, s, k in tensor_specs(c):
        if k == "lora" and n.endswith(".A"):
            assert not eng.get(n, s, grad=True).any(), n


@pytest.mark.parametrize("qtype", [QTYPE_Q8_0, QTYPE_Q4_K])
def test_device_encoder_bitexact(orc, dev, qtype):
    """smhip_quantize == TensorQuantizer restatement, byte for byte (incl. zero and constant blocks)."""
    import sharpmind_amd
    rng = np.random.default_rng(qtype)
    x = (rng.standard_normal(256 * 257) * 0.02).astype(np.float32)
    x[:256] = 0.0
    x[256:512] = 0.013
    x[512:544] = -1e-30
    raw_ref, _ = _quant(orc, x, qtype)
    out = torch.zeros(raw_ref.size, dtype=torch.uint8, device=dev)
    xt = torch.from_numpy(x).to(dev)
    sharpmind_amd.check(sharpmind_amd.lib().smhip_quantize(qtype, xt.data_ptr(), x.size, out.data_ptr(),
                                                           torch.cuda.current_stream().cuda_stream))
    torch.cuda.synchronize()
    assert np.array_equal(out.cpu().numpy(), raw_ref)


def test_engine_graph_replay_matches_eager(orc, dev):
    """Graph mode: the recorded step replayed several times, with unrelated eager work and
    synchronisations in between, gives gradients and loss bit-identical to eager launches."""
    c = ModelConfig(n_layers=2, d_model=256, n_heads=4, n_kv_heads=2, head_dim=64, ffn_dim=512, vocab=512, batch=2,
                    seq=128, rope_theta=1e6, rope_neox=1, qk_norm=1, base_qtype=QTYPE_Q8_0, lora_rank=8,
                    lora_alpha=16.0, precision=PREC_BF16)
    eng, P, G = build(orc, c, 21)
    rng = np.random.default_rng(22)
    batches = [torch.from_numpy(rng.integers(0, c.vocab, c.tokens).astype(np.int32)).to(dev) for _ in range(2)]
    loss = torch.zeros(1, device=dev)

    def grads():
        return {n: eng.get(n, g.shape, grad=True) for n, g in G.items()}

    ref = []
    for ids in batches:  # eager
        eng.forward_backward(ids, next_token_labels(ids, c.seq), loss)
        torch.cuda.synchronize()
        ref.append((float(loss.cpu()[0]), grads()))
    eng.use_graph(True)
    for rep in range(3):
        for i, ids in enumerate(batches):
            scratch = torch.randn(1 << 20, device=dev)  # unrelated eager work between replays
            scratch.mul_(2.0).sum().item()
            eng.forward_backward(ids, next_token_labels(ids, c.seq), loss)
            torch.cuda.synchronize()
            assert float(loss.cpu()[0]) == ref[i][0], (rep, i)
            got = grads()
            for n in got:
                assert np.array_equal(got[n], ref[i][1][n]), (rep, i, n)


def test_engine_full_optimizer_decay_groups(orc, dev):
    """Full-parameter AdamW with weight decay: biases are exempt and norm weights decay, as the
    reference's name rule gives for its parameter names (AdamW.cs:38-41, 119-125)."""
    c = ModelConfig(n_layers=1, d_model=128, n_heads=4, n_kv_heads=2, head_dim=32, ffn_dim=192, vocab=256, batch=1,
                    seq=64, rope_theta=1e4, rope_neox=0, qk_norm=1, use_bias=1, precision=PREC_FP32)
    eng, P, G = build(orc, c, 5)
    ids = torch.from_numpy(np.random.default_rng(2).integers(0, c.vocab, c.tokens).astype(np.int32)).to(dev)
    eng.forward_backward(ids, next_token_labels(ids, c.seq))
    specs = tensor_specs(c)
    before = {n: eng.get(n, s) for n, s, _ in specs}
    grads = {n: eng.get(n, s, grad=True) for n, s, _ in specs}
    eng.optimizer_step()
    bc1 = float(np.float32(1) - np.float32(0.9))
    bc2 = float(np.float32(1) - np.float32(0.95))
    for n, s, kind in specs:
        ref = before[n].copy().ravel()
        m, v = np.zeros_like(ref), np.zeros_like(ref)
        decay = 0.0 if kind == "bias" else 0.1
        orc.orc_adamw(ref, np.ascontiguousarray(grads[n].ravel()), m, v, ref.size, 0.9, 0.95, bc1, bc2, 1e-3, 1e-8, decay)
        assert np.array_equal(eng.get(n, s).ravel(), ref), n
