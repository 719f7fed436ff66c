"""GGUF base loading into a LoRA engine: a file written by the format restatement (separate
q/k/v and gate/up tensors, shuffled order, extra tensors and metadata) must give exactly the
engine that set_tensor builds from the same bytes."""
import numpy as np
import pytest
import torch

from oracle import gguf as og
from sharpmind_amd import SmHipError
from sharpmind_amd.engine import Engine, next_token_labels
from sharpmind_amd.model import PREC_BF16, QTYPE_Q4_K, QTYPE_Q8_0, ModelConfig, tensor_specs

pytestmark = pytest.mark.gpu


def _cfg(qtype):
    return ModelConfig(n_layers=2, d_model=256, n_heads=4, n_kv_heads=2, head_dim=64, ffn_dim=512, vocab=512, batch=2,
                       seq=128, rope_theta=1e6, rope_neox=1, qk_norm=1, base_qtype=qtype, lora_rank=8,
                       lora_alpha=16.0, precision=PREC_BF16)


def _quant(orc, w, qtype):
    w = np.ascontiguousarray(w, np.float32).ravel()
    if qtype == QTYPE_Q8_0:
        raw = np.zeros(w.size // 32 * 34, np.uint8)
        assert orc.orc_quantize_q8_0(w, w.size, raw) == 0
    else:
        raw = np.zeros(w.size // 256 * 144, np.uint8)
        assert orc.orc_quantize_q4k(w, w.size, raw) == 0
    return raw.tobytes()


def _model(orc, c, rng, norm_f16=False):
    """GGUF tensor list and the engine tensors (fused raw bytes, norms, LoRA) built from it."""
    d, F, D, qd, kvd = c.d_model, c.ffn_dim, c.head_dim, c.q_dim, c.kv_dim
    qt = og.Q8_0 if c.base_qtype == QTYPE_Q8_0 else og.Q4_K
    gg, eng = [], {}

    def lin(name, In, Out):
        raw = _quant(orc, 0.02 * rng.standard_normal((Out, In)), c.base_qtype)
        gg.append((name, (In, Out), qt, raw))
        return raw

    def norm(name, n):
        w = (1 + 0.1 * rng.standard_normal(n)).astype(np.float32)
        if norm_f16:
            w = w.astype(np.float16)
            gg.append((name, (n,), og.F16, w.tobytes()))
            return w.astype(np.float32)
        gg.append((name, (n,), og.F32, w.tobytes()))
        return w

    eng["emb"] = np.frombuffer(lin("token_embd.weight", d, c.vocab), np.uint8)
    eng["norm_f"] = norm("output_norm.weight", d)
    for l in range(c.n_layers):
        b = f"blk.{l}."
        q, k, v = lin(b + "attn_q.weight", d, qd), lin(b + "attn_k.weight", d, kvd), lin(b + "attn_v.weight", d, kvd)
        eng[f"l{l}.wqkv"] = np.frombuffer(q + k + v, np.uint8)
        eng[f"l{l}.wo"] = np.frombuffer(lin(b + "attn_output.weight", qd, d), np.uint8)
        g, u = lin(b + "ffn_gate.weight", d, F), lin(b + "ffn_up.weight", d, F)
        eng[f"l{l}.wgu"] = np.frombuffer(g + u, np.uint8)
        eng[f"l{l}.wd"] = np.frombuffer(lin(b + "ffn_down.weight", F, d), np.uint8)
        eng[f"l{l}.norm1"] = norm(b + "attn_norm.weight", d)
        eng[f"l{l}.norm2"] = norm(b + "ffn_norm.weight", d)
        eng[f"l{l}.q_norm"] = norm(b + "attn_q_norm.weight", D)
        eng[f"l{l}.k_norm"] = norm(b + "attn_k_norm.weight", D)
    for name, shape, kind in tensor_specs(c):
        if kind == "lora":
            eng[name] = (0.05 * rng.standard_normal(shape)).astype(np.float32)
    gg.append(("rope_freqs.weight", (32,), og.F32, np.ones(32, np.float32).tobytes()))  # not a model tensor
    order = rng.permutation(len(gg))
    return [gg[i] for i in order], eng


KV = [("general.architecture", "qwen3"), ("qwen3.block_count", (4, 2)), ("qwen3.embedding_length", (4, 256)),
      ("tokenizer.ggml.tokens", ["a", "b"]), ("general.alignment", (4, 32))]


def _step(e, c, dev):
    ids = torch.from_numpy(np.random.default_rng(4).integers(0, c.vocab, c.tokens).astype(np.int32)).to(dev)
    loss = torch.zeros(1, device=dev)
    e.forward_backward(ids, next_token_labels(ids, c.seq), loss)
    torch.cuda.synchronize()
    return loss.item()


@pytest.mark.parametrize("qtype,f16", [(QTYPE_Q8_0, False), (QTYPE_Q4_K, True)])
def test_gguf_base_equals_set_tensor(orc, dev, tmp_path, qtype, f16):
    c = _cfg(qtype)
    gg, tensors = _model(orc, c, np.random.default_rng(int(qtype)), norm_f16=f16)
    path = tmp_path / "base.gguf"
    og.write(str(path), KV, gg)
    a, b = Engine(c), Engine(c)
    a.load_gguf(path)
    for name, arr in tensors.items():
        b.set(name, arr)
        if ".lora." in name:
            a.set(name, arr)
    la, lb = _step(a, c, dev), _step(b, c, dev)
    assert la == lb
    for name, shape, kind in tensor_specs(c):
        if kind in ("lora", "norm"):
            assert np.array_equal(a.get(name, shape), b.get(name, shape)), name
        if kind == "lora":
            assert np.array_equal(a.get(name, shape, grad=True), b.get(name, shape, grad=True)), name
    a.close()
    b.close()


def _expect_error(c, tmp_path, gg, kv, match):
    path = tmp_path / "bad.gguf"
    og.write(str(path), kv, gg)
    e = Engine(c)
    with pytest.raises(SmHipError, match=match):
        e.load_gguf(path)
    e.close()


def test_gguf_errors(orc, dev, tmp_path):
    c = _cfg(QTYPE_Q8_0)
    gg, _ = _model(orc, c, np.random.default_rng(0))
    # another quantisation than the engine's base
    c4 = _cfg(QTYPE_Q4_K)
    _expect_error(c4, tmp_path, gg, KV, "ggml type")
    # a missing tensor
    _expect_error(c, tmp_path, [t for t in gg if t[0] != "blk.1.ffn_up.weight"], KV, "missing tensor blk.1.ffn_up")
    # an untied head
    head = next(t for t in gg if t[0] == "token_embd.weight")
    _expect_error(c, tmp_path, gg + [("output.weight", head[1], head[2], head[3])], KV, "untied")
    # a file for a deeper model
    kv3 = [(k, (4, 3) if k == "qwen3.block_count" else v) for k, v in KV]
    _expect_error(c, tmp_path, gg, kv3, "3 blocks")
    # a wrong shape
    bad = [(n, (dims[1], dims[0]) if n == "blk.0.attn_k.weight" else dims, t, raw) for n, dims, t, raw in gg]
    _expect_error(c, tmp_path, bad, KV, "unexpected shape")
