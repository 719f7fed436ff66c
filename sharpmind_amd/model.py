"""Model configuration and tensor naming of the training engine.

Tensor names follow the engine's C ABI (smhip_engine_set_tensor / get_tensor).
Linear weights are stored [Out][In] (GradientMapping layout,
SharpMind.Core/Training/GradientMapping.cs:30-34); the reference's training
LinearLayer keeps [In][Out] (SharpMind.Model/Layers/Linearlayer.cs:31), so a
reference checkpoint is transposed once on load.  Per layer the q|k|v and
gate|up projections are fused row-wise ([Wq; Wk; Wv], [Wgate; Wup]), exactly as
the reference fuses gate|up (ModelFactory.cs:157-196).
"""
from dataclasses import dataclass, field

QTYPE_F32, QTYPE_Q8_0, QTYPE_Q4_K = 0, 8, 12
PREC_FP32, PREC_BF16 = 0, 1
LORA_TARGETS = ("q", "k", "v", "o", "gate", "up", "down")


@dataclass
class ModelConfig:
    n_layers: int
    d_model: int
    n_heads: int
    n_kv_heads: int
    head_dim: int
    ffn_dim: int
    vocab: int
    batch: int
    seq: int
    norm_eps: float = 1e-6
    rope_theta: float = 1e4
    rope_neox: int = 0
    qk_norm: int = 0
    base_qtype: int = QTYPE_F32      # F32 = full-parameter training
    lora_rank: int = 0                # 0 = no adapters
    lora_alpha: float = 0.0
    precision: int = PREC_FP32
    use_bias: int = 0
    extra: dict = field(default_factory=dict)

    @property
    def tokens(self):
        return self.batch * self.seq

    @property
    def q_dim(self):
        return self.n_heads * self.head_dim

    @property
    def kv_dim(self):
        return self.n_kv_heads * self.head_dim

    def lora_geom(self, p):
        """(In, Out) of LoRA target p."""
        d, F = self.d_model, self.ffn_dim
        return {"q": (d, self.q_dim), "k": (d, self.kv_dim), "v": (d, self.kv_dim), "o": (self.q_dim, d),
                "gate": (d, F), "up": (d, F), "down": (F, d)}[p]


def tensor_specs(c: ModelConfig):
    """Ordered [(name, shape, kind)] with kind in {"base", "norm", "bias", "lora"}."""
    d, F, V = c.d_model, c.ffn_dim, c.vocab
    nqkv = c.q_dim + 2 * c.kv_dim
    out = [("emb", (V, d), "base"), ("norm_f", (d,), "norm")]
    for l in range(c.n_layers):
        p = f"l{l}."
        out += [(p + "norm1", (d,), "norm"), (p + "wqkv", (nqkv, d), "base")]
        if c.use_bias:
            out.append((p + "bqkv", (nqkv,), "bias"))
        if c.qk_norm:
            out += [(p + "q_norm", (c.head_dim,), "norm"), (p + "k_norm", (c.head_dim,), "norm")]
        out.append((p + "wo", (d, c.q_dim), "base"))
        if c.use_bias:
            out.append((p + "bo", (d,), "bias"))
        out += [(p + "norm2", (d,), "norm"), (p + "wgu", (2 * F, d), "base")]
        if c.use_bias:
            out.append((p + "bgu", (2 * F,), "bias"))
        out.append((p + "wd", (d, F), "base"))
        if c.use_bias:
            out.append((p + "bd", (d,), "bias"))
        if c.lora_rank:
            for t in LORA_TARGETS:
                In, Out = c.lora_geom(t)
                out += [(p + f"lora.{t}.A", (In, c.lora_rank), "lora"), (p + f"lora.{t}.B", (c.lora_rank, Out), "lora")]
    return out


def trainable(c: ModelConfig, kind):
    return kind == "lora" if c.lora_rank else kind in ("base", "norm", "bias")


# ------------------------------------------------------------------ the benchmark configurations
def tiny_llama(batch=4, seq=128):
    """Config 1: 2 layers, d 256, 4x64 heads, SwiGLU 688, eps 1e-6, RoPE 1e4 adjacent, vocab 512, fp32."""
    return ModelConfig(n_layers=2, d_model=256, n_heads=4, n_kv_heads=4, head_dim=64, ffn_dim=688, vocab=512,
                       batch=batch, seq=seq, norm_eps=1e-6, rope_theta=1e4, rope_neox=0, qk_norm=0,
                       base_qtype=QTYPE_F32, precision=PREC_FP32, use_bias=1)


def qwen3_0_6b(batch=4, seq=1024, qtype=QTYPE_Q8_0, rank=16, alpha=32.0, precision=PREC_BF16, layers=28):
    """Configs 3/4: Qwen3-0.6B shape (28 x d1024, 16q/8kv x 128, FFN 3072, vocab 151936, QK-norm, RoPE 1e6 NeoX)."""
    return ModelConfig(n_layers=layers, d_model=1024, n_heads=16, n_kv_heads=8, head_dim=128, ffn_dim=3072,
                       vocab=151936, batch=batch, seq=seq, norm_eps=1e-6, rope_theta=1e6, rope_neox=1, qk_norm=1,
                       base_qtype=qtype, lora_rank=rank, lora_alpha=alpha, precision=precision)


def qwen3_1_7b(batch=2, seq=2048, qtype=QTYPE_Q4_K, rank=32, alpha=64.0, precision=PREC_BF16, layers=28):
    """Config 5: Qwen3-1.7B shape (28 x d2048, 16q/8kv x 128, FFN 6144, vocab 151936)."""
    return ModelConfig(n_layers=layers, d_model=2048, n_heads=16, n_kv_heads=8, head_dim=128, ffn_dim=6144,
                       vocab=151936, batch=batch, seq=seq, norm_eps=1e-6, rope_theta=1e6, rope_neox=1, qk_norm=1,
                       base_qtype=qtype, lora_rank=rank, lora_alpha=alpha, precision=precision)
