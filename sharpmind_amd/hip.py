"""Python mirror of the reference's slot interfaces over device tensors.

Method names, argument meaning and accumulate/overwrite behaviour follow the
reference's JigSaw slot classes:
  GradientMapping  (SharpMind.Core/Training/GradientMapping.cs:26-106)
  TrainingOps      (SharpMind.Training/TrainingOps.cs:17-33)
  QuantizationOps  (SharpMind.Core/Quantization/QuantizationOps.cs:8-9,142-166)
Tensors are torch CUDA(HIP) tensors used purely as device buffers; all
arithmetic happens in libsharpmind_hip.so.  Shape errors raise ValueError
(the reference throws ArgumentException).
"""
import torch

from . import check, lib

PREC_FP32 = 0
PREC_BF16 = 1
QTYPE_F32 = 0
QTYPE_Q8_0 = 8
QTYPE_Q4_K = 12


def _p(t):
    if t is None:
        return None
    if not t.is_cuda:
        raise ValueError("sharpmind_amd.hip expects device tensors")
    if not t.is_contiguous():
        raise ValueError("sharpmind_amd.hip expects contiguous tensors")
    return t.data_ptr()


def _stream():
    return torch.cuda.current_stream().cuda_stream


class AttentionGradients:
    """(dQ, dK, dV) as returned by GradientMapping.Attention."""

    def __init__(self, dq, dk, dv):
        self.DQ, self.DK, self.DV = dq, dk, dv


class Parameter:
    """Data + Grad pair with accumulate semantics (SharpMind.Core/Training/Parameter.cs:19-74)."""

    def __init__(self, name, data):
        self.Name = name
        self.Data = data
        self.Grad = torch.zeros_like(data)

    def ZeroGrad(self):
        self.Grad.zero_()


class GradientMapping:
    """HIP implementation of every GradientMapping slot ("hip" variant)."""

    def __init__(self, precision=PREC_FP32):
        self.precision = precision

    def Linear(self, dOutput, input, weight, bias=None):
        B, Out = dOutput.shape
        In = input.shape[1]
        if input.shape[0] != B or tuple(weight.Data.shape) != (Out, In):
            raise ValueError("Linear: shape mismatch")
        dInput = torch.empty(B, In, device=dOutput.device, dtype=torch.float32)
        check(lib().smhip_grad_linear(_p(dOutput), _p(input), _p(weight.Data), _p(weight.Grad),
                                      _p(bias.Grad) if bias is not None else None, _p(dInput),
                                      B, In, Out, self.precision, _stream()))
        return dInput

    def RMSNorm(self, dOutput, xNorm, rmsInv, weight):
        T, D = dOutput.shape
        dInput = torch.empty_like(dOutput)
        check(lib().smhip_grad_rmsnorm(_p(dOutput), _p(xNorm), _p(rmsInv), _p(weight.Data),
                                       _p(weight.Grad), _p(dInput), T, D, _stream()))
        return dInput

    def LayerNorm(self, dOutput, input, weight, bias, eps=1e-5):
        T, D = dOutput.shape
        dInput = torch.empty_like(dOutput)
        check(lib().smhip_grad_layernorm(_p(dOutput), _p(input), _p(weight.Data), _p(weight.Grad),
                                         _p(bias.Grad), _p(dInput), T, D, eps, _stream()))
        return dInput

    def Attention(self, dOut, q, k, v, probs, scale):
        S, D = q.shape
        dq, dk, dv = (torch.empty_like(q) for _ in range(3))
        check(lib().smhip_grad_attention(_p(dOut), _p(q), _p(k), _p(v), _p(probs), _p(dq), _p(dk),
                                         _p(dv), S, D, scale, _stream()))
        return AttentionGradients(dq, dk, dv)

    def Embedding(self, dOutput, tokenIds, weight):
        T, D = dOutput.shape
        V = weight.Data.shape[0]
        if tokenIds.dtype != torch.int32:
            raise ValueError("Embedding: token ids must be int32")
        check(lib().smhip_grad_embedding(_p(dOutput), _p(tokenIds), _p(weight.Grad), T, D, V,
                                         _stream()))

    def ActivationSiLU(self, dOutput, preAct):
        dInput = torch.empty_like(dOutput)
        check(lib().smhip_grad_silu(_p(dOutput), _p(preAct), _p(dInput), dOutput.numel(), _stream()))
        return dInput

    def ActivationGELU(self, dOutput, preAct):
        dInput = torch.empty_like(dOutput)
        check(lib().smhip_grad_gelu(_p(dOutput), _p(preAct), _p(dInput), dOutput.numel(), _stream()))
        return dInput


class TrainingOps:
    """HIP implementation of the TrainingOps slots."""

    def AdamWUpdate(self, data, grad, m, v, beta1, beta2, bc1, bc2, lr, epsilon, decay):
        check(lib().smhip_adamw_update(_p(data), _p(grad), _p(m), _p(v), data.numel(), beta1, beta2,
                                       bc1, bc2, lr, epsilon, decay, _stream()))

    def L2NormSq(self, data):
        out = torch.zeros(1, device=data.device, dtype=torch.float32)
        check(lib().smhip_l2normsq(_p(data), data.numel(), _p(out), _stream()))
        return out


class QuantizationOps:
    """QuantizedMatMulFn for F32 / Q8_0 / Q4_K raw weights on the device."""

    def __init__(self, precision=PREC_FP32):
        self.precision = precision

    def QuantizedMatMul(self, qtype, input, rawWeights, M, K, N):
        out = torch.empty(M, N, device=input.device, dtype=torch.float32)
        check(lib().smhip_qmatmul(qtype, _p(input), _p(rawWeights), _p(out), M, K, N,
                                  self.precision, _stream()))
        return out

    def Dequantize(self, qtype, raw, n):
        out = torch.empty(n, device=raw.device, dtype=torch.float32)
        check(lib().smhip_dequant(qtype, _p(raw), _p(out), n, _stream()))
        return out


# ---- BackpropEngine inline math (no slot in the reference) ----------------------------
def swiglu_backward(dAct, gate, up):
    T, F = dAct.shape
    out = torch.empty(T, 2 * F, device=dAct.device, dtype=torch.float32)
    check(lib().smhip_grad_swiglu(_p(dAct), _p(gate), _p(up), _p(out), T, F, _stream()))
    return out


def swiglu_forward(gate, up):
    out = torch.empty_like(gate)
    check(lib().smhip_swiglu_forward(_p(gate), _p(up), _p(out), gate.numel(), _stream()))
    return out


def rope_tables(theta, rope_dim, max_seq):
    import numpy as np
    c = np.zeros((max_seq, rope_dim // 2), np.float32)
    s = np.zeros_like(c)
    check(lib().smhip_rope_tables(theta, rope_dim, max_seq, c.ctypes.data, s.ctypes.data))
    return c, s


def rope_backward(dx, cos_t, sin_t, neox):
    B, S, H, D = dx.shape
    check(lib().smhip_rope_backward(_p(dx), _p(cos_t), _p(sin_t), B, S, H, D, int(neox), _stream()))


def rope_forward(x, cos_t, sin_t, neox):
    B, S, H, D = x.shape
    check(lib().smhip_rope_forward(_p(x), _p(cos_t), _p(sin_t), B, S, H, D, int(neox), _stream()))


def rmsnorm_forward(x, w, eps):
    T, D = x.shape
    y = torch.empty_like(x)
    rinv = torch.empty(T, device=x.device, dtype=torch.float32)
    check(lib().smhip_rmsnorm_forward(_p(x), _p(w), _p(y), _p(rinv), T, D, eps, _stream()))
    return y, rinv


def cross_entropy_softmax(logits, labels, ignore_id=-100, smoothing=0.0, out=None):
    T, V = logits.shape
    d = torch.empty_like(logits) if out is None else out
    loss = torch.zeros(1, device=logits.device, dtype=torch.float32)
    check(lib().smhip_ce_softmax_grad(_p(logits), _p(labels), _p(d), _p(loss), T, V, ignore_id,
                                      smoothing, _stream()))
    return d, loss


def attention_forward_probs(q, k, v):
    B, S, Hq, D = q.shape
    Hkv = k.shape[2]
    probs = torch.empty(B, Hq, S, S, device=q.device, dtype=torch.float32)
    out = torch.empty(B, S, Hq * D, device=q.device, dtype=torch.float32)
    check(lib().smhip_attention_forward_probs(_p(q), _p(k), _p(v), _p(probs), _p(out), B, S, Hq,
                                              Hkv, D, _stream()))
    return probs, out
