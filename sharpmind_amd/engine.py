"""Python handle on the resident training engine (smhip_engine_* in include/sharpmind_hip.h).

Mirrors how the reference drives a step: TrainLoop.ForwardBackward
(SharpMind.Training/TrainLoop.cs:222-243) then Gradients.ClipGlobalNorm and
AdamW.Update (TrainLoop.cs:122-129).  Token ids / labels are device int32
tensors; parameters and gradients are read back by name.
"""
import ctypes

import numpy as np
import torch

from . import check, lib
from .model import ModelConfig


class CModelConfig(ctypes.Structure):
    _fields_ = [(n, ctypes.c_int) for n in ("n_layers", "d_model", "n_heads", "n_kv_heads", "head_dim", "ffn_dim",
                                             "vocab", "batch", "seq")] + \
        [("norm_eps", ctypes.c_float), ("rope_theta", ctypes.c_float), ("rope_neox", ctypes.c_int),
         ("qk_norm", ctypes.c_int), ("base_qtype", ctypes.c_int), ("lora_rank", ctypes.c_int),
         ("lora_alpha", ctypes.c_float), ("precision", ctypes.c_int), ("use_bias", ctypes.c_int),
         ("lr", ctypes.c_float), ("beta1", ctypes.c_float), ("beta2", ctypes.c_float),
         ("adam_eps", ctypes.c_float), ("weight_decay", ctypes.c_float), ("max_grad_norm", ctypes.c_float)]


class Engine:
    """One model + optimizer state resident on cuda:0."""

    def __init__(self, cfg: ModelConfig, lr=1e-3, beta1=0.9, beta2=0.95, adam_eps=1e-8, weight_decay=0.1,
                 max_grad_norm=1.0):
        self.cfg = cfg
        c = CModelConfig()
        for name, _ in CModelConfig._fields_:
            if hasattr(cfg, name):
                setattr(c, name, getattr(cfg, name))
        c.lr, c.beta1, c.beta2, c.adam_eps, c.weight_decay, c.max_grad_norm = lr, beta1, beta2, adam_eps, weight_decay, max_grad_norm
        self._c = c
        h = ctypes.c_void_p()
        check(lib().smhip_engine_create(ctypes.byref(c), ctypes.byref(h)))
        self.h = h

    def close(self):
        if self.h:
            lib().smhip_engine_destroy(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def param_count(self):
        t, f = ctypes.c_int64(), ctypes.c_int64()
        check(lib().smhip_engine_param_count(self.h, ctypes.byref(t), ctypes.byref(f)))
        return t.value, f.value

    def set(self, name, arr):
        a = np.ascontiguousarray(arr)
        check(lib().smhip_engine_set_tensor(self.h, name.encode(), a.ctypes.data, a.nbytes))

    def get(self, name, shape, grad=False, state=None):
        """Parameter (default), its gradient (grad=True) or AdamW state (state='m' | 'v')."""
        which = {None: 1 if grad else 0, "m": 2, "v": 3}[state]
        out = np.zeros(shape, np.float32)
        check(lib().smhip_engine_get_tensor(self.h, name.encode(), which, out.ctypes.data, out.nbytes))
        return out

    def load_gguf(self, path):
        """Frozen quantised base from a GGUF file (GgufLoader.LoadAllWeights, GgufLoader.cs:435-600)."""
        check(lib().smhip_engine_load_gguf(self.h, str(path).encode()))

    def save_checkpoint(self, directory, step=0, loss=float("nan"), note=None, optimizer=True):
        """Checkpoint.Save (Checkpoint.cs:27-82): model.bin, optimizer.bin, meta.json."""
        check(lib().smhip_engine_save_checkpoint(self.h, str(directory).encode(), 1 if optimizer else 0, int(step),
                                                 float(loss), note.encode() if note is not None else None))

    def load_checkpoint(self, directory, optimizer=True):
        """Checkpoint.Load (Checkpoint.cs:161-237); returns meta.json's (step, loss)."""
        st, ls = ctypes.c_int(), ctypes.c_float()
        check(lib().smhip_engine_load_checkpoint(self.h, str(directory).encode(), 1 if optimizer else 0,
                                                 ctypes.byref(st), ctypes.byref(ls)))
        return st.value, ls.value

    def init_synthetic(self, seed=0):
        check(lib().smhip_engine_init_synthetic(self.h, seed))

    @staticmethod
    def _stream():
        return torch.cuda.current_stream().cuda_stream

    def forward_backward(self, ids, labels, loss=None, accumulate=False):
        """TrainLoop.ForwardBackward; accumulate=True adds to the held gradients (a later micro-batch of a
        GradAccumSteps window, TrainLoop.cs:104-120), otherwise they are zeroed first."""
        check(lib().smhip_engine_forward_backward_accum(self.h, ids.data_ptr(), labels.data_ptr(),
                                                        loss.data_ptr() if loss is not None else None,
                                                        1 if accumulate else 0, self._stream()))

    def zero_grad(self):
        check(lib().smhip_engine_zero_grad(self.h, self._stream()))

    @property
    def lr(self):
        v = ctypes.c_float()
        check(lib().smhip_engine_get_lr(self.h, ctypes.byref(v)))
        return v.value

    @lr.setter
    def lr(self, value):
        """_optimizer.LearningRate = scheduler.GetLr(step + 1) (TrainLoop.cs:122-123)."""
        check(lib().smhip_engine_set_lr(self.h, float(value)))

    def optimizer_step(self, grad_norm_sq=None):
        check(lib().smhip_engine_optimizer_step(self.h, grad_norm_sq.data_ptr() if grad_norm_sq is not None else None,
                                                self._stream()))

    def use_graph(self, on=True):
        """Replay forward_backward as a recorded HIP graph (bit-identical to eager launches)."""
        check(lib().smhip_engine_use_graph(self.h, 1 if on else 0))

    def step(self, ids, labels, loss=None):
        check(lib().smhip_engine_step(self.h, ids.data_ptr(), labels.data_ptr(),
                                      loss.data_ptr() if loss is not None else None, self._stream()))


def gguf_tensor_table(path):
    """[(name, dims innermost first, ggml type, absolute file offset)] of a GGUF file."""
    n = ctypes.c_int64()
    check(lib().smhip_gguf_tensor_count(str(path).encode(), ctypes.byref(n)))
    out = []
    for i in range(n.value):
        name = ctypes.create_string_buffer(1024)
        t, nd, off = ctypes.c_int(), ctypes.c_int(), ctypes.c_int64()
        dims = (ctypes.c_int64 * 8)()
        check(lib().smhip_gguf_tensor_info(str(path).encode(), i, name, len(name), ctypes.byref(t), ctypes.byref(nd),
                                           dims, ctypes.byref(off)))
        out.append((name.value.decode(), tuple(dims[:nd.value]), t.value, off.value))
    return out


def find_latest_checkpoint(directory):
    """Checkpoint.FindLatest (Checkpoint.cs:117-145): latest step-* directory, or None."""
    buf = ctypes.create_string_buffer(4096)
    rc = lib().smhip_checkpoint_find_latest(str(directory).encode() if directory is not None else None, buf, len(buf))
    if rc < 0:
        check(rc)
    return buf.value.decode() if rc == 1 else None


def next_token_labels(ids, seq):
    """labels[b, s] = ids[b, s+1], -100 at the end of each sequence (CLM shift, TrainingBatch.cs:8)."""
    lab = torch.roll(ids, -1)
    lab = lab.view(-1, seq).clone()
    lab[:, -1] = -100
    return lab.view(-1).contiguous()
