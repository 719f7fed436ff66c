"""ctypes binding of the CPU oracle (liboracle.so) and the reference C tool.

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and the
cpu_baseline leg of bench.py, never by the sharpmind_amd package.  Every
function wraps a C restatement in oracle.c that cites the reference file:line
it follows.
"""
import ctypes
import os

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB = None
_REF = None

F32P = np.ctypeslib.ndpointer(dtype=np.float32, flags="C_CONTIGUOUS")
U8P = np.ctypeslib.ndpointer(dtype=np.uint8, flags="C_CONTIGUOUS")
I32P = np.ctypeslib.ndpointer(dtype=np.int32, flags="C_CONTIGUOUS")
c_int, c_float, c_i64 = ctypes.c_int, ctypes.c_float, ctypes.c_int64


class Rng(ctypes.Structure):
    """.NET System.Random(seed) state (legacy seeded generator)."""
    _fields_ = [("seed", ctypes.c_int32 * 56), ("inext", c_int), ("inextp", c_int)]


_SIGS = {
    "orc_rng_init": (None, [ctypes.POINTER(Rng), ctypes.c_int32]),
    "orc_rng_sample": (ctypes.c_int32, [ctypes.POINTER(Rng)]),
    "orc_rng_next_double": (ctypes.c_double, [ctypes.POINTER(Rng)]),
    "orc_rng_next_bytes": (None, [ctypes.POINTER(Rng), U8P, c_i64]),
    "orc_fill_normal": (None, [ctypes.POINTER(Rng), F32P, c_i64, c_float]),
    "orc_fill_uniform_pm1": (None, [ctypes.POINTER(Rng), F32P, c_i64]),
    "orc_half_to_float": (c_float, [ctypes.c_uint16]),
    "orc_float_to_half_rne": (ctypes.c_uint16, [c_float]),
    "orc_dequant_q8_0": (None, [U8P, F32P, c_i64]),
    "orc_dequant_q4k": (None, [U8P, F32P, c_i64]),
    "orc_vecdot_q8_0": (c_float, [F32P, U8P, c_int, c_int]),
    "orc_vecdot_q4k": (c_float, [F32P, U8P, c_int, c_int]),
    "orc_qmatmul_q8_0": (None, [F32P, U8P, F32P, c_int, c_int, c_int]),
    "orc_qmatmul_q4k": (None, [F32P, U8P, F32P, c_int, c_int, c_int]),
    "orc_qmatmul_f32": (None, [F32P, F32P, F32P, c_int, c_int, c_int]),
    "orc_quantize_q8_0": (c_int, [F32P, c_i64, U8P]),
    "orc_quantize_q4k": (c_int, [F32P, c_i64, U8P]),
    "orc_grad_linear": (None, [F32P, F32P, F32P, F32P, ctypes.c_void_p, F32P, c_int, c_int, c_int]),
    "orc_grad_rmsnorm": (None, [F32P, F32P, F32P, F32P, F32P, F32P, c_int, c_int]),
    "orc_grad_layernorm": (None, [F32P, F32P, F32P, F32P, F32P, F32P, c_int, c_int, c_float]),
    "orc_grad_attention": (None, [F32P] * 8 + [c_int, c_int, c_float]),
    "orc_grad_embedding": (None, [F32P, I32P, F32P, c_int, c_int]),
    "orc_grad_silu": (None, [F32P, F32P, F32P, c_i64]),
    "orc_grad_gelu": (None, [F32P, F32P, F32P, c_i64]),
    "orc_grad_swiglu": (None, [F32P, F32P, F32P, F32P, c_int, c_int]),
    "orc_swiglu_fwd": (None, [F32P, F32P, F32P, c_i64]),
    "orc_rope_tables": (None, [c_float, c_int, c_int, F32P, F32P]),
    "orc_rope_fwd": (None, [F32P, F32P, F32P, c_int, c_int, c_int, c_int]),
    "orc_rope_bwd": (None, [F32P, F32P, F32P, c_int, c_int, c_int, c_int]),
    "orc_rmsnorm_param": (c_float, [F32P, c_int, c_float]),
    "orc_rmsnorm_fwd": (None, [F32P, F32P, F32P, F32P, c_int, c_int, c_float]),
    "orc_ce_softmax_grad": (None, [F32P, I32P, F32P, c_int, c_int, c_int, c_float]),
    "orc_ce_loss": (c_float, [F32P, I32P, c_int, c_int, c_int, c_float]),
    "orc_adamw": (None, [F32P, F32P, F32P, F32P, c_i64] + [c_float] * 7),
    "orc_l2normsq": (c_float, [F32P, c_i64]),
    "orc_attention_fwd": (None, [F32P] * 5 + [c_int] * 5),
    "orc_lora_fwd": (None, [F32P] * 5 + [c_int] * 4 + [c_float]),
    "orc_lora_bwd": (None, [F32P] * 8 + [c_int] * 4 + [c_float]),
}


def build():
    """Compile liboracle.so (and oracle/_ref when the reference checkout exists)."""
    import subprocess
    subprocess.run(["make", "-s", "-C", _HERE], check=True)


def lib():
    global _LIB
    if _LIB is None:
        path = os.path.join(_HERE, "liboracle.so")
        if not os.path.exists(path):
            build()
        L = ctypes.CDLL(path)
        for name, (res, args) in _SIGS.items():
            f = getattr(L, name)
            f.restype = res
            f.argtypes = args
        _LIB = L
    return _LIB


def ref_lib():
    """The reference's own vecdot_ref.c built as a library, or None if not built."""
    global _REF
    if _REF is None:
        path = os.path.join(_HERE, "_ref", "libvecdot_ref.so")
        if not os.path.exists(path):
            return None
        R = ctypes.CDLL(path)
        R.half_to_float.restype = c_float
        R.half_to_float.argtypes = [ctypes.c_uint16]
        for n in ("vecdot_q8_0", "vecdot_q4_K"):
            f = getattr(R, n)
            f.restype = c_float
            f.argtypes = [F32P, U8P, c_int, c_int]
        _REF = R
    return _REF


class DotNetRandom:
    """.NET System.Random(seed) restated in oracle.c (Knuth subtractive)."""

    def __init__(self, seed):
        self._s = Rng()
        lib().orc_rng_init(ctypes.byref(self._s), seed)

    def sample(self):
        return lib().orc_rng_sample(ctypes.byref(self._s))

    def next_double(self):
        return lib().orc_rng_next_double(ctypes.byref(self._s))

    def next_bytes(self, n):
        b = np.zeros(n, np.uint8)
        lib().orc_rng_next_bytes(ctypes.byref(self._s), b, n)
        return b

    def uniform_pm1(self, n):
        a = np.zeros(n, np.float32)
        lib().orc_fill_uniform_pm1(ctypes.byref(self._s), a, n)
        return a

    def normal(self, n, std):
        a = np.zeros(n, np.float32)
        lib().orc_fill_normal(ctypes.byref(self._s), a, n, std)
        return a


def f32(a):
    return np.ascontiguousarray(a, dtype=np.float32)


# ---------------------------------------------------------------- engine (oracle/engine.c)
class EngineCfg(ctypes.Structure):
    _fields_ = [("L", c_int), ("d", c_int), ("Hq", c_int), ("Hkv", c_int), ("D", c_int), ("F", c_int),
                ("V", c_int), ("B", c_int), ("S", c_int), ("eps", c_float), ("theta", c_float),
                ("neox", c_int), ("qk_norm", c_int), ("lora_rank", c_int), ("lora_alpha", c_float)]


PER_LAYER = ["norm1", "wqkv", "bqkv", "q_norm", "k_norm", "wo", "bo", "norm2", "wgu", "bgu", "wd", "bd"] + \
    [f"lora.{p}.{m}" for p in ("q", "k", "v", "o", "gate", "up", "down") for m in ("A", "B")]


def engine_index(name):
    """Tensor index used by orc_engine_step: 0 emb, 1 norm_f, then 26 per layer."""
    if name == "emb":
        return 0
    if name == "norm_f":
        return 1
    layer, rest = name.split(".", 1)
    return 2 + int(layer[1:]) * len(PER_LAYER) + PER_LAYER.index(rest)


def engine_step(cfg, params, grads, ids, labels, want_logits=False):
    """Run orc_engine_step.  params/grads: dict name -> float32 ndarray (grads accumulate in place)."""
    L = lib()
    if not hasattr(L, "_engine_declared"):
        L.orc_engine_step.restype = c_int
        L.orc_engine_step.argtypes = [ctypes.POINTER(EngineCfg), ctypes.POINTER(ctypes.c_void_p),
                                      ctypes.POINTER(ctypes.c_void_p), I32P, I32P,
                                      ctypes.POINTER(c_float), ctypes.c_void_p]
        L._engine_declared = True
    n = 2 + cfg.L * len(PER_LAYER)
    P = (ctypes.c_void_p * n)()
    G = (ctypes.c_void_p * n)()
    for k, a in params.items():
        assert a.dtype == np.float32 and a.flags.c_contiguous
        P[engine_index(k)] = a.ctypes.data
    for k, a in grads.items():
        assert a.dtype == np.float32 and a.flags.c_contiguous
        G[engine_index(k)] = a.ctypes.data
    loss = c_float(0)
    logits = np.zeros((cfg.B * cfg.S, cfg.V), np.float32) if want_logits else None
    rc = L.orc_engine_step(ctypes.byref(cfg), P, G, np.ascontiguousarray(ids, np.int32),
                           np.ascontiguousarray(labels, np.int32), ctypes.byref(loss),
                           logits.ctypes.data if want_logits else None)
    assert rc == 0
    return (loss.value, logits) if want_logits else loss.value


class TwinCfg(ctypes.Structure):
    _fields_ = [(n, c_int) for n in ("d", "Hq", "Hkv", "D", "F", "V", "B", "S", "r", "head_tokens", "full")]


def twin_time_step(d, Hq, Hkv, D, F, V, B, S, r, head_tokens, full=0):
    """cpu_twin.c: (block seconds, head seconds on head_tokens tokens, threads) of the reference's
    AVX2/FMA CPU tiers at this shape.  Measurement infrastructure for bench.py's cpu_baseline."""
    path = os.path.join(_HERE, "libcputwin.so")
    if not os.path.exists(path):
        build()
    L = ctypes.CDLL(path)
    L.twin_time_step.restype = c_int
    L.twin_time_step.argtypes = [ctypes.POINTER(TwinCfg), ctypes.POINTER(ctypes.c_double)]
    out = (ctypes.c_double * 3)()
    cfg = TwinCfg(d, Hq, Hkv, D, F, V, B, S, r, head_tokens, full)
    if L.twin_time_step(ctypes.byref(cfg), out) != 0:
        raise RuntimeError("twin_time_step failed")
    return out[0], out[1], int(out[2])
