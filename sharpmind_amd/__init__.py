"""sharpmind_amd — MI355X (gfx950) backward-pass backend for SharpMind.

The product is libsharpmind_hip.so (hand-written HIP kernels behind the C ABI
declared in include/sharpmind_hip.h).  This package only locates and loads it;
`sharpmind_amd.hip` mirrors the reference's GradientMapping / TrainingOps /
QuantizationOps slot names over device tensors for Python callers and tests.

There is no CPU fallback: if the library is missing or fails to load, every
entry point raises.
"""
import ctypes
import os

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "libsharpmind_hip.so")
_lib = None


class SmHipError(RuntimeError):
    pass


def lib():
    """Load libsharpmind_hip.so (built in-tree by sharpmind_amd.build)."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise SmHipError(
                f"{LIB_PATH} is missing: build it with `python -m sharpmind_amd.build` "
                "(no CPU fallback exists)")
        _lib = ctypes.CDLL(LIB_PATH)
        from . import _abi
        _abi.declare(_lib)
    return _lib


def check(rc):
    if rc != 0:
        msg = lib().smhip_last_error().decode(errors="replace")
        raise SmHipError(f"libsharpmind_hip error {rc}: {msg}")
    return rc
