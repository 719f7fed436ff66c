"""ctypes declarations generated from include/sharpmind_hip.h.

The header is the single source of truth for the C ABI: each prototype is
parsed here (plain C types only) so Python callers, the symbol-export test and
the C# P/Invoke shim all bind the same signatures.
"""
import ctypes
import os
import re

HEADER = os.path.join(os.path.dirname(os.path.abspath(__file__)), "..", "include", "sharpmind_hip.h")

_SCALARS = {
    "int": ctypes.c_int, "int32_t": ctypes.c_int32, "int64_t": ctypes.c_int64, "uint64_t": ctypes.c_uint64,
    "float": ctypes.c_float, "double": ctypes.c_double, "size_t": ctypes.c_size_t,
    "smhip_stream_t": ctypes.c_void_p, "void": None,
}


def _ctype(decl):
    decl = decl.replace("const ", "").strip()
    if "*" in decl:
        base = decl.split("*")[0].strip()
        return ctypes.c_char_p if base == "char" else ctypes.c_void_p
    toks = decl.split()
    return _SCALARS[toks[0]]


def prototypes(path=HEADER):
    """[(name, restype, [argtypes])] for every function declared in the header."""
    text = open(path).read()
    text = re.sub(r"/\*.*?\*/", " ", text, flags=re.S)
    out = []
    for m in re.finditer(r"\b(int|const char\s*\*|void)\s+(smhip_\w+)\s*\(([^)]*)\)\s*;", text):
        ret, name, args = m.group(1), m.group(2), m.group(3).strip()
        restype = ctypes.c_char_p if "char" in ret else (_SCALARS[ret] if ret != "void" else None)
        argtypes = []
        if args and args != "void":
            for a in args.split(","):
                a = a.strip()
                # drop the parameter name
                decl = re.sub(r"\b\w+\s*$", "", a) if not a.endswith("*") else a
                argtypes.append(_ctype(decl))
        out.append((name, restype, argtypes))
    return out


def declare(lib):
    for name, res, args in prototypes():
        f = getattr(lib, name)
        f.restype = res
        f.argtypes = args
