"""Python restatement of the reference's GGUF writer and header reader.

TEST INFRASTRUCTURE ONLY: imported by tests/, never by the sharpmind_amd package.

Follows SharpMind.Model/Format/GgufWriter.cs (Write :50-100, WriteString :102-107, WriteValue
:109-140, Align :172-173) and GgufLoader.LoadMeta (GgufLoader.cs:124-177); byte counts follow
QuantizationOps.GetRawTensorByteCount (QuantizationOps.cs:15-72).
"""
import struct

import numpy as np

MAGIC = 0x46554747
F32, F16, Q8_0, Q4_K = 0, 1, 8, 12


def tensor_bytes(dims, dtype):
    """QuantizationOps.GetRawTensorByteCount for the types used here (dims as stored)."""
    n = int(np.prod(dims))
    if dtype == F32:
        return 4 * n
    if dtype == F16:
        return 2 * n
    if dtype == Q4_K:
        return (n + 255) // 256 * 144
    if dtype == Q8_0:  # GetBlockQuantByteCount(shape, 32, 34): blocks along the last stored dim
        outer = int(np.prod(dims[:-1])) if len(dims) > 1 else 1
        return outer * ((dims[-1] + 31) // 32) * 34
    raise ValueError(dtype)


def _align(x, a):
    return (x + a - 1) & ~(a - 1)


def _string(s):
    b = s.encode("utf-8")
    return struct.pack("<Q", len(b)) + b


def _value(v):
    """(type id, payload) as WriteValue encodes .NET values; tuples tag the scalar type."""
    if isinstance(v, tuple):  # (type id, python value)
        t, x = v
        fmt = {0: "<B", 1: "<b", 2: "<H", 3: "<h", 4: "<I", 5: "<i", 6: "<f", 7: "<?", 10: "<Q", 11: "<q", 12: "<d"}[t]
        return struct.pack("<I", t) + struct.pack(fmt, x)
    if isinstance(v, bool):
        return struct.pack("<I", 7) + struct.pack("<?", v)
    if isinstance(v, int):
        return struct.pack("<I", 5) + struct.pack("<i", v)
    if isinstance(v, float):
        return struct.pack("<I", 6) + struct.pack("<f", v)
    if isinstance(v, str):
        return struct.pack("<I", 8) + _string(v)
    if isinstance(v, list):  # arrays: element type from the first element (strings, int32, float32)
        if v and isinstance(v[0], str):
            return struct.pack("<IIQ", 9, 8, len(v)) + b"".join(_string(x) for x in v)
        if v and isinstance(v[0], float):
            return struct.pack("<IIQ", 9, 6, len(v)) + b"".join(struct.pack("<f", x) for x in v)
        return struct.pack("<IIQ", 9, 5, len(v)) + b"".join(struct.pack("<i", x) for x in v)
    raise TypeError(type(v))


def write(path, kv, tensors, alignment=32):
    """GgufWriter.Write: kv = [(key, value)], tensors = [(name, dims innermost first, dtype, bytes)]."""
    head = struct.pack("<IIqq", MAGIC, 3, len(tensors), len(kv))
    for k, v in kv:
        head += _string(k) + _value(v)
    cursor = 0
    for name, dims, dtype, data in tensors:
        assert len(data) == tensor_bytes(dims, dtype), name
        head += _string(name) + struct.pack("<I", len(dims)) + b"".join(struct.pack("<Q", d) for d in dims)
        head += struct.pack("<IQ", dtype, cursor)
        cursor = _align(cursor + len(data), alignment)
    with open(path, "wb") as f:
        f.write(head)
        f.write(b"\0" * (_align(len(head), alignment) - len(head)))
        for _, _, _, data in tensors:
            f.write(data)
            pad = _align(f.tell(), alignment) - f.tell()
            f.write(b"\0" * pad)


def read_table(path):
    """GgufLoader.LoadMeta: [(name, dims, dtype, absolute data offset)] and the kv dict of scalars."""
    with open(path, "rb") as f:
        buf = f.read()
    pos = 0

    def take(fmt):
        nonlocal pos
        out = struct.unpack_from(fmt, buf, pos)
        pos += struct.calcsize(fmt)
        return out

    def string():
        (n,) = take("<Q")
        nonlocal pos
        s = buf[pos:pos + n].decode("utf-8")
        pos += n
        return s

    sizes = {0: "<B", 1: "<b", 2: "<H", 3: "<h", 4: "<I", 5: "<i", 6: "<f", 7: "<?", 10: "<Q", 11: "<q", 12: "<d"}

    def value(t):
        if t == 8:
            return string()
        if t == 9:
            et, n = take("<IQ")
            return [value(et) for _ in range(n)]
        return take(sizes[t])[0]

    magic, version, nt, nkv = take("<IIqq")
    assert magic == MAGIC
    kv = {}
    for _ in range(nkv):
        k = string()
        (t,) = take("<I")
        kv[k] = value(t)
    table = []
    for _ in range(nt):
        name = string()
        (nd,) = take("<I")
        dims = take("<%dQ" % nd)
        dtype, off = take("<IQ")
        table.append([name, tuple(dims), dtype, off])
    data = _align(pos, int(kv.get("general.alignment", 32)))
    for t in table:
        t[3] += data
    return [tuple(t) for t in table], kv
