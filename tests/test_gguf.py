"""GGUF container reading on the CPU: the library's tensor table against the format restatement
(GgufWriter.cs / GgufLoader.LoadMeta), over every metadata value type the format has."""
import numpy as np
import pytest

from oracle import gguf as og
from sharpmind_amd import SmHipError
from sharpmind_amd.engine import gguf_tensor_table

KV = [
    ("general.architecture", "qwen3"),
    ("general.alignment", (4, 64)),
    ("qwen3.block_count", (4, 2)),
    ("qwen3.rope.freq_base", 1e6),
    ("qwen3.tie_word_embeddings", True),
    ("tokenizer.ggml.tokens", ["<s>", "</s>", "hello"]),
    ("tokenizer.ggml.token_type", [1, 3, 1]),
    ("tokenizer.ggml.scores", [0.0, -1.5, 2.25]),
    ("big.u64", (10, 2 ** 40)), ("small.i8", (1, -3)), ("half.u16", (2, 7)), ("dbl", (12, 0.5)), ("i64", (11, -9)),
]


def _tensors(rng):
    return [
        ("token_embd.weight", (64, 10), og.Q8_0, rng.integers(0, 256, og.tensor_bytes((64, 10), og.Q8_0), np.uint8).tobytes()),
        ("blk.0.attn_norm.weight", (64,), og.F32, rng.standard_normal(64).astype(np.float32).tobytes()),
        ("blk.0.ffn_down.weight", (256, 64), og.Q4_K, rng.integers(0, 256, og.tensor_bytes((256, 64), og.Q4_K), np.uint8).tobytes()),
        ("blk.1.attn_q_norm.weight", (32,), og.F16, rng.standard_normal(32).astype(np.float16).tobytes()),
    ]


def test_table_matches_restatement(tmp_path):
    path = tmp_path / "m.gguf"
    og.write(str(path), KV, _tensors(np.random.default_rng(0)), alignment=64)
    ref, kv = og.read_table(str(path))
    assert kv["qwen3.block_count"] == 2 and kv["tokenizer.ggml.tokens"][2] == "hello"
    got = gguf_tensor_table(path)
    assert got == ref
    assert all(off % 64 == 0 for *_, off in got)
    # the data really is where the table says
    data = path.read_bytes()
    for (name, dims, dtype, off), (_, _, _, raw) in zip(got, _tensors(np.random.default_rng(0))):
        assert data[off:off + len(raw)] == raw, name


def test_default_alignment(tmp_path):
    path = tmp_path / "m.gguf"
    og.write(str(path), [("general.architecture", "llama")], _tensors(np.random.default_rng(1)))
    assert gguf_tensor_table(path) == og.read_table(str(path))[0]


def test_tensor_bytes_kats():
    """GetRawTensorByteCount (QuantizationOps.cs:15-72): Q8_0 34 B per 32, Q4_K 144 B per 256."""
    assert og.tensor_bytes((1024, 2048), og.Q8_0) == 1024 * 2048 // 32 * 34
    assert og.tensor_bytes((1024, 3072), og.Q4_K) == 1024 * 3072 // 256 * 144
    assert og.tensor_bytes((7,), og.F16) == 14 and og.tensor_bytes((7,), og.F32) == 28


def test_not_gguf_is_an_error(tmp_path):
    bad = tmp_path / "x.gguf"
    bad.write_bytes(b"GGML" + b"\0" * 64)
    with pytest.raises(SmHipError, match="not a GGUF"):
        gguf_tensor_table(bad)
    path = tmp_path / "t.gguf"
    og.write(str(path), KV, _tensors(np.random.default_rng(0)))
    trunc = tmp_path / "trunc.gguf"
    trunc.write_bytes(path.read_bytes()[:200])
    with pytest.raises(SmHipError):
        gguf_tensor_table(trunc)


def test_hand_assembled_header(tmp_path):
    """A file laid out byte by byte from the published GGUF v3 layout (magic "GGUF", u32 version,
    u64 tensor and KV counts, u64-length strings, u32 value types, tensor infos of name / u32 n_dims /
    u64 dims innermost first / u32 ggml type / u64 offset from the data section, the data section
    aligned to general.alignment), written without oracle/gguf.py's writer.  Offsets by hand:
    header = 24 + 45 (architecture) + 33 (alignment) + 57 + 50 (tensor infos) = 209 bytes, data at
    256; token_embd (Q8_0, 4 rows x 64) takes 4*2*34 = 272 bytes, so output_norm sits at 320."""
    import struct

    def s(x):
        return struct.pack("<Q", len(x)) + x.encode()

    hdr = b"GGUF" + struct.pack("<IQQ", 3, 2, 2)
    hdr += s("general.architecture") + struct.pack("<I", 8) + s("qwen3")
    hdr += s("general.alignment") + struct.pack("<II", 4, 64)
    hdr += s("token_embd.weight") + struct.pack("<IQQIQ", 2, 64, 4, 8, 0)
    hdr += s("output_norm.weight") + struct.pack("<IQIQ", 1, 64, 0, 320)
    assert len(hdr) == 209
    q8 = bytes(range(256)) + bytes(16)
    norm = np.arange(64, dtype=np.float32).tobytes()
    blob = hdr + bytes(256 - 209) + q8 + bytes(320 - 272) + norm
    path = tmp_path / "hand.gguf"
    path.write_bytes(blob)
    want = [("token_embd.weight", (64, 4), 8, 256), ("output_norm.weight", (64,), 0, 576)]
    assert gguf_tensor_table(path) == want
    table, kv = og.read_table(str(path))
    assert table == want and kv["general.architecture"] == "qwen3"
    assert blob[576:576 + 256] == norm
