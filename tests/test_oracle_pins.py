"""Pins the CPU oracle (oracle/oracle.c) before it is trusted as the GPU checker.

Each oracle function is checked against something independent of its own
formula: the reference's golden files (tests/golden/dataref, copied from
SharpMind.Tests/DataRef), the reference's known-answer tests (cited), the
reference's own C tool built from its sources (oracle/_ref), IEEE identities
checked with numpy, or float64 finite differences of the forward function.
"""
import os

import numpy as np
import pytest

import oracle
from oracle import DotNetRandom, f32

from conftest import rel_err

GOLD = os.path.join(os.path.dirname(__file__), "golden", "dataref")


def _parse(path):
    return np.array([float(s.replace("∞", "inf")) for s in open(path, encoding="utf-8").read().split()],
                    np.float32)


# ------------------------------------------------------------------ .NET Random + DataRef goldens
@pytest.mark.parametrize("dtype,qk,bb,fn", [(8, 32, 34, "orc_dequant_q8_0"), (12, 256, 144, "orc_dequant_q4k")])
def test_dataref_read_bitexact(orc, dtype, qk, bb, fn):
    """VecDotTests.Read_AgreesWithCReference (VecDotTests.cs:597-627): raw = Random(42).NextBytes."""
    assert open(os.path.join(GOLD, "seed.txt")).read().strip() == "42"
    n = 4 * qk
    raw = DotNetRandom(42).next_bytes(2 * 4 * bb)
    for c in range(2):
        ref = _parse(os.path.join(GOLD, f"refread_{dtype}_c{c}.bin"))
        out = np.zeros(n, np.float32)
        getattr(orc, fn)(np.ascontiguousarray(raw[c * 4 * bb:(c + 1) * 4 * bb]), out, n)
        same = (out.view(np.uint32) == ref.view(np.uint32)) | (np.isnan(out) & np.isnan(ref))
        assert same.all(), f"dtype {dtype} col {c}: {np.flatnonzero(~same)[:5]}"


@pytest.mark.parametrize("dtype,qk,bb,fn", [(8, 32, 34, "orc_vecdot_q8_0"), (12, 256, 144, "orc_vecdot_q4k")])
def test_dataref_vecdot_exact(orc, dtype, qk, bb, fn):
    """VecDotTests.VecDot_AgreesWithCReference (VecDotTests.cs:522-590): input then weights from one Random(42)."""
    n = 4 * qk
    r = DotNetRandom(42)
    inp = r.uniform_pm1(n)
    raw = r.next_bytes(2 * 4 * bb)
    for c in range(2):
        gold = np.float32(float(open(os.path.join(GOLD, f"ref_{dtype}_c{c}.bin")).read()))
        assert np.float32(getattr(orc, fn)(inp, raw, c, n)) == gold


def test_vecdot_matches_reference_c_tool(orc):
    """oracle vs tools/ReferenceDataGenerator/vecdot_ref.c compiled from the reference sources."""
    R = oracle.ref_lib()
    if R is None:
        pytest.skip("oracle/_ref not built (no reference checkout)")
    rng = np.random.default_rng(5)
    for K in (32, 256, 1024):
        inp = f32(rng.standard_normal(K))
        for dtype_fn, rfn, bb, qk in (("orc_vecdot_q8_0", R.vecdot_q8_0, 34, 32), ("orc_vecdot_q4k", R.vecdot_q4_K, 144, 256)):
            if K % qk:  # whole blocks only: a shorter K would have both read past the buffer
                continue
            raw = rng.integers(0, 256, size=(K // qk) * bb, dtype=np.uint8)
            if bb == 34:  # keep scales finite so sums are comparable
                for b in range(K // qk):
                    raw[b * 34 + 1] &= 0x3B
            else:
                for b in range(K // qk):
                    raw[b * 144 + 1] &= 0x3B
                    raw[b * 144 + 3] &= 0x3B
            a = getattr(orc, dtype_fn)(inp, raw, 0, K)
            b = rfn(inp, raw, 0, K)
            assert np.float32(a) == np.float32(b)


# ------------------------------------------------------------------ half <-> float
HALF_KATS = [(0x0000, 0x00000000), (0x8000, 0x80000000), (0x3C00, 0x3F800000), (0xBC00, 0xBF800000),
             (0x3800, 0x3F000000), (0x4000, 0x40000000), (0x7BFF, 0x477FE000), (0x0400, 0x38800000),
             (0x0001, 0x33800000), (0x03FF, 0x387FC000), (0x1955, 0x3B2AA000), (0x67FF, 0x44FFE000)]


def test_half_to_float_kats(orc):
    """HalfToFloatTests.HalfToFloat_Scalar_ReturnsCorrectBits (HalfToFloatTests.cs:11-28)."""
    for h, bits in HALF_KATS:
        assert np.float32(orc.orc_half_to_float(h)).view(np.uint32) == bits


def test_half_to_float_exhaustive(orc):
    """All 65536 patterns against IEEE binary16->binary32 (numpy) and the reference C tool."""
    allh = np.arange(65536, dtype=np.uint16)
    ieee = allh.view(np.float16).astype(np.float32)
    mine = np.array([orc.orc_half_to_float(int(h)) for h in allh], np.float32)
    nan = np.isnan(ieee)
    assert (np.isnan(mine) == nan).all()
    assert (mine[~nan].view(np.uint32) == ieee[~nan].view(np.uint32)).all()
    R = oracle.ref_lib()
    if R is not None:
        refc = np.array([R.half_to_float(int(h)) for h in allh], np.float32)
        assert (np.isnan(refc) == nan).all()
        assert (refc[~nan].view(np.uint32) == mine[~nan].view(np.uint32)).all()


def test_float_to_half_rne(orc):
    """(Half)f is IEEE round-to-nearest-even: compare with numpy on edge and random values."""
    rng = np.random.default_rng(1)
    vals = np.concatenate([
        rng.standard_normal(20000).astype(np.float32) * np.float32(10.0) ** rng.integers(-9, 6, 20000).astype(np.float32),
        np.array([0.0, -0.0, 65504, 65519.99, 65520, 1e9, -1e9, 5.96e-8, 2.98e-8, 2.99e-8, 1e-10,
                  6.103515625e-05, 6.1e-05, np.inf, -np.inf], np.float32)])
    ref = vals.astype(np.float16).view(np.uint16)
    mine = np.array([orc.orc_float_to_half_rne(float(v)) for v in vals], np.uint16)
    assert (mine == ref).all()


# ------------------------------------------------------------------ encoders
def test_q8_0_encoder_roundtrip(orc):
    """TensorQuantizer.WriteBlock (TensorQuantizer.cs:80-144): |x - deq| <= d/2 (+half rounding), amax -> +-127, zero block."""
    rng = np.random.default_rng(2)
    x = f32(rng.standard_normal(32 * 64) * 0.02)
    x[:32] = 0.0
    raw = np.zeros(64 * 34, np.uint8)
    assert orc.orc_quantize_q8_0(x, x.size, raw) == 0
    deq = np.zeros_like(x)
    orc.orc_dequant_q8_0(raw, deq, x.size)
    assert (deq[:32] == 0).all() and (raw[:34] == 0).all()
    for b in range(1, 64):
        blk = x[b * 32:(b + 1) * 32]
        d = np.abs(blk).max() / 127.0
        dh = raw[b * 34:b * 34 + 2].view(np.float16)[0].astype(np.float64)
        assert abs(dh - d) <= d * 2 ** -10
        q = raw[b * 34 + 2:(b + 1) * 34].view(np.int8)
        assert np.abs(q).max() == 127
        err = np.abs(deq[b * 32:(b + 1) * 32].astype(np.float64) - blk)
        assert err.max() <= 0.5 * dh + 128 * abs(dh - d) + 1e-12


def test_q4k_encoder_roundtrip(orc):
    """KQuantEncoderTests (KQuantEncoderTests.cs:48-95): rel RMS < 0.12, all-zero block encodes to zeros."""
    rng = np.random.default_rng(3)
    x = f32(rng.standard_normal(256 * 32) * 0.02)
    x[:256] = 0
    raw = np.zeros(32 * 144, np.uint8)
    assert orc.orc_quantize_q4k(x, x.size, raw) == 0
    deq = np.zeros_like(x)
    orc.orc_dequant_q4k(raw, deq, x.size)
    assert (raw[:144] == 0).all() and (deq[:256] == 0).all()
    rel_rms = np.sqrt(np.mean((deq[256:] - x[256:]) ** 2)) / np.sqrt(np.mean(x[256:] ** 2))
    assert rel_rms < 0.12


# ------------------------------------------------------------------ GradientMapping slots
def test_linear_kat(orc):
    """GradientMappingTests.Linear_ReturnsDInput_AndAccumulatesGradients (GradientMappingTests.cs:26-48)."""
    dY = f32([[1, 2, 3], [4, 5, 6]])
    X = f32([[1, 1, 1, 1], [2, 2, 2, 2]])
    W = np.ones((3, 4), np.float32)
    dW = np.zeros((3, 4), np.float32)
    db = np.zeros(3, np.float32)
    dX = np.zeros((2, 4), np.float32)
    orc.orc_grad_linear(dY, X, W, dW, db.ctypes.data, dX, 2, 4, 3)
    assert dW[0, 0] == 9 and dW[2, 3] == 15 and db[0] == 5 and db[2] == 9


def test_linear_brute_force(orc):
    rng = np.random.default_rng(4)
    B, In, Out = 7, 13, 11
    dY, X, W = (f32(rng.standard_normal(s)) for s in ((B, Out), (B, In), (Out, In)))
    dW0 = f32(rng.standard_normal((Out, In)))
    dW = dW0.copy()
    db = np.zeros(Out, np.float32)
    dX = np.zeros((B, In), np.float32)
    orc.orc_grad_linear(dY, X, W, dW, db.ctypes.data, dX, B, In, Out)
    d64 = dY.astype(np.float64)
    assert rel_err(dX, d64 @ W) < 1e-6
    assert rel_err(dW - dW0, d64.T @ X) < 1e-6
    assert rel_err(db, d64.sum(0)) < 1e-6


def _fd(f, x, h=1e-6):
    g = np.zeros_like(x)
    it = np.nditer(x, flags=["multi_index"])
    for _ in it:
        i = it.multi_index
        old = x[i]
        x[i] = old + h
        fp = f(x)
        x[i] = old - h
        fm = f(x)
        x[i] = old
        g[i] = (fp - fm) / (2 * h)
    return g


def test_rmsnorm_kat_and_fd(orc):
    """KAT GradientMappingTests.cs:50-65 (dw[0]=2) and finite differences of y = x*rinv(x)*w."""
    T, D = 2, 3
    dY = np.ones((T, D), np.float32)
    xn = np.ones((T, D), np.float32)
    rinv = f32([2, 2])
    w = np.ones(D, np.float32)
    dw = np.zeros(D, np.float32)
    dX = np.zeros((T, D), np.float32)
    orc.orc_grad_rmsnorm(dY, xn, rinv, w, dw, dX, T, D)
    assert dw[0] == 2
    rng = np.random.default_rng(6)
    T, D, eps = 3, 16, 1e-6
    x = rng.standard_normal((T, D))
    w = 1 + 0.1 * rng.standard_normal(D)
    g = rng.standard_normal((T, D))

    def loss(xx):
        r = 1 / np.sqrt((xx ** 2).mean(1, keepdims=True) + eps)
        return float((xx * r * w * g).sum())

    def lossw(ww):
        r = 1 / np.sqrt((x ** 2).mean(1, keepdims=True) + eps)
        return float((x * r * ww * g).sum())

    r = 1 / np.sqrt((x ** 2).mean(1) + eps)
    dw = np.zeros(D, np.float32)
    dX = np.zeros((T, D), np.float32)
    orc.orc_grad_rmsnorm(f32(g), f32(x * r[:, None]), f32(r), f32(w), dw, dX, T, D)
    assert rel_err(dX, _fd(loss, x.copy())) < 1e-5
    assert rel_err(dw, _fd(lossw, w.copy())) < 1e-5


def test_rmsnorm_forward_param(orc):
    rng = np.random.default_rng(7)
    for n in (5, 64, 1024, 1027):
        x = f32(rng.standard_normal(n) * 3)
        ref = 1 / np.sqrt((x.astype(np.float64) ** 2).mean() + 1e-6)
        assert abs(orc.orc_rmsnorm_param(x, n, 1e-6) - ref) / ref < 1e-6


def test_layernorm_kat_and_fd(orc):
    """KAT GradientMappingTests.cs:67-84 (db[0]=2) and finite differences."""
    T, D = 2, 3
    dY = np.ones((T, D), np.float32)
    x = f32([[1, 1, 1], [2, 2, 2]])
    w = np.ones(D, np.float32)
    dw = np.zeros(D, np.float32)
    db = np.zeros(D, np.float32)
    dX = np.zeros((T, D), np.float32)
    orc.orc_grad_layernorm(dY, x, w, dw, db, dX, T, D, 1e-5)
    assert db[0] == 2
    rng = np.random.default_rng(8)
    T, D, eps = 3, 12, 1e-5
    x = rng.standard_normal((T, D))
    w = 1 + 0.1 * rng.standard_normal(D)
    g = rng.standard_normal((T, D))

    def loss(xx):
        mu = xx.mean(1, keepdims=True)
        var = ((xx - mu) ** 2).mean(1, keepdims=True)
        return float(((xx - mu) / np.sqrt(var + eps) * w * g).sum())

    dw = np.zeros(D, np.float32)
    db = np.zeros(D, np.float32)
    dX = np.zeros((T, D), np.float32)
    orc.orc_grad_layernorm(f32(g), f32(x), f32(w), dw, db, dX, T, D, eps)
    assert rel_err(dX, _fd(loss, x.copy())) < 1e-4
    assert rel_err(db, g.sum(0)) < 1e-6


def _softmax_causal(s):
    S = s.shape[0]
    m = np.triu(np.ones((S, S), bool), 1)
    s = np.where(m, -np.inf, s)
    e = np.exp(s - s.max(1, keepdims=True))
    return e / e.sum(1, keepdims=True)


def test_attention_forward_and_backward_fd(orc):
    """Forward probs: causal rows sum to 1; backward (GradientKernels.cs:408-481) vs finite differences."""
    rng = np.random.default_rng(9)
    S, D = 6, 4
    q, k, v, dO = (rng.standard_normal((S, D)) for _ in range(4))
    scale = 1 / np.sqrt(D)
    probs = np.zeros((1, 1, S, S), np.float32)
    out = np.zeros((1, S, D), np.float32)
    orc.orc_attention_fwd(f32(q), f32(k), f32(v), probs, out, 1, S, 1, 1, D)
    P = _softmax_causal(q @ k.T * scale)
    assert rel_err(probs[0, 0], P) < 1e-6 and rel_err(out[0], P @ v) < 1e-6

    def L(qq, kk, vv):
        return float((_softmax_causal(qq @ kk.T * scale) @ vv * dO).sum())

    dQ, dK, dV = (np.zeros((S, D), np.float32) for _ in range(3))
    orc.orc_grad_attention(f32(dO), f32(q), f32(k), f32(v), f32(P), dQ, dK, dV, S, D, scale)
    assert rel_err(dQ, _fd(lambda x: L(x, k, v), q.copy())) < 1e-5
    assert rel_err(dK, _fd(lambda x: L(q, x, v), k.copy())) < 1e-5
    assert rel_err(dV, _fd(lambda x: L(q, k, x), v.copy())) < 1e-5


def test_attention_forward_gqa_group_mapping(orc):
    """GQA: query head h reads kv head h // (Hq/Hkv) (BackpropEngine.cs:283)."""
    rng = np.random.default_rng(10)
    B, S, Hq, Hkv, D = 2, 5, 4, 2, 3
    q = f32(rng.standard_normal((B, S, Hq, D)))
    k = f32(rng.standard_normal((B, S, Hkv, D)))
    v = f32(rng.standard_normal((B, S, Hkv, D)))
    probs = np.zeros((B, Hq, S, S), np.float32)
    out = np.zeros((B, S, Hq * D), np.float32)
    orc.orc_attention_fwd(q, k, v, probs, out, B, S, Hq, Hkv, D)
    for b in range(B):
        for h in range(Hq):
            P = _softmax_causal(q[b, :, h].astype(np.float64) @ k[b, :, h // 2].T / np.sqrt(D))
            assert rel_err(probs[b, h], P) < 1e-6
            assert rel_err(out[b, :, h * D:(h + 1) * D], P @ v[b, :, h // 2]) < 1e-6


def test_embedding_kat(orc):
    """GradientMappingTests.Embedding_AccumulatesIntoSelectedRows (GradientMappingTests.cs:108-122)."""
    dY = np.ones((2, 3), np.float32)
    ids = np.array([1, 3], np.int32)
    dE = np.zeros((5, 3), np.float32)
    orc.orc_grad_embedding(dY, ids, dE, 2, 3)
    assert dE[1, 0] == 1 and dE[0, 0] == 0 and dE[3, 2] == 1


def test_silu_gelu_fd(orc):
    rng = np.random.default_rng(11)
    x = rng.standard_normal(50) * 3
    g = rng.standard_normal(50)
    silu = lambda z: z / (1 + np.exp(-z))
    gelu = lambda z: 0.5 * z * (1 + np.tanh(0.7978845608 * (z + 0.044715 * z ** 3)))
    for fn, f in (("orc_grad_silu", silu), ("orc_grad_gelu", gelu)):
        dx = np.zeros(50, np.float32)
        getattr(orc, fn)(f32(g), f32(x), dx, 50)
        num = (f(x + 1e-6) - f(x - 1e-6)) / 2e-6 * g
        assert rel_err(dx, num) < 1e-5


def test_swiglu_fd(orc):
    rng = np.random.default_rng(12)
    T, F = 3, 10
    g, u, da = (rng.standard_normal((T, F)) * 2 for _ in range(3))
    out = np.zeros((T, 2 * F), np.float32)
    orc.orc_grad_swiglu(f32(da), f32(g), f32(u), out, T, F)
    act = lambda gg, uu: gg / (1 + np.exp(-gg)) * uu
    dg = (act(g + 1e-6, u) - act(g - 1e-6, u)) / 2e-6 * da
    du = (act(g, u + 1e-6) - act(g, u - 1e-6)) / 2e-6 * da
    assert rel_err(out[:, :F], dg) < 1e-5 and rel_err(out[:, F:], du) < 1e-5
    a = np.zeros(T * F, np.float32)
    orc.orc_swiglu_fwd(f32(g).ravel(), f32(u).ravel(), a, T * F)
    assert rel_err(a, act(g, u).ravel()) < 1e-6


# ------------------------------------------------------------------ RoPE
def test_rope_forward_kats(orc):
    """RoPETests.Apply_AdjacentPairing_* (RoPETests.cs:44-78), RoPEConventionTests (RoPEConventionTests.cs:34-73)."""
    for D in (4, 8):
        cos_t = np.zeros((8, D // 2), np.float32)
        sin_t = np.zeros_like(cos_t)
        orc.orc_rope_tables(10000.0, D, 8, cos_t, sin_t)
        for neox in (0, 1):
            x = np.zeros((2, 1, D), np.float32)
            x[1, 0] = np.arange(1, D + 1)
            x[0, 0] = np.arange(1, D + 1)
            orc.orc_rope_fwd(x, cos_t, sin_t, 2, 1, D, neox)
            assert np.allclose(x[0, 0], np.arange(1, D + 1), atol=1e-6)  # position 0 is identity
            for i in range(D // 2):
                th = np.float32(10000.0) ** np.float32(-2.0 * i / D)
                i0, i1 = (i, i + D // 2) if neox else (2 * i, 2 * i + 1)
                a, b = i0 + 1.0, i1 + 1.0
                assert abs(x[1, 0, i0] - (a * np.cos(th) - b * np.sin(th))) < 1e-5
                assert abs(x[1, 0, i1] - (b * np.cos(th) + a * np.sin(th))) < 1e-5


def test_rope_backward_is_transpose(orc):
    """<R x, y> == <x, R^T y>: pins ApplyBackward (RoPE.cs:300-347) to Apply."""
    rng = np.random.default_rng(13)
    S, H, D = 9, 3, 16
    cos_t = np.zeros((S, D // 2), np.float32)
    sin_t = np.zeros_like(cos_t)
    orc.orc_rope_tables(1e6, D, S, cos_t, sin_t)
    for neox in (0, 1):
        x = f32(rng.standard_normal((S, H, D)))
        y = f32(rng.standard_normal((S, H, D)))
        rx = x.copy()
        orc.orc_rope_fwd(rx, cos_t, sin_t, S, H, D, neox)
        ry = y.copy()
        orc.orc_rope_bwd(ry, cos_t, sin_t, S, H, D, neox)
        a = float((rx.astype(np.float64) * y).sum())
        b = float((x.astype(np.float64) * ry).sum())
        assert abs(a - b) < 1e-4 * (abs(a) + 1)
        back = rx.copy()
        orc.orc_rope_bwd(back, cos_t, sin_t, S, H, D, neox)
        assert rel_err(back, x) < 1e-6  # rotation is orthogonal


# ------------------------------------------------------------------ loss / optimizer
def _ce_loss64(z, lab, sm, ignore=-100):
    m = lab != ignore
    zz = z[m]
    lse = np.log(np.exp(zz - zz.max(1, keepdims=True)).sum(1)) + zz.max(1)
    logp = zz - lse[:, None]
    V = z.shape[1]
    u = np.full(zz.shape, sm / V)
    u[np.arange(zz.shape[0]), lab[m]] += 1 - sm
    return float(-(u * logp).sum(1).mean())


def test_ce_grad_fd_and_invariants(orc):
    """CrossEntropyLossTests (CrossEntropyLossTests.cs:172-255): FD, ignore id, smoothing; sum_v dz = 0."""
    rng = np.random.default_rng(14)
    T, V = 5, 17
    z = rng.standard_normal((T, V)) * 2
    lab = rng.integers(0, V, T).astype(np.int32)
    lab[2] = -100
    for sm in (0.0, 0.1):
        d = np.zeros((T, V), np.float32)
        orc.orc_ce_softmax_grad(f32(z), lab, d, T, V, -100, sm)
        assert (d[2] == 0).all()
        num = _fd(lambda zz: _ce_loss64(zz, lab, sm), z.copy())
        assert rel_err(d, num) < 1e-5
        assert abs(orc.orc_ce_loss(f32(z), lab, T, V, -100, sm) - _ce_loss64(z, lab, sm)) < 1e-5
        assert np.abs(d.sum(1)).max() < 1e-6


def test_adamw_first_step_closed_form(orc):
    """t=1: m_hat = g, v_hat = g^2, so theta -= lr*(g/(|g|+eps) + decay*theta)."""
    rng = np.random.default_rng(15)
    n = 1000
    th = f32(rng.standard_normal(n) * 0.02)
    g = f32(rng.standard_normal(n) * 0.02)
    m = np.zeros(n, np.float32)
    v = np.zeros(n, np.float32)
    b1, b2, lr, eps, wd = 0.9, 0.95, 1e-3, 1e-8, 0.1
    new = th.copy()
    orc.orc_adamw(new, g, m, v, n, b1, b2, 1 - b1, 1 - b2, lr, eps, wd)
    g64 = g.astype(np.float64)
    ref = th - lr * (g64 / (np.abs(g64) + eps) + wd * th)
    assert np.abs(new - ref).max() < 1e-6
    assert rel_err(m, (1 - b1) * g64) < 1e-6 and rel_err(v, (1 - b2) * g64 ** 2) < 1e-6


def test_l2normsq(orc):
    rng = np.random.default_rng(16)
    x = f32(rng.standard_normal(10001))
    ref = float((x.astype(np.float64) ** 2).sum())
    assert abs(orc.orc_l2normsq(x, x.size) - ref) < 1e-5 * ref


# ------------------------------------------------------------------ LoRA (no reference backward)
def test_lora_forward_contract_and_backward_fd(orc):
    """Forward y = xW^T + s(xA)B (LoRALayer.cs:52-80, LoRATests.cs:53-98); backward vs FD; B=0 invariant."""
    rng = np.random.default_rng(17)
    T, In, Out, r, s = 4, 6, 5, 3, 2.0
    x, W, A, Bm, dY = (rng.standard_normal(sh) for sh in ((T, In), (Out, In), (In, r), (r, Out), (T, Out)))
    y = np.zeros((T, Out), np.float32)
    orc.orc_lora_fwd(f32(x), f32(W), f32(A), f32(Bm), y, T, In, Out, r, s)
    assert rel_err(y, x @ W.T + s * (x @ A) @ Bm) < 1e-6

    def L(xx, AA, BB):
        return float(((xx @ W.T + s * (xx @ AA) @ BB) * dY).sum())

    dA = np.zeros((In, r), np.float32)
    dB = np.zeros((r, Out), np.float32)
    dX = np.zeros((T, In), np.float32)
    orc.orc_lora_bwd(f32(dY), f32(x), f32(W), f32(A), f32(Bm), dA, dB, dX, T, In, Out, r, s)
    assert rel_err(dA, _fd(lambda a: L(x, a, Bm), A.copy())) < 1e-5
    assert rel_err(dB, _fd(lambda b: L(x, A, b), Bm.copy())) < 1e-5
    assert rel_err(dX, _fd(lambda a: L(a, A, Bm), x.copy())) < 1e-5
    dA[:] = 0
    dB[:] = 0
    orc.orc_lora_bwd(f32(dY), f32(x), f32(W), f32(A), np.zeros((r, Out), np.float32), dA, dB, dX, T, In, Out, r, s)
    assert (dA == 0).all() and rel_err(dX, dY @ W) < 1e-6


# ------------------------------------------------------------------ encoder known-answer blocks
# Bytes derived by hand from TensorQuantizer.WriteBlock (TensorQuantizer.cs:80-144: d = amax/127
# stored as (Half)d, q = Round(x/d, AwayFromZero) with the float d) and WriteKQ4 /
# PackScaleMinK4 (TensorQuantizer.KQuant.cs:173-225, 451-459).  Each block holds values where a
# plausible mistake gives other bytes: round-half-even or truncation of x/d, truncation of d to
# half, dividing by the half-rounded d, the sc clamp at 1, the mn clamp at 0, mn = 63 in the packed
# high bits, sc/mn of an upper sub-block, and the zero-range branch.
def test_q8_0_encoder_known_blocks(orc):
    a = np.zeros(32, np.float32)  # amax 127 -> d = 1.0 (half 0x3C00)
    a[:7] = [127.0, 2.5, -2.5, 0.5, -0.5, 1.4999999, -127.0]
    b = np.zeros(32, np.float32)  # amax/127 = 1 + 3*2^-12: (Half) rounds to nearest even -> 0x3C01
    b[0], b[1] = 127.093017578125, 99.583   # 99.583 / 1.000732421875 = 99.51 -> 100 (99 with the half d)
    c = np.zeros(32, np.float32)  # zero block: d = 0, codes 0
    x = np.concatenate([a, b, c])
    raw = np.zeros(3 * 34, np.uint8)
    assert orc.orc_quantize_q8_0(x, x.size, raw) == 0
    ea = [0x00, 0x3C, 0x7F, 0x03, 0xFD, 0x01, 0xFF, 0x01, 0x81] + [0] * 25
    eb = [0x01, 0x3C, 0x7F, 0x64] + [0] * 30
    assert raw.tolist() == ea + eb + [0] * 34


def test_q4k_encoder_known_blocks(orc):
    # block 1: amax 63 -> step 1.0 (d = dmin = 0x3C00); per sub-block (sc, mn) by hand:
    #   0: [-2, 28, -1, 1, 3, 0...]  range 30 -> sc 2, mn 2; codes (x+2)/2: 0, 15, 1 (0.5 away), 2, 3 (2.5 away), 1...
    #   1: [0.1, 0...]               range 0.1 -> sc round(0.0067) = 0 -> clamp 1; mn -0 -> 0; codes 0
    #   2: [5, 10, 7.5...]           range 5 -> sc 0 -> 1; mn round(-5) -> clamp 0; codes 5, 10, 8 (7.5 away)
    #   3: all -3                    zero range: sc 0, mn 3, codes 0
    #   4: [-10, 27.5, 0...]         range 37.5 -> sc round(2.5) = 3 (away), mn 10; codes 0, 13 (12.5), 3 (3.33)
    #   5: [-63, 1, 0...]            range 64 -> sc 4, mn 63; codes 0, 15 (16 clamped), 15 (15.75 -> 16 clamped)
    #   6: all 0                     zero range: sc 0, mn 0
    #   7: [63, 0...]                range 63 -> sc 4, mn 0; codes 15 (15.75 -> 16 clamped), 0
    # block 2: amax 63.046142578125 -> step 1 + 3*2^-12, half RNE 0x3C01; sub-block 0 = [amax, 0...]: sc 4, mn 0
    blk = np.zeros((8, 32), np.float32)
    blk[0, :5] = [-2, 28, -1, 1, 3]
    blk[1, 0] = 0.1
    blk[2, :] = 7.5
    blk[2, :2] = [5, 10]
    blk[3, :] = -3
    blk[4, :2] = [-10, 27.5]
    blk[5, :2] = [-63, 1]
    blk[7, 0] = 63
    blk2 = np.zeros(256, np.float32)
    blk2[0] = 63.046142578125
    x = np.concatenate([blk.ravel(), blk2])
    raw = np.zeros(2 * 144, np.uint8)
    assert orc.orc_quantize_q4k(x, x.size, raw) == 0
    e1 = [0x00, 0x3C, 0x00, 0x3C]
    e1 += [0x02, 0x01, 0x01, 0x00, 0x02, 0xC0, 0x00, 0x03, 0xA3, 0xF4, 0x00, 0x04]
    qs = [0x01] * 128
    qs[0:5] = [0x00, 0x0F, 0x01, 0x02, 0x03]              # sub 0 low nibbles, sub 1 high nibbles (0)
    qs[32:64] = [0x05, 0x0A] + [0x08] * 30                 # sub 2 low, sub 3 high (0)
    qs[64:96] = [0x00, 0xFD] + [0xF3] * 30                 # sub 4 low, sub 5 high
    qs[96:128] = [0xF0] + [0x00] * 31                      # sub 6 low (0), sub 7 high
    e1 += qs
    e2 = [0x01, 0x3C, 0x01, 0x3C] + [0x04] + [0x00] * 11 + [0x0F] + [0x00] * 127
    assert raw[:144].tolist() == e1
    assert raw[144:].tolist() == e2
