"""GPU parity of every slot entry point against the pinned CPU oracle.

Calls go through libsharpmind_hip's C ABI (sharpmind_amd.hip is a thin ctypes
layer; torch only allocates device memory).  Tolerances (norm-wise relative
error, see conftest.rel_err): fp32 paths <= 1e-5, bf16 MFMA paths <= 2e-2,
dequantisation, AdamW and the embedding scatter bit-exact.
"""
import os

import numpy as np
import pytest
import torch

import oracle
from oracle import DotNetRandom, f32
from sharpmind_amd import hip

from conftest import rel_err

pytestmark = pytest.mark.gpu
GOLD = os.path.join(os.path.dirname(__file__), "golden", "dataref")
FP32_TOL = 1e-5
BF16_TOL = 2e-2


def T(a, dev):
    return torch.from_numpy(np.ascontiguousarray(a)).to(dev)


def H(t):
    torch.cuda.synchronize()
    return t.detach().cpu().numpy()


def _parse(path):
    return np.array([float(s.replace("∞", "inf")) for s in open(path, encoding="utf-8").read().split()], np.float32)


def _bits_equal(a, b):
    a = np.asarray(a, np.float32)
    b = np.asarray(b, np.float32)
    return bool(((a.view(np.uint32) == b.view(np.uint32)) | (np.isnan(a) & np.isnan(b))).all())


# ------------------------------------------------------------------ dequantisation
@pytest.mark.parametrize("qtype,qk,bb", [(8, 32, 34), (12, 256, 144)])
def test_dequant_dataref_bitexact(dev, qtype, qk, bb):
    raw = DotNetRandom(42).next_bytes(2 * 4 * bb)
    out = H(hip.QuantizationOps().Dequantize(qtype, T(raw, dev), 2 * 4 * qk))
    for c in range(2):
        ref = _parse(os.path.join(GOLD, f"refread_{qtype}_c{c}.bin"))
        assert _bits_equal(out[c * 4 * qk:(c + 1) * 4 * qk], ref)


@pytest.mark.parametrize("qtype,qk,bb", [(8, 32, 34), (12, 256, 144)])
def test_dequant_random_stream_bitexact(orc, dev, qtype, qk, bb):
    nb = 4099
    raw = np.random.default_rng(qtype).integers(0, 256, nb * bb, dtype=np.uint8)
    n = nb * qk
    ref = np.zeros(n, np.float32)
    (orc.orc_dequant_q8_0 if qtype == 8 else orc.orc_dequant_q4k)(raw, ref, n)
    out = H(hip.QuantizationOps().Dequantize(qtype, T(raw, dev), n))
    assert _bits_equal(out, ref)


def _quantized(orc, qtype, N, K, seed):
    w = f32(np.random.default_rng(seed).standard_normal((N, K)) * 0.02)
    if qtype == 8:
        raw = np.zeros(N * K // 32 * 34, np.uint8)
        assert orc.orc_quantize_q8_0(w.ravel(), w.size, raw) == 0
    else:
        raw = np.zeros(N * K // 256 * 144, np.uint8)
        assert orc.orc_quantize_q4k(w.ravel(), w.size, raw) == 0
    return raw


@pytest.mark.parametrize("qtype", [0, 8, 12])
@pytest.mark.parametrize("prec,tol", [(0, FP32_TOL), (1, BF16_TOL)])
def test_qmatmul(orc, dev, qtype, prec, tol):
    M, K, N = 37, 512, 300
    rng = np.random.default_rng(20)
    x = f32(rng.standard_normal((M, K)))
    ref = np.zeros((M, N), np.float32)
    if qtype == 0:
        w = f32(rng.standard_normal((N, K)) * 0.02)
        orc.orc_qmatmul_f32(x, w, ref, M, K, N)
        raw = w.view(np.uint8).ravel()
    else:
        raw = _quantized(orc, qtype, N, K, 21)
        (orc.orc_qmatmul_q8_0 if qtype == 8 else orc.orc_qmatmul_q4k)(x, raw, ref, M, K, N)
    out = H(hip.QuantizationOps(prec).QuantizedMatMul(qtype, T(x, dev), T(raw, dev), M, K, N))
    assert rel_err(out, ref) <= tol


# ------------------------------------------------------------------ Linear
def test_linear_kat(dev):
    """GradientMappingTests.cs:26-48 through the HIP slot."""
    gm = hip.GradientMapping(hip.PREC_FP32)
    w = hip.Parameter("w", torch.ones(3, 4, device=dev))
    b = hip.Parameter("b", torch.ones(3, device=dev))
    dX = gm.Linear(T(f32([[1, 2, 3], [4, 5, 6]]), dev), T(f32([[1, 1, 1, 1], [2, 2, 2, 2]]), dev), w, b)
    g = H(w.Grad)
    assert g[0, 0] == 9 and g[2, 3] == 15
    assert H(b.Grad)[0] == 5 and H(b.Grad)[2] == 9
    assert np.allclose(H(dX), [[6, 6, 6, 6], [15, 15, 15, 15]])


@pytest.mark.parametrize("B,In,Out", [(129, 200, 77), (256, 512, 384), (1, 48, 1000), (512, 688, 256)])
@pytest.mark.parametrize("prec,tol", [(0, FP32_TOL), (1, BF16_TOL)])
def test_linear_random(orc, dev, B, In, Out, prec, tol):
    rng = np.random.default_rng(B + In + Out)
    dY, X, W = f32(rng.standard_normal((B, Out))), f32(rng.standard_normal((B, In))), f32(rng.standard_normal((Out, In)))
    dW0, db0 = f32(rng.standard_normal((Out, In))), f32(rng.standard_normal(Out))
    rdW, rdb, rdX = dW0.copy(), db0.copy(), np.zeros((B, In), np.float32)
    orc.orc_grad_linear(dY, X, W, rdW, rdb.ctypes.data, rdX, B, In, Out)
    w = hip.Parameter("w", T(W, dev))
    w.Grad.copy_(T(dW0, dev))
    b = hip.Parameter("b", torch.zeros(Out, device=dev))
    b.Grad.copy_(T(db0, dev))
    dX = hip.GradientMapping(prec).Linear(T(dY, dev), T(X, dev), w, b)
    assert rel_err(H(dX), rdX) <= tol
    assert rel_err(H(w.Grad) - dW0, rdW - dW0) <= tol  # accumulated part
    assert rel_err(H(b.Grad), rdb) <= FP32_TOL


# ------------------------------------------------------------------ RMSNorm / LayerNorm
@pytest.mark.parametrize("Tn,D", [(2, 3), (8192, 1024), (300, 128), (77, 1001), (64, 2048)])
def test_rmsnorm(orc, dev, Tn, D):
    rng = np.random.default_rng(Tn * 7 + D)
    x = f32(rng.standard_normal((Tn, D)))
    dY = f32(rng.standard_normal((Tn, D)))
    w = f32(1 + 0.1 * rng.standard_normal(D))
    rinv = f32(1 / np.sqrt((x.astype(np.float64) ** 2).mean(1) + 1e-6))
    xn = f32(x * rinv[:, None])
    dw0 = f32(rng.standard_normal(D))
    rdw, rdx = dw0.copy(), np.zeros_like(x)
    orc.orc_grad_rmsnorm(dY, xn, rinv, w, rdw, rdx, Tn, D)
    p = hip.Parameter("w", T(w, dev))
    p.Grad.copy_(T(dw0, dev))
    dx = hip.GradientMapping().RMSNorm(T(dY, dev), T(xn, dev), T(rinv, dev), p)
    assert rel_err(H(dx), rdx) <= FP32_TOL
    assert rel_err(H(p.Grad) - dw0, rdw - dw0) <= FP32_TOL


def test_rmsnorm_forward(orc, dev):
    rng = np.random.default_rng(30)
    Tn, D = 513, 1024
    x = f32(rng.standard_normal((Tn, D)))
    w = f32(1 + 0.1 * rng.standard_normal(D))
    ry, rr = np.zeros_like(x), np.zeros(Tn, np.float32)
    orc.orc_rmsnorm_fwd(x, w, ry, rr, Tn, D, 1e-6)
    y, r = hip.rmsnorm_forward(T(x, dev), T(w, dev), 1e-6)
    assert rel_err(H(y), ry) <= FP32_TOL and rel_err(H(r), rr) <= FP32_TOL


def test_layernorm(orc, dev):
    rng = np.random.default_rng(31)
    Tn, D = 333, 256
    x, dY = f32(rng.standard_normal((Tn, D))), f32(rng.standard_normal((Tn, D)))
    w = f32(1 + 0.1 * rng.standard_normal(D))
    rdw, rdb, rdx = np.zeros(D, np.float32), np.zeros(D, np.float32), np.zeros_like(x)
    orc.orc_grad_layernorm(dY, x, w, rdw, rdb, rdx, Tn, D, 1e-5)
    pw, pb = hip.Parameter("w", T(w, dev)), hip.Parameter("b", torch.zeros(D, device=dev))
    dx = hip.GradientMapping().LayerNorm(T(dY, dev), T(x, dev), pw, pb, 1e-5)
    assert rel_err(H(dx), rdx) <= FP32_TOL
    assert rel_err(H(pw.Grad), rdw) <= FP32_TOL and rel_err(H(pb.Grad), rdb) <= FP32_TOL


# ------------------------------------------------------------------ attention
@pytest.mark.parametrize("S,D", [(2, 3), (128, 64), (200, 128)])
def test_attention_slot(orc, dev, S, D):
    rng = np.random.default_rng(S + D)
    q, k, v, dO = (f32(rng.standard_normal((S, D))) for _ in range(4))
    probs = np.zeros((1, 1, S, S), np.float32)
    out = np.zeros((1, S, D), np.float32)
    orc.orc_attention_fwd(q, k, v, probs, out, 1, S, 1, 1, D)
    P = probs[0, 0].copy()
    scale = float(1 / np.sqrt(D))
    rq, rk, rv = (np.zeros((S, D), np.float32) for _ in range(3))
    orc.orc_grad_attention(dO, q, k, v, P, rq, rk, rv, S, D, scale)
    g = hip.GradientMapping().Attention(T(dO, dev), T(q, dev), T(k, dev), T(v, dev), T(P, dev), scale)
    assert rel_err(H(g.DQ), rq) <= FP32_TOL
    assert rel_err(H(g.DK), rk) <= FP32_TOL
    assert rel_err(H(g.DV), rv) <= FP32_TOL


def test_attention_forward_probs(orc, dev):
    rng = np.random.default_rng(40)
    B, S, Hq, Hkv, D = 2, 64, 4, 2, 64
    q, k, v = f32(rng.standard_normal((B, S, Hq, D))), f32(rng.standard_normal((B, S, Hkv, D))), f32(rng.standard_normal((B, S, Hkv, D)))
    rp, ro = np.zeros((B, Hq, S, S), np.float32), np.zeros((B, S, Hq * D), np.float32)
    orc.orc_attention_fwd(q, k, v, rp, ro, B, S, Hq, Hkv, D)
    p, o = hip.attention_forward_probs(T(q, dev), T(k, dev), T(v, dev))
    assert rel_err(H(p), rp) <= FP32_TOL and rel_err(H(o), ro) <= FP32_TOL


# ------------------------------------------------------------------ embedding / activations
def test_embedding_bitexact(orc, dev):
    rng = np.random.default_rng(50)
    Tn, D, V = 4096, 256, 512
    dY = f32(rng.standard_normal((Tn, D)))
    ids = rng.integers(0, V, Tn).astype(np.int32)
    E0 = f32(rng.standard_normal((V, D)))
    rE = E0.copy()
    orc.orc_grad_embedding(dY, ids, rE, Tn, D)
    p = hip.Parameter("embedding.weight", torch.zeros(V, D, device=dev))
    p.Grad.copy_(T(E0, dev))
    hip.GradientMapping().Embedding(T(dY, dev), T(ids, dev), p)
    assert _bits_equal(H(p.Grad), rE)


def test_embedding_kat(dev):
    p = hip.Parameter("embedding.weight", torch.zeros(5, 3, device=dev))
    hip.GradientMapping().Embedding(torch.ones(2, 3, device=dev), torch.tensor([1, 3], dtype=torch.int32, device=dev), p)
    g = H(p.Grad)
    assert g[1, 0] == 1 and g[0, 0] == 0 and g[3, 2] == 1


@pytest.mark.parametrize("fn", ["silu", "gelu"])
def test_activation_backward(orc, dev, fn):
    rng = np.random.default_rng(51)
    n = 100003
    x, dy = f32(rng.standard_normal(n) * 3), f32(rng.standard_normal(n))
    ref = np.zeros(n, np.float32)
    getattr(orc, f"orc_grad_{fn}")(dy, x, ref, n)
    gm = hip.GradientMapping()
    out = (gm.ActivationSiLU if fn == "silu" else gm.ActivationGELU)(T(dy, dev), T(x, dev))
    assert rel_err(H(out), ref) <= FP32_TOL


@pytest.mark.parametrize("Tn,F", [(8192, 3072), (512, 3072), (33, 1001)])
def test_swiglu(orc, dev, Tn, F):
    rng = np.random.default_rng(Tn + F)
    g, u, da = (f32(rng.standard_normal((Tn, F))) for _ in range(3))
    ref = np.zeros((Tn, 2 * F), np.float32)
    orc.orc_grad_swiglu(da, g, u, ref, Tn, F)
    out = hip.swiglu_backward(T(da, dev), T(g, dev), T(u, dev))
    assert rel_err(H(out), ref) <= FP32_TOL
    ra = np.zeros(Tn * F, np.float32)
    orc.orc_swiglu_fwd(g.ravel(), u.ravel(), ra, Tn * F)
    assert rel_err(H(hip.swiglu_forward(T(g, dev), T(u, dev))).ravel(), ra) <= FP32_TOL


@pytest.mark.parametrize("neox,theta,D", [(0, 1e4, 64), (1, 1e6, 128)])
def test_rope(orc, dev, neox, theta, D):
    rng = np.random.default_rng(D)
    B, S, Hh = 2, 300, 3
    c, s = hip.rope_tables(theta, D, S)
    x = f32(rng.standard_normal((B, S, Hh, D)))
    rf, rb = x.copy(), x.copy()
    for b in range(B):
        orc.orc_rope_fwd(rf[b], c, s, S, Hh, D, neox)
        orc.orc_rope_bwd(rb[b], c, s, S, Hh, D, neox)
    tf, tb = T(x, dev), T(x, dev)
    hip.rope_forward(tf, T(c, dev), T(s, dev), neox)
    hip.rope_backward(tb, T(c, dev), T(s, dev), neox)
    assert rel_err(H(tf), rf) <= FP32_TOL and rel_err(H(tb), rb) <= FP32_TOL


# ------------------------------------------------------------------ loss
@pytest.mark.parametrize("Tn,V,sm", [(8192, 32000, 0.0), (256, 32000, 0.0), (64, 32000, 0.1), (8, 151936, 0.0), (40, 513, 0.0), (16, 1000, 0.2)])
def test_cross_entropy(orc, dev, Tn, V, sm):
    rng = np.random.default_rng(Tn + V)
    z = f32(rng.standard_normal((Tn, V)) * 2)
    lab = rng.integers(0, V, Tn).astype(np.int32)
    lab[::7] = -100
    ref = np.zeros_like(z)
    orc.orc_ce_softmax_grad(z, lab, ref, Tn, V, -100, sm)
    rloss = orc.orc_ce_loss(z, lab, Tn, V, -100, sm)
    d, loss = hip.cross_entropy_softmax(T(z, dev), T(lab, dev), -100, sm)
    assert rel_err(H(d), ref) <= FP32_TOL
    assert abs(float(H(loss)[0]) - rloss) <= FP32_TOL * abs(rloss)


@pytest.mark.parametrize("Tn,V", [(64, 512), (32, 32000), (4, 151936)])
def test_cross_entropy_in_place(orc, dev, Tn, V):
    """dLogits written over the logits buffer (the fp32 engine does this): loss must use the original row."""
    rng = np.random.default_rng(V)
    z = f32(rng.standard_normal((Tn, V)) * 2)
    lab = rng.integers(0, V, Tn).astype(np.int32)
    lab[1] = -100
    ref = np.zeros_like(z)
    orc.orc_ce_softmax_grad(z, lab, ref, Tn, V, -100, 0.0)
    rloss = orc.orc_ce_loss(z, lab, Tn, V, -100, 0.0)
    tz = T(z, dev)
    d, loss = hip.cross_entropy_softmax(tz, T(lab, dev), -100, 0.0, out=tz)
    assert rel_err(H(tz), ref) <= FP32_TOL
    assert abs(float(H(loss)[0]) - rloss) <= FP32_TOL * abs(rloss)


# ------------------------------------------------------------------ TrainingOps
@pytest.mark.parametrize("n", [100_000_000, 1_000_003, 7])
def test_adamw_bitexact(orc, dev, n):
    rng = np.random.default_rng(60)
    d, g = f32(rng.standard_normal(n) * 0.02), f32(rng.standard_normal(n) * 0.02)
    m, v = f32(rng.standard_normal(n) * 0.01), f32(np.abs(rng.standard_normal(n)) * 1e-4)
    args = (0.9, 0.95, 1 - 0.9 ** 3, 1 - 0.95 ** 3, 1e-3, 1e-8, 0.1)
    rd, rm, rv = d.copy(), m.copy(), v.copy()
    orc.orc_adamw(rd, g, rm, rv, n, *args)
    td, tm, tv = T(d, dev), T(m, dev), T(v, dev)
    hip.TrainingOps().AdamWUpdate(td, T(g, dev), tm, tv, *args)
    assert _bits_equal(H(td), rd) and _bits_equal(H(tm), rm) and _bits_equal(H(tv), rv)


def test_l2normsq(dev):
    rng = np.random.default_rng(61)
    x = f32(rng.standard_normal(3_000_017))
    ref = float((x.astype(np.float64) ** 2).sum())
    out = float(H(hip.TrainingOps().L2NormSq(T(x, dev)))[0])
    assert abs(out - ref) <= 1e-6 * ref
