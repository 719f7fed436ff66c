"""The host-pointer slot entries (smhip_host_*), the surface the C# plugin P/Invokes.

Each entry is called through ctypes with plain host arrays, as the SharpMind.HIP shim
would call it, and compared with the pinned CPU oracle at the fp32 bar (norm-wise
relative error <= 1e-5; AdamW bit-exact).  The reference calls its Attention slot
concurrently from Parallel.For bodies (BackpropEngine.cs:563-582), so one test runs
smhip_host_grad_attention from several Python threads at once (ctypes releases the
GIL during the call) and checks every result; another grows a thread's buffers
between calls and checks the results stay right.
"""
import ctypes
import threading

import numpy as np
import pytest

import sharpmind_amd
from sharpmind_amd import check

from conftest import rel_err

pytestmark = pytest.mark.gpu
TOL = 1e-5


def P(a):
    return a.ctypes.data_as(ctypes.c_void_p)


@pytest.fixture(scope="module")
def L(dev):
    return sharpmind_amd.lib()


def _attn_case(orc, rng, S, D):
    q, k, v, dO = (rng.standard_normal((S, D)).astype(np.float32) for _ in range(4))
    probs = np.zeros((1, 1, S, S), np.float32)
    out = np.zeros((S, D), np.float32)
    orc.orc_attention_fwd(q, k, v, probs, out, 1, S, 1, 1, D)
    ref = [np.zeros((S, D), np.float32) for _ in range(3)]
    orc.orc_grad_attention(dO, q, k, v, probs, *ref, S, D, np.float32(1 / np.sqrt(D)))
    return (dO, q, k, v, probs), ref


def _host_attention(L, ins, S, D):
    outs = [np.full((S, D), np.nan, np.float32) for _ in range(3)]
    check(L.smhip_host_grad_attention(*map(P, ins), *map(P, outs), S, D, ctypes.c_float(1 / np.sqrt(D))))
    return outs


def test_host_grad_linear(orc, L):
    rng = np.random.default_rng(1)
    M, In, Out = 77, 96, 130
    dY, X = rng.standard_normal((M, Out)).astype(np.float32), rng.standard_normal((M, In)).astype(np.float32)
    W = rng.standard_normal((Out, In)).astype(np.float32)
    dW0, db0 = rng.standard_normal((Out, In)).astype(np.float32), rng.standard_normal(Out).astype(np.float32)
    dW, db, dX = dW0.copy(), db0.copy(), np.zeros((M, In), np.float32)
    check(L.smhip_host_grad_linear(P(dY), P(X), P(W), P(dW), P(db), P(dX), M, In, Out, 0))
    rdW, rdb, rdX = dW0.copy(), db0.copy(), np.zeros((M, In), np.float32)
    orc.orc_grad_linear(dY, X, W, rdW, rdb.ctypes.data, rdX, M, In, Out)
    assert rel_err(dX, rdX) <= TOL and rel_err(dW, rdW) <= TOL and rel_err(db, rdb) <= TOL


def test_host_grad_rmsnorm_layernorm(orc, L):
    rng = np.random.default_rng(2)
    T, D = 64, 320
    dY, x = rng.standard_normal((T, D)).astype(np.float32), rng.standard_normal((T, D)).astype(np.float32)
    w = (1 + 0.1 * rng.standard_normal(D)).astype(np.float32)
    y, rinv = np.zeros_like(x), np.zeros(T, np.float32)
    orc.orc_rmsnorm_fwd(x, w, y, rinv, T, D, 1e-6)
    xn = (x * rinv[:, None]).astype(np.float32)
    dw, dX = np.ones(D, np.float32), np.zeros_like(x)
    check(L.smhip_host_grad_rmsnorm(P(dY), P(xn), P(rinv), P(w), P(dw), P(dX), T, D))
    rdw, rdX = np.ones(D, np.float32), np.zeros_like(x)
    orc.orc_grad_rmsnorm(dY, xn, rinv, w, rdw, rdX, T, D)
    assert rel_err(dX, rdX) <= TOL and rel_err(dw, rdw) <= TOL
    dw, db, dX = np.zeros(D, np.float32), np.zeros(D, np.float32), np.zeros_like(x)
    check(L.smhip_host_grad_layernorm(P(dY), P(x), P(w), P(dw), P(db), P(dX), T, D, ctypes.c_float(1e-5)))
    rdw, rdb, rdX = np.zeros(D, np.float32), np.zeros(D, np.float32), np.zeros_like(x)
    orc.orc_grad_layernorm(dY, x, w, rdw, rdb, rdX, T, D, 1e-5)
    assert rel_err(dX, rdX) <= TOL and rel_err(dw, rdw) <= TOL and rel_err(db, rdb) <= TOL


def test_host_grad_embedding_silu_gelu(orc, L):
    rng = np.random.default_rng(3)
    T, D, V = 200, 64, 50
    dY = rng.standard_normal((T, D)).astype(np.float32)
    ids = rng.integers(0, V, T).astype(np.int32)
    dE, rdE = np.ones((V, D), np.float32), np.ones((V, D), np.float32)
    check(L.smhip_host_grad_embedding(P(dY), P(ids), P(dE), T, D, V))
    orc.orc_grad_embedding(dY, ids, rdE, T, D)
    assert np.array_equal(dE, rdE)
    n = 10007
    g, x = rng.standard_normal(n).astype(np.float32), (3 * rng.standard_normal(n)).astype(np.float32)
    for name in ("silu", "gelu"):
        out, ref = np.zeros(n, np.float32), np.zeros(n, np.float32)
        check(getattr(L, f"smhip_host_grad_{name}")(P(g), P(x), P(out), n))
        getattr(orc, f"orc_grad_{name}")(g, x, ref, n)
        assert rel_err(out, ref) <= TOL, name


def test_host_adamw_l2normsq(orc, L):
    rng = np.random.default_rng(4)
    n = 100003
    data = (0.02 * rng.standard_normal(n)).astype(np.float32)
    grad = (0.01 * rng.standard_normal(n)).astype(np.float32)
    m = (0.001 * rng.standard_normal(n)).astype(np.float32)
    v = np.abs(0.0001 * rng.standard_normal(n)).astype(np.float32)
    args = [ctypes.c_float(a) for a in (0.9, 0.95, 0.271, 0.143, 1e-3, 1e-8, 0.1)]
    d2, m2, v2 = data.copy(), m.copy(), v.copy()
    check(L.smhip_host_adamw_update(P(d2), P(grad), P(m2), P(v2), n, *args))
    orc.orc_adamw(data, grad, m, v, n, 0.9, 0.95, 0.271, 0.143, 1e-3, 1e-8, 0.1)
    assert np.array_equal(d2, data) and np.array_equal(m2, m) and np.array_equal(v2, v)
    out = np.zeros(1, np.float32)
    check(L.smhip_host_l2normsq(P(grad), n, P(out)))
    assert abs(out[0] - np.sum(grad.astype(np.float64) ** 2)) <= 1e-6 * out[0]


@pytest.mark.parametrize("qtype", [0, 8, 12])
def test_host_qmatmul(orc, L, qtype):
    rng = np.random.default_rng(5 + qtype)
    M, K, N = 33, 512, 96
    x = rng.standard_normal((M, K)).astype(np.float32)
    W = (0.05 * rng.standard_normal((N, K))).astype(np.float32)
    if qtype == 8:
        raw = np.zeros(N * K // 32 * 34, np.uint8)
        orc.orc_quantize_q8_0(W.ravel(), W.size, raw)
    elif qtype == 12:
        raw = np.zeros(N * K // 256 * 144, np.uint8)
        orc.orc_quantize_q4k(W.ravel(), W.size, raw)
    else:
        raw = W.view(np.uint8).ravel()
    out, ref = np.zeros((M, N), np.float32), np.zeros((M, N), np.float32)
    check(L.smhip_host_qmatmul(qtype, P(x), P(raw), P(out), M, K, N))
    {0: orc.orc_qmatmul_f32, 8: orc.orc_qmatmul_q8_0, 12: orc.orc_qmatmul_q4k}[qtype](
        x, raw if qtype else W, ref, M, K, N)
    assert rel_err(out, ref) <= TOL


def test_host_attention_grows_buffers(orc, L):
    """A thread's reused device buffers grow when a larger call follows a smaller one."""
    rng = np.random.default_rng(6)
    for S, D in ((32, 16), (160, 64), (48, 32)):
        ins, ref = _attn_case(orc, rng, S, D)
        got = _host_attention(L, ins, S, D)
        for g, r in zip(got, ref):
            assert rel_err(g, r) <= TOL, (S, D)


def test_host_attention_concurrent_threads(orc, L):
    """Four threads call the Attention slot at once, as Parallel.For does (BackpropEngine.cs:563-582):
    each gets its own case's gradients (a shared dP or split-K buffer would mix them up)."""
    rng = np.random.default_rng(7)
    S, D, nthr, reps = 256, 64, 4, 6
    cases = [_attn_case(orc, rng, S, D) for _ in range(nthr)]
    errs, fails = {}, []
    start = threading.Barrier(nthr)

    def work(i):
        try:
            start.wait()
            worst = 0.0
            for _ in range(reps):
                got = _host_attention(L, cases[i][0], S, D)
                worst = max(worst, max(rel_err(g, r) for g, r in zip(got, cases[i][1])))
            errs[i] = worst
        except Exception as ex:  # reported below
            fails.append((i, repr(ex)))

    ths = [threading.Thread(target=work, args=(i,)) for i in range(nthr)]
    for t in ths:
        t.start()
    for t in ths:
        t.join(timeout=120)
    assert not fails, fails
    assert len(errs) == nthr and max(errs.values()) <= TOL, errs
