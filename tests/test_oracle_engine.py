"""Pins the oracle's whole-step restatement (oracle/engine.c) with float64 finite differences.

Recipe after BackpropEngineTests.cs:57-93 (central differences on sampled
elements of every parameter), but run in float64 on an independent numpy
forward (tests/npmodel.py), so the tolerance can be 1e-3 relative instead of
the reference's 2e-2*(1+|fd|).
"""
import numpy as np
import pytest

import oracle
from npmodel import loss as np_loss


def make(neox, qk_norm, lora, bias, seed=0):
    cfg = oracle.EngineCfg(L=2, d=32, Hq=4, Hkv=2, D=8, F=24, V=40, B=2, S=6, eps=1e-6, theta=1e4 if not neox else 1e6,
                           neox=neox, qk_norm=qk_norm, lora_rank=4 if lora else 0, lora_alpha=8.0 if lora else 0.0)
    rng = np.random.default_rng(seed)
    qd, kvd = cfg.Hq * cfg.D, cfg.Hkv * cfg.D
    P = {"emb": rng.standard_normal((cfg.V, cfg.d)) * 0.3, "norm_f": 1 + 0.1 * rng.standard_normal(cfg.d)}
    for l in range(cfg.L):
        p = f"l{l}."
        P[p + "norm1"] = 1 + 0.1 * rng.standard_normal(cfg.d)
        P[p + "norm2"] = 1 + 0.1 * rng.standard_normal(cfg.d)
        P[p + "wqkv"] = rng.standard_normal((qd + 2 * kvd, cfg.d)) * 0.3
        P[p + "wo"] = rng.standard_normal((cfg.d, qd)) * 0.3
        P[p + "wgu"] = rng.standard_normal((2 * cfg.F, cfg.d)) * 0.3
        P[p + "wd"] = rng.standard_normal((cfg.d, cfg.F)) * 0.3
        if qk_norm:
            P[p + "q_norm"] = 1 + 0.1 * rng.standard_normal(cfg.D)
            P[p + "k_norm"] = 1 + 0.1 * rng.standard_normal(cfg.D)
        if bias:
            for k, n in (("bqkv", qd + 2 * kvd), ("bo", cfg.d), ("bgu", 2 * cfg.F), ("bd", cfg.d)):
                P[p + k] = rng.standard_normal(n) * 0.1
        if lora:
            geo = {"q": (cfg.d, qd), "k": (cfg.d, kvd), "v": (cfg.d, kvd), "o": (qd, cfg.d),
                   "gate": (cfg.d, cfg.F), "up": (cfg.d, cfg.F), "down": (cfg.F, cfg.d)}
            for t, (In, Out) in geo.items():
                P[p + f"lora.{t}.A"] = rng.standard_normal((In, 4)) * 0.3
                P[p + f"lora.{t}.B"] = rng.standard_normal((4, Out)) * 0.3
    ids = rng.integers(0, cfg.V, cfg.B * cfg.S).astype(np.int32)
    lab = np.roll(ids, -1).astype(np.int32)
    lab[cfg.S - 1::cfg.S] = -100
    return cfg, P, ids, lab


@pytest.mark.parametrize("neox,qk_norm,lora,bias", [(0, 0, 0, 1), (1, 1, 0, 0), (1, 1, 1, 0)])
def test_engine_grads_match_float64_fd(neox, qk_norm, lora, bias):
    cfg, P64, ids, lab = make(neox, qk_norm, lora, bias)
    P32 = {k: np.ascontiguousarray(v, np.float32) for k, v in P64.items()}
    P64 = {k: v.astype(np.float32).astype(np.float64) for k, v in P64.items()}
    train = [k for k in P32 if ".lora." in k] if lora else list(P32)
    G = {k: np.zeros_like(P32[k]) for k in train}
    L32 = oracle.engine_step(cfg, P32, G, ids, lab)
    L64 = np_loss(cfg, P64, ids, lab)
    assert abs(L32 - L64) < 1e-5 * abs(L64)
    rng = np.random.default_rng(1)
    for k in train:
        flat = P64[k].ravel()
        idx = rng.choice(flat.size, size=min(12, flat.size), replace=False)
        num = []
        for i in idx:
            old = flat[i]
            flat[i] = old + 1e-5
            lp = np_loss(cfg, P64, ids, lab)
            flat[i] = old - 1e-5
            lm = np_loss(cfg, P64, ids, lab)
            flat[i] = old
            num.append((lp - lm) / 2e-5)
        num = np.array(num)
        got = G[k].ravel()[idx]
        scale = max(np.abs(num).max(), 1e-3)
        assert np.abs(got - num).max() <= 1e-3 * scale, (k, got, num)
