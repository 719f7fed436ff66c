"""Float64 numpy forward of the decoder, written independently of oracle/engine.c.

Used only to pin the oracle engine: its loss must agree with the oracle's, and
central differences of this loss must agree with the oracle's gradients.
"""
import numpy as np


def rope(x, theta, neox):
    """x [B,S,H,D] rotated at positions 0..S-1 (RoPE.cs:168-259 conventions)."""
    B, S, H, D = x.shape
    half = D // 2
    freqs = 1.0 / theta ** (2.0 * np.arange(half) / D)
    ang = np.arange(S)[:, None] * freqs[None, :]
    c, s = np.cos(ang)[None, :, None, :], np.sin(ang)[None, :, None, :]
    if neox:
        a, b = x[..., :half], x[..., half:]
        return np.concatenate([a * c - b * s, b * c + a * s], -1)
    a, b = x[..., 0::2], x[..., 1::2]
    out = np.empty_like(x)
    out[..., 0::2] = a * c - b * s
    out[..., 1::2] = b * c + a * s
    return out


def rms(x, w, eps):
    return x / np.sqrt((x ** 2).mean(-1, keepdims=True) + eps) * w


def loss(cfg, P, ids, labels):
    g = lambda k: P.get(k)
    B, S, d, Hq, Hkv, D, F = cfg.B, cfg.S, cfg.d, cfg.Hq, cfg.Hkv, cfg.D, cfg.F
    qd, kvd = Hq * D, Hkv * D
    s_l = cfg.lora_alpha / cfg.lora_rank if cfg.lora_rank else 0.0

    def lin(x, W, b, lora):
        y = x @ W.T
        if b is not None:
            y = y + b
        for (A, Bm, sl) in lora:
            if A is not None:
                y[:, sl] += s_l * (x @ A) @ Bm
        return y

    h = P["emb"][ids]
    for l in range(cfg.L):
        p = f"l{l}."
        xn = rms(h, P[p + "norm1"], cfg.eps)
        qkv = lin(xn, P[p + "wqkv"], g(p + "bqkv"), [
            (g(p + "lora.q.A"), g(p + "lora.q.B"), slice(0, qd)),
            (g(p + "lora.k.A"), g(p + "lora.k.B"), slice(qd, qd + kvd)),
            (g(p + "lora.v.A"), g(p + "lora.v.B"), slice(qd + kvd, qd + 2 * kvd))])
        q = qkv[:, :qd].reshape(B, S, Hq, D)
        k = qkv[:, qd:qd + kvd].reshape(B, S, Hkv, D)
        v = qkv[:, qd + kvd:].reshape(B, S, Hkv, D)
        if cfg.qk_norm:
            q = rms(q, P[p + "q_norm"], cfg.eps)
            k = rms(k, P[p + "k_norm"], cfg.eps)
        q, k = rope(q, cfg.theta, cfg.neox), rope(k, cfg.theta, cfg.neox)
        grp = Hq // Hkv
        o = np.zeros((B, S, Hq, D))
        mask = np.triu(np.ones((S, S), bool), 1)
        for b in range(B):
            for hh in range(Hq):
                sc = q[b, :, hh] @ k[b, :, hh // grp].T / np.sqrt(D)
                sc = np.where(mask, -np.inf, sc)
                e = np.exp(sc - sc.max(1, keepdims=True))
                o[b, :, hh] = (e / e.sum(1, keepdims=True)) @ v[b, :, hh // grp]
        o = o.reshape(B * S, qd)
        h = h + lin(o, P[p + "wo"], g(p + "bo"), [(g(p + "lora.o.A"), g(p + "lora.o.B"), slice(0, d))])
        xn2 = rms(h, P[p + "norm2"], cfg.eps)
        gu = lin(xn2, P[p + "wgu"], g(p + "bgu"), [(g(p + "lora.gate.A"), g(p + "lora.gate.B"), slice(0, F)),
                                                   (g(p + "lora.up.A"), g(p + "lora.up.B"), slice(F, 2 * F))])
        gt, up = gu[:, :F], gu[:, F:]
        act = gt / (1 + np.exp(-gt)) * up
        h = h + lin(act, P[p + "wd"], g(p + "bd"), [(g(p + "lora.down.A"), g(p + "lora.down.B"), slice(0, d))])
    xf = rms(h, P["norm_f"], cfg.eps)
    z = xf @ P["emb"].T
    m = labels != -100
    zz = z[m]
    lse = np.log(np.exp(zz - zz.max(1, keepdims=True)).sum(1)) + zz.max(1)
    return float((lse - zz[np.arange(zz.shape[0]), labels[m]]).mean())
