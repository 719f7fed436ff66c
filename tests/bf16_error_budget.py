"""Where the bf16 whole-step gradient error comes from: the decoder of the engine tests in
float64 torch, with bf16 rounding (straight-through in backward) switched on at chosen points
of the forward, one at a time or all together.  Used by tests/test_bf16_error_budget.py and
runnable on its own (python tests/bf16_error_budget.py) for the full table."""
import math

import torch

F64 = torch.float64


class RND(torch.autograd.Function):  # round the value to bf16, pass the gradient through
    @staticmethod
    def forward(ctx, x): return x.to(torch.bfloat16).to(torch.float64)
    @staticmethod
    def backward(ctx, g): return g
class GRND(torch.autograd.Function):  # round the gradient flowing back
    @staticmethod
    def forward(ctx, x): return x.clone()
    @staticmethod
    def backward(ctx, g): return g.to(torch.bfloat16).to(torch.float64)
L, d, Hq, Hkv, D, F, V, B, S = 2, 256, 4, 2, 64, 512, 512, 2, 128
r, alpha = 8, 16.0
def run(active, init, seed=7):
    """Adapter gradients of one step with bf16 rounding at the forward points named in active."""
    R = lambda x, tag: RND.apply(x) if tag in active else x
    G = lambda x, tag: GRND.apply(x) if tag in active else x
    g = torch.Generator().manual_seed(seed)
    sd = 0.05 if init == "wide" else 0.02
    def W(*sh, std=sd): return torch.randn(*sh, generator=g, dtype=F64) * std
    P = {"emb": W(V, d)}
    for l in range(L):
        P[f"{l}.wqkv"] = W(Hq * D + 2 * Hkv * D, d); P[f"{l}.wo"] = W(d, Hq * D); P[f"{l}.wgu"] = W(2 * F, d); P[f"{l}.wd"] = W(d, F)
        for n in ["norm1", "norm2"]: P[f"{l}.{n}"] = 1 + 0.1 * torch.randn(d, generator=g, dtype=F64)
        P[f"{l}.qn"] = 1 + 0.1 * torch.randn(D, generator=g, dtype=F64); P[f"{l}.kn"] = 1 + 0.1 * torch.randn(D, generator=g, dtype=F64)
        for t, (In, Out) in {"qkv": (d, Hq * D + 2 * Hkv * D), "o": (Hq * D, d), "gu": (d, 2 * F), "d": (F, d)}.items():
            if init == "wide":
                P[f"{l}.{t}.A"] = W(In, r); P[f"{l}.{t}.B"] = W(r, Out)
            else:
                P[f"{l}.{t}.A"] = (torch.rand(In, r, generator=g, dtype=F64) * 2 - 1) / math.sqrt(In); P[f"{l}.{t}.B"] = W(r, Out, std=1e-3)
    P["normf"] = 1 + 0.1 * torch.randn(d, generator=g, dtype=F64)
    ids = torch.randint(0, V, (B * S,), generator=g)
    lab = torch.cat([ids.view(B, S)[:, 1:], torch.full((B, 1), -100)], 1).view(-1)
    for k in P: P[k].requires_grad_(k.endswith(".A") or k.endswith(".B"))
    def rms(x, w): return x / torch.sqrt((x * x).mean(-1, keepdim=True) + 1e-6) * w
    def lin(x, l, t, Wt):
        y = R(x, "act") @ R(Wt, "w").T
        u = R(R(x, "act") @ R(P[f"{l}.{t}.A"], "w"), "u")
        return y + (alpha / r) * (u @ R(P[f"{l}.{t}.B"], "w"))
    half = D // 2
    freqs = 1.0 / 1e6 ** (2.0 * torch.arange(half, dtype=F64) / D)
    ang = torch.arange(S, dtype=F64)[:, None] * freqs[None]
    c, s_ = torch.cos(ang)[None, :, None], torch.sin(ang)[None, :, None]
    def rope(x):
        a, b_ = x[..., :half], x[..., half:]
        return torch.cat([a * c - b_ * s_, b_ * c + a * s_], -1)
    h = P["emb"][ids]
    mask = torch.triu(torch.ones(S, S, dtype=torch.bool), 1)
    for l in range(L):
        xn = rms(h, P[f"{l}.norm1"])
        qkv = R(lin(xn, l, "qkv", P[f"{l}.wqkv"]), "qkvout")
        q = qkv[:, :Hq * D].view(B, S, Hq, D); k = qkv[:, Hq * D:Hq * D + Hkv * D].view(B, S, Hkv, D); v = qkv[:, Hq * D + Hkv * D:].view(B, S, Hkv, D)
        q = rope(rms(q, P[f"{l}.qn"])); k = rope(rms(k, P[f"{l}.kn"]))
        q, k, v = R(q, "qk"), R(k, "qk"), R(v, "v")
        grp = Hq // Hkv
        kk = k.repeat_interleave(grp, 2); vv = v.repeat_interleave(grp, 2)
        sc = torch.einsum("bqhd,bkhd->bhqk", q, kk) / math.sqrt(D)
        sc = sc.masked_fill(mask, -math.inf)
        p = torch.softmax(sc, -1)
        p = R(p, "p")
        o = torch.einsum("bhqk,bkhd->bqhd", p, vv).reshape(B * S, Hq * D)
        o = G(o, "do")
        h = h + lin(R(o, "o"), l, "o", P[f"{l}.wo"])
        xn2 = rms(h, P[f"{l}.norm2"])
        gu = R(lin(xn2, l, "gu", P[f"{l}.wgu"]), "gu")
        a = gu[:, :F] * torch.sigmoid(gu[:, :F]) * gu[:, F:]
        h = h + lin(R(a, "act2"), l, "d", P[f"{l}.wd"])
    z = rms(h, P["normf"]) @ P["emb"].T
    loss = torch.nn.functional.cross_entropy(z, lab, ignore_index=-100)
    grads = torch.autograd.grad(loss, [P[k] for k in P if P[k].requires_grad])
    return {k: gr for k, gr in zip([k for k in P if P[k].requires_grad], grads)}
TAGS = ["act", "w", "u", "qkvout", "qk", "v", "p", "o", "gu", "act2", "do"]


def worst_errors(active, init, ref=None, k=3):
    """Norm-wise relative error of every adapter gradient against the unrounded run; the k worst."""
    ref = ref if ref is not None else run(set(), init)
    gr = run(active, init)
    e = {n: float((gr[n] - ref[n]).norm() / ref[n].norm()) for n in ref}
    return sorted(e.items(), key=lambda kv: -kv[1])[:k]


if __name__ == "__main__":
    for init in ["wide", "config"]:
        ref = run(set(), init)
        print(init, "all", worst_errors(set(TAGS), init, ref), flush=True)
        for t in TAGS:
            print(init, "only", t, worst_errors({t}, init, ref), flush=True)
        for t in ["qk", "p", "act", "w"]:
            print(init, "all but", t, worst_errors(set(TAGS) - {t}, init, ref), flush=True)
