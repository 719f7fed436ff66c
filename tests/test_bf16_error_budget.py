"""The bf16 whole-step error is a sum of many roundings, not one (CPU, float64 torch emulation).

Rounding the weights, activations, q|k|v projection, rotated q/k, v, probabilities, attention
output, gate|up and the SwiGLU output to bf16 in the forward (what the MFMA operands require)
gives the adapter gradients a worst relative error near 2e-2 at large weights (N(0, 0.05));
leaving q/k unrounded before QK^T (the hi/lo-split remedy) barely moves it, and no single
rounding point accounts for more than about two thirds of it."""
import pytest

torch = pytest.importorskip("torch")
import bf16_error_budget as B


def test_error_budget_is_spread_over_roundings():
    init = "wide"
    ref = B.run(set(), init)
    worst_all = B.worst_errors(set(B.TAGS), init, ref)[0][1]
    worst_no_qk = B.worst_errors(set(B.TAGS) - {"qk"}, init, ref)[0][1]
    worst_w = B.worst_errors({"w"}, init, ref)[0][1]
    worst_qk = B.worst_errors({"qk"}, init, ref)[0][1]
    assert 5e-3 < worst_all < 3e-2, worst_all
    assert worst_no_qk > 0.85 * worst_all, (worst_no_qk, worst_all)  # q/k rounding is a small share
    assert worst_qk < 0.5 * worst_all, (worst_qk, worst_all)
    assert worst_w < 0.75 * worst_all, (worst_w, worst_all)             # not one dominant point
