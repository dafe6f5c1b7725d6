"""Pins the oracle's math-path pieces (softmax, its gradient, bmm, the composed math path)
before they check the GPU's composed path.

  * softmax_lastdim (src/torch_softmax.rs:57-67) against float64 softmax (an error bound in
    ulp), exactly on rows of equal values (every weight 1/W), and bit-invariant under an exact
    shift of the row (it subtracts the row max); NaN and +inf rows;
  * softmax_backward_lastdim (src/torch_softmax.rs:90-97) against the float64 Jacobian product
    (diag(y) - y y^T) g;
  * bmm (src/torch_blas.rs:404-449, 95-134) exactly on small integers (any summation order is
    exact there, so a wrong index or transpose fails) and against float64 on random inputs;
  * the composed math path (python/densecore/functional.py:318-340) against the float64 brute
    force and torch.autograd in float64: rank 3 and 4, Ev != E, causal, float and bool masks with
    fully masked rows (out 0, zero gradients), and the gradient of a float mask.
"""
import math

import numpy as np
import pytest

import oracle
from oracle import brute
from tests._data import assert_f32

RNG = np.random.default_rng(77)


def test_softmax_against_float64():
    for width in (1, 3, 4, 5, 8, 37, 64, 513):
        x = (RNG.standard_normal((9, width)) * 4).astype(np.float32)
        y = oracle.softmax(x)
        x64 = x.astype(np.float64)
        e = np.exp(x64 - x64.max(-1, keepdims=True))
        ref = e / e.sum(-1, keepdims=True)
        ulp = np.spacing(ref.astype(np.float32)).astype(np.float64)
        # 1-ulp expf and the reciprocal; the rounding of x - max, relative to |x - max| and
        # amplified by exp into that many ulps; the sum's rounding, at most one per addition
        # along a lane of the 4-lane tree (width / 4 of them).
        bound = 4.0 + np.abs(x64 - x64.max(-1, keepdims=True)) + width / 4
        assert (np.abs(y - ref) / ulp <= bound).all(), width


def test_softmax_equal_rows_and_shift():
    for width in (1, 2, 7, 64, 1000):
        y = oracle.softmax(np.full((2, width), 3.25, np.float32))
        assert np.array_equal(y, np.full((2, width), np.float32(1) / np.float32(width)))
    x = RNG.integers(-20, 1, size=(5, 33)).astype(np.float32)
    assert np.array_equal(oracle.softmax(x), oracle.softmax(x + np.float32(64)))


def test_softmax_special_rows():
    y = oracle.softmax(np.array([[0.0, np.nan, 1.0], [np.inf, 0.0, 1.0], [0.0, -np.inf, 0.0]],
                                np.float32))
    assert np.isnan(y[0]).all() and np.isnan(y[1]).all()
    assert np.array_equal(y[2], np.array([0.5, 0.0, 0.5], np.float32))


def test_softmax_backward_against_jacobian():
    for width in (1, 3, 4, 9, 130):
        y = oracle.softmax(RNG.standard_normal((6, width)).astype(np.float32))
        g = RNG.standard_normal((6, width)).astype(np.float32)
        dx = oracle.softmax_backward(g, y)
        y64, g64 = y.astype(np.float64), g.astype(np.float64)
        ref = y64 * g64 - y64 * (y64 * g64).sum(-1, keepdims=True)
        assert np.abs(dx - ref).max() <= 1e-6 * (1 + np.abs(g64).max()), width


def test_bmm_exact_on_integers_and_close_on_random():
    for (b, m, k, n) in ((3, 5, 7, 4), (2, 1, 1, 1), (2, 33, 65, 17), (1, 3, 4, 2)):
        a = RNG.integers(-8, 9, size=(b, m, k)).astype(np.float32)
        c = RNG.integers(-8, 9, size=(b, k, n)).astype(np.float32)
        assert np.array_equal(oracle.bmm(a, c), a @ c)
        assert np.array_equal(oracle.bmm(a, np.swapaxes(np.ascontiguousarray(np.swapaxes(c, 1, 2)), 1, 2),
                                         b_k_contiguous=True), a @ c)
        a = RNG.standard_normal((b, m, k)).astype(np.float32)
        c = RNG.standard_normal((b, k, n)).astype(np.float32)
        ref = a.astype(np.float64) @ c.astype(np.float64)
        assert np.abs(oracle.bmm(a, c) - ref).max() <= 4 * k * 2**-24 * (np.abs(a) @ np.abs(c)).max()


def _brute(q, k, v, mask, causal, scale, g):
    """float64 dense attention (and grads) on rank-4 inputs, any Ev."""
    out, _ = brute.sdpa(q, k, v, causal, scale, mask)
    grads = brute.sdpa_grads(g, q, k, v, causal, scale, mask) if g is not None else None
    return out, grads


@pytest.mark.parametrize("case", ["rank4", "rank3", "ev", "causal", "bool_mask", "float_mask"])
def test_math_attention_against_float64(case):
    B, H, L, S, E, Ev = 2, 3, 19, 23, 16, 16
    if case == "ev":
        Ev = 24
    if case == "causal":
        S = L
    q = RNG.standard_normal((B, H, L, E)).astype(np.float32)
    k = RNG.standard_normal((B, H, S, E)).astype(np.float32)
    v = RNG.standard_normal((B, H, S, Ev)).astype(np.float32)
    g = RNG.standard_normal((B, H, L, Ev)).astype(np.float32)
    mask = None
    if case == "bool_mask":
        allowed = RNG.random((B, 1, L, S)) < 0.6
        allowed[0, 0, 3] = False  # a fully masked row
        mask = allowed
    if case == "float_mask":
        mask = (RNG.standard_normal((1, H, L, S)) * 2).astype(np.float32)
        mask[0, 1, 5] = -np.inf
    scale = 1.0 / math.sqrt(E)
    args = (q, k, v) if case != "rank3" else (q[0], k[0], v[0])
    out, (dq, dk, dv, _) = oracle.math_attention(*args, attn_mask=mask, is_causal=case == "causal",
                                                 grad_out=g if case != "rank3" else g[0])
    add = None if mask is None else (np.where(mask, 0.0, -np.inf) if mask.dtype == bool else mask)
    if add is not None:
        add = np.broadcast_to(add, (B, H, L, S))
    ref_out, ref_g = _brute(q, k, v, add, case == "causal", np.float32(scale), g)
    if case == "rank3":
        ref_out, ref_g = ref_out[0], tuple(x[0] for x in ref_g)
    assert_f32(out, ref_out, f"{case} out")
    for name, got, ref in zip(("dq", "dk", "dv"), (dq, dk, dv), ref_g):
        assert_f32(got, ref, f"{case} {name}")
    if case == "bool_mask":
        assert np.all(out[0, :, 3] == 0) and np.all(dq[0, :, 3] == 0)


def test_math_attention_mask_gradient():
    import torch
    B, H, L, S, E = 2, 2, 7, 9, 8
    q, k, v, g = (RNG.standard_normal(s).astype(np.float32)
                  for s in ((B, H, L, E), (B, H, S, E), (B, H, S, E), (B, H, L, E)))
    mask = RNG.standard_normal((1, H, L, S)).astype(np.float32)
    _, (_, _, _, da) = oracle.math_attention(q, k, v, attn_mask=mask, grad_out=g)
    dmask = da.sum(0, keepdims=True)
    t = [torch.tensor(x.astype(np.float64), requires_grad=True) for x in (q, k, v, mask)]
    s = t[0] @ t[1].transpose(-1, -2) / math.sqrt(E) + t[3]
    out = torch.softmax(s, -1) @ t[2]
    out.backward(torch.tensor(g.astype(np.float64)))
    assert_f32(dmask, t[3].grad.numpy(), "dmask")
