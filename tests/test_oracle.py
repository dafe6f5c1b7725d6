"""Pins the CPU oracle (oracle/sdpa_oracle.c) before it is trusted as the checker.

The reference holds no golden vectors for this path (its attention tests compare against live
torch), so each part is pinned by what the mathematics fixes, chosen so that a plausible
restatement mistake fails at least one check:
  * exp_u20 / SLEEF expf against float64 exp (error bounds), special values, and the
    per-4-lane-group fallback of exp_u20 (src/sleef.rs:1225-1255);
  * reduce_all's tree order op(op(a0, a2), op(a1, a3)) on inputs where the order changes the
    float32 result (src/torch_softmax.rs:14-37);
  * gemm_raw against a float64 matmul for every transpose combination and alpha/beta,
    normalize_last_dims and the layout error (src/torch_blas.rs:59-79, 95-134, 583-642);
  * forward/backward against the float64 brute force and torch's CPU SDPA on the reference's
    test shapes, and closed forms (constant V, q = 0, one key, fully masked rows,
    shift invariance);
  * the committed golden fixtures (tests/golden/sdpa_golden.npz).
"""
import math

import numpy as np
import pytest

from oracle import brute
from tests._data import additive, make_inputs

RNG = np.random.default_rng(1234)


def ulp_err(got, ref64):
    got = np.asarray(got, np.float64)
    ulp = np.spacing(np.abs(ref64).astype(np.float32)).astype(np.float64)
    return np.abs(got - ref64) / ulp


# ---------------- exp kernels ----------------

def test_exp_u20_accuracy(oracle_lib):
    x = np.linspace(-87.0, 87.0, 400_000, dtype=np.float32)
    y = oracle_lib.exp_u20(x)
    ref = np.exp(x.astype(np.float64))
    assert ulp_err(y, ref).max() < 3.0  # Arm Optimized Routines expf: ~2 ulp


def test_sleef_expf_accuracy_and_specials(oracle_lib):
    x = np.linspace(-103.0, 88.5, 400_000, dtype=np.float32)
    y = oracle_lib.sleef_expf(x)
    ref = np.exp(x.astype(np.float64))
    normal = ref > np.finfo(np.float32).tiny
    assert ulp_err(y[normal], ref[normal]).max() <= 1.0  # SLEEF xexpf is a 1.0-ulp function
    s = oracle_lib.sleef_expf(np.array([0.0, -np.inf, -105.0, 101.0, np.inf], np.float32))
    assert s[0] == 1.0 and s[1] == 0.0 and s[2] == 0.0 and np.isposinf(s[3]) and np.isposinf(s[4])


def test_exp_u20_group_fallback(oracle_lib):
    """One lane past the bound sends all four lanes of its group to SLEEF's expf."""
    base = np.array([0.3, -1.7, 2.9, -5.1], np.float32)
    grp = base.copy()
    grp[3] = -100.0
    y = oracle_lib.exp_u20(np.concatenate([base, grp]))
    assert np.array_equal(y[4:], oracle_lib.sleef_expf(grp))
    assert np.array_equal(y[:4], oracle_lib.exp_u20(base))
    # The two formulas differ in the last bit somewhere on a dense grid, so the fallback is
    # observable (a restatement without the group rule would fail the line above).
    x = np.linspace(-5, 5, 4096, dtype=np.float32)
    assert not np.array_equal(oracle_lib.exp_u20(x), oracle_lib.sleef_expf(x))


def test_exp_reduce_sum(oracle_lib):
    row = RNG.standard_normal(37).astype(np.float32) * 3
    mx = float(row.max())
    out, s = oracle_lib.exp_reduce_sum(row, mx)
    ref = np.exp((row - np.float32(mx)).astype(np.float64))  # exp of the float32 difference
    np.testing.assert_allclose(out, ref, rtol=3e-7)
    np.testing.assert_allclose(s, ref.sum(), rtol=1e-6)


# ---------------- reductions ----------------

def test_reduce_all_tree_order(oracle_lib):
    # Tree: (a0 + a2) + (a1 + a3) = (1e8 - 1e8) + (1 + 1) = 2; a left-to-right float32 sum
    # gives ((1e8 + 1) - 1e8) + 1 = 1.
    a = np.array([1e8, 1.0, -1e8, 1.0], np.float32)
    assert oracle_lib.reduce_dot(a, np.ones(4, np.float32)) == 2.0
    # Fewer than four elements combine in order; a tail lane updates its partial.
    assert oracle_lib.reduce_dot(np.array([1e8, 1.0, -1e8], np.float32), np.ones(3, np.float32)) == 0.0
    # The tail element is added into lane 0 (1e8 + 1 rounds to 1e8), so the tree gives 0
    # where an in-order sum gives 1.
    a5 = np.array([1e8, 0.0, -1e8, 0.0, 1.0], np.float32)
    assert oracle_lib.reduce_dot(a5, np.ones(5, np.float32)) == 0.0
    x = RNG.standard_normal(1001).astype(np.float32)
    assert oracle_lib.reduce_max(x) == x.max()
    x[500] = np.nan
    assert np.isnan(oracle_lib.reduce_max(x))


def test_mul_reduce_max(oracle_lib):
    row = RNG.standard_normal(29).astype(np.float32)
    out, m = oracle_lib.mul_reduce_max(row, 0.125)
    assert np.array_equal(out, row * np.float32(0.125))
    assert m == (row * np.float32(0.125)).max()
    row[3] = np.nan
    assert np.isnan(oracle_lib.mul_reduce_max(row, 0.5)[1])


# ---------------- gemm_raw ----------------

@pytest.mark.parametrize("ta,tb", [(0, 0), (0, 1), (1, 0), (1, 1)])
@pytest.mark.parametrize("alpha,beta", [(1.0, 0.0), (0.3, 1.0), (-2.0, 0.5)])
def test_gemm_raw_matches_matmul(oracle_lib, ta, tb, alpha, beta):
    m, n, k = 7, 5, 9
    A = RNG.standard_normal((k, m) if ta else (m, k)).astype(np.float32)  # logical op(A) is m x k
    Bm = RNG.standard_normal((n, k) if tb else (k, n)).astype(np.float32)
    C0 = RNG.standard_normal((m, n)).astype(np.float32)
    # Column-major storage: a column-major X is the row-major X^T.
    a_cm = np.ascontiguousarray(A.T).ravel()
    b_cm = np.ascontiguousarray(Bm.T).ravel()
    c_cm = np.ascontiguousarray(C0.T).ravel()
    lda, ldb = A.shape[0], Bm.shape[0]
    got = oracle_lib.gemm_raw(ta, tb, m, n, k, alpha, a_cm, lda, b_cm, ldb, beta, c_cm, m)
    opA = A.T if ta else A
    opB = Bm.T if tb else Bm
    ref = alpha * (opA.astype(np.float64) @ opB.astype(np.float64)) + beta * C0
    np.testing.assert_allclose(got.reshape(n, m).T, ref, rtol=1e-5, atol=1e-5)


def test_gemm_raw_layout_error_and_normalize(oracle_lib):
    with pytest.raises(RuntimeError, match="gemm layout"):
        oracle_lib.gemm_raw(0, 0, 4, 2, 3, 1.0, np.zeros(12, np.float32), 2,  # lda < m
                            np.zeros(6, np.float32), 3, 0.0, np.zeros(8, np.float32), 4)
    # n == 1: ldc is normalised to m, so a too-small ldc is accepted (normalize_last_dims).
    a = RNG.standard_normal(6).astype(np.float32)
    b = RNG.standard_normal(3).astype(np.float32)
    got = oracle_lib.gemm_raw(0, 0, 2, 1, 3, 1.0, a, 2, b, 3, 0.0, np.zeros(2, np.float32), 1)
    np.testing.assert_allclose(got, a.reshape(3, 2).T @ b, rtol=1e-6)


def test_split_policy_and_scale(oracle_lib):
    assert [oracle_lib.q_split(n) for n in (1, 191, 192, 767, 768, 4096)] == [32, 32, 64, 64, 256, 256]
    assert oracle_lib.scale_factor(64) == np.float32(0.125)
    assert oracle_lib.scale_factor(12) == np.float32(1.0 / math.sqrt(12.0))
    assert oracle_lib.scale_factor(12, 0.3) == np.float32(0.3)


# ---------------- attention against independent references ----------------

SHAPES = [(2, 2, 7, 7, 5, False, None), (2, 2, 7, 7, 5, True, None), (1, 3, 33, 33, 16, True, None),
          (1, 2, 100, 37, 12, False, None), (1, 1, 200, 200, 8, True, None),
          (1, 2, 9, 1030, 6, False, None), (1, 2, 64, 64, 16, True, 0.3)]


@pytest.mark.parametrize("B,H,L,S,E,causal,scale", SHAPES)
def test_forward_backward_vs_float64(oracle_lib, B, H, L, S, E, causal, scale):
    rng = np.random.default_rng(L * 31 + S)
    q, g = (rng.normal(size=(B, H, L, E)).astype(np.float32) for _ in range(2))
    k, v = (rng.normal(size=(B, H, S, E)).astype(np.float32) for _ in range(2))
    out, lse = oracle_lib.forward(q, k, v, causal, scale)
    bo, bl = brute.sdpa(q, k, v, causal, scale)
    np.testing.assert_allclose(out, bo, rtol=1e-5, atol=2e-6)
    np.testing.assert_allclose(lse, bl, rtol=1e-5, atol=2e-6)
    for a, b in zip(oracle_lib.backward(g, q, k, v, out, lse, causal, scale),
                    brute.sdpa_grads(g, q, k, v, causal, scale)):
        np.testing.assert_allclose(a, b, rtol=1e-4, atol=1e-5)


@pytest.mark.parametrize("mode", ["none", "causal", "bool", "float"])
def test_vs_torch_cpu_sdpa(oracle_lib, mode):
    """tests/test_attention.py:12-39 of the reference, with torch's CPU SDPA as the oracle's
    oracle (same algorithm family, float32) at the reference's tolerances."""
    torch = pytest.importorskip("torch")
    rng = np.random.default_rng(21)
    q, k, v, g = (rng.normal(size=(2, 3, 40, 8)).astype(np.float32) for _ in range(4))
    mask, tm = None, None
    if mode == "bool":
        mb = rng.random((40, 40)) > .3
        mb[:, 0] = True
        mask, tm = additive(mb, (2, 3, 40, 40)), torch.from_numpy(mb)
    elif mode == "float":
        mf = rng.normal(size=(40, 40)).astype(np.float32)
        mask, tm = np.ascontiguousarray(np.broadcast_to(mf, (2, 3, 40, 40))), torch.from_numpy(mf)
    causal = mode == "causal"
    out, lse = oracle_lib.forward(q, k, v, causal, None, mask)
    t = [torch.tensor(x, requires_grad=True) for x in (q, k, v)]
    y = torch.nn.functional.scaled_dot_product_attention(*t, attn_mask=tm, is_causal=causal)
    np.testing.assert_allclose(out, y.detach().numpy(), rtol=1e-5, atol=1e-6)
    y.backward(torch.from_numpy(g))
    for a, tt in zip(oracle_lib.backward(g, q, k, v, out, lse, causal, None, mask), t):
        np.testing.assert_allclose(a, tt.grad.numpy(), rtol=1e-4, atol=1e-5)


def test_grouped_heads_equal_widened(oracle_lib):
    """Hkv < H is the same as widening k and v (src/torch_attention.rs:159-167, 321-324)."""
    rng = np.random.default_rng(3)
    q, g = (rng.standard_normal((2, 4, 9, 8), dtype=np.float32) for _ in range(2))
    k, v = (rng.standard_normal((2, 2, 9, 8), dtype=np.float32) for _ in range(2))
    out, lse = oracle_lib.forward(q, k, v, True)
    kw, vw = np.repeat(k, 2, axis=1), np.repeat(v, 2, axis=1)
    ow, lw = oracle_lib.forward(q, kw, vw, True)
    assert np.array_equal(out, ow) and np.array_equal(lse, lw)
    dq, dk, dv = oracle_lib.backward(g, q, k, v, out, lse, True)
    dqw, dkw, dvw = oracle_lib.backward(g, q, kw, vw, out, lse, True)
    assert np.array_equal(dq, dqw)
    np.testing.assert_allclose(dk, dkw.reshape(2, 2, 2, 9, 8).sum(2), rtol=1e-6, atol=1e-7)
    np.testing.assert_allclose(dv, dvw.reshape(2, 2, 2, 9, 8).sum(2), rtol=1e-6, atol=1e-7)


# ---------------- closed forms ----------------

def test_closed_forms(oracle_lib):
    rng = np.random.default_rng(11)
    B, H, L, S, E = 1, 2, 70, 70, 16
    q, k = (rng.standard_normal((B, H, n, E), dtype=np.float32) for n in (L, S))
    # Constant V rows: out is that row, whatever the weights.
    c = rng.standard_normal((B, H, 1, E), dtype=np.float32)
    out, _ = oracle_lib.forward(q, k, np.ascontiguousarray(np.broadcast_to(c, (B, H, S, E))), True)
    np.testing.assert_allclose(out, np.broadcast_to(c, out.shape), rtol=1e-6, atol=1e-6)
    # q = 0: uniform weights over the allowed keys: causal prefix means, lse = ln(#allowed).
    v = rng.standard_normal((B, H, S, E), dtype=np.float32)
    out, lse = oracle_lib.forward(np.zeros_like(q), k, v, True)
    prefix = np.cumsum(v.astype(np.float64), axis=2) / np.arange(1, S + 1)[:, None]
    np.testing.assert_allclose(out, prefix, rtol=1e-5, atol=1e-6)
    np.testing.assert_allclose(lse, np.broadcast_to(np.log(np.arange(1, L + 1)), lse.shape), rtol=1e-6)
    # One key: out = v0 and lse = scale * q . k0.
    k1, v1 = k[:, :, :1], v[:, :, :1]
    out, lse = oracle_lib.forward(q, k1, v1, False)
    np.testing.assert_allclose(out, np.broadcast_to(v1, out.shape), rtol=1e-6, atol=1e-7)
    np.testing.assert_allclose(lse, (q @ k1.transpose(0, 1, 3, 2))[..., 0] * 0.25, rtol=1e-5, atol=1e-6)
    # Shift invariance: a constant added to every score of a row moves lse by it, not out.
    m = rng.standard_normal((B, H, L, S)).astype(np.float32)
    o1, l1 = oracle_lib.forward(q, k, v, False, None, m)
    o2, l2 = oracle_lib.forward(q, k, v, False, None, m + np.float32(3.0))
    np.testing.assert_allclose(o2, o1, rtol=1e-5, atol=1e-6)
    np.testing.assert_allclose(l2, l1 + 3.0, rtol=1e-6, atol=1e-5)


def test_fully_masked_rows(oracle_lib):
    """src/torch_attention.rs:223-226, 258-264: out 0, lse 0 and zero gradients."""
    rng = np.random.default_rng(12)
    q, k, v, g = (rng.standard_normal((1, 1, 6, 8), dtype=np.float32) for _ in range(4))
    mask = np.zeros((1, 1, 6, 6), np.float32)
    mask[0, 0, 2, :] = -np.inf
    out, lse = oracle_lib.forward(q, k, v, False, None, mask)
    assert not out[0, 0, 2].any() and lse[0, 0, 2] == 0.0
    dq, dk, dv = oracle_lib.backward(g, q, k, v, out, lse, False, None, mask)
    assert not dq[0, 0, 2].any()
    # The other rows are unaffected by the dead row.
    o2, _ = oracle_lib.forward(q, k, v, False, None, np.zeros_like(mask))
    np.testing.assert_array_equal(np.delete(out, 2, axis=2), np.delete(o2, 2, axis=2))


def test_threads_do_not_change_bits(oracle_lib):
    """src/torch_attention.rs:8: the (batch, head) split never changes the result."""
    d = make_inputs("C1", B=3, H=2, L=80, S=80, E=16)
    n = oracle_lib.get_num_threads()
    try:
        oracle_lib.set_num_threads(1)
        a = oracle_lib.forward(d["q"], d["k"], d["v"], True)
        oracle_lib.set_num_threads(5)
        b = oracle_lib.forward(d["q"], d["k"], d["v"], True)
    finally:
        oracle_lib.set_num_threads(n)
    assert all(np.array_equal(x, y) for x, y in zip(a, b))


# ---------------- committed fixtures ----------------

def _golden():
    import os
    path = os.path.join(os.path.dirname(__file__), "golden", "sdpa_golden.npz")
    return np.load(path)


def golden_cases():
    z = _golden()
    tags = sorted({k.split("/")[0] for k in z.files if not k.startswith("in_")})
    return tags


@pytest.mark.parametrize("tag", golden_cases())
def test_oracle_reproduces_golden(oracle_lib, tag):
    z = _golden()
    src = str(z[f"{tag}/inputs"])
    q, k, v, g = (z[f"{src}/{n}"] for n in "qkvg")
    causal, scale = z[f"{tag}/meta"]
    scale = None if np.isnan(scale) else float(scale)
    mask = z[f"{tag}/mask"] if f"{tag}/mask" in z.files else None
    out, lse = oracle_lib.forward(q, k, v, bool(causal), scale, mask)
    assert np.array_equal(out, z[f"{tag}/out"]) and np.array_equal(lse, z[f"{tag}/lse"])
    for name, a in zip(("dq", "dk", "dv"), oracle_lib.backward(g, q, k, v, out, lse, bool(causal), scale, mask)):
        assert np.array_equal(a, z[f"{tag}/{name}"]), name
