"""GPU parity: the HIP kernels (through the C ABI) against the CPU oracle on identical inputs.

Tolerance (written here, the target's): float32 outputs, lse and gradients must satisfy
|gpu - ref| <= 2e-5 + 1e-5 |ref| elementwise.

Shapes are the ones the reference's own tests pin (tests/test_sdpa_exact.py:10-14, 33-41;
tests/test_attention.py:12-39; tests/test_torch_api_f1.py:78-84) plus the edge cases the
kernels' tiling creates (partial tiles, head dims that are not a multiple of 4, L != S,
fully masked rows, one key, grouped heads).
"""
import numpy as np
import pytest

from tests._data import additive, assert_f32, assert_f32_nan

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu

DEV = "cuda:0"


def _t(x):
    return torch.from_numpy(np.ascontiguousarray(x)).to(DEV)


def _run_fwd(q, k, v, causal, scale, mask):
    from densecore_amd import _native
    m = None if mask is None else _t(mask)
    out, lse = _native._flash_attention(_t(q), _t(k), _t(v), causal, scale, m)
    torch.cuda.synchronize()
    return out.cpu().numpy(), lse.cpu().numpy()


def _run_bwd(g, q, k, v, out, lse, causal, scale, mask):
    from densecore_amd import _native
    m = None if mask is None else _t(mask)
    grads = _native._flash_attention_backward(_t(g), _t(q), _t(k), _t(v), _t(out), _t(lse), causal,
                                              scale, m)
    torch.cuda.synchronize()
    return [x.cpu().numpy() for x in grads]


def _check(oracle, q, k, v, g, causal, scale=None, mask=None, tag=""):
    print(f"[case] {tag} q{q.shape} k{k.shape} causal={causal} scale={scale} "
          f"mask={None if mask is None else mask.shape}", flush=True)
    ref_o, ref_l = oracle.forward(q, k, v, causal, scale, mask)
    out, lse = _run_fwd(q, k, v, causal, scale, mask)
    assert_f32(out, ref_o, f"{tag} out")
    assert_f32(lse, ref_l, f"{tag} lse")
    if g is None:
        return
    # Backward from the oracle's saved (out, lse), so the gradients are compared on equal inputs.
    ref = oracle.backward(g, q, k, v, ref_o, ref_l, causal, scale, mask)
    got = _run_bwd(g, q, k, v, ref_o, ref_l, causal, scale, mask)
    for name, a, b in zip(("dq", "dk", "dv"), got, ref):
        assert_f32(a, b, f"{tag} {name}")


EXACT_SHAPES = [  # tests/test_sdpa_exact.py:10-14
    (2, 2, 7, 7, 5, False, None), (2, 2, 7, 7, 5, True, None), (1, 3, 33, 33, 16, True, None),
    (1, 2, 100, 37, 12, False, None), (1, 1, 200, 200, 8, True, None), (1, 1, 600, 600, 8, False, None),
    (1, 1, 800, 800, 4, True, None), (1, 2, 9, 1030, 6, False, None), (1, 2, 64, 64, 16, True, 0.3),
]


@pytest.mark.parametrize("B,H,L,S,E,causal,scale", EXACT_SHAPES)
def test_exact_shapes(oracle_lib, B, H, L, S, E, causal, scale):
    rng = np.random.default_rng(L * 31 + S)
    q, g = (rng.normal(size=(B, H, L, E)).astype(np.float32) for _ in range(2))
    k, v = (rng.normal(size=(B, H, S, E)).astype(np.float32) for _ in range(2))
    _check(oracle_lib, q, k, v, g, causal, scale, tag=f"exact{(B, H, L, S, E)}")


MASK_SHAPES = [(2, 2, 7, 7, 5), (1, 2, 200, 37, 12), (1, 1, 9, 1030, 6), (2, 3, 64, 64, 16)]


@pytest.mark.parametrize("B,H,L,S,E", MASK_SHAPES)
@pytest.mark.parametrize("kind", ["bool2d", "float2d", "bool4d_b1", "float4d_1h", "row"])
def test_masked_shapes(oracle_lib, B, H, L, S, E, kind):
    """tests/test_sdpa_exact.py:32-51: five mask kinds; "row" masks every key of every row."""
    rng = np.random.default_rng(L + S)
    q, g = (rng.normal(size=(B, H, L, E)).astype(np.float32) for _ in range(2))
    k, v = (rng.normal(size=(B, H, S, E)).astype(np.float32) for _ in range(2))
    mask = {"bool2d": rng.random((L, S)) > 0.3, "float2d": rng.normal(size=(L, S)).astype(np.float32),
            "bool4d_b1": rng.random((B, 1, L, S)) > 0.5,
            "float4d_1h": rng.normal(size=(1, H, 1, S)).astype(np.float32),
            "row": np.zeros((L, S), bool)}[kind]
    full = additive(mask, (B, H, L, S)) if mask.dtype == np.bool_ else \
        np.ascontiguousarray(np.broadcast_to(mask, (B, H, L, S)), np.float32)
    _check(oracle_lib, q, k, v, g, False, None, full, tag=f"mask-{kind}{(B, H, L, S, E)}")


@pytest.mark.parametrize("B,H,L,S,E,kind", [
    (2, 3, 70, 300, 64, "padding"), (2, 2, 130, 257, 64, "holes"), (1, 4, 64, 200, 128, "holes"),
    (2, 2, 100, 100, 32, "per_head"), (1, 2, 50, 129, 48, "holes"), (2, 1, 40, 64, 64, "closed"),
    (5, 7, 90, 333, 64, "per_bh"), (16, 16, 64, 512, 64, "padding"), (3, 11, 40, 1000, 32, "per_bh"),
])
def test_row_broadcast_masks(oracle_lib, B, H, L, S, E, kind):
    """Masks that do not depend on the query (a stride-0 view along L: key padding and the like)
    take their own path in the float32 forward (one mask load per key and tile, sub-tile liveness
    from a ballot).  Padding, random holes, per-head rows, a fully masked batch row ("closed":
    out 0, lse 0), 32-key tiles (E = 128) and the unaligned generic path (E = 48).  Such masks
    also order the forward's workgroups by each head's live key tiles (longest first, a head's
    query tiles on one XCD): per-(batch, head) prefix lengths including empty heads ("per_bh"),
    batch * heads not a multiple of 8, and C3's 256 heads check that every (head, query tile) is
    computed exactly once."""
    from densecore_amd import _native
    rng = np.random.default_rng(B * 7 + H * 11 + L + S + E)
    q, g = (rng.standard_normal((B, H, L, E), dtype=np.float32) for _ in range(2))
    k, v = (rng.standard_normal((B, H, S, E), dtype=np.float32) for _ in range(2))
    if kind == "padding":
        lens = rng.integers(1, S + 1, size=B)
        allowed = np.arange(S)[None, None, None, :] < lens[:, None, None, None]
    elif kind == "holes":
        allowed = rng.random((B, 1, 1, S)) > 0.6
    elif kind == "per_head":
        allowed = rng.random((1, H, 1, S)) > 0.5
    elif kind == "per_bh":
        lens = rng.integers(0, S + 1, size=(B, H))
        lens[0, 0], lens[-1, -1] = 0, S
        allowed = np.arange(S)[None, None, None, :] < lens[:, :, None, None]
    else:
        allowed = np.ones((B, 1, 1, S), bool)
        allowed[0] = False
    small = np.where(allowed, np.float32(0), np.float32(-np.inf)).astype(np.float32)
    view = _t(small).expand(B, H, L, S)
    assert view.stride(2) == 0
    full = additive(allowed, (B, H, L, S))
    print(f"[case] row mask {kind} q{q.shape} k{k.shape}", flush=True)
    ref_o, ref_l = oracle_lib.forward(q, k, v, False, None, full)
    out, lse = _native._flash_attention(_t(q), _t(k), _t(v), False, None, view)
    torch.cuda.synchronize()
    assert_f32(out.cpu().numpy(), ref_o, f"row-{kind} out")
    assert_f32(lse.cpu().numpy(), ref_l, f"row-{kind} lse")
    ref = oracle_lib.backward(g, q, k, v, ref_o, ref_l, False, None, full)
    got = _native._flash_attention_backward(_t(g), _t(q), _t(k), _t(v), _t(ref_o), _t(ref_l), False,
                                            None, view)
    for name, a, b in zip(("dq", "dk", "dv"), got, ref):
        assert_f32(a.cpu().numpy(), b, f"row-{kind} {name}")


@pytest.mark.parametrize("shape", [(1, 1, 70, 1), (2, 1, 70, 1), (2, 3, 70, 1)])
def test_key_broadcast_masks(oracle_lib, shape):
    """A mask constant along the keys (an (L, 1)-shaped row bias, stride 0 over S) is copied
    along the key axis only and keeps its other broadcast strides; rows at -inf are fully
    masked (out 0, lse 0, zero gradients)."""
    from densecore_amd import _native
    B, H, L, S, E = 2, 3, 70, 90, 64
    rng = np.random.default_rng(sum(shape))
    q, g = (rng.standard_normal((B, H, L, E), dtype=np.float32) for _ in range(2))
    k, v = (rng.standard_normal((B, H, S, E), dtype=np.float32) for _ in range(2))
    small = rng.standard_normal(shape).astype(np.float32)
    small[..., ::7, :] = -np.inf
    view = _t(small).expand(B, H, L, S)
    m, _ = _native._mask_arg(view, (B, H, H, L, S, E), view.device)
    assert m.untyped_storage().nbytes() == small.size * S * 4
    full = np.ascontiguousarray(np.broadcast_to(small, (B, H, L, S)))
    print(f"[case] key-broadcast mask {shape}", flush=True)
    ref_o, ref_l = oracle_lib.forward(q, k, v, False, None, full)
    out, lse = _native._flash_attention(_t(q), _t(k), _t(v), False, None, view)
    torch.cuda.synchronize()
    assert_f32(out.cpu().numpy(), ref_o, "key-broadcast out")
    assert_f32(lse.cpu().numpy(), ref_l, "key-broadcast lse")
    ref = oracle_lib.backward(g, q, k, v, ref_o, ref_l, False, None, full)
    got = _native._flash_attention_backward(_t(g), _t(q), _t(k), _t(v), _t(ref_o), _t(ref_l), False,
                                            None, view)
    for name, a, b in zip(("dq", "dk", "dv"), got, ref):
        assert_f32(a.cpu().numpy(), b, f"key-broadcast {name}")


@pytest.mark.parametrize("mode", ["none", "causal", "bool", "float"])
def test_attention_rank4(oracle_lib, mode):
    """tests/test_attention.py:12-39, rank-4 (2, 3, 4, 8) cases."""
    rng = np.random.default_rng(21)
    q, k, v, g = (rng.normal(size=(2, 3, 4, 8)).astype(np.float32) for _ in range(4))
    mask = None
    if mode == "bool":
        m = rng.random((4, 4)) > .3
        m[:, 0] = True
        mask = additive(m, (2, 3, 4, 4))
    elif mode == "float":
        mask = np.ascontiguousarray(np.broadcast_to(rng.normal(size=(4, 4)).astype(np.float32),
                                                    (2, 3, 4, 4)))
    _check(oracle_lib, q, k, v, g, mode == "causal", None, mask, tag=f"rank4-{mode}")


@pytest.mark.parametrize("B,H,Hkv,L,S,E,causal", [
    (2, 4, 2, 5, 5, 8, True),        # tests/test_torch_api_f1.py:78-84
    (1, 6, 2, 300, 300, 64, True),
    (2, 8, 1, 130, 250, 32, False),
    (1, 4, 2, 200, 200, 32, True),   # short causal rows: one-wave forward, D = 32
])
def test_grouped_heads(oracle_lib, B, H, Hkv, L, S, E, causal):
    rng = np.random.default_rng(B * 1000 + H * 10 + Hkv)
    q, g = (rng.standard_normal((B, H, L, E), dtype=np.float32) for _ in range(2))
    k, v = (rng.standard_normal((B, Hkv, S, E), dtype=np.float32) for _ in range(2))
    _check(oracle_lib, q, k, v, g, causal, tag="gqa")


@pytest.mark.parametrize("scale", [-0.4, 0.0, -0.0, float("nan")])
@pytest.mark.parametrize("B,H,L,S,E,causal,masked", [
    (2, 2, 100, 100, 64, True, False),    # one-wave forward
    (1, 3, 300, 300, 64, True, False),    # 4-wave forward
    (1, 2, 600, 600, 64, True, False),    # split key ranges
    (1, 1, 1100, 1100, 32, True, False),  # q blocks of 256, two key blocks of 512
    (1, 2, 100, 300, 64, True, False),    # L < S: keys no query sees
    (1, 2, 300, 100, 64, True, False),    # L > S
    (1, 1, 3, 3, 16, True, False),        # one block narrower than 4 keys
    (1, 2, 150, 150, 64, True, True),     # a float mask as well
    (1, 2, 130, 130, 160, True, False),   # head dim above 128 (materialized rows)
    (1, 2, 200, 300, 32, False, False),   # non-causal: only a NaN scale changes anything
])
def test_negative_and_zero_scale(oracle_lib, B, H, L, S, E, causal, masked, scale):
    """An explicit scale may be negative, zero or NaN (the reference takes any float), and the
    result is the reference's, NaN rows included: it writes -inf into causally masked scores
    before it scales them (src/torch_attention.rs:202-216), so -inf times a negative scale is
    +inf and times 0 NaN, and every row with such a score in its last key block comes out NaN;
    a NaN scale makes every row NaN (0 without a mask when the only block is narrower than 4
    keys).  torch's CPU SDPA gives the same rows.  Out and lse are compared with the oracle's
    causal forward on the same inputs: the same NaN elements, the float32 bar elsewhere; the
    backward from the oracle's (out, lse) must spread those NaN to the same gradient elements."""
    rng = np.random.default_rng(B + 3 * H + 5 * L + 7 * S + 11 * E)
    q, g = (rng.standard_normal((B, H, L, E), dtype=np.float32) for _ in range(2))
    k, v = (rng.standard_normal((B, H, S, E), dtype=np.float32) for _ in range(2))
    mask = None
    if masked:
        mask = rng.standard_normal((B, H, L, S)).astype(np.float32)
        mask[rng.random((B, H, L, S)) < 0.2] = -np.inf
    print(f"[case] scale {scale} q{q.shape} k{k.shape} causal={causal} mask={masked}", flush=True)
    ref_o, ref_l = oracle_lib.forward(q, k, v, causal, scale, mask)
    out, lse = _run_fwd(q, k, v, causal, scale, mask)
    assert_f32_nan(out, ref_o, f"scale {scale} out")
    assert_f32_nan(lse, ref_l, f"scale {scale} lse")
    if causal and scale == scale and (S >= 4 or masked):
        assert bool(np.isnan(ref_l).any()), "the case must be one the reference makes NaN"
    ref = oracle_lib.backward(g, q, k, v, ref_o, ref_l, causal, scale, mask)
    got = _run_bwd(g, q, k, v, ref_o, ref_l, causal, scale, mask)
    for name, x, y in zip(("dq", "dk", "dv"), got, ref):
        assert_f32_nan(x, y, f"scale {scale} {name}")


@pytest.mark.parametrize("B,H,L,S,E,causal", [
    (1, 1, 1, 1, 64, False), (1, 2, 1, 700, 64, False), (1, 1, 129, 1, 64, True),
    (2, 2, 257, 191, 64, True), (1, 3, 191, 257, 64, False), (1, 2, 130, 70, 128, True),
    (1, 2, 65, 300, 128, False), (1, 1, 40, 40, 100, True), (1, 1, 33, 47, 1, False),
    (1, 1, 50, 60, 31, True), (3, 1, 200, 200, 64, True),
    # short causal rows (L <= 256, no mask) take the one-wave forward: aligned D = 32 and 64, keys
    # beyond the queries, a ragged last tile
    (2, 3, 100, 100, 32, True), (1, 2, 96, 160, 64, True), (2, 1, 256, 256, 32, True),
])
def test_tile_edges(oracle_lib, B, H, L, S, E, causal):
    rng = np.random.default_rng(B + 7 * H + 13 * L + 17 * S + 19 * E)
    q, g = (rng.standard_normal((B, H, L, E), dtype=np.float32) for _ in range(2))
    k, v = (rng.standard_normal((B, H, S, E), dtype=np.float32) for _ in range(2))
    _check(oracle_lib, q, k, v, g, causal, tag="edge")


def test_causal_with_mask(oracle_lib):
    """The native boundary accepts causal and a mask together (src/torch_attention.rs:202-215)."""
    rng = np.random.default_rng(5)
    q, k, v, g = (rng.standard_normal((2, 2, 150, 64), dtype=np.float32) for _ in range(4))
    mask = rng.standard_normal((2, 2, 150, 150)).astype(np.float32)
    _check(oracle_lib, q, k, v, g, True, 0.2, mask, tag="causal+mask")


@pytest.fixture
def consistent_scores(request):
    """Run the test with DC_FLAG_CONSISTENT_SCORES on (param True) or off, restoring the setting."""
    from densecore_amd import _native
    previous = _native.consistent_scores(getattr(request, "param", False))
    yield getattr(request, "param", False)
    _native.consistent_scores(previous)


@pytest.mark.parametrize("E,factor,consistent_scores", [(64, 2, False), (128, 8, False), (128, 2, True)],
                         indirect=["consistent_scores"])
def test_large_logits(oracle_lib, E, factor, consistent_scores):
    """Scores far past the exp_u20 bound (|x - max| > 87.3, the reference's SLEEF fallback).

    Forward at the standard tolerance.  The gradients of such a peaked softmax are
    ill-conditioned: a one-ulp change of a score of magnitude ~100 moves P by ~1e-5
    relative, so two correct float32 summation orders differ by more than 2e-5.  There the
    GPU is held to float64 truth instead, each side running end to end on its own forward
    (out, lse): its error may not exceed twice the oracle's.  (Feeding one side's lse to the
    other's backward would mix two summation orders of the same scores, so that P no longer
    sums to one by ~1e-5, an error of the test, not of either implementation.)  At head dim 128
    the backward's scores run on 16x16x4 products in another order than the forward's 32x32x2
    (its 8-wave layout), which is that same mixing inside the GPU: its error there is held to
    8x the oracle's (measured up to 5.3x, in dV).  With DC_FLAG_CONSISTENT_SCORES the head-dim-128
    backward forms its scores in the forward's order and is held to 2x, as at head dim 64.  q and
    k scale with E^(-1/4), so the score gaps within a row stay of the order of 100 at both head
    dims."""
    from oracle import brute
    rng = np.random.default_rng(9)
    q, k, v, g = (rng.standard_normal((1, 2, 96, E), dtype=np.float32) for _ in range(4))
    q, k = q * 6 * (64 / E) ** 0.25, k * 6 * (64 / E) ** 0.25
    ref_o, ref_l = oracle_lib.forward(q, k, v, True)
    out, lse = _run_fwd(q, k, v, True, None, None)
    assert_f32(out, ref_o, "large-logits out")
    assert_f32(lse, ref_l, "large-logits lse")
    truth = brute.sdpa_grads(g, q, k, v, True)
    ref = oracle_lib.backward(g, q, k, v, ref_o, ref_l, True)
    got = _run_bwd(g, q, k, v, out, lse, True, None, None)
    for name, a, b, t in zip(("dq", "dk", "dv"), got, ref, truth):
        err_gpu, err_ref = np.abs(a - t).max(), np.abs(b - t).max()
        assert err_gpu <= factor * err_ref + 2e-6, f"{name}: gpu err {err_gpu:.3e} vs oracle {err_ref:.3e}"


@pytest.mark.parametrize("causal", [False, True])
def test_nan_scores_propagate(oracle_lib, causal):
    """A NaN in q or k makes every row that sees it NaN, out and lse, as the reference's
    NaN-propagating row max does (src/torch_attention.rs:42-87, src/torch_softmax.rs:43-54); a
    causally hidden NaN key leaves the rows before it untouched (its score is -inf either way).
    (NaN in v, or the backward, also reach rows through 0 * NaN inside a tile whose keys a row does
    not see; which rows depends on each implementation's tiling, so those are not compared.)"""
    rng = np.random.default_rng(5)
    q, k, v = (rng.standard_normal((1, 2, 70, 16), dtype=np.float32) for _ in range(3))
    k[0, 1, 5, 3] = np.nan
    k[0, 0, 60, 2] = np.nan
    q[0, 1, 33, 0] = np.nan
    ref_o, ref_l = oracle_lib.forward(q, k, v, causal)
    out, lse = _run_fwd(q, k, v, causal, None, None)
    assert (np.isnan(out) == np.isnan(ref_o)).all() and (np.isnan(lse) == np.isnan(ref_l)).all()
    assert np.isnan(ref_l).sum() == (70 + 70 if not causal else 10 + 65)
    fin = ~np.isnan(ref_o)
    assert_f32(out[fin], ref_o[fin], "finite out")
    assert_f32(lse[~np.isnan(ref_l)], ref_l[~np.isnan(ref_l)], "finite lse")


def test_errors_match_reference():
    """src/lib.rs:561-571, 599-606, 658-663: ValueError with the reference's messages."""
    from densecore_amd import _native
    x = torch.zeros((1, 2, 3, 4), device=DEV)
    with pytest.raises(ValueError, match=r"takes \(B, H, L, E\) tensors"):
        _native._flash_attention(x[0], x, x, False)
    with pytest.raises(ValueError, match="q/k/v shapes do not match"):
        _native._flash_attention(x, torch.zeros((1, 3, 3, 4), device=DEV), x, False)
    with pytest.raises(ValueError, match="mask must be"):
        _native._flash_attention(x, x, x, False, None, torch.zeros((1, 2, 3, 2), device=DEV))
    out, lse = _native._flash_attention(x, x, x, False)
    with pytest.raises(ValueError, match="backward shapes do not match"):
        _native._flash_attention_backward(out, x, x, x, out, lse[..., :2], False)


def _golden_tags():
    import os
    z = np.load(os.path.join(os.path.dirname(__file__), "golden", "sdpa_golden.npz"))
    return z, sorted({k.split("/")[0] for k in z.files if not k.startswith("in_")})


@pytest.mark.parametrize("tag", _golden_tags()[1])
def test_golden_fixtures(tag):
    """The committed fixtures (tests/golden/sdpa_golden.npz), no live oracle involved."""
    z, _ = _golden_tags()
    src = str(z[f"{tag}/inputs"])
    q, k, v, g = (z[f"{src}/{n}"] for n in "qkvg")
    causal, scale = z[f"{tag}/meta"]
    scale = None if np.isnan(scale) else float(scale)
    mask = z[f"{tag}/mask"] if f"{tag}/mask" in z.files else None
    print(f"[case] golden {tag}", flush=True)
    out, lse = _run_fwd(q, k, v, bool(causal), scale, mask)
    assert_f32(out, z[f"{tag}/out"], f"{tag} out")
    assert_f32(lse, z[f"{tag}/lse"], f"{tag} lse")
    got = _run_bwd(g, q, k, v, z[f"{tag}/out"], z[f"{tag}/lse"], bool(causal), scale, mask)
    for name, a in zip(("dq", "dk", "dv"), got):
        assert_f32(a, z[f"{tag}/{name}"], f"{tag} {name}")


def _misaligned(x):
    """A contiguous float32 device copy of x whose data pointer is 4 bytes past a 16-byte
    boundary."""
    x = np.ascontiguousarray(x, np.float32)
    flat = torch.empty(x.size + 4, dtype=torch.float32, device=DEV)
    view = flat[1:1 + x.size].view(x.shape)
    view.copy_(torch.from_numpy(x).to(DEV))
    assert view.data_ptr() % 16 != 0
    return view


@pytest.mark.parametrize("E", [32, 64, 128])
def test_unaligned_pointers(oracle_lib, E):
    """Inputs not 16-byte aligned take the element-wise load paths of the forward and backward
    kernels at head dims equal to the instantiated ones."""
    from densecore_amd import _native
    rng = np.random.default_rng(400 + E)
    q, k, v, g = (rng.standard_normal((1, 2, 150, E), dtype=np.float32) for _ in range(4))
    print(f"[case] fp32 unaligned E{E}", flush=True)
    ref_o, ref_l = oracle_lib.forward(q, k, v, True)
    out, lse = _native._flash_attention(_misaligned(q), _misaligned(k), _misaligned(v), True)
    torch.cuda.synchronize()
    assert_f32(out.cpu().numpy(), ref_o, "unaligned out")
    assert_f32(lse.cpu().numpy(), ref_l, "unaligned lse")
    ref = oracle_lib.backward(g, q, k, v, ref_o, ref_l, True)
    got = _native._flash_attention_backward(_misaligned(g), _misaligned(q), _misaligned(k),
                                            _misaligned(v), _misaligned(ref_o), _t(ref_l), True)
    torch.cuda.synchronize()
    for name, a, b in zip(("dq", "dk", "dv"), got, ref):
        assert_f32(a.cpu().numpy(), b, f"unaligned {name}")


@pytest.mark.parametrize("B,H,Hkv,L,S,causal,masked", [
    (1, 8, 8, 2048, 2048, True, False),    # stream-K ranges
    (8, 12, 12, 512, 512, True, False),    # whole tiles
    (2, 4, 2, 300, 700, True, False),      # grouped heads, keys past the queries
    (1, 2, 2, 700, 300, False, True),      # float mask, L > S
    (2, 3, 3, 190, 190, True, True),       # causal and a mask
])
def test_consistent_scores_backward(oracle_lib, B, H, Hkv, L, S, causal, masked):
    """DC_FLAG_CONSISTENT_SCORES at head dim 128 (the forward-ordered 4-wave backward tile): the
    float32 bar against the oracle, on the whole-tile and stream-K schedules, with grouped heads,
    L != S and masks; and the same results as the default tile to the bar."""
    from densecore_amd import _native
    rng = np.random.default_rng(B * 100 + H + L + S)
    q, g = (rng.standard_normal((B, H, L, 128), dtype=np.float32) for _ in range(2))
    k, v = (rng.standard_normal((B, Hkv, S, 128), dtype=np.float32) for _ in range(2))
    mask = None
    if masked:
        mask = rng.standard_normal((B, H, L, S)).astype(np.float32)
        mask[rng.random((B, H, L, S)) < 0.2] = -np.inf
    print(f"[case] consistent scores B{B} H{H} Hkv{Hkv} L{L} S{S} causal={causal} mask={masked}", flush=True)
    previous = _native.consistent_scores(True)
    try:
        _check(oracle_lib, q, k, v, g, causal, None, mask, tag="consistent")
    finally:
        _native.consistent_scores(previous)
