"""GPU parity of the composed ("math") attention path: the softmax kernels through the C ABI
against the oracle's softmax_lastdim / softmax_backward_lastdim, the math path of
scaled_dot_product_attention against the oracle's composition of the reference's ops
(python/densecore/functional.py:318-340), and multi_head_attention_forward against torch's own
reference algorithm in float64 on the CPU (the algorithm functional.py:400-461 restates).

Tolerance (written here, the target's): |gpu - ref| <= 2e-5 + 1e-5 |ref| elementwise for every
float32 output and gradient.
"""
import math

import numpy as np
import pytest

import oracle
from tests._data import assert_f32

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu

DEV = "cuda:0"
RNG = np.random.default_rng(2024)


def _t(x, requires_grad=False):
    t = torch.from_numpy(np.ascontiguousarray(x)).to(DEV)
    return t.requires_grad_(requires_grad)


def _np(t):
    torch.cuda.synchronize()
    return t.detach().cpu().numpy()


@pytest.mark.parametrize("width", [1, 3, 4, 5, 63, 64, 65, 255, 256, 257, 1000, 1024, 2047, 4096,
                                   4097, 9000])
def test_softmax_widths(width):
    from densecore_amd import _native
    print(f"[case] softmax width={width}", flush=True)
    rows = 37
    x = (RNG.standard_normal((rows, width)) * 3).astype(np.float32)
    y = _np(_native._softmax(_t(x)))
    ref = oracle.softmax(x)
    assert_f32(y, ref, f"softmax w{width}")
    g = RNG.standard_normal((rows, width)).astype(np.float32)
    dx = _np(_native._softmax_backward(_t(g), _t(ref)))
    assert_f32(dx, oracle.softmax_backward(g, ref), f"softmax backward w{width}")


@pytest.mark.parametrize("width", [8, 300, 6000])
def test_softmax_unaligned_rows(width):
    """Storage offset by one element: rows are not 16-byte aligned (the 4-byte load path)."""
    from densecore_amd import _native
    print(f"[case] softmax unaligned width={width}", flush=True)
    x = (RNG.standard_normal((9, width)) * 2).astype(np.float32)
    buf = _t(np.concatenate([[0.0], x.ravel()]).astype(np.float32))
    xv = buf[1:].view(9, width)
    assert xv.data_ptr() % 16 != 0
    assert_f32(_np(_native._softmax(xv)), oracle.softmax(x), "unaligned softmax")


@pytest.mark.parametrize("mshape", [(2, 1, 1, 40), (1, 1, 7, 40), (2, 3, 7, 40), (7, 40),
                                    (2, 3, 7, 1), (2, 1, 7, 41)])
@pytest.mark.parametrize("safe", [False, True])
def test_softmax_masks(mshape, safe):
    """Broadcast masks are read through strides; safe rows that are all -inf give 0."""
    from densecore_amd import _native
    print(f"[case] softmax mask {mshape} safe={safe}", flush=True)
    S = mshape[-1] if mshape[-1] != 1 else 40
    shape = (2, 3, 7, S)
    x = RNG.standard_normal(shape).astype(np.float32)
    m = np.where(RNG.random(mshape) < 0.3, -np.inf, RNG.standard_normal(mshape)).astype(np.float32)
    if len(mshape) == 4 and mshape[-2] == 7 and mshape[-1] != 1:
        m[(0,) * (len(mshape) - 2) + (2,)] = -np.inf  # a fully masked row
    y = _np(_native._softmax(_t(x), _t(m), safe))
    s = x + np.broadcast_to(m, shape)
    empty = np.isneginf(s).all(-1, keepdims=True)
    if safe:
        ref = np.where(empty, np.float32(0), oracle.softmax(np.where(empty, np.float32(0), s)))
        assert_f32(y, ref, "masked softmax")
    else:
        ref = oracle.softmax(s)
        assert np.array_equal(np.isnan(y), np.isnan(ref))
        ok = ~np.isnan(ref)
        assert_f32(y[ok], ref[ok], "masked softmax")


def test_softmax_special_rows():
    from densecore_amd import _native
    x = np.array([[0.0, np.nan, 1.0, 2.0], [np.inf, 0.0, 1.0, 2.0], [0.0, -np.inf, 0.0, -np.inf],
                  [-np.inf] * 4], np.float32)
    y = _np(_native._softmax(_t(x)))
    assert np.isnan(y[0]).all() and np.isnan(y[1]).all() and np.isnan(y[3]).all()
    assert np.array_equal(y[2], np.array([0.5, 0.0, 0.5, 0.0], np.float32))


def _sdpa_case(case):
    B, H, L, S, E, Ev = 2, 3, 37, 45, 32, 32
    mask, causal = None, False
    if case == "ev":
        Ev = 48
    q = RNG.standard_normal((B, H, L, E)).astype(np.float32)
    k = RNG.standard_normal((B, H, S, E)).astype(np.float32)
    v = RNG.standard_normal((B, H, S, Ev)).astype(np.float32)
    g = RNG.standard_normal((B, H, L, Ev)).astype(np.float32)
    if case == "rank3":
        q, k, v, g = q[0], k[0], v[0], g[0]
    if case == "mask3d":  # a 3-D (H, L, S) bool mask: the flash path takes only 2-D or 4-D
        mask = RNG.random((H, L, S)) < 0.7
        mask[1, 4] = False
    if case == "ev":
        mask = np.where(RNG.random((L, S)) < 0.8, 0.0, -np.inf).astype(np.float32)
    if case == "ev_causal":
        v = RNG.standard_normal((B, H, S, 40)).astype(np.float32)
        g = RNG.standard_normal((B, H, L, 40)).astype(np.float32)
        causal = True
    return q, k, v, g, mask, causal


@pytest.mark.parametrize("case", ["rank3", "mask3d", "ev", "ev_causal"])
def test_math_path_against_oracle(case):
    from densecore_amd.functional import scaled_dot_product_attention
    print(f"[case] math path {case}", flush=True)
    q, k, v, g, mask, causal = _sdpa_case(case)
    tq, tk, tv = _t(q, True), _t(k, True), _t(v, True)
    out = scaled_dot_product_attention(tq, tk, tv, attn_mask=None if mask is None else _t(mask),
                                       is_causal=causal)
    out.backward(_t(g))
    ref_out, (dq, dk, dv, _) = oracle.math_attention(q, k, v, attn_mask=mask, is_causal=causal,
                                                     grad_out=g)
    assert_f32(_np(out), ref_out, f"{case} out")
    for name, t, ref in (("dq", tq, dq), ("dk", tk, dk), ("dv", tv, dv)):
        assert_f32(_np(t.grad), ref, f"{case} {name}")


def test_math_path_float_mask_gradient():
    """A float mask that requires a gradient takes the math path and receives dS summed over
    its broadcast dims."""
    from densecore_amd.functional import scaled_dot_product_attention
    B, H, L, S, E = 2, 2, 19, 23, 16
    q, k, v, g = (RNG.standard_normal(s).astype(np.float32)
                  for s in ((B, H, L, E), (B, H, S, E), (B, H, S, E), (B, H, L, E)))
    m = RNG.standard_normal((1, H, L, S)).astype(np.float32)
    tq, tk, tv, tm = _t(q, True), _t(k, True), _t(v, True), _t(m, True)
    out = scaled_dot_product_attention(tq, tk, tv, attn_mask=tm)
    out.backward(_t(g))
    ref_out, (dq, dk, dv, da) = oracle.math_attention(q, k, v, attn_mask=m, grad_out=g)
    assert_f32(_np(out), ref_out, "out")
    assert_f32(_np(tq.grad), dq, "dq")
    assert_f32(_np(tm.grad), da.sum(0, keepdims=True), "dmask")


def _mha_inputs(L, S, N, E, kdim=None, vdim=None):
    q = RNG.standard_normal((L, N, E)).astype(np.float32)
    k = RNG.standard_normal((S, N, kdim or E)).astype(np.float32)
    v = RNG.standard_normal((S, N, vdim or E)).astype(np.float32)
    return q, k, v


MHA_CASES = ["plain", "key_padding", "bool_mask", "bias_kv", "zero_attn", "kvdim", "unbatched",
             "per_head_weights"]


@pytest.mark.parametrize("case", MHA_CASES)
def test_multi_head_attention_against_torch_float64(case):
    from densecore_amd import nn
    F = torch.nn.functional
    print(f"[case] mha {case}", flush=True)
    E, heads, L, S, N = 64, 4, 13, 17, 3
    kdim = vdim = None
    if case == "kvdim":
        kdim, vdim = 40, 24
    torch.manual_seed(0)
    mod = nn.MultiheadAttention(E, heads, bias=True, add_bias_kv=case == "bias_kv",
                                add_zero_attn=case == "zero_attn", kdim=kdim, vdim=vdim)
    with torch.no_grad():
        mod.out_proj.bias.normal_()
        if mod.in_proj_bias is not None:
            mod.in_proj_bias.normal_()
    q, k, v = _mha_inputs(L, S, N, E, kdim, vdim)
    kpm = am = None
    if case == "key_padding":
        kpm = RNG.random((N, S)) < 0.3
        kpm[:, 0] = False
    if case == "bool_mask":
        am = RNG.random((L, S)) < 0.3
        am[:, 0] = False
    avg = case != "per_head_weights"
    if case == "unbatched":
        q, k, v = q[:, 0], k[:, 0], v[:, 0]
    tq, tk, tv = _t(q, True), _t(k, True), _t(v, True)
    out, w = mod(tq, tk, tv, key_padding_mask=None if kpm is None else _t(kpm),
                 attn_mask=None if am is None else _t(am), average_attn_weights=avg)
    go = RNG.standard_normal(tuple(out.shape)).astype(np.float32)
    out.backward(_t(go))
    # torch's reference algorithm in float64 on the CPU with the same parameters.
    P = {n: p.detach().cpu().double().requires_grad_(True) for n, p in mod.named_parameters()}
    cq, ck, cv = (torch.tensor(x, dtype=torch.float64, requires_grad=True) for x in (q, k, v))
    sep = not mod._qkv_same_embed_dim
    ref_out, ref_w = F.multi_head_attention_forward(
        cq, ck, cv, E, heads, P.get("in_proj_weight"), P.get("in_proj_bias"), P.get("bias_k"),
        P.get("bias_v"), mod.add_zero_attn, 0.0, P["out_proj.weight"], P["out_proj.bias"],
        training=False, key_padding_mask=None if kpm is None else torch.tensor(kpm),
        need_weights=True, attn_mask=None if am is None else torch.tensor(am),
        use_separate_proj_weight=sep, q_proj_weight=P.get("q_proj_weight"),
        k_proj_weight=P.get("k_proj_weight"), v_proj_weight=P.get("v_proj_weight"),
        average_attn_weights=avg)
    ref_out.backward(torch.tensor(go, dtype=torch.float64))
    assert_f32(_np(out), ref_out.detach().numpy(), f"mha {case} out")
    assert_f32(_np(w), ref_w.detach().numpy(), f"mha {case} weights")
    for name, t, r in (("dq", tq, cq), ("dk", tk, ck), ("dv", tv, cv)):
        assert_f32(_np(t.grad), r.grad.numpy(), f"mha {case} {name}")
    for n, p in mod.named_parameters():
        assert_f32(_np(p.grad), P[n].grad.numpy(), f"mha {case} grad {n}")


def test_multi_head_attention_batch_first_and_no_weights():
    from densecore_amd import nn
    torch.manual_seed(1)
    mod = nn.MultiheadAttention(32, 2, batch_first=True)
    x = RNG.standard_normal((3, 11, 32)).astype(np.float32)
    out, w = mod(_t(x), _t(x), _t(x), need_weights=False)
    assert w is None and tuple(out.shape) == (3, 11, 32)
    mod.batch_first = False
    ref, _ = mod(_t(x).transpose(0, 1), _t(x).transpose(0, 1), _t(x).transpose(0, 1))
    assert_f32(_np(out), _np(ref.transpose(0, 1)), "batch_first")


@pytest.mark.parametrize("shape", [
    ((0, 2, 5, 4), (0, 2, 6, 4), (0, 2, 6, 3)),   # B = 0
    ((2, 3, 0, 4), (2, 3, 6, 4), (2, 3, 6, 3)),   # L = 0
    ((2, 3, 5, 0), (2, 3, 6, 0), (2, 3, 6, 3)),   # E = 0: scores are 0, out = mean of v
    ((2, 5, 0), (2, 7, 0), (2, 7, 4)),            # rank 3, E = 0
])
@pytest.mark.parametrize("causal", [False, True])
def test_math_path_empty_dims(shape, causal):
    """Shapes with a zero length, batch or head dim go to the math path (the reference's flash
    predicate needs L, S and E non-zero, functional.py:310-312), and its products accept them:
    out has the query's leading shape and v's last dim; with E = 0 every score is 0, so out is the
    mean of v over the keys each row sees, and the gradients follow."""
    from densecore_amd import functional as F
    qs, ks, vs = shape
    print(f"[case] math path empty dims q{qs} k{ks} v{vs} causal={causal}", flush=True)
    q, k, v = (RNG.standard_normal(s).astype(np.float32) for s in (qs, ks, vs))
    tq, tk, tv = _t(q, True), _t(k, True), _t(v, True)
    out = F.scaled_dot_product_attention(tq, tk, tv, is_causal=causal)
    assert tuple(out.shape) == qs[:-1] + vs[-1:]
    L, S = qs[-2], ks[-2]
    allowed = np.tril(np.ones((L, S), bool)) if causal else np.ones((L, S), bool)
    w = allowed / np.maximum(allowed.sum(-1, keepdims=True), 1)
    if qs[-1] == 0 and out.numel():
        assert_f32(_np(out), np.matmul(w, v).astype(np.float32), "E = 0 out")
    g = RNG.standard_normal(tuple(out.shape)).astype(np.float32)
    out.backward(_t(g))
    for t, s in ((tq, qs), (tk, ks), (tv, vs)):
        assert t.grad is not None and tuple(t.grad.shape) == s
    if qs[-1] == 0 and out.numel():
        assert_f32(_np(tv.grad), np.matmul(np.swapaxes(w, -1, -2), g).astype(np.float32), "E = 0 dv")


@pytest.mark.parametrize("kw", [dict(), dict(bias=False), dict(add_bias_kv=True), dict(kdim=40, vdim=24),
                                dict(add_zero_attn=True, batch_first=True)])
def test_multi_head_attention_parameters_as_torch(kw):
    """The module's parameters are torch.nn.MultiheadAttention's: the same names and shapes for
    the same arguments, and its initial rules (zero projection biases, xavier-scaled weights)."""
    from densecore_amd import nn
    E, heads = 64, 4
    ours = nn.MultiheadAttention(E, heads, **kw)
    theirs = torch.nn.MultiheadAttention(E, heads, device=DEV, **kw)
    got = {n: tuple(p.shape) for n, p in ours.named_parameters()}
    want = {n: tuple(p.shape) for n, p in theirs.named_parameters()}
    assert got == want
    if kw.get("bias", True):
        assert not ours.in_proj_bias.any() and not ours.out_proj.bias.any()
    for n, p in ours.named_parameters():
        if n.endswith("proj_weight"):  # xavier-uniform: |w| <= sqrt(6 / (fan_in + fan_out))
            bound = (6.0 / (p.shape[0] + p.shape[1])) ** 0.5
            assert float(p.abs().max()) <= bound and float(p.abs().max()) > 0.5 * bound, n
