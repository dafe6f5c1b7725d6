"""GPU parity of the public drop-in path: ``functional.scaled_dot_product_attention`` with autograd.

The reference's users reach the flash kernels through ``scaled_dot_product_attention`` and the
``FlashAttention`` autograd function (``python/densecore/functional.py:276-388``); its own tests
drive exactly that (``tests/test_attention.py:12-39``: forward, ``.backward``, grads;
``tests/test_torch_api_f1.py:78-84``: ``enable_gqa=True``).  These cases do the same on the
GPU: leaf tensors with ``requires_grad``, one forward, ``out.backward(g)``, and out, q.grad,
k.grad, v.grad against the oracle run the way the reference runs them:

  * bool masks become 0 / -inf and are broadcast to (B, H, L, S) (``functional.py:343-364``);
  * ``enable_gqa`` widens K and V over the query heads first (``functional.py:287-297``), so the
    reference's dK / dV are the widened gradients summed over each kv head's query heads;
  * float32: the oracle's forward, then its backward from its own (out, lse), end to end, to
    |gpu - ref| <= 2e-5 + 1e-5 |ref|;
  * bf16 (new here; the reference's flash path is float32): the oracle on the exact float32
    upcast of the bf16 inputs; its backward takes the GPU's own out and lse, as the autograd
    node saved them (a bf16-rounded out changes dsum by ~2^-9 |dO||out|), to
    |gpu - ref| <= 1e-2 |ref| + 1e-2 rms(ref).

Every case asserts that the flash branch ran: ``out.grad_fn`` is the flash autograd node, and
the math path, its batched products (``dc_bmm``) and the device BLAS (``torch.matmul`` /
``torch.bmm``) are never entered.
"""
import numpy as np
import pytest

from tests._data import assert_bf16, assert_bf16_nan, assert_f32, assert_f32_nan, bf16_round

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu

DEV = "cuda:0"


@pytest.fixture
def flash_only(monkeypatch):
    """Fail the test if anything but the flash kernels would compute attention."""
    from densecore_amd import functional as F

    def boom(*args, **kwargs):
        raise AssertionError("the math path / device BLAS ran instead of the flash kernels")

    monkeypatch.setattr(F, "_math_attention", boom)
    monkeypatch.setattr(F._native, "_bmm", boom)
    monkeypatch.setattr(torch, "matmul", boom)
    monkeypatch.setattr(torch, "bmm", boom)
    return F


def _same_bits(a, b):
    """Equal element by element, NaN matching NaN (the reference's NaN rows)."""
    return a.shape == b.shape and bool(torch.equal(a.view(torch.int16) if a.dtype == torch.bfloat16 else a.view(torch.int32),
                                                  b.view(torch.int16) if b.dtype == torch.bfloat16 else b.view(torch.int32)))


def _leaf(x, dtype):
    return torch.from_numpy(np.ascontiguousarray(x)).to(DEV, dtype).requires_grad_(True)


def _reference(oracle, q, k, v, g, causal, scale, mask, out_gpu=None, lse_gpu=None):
    """The reference's result for (q, k, v) whose K / V already have H heads."""
    ref_o, ref_l = oracle.forward(q, k, v, causal, scale, mask)
    o_in, l_in = (ref_o, ref_l) if out_gpu is None else (out_gpu, lse_gpu)
    return ref_o, ref_l, oracle.backward(g, q, k, v, o_in, l_in, causal, scale, mask)


def _run(F, q, k, v, g, dtype, **kw):
    tq, tk, tv = _leaf(q, dtype), _leaf(k, dtype), _leaf(v, dtype)
    out = F.scaled_dot_product_attention(tq, tk, tv, **kw)
    assert type(out.grad_fn).__name__ == "_FlashAttentionBackward", type(out.grad_fn).__name__
    out.backward(torch.from_numpy(g).to(DEV, dtype))
    torch.cuda.synchronize()
    grads = [t.grad.float().cpu().numpy() for t in (tq, tk, tv)]
    return out, grads


def _mask_np(kind, rng, B, H, L, S):
    """(API mask as numpy, additive (B, H, L, S) float32 mask the reference's kernel receives)."""
    if kind is None:
        return None, None
    if kind == "bool2d":
        m = rng.random((L, S)) < 0.8
        m[min(3, L - 1)] = False  # one fully masked row: out 0, lse 0, zero gradients
    elif kind == "bool4d_padding":  # key padding, (B, 1, 1, S)
        lengths = rng.integers(1, S + 1, size=B)
        m = (np.arange(S)[None, :] < lengths[:, None])[:, None, None, :]
    elif kind == "float4d":
        m = rng.standard_normal((B, H, L, S)).astype(np.float32)
        m[rng.random((B, H, L, S)) < 0.25] = -np.inf
        m[0, 0, 0] = -np.inf  # a fully masked row
    elif kind == "float2d":
        m = rng.standard_normal((L, S)).astype(np.float32)
    else:
        raise ValueError(kind)
    add = np.where(m, np.float32(0), np.float32(-np.inf)) if m.dtype == np.bool_ else m
    return m, np.ascontiguousarray(np.broadcast_to(add, (B, H, L, S)), np.float32)


CASES = [  # tag, B, H, Hkv, L, S, E, causal, mask kind, scale, gqa
    ("causal", 2, 3, 3, 150, 150, 64, True, None, None, False),
    ("causal_scale", 2, 2, 2, 97, 97, 32, True, None, 0.3, False),
    ("plain_l_ne_s", 1, 4, 4, 70, 130, 64, False, None, None, False),
    ("bool2d_full_row", 2, 2, 2, 64, 96, 64, False, "bool2d", None, False),
    ("bool4d_padding", 3, 2, 2, 80, 200, 128, False, "bool4d_padding", None, False),
    ("float4d_holes", 1, 3, 3, 45, 77, 40, False, "float4d", 0.3, False),
    ("float2d", 2, 2, 2, 33, 65, 16, False, "float2d", None, False),
    ("gqa_causal", 2, 8, 2, 130, 130, 64, True, None, None, True),
    ("gqa_padding", 2, 6, 3, 64, 150, 128, False, "bool4d_padding", 0.3, True),
    # the reference scales its causal -inf fill: NaN rows (src/torch_attention.rs:202-216)
    ("causal_negative_scale", 1, 2, 2, 100, 100, 64, True, None, -0.4, False),
    ("causal_zero_scale", 2, 2, 2, 300, 300, 32, True, None, 0.0, False),
]


@pytest.mark.parametrize("dtype", ["f32", "bf16"])
@pytest.mark.parametrize("tag,B,H,Hkv,L,S,E,causal,mask,scale,gqa", CASES, ids=[c[0] for c in CASES])
def test_public_flash_autograd(oracle_lib, flash_only, dtype, tag, B, H, Hkv, L, S, E, causal, mask,
                               scale, gqa):
    bf16 = dtype == "bf16"
    rng = np.random.default_rng(sum(map(ord, tag)) + (7 if bf16 else 0))
    q = rng.standard_normal((B, H, L, E), dtype=np.float32)
    k = rng.standard_normal((B, Hkv, S, E), dtype=np.float32)
    v = rng.standard_normal((B, Hkv, S, E), dtype=np.float32)
    g = rng.standard_normal((B, H, L, E), dtype=np.float32)
    if bf16:
        q, k, v, g = (bf16_round(x) for x in (q, k, v, g))
    api_mask, add_mask = _mask_np(mask, rng, B, H, L, S)
    print(f"[case] public {dtype} {tag} B{B} H{H} Hkv{Hkv} L{L} S{S} E{E} causal={causal} "
          f"mask={mask} scale={scale} gqa={gqa}", flush=True)
    tdt = torch.bfloat16 if bf16 else torch.float32
    kw = {"is_causal": causal, "scale": scale, "enable_gqa": gqa}
    if api_mask is not None:
        kw["attn_mask"] = torch.from_numpy(api_mask).to(DEV)
    out, (dq, dk, dv) = _run(flash_only, q, k, v, g, tdt, **kw)

    # The reference widens K / V over the query heads (enable_gqa) before its kernel.
    rep = H // Hkv
    kw_, vw_ = np.repeat(k, rep, axis=1), np.repeat(v, rep, axis=1)
    if bf16:
        # The GPU's saved (out, lse), recomputed by the flash forward alone (the autograd node
        # saved the same tensors: the forward is deterministic).
        from densecore_amd import _native
        m = None if add_mask is None else torch.from_numpy(add_mask).to(DEV)
        o_gpu, l_gpu = _native._flash_attention(*(torch.from_numpy(x).to(DEV, tdt) for x in (q, k, v)),
                                                causal, scale, m)
        assert _same_bits(o_gpu, out.detach()), "bf16 forward is not deterministic"
        ref_o, ref_l, ref = _reference(oracle_lib, q, kw_, vw_, g, causal, scale, add_mask,
                                       o_gpu.float().cpu().numpy(), l_gpu.cpu().numpy())
    else:
        ref_o, ref_l, ref = _reference(oracle_lib, q, kw_, vw_, g, causal, scale, add_mask)
    rdq, rdk, rdv = ref
    if rep > 1:
        rdk = rdk.reshape(B, Hkv, rep, S, E).sum(axis=2)
        rdv = rdv.reshape(B, Hkv, rep, S, E).sum(axis=2)
    check = assert_bf16 if bf16 else assert_f32
    if scale is not None and not scale > 0:
        check = assert_bf16_nan if bf16 else assert_f32_nan
        assert np.isnan(ref_o).any()
    check(out.detach().float().cpu().numpy(), ref_o, f"{tag} out")
    for name, a, b in (("dq", dq, rdq), ("dk", dk, rdk), ("dv", dv, rdv)):
        check(a, b, f"{tag} {name}")


def test_public_c2_autograd(oracle_lib, flash_only):
    """C2 (causal fp32, B8 H12 T1024 D64) end to end through the public API and autograd."""
    from tests._data import make_inputs
    d = make_inputs("C2")
    print("[case] public C2 fp32 causal B8 H12 T1024 D64", flush=True)
    out, (dq, dk, dv) = _run(flash_only, d["q"], d["k"], d["v"], d["g"], torch.float32, is_causal=True)
    ref_o, _, (rdq, rdk, rdv) = _reference(oracle_lib, d["q"], d["k"], d["v"], d["g"], True, None, None)
    assert_f32(out.detach().cpu().numpy(), ref_o, "C2 out")
    for name, a, b in (("dq", dq, rdq), ("dk", dk, rdk), ("dv", dv, rdv)):
        assert_f32(a, b, f"C2 {name}")


def test_public_bool_mask_stays_on_device(flash_only):
    """The flash mask handed to the kernels is a device broadcast view of 0 / -inf (never a
    host copy, never materialised to (B, H, L, S)): ``_flash_mask`` (functional.py:343-364)."""
    F = flash_only
    m = torch.tensor([[True, False, True]], device=DEV)  # (1, 3): broadcast over B, H, L
    fm = F._flash_mask(m, (2, 4, 5, 3), 3, torch.device(DEV))
    assert fm.device.type == "cuda" and fm.dtype == torch.float32 and tuple(fm.shape) == (2, 4, 5, 3)
    assert fm.stride()[:3] == (0, 0, 0)
    assert fm[1, 3, 4].tolist() == [0.0, float("-inf"), 0.0]


@pytest.mark.parametrize("dtype", ["f32", "bf16"])
@pytest.mark.parametrize("B,T,H,D", [(2, 96, 4, 32), (3, 257, 6, 64), (1, 130, 2, 128)])
def test_public_transposed_views(oracle_lib, flash_only, dtype, B, T, H, D):
    """The reference's own consumer (examples/tiny_gpt.py:30-38) hands attention (B, T, H, D)
    projections viewed as (B, H, T, D) through .transpose(1, 2), is_causal=True.  The same views
    here, with autograd back to the (B, T, H * D) leaves: out and the leaves' gradients against the
    oracle on the contiguous (B, H, T, D) copies."""
    bf16 = dtype == "bf16"
    tdt = torch.bfloat16 if bf16 else torch.float32
    rng = np.random.default_rng(B * 1000 + T + H * D + (7 if bf16 else 0))
    x = [rng.standard_normal((B, T, H * D), dtype=np.float32) for _ in range(3)]
    g = rng.standard_normal((B, H, T, D), dtype=np.float32)
    if bf16:
        x, g = [bf16_round(a) for a in x], bf16_round(g)
    print(f"[case] public {dtype} transposed views B{B} T{T} H{H} D{D}", flush=True)
    leaves = [_leaf(a, tdt) for a in x]
    q, k, v = (t.reshape(B, T, H, D).transpose(1, 2) for t in leaves)
    assert not q.is_contiguous()
    out = flash_only.scaled_dot_product_attention(q, k, v, is_causal=True)
    assert type(out.grad_fn).__name__ == "_FlashAttentionBackward", type(out.grad_fn).__name__
    out.backward(torch.from_numpy(g).to(DEV, tdt))
    torch.cuda.synchronize()
    qn, kn, vn = (np.ascontiguousarray(a.reshape(B, T, H, D).transpose(0, 2, 1, 3)) for a in x)
    if bf16:
        from densecore_amd import _native
        o_gpu, l_gpu = _native._flash_attention(*(torch.from_numpy(a).to(DEV, tdt) for a in (qn, kn, vn)), True)
        assert _same_bits(o_gpu, out.detach()), "bf16 forward differs on a transposed view"
        ref_o, _, ref = _reference(oracle_lib, qn, kn, vn, g, True, None, None,
                                   o_gpu.float().cpu().numpy(), l_gpu.cpu().numpy())
    else:
        ref_o, _, ref = _reference(oracle_lib, qn, kn, vn, g, True, None, None)
    check = assert_bf16 if bf16 else assert_f32
    check(out.detach().float().cpu().numpy(), ref_o, "transposed out")
    for name, leaf, r in zip(("dq", "dk", "dv"), leaves, ref):
        got = leaf.grad.float().cpu().numpy().reshape(B, T, H, D).transpose(0, 2, 1, 3)
        check(got, r, f"transposed {name}")
