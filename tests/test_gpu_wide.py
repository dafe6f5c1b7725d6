"""GPU parity at head dims above 128 (the reference's kernels take any head dim,
src/torch_attention.rs:150-171, 300-320).

The float32 flash kernels instantiate head dims up to 128 and the bf16 ones up to 256; wider heads
run materialized over blocks of query rows (scores through dc_bmm's MFMA kernel, row kernels for
the softmax, P and dS), and decode up to 256 runs its split-KV kernel.  So the bf16 cases up to 256
here run the flash kernels (their own tests: tests/test_gpu_bf16.py) and the rest materialized.  Each case is checked against the oracle: float32 to
|gpu - ref| <= 2e-5 + 1e-5 |ref|; bf16 (the oracle on the exact float32 upcast, its backward from
the GPU's own bf16 out and lse) to |gpu - ref| <= 1e-2 |ref| + 1e-2 rms(ref).  Outputs start as
NaN, so a row no block writes fails.
"""
import ctypes

import numpy as np
import pytest

from tests._data import assert_bf16, assert_f32, bf16_round

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu

DEV = "cuda:0"


def _t(x, dtype=torch.float32):
    return torch.from_numpy(np.ascontiguousarray(x)).to(DEV, dtype)


def _fwd(q, k, v, causal, mask, ws_bytes=None):
    from densecore_amd import _lib, _native
    dims = _native._attention_dims(q, k, v)
    B, H, _, L, _, E = dims
    m, ms = _native._mask_arg(mask, dims, q.device)
    d = _native._desc(dims, causal, None, q.dtype, ms)
    L_ = _lib.lib()
    full = L_.dc_sdpa_fwd_workspace_size(ctypes.byref(d))
    nbytes = full if ws_bytes is None else ws_bytes
    ws = torch.empty(max(nbytes, 1), dtype=torch.uint8, device=DEV)
    out = torch.full((B, H, L, E), float("nan"), device=DEV, dtype=q.dtype)
    lse = torch.full((B, H, L), float("nan"), device=DEV)
    sched = _native._schedule(False, q, k, v, causal, mask=m, workspace_bytes=nbytes)
    _lib.check(L_.dc_sdpa_fwd(d, _native._ptr(q), _native._ptr(k), _native._ptr(v), _native._ptr(m),
                              _native._ptr(out), _native._ptr(lse), _native._ptr(ws), nbytes,
                              _native._stream(q.device)))
    torch.cuda.synchronize()
    return out, lse, sched


def _bwd(g, q, k, v, out, lse, causal, mask, ws_bytes=None):
    from densecore_amd import _lib, _native
    dims = _native._attention_dims(q, k, v)
    B, H, Hkv, L, S, E = dims
    m, ms = _native._mask_arg(mask, dims, q.device)
    d = _native._desc(dims, causal, None, q.dtype, ms)
    L_ = _lib.lib()
    nbytes = L_.dc_sdpa_bwd_workspace_size(ctypes.byref(d)) if ws_bytes is None else ws_bytes
    ws = torch.full((max(nbytes, 4) // 4,), float("nan"), device=DEV)
    dq = torch.full((B, H, L, E), float("nan"), device=DEV, dtype=q.dtype)
    dk = torch.full((B, Hkv, S, E), float("nan"), device=DEV, dtype=q.dtype)
    dv = torch.full((B, Hkv, S, E), float("nan"), device=DEV, dtype=q.dtype)
    sched = _native._schedule(True, q, k, v, causal, mask=m, workspace_bytes=nbytes)
    _lib.check(L_.dc_sdpa_bwd(d, _native._ptr(g), _native._ptr(q), _native._ptr(k), _native._ptr(v),
                              _native._ptr(out), _native._ptr(lse), _native._ptr(m), _native._ptr(dq),
                              _native._ptr(dk), _native._ptr(dv), _native._ptr(ws), nbytes,
                              _native._stream(q.device)))
    torch.cuda.synchronize()
    return (dq, dk, dv), sched


def _np(t):
    return t.float().cpu().numpy()


CASES = [  # tag, B, H, Hkv, L, S, E, causal, mask
    ("e160_causal", 2, 4, 2, 300, 300, 160, True, None),
    ("e192_full", 2, 3, 3, 130, 257, 192, False, None),
    ("e256_causal", 1, 4, 4, 333, 333, 256, True, None),
    ("e256_float_mask", 2, 2, 1, 97, 150, 256, False, "float"),
    ("e256_padding", 3, 2, 2, 64, 200, 256, False, "padding"),
    ("e320_causal_l_gt_s", 1, 2, 2, 200, 120, 320, True, None),
    ("e129_few_keys", 2, 2, 2, 40, 5, 129, False, None),  # (one key makes dq pure rounding noise)
]


@pytest.mark.parametrize("dtype", ["f32", "bf16"])
@pytest.mark.parametrize("tag,B,H,Hkv,L,S,E,causal,mask", CASES, ids=[c[0] for c in CASES])
def test_wide_forward_backward(oracle_lib, dtype, tag, B, H, Hkv, L, S, E, causal, mask):
    bf16 = dtype == "bf16"
    rng = np.random.default_rng(sum(map(ord, tag)) + (5 if bf16 else 0))
    q, g = (rng.standard_normal((B, H, L, E), dtype=np.float32) for _ in range(2))
    k, v = (rng.standard_normal((B, Hkv, S, E), dtype=np.float32) for _ in range(2))
    if bf16:
        q, k, v, g = (bf16_round(x) for x in (q, k, v, g))
    mk = tm = None
    if mask == "float":
        mk = rng.standard_normal((B, H, L, S), dtype=np.float32)
        mk[rng.random((B, H, L, S)) < 0.25] = -np.inf
        mk[0, 0, 1] = -np.inf  # a fully masked row: out 0, lse 0, zero gradients
        tm = _t(mk)
    elif mask == "padding":
        lengths = rng.integers(1, S + 1, size=B)
        mk = np.where(np.arange(S)[None, :] < lengths[:, None], np.float32(0), np.float32(-np.inf))
        tm = _t(mk[:, None, None, :]).expand(B, H, L, S)  # a broadcast view, never materialised
        mk = np.ascontiguousarray(np.broadcast_to(mk[:, None, None, :], (B, H, L, S)))
    print(f"[case] wide {dtype} {tag} B{B} H{H} Hkv{Hkv} L{L} S{S} E{E} causal={causal} mask={mask}", flush=True)
    tdt = torch.bfloat16 if bf16 else torch.float32
    tq, tk, tv, tg = (_t(x, tdt) for x in (q, k, v, g))
    out, lse, sched = _fwd(tq, tk, tv, causal, tm)
    rows = 0 if bf16 and E <= 256 else (H // Hkv) * L  # bf16 up to 256: the flash kernels
    assert sched["materialized_rows"] == rows, sched
    ref_o, ref_l = oracle_lib.forward(q, k, v, causal, None, mk)
    check = assert_bf16 if bf16 else assert_f32
    check(_np(out), ref_o, f"{tag} out")
    check(_np(lse), ref_l, f"{tag} lse")
    o_in, l_in = (_np(out), _np(lse)) if bf16 else (ref_o, ref_l)
    (dq, dk, dv), bs = _bwd(tg, tq, tk, tv, out if bf16 else _t(ref_o), lse if bf16 else _t(ref_l), causal, tm)
    assert bs["materialized_rows"] == rows and bs["deterministic"] == 1, bs
    ref = oracle_lib.backward(g, q, k, v, o_in, l_in, causal, None, mk)
    for name, a, b in zip(("dq", "dk", "dv"), (dq, dk, dv), ref):
        check(_np(a), b, f"{tag} {name}")


@pytest.mark.parametrize("dtype", ["f32", "bf16"])
def test_wide_small_workspace_row_blocks(oracle_lib, dtype):
    """A workspace that holds a few rows of scores per kv head: many row blocks, the same results
    (to the bar) and bit-identical from run to run."""
    from densecore_amd import _lib, _native
    bf16 = dtype == "bf16"
    B, H, Hkv, L, S, E, causal = 2, 4, 2, 150, 150, 320 if bf16 else 192, True  # bf16: above its flash 256
    rng = np.random.default_rng(192 + bf16)
    q, g = (rng.standard_normal((B, H, L, E), dtype=np.float32) for _ in range(2))
    k, v = (rng.standard_normal((B, Hkv, S, E), dtype=np.float32) for _ in range(2))
    if bf16:
        q, k, v, g = (bf16_round(x) for x in (q, k, v, g))
    tdt = torch.bfloat16 if bf16 else torch.float32
    tq, tk, tv, tg = (_t(x, tdt) for x in (q, k, v, g))
    d = _native._desc(_native._attention_dims(tq, tk, tv), causal, None, tdt, (0, 0, 0))
    L_ = _lib.lib()
    row = B * Hkv * S * 4  # one row of scores for every (batch, kv head)
    fwd_small = L_.dc_sdpa_fwd_workspace_size(ctypes.byref(d)) - (2 * L - 7) * row
    bwd_small = L_.dc_sdpa_bwd_workspace_size(ctypes.byref(d)) - 2 * (2 * L - 7) * row
    print(f"[case] wide {dtype} small workspace: 7 rows per block", flush=True)
    out, lse, sched = _fwd(tq, tk, tv, causal, None, fwd_small)
    assert 1 <= sched["materialized_rows"] <= 8, sched
    ref_o, ref_l = oracle_lib.forward(q, k, v, causal)
    check = assert_bf16 if bf16 else assert_f32
    check(_np(out), ref_o, "out (row blocks)")
    check(_np(lse), ref_l, "lse (row blocks)")
    o_in, l_in = (out, lse) if bf16 else (_t(ref_o), _t(ref_l))
    first, bs = _bwd(tg, tq, tk, tv, o_in, l_in, causal, None, bwd_small)
    second, _ = _bwd(tg, tq, tk, tv, o_in, l_in, causal, None, bwd_small)
    assert 1 <= bs["materialized_rows"] <= 8, bs
    for name, a, b in zip(("dq", "dk", "dv"), first, second):
        assert torch.equal(a, b), f"{name}: runs differ"
    ref = oracle_lib.backward(g, q, k, v, _np(o_in), _np(l_in), causal)
    for name, a, b in zip(("dq", "dk", "dv"), first, ref):
        check(_np(a), b, f"{name} (row blocks)")


@pytest.mark.parametrize("E", [192, 256, 300])
@pytest.mark.parametrize("dtype", ["f32", "bf16"])
def test_wide_decode(oracle_lib, E, dtype):
    """Decode at head dims above 128: the split-KV kernel up to 256, materialized above."""
    from densecore_amd import _native
    bf16 = dtype == "bf16"
    B, H, Hkv, S = 3, 8, 2, 1000
    rng = np.random.default_rng(E + 17 * bf16)
    q = rng.standard_normal((B, H, 1, E), dtype=np.float32)
    k, v = (rng.standard_normal((B, Hkv, S, E), dtype=np.float32) * np.float32(0.5) for _ in range(2))
    if bf16:
        q, k, v = (bf16_round(x) for x in (q, k, v))
    print(f"[case] wide decode {dtype} E{E}", flush=True)
    tdt = torch.bfloat16 if bf16 else torch.float32
    out, lse = _native._flash_decode(_t(q, tdt), _t(k, tdt), _t(v, tdt))
    torch.cuda.synchronize()
    ref_o, ref_l = oracle_lib.forward(q, k, v, False)
    check = assert_bf16 if bf16 else assert_f32
    check(_np(out), ref_o, f"decode E{E} out")
    check(_np(lse), ref_l, f"decode E{E} lse")


def test_wide_public_autograd(oracle_lib):
    """E = 256 through functional.scaled_dot_product_attention and autograd (the flash autograd
    node: the materialized path sits behind the same entry points)."""
    from densecore_amd import functional as F
    rng = np.random.default_rng(256)
    B, H, L, E = 2, 3, 120, 256
    q, k, v, g = (rng.standard_normal((B, H, L, E), dtype=np.float32) for _ in range(4))
    tq, tk, tv = (_t(x).requires_grad_(True) for x in (q, k, v))
    out = F.scaled_dot_product_attention(tq, tk, tv, is_causal=True)
    assert type(out.grad_fn).__name__ == "_FlashAttentionBackward"
    out.backward(_t(g))
    torch.cuda.synchronize()
    ref_o, ref_l = oracle_lib.forward(q, k, v, True)
    ref = oracle_lib.backward(g, q, k, v, ref_o, ref_l, True)
    assert_f32(_np(out.detach()), ref_o, "public E256 out")
    for name, t, r in zip(("dq", "dk", "dv"), (tq, tk, tv), ref):
        assert_f32(_np(t.grad), r, f"public E256 {name}")
