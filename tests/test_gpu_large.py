"""Tensors of more than 2^31 elements (each dimension still below 2^31): 64-bit offsets everywhere.

The reference sizes nothing by 32-bit products (src/torch_attention.rs indexes with usize), so a
key / value cache of B * Hkv * S * E > 2^31 elements is valid input.  Here K and V hold 16 heads of
1,048,640 keys x 128 dims (2,147,614,720 elements, 4.3 GB in bf16, 8.6 GB in float32), and the
last head's rows start 2.01e9 elements in, so its reads and its dK / dV writes cross the 2^31
element (and, for float32, byte) offsets.  The forward, the backward and, for bf16, the fp16
copies of K and V all address it.  The reference for that head is exact arithmetic (float64 NumPy
on the same inputs): out and lse of every query, dQ of every query, dK and dV of the first and the
last 2048 keys, and the decode entry's out and lse for the first query.  The bar is loose (1e-2
|ref| + 1e-2 rms(ref) for bf16, 1e-4 for float32, whose sums run over a million keys): an offset
error gives wrong rows, not rounding.
"""
import numpy as np
import pytest

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu

DEV = "cuda:0"
B, H, L, S, E = 1, 16, 64, (1 << 20) + 64, 128


def _check(got, ref, rel, name):
    got, ref = np.asarray(got, np.float64), np.asarray(ref, np.float64)
    rms = float(np.sqrt(np.mean(ref ** 2)))
    err = np.abs(got - ref)
    bad = ~(err <= rel * np.abs(ref) + rel * rms)
    assert not bad.any(), (f"{name}: {int(bad.sum())} of {bad.size} elements outside {rel}|ref| + {rel} rms "
                           f"(max err {float(np.nanmax(err)):.3e}, rms {rms:.3e})")


@pytest.mark.parametrize("dtype", ["bf16", "f32"])
def test_kv_over_2_31_elements(dtype):
    from densecore_amd import _native
    assert B * H * S * E > 1 << 31 and (H - 1) * S * E + S * E > 1 << 31
    dt = torch.bfloat16 if dtype == "bf16" else torch.float32
    rel = 1e-2 if dtype == "bf16" else 1e-4
    print(f"[case] large K/V {dtype} B{B} H{H} L{L} S{S} E{E} non-causal", flush=True)
    gen = torch.Generator(device=DEV).manual_seed(231)
    q = torch.randn(B, H, L, E, device=DEV, generator=gen, dtype=dt)
    g = torch.randn(B, H, L, E, device=DEV, generator=gen, dtype=dt)
    k = torch.randn(B, H, S, E, device=DEV, generator=gen, dtype=dt)
    v = torch.randn(B, H, S, E, device=DEV, generator=gen, dtype=dt)
    try:
        if dtype == "f32":  # the deterministic slots (4.3 GB) exceed the bound: pieces of kv heads
            assert _native._schedule(True, q, k, v, False)["chunks"] > 1
        out, lse = _native._flash_attention(q, k, v, False)
        dq, dk, dv = _native._flash_attention_backward(g, q, k, v, out, lse, False)
        torch.cuda.synchronize()

        hh = H - 1  # the head whose rows cross the 2^31 offsets
        f64 = lambda t: t[0, hh].float().cpu().numpy().astype(np.float64)
        qh, gh, kh, vh = f64(q), f64(g), f64(k), f64(v)
        scale = 1.0 / np.sqrt(E)
        s = (qh @ kh.T) * scale                       # (L, S)
        m = s.max(axis=1, keepdims=True)
        p = np.exp(s - m)
        lsum = p.sum(axis=1, keepdims=True)
        ref_out = (p @ vh) / lsum
        ref_lse = (m + np.log(lsum))[:, 0]
        _check(out[0, hh].float().cpu().numpy(), ref_out, rel, "out")
        _check(lse[0, hh].cpu().numpy(), ref_lse, rel, "lse")

        # The backward differentiates the GPU's own forward (its out and lse), as the reference's
        # backward takes what its forward saved.
        oh = out[0, hh].float().cpu().numpy().astype(np.float64)
        lh = lse[0, hh].cpu().numpy().astype(np.float64)
        p = np.exp(s - lh[:, None])
        dsum = (gh * oh).sum(axis=1, keepdims=True)
        ds = p * (gh @ vh.T - dsum)
        _check(dq[0, hh].float().cpu().numpy(), scale * (ds @ kh), rel, "dq")
        keys = np.r_[0:2048, S - 2048:S]
        _check(dk[0, hh, keys].float().cpu().numpy(), scale * (ds[:, keys].T @ qh), rel, "dk")
        _check(dv[0, hh, keys].float().cpu().numpy(), p[:, keys].T @ gh, rel, "dv")

        # Decode (one query per head) over the same cache: the split-KV kernels' reads of the last
        # head cross the same offsets.
        print(f"[case] large K/V decode {dtype}", flush=True)
        q1 = q[:, :, :1].contiguous()
        out1, lse1 = _native._flash_decode(q1, k, v)
        torch.cuda.synchronize()
        _check(out1[0, hh, 0].float().cpu().numpy(), ref_out[0], rel, "decode out")
        _check(lse1[0, hh, 0].cpu().numpy(), ref_lse[:1], rel, "decode lse")
    finally:
        del q, g, k, v
        _native.release_workspaces()
        torch.cuda.empty_cache()


LQ, SQ = (1 << 20) + 64, 64


@pytest.mark.parametrize("dtype", ["bf16", "f32"])
def test_q_over_2_31_elements(dtype):
    """The query side: Q, dO, out and dQ of 16 heads x 1,048,640 queries x 128 dims (more than 2^31
    elements) over 64 keys, non-causal; the last head checked in float64 NumPy (out, lse and dQ of
    every query, dK and dV of every key)."""
    from densecore_amd import _native
    assert B * H * LQ * E > 1 << 31
    dt = torch.bfloat16 if dtype == "bf16" else torch.float32
    rel = 1e-2 if dtype == "bf16" else 1e-4
    print(f"[case] large Q {dtype} B{B} H{H} L{LQ} S{SQ} E{E} non-causal", flush=True)
    gen = torch.Generator(device=DEV).manual_seed(232)
    q = torch.randn(B, H, LQ, E, device=DEV, generator=gen, dtype=dt)
    g = torch.randn(B, H, LQ, E, device=DEV, generator=gen, dtype=dt)
    k = torch.randn(B, H, SQ, E, device=DEV, generator=gen, dtype=dt)
    v = torch.randn(B, H, SQ, E, device=DEV, generator=gen, dtype=dt)
    try:
        out, lse = _native._flash_attention(q, k, v, False)
        dq, dk, dv = _native._flash_attention_backward(g, q, k, v, out, lse, False)
        torch.cuda.synchronize()

        hh = H - 1
        f64 = lambda t: t[0, hh].float().cpu().numpy().astype(np.float64)
        qh, gh, kh, vh = f64(q), f64(g), f64(k), f64(v)
        scale = 1.0 / np.sqrt(E)
        s = (qh @ kh.T) * scale                       # (LQ, SQ)
        m = s.max(axis=1, keepdims=True)
        p = np.exp(s - m)
        lsum = p.sum(axis=1, keepdims=True)
        _check(out[0, hh].float().cpu().numpy(), (p @ vh) / lsum, rel, "out")
        _check(lse[0, hh].cpu().numpy(), (m + np.log(lsum))[:, 0], rel, "lse")
        oh = f64(out)
        lh = lse[0, hh].cpu().numpy().astype(np.float64)
        p = np.exp(s - lh[:, None])
        ds = p * (gh @ vh.T - (gh * oh).sum(axis=1, keepdims=True))
        _check(dq[0, hh].float().cpu().numpy(), scale * (ds @ kh), rel, "dq")
        _check(dk[0, hh].float().cpu().numpy(), scale * (ds.T @ qh), rel, "dk")
        _check(dv[0, hh].float().cpu().numpy(), p.T @ gh, rel, "dv")
    finally:
        del q, g, k, v
        _native.release_workspaces()
        torch.cuda.empty_cache()
