"""Writes tests/golden/sdpa_golden.npz: inputs and the oracle's outputs for the shapes the
reference's own attention tests pin (tests/test_sdpa_exact.py:10-14 and :32-41 of the
reference; it holds no golden vectors of its own, its tests compare against live torch).

Before anything is written, every case is cross-checked against two independent references:
the float64 brute force (oracle/brute.py: dense softmax forward, torch.autograd gradients) and
torch's float32 CPU scaled_dot_product_attention, at the reference's own test tolerances
(tests/test_attention.py:33-39: forward rtol 1e-5 atol 1e-6, gradients rtol 1e-4 atol 1e-5).

    python tests/golden/gen_golden.py
"""
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, ROOT)

EXACT = [(2, 2, 7, 7, 5, False, None), (2, 2, 7, 7, 5, True, None), (1, 3, 33, 33, 16, True, None),
         (1, 2, 100, 37, 12, False, None), (1, 1, 200, 200, 8, True, None),
         (1, 1, 600, 600, 8, False, None), (1, 1, 800, 800, 4, True, None),
         (1, 2, 9, 1030, 6, False, None), (1, 2, 64, 64, 16, True, 0.3)]
MASKED = [(2, 2, 7, 7, 5), (1, 2, 200, 37, 12), (1, 1, 9, 1030, 6), (2, 3, 64, 64, 16)]
KINDS = ["bool2d", "float2d", "bool4d_b1", "float4d_1h", "row"]


def cases():
    """(tag, seed, q, k, v, g, causal, scale, mask (B,H,L,S) additive or None), drawn like the
    reference's tests draw them."""
    for B, H, L, S, E, causal, scale in EXACT:
        rng = np.random.default_rng(L * 31 + S)
        q, g = (rng.normal(size=(B, H, L, E)).astype(np.float32) for _ in range(2))
        k, v = (rng.normal(size=(B, H, S, E)).astype(np.float32) for _ in range(2))
        yield f"exact_{B}_{H}_{L}_{S}_{E}_{int(causal)}_{scale}", L * 31 + S, q, k, v, g, causal, scale, None
    for B, H, L, S, E in MASKED:
        # The 1030-key shape keeps two kinds to hold the file small; all five run live on the GPU.
        for kind in (KINDS if S < 1000 else ["bool2d", "row"]):
            rng = np.random.default_rng(L + S)
            q, g = (rng.normal(size=(B, H, L, E)).astype(np.float32) for _ in range(2))
            k, v = (rng.normal(size=(B, H, S, E)).astype(np.float32) for _ in range(2))
            m = {"bool2d": rng.random((L, S)) > 0.3, "float2d": rng.normal(size=(L, S)).astype(np.float32),
                 "bool4d_b1": rng.random((B, 1, L, S)) > 0.5,
                 "float4d_1h": rng.normal(size=(1, H, 1, S)).astype(np.float32),
                 "row": np.zeros((L, S), bool)}[kind]
            if m.dtype == np.bool_:
                m = np.where(m, np.float32(0.0), np.float32(-np.inf))
            full = np.ascontiguousarray(np.broadcast_to(m, (B, H, L, S)), np.float32)
            yield f"mask_{kind}_{B}_{H}_{L}_{S}_{E}", L + S, q, k, v, g, False, None, full


def cross_check(tag, q, k, v, g, causal, scale, mask, out, lse, grads):
    import torch
    from oracle import brute
    bo, bl = brute.sdpa(q, k, v, causal, scale, mask)
    np.testing.assert_allclose(out, bo, rtol=1e-5, atol=2e-6, err_msg=f"{tag} out vs float64")
    np.testing.assert_allclose(lse, bl, rtol=1e-5, atol=2e-6, err_msg=f"{tag} lse vs float64")
    for name, a, b in zip("qkv", grads, brute.sdpa_grads(g, q, k, v, causal, scale, mask)):
        np.testing.assert_allclose(a, b, rtol=1e-4, atol=1e-5, err_msg=f"{tag} d{name} vs float64")
    t = [torch.tensor(x, requires_grad=True) for x in (q, k, v)]
    tm = None if mask is None else torch.tensor(mask)
    y = torch.nn.functional.scaled_dot_product_attention(*t, attn_mask=tm, is_causal=causal, scale=scale)
    y.backward(torch.tensor(g))
    if not np.isneginf(mask).all(-1).any() if mask is not None else True:
        # (torch's CPU SDPA gives NaN for fully masked rows; the reference gives 0)
        np.testing.assert_allclose(out, y.detach().numpy(), rtol=1e-5, atol=1e-6, err_msg=f"{tag} torch")
        for name, a, tt in zip("qkv", grads, t):
            np.testing.assert_allclose(a, tt.grad.numpy(), rtol=1e-4, atol=1e-5, err_msg=f"{tag} torch d{name}")


def main():
    import oracle
    oracle.build()
    arrays = {}
    for tag, seed, q, k, v, g, causal, scale, mask in cases():
        out, lse = oracle.forward(q, k, v, causal, scale, mask)
        grads = oracle.backward(g, q, k, v, out, lse, causal, scale, mask)
        cross_check(tag, q, k, v, g, causal, scale, mask, out, lse, grads)
        # Inputs are stored once per shape (the masked kinds of one shape share them).
        src = "in_" + "_".join(map(str, q.shape + k.shape[2:3] + (seed,)))
        for name, x in (("q", q), ("k", k), ("v", v), ("g", g)):
            if f"{src}/{name}" in arrays:
                assert np.array_equal(arrays[f"{src}/{name}"], x)
            arrays[f"{src}/{name}"] = x
        arrays.update({f"{tag}/out": out, f"{tag}/lse": lse, f"{tag}/dq": grads[0],
                       f"{tag}/dk": grads[1], f"{tag}/dv": grads[2],
                       f"{tag}/inputs": np.array(src),
                       f"{tag}/meta": np.array([float(causal), np.nan if scale is None else scale])})
        if mask is not None:
            # The additive mask before broadcasting to (B, H, L, S) is not kept by cases(), so
            # keep the full one; -inf runs compress well.
            arrays[f"{tag}/mask"] = mask
    path = os.path.join(HERE, "sdpa_golden.npz")
    np.savez_compressed(path, **arrays)
    print(f"wrote {path}: {len(arrays)} arrays, {os.path.getsize(path) / 1e6:.2f} MB")


if __name__ == "__main__":
    main()
