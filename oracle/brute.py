"""TEST INFRASTRUCTURE ONLY: float64 brute-force attention, the textbook formula.

This is the independent check the C oracle is pinned against: dense scores, a plain
(non-blockwise) softmax, no online rescaling, no tiling, float64 throughout.  It restates
nothing of the reference's blockwise algorithm; it states what that algorithm computes
(``src/torch_attention.rs:143-284``): out = softmax(scale * q k^T + mask, causal) v and
lse = log(sum(exp(scores))), with fully masked rows giving out = 0 and lse = 0
(``src/torch_attention.rs:223-226, 258-264``).  Gradients come from torch's autograd in
float64 on the CPU, a separate implementation of the chain rule.
"""
import math

import numpy as np


def _scores(q, k, causal, scale, mask):
    q = np.asarray(q, np.float64)
    k = np.asarray(k, np.float64)
    B, H, L, E = q.shape
    Hkv, S = k.shape[1], k.shape[2]
    k = np.repeat(k, H // Hkv, axis=1)
    if scale is None:
        scale = 1.0 / math.sqrt(E)
    s = np.einsum("bhld,bhsd->bhls", q, k) * float(np.float32(scale))
    if mask is not None:
        s = s + np.asarray(mask, np.float64)
    if causal:
        allowed = np.arange(S)[None, :] <= np.arange(L)[:, None]
        s = np.where(allowed, s, -np.inf)
    return s


def sdpa(q, k, v, causal=False, scale=None, mask=None):
    """Dense float64 attention: (out, lse)."""
    s = _scores(q, k, causal, scale, mask)
    H = np.asarray(q).shape[1]
    v = np.repeat(np.asarray(v, np.float64), H // np.asarray(v).shape[1], axis=1)
    m = s.max(-1, keepdims=True)
    empty = np.isneginf(m)
    m = np.where(empty, 0.0, m)
    p = np.exp(s - m)
    tot = p.sum(-1, keepdims=True)
    lse = np.where(empty, 0.0, m + np.log(np.where(tot == 0, 1.0, tot)))[..., 0]
    w = np.where(tot == 0, 0.0, p / np.where(tot == 0, 1.0, tot))
    return np.einsum("bhls,bhsd->bhld", w, v), lse


def sdpa_grads(grad_out, q, k, v, causal=False, scale=None, mask=None):
    """(dq, dk, dv) in float64 from torch.autograd over the dense formula."""
    import torch
    t = [torch.tensor(np.asarray(x, np.float64), requires_grad=True) for x in (q, k, v)]
    tq, tk, tv = t
    B, H, L, E = tq.shape
    rep = H // tk.shape[1]
    kk = tk.repeat_interleave(rep, dim=1)
    vv = tv.repeat_interleave(rep, dim=1)
    sc = float(np.float32(1.0 / math.sqrt(E) if scale is None else scale))
    s = torch.matmul(tq, kk.transpose(-1, -2).contiguous()) * sc
    if mask is not None:
        s = s + torch.tensor(np.asarray(mask, np.float64))
    if causal:
        S = tk.shape[2]
        allowed = torch.arange(S)[None, :] <= torch.arange(L)[:, None]
        s = s.masked_fill(~allowed, float("-inf"))
    empty = torch.isneginf(s).all(-1, keepdim=True)
    w = torch.softmax(s.masked_fill(empty, 0.0), -1).masked_fill(empty, 0.0)
    out = torch.matmul(w, vv)
    out.backward(torch.tensor(np.asarray(grad_out, np.float64)))
    return tuple(x.grad.numpy() for x in t)
