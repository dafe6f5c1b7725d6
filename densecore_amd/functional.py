"""``scaled_dot_product_attention`` for device tensors, mirroring DenseCore's Python API.

Follows ``python/densecore/functional.py:276-388`` of the reference: the same argument checks
and messages, the same scale rule (``None`` means the double ``1/sqrt(E)``), the same
"flash eligibility" predicate and the same mask conversion (a bool mask is True where
attention is allowed and becomes 0 / -inf; a float mask is added), feeding the native
``_flash_attention`` / ``_flash_attention_backward`` pair through an autograd Function that
saves (q, k, v, out, lse) for the backward.

Differences, all on the device side of the boundary:
  * tensors are ``torch`` tensors on the GPU, float32 or bfloat16 (bf16 is new: the reference
    flash path is float32 only, ``functional.py:314``);
  * masks are passed as broadcast views, not materialised to (B, H, L, S) on the host;
  * ``enable_gqa`` passes the kv heads straight to the kernels (they index kv head h // repeat,
    as ``src/torch_attention.rs:159-167`` does) instead of widening K and V first;
  * inputs that would take the reference's math path (dropout, rank 3, Ev != E, masks the
    flash path rejects) raise ``NotImplementedError``: only the flash path is built here, and
    there is no silent CPU or composed-op fallback.
"""
import math
import numbers

import numpy as np
import torch

from . import _native


def scaled_dot_product_attention(query, key, value, attn_mask=None, dropout_p=0.0, is_causal=False,
                                 scale=None, enable_gqa=False):
    """softmax(query @ key^T * scale + mask) @ value for rank-4 (N, H, L, E) device tensors."""
    for name, t in (("query", query), ("key", key), ("value", value)):
        if not isinstance(t, torch.Tensor):
            raise TypeError(f"attention {name} must be a Tensor")
    rank = query.dim()
    gqa = enable_gqa and rank == 4 and key.dim() == 4 and key.shape[1] != query.shape[1]
    if rank not in (3, 4) or key.dim() != rank or value.dim() != rank:
        raise ValueError("attention query, key and value must all be rank 3 or all rank 4")
    lead, (length, embed) = tuple(query.shape[:-2]), tuple(query.shape[-2:])
    source = key.shape[-2]
    klead, vlead = tuple(key.shape[:-2]), tuple(value.shape[:-2])
    if gqa:
        if query.shape[1] % key.shape[1]:
            raise ValueError("attention shapes must be (..., L, E), (..., S, E), (..., S, Ev)")
        klead = vlead = lead  # each kv head serves H // Hkv query heads
        if tuple(key.shape[:2]) != tuple(value.shape[:2]) or key.shape[0] != query.shape[0]:
            raise ValueError("attention shapes must be (..., L, E), (..., S, E), (..., S, Ev)")
    if klead != lead or vlead != lead or key.shape[-1] != embed or value.shape[-2] != source:
        raise ValueError("attention shapes must be (..., L, E), (..., S, E), (..., S, Ev)")
    if type(is_causal) is not bool:
        raise TypeError("is_causal must be a bool")
    if is_causal and attn_mask is not None:
        raise ValueError("attn_mask and is_causal cannot both be set")
    if scale is None:
        scale = 1.0 / math.sqrt(embed) if embed else 1.0
    elif isinstance(scale, (bool, np.bool_)) or not isinstance(scale, numbers.Real):
        raise TypeError("scale must be real")
    flash_dtypes = (torch.float32, torch.bfloat16)
    if (rank == 4 and not dropout_p and value.shape[-1] == embed and length and source and embed
            and query.dtype in flash_dtypes and key.dtype == query.dtype and value.dtype == query.dtype):
        flash_mask = _flash_mask(attn_mask, tuple(query.shape), source, query.device)
        if attn_mask is None or flash_mask is not None:
            return _flash_attention(query, key, value, is_causal, float(scale), flash_mask)
    raise NotImplementedError(
        "only DenseCore's flash path is built on the GPU (rank 4, no dropout, Ev == E, "
        "float32/bfloat16, masks of shape (L|1, S|1) or (B|1, H|1, L|1, S|1)); "
        "this call would take the reference's math path")


def _flash_mask(attn_mask, qshape, source, device):
    """The additive float32 (B, H, L, S) mask the flash kernels read, as a broadcast view, or
    None when the reference would not take the flash path for this mask
    (``python/densecore/functional.py:343-364``)."""
    if attn_mask is None:
        return None
    if isinstance(attn_mask, torch.Tensor):
        if attn_mask.requires_grad or attn_mask.dtype not in (torch.bool, torch.float32):
            return None
        values = attn_mask.to(device)
    else:
        arr = np.asarray(attn_mask)
        if arr.dtype not in (np.bool_, np.float32):
            return None
        values = torch.from_numpy(np.ascontiguousarray(arr)).to(device)
    batch, heads, length = qshape[:3]
    if values.dim() not in (2, 4) or values.shape[-2] not in (1, length) or values.shape[-1] not in (1, source):
        return None
    if values.dim() == 4 and (values.shape[0] not in (1, batch) or values.shape[1] not in (1, heads)):
        return None
    if values.dtype == torch.bool:
        values = torch.where(values, torch.zeros((), dtype=torch.float32, device=device),
                             torch.full((), float("-inf"), dtype=torch.float32, device=device))
    return values.expand(batch, heads, length, source)


class _FlashAttention(torch.autograd.Function):
    """``FlashAttention`` (``python/densecore/functional.py:371-386``)."""

    @staticmethod
    def forward(ctx, q, k, v, causal, scale, mask):
        out, lse = _native._flash_attention(q, k, v, causal, scale, mask)
        ctx.save_for_backward(q, k, v, out, lse)
        ctx.causal, ctx.scale, ctx.mask = causal, scale, mask
        return out

    @staticmethod
    def backward(ctx, grad):
        q, k, v, out, lse = ctx.saved_tensors
        dq, dk, dv = _native._flash_attention_backward(grad, q, k, v, out, lse, ctx.causal,
                                                       ctx.scale, ctx.mask)
        return dq, dk, dv, None, None, None


def _flash_attention(query, key, value, causal, scale, mask=None):
    """The fused path (``python/densecore/functional.py:367-388``)."""
    return _FlashAttention.apply(query, key, value, causal, scale, mask)


def flash_decode(query, key, value, scale=None):
    """One decode step: query (B, H, 1, E) against the whole KV cache (B, Hkv, S, E)."""
    return _native._flash_decode(query, key, value, None if scale is None else float(scale))[0]
