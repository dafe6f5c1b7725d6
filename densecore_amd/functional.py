"""``scaled_dot_product_attention`` for device tensors, mirroring DenseCore's Python API.

Follows ``python/densecore/functional.py:276-388`` of the reference: the same argument checks
and messages, the same scale rule (``None`` means the double ``1/sqrt(E)``), the same
"flash eligibility" predicate and the same mask conversion (a bool mask is True where
attention is allowed and becomes 0 / -inf; a float mask is added), feeding the native
``_flash_attention`` / ``_flash_attention_backward`` pair through an autograd Function that
saves (q, k, v, out, lse) for the backward.

Inputs the flash path does not take (dropout, rank 3, Ev != E, masks the flash path rejects,
float masks that require a gradient) go through the reference's math path
(``functional.py:318-340``), composed on the device from this library's kernels
(``include/dc_math.h``): the two batched products are ``dc_bmm`` (the device entry of the
reference's bmm registry, ``src/batched_matmul.rs:28-49``, with its gradient as two more bmm
calls on transposed views), the mask add, safe softmax and its gradient are the softmax
kernels.  ``multi_head_attention_forward`` (``functional.py:400-461``) composes the same pieces
around its input and output projections.

Differences, all on the device side of the boundary:
  * tensors are ``torch`` tensors on the GPU, float32 or bfloat16 (bf16 is new: the reference
    flash path is float32 only, ``functional.py:314``); the math path is float32 only, as the
    reference's is;
  * masks are passed as broadcast views, not materialised to (B, H, L, S) on the host;
  * ``enable_gqa`` passes the kv heads straight to the flash kernels (they index kv head
    h // repeat, as ``src/torch_attention.rs:159-167`` does) instead of widening K and V first;
    the math path widens them as the reference does;
  * nothing falls back to the CPU: an input no device path takes raises ``NotImplementedError``.
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
    if gqa:
        # Each kv head serves H // Hkv query heads (functional.py:287-293).
        groups = query.shape[1] // key.shape[1]
        key = key.repeat_interleave(groups, dim=1)
        value = value.repeat_interleave(groups, dim=1)
    return _math_attention(query, key, value, attn_mask, dropout_p, is_causal, float(scale))


def _math_attention(query, key, value, attn_mask, dropout_p, is_causal, scale):
    """PyTorch's math path as the reference composes it (``functional.py:318-340``): q and k^T
    each scaled by sqrt(|scale|), one batched product, the additive mask, the safe softmax
    (rows that are all -inf give 0), dropout, and the product with v."""
    if any(t.dtype != torch.float32 for t in (query, key, value)):
        raise NotImplementedError("the math attention path on the GPU takes float32 tensors "
                                  "(the reference's math path is float32)")
    if query.device.type != "cuda" or key.device != query.device or value.device != query.device:
        raise ValueError("attention tensors must be on one GPU")
    factor = math.sqrt(abs(scale))
    q = query * float(-factor if scale < 0 else factor)
    attn = _matmul(q, (key * float(factor)).transpose(-2, -1))
    length, source = attn.shape[-2], attn.shape[-1]
    if is_causal:
        attn_mask = torch.ones((length, source), dtype=torch.bool, device=attn.device).tril()
    additive = None
    if attn_mask is not None:
        if isinstance(attn_mask, torch.Tensor):
            m = attn_mask.to(attn.device)
        else:
            m = torch.from_numpy(np.ascontiguousarray(np.asarray(attn_mask))).to(attn.device)
        if m.dtype == torch.bool:
            additive = torch.zeros(m.shape, dtype=torch.float32, device=attn.device).masked_fill_(
                ~m, float("-inf"))
        else:
            additive = m if m.dtype == torch.float32 else m.float()
    weights = softmax_masked(attn, additive, safe=additive is not None)
    if dropout_p:
        weights = dropout(weights, dropout_p, True)
    return _matmul(weights, value)


class _Bmm(torch.autograd.Function):
    """``bmm`` with its gradient: dA = dC B^T and dB = A^T dC, both ``dc_bmm`` on transposed
    views (no copies)."""

    @staticmethod
    def forward(ctx, a, b):
        ctx.save_for_backward(a, b)
        return _native._bmm(a, b)

    @staticmethod
    def backward(ctx, grad):
        a, b = ctx.saved_tensors
        da = _native._bmm(grad, b.transpose(1, 2)) if ctx.needs_input_grad[0] else None
        db = _native._bmm(a.transpose(1, 2), grad) if ctx.needs_input_grad[1] else None
        return da, db


def bmm(a, b):
    """The reference's ``bmm`` (``src/batched_matmul.rs:9-49``) on float32 GPU tensors:
    (batch, m, k) x (batch, k, n) -> (batch, m, n), strided operands, autograd."""
    return _Bmm.apply(a, b)


def _matmul(x, y):
    """x @ y for x (..., m, k) and y (..., k, n) with equal leading dimensions (rank 3 or 4), as
    one ``bmm`` over the flattened leading dimensions."""
    lead = tuple(x.shape[:-2])
    if tuple(y.shape[:-2]) != lead:
        raise ValueError("bmm batch or inner dimensions mismatch")
    batch = math.prod(lead)  # explicit: reshape cannot infer -1 for tensors with no elements
    out = bmm(x.reshape((batch,) + tuple(x.shape[-2:])), y.reshape((batch,) + tuple(y.shape[-2:])))
    return out.reshape(lead + tuple(out.shape[-2:]))


class _Softmax(torch.autograd.Function):
    """Softmax over the last axis with the additive mask fused in; gradient
    ``softmax_backward_lastdim`` (``src/torch_softmax.rs:90-97``).  A mask that requires a
    gradient receives the scores' gradient summed over its broadcast dimensions, as the
    reference's separate ``attn + additive`` would give it."""

    @staticmethod
    def forward(ctx, scores, mask, safe):
        y = _native._softmax(scores, mask, safe)
        ctx.save_for_backward(y)
        ctx.mask_shape = None if mask is None else tuple(mask.shape)
        return y

    @staticmethod
    def backward(ctx, grad):
        (y,) = ctx.saved_tensors
        dx = _native._softmax_backward(grad, y)
        dmask = None
        if ctx.needs_input_grad[1]:
            dmask = dx.sum_to_size(ctx.mask_shape) if ctx.mask_shape else dx.sum()
        return dx, dmask, None


def softmax_masked(scores, mask=None, safe=False):
    """``softmax(scores + mask, -1)`` on the GPU; ``safe`` makes rows that are all -inf give 0
    (the math path's ``_safe_softmax``, ``functional.py:334-337``)."""
    return _Softmax.apply(scores, mask, bool(safe))


def softmax(input, dim=-1):
    """``Tensor.softmax`` over the last axis (``src/torch_softmax.rs:57-67``) for float32 GPU
    tensors (other axes are moved last and back)."""
    if dim < 0:
        dim += input.dim()
    if dim != input.dim() - 1:
        return softmax(input.movedim(dim, -1), -1).movedim(-1, dim)
    return _Softmax.apply(input, None, False)


def _dropout_probability(p):
    """``python/densecore/functional.py:219-226``."""
    if isinstance(p, (bool, np.bool_)) or not isinstance(p, numbers.Real):
        raise TypeError("dropout probability must be real")
    p = float(p)
    if not 0.0 <= p <= 1.0:
        raise ValueError("dropout probability must be in [0, 1]")
    return p


class _Dropout(torch.autograd.Function):
    """``input * noise`` with noise = keep / float32(1 - p): the same product forward and
    backward (``dc_dropout_apply``)."""

    @staticmethod
    def forward(ctx, x, bits, scale):
        ctx.save_for_backward(bits)
        ctx.scale = scale
        return _native._dropout_apply(bits, x, scale)

    @staticmethod
    def backward(ctx, grad):
        (bits,) = ctx.saved_tensors
        return _native._dropout_apply(bits, grad, ctx.scale), None, None


def dropout(input, p=0.5, training=True, generator=None):
    """``functional.dropout`` (``python/densecore/functional.py:229-244``): zero elements with
    probability p and scale survivors by 1/(1-p) while training.  The mask is
    ``Generator::bernoulli(n, 1 - p)`` drawn on the GPU from the reference's generator stream
    (``densecore_amd.random``), so a seed gives the reference's mask bit for bit; the noise
    value is float32(1) / float32(1 - p) as ``_dropout_noise`` (:638-641) rounds it."""
    from . import random as _random
    if not isinstance(input, torch.Tensor):
        raise TypeError("dropout input must be a Tensor")
    p = _dropout_probability(p)
    if type(training) is not bool:
        raise TypeError("training must be a bool")
    if not training or p == 0.0:
        return input
    if p == 1.0:
        return input * torch.zeros((), dtype=input.dtype, device=input.device)
    if input.device.type != "cuda":
        raise ValueError("dropout on this path takes tensors on the GPU")
    if input.dtype != torch.float32:
        raise NotImplementedError("dropout on the GPU takes float32 tensors")
    gen = _random.default_generator(input.device) if generator is None else generator
    bits = gen._bernoulli_bits(input.numel(), 1 - p)
    scale = float(np.float32(1.0) / np.float32(1 - p))
    return _Dropout.apply(input, bits, scale)


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


def _float_mask(mask):
    """MHA masks (``functional.py:391-397``): a bool mask is True where attention is NOT
    allowed (-inf); a float mask is added."""
    if mask is None:
        return None
    if mask.dtype == torch.bool:
        return torch.zeros(mask.shape, dtype=torch.float32, device=mask.device).masked_fill_(
            mask, float("-inf"))
    return mask


def _append_position(mask):
    """A mask over the keys with one more key at the end, always visible (a zero column)."""
    return None if mask is None else torch.nn.functional.pad(mask, (0, 1))


def multi_head_attention_forward(query, key, value, embed_dim_to_check, num_heads, in_proj_weight,
                                 in_proj_bias, bias_k, bias_v, add_zero_attn, dropout_p,
                                 out_proj_weight, out_proj_bias, training=True,
                                 key_padding_mask=None, need_weights=True, attn_mask=None,
                                 use_separate_proj_weight=False, q_proj_weight=None,
                                 k_proj_weight=None, v_proj_weight=None, static_k=None,
                                 static_v=None, average_attn_weights=True, is_causal=False):
    """Multi-head attention with PyTorch's ``F.multi_head_attention_forward`` signature and
    semantics (the reference composes the same steps, ``functional.py:400-461``), on the GPU.

    query is (L, N, E) or unbatched (L, E); key and value (S, N, kdim / vdim) or (S, kdim / vdim).
    The steps, in PyTorch's order: project q, k, v (the packed ``in_proj_weight`` holds the three
    projections in that order, or the three separate weights); append ``bias_k`` / ``bias_v`` as
    one more key position; split the heads; substitute ``static_k`` / ``static_v``; append a zero
    key position (``add_zero_attn``); fold ``key_padding_mask`` into the additive mask; attention
    weights softmax(q k^T / sqrt(head_dim) + mask), dropped out when training; their product with
    v, merged heads, output projection.  Masks that gain a key position gain a zero column.  Bool
    masks are True where attention is not allowed.  ``is_causal`` is only a hint: ``attn_mask``
    must still be given, and is what is applied.  The projections are device BLAS calls
    (``F.linear``); the two batched products are this library's ``bmm``, the mask add and the
    softmax its softmax kernel (rows whose keys are all masked come out NaN, as PyTorch's do), and
    the dropout its dropout."""
    F = torch.nn.functional
    if is_causal and attn_mask is None:
        raise RuntimeError("Need attn_mask if specifying the is_causal hint")
    unbatched = query.dim() != 3
    if unbatched:  # one sequence: a batch of one along dim 1
        query, key, value = (x.unsqueeze(1) for x in (query, key, value))
        key_padding_mask = None if key_padding_mask is None else key_padding_mask.unsqueeze(0)
    tgt_len, batch, embed_dim = query.shape
    if embed_dim != embed_dim_to_check:
        raise ValueError(f"was expecting embedding dimension of {embed_dim_to_check}, but got {embed_dim}")
    head_dim = embed_dim // num_heads
    rows = batch * num_heads

    # Input projections.
    if use_separate_proj_weight:
        proj_w = (q_proj_weight, k_proj_weight, v_proj_weight)
    else:
        proj_w = in_proj_weight.chunk(3)
    proj_b = in_proj_bias.chunk(3) if in_proj_bias is not None else (None, None, None)
    q = F.linear(query, proj_w[0], proj_b[0])
    k = F.linear(key, proj_w[1], proj_b[1])
    v = F.linear(value, proj_w[2], proj_b[2])

    mask = _float_mask(attn_mask)
    if mask is not None and mask.dim() == 2:
        mask = mask.unsqueeze(0)  # one (L, S) mask for every (batch, head)
    key_pad = _float_mask(key_padding_mask)
    if bias_k is not None and bias_v is not None:
        k = torch.cat([k, bias_k.expand(1, batch, embed_dim)])
        v = torch.cat([v, bias_v.expand(1, batch, embed_dim)])
        mask, key_pad = _append_position(mask), _append_position(key_pad)

    # (seq, batch, heads * head_dim) -> (batch * heads, seq, head_dim)
    def heads(x):
        return x.reshape(x.shape[0], rows, head_dim).transpose(0, 1)

    q = heads(q)
    k = heads(k) if static_k is None else static_k
    v = heads(v) if static_v is None else static_v
    if add_zero_attn:
        k = torch.cat([k, k.new_zeros(rows, 1, head_dim)], 1)
        v = torch.cat([v, v.new_zeros(rows, 1, head_dim)], 1)
        mask, key_pad = _append_position(mask), _append_position(key_pad)
    src_len = k.shape[1]
    if key_pad is not None:
        per_row = key_pad.reshape(batch, 1, 1, src_len).expand(batch, num_heads, 1, src_len)
        per_row = per_row.reshape(rows, 1, src_len)
        mask = per_row if mask is None else mask + per_row

    attn = softmax_masked(bmm(q * math.sqrt(1.0 / head_dim), k.transpose(1, 2)), mask, safe=False)
    if training and dropout_p > 0:
        attn = dropout(attn, dropout_p, True)
    merged = bmm(attn, v).transpose(0, 1).reshape(tgt_len * batch, embed_dim)
    out = F.linear(merged, out_proj_weight, out_proj_bias).reshape(tgt_len, batch, -1)
    if unbatched:
        out = out.squeeze(1)
    if not need_weights:
        return out, None
    attn = attn.reshape(batch, num_heads, tgt_len, src_len)
    if average_attn_weights:
        attn = attn.mean(1)
    return out, attn.squeeze(0) if unbatched else attn

