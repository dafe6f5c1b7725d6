"""Device-side counterpart of DenseCore's native flash-attention boundary.

``_flash_attention`` and ``_flash_attention_backward`` keep the names, argument meaning and
error behaviour of the reference's pyo3 functions (``src/lib.rs:555-683``): rank and shape
checks raise ``ValueError`` with the same messages, kernel failures raise ``RuntimeError``,
and the results are fresh tensors.  The difference is where the data lives: tensors are
device-resident ``torch`` tensors on the GPU (torch is used for device memory and streams
only), and the work is done by the HIP kernels behind ``include/dc_attn.h``.  Calls are
ordered on torch's current stream of the tensors' device.

``_flash_decode`` is the new single-query entry point (split-KV), equivalent to
``_flash_attention`` at L = 1 without causal masking.
"""
import collections
import math

import torch

from . import _lib

_DTYPES = {torch.float32: _lib.DC_F32, torch.bfloat16: _lib.DC_BF16}


def _attention_dims(q, k, v):
    """``attention_dims`` (src/lib.rs:555-580)."""
    if q.dim() != 4 or k.dim() != 4 or v.dim() != 4:
        raise ValueError("flash attention takes (B, H, L, E) tensors")
    qs, ks = tuple(q.shape), tuple(k.shape)
    ok = ks == tuple(v.shape) and ks[0] == qs[0] and ks[3] == qs[3] and ks[1] > 0 and qs[1] % ks[1] == 0
    if not ok:
        raise ValueError("flash attention q/k/v shapes do not match")
    return qs[0], qs[1], ks[1], qs[2], ks[2], qs[3]


def _check_device(*tensors):
    dev = tensors[0].device
    if dev.type != "cuda":
        raise ValueError("flash attention tensors must be on the GPU")
    dtype = tensors[0].dtype
    if dtype not in _DTYPES:
        raise ValueError("flash attention takes float32 or bfloat16 tensors")
    for t in tensors[1:]:
        if t.device != dev:
            raise ValueError("flash attention tensors must be on one device")
        if t.dtype != dtype:
            raise ValueError("flash attention tensors must share one dtype")
    return dev, dtype


def _mask_arg(mask, dims, dev):
    """``attention_mask`` (src/lib.rs:594-607): an additive float32 (B, H, L, S) mask.
    Broadcast views (stride 0) are passed through without materialising them.  The kernels read
    a row's keys with unit stride, so a mask without it (e.g. an (L, 1) mask expanded over the keys)
    is copied along the key axis only: its broadcast batch / head / query dims stay stride 0."""
    if mask is None:
        return None, (0, 0, 0)
    B, H, _, L, S, _ = dims
    if tuple(mask.shape) != (B, H, L, S):
        raise ValueError("flash attention mask must be (B, H, L, S)")
    if mask.device != dev or mask.dtype != torch.float32:
        mask = mask.to(device=dev, dtype=torch.float32)
    if S > 1 and mask.stride(3) != 1:
        distinct = tuple(slice(0, 1) if mask.stride(i) == 0 else slice(None) for i in range(3))
        mask = mask[distinct].contiguous().expand(B, H, L, S)
    return mask, (mask.stride(0), mask.stride(1), mask.stride(2))


# DC_FLAG_CONSISTENT_SCORES on every call when set (include/dc_attn.h): the float32 backward at
# head dims 65-128 forms its scores in the forward's order of products, so that exp(score - lse)
# normalizes exactly as the forward's did (slower); see consistent_scores().
CONSISTENT_SCORES = False


def consistent_scores(enabled=True):
    """Make the float32 backward at head dims 65-128 form its scores in the forward's order
    (``DC_FLAG_CONSISTENT_SCORES``) for the calls that follow, or go back to the faster 8-wave
    tile.  Head dims up to 64 always use the forward's order.  Returns the previous setting."""
    global CONSISTENT_SCORES
    previous, CONSISTENT_SCORES = CONSISTENT_SCORES, bool(enabled)
    return previous


def _desc(dims, causal, scale, dtype, mstrides):
    B, H, Hkv, L, S, E = dims
    flags = _lib.DC_FLAG_CONSISTENT_SCORES if CONSISTENT_SCORES else 0
    return _lib.Desc(B, H, Hkv, L, S, E, int(bool(causal)), int(scale is not None),
                     float(scale) if scale is not None else 0.0, _DTYPES[dtype], flags, *mstrides)


def _ptr(t):
    return None if t is None or t.numel() == 0 else t.data_ptr()


def _stream(dev):
    return torch.cuda.current_stream(dev).cuda_stream


# One workspace per (device, stream), grown on demand and reused: calls on one stream run in
# order, so a call never overlaps the previous user of its stream's workspace.  At most
# _MAX_WORKSPACES streams keep one (the least recently used is dropped; torch's caching allocator
# frees its memory once the last call using it has run), and release_workspaces() drops them all.
# Under stream capture (a CUDA graph) every call gets a workspace of its own instead: a captured
# graph keeps its addresses, and two graphs replayed on different streams must not share one.
_WORKSPACES = collections.OrderedDict()
_MAX_WORKSPACES = 4


def release_workspaces():
    """Drop every cached workspace (their memory returns to torch's caching allocator)."""
    _WORKSPACES.clear()


def _workspace(nbytes, dev):
    nbytes = max(int(nbytes), 1)
    if torch.cuda.is_current_stream_capturing():
        return torch.empty(nbytes, dtype=torch.uint8, device=dev)
    key = (dev.index, _stream(dev))
    ws = _WORKSPACES.pop(key, None)
    if ws is None or ws.numel() < nbytes:
        ws = None  # release the smaller buffer before allocating its replacement
        ws = torch.empty(nbytes, dtype=torch.uint8, device=dev)
    _WORKSPACES[key] = ws
    while len(_WORKSPACES) > _MAX_WORKSPACES:
        _WORKSPACES.popitem(last=False)
    return ws


# The float32 backward's full workspace holds one dQ-sized slot per 128-key tile (for sums in a
# fixed order), which grows as S / 128 * |dq|: about 4 GiB at B1 H32 L=S=8192 E128 causal.  Above
# max(this many bytes, 8 |dq|) a call passes that bound instead; the library then runs the problem
# in pieces (whole batches, or kv heads of one batch) whose slots fit, with the same fixed-order
# sums, and only when not even one kv head's slots fit, with float atomics.
DETERMINISTIC_WORKSPACE_BYTES = 1 << 30


def _bwd_workspace_bytes(L_, d, dims, dtype):
    full = int(L_.dc_sdpa_bwd_workspace_size(d))
    B, H, _, L, _, E = dims
    if dtype != torch.float32 or E > 128:
        return full
    return min(full, max(DETERMINISTIC_WORKSPACE_BYTES, 8 * B * H * L * E * 4))


def _schedule(backward, q, k, v, causal, scale=None, mask=None, workspace_bytes=None):
    """The schedule ``dc_sdpa_fwd`` (or ``dc_sdpa_bwd``) takes for these arguments on the current
    device, with the workspace ``_flash_attention`` passes (or ``workspace_bytes``)."""
    dims = _attention_dims(q, k, v)
    _, dtype = _check_device(q, k, v)
    ms = _mask_arg(mask, dims, q.device)[1] if mask is not None else (0, 0, 0)
    d = _desc(dims, causal, scale, dtype, ms)
    L_ = _lib.lib()
    if workspace_bytes is None:
        size = (_bwd_workspace_bytes(L_, d, dims, dtype) if backward
                else int(L_.dc_sdpa_fwd_workspace_size(d)))
        workspace_bytes = max(size, 1)
    out = _lib.Schedule()
    query = L_.dc_sdpa_bwd_schedule if backward else L_.dc_sdpa_fwd_schedule
    _lib.check(query(d, int(mask is not None), int(workspace_bytes), out))
    return out.as_dict()


def _flash_attention(q, k, v, causal, scale=None, mask=None):
    """Forward: (out, lse).  ``_flash_attention`` (src/lib.rs:609-638)."""
    dims = _attention_dims(q, k, v)
    dev, dtype = _check_device(q, k, v)
    mask, ms = _mask_arg(mask, dims, dev)
    q, k, v = q.contiguous(), k.contiguous(), v.contiguous()
    B, H, _, L, _, E = dims
    out = torch.empty((B, H, L, E), dtype=dtype, device=dev)
    lse = torch.empty((B, H, L), dtype=torch.float32, device=dev)
    d = _desc(dims, causal, scale, dtype, ms)
    L_ = _lib.lib()
    ws = _workspace(L_.dc_sdpa_fwd_workspace_size(d), dev)
    _lib.check(L_.dc_sdpa_fwd(d, _ptr(q), _ptr(k), _ptr(v), _ptr(mask), _ptr(out), _ptr(lse),
                              _ptr(ws), ws.numel(), _stream(dev)))
    return out, lse


def _flash_attention_backward(grad_out, q, k, v, out, lse, causal, scale=None, mask=None):
    """Backward: (dq, dk, dv).  ``_flash_attention_backward`` (src/lib.rs:640-683)."""
    dims = _attention_dims(q, k, v)
    B, H, Hkv, L, S, E = dims
    if (tuple(grad_out.shape) != tuple(q.shape) or tuple(out.shape) != tuple(q.shape)
            or tuple(lse.shape) != (B, H, L)):
        raise ValueError("flash attention backward shapes do not match")
    dev, dtype = _check_device(q, k, v, grad_out, out)
    if lse.device != dev or lse.dtype != torch.float32:
        raise ValueError("flash attention lse must be float32 on the tensors' device")
    mask, ms = _mask_arg(mask, dims, dev)
    grad_out, q, k, v, out, lse = (t.contiguous() for t in (grad_out, q, k, v, out, lse))
    dq = torch.empty((B, H, L, E), dtype=dtype, device=dev)
    dk = torch.empty((B, Hkv, S, E), dtype=dtype, device=dev)
    dv = torch.empty((B, Hkv, S, E), dtype=dtype, device=dev)
    d = _desc(dims, causal, scale, dtype, ms)
    L_ = _lib.lib()
    ws = _workspace(_bwd_workspace_bytes(L_, d, dims, dtype), dev)
    _lib.check(L_.dc_sdpa_bwd(d, _ptr(grad_out), _ptr(q), _ptr(k), _ptr(v), _ptr(out), _ptr(lse),
                              _ptr(mask), _ptr(dq), _ptr(dk), _ptr(dv), _ptr(ws), ws.numel(),
                              _stream(dev)))
    return dq, dk, dv


def _flash_decode(q, k, v, scale=None):
    """Single-query attention (q is (B, H, 1, E)) over a contiguous KV cache: (out, lse)."""
    dims = _attention_dims(q, k, v)
    B, H, _, L, _, E = dims
    if L != 1:
        raise ValueError("flash attention decode takes q_len == 1")
    dev, dtype = _check_device(q, k, v)
    q, k, v = q.contiguous(), k.contiguous(), v.contiguous()
    out = torch.empty((B, H, 1, E), dtype=dtype, device=dev)
    lse = torch.empty((B, H, 1), dtype=torch.float32, device=dev)
    d = _desc(dims, False, scale, dtype, (0, 0, 0))
    L_ = _lib.lib()
    ws = _workspace(L_.dc_sdpa_decode_workspace_size(d), dev)
    _lib.check(L_.dc_sdpa_decode(d, _ptr(q), _ptr(k), _ptr(v), _ptr(out), _ptr(lse), _ptr(ws),
                                 ws.numel(), _stream(dev)))
    return out, lse


def _bmm(a, b):
    """``bmm`` (``src/batched_matmul.rs:9-49``): (batch, m, k) x (batch, k, n) -> (batch, m, n),
    float32, with the reference's shape errors.  The operands are read through their strides (a
    transposed view is not copied); the result is a fresh contiguous tensor."""
    if a.dim() != 3 or b.dim() != 3:
        raise ValueError("bmm requires rank-3 operands")
    if a.shape[0] != b.shape[0] or a.shape[2] != b.shape[1]:
        raise ValueError("bmm batch or inner dimensions mismatch")
    if a.device.type != "cuda" or b.device != a.device:
        raise ValueError("bmm takes tensors on one GPU")
    if a.dtype != torch.float32 or b.dtype != torch.float32:
        raise ValueError("no registered bmm kernel for device/dtype")
    batch, m, k = a.shape
    n = b.shape[2]
    c = torch.empty((batch, m, n), dtype=torch.float32, device=a.device)
    sa, sb = a.stride(), b.stride()
    d = _lib.BmmDesc(batch, m, n, k, sa[0], sa[1], sa[2], sb[0], sb[1], sb[2])
    # A data pointer of an empty tensor may be anything: the library reads nothing then.
    _lib.check(_lib.lib().dc_bmm(d, _ptr(a), _ptr(b), _ptr(c), _stream(a.device)))
    return c


def _softmax_desc(rows, width, heads=1, q_len=1, mstrides=(0, 0, 0), safe=False):
    return _lib.SoftmaxDesc(int(rows), int(width), int(heads), int(q_len), *map(int, mstrides),
                            int(bool(safe)), 0)


def _softmax(scores, mask=None, safe=False):
    """``Tensor.softmax(-1)`` of float32 scores (``src/torch_softmax.rs:57-67``) with the math
    path's additive mask and safe rows fused (``python/densecore/functional.py:330-337``).

    ``scores`` is (..., L, S); ``mask`` is None or a float32 tensor broadcastable to it; it is
    read through the strides of its broadcast view (a stride of 0 is never materialised).
    """
    if scores.device.type != "cuda" or scores.dtype != torch.float32:
        raise ValueError("softmax takes a float32 tensor on the GPU")
    if scores.dim() == 0:
        raise ValueError("softmax axis out of range")
    x = scores.contiguous()
    width = x.shape[-1]
    rows = x.numel() // width if width else 0
    y = torch.empty_like(x)
    heads = q_len = 1
    ms = (0, 0, 0)
    m = None
    if mask is not None:
        m = mask.to(device=x.device, dtype=torch.float32).expand(*x.shape)
        if width > 1 and m.stride(-1) != 1:
            m = m.contiguous()
        # A (B, H, L, S) view of the mask: the kernel addresses row (b, h, l) by strides.
        lead = x.dim() - 2
        if lead < 0:
            m = m.reshape(1, 1, 1, width)
        elif lead <= 2:
            m = m[(None,) * (2 - lead)]
        else:
            m = m.reshape(-1, x.shape[-3], x.shape[-2], width)
        heads, q_len = m.shape[1], m.shape[2]
        ms = (m.stride(0), m.stride(1), m.stride(2))
    d = _softmax_desc(rows, width, heads, q_len, ms, safe)
    _lib.check(_lib.lib().dc_softmax_fwd(d, _ptr(x), _ptr(m), _ptr(y), _stream(x.device)))
    return y


def _softmax_backward(grad_y, y):
    """``softmax_backward_lastdim`` (``src/torch_softmax.rs:90-97``): (g - sum(g * y)) * y."""
    if tuple(grad_y.shape) != tuple(y.shape):
        raise ValueError("softmax backward shapes do not match")
    g, y = grad_y.contiguous(), y.contiguous()
    if g.dtype != torch.float32 or y.dtype != torch.float32 or g.device != y.device:
        raise ValueError("softmax backward takes float32 tensors on one GPU")
    width = y.shape[-1] if y.dim() else 1
    rows = y.numel() // width if width else 0
    dx = torch.empty_like(y)
    d = _softmax_desc(rows, width)
    _lib.check(_lib.lib().dc_softmax_bwd(d, _ptr(g), _ptr(y), _ptr(dx), _stream(y.device)))
    return dx


def _dropout_apply(bits, x, scale):
    """``x * noise`` for the keep bits of ``x``'s elements in row-major order:
    y = x * (kept ? scale : 0) (``dc_dropout_apply``)."""
    if x.device.type != "cuda" or x.dtype != torch.float32 or bits.device != x.device:
        raise ValueError("dropout takes float32 tensors and keep bits on one GPU")
    x = x.contiguous()
    if bits.numel() * 32 < x.numel():
        raise ValueError("dropout keep bits do not cover the tensor")
    y = torch.empty_like(x)
    _lib.check(_lib.lib().dc_dropout_apply(_ptr(bits), x.numel(), float(scale), _ptr(x), _ptr(y),
                                           _stream(x.device)))
    return y


def default_scale(head_dim):
    """``sdp::calculate_scale`` as the Python layer passes it (a double)."""
    return 1.0 / math.sqrt(head_dim) if head_dim else 1.0
