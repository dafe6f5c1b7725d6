"""TEST INFRASTRUCTURE ONLY: ctypes front end of the CPU oracle (``sdpa_oracle.c``).

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s ``cpu_baseline`` leg import
this package, and only as the checker (or the timed CPU baseline).  The product package
``densecore_amd`` never imports it.

``forward`` / ``backward`` mirror DenseCore's ``torch_attention::forward`` /
``torch_attention::backward`` (``src/torch_attention.rs:143-284, 286-468``) on contiguous
float32 NumPy arrays laid out (B, H, L, E) for q/out/grad_out, (B, Hkv, S, E) for k/v and
(B, H, L) for lse; ``mask`` is the additive float (B, H, L, S) mask the reference's boundary
accepts (``src/lib.rs:594-607``).
"""
import ctypes
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
# DC_ORACLE_LIB names another build of the same source (the sanitizer build, oracle_asan.so).
_LIB_PATH = os.environ.get("DC_ORACLE_LIB") or os.path.join(_HERE, "liboracle_sdpa.so")
_lib = None

_F = ctypes.POINTER(ctypes.c_float)
_SZ = ctypes.c_size_t

ERRORS = {1: "gemm layout outside PyTorch's BLAS path", 2: "out of memory",
          3: "flash attention q/k/v shapes do not match"}


def build(force=False):
    """Compile the oracle with its Makefile (gcc, -ffp-contract=off)."""
    if force or not os.path.exists(_LIB_PATH):
        subprocess.run(["make", "-s", "-C", _HERE, "-B" if force else "all", "liboracle_sdpa.so"],
                       check=True)


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            raise RuntimeError(f"oracle library not built: {_LIB_PATH} (run oracle.build())")
        L = ctypes.CDLL(_LIB_PATH)
        L.oracle_forward.argtypes = [_F, _F, _F, _F] + [_SZ] * 6 + [ctypes.c_int, ctypes.c_int,
                                                                     ctypes.c_double, _F, _F]
        L.oracle_forward.restype = ctypes.c_int
        L.oracle_backward.argtypes = [_F] * 7 + [_SZ] * 6 + [ctypes.c_int, ctypes.c_int,
                                                              ctypes.c_double, _F, _F, _F]
        L.oracle_backward.restype = ctypes.c_int
        L.oracle_set_num_threads.argtypes = [_SZ]
        L.oracle_get_num_threads.restype = _SZ
        L.oracle_exp_u20.argtypes = [_F, _F, _SZ]
        L.oracle_sleef_expf.argtypes = [_F, _F, _SZ]
        L.oracle_reduce_max.argtypes = [_F, _SZ]
        L.oracle_reduce_max.restype = ctypes.c_float
        L.oracle_reduce_dot.argtypes = [_F, _F, _SZ]
        L.oracle_reduce_dot.restype = ctypes.c_float
        L.oracle_mul_reduce_max.argtypes = [_F, _SZ, ctypes.c_float]
        L.oracle_mul_reduce_max.restype = ctypes.c_float
        L.oracle_exp_reduce_sum.argtypes = [_F, _SZ, ctypes.c_float]
        L.oracle_exp_reduce_sum.restype = ctypes.c_float
        L.oracle_gemm_raw.argtypes = [ctypes.c_int, ctypes.c_int, _SZ, _SZ, _SZ, ctypes.c_float,
                                      _F, _SZ, _F, _SZ, ctypes.c_float, _F, _SZ]
        L.oracle_gemm_raw.restype = ctypes.c_int
        L.oracle_scale_factor.argtypes = [_SZ, ctypes.c_int, ctypes.c_double]
        L.oracle_scale_factor.restype = ctypes.c_float
        L.oracle_q_split.argtypes = [_SZ]
        L.oracle_q_split.restype = _SZ
        L.oracle_softmax.argtypes = [_F, _SZ, _SZ, _F]
        L.oracle_softmax_backward.argtypes = [_F, _F, _SZ, _SZ, _F]
        MT = ctypes.c_void_p
        L.oracle_mt_seed.argtypes = [MT, ctypes.c_uint64]
        L.oracle_mt_random.argtypes = [MT, ctypes.POINTER(ctypes.c_uint32), _SZ]
        L.oracle_mt_uniform_f64.argtypes = [MT, ctypes.POINTER(ctypes.c_double), _SZ]
        L.oracle_mt_bernoulli.argtypes = [MT, ctypes.c_double, _F, _SZ]
        _lib = L
    return _lib


def _p(a):
    return None if a is None else a.ctypes.data_as(_F)


def _f32(a):
    return np.ascontiguousarray(a, dtype=np.float32)


def set_num_threads(n):
    lib().oracle_set_num_threads(int(n))


def get_num_threads():
    return int(lib().oracle_get_num_threads())


def _dims(q, k, v):
    if q.ndim != 4 or k.ndim != 4 or v.ndim != 4:
        raise ValueError("flash attention takes (B, H, L, E) tensors")
    if not (k.shape == v.shape and k.shape[0] == q.shape[0] and k.shape[3] == q.shape[3]
            and k.shape[1] > 0 and q.shape[1] % k.shape[1] == 0):
        raise ValueError("flash attention q/k/v shapes do not match")
    return q.shape[0], q.shape[1], k.shape[1], q.shape[2], k.shape[2], q.shape[3]


def forward(q, k, v, causal, scale=None, mask=None):
    """``torch_attention::forward`` (``src/torch_attention.rs:143-284``): (out, lse)."""
    q, k, v = _f32(q), _f32(k), _f32(v)
    B, H, Hkv, L, S, E = _dims(q, k, v)
    if mask is not None:
        mask = _f32(mask)
        if mask.shape != (B, H, L, S):
            raise ValueError("flash attention mask must be (B, H, L, S)")
    out = np.empty((B, H, L, E), np.float32)
    lse = np.empty((B, H, L), np.float32)
    r = lib().oracle_forward(_p(q), _p(k), _p(v), _p(mask), B, H, Hkv, L, S, E, int(bool(causal)),
                             int(scale is not None), float(scale or 0.0), _p(out), _p(lse))
    if r:
        raise RuntimeError(ERRORS.get(r, f"oracle error {r}"))
    return out, lse


def backward(grad_out, q, k, v, out, lse, causal, scale=None, mask=None):
    """``torch_attention::backward`` (``src/torch_attention.rs:286-468``): (dq, dk, dv)."""
    g, q, k, v, o, lse = (_f32(x) for x in (grad_out, q, k, v, out, lse))
    B, H, Hkv, L, S, E = _dims(q, k, v)
    if g.shape != q.shape or o.shape != q.shape or lse.shape != (B, H, L):
        raise ValueError("flash attention backward shapes do not match")
    if mask is not None:
        mask = _f32(mask)
        if mask.shape != (B, H, L, S):
            raise ValueError("flash attention mask must be (B, H, L, S)")
    dq = np.empty((B, H, L, E), np.float32)
    dk = np.empty((B, Hkv, S, E), np.float32)
    dv = np.empty((B, Hkv, S, E), np.float32)
    r = lib().oracle_backward(_p(g), _p(q), _p(k), _p(v), _p(o), _p(lse), _p(mask), B, H, Hkv, L, S,
                              E, int(bool(causal)), int(scale is not None), float(scale or 0.0),
                              _p(dq), _p(dk), _p(dv))
    if r:
        raise RuntimeError(ERRORS.get(r, f"oracle error {r}"))
    return dq, dk, dv


# ---- single functions, for pinning each piece against the mathematics ----

def exp_u20(x):
    x = _f32(x)
    assert x.size % 4 == 0
    y = np.empty_like(x)
    lib().oracle_exp_u20(_p(x), _p(y), x.size)
    return y


def sleef_expf(x):
    x = _f32(x)
    y = np.empty_like(x)
    lib().oracle_sleef_expf(_p(x), _p(y), x.size)
    return y


def reduce_max(x):
    x = _f32(x)
    return float(lib().oracle_reduce_max(_p(x), x.size))


def reduce_dot(a, b):
    a, b = _f32(a), _f32(b)
    return float(lib().oracle_reduce_dot(_p(a), _p(b), a.size))


def mul_reduce_max(row, scale):
    row = _f32(row).copy()
    m = float(lib().oracle_mul_reduce_max(_p(row), row.size, scale))
    return row, m


def exp_reduce_sum(row, mx):
    row = _f32(row).copy()
    s = float(lib().oracle_exp_reduce_sum(_p(row), row.size, mx))
    return row, s


def gemm_raw(ta, tb, m, n, k, alpha, a, lda, b, ldb, beta, c, ldc):
    a, b = _f32(a), _f32(b)
    c = _f32(c).copy()
    r = lib().oracle_gemm_raw(int(ta), int(tb), m, n, k, alpha, _p(a), lda, _p(b), ldb, beta, _p(c), ldc)
    if r:
        raise RuntimeError(ERRORS.get(r, f"oracle error {r}"))
    return c


def scale_factor(e, scale=None):
    return float(lib().oracle_scale_factor(e, int(scale is not None), float(scale or 0.0)))


def q_split(q_len):
    return int(lib().oracle_q_split(q_len))


# ---- the math path's pieces (python/densecore/functional.py:318-340) ----

def softmax(x):
    """``softmax_lastdim`` (``src/torch_softmax.rs:57-67``) over the last axis."""
    x = _f32(x)
    width = x.shape[-1]
    y = np.empty_like(x)
    if x.size:
        lib().oracle_softmax(_p(x), x.size // width, width, _p(y))
    return y


def softmax_backward(g, y):
    """``softmax_backward_lastdim`` (``src/torch_softmax.rs:90-97``)."""
    g, y = _f32(g), _f32(y)
    width = y.shape[-1]
    dx = np.empty_like(y)
    if y.size:
        lib().oracle_softmax_backward(_p(g), _p(y), y.size // width, width, _p(dx))
    return dx


def bmm(a, b, b_k_contiguous=False):
    """``torch_blas::bmm`` (``src/torch_blas.rs:404-449``) over leading dims, float32.

    Products with k*rows*cols >= 400 go through ``addmm`` to the Linux naive ``sgemm_``
    (``src/torch_blas.rs:95-134``): each output is the float32 sum of rounded products in k
    order.  Smaller ones take the plain loop of ``:414-442``: the first k - k % 4 products
    rounded and added in order when k > 3 and both operands are contiguous along k (a is taken
    as contiguous; ``b_k_contiguous`` says whether b is a transposed view), the rest fused
    (emulated in float64: the product is exact there, then the sum is rounded once)."""
    a, b = np.asarray(a, np.float32), np.asarray(b, np.float32)
    rows, k = a.shape[-2], a.shape[-1]
    cols = b.shape[-1]
    lead = np.broadcast_shapes(a.shape[:-2], b.shape[:-2])
    a = np.broadcast_to(a, lead + a.shape[-2:])
    b = np.broadcast_to(b, lead + b.shape[-2:])
    acc = np.zeros(lead + (rows, cols), np.float32)
    small = k * rows * cols < 400
    unfused = (k - k % 4 if (k > 3 and b_k_contiguous) else 0) if small else k
    for t in range(k):
        x = a[..., :, t][..., :, None]
        y = b[..., t, :][..., None, :]
        if t < unfused:
            acc = acc + x * y
        else:
            acc = (acc.astype(np.float64) + x.astype(np.float64) * y.astype(np.float64)).astype(np.float32)
    return acc


def math_attention(query, key, value, attn_mask=None, is_causal=False, scale=None, noise=None,
                   grad_out=None):
    """The reference's math path (``python/densecore/functional.py:318-340``) composed from the
    restated pieces: q and k each scaled by float32(sqrt(|scale|)), ``bmm``, the additive mask,
    the safe softmax, an optional dropout noise tensor (keep / (1 - p) as float32), ``bmm`` with
    v.  With ``grad_out`` it also returns (dq, dk, dv, dmask) by the chain rule of those ops
    (``mm_mat1_backward`` / ``mm_mat2_backward``, ``softmax_backward_lastdim``, the masked
    fills zeroing the empty rows)."""
    import math
    q, k, v = _f32(query), _f32(key), _f32(value)
    E, L, S = q.shape[-1], q.shape[-2], k.shape[-2]
    if scale is None:
        scale = 1.0 / math.sqrt(E) if E else 1.0
    factor = math.sqrt(abs(scale))
    fq = np.float32(-factor if scale < 0 else factor)
    fk = np.float32(factor)
    qs, ks = q * fq, k * fk
    attn = bmm(qs, np.swapaxes(ks, -1, -2), b_k_contiguous=True)
    mask = np.tril(np.ones((L, S), bool)) if is_causal else attn_mask
    empty = None
    if mask is not None:
        mask = np.asarray(mask)
        additive = np.where(mask, np.float32(0), np.float32(-np.inf)) if mask.dtype == np.bool_ \
            else mask.astype(np.float32)
        attn = attn + additive
        empty = np.isneginf(attn).all(-1, keepdims=True)
    if empty is not None and empty.any():
        w = np.where(empty, np.float32(0), softmax(np.where(empty, np.float32(0), attn)))
    else:
        w = softmax(attn)
    wd = w if noise is None else w * _f32(noise)
    out = bmm(wd, v)
    if grad_out is None:
        return out
    g = _f32(grad_out)
    dwd = bmm(g, np.swapaxes(v, -1, -2))
    dv = bmm(np.swapaxes(wd, -1, -2), g)
    dw = dwd if noise is None else dwd * _f32(noise)
    if empty is not None and empty.any():
        dw = np.where(empty, np.float32(0), dw)
        ws = softmax(np.where(empty, np.float32(0), attn))
        da = np.where(empty, np.float32(0), softmax_backward(dw, ws))
    else:
        da = softmax_backward(dw, w)
    dqs = bmm(da, ks)
    dks = bmm(np.swapaxes(da, -1, -2), qs)
    return out, (dqs * fq, dks * fk, dv, da)


# ---- the reference's generator (src/torch_random.rs:9-110, 241-254), one output at a time ----

class _MT(ctypes.Structure):
    _fields_ = [("state", ctypes.c_uint32 * 624), ("left", ctypes.c_int64), ("next", ctypes.c_int64)]


class Generator:
    """``torch_random::Generator``'s engine and the draws the dropout path uses."""

    def __init__(self, seed=67_280_421_310_721):
        self._g = _MT()
        self.manual_seed(seed)

    def manual_seed(self, seed):
        lib().oracle_mt_seed(ctypes.addressof(self._g), int(seed) & (2**64 - 1))

    @property
    def words(self):
        return np.frombuffer(self._g.state, np.uint32).copy()

    @property
    def position(self):
        return int(self._g.left), int(self._g.next)

    def set(self, words, left, next_):
        self._g.state[:] = [int(w) for w in np.asarray(words, np.uint32)]
        self._g.left, self._g.next = int(left), int(next_)

    def random(self, n):
        out = np.empty(int(n), np.uint32)
        lib().oracle_mt_random(ctypes.addressof(self._g), out.ctypes.data_as(ctypes.POINTER(ctypes.c_uint32)),
                               out.size)
        return out

    def uniform_doubles(self, n):
        out = np.empty(int(n), np.float64)
        lib().oracle_mt_uniform_f64(ctypes.addressof(self._g),
                                    out.ctypes.data_as(ctypes.POINTER(ctypes.c_double)), out.size)
        return out

    def bernoulli(self, n, p):
        """``Generator::bernoulli(n, p)``: float32 0/1."""
        out = np.empty(int(n), np.float32)
        lib().oracle_mt_bernoulli(ctypes.addressof(self._g), float(p), _p(out), out.size)
        return out


def dropout_noise(gen, shape, p):
    """``_dropout_noise`` (``python/densecore/functional.py:638-641``): bernoulli(1 - p) divided
    by float32(1 - p), in float32."""
    n = int(np.prod(shape))
    return (gen.bernoulli(n, 1 - p) / np.float32(1 - p)).reshape(shape)
