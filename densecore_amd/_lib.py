"""ctypes binding of ``libdcattn.so`` (the C ABI in ``include/dc_attn.h`` and ``include/dc_math.h``).

The library is built in-tree (``densecore_amd/libdcattn.so``) by ``densecore_amd.build``.
If it is missing, every entry point raises: there is no CPU fallback on this path.
"""
import ctypes
import os

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "libdcattn.so")

DC_OK, DC_INVALID_ARGUMENT, DC_UNSUPPORTED, DC_EXECUTION_FAILED = 0, 1, 2, 3
DC_F32, DC_BF16 = 0, 1
DC_FLAG_CONSISTENT_SCORES = 1

# Every symbol include/dc_attn.h and include/dc_math.h declare.
EXPORTS = ("dc_abi_version", "dc_last_error",
           "dc_sdpa_fwd_workspace_size", "dc_sdpa_fwd",
           "dc_sdpa_bwd_workspace_size", "dc_sdpa_bwd",
           "dc_sdpa_decode_workspace_size", "dc_sdpa_decode",
           "dc_sdpa_fwd_schedule", "dc_sdpa_bwd_schedule", "dc_sdpa_decode_noalloc",
           "dc_bmm", "dc_softmax_fwd", "dc_softmax_bwd",
           "dc_mt19937_seed", "dc_mt19937_advance", "dc_mt19937_table_bytes",
           "dc_mt19937_table_init", "dc_bernoulli_max_draws", "dc_bernoulli_workspace_size",
           "dc_bernoulli", "dc_dropout_apply")


class Desc(ctypes.Structure):
    """``dc_attn_desc``."""
    _fields_ = [("batch", ctypes.c_int64), ("heads", ctypes.c_int64), ("kv_heads", ctypes.c_int64),
                ("q_len", ctypes.c_int64), ("kv_len", ctypes.c_int64), ("head_dim", ctypes.c_int64),
                ("causal", ctypes.c_int32), ("has_scale", ctypes.c_int32), ("scale", ctypes.c_double),
                ("dtype", ctypes.c_int32), ("flags", ctypes.c_int32),
                ("mask_stride_b", ctypes.c_int64), ("mask_stride_h", ctypes.c_int64),
                ("mask_stride_l", ctypes.c_int64)]


class Schedule(ctypes.Structure):
    """``dc_sdpa_schedule``."""
    _fields_ = [("split_chunk", ctypes.c_int32), ("split_pieces", ctypes.c_int32),
                ("streamk_ranges", ctypes.c_int32), ("split_chunk_k", ctypes.c_int32),
                ("split_chunk_q", ctypes.c_int32), ("f16_products", ctypes.c_int32),
                ("deterministic", ctypes.c_int32), ("materialized_rows", ctypes.c_int32),
                ("workgroups", ctypes.c_int64), ("chunks", ctypes.c_int32), ("reserved", ctypes.c_int32)]

    def as_dict(self):
        return {name: getattr(self, name) for name, _ in self._fields_}


class BmmDesc(ctypes.Structure):
    """``dc_bmm_desc``."""
    _fields_ = [("batch", ctypes.c_int64), ("m", ctypes.c_int64), ("n", ctypes.c_int64),
                ("k", ctypes.c_int64), ("a_stride_batch", ctypes.c_int64), ("a_stride_m", ctypes.c_int64),
                ("a_stride_k", ctypes.c_int64), ("b_stride_batch", ctypes.c_int64),
                ("b_stride_k", ctypes.c_int64), ("b_stride_n", ctypes.c_int64)]


class SoftmaxDesc(ctypes.Structure):
    """``dc_softmax_desc``."""
    _fields_ = [("rows", ctypes.c_int64), ("width", ctypes.c_int64), ("heads", ctypes.c_int64),
                ("q_len", ctypes.c_int64), ("mask_stride_b", ctypes.c_int64),
                ("mask_stride_h", ctypes.c_int64), ("mask_stride_l", ctypes.c_int64),
                ("safe", ctypes.c_int32), ("reserved", ctypes.c_int32)]


_lib = None


def lib():
    """The loaded library; raises if it has not been built."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"densecore_amd: HIP library not built ({LIB_PATH}); "
                               "run densecore_amd.build.build() (hipcc, gfx950)")
        L = ctypes.CDLL(LIB_PATH)
        P, SZ, D = ctypes.c_void_p, ctypes.c_size_t, ctypes.POINTER(Desc)
        L.dc_abi_version.restype = ctypes.c_int
        L.dc_last_error.restype = ctypes.c_char_p
        for name in ("dc_sdpa_fwd_workspace_size", "dc_sdpa_bwd_workspace_size",
                     "dc_sdpa_decode_workspace_size"):
            getattr(L, name).argtypes = [D]
            getattr(L, name).restype = SZ
        L.dc_sdpa_fwd.argtypes = [D, P, P, P, P, P, P, P, SZ, P]
        L.dc_sdpa_bwd.argtypes = [D, P, P, P, P, P, P, P, P, P, P, P, SZ, P]
        L.dc_sdpa_decode.argtypes = [D, P, P, P, P, P, P, SZ, P]
        L.dc_sdpa_decode_noalloc.argtypes = [D, P, P, P, P, P, P]
        L.dc_sdpa_decode_noalloc.restype = ctypes.c_int
        for name in ("dc_sdpa_fwd_schedule", "dc_sdpa_bwd_schedule"):
            getattr(L, name).argtypes = [D, ctypes.c_int, SZ, ctypes.POINTER(Schedule)]
            getattr(L, name).restype = ctypes.c_int
        L.dc_bmm.argtypes = [ctypes.POINTER(BmmDesc), P, P, P, P]
        L.dc_bmm.restype = ctypes.c_int
        SD = ctypes.POINTER(SoftmaxDesc)
        L.dc_softmax_fwd.argtypes = [SD, P, P, P, P]
        L.dc_softmax_bwd.argtypes = [SD, P, P, P, P]
        I64P = ctypes.POINTER(ctypes.c_int64)
        L.dc_mt19937_seed.argtypes = [ctypes.c_uint64, P]
        L.dc_mt19937_seed.restype = None
        L.dc_mt19937_advance.argtypes = [P, I64P, I64P, ctypes.c_uint64]
        L.dc_mt19937_table_bytes.argtypes = []
        L.dc_mt19937_table_bytes.restype = SZ
        L.dc_mt19937_table_init.argtypes = [P, P]
        L.dc_bernoulli_max_draws.argtypes = []
        L.dc_bernoulli_max_draws.restype = ctypes.c_int64
        L.dc_bernoulli_workspace_size.argtypes = [ctypes.c_int64]
        L.dc_bernoulli_workspace_size.restype = SZ
        L.dc_bernoulli.argtypes = [P, P, I64P, I64P, ctypes.c_int64, ctypes.c_double, P, P, SZ, P]
        L.dc_dropout_apply.argtypes = [P, ctypes.c_int64, ctypes.c_float, P, P, P]
        for name in ("dc_sdpa_fwd", "dc_sdpa_bwd", "dc_sdpa_decode", "dc_softmax_fwd",
                     "dc_softmax_bwd", "dc_mt19937_advance", "dc_mt19937_table_init",
                     "dc_bernoulli", "dc_dropout_apply"):
            getattr(L, name).restype = ctypes.c_int
        _lib = L
    return _lib


def check(status):
    """Map a dc_status to the exception the reference raises for it (src/lib.rs:555-683)."""
    if status == DC_OK:
        return
    msg = lib().dc_last_error().decode()
    if status == DC_INVALID_ARGUMENT:
        raise ValueError(msg)
    if status == DC_UNSUPPORTED:
        raise NotImplementedError(msg)
    raise RuntimeError(msg)
