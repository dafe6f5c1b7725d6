"""The allocation-free decode entry point (dc_sdpa_decode_noalloc) against dc_sdpa_decode.

dc_sdpa_decode_noalloc runs the same split-KV kernels as dc_sdpa_decode, with the split partials
in a static device array instead of a caller's workspace, so its out and lse must be bit-identical
to dc_sdpa_decode's on the same inputs.  Each case makes two calls in a row through the C ABI, the
second on a smaller input (the array keeps the first call's contents; nothing may leak into the
second), and compares both with dc_sdpa_decode.  The full C4 shape (B32 H32 S4096 D128) is one of
the calls.
"""
import ctypes

import numpy as np
import pytest

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu

DEV = "cuda:0"


def _inputs(rng, B, H, Hkv, S, E, dtype):
    q = torch.from_numpy(rng.standard_normal((B, H, 1, E), dtype=np.float32)).to(DEV, dtype)
    k = torch.from_numpy(rng.standard_normal((B, Hkv, S, E), dtype=np.float32) * 0.5).to(DEV, dtype)
    v = torch.from_numpy(rng.standard_normal((B, Hkv, S, E), dtype=np.float32) * 0.5).to(DEV, dtype)
    return q, k, v


def _noalloc(q, k, v, scale=None):
    from densecore_amd import _lib, _native
    dims = _native._attention_dims(q, k, v)
    B, H, _, _, _, E = dims
    out = torch.empty((B, H, 1, E), dtype=q.dtype, device=DEV)
    lse = torch.empty((B, H, 1), dtype=torch.float32, device=DEV)
    d = _native._desc(dims, False, scale, q.dtype, (0, 0, 0))
    _lib.check(_lib.lib().dc_sdpa_decode_noalloc(ctypes.byref(d), _native._ptr(q), _native._ptr(k),
                                                 _native._ptr(v), _native._ptr(out), _native._ptr(lse),
                                                 _native._stream(q.device)))
    return out, lse


PAIRS = [  # (first call, second smaller call): B, H, Hkv, S, E, dtype
    ((32, 32, 32, 4096, 128, "f32"), (2, 4, 4, 700, 64, "f32")),
    ((4, 16, 4, 5000, 128, "bf16"), (1, 2, 1, 33, 40, "bf16")),
    ((8, 8, 8, 2048, 64, "f32"), (3, 2, 2, 129, 128, "bf16")),
]


@pytest.mark.parametrize("first,second", PAIRS, ids=["c4_then_small", "bf16_gqa", "f32_then_bf16"])
def test_noalloc_decode_matches_workspace_decode(first, second):
    from densecore_amd import _native
    rng = np.random.default_rng(2024)
    for B, H, Hkv, S, E, dt in (first, second):
        dtype = torch.bfloat16 if dt == "bf16" else torch.float32
        print(f"[case] decode_noalloc {dt} B{B} H{H} Hkv{Hkv} S{S} E{E}", flush=True)
        q, k, v = _inputs(rng, B, H, Hkv, S, E, dtype)
        out, lse = _noalloc(q, k, v)
        ref_out, ref_lse = _native._flash_decode(q, k, v)
        torch.cuda.synchronize()
        assert torch.isfinite(out.float()).all() and torch.isfinite(lse).all()
        assert torch.equal(out, ref_out), f"{dt} B{B} H{H} S{S} E{E}: out differs from dc_sdpa_decode"
        assert torch.equal(lse, ref_lse), f"{dt} B{B} H{H} S{S} E{E}: lse differs from dc_sdpa_decode"
        del q, k, v


def test_noalloc_decode_rejects_oversized_scratch():
    """More split partials than the static array holds: DC_UNSUPPORTED before any launch."""
    from densecore_amd import _lib
    d = _lib.Desc(1, 40000, 40000, 1, 64, 128, 0, 0, 0.0, _lib.DC_F32, 0, 0, 0, 0)
    st = _lib.lib().dc_sdpa_decode_noalloc(ctypes.byref(d), None, None, None, None, None, None)
    assert st == _lib.DC_UNSUPPORTED
    assert b"scratch" in _lib.lib().dc_last_error()
