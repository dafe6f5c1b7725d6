"""Every kernel writes only inside its outputs and its workspace.

Each output (out, lse; dq, dk, dv) and the workspace sit inside a larger buffer whose guard bands
before and after are filled with a byte pattern; after the call (through the C ABI, on the
schedule the case is for, which the schedule query confirms) every guard byte must be unchanged
and the outputs must meet the bar against the oracle, so a write past the end of any output or
of the workspace region the call was given fails the test.  Cases: the float32 and bf16 forwards
whole and split, the key-padding order, the float32 backward whole, stream-K, in pieces and with
only dsum (atomics), the bf16 backward whole and split, head dims above 128 over several row
blocks, decode with a workspace, and the allocation-free decode.
"""
import numpy as np
import pytest

from tests._data import assert_bf16, assert_f32, bf16_round

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu

DEV = "cuda:0"
GUARD = 4096          # bytes on each side (keeps the inner region 256-byte aligned)
PATTERN = 0xA5


class Guarded:
    """A tensor of `shape` / `dtype` (or `nbytes` raw bytes) inside guard bands of PATTERN."""

    def __init__(self, shape=None, dtype=torch.float32, nbytes=None, fill=float("nan")):
        esize = torch.empty((), dtype=dtype).element_size()
        self.nbytes = int(nbytes) if nbytes is not None else int(np.prod(shape)) * esize
        self.buf = torch.full((GUARD + self.nbytes + GUARD,), PATTERN, dtype=torch.uint8, device=DEV)
        inner = self.buf[GUARD:GUARD + self.nbytes]
        self.t = inner.view(dtype).view(shape) if shape is not None else inner
        if shape is not None and fill is not None:
            self.t.fill_(fill)

    def ptr(self):
        return self.t.data_ptr() if self.nbytes else None

    def intact(self):
        torch.cuda.synchronize()
        g = torch.cat([self.buf[:GUARD], self.buf[GUARD + self.nbytes:]])
        return bool((g == PATTERN).all())


def _ws_for_rows(backward, tq, tk, tv, causal, full, rows):
    """A workspace size (multiple of 256) whose materialized row blocks (head dims above 128) hold
    at most `rows` rows, found with the schedule query."""
    from densecore_amd import _native
    nbytes = full
    while True:
        s = _native._schedule(backward, tq, tk, tv, causal, workspace_bytes=nbytes)
        if 0 < s["materialized_rows"] <= rows:
            return nbytes
        assert s["materialized_rows"] > rows, s
        nbytes = (nbytes - nbytes // 16) // 256 * 256


def _inputs(rng, B, H, Hkv, L, S, E, bf16):
    q, g = (rng.standard_normal((B, H, L, E), dtype=np.float32) for _ in range(2))
    k, v = (rng.standard_normal((B, Hkv, S, E), dtype=np.float32) for _ in range(2))
    if bf16:
        q, k, v, g = (bf16_round(x) for x in (q, k, v, g))
    return q, k, v, g


def _dev(x, bf16):
    return torch.from_numpy(np.ascontiguousarray(x)).to(DEV, torch.bfloat16 if bf16 else torch.float32)


FWD = [  # tag, B, H, Hkv, L, S, E, causal, bf16, mask, expected plan
    ("f32_whole", 8, 12, 12, 1024, 1024, 64, True, False, None, "whole"),
    ("f32_one_wave", 2, 4, 4, 200, 200, 64, True, False, None, "any"),
    ("f32_split", 1, 2, 2, 2048, 2048, 64, True, False, None, "split"),
    ("f32_padding_order", 3, 4, 4, 256, 384, 64, False, False, "padding", "any"),
    ("bf16_split", 1, 2, 2, 2048, 2048, 128, True, True, None, "split"),
    ("bf16_grouped", 2, 16, 8, 1024, 1024, 128, True, True, None, "any"),
    ("f32_wide_rows", 1, 2, 2, 200, 300, 160, True, False, None, "rows"),
    ("bf16_wide_rows", 2, 2, 1, 150, 150, 320, False, True, None, "rows"),
    ("bf16_flash_d256", 2, 4, 2, 300, 300, 256, True, True, None, "whole"),
    ("bf16_flash_d200_padding", 3, 2, 2, 100, 250, 200, False, True, "padding", "any"),
]


@pytest.mark.parametrize("tag,B,H,Hkv,L,S,E,causal,bf16,mask,plan", FWD, ids=[c[0] for c in FWD])
def test_forward_writes_in_bounds(oracle_lib, tag, B, H, Hkv, L, S, E, causal, bf16, mask, plan):
    from densecore_amd import _lib, _native
    rng = np.random.default_rng(sum(map(ord, tag)))
    q, k, v, _ = _inputs(rng, B, H, Hkv, L, S, E, bf16)
    madd, tm = None, None
    if mask == "padding":
        lengths = rng.integers(1, S + 1, size=B)
        madd = np.where(np.arange(S)[None, :] < lengths[:, None], np.float32(0), np.float32(-np.inf))
        madd = np.ascontiguousarray(np.broadcast_to(madd[:, None, None, :], (B, H, L, S)))
        tm = torch.from_numpy(np.ascontiguousarray(madd[:, :1, :1, :])).to(DEV).expand(B, H, L, S)
    print(f"[case] bounds forward {tag}", flush=True)
    dt = torch.bfloat16 if bf16 else torch.float32
    tq, tk, tv = (_dev(x, bf16) for x in (q, k, v))
    dims = (B, H, Hkv, L, S, E)
    ms = (0, 0, 0) if tm is None else (tm.stride(0), tm.stride(1), tm.stride(2))
    d = _native._desc(dims, causal, None, dt, ms)
    L_ = _lib.lib()
    nbytes = int(L_.dc_sdpa_fwd_workspace_size(d))
    if plan == "rows":
        nbytes = _ws_for_rows(False, tq, tk, tv, causal, nbytes, (H // Hkv) * L // 3)
    sched = _native._schedule(False, tq, tk, tv, causal, mask=tm, workspace_bytes=nbytes)
    print(f"[schedule] {sched}", flush=True)
    if plan == "split":
        assert sched["split_chunk"] > 0, sched
    elif plan == "whole":
        assert sched["split_chunk"] == 0 and sched["materialized_rows"] == 0, sched
    elif plan == "rows":
        assert 0 < sched["materialized_rows"] < (H // Hkv) * L, sched
    out, lse = Guarded((B, H, L, E), dt), Guarded((B, H, L))
    ws = Guarded(nbytes=nbytes, fill=None)
    ws.t.fill_(0xFF)  # NaN as float32
    _lib.check(L_.dc_sdpa_fwd(d, tq.data_ptr(), tk.data_ptr(), tv.data_ptr(),
                              None if tm is None else tm.data_ptr(), out.ptr(), lse.ptr(), ws.ptr(),
                              nbytes, _native._stream(tq.device)))
    for name, gbuf in (("out", out), ("lse", lse), ("workspace", ws)):
        assert gbuf.intact(), f"{tag}: a write landed outside {name}"
    ref_o, ref_l = oracle_lib.forward(q, k, v, causal, None, madd)
    check = assert_bf16 if bf16 else assert_f32
    check(out.t.float().cpu().numpy(), ref_o, f"{tag} out")
    check(lse.t.cpu().numpy(), ref_l, f"{tag} lse")


BWD = [  # tag, B, H, Hkv, L, S, E, causal, bf16, workspace bytes ("full", "min" or a number), plan
    ("f32_whole", 8, 12, 12, 1024, 1024, 64, True, False, "full", "whole"),
    ("f32_streamk", 1, 8, 8, 2048, 2048, 64, True, False, "full", "streamk"),
    ("f32_streamk_grouped_e128", 2, 8, 2, 640, 640, 128, True, False, "full", "streamk"),
    ("f32_min_atomics", 1, 4, 4, 700, 900, 64, False, False, "min", "atomics"),
    ("f32_pieces", 16, 16, 16, 1024, 1024, 64, True, False, 160 << 20, "pieces"),
    ("bf16_masked_whole", 2, 8, 4, 600, 700, 128, False, True, "full", "whole"),
    ("bf16_split", 1, 2, 2, 2048, 2048, 128, True, True, "full", "split"),
    ("f32_wide_rows", 1, 2, 2, 200, 300, 192, True, False, "rows", "rows"),
    ("bf16_flash_d256", 2, 4, 2, 300, 300, 256, True, True, "full", "whole"),
    ("bf16_flash_d256_min", 1, 2, 2, 200, 260, 256, False, True, "min", "any"),
]


@pytest.mark.parametrize("tag,B,H,Hkv,L,S,E,causal,bf16,wsb,plan", BWD, ids=[c[0] for c in BWD])
def test_backward_writes_in_bounds(oracle_lib, tag, B, H, Hkv, L, S, E, causal, bf16, wsb, plan):
    from densecore_amd import _lib, _native
    rng = np.random.default_rng(sum(map(ord, tag)) + 1)
    q, k, v, g = _inputs(rng, B, H, Hkv, L, S, E, bf16)
    print(f"[case] bounds backward {tag}", flush=True)
    dt = torch.bfloat16 if bf16 else torch.float32
    tq, tk, tv, tg = (_dev(x, bf16) for x in (q, k, v, g))
    mk, tm = None, None
    if "masked" in tag:  # a float mask with -inf holes (no split grids under a mask)
        mk = rng.standard_normal((B, H, L, S)).astype(np.float32)
        mk[rng.random((B, H, L, S)) < 0.2] = -np.inf
        tm = torch.from_numpy(mk).to(DEV)
    out, lse = _native._flash_attention(tq, tk, tv, causal, None, tm)
    dims = (B, H, Hkv, L, S, E)
    ms = (0, 0, 0) if tm is None else (tm.stride(0), tm.stride(1), tm.stride(2))
    d = _native._desc(dims, causal, None, dt, ms)
    L_ = _lib.lib()
    full = int(L_.dc_sdpa_bwd_workspace_size(d))
    dsum = (B * H * L * 4 + 255) // 256 * 256
    nbytes = {"full": full, "min": dsum}.get(wsb, wsb)
    if wsb == "rows":
        nbytes = _ws_for_rows(True, tq, tk, tv, causal, full, (H // Hkv) * L // 3)
    sched = _native._schedule(True, tq, tk, tv, causal, mask=tm, workspace_bytes=nbytes)
    print(f"[schedule] {sched}", flush=True)
    expect = {"whole": lambda s: s["streamk_ranges"] == 0 and s["split_chunk_k"] == 0 and s["chunks"] == 1
                       and s["materialized_rows"] == 0,
              "any": lambda s: True,
              "streamk": lambda s: s["streamk_ranges"] > 0 and s["deterministic"] == 1,
              "atomics": lambda s: s["deterministic"] == 0,
              "pieces": lambda s: s["chunks"] > 1 and s["deterministic"] == 1,
              "split": lambda s: s["split_chunk_k"] > 0 or s["split_chunk_q"] > 0,
              "rows": lambda s: 0 < s["materialized_rows"] < (H // Hkv) * L}[plan]
    assert expect(sched), sched
    dq, dk, dv = Guarded((B, H, L, E), dt), Guarded((B, Hkv, S, E), dt), Guarded((B, Hkv, S, E), dt)
    ws = Guarded(nbytes=nbytes, fill=None)
    ws.t.fill_(0xFF)
    _lib.check(L_.dc_sdpa_bwd(d, tg.data_ptr(), tq.data_ptr(), tk.data_ptr(), tv.data_ptr(), out.data_ptr(),
                              lse.data_ptr(), None if tm is None else tm.data_ptr(), dq.ptr(), dk.ptr(),
                              dv.ptr(), ws.ptr(), nbytes,
                              _native._stream(tq.device)))
    for name, gbuf in (("dq", dq), ("dk", dk), ("dv", dv), ("workspace", ws)):
        assert gbuf.intact(), f"{tag}: a write landed outside {name}"
    on, ln = out.float().cpu().numpy(), lse.cpu().numpy()
    ref = oracle_lib.backward(g, q, k, v, on, ln, causal, None, mk)
    check = assert_bf16 if bf16 else assert_f32
    for name, a, r in zip(("dq", "dk", "dv"), (dq, dk, dv), ref):
        check(a.t.float().cpu().numpy(), r, f"{tag} {name}")


@pytest.mark.parametrize("noalloc", [False, True])
@pytest.mark.parametrize("B,H,Hkv,S,E,bf16", [(4, 8, 8, 4096, 128, False), (3, 6, 2, 1000, 64, True),
                                             (2, 4, 4, 333, 256, False)])
def test_decode_writes_in_bounds(oracle_lib, noalloc, B, H, Hkv, S, E, bf16):
    from densecore_amd import _lib, _native
    rng = np.random.default_rng(B * 7 + S + E)
    q, k, v, _ = _inputs(rng, B, H, Hkv, 1, S, E, bf16)
    print(f"[case] bounds decode noalloc={noalloc} B{B} H{H} Hkv{Hkv} S{S} E{E} bf16={bf16}", flush=True)
    dt = torch.bfloat16 if bf16 else torch.float32
    tq, tk, tv = (_dev(x, bf16) for x in (q, k, v))
    d = _native._desc((B, H, Hkv, 1, S, E), False, None, dt, (0, 0, 0))
    L_ = _lib.lib()
    out, lse = Guarded((B, H, 1, E), dt), Guarded((B, H, 1))
    stream = _native._stream(tq.device)
    if noalloc:
        _lib.check(L_.dc_sdpa_decode_noalloc(d, tq.data_ptr(), tk.data_ptr(), tv.data_ptr(), out.ptr(),
                                             lse.ptr(), stream))
        gbufs = (("out", out), ("lse", lse))
    else:
        nbytes = int(L_.dc_sdpa_decode_workspace_size(d))
        ws = Guarded(nbytes=nbytes, fill=None)
        _lib.check(L_.dc_sdpa_decode(d, tq.data_ptr(), tk.data_ptr(), tv.data_ptr(), out.ptr(), lse.ptr(),
                                     ws.ptr(), nbytes, stream))
        gbufs = (("out", out), ("lse", lse), ("workspace", ws))
    for name, gbuf in gbufs:
        assert gbuf.intact(), f"decode: a write landed outside {name}"
    ref_o, ref_l = oracle_lib.forward(q, k, v, False)
    check = assert_bf16 if bf16 else assert_f32
    check(out.t.float().cpu().numpy(), ref_o, "decode out")
    check(lse.t.cpu().numpy(), ref_l, "decode lse")
