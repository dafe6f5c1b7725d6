"""GPU parity of the kernels under their alternative schedules.

Forward (float32, and bf16 with its fp16 copy of V): when the grid of query tiles fills at most
half of the workgroups that fit at once (few heads, long rows; no mask), the key tiles of each
query tile run as pieces of at least 4 tiles,
each writing a normalized partial output and lse, merged by a second kernel (rows of query tiles
that ran whole are written directly).  The cases below take that path on MI355X; out and lse
start as NaN, so a row neither path writes fails.

Backward (bf16, with its fp16 copies): on grids that fill at most half of the device, the dK/dV
kernel's key tiles run as pieces over their query steps and the dQ kernel's query tiles as pieces
over their key tiles, each piece writing float32 partials that a reduction sums in piece order.

Backward (float32): the backward either gives each key tile (128 keys of one kv head) to one workgroup, or, when
whole tiles would leave part of the device idle (fewer tiles than resident workgroups, or a
ragged last wave of equal non-causal tiles), cuts the steps of all tiles into equal ranges, one
per resident workgroup (stream-K).  A tile cut between ranges leaves each range's dK / dV share in a slot
of the workspace, summed in range order by a reduction (with only dsum in the workspace, the
shares are added atomically into rows the pre-kernel cleared; tiles without steps, causal keys
past the last query, are cleared there too).  These
cases call the C ABI with dQ, dK and dV pre-filled with NaN, so a row neither schedule writes
fails.  On MI355X (256 CUs) the shapes marked "whole" take the one-tile-per-workgroup grid, the
others stream-K.  Tolerance, as for every float32 output: |gpu - ref| <= 2e-5 + 1e-5 |ref|.
"""
import numpy as np
import pytest

from tests._data import assert_bf16, assert_f32, bf16_round

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu

DEV = "cuda:0"


def _t(x):
    return torch.from_numpy(np.ascontiguousarray(x)).to(DEV)


def _forward_nan_filled(q, k, v, causal, dtype=None):
    from densecore_amd import _lib, _native
    dtype = dtype or torch.float32
    q, k, v = (_t(x).to(dtype) for x in (q, k, v))
    dims = _native._attention_dims(q, k, v)
    B, H, Hkv, L, S, E = dims
    out = torch.full((B, H, L, E), float("nan"), device=DEV, dtype=dtype)
    lse = torch.full((B, H, L), float("nan"), device=DEV)
    d = _native._desc(dims, causal, None, dtype, (0, 0, 0))
    L_ = _lib.lib()
    ws = _native._workspace(L_.dc_sdpa_fwd_workspace_size(d), q.device)
    sched = _native._schedule(False, q, k, v, causal, workspace_bytes=ws.numel())
    print(f"[schedule] {sched}", flush=True)
    _lib.check(L_.dc_sdpa_fwd(d, _native._ptr(q), _native._ptr(k), _native._ptr(v), None,
                              _native._ptr(out), _native._ptr(lse), _native._ptr(ws), ws.numel(),
                              _native._stream(q.device)))
    torch.cuda.synchronize()
    return out.float().cpu().numpy(), lse.cpu().numpy(), sched


FWD_CASES = [  # tag, B, H, Hkv, L, S, E, causal
    ("causal_long", 1, 2, 2, 2048, 2048, 64, True),
    ("full_l_ne_s", 1, 3, 3, 1500, 1700, 64, False),
    ("causal_e128", 1, 2, 2, 700, 700, 128, True),
    ("causal_e32", 1, 2, 2, 2048, 2048, 32, True),
    ("grouped", 2, 4, 2, 1024, 1024, 64, True),
    ("unaligned_e40", 1, 1, 1, 333, 2000, 40, False),
    ("single_query", 1, 2, 2, 1, 5000, 64, False),
    ("causal_l_gt_s", 1, 2, 2, 1200, 600, 64, True),
]


@pytest.mark.parametrize("tag,B,H,Hkv,L,S,E,causal", FWD_CASES, ids=[c[0] for c in FWD_CASES])
def test_forward_split_ranges(oracle_lib, tag, B, H, Hkv, L, S, E, causal):
    rng = np.random.default_rng(sum(map(ord, tag)) + 1)
    q = rng.standard_normal((B, H, L, E), dtype=np.float32)
    k = rng.standard_normal((B, Hkv, S, E), dtype=np.float32)
    v = rng.standard_normal((B, Hkv, S, E), dtype=np.float32)
    print(f"[case] forward split {tag} B{B} H{H} Hkv{Hkv} L{L} S{S} E{E} causal={causal}", flush=True)
    ref_o, ref_l = oracle_lib.forward(q, k, v, causal)
    out, lse, sched = _forward_nan_filled(q, k, v, causal)
    assert sched["split_chunk"] > 0 and sched["split_pieces"] > 1, f"{tag}: no split ran: {sched}"
    assert_f32(out, ref_o, f"{tag} out")
    assert_f32(lse, ref_l, f"{tag} lse")


BF16_FWD_CASES = [  # tag, B, H, Hkv, L, S, E, causal (256-query tiles, 64-key tiles)
    ("causal_e128", 1, 2, 2, 2048, 2048, 128, True),
    ("full_e64", 1, 1, 1, 1000, 4096, 64, False),
    ("grouped_e128", 1, 4, 2, 1024, 1024, 128, True),
    ("causal_e32", 2, 1, 1, 1536, 1536, 32, True),
    ("unaligned_e40", 1, 1, 1, 700, 2500, 40, False),
    ("single_query", 1, 3, 3, 1, 5000, 128, False),
]


@pytest.mark.parametrize("tag,B,H,Hkv,L,S,E,causal", BF16_FWD_CASES, ids=[c[0] for c in BF16_FWD_CASES])
def test_bf16_forward_split_ranges(oracle_lib, tag, B, H, Hkv, L, S, E, causal):
    """The bf16 forward's split path (fp16 P V product, pieces merged into bf16 out) against the
    oracle on the bf16-rounded inputs, to the bf16 bar |gpu - ref| <= 1e-2 |ref| + 1e-2 rms."""
    rng = np.random.default_rng(sum(map(ord, tag)) + 2)
    q = bf16_round(rng.standard_normal((B, H, L, E), dtype=np.float32))
    k = bf16_round(rng.standard_normal((B, Hkv, S, E), dtype=np.float32))
    v = bf16_round(rng.standard_normal((B, Hkv, S, E), dtype=np.float32))
    print(f"[case] bf16 forward split {tag} B{B} H{H} Hkv{Hkv} L{L} S{S} E{E} causal={causal}", flush=True)
    ref_o, ref_l = oracle_lib.forward(q, k, v, causal)
    out, lse, sched = _forward_nan_filled(q, k, v, causal, torch.bfloat16)
    assert sched["split_chunk"] > 0 and sched["f16_products"] == 1, f"{tag}: no split ran: {sched}"
    assert_bf16(out, ref_o, f"{tag} out")
    assert_bf16(lse, ref_l, f"{tag} lse")


BF16_BWD_CASES = [  # tag, B, H, Hkv, L, S, E, causal
    ("causal_e128", 1, 2, 2, 2048, 2048, 128, True),
    ("full_e64", 1, 1, 1, 4096, 4096, 64, False),
    ("grouped_e128", 1, 4, 2, 1024, 1024, 128, True),
    ("causal_s_gt_l", 1, 2, 2, 700, 1500, 64, True),   # key tiles past L have no steps
    ("causal_l_gt_s", 1, 2, 2, 1500, 600, 128, True),
    ("causal_e32", 2, 1, 1, 1536, 1536, 32, True),
    ("unaligned_e40", 1, 1, 1, 700, 900, 40, False),
]


@pytest.mark.parametrize("tag,B,H,Hkv,L,S,E,causal", BF16_BWD_CASES, ids=[c[0] for c in BF16_BWD_CASES])
def test_bf16_backward_split_grids(oracle_lib, tag, B, H, Hkv, L, S, E, causal):
    """The bf16 backward's split grids (dK/dV pieces over query steps, dQ pieces over key tiles,
    float32 partials summed in piece order) against the oracle's backward from the GPU's own bf16
    out and lse, to the bf16 bar; dq, dk, dv start as NaN."""
    from densecore_amd import _lib, _native
    rng = np.random.default_rng(sum(map(ord, tag)) + 3)
    q, g = (bf16_round(rng.standard_normal((B, H, L, E), dtype=np.float32)) for _ in range(2))
    k, v = (bf16_round(rng.standard_normal((B, Hkv, S, E), dtype=np.float32)) for _ in range(2))
    print(f"[case] bf16 backward split {tag} B{B} H{H} Hkv{Hkv} L{L} S{S} E{E} causal={causal}", flush=True)
    tq, tk, tv, tg = (_t(x).to(torch.bfloat16) for x in (q, k, v, g))
    out, lse = _native._flash_attention(tq, tk, tv, causal)
    torch.cuda.synchronize()
    ref = oracle_lib.backward(g, q, k, v, out.float().cpu().numpy(), lse.cpu().numpy(), causal)
    dims = _native._attention_dims(tq, tk, tv)
    dq = torch.full((B, H, L, E), float("nan"), device=DEV, dtype=torch.bfloat16)
    dk = torch.full((B, Hkv, S, E), float("nan"), device=DEV, dtype=torch.bfloat16)
    dv = torch.full((B, Hkv, S, E), float("nan"), device=DEV, dtype=torch.bfloat16)
    d = _native._desc(dims, causal, None, torch.bfloat16, (0, 0, 0))
    L_ = _lib.lib()
    ws = _native._workspace(L_.dc_sdpa_bwd_workspace_size(d), tq.device)
    sched = _native._schedule(True, tq, tk, tv, causal, workspace_bytes=ws.numel())
    print(f"[schedule] {sched}", flush=True)
    assert sched["f16_products"] == 1 and (sched["split_chunk_k"] > 0 or sched["split_chunk_q"] > 0), \
        f"{tag}: no split grid ran: {sched}"
    assert sched["deterministic"] == 1
    _lib.check(L_.dc_sdpa_bwd(d, _native._ptr(tg), _native._ptr(tq), _native._ptr(tk), _native._ptr(tv),
                              _native._ptr(out), _native._ptr(lse), None, _native._ptr(dq), _native._ptr(dk),
                              _native._ptr(dv), _native._ptr(ws), ws.numel(), _native._stream(tq.device)))
    torch.cuda.synchronize()
    for name, a, b in zip(("dq", "dk", "dv"), (dq, dk, dv), ref):
        assert_bf16(a.float().cpu().numpy(), b, f"{tag} {name}")


def _backward_nan_filled(g, q, k, v, out, lse, causal, mask=None):
    from densecore_amd import _lib, _native
    g, q, k, v, out, lse = (_t(x) for x in (g, q, k, v, out, lse))
    dims = _native._attention_dims(q, k, v)
    B, H, Hkv, L, S, E = dims
    m, ms = _native._mask_arg(None if mask is None else _t(mask), dims, q.device)
    dq = torch.full((B, H, L, E), float("nan"), device=DEV)
    dk = torch.full((B, Hkv, S, E), float("nan"), device=DEV)
    dv = torch.full((B, Hkv, S, E), float("nan"), device=DEV)
    d = _native._desc(dims, causal, None, torch.float32, ms)
    L_ = _lib.lib()
    ws = _native._workspace(L_.dc_sdpa_bwd_workspace_size(d), q.device)
    sched = _native._schedule(True, q, k, v, causal, mask=m, workspace_bytes=ws.numel())
    print(f"[schedule] {sched}", flush=True)
    _lib.check(L_.dc_sdpa_bwd(d, _native._ptr(g), _native._ptr(q), _native._ptr(k), _native._ptr(v),
                              _native._ptr(out), _native._ptr(lse), _native._ptr(m), _native._ptr(dq),
                              _native._ptr(dk), _native._ptr(dv), _native._ptr(ws), ws.numel(),
                              _native._stream(q.device)))
    torch.cuda.synchronize()
    return [x.cpu().numpy() for x in (dq, dk, dv)], sched


CASES = [  # tag, B, H, Hkv, L, S, E, causal, mask
    ("c2_like", 2, 6, 6, 1024, 1024, 64, True, None),
    ("causal_s_gt_l", 1, 4, 4, 300, 700, 64, True, None),     # tiles 3..5 have no steps
    ("causal_l_gt_s", 2, 2, 2, 900, 260, 32, True, None),
    ("noncausal_e128", 1, 3, 3, 500, 640, 128, False, None),
    ("grouped", 2, 8, 2, 640, 640, 64, True, None),
    ("masked_causal", 1, 2, 2, 384, 384, 64, True, "float"),
    ("unaligned_e40", 1, 3, 3, 333, 333, 40, True, None),
    ("ragged_noncausal", 6, 16, 16, 1024, 1024, 32, False, None),  # 1.5 waves of tiles
    ("whole_causal", 16, 16, 16, 1024, 1024, 32, True, None),
    ("whole_noncausal", 16, 16, 16, 512, 512, 32, False, None),
]


@pytest.mark.parametrize("tag,B,H,Hkv,L,S,E,causal,mask", CASES, ids=[c[0] for c in CASES])
def test_backward_schedules(oracle_lib, tag, B, H, Hkv, L, S, E, causal, mask):
    rng = np.random.default_rng(sum(map(ord, tag)))
    q = rng.standard_normal((B, H, L, E), dtype=np.float32)
    k = rng.standard_normal((B, Hkv, S, E), dtype=np.float32)
    v = rng.standard_normal((B, Hkv, S, E), dtype=np.float32)
    g = rng.standard_normal((B, H, L, E), dtype=np.float32)
    m = None
    if mask == "float":
        m = rng.standard_normal((B, H, L, S), dtype=np.float32)
        m[rng.random((B, H, L, S)) < 0.2] = -np.inf
    print(f"[case] backward schedule {tag} B{B} H{H} Hkv{Hkv} L{L} S{S} E{E} causal={causal}",
          flush=True)
    ref_o, ref_l = oracle_lib.forward(q, k, v, causal, None, m)
    rq, rk, rv = oracle_lib.backward(g, q, k, v, ref_o, ref_l, causal, None, m)
    (dq, dk, dv), sched = _backward_nan_filled(g, q, k, v, ref_o, ref_l, causal, m)
    if tag.startswith("whole"):
        assert sched["streamk_ranges"] == 0, f"{tag}: expected whole key tiles: {sched}"
    else:
        assert sched["streamk_ranges"] > 0, f"{tag}: expected the stream-K schedule: {sched}"
    assert_f32(dq, rq, f"{tag} dq")
    assert_f32(dk, rk, f"{tag} dk")
    assert_f32(dv, rv, f"{tag} dv")


@pytest.mark.parametrize("dtype", ["f32", "bf16"])
def test_split_shapes_without_split_workspace(oracle_lib, dtype):
    """Shapes that split when given the full workspace, run with less: the forward with none at
    all (whole query tiles, and for bf16 the hi + lo P V product), the backward with the float32
    minimum (dsum only) or, for bf16, exactly the fp16 copies without the split partials (the
    whole-tile grids).  Results still meet the bar."""
    from densecore_amd import _lib, _native
    B, H, L, E, causal = 1, 2, 1536, 128, True
    bf16 = dtype == "bf16"
    rng = np.random.default_rng(77 if bf16 else 78)
    q, k, v, g = (rng.standard_normal((B, H, L, E), dtype=np.float32) for _ in range(4))
    if bf16:
        q, k, v, g = (bf16_round(x) for x in (q, k, v, g))
    dt = torch.bfloat16 if bf16 else torch.float32
    tq, tk, tv, tg = (_t(x).to(dt) for x in (q, k, v, g))
    dims = _native._attention_dims(tq, tk, tv)
    d = _native._desc(dims, causal, None, dt, (0, 0, 0))
    L_ = _lib.lib()
    stream = _native._stream(tq.device)
    print(f"[case] reduced workspaces {dtype} B{B} H{H} L{L} E{E}", flush=True)
    assert L_.dc_sdpa_fwd_workspace_size(d) > 256  # the full size holds split partials
    assert _native._schedule(False, tq, tk, tv, causal)["split_chunk"] > 0
    assert _native._schedule(False, tq, tk, tv, causal, workspace_bytes=0)["split_chunk"] == 0
    out = torch.full((B, H, L, E), float("nan"), device=DEV, dtype=dt)
    lse = torch.full((B, H, L), float("nan"), device=DEV)
    _lib.check(L_.dc_sdpa_fwd(d, _native._ptr(tq), _native._ptr(tk), _native._ptr(tv), None, _native._ptr(out),
                              _native._ptr(lse), None, 0, stream))
    torch.cuda.synchronize()
    ref_o, ref_l = oracle_lib.forward(q, k, v, causal)
    check = assert_bf16 if bf16 else assert_f32
    check(out.float().cpu().numpy(), ref_o, f"{dtype} out, no workspace")
    check(lse.cpu().numpy(), ref_l, f"{dtype} lse, no workspace")
    full = L_.dc_sdpa_bwd_workspace_size(d)
    # bf16: dsum + the fp16 copies = the full size minus the split partials; float32: dsum only.
    dsum_bytes = (B * H * L * 4 + 255) // 256 * 256
    less = full - 1 if bf16 else dsum_bytes
    ws = _native._workspace(less, tq.device)
    full_sched = _native._schedule(True, tq, tk, tv, causal)
    less_sched = _native._schedule(True, tq, tk, tv, causal, workspace_bytes=less)
    print(f"[schedule] full {full_sched} reduced {less_sched}", flush=True)
    if bf16:
        assert full_sched["split_chunk_k"] > 0 or full_sched["split_chunk_q"] > 0
        assert less_sched["split_chunk_k"] == 0 and less_sched["split_chunk_q"] == 0
        assert less_sched["f16_products"] == 1
    dq, dk, dv = (torch.full((B, H, L, E), float("nan"), device=DEV, dtype=dt) for _ in range(3))
    o_in = out if bf16 else _t(ref_o)
    l_in = lse if bf16 else torch.from_numpy(ref_l).to(DEV)
    _lib.check(L_.dc_sdpa_bwd(d, _native._ptr(tg), _native._ptr(tq), _native._ptr(tk), _native._ptr(tv),
                              _native._ptr(o_in), _native._ptr(l_in), None, _native._ptr(dq), _native._ptr(dk),
                              _native._ptr(dv), _native._ptr(ws), less, stream))
    torch.cuda.synchronize()
    if bf16:
        ref = oracle_lib.backward(g, q, k, v, out.float().cpu().numpy(), lse.cpu().numpy(), causal)
    else:
        ref = oracle_lib.backward(g, q, k, v, ref_o, ref_l, causal)
    for name, a, b in zip(("dq", "dk", "dv"), (dq, dk, dv), ref):
        check(a.float().cpu().numpy(), b, f"{dtype} {name}, reduced workspace")
