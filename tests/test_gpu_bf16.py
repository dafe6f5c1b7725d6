"""GPU parity of the bfloat16 kernels (fp32 accumulation) against the float32 oracle run on
the exact float32 upcast of the same bf16 inputs.

Tolerance (the target's for bf16): |gpu - ref| <= 1e-2 |ref| + 1e-2 rms(ref), elementwise.

Each function is compared on identical inputs.  The backward takes (out, lse) as inputs, so
the oracle's backward is given the GPU forward's bf16 out (upcast) and lse: dsum = rowsum(dO *
out) formed from a bf16-rounded out differs from one formed from a float32 out by about
2^-9 |dO| |out|, which alone can exceed the elementwise bound for small gradients.

C5 (B2 H32 T8192 D128, causal) runs at full size on the GPU; the oracle checks it through
causal row windows, which is exact: query rows [a, b) of a causal problem depend only on keys
[0, b), so the oracle on (q[a:b], k[:b], v[:b]) with the mask "key <= row + a" gives those
rows' out, lse and dq; with b = T it also gives dk and dv of every key >= a."""
import numpy as np
import pytest

from tests._data import assert_bf16, assert_bf16_nan, bf16_round, make_inputs

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu

DEV = "cuda:0"


def _bf(x):
    return torch.from_numpy(np.ascontiguousarray(x, np.float32)).to(DEV).to(torch.bfloat16)


def _np(t):
    torch.cuda.synchronize()
    return t.float().cpu().numpy()


def _offset_causal(rows, keys, a):
    allowed = np.arange(keys)[None, :] <= np.arange(rows)[:, None] + a
    return np.where(allowed, np.float32(0), np.float32(-np.inf))


@pytest.mark.parametrize("B,H,Hkv,L,S,E,causal", [
    (2, 2, 2, 7, 7, 5, False), (1, 3, 3, 33, 33, 16, True), (1, 2, 2, 100, 37, 12, False),
    (1, 1, 1, 200, 200, 64, True), (2, 4, 2, 300, 300, 128, True), (1, 2, 1, 129, 257, 128, False),
    (1, 2, 2, 64, 64, 32, True), (2, 2, 2, 190, 190, 100, True),
    # one query (three keys: with one key dq is exactly 0 and the relative bar would compare
    # rounding noise), L > S and L < S under causal masking, 4 query heads per kv head, head
    # dim 1 (every tile of every kernel is partial)
    (1, 1, 1, 1, 3, 64, False), (1, 2, 2, 1, 300, 64, False), (1, 2, 2, 300, 100, 64, True),
    (1, 2, 2, 100, 300, 64, True), (1, 4, 1, 70, 70, 64, True), (2, 2, 2, 40, 40, 1, True),
])
def test_bf16_shapes(oracle_lib, B, H, Hkv, L, S, E, causal):
    from densecore_amd import _native
    rng = np.random.default_rng(L * 7 + S + E)
    q, g = (bf16_round(rng.standard_normal((B, H, L, E), dtype=np.float32)) for _ in range(2))
    k, v = (bf16_round(rng.standard_normal((B, Hkv, S, E), dtype=np.float32)) for _ in range(2))
    print(f"[case] bf16 B{B} H{H} Hkv{Hkv} L{L} S{S} E{E} causal={causal}", flush=True)
    ref_o, ref_l = oracle_lib.forward(q, k, v, causal)
    tq, tk, tv, tg = (_bf(x) for x in (q, k, v, g))
    out, lse = _native._flash_attention(tq, tk, tv, causal)
    assert out.dtype == torch.bfloat16 and lse.dtype == torch.float32
    assert_bf16(_np(out), ref_o, "out")
    assert_bf16(_np(lse), ref_l, "lse")
    ref = oracle_lib.backward(g, q, k, v, _np(out), _np(lse), causal)
    got = _native._flash_attention_backward(tg, tq, tk, tv, out, lse, causal)
    for name, a, b in zip(("dq", "dk", "dv"), got, ref):
        assert a.dtype == torch.bfloat16
        assert_bf16(_np(a), b, name)


@pytest.mark.parametrize("scale", [-0.4, 0.0, float("nan")])
@pytest.mark.parametrize("B,H,L,S,E,causal", [
    (1, 2, 300, 300, 128, True), (2, 2, 200, 200, 64, True), (1, 2, 100, 300, 64, True),
    (1, 2, 150, 170, 64, False),
])
def test_bf16_negative_and_zero_scale(oracle_lib, B, H, L, S, E, causal, scale):
    """Explicit negative, zero and NaN scales give the reference's result, NaN rows included (the
    reference scales its causal -inf fill: src/torch_attention.rs:202-216): out and lse against
    the oracle's causal forward on the upcast inputs, the same NaN elements and the bf16 bar
    elsewhere; the backward from the GPU's (out, lse) against the oracle's from the same."""
    from densecore_amd import _native
    rng = np.random.default_rng(L + 3 * S + 5 * E)
    q, g = (bf16_round(rng.standard_normal((B, H, L, E), dtype=np.float32)) for _ in range(2))
    k, v = (bf16_round(rng.standard_normal((B, H, S, E), dtype=np.float32)) for _ in range(2))
    print(f"[case] bf16 scale {scale} B{B} H{H} L{L} S{S} E{E} causal={causal}", flush=True)
    ref_o, ref_l = oracle_lib.forward(q, k, v, causal, scale)
    tq, tk, tv, tg = (_bf(x) for x in (q, k, v, g))
    out, lse = _native._flash_attention(tq, tk, tv, causal, scale)
    assert_bf16_nan(_np(out), ref_o, "out")
    assert_bf16_nan(_np(lse), ref_l, "lse")
    ref = oracle_lib.backward(g, q, k, v, _np(out), _np(lse), causal, scale)
    got = _native._flash_attention_backward(tg, tq, tk, tv, out, lse, causal, scale)
    for name, x, y in zip(("dq", "dk", "dv"), got, ref):
        assert_bf16_nan(_np(x), y, name)


def test_bf16_masked(oracle_lib):
    from densecore_amd import _native
    rng = np.random.default_rng(77)
    B, H, L, S, E = 2, 3, 150, 170, 64
    q, g = (bf16_round(rng.standard_normal((B, H, L, E), dtype=np.float32)) for _ in range(2))
    k, v = (bf16_round(rng.standard_normal((B, H, S, E), dtype=np.float32)) for _ in range(2))
    mask = np.where(rng.random((B, 1, L, S)) > 0.3, np.float32(0), np.float32(-np.inf))
    mask[0, 0, 5, :] = -np.inf  # a fully masked row
    full = np.ascontiguousarray(np.broadcast_to(mask, (B, H, L, S)))
    ref_o, ref_l = oracle_lib.forward(q, k, v, False, None, full)
    tq, tk, tv, tg = (_bf(x) for x in (q, k, v, g))
    tm = torch.from_numpy(mask).to(DEV).expand(B, H, L, S)
    out, lse = _native._flash_attention(tq, tk, tv, False, None, tm)
    assert_bf16(_np(out), ref_o, "out")
    assert_bf16(_np(lse), ref_l, "lse")
    ref = oracle_lib.backward(g, q, k, v, _np(out), _np(lse), False, None, full)
    got = _native._flash_attention_backward(tg, tq, tk, tv, out, lse, False, None, tm)
    for name, a, b in zip(("dq", "dk", "dv"), got, ref):
        assert_bf16(_np(a), b, name)


@pytest.mark.parametrize("B,H,Hkv,S,E", [(4, 8, 8, 4096, 128), (2, 4, 2, 1000, 64), (1, 2, 2, 77, 100)])
def test_bf16_decode(oracle_lib, B, H, Hkv, S, E):
    from densecore_amd import _native
    rng = np.random.default_rng(S)
    q = bf16_round(rng.standard_normal((B, H, 1, E), dtype=np.float32))
    k, v = (bf16_round(rng.standard_normal((B, Hkv, S, E), dtype=np.float32) * 0.5) for _ in range(2))
    ref_o, ref_l = oracle_lib.forward(q, k, v, False)
    out, lse = _native._flash_decode(_bf(q), _bf(k), _bf(v))
    assert_bf16(_np(out), ref_o, "decode out")
    assert_bf16(_np(lse), ref_l, "decode lse")


@pytest.fixture(scope="module")
def c5_run():
    """Full C5 forward + backward on the GPU, kept on the host for the window checks."""
    from densecore_amd import _native
    d = make_inputs("C5")
    print("[case] C5 full forward+backward (B2 H32 T8192 D128 bf16)", flush=True)
    tq, tk, tv, tg = (_bf(d[n]) for n in "qkvg")
    out, lse = _native._flash_attention(tq, tk, tv, True)
    dq, dk, dv = _native._flash_attention_backward(tg, tq, tk, tv, out, lse, True)
    res = {n: _np(x) for n, x in (("out", out), ("lse", lse), ("dq", dq), ("dk", dk), ("dv", dv))}
    for n, x in res.items():
        assert np.isfinite(x).all(), n
    return d, res


HEADS = [(0, 0), (1, 17), (0, 31), (1, 31)]  # (batch, head): first, middle and last heads


@pytest.mark.parametrize("a,b", [(0, 1024), (4096, 4224), (7168, 8192)])
def test_c5_windows(oracle_lib, c5_run, a, b):
    d, res = c5_run
    sel = lambda x, rows: np.stack([x[bi, hi, rows] for bi, hi in HEADS])[None]  # (1, len(HEADS), n, E)
    q, g = sel(d["q"], slice(a, b)), sel(d["g"], slice(a, b))
    k, v = sel(d["k"], slice(0, b)), sel(d["v"], slice(0, b))
    mask = np.ascontiguousarray(np.broadcast_to(_offset_causal(b - a, b, a), (1, len(HEADS), b - a, b)))
    print(f"[case] C5 window rows [{a}, {b})", flush=True)
    ref_o, ref_l = oracle_lib.forward(q, k, v, False, None, mask)
    assert_bf16(sel(res["out"], slice(a, b)), ref_o, f"C5 out[{a}:{b}]")
    assert_bf16(sel(res["lse"][..., None], slice(a, b))[..., 0], ref_l, f"C5 lse[{a}:{b}]")
    go, gl = sel(res["out"], slice(a, b)), sel(res["lse"][..., None], slice(a, b))[..., 0]
    rq, rk, rv = oracle_lib.backward(g, q, k, v, go, gl, False, None, mask)
    assert_bf16(sel(res["dq"], slice(a, b)), rq, f"C5 dq[{a}:{b}]")
    if b == d["q"].shape[2]:
        assert_bf16(sel(res["dk"], slice(a, b)), rk[:, :, a:], f"C5 dk[{a}:]")
        assert_bf16(sel(res["dv"], slice(a, b)), rv[:, :, a:], f"C5 dv[{a}:]")


def _bf_misaligned(x):
    """A contiguous bf16 device copy of x whose data pointer is 2 bytes past a 16-byte boundary."""
    x = np.ascontiguousarray(x, np.float32)
    flat = torch.empty(x.size + 8, dtype=torch.bfloat16, device=DEV)
    view = flat[1:1 + x.size].view(x.shape)
    view.copy_(torch.from_numpy(x).to(DEV).to(torch.bfloat16))
    assert view.data_ptr() % 16 != 0
    return view


@pytest.mark.parametrize("E", [32, 64, 128])
def test_bf16_unaligned_pointers(oracle_lib, E):
    """Inputs not 16-byte aligned take the element-wise tile fills (no global_load_lds) of the
    forward, dK/dV and dQ kernels at head dims equal to the instantiated ones."""
    from densecore_amd import _native
    rng = np.random.default_rng(300 + E)
    B, H, L, E_ = 1, 2, 150, E
    q, k, v, g = (bf16_round(rng.standard_normal((B, H, L, E_), dtype=np.float32)) for _ in range(4))
    print(f"[case] bf16 unaligned E{E}", flush=True)
    tq, tk, tv, tg = (_bf_misaligned(x) for x in (q, k, v, g))
    out, lse = _native._flash_attention(tq, tk, tv, True)
    ref_o, ref_l = oracle_lib.forward(q, k, v, True)
    assert_bf16(_np(out), ref_o, "out")
    assert_bf16(_np(lse), ref_l, "lse")
    ref = oracle_lib.backward(g, q, k, v, _np(out), _np(lse), True)
    got = _native._flash_attention_backward(tg, tq, tk, tv, out, lse, True)
    for name, a, b in zip(("dq", "dk", "dv"), got, ref):
        assert_bf16(_np(a), b, name)


def test_bf16_high_half_addresses(oracle_lib):
    """Inputs whose addresses have bit 31 set in their low 32 bits: the tile fills split each
    tile's base address into two 32-bit halves (scalar registers), and the low half must be
    widened without sign extension.  The tensors are in-bounds views into one 4.1 GiB
    buffer, placed so that every one of them starts 3 GiB into a 4 GiB window."""
    from densecore_amd import _native
    rng = np.random.default_rng(31)
    B, H, L, E = 1, 2, 300, 128
    xs = [bf16_round(rng.standard_normal((B, H, L, E), dtype=np.float32)) for _ in range(4)]
    n = B * H * L * E
    buf = torch.empty((1 << 31) + 4 * n + 64, dtype=torch.bfloat16, device=DEV)
    target = 3 << 30  # low 32 bits of the first tensor's address
    off = ((target - buf.data_ptr()) % (1 << 32)) // 2  # in elements; data_ptr is 256-aligned
    views = []
    for i, x in enumerate(xs):
        v = buf[off + i * n: off + (i + 1) * n].view(B, H, L, E)
        v.copy_(_bf(x))
        assert v.data_ptr() % 16 == 0 and (v.data_ptr() & 0xFFFFFFFF) >= 1 << 31
        views.append(v)
    tq, tk, tv, tg = views
    q, k, v, g = xs
    print("[case] bf16 high-half addresses", flush=True)
    out, lse = _native._flash_attention(tq, tk, tv, True)
    ref_o, ref_l = oracle_lib.forward(q, k, v, True)
    assert_bf16(_np(out), ref_o, "out")
    assert_bf16(_np(lse), ref_l, "lse")
    ref = oracle_lib.backward(g, q, k, v, _np(out), _np(lse), True)
    got = _native._flash_attention_backward(tg, tq, tk, tv, out, lse, True)
    for name, a, b in zip(("dq", "dk", "dv"), got, ref):
        assert_bf16(_np(a), b, name)


def test_bf16_backward_bit_reproducible():
    """The bf16 backward has no atomics: two runs give bit-identical dq, dk and dv."""
    from densecore_amd import _native
    rng = np.random.default_rng(11)
    q, k, v, g = (_bf(bf16_round(rng.standard_normal((2, 4, 700, 128), dtype=np.float32)))
                  for _ in range(4))
    out, lse = _native._flash_attention(q, k, v, True)
    first = _native._flash_attention_backward(g, q, k, v, out, lse, True)
    second = _native._flash_attention_backward(g, q, k, v, out, lse, True)
    torch.cuda.synchronize()
    for name, a, b in zip(("dq", "dk", "dv"), first, second):
        assert torch.equal(a, b), name


@pytest.mark.parametrize("vscale_log2", [-100, 0, 20, 100])
def test_bf16_value_scales(oracle_lib, vscale_log2):
    """The forward's P V product runs on an fp16 copy of V scaled per (batch, kv head) by a power
    of two: values of magnitude 2^+-100 (far outside fp16's range) and per-head scales that differ
    by 2^20 must come out as exactly as N(0, 1) values do."""
    from densecore_amd import _native
    rng = np.random.default_rng(vscale_log2 + 500)
    B, H, L, E = 2, 3, 150, 64
    q = bf16_round(rng.standard_normal((B, H, L, E), dtype=np.float32))
    k = bf16_round(rng.standard_normal((B, H, L, E), dtype=np.float32))
    v = bf16_round(rng.standard_normal((B, H, L, E), dtype=np.float32))
    v *= np.float32(2.0 ** vscale_log2)
    v[1, 2] *= np.float32(2.0 ** -20)  # a head 2^20 smaller than the others
    print(f"[case] bf16 V scale 2^{vscale_log2}", flush=True)
    ref_o, ref_l = oracle_lib.forward(q, k, v, True)
    out, lse = _native._flash_attention(_bf(q), _bf(k), _bf(v), True)
    got = _np(out)
    for b in range(B):
        for h in range(H):
            assert_bf16(got[b, h], ref_o[b, h], f"out b{b} h{h}")
    assert_bf16(_np(lse), ref_l, "lse")


def test_bf16_without_fp16_copies(oracle_lib):
    """A caller that passes no forward workspace and only dsum for the backward gets the bf16
    hi + lo products (no fp16 copies): the same bar on the same shape."""
    import ctypes
    from densecore_amd import _lib, _native
    rng = np.random.default_rng(77)
    B, H, L, E = 1, 4, 300, 128
    q, k, v, g = (bf16_round(rng.standard_normal((B, H, L, E), dtype=np.float32)) for _ in range(4))
    print("[case] bf16 minimal workspaces", flush=True)
    ref_o, ref_l = oracle_lib.forward(q, k, v, True)
    tq, tk, tv, tg = (_bf(x) for x in (q, k, v, g))
    out = torch.empty_like(tq)
    lse = torch.empty((B, H, L), dtype=torch.float32, device=DEV)
    d = _native._desc((B, H, H, L, L, E), True, None, torch.bfloat16, (0, 0, 0))
    Lb = _lib.lib()
    stream = torch.cuda.current_stream().cuda_stream
    _lib.check(Lb.dc_sdpa_fwd(d, tq.data_ptr(), tk.data_ptr(), tv.data_ptr(), None, out.data_ptr(),
                              lse.data_ptr(), None, 0, stream))
    assert_bf16(_np(out), ref_o, "out")
    ref = oracle_lib.backward(g, q, k, v, _np(out), _np(lse), True)
    dq, dk, dv = (torch.empty_like(tq) for _ in range(3))
    ws = torch.empty(B * H * L * 4 + 256, dtype=torch.uint8, device=DEV)
    assert ws.numel() < Lb.dc_sdpa_bwd_workspace_size(d)
    _lib.check(Lb.dc_sdpa_bwd(d, tg.data_ptr(), tq.data_ptr(), tk.data_ptr(), tv.data_ptr(), out.data_ptr(),
                              lse.data_ptr(), None, dq.data_ptr(), dk.data_ptr(), dv.data_ptr(),
                              ws.data_ptr(), ws.numel(), stream))
    for name, a, r in zip(("dq", "dk", "dv"), (dq, dk, dv), ref):
        assert_bf16(_np(a), r, name)


def test_bf16_long_causal_early_keys():
    """dV and dK of the first keys of a long causal row.  Key j < 64 is seen by every later query,
    the nearby ones with P ~ 1 / (query + 1): thousands of terms, the large ones of either sign,
    cancel to a small sum.  P and dS rounded once to fp16 (2^-12 per term) left errors of ~1% of
    rms(dV) there at L = 8192; blocks with large P now also carry the rounding error.  Checked
    against float64 (P from the GPU's lse, dsum from its bf16 out, as the backward takes them):
    |gpu - ref| <= 2^-7 |ref| + 3e-4 rms(ref), i.e. twice the outputs' own bf16 rounding (up to
    2^-8 |ref|) plus a small allowance.  A float64 emulation of these inputs gives 0.49 (dV) and
    0.63 (dK) of this bound for the kernels' products, 1.59 and 1.84 for fp16-only products."""
    from densecore_amd import _native
    B, H, L, E = 1, 1, 8192, 128
    rng = np.random.default_rng(8192)
    q, k, v, g = (bf16_round(rng.standard_normal((B, H, L, E), dtype=np.float32)) for _ in range(4))
    print("[case] bf16 causal L8192 D128 early keys vs float64", flush=True)
    tq, tk, tv, tg = (_bf(x) for x in (q, k, v, g))
    out, lse = _native._flash_attention(tq, tk, tv, True)
    dq, dk, dv = _native._flash_attention_backward(tg, tq, tk, tv, out, lse, True)
    torch.cuda.synchronize()
    o, l = _np(out)[0, 0].astype(np.float64), lse.cpu().numpy()[0, 0].astype(np.float64)
    q64, k64, v64, g64 = (x[0, 0].astype(np.float64) for x in (q, k, v, g))
    scale = 1.0 / np.sqrt(E)
    J = 64
    s = q64 @ k64[:J].T * scale                              # (L, J): every query, the first keys
    s[np.arange(L)[:, None] < np.arange(J)[None, :]] = -np.inf
    p = np.exp(s - l[:, None])
    dsum = np.sum(g64 * o, axis=1)
    ds = p * (g64 @ v64[:J].T - dsum[:, None])
    ref = {"dv": p.T @ g64, "dk": scale * (ds.T @ q64)}
    got = {"dv": _np(dv)[0, 0, :J], "dk": _np(dk)[0, 0, :J]}
    for name in ("dv", "dk"):
        r = ref[name]
        bar = 2.0 ** -7 * np.abs(r) + 3e-4 * np.sqrt(np.mean(r ** 2))
        err = np.abs(got[name] - r)
        assert np.all(err <= bar), f"{name}: max err / bar {np.max(err / bar):.3f}"


@pytest.mark.parametrize("B,H,Hkv,L,S,E,causal,mask", [
    (2, 4, 2, 300, 300, 256, True, None),
    (1, 2, 2, 2048, 2048, 256, True, None),     # long causal rows (fp16 P with its low part)
    (2, 3, 3, 130, 257, 192, False, None),
    (1, 2, 1, 200, 120, 256, True, None),       # L > S, grouped heads
    (2, 2, 2, 97, 150, 256, False, "float"),   # a float mask with -inf holes, a fully masked row
    (3, 2, 2, 64, 200, 200, False, "padding"),  # key padding, head dim not a multiple of 32
    (2, 2, 2, 40, 5, 129, False, None),
])
def test_bf16_flash_head_dims_to_256(oracle_lib, B, H, Hkv, L, S, E, causal, mask):
    """bf16 head dims 129-256 on the flash kernels (4-wave forward, dQ and dK/dV kernels at head
    dim 256, one wave per SIMD): no materialized rows; out and lse against the oracle on the upcast
    inputs, the backward from the GPU's own (out, lse), bf16 bar; the backward bit-identical from
    run to run."""
    from densecore_amd import _native
    rng = np.random.default_rng(L * 3 + S + E + B)
    q, g = (bf16_round(rng.standard_normal((B, H, L, E), dtype=np.float32)) for _ in range(2))
    k, v = (bf16_round(rng.standard_normal((B, Hkv, S, E), dtype=np.float32)) for _ in range(2))
    mk = tm = None
    if mask == "float":
        mk = rng.standard_normal((B, H, L, S)).astype(np.float32)
        mk[rng.random((B, H, L, S)) < 0.25] = -np.inf
        mk[0, 0, 1] = -np.inf
        tm = torch.from_numpy(mk).to(DEV)
    elif mask == "padding":
        lengths = rng.integers(1, S + 1, size=B)
        m1 = np.where(np.arange(S)[None, :] < lengths[:, None], np.float32(0), np.float32(-np.inf))
        tm = torch.from_numpy(m1[:, None, None, :]).to(DEV).expand(B, H, L, S)
        mk = np.ascontiguousarray(np.broadcast_to(m1[:, None, None, :], (B, H, L, S)))
    print(f"[case] bf16 flash B{B} H{H} Hkv{Hkv} L{L} S{S} E{E} causal={causal} mask={mask}", flush=True)
    tq, tk, tv, tg = (_bf(x) for x in (q, k, v, g))
    fs = _native._schedule(False, tq, tk, tv, causal, mask=tm)
    bs = _native._schedule(True, tq, tk, tv, causal, mask=tm)
    assert fs["materialized_rows"] == 0 and bs["materialized_rows"] == 0 and bs["deterministic"] == 1, (fs, bs)
    ref_o, ref_l = oracle_lib.forward(q, k, v, causal, None, mk)
    out, lse = _native._flash_attention(tq, tk, tv, causal, None, tm)
    assert_bf16(_np(out), ref_o, "out")
    assert_bf16(_np(lse), ref_l, "lse")
    ref = oracle_lib.backward(g, q, k, v, _np(out), _np(lse), causal, None, mk)
    got = _native._flash_attention_backward(tg, tq, tk, tv, out, lse, causal, None, tm)
    again = _native._flash_attention_backward(tg, tq, tk, tv, out, lse, causal, None, tm)
    for name, a, b, c in zip(("dq", "dk", "dv"), got, ref, again):
        assert_bf16(_np(a), b, name)
        assert torch.equal(a, c), f"{name}: runs differ"
