"""GPU parity of dc_bmm, the device entry of the reference's bmm registry.

The reference's bmm (src/batched_matmul.rs:9-49 -> src/torch_blas.rs:404-449) multiplies strided
(batch, m, k) and (batch, k, n) float32 operands into a fresh (batch, m, n).  dc_bmm reads A and B
through their strides: row-major operands, transposed views (the math path's k^T), and strided
views without a unit stride each take their own load path.  Every case is checked against the
oracle's bmm (oracle.bmm, the k-order float32 sum of the reference's Linux sgemm) at the float32
bar |gpu - ref| <= 2e-5 + 1e-5 |ref|, with C pre-filled with NaN so an element no tile writes
fails.  The gradient (functional.bmm: dA = dC B^T, dB = A^T dC, both dc_bmm on transposed views)
is checked the same way.
"""
import numpy as np
import pytest

from tests._data import assert_f32

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu

DEV = "cuda:0"


def _operand(x, layout):
    """x (batch, r, c) on the GPU as a view of the given layout (same values)."""
    t = torch.from_numpy(np.ascontiguousarray(x)).to(DEV)
    if layout == "row":        # contiguous: unit stride along the last dim
        return t
    if layout == "col":        # transposed storage: unit stride along the middle dim
        return t.transpose(1, 2).contiguous().transpose(1, 2)
    if layout == "strided":    # no unit stride: every other element of a wider buffer
        wide = torch.zeros(x.shape[0], x.shape[1], 2 * x.shape[2], device=DEV)
        wide[:, :, ::2] = t
        return wide[:, :, ::2]
    if layout == "offset":     # row-major, rows 4-byte aligned but not 16-byte aligned
        buf = torch.zeros(x.size + 1, device=DEV)
        view = buf[1:].view(x.shape)
        view.copy_(t)
        return view
    raise ValueError(layout)


def _bmm_nan_filled(a, b):
    from densecore_amd import _lib, _native
    batch, m, k = a.shape
    n = b.shape[2]
    c = torch.full((batch, m, n), float("nan"), device=DEV)
    sa, sb = a.stride(), b.stride()
    d = _lib.BmmDesc(batch, m, n, k, sa[0], sa[1], sa[2], sb[0], sb[1], sb[2])
    _lib.check(_lib.lib().dc_bmm(d, _native._ptr(a), _native._ptr(b), _native._ptr(c),
                                 _native._stream(a.device)))
    torch.cuda.synchronize()
    return c.cpu().numpy()


LAYOUTS = ["row", "col", "strided", "offset"]
SHAPES = [(3, 37, 45, 29), (2, 130, 70, 64), (2, 200, 257, 36), (4, 1, 1, 1), (1, 129, 65, 131)]


@pytest.mark.parametrize("la", LAYOUTS)
@pytest.mark.parametrize("lb", LAYOUTS)
@pytest.mark.parametrize("shape", SHAPES, ids=[f"b{s[0]}m{s[1]}n{s[2]}k{s[3]}" for s in SHAPES])
def test_bmm_layouts(oracle_lib, la, lb, shape):
    batch, m, n, k = shape
    rng = np.random.default_rng(batch * 1000 + m + n + k + 7 * LAYOUTS.index(la) + LAYOUTS.index(lb))
    a = rng.standard_normal((batch, m, k), dtype=np.float32)
    b = rng.standard_normal((batch, k, n), dtype=np.float32)
    print(f"[case] bmm {shape} A {la} B {lb}", flush=True)
    got = _bmm_nan_filled(_operand(a, la), _operand(b, lb))
    assert_f32(got, oracle_lib.bmm(a, b, b_k_contiguous=lb == "col"), f"bmm {shape} {la} {lb}")


def test_bmm_attention_shapes(oracle_lib):
    """The math path's two products at C3's shape (B16 H16 L = S = 512, D64), 16 of the 256
    (batch, head) items: scores = q k^T with k^T a transposed view, then weights v."""
    rng = np.random.default_rng(3)
    q = rng.standard_normal((16, 512, 64), dtype=np.float32) * np.float32(0.35)
    k = rng.standard_normal((16, 512, 64), dtype=np.float32) * np.float32(0.35)
    v = rng.standard_normal((16, 512, 64), dtype=np.float32)
    print("[case] bmm C3 shapes: q k^T and weights v", flush=True)
    tk = torch.from_numpy(k).to(DEV)
    scores = _bmm_nan_filled(torch.from_numpy(q).to(DEV), tk.transpose(1, 2))
    ref = oracle_lib.bmm(q, np.ascontiguousarray(k.transpose(0, 2, 1)), b_k_contiguous=True)
    assert_f32(scores, ref, "q k^T")
    w = np.exp(ref - ref.max(axis=-1, keepdims=True))
    w = (w / w.sum(axis=-1, keepdims=True)).astype(np.float32)
    got = _bmm_nan_filled(torch.from_numpy(w).to(DEV), torch.from_numpy(v).to(DEV))
    assert_f32(got, oracle_lib.bmm(w, v), "weights v")


def test_bmm_empty_and_zero_k():
    from densecore_amd import _native
    a = torch.randn(3, 5, 0, device=DEV)
    b = torch.randn(3, 0, 7, device=DEV)
    c = _native._bmm(a, b)
    torch.cuda.synchronize()
    assert tuple(c.shape) == (3, 5, 7) and torch.count_nonzero(c) == 0
    assert tuple(_native._bmm(torch.randn(0, 5, 4, device=DEV), torch.randn(0, 4, 7, device=DEV)).shape) == (0, 5, 7)
    with pytest.raises(ValueError, match="bmm requires rank-3 operands"):
        _native._bmm(torch.randn(5, 4, device=DEV), torch.randn(1, 4, 7, device=DEV))
    with pytest.raises(ValueError, match="bmm batch or inner dimensions mismatch"):
        _native._bmm(torch.randn(2, 5, 4, device=DEV), torch.randn(2, 3, 7, device=DEV))


def test_bmm_gradient(oracle_lib):
    """functional.bmm's backward: dA = dC B^T and dB = A^T dC against the oracle's bmm."""
    from densecore_amd import functional as F
    rng = np.random.default_rng(44)
    a = rng.standard_normal((3, 70, 40), dtype=np.float32)
    b = rng.standard_normal((3, 40, 90), dtype=np.float32)
    g = rng.standard_normal((3, 70, 90), dtype=np.float32)
    ta = torch.from_numpy(a).to(DEV).requires_grad_(True)
    tb = torch.from_numpy(b).to(DEV).transpose(1, 2).contiguous().transpose(1, 2).requires_grad_(True)
    out = F.bmm(ta, tb)
    out.backward(torch.from_numpy(g).to(DEV))
    torch.cuda.synchronize()
    assert_f32(out.detach().cpu().numpy(), oracle_lib.bmm(a, b), "bmm out")
    assert_f32(ta.grad.cpu().numpy(), oracle_lib.bmm(g, np.ascontiguousarray(b.transpose(0, 2, 1))), "dA")
    assert_f32(tb.grad.cpu().numpy(), oracle_lib.bmm(np.ascontiguousarray(a.transpose(0, 2, 1)), g), "dB")
