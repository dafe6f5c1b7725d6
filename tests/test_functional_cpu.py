"""Host-side logic of the Python mirror, without a GPU: argument checks and messages follow
python/densecore/functional.py:276-364 and src/lib.rs:555-683 of the reference; inputs the
flash path does not take go to the device math path and never run on the host; masks become
broadcast views."""
import numpy as np
import pytest

torch = pytest.importorskip("torch")

from densecore_amd import _native, functional as F  # noqa: E402


def t(*shape, dtype=torch.float32):
    return torch.zeros(shape, dtype=dtype)


def test_reference_argument_errors():
    """tests/test_attention.py:50-64 of the reference."""
    sdpa = F.scaled_dot_product_attention
    q, k, v = t(1, 1, 2, 4), t(1, 1, 3, 4), t(1, 1, 3, 5)
    with pytest.raises(ValueError, match="both"):
        sdpa(q, k, k, attn_mask=np.ones((2, 3), bool), is_causal=True)
    with pytest.raises(ValueError, match="shapes"):
        sdpa(q, t(1, 1, 3, 3), k)
    with pytest.raises(ValueError, match="rank"):
        sdpa(q.reshape(2, 4), k, k)
    with pytest.raises(TypeError):
        sdpa(q, k, k, is_causal=1)
    with pytest.raises(TypeError):
        sdpa(q, k, k, scale="x")
    with pytest.raises(TypeError):
        sdpa(np.zeros((1, 1, 2, 4)), k, k)


def test_math_path_inputs_never_run_on_the_cpu():
    """Inputs the flash path does not take go to the composed math path, which runs on the GPU
    only: CPU tensors are rejected rather than computed on the host."""
    sdpa = F.scaled_dot_product_attention
    q, k = t(1, 1, 2, 4), t(1, 1, 3, 4)
    for call in (lambda: sdpa(q, k, k, dropout_p=0.5),
                 lambda: sdpa(t(1, 2, 4), t(1, 3, 4), t(1, 3, 4)),          # rank 3
                 lambda: sdpa(q, k, t(1, 1, 3, 5)),                          # Ev != E
                 lambda: sdpa(q, k, k, attn_mask=np.zeros((1, 2, 3), np.float32))):  # 3-D mask
        with pytest.raises(ValueError, match="GPU"):
            call()
    with pytest.raises(NotImplementedError, match="float32"):
        sdpa(q.double(), k.double(), k.double())
    with pytest.raises(ValueError, match="GPU"):
        _native._softmax(t(2, 3))
    with pytest.raises(ValueError, match="GPU"):
        F.softmax(t(2, 3))


def test_cpu_tensors_are_rejected_no_fallback():
    with pytest.raises(ValueError, match="on the GPU"):
        F.scaled_dot_product_attention(t(1, 1, 2, 4), t(1, 1, 3, 4), t(1, 1, 3, 4))


def test_native_boundary_messages():
    x = t(1, 2, 3, 4)
    with pytest.raises(ValueError, match=r"takes \(B, H, L, E\) tensors"):
        _native._flash_attention(x[0], x, x, False)
    with pytest.raises(ValueError, match="q/k/v shapes do not match"):
        _native._flash_attention(x, t(1, 3, 3, 4), t(1, 3, 3, 4), False)
    with pytest.raises(ValueError, match="q/k/v shapes do not match"):
        _native._flash_attention(x, x, t(1, 2, 3, 5), False)
    with pytest.raises(ValueError, match="backward shapes do not match"):
        _native._flash_attention_backward(x, x, x, x, x, t(1, 2, 2), False)
    with pytest.raises(ValueError, match="decode takes q_len == 1"):
        _native._flash_decode(x, x, x)


@pytest.mark.parametrize("shape", [(3, 5), (1, 5), (3, 1), (2, 4, 3, 5), (1, 4, 1, 5), (2, 1, 3, 1)])
def test_flash_mask_bool_and_float(shape):
    rng = np.random.default_rng(0)
    qshape, source = (2, 4, 3, 8), 5
    b = rng.random(shape) > 0.4
    m = F._flash_mask(b, qshape, source, "cpu")
    assert tuple(m.shape) == (2, 4, 3, 5)
    expect = np.broadcast_to(np.where(b, 0.0, -np.inf), (2, 4, 3, 5))
    np.testing.assert_array_equal(m.numpy(), expect)
    # broadcast, not materialised: the broadcast dims have stride 0
    if len(shape) == 4:
        for dim in range(4):
            if shape[dim] == 1 and (2, 4, 3, 5)[dim] > 1:
                assert m.stride(dim) == 0
    f = rng.normal(size=shape).astype(np.float32)
    mf = F._flash_mask(torch.from_numpy(f), qshape, source, "cpu")
    np.testing.assert_array_equal(mf.numpy(), np.broadcast_to(f, (2, 4, 3, 5)))


@pytest.mark.parametrize("mask", [
    np.zeros((2, 3, 5), np.float32),          # 3-D
    np.zeros((3, 4), np.float32),             # wrong S
    np.zeros((2, 2, 3, 5), np.float32),       # wrong H
    np.zeros((3, 5), np.int32),               # dtype
])
def test_flash_mask_rejections(mask):
    assert F._flash_mask(mask, (2, 4, 3, 8), 5, "cpu") is None
    req = torch.zeros((3, 5), requires_grad=True)
    assert F._flash_mask(req, (2, 4, 3, 8), 5, "cpu") is None


@pytest.mark.parametrize("shape", [(3, 1), (1, 1, 3, 1), (2, 1, 3, 1), (1, 4, 1, 1), (2, 4, 3, 1)])
def test_mask_broadcast_over_keys_copies_the_key_axis_only(shape):
    """A mask without unit key stride (an (L, 1) mask expanded over S, say) reaches the kernels
    as a copy along the key axis whose other broadcast dims keep stride 0: never B*H*L*S floats
    unless the mask really has B*H*L distinct rows."""
    B, H, L, S = 2, 4, 3, 5
    rng = np.random.default_rng(1)
    src = torch.from_numpy(rng.normal(size=shape).astype(np.float32))
    full = (1,) * (4 - len(shape)) + tuple(shape)  # the mask's own (B|1, H|1, L|1, 1)
    view = src.reshape(full).expand(B, H, L, S)
    m, strides = _native._mask_arg(view, (B, H, H, L, S, 8), torch.device("cpu"))
    assert m.stride(3) == 1 and strides == (m.stride(0), m.stride(1), m.stride(2))
    np.testing.assert_array_equal(m.numpy(), view.numpy())
    for dim in range(3):
        if full[dim] == 1:
            assert m.stride(dim) == 0, (dim, m.stride())
    assert m.untyped_storage().nbytes() == 4 * S * int(np.prod([full[d] for d in range(3)]))
