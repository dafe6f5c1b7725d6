"""GPU parity of dropout: the mask drawn on the GPU from the reference's generator stream
against the oracle's sequential restatement of Generator::bernoulli (src/torch_random.rs:
241-254), bit for bit, then dropout, the math path with dropout and MHA with dropout against
the oracle composed with that same noise.

Bars (written here): keep bits and the generator state after each draw are identical (integer
work); dropout's product is bit-identical to x * noise; attention outputs and gradients meet
|gpu - ref| <= 2e-5 + 1e-5 |ref| elementwise.
"""
import numpy as np
import pytest

import oracle
from tests._data import assert_f32

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu

DEV = "cuda:0"


def _unpack(bits, n):
    torch.cuda.synchronize()
    return np.unpackbits(bits.cpu().numpy().view(np.uint8), bitorder="little")[:n].astype(bool)


def _gen(seed, pre=0):
    """A device generator and the oracle generator, both seeded and advanced by `pre` outputs."""
    from densecore_amd import random as R
    o = oracle.Generator(seed)
    o.random(pre)
    g = R.Generator(DEV)
    s = np.concatenate([np.array([seed, *o.position, 2**64 - 1, 0, 0, 0], np.uint64),
                        o.words.astype(np.uint64)])
    g.set_state(s.view(np.uint8))
    return g, o


def _state_equal(g, o):
    st = g.get_state().numpy().view(np.uint64)
    return tuple(int(x) for x in st[1:3]) == o.position and np.array_equal(st[7:].astype(np.uint32), o.words)


@pytest.mark.parametrize("pre", [0, 1, 2, 623, 624, 625, 1001])
@pytest.mark.parametrize("n", [1, 31, 32, 63, 64, 65, 100, 1000, 65_536 + 63, 65_536 + 64, 65_536 + 65,
                               200_000])
def test_bernoulli_bits_match_the_oracle(n, pre):
    print(f"[case] bernoulli n={n} pre={pre}", flush=True)
    g, o = _gen(1234 + n, pre)
    p = 0.7
    got = _unpack(g._bernoulli_bits(n, p), n)
    ref = o.bernoulli(n, p).astype(bool)
    assert np.array_equal(got, ref), f"first mismatch at {int(np.argmax(got != ref))}"
    assert _state_equal(g, o)


@pytest.mark.parametrize("p", [0.0, 1e-9, 0.25, 0.5, 0.999, 1.0])
def test_bernoulli_probabilities(p):
    g, o = _gen(99, 5)
    n = 70_001
    assert np.array_equal(_unpack(g._bernoulli_bits(n, p), n), o.bernoulli(n, p).astype(bool))


def test_consecutive_draws_keep_the_stream():
    """Draws of odd sizes one after the other: the engine block stays on the GPU between them."""
    g, o = _gen(7)
    for n in (3, 1000, 131_071, 1, 624, 300_000, 77):
        print(f"[case] consecutive n={n}", flush=True)
        assert np.array_equal(_unpack(g._bernoulli_bits(n, 0.4), n), o.bernoulli(n, 0.4).astype(bool))
    assert _state_equal(g, o)


def test_many_chunks_and_every_jump_level():
    """40M draws: 611 chunks, so the first jump level takes digits 0-2, the second every digit."""
    print("[case] bernoulli n=40M", flush=True)
    g, o = _gen(2026, 333)
    n = 40_000_000
    got = _unpack(g._bernoulli_bits(n, 0.9), n)
    ref = o.bernoulli(n, 0.9).astype(bool)
    assert np.array_equal(got, ref), f"{int((got != ref).sum())} mismatches"
    assert _state_equal(g, o)


def test_dropout_is_x_times_the_reference_noise():
    from densecore_amd import functional as F, random as R
    print("[case] dropout exact", flush=True)
    x = np.random.default_rng(3).standard_normal((3, 5, 777)).astype(np.float32)
    for p in (0.1, 0.5, 0.8):
        R.manual_seed(42)
        t = torch.from_numpy(x).to(DEV).requires_grad_(True)
        y = F.dropout(t, p)
        gy = torch.ones_like(y)
        y.backward(gy)
        noise = oracle.dropout_noise(oracle.Generator(42), x.shape, p)
        torch.cuda.synchronize()
        assert np.array_equal(y.detach().cpu().numpy(), x * noise)
        assert np.array_equal(t.grad.cpu().numpy(), np.ones_like(x) * noise)


def test_math_path_with_dropout_against_oracle():
    from densecore_amd import functional as F, random as R
    print("[case] sdpa dropout", flush=True)
    rng = np.random.default_rng(11)
    B, H, L, S, E = 2, 3, 33, 47, 32
    q, k, v, g = (rng.standard_normal(s).astype(np.float32)
                  for s in ((B, H, L, E), (B, H, S, E), (B, H, S, E), (B, H, L, E)))
    p = 0.3
    R.manual_seed(5)
    tq, tk, tv = (torch.from_numpy(a).to(DEV).requires_grad_(True) for a in (q, k, v))
    out = F.scaled_dot_product_attention(tq, tk, tv, dropout_p=p, is_causal=True)
    out.backward(torch.from_numpy(g).to(DEV))
    noise = oracle.dropout_noise(oracle.Generator(5), (B, H, L, S), p)
    ref, (dq, dk, dv, _) = oracle.math_attention(q, k, v, is_causal=True, noise=noise, grad_out=g)
    torch.cuda.synchronize()
    assert_f32(out.detach().cpu().numpy(), ref, "out")
    for name, t, r in (("dq", tq, dq), ("dk", tk, dk), ("dv", tv, dv)):
        assert_f32(t.grad.cpu().numpy(), r, name)


def test_multi_head_attention_dropout_weights():
    """Training-mode MHA returns the dropped weights: softmax weights times the noise."""
    from densecore_amd import nn, random as R
    print("[case] mha dropout", flush=True)
    torch.manual_seed(0)
    E, heads, L, N = 32, 4, 9, 2
    mod = nn.MultiheadAttention(E, heads, dropout=0.25)
    x = torch.from_numpy(np.random.default_rng(8).standard_normal((L, N, E)).astype(np.float32)).to(DEV)
    mod.eval()
    _, w = mod(x, x, x, average_attn_weights=False)
    mod.train()
    R.manual_seed(77)
    _, wd = mod(x, x, x, average_attn_weights=False)
    noise = oracle.dropout_noise(oracle.Generator(77), (N * heads, L, L), 0.25).reshape(N, heads, L, L)
    torch.cuda.synchronize()
    assert np.array_equal(wd.detach().cpu().numpy(), w.detach().cpu().numpy() * noise)
