"""The reference's generator on the CPU side: the oracle's restatement of the engine
(src/torch_random.rs) pinned against independent implementations, the library's host
functions (seeding, jump-ahead skip) against the oracle, and the Python Generator's state API.

Pins of the oracle's engine, chosen so that a wrong constant, shift, twist index or word order
fails: the reference's own known answer (seed 5489: the 10000th output is 4123659995,
src/torch_random.rs:313-322); numpy's MT19937 (legacy seeding = the same init_genrand) raw
32-bit stream; and torch's CPU generator, whose float64 ``rand`` is the same uniform_real
(random64 with the first output high, 53 bits, times 2^-53), for seeds above and below 2^32
including the default seed.  Bernoulli is then the comparison of those doubles with p.
"""
import ctypes

import numpy as np
import pytest

import oracle

torch = pytest.importorskip("torch")

SEEDS = [0, 1, 5489, 67_280_421_310_721, 2**40 + 7, 2**64 - 1]


def test_known_answer_of_the_reference():
    assert oracle.Generator(5489).random(10_000)[-1] == 4_123_659_995


@pytest.mark.parametrize("seed", [0, 1, 5489, 2**32 - 1])
def test_engine_matches_numpy_mt19937(seed):
    bg = np.random.MT19937()
    bg._legacy_seeding(seed)
    ref = bg.random_raw(5000).astype(np.uint32)
    assert np.array_equal(oracle.Generator(seed).random(5000), ref)


@pytest.mark.parametrize("seed", SEEDS)
def test_uniform_doubles_and_bernoulli_match_torch(seed):
    u = oracle.Generator(seed).uniform_doubles(3000)
    tg = torch.Generator().manual_seed(seed)
    ref = torch.rand(3000, dtype=torch.float64, generator=tg).numpy()
    assert np.array_equal(u, ref)
    for p in (0.0, 0.1, 0.5, 0.9, 1.0):
        b = oracle.Generator(seed).bernoulli(3000, p)
        assert np.array_equal(b, (ref < p).astype(np.float32))


def _lib():
    from densecore_amd import _lib
    return _lib.lib()


def test_library_seed_matches_oracle():
    for seed in SEEDS:
        w = np.zeros(624, np.uint32)
        _lib().dc_mt19937_seed(seed, w.ctypes.data)
        assert np.array_equal(w, oracle.Generator(seed).words)


def _advance(words, left, nxt, count):
    w = np.ascontiguousarray(words, np.uint32).copy()
    l, n = ctypes.c_int64(left), ctypes.c_int64(nxt)
    st = _lib().dc_mt19937_advance(w.ctypes.data, ctypes.byref(l), ctypes.byref(n), count)
    return st, w, (l.value, n.value)


@pytest.mark.parametrize("pre", [0, 1, 2, 623, 624, 625, 1000])
@pytest.mark.parametrize("count", [0, 1, 2, 623, 624, 625, 1247, 1248, 19937, 100_003, 2_000_001])
def test_advance_matches_sequential_draws(pre, count):
    g = oracle.Generator(987)
    g.random(pre)
    st, w, pos = _advance(g.words, *g.position, count)
    assert st == 0
    g.random(count)
    assert np.array_equal(w, g.words) and pos == g.position


@pytest.mark.parametrize("left,nxt", [(0, 0), (625, 0), (5, 5), (1, 625), (624, -1)])
def test_invalid_positions_rejected(left, nxt):
    from densecore_amd import _lib as L
    st, _, _ = _advance(np.zeros(624, np.uint32), left, nxt, 3)
    assert st == L.DC_INVALID_ARGUMENT
    assert "invalid generator state" in _lib().dc_last_error().decode()


def test_bernoulli_argument_errors():
    from densecore_amd import _lib as L
    lib = _lib()
    w = np.zeros(624, np.uint32)
    l, n = ctypes.c_int64(1), ctypes.c_int64(0)
    for count, p, status, msg in ((-1, 0.5, L.DC_INVALID_ARGUMENT, "negative"),
                                  (10, 1.5, L.DC_INVALID_ARGUMENT, "0 <= p <= 1"),
                                  (10, float("nan"), L.DC_INVALID_ARGUMENT, "0 <= p <= 1"),
                                  (lib.dc_bernoulli_max_draws() + 1, 0.5, L.DC_UNSUPPORTED, "max_draws"),
                                  (10, 0.5, L.DC_INVALID_ARGUMENT, "null pointer")):
        st = lib.dc_bernoulli(None, w.ctypes.data, ctypes.byref(l), ctypes.byref(n), count, p,
                              None, None, 0, None)
        assert st == status and msg in lib.dc_last_error().decode()
    assert lib.dc_bernoulli(None, w.ctypes.data, ctypes.byref(l), ctypes.byref(n), 0, 0.5, None,
                            None, 0, None) == L.DC_OK
    assert (l.value, n.value) == (1, 0)
    assert lib.dc_bernoulli_workspace_size(-1) == 0


def test_python_generator_state_layout():
    from densecore_amd import random as R
    g = R.Generator("cuda")
    assert g.initial_seed() == R.DEFAULT_SEED
    st = g.get_state().numpy().view(np.uint64)
    assert st.size == 7 + 624
    assert list(st[:3]) == [R.DEFAULT_SEED, 1, 0] and st[3] == 2**64 - 1 and st[4] == 0
    assert np.array_equal(st[7:].astype(np.uint32), oracle.Generator(R.DEFAULT_SEED).words)
    g.manual_seed(-1)
    assert g.initial_seed() == 2**64 - 1
    o = oracle.Generator(12)
    o.random(777)
    s = np.concatenate([np.array([12, *o.position, 2**64 - 1, 0, 0, 0], np.uint64),
                        o.words.astype(np.uint64)])
    g.set_state(torch.from_numpy(s.view(np.uint8).copy()))
    assert np.array_equal(g.get_state().numpy().view(np.uint64), s)
    bad = s.copy()
    bad[1] = 0
    with pytest.raises(ValueError, match="invalid generator state"):
        g.set_state(bad.view(np.uint8))
    with pytest.raises(ValueError, match="invalid generator state"):
        g.set_state(np.zeros(13, np.uint8))
    with pytest.raises(TypeError):
        g.manual_seed(True)
    with pytest.raises(RuntimeError, match="Overflow"):
        g.manual_seed(2**64)


def test_dropout_arguments_and_no_cpu_path():
    from densecore_amd import functional as F
    x = torch.ones(4, 5)
    with pytest.raises(TypeError):
        F.dropout(x, p=True)
    with pytest.raises(ValueError, match=r"\[0, 1\]"):
        F.dropout(x, p=1.5)
    with pytest.raises(TypeError):
        F.dropout(x, p=0.5, training=1)
    assert F.dropout(x, 0.5, training=False) is x and F.dropout(x, 0.0) is x
    assert torch.equal(F.dropout(x, 1.0), torch.zeros(4, 5))
    with pytest.raises(ValueError, match="GPU"):
        F.dropout(x, 0.5)
