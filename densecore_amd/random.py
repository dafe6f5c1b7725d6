"""The reference's generator for the GPU path (``python/densecore/_random.py:31-131``).

Same engine (PyTorch's mt19937, ``src/torch_random.rs``), same seeding rules, same default seed
and the same ``get_state`` layout, so a seed gives the reference's draws bit for bit.  The
engine's 624 words move to the GPU on the first device draw and stay there between draws (no
host round trip per call); ``left`` / ``next`` are tracked on the host exactly as the
reference's ``random()`` moves them.  The draws the attention path needs (dropout's Bernoulli
mask) are made on the GPU by ``dc_bernoulli`` (``include/dc_math.h``).
"""
import ctypes
import operator
import os

import numpy as np
import torch

from . import _lib

DEFAULT_SEED = 67_280_421_310_721  # default_rng_seed_val (src/torch_random.rs:15-16)
_WORDS = 624
_tables = {}


def _seed_value(seed):
    """torch.manual_seed's accepted range; negatives wrap to 0xffff_ffff_ffff_ffff + seed + 1
    (``python/densecore/_random.py:17-24``)."""
    if isinstance(seed, (bool, np.bool_)):
        raise TypeError("seed must be an integer")
    seed = operator.index(seed)
    if not -0x8000_0000_0000_0000 <= seed <= 0xFFFF_FFFF_FFFF_FFFF:
        raise RuntimeError("Overflow when unpacking long long")
    return seed & 0xFFFF_FFFF_FFFF_FFFF


def _table(device):
    """The jump-ahead polynomials dc_bernoulli reads, uploaded once per device."""
    key = (device.type, device.index)
    if key not in _tables:
        L = _lib.lib()
        t = torch.empty(int(L.dc_mt19937_table_bytes()), dtype=torch.uint8, device=device)
        _lib.check(L.dc_mt19937_table_init(t.data_ptr(), torch.cuda.current_stream(device).cuda_stream))
        _tables[key] = t
    return _tables[key]


class Generator:
    """The reference's CPU generator with its engine words kept on ``device`` for GPU draws."""

    def __init__(self, device="cuda"):
        device = torch.device(device)
        if device.type != "cuda":
            raise NotImplementedError("this generator draws on the GPU: device must be cuda")
        self.device = device
        self._seed = 0
        self._host = np.zeros(_WORDS, np.uint32)  # current when self._dev is None
        self._dev = None
        self._left, self._next = 1, 0
        self._normals = (0xFFFF_FFFF_FFFF_FFFF, 0, 0, 0)  # opaque cached-normal words of a set state
        self.manual_seed(DEFAULT_SEED)

    # ---- torch.Generator API (python/densecore/_random.py:40-66) ----

    def manual_seed(self, seed):
        seed = _seed_value(seed)
        words = np.empty(_WORDS, np.uint32)
        _lib.lib().dc_mt19937_seed(seed, words.ctypes.data)
        self._seed, self._host, self._dev = seed, words, None
        self._left, self._next = 1, 0
        self._normals = (0xFFFF_FFFF_FFFF_FFFF, 0, 0, 0)
        return self

    def initial_seed(self):
        return self._seed

    def seed(self):
        """Reseed from the operating system and return the new seed (like torch)."""
        seed = int.from_bytes(os.urandom(8), "little") & 0x7FFF_FFFF_FFFF_FFFF
        self.manual_seed(seed)
        return seed

    def _words_host(self):
        if self._dev is not None:
            self._host = self._dev.cpu().numpy().view(np.uint32).copy()
            self._dev = None
        return self._host

    def get_state(self):
        """Engine state as a uint8 CPU tensor in the reference's layout (``to_words``,
        ``src/torch_random.rs:276-288``): seed, left, next, the two cached normals, 624 words."""
        w = np.empty(7 + _WORDS, np.uint64)
        w[:7] = (self._seed, self._left, self._next) + self._normals
        w[7:] = self._words_host()
        return torch.from_numpy(w.view(np.uint8).copy())

    def set_state(self, state):
        """``from_words`` (``src/torch_random.rs:290-311``) with its validation."""
        array = state.cpu().numpy() if isinstance(state, torch.Tensor) else np.asarray(state)
        array = np.ascontiguousarray(array, np.uint8)
        if array.size % 8:
            raise ValueError("invalid generator state")
        w = array.view(np.uint64)
        if (w.size != 7 + _WORDS or w[1] == 0 or w[1] > _WORDS or w[2] > _WORDS
                or (w[7:] > 0xFFFF_FFFF).any()):
            raise ValueError("invalid generator state")
        self._seed, self._left, self._next = int(w[0]), int(w[1]), int(w[2])
        self._normals = tuple(int(x) for x in w[3:7])
        self._host, self._dev = w[7:].astype(np.uint32), None
        return self

    # ---- GPU draws ----

    def _words_device(self):
        if self._dev is None:
            self._dev = torch.from_numpy(self._host.view(np.int32).copy()).to(self.device)
        return self._dev

    def _bernoulli_bits(self, n, p):
        """Keep bits of ``Generator::bernoulli(n, p)`` (``src/torch_random.rs:241-254``) drawn on
        the GPU: element e is bit e % 32 of int32 word e / 32."""
        L = _lib.lib()
        n = int(n)
        bits = torch.empty((n + 31) // 32, dtype=torch.int32, device=self.device)  # all written
        if n == 0:
            return bits
        words = self._words_device()
        table = _table(self.device)
        stream = torch.cuda.current_stream(self.device).cuda_stream
        left, nxt = ctypes.c_int64(self._left), ctypes.c_int64(self._next)
        step = int(L.dc_bernoulli_max_draws()) // 32 * 32
        for start in range(0, n, step):
            m = min(step, n - start)
            ws = torch.empty(max(int(L.dc_bernoulli_workspace_size(m)), 1), dtype=torch.uint8,
                             device=self.device)
            _lib.check(L.dc_bernoulli(table.data_ptr(), words.data_ptr(), ctypes.byref(left),
                                      ctypes.byref(nxt), m, float(p), bits[start // 32:].data_ptr(),
                                      ws.data_ptr(), ws.numel(), stream))
            self._left, self._next = left.value, nxt.value
        return bits


_default = {}


def default_generator(device=None):
    """The default generator of ``device`` (the current GPU when None)."""
    device = torch.device("cuda", torch.cuda.current_device()) if device is None else torch.device(device)
    if device.type == "cuda" and device.index is None:
        device = torch.device("cuda", torch.cuda.current_device())
    key = (device.type, device.index)
    if key not in _default:
        _default[key] = Generator(device)
        if _pending_seed is not None:
            _default[key].manual_seed(_pending_seed)
    return _default[key]


_pending_seed = None


def manual_seed(seed):
    """Seed the default generator(s); the same seed gives the reference's draws
    (``python/densecore/_random.py:113-115``).  Returns the current GPU's default generator
    (None on a machine without a GPU, where the seed still applies to generators made later)."""
    global _pending_seed
    _pending_seed = _seed_value(seed)
    for g in _default.values():
        g.manual_seed(_pending_seed)
    return default_generator() if torch.cuda.is_available() else None


def initial_seed():
    return default_generator().initial_seed()


def get_rng_state():
    return default_generator().get_state()


def set_rng_state(new_state):
    default_generator().set_state(new_state)
