"""Seeded synthetic inputs and tolerance checks shared by the tests and bench.py.

Inputs follow the measurement protocol: ``np.random.default_rng(seed)`` and
``standard_normal(dtype=float32)`` drawn in the order q, k, v, dO; C3 draws its per-sequence
valid lengths first; C4 scales k and v by 0.5; C5 rounds to bf16 (round to nearest even) and
the CPU reference runs on the exact float32 upcast of those values.
"""
import numpy as np

CONFIGS = {
    # name: (B, H, L, S, E, causal, backward, seed)
    "C1": (64, 6, 256, 256, 64, True, False, 1),
    "C2": (8, 12, 1024, 1024, 64, True, True, 2),
    "C3": (16, 16, 512, 512, 64, False, False, 3),
    "C4": (32, 32, 1, 4096, 128, False, False, 4),
    "C5": (2, 32, 8192, 8192, 128, True, True, 5),
}


def bf16_round(x):
    """float32 -> nearest-even bfloat16, returned as float32 (exact upcast)."""
    u = np.ascontiguousarray(x, np.float32).view(np.uint32).astype(np.uint64)
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16) << 16
    return r.astype(np.uint32).view(np.float32)


def make_inputs(name, B=None, H=None, L=None, S=None, E=None):
    """Inputs of config ``name``, optionally at reduced sizes (same seed and draw order)."""
    B0, H0, L0, S0, E0, causal, bwd, seed = CONFIGS[name]
    B, H, L, S, E = B or B0, H or H0, L or L0, S or S0, E or E0
    rng = np.random.default_rng(seed)
    out = {"causal": causal, "backward": bwd, "mask_bool": None, "lengths": None}
    if name == "C3":
        out["lengths"] = rng.integers(64, 513, size=B) if S >= 512 else rng.integers(1, S + 1, size=B)
    q = rng.standard_normal((B, H, L, E), dtype=np.float32)
    k = rng.standard_normal((B, H, S, E), dtype=np.float32)
    v = rng.standard_normal((B, H, S, E), dtype=np.float32)
    if name == "C4":
        k *= np.float32(0.5)
        v *= np.float32(0.5)
    g = rng.standard_normal((B, H, L, E), dtype=np.float32) if bwd else None
    if name == "C5":
        q, k, v, g = (bf16_round(x) for x in (q, k, v, g))
    if name == "C3":
        allowed = np.arange(S)[None, :] < out["lengths"][:, None]  # (B, S)
        out["mask_bool"] = allowed[:, None, None, :]
    out.update(q=q, k=k, v=v, g=g)
    return out


def additive(mask_bool, shape):
    """The reference's bool -> 0/-inf conversion, broadcast to (B, H, L, S)."""
    m = np.where(mask_bool, np.float32(0.0), np.float32(-np.inf))
    return np.ascontiguousarray(np.broadcast_to(m, shape), np.float32)


def f32_violations(got, ref):
    """Elements outside |got - ref| <= 2e-5 + 1e-5 |ref| (NaN counts as a violation)."""
    got, ref = np.asarray(got, np.float64), np.asarray(ref, np.float64)
    diff = np.abs(got - ref)
    bad = ~(diff <= 2e-5 + 1e-5 * np.abs(ref))
    return int(bad.sum()), float(np.nanmax(diff)) if diff.size else 0.0


def assert_f32(got, ref, name):
    n, mx = f32_violations(got, ref)
    assert n == 0, f"{name}: {n} elements outside 2e-5 + 1e-5|ref| (max abs diff {mx:.3e})"


def assert_bf16(got, ref, name):
    """|got - ref| <= 1e-2 |ref| + 1e-2 rms(ref) elementwise."""
    got, ref = np.asarray(got, np.float64), np.asarray(ref, np.float64)
    rms = float(np.sqrt(np.mean(ref ** 2))) if ref.size else 0.0
    diff = np.abs(got - ref)
    bad = ~(diff <= 1e-2 * np.abs(ref) + 1e-2 * rms)
    assert not bad.any(), (f"{name}: {int(bad.sum())} elements outside 1e-2|ref| + 1e-2 rms "
                           f"(max abs diff {float(np.nanmax(diff)):.3e}, rms {rms:.3e})")


def _same_nans(got, ref, name):
    got, ref = np.asarray(got, np.float64), np.asarray(ref, np.float64)
    gn, rn = np.isnan(got), np.isnan(ref)
    assert (gn == rn).all(), (f"{name}: NaN at {int((gn & ~rn).sum())} elements the reference has "
                              f"finite, finite at {int((rn & ~gn).sum())} it has NaN")
    return got[~rn], ref[~rn]


def assert_f32_nan(got, ref, name):
    """The reference's NaN elements exactly, and the float32 bar on every other element."""
    g, r = _same_nans(got, ref, name)
    assert_f32(g, r, name)


def assert_bf16_nan(got, ref, name):
    """The reference's NaN elements exactly, and the bf16 bar (rms over the finite elements) on
    every other element."""
    g, r = _same_nans(got, ref, name)
    assert_bf16(g, r, name)
