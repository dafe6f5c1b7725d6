"""Benchmark of the SDPA hot path on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu] [--only C2,C4,math,sched]

A step is one pass of the hot path over one batch of synthetic, HBM-resident input:
C2 (the headline) is causal fp32 forward + backward at B8 H12 T1024
D64 through the C ABI (dc_sdpa_fwd then dc_sdpa_bwd).  ``value`` is C2's algorithmic TFLOP/s
(4*B*H*T^2*D/2 forward, 2.5x that backward), after exactly W untimed steps.  The same line
carries the decode figure the
metric names (C4, dc_sdpa_decode, GB/s of K + V + q + out + lse), the other configurations'
throughput (wall clock over K steps between two synchronizations, each config warmed up for at
least W steps and 100 ms of its own work, so that it is timed at steady clocks), a roofline entry per
entry point whose kernel time comes from HIP events on the launch stream around back-to-back
calls of that entry point alone (``in_step`` gives the same entry points timed inside the step, by
events in a separate loop of the same steps), and the CPU baseline: the oracle (a C port of
DenseCore's CPU path) timed on this host.
C2 runs last, straight after C1's GPU work (float32 MFMA work like its own) with its inputs already
on the device, so that its W warm-up steps start at the clocks the device holds under that load.
``math_path`` reports the composed path's own kernels (softmax forward/backward, the Bernoulli
mask from the reference's generator stream, the dropout product) at C3's shape.  ``--only sched``
(not in the default run) times the few-heads shapes that take the split / stream-K schedules.
"""
import argparse
import json
import os
import sys
import time

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, HERE)

PEAK_FP32_MFMA = 157.3   # TFLOP/s, MI355X dense
PEAK_BF16_MFMA = 2500.0  # TFLOP/s, MI355X dense
PEAK_HBM = 8000.0        # GB/s

METRIC = "SDPA fwd+bwd TFLOP/s & %MFMA peak (B8 H12 T1024 D64); decode GB/s"


def flops(B, H, L, S, E, causal, backward):
    """Algorithmic FLOPs: 4*B*H*L*S*E (two GEMMs), halved when causal; backward is 2.5x."""
    f = 4.0 * B * H * L * S * E / (2 if causal else 1)
    return f, 2.5 * f if backward else 0.0


def decode_bytes(B, H, S, E, elem=4):
    """K + V + q + out (elem bytes each) + lse (float32)."""
    return 2 * B * H * S * E * elem + 2 * B * H * E * elem + B * H * 4


def load_traffic():
    """Measured HBM bytes per launch (rocprofv3 FETCH_SIZE + WRITE_SIZE, copy-kernel scaled)."""
    path = os.path.join(HERE, "profiles", "traffic.json")
    if os.path.exists(path):
        with open(path) as f:
            return json.load(f)
    return {}


# Secondary configs warm up for at least this long (and at least --warmup steps): after the host
# has built a config's inputs the GPU has idled and its clock has dropped, and a few steps of a
# 50 us config do not bring it back.  The headline C2 step takes exactly --warmup steps.
MIN_WARMUP_MS = 100.0


def warm_up(torch, fn, steps, headline):
    """Run ``fn`` untimed: ``steps`` times, and for secondary configs until MIN_WARMUP_MS of it
    has run."""
    for _ in range(steps):
        fn()
    torch.cuda.synchronize()
    if headline:
        return
    t0 = time.perf_counter()
    while (time.perf_counter() - t0) * 1e3 < MIN_WARMUP_MS:
        for _ in range(10):
            fn()
        torch.cuda.synchronize()


def kernel_ms(torch, stream, fn, n):
    """Average duration of one call of ``fn`` (its kernels only, launched back to back) from one
    pair of HIP events around n calls on the launch stream.  An event pair around every call
    would add two marker packets, and their waits, to each call's time."""
    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    a.record(stream)
    for _ in range(n):
        fn()
    b.record(stream)
    b.synchronize()
    return a.elapsed_time(b) / n


def in_step_ms(torch, stream, fwd, bwd, n):
    """Mean per-entry-point time inside the step itself: n more steps, with pre-made HIP events
    recorded before the forward, between it and the backward, and after (a separate loop, so the
    timed steps carry no event packets).  Their sum is the step's GPU time plus the events' own
    cost (a few us per interval on this part), against which ms_per_step can be compared."""
    ev = [[torch.cuda.Event(enable_timing=True) for _ in range(3 if bwd else 2)] for _ in range(n)]
    for e in ev:
        e[0].record(stream)
        out, lse = fwd()
        e[1].record(stream)
        if bwd is not None:
            bwd(out, lse)
            e[2].record(stream)
    torch.cuda.synchronize()
    f = sum(e[0].elapsed_time(e[1]) for e in ev) / n
    if bwd is None:
        return {"fwd_ms": round(f, 4), "steps": n}
    b = sum(e[1].elapsed_time(e[2]) for e in ev) / n
    return {"fwd_ms": round(f, 4), "bwd_ms": round(b, 4), "sum_ms": round(f + b, 4), "steps": n}


def roofline(achieved, peak, unit, bound, traffic, kernel, work_note):
    return {"bound": bound, "achieved": round(achieved, 3), "peak": peak, "unit": unit,
            "frac": round(achieved / peak, 4), "traffic": traffic, "kernel": kernel,
            "work": work_note}


def parity(got, ref, bf16=False):
    """Margins of one output against the oracle: max |gpu - ref|, the normwise relative error,
    and the largest fraction of the elementwise bar used (<= 1 passes): float32
    |gpu - ref| <= 2e-5 + 1e-5 |ref|; bf16 |gpu - ref| <= 1e-2 |ref| + 1e-2 rms(ref)."""
    got, ref = np.asarray(got, np.float64), np.asarray(ref, np.float64)
    diff = np.abs(got - ref)
    if bf16:
        bar = 1e-2 * np.abs(ref) + 1e-2 * float(np.sqrt(np.mean(ref ** 2)))
    else:
        bar = 2e-5 + 1e-5 * np.abs(ref)
    used = diff / np.maximum(bar, 1e-300)
    nref = float(np.linalg.norm(ref))
    return {"max_abs": float(np.nanmax(diff)) if diff.size else 0.0,
            "normwise_rel": float(np.linalg.norm(diff) / nref) if nref else 0.0,
            "bar_used": float(np.nanmax(used)) if used.size else 0.0,
            "allclose": bool(np.all(diff <= bar))}


def host_cpus():
    """This host's CPUs as the CPU baseline sees them: `nproc` (the affinity mask), the cgroup
    CPU quota when one is set, and the CPU model."""
    nproc = len(os.sched_getaffinity(0))
    quota = None
    try:
        with open("/sys/fs/cgroup/cpu.max") as f:
            q, per = f.read().split()[:2]
            if q != "max":
                quota = float(q) / float(per)
    except (OSError, ValueError):
        pass
    model = None
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    model = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    return nproc, quota, model


def prepare_prefill(torch, name, dev):
    """A prefill config's inputs, drawn on the host and copied to the device."""
    from tests._data import CONFIGS, make_inputs, additive
    B, H, L, S, E, causal, bwd, _ = CONFIGS[name]
    d = make_inputs(name)
    dt = torch.bfloat16 if name == "C5" else torch.float32
    t = {n: torch.from_numpy(d[n]).to(dev, dt) for n in "qkv"}
    t["g"] = torch.from_numpy(d["g"]).to(dev, dt) if bwd else None
    t["mask"] = None
    if d["mask_bool"] is not None:  # C3: key padding as a broadcast (B, 1, 1, S) additive mask
        t["mask"] = torch.from_numpy(additive(d["mask_bool"], (B, 1, 1, S)).copy()).to(dev).expand(B, H, L, S)
    t["lengths"] = d["lengths"]
    torch.cuda.synchronize()
    return t


def bench_prefill(torch, native, name, steps, warmup, dev, inputs=None):
    """Forward (+ backward) of a prefill config; returns per-call mean ms and throughput."""
    from tests._data import CONFIGS
    B, H, L, S, E, causal, bwd, _ = CONFIGS[name]
    t = inputs if inputs is not None else prepare_prefill(torch, name, dev)
    q, k, v, g, mask = t["q"], t["k"], t["v"], t["g"], t["mask"]
    scale = 1.0 / np.sqrt(E)
    stream = torch.cuda.current_stream(dev)

    def fwd():
        return native._flash_attention(q, k, v, causal, scale, mask)

    def step():
        out, lse = fwd()
        if bwd:
            native._flash_attention_backward(g, q, k, v, out, lse, causal, scale, mask)

    warm_up(torch, step, warmup, headline=name == "C2")
    t0 = time.perf_counter()
    for _ in range(steps):
        step()
    torch.cuda.synchronize()
    wall = (time.perf_counter() - t0) / steps * 1e3
    # Per-entry-point kernel time, for the roofline: the same calls, back to back; and the same
    # steps with an event pair around each entry point.
    n = max(steps, 10)
    res = {"ms_per_step": wall, "fwd_ms": kernel_ms(torch, stream, fwd, n), "bwd_ms": 0.0,
           "timing_calls": n}
    res["in_step"] = in_step_ms(torch, stream, fwd, (lambda o, l: native._flash_attention_backward(
        g, q, k, v, o, l, causal, scale, mask)) if bwd else None, n)
    if bwd:
        out, lse = fwd()
        res["bwd_ms"] = kernel_ms(torch, stream, lambda: native._flash_attention_backward(
            g, q, k, v, out, lse, causal, scale, mask), n)
    # One more call whose outputs the CPU-baseline leg checks against the oracle (C5: the
    # (b = 0, h < 16) slice the CPU leg computes).
    sl = (slice(0, 1), slice(0, 16)) if name == "C5" else (slice(None), slice(None))
    out, lse = fwd()
    keep = {"out": out[sl].float().cpu().numpy(), "lse": lse[sl].cpu().numpy()}
    if bwd:
        grads = native._flash_attention_backward(g, q, k, v, out, lse, causal, scale, mask)
        keep.update({n: t[sl].float().cpu().numpy() for n, t in zip(("dq", "dk", "dv"), grads)})
        del grads
    torch.cuda.synchronize()
    res["outputs"] = keep
    ff, fb = flops(B, H, L, S, E, causal, bwd)
    if name == "C2":
        res["public"] = bench_public(torch, q, k, v, g, steps, warmup, ff + fb)
    if name == "C3":  # useful work counts valid keys only
        ff = 4.0 * H * L * E * float(np.sum(t["lengths"]))
    res.update({"fwd_flop": ff, "bwd_flop": fb})
    res["tflops"] = (ff + fb) / (wall * 1e-3) / 1e12
    res["fwd_tflops"] = ff / (res["fwd_ms"] * 1e-3) / 1e12
    if bwd:
        res["bwd_tflops"] = fb / (res["bwd_ms"] * 1e-3) / 1e12
    return res


def bench_public(torch, q, k, v, g, steps, warmup, work):
    """C2 through the public API: ``functional.scaled_dot_product_attention`` on leaf tensors
    that require gradients, then the gradients by autograd (the flash autograd node saves out
    and lse and calls the backward), wall clock over the steps."""
    from densecore_amd import functional as F
    qr, kr, vr = (t.detach().clone().requires_grad_(True) for t in (q, k, v))

    def step():
        out = F.scaled_dot_product_attention(qr, kr, vr, is_causal=True)
        torch.autograd.grad(out, (qr, kr, vr), g)

    for _ in range(warmup):
        step()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        step()
    torch.cuda.synchronize()
    ms = (time.perf_counter() - t0) / steps * 1e3
    return {"ms_per_step": round(ms, 4), "tflops": round(work / (ms * 1e-3) / 1e12, 3),
            "path": "functional.scaled_dot_product_attention + torch.autograd.grad (flash node)"}


def bench_decode(torch, native, steps, warmup, dev):
    from tests._data import CONFIGS, make_inputs
    B, H, L, S, E, _, _, _ = CONFIGS["C4"]
    d = make_inputs("C4")
    q, k, v = (torch.from_numpy(d[n]).to(dev) for n in "qkv")
    del d
    stream = torch.cuda.current_stream(dev)
    warm_up(torch, lambda: native._flash_decode(q, k, v), warmup, headline=False)
    t0 = time.perf_counter()
    for _ in range(steps):
        native._flash_decode(q, k, v)
    torch.cuda.synchronize()
    wall = (time.perf_counter() - t0) / steps * 1e3
    n = max(steps, 10)
    ev = kernel_ms(torch, stream, lambda: native._flash_decode(q, k, v), n)
    nbytes = decode_bytes(B, H, S, E)
    out, lse = native._flash_decode(q, k, v)
    keep = {"out": out.cpu().numpy(), "lse": lse.cpu().numpy()}
    return {"ms_per_step": wall, "event_ms": ev, "bytes": nbytes, "timing_calls": n,
            "gbps": nbytes / (ev * 1e-3) / 1e9, "outputs": keep}


def bench_math(torch, steps, warmup, dev):
    """The composed math path's own kernels at C3's shape (B16 H16 L=S=512, key-padding mask)
    with dropout p = 0.1: softmax forward (scores + broadcast mask -> probabilities, 8 B per
    score) and backward (12 B per score) against HBM, the Bernoulli mask drawn from the
    reference's generator stream (draws/s), the dropout product (8 B per score plus the bits),
    the two batched products (dc_bmm, next to the device BLAS), and one whole math-path step
    (forward + backward through autograd, every product on dc_bmm)."""
    import densecore_amd._native as native
    from densecore_amd import functional as F, random as R
    from tests._data import CONFIGS, additive, make_inputs
    B, H, L, S, E, _, _, _ = CONFIGS["C3"]
    d = make_inputs("C3")
    n = B * H * L * S
    stream = torch.cuda.current_stream(dev)
    x = torch.randn((B, H, L, S), device=dev)
    mask = torch.from_numpy(additive(d["mask_bool"], (B, 1, 1, S)).copy()).to(dev)
    y = native._softmax(x, mask, True)
    g = torch.randn_like(x)
    reps = max(steps, 10)
    warm_up(torch, lambda: native._softmax(x, mask, True), warmup, headline=False)
    res = {"workload": "C3 shape B16 H16 L=S=512, key-padding mask, dropout p=0.1",
           "timing_calls": reps}
    ms = kernel_ms(torch, stream, lambda: native._softmax(x, mask, True), reps)
    res["softmax_fwd"] = {"ms": round(ms, 4), "gbps": round(8 * n / (ms * 1e-3) / 1e9, 1),
                          "frac_hbm": round(8 * n / (ms * 1e-3) / 1e9 / PEAK_HBM, 4)}
    ms = kernel_ms(torch, stream, lambda: native._softmax_backward(g, y), reps)
    res["softmax_bwd"] = {"ms": round(ms, 4), "gbps": round(12 * n / (ms * 1e-3) / 1e9, 1),
                          "frac_hbm": round(12 * n / (ms * 1e-3) / 1e9 / PEAK_HBM, 4)}
    gen = R.Generator(dev).manual_seed(0)
    gen._bernoulli_bits(n, 0.9)
    ms = kernel_ms(torch, stream, lambda: gen._bernoulli_bits(n, 0.9), reps)
    res["bernoulli"] = {"ms": round(ms, 4), "gdraws_per_s": round(n / (ms * 1e-3) / 1e9, 2),
                        "mt19937_words_per_s_g": round(2 * n / (ms * 1e-3) / 1e9, 2)}
    bits = gen._bernoulli_bits(n, 0.9)
    scale = float(np.float32(1) / np.float32(0.9))
    ms = kernel_ms(torch, stream, lambda: native._dropout_apply(bits, y, scale), reps)
    nb = 8 * n + n // 8
    res["dropout_apply"] = {"ms": round(ms, 4), "gbps": round(nb / (ms * 1e-3) / 1e9, 1),
                            "frac_hbm": round(nb / (ms * 1e-3) / 1e9 / PEAK_HBM, 4)}
    del x, y, g, bits
    # The two batched products of the math path at C3's shape (256 (batch, head) items):
    # scores = q k^T (k^T a transposed view, 512 x 64 x 512) and weights v (512 x 512 x 64), by
    # dc_bmm and, for comparison, by the device BLAS (torch.bmm -> hipBLASLt).
    qa, ka = torch.randn(B * H, L, E, device=dev), torch.randn(B * H, S, E, device=dev)
    wa, va = torch.randn(B * H, L, S, device=dev), torch.randn(B * H, S, E, device=dev)
    work = 2.0 * B * H * L * S * E
    res["bmm"] = {"note": "TFLOP/s of 2*m*n*k per product, HIP events around back-to-back calls"}
    for name, fn, ref in (("q_kT", lambda: native._bmm(qa, ka.transpose(1, 2)),
                           lambda: torch.bmm(qa, ka.transpose(1, 2))),
                          ("weights_v", lambda: native._bmm(wa, va), lambda: torch.bmm(wa, va))):
        fn(), ref()
        ms_dc = kernel_ms(torch, stream, fn, reps)
        ms_bl = kernel_ms(torch, stream, ref, reps)
        res["bmm"][name] = {"dc_bmm_ms": round(ms_dc, 4), "dc_bmm_tflops": round(work / (ms_dc * 1e-3) / 1e12, 2),
                            "hipblaslt_ms": round(ms_bl, 4),
                            "hipblaslt_tflops": round(work / (ms_bl * 1e-3) / 1e12, 2),
                            "frac_fp32_mfma": round(work / (ms_dc * 1e-3) / 1e12 / PEAK_FP32_MFMA, 4)}
    del qa, ka, wa, va
    q, k, v = (torch.from_numpy(d[c]).to(dev).requires_grad_(True) for c in "qkv")
    am = torch.from_numpy(d["mask_bool"]).to(dev)
    go = torch.randn((B, H, L, E), device=dev)

    def step():
        out = F.scaled_dot_product_attention(q, k, v, attn_mask=am, dropout_p=0.1)
        out.backward(go)

    for _ in range(2):
        step()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    k_steps = max(3, steps // 10)
    for _ in range(k_steps):
        step()
    torch.cuda.synchronize()
    res["math_path_step_ms"] = round((time.perf_counter() - t0) / k_steps * 1e3, 3)
    return res


def cpu_baseline(threads, gpu):
    """The oracle (C port of DenseCore's CPU SDPA) on this host's cores, in the units of the GPU
    figures: the full C2 workload (the headline figure, median of 2), full C1, C3 (the
    reference's materialised (B, H, L, S) mask) and C4 once each, and a slice of C5 (b = 0,
    h < 16: 16 of its 64 whole (batch, head) tasks, forward and backward) extrapolated to the
    whole config; plus the math path's softmax and Bernoulli draws on a slice of C3's shape.

    The oracle's outputs of these runs are also the checker of the GPU's outputs of the same
    inputs (``gpu``: name -> host copies): ``parity`` gives each output's margins against the
    bar.  C5's backward takes the GPU's own bf16 out and lse, as the GPU backward did."""
    import oracle
    from tests._data import additive, make_inputs
    oracle.build()
    oracle.set_num_threads(threads)
    checks = {}

    def check(name, got, ref, bf16=False):
        if got is not None:
            checks[name] = {k: parity(got[k], r, bf16) for k, r in ref.items()}

    d = make_inputs("C2")
    times = []
    for _ in range(2):
        t0 = time.perf_counter()
        o, l = oracle.forward(d["q"], d["k"], d["v"], True)
        grads = oracle.backward(d["g"], d["q"], d["k"], d["v"], o, l, True)
        times.append(time.perf_counter() - t0)
    check("C2", gpu.get("C2"), dict(zip(("out", "lse", "dq", "dk", "dv"), (o, l) + tuple(grads))))
    ff, fb = flops(8, 12, 1024, 1024, 64, True, True)
    best = float(np.median(times))
    per = {}
    d = make_inputs("C1")
    t0 = time.perf_counter()
    o, l = oracle.forward(d["q"], d["k"], d["v"], True)
    dt = time.perf_counter() - t0
    check("C1", gpu.get("C1"), {"out": o, "lse": l})
    per["C1"] = {"tflops": round(flops(64, 6, 256, 256, 64, True, False)[0] / dt / 1e12, 5),
                 "s": round(dt, 3)}
    d = make_inputs("C3")
    mask = additive(d["mask_bool"], (16, 16, 512, 512))
    t0 = time.perf_counter()
    o, l = oracle.forward(d["q"], d["k"], d["v"], False, None, mask)
    dt = time.perf_counter() - t0
    check("C3", gpu.get("C3"), {"out": o, "lse": l})
    per["C3"] = {"tflops": round(4.0 * 16 * 512 * 64 * float(np.sum(d["lengths"])) / dt / 1e12, 5),
                 "s": round(dt, 3), "note": "useful FLOPs (valid keys); the CPU path computes every key"}
    del mask
    d = make_inputs("C4")
    t0 = time.perf_counter()
    o, l = oracle.forward(d["q"], d["k"], d["v"], False)
    dt = time.perf_counter() - t0
    check("C4", gpu.get("C4"), {"out": o, "lse": l})
    per["C4"] = {"gbps": round(decode_bytes(32, 32, 4096, 128) / dt / 1e9, 2), "s": round(dt, 3)}
    del d, o, l
    # C5: 16 whole (batch, head) tasks (each independent, bit-identical under any thread split,
    # src/torch_attention.rs:8) on the exact float32 upcast of the bf16 inputs.
    c5 = gpu.get("C5")
    if c5 is not None:
        d = make_inputs("C5")
        sl = (slice(0, 1), slice(0, 16))
        q, k, v, g = (np.ascontiguousarray(d[n][sl]) for n in ("q", "k", "v", "g"))
        del d
        t0 = time.perf_counter()
        o, l = oracle.forward(q, k, v, True)
        tf = time.perf_counter() - t0
        t0 = time.perf_counter()
        grads = oracle.backward(g, q, k, v, c5["out"], c5["lse"], True)
        tb = time.perf_counter() - t0
        check("C5", c5, dict(zip(("out", "lse", "dq", "dk", "dv"), (o, l) + tuple(grads))), bf16=True)
        fwd5, bwd5 = flops(2, 32, 8192, 8192, 128, True, True)
        scale = 64 / 16
        per["C5"] = {"tflops": round((fwd5 + bwd5) / ((tf + tb) * scale) / 1e12, 5),
                     "s_slice": round(tf + tb, 3), "s_full_extrapolated": round((tf + tb) * scale, 3),
                     "extrapolated": True,
                     "sample": "b = 0, h < 16: 16 of C5's 64 (batch, head) tasks, forward + backward, "
                               "x4 for the whole config"}
        del q, k, v, g, o, l, grads
    # The math path's pieces at C3's shape, single-threaded as the reference runs them:
    # softmax_lastdim over 8 of the 256 (b, h) score blocks and Generator::bernoulli draws.
    x = np.random.default_rng(0).standard_normal((8, 512, 512), dtype=np.float32)
    t0 = time.perf_counter()
    oracle.softmax(x)
    dt = time.perf_counter() - t0
    n = 16 * 16 * 512 * 512 // 8
    gen = oracle.Generator(0)
    t1 = time.perf_counter()
    gen.bernoulli(n, 0.9)
    db = time.perf_counter() - t1
    per["math_path"] = {"softmax_gbps": round(8 * x.size / dt / 1e9, 3),
                        "bernoulli_gdraws_per_s": round(n / db / 1e9, 4), "threads": 1,
                        "sample": f"softmax of {x.size} scores (8 of C3's 256 blocks, {dt:.3f} s), "
                                  f"{n} Bernoulli draws (an eighth of C3's, {db:.3f} s)"}
    nproc, quota, model = host_cpus()
    base = {"value": round((ff + fb) / best / 1e12, 5), "unit": "TFLOP/s", "cores": threads,
            "kind": "port", "nproc": nproc, "cgroup_cpus": quota, "cpu_model": model,
            "sample": f"full C2 fwd+bwd (B8 H12 T1024 D64 fp32) x{len(times)}, median "
                      f"{best:.2f} s; oracle/sdpa_oracle.c, {threads} threads",
            "configs": per}
    return base, checks


# Shapes whose whole-tile grids fill little of the device (few heads, long rows), where the
# alternative schedules run: the split forward (float32, bf16), the float32 backward's stream-K
# ranges and the bf16 backward's split grids; and head dim 256, which runs materialized over row
# blocks (its FLOPs count the causal half only, as everywhere).  Not part of the default run
# (--only sched).
SCHED_SHAPES = [  # B, H, L, E, causal, dtype
    (1, 8, 2048, 64, True, "f32"), (1, 4, 4096, 64, True, "f32"), (1, 8, 2048, 128, True, "f32"),
    (8, 12, 512, 64, True, "f32"), (6, 16, 1024, 64, False, "f32"),
    (1, 1, 16384, 128, True, "bf16"), (1, 2, 8192, 128, True, "bf16"), (1, 4, 4096, 128, True, "bf16"),
    (2, 16, 2048, 256, True, "f32"), (2, 16, 2048, 256, True, "bf16"),
]


def bench_schedules(torch, native, steps, dev):
    """Kernel time per call (HIP events around back-to-back calls) of dc_sdpa_fwd and dc_sdpa_bwd
    on SCHED_SHAPES, synthetic N(0, 1) inputs."""
    out = {}
    stream = torch.cuda.current_stream(dev)
    gen = torch.Generator(device=dev).manual_seed(0)
    n = max(steps, 10)
    for B, H, L, E, causal, dtn in SCHED_SHAPES:
        dt = torch.bfloat16 if dtn == "bf16" else torch.float32
        q, k, v, g = (torch.randn(B, H, L, E, device=dev, generator=gen).to(dt) for _ in range(4))
        o, lse = native._flash_attention(q, k, v, causal)
        for _ in range(3):
            native._flash_attention(q, k, v, causal)
            native._flash_attention_backward(g, q, k, v, o, lse, causal)
        fms = kernel_ms(torch, stream, lambda: native._flash_attention(q, k, v, causal), n)
        bms = kernel_ms(torch, stream, lambda: native._flash_attention_backward(g, q, k, v, o, lse, causal), n)
        ff, fb = flops(B, H, L, L, E, causal, True)
        out[f"{dtn} B{B} H{H} L{L} D{E} {'causal' if causal else 'full'}"] = {
            "fwd_ms": round(fms, 4), "bwd_ms": round(bms, 4),
            "fwd_tflops": round(ff / (fms * 1e-3) / 1e12, 1), "bwd_tflops": round(fb / (bms * 1e-3) / 1e12, 1)}
        del q, k, v, g, o, lse
        torch.cuda.empty_cache()
    return out


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--only", default="", help="comma list of configs to run (C1..C5, math, sched)")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="only run a plain 1 GiB device-to-device copy (torch copy_), the kernel "
                         "of known traffic that scales rocprofv3 FETCH_SIZE / WRITE_SIZE")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py: this build runs on one GPU only (asked for --gpus {args.gpus}); the "
              "path shards over (batch, head) with no collectives, each GPU running its share of "
              "the heads on its own", file=sys.stderr)
        sys.exit(2)

    import torch
    if args.copy_calibration:
        src = torch.ones(1 << 28, dtype=torch.float32, device="cuda:0")
        dst = torch.empty_like(src)
        for _ in range(5):
            dst.copy_(src)
        torch.cuda.synchronize()
        print(json.dumps({"copy_calibration_bytes_each_way": src.numel() * 4, "calls": 5}))
        return
    import densecore_amd._native as native
    from densecore_amd import _lib
    _lib.lib()  # fail loudly if the HIP library is missing
    dev = torch.device("cuda:0")
    only = set(args.only.split(",")) if args.only else {"C1", "C2", "C3", "C4", "C5"}

    results = {}
    for name in ("C3", "C5"):
        if name not in only:
            continue
        try:
            results[name] = bench_prefill(torch, native, name, args.steps, args.warmup, dev)
        except NotImplementedError as e:
            results[name] = {"skipped": str(e)}
        torch.cuda.empty_cache()
    if "math" in only or not args.only:
        results["math"] = bench_math(torch, args.steps, args.warmup, dev)
        torch.cuda.empty_cache()
    if "sched" in only:
        results["sched"] = bench_schedules(torch, native, args.steps, dev)
    if "C4" in only:
        results["C4"] = bench_decode(torch, native, args.steps, args.warmup, dev)
        torch.cuda.empty_cache()
    # The headline runs last, its inputs already on the device, straight after C1 (float32 MFMA
    # work like its own): its W warm-up steps then start at the clocks the device holds under such
    # load.  Started cold, after the host has drawn its inputs, the device ramps its clocks over
    # tens of milliseconds: a kernel trace of that loop shows the step falling from 573 to 490 us
    # over the timed steps; after the memory-bound decode config, from 513 to 485 us.
    c2_inputs = prepare_prefill(torch, "C2", dev) if "C2" in only else None
    if "C1" in only:
        results["C1"] = bench_prefill(torch, native, "C1", args.steps, args.warmup, dev)
    if c2_inputs is not None:
        results["C2"] = bench_prefill(torch, native, "C2", args.steps, args.warmup, dev, c2_inputs)
        del c2_inputs
        torch.cuda.empty_cache()

    traffic = load_traffic()
    line = {"metric": METRIC, "value": None, "unit": "TFLOP/s", "n_gpus": 1, "steps": args.steps,
            "warmup": args.warmup, "ms_per_step": None, "higher_is_better": True, "scaling": "weak",
            "vs_baseline": None, "dtype": "f32", "data": "synthetic (seeded N(0,1), HBM-resident)",
            "config": {"workload": "C2: causal SDPA fwd+bwd fp32, B=8 H=12 T=1024 D=64",
                       "global_batch": 8, "seq_len": 1024, "parallelism": "none (1 GPU)"}}
    c2 = results.get("C2")
    if c2:
        line["value"] = round(c2["tflops"], 3)
        line["ms_per_step"] = round(c2["ms_per_step"], 4)
        line["roofline"] = roofline(
            c2["bwd_tflops"], PEAK_FP32_MFMA, "TFLOP/s", "mfma", traffic.get("C2_bwd"),
            "dc_sdpa_bwd (bwd_pre_f32_kernel + bwd_f32_kernel + bwd_reduce_f32_kernel)",
            f"{c2['bwd_flop'] / 1e9:.3f} GFLOP per call / {c2['bwd_ms']:.4f} ms (HIP events around "
            f"{c2['timing_calls']} back-to-back calls)")
        line["forward_roofline"] = roofline(
            c2["fwd_tflops"], PEAK_FP32_MFMA, "TFLOP/s", "mfma", traffic.get("C2_fwd"),
            "dc_sdpa_fwd (fwd_f32_kernel)",
            f"{c2['fwd_flop'] / 1e9:.3f} GFLOP per call / {c2['fwd_ms']:.4f} ms (HIP events around "
            f"{c2['timing_calls']} back-to-back calls)")
        line["mfma_frac"] = round(c2["tflops"] / PEAK_FP32_MFMA, 4)
        line["in_step"] = c2["in_step"]
        line["public_api"] = c2["public"]
    c4 = results.get("C4")
    if c4:
        line["decode"] = {"workload": "C4: decode fp32, B=32 H=32 S=4096 D=128, split-KV",
                          "value": round(c4["gbps"], 1), "unit": "GB/s",
                          "ms_per_step": round(c4["ms_per_step"], 4),
                          "kernel_ms": round(c4["event_ms"], 4),
                          "roofline": roofline(c4["gbps"], PEAK_HBM, "GB/s", "hbm",
                                               traffic.get("C4_decode"),
                                               "dc_sdpa_decode (decode_split + decode_merge)",
                                               f"{c4['bytes']} B per call / {c4['event_ms']:.4f} ms (HIP events "
                                               f"around {c4['timing_calls']} back-to-back calls)")}
    others = {}
    for name in ("C1", "C3", "C5"):
        r = results.get(name)
        if not r:
            continue
        if "skipped" in r:
            others[name] = r
            continue
        peak = PEAK_BF16_MFMA if name == "C5" else PEAK_FP32_MFMA
        others[name] = {"tflops": round(r["tflops"], 3), "ms_per_step": round(r["ms_per_step"], 4),
                        "frac": round(r["tflops"] / peak, 4), "fwd_ms": round(r["fwd_ms"], 4)}
        if r.get("bwd_ms"):
            others[name]["bwd_ms"] = round(r["bwd_ms"], 4)
        others[name]["in_step"] = r["in_step"]
    if others:
        line["other_configs"] = others
    if results.get("math"):
        line["math_path"] = results["math"]
    if results.get("sched"):
        line["schedules"] = results["sched"]
    if not args.no_cpu:
        # The reference's default is every core it may run on (std::thread::available_parallelism,
        # src/torch_sum.rs:48): `nproc`, bounded by the cgroup's CPU quota and by the GPU box's CPU
        # share (16 per GPU).
        nproc, quota, _ = host_cpus()
        threads = max(1, min(nproc, int(quota) if quota else nproc, 16))
        gpu = {name: r["outputs"] for name, r in results.items() if isinstance(r, dict) and "outputs" in r}
        line["cpu_baseline"], line["parity"] = cpu_baseline(threads, gpu)
        line["parity_note"] = ("GPU outputs of the bench configs against the oracle's outputs of the "
                               "same inputs from the cpu_baseline leg; bar_used <= 1 passes")
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
