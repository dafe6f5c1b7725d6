"""The flash path under HIP graph capture (torch.cuda.CUDAGraph), as a serving loop would run it.

A forward + backward (and a decode) is captured once, then replayed several times with new input
values copied into the captured tensors between replays and other eager GPU work around them; every
replay must give bit-identical results to eager calls on the same values (the float32 backward
with its full workspace and the bf16 backward are deterministic).  The library's kernels record no
memset nodes (workspaces are written by kernels only), and the Python boundary gives a captured call
a workspace of its own from the graph's memory pool.
"""
import pytest

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu

DEV = "cuda:0"
REPLAYS = 3


@pytest.mark.parametrize("dtype,B,H,Hkv,L,S,E,causal", [
    ("f32", 2, 4, 4, 300, 300, 64, True),
    ("f32", 1, 8, 8, 2048, 2048, 64, True),    # stream-K backward, split forward
    ("bf16", 1, 4, 2, 512, 700, 128, False),   # fp16 copies, grouped heads
    ("bf16", 1, 2, 2, 4096, 4096, 128, True),  # split bf16 grids
])
def test_flash_graph_replays(dtype, B, H, Hkv, L, S, E, causal):
    from densecore_amd import _native
    dt = torch.bfloat16 if dtype == "bf16" else torch.float32
    print(f"[case] graph {dtype} B{B} H{H} Hkv{Hkv} L{L} S{S} E{E} causal={causal}", flush=True)
    gen = torch.Generator(device=DEV).manual_seed(L + S + E)
    draw = lambda *shape: torch.randn(*shape, device=DEV, generator=gen, dtype=dt)
    inputs = [(draw(B, H, L, E), draw(B, Hkv, S, E), draw(B, Hkv, S, E), draw(B, H, L, E))
              for _ in range(REPLAYS + 1)]
    # Eager results for every set of values.
    want = []
    for q, k, v, g in inputs:
        out, lse = _native._flash_attention(q, k, v, causal)
        want.append((out, lse) + tuple(_native._flash_attention_backward(g, q, k, v, out, lse, causal)))
    torch.cuda.synchronize()

    sq, sk, sv, sg = (t.clone() for t in inputs[0])
    side = torch.cuda.Stream(device=DEV)
    side.wait_stream(torch.cuda.current_stream(DEV))
    with torch.cuda.stream(side):  # warm-up on the capture stream, as torch asks
        out, lse = _native._flash_attention(sq, sk, sv, causal)
        _native._flash_attention_backward(sg, sq, sk, sv, out, lse, causal)
    torch.cuda.current_stream(DEV).wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        gout, glse = _native._flash_attention(sq, sk, sv, causal)
        gdq, gdk, gdv = _native._flash_attention_backward(sg, sq, sk, sv, gout, glse, causal)
    scratch = torch.randn(1024, 1024, device=DEV)
    for r in range(REPLAYS + 1):
        for dst, src in zip((sq, sk, sv, sg), inputs[r]):
            dst.copy_(src)
        scratch = scratch @ scratch.T / 1024.0  # unrelated eager work before the replay
        graph.replay()
        torch.cuda.synchronize()
        for name, got, ref in zip(("out", "lse", "dq", "dk", "dv"), (gout, glse, gdq, gdk, gdv), want[r]):
            assert torch.equal(got, ref), f"replay {r}: {name} differs from the eager call"


def test_decode_graph_replays():
    from densecore_amd import _native
    print("[case] graph decode f32 B4 H8 S3000 E128", flush=True)
    gen = torch.Generator(device=DEV).manual_seed(7)
    draw = lambda *shape: torch.randn(*shape, device=DEV, generator=gen)
    inputs = [(draw(4, 8, 1, 128), draw(4, 8, 3000, 128), draw(4, 8, 3000, 128)) for _ in range(REPLAYS + 1)]
    want = [_native._flash_decode(q, k, v) for q, k, v in inputs]
    torch.cuda.synchronize()
    sq, sk, sv = (t.clone() for t in inputs[0])
    side = torch.cuda.Stream(device=DEV)
    side.wait_stream(torch.cuda.current_stream(DEV))
    with torch.cuda.stream(side):
        _native._flash_decode(sq, sk, sv)
    torch.cuda.current_stream(DEV).wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        gout, glse = _native._flash_decode(sq, sk, sv)
    for r in range(REPLAYS + 1):
        for dst, src in zip((sq, sk, sv), inputs[r]):
            dst.copy_(src)
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(gout, want[r][0]) and torch.equal(glse, want[r][1]), f"replay {r} differs"


@pytest.mark.parametrize("dtype", ["f32", "bf16"])
def test_public_api_graphed_callable(dtype):
    """functional.scaled_dot_product_attention with autograd through
    torch.cuda.make_graphed_callables (forward and backward each one captured graph): outputs and
    input gradients of every call equal eager ones on the same values."""
    from densecore_amd import functional as F
    dt = torch.bfloat16 if dtype == "bf16" else torch.float32
    print(f"[case] graphed callable {dtype}", flush=True)
    B, H, L, E = 2, 4, 256, 64

    def fn(q, k, v):
        return F.scaled_dot_product_attention(q, k, v, is_causal=True)

    gen = torch.Generator(device=DEV).manual_seed(3)
    draw = lambda: torch.randn(B, H, L, E, device=DEV, generator=gen, dtype=dt)
    sample = tuple(draw().requires_grad_() for _ in range(3))
    graphed = torch.cuda.make_graphed_callables(fn, sample)
    for r in range(REPLAYS):
        vals = [draw() for _ in range(4)]
        eager = [x.clone().requires_grad_() for x in vals[:3]]
        y_ref = fn(*eager)
        y_ref.backward(vals[3])
        cap = [x.clone().requires_grad_() for x in vals[:3]]
        y = graphed(*cap)
        y.backward(vals[3])
        torch.cuda.synchronize()
        assert torch.equal(y, y_ref), f"call {r}: output differs"
        for name, a, b in zip("qkv", cap, eager):
            assert torch.equal(a.grad, b.grad), f"call {r}: d{name} differs"
