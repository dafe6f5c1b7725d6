"""The C ABI on a machine without a GPU: the library loads, exports every function the header
declares, agrees with the header on the descriptor layout, and rejects bad arguments with the
reference's messages (src/lib.rs:555-607, 658-663) before any kernel is launched."""
import ctypes
import os
import re
import subprocess

import pytest

from densecore_amd import _lib

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
INCLUDE = os.path.join(ROOT, "include")


def header_functions():
    """Every function any header under include/ declares."""
    names = set()
    for h in sorted(os.listdir(INCLUDE)):
        if h.endswith(".h"):
            names |= set(re.findall(r"\b(dc_[a-z_0-9]+)\s*\(", open(os.path.join(INCLUDE, h)).read()))
    return sorted(names)


def test_library_exports_every_declared_function():
    L = _lib.lib()
    declared = header_functions()
    assert declared, "no functions parsed from the header"
    assert set(declared) == set(_lib.EXPORTS)
    for name in declared:
        assert hasattr(L, name), name
    out = subprocess.run(["nm", "-D", "--defined-only", _lib.LIB_PATH], capture_output=True,
                         text=True, check=True).stdout
    exported = set(re.findall(r" T (dc_[a-z_0-9]+)$", out, re.M))
    assert set(declared) <= exported


def test_descriptor_layout_matches_header(tmp_path):
    src = tmp_path / "layout.c"
    src.write_text('#include <stddef.h>\n#include <stdio.h>\n#include "dc_attn.h"\n'
                   "int main(void){printf(\"%zu %zu %zu %zu %zu\\n\", sizeof(dc_attn_desc),"
                   " offsetof(dc_attn_desc, causal), offsetof(dc_attn_desc, scale),"
                   " offsetof(dc_attn_desc, dtype), offsetof(dc_attn_desc, mask_stride_l));"
                   "printf(\"%zu %d\\n\", offsetof(dc_attn_desc, flags), DC_FLAG_CONSISTENT_SCORES);"
                   "return 0;}\n")
    exe = tmp_path / "layout"
    subprocess.run(["gcc", "-I", os.path.join(ROOT, "include"), str(src), "-o", str(exe)], check=True)
    got = list(map(int, subprocess.run([str(exe)], capture_output=True, text=True,
                                       check=True).stdout.split()))
    D = _lib.Desc
    assert got == [ctypes.sizeof(D), D.causal.offset, D.scale.offset, D.dtype.offset,
                   D.mask_stride_l.offset, D.flags.offset, _lib.DC_FLAG_CONSISTENT_SCORES]


def test_softmax_descriptor_layout_matches_header(tmp_path):
    src = tmp_path / "layout.c"
    src.write_text('#include <stddef.h>\n#include <stdio.h>\n#include "dc_math.h"\n'
                   "int main(void){printf(\"%zu %zu %zu %zu\\n\", sizeof(dc_softmax_desc),"
                   " offsetof(dc_softmax_desc, q_len), offsetof(dc_softmax_desc, mask_stride_l),"
                   " offsetof(dc_softmax_desc, safe));return 0;}\n")
    exe = tmp_path / "layout"
    subprocess.run(["gcc", "-I", INCLUDE, str(src), "-o", str(exe)], check=True)
    got = list(map(int, subprocess.run([str(exe)], capture_output=True, text=True,
                                       check=True).stdout.split()))
    D = _lib.SoftmaxDesc
    assert got == [ctypes.sizeof(D), D.q_len.offset, D.mask_stride_l.offset, D.safe.offset]


def softmax_desc(**kw):
    d = dict(rows=6, width=5, heads=1, q_len=1, mask_stride_b=0, mask_stride_h=0,
             mask_stride_l=0, safe=0, reserved=0)
    d.update(kw)
    return _lib.SoftmaxDesc(**d)


@pytest.mark.parametrize("kw,use_mask,status,msg", [
    (dict(width=0), False, _lib.DC_INVALID_ARGUMENT, "nonempty reduction axis"),
    (dict(rows=0, width=0), False, _lib.DC_INVALID_ARGUMENT, "nonempty reduction axis"),
    (dict(rows=-1), False, _lib.DC_INVALID_ARGUMENT, "negative"),
    (dict(width=2**31), False, _lib.DC_UNSUPPORTED, "2\\^31"),
    (dict(heads=4, q_len=4), True, _lib.DC_INVALID_ARGUMENT, "rows == B\\*H\\*L"),
    (dict(heads=0), True, _lib.DC_INVALID_ARGUMENT, "rows == B\\*H\\*L"),
    (dict(heads=2, q_len=3, mask_stride_l=-5), True, _lib.DC_INVALID_ARGUMENT, "non-negative"),
    (dict(), False, _lib.DC_INVALID_ARGUMENT, "null pointer"),
])
def test_softmax_argument_errors(kw, use_mask, status, msg):
    L = _lib.lib()
    d = softmax_desc(**kw)
    mask = ctypes.c_void_p(16) if use_mask else None   # never dereferenced: rejected first
    assert L.dc_softmax_fwd(ctypes.byref(d), None, mask, None, None) == status
    assert re.search(msg, L.dc_last_error().decode())


def test_softmax_empty_rows_accepted():
    L = _lib.lib()
    assert L.dc_softmax_fwd(ctypes.byref(softmax_desc(rows=0)), None, None, None, None) == _lib.DC_OK
    assert L.dc_softmax_bwd(ctypes.byref(softmax_desc(rows=0)), None, None, None, None) == _lib.DC_OK


def desc(**kw):
    d = dict(batch=2, heads=4, kv_heads=2, q_len=8, kv_len=8, head_dim=16, causal=0, has_scale=0,
             scale=0.0, dtype=_lib.DC_F32, flags=0, mask_stride_b=0, mask_stride_h=0,
             mask_stride_l=0)
    d.update(kw)
    return _lib.Desc(**d)


def fwd(d, mask=None):
    L = _lib.lib()
    return L.dc_sdpa_fwd(ctypes.byref(d), None, None, None, mask, None, None, None, 0, None)


@pytest.mark.parametrize("kw,status,msg", [
    (dict(kv_heads=3), _lib.DC_INVALID_ARGUMENT, "q/k/v shapes do not match"),
    (dict(kv_heads=0), _lib.DC_INVALID_ARGUMENT, "q/k/v shapes do not match"),
    (dict(q_len=-1), _lib.DC_INVALID_ARGUMENT, r"takes \(B, H, L, E\) tensors"),
    (dict(dtype=7), _lib.DC_INVALID_ARGUMENT, "dtype"),
    (dict(flags=2), _lib.DC_INVALID_ARGUMENT, "flags has unknown bits"),
    (dict(q_len=2**31), _lib.DC_UNSUPPORTED, "2\\^31"),
])
def test_forward_argument_errors(kw, status, msg):
    assert fwd(desc(**kw)) == status
    assert re.search(msg, _lib.lib().dc_last_error().decode())
    with pytest.raises(ValueError if status == _lib.DC_INVALID_ARGUMENT else NotImplementedError,
                       match=msg):
        _lib.check(status)


def test_null_pointers_rejected_and_empty_accepted():
    assert fwd(desc()) == _lib.DC_INVALID_ARGUMENT
    assert "null pointer" in _lib.lib().dc_last_error().decode()
    assert fwd(desc(batch=0)) == _lib.DC_OK  # nothing to do: no launch, no pointers needed
    assert fwd(desc(q_len=0)) == _lib.DC_OK


def test_mask_strides_and_workspace_checks():
    L = _lib.lib()
    d = desc(mask_stride_b=-1)
    assert fwd(d, mask=ctypes.c_void_p(16)) == _lib.DC_INVALID_ARGUMENT
    assert "mask must be (B, H, L, S)" in L.dc_last_error().decode()
    d = desc()
    need = L.dc_sdpa_bwd_workspace_size(ctypes.byref(d))
    dsum = 256  # the minimum: dsum, float32 per (b, h, l) = 2 * 4 * 8 * 4 bytes, 256-byte aligned
    # float32 asks for dsum plus the deterministic dQ slots (one key tile: 8 rows of each of the
    # 8 (b, h), 16 floats each); with only dsum it still runs (dQ by float atomics).
    assert need >= dsum + 8 * 8 * 16 * 4
    st = L.dc_sdpa_bwd(ctypes.byref(d), *([None] * 11), dsum - 1, None)
    assert st == _lib.DC_INVALID_ARGUMENT and "workspace" in L.dc_last_error().decode()
    bf = desc(dtype=_lib.DC_BF16)
    # bf16 asks for dsum plus the fp16 copies of q, k, v, dout (B2 H4 L8 E16: 2 x 1024 + 2 x 512
    # halves) and their scratch; with only dsum it still runs (the bf16 hi + lo products).
    need_bf = L.dc_sdpa_bwd_workspace_size(ctypes.byref(bf))
    assert need_bf >= dsum + 2 * (2 * 4 * 8 * 16) * 2 + 2 * (2 * 2 * 8 * 16) * 2
    st = L.dc_sdpa_bwd(ctypes.byref(bf), *([None] * 11), dsum - 1, None)
    assert st == _lib.DC_INVALID_ARGUMENT and "workspace" in L.dc_last_error().decode()
    fw = L.dc_sdpa_fwd_workspace_size(ctypes.byref(bf))
    assert fw >= L.dc_sdpa_fwd_workspace_size(ctypes.byref(d)) + 2 * 2 * 8 * 16 * 2  # + V's fp16 copy
    dd = desc(q_len=2)
    st = L.dc_sdpa_decode(ctypes.byref(dd), *([None] * 6), 1 << 20, None)
    assert st == _lib.DC_INVALID_ARGUMENT and "q_len == 1" in L.dc_last_error().decode()
    dc = desc(q_len=1, causal=1)
    st = L.dc_sdpa_decode(ctypes.byref(dc), *([None] * 6), 1 << 20, None)
    assert st == _lib.DC_INVALID_ARGUMENT and "non-causal" in L.dc_last_error().decode()


def test_decode_workspace_covers_splits():
    L = _lib.lib()
    for B, H, S, E in [(32, 32, 4096, 128), (1, 1, 1, 64), (1, 1, 100000, 64), (4, 8, 0, 32)]:
        d = desc(batch=B, heads=H, kv_heads=H, q_len=1, kv_len=S, head_dim=E)
        ws = L.dc_sdpa_decode_workspace_size(ctypes.byref(d))
        # at least one (acc[E], max, sum) record per (batch, head), and no more than 2048 keys
        # per split
        splits = max(1, -(-S // 2048))
        assert ws >= B * H * splits * (E + 2) * 4


def test_schedule_layout_matches_header(tmp_path):
    src = tmp_path / "layout.c"
    src.write_text('#include <stddef.h>\n#include <stdio.h>\n#include "dc_attn.h"\n'
                   "int main(void){printf(\"%zu %zu %zu %zu\\n\", sizeof(dc_sdpa_schedule),"
                   " offsetof(dc_sdpa_schedule, deterministic), offsetof(dc_sdpa_schedule, workgroups),"
                   " offsetof(dc_sdpa_schedule, chunks));"
                   "return 0;}\n")
    exe = tmp_path / "layout"
    subprocess.run(["gcc", "-I", INCLUDE, str(src), "-o", str(exe)], check=True)
    got = list(map(int, subprocess.run([str(exe)], capture_output=True, text=True,
                                       check=True).stdout.split()))
    S = _lib.Schedule
    assert got == [ctypes.sizeof(S), S.deterministic.offset, S.workgroups.offset, S.chunks.offset]


def test_schedule_query_is_a_dry_run():
    """The schedule query runs the launchers' decisions without launching: it works without a GPU
    (no device: no split, no stream-K; the grids are the whole-tile ones) and reports the
    workgroups each launch would take."""
    L = _lib.lib()
    d = _lib.Desc(8, 12, 12, 1024, 1024, 64, 1, 0, 0.0, _lib.DC_F32, 0, 0, 0, 0)
    out = _lib.Schedule()
    assert L.dc_sdpa_fwd_schedule(ctypes.byref(d), 0, 1 << 20, ctypes.byref(out)) == _lib.DC_OK
    assert out.split_chunk == 0 and out.split_pieces == 1
    assert out.workgroups == (1024 // 128) * 8 * 12  # 128-query tiles of every (b, h)
    ws = L.dc_sdpa_bwd_workspace_size(ctypes.byref(d))
    assert L.dc_sdpa_bwd_schedule(ctypes.byref(d), 0, ws, ctypes.byref(out)) == _lib.DC_OK
    assert out.streamk_ranges == 0
    assert out.workgroups > (1024 // 128) * 8 * 12  # the pre-kernel, then one per key tile
    # Errors are the call's own: a backward workspace below dsum is rejected.
    assert L.dc_sdpa_bwd_schedule(ctypes.byref(d), 0, 0, ctypes.byref(out)) == _lib.DC_INVALID_ARGUMENT
    bad = _lib.Desc(1, 3, 2, 4, 4, 8, 0, 0, 0.0, _lib.DC_F32, 0, 0, 0, 0)
    assert L.dc_sdpa_fwd_schedule(ctypes.byref(bad), 0, 0, ctypes.byref(out)) == _lib.DC_INVALID_ARGUMENT
    assert L.dc_last_error() == b"flash attention q/k/v shapes do not match"


def test_bmm_argument_errors():
    """dc_bmm rejects bad shapes before any launch (no GPU needed)."""
    L = _lib.lib()

    def bmm(batch, m, n, k, a=None, b=None, c=None):
        d = _lib.BmmDesc(batch, m, n, k, m * k, k, 1, k * n, n, 1)
        return L.dc_bmm(ctypes.byref(d), a, b, c, None)

    assert bmm(-1, 2, 2, 2) == _lib.DC_INVALID_ARGUMENT
    assert L.dc_last_error() == b"bmm requires rank-3 operands"
    assert bmm(1, 2 ** 31, 2, 2) == _lib.DC_UNSUPPORTED
    assert bmm(0, 5, 5, 5) == _lib.DC_OK  # nothing to compute: no pointers needed
    assert bmm(3, 0, 5, 5) == _lib.DC_OK
    assert bmm(2, 3, 4, 5) == _lib.DC_INVALID_ARGUMENT
    assert b"null pointer" in L.dc_last_error()


def test_bmm_descriptor_layout_matches_header(tmp_path):
    src = tmp_path / "layout.c"
    src.write_text('#include <stddef.h>\n#include <stdio.h>\n#include "dc_math.h"\n'
                   "int main(void){printf(\"%zu %zu %zu\\n\", sizeof(dc_bmm_desc),"
                   " offsetof(dc_bmm_desc, a_stride_batch), offsetof(dc_bmm_desc, b_stride_n));return 0;}\n")
    exe = tmp_path / "layout"
    subprocess.run(["gcc", "-I", INCLUDE, str(src), "-o", str(exe)], check=True)
    got = list(map(int, subprocess.run([str(exe)], capture_output=True, text=True,
                                       check=True).stdout.split()))
    D = _lib.BmmDesc
    assert got == [ctypes.sizeof(D), D.a_stride_batch.offset, D.b_stride_n.offset]


def test_wide_head_dims_take_the_materialized_path():
    """Head dims above the flash kernels' (128 float32, 256 bf16) run materialized over row blocks in the workspace (any head dim, as
    the reference's kernels take any): the schedule query reports the rows per block, the
    workspace is required, and a smaller one only shortens the blocks."""
    L = _lib.lib()
    out = _lib.Schedule()
    for dtype in (_lib.DC_F32, _lib.DC_BF16):
        d = desc(head_dim=300, dtype=dtype, q_len=50, kv_len=70)
        full = L.dc_sdpa_fwd_workspace_size(ctypes.byref(d))
        assert L.dc_sdpa_fwd_schedule(ctypes.byref(d), 0, full, ctypes.byref(out)) == _lib.DC_OK
        assert out.materialized_rows == 2 * 50  # repeat (4 / 2) x L rows per (batch, kv head)
        assert L.dc_sdpa_fwd_schedule(ctypes.byref(d), 0, 0, ctypes.byref(out)) == _lib.DC_INVALID_ARGUMENT
        assert b"head_dim above the flash kernels' (128 for float32, 256 for bfloat16)" in L.dc_last_error()
        one_row = full - (2 * 50 - 1) * 2 * 2 * 70 * 4  # full minus 99 rows of (items x S) floats
        assert L.dc_sdpa_fwd_schedule(ctypes.byref(d), 0, one_row, ctypes.byref(out)) == _lib.DC_OK
        assert 1 <= out.materialized_rows < 2 * 50
        bw = L.dc_sdpa_bwd_workspace_size(ctypes.byref(d))
        assert L.dc_sdpa_bwd_schedule(ctypes.byref(d), 0, bw, ctypes.byref(out)) == _lib.DC_OK
        assert out.materialized_rows == 2 * 50 and out.deterministic == 1


def test_bf16_head_dims_to_256_take_the_flash_kernels():
    """bf16 head dims 129-256 run on the flash kernels (no materialized rows, no workspace needed);
    float32 ones run materialized."""
    L = _lib.lib()
    out = _lib.Schedule()
    for E in (129, 200, 256):
        d = desc(head_dim=E, dtype=_lib.DC_BF16, q_len=50, kv_len=70)
        assert L.dc_sdpa_fwd_schedule(ctypes.byref(d), 0, 0, ctypes.byref(out)) == _lib.DC_OK
        assert out.materialized_rows == 0
        bw = L.dc_sdpa_bwd_workspace_size(ctypes.byref(d))
        assert L.dc_sdpa_bwd_schedule(ctypes.byref(d), 0, bw, ctypes.byref(out)) == _lib.DC_OK
        assert out.materialized_rows == 0 and out.f16_products == 1 and out.deterministic == 1
        d32 = desc(head_dim=E, dtype=_lib.DC_F32, q_len=50, kv_len=70)
        full = L.dc_sdpa_fwd_workspace_size(ctypes.byref(d32))
        assert L.dc_sdpa_fwd_schedule(ctypes.byref(d32), 0, full, ctypes.byref(out)) == _lib.DC_OK
        assert out.materialized_rows > 0
