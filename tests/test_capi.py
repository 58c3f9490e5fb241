"""CPU: the C-ABI library loads, exports everything include/nimbus_attn.h
declares, and rejects bad arguments before any launch (no GPU needed)."""

from __future__ import annotations

import os
import re
import subprocess

import pytest

from nimbus_amd import _lib

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "nimbus_attn.h")


def declared_functions() -> list[str]:
    text = open(HEADER).read()
    return re.findall(r"^(?:int|int64_t|const char\*)\s+(nimbus_\w+)\(", text, flags=re.M)


def test_header_declares_the_four_launch_paths():
    names = declared_functions()
    for want in ("nimbus_write_kv", "nimbus_paged_decode", "nimbus_paged_decode_workspace_bytes",
                 "nimbus_paged_prefill", "nimbus_paged_verify", "nimbus_paged_verify_workspace_bytes",
                 "nimbus_paged_prefill_pieces", "nimbus_paged_prefill_pieces_workspace_bytes",
                 "nimbus_add_rms_norm", "nimbus_int8_matmul", "nimbus_int8_matmul_workspace_bytes",
                 "nimbus_attn_abi_version",
                 "nimbus_attn_error_string"):
        assert want in names


def test_library_exports_every_declared_symbol():
    lib = _lib.load()
    nm = subprocess.run(["nm", "-D", "--defined-only", _lib.LIB_PATH], capture_output=True, text=True, check=True)
    exported = set(re.findall(r"\bT (nimbus_\w+)", nm.stdout))
    for name in declared_functions():
        assert name in exported, name
        assert hasattr(lib, name)
        assert name in _lib.SIGNATURES, f"{name} has no ctypes signature"


def test_abi_version_and_error_strings():
    lib = _lib.load()
    assert lib.nimbus_attn_abi_version() == _lib.ABI_VERSION
    for code in (0, -1, -2, -3, -4, -5):
        assert lib.nimbus_attn_error_string(code)
    assert b"unknown" in lib.nimbus_attn_error_string(-99)


def test_one_hip_runtime_in_process():
    import torch  # noqa: F401

    _lib.load()
    assert len(_lib.hip_runtimes()) == 1, _lib.hip_runtimes()


def test_workspace_bytes_is_a_pure_size_formula():
    lib = _lib.load()
    f = lib.nimbus_paged_decode_workspace_bytes

    def r256(n):
        return -(-n // 256) * 256

    def want(b, h, d, maxc):
        waves = max(1, min(256 * 8, b * -(-maxc // 16) // 2))  # slices of >= 2 pages, <= resident waves
        slots = waves + b  # one per (wave, sequence) piece
        return r256((b + 1) * 4) + r256(slots * h * 2 * 4) + slots * h * d * 4  # prefix, (m, l), O

    assert f(64, 32, 128, 8192) == want(64, 32, 128, 8192) == 512 + 2112 * 32 * 8 + 2112 * 32 * 512
    assert f(1, 32, 128, 100) == want(1, 32, 128, 100) == 256 + 1024 + 4 * 32 * 512  # 7 pages: 3 slices + 1
    assert f(16, 32, 64, 1024) == want(16, 32, 64, 1024)
    assert f(-1, 32, 128, 8192) == -1


def test_verify_workspace_scales_the_decode_formula_by_queries():
    """A verify call holds pieces for queries_per_seq columns per head: the
    decode workspace of queries_per_seq x num_heads heads."""
    lib = _lib.load()
    f, dec = lib.nimbus_paged_verify_workspace_bytes, lib.nimbus_paged_decode_workspace_bytes
    assert f(16, 1, 32, 128, 8192) == dec(16, 32, 128, 8192)
    assert f(16, 5, 32, 128, 8192) == dec(16, 160, 128, 8192)
    assert f(3, 16, 8, 64, 100) == dec(3, 128, 64, 100)
    for bad in (0, 17, -1):
        assert f(16, bad, 32, 128, 8192) == -1


DUMMY = 1 << 20  # a 16-byte aligned fake address: these calls must return before touching it


def _decode(**kw):
    a = dict(q=DUMMY, qsb=32 * 128, qsh=128, k=DUMMY, v=DUMMY, nb=100, csb=16 * 8 * 128, cst=8 * 128, csh=128,
             bt=DUMMY, bts=4, btw=4, ctx=DUMMY, out=DUMMY, osb=32 * 128, osh=128, ws=None, wsb=0, b=2, h=32,
             kv=8, d=128, bs=16, maxc=64, scale=0.1, dt=1, stream=None)
    a.update(kw)
    return _lib.load().nimbus_paged_decode(*a.values())


@pytest.mark.parametrize("kw,code", [
    # other page sizes and head dims run the general kernel; past it they are refused before launch
    (dict(bs=0), _lib.NIMBUS_ERR_UNSUPPORTED),
    (dict(d=264), _lib.NIMBUS_ERR_UNSUPPORTED),
    (dict(d=96, bs=8, q=None), _lib.NIMBUS_ERR_INVALID),
    (dict(d=96, bs=8, b=0), 0),
    (dict(d=96, bs=8, dt=7), _lib.NIMBUS_ERR_UNSUPPORTED),
    (dict(dt=7), _lib.NIMBUS_ERR_UNSUPPORTED),
    (dict(h=30), _lib.NIMBUS_ERR_INVALID),
    (dict(q=None), _lib.NIMBUS_ERR_INVALID),
    (dict(qsh=100), _lib.NIMBUS_ERR_ALIGNMENT),
    (dict(q=DUMMY + 2), _lib.NIMBUS_ERR_ALIGNMENT),
    (dict(maxc=4096), _lib.NIMBUS_ERR_WORKSPACE),
    (dict(maxc=64), _lib.NIMBUS_ERR_WORKSPACE),  # the chunk prefix is always needed
    (dict(b=4097), _lib.NIMBUS_ERR_UNSUPPORTED),
    (dict(b=0), 0),
    (dict(maxc=0), 0),
])
def test_decode_argument_checks(kw, code):
    assert _decode(**kw) == code


def test_verify_argument_checks():
    """queries_per_seq outside 1..16 is refused; the rest are the decode
    checks, with the workspace sized for every query column."""
    lib = _lib.load()

    def verify(nq, **kw):
        a = dict(q=DUMMY, qsb=32 * 128, qsh=128, k=DUMMY, v=DUMMY, nb=100, csb=16 * 8 * 128, cst=8 * 128, csh=128,
                 bt=DUMMY, bts=4, btw=4, ctx=DUMMY, out=DUMMY, osb=32 * 128, osh=128, ws=None, wsb=0, b=2, h=32,
                 kv=8, d=128, bs=16, maxc=64, scale=0.1, dt=1, stream=None)
        a.update(kw)
        return lib.nimbus_paged_verify(nq, *a.values())

    assert verify(0) == _lib.NIMBUS_ERR_INVALID
    assert verify(17) == _lib.NIMBUS_ERR_UNSUPPORTED
    assert verify(5, bs=0) == _lib.NIMBUS_ERR_UNSUPPORTED
    assert verify(5, d=264) == _lib.NIMBUS_ERR_UNSUPPORTED
    assert verify(5, b=0) == 0
    # a workspace big enough for decode is too small for five query columns
    dec = lib.nimbus_paged_decode_workspace_bytes(2, 32, 128, 64)
    assert verify(5, ws=DUMMY, wsb=dec) == _lib.NIMBUS_ERR_WORKSPACE


def test_prefill_and_write_kv_argument_checks():
    lib = _lib.load()
    base = [DUMMY, 32 * 128, 128, DUMMY, DUMMY, 100, 16 * 8 * 128, 8 * 128, 128, DUMMY, 4, 4, DUMMY, DUMMY, DUMMY,
            DUMMY, 3, DUMMY, 32 * 128, 128, 32, 8, 128, 16, 0.1, 1, None]
    # other page sizes and head dims run the general kernel; past it they are refused before launch
    assert lib.nimbus_paged_prefill(*base[:23], 0, *base[24:]) == _lib.NIMBUS_ERR_UNSUPPORTED  # block size
    assert lib.nimbus_paged_prefill(*base[:16], 0, *base[17:]) == 0  # no tiles: nothing to launch
    assert lib.nimbus_paged_prefill(*base[:22], 264, *base[23:]) == _lib.NIMBUS_ERR_UNSUPPORTED  # head dim
    assert lib.nimbus_paged_prefill(*base[:22], 80, 8, *base[24:25], 7, None) == _lib.NIMBUS_ERR_UNSUPPORTED  # dtype
    assert lib.nimbus_paged_prefill(*base[:16], 0, *base[17:22], 80, 8, *base[24:]) == 0  # general, no tiles
    # page offsets are 32 x 32-bit products: block strides of 2^30 elements and up are refused
    assert lib.nimbus_paged_prefill(*base[:6], 1 << 30, *base[7:]) == _lib.NIMBUS_ERR_UNSUPPORTED
    wk =[DUMMY, DUMMY, DUMMY, DUMMY, DUMMY, 0, 8, 128, 8 * 128, 128, 8 * 128, 128, 1600, 1, None]
    assert lib.nimbus_write_kv(*wk) == 0  # zero tokens
    wk[13] = 3
    wk[5] = 5
    assert lib.nimbus_write_kv(*wk) == _lib.NIMBUS_ERR_UNSUPPORTED


def test_rope_write_kv_rejects_before_launch():
    """Every argument the fused rotary + slot write refuses returns its code
    before any pointer is touched."""
    lib = _lib.load()

    def call(**kw):
        a = dict(qkv=DUMMY, qs=48 * 128, t=5, h=32, kv=8, d=128, pos=DUMMY, cos=DUMMY, sin=DUMMY, ts=128, mp=4096,
                 kc=DUMMY, vc=DUMMY, slots=DUMMY, ns=1600, dt=1)
        a.update(kw)
        return lib.nimbus_rope_write_kv(a["qkv"], a["qs"], a["t"], a["h"], a["kv"], a["d"], a["pos"], a["cos"],
                                        a["sin"], a["ts"], a["mp"], a["kc"], a["vc"], a["slots"], a["ns"], a["dt"],
                                        None)

    assert call(t=0) == 0  # no tokens: nothing to launch
    assert call(d=72) == _lib.NIMBUS_ERR_UNSUPPORTED  # head_dim % 16
    assert call(dt=4) == _lib.NIMBUS_ERR_UNSUPPORTED
    assert call(kv=0) == _lib.NIMBUS_ERR_INVALID
    assert call(slots=None) == _lib.NIMBUS_ERR_INVALID
    assert call(qs=40 * 128) == _lib.NIMBUS_ERR_INVALID  # row narrower than q + k + v heads
    assert call(ts=64) == _lib.NIMBUS_ERR_INVALID  # table row narrower than head_dim
    assert call(kc=DUMMY + 8) == _lib.NIMBUS_ERR_ALIGNMENT
    assert call(qs=48 * 128 + 4) == _lib.NIMBUS_ERR_ALIGNMENT
    assert call(ts=130) == _lib.NIMBUS_ERR_ALIGNMENT


def test_rms_norm_rejects_before_launch():
    """Shapes outside the kernel and null pointers return an error code; no
    pointer is dereferenced on the host, so null is safe to pass here."""
    lib = _lib.load()
    f = lib.nimbus_add_rms_norm
    for cols in (12, 0, 8200, 16384):  # not a multiple of 8, empty, too long
        assert f(None, 0, None, 0, None, None, 0, None, 0, 4, cols, 1e-5, 0, None) in (-1, -2)
    assert f(None, 0, None, 0, None, None, 0, None, 0, 4, 16, 1e-5, 7, None) == -2  # dtype
    assert f(None, 0, None, 0, None, None, 0, None, 0, 4, 16, 1e-5, 0, None) == -1  # null x
    assert f(None, 0, None, 0, None, None, 0, None, 0, 0, 16, 1e-5, 0, None) == 0  # no rows: nothing to do


def test_int8_matmul_rejects_before_launch():
    """Null pointers, misaligned elements, short strides and a missing
    split-K workspace return an error code without touching memory; shapes
    the tiled kernel does not take need no workspace (the general kernel)."""
    lib = _lib.load()
    f = lib.nimbus_int8_matmul
    ws = lib.nimbus_int8_matmul_workspace_bytes
    args = lambda m, n, k, **kw: dict(x=DUMMY, xs=k, w=DUMMY, wsd=k, s=DUMMY, y=DUMMY, ys=n, m=m, n=n, k=k,
                                      ws=None, wsb=0, dt=0, stream=None) | kw
    call = lambda **kw: f(*kw.values())
    assert call(**args(4, 4098, 2048, x=None)) == _lib.NIMBUS_ERR_INVALID  # n % 4: checked like any shape
    assert call(**args(4, 4096, 2040, y=None)) == _lib.NIMBUS_ERR_INVALID  # k % 16
    assert ws(4, 4098, 2048) == 0 and ws(4, 4096, 2040) == 0  # the general kernel takes no workspace
    assert call(**args(4, 4096, 2048, dt=5)) == _lib.NIMBUS_ERR_UNSUPPORTED
    assert call(**args(0, 4096, 2048)) == 0
    assert call(**args(4, 4096, 2048, x=None)) == _lib.NIMBUS_ERR_INVALID
    assert call(**args(4, 4096, 2048, xs=2044)) == _lib.NIMBUS_ERR_INVALID  # stride below k
    assert call(**args(4, 4096, 2048, x=DUMMY + 1)) == _lib.NIMBUS_ERR_ALIGNMENT  # not on a 2-byte element
    assert call(**args(4, 4096, 2048, s=DUMMY + 3)) == _lib.NIMBUS_ERR_ALIGNMENT
    assert ws(4, 4096, 2048) > 0  # 32 channel tiles: K is split, so a workspace is needed
    assert call(**args(4, 4096, 2048)) == _lib.NIMBUS_ERR_WORKSPACE
    assert ws(300, 11264, 2048) == 0  # 88 x 5 tiles fill the chip: no split
    assert ws(-1, 4, 16) == -1


def test_split_partials_entries_reject_before_launch():
    """The split-K partials of a projection and the norm that folds them in
    refuse plans that do not split, short workspaces, rows the norm's chunked
    kernel does not take, missing pointers and misalignment, before any
    launch."""
    lib = _lib.load()
    part = lib.nimbus_int8_matmul_packed_partials
    pargs = lambda **kw: dict(x=DUMMY, xs=4096, w=DUMMY, m=64, n=4096, k=4096, bm=64, ks=1, splits=4, rw=1,
                              ws=DUMMY, wsb=1 << 30, dt=1, stream=None) | kw
    call = lambda f, d: f(*d.values())
    assert call(part, pargs(m=-1)) == _lib.NIMBUS_ERR_INVALID
    assert call(part, pargs(splits=1)) == _lib.NIMBUS_ERR_UNSUPPORTED  # no split: nothing to leave unreduced
    assert call(part, pargs(bm=48)) == _lib.NIMBUS_ERR_UNSUPPORTED
    assert call(part, pargs(dt=5)) == _lib.NIMBUS_ERR_UNSUPPORTED
    assert call(part, pargs(m=0)) == 0
    assert call(part, pargs(x=None)) == _lib.NIMBUS_ERR_INVALID
    assert call(part, pargs(ws=None)) == _lib.NIMBUS_ERR_WORKSPACE
    assert call(part, pargs(wsb=4 * 64 * 4096 * 4 - 4)) == _lib.NIMBUS_ERR_WORKSPACE
    assert call(part, pargs(x=DUMMY + 8)) == _lib.NIMBUS_ERR_ALIGNMENT
    norm = lib.nimbus_add_rms_norm_partials
    nargs = lambda **kw: dict(p=DUMMY, splits=4, s=DUMMY, r=DUMMY, rs=4096, w=DUMMY, o=DUMMY, os=4096, ro=DUMMY,
                              ros=4096, rows=64, cols=4096, eps=1e-5, dt=1, stream=None) | kw
    assert call(norm, nargs(splits=0)) == _lib.NIMBUS_ERR_INVALID
    assert call(norm, nargs(cols=4100)) == _lib.NIMBUS_ERR_UNSUPPORTED  # not a multiple of 8
    assert call(norm, nargs(cols=16384, rs=16384, os=16384, ros=16384)) == _lib.NIMBUS_ERR_UNSUPPORTED  # past 8192
    assert call(norm, nargs(rows=0)) == 0
    assert call(norm, nargs(r=None)) == _lib.NIMBUS_ERR_INVALID  # the residual is required
    assert call(norm, nargs(rs=4000)) == _lib.NIMBUS_ERR_INVALID
    assert call(norm, nargs(s=DUMMY + 8)) == _lib.NIMBUS_ERR_ALIGNMENT


def test_int8_packed_silu_rejects_before_launch():
    """The fused gate_up + SiLU entry refuses shapes, plans, null pointers,
    short strides and misalignment with an error code, before any launch."""
    lib = _lib.load()
    f = lib.nimbus_int8_matmul_packed_silu
    args = lambda m, n, k, **kw: dict(x=DUMMY, xs=k, w=DUMMY, s=DUMMY, y=DUMMY, ys=n // 2, m=m, n=n, k=k, bm=0,
                                      ks=1, rw=1, dt=1, stream=None) | kw
    call = lambda **kw: f(*kw.values())
    assert call(**args(-1, 28672, 4096)) == _lib.NIMBUS_ERR_INVALID
    assert call(**args(4, 4112, 4096)) == _lib.NIMBUS_ERR_UNSUPPORTED  # n not a multiple of 32
    assert call(**args(4, 28672, 4092)) == _lib.NIMBUS_ERR_UNSUPPORTED  # k not a multiple of 8
    assert call(**args(4, 28672, 4096, dt=5)) == _lib.NIMBUS_ERR_UNSUPPORTED
    for bad in [dict(bm=48), dict(bm=16, ks=8), dict(bm=128, ks=2), dict(bm=64, rw=3), dict(bm=64, ks=3)]:
        assert call(**args(4, 28672, 4096, **bad)) == _lib.NIMBUS_ERR_UNSUPPORTED, bad
    assert call(**args(0, 28672, 4096)) == 0  # no rows: nothing to launch
    # 65536 token tiles of 16: more than the grid's z dimension takes (65535 of them are still accepted
    # as a plan: the workspace query answers for it)
    assert call(**args(16 * 65536, 64, 64, bm=16)) == _lib.NIMBUS_ERR_UNSUPPORTED
    assert lib.nimbus_int8_matmul_packed_plan_workspace_bytes(16 * 65536, 64, 64, 16, 1, 1, 1) == -1
    assert lib.nimbus_int8_matmul_packed_plan_workspace_bytes(16 * 65535, 64, 64, 16, 1, 1, 1) == 0
    assert call(**args(4, 28672, 4096, x=None)) == _lib.NIMBUS_ERR_INVALID
    assert call(**args(4, 28672, 4096, xs=4088)) == _lib.NIMBUS_ERR_INVALID  # stride below k
    assert call(**args(4, 28672, 4096, ys=14332)) == _lib.NIMBUS_ERR_INVALID  # stride below n / 2
    assert call(**args(4, 28672, 4096, x=DUMMY + 1)) == _lib.NIMBUS_ERR_ALIGNMENT
    assert call(**args(4, 28672, 4096, x=DUMMY + 2)) == _lib.NIMBUS_ERR_ALIGNMENT  # not 16-byte aligned
    assert call(**args(4, 28672, 4096, s=DUMMY + 4)) == _lib.NIMBUS_ERR_ALIGNMENT
    assert call(**args(4, 28672, 4096, ys=14338)) == _lib.NIMBUS_ERR_ALIGNMENT  # y stride not a multiple of 4


def test_stream_flag_area_is_the_same_for_every_plan():
    """The stream-K workspace keeps its flags and error word at the same
    offsets whatever the plan, so calls with different plans can share one
    workspace; the slots after them grow with the plan."""
    lib = _lib.load()
    fb = lib.nimbus_paged_prefill_stream_flag_bytes
    ws = lib.nimbus_paged_prefill_stream_workspace_bytes
    sizes = {fb(s, h, kv) for s, h, kv in [(1, 8, 8), (128, 32, 1), (64, 32, 8), (512, 64, 8), (7, 28, 4)]}
    assert len(sizes) == 1 and sizes.pop() > 0
    assert fb(-1, 32, 8) == -1 and fb(4, 30, 8) == -1
    assert fb(4, 32, 8) < ws(4, 32, 8, 64) < ws(8, 32, 8, 64) < ws(8, 32, 8, 128)


def test_int8_workspace_is_splits_times_fp32_output():
    lib = _lib.load()
    ws = lib.nimbus_int8_matmul_workspace_bytes
    # 4096 channels = 32 tiles of 128, one 16-token tile: 8 splits of 14336 / 8 = 1792 -> 2048 (whole
    # rings of 512) -> 7 splits
    assert ws(16, 4096, 14336) == 7 * 16 * 4096 * 4
    assert ws(1, 3072, 2048) == 4 * 1 * 3072 * 4  # 24 tiles want 11 splits; 2048 / 512 allows 4


def test_int8_explicit_plan_workspace_and_validation():
    lib = _lib.load()
    ws = lib.nimbus_int8_matmul_packed_plan_workspace_bytes
    assert ws(64, 4096, 14336, 64, 2, 4, 1) == 4 * 64 * 4096 * 4
    assert ws(64, 4096, 14336, 32, 2, 4, 2) == 4 * 64 * 4096 * 4  # rows per wave does not change the split
    assert ws(64, 28672, 4096, 64, 2, 1, 2) == 0
    for bad in [(48, 1, 1, 1), (64, 4, 1, 1), (16, 3, 1, 1), (16, 1, 17, 1), (16, 1, 1, 0), (16, 1, 1, 3)]:
        assert ws(64, 4096, 4096, *bad) == -1, bad
    # shapes the tiled kernel does not take have no plan, and the default call needs no workspace
    assert ws(64, 4098, 4096, 64, 2, 1, 1) == -1 and ws(64, 4096, 4092, 64, 2, 1, 1) == -1
    assert lib.nimbus_int8_matmul_packed_workspace_bytes(64, 4098, 4096) == 0


def test_prefill_pieces_checks():
    lib = _lib.load()
    assert lib.nimbus_paged_prefill_pieces_workspace_bytes(3, 32, 128) == 3 * 64 * 32 * 130 * 4
    assert lib.nimbus_paged_prefill_pieces_workspace_bytes(-1, 32, 128) == -1
    base = [DUMMY, 32 * 128, 128, DUMMY, DUMMY, 100, 16 * 8 * 128, 8 * 128, 128, DUMMY, 4, 4, DUMMY, DUMMY]
    tail = [DUMMY, 32 * 128, 128, 32, 8, 128, 16, 0.1, 1, None]
    f = lib.nimbus_paged_prefill_pieces
    assert f(*base, None, 3, None, 0, 0, None, 0, *tail) == _lib.NIMBUS_ERR_INVALID  # no piece table
    assert f(*base, DUMMY, 3, DUMMY, 1, 2, None, 0, *tail) == _lib.NIMBUS_ERR_WORKSPACE  # slots need a workspace
    assert f(*base, DUMMY, 0, None, 0, 0, None, 0, *tail) == 0  # no pieces: nothing to launch
