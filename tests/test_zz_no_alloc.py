"""GPU: the allocation-free decode entry point (nimbus_paged_decode_noalloc)
against nimbus_paged_decode with a caller-owned workspace, through the C ABI.

Two calls in a row on the library's scratch array, the second with a
smaller input than the first (the array keeps the first call's contents),
each equal bit for bit to nimbus_paged_decode on the same inputs (the same
kernels and grid) and so within the output bar of it; a call that needs more
workspace than the array holds is refused before launch."""

from __future__ import annotations

import ctypes

import pytest
import torch

from nimbus_amd import _lib, workloads
from nimbus_amd.kernels.paged_attention import (decode_workspace_bytes, new_decode_workspace,
                                                paged_decode_attention, paged_decode_attention_noalloc)
from tests.gpu_helpers import announce
from tests.helpers import assert_within

pytestmark = pytest.mark.gpu


def _noalloc_c(q, kc, vc, ctx, bt, maxc, scale, out):
    """One call straight through the C ABI; returns its code."""
    lib = _lib.load()
    return lib.nimbus_paged_decode_noalloc(
        q.data_ptr(), q.stride(0), q.stride(1), kc.data_ptr(), vc.data_ptr(), kc.shape[0], kc.stride(0),
        kc.stride(1), kc.stride(2), bt.data_ptr(), bt.stride(0), bt.shape[1], ctx.data_ptr(), out.data_ptr(),
        out.stride(0), out.stride(1), q.shape[0], q.shape[1], kc.shape[2], q.shape[2], kc.shape[1], int(maxc),
        ctypes.c_float(scale), _lib.dtype_code(q.dtype), _lib.stream_of(q))


def _with_workspace(q, kc, vc, ctx, bt, maxc, scale):
    ws = new_decode_workspace(decode_workspace_bytes(q.shape[0], q.shape[1], q.shape[2], maxc), q.device)
    return paged_decode_attention(q, kc, vc, ctx, bt, maxc, scale, workspace=ws)


def test_noalloc_matches_workspace_entry_point_twice():
    # Call 1: config 3 (B=64, Llama-3-8B heads, bf16, contexts up to 8192).
    announce("noalloc call 1: llama3_decode (config 3)")
    big = workloads.llama3_decode("cuda")
    a = big.decode_args()
    want1 = _with_workspace(a[0], a[1], a[2], a[3], a[4], 8192, a[6])
    got1 = torch.full_like(a[0], float("nan"))
    assert _noalloc_c(a[0], a[1], a[2], a[3], a[4], 8192, a[6], got1) == 0
    torch.cuda.synchronize()
    assert torch.equal(got1, want1)
    assert_within(got1.cpu(), want1.cpu().double(), what="call 1 vs nimbus_paged_decode")
    # Call 2, right after on the same scratch: a smaller batch, TinyLlama heads, fp16.
    announce("noalloc call 2: 5 sequences, TinyLlama heads, fp16")
    small = workloads.build_batch([(700, 1), (1, 1), (33, 1), (2048, 1), (17, 1)], heads=32, kv_heads=4,
                                  head_dim=64, dtype=torch.float16, device="cuda", seed=9, write_first=False)
    s = small.decode_args()
    want2 = _with_workspace(s[0], s[1], s[2], s[3], s[4], s[5], s[6])
    got2 = torch.full_like(s[0], float("nan"))
    assert _noalloc_c(s[0], s[1], s[2], s[3], s[4], s[5], s[6], got2) == 0
    torch.cuda.synchronize()
    assert torch.equal(got2, want2)
    assert_within(got2.cpu(), want2.cpu().double(), what="call 2 vs nimbus_paged_decode")
    # And through the Python wrapper once more.
    got3 = paged_decode_attention_noalloc(s[0], s[1], s[2], s[3], s[4], s[5], s[6], torch.empty_like(s[0]))
    torch.cuda.synchronize()
    assert torch.equal(got3, want2)


def test_noalloc_refuses_calls_beyond_its_scratch():
    announce("noalloc refuses an oversized call")
    q = torch.zeros(4096, 64, 128, dtype=torch.bfloat16, device="cuda")
    kc = torch.zeros(8, 16, 8, 128, dtype=torch.bfloat16, device="cuda")
    ctx = torch.ones(4096, dtype=torch.int32, device="cuda")
    bt = torch.zeros(4096, 2048, dtype=torch.int32, device="cuda")
    assert decode_workspace_bytes(4096, 64, 128, 32768) > _lib.NOALLOC_SCRATCH_BYTES
    out = torch.full_like(q, 7.0)
    assert _noalloc_c(q, kc, kc, ctx, bt, 32768, 0.1, out) == _lib.NIMBUS_ERR_SCRATCH
    torch.cuda.synchronize()
    assert bool((out == 7.0).all())  # nothing was launched
    with pytest.raises(ValueError):
        paged_decode_attention_noalloc(q, kc, kc, ctx, bt, 32768, 0.1, out)
