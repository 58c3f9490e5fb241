"""GPU: the one-launch decode (merge workgroups appended to the page pass's
grid, waiting on per-(sequence, kv group) piece counters) gives the bits of
the two-launch path, and leaves the workspace's counters at zero.

Both paths run the same page pass and combine the same pieces in the same
order; only where the merge runs differs, so the outputs must be identical.
The counters sit at a fixed place at the start of the workspace, so calls of
different shapes (decode and verify) can share one workspace.
"""

from __future__ import annotations

import pytest
import torch

from nimbus_amd import workloads
from nimbus_amd.kernels.paged_attention import (COUNTER_BYTES, decode_workspace_bytes, decode_workspace_error,
                                                new_decode_workspace, paged_decode_attention, paged_verify_attention,
                                                verify_workspace_bytes)
from tests.gpu_helpers import announce, oracle_decode
from tests.helpers import assert_within, random_tables, scattered_cache

pytestmark = pytest.mark.gpu


def _case(heads, kv, d, ctx_lens, dtype, seed=0, nq=1):
    pool = max(64, sum(-(-c // 16) for c in ctx_lens) + 8)
    k, v = scattered_cache(pool, 16, kv, d, seed=seed, dtype=dtype, device="cuda")
    bt = random_tables(ctx_lens, 16, pool, seed=seed, device="cuda")
    ctx = torch.tensor(ctx_lens, dtype=torch.int32, device="cuda")
    g = torch.Generator(device="cuda").manual_seed(seed + 1)
    q = torch.randn(len(ctx_lens) * nq, heads, d, generator=g, device="cuda").to(dtype)
    return q, k, v, ctx, bt, d ** -0.5


def _clear(ws):
    return bool(ws[:COUNTER_BYTES].eq(0).all())


def _two_launch(q, k, v, ctx, bt, maxc, scale, ws):
    out = torch.empty_like(q)
    paged_decode_attention(q, k, v, ctx, bt, maxc, scale, out=out, workspace=ws, _entry="nimbus_paged_decode_pages")
    paged_decode_attention(q, k, v, ctx, bt, maxc, scale, out=out, workspace=ws, _entry="nimbus_paged_decode_merge")
    return out


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("heads,kv,d,batch", [(32, 8, 128, 64), (32, 8, 128, 65), (32, 8, 128, 130),
                                              (32, 8, 128, 3), (32, 4, 64, 16), (32, 4, 128, 64),
                                              (16, 2, 64, 200), (32, 16, 128, 64)])
def test_one_launch_equals_two_launches(dtype, heads, kv, d, batch):
    announce(f"fused decode H={heads} KV={kv} D={d} B={batch} {dtype}")
    ctx_lens = workloads.llama3_decode_lens(seed=batch, batch=batch)
    q, k, v, ctx, bt, scale = _case(heads, kv, d, ctx_lens, dtype, seed=batch)
    maxc = max(ctx_lens)
    ws = new_decode_workspace(decode_workspace_bytes(batch, heads, d, maxc), "cuda")
    two = _two_launch(q, k, v, ctx, bt, maxc, scale, ws)
    one = paged_decode_attention(q, k, v, ctx, bt, maxc, scale, workspace=ws)
    torch.cuda.synchronize()
    assert _clear(ws) and decode_workspace_error(ws) == 0
    assert torch.equal(one, two)
    assert_within(one.cpu(), oracle_decode(q, k, v, ctx_lens, bt, scale), what="vs oracle")


def test_one_workspace_across_shapes_and_a_graph():
    """One workspace serves decode calls of 64, then 20 sequences, a verify
    call of 5 queries a sequence, and graph replays of the 64-sequence call
    with eager calls between them: every result has the two-launch bits and
    the counters are back at zero after each call."""
    announce("fused decode: shared workspace across shapes, graph replay")
    lens64 = workloads.llama3_decode_lens(seed=1, batch=64)
    q, k, v, ctx, bt, scale = _case(32, 8, 128, lens64, torch.bfloat16, seed=1)
    ws = new_decode_workspace(max(decode_workspace_bytes(64, 32, 128, 8192),
                                  verify_workspace_bytes(20, 5, 32, 128, 8192)), "cuda")
    ref64 = _two_launch(q, k, v, ctx, bt, 8192, scale, ws)
    got = paged_decode_attention(q, k, v, ctx, bt, 8192, scale, workspace=ws)
    torch.cuda.synchronize()
    assert torch.equal(got, ref64) and _clear(ws)
    q20, ctx20, bt20 = q[:20].contiguous(), ctx[:20].contiguous(), bt[:20].contiguous()
    ref20 = _two_launch(q20, k, v, ctx20, bt20, 8192, scale, ws)
    got20 = paged_decode_attention(q20, k, v, ctx20, bt20, 8192, scale, workspace=ws)
    torch.cuda.synchronize()
    assert torch.equal(got20, ref20) and _clear(ws)
    g = torch.Generator(device="cuda").manual_seed(7)
    qv = torch.randn(20 * 5, 32, 128, generator=g, device="cuda").bfloat16()
    ver = paged_verify_attention(qv, k, v, ctx20, bt20, 5, 8192, scale, workspace=ws)
    torch.cuda.synchronize()
    assert _clear(ws)
    last = qv.view(20, 5, 32, 128)[:, 4].contiguous()  # each sequence's newest query sees its whole context
    assert_within(ver.view(20, 5, 32, 128)[:, 4].cpu(), oracle_decode(last, k, v, lens64[:20], bt20, scale),
                  what="verify, newest queries vs oracle")
    out = torch.empty_like(q)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        paged_decode_attention(q, k, v, ctx, bt, 8192, scale, out=out, workspace=ws)
    for i in range(4):
        out.zero_()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, ref64), f"replay {i}"
        assert _clear(ws)
        paged_decode_attention(q20, k, v, ctx20, bt20, 8192, scale, workspace=ws)  # eager work between replays
    assert decode_workspace_error(ws) == 0


def test_other_kernels_leave_the_cached_decode_workspace_alone():
    """The INT8 matmul's split-K partials and the prefill pieces' slots write
    their workspaces from the first byte: they keep caches of their own, so
    the decode workspace cached per stream keeps zero counters and the next
    decode and verify calls (taking it by default) stay right."""
    announce("fused decode after INT8 split-K and prefill pieces")
    from nimbus_amd.kernels import paged_attention as pa
    from nimbus_amd.kernels.int8_matmul import int8_matmul, int8_matmul_workspace_bytes
    from nimbus_amd.kernels.prefill_attention import paged_prefill_attention, plan_pieces
    from nimbus_amd.quant import quantize_weight

    g = torch.Generator(device="cuda").manual_seed(3)
    used = 0
    for m, n, kdim in ((64, 6144, 4096), (64, 4096, 14336), (16, 4096, 4096), (1, 28672, 4096)):
        if int8_matmul_workspace_bytes(m, n, kdim) > 0:
            used += 1
            wq, sc = quantize_weight((torch.randn(n, kdim, generator=g, device="cuda") * 0.02).bfloat16())
            int8_matmul(torch.randn(m, kdim, generator=g, device="cuda").bfloat16(), wq, sc)
    assert used > 0
    b = workloads.build_batch([(8192 + 64, 64)], heads=32, kv_heads=8, head_dim=128, dtype=torch.bfloat16,
                              device="cuda", seed=4, write_first=False)
    args = b.prefill_args()
    plan = plan_pieces(args[7], args[8], 32, 8, "cuda")
    assert plan is not None
    paged_prefill_attention(*args, plan)
    lens = workloads.llama3_decode_lens(seed=5, batch=64)
    q, k, v, ctx, bt, scale = _case(32, 8, 128, lens, torch.bfloat16, seed=5)
    got = paged_decode_attention(q, k, v, ctx, bt, max(lens), scale)  # the cached workspace
    torch.cuda.synchronize()
    ws = pa._WORKSPACES[(torch.cuda.current_device(), torch._C._cuda_getCurrentRawStream(torch.cuda.current_device()))]
    assert _clear(ws) and decode_workspace_error(ws) == 0
    own = new_decode_workspace(decode_workspace_bytes(64, 32, 128, max(lens)), "cuda")
    assert torch.equal(got, _two_launch(q, k, v, ctx, bt, max(lens), scale, own))
