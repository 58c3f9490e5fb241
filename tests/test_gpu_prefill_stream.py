"""GPU: the stream-K prefill (nimbus_paged_prefill_stream) matches the
oracle within the bar, leaves its workspace flags at zero, and replays from
a hipGraph.

The plan cuts every kv-head group's (unit, key block) work into equal
shares, one resident workgroup each; units cut by share boundaries are
finished by the share holding their last blocks, which folds in the other
shares' fp32 (O, m, l) pieces by the log-sum-exp rule. The `resident`
override makes short batches cut their units into many pieces, and long
ones run many units per share.
"""

from __future__ import annotations

import pytest
import torch

from nimbus_amd import workloads
from nimbus_amd.kernels.prefill_attention import (paged_prefill_attention, plan_stream, stream_error,
                                                  stream_workspace_bytes, new_stream_workspace)
from nimbus_amd import _lib
from tests.gpu_helpers import announce, oracle_prefill
from tests.helpers import assert_within, query_starts, random_tables, scattered_cache

pytestmark = pytest.mark.gpu


def _case(heads, kv, d, seqs, dtype, seed=1):
    ctx_lens = [c for _, c in seqs]
    pool = max(64, sum(-(-c // 16) for c in ctx_lens) + 8)
    k, v = scattered_cache(pool, 16, kv, d, seed=seed, dtype=dtype, device="cuda")
    bt = random_tables(ctx_lens, 16, pool, seed=seed, device="cuda")
    qs = query_starts([ql for ql, _ in seqs])
    g = torch.Generator(device="cuda").manual_seed(seed + 2)
    q = torch.randn(qs[-1], heads, d, generator=g, device="cuda").to(dtype)
    return (q, k, v, torch.tensor(qs, dtype=torch.int32, device="cuda"),
            torch.tensor(ctx_lens, dtype=torch.int32, device="cuda"), bt, d ** -0.5, qs, ctx_lens)


def _flags_clear(ws, plan, heads, kv):
    n = int(_lib.load().nimbus_paged_prefill_stream_flag_bytes(plan.num_shares, heads, kv))
    return bool(ws[:n].eq(0).all())


SEQS = [(1, 1), (64, 64), (65, 65), (3, 700), (130, 1000), (512, 1536), (200, 201), (0, 40)]


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("heads,kv,d", [(32, 8, 128), (32, 4, 64), (32, 4, 128), (8, 8, 64), (12, 4, 64),
                                        (32, 16, 128), (16, 2, 64), (28, 4, 128)])
@pytest.mark.parametrize("resident", [512, 64])
def test_stream_matches_oracle(dtype, heads, kv, d, resident):
    announce(f"prefill stream H={heads} KV={kv} D={d} {dtype} resident={resident}")
    q, k, v, qst, ctxt, bt, scale, qs, ctx = _case(heads, kv, d, SEQS, dtype, seed=4)
    plan = plan_stream(qs, ctx, heads, kv, "cuda", resident=resident)
    ws = new_stream_workspace(stream_workspace_bytes(plan.num_shares, heads, kv, d), "cuda")
    got = paged_prefill_attention(q, k, v, qst, ctxt, bt, scale, qs, ctx, plan, workspace=ws)
    torch.cuda.synchronize()
    assert stream_error(ws, plan.num_shares, heads, kv) == 0 and _flags_clear(ws, plan, heads, kv)
    assert_within(got.cpu(), oracle_prefill(q, k, v, qs, ctx, bt, scale), what="stream vs oracle")


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("seqs", [
    [(64, 8192), (130, 4000), (40, 300)],      # short chunks on long prefixes: units cut over many shares
    [(2048, 2048)],                            # one fresh prompt
    [(5, 40), (0, 17), (64, 64), (0, 30), (3, 3), (0, 1)],  # zero-length sequences between others
])
def test_stream_cut_units_and_whole_prompts(dtype, seqs):
    announce(f"prefill stream {dtype} seqs={seqs}")
    q, k, v, qst, ctxt, bt, scale, qs, ctx = _case(32, 8, 128, seqs, dtype, seed=8)
    plan = plan_stream(qs, ctx, 32, 8, "cuda")
    got = paged_prefill_attention(q, k, v, qst, ctxt, bt, scale, qs, ctx, plan)
    tile = paged_prefill_attention(q, k, v, qst, ctxt, bt, scale, qs, ctx, kernel="tile")
    torch.cuda.synchronize()
    want = oracle_prefill(q, k, v, qs, ctx, bt, scale)
    rows = torch.zeros(qs[-1], dtype=torch.bool)
    for i, (ql, _) in enumerate(seqs):
        rows[qs[i]:qs[i] + ql] = True
    assert_within(got.cpu()[rows], want[rows], what="stream vs oracle")
    assert_within(got.cpu()[rows], tile.cpu()[rows].double(), what="stream vs tile kernel")


def test_stream_plans_of_different_shapes_share_one_workspace():
    """Calls whose plans differ (head shapes, head dims, share counts) one
    after another on one workspace, twice round: each matches the oracle, the
    flags are back at zero and the error word stays zero after every call.
    (Flag areas sized to the plan once let a call's partial slots lie where a
    later plan's flags did, and that later call folded in stale pieces.)"""
    cases = [((32, 8, 128), [(512, 1343), (512, 599), (300, 900), (64, 5000)], torch.bfloat16, 512),
             ((32, 1, 64), [(199, 199), (540, 540)], torch.bfloat16, 512),
             ((32, 2, 64), [(542, 5223), (83, 83), (302, 302), (665, 4735)], torch.float16, 512),
             ((32, 4, 128), [(212, 2633), (629, 6031), (456, 456)], torch.float16, 64)]
    built = []
    for i, ((heads, kv, d), seqs, dtype, resident) in enumerate(cases):
        q, k, v, qst, ctxt, bt, scale, qs, ctx = _case(heads, kv, d, seqs, dtype, seed=30 + i)
        plan = plan_stream(qs, ctx, heads, kv, "cuda", resident=resident)
        built.append((heads, kv, d, plan, (q, k, v, qst, ctxt, bt, scale, qs, ctx),
                      oracle_prefill(q, k, v, qs, ctx, bt, scale)))
    ws = new_stream_workspace(max(stream_workspace_bytes(b[3].num_shares, b[0], b[1], b[2]) for b in built), "cuda")
    for rnd in range(2):
        for heads, kv, d, plan, args, want in built:
            announce(f"prefill stream shared workspace round {rnd} H={heads} KV={kv} D={d} shares={plan.num_shares}")
            got = paged_prefill_attention(*args, plan, workspace=ws)
            torch.cuda.synchronize()
            assert stream_error(ws, plan.num_shares, heads, kv) == 0 and _flags_clear(ws, plan, heads, kv)
            assert_within(got.cpu(), want, what=f"H={heads} KV={kv} D={d} round {rnd}")


@pytest.mark.parametrize("config", ["tinyllama_prefill", "llama3_mixed"])
def test_stream_configs_full(config):
    announce(f"prefill stream config {config}")
    b = workloads.CONFIGS[config]("cuda")
    q, k, v, qst, ctxt, bt, scale, qs, ctx = b.prefill_args()
    plan = plan_stream(qs, ctx, q.shape[1], k.shape[2], "cuda")
    got = paged_prefill_attention(q, k, v, qst, ctxt, bt, scale, qs, ctx, plan)
    assert_within(got.cpu(), oracle_prefill(q, k, v, qs, ctx, bt, scale), what=config)


def test_stream_calls_repeat_bit_for_bit_and_replay_from_a_graph():
    """Three eager calls on one workspace give identical bits (the fix-up
    order is fixed by the plan), the flags are back at zero after each, and
    graph replays (with eager work and synchronisations between them) give
    the eager bits every time."""
    announce("prefill stream repeat + graph replay")
    q, k, v, qst, ctxt, bt, scale, qs, ctx = _case(32, 8, 128, [(512, 1343), (512, 599), (300, 900)],
                                                   torch.bfloat16, seed=11)
    plan = plan_stream(qs, ctx, 32, 8, "cuda")
    ws = new_stream_workspace(stream_workspace_bytes(plan.num_shares, 32, 8, 128), "cuda")
    outs = []
    for _ in range(3):
        outs.append(paged_prefill_attention(q, k, v, qst, ctxt, bt, scale, qs, ctx, plan, workspace=ws))
        torch.cuda.synchronize()
        assert _flags_clear(ws, plan, 32, 8)
    assert all(torch.equal(outs[0], o) for o in outs[1:])
    out = torch.empty_like(q)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        paged_prefill_attention(q, k, v, qst, ctxt, bt, scale, qs, ctx, plan, out=out, workspace=ws)
    for i in range(4):
        out.zero_()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, outs[0]), f"replay {i}"
        assert _flags_clear(ws, plan, 32, 8)
        paged_prefill_attention(q, k, v, qst, ctxt, bt, scale, qs, ctx, plan, workspace=ws)  # eager between
    assert stream_error(ws, plan.num_shares, 32, 8) == 0
    assert_within(outs[0].cpu(), oracle_prefill(q, k, v, qs, ctx, bt, scale), what="vs oracle")
