"""GPU: the verify form of prefill attention (nimbus_paged_verify) against
the oracle, the tile kernel and the decode kernel.

The verify form computes nimbus/kernels/prefill_attention.py:93-119 for a
batch in which every sequence has the same q_len <= 16 (the batches
nimbus/spec/engine.py:84-96 builds, q_len = k + 1). The bar is the
prefill bar: within 2e-3 + 1e-2 |ref| of the oracle's fp32-accumulated
attention. Cases: the query run inside one page and across a page edge,
contexts that equal q_len (a fresh short prompt), sequences long enough that
their pages are split between waves (the merge pass), GQA groups 1..8 with
one and two 16-column chunks (two chunks in workgroups of 2, 4, 5, 6 and 8
waves), both dtypes and head dims.
"""

from __future__ import annotations

import pytest
import torch

from nimbus_amd.kernels.paged_attention import paged_decode_attention, paged_verify_attention
from nimbus_amd.kernels.prefill_attention import paged_prefill_attention, verify_queries
from tests.gpu_helpers import announce, oracle_decode, oracle_prefill
from tests.helpers import assert_within, query_starts, random_tables, scattered_cache

pytestmark = pytest.mark.gpu


def _case(heads, kv, d, nq, ctx_lens, dtype, seed=1):
    pool = sum(-(-c // 16) for c in ctx_lens) + 8
    k, v = scattered_cache(pool, 16, kv, d, seed=seed, dtype=dtype, device="cuda")
    bt = random_tables(ctx_lens, 16, pool, seed=seed, device="cuda")
    qs = query_starts([nq] * len(ctx_lens))
    g = torch.Generator(device="cuda").manual_seed(seed + 2)
    q = torch.randn(qs[-1], heads, d, generator=g, device="cuda").to(dtype)
    ctx = torch.tensor(ctx_lens, dtype=torch.int32, device="cuda")
    return q, k, v, qs, ctx, bt


CASES = [
    # heads, kv, d, nq, contexts
    (32, 8, 128, 5, [5, 16, 17, 21, 100, 1000, 4000]),        # Llama-3-8B, k = 4: two 16-column chunks
    (32, 8, 128, 4, [4, 31, 32, 33, 47, 48, 49, 2500]),       # one chunk, runs across page edges
    (32, 4, 64, 4, [4, 19, 300, 3000]),                       # G = 8: 32 columns
    (8, 8, 64, 16, [16, 17, 40, 1500]),                       # MHA, a whole page of queries
    (12, 4, 64, 3, [3, 9, 700, 5000, 6]),                     # G = 3: 9 columns, a ragged chunk
    (16, 2, 128, 2, [2, 18, 33, 8000]),                       # G = 8: 16 columns
    # two chunks with the chip filled, workgroups of 4, 6 and 2 waves holding both chunks of their kv heads,
    # and 5-wave workgroups (10 kv groups), which keep a workgroup per chunk
    (16, 2, 64, 3, [3, 40, 4200, 700]),
    (24, 3, 64, 3, [3, 4000, 90]),
    (8, 1, 128, 3, [17000, 3]),
    (20, 5, 64, 5, [5, 2500, 600]),
]


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("heads,kv,d,nq,ctx_lens", CASES)
def test_verify_matches_oracle_and_tile_kernel(dtype, heads, kv, d, nq, ctx_lens):
    announce(f"verify H={heads} KV={kv} D={d} nq={nq} ctx={ctx_lens} {dtype}")
    q, k, v, qs, ctx, bt = _case(heads, kv, d, nq, ctx_lens, dtype)
    assert verify_queries(qs, heads, kv) == nq  # the prefill call routes these here
    scale = d ** -0.5
    got = paged_verify_attention(q, k, v, ctx, bt, nq, max(ctx_lens), scale)
    routed = paged_prefill_attention(q, k, v, torch.tensor(qs, dtype=torch.int32, device="cuda"), ctx, bt, scale,
                                     qs, ctx_lens)
    tile = paged_prefill_attention(q, k, v, torch.tensor(qs, dtype=torch.int32, device="cuda"), ctx, bt, scale,
                                   qs, ctx_lens, kernel="tile")
    torch.cuda.synchronize()
    want = oracle_prefill(q, k, v, qs, ctx_lens, bt, scale)
    assert_within(got.cpu(), want, what="verify vs oracle")
    assert_within(routed.cpu(), want, what="prefill call (verify form) vs oracle")
    assert_within(tile.cpu(), want, what="tile kernel vs oracle")
    # the routed call bounds contexts by the table width: same kernels, same pieces only if the
    # grid matches, so compare to the bar rather than bit for bit
    assert_within(routed.cpu(), got.cpu().double(), what="routed vs direct")


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_one_query_is_decode_bit_for_bit(dtype):
    """queries_per_seq = 1 runs the decode kernels on the decode grid."""
    announce(f"verify nq=1 vs decode {dtype}")
    ctx_lens = [1, 15, 16, 17, 900, 3000, 64, 5000]
    q, k, v, qs, ctx, bt = _case(32, 8, 128, 1, ctx_lens, dtype, seed=4)
    got = paged_verify_attention(q, k, v, ctx, bt, 1, 5000, 128 ** -0.5)
    dec = paged_decode_attention(q, k, v, ctx, bt, 5000, 128 ** -0.5)
    torch.cuda.synchronize()
    assert torch.equal(got.view(torch.int16), dec.view(torch.int16))
    assert_within(got.cpu(), oracle_decode(q, k, v, ctx_lens, bt, 128 ** -0.5), what="vs oracle")


def test_queries_before_the_first_key_give_zero():
    """A context shorter than queries_per_seq puts the first queries before
    position 0: they see no key and give 0; each later query j sees keys
    0 .. ctx - nq + j, i.e. decode attention over that prefix."""
    announce("verify ctx < nq")
    nq, ctx_lens = 5, [3, 40]
    q, k, v, qs, ctx, bt = _case(32, 8, 128, nq, ctx_lens, torch.bfloat16, seed=9)
    got = paged_verify_attention(q, k, v, ctx, bt, nq, 40, 128 ** -0.5).cpu()
    assert torch.equal(got[:2], torch.zeros_like(got[:2]))
    rows = [2, 3, 4]  # positions 0, 1, 2 of the short sequence
    want = oracle_decode(q[rows], k, v, [1, 2, 3], bt[:1].expand(3, -1), 128 ** -0.5)
    assert_within(got[rows], want, what="short sequence vs decode over its prefix")
    want_long = oracle_prefill(q[nq:], k, v, [0, nq], [40], bt[1:], 128 ** -0.5)
    assert_within(got[nq:], want_long, what="full sequence")


def test_many_sequences_and_strided_output():
    """A wide batch (every wave's slice crosses sequences) written into a
    column slice of a wider output buffer."""
    announce("verify 300 sequences, strided out")
    g = torch.Generator().manual_seed(5)
    ctx_lens = [int(c) for c in torch.randint(5, 600, (300,), generator=g)]
    q, k, v, qs, ctx, bt = _case(32, 8, 64, 5, ctx_lens, torch.float16, seed=6)
    wide = torch.full((q.shape[0], 40, 64), 7.0, dtype=q.dtype, device="cuda")
    out = wide[:, 4:36]
    paged_verify_attention(q, k, v, ctx, bt, 5, 600, 0.125, out=out)
    torch.cuda.synchronize()
    assert_within(out.cpu(), oracle_prefill(q, k, v, qs, ctx_lens, bt, 0.125), what="vs oracle")
    assert torch.all(wide[:, :4] == 7) and torch.all(wide[:, 36:] == 7)
