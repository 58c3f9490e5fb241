"""GPU: page sizes other than 16 and head dims other than 64 and 128.

The reference's Triton kernels take BLOCK_SIZE = k_cache.shape[1] and any
power-of-two head dim (nimbus/kernels/paged_attention.py:139-140,
nimbus/kernels/prefill_attention.py:115); here those shapes run the general
kernel (nimbus_amd/csrc/paged_general.hip) through the same entry points.
Decode, verify and varlen prefill calls are checked against the oracle
(which gathers pages by the cache's own block size) within
2e-3 + 1e-2 |ref|, at pages of 1, 8 and 32 tokens and head dims 32, 80, 96
and 256 (and 128 on 32-token pages), GQA groups 1-32 (at 32 the heads of a
kv head split over several workgroups), both dtypes; contexts
at and around page edges, rows longer than the block table covers cut to
it, and a graph-captured decode call that replays bit for bit; and six
seeded random shapes (head dims 16-256, pages of 1-64 tokens).
"""

from __future__ import annotations

import pytest
import torch

from nimbus_amd.kernels.paged_attention import paged_decode_attention, paged_verify_attention
from nimbus_amd.kernels.prefill_attention import paged_prefill_attention
from tests.gpu_helpers import announce, oracle_decode, oracle_prefill
from tests.helpers import assert_within, query_starts, random_tables, scattered_cache

pytestmark = pytest.mark.gpu

SHAPES = [
    # heads, kv, head dim, block size
    (32, 8, 96, 16),
    (16, 4, 256, 16),
    (8, 8, 32, 32),
    (12, 4, 80, 8),
    (32, 8, 128, 32),
    (4, 1, 64, 1),
    (32, 1, 256, 8),    # G = 32 at D = 256: four workgroups of 8 heads per kv head
    (64, 2, 96, 16),    # G = 32 at D = 96: two chunks, 21 + 11 heads
]


def _cache(kv, d, bs, ctx_lens, dtype, seed):
    pool = sum(-(-c // bs) for c in ctx_lens) + 4
    k, v = scattered_cache(pool, bs, kv, d, seed=seed, dtype=dtype, device="cuda")
    bt = random_tables(ctx_lens, bs, pool, seed=seed, device="cuda")
    return k, v, bt


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("heads,kv,d,bs", SHAPES)
def test_general_decode_matches_oracle(dtype, heads, kv, d, bs):
    ctx_lens = [1, bs, bs + 1, 2 * bs - 1, 700, 3000]
    announce(f"general decode H={heads} KV={kv} D={d} bs={bs} {dtype}")
    k, v, bt = _cache(kv, d, bs, ctx_lens, dtype, seed=d + bs)
    g = torch.Generator(device="cuda").manual_seed(3)
    q = torch.randn(len(ctx_lens), heads, d, generator=g, device="cuda").to(dtype)
    ctx = torch.tensor(ctx_lens, dtype=torch.int32, device="cuda")
    got = paged_decode_attention(q, k, v, ctx, bt, max(ctx_lens), d ** -0.5)
    torch.cuda.synchronize()
    assert_within(got.cpu(), oracle_decode(q, k, v, ctx_lens, bt, d ** -0.5), what="general decode vs oracle")


@pytest.mark.parametrize("heads,kv,d,bs", [(32, 8, 96, 32), (12, 4, 256, 8), (32, 1, 256, 16)])
def test_general_verify_matches_oracle(heads, kv, d, bs):
    nq = 3
    ctx_lens = [3, bs + 2, 900, 2500]
    announce(f"general verify H={heads} KV={kv} D={d} bs={bs} nq={nq}")
    k, v, bt = _cache(kv, d, bs, ctx_lens, torch.bfloat16, seed=11)
    qs = query_starts([nq] * len(ctx_lens))
    g = torch.Generator(device="cuda").manual_seed(4)
    q = torch.randn(qs[-1], heads, d, generator=g, device="cuda").bfloat16()
    ctx = torch.tensor(ctx_lens, dtype=torch.int32, device="cuda")
    got = paged_verify_attention(q, k, v, ctx, bt, nq, max(ctx_lens), d ** -0.5)
    routed = paged_prefill_attention(q, k, v, torch.tensor(qs, dtype=torch.int32, device="cuda"), ctx, bt,
                                     d ** -0.5, qs, ctx_lens)
    tile = paged_prefill_attention(q, k, v, torch.tensor(qs, dtype=torch.int32, device="cuda"), ctx, bt,
                                   d ** -0.5, qs, ctx_lens, kernel="tile")
    torch.cuda.synchronize()
    want = oracle_prefill(q, k, v, qs, ctx_lens, bt, d ** -0.5)
    assert_within(got.cpu(), want, what="general verify vs oracle")
    assert_within(routed.cpu(), want, what="routed prefill call vs oracle")
    assert_within(tile.cpu(), want, what="tile-table prefill vs oracle")


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("heads,kv,d,bs", [(32, 8, 96, 32), (16, 2, 256, 8), (8, 8, 32, 1), (32, 8, 128, 32),
                                         (64, 2, 96, 16)])
def test_general_prefill_matches_oracle(dtype, heads, kv, d, bs):
    """Varlen causal chunks on cached prefixes, the chunks 1-200 tokens (more
    than one 64-position tile), a fresh prompt and a chunk on a long prefix."""
    q_lens = [1, 70, 200, 5, 64]
    prefixes = [0, 33, 500, 1200, 0]
    ctx_lens = [a + b for a, b in zip(q_lens, prefixes)]
    announce(f"general prefill H={heads} KV={kv} D={d} bs={bs} {dtype}")
    k, v, bt = _cache(kv, d, bs, ctx_lens, dtype, seed=5)
    qs = query_starts(q_lens)
    g = torch.Generator(device="cuda").manual_seed(6)
    q = torch.randn(qs[-1], heads, d, generator=g, device="cuda").to(dtype)
    ctx = torch.tensor(ctx_lens, dtype=torch.int32, device="cuda")
    got = paged_prefill_attention(q, k, v, torch.tensor(qs, dtype=torch.int32, device="cuda"), ctx, bt,
                                  d ** -0.5, qs, ctx_lens)
    torch.cuda.synchronize()
    assert_within(got.cpu(), oracle_prefill(q, k, v, qs, ctx_lens, bt, d ** -0.5), what="general prefill vs oracle")


def test_general_decode_cut_to_table_and_graph_replay():
    """max_context and the block table's width bound the keys read (a context
    past them is cut, as in the tuned kernels); a graph-captured call replays
    bit for bit."""
    heads, kv, d, bs = 16, 4, 96, 8
    ctx_lens = [40, 90, 7]
    announce("general decode bounds and graph replay")
    k, v, bt = _cache(kv, d, bs, ctx_lens, torch.bfloat16, seed=9)
    g = torch.Generator(device="cuda").manual_seed(7)
    q = torch.randn(len(ctx_lens), heads, d, generator=g, device="cuda").bfloat16()
    ctx = torch.tensor(ctx_lens, dtype=torch.int32, device="cuda")
    cut = paged_decode_attention(q, k, v, ctx, bt, 48, d ** -0.5)  # max_context 48: the 90-token row sees 48
    want = oracle_decode(q, k, v, [40, 48, 7], bt, d ** -0.5)
    assert_within(cut.cpu(), want, what="cut to max_context")
    out = torch.empty_like(q)
    eager = paged_decode_attention(q, k, v, ctx, bt, 96, d ** -0.5)
    paged_decode_attention(q, k, v, ctx, bt, 96, d ** -0.5, out=out)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        paged_decode_attention(q, k, v, ctx, bt, 96, d ** -0.5, out=out)
    for _ in range(3):
        out.zero_()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, eager)


def test_backend_step_on_32_token_pages():
    """A flat step (prefill chunks then decodes, as runner.prepare lays it
    out) through AttentionBackend.forward on 32-token pages and D = 96: the
    slot write (any page size: a flat slot view) is bit-exact and both
    attention parts match the oracle."""
    from nimbus_amd.model.attention import AttentionBackend, AttnMetadata

    heads, kv, d, bs = 16, 4, 96, 32
    prefills = [(100, 40), (0, 5)]  # (cached prefix, new tokens)
    decodes = [300, 65, 1]           # context lengths, the newest token included
    ctx_all = [p + q for p, q in prefills] + decodes
    announce("general backend step bs=32 D=96")
    k_cache, v_cache, bt = _cache(kv, d, bs, ctx_all, torch.bfloat16, seed=12)
    bt_host = bt.cpu()
    positions, rows = [], []
    for s, (p, q) in enumerate(prefills):
        positions += list(range(p, p + q))
        rows += [s] * q
    for s, c in enumerate(decodes, start=len(prefills)):
        positions.append(c - 1)
        rows.append(s)
    slots = torch.tensor([int(bt_host[r, pos // bs]) * bs + pos % bs for r, pos in zip(rows, positions)],
                         dtype=torch.int64, device="cuda")
    t = len(positions)
    g = torch.Generator(device="cuda").manual_seed(13)
    q = torch.randn(t, heads, d, generator=g, device="cuda").bfloat16()
    k_new = torch.randn(t, kv, d, generator=g, device="cuda").bfloat16()
    v_new = torch.randn(t, kv, d, generator=g, device="cuda").bfloat16()
    qs_host = [0]
    for _, n in prefills:
        qs_host.append(qs_host[-1] + n)
    ctx_pre = [p + n for p, n in prefills]
    n_pre = qs_host[-1]
    meta = AttnMetadata(
        slot_mapping=slots, num_prefill_tokens=n_pre,
        prefill_query_start=torch.tensor(qs_host, dtype=torch.int32, device="cuda"),
        prefill_context_lens=torch.tensor(ctx_pre, dtype=torch.int32, device="cuda"),
        prefill_block_tables=bt[:len(prefills)],
        decode_context_lens=torch.tensor(decodes, dtype=torch.int32, device="cuda"),
        decode_block_tables=bt[len(prefills):], max_decode_context=max(decodes),
        prefill_query_start_host=qs_host, prefill_context_lens_host=ctx_pre)
    k_before = k_cache.clone()
    out = AttentionBackend().forward(q, k_new, v_new, k_cache, v_cache, meta, d ** -0.5)
    torch.cuda.synchronize()
    kref = k_before.view(-1, kv, d)
    kref[slots] = k_new
    assert torch.equal(k_cache.view(-1, kv, d).view(torch.int16), kref.view(torch.int16))
    assert_within(out[:n_pre].cpu(), oracle_prefill(q[:n_pre], k_cache, v_cache, qs_host, ctx_pre,
                                                    bt[:len(prefills)], d ** -0.5), what="prefill part")
    assert_within(out[n_pre:].cpu(), oracle_decode(q[n_pre:], k_cache, v_cache, decodes, bt[len(prefills):],
                                                   d ** -0.5), what="decode part")


@pytest.mark.parametrize("seed", range(6))
def test_general_random_shapes_match_oracle(seed):
    """Seeded random shapes the general kernel takes: head dims 16-256,
    pages of 1-64 tokens, GQA groups 1-32, both dtypes; decode over 1-24
    log-uniform contexts up to 4,000 tokens, and prefill chunks over
    prefixes, against the oracle."""
    import numpy as np

    rng = np.random.default_rng(7000 + seed)
    kv = int(rng.choice([1, 2, 4, 8]))
    heads = kv * int(rng.choice([1, 2, 3, 4, 5, 7, 8, 16, 32]))
    d = int(rng.choice([16, 32, 48, 64, 80, 96, 112, 128, 160, 192, 256]))
    bs = int(rng.choice([1, 2, 4, 8, 16, 32, 64]))
    if bs == 16 and d in (64, 128):
        bs = 32  # (the tuned kernels' shape)
    dtype = [torch.float16, torch.bfloat16][seed % 2]
    n = int(rng.integers(1, 24))
    ctx_lens = [max(1, int(np.exp(rng.uniform(0, np.log(4000))))) for _ in range(n)]
    announce(f"general random seed={seed} H={heads} KV={kv} D={d} bs={bs} {dtype} n={n}")
    k, v, bt = _cache(kv, d, bs, ctx_lens, dtype, seed=seed)
    g = torch.Generator(device="cuda").manual_seed(seed)
    q = torch.randn(n, heads, d, generator=g, device="cuda").to(dtype)
    ctx = torch.tensor(ctx_lens, dtype=torch.int32, device="cuda")
    got = paged_decode_attention(q, k, v, ctx, bt, max(ctx_lens), d ** -0.5)
    assert_within(got.cpu(), oracle_decode(q, k, v, ctx_lens, bt, d ** -0.5), what="general decode vs oracle")
    q_lens = [int(rng.integers(1, 300)) for _ in range(min(n, 6))]
    p_lens = [ql + int(rng.choice([0, int(rng.integers(1, 1500))])) for ql in q_lens]
    k, v, bt = _cache(kv, d, bs, p_lens, dtype, seed=seed + 1)
    qs = query_starts(q_lens)
    qp = torch.randn(qs[-1], heads, d, generator=g, device="cuda").to(dtype)
    got = paged_prefill_attention(qp, k, v, torch.tensor(qs, dtype=torch.int32, device="cuda"),
                                  torch.tensor(p_lens, dtype=torch.int32, device="cuda"), bt, d ** -0.5, qs, p_lens)
    assert_within(got.cpu(), oracle_prefill(qp, k, v, qs, p_lens, bt, d ** -0.5), what="general prefill vs oracle")
