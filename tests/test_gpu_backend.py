"""GPU: the drop-in backend (write -> prefill -> decode on one flat batch),
decode attention replayed from hipGraphs at padded batch sizes, and
speculative verification's prefill attention replayed from hipGraphs."""

from __future__ import annotations

import pytest
import torch

from nimbus_amd import workloads
from nimbus_amd.graphs import DecodeAttentionGraphs, VerifyAttentionGraphs
from nimbus_amd.model.attention import AttentionBackend, AttnMetadata
from tests.gpu_helpers import announce, oracle_decode, oracle_prefill
from tests.helpers import assert_within

pytestmark = pytest.mark.gpu


def _meta(b: workloads.PagedBatch) -> AttnMetadata:
    p = b.num_prefills
    pa = b.prefill_args()
    da = b.decode_args()
    return AttnMetadata(
        slot_mapping=b.slot_mapping, num_prefill_tokens=b.num_prefill_tokens, prefill_query_start=pa[3],
        prefill_context_lens=pa[4], prefill_block_tables=b.block_tables[:p], decode_context_lens=da[3],
        decode_block_tables=da[4], max_decode_context=da[5], prefill_query_start_host=pa[7],
        prefill_context_lens_host=pa[8])


def test_mixed_step_matches_oracle():
    """config 4 layout: 4 prefill chunks of 512 over cached prefixes,
    then 60 decodes, flat and prefill-first; the backend writes the new K/V
    first (write_first=False here so the backend's own write is what counts)."""
    announce("backend mixed step (llama3_mixed)")
    b = workloads.llama3_mixed("cuda")
    # Rebuild with the new tokens NOT yet in the cache.
    b = workloads.build_batch(b.seqs, heads=32, kv_heads=8, head_dim=128, dtype=torch.bfloat16, device="cuda",
                              seed=0, write_first=False)
    k_before = b.k_cache.clone()
    out = AttentionBackend().forward(b.q, b.k, b.v, b.k_cache, b.v_cache, _meta(b), b.scale)
    torch.cuda.synchronize()
    # the slot write is bit-exact
    kref = k_before.view(-1, 8, 128)
    kref[b.slot_mapping] = b.k
    assert torch.equal(b.k_cache.view(-1, 8, 128).view(torch.int16), kref.view(torch.int16))
    p = b.num_prefill_tokens
    q, k, v, _, _, bt, scale, qs, ctx = b.prefill_args()
    assert_within(out[:p].cpu(), oracle_prefill(q, k, v, qs, ctx, bt, scale), what="prefill part")
    da = b.decode_args()
    assert_within(out[p:].cpu(), oracle_decode(da[0], b.k_cache, b.v_cache, b.decode_context_host(), da[4], scale),
                  what="decode part")


def test_config4_step_with_graph_replayed_decode():
    """config 4 as the bench runs it: the slot write of the prefill
    tokens and the prefill (eager), then the 60 decodes (contexts U[256,
    4096]) replayed from DecodeAttentionGraphs padded to 64, whose graph
    writes the decode tokens' K/V itself. Both parts against the oracle, the
    cache bit-exact, and every replay (eager work between them) identical."""
    announce("config 4 step: eager prefill + decode graph padded to 64")
    from nimbus_amd.kernels.cache_ops import write_kv
    from nimbus_amd.kernels.prefill_attention import build_programs, paged_prefill_attention

    ref = workloads.llama3_mixed("cuda")
    b = workloads.build_batch(ref.seqs, heads=32, kv_heads=8, head_dim=128, dtype=torch.bfloat16, device="cuda",
                              seed=0, write_first=False)
    nb = b.k_cache.shape[0]
    kc = torch.cat([b.k_cache, torch.zeros_like(b.k_cache[:1])])  # + the scratch block
    vc = torch.cat([b.v_cache, torch.zeros_like(b.v_cache[:1])])
    k_before = kc[:nb].clone()
    graphs = DecodeAttentionGraphs(kc, vc, num_heads=32, scale=b.scale, max_model_len=8192, max_batch=64,
                                   scratch_block=nb)
    graphs.capture()
    p_tok = b.num_prefill_tokens
    pa, da = b.prefill_args(), b.decode_args()
    assert len(b.decode_context_host()) == 60
    write_kv(b.k[:p_tok], b.v[:p_tok], kc, vc, b.slot_mapping[:p_tok])
    out_p = paged_prefill_attention(pa[0], kc, vc, pa[3], pa[4], pa[5], pa[6], pa[7], pa[8],
                                    build_programs(pa[7], "cuda", pa[8]))
    gb = graphs.load(da[0], b.k[p_tok:], b.v[p_tok:], b.slot_mapping[p_tok:], da[3], da[4])
    assert gb == 64
    replays = []
    for _ in range(3):
        replays.append(graphs.replay(gb)[:60].clone())
        torch.cuda.synchronize()
        _ = (torch.randn(1000, device="cuda") * 2).sum().item()  # eager work between replays
    for r in replays[1:]:
        assert torch.equal(r, replays[0])
    kref = k_before.view(-1, 8, 128)
    kref[b.slot_mapping] = b.k
    assert torch.equal(kc[:nb].view(-1, 8, 128).view(torch.int16), kref.view(torch.int16))
    q, _, _, _, _, bt, scale, qs, ctx = b.prefill_args()
    assert_within(out_p.cpu(), oracle_prefill(q, kc, vc, qs, ctx, bt, scale), what="config 4 prefill part")
    want = oracle_decode(da[0], kc, vc, b.decode_context_host(), da[4], scale)
    assert_within(replays[0].cpu(), want, what="config 4 decode part, graph replay at 64")


def test_eager_chunked_prefill_after_decode_graph_setup():
    """A backend holding a workspace sized for decode alone (DecodeGraphs gives
    a model's backend one sized for its largest batch, here 2 rows up to 8192
    tokens) still runs an eager 64-token chunk over an 8192-token prefix,
    whose key-range plan needs more workspace than that, and matches the
    oracle."""
    announce("eager chunked prefill through a backend with a decode-sized workspace")
    from nimbus_amd.kernels.paged_attention import decode_workspace_bytes, new_decode_workspace
    from nimbus_amd.kernels.prefill_attention import PrefillPieces, pieces_workspace_bytes, plan_pieces

    b = workloads.build_batch([(8192 + 64, 64)], heads=32, kv_heads=8, head_dim=128, dtype=torch.bfloat16,
                              device="cuda", seed=4, write_first=False)
    small = new_decode_workspace(decode_workspace_bytes(2, 32, 128, 8192), "cuda")
    plan = plan_pieces([0, 64], [8256], 32, 8, "cuda")
    assert isinstance(plan, PrefillPieces) and pieces_workspace_bytes(plan.num_slots, 32, 128) > small.numel()
    backend = AttentionBackend(decode_workspace=small)
    out = backend.forward(b.q, b.k, b.v, b.k_cache, b.v_cache, _meta(b), b.scale)
    q, k, v, _, _, bt, scale, qs, ctx = b.prefill_args()
    assert_within(out.cpu(), oracle_prefill(q, k, v, qs, ctx, bt, scale), what="chunk over an 8192 prefix")


@pytest.mark.parametrize("n", [60, 3, 1])
def test_decode_graph_replay_matches_eager(n):
    """Decode attention captured at padded sizes (padding rows on a scratch
    block): every replay, with eager work and synchronisations between
    replays, is bit-identical to the eager call on the same padded inputs,
    and the real rows agree with the eager call on the unpadded batch and
    with the oracle within the output tolerance. (The decode kernel splits
    the batch's chunks evenly over its waves, so padding rows move the split
    points and change the fp32 summation order of the real rows: bitwise
    equality holds only for identical inputs.)"""
    announce(f"graph replay n={n}")
    ctx = workloads.llama3_decode_lens(seed=n, batch=n)
    b = workloads.build_batch([(c, 1) for c in ctx], heads=32, kv_heads=8, head_dim=128, dtype=torch.bfloat16,
                              device="cuda", seed=n, pool_factor=1.3, write_first=False)
    nb = b.k_cache.shape[0]
    # one extra block that no sequence owns absorbs the padding rows
    kc = torch.cat([b.k_cache, torch.zeros_like(b.k_cache[:1])])
    vc = torch.cat([b.v_cache, torch.zeros_like(b.v_cache[:1])])
    graphs = DecodeAttentionGraphs(kc, vc, num_heads=32, scale=b.scale, max_model_len=8192, max_batch=64,
                                   scratch_block=nb)
    graphs.capture()
    da = b.decode_args()
    k_new = torch.randn(n, 8, 128, device="cuda").bfloat16()
    v_new = torch.randn(n, 8, 128, device="cuda").bfloat16()
    # decode writes its token's K/V at position ctx-1 first
    slots = torch.tensor([t[(c - 1) // 16] * 16 + (c - 1) % 16 for t, c in zip(b.tables_host, ctx)],
                         dtype=torch.int64, device="cuda")
    kc_e, vc_e = kc.clone(), vc.clone()
    eager_meta = AttnMetadata(
        slot_mapping=slots, num_prefill_tokens=0,
        prefill_query_start=torch.zeros(1, dtype=torch.int32, device="cuda"),
        prefill_context_lens=torch.zeros(0, dtype=torch.int32, device="cuda"),
        prefill_block_tables=torch.zeros(0, 1, dtype=torch.int32, device="cuda"),
        decode_context_lens=da[3], decode_block_tables=da[4], max_decode_context=da[5],
        prefill_query_start_host=[0], prefill_context_lens_host=[])
    eager = AttentionBackend().forward(da[0], k_new, v_new, kc_e, vc_e, eager_meta, b.scale)
    replays = []
    for rep in range(3):
        replays.append(graphs.run(da[0], k_new, v_new, slots, da[3], da[4]).clone())
        torch.cuda.synchronize()
        _ = (torch.randn(1000, device="cuda") * 2).sum().item()  # eager work between replays
    bp = graphs.padded_size(n)
    padded_meta = graphs.graphs[bp][2]
    kc_p, vc_p = kc.clone(), vc.clone()
    padded = AttentionBackend().forward(graphs.q[:bp], graphs.k[:bp], graphs.v[:bp], kc_p, vc_p, padded_meta,
                                        b.scale)[:n]
    for rep, got in enumerate(replays):
        assert torch.equal(got, padded), f"replay {rep} differs from eager on the padded batch"
        assert_within(got.cpu(), eager.cpu().double(), what=f"replay {rep} vs eager")
    assert torch.equal(kc[:nb], kc_e[:nb]) and torch.equal(vc[:nb], vc_e[:nb])
    want = oracle_decode(da[0], kc_e, vc_e, ctx, da[4], b.scale)
    assert_within(eager.cpu(), want, what="eager vs oracle")
    assert_within(replays[0].cpu(), want, what="replay vs oracle")


@pytest.mark.parametrize("n,q_len,dtype", [(3, 5, torch.bfloat16), (7, 5, torch.bfloat16), (16, 5, torch.bfloat16),
                                           (5, 16, torch.float16)])
def test_verify_graph_replay_matches_eager_and_oracle(n, q_len, dtype):
    """Speculative verification (nimbus/spec/engine.py:60-150): n sequences of
    q_len = k + 1 new tokens on cached contexts, captured once per padded size
    with the precomputed tile table (arange(b), zeros(b)) and placeholder host
    lists. Each replay, with eager work and synchronisations between
    replays, is bit-identical to the eager backend call on the padded batch
    with the graph's metadata (same kernels, same grid), within the bar of
    the eager call on the unpadded batch (the verify form splits pages
    between waves by batch and table width), writes the same cache, and
    matches the oracle. q_len 5 takes the verify form, q_len 16 at G = 8
    the tile kernel."""
    announce(f"verify graph n={n} q_len={q_len} dtype={dtype}")
    g = torch.Generator().manual_seed(n * 100 + q_len)
    ctx = [int(c) for c in torch.randint(q_len + 1, 3000, (n,), generator=g)]
    heads, kv, d = (32, 8, 128) if dtype == torch.bfloat16 else (32, 4, 64)
    b = workloads.build_batch([(c, q_len) for c in ctx], heads=heads, kv_heads=kv, head_dim=d, dtype=dtype,
                              device="cuda", seed=n, pool_factor=1.3, write_first=False)
    nb = b.k_cache.shape[0]
    kc = torch.cat([b.k_cache, torch.zeros_like(b.k_cache[:1])])  # + the scratch block
    vc = torch.cat([b.v_cache, torch.zeros_like(b.v_cache[:1])])
    graphs = VerifyAttentionGraphs(kc, vc, num_heads=heads, scale=b.scale, max_model_len=4096, max_batch=16,
                                   k=q_len - 1, scratch_block=nb)
    graphs.capture()
    pa = b.prefill_args()
    empty = torch.zeros(0, dtype=torch.int32, device="cuda")
    meta = AttnMetadata(
        slot_mapping=b.slot_mapping, num_prefill_tokens=n * q_len, prefill_query_start=pa[3],
        prefill_context_lens=pa[4], prefill_block_tables=b.block_tables, decode_context_lens=empty,
        decode_block_tables=empty.view(0, 1), max_decode_context=0, prefill_query_start_host=pa[7],
        prefill_context_lens_host=pa[8])
    kc_e, vc_e = kc.clone(), vc.clone()
    eager = AttentionBackend().forward(b.q, b.k, b.v, kc_e, vc_e, meta, b.scale)
    replays = []
    for rep in range(3):
        replays.append(graphs.run(b.q, b.k, b.v, b.slot_mapping, pa[4], b.block_tables).clone())
        torch.cuda.synchronize()
        _ = (torch.randn(1000, device="cuda") * 2).sum().item()  # eager work between replays
    bp = graphs.padded_size(n)
    padded_meta = graphs.graphs[bp][2]
    assert padded_meta.prefill_kernel == ("verify" if q_len * heads // kv <= 32 else "tile")
    kc_p, vc_p = kc.clone(), vc.clone()
    rows = bp * q_len
    padded = AttentionBackend(decode_workspace=graphs.backend.decode_workspace).forward(
        graphs.q[:rows], graphs.k[:rows], graphs.v[:rows], kc_p, vc_p, padded_meta, b.scale)[:n * q_len]
    for rep, got in enumerate(replays):
        assert torch.equal(got, padded), f"replay {rep} differs from eager on the padded batch"
        assert_within(got.cpu(), eager.cpu().double(), what=f"replay {rep} vs eager")
    assert torch.equal(kc[:nb], kc_e[:nb]) and torch.equal(vc[:nb], vc_e[:nb])
    want = oracle_prefill(b.q, kc_e, vc_e, pa[7], pa[8], b.block_tables, b.scale)
    assert_within(replays[0].cpu(), want, what="verify replay vs oracle")


@pytest.mark.parametrize("seed", range(12))
def test_random_mixed_batches_match_oracle(seed):
    """Seeded random flat batches through the backend, as runner.prepare lays
    them out: a few prefill chunks (fresh prompts and chunks over cached
    prefixes, lengths crossing tile and page edges) then decodes, over
    random head shapes, head dims and dtypes. The slot write is bit-exact and
    both parts match the oracle."""
    import numpy as np

    rng = np.random.default_rng(100 + seed)
    heads, kv = [(32, 8), (32, 4), (16, 16), (28, 4), (32, 1)][int(rng.integers(0, 5))]
    d = int(rng.choice([64, 128]))
    dtype = [torch.float16, torch.bfloat16][seed % 2]
    seqs = []
    for _ in range(int(rng.integers(1, 5))):
        q_len = int(rng.integers(1, 700))
        prefix = int(rng.choice([0, int(rng.integers(1, 1500))]))
        seqs.append((prefix + q_len, q_len))
    seqs = [s for s in seqs if s[1] > 1 or s[0] == 1] or [(65, 65)]
    seqs += [(int(rng.integers(1, 3000)), 1) for _ in range(int(rng.integers(0, 40)))]
    announce(f"backend random batch seed={seed} H={heads} KV={kv} D={d} {dtype} prefills={sum(q > 1 for _, q in seqs)} "
             f"decodes={sum(q == 1 for _, q in seqs)}")
    b = workloads.build_batch(seqs, heads=heads, kv_heads=kv, head_dim=d, dtype=dtype, device="cuda", seed=seed,
                              write_first=False)
    k_before = b.k_cache.clone()
    out = AttentionBackend().forward(b.q, b.k, b.v, b.k_cache, b.v_cache, _meta(b), b.scale)
    torch.cuda.synchronize()
    kref = k_before.view(-1, kv, d)
    kref[b.slot_mapping] = b.k
    assert torch.equal(b.k_cache.view(-1, kv, d).view(torch.int16), kref.view(torch.int16))
    p = b.num_prefill_tokens
    if p:
        q, k, v, _, _, bt, scale, qs, ctx = b.prefill_args()
        assert_within(out[:p].cpu(), oracle_prefill(q, k, v, qs, ctx, bt, scale), what="prefill part")
    if b.num_prefills < len(seqs):
        da = b.decode_args()
        assert_within(out[p:].cpu(),
                      oracle_decode(da[0], b.k_cache, b.v_cache, b.decode_context_host(), da[4], b.scale),
                      what="decode part")
