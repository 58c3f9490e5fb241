"""CPU: host-side logic of the boundary (tile table, metadata, workloads,
algorithmic work formulas) and the absence of any CPU fallback."""

from __future__ import annotations

import dataclasses
import math
import os

import numpy as np
import pytest
import torch

from nimbus_amd import workloads
from nimbus_amd.kernels import cache_ops, paged_attention, prefill_attention, rmsnorm
from nimbus_amd.model.attention import AttentionBackend, AttnMetadata


def _programs_loop(query_start_host, block_m=64):
    """The reference's build_programs loop (prefill_attention.py:81-90), restated."""
    seqs, starts = [], []
    for i in range(len(query_start_host) - 1):
        q_len = query_start_host[i + 1] - query_start_host[i]
        for m0 in range(0, q_len, block_m):
            seqs.append(i)
            starts.append(m0)
    return seqs, starts


@pytest.mark.parametrize("qs", [[0], [0, 1], [0, 64], [0, 65], [0, 5, 69, 72, 72, 202], [0, 512, 1024, 1600]])
def test_build_programs_matches_reference_loop(qs):
    s, m = prefill_attention.build_programs(qs, "cpu")
    want_s, want_m = _programs_loop(qs)
    assert s.tolist() == want_s and m.tolist() == want_m
    assert s.dtype == m.dtype == torch.int32


@pytest.mark.parametrize("qs,ctx", [([0, 512, 1024, 1536, 2048], [700, 1536, 512, 1000]),
                                    ([0, 5, 69, 72], [5, 100, 3]), ([0, 64], [64]),
                                    ([0] + [512 * (i + 1) for i in range(6)], [2560] * 6),
                                    ([0] + [200 * (i + 1) for i in range(12)], [300 + 50 * i for i in range(12)]),
                                    ([0] + [300 * (i + 1) for i in range(8)], [400 + 90 * i for i in range(8)]),
                                    ([0] + [600 * (i + 1) for i in range(8)], [900 + 90 * i for i in range(8)])])
def test_build_programs_cost_order_keeps_the_entries(qs, ctx):
    """With context lengths the table holds the reference's entries: sequences
    heaviest first, each sequence's tiles adjacent and heaviest first, and,
    for a table short enough to start at once, the second half reversed; a
    table of up to LPT_TILES tiles goes heaviest tile first."""
    s, m = prefill_attention.build_programs(qs, "cpu", ctx)
    got = list(zip(s.tolist(), m.tolist()))
    entries = _programs_loop(qs)
    assert sorted(got) == sorted(zip(*entries))
    lens = [qs[i + 1] - qs[i] for i in range(len(ctx))]
    cost = {(a, b): min(ctx[a], ctx[a] - lens[a] + b + 64) for a, b in zip(*entries)}
    seq_cost = {a: sum(c for (x, _), c in cost.items() if x == a) for a in range(len(ctx))}
    half = (len(got) + 1) // 2
    paired = len(got) <= prefill_attention.PAIRED_TILES
    listed = got[:half] + got[half:][::-1] if paired else got
    if prefill_attention.PAIRED_TILES < len(got) <= prefill_attention.LPT_TILES:
        keys = [(-cost[(a, b)], a, b) for a, b in listed]
        assert keys == sorted(keys)
        return
    keys = [(-seq_cost[a], a, -cost[(a, b)]) for a, b in listed]
    assert keys == sorted(keys)
    # each sequence's tiles stay together in the listed order
    seen = []
    for a, _ in listed:
        if not seen or seen[-1] != a:
            assert a not in seen
            seen.append(a)


def test_attn_metadata_fields_match_reference():
    # nimbus/model/attention.py:24-50, in order
    want = ["slot_mapping", "num_prefill_tokens", "prefill_query_start", "prefill_context_lens",
            "prefill_block_tables", "decode_context_lens", "decode_block_tables", "max_decode_context",
            "prefill_query_start_host", "prefill_context_lens_host", "prefill_programs", "decode_partitions"]
    names = [f.name for f in dataclasses.fields(AttnMetadata)]
    assert names[:len(want)] == want
    assert names[len(want):] == ["prefill_kernel"]  # ours, defaulted, after the reference's fields


@pytest.mark.parametrize("qs,heads,kv,want", [
    ([0, 5, 10, 15], 32, 8, 5),     # k = 4 draft tokens, Llama-3-8B groups: 20 columns
    ([0, 8, 16], 32, 8, 8),         # 32 columns: the limit
    ([0, 9, 18], 32, 8, 0),         # 36 columns: the tile kernel
    ([0, 5, 10, 16], 32, 8, 0),     # ragged
    ([0, 1], 32, 32, 1),            # one token, MHA
    ([0, 17, 34], 8, 8, 0),         # more queries than a page
    ([0], 32, 8, 0),                # no sequences
    ([0, 3, 6, 9], 12, 4, 3),
])
def test_verify_form_takes_uniform_short_runs(qs, heads, kv, want):
    assert prefill_attention.verify_queries(qs, heads, kv) == want


def test_verify_form_batch_limit():
    n = prefill_attention.MAX_VERIFY_SEQUENCES
    assert prefill_attention.verify_queries(list(range(0, 2 * (n + 1), 2)), 32, 8) == 2
    assert prefill_attention.verify_queries(list(range(0, 2 * (n + 2), 2)), 32, 8) == 0


def test_backend_has_no_cpu_path():
    with pytest.raises(ValueError):
        AttentionBackend(False)


def test_kernels_refuse_cpu_tensors():
    k = torch.zeros(4, 16, 2, 64, dtype=torch.float16)
    q = torch.zeros(2, 4, 64, dtype=torch.float16)
    ctx = torch.ones(2, dtype=torch.int32)
    bt = torch.zeros(2, 1, dtype=torch.int32)
    with pytest.raises(ValueError, match="GPU"):
        paged_attention.paged_decode_attention(q, k, k, ctx, bt, 1, 0.125)
    with pytest.raises(ValueError, match="GPU"):
        prefill_attention.paged_prefill_attention(q, k, k, torch.tensor([0, 2], dtype=torch.int32), ctx[:1],
                                                  bt[:1], 0.125, [0, 2], [2])
    with pytest.raises(ValueError, match="GPU"):
        cache_ops.write_kv(q[:, :2], q[:, :2], k, k, torch.zeros(2, dtype=torch.int64))
    x = torch.zeros(3, 64, dtype=torch.float16)
    with pytest.raises(ValueError, match="GPU"):
        rmsnorm.add_rms_norm(x, x, torch.ones(64, dtype=torch.float16), 1e-5)


def test_rms_norm_wrapper_checks_shapes():
    # any row length is taken (60 is not a multiple of 8: the general kernel); CPU tensors are refused
    with pytest.raises(ValueError, match="GPU only"):
        rmsnorm.rms_norm(torch.zeros(3, 60, dtype=torch.float16), torch.ones(60, dtype=torch.float16), 1e-5)
    with pytest.raises(NotImplementedError):
        rmsnorm.rms_norm(torch.zeros(2, 64), torch.ones(64), 1e-5)  # float32
    with pytest.raises(ValueError):
        rmsnorm.rms_norm(torch.zeros(2, 64, dtype=torch.float16), torch.ones(32, dtype=torch.float16), 1e-5)


def test_batch_layout_follows_runner():
    b = workloads.build_batch([(40, 40), (70, 30), (100, 1), (17, 1)], heads=4, kv_heads=2, head_dim=64,
                              dtype=torch.float16, device="cpu", seed=3)
    assert b.num_prefills == 2 and b.num_prefill_tokens == 70
    # slot formula nimbus/runner.py:61
    slots = []
    for (c, ql), t in zip(b.seqs, b.tables_host):
        slots += [t[p // 16] * 16 + p % 16 for p in range(c - ql, c)]
    assert b.slot_mapping.tolist() == slots
    # zero-padded tables (runner.py:24-30)
    assert b.block_tables.shape == (4, 7)
    assert b.block_tables[3, 2:].eq(0).all()
    # the new tokens are in the cache (write first)
    kc = b.k_cache.view(-1, 2, 64)
    assert torch.equal(kc[b.slot_mapping], b.k)
    pa = b.prefill_args()
    assert pa[7] == [0, 40, 70] and pa[8] == [40, 70]
    da = b.decode_args()
    assert da[5] == 100 and da[0].shape == (2, 4, 64)


def test_flat_step_follows_runner_layout():
    """flat_step against the layout contract written out token by token
    (nimbus/runner.py:33-96): fed tokens back to back, prefills first, slot
    = table[p // 16] * 16 + p % 16, per-group zero-padded tables, host lists,
    and the rows sampled (sequences whose pending tokens the step finishes)."""
    rng = np.random.default_rng(7)
    fresh = workloads.SeqState(list(rng.integers(0, 99, 23)), [5, 9])
    chunk = workloads.SeqState(list(rng.integers(0, 99, 70)), [1, 2, 3, 4, 8], num_computed=32)
    dec_a = workloads.SeqState(list(rng.integers(0, 99, 18)), [7, 6], num_computed=17)
    dec_b = workloads.SeqState(list(rng.integers(0, 99, 3)), [11], num_computed=2)
    entries = [(fresh, 23), (chunk, 20), (dec_a, 1), (dec_b, 1)]
    st = workloads.flat_step(entries, "cpu")
    ids, pos, slots, sample = [], [], [], []
    for s, n in entries:
        for p in range(s.num_computed, s.num_computed + n):
            ids.append(s.token_ids[p])
            pos.append(p)
            slots.append(s.block_table[p // 16] * 16 + p % 16)
        if s.num_computed + n == len(s):
            sample.append(len(ids) - 1)
    assert st.input_ids.tolist() == ids and st.positions.tolist() == pos
    m = st.meta
    assert m.slot_mapping.tolist() == slots and m.slot_mapping.dtype == torch.int64
    assert st.sample_rows.tolist() == sample  # the chunk (52 of 70 done) is not sampled
    assert m.num_prefill_tokens == 43 and m.prefill_query_start_host == [0, 23, 43]
    assert m.prefill_context_lens_host == [23, 52] and m.prefill_context_lens.tolist() == [23, 52]
    assert m.prefill_block_tables.tolist() == [[5, 9, 0, 0, 0], [1, 2, 3, 4, 8]]
    assert m.decode_context_lens.tolist() == [18, 3] and m.max_decode_context == 18
    assert m.decode_block_tables.tolist() == [[7, 6], [11, 0]]
    assert m.decode_block_tables.dtype == torch.int32 and m.num_decodes == 2 and m.num_prefills == 2
    with pytest.raises(ValueError):
        workloads.flat_step([(dec_a, 1), (fresh, 23)], "cpu")  # a decode before a prefill
    with pytest.raises(ValueError):
        workloads.flat_step([(workloads.SeqState([1] * 40, [3]), 40)], "cpu")  # 40 tokens on one page
    with pytest.raises(ValueError):
        workloads.flat_step([(dec_b, 2)], "cpu")  # more tokens than pending


def test_flat_step_matches_build_batch():
    """The two generators of the runner's layout agree: a prefill chunk over
    a prefix and decodes, with build_batch's tables."""
    b = workloads.build_batch([(40, 40), (70, 30), (100, 1), (17, 1)], heads=4, kv_heads=2, head_dim=64,
                              dtype=torch.float16, device="cpu", seed=3)
    entries = [(workloads.SeqState(list(range(c)), t, c - ql), ql) for (c, ql), t in zip(b.seqs, b.tables_host)]
    st = workloads.flat_step(entries, "cpu")
    assert torch.equal(st.meta.slot_mapping, b.slot_mapping)
    pa, da = b.prefill_args(), b.decode_args()
    assert st.meta.prefill_query_start_host == pa[7] and st.meta.prefill_context_lens_host == pa[8]
    assert torch.equal(st.meta.decode_context_lens, da[3])
    assert st.meta.max_decode_context == da[5]


def test_weight_bytes_counts_each_storage_once():
    from torch import nn

    from nimbus_amd.quant import weight_bytes

    emb = nn.Embedding(10, 4)
    head = nn.Linear(4, 10, bias=False)
    head.weight = emb.weight  # tied
    model = nn.Sequential(emb, nn.Linear(4, 6, bias=False), head)
    model.register_buffer("table", torch.zeros(3, dtype=torch.float16))
    assert weight_bytes(model) == 10 * 4 * 4 + 6 * 4 * 4 + 3 * 2


def test_pages_are_distinct():
    b = workloads.tinyllama_decode("cpu")
    pages = [p for t in b.tables_host for p in t]
    assert len(pages) == len(set(pages)) and max(pages) < 1100


def test_config_generators_shapes():
    assert len(workloads.llama3_decode_lens()) == 64
    lens = workloads.llama3_decode_lens()
    assert min(lens) >= 128 and max(lens) <= 8192
    long_ = workloads.llama3_long_lens()
    assert len(long_) == 256 and max(long_) <= 32768
    assert sum(c >= 16384 for c in long_) >= 10


def test_decode_bytes_formula():
    # sum ctx * 2 * KV * D * 2 + 2 * B * H * D * 2 + 4 * sum pages + 4 * B
    assert workloads.decode_bytes([512], 32, 4, 64) == 512 * 2 * 4 * 64 * 2 + 2 * 32 * 64 * 2 + 4 * 32 + 4
    assert workloads.decode_bytes([1, 17], 32, 8, 128) == 18 * 4096 + 2 * 2 * 32 * 128 * 2 + 4 * 3 + 8


def test_prefill_flops_formula():
    # fresh prompt of n: 4*D*H*n(n+1)/2
    assert workloads.prefill_flops([(512, 512)], 32, 64) == 4 * 64 * 32 * 512 * 513 // 2
    # 3 new on a prefix of 37: 3*37 + 3*4/2 pairs
    assert workloads.prefill_flops([(40, 3)], 1, 1) == 4 * (3 * 37 + 6)
    assert math.isclose(workloads.prefill_flops([(40, 3)], 2, 2), 4 * 4 * 117)


def test_int8_matmul_wrapper_checks():
    from nimbus_amd.kernels.int8_matmul import int8_matmul
    from nimbus_amd.quant import Int8Linear

    x = torch.zeros(2, 64, dtype=torch.float16)
    q = torch.zeros(32, 64, dtype=torch.int8)
    s = torch.ones(32, dtype=torch.float16)
    with pytest.raises(ValueError):  # CPU tensors: no CPU path
        int8_matmul(x, q, s)
    with pytest.raises(ValueError):
        int8_matmul(x, q.float(), s)
    with pytest.raises(ValueError):
        int8_matmul(x[:, :32], q, s)
    with pytest.raises(ValueError):
        int8_matmul(x, q, s.bfloat16())
    with pytest.raises(NotImplementedError):
        int8_matmul(x.float(), q, s.float())
    with pytest.raises(ValueError):
        Int8Linear(torch.nn.Linear(64, 32, bias=False), use_hip=False)


def test_plan_pieces_covers_every_block_once():
    """Short chunks over long prefixes (6 tiles, Llama-3 heads): heavy tiles
    are cut into near-equal ranges that tile their key blocks exactly, slots
    are consecutive per tile, light tiles stay whole."""
    from nimbus_amd.kernels.prefill_attention import KEY_BLOCK, plan_pieces

    lens, prefix = [130, 64, 40], [4000, 8000, 300]  # few tiles over long prefixes: the chip is underfilled
    qs = [0]
    for n in lens:
        qs.append(qs[-1] + n)
    ctx = [p + n for p, n in zip(prefix, lens)]
    plan = plan_pieces(qs, ctx, 32, 8, "cpu")
    assert plan is not None
    pieces, merges = plan.pieces.numpy(), plan.merges.numpy()
    for seq, m0 in {(int(r[0]), int(r[1])) for r in pieces}:
        rows = sorted((int(r[2]), int(r[3]), int(r[4])) for r in pieces if r[0] == seq and r[1] == m0)
        blocks = -(-min(ctx[seq], ctx[seq] - lens[seq] + m0 + 64) // KEY_BLOCK)
        if len(rows) == 1:
            assert rows[0][2] == -1 and rows[0][0] == 0
            continue
        assert rows[0][0] == 0 and rows[-1][1] == blocks
        assert all(a[1] == b[0] for a, b in zip(rows, rows[1:]))
        slots = [r[2] for r in rows]
        assert slots == list(range(slots[0], slots[0] + len(rows)))
        assert [seq, m0, slots[0], len(rows)] in merges.tolist()
    assert plan.num_slots == sum(int(m[3]) for m in merges) > 0


def test_plan_pieces_declines_when_tiles_fill_the_chip():
    from nimbus_amd.kernels.prefill_attention import plan_pieces

    qs = list(range(0, 64 * 2048 + 1, 2048))  # 64 sequences x 32 tiles: far more than the chip holds at once
    assert plan_pieces(qs, [4096] * 64, 32, 8, "cpu") is None
    qs4 = [0, 512, 1024, 1536, 2048]  # config 4: 32 tiles fill the chip, two per CU
    assert plan_pieces(qs4, [1512, 529, 1152, 1536], 32, 8, "cpu") is None
    assert plan_pieces([0, 64], [64], 32, 8, "cpu") is None  # one short tile: nothing to cut


def test_index_checks_raise_like_the_reference():
    """The opt-in checks raise IndexError where the reference's index_copy_
    and table gathers would fail, and pass padding past a row's context."""
    from nimbus_amd.kernels import index_checks

    index_checks.check_slots(torch.tensor([0, 5, 63]), 64)
    with pytest.raises(IndexError):
        index_checks.check_slots(torch.tensor([0, 64]), 64)
    with pytest.raises(IndexError):
        index_checks.check_slots(torch.tensor([-1]), 64)
    bt = torch.tensor([[3, 1, 999], [2, 0, 0]], dtype=torch.int32)  # 999: padding past row 0's 2 pages
    index_checks.check_tables(bt, torch.tensor([20, 16], dtype=torch.int32), 4, 16)
    with pytest.raises(IndexError):  # row 0 now reads its third page, id 999
        index_checks.check_tables(bt, torch.tensor([40, 16], dtype=torch.int32), 4, 16)
    with pytest.raises(IndexError):  # 4 pages needed, table 3 wide
        index_checks.check_tables(bt, torch.tensor([20, 49], dtype=torch.int32), 4, 16)
    with pytest.raises(IndexError):
        index_checks.check_tables(torch.tensor([[-2]], dtype=torch.int32), torch.tensor([1], dtype=torch.int32),
                                  4, 16)
    assert not index_checks.enabled() or os.environ.get("NIMBUS_CHECK_INDICES")


def _bare_loader(cls, max_batch=8, width=4, q_len=None):
    """A graph set's host-side loader state alone (plain host buffers, no
    capture): enough to run _load's checks, which come before any copy."""
    from nimbus_amd import graphs

    g = object.__new__(getattr(graphs, cls))
    g.block_size, g.max_batch, g.scratch_block = 16, max_batch, 99
    g.scratch_slot = 99 * 16
    g.sizes = [1, 2, 4, 8]
    g._staged = None
    rows = 4 if q_len is None else 3
    g._host = torch.zeros((rows, max_batch * (q_len or 1)), dtype=torch.int64)
    g._host_tables = torch.zeros((max_batch, width), dtype=torch.int32)
    if q_len is not None:
        g.q_len = q_len
        g._host_ctx = torch.zeros(max_batch, dtype=torch.int32)
    return g


def test_decode_graph_loader_refuses_a_short_block_table():
    # Position 32 needs a third block; the table holds two. The zero padding past
    # it must not become block 0 (nimbus/cuda_graph.py:118-135 raises IndexError).
    g = _bare_loader("DecodeGraphs")
    seqs = [workloads.SeqState(list(range(10)), [5], 9), workloads.SeqState(list(range(33)), [3, 4], 32)]
    with pytest.raises(IndexError, match="sequence 1"):
        g._load(seqs)


def test_verify_graph_loader_refuses_a_short_block_table():
    # The last of 5 fed tokens of sequence 1 sits at position 16: a second block is needed.
    g = _bare_loader("VerifyGraphs", q_len=5)
    seqs = [workloads.SeqState(list(range(9)), [1]), workloads.SeqState(list(range(17)), [2])]
    with pytest.raises(IndexError, match="sequence 1"):
        g._load(seqs, 2)


def _stream_case(lens, prefix):
    qs = [0]
    for n in lens:
        qs.append(qs[-1] + n)
    return qs, [p + n for p, n in zip(prefix, lens)]


@pytest.mark.parametrize("lens,prefix,heads,kv", [
    ([512] * 4, [831, 87, 183, 242], 32, 8),   # config 4's prefill part (its seed's prefixes)
    ([300, 17, 64, 0, 1, 900], [0, 5000, 64, 12, 0, 33], 32, 8),
    ([8192], [0], 32, 8),                       # one long prompt: many units per share
    ([130, 64, 40], [4000, 8000, 300], 32, 8),  # few heavy units: units cut across many shares
    ([100, 250, 33], [10, 0, 700], 32, 4),      # TinyLlama heads (GS 8)
    ([70, 9], [0, 3], 28, 4),                   # GQA 7: GS 1, 64-position units
    ([1], [0], 32, 32),                         # MHA, a single query
])
def test_stream_plan_covers_every_block_once(lens, prefix, heads, kv):
    """Every unit's key blocks are covered exactly once by its pieces; a cut
    unit is finished by the share holding its last blocks, which folds in
    exactly the lower shares that wrote its other pieces (each into its own
    share's slot, at most one per share); each share runs its pieces
    last-first; shares are balanced to a block and fit the resident
    workgroups."""
    from nimbus_amd.kernels.prefill_attention import plan_stream, stream_units

    qs, ctx = _stream_case(lens, prefix)
    resident = 512
    plan = plan_stream(qs, ctx, heads, kv, "cpu", resident=resident)
    useq, um0, nb, kvg = stream_units(qs, ctx, heads, kv)
    assert plan.num_shares * kvg <= resident
    start, rec = plan.share_start.numpy(), plan.pieces.numpy()
    assert start[0] == 0 and start[-1] == len(rec) and np.all(np.diff(start) >= 0)
    share_of = np.repeat(np.arange(plan.num_shares), np.diff(start))
    unit_index = {(int(s), int(m)): i for i, (s, m) in enumerate(zip(useq, um0))}
    pieces_of = {}
    loads = np.zeros(plan.num_shares, dtype=np.int64)
    for j, r in zip(share_of, rec):
        u = unit_index[(int(r[0]), int(r[1]))]
        hi = min(int(r[3]), int(nb[u]))
        pieces_of.setdefault(u, []).append((int(r[2]), hi, int(r[4]), int(r[5]), int(r[6]), int(j)))
        loads[j] += max(hi - int(r[2]), 0) + (1 if nb[u] == 0 else 0)
    assert sorted(pieces_of) == list(range(len(useq)))
    for u, ps in pieces_of.items():
        ps.sort()
        assert ps[0][0] == 0 and ps[-1][1] == nb[u]
        assert all(a[1] == b[0] for a, b in zip(ps, ps[1:]))
        finishers = [p for p in ps if p[2] == -1]
        assert len(finishers) == 1
        fin = finishers[0]
        contributors = sorted(p[5] for p in ps if p[2] != -1)
        assert all(p[2] == p[5] for p in ps if p[2] != -1)  # a contributor writes its own share's slot
        if contributors:
            assert fin[5] > contributors[-1] and (fin[3], fin[4]) == (contributors[0], fin[5])
            assert contributors == list(range(contributors[0], fin[5]))
        else:
            assert (fin[3], fin[4]) == (0, 0)
    for j in range(plan.num_shares):
        rows = rec[start[j]:start[j + 1]]
        assert sum(1 for r in rows if r[4] != -1) <= 1
        order = [unit_index[(int(r[0]), int(r[1]))] for r in rows]
        assert order == sorted(order, reverse=True)  # last piece first
    total = int(np.maximum(nb, 1).sum())
    assert loads.sum() == total and loads.max() - loads.min() <= 1


def test_stream_plan_of_an_empty_batch_is_none():
    from nimbus_amd.kernels.prefill_attention import plan_stream

    assert plan_stream([0], [], 32, 8, "cpu") is None
    assert plan_stream([0, 0, 0], [5, 9], 32, 8, "cpu") is None
