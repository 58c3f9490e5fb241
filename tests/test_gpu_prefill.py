"""GPU: causal varlen paged prefill matches the oracle within the bar.

Covers the reference's test matrix (tests/test_kernels.py:54-75 of Nimbus:
fresh prompts across 64-query tile edges, cached prefixes, a single token)
plus bf16, D=128, GQA groups 1..8, long chunks over long prefixes, and the
two prefill configurations at full size.
"""

from __future__ import annotations

import pytest
import torch

from nimbus_amd import workloads
from nimbus_amd.kernels.prefill_attention import (PrefillPieces, build_programs, paged_prefill_attention,
                                                  plan_pieces)
from oracle import closed_form
from tests import golden_io
from tests.gpu_helpers import announce, oracle_prefill
from tests.helpers import assert_within, query_starts, random_tables, scattered_cache

pytestmark = pytest.mark.gpu


def _case(heads, kv, d, seqs, dtype, seed=1, pool=None):
    ctx_lens = [c for _, c in seqs]
    pool = pool or max(64, sum(-(-c // 16) for c in ctx_lens) + 8)
    k, v = scattered_cache(pool, 16, kv, d, seed=seed, dtype=dtype, device="cuda")
    bt = random_tables(ctx_lens, 16, pool, seed=seed, device="cuda")
    qs = query_starts([ql for ql, _ in seqs])
    g = torch.Generator(device="cuda").manual_seed(seed + 2)
    q = torch.randn(qs[-1], heads, d, generator=g, device="cuda").to(dtype)
    args = (q, k, v, torch.tensor(qs, dtype=torch.int32, device="cuda"),
            torch.tensor(ctx_lens, dtype=torch.int32, device="cuda"), bt, d ** -0.5, qs, ctx_lens)
    return args


REF_SEQS = [[(5, 5), (64, 64), (130, 130)], [(3, 40), (17, 17), (1, 9), (70, 200)], [(1, 1)]]


@pytest.mark.parametrize("kernel", ["auto", "tile"])  # auto: [(1, 1)] takes the verify form
@pytest.mark.parametrize("heads,kv", [(32, 4), (8, 8)])
@pytest.mark.parametrize("seqs", REF_SEQS)
def test_reference_matrix_fp16_d64(heads, kv, seqs, kernel):
    announce(f"prefill ref-matrix H={heads} KV={kv} seqs={seqs} kernel={kernel}")
    args = _case(heads, kv, 64, seqs, torch.float16, pool=400)
    got = paged_prefill_attention(*args, kernel=kernel)
    q, k, v, _, _, bt, scale, qs, ctx = args
    want = oracle_prefill(q, k, v, qs, ctx, bt, scale)
    assert_within(got.cpu(), want, what="vs oracle (fp32 accumulation)")
    assert_within(got.cpu(), oracle_prefill(q, k, v, qs, ctx, bt, scale, in_dtype=True), what="vs oracle in fp16")
    assert_within(got.cpu(), closed_form.prefill(q.cpu(), k.cpu(), v.cpu(), qs, ctx, bt.cpu(), scale),
                  what="vs float64")


SEQS = [(1, 1), (64, 64), (65, 65), (3, 700), (130, 1000), (512, 1536), (200, 201)]


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("heads,kv,d", [(32, 8, 128), (32, 4, 64), (32, 4, 128), (8, 8, 64), (12, 4, 64),
                                        (32, 16, 128), (16, 2, 64)])
def test_group_sizes_dtypes_and_long_chunks(dtype, heads, kv, d):
    announce(f"prefill H={heads} KV={kv} D={d} {dtype}")
    args = _case(heads, kv, d, SEQS, dtype, seed=4)
    got = paged_prefill_attention(*args)
    q, k, v, _, _, bt, scale, qs, ctx = args
    assert_within(got.cpu(), oracle_prefill(q, k, v, qs, ctx, bt, scale), what="vs oracle")


@pytest.mark.parametrize("kernel", ["auto", "tile"])
def test_zero_length_sequences_inside_a_batch(kernel):
    """Sequences feeding no query (q_len 0, with or without a cached
    context) between others: they get no tile, and the other sequences'
    rows match the oracle (the reference's loop builds no program for them,
    prefill_attention.py:81-90)."""
    announce(f"prefill zero-length sequences kernel={kernel}")
    seqs = [(5, 40), (0, 17), (64, 64), (0, 30), (3, 3), (0, 1)]
    args = _case(32, 8, 128, seqs, torch.bfloat16, seed=6)
    got = paged_prefill_attention(*args, kernel=kernel)
    q, k, v, _, _, bt, scale, qs, ctx = args
    assert got.shape == q.shape
    assert_within(got.cpu(), oracle_prefill(q, k, v, qs, ctx, bt, scale), what="vs oracle")


def test_empty_batches_return_empty():
    """A prefill with no sequences, one whose sequences all feed no query,
    and a decode of zero sequences launch nothing and return empty outputs."""
    from nimbus_amd.kernels.paged_attention import paged_decode_attention

    announce("empty prefill and decode batches")
    k, v = scattered_cache(8, 16, 8, 128, seed=1, dtype=torch.bfloat16, device="cuda")
    q0 = torch.empty(0, 32, 128, dtype=torch.bfloat16, device="cuda")
    none = torch.zeros(0, 1, dtype=torch.int32, device="cuda")
    got = paged_prefill_attention(q0, k, v, torch.zeros(1, dtype=torch.int32, device="cuda"),
                                  torch.zeros(0, dtype=torch.int32, device="cuda"), none, 0.1, [0], [])
    assert got.shape == (0, 32, 128)
    bt = random_tables([20, 9], 16, 8, seed=2, device="cuda")
    got = paged_prefill_attention(q0, k, v, torch.zeros(3, dtype=torch.int32, device="cuda"),
                                  torch.tensor([20, 9], dtype=torch.int32, device="cuda"), bt, 0.1, [0, 0, 0],
                                  [20, 9])
    assert got.shape == (0, 32, 128)
    got = paged_decode_attention(q0, k, v, torch.zeros(0, dtype=torch.int32, device="cuda"), none, 4096, 0.1)
    torch.cuda.synchronize()
    assert got.shape == (0, 32, 128)


def test_prebuilt_programs_and_out_slice():
    announce("prefill programs + out slice")
    seqs = [(70, 90), (5, 5)]
    q, k, v, qst, ctxt, bt, scale, qs, ctx = _case(32, 8, 128, seqs, torch.bfloat16, seed=6)
    progs = build_programs(qs, "cuda")
    flat = torch.full((qs[-1] + 3, 32, 128), 5.0, device="cuda").bfloat16()
    paged_prefill_attention(q, k, v, qst, ctxt, bt, scale, qs, ctx, progs, out=flat[:qs[-1]])
    assert flat[qs[-1]:].eq(5).all()
    assert_within(flat[:qs[-1]].cpu(), oracle_prefill(q, k, v, qs, ctx, bt, scale), what="vs oracle")


@pytest.mark.parametrize("name", golden_io.names("prefill"))
def test_golden_fixture(name):
    announce(f"prefill golden {name}")
    f = golden_io.load(name, device="cuda")
    qs = f["query_start"].tolist()
    got = paged_prefill_attention(f["q"], f["k_cache"], f["v_cache"], f["query_start"], f["context_lens"],
                                  f["block_tables"], f["scale"], qs, f["context_lens"].tolist())
    assert_within(got.cpu(), f["out"], what=name)


@pytest.mark.parametrize("config", ["tinyllama_prefill", "llama3_mixed"])
def test_prefill_configs_full(config):
    announce(f"prefill config {config}")
    b = workloads.CONFIGS[config]("cuda")
    args = b.prefill_args()
    got = paged_prefill_attention(*args)
    q, k, v, _, _, bt, scale, qs, ctx = args
    assert_within(got.cpu(), oracle_prefill(q, k, v, qs, ctx, bt, scale), what=config)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("heads,kv,d,seqs,resident", [
    (32, 8, 128, [(64, 8192), (130, 4000), (40, 300)], 512),                # short chunks on long prefixes
    # a larger chip share per tile (resident) forces cuts on small batches
    (32, 4, 64, [(130, 1000), (64, 64), (3, 700), (200, 201)], 2048),         # mixed batch
    (8, 8, 64, [(70, 2000), (1, 9)], 2048),                                  # MHA, a single-token sequence
    (12, 4, 128, [(100, 3000), (40, 1000)], 2048),                            # G = 3, partial tiles
])
def test_key_range_pieces_match_oracle(dtype, heads, kv, d, seqs, resident):
    """Heavy tiles' key ranges cut into pieces (fp32 partials merged by the
    log-sum-exp rule) give the oracle's output, and the uncut tile kernel's
    within the bar."""
    announce(f"prefill pieces H={heads} KV={kv} D={d} {dtype} seqs={seqs} resident={resident}")
    q, k, v, qst, ctxt, bt, scale, qs, ctx = _case(heads, kv, d, seqs, dtype, seed=8)
    plan = plan_pieces(qs, ctx, heads, kv, "cuda", resident=resident)
    assert plan is not None and plan.num_slots > 0
    got = paged_prefill_attention(q, k, v, qst, ctxt, bt, scale, qs, ctx, plan)
    whole = paged_prefill_attention(q, k, v, qst, ctxt, bt, scale, qs, ctx, kernel="tile")
    torch.cuda.synchronize()
    assert_within(got.cpu(), oracle_prefill(q, k, v, qs, ctx, bt, scale), what="pieces vs oracle")
    assert_within(got.cpu(), whole.cpu().double(), what="pieces vs whole tiles")


def test_pieces_with_an_empty_sub_tile_range():
    """A 64-query tile at context 660 (Llama-3 heads: two 32-position
    sub-tiles): the second sub-tile sees 11 key blocks, the first only 10, so
    the piece [10, end) holds nothing for the first sub-tile, whose rows must
    write m = -inf, l = 0 and weigh nothing in the merge."""
    announce("prefill pieces: empty sub-tile range")
    q, k, v, qst, ctxt, bt, scale, qs, ctx = _case(32, 8, 128, [(64, 660)], torch.bfloat16, seed=9)
    end = 2**31 - 1
    pieces = torch.tensor([[0, 0, 10, end, 2], [0, 0, 4, 10, 1], [0, 0, 0, 4, 0]], dtype=torch.int32, device="cuda")
    merges = torch.tensor([[0, 0, 0, 3]], dtype=torch.int32, device="cuda")
    got = paged_prefill_attention(q, k, v, qst, ctxt, bt, scale, qs, ctx, PrefillPieces(pieces, merges, 3))
    torch.cuda.synchronize()
    assert_within(got.cpu(), oracle_prefill(q, k, v, qs, ctx, bt, scale), what="vs oracle")


@pytest.mark.parametrize("v_scale", [1e-3, 1e-4, 1e-5])
def test_small_magnitude_bf16_v_keeps_relative_accuracy(v_scale):
    """bf16 V of small magnitude. The prefill kernel's P.V product runs in
    fp16: a bf16 V element converts exactly down to 2^-17 (fp16 subnormals
    hold bf16's 8 significant bits that far), and below that loses bits,
    with an absolute error under 2^-24 an element, so an output (a convex
    combination of V rows) is off by less than 2^-24 beyond P's rounding.
    Down to V ~ 1e-4 the output bar scaled to V's magnitude holds
    (|got - ref| <= 2e-3 * v_scale + 1e-2 |ref|, which a relative loss the
    unscaled 2e-3 floor hides would fail); at 1e-5 the documented 2^-24
    floor takes the place of the scaled one."""
    announce(f"prefill bf16 small V scale={v_scale}")
    q, k, v, qs_t, ctx_t, bt, scale, qs, ctx = _case(32, 8, 128, [(512, 1536), (200, 201), (64, 700)],
                                                     torch.bfloat16, seed=3)
    v = (v.float() * v_scale).to(torch.bfloat16)
    got = paged_prefill_attention(q, k, v, qs_t, ctx_t, bt, scale, qs, ctx, kernel="tile")
    want = oracle_prefill(q, k, v, qs, ctx, bt, scale)
    atol = max(2e-3 * v_scale, 2.0 ** -24)
    assert_within(got.cpu(), want, atol=atol, what=f"V scaled by {v_scale}")
