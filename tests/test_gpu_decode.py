"""GPU: paged decode attention matches the oracle within |d| <= 2e-3 + 1e-2|ref|.

Covers the reference's own test matrix (tests/test_kernels.py:33-51 of
Nimbus: heads/KV (32,4) and (8,8), D=64, fp16, contexts that take the one-
and multi-partition paths), plus what the reference never tested: bf16,
D=128, GQA groups of 1..32, long contexts, the three decode configurations
at full size, split-grid invariance, padding rows and strided q/out.
"""

from __future__ import annotations

import pytest
import torch

from nimbus_amd import workloads
from nimbus_amd.kernels.paged_attention import PAGE, paged_decode_attention
from oracle import closed_form
from tests import golden_io
from tests.gpu_helpers import announce, oracle_decode
from tests.helpers import assert_within, random_tables, scattered_cache

pytestmark = pytest.mark.gpu


def _case(heads, kv, d, ctx_lens, dtype, seed=0, pool=None):
    pool = pool or max(64, sum(-(-c // 16) for c in ctx_lens) + 8)
    k, v = scattered_cache(pool, 16, kv, d, seed=seed, dtype=dtype, device="cuda")
    bt = random_tables(ctx_lens, 16, pool, seed=seed, device="cuda")
    ctx = torch.tensor(ctx_lens, dtype=torch.int32, device="cuda")
    g = torch.Generator(device="cuda").manual_seed(seed + 1)
    q = torch.randn(len(ctx_lens), heads, d, generator=g, device="cuda").to(dtype)
    return q, k, v, ctx, bt, d ** -0.5


REF_CTX = [[1, 17, 64, 100, 255, 300], [1500], [700, 33], list(range(1, 200, 7))]


@pytest.mark.parametrize("heads,kv", [(32, 4), (8, 8)])
@pytest.mark.parametrize("ctx_lens", REF_CTX)
def test_reference_matrix_fp16_d64(heads, kv, ctx_lens):
    announce(f"decode ref-matrix H={heads} KV={kv} ctx={ctx_lens[:6]}")
    q, k, v, ctx, bt, scale = _case(heads, kv, 64, ctx_lens, torch.float16, pool=800)
    got = paged_decode_attention(q, k, v, ctx, bt, max(ctx_lens), scale)
    want = oracle_decode(q, k, v, ctx_lens, bt, scale, batched=True)
    assert_within(got.cpu(), want, what="vs oracle (fp32 accumulation)")
    # fp16, as the reference's own test: the oracle in the input dtype holds too
    assert_within(got.cpu(), oracle_decode(q, k, v, ctx_lens, bt, scale, batched=True, in_dtype=True),
                  what="vs oracle in fp16")
    assert_within(got.cpu(), closed_form.decode(q.cpu(), k.cpu(), v.cpu(), ctx.cpu(), bt.cpu(), scale),
                  what="vs float64")


LONG = [1, 15, 16, 17, 511, 512, 513, 1024, 1025, 4096, 8199]


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("heads,kv,d", [(32, 8, 128), (32, 4, 64), (32, 4, 128), (8, 8, 64), (12, 4, 64),
                                        (32, 2, 128), (32, 1, 64), (16, 1, 128)])
def test_group_sizes_dtypes_and_long_contexts(dtype, heads, kv, d):
    announce(f"decode H={heads} KV={kv} D={d} {dtype}")
    q, k, v, ctx, bt, scale = _case(heads, kv, d, LONG, dtype, seed=3)
    got = paged_decode_attention(q, k, v, ctx, bt, max(LONG), scale)
    want = oracle_decode(q, k, v, LONG, bt, scale)
    assert_within(got.cpu(), want, what="vs oracle")


@pytest.mark.parametrize("heads,kv,d,batch,max_ctx", [
    (32, 32, 64, 48, 3000),   # 32 kv groups: 4 workgroups of 8 waves per slice
    (24, 12, 64, 40, 4000),   # 12 groups: workgroups of 6 waves, 170 slices (a ragged last group of 8)
    (20, 5, 128, 48, 3000),   # 5 groups: workgroups of 5 waves, 409 slices
    (32, 2, 128, 16, 8192),   # 2 groups (G = 16): workgroups of 2 waves, 1024 slices
])
def test_lockstep_workgroup_shapes(heads, kv, d, batch, max_ctx):
    """Batches that fill the chip put the kv groups of a slice in one
    workgroup: every group count (divisors, several workgroups per slice,
    a slice count that is not a multiple of 8) against the oracle."""
    announce(f"decode lockstep H={heads} KV={kv} D={d} B={batch}")
    g = torch.Generator().manual_seed(batch + heads)
    ctx_lens = [int(c) for c in torch.randint(1, max_ctx + 1, (batch,), generator=g)]
    ctx_lens[0] = max_ctx
    q, k, v, ctx, bt, scale = _case(heads, kv, d, ctx_lens, torch.bfloat16, seed=11)
    got = paged_decode_attention(q, k, v, ctx, bt, max_ctx, scale)
    assert_within(got.cpu(), oracle_decode(q, k, v, ctx_lens, bt, scale), what="vs oracle")


@pytest.mark.parametrize("batch", [1, 2, 63, 64, 65, 130])
def test_prefix_in_registers_and_in_lds(batch):
    """Up to 64 sequences the page prefix lives in registers (a lane per
    sequence, a ballot per page); past that, in LDS. Both sides of the
    boundary, with runs of one-page sequences (several sequences in one
    wave's slice) between long ones, against the oracle."""
    announce(f"decode prefix path B={batch}")
    g = torch.Generator().manual_seed(batch)
    ctx_lens = [int(c) for c in torch.randint(1, 1200, (batch,), generator=g)]
    for i in range(0, batch, 3):
        ctx_lens[i] = 1 + i % 17  # one page (up to 17 tokens: two)
    q, k, v, ctx, bt, scale = _case(32, 8, 128, ctx_lens, torch.bfloat16, seed=batch + 1)
    got = paged_decode_attention(q, k, v, ctx, bt, max(ctx_lens), scale)
    assert_within(got.cpu(), oracle_decode(q, k, v, ctx_lens, bt, scale), what="vs oracle")


def test_largest_batch():
    """4096 sequences, the most the page prefix in LDS holds (4097 is refused
    before launch, tests/test_capi.py): short contexts of 1-40 tokens, so most
    slices hold several whole sequences, against the batched oracle."""
    announce("decode B=4096 (largest batch)")
    g = torch.Generator().manual_seed(4096)
    ctx_lens = [int(c) for c in torch.randint(1, 41, (4096,), generator=g)]
    q, k, v, ctx, bt, scale = _case(32, 8, 128, ctx_lens, torch.bfloat16, seed=4096)
    got = paged_decode_attention(q, k, v, ctx, bt, max(ctx_lens), scale)
    assert_within(got.cpu(), oracle_decode(q, k, v, ctx_lens, bt, scale, batched=True), what="vs oracle")


@pytest.mark.parametrize("seed", range(8))
def test_random_decode_batches_match_oracle(seed):
    """Seeded random batches: head shapes with GQA groups of 1-32, D 64 or
    128, both dtypes, 1-300 sequences with log-uniform contexts of 1-12,000
    tokens and a few on page edges, pages scattered over the pool."""
    import numpy as np

    rng = np.random.default_rng(1000 + seed)
    shapes = [(32, 8), (32, 4), (16, 16), (28, 4), (32, 1), (64, 8), (8, 8), (40, 8), (56, 8), (32, 2)]
    heads, kv = shapes[int(rng.integers(len(shapes)))]
    d = int(rng.choice([64, 128]))
    dtype = [torch.float16, torch.bfloat16][seed % 2]
    b = max(1, int(np.exp(rng.uniform(0, np.log(300)))))
    ctx = [max(1, int(np.exp(rng.uniform(0, np.log(12000))))) for _ in range(b)]
    for _ in range(min(b, 4)):
        ctx[int(rng.integers(b))] = max(1, int(16 * rng.integers(1, 200) + rng.integers(-1, 2)))
    announce(f"decode random batch seed={seed} H={heads} KV={kv} D={d} {dtype} B={b} sum_ctx={sum(ctx)}")
    batch = workloads.build_batch([(c, 1) for c in ctx], heads=heads, kv_heads=kv, head_dim=d, dtype=dtype,
                                  device="cuda", seed=seed, fill="used")
    da = batch.decode_args()
    got = paged_decode_attention(*da)
    want = oracle_decode(da[0], batch.k_cache, batch.v_cache, batch.decode_context_host(), da[4], batch.scale)
    assert_within(got.cpu(), want, what="vs oracle")


def test_grid_width_does_not_change_results():
    """A wider grid (larger max_context, as under graph capture) only adds
    partitions that exit at once: results are bit-identical."""
    announce("decode grid invariance")
    ctx_lens = [3, 600, 1500, 2049]
    q, k, v, ctx, bt, scale = _case(32, 8, 128, ctx_lens, torch.bfloat16, seed=5)
    a = paged_decode_attention(q, k, v, ctx, bt, max(ctx_lens), scale)
    b = paged_decode_attention(q, k, v, ctx, bt, 4 * max(ctx_lens) + 3, scale, num_partitions=1)
    assert torch.equal(a, b)


def test_page_boundaries_match_oracle():
    announce("decode page boundaries")
    ctx_lens = [PAGE - 1, PAGE, PAGE + 1, 2 * PAGE, 511, 512, 513, 1024 + PAGE, 1536 + 31]
    q, k, v, ctx, bt, scale = _case(32, 8, 128, ctx_lens, torch.bfloat16, seed=6)
    got = paged_decode_attention(q, k, v, ctx, bt, max(ctx_lens), scale)
    assert_within(got.cpu(), oracle_decode(q, k, v, ctx_lens, bt, scale), what="vs oracle")


def test_strided_q_and_out_slice():
    """q as the slice of a fused qkv projection; out as a slice of a flat batch."""
    announce("decode strided q/out")
    heads, kv, d = 32, 8, 128
    ctx_lens = [77, 1030, 5]
    _, k, v, ctx, bt, scale = _case(heads, kv, d, ctx_lens, torch.bfloat16, seed=7)
    qkv = torch.randn(3, (heads + 2 * kv) * d, device="cuda").bfloat16()
    q = qkv[:, :heads * d].view(3, heads, d)
    flat = torch.full((5, heads, d), 7.0, device="cuda").bfloat16()
    paged_decode_attention(q, k, v, ctx, bt, max(ctx_lens), scale, out=flat[2:])
    assert flat[:2].eq(7).all()
    assert_within(flat[2:].cpu(), oracle_decode(q, k, v, ctx_lens, bt, scale), what="vs oracle")


def test_padding_rows_on_scratch_block():
    """Graph padding rows: ctx=1 on a scratch block (nimbus/cuda_graph.py:133-138)."""
    announce("decode padding rows")
    ctx_lens = [300, 1, 1, 1]
    q, k, v, ctx, bt, scale = _case(32, 8, 128, ctx_lens, torch.bfloat16, seed=8)
    scratch = k.shape[0] - 1
    bt[1:, 0] = scratch
    got = paged_decode_attention(q, k, v, ctx, bt, 4096, scale)
    want = v[scratch, 0].float().repeat_interleave(4, 0)
    for r in (1, 2, 3):
        assert_within(got[r].cpu(), want.cpu().to(got.dtype), what="padding row")
    assert_within(got[:1].cpu(), oracle_decode(q[:1], k, v, [300], bt[:1], scale), what="real row")


def test_stale_table_entries_past_context_are_not_read():
    announce("decode stale tables")
    ctx_lens = [40, 20]
    q, k, v, ctx, bt, scale = _case(8, 2, 64, ctx_lens, torch.float16, seed=9)
    bt2 = torch.cat([bt, torch.full((2, 6), 10 ** 6, dtype=torch.int32, device="cuda")], dim=1)
    bt2[1, 2] = -5
    a = paged_decode_attention(q, k, v, ctx, bt, 40, scale)
    b = paged_decode_attention(q, k, v, ctx, bt2, 40, scale)
    assert torch.equal(a, b)


@pytest.mark.parametrize("name", golden_io.names("decode"))
def test_golden_fixture(name):
    announce(f"decode golden {name}")
    f = golden_io.load(name, device="cuda")
    got = paged_decode_attention(f["q"], f["k_cache"], f["v_cache"], f["context_lens"], f["block_tables"],
                                 int(f["context_lens"].max()), f["scale"])
    assert_within(got.cpu(), f["out"], what=name)


def test_config1_tinyllama_decode_full():
    announce("decode config tinyllama_decode")
    b = workloads.tinyllama_decode("cuda")
    args = b.decode_args()
    got = paged_decode_attention(*args)
    want = oracle_decode(args[0], b.k_cache, b.v_cache, b.decode_context_host(), args[4], b.scale, batched=True)
    assert_within(got.cpu(), want, what="config 1")


def test_config3_llama3_decode_full():
    announce("decode config llama3_decode")
    b = workloads.llama3_decode("cuda")
    args = b.decode_args()
    got = paged_decode_attention(*args)
    want = oracle_decode(args[0], b.k_cache, b.v_cache, b.decode_context_host(), args[4], b.scale)
    assert_within(got.cpu(), want, what="config 3")


def test_config5_long_context_rows():
    """B=256 with 16k-32k rows in a ~40 GB pool: every long row and 64 random
    short rows (plus the first and last rows) against the per-row oracle;
    all rows finite."""
    announce("decode config llama3_long_decode (40 GB pool)")
    import numpy as np

    b = workloads.llama3_long_decode("cuda")
    args = b.decode_args()
    got = paged_decode_attention(*args)
    torch.cuda.synchronize()
    assert torch.isfinite(got.float()).all()
    lens = b.decode_context_host()
    long_rows = [i for i, c in enumerate(lens) if c >= 16384]
    short = [i for i, c in enumerate(lens) if c < 16384]
    picked = np.random.default_rng(5).choice(short, size=64, replace=False).tolist()
    rows = sorted(set(long_rows + picked + [0, len(lens) - 1]))
    assert len(long_rows) >= 10 and len(rows) >= 74
    sel = torch.tensor(rows, device="cuda")
    want = oracle_decode(args[0][sel], b.k_cache, b.v_cache, [lens[i] for i in rows], args[4][sel], b.scale)
    assert_within(got[sel].cpu(), want, what="config 5 rows")
    del b, got
