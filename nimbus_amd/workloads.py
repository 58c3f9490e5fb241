"""Seeded synthetic inputs for the paged-attention path.

Builds paged K/V pools, block tables, context lengths and slot mappings in
the layout Nimbus's runner produces (nimbus/runner.py:33-96): caches are
[num_blocks, 16, KV, D]; token p of a sequence lives in slot
table[p // 16] * 16 + p % 16 (runner.py:61); tables are zero-padded to the
widest row (runner.py:24-30); a flat batch is ordered prefill-first.

The five named configurations are the ones the benchmark and the parity tests
use, numbered 1-5 as comments elsewhere refer to them ("config 3"), values
N(0,1) unless stated, scale 1/sqrt(D):

  1 tinyllama_decode     B=16, H=32, KV=4, D=64, fp16, ctx U[16,1024], tables
                         consecutive slices of a permutation of a 1,100 pool
  2 tinyllama_prefill    8 seqs, new q_len U[32,512] on prefix U[0,256],
                         H=32, KV=4, D=64, fp16
  3 llama3_decode        B=64, H=32, KV=8, D=128, bf16, ctx log-U[128,8192],
                         K/V 0.5*N(0,1), pool 1.2x the pages needed (the
                         benchmark's headline)
  4 llama3_mixed         4 prefill chunks of 512 on prefix U[0,1024], then 60
                         decodes with ctx U[256,4096], bf16
  5 llama3_long_decode   B=256, 90% ctx U[512,4096], 10% U[16384,32768], pool
                         of ~40 GB K+V, tables random pages from it
"""

from __future__ import annotations

import math
from dataclasses import dataclass, field

import numpy as np
import torch

BLOCK_SIZE = 16


@dataclass
class PagedBatch:
    """One flat batch: `seqs[i] = (ctx, q_len)`; q_len == 1 rows after the
    prefills are decodes. All tensors live on `device`."""

    q: torch.Tensor  # [T, H, D]
    k: torch.Tensor  # [T, KV, D] new keys (already written unless write_first=False)
    v: torch.Tensor
    k_cache: torch.Tensor  # [NB, 16, KV, D]
    v_cache: torch.Tensor
    slot_mapping: torch.Tensor  # [T] int64
    block_tables: torch.Tensor  # [S, W] int32 (all sequences)
    context_lens: torch.Tensor  # [S] int32
    seqs: list  # [(ctx, q_len)]
    tables_host: list  # per sequence page lists
    scale: float
    num_prefills: int
    extra: dict = field(default_factory=dict)

    # ---- views in the reference's argument order ----
    @property
    def num_prefill_tokens(self) -> int:
        return sum(q for _, q in self.seqs[: self.num_prefills])

    def prefill_args(self):
        """(q, k_cache, v_cache, query_start, context_lens, block_tables, scale,
        query_start_host, context_lens_host) for paged_prefill_attention."""
        p = self.num_prefills
        qs = [0]
        for _, ql in self.seqs[:p]:
            qs.append(qs[-1] + ql)
        ctx = [c for c, _ in self.seqs[:p]]
        dev = self.q.device
        return (self.q[: qs[-1]], self.k_cache, self.v_cache,
                torch.tensor(qs, dtype=torch.int32, device=dev),
                torch.tensor(ctx, dtype=torch.int32, device=dev),
                self.block_tables[:p], self.scale, qs, ctx)

    def decode_args(self):
        """(q, k_cache, v_cache, context_lens, block_tables, max_context, scale)
        for paged_decode_attention."""
        p = self.num_prefills
        t0 = self.num_prefill_tokens
        ctx = [c for c, _ in self.seqs[p:]]
        return (self.q[t0:], self.k_cache, self.v_cache, self.context_lens[p:],
                self.block_tables[p:], max(ctx, default=0), self.scale)

    def decode_context_host(self):
        return [c for c, _ in self.seqs[self.num_prefills:]]


def _pages(ctx: int) -> int:
    return -(-ctx // BLOCK_SIZE)


def build_batch(seqs, *, heads: int, kv_heads: int, head_dim: int, dtype, device, seed: int,
                pool_blocks: int | None = None, pool_factor: float = 1.2, kv_scale: float = 1.0,
                contiguous_slices: bool = False, write_first: bool = True,
                fill: str = "pool") -> PagedBatch:
    """seqs: list of (ctx, q_len). The first rows with q_len > 1 (or
    q_len == ctx) are prefills; rows after them must be decodes (q_len == 1).

    Pages come from a seeded permutation of the pool: consecutive slices of it
    (contiguous_slices, as tests/test_kernels.py:18-30 of the reference) or a
    sample without replacement spread across the whole pool. Cached prefix
    tokens are random; the new tokens' K/V are written through slot_mapping
    when write_first is set (the order of model/attention.py:78).

    fill="pool" fills the whole pool with N(0,1)*kv_scale; fill="used" fills
    only the pages the tables reference (the rest stays uninitialised), for
    pools too big to fill cheaply.
    """
    rng = np.random.default_rng(seed)
    need = sum(_pages(c) for c, _ in seqs)
    nb = pool_blocks if pool_blocks is not None else max(need, int(math.ceil(pool_factor * need)))
    if nb < need:
        raise ValueError(f"pool of {nb} blocks cannot hold {need} pages")
    if contiguous_slices:
        perm = rng.permutation(nb)[:need]
    else:
        perm = rng.choice(nb, size=need, replace=False)
    tables, i = [], 0
    for c, _ in seqs:
        n = _pages(c)
        tables.append([int(x) for x in perm[i:i + n]])
        i += n
    width = max((len(t) for t in tables), default=1) or 1
    bt = np.zeros((len(seqs), width), dtype=np.int32)
    for r, t in enumerate(tables):
        bt[r, :len(t)] = t

    num_prefills = 0
    for c, ql in seqs:
        if ql == 1 and c > 1:
            break
        num_prefills += 1
    for c, ql in seqs[num_prefills:]:
        if ql != 1:
            raise ValueError("prefill sequences must come before decodes")

    gen = torch.Generator(device=device).manual_seed(seed)
    shape = (nb, BLOCK_SIZE, kv_heads, head_dim)
    if fill == "pool":
        k_cache = (torch.randn(shape, generator=gen, device=device, dtype=torch.float32) * kv_scale).to(dtype) \
            if nb * BLOCK_SIZE * kv_heads * head_dim < (1 << 28) else _randn_big(shape, gen, device, dtype, kv_scale)
        v_cache = (torch.randn(shape, generator=gen, device=device, dtype=torch.float32) * kv_scale).to(dtype) \
            if nb * BLOCK_SIZE * kv_heads * head_dim < (1 << 28) else _randn_big(shape, gen, device, dtype, kv_scale)
    elif fill == "used":
        k_cache = torch.empty(shape, device=device, dtype=dtype)
        v_cache = torch.empty(shape, device=device, dtype=dtype)
        used = torch.as_tensor(perm.astype(np.int64), device=device)
        for cache in (k_cache, v_cache):
            for s in range(0, need, 8192):
                idx = used[s:s + 8192]
                vals = torch.randn((idx.numel(),) + shape[1:], generator=gen, device=device,
                                   dtype=torch.float32) * kv_scale
                cache.index_copy_(0, idx, vals.to(dtype))
    else:
        raise ValueError(fill)

    total_q = sum(ql for _, ql in seqs)
    q = torch.randn((total_q, heads, head_dim), generator=gen, device=device, dtype=torch.float32).to(dtype)
    k = (torch.randn((total_q, kv_heads, head_dim), generator=gen, device=device, dtype=torch.float32)
         * kv_scale).to(dtype)
    v = (torch.randn((total_q, kv_heads, head_dim), generator=gen, device=device, dtype=torch.float32)
         * kv_scale).to(dtype)
    slots = []
    for (c, ql), t in zip(seqs, tables):
        slots.extend(t[p // BLOCK_SIZE] * BLOCK_SIZE + p % BLOCK_SIZE for p in range(c - ql, c))
    slot_mapping = torch.tensor(slots, dtype=torch.int64, device=device)
    if write_first and total_q:
        kv_ = k_cache.view(-1, kv_heads, head_dim)
        kv_.index_copy_(0, slot_mapping, k)
        v_cache.view(-1, kv_heads, head_dim).index_copy_(0, slot_mapping, v)
    return PagedBatch(
        q=q, k=k, v=v, k_cache=k_cache, v_cache=v_cache, slot_mapping=slot_mapping,
        block_tables=torch.as_tensor(bt, device=device),
        context_lens=torch.tensor([c for c, _ in seqs], dtype=torch.int32, device=device),
        seqs=list(seqs), tables_host=tables, scale=head_dim ** -0.5, num_prefills=num_prefills,
    )


def _randn_big(shape, gen, device, dtype, kv_scale):
    out = torch.empty(shape, device=device, dtype=dtype)
    flat = out.view(shape[0], -1)
    step = max(1, (1 << 26) // flat.shape[1])
    for s in range(0, shape[0], step):
        blk = flat[s:s + step]
        blk.copy_(torch.randn(blk.shape, generator=gen, device=device, dtype=torch.float32) * kv_scale)
    return out


# ---------------------------------------------------------------- configs

def tinyllama_decode(device, seed: int = 0, batch: int = 16) -> PagedBatch:
    rng = np.random.default_rng(seed)
    ctx = rng.integers(16, 1024, size=batch, endpoint=True)
    return build_batch([(int(c), 1) for c in ctx], heads=32, kv_heads=4, head_dim=64, dtype=torch.float16,
                       device=device, seed=seed, pool_blocks=1100, contiguous_slices=True, write_first=False)


def tinyllama_prefill(device, seed: int = 0, n_seqs: int = 8) -> PagedBatch:
    rng = np.random.default_rng(seed + 1)
    q_len = rng.integers(32, 512, size=n_seqs, endpoint=True)
    prefix = rng.integers(0, 256, size=n_seqs, endpoint=True)
    return build_batch([(int(p + ql), int(ql)) for p, ql in zip(prefix, q_len)], heads=32, kv_heads=4,
                       head_dim=64, dtype=torch.float16, device=device, seed=seed)


def llama3_decode_lens(seed: int = 0, batch: int = 64) -> list[int]:
    rng = np.random.default_rng(seed + 2)
    return [int(round(math.exp(x))) for x in rng.uniform(math.log(128), math.log(8192), size=batch)]


def llama3_decode(device, seed: int = 0, batch: int = 64) -> PagedBatch:
    ctx = llama3_decode_lens(seed, batch)
    return build_batch([(c, 1) for c in ctx], heads=32, kv_heads=8, head_dim=128, dtype=torch.bfloat16,
                       device=device, seed=seed, pool_factor=1.2, kv_scale=0.5, write_first=False)


def llama3_mixed(device, seed: int = 0) -> PagedBatch:
    rng = np.random.default_rng(seed + 3)
    prefix = rng.integers(0, 1024, size=4, endpoint=True)
    dec = rng.integers(256, 4096, size=60, endpoint=True)
    seqs = [(int(p) + 512, 512) for p in prefix] + [(int(c), 1) for c in dec]
    return build_batch(seqs, heads=32, kv_heads=8, head_dim=128, dtype=torch.bfloat16, device=device,
                       seed=seed, pool_factor=1.2)


def llama3_long_lens(seed: int = 0, batch: int = 256) -> list[int]:
    rng = np.random.default_rng(seed + 4)
    long_rows = rng.random(batch) < 0.1
    short = rng.integers(512, 4096, size=batch, endpoint=True)
    long_ = rng.integers(16384, 32768, size=batch, endpoint=True)
    return [int(l if f else s) for f, s, l in zip(long_rows, short, long_)]


def llama3_long_decode(device, seed: int = 0, batch: int = 256, pool_gb: float = 40.0) -> PagedBatch:
    ctx = llama3_long_lens(seed, batch)
    block_bytes = 2 * BLOCK_SIZE * 8 * 128 * 2  # K and V page bytes, bf16
    nb = int(pool_gb * 1e9 // block_bytes)
    return build_batch([(c, 1) for c in ctx], heads=32, kv_heads=8, head_dim=128, dtype=torch.bfloat16,
                       device=device, seed=seed, pool_blocks=nb, kv_scale=0.5, write_first=False, fill="used")


CONFIGS = {
    "tinyllama_decode": tinyllama_decode,
    "tinyllama_prefill": tinyllama_prefill,
    "llama3_decode": llama3_decode,
    "llama3_mixed": llama3_mixed,
    "llama3_long_decode": llama3_long_decode,
}


# ---------------------------------------------------------------- algorithmic work

def decode_bytes(ctx_lens, heads: int, kv_heads: int, head_dim: int, elem: int = 2) -> int:
    """Algorithmic HBM bytes of one decode call: every visible K and V row once,
    q in and out once, the page ids and context lengths."""
    b = len(ctx_lens)
    return (sum(ctx_lens) * 2 * kv_heads * head_dim * elem + 2 * b * heads * head_dim * elem
            + 4 * sum(_pages(c) for c in ctx_lens) + 4 * b)


def prefill_flops(seqs, heads: int, head_dim: int) -> int:
    """Causal pairs only: 4*D*H*sum(q*prefix + q(q+1)/2)."""
    return 4 * head_dim * heads * sum(ql * (c - ql) + ql * (ql + 1) // 2 for c, ql in seqs)


def prefill_bytes(seqs, heads: int, kv_heads: int, head_dim: int, elem: int = 2) -> int:
    tq = sum(ql for _, ql in seqs)
    return 2 * tq * heads * head_dim * elem + sum(c for c, _ in seqs) * 2 * kv_heads * head_dim * elem


def write_kv_bytes(tokens: int, kv_heads: int, head_dim: int, elem: int = 2) -> int:
    return 4 * tokens * kv_heads * head_dim * elem + 8 * tokens


# ---------------------------------------------------------------- flat steps from sequence states

@dataclass
class SeqState:
    """What a forward step reads of a sequence: its tokens so far, how many of
    them already have K/V in the cache, and its pages. The attribute names are
    those of Nimbus's Sequence (nimbus/sequence.py), so DecodeGraphs takes
    either."""

    token_ids: list
    block_table: list = field(default_factory=list)
    num_computed: int = 0

    def __len__(self) -> int:
        return len(self.token_ids)

    def feed(self, token: int) -> None:
        """Every pending token was computed and `token` was sampled after them."""
        self.num_computed = len(self.token_ids)
        self.token_ids.append(int(token))

    def copy(self) -> "SeqState":
        return SeqState(list(self.token_ids), list(self.block_table), self.num_computed)


def is_decode(seq, n: int) -> bool:
    """A sequence feeding its single last pending token on top of a cached
    prefix is a decode; anything else is a prefill (possibly a chunk that
    continues a cached prefix)."""
    return n == 1 and 0 < seq.num_computed == len(seq) - 1


@dataclass
class FlatStep:
    input_ids: torch.Tensor  # [T] int64
    positions: torch.Tensor  # [T] int64
    meta: object  # model.attention.AttnMetadata
    sample_rows: torch.Tensor  # [S'] int64: last row of every sequence whose pending tokens this step finishes


def flat_step(entries, device, block_size: int = BLOCK_SIZE) -> FlatStep:
    """One forward pass over `entries` = [(sequence, tokens to feed)], laid out
    as Nimbus's runner lays it (nimbus/runner.py:33-96): the fed tokens of
    every sequence back to back, prefills first; token p of a sequence goes to
    slot table[p // block_size] * block_size + p % block_size; each group's
    block tables are zero-padded to its widest row."""
    from nimbus_amd.model.attention import AttnMetadata

    if not entries:
        raise ValueError("empty step")
    feed = np.array([n for _, n in entries], dtype=np.int64)
    start = np.array([s.num_computed for s, _ in entries], dtype=np.int64)
    end = start + feed
    if (feed < 1).any() or (end > np.array([len(s) for s, _ in entries])).any():
        raise ValueError("a sequence is asked for tokens it does not have")
    dec = np.array([is_decode(s, int(n)) for s, n in entries])
    if dec.any() and not dec[int(np.argmax(dec)):].all():
        raise ValueError("prefill sequences must come before decodes")
    widths = np.array([len(s.block_table) for s, _ in entries], dtype=np.int64)
    if (widths * block_size < end).any():
        raise ValueError("a sequence has too few blocks for its tokens")
    tables = np.zeros((len(entries), max(1, int(widths.max()))), dtype=np.int32)
    for r, (s, _) in enumerate(entries):
        tables[r, :widths[r]] = s.block_table
    row_of = np.repeat(np.arange(len(entries)), feed)
    first_row = np.cumsum(feed) - feed
    pos = start[row_of] + np.arange(row_of.size) - first_row[row_of]
    slots = tables[row_of, pos // block_size].astype(np.int64) * block_size + pos % block_size
    ids = np.concatenate([np.asarray(s.token_ids[a:b], dtype=np.int64) for (s, _), a, b in zip(entries, start, end)])
    done = end == np.array([len(s) for s, _ in entries])
    sample = (first_row + feed - 1)[done]

    def group(mask):
        w = max(1, int(widths[mask].max())) if mask.any() else 1
        return torch.from_numpy(np.ascontiguousarray(tables[mask, :w])).to(device)

    pf = ~dec
    qs_host = [0] + np.cumsum(feed[pf]).tolist()
    pf_ctx = end[pf].tolist()
    dc_ctx = end[dec].tolist()
    dev_i32 = lambda x: torch.tensor(x, dtype=torch.int32).to(device)  # noqa: E731
    meta = AttnMetadata(
        slot_mapping=torch.from_numpy(slots).to(device), num_prefill_tokens=qs_host[-1],
        prefill_query_start=dev_i32(qs_host), prefill_context_lens=dev_i32(pf_ctx), prefill_block_tables=group(pf),
        decode_context_lens=dev_i32(dc_ctx), decode_block_tables=group(dec), max_decode_context=max(dc_ctx, default=0),
        prefill_query_start_host=qs_host, prefill_context_lens_host=pf_ctx)
    return FlatStep(torch.from_numpy(ids).to(device), torch.from_numpy(pos).to(device), meta,
                    torch.from_numpy(sample).to(device))
