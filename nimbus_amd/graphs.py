"""Decode steps and speculative-verify attention replayed from hipGraphs at
padded batch sizes.

DecodeGraphs replays the whole model's decode step (nimbus/cuda_graph.py:
28-144): embedding, every layer, final norm and logits, captured once per
padded batch size; greedy_chain runs many greedy steps without returning
to the host, each one a replay of the step graph and of a one-kernel graph
that picks the tokens and advances positions, context lengths and slots on
the device. DecodeAttentionGraphs and VerifyAttentionGraphs replay the
attention layer alone.

Follows the capture contract of Nimbus's DecodeGraphs (nimbus/cuda_graph.py:
38-79 and 118-144), restricted to the attention layer (the slot write plus
paged decode attention) instead of the whole model:

- inputs live in static device buffers sized for the largest batch, and a
  step's real batch is padded up to the nearest captured size
  (1, 2, 4, 8, 16, 24, 32, 48, 64, 96, 128 below max_batch, then max_batch);
- padding rows have context length 1, write their K/V into a scratch slot and
  read a scratch block that no sequence owns (cuda_graph.py:133-138);
- max_decode_context is pinned to max_model_len, which pins the decode grid,
  so one graph per size serves every mix of context lengths.

Nothing inside a captured region allocates outside the graph pool, reads
device memory on the host or issues a memset.

VerifyAttentionGraphs does the same for speculative verification
(nimbus/spec/engine.py:60-150): there every sequence feeds k + 1 tokens, all
through the prefill call, which runs them in its verify form (the page-split
decode kernels with k + 1 query columns per head) when they fit it.
VerifyGraphs replays the target model's whole verification pass the same
way, as the reference's VerifyGraphs does.
"""

from __future__ import annotations

import bisect

import numpy as np
import torch

from nimbus_amd.kernels.elementwise import greedy_step
from nimbus_amd.kernels.paged_attention import (decode_workspace_bytes, new_decode_workspace,
                                                verify_workspace_bytes)
from nimbus_amd.kernels.prefill_attention import verify_queries
from nimbus_amd.model.attention import AttentionBackend, AttnMetadata
from nimbus_amd.workloads import is_decode

PADDED_SIZES = (1, 2, 4, 8, 16, 24, 32, 48, 64, 96, 128)


class DecodeAttentionGraphs:
    def __init__(self, k_cache: torch.Tensor, v_cache: torch.Tensor, num_heads: int, scale: float,
                 max_model_len: int, max_batch: int, scratch_block: int):
        self.k_cache, self.v_cache = k_cache, v_cache
        self.block_size = k_cache.shape[1]
        kv, d = k_cache.shape[2], k_cache.shape[3]
        dev, dt = k_cache.device, k_cache.dtype
        self.scale = scale
        self.max_model_len = max_model_len
        self.max_batch = max_batch
        self.scratch_block = scratch_block
        self.scratch_slot = scratch_block * self.block_size
        self.sizes = [b for b in PADDED_SIZES if b < max_batch] + [max_batch]
        width = -(-max_model_len // self.block_size)
        self.q = torch.zeros(max_batch, num_heads, d, dtype=dt, device=dev)
        self.k = torch.zeros(max_batch, kv, d, dtype=dt, device=dev)
        self.v = torch.zeros(max_batch, kv, d, dtype=dt, device=dev)
        self.slots = torch.full((max_batch,), self.scratch_slot, dtype=torch.int64, device=dev)
        self.ctx = torch.ones(max_batch, dtype=torch.int32, device=dev)
        self.tables = torch.full((max_batch, width), scratch_block, dtype=torch.int32, device=dev)
        # The graphs' own decode workspace (page prefix + split pieces), sized for the largest batch.
        self.workspace = new_decode_workspace(decode_workspace_bytes(max_batch, num_heads, d, max_model_len), dev)
        self.backend = AttentionBackend(decode_workspace=self.workspace)
        self.graphs: dict[int, tuple[torch.cuda.CUDAGraph, torch.Tensor, AttnMetadata]] = {}

    def _meta(self, b: int) -> AttnMetadata:
        dev = self.k_cache.device
        empty = torch.zeros(0, dtype=torch.int32, device=dev)
        return AttnMetadata(
            slot_mapping=self.slots[:b], num_prefill_tokens=0,
            prefill_query_start=torch.zeros(1, dtype=torch.int32, device=dev),
            prefill_context_lens=empty, prefill_block_tables=empty.view(0, 1),
            decode_context_lens=self.ctx[:b], decode_block_tables=self.tables[:b],
            max_decode_context=self.max_model_len,
            prefill_query_start_host=[0], prefill_context_lens_host=[],
        )

    def _forward(self, b: int, meta: AttnMetadata) -> torch.Tensor:
        return self.backend.forward(self.q[:b], self.k[:b], self.v[:b], self.k_cache, self.v_cache, meta,
                                    self.scale)

    @torch.inference_mode()
    def capture(self) -> None:
        pool = torch.cuda.graph_pool_handle()
        for b in reversed(self.sizes):  # largest first, so the pool is sized once
            meta = self._meta(b)
            for _ in range(2):
                self._forward(b, meta)
            torch.cuda.synchronize()
            g = torch.cuda.CUDAGraph()
            with torch.cuda.graph(g, pool=pool):
                out = self._forward(b, meta)
            self.graphs[b] = (g, out, meta)  # meta's tensors must outlive the graph
        torch.cuda.synchronize()

    def padded_size(self, n: int) -> int:
        return self.sizes[bisect.bisect_left(self.sizes, n)]

    @torch.inference_mode()
    def load(self, q, k, v, slot_mapping, context_lens, block_tables) -> int:
        """Copies one decode batch into the static buffers (device to device)
        and pads it; returns the captured size that will run."""
        n = q.shape[0]
        if not 0 < n <= self.max_batch:
            raise ValueError(f"batch {n} outside 1..{self.max_batch}")
        b = self.padded_size(n)
        w = block_tables.shape[1]
        if w > self.tables.shape[1]:
            raise ValueError("block tables wider than max_model_len allows")
        self.q[:n].copy_(q)
        self.k[:n].copy_(k)
        self.v[:n].copy_(v)
        self.slots[:n].copy_(slot_mapping)
        self.ctx[:n].copy_(context_lens)
        self.tables[:n, :w].copy_(block_tables)
        if b > n:
            self.slots[n:b].fill_(self.scratch_slot)
            self.ctx[n:b].fill_(1)
            self.tables[n:b, 0].fill_(self.scratch_block)
        return b

    def replay(self, b: int) -> torch.Tensor:
        g, out, _ = self.graphs[b]
        g.replay()
        return out

    def run(self, q, k, v, slot_mapping, context_lens, block_tables) -> torch.Tensor:
        """One decode attention step: returns [n, H, D] for the n real rows."""
        n = q.shape[0]
        return self.replay(self.load(q, k, v, slot_mapping, context_lens, block_tables))[:n]


VERIFY_SIZES = (1, 2, 4, 8, 16)


class VerifyAttentionGraphs:
    """Speculative verification's attention replayed from hipGraphs.

    Follows Nimbus's VerifyGraphs (nimbus/spec/engine.py:60-150), restricted
    to the attention layer (slot write + paged prefill attention):

    - every sequence feeds exactly q = k + 1 <= block_size tokens, all of
      them prefill tokens, so a step's metadata differs only in device data;
    - the tile table is precomputed as (arange(b), zeros(b)) (:86-87): one
      entry per sequence, since q <= 16 < BLOCK_M;
    - the host lists are placeholders ([q] * b context lengths, :96) that the
      kernels never read: context lengths and query starts come from the
      device buffers each replay;
    - padding sequences (up to the captured sizes 1, 2, 4, 8, 16 below
      max_batch, then max_batch) have context q and write and read the
      scratch block, which holds q <= block_size tokens (:118-126).

    kernel: "auto" lets the prefill call pick its verify form (a workspace
    for it, sized for max_batch and max_model_len, is owned here); "tile"
    pins the tile kernel, as in the reference.
    """

    def __init__(self, k_cache: torch.Tensor, v_cache: torch.Tensor, num_heads: int, scale: float,
                 max_model_len: int, max_batch: int, k: int, scratch_block: int, kernel: str = "auto"):
        if kernel not in ("auto", "tile"):
            raise ValueError(f"kernel must be 'auto' or 'tile', got {kernel!r}")
        self.block_size = k_cache.shape[1]
        if not 0 < k + 1 <= self.block_size:
            raise ValueError(f"k + 1 = {k + 1} must fit one block of {self.block_size}")
        self.k_cache, self.v_cache = k_cache, v_cache
        self.q_len = q = k + 1
        kv, d = k_cache.shape[2], k_cache.shape[3]
        dev, dt = k_cache.device, k_cache.dtype
        self.scale = scale
        self.max_batch = max_batch
        self.scratch_block = scratch_block
        self.sizes = [b for b in VERIFY_SIZES if b < max_batch] + [max_batch]
        width = -(-max_model_len // self.block_size)
        self.q = torch.zeros(max_batch * q, num_heads, d, dtype=dt, device=dev)
        self.k = torch.zeros(max_batch * q, kv, d, dtype=dt, device=dev)
        self.v = torch.zeros(max_batch * q, kv, d, dtype=dt, device=dev)
        self.pad_slots = scratch_block * self.block_size + torch.arange(q, dtype=torch.int64, device=dev)
        self.slots = self.pad_slots.repeat(max_batch)
        self.ctx = torch.full((max_batch,), q, dtype=torch.int32, device=dev)
        self.tables = torch.full((max_batch, width), scratch_block, dtype=torch.int32, device=dev)
        self.qstart = torch.arange(0, (max_batch + 1) * q, q, dtype=torch.int32, device=dev)
        self.kernel = kernel
        workspace = None
        if kernel == "auto" and verify_queries(list(range(0, (max_batch + 1) * q, q)), num_heads, kv):
            # the verify form bounds contexts by the block-table width
            nbytes = verify_workspace_bytes(max_batch, q, num_heads, d, width * self.block_size)
            workspace = new_decode_workspace(nbytes, dev)
        self.backend = AttentionBackend(decode_workspace=workspace)
        self.graphs: dict[int, tuple[torch.cuda.CUDAGraph, torch.Tensor, AttnMetadata]] = {}

    def _meta(self, b: int) -> AttnMetadata:
        dev = self.k_cache.device
        empty = torch.zeros(0, dtype=torch.int32, device=dev)
        q = self.q_len
        progs = (torch.arange(b, dtype=torch.int32, device=dev), torch.zeros(b, dtype=torch.int32, device=dev))
        return AttnMetadata(
            slot_mapping=self.slots[:b * q], num_prefill_tokens=b * q,
            prefill_query_start=self.qstart[:b + 1], prefill_context_lens=self.ctx[:b],
            prefill_block_tables=self.tables[:b],
            decode_context_lens=empty, decode_block_tables=empty.view(0, 1), max_decode_context=0,
            prefill_query_start_host=list(range(0, (b + 1) * q, q)), prefill_context_lens_host=[q] * b,
            prefill_programs=progs, prefill_kernel=None if self.kernel == "auto" else self.kernel,
        )

    def _forward(self, b: int, meta: AttnMetadata) -> torch.Tensor:
        n = b * self.q_len
        return self.backend.forward(self.q[:n], self.k[:n], self.v[:n], self.k_cache, self.v_cache, meta,
                                    self.scale)

    @torch.inference_mode()
    def capture(self) -> None:
        pool = torch.cuda.graph_pool_handle()
        for b in reversed(self.sizes):
            meta = self._meta(b)
            for _ in range(2):
                self._forward(b, meta)
            torch.cuda.synchronize()
            g = torch.cuda.CUDAGraph()
            with torch.cuda.graph(g, pool=pool):
                out = self._forward(b, meta)
            self.graphs[b] = (g, out, meta)  # meta's tensors (the tile table) must outlive the graph
        torch.cuda.synchronize()

    def padded_size(self, n: int) -> int:
        return self.sizes[bisect.bisect_left(self.sizes, n)]

    @torch.inference_mode()
    def load(self, q, k, v, slot_mapping, context_lens, block_tables) -> int:
        """Copies one verification batch (n sequences, n * q tokens in sequence
        order) into the static buffers and pads it; returns the captured size
        that will run."""
        qn = self.q_len
        n = context_lens.shape[0]
        if not 0 < n <= self.max_batch or q.shape[0] != n * qn:
            raise ValueError(f"{n} sequences of {qn} tokens expected, got q {tuple(q.shape)}")
        b = self.padded_size(n)
        w = block_tables.shape[1]
        if w > self.tables.shape[1]:
            raise ValueError("block tables wider than max_model_len allows")
        self.q[:n * qn].copy_(q)
        self.k[:n * qn].copy_(k)
        self.v[:n * qn].copy_(v)
        self.slots[:n * qn].copy_(slot_mapping)
        self.ctx[:n].copy_(context_lens)
        self.tables[:n, :w].copy_(block_tables)
        if b > n:
            self.slots[n * qn:b * qn].copy_(self.pad_slots.repeat(b - n))
            self.ctx[n:b].fill_(qn)
            self.tables[n:b, 0].fill_(self.scratch_block)
        return b

    def replay(self, b: int) -> torch.Tensor:
        g, out, _ = self.graphs[b]
        g.replay()
        return out

    def run(self, q, k, v, slot_mapping, context_lens, block_tables) -> torch.Tensor:
        """One verification step's attention: returns [n * q, H, D]."""
        n = context_lens.shape[0]
        return self.replay(self.load(q, k, v, slot_mapping, context_lens, block_tables))[:n * self.q_len]


class DecodeGraphs:
    """Whole decode steps of `model` replayed from hipGraphs.

    Follows nimbus/cuda_graph.py:28-144: static input buffers sized for
    max_batch, a step's batch padded up to the nearest captured size
    (PADDED_SIZES below max_batch, then max_batch), padding rows at position
    0 with context 1 writing and reading the scratch block, and the decode
    grid pinned by max_model_len so one graph per size serves every mix of
    context lengths. The model's attention backend gets a decode workspace
    of its own (sized for max_batch and max_model_len) unless it has one.

    greedy_chain keeps every step on the device: after each replay of the
    step graph, a second captured graph (one nimbus_greedy_step kernel)
    takes each row's argmax as its next token, records it, and advances the
    real rows' positions, context lengths and slots; the host only reads the
    recorded tokens at the end. A chain is at most max_chain steps.
    """

    def __init__(self, model, kv_layers, block_size: int, max_model_len: int, max_batch: int, scratch_block: int,
                 num_kv_heads: int, device, max_chain: int = 256):
        self.model = model
        self.kv_layers = kv_layers
        self.block_size = block_size
        self.max_model_len = max_model_len
        self.scratch_block = scratch_block
        self.scratch_slot = scratch_block * block_size
        self.sizes = [b for b in PADDED_SIZES if b < max_batch] + [max_batch]
        self.max_batch = max_batch
        self.max_chain = max_chain
        self.kv_heads = num_kv_heads
        self.device = device
        width = -(-max_model_len // block_size)
        i64, i32 = torch.int64, torch.int32
        self.input_ids = torch.zeros(max_batch, dtype=i64, device=device)
        self.positions = torch.zeros(max_batch, dtype=i64, device=device)
        self.slots = torch.full((max_batch,), self.scratch_slot, dtype=i64, device=device)
        self.ctx = torch.ones(max_batch, dtype=i32, device=device)
        self.tables = torch.full((max_batch, width), scratch_block, dtype=i32, device=device)
        self.active = torch.zeros(max_batch, dtype=i32, device=device)
        self.ctx_start = torch.ones(max_batch, dtype=i32, device=device)
        self.tokens = torch.zeros(max_batch, max_chain, dtype=i64, device=device)
        # Pinned staging for _load (allocated pinned, never registered).
        self._host = torch.empty((4, max_batch), dtype=i64, pin_memory=True)
        self._host_tables = torch.empty((max_batch, width), dtype=i32, pin_memory=True)
        self._staged = None  # event after the last staged copies: the pinned rows are reused only after it
        backend = model.backend
        if backend.decode_workspace is None:
            cfg = model.cfg
            backend.decode_workspace = new_decode_workspace(
                decode_workspace_bytes(max_batch, cfg.num_heads, cfg.head_dim, max_model_len), device)
        self.graphs: dict[int, tuple[torch.cuda.CUDAGraph, torch.Tensor, AttnMetadata, torch.cuda.CUDAGraph]] = {}

    def _meta(self, b: int) -> AttnMetadata:
        empty = torch.zeros(0, dtype=torch.int32, device=self.device)
        return AttnMetadata(
            slot_mapping=self.slots[:b], num_prefill_tokens=0,
            prefill_query_start=torch.zeros(1, dtype=torch.int32, device=self.device),
            prefill_context_lens=empty, prefill_block_tables=empty.view(0, 1),
            decode_context_lens=self.ctx[:b], decode_block_tables=self.tables[:b],
            max_decode_context=self.max_model_len, prefill_query_start_host=[0], prefill_context_lens_host=[])

    def _step(self, b: int, meta: AttnMetadata) -> torch.Tensor:
        return self.model.logits(self.model(self.input_ids[:b], self.positions[:b], self.kv_layers, meta))

    def _advance(self, b: int, logits: torch.Tensor) -> None:
        greedy_step(logits, self.input_ids, self.positions, self.ctx, self.slots, self.tables, self.block_size,
                    self.active, self.ctx_start, self.tokens, self.scratch_slot)

    @torch.inference_mode()
    def capture(self) -> None:
        pool = torch.cuda.graph_pool_handle()
        for b in reversed(self.sizes):  # largest first, so the pool is sized once
            meta = self._meta(b)
            for _ in range(2):
                self._step(b, meta)
            torch.cuda.synchronize()
            g = torch.cuda.CUDAGraph()
            with torch.cuda.graph(g, pool=pool):
                logits = self._step(b, meta)
            adv = torch.cuda.CUDAGraph()
            with torch.cuda.graph(adv, pool=pool):
                self._advance(b, logits)
            self.graphs[b] = (g, logits, meta, adv)  # meta's tensors must outlive the graph
        torch.cuda.synchronize()

    def can_run(self, batch) -> bool:
        """True for (sequence, tokens) pairs that are all plain decodes and fit
        the captured sizes (the condition of cuda_graph.py:83-85)."""
        return 0 < len(batch) <= self.max_batch and all(is_decode(s, n) for s, n in batch)

    @torch.inference_mode()
    def run(self, seqs) -> torch.Tensor:
        """One decode step for seqs; returns their logits [len(seqs), vocab]
        (fp32, a view of the graph's output, valid until the next replay)."""
        g, logits, _, _ = self.graphs[self._load(seqs)]
        g.replay()
        return logits[:len(seqs)]

    @torch.inference_mode()
    def greedy_chain(self, seqs, steps: int) -> torch.Tensor:
        """`steps` greedy decode steps without returning to the host; returns
        the chosen tokens [len(seqs), steps]. Every block table must already
        cover `steps` more tokens (cuda_graph.py:92-99)."""
        if not 0 < steps <= self.max_chain:
            raise ValueError(f"steps must be in 1..{self.max_chain}")
        n = len(seqs)
        g, _, _, adv = self.graphs[self._load(seqs)]
        for _ in range(steps):
            g.replay()
            adv.replay()
        return self.tokens[:n, :steps].clone()

    def _load(self, seqs) -> int:
        """Stages seqs' next-token inputs into the static buffers and pads the
        batch to a captured size (the contract of cuda_graph.py:118-144):
        each real row feeds token num_computed at that position, writing slot
        table[p // bs] * bs + p % bs, with context p + 1; padding rows feed
        token 0 at position 0 with context 1 on the scratch block. The rows
        are assembled in pinned host memory and copied in one go per buffer.
        Returns the captured size."""
        n = len(seqs)
        if not 0 < n <= self.max_batch:
            raise ValueError(f"batch {n} outside 1..{self.max_batch}")
        b = self.sizes[bisect.bisect_left(self.sizes, n)]
        bs = self.block_size
        if self._staged is not None:
            self._staged.synchronize()  # the previous call's copies have read the pinned rows
        rows, tables = self._host.numpy(), self._host_tables.numpy()
        widths = [len(s.block_table) for s in seqs]
        if max(widths) > tables.shape[1]:
            raise ValueError("a block table is wider than max_model_len allows")
        tables[:n] = 0
        for i, s in enumerate(seqs):
            tables[i, :widths[i]] = s.block_table
        pos = np.fromiter((s.num_computed for s in seqs), dtype=np.int64, count=n)
        short = np.flatnonzero(pos // bs >= np.asarray(widths, dtype=np.int64))
        if short.size:
            # (the zero padding past a table's width would send the token's K/V to block 0, which another
            # sequence may own; nimbus/cuda_graph.py:118-135 raises IndexError on block_table[p // bs])
            i = int(short[0])
            raise IndexError(f"sequence {i} has {widths[i]} blocks, too few for position {int(pos[i])}")
        rows[0, :n] = [s.token_ids[p] for s, p in zip(seqs, pos.tolist())]
        rows[1, :n] = pos
        rows[2, :n] = tables[np.arange(n), pos // bs].astype(np.int64) * bs + pos % bs
        rows[3, :n] = pos + 1
        rows[:, n:b] = np.array([[0], [0], [self.scratch_slot], [1]])
        tables[n:b, 0] = self.scratch_block
        for dst, src in ((self.input_ids, self._host[0]), (self.positions, self._host[1]),
                         (self.slots, self._host[2]), (self.ctx, self._host[3])):
            dst[:b].copy_(src[:b], non_blocking=True)
        self.tables[:b].copy_(self._host_tables[:b], non_blocking=True)
        self._staged = torch.cuda.Event()
        self._staged.record()
        self.ctx_start[:b].copy_(self.ctx[:b])
        self.active[:n].fill_(1)
        self.active[n:b].fill_(0)
        return b


class VerifyGraphs:
    """The target model's whole verification pass replayed from hipGraphs.

    Follows Nimbus's VerifyGraphs (nimbus/spec/engine.py:60-150): every
    sequence feeds its last q = k + 1 <= block_size tokens (the pending token
    and k drafts) through one forward pass of `model` (embedding, every
    layer, final norm, logits), all as prefill tokens, so a step differs from
    the captured one only in device data. One graph per batch size (1, 2, 4,
    8, 16 below max_batch, then max_batch); padding sequences sit at
    positions 0..q - 1 of the scratch block with context q. The tile table
    is fixed at capture (one entry per sequence, q < 64 query rows) and the
    host lists are placeholders the kernels never read.

    kernel: "auto" lets the prefill call take its verify form (the page-split
    decode kernels with q query columns per head) when the heads fit it;
    "tile" pins the tile kernel, as in the reference. The graphs own a
    workspace sized for max_batch and max_model_len, which the model's
    backend holds while they are captured (and is restored afterwards).
    """

    def __init__(self, model, kv_layers, block_size: int, max_model_len: int, max_batch: int, k: int,
                 scratch_block: int, device, kernel: str = "auto"):
        if kernel not in ("auto", "tile"):
            raise ValueError(f"kernel must be 'auto' or 'tile', got {kernel!r}")
        if not 0 < k + 1 <= block_size:
            raise ValueError(f"k + 1 = {k + 1} must fit one block of {block_size}")
        self.model = model
        self.kv_layers = kv_layers
        self.block_size = block_size
        self.q_len = q = k + 1
        self.max_batch = max_batch
        self.scratch_block = scratch_block
        self.kernel = kernel
        self.device = device
        self.sizes = [b for b in VERIFY_SIZES if b < max_batch] + [max_batch]
        width = -(-max_model_len // block_size)
        i64, i32 = torch.int64, torch.int32
        self.input_ids = torch.zeros(max_batch * q, dtype=i64, device=device)
        self.positions = torch.zeros(max_batch * q, dtype=i64, device=device)
        self.slots = torch.zeros(max_batch * q, dtype=i64, device=device)
        self.ctx = torch.full((max_batch,), q, dtype=i32, device=device)
        self.tables = torch.full((max_batch, width), scratch_block, dtype=i32, device=device)
        self.qstart = torch.arange(0, (max_batch + 1) * q, q, dtype=i32, device=device)
        self._host = torch.empty((3, max_batch * q), dtype=i64, pin_memory=True)
        self._host_ctx = torch.empty(max_batch, dtype=i32, pin_memory=True)
        self._host_tables = torch.empty((max_batch, width), dtype=i32, pin_memory=True)
        self._staged = None  # event after the last staged copies: the pinned rows are reused only after it
        cfg = model.cfg
        self.workspace = None
        if kernel == "auto" and verify_queries(list(range(0, (max_batch + 1) * q, q)), cfg.num_heads,
                                               cfg.num_kv_heads):
            need = verify_workspace_bytes(max_batch, q, cfg.num_heads, cfg.head_dim, width * block_size)
            self.workspace = new_decode_workspace(need, device)
        self.graphs: dict[int, tuple[torch.cuda.CUDAGraph, torch.Tensor, AttnMetadata]] = {}

    def _meta(self, b: int) -> AttnMetadata:
        empty = torch.zeros(0, dtype=torch.int32, device=self.device)
        q = self.q_len
        progs = (torch.arange(b, dtype=torch.int32, device=self.device),
                 torch.zeros(b, dtype=torch.int32, device=self.device))
        return AttnMetadata(
            slot_mapping=self.slots[:b * q], num_prefill_tokens=b * q,
            prefill_query_start=self.qstart[:b + 1], prefill_context_lens=self.ctx[:b],
            prefill_block_tables=self.tables[:b],
            decode_context_lens=empty, decode_block_tables=empty.view(0, 1), max_decode_context=0,
            prefill_query_start_host=list(range(0, (b + 1) * q, q)), prefill_context_lens_host=[q] * b,
            prefill_programs=progs, prefill_kernel=None if self.kernel == "auto" else self.kernel,
        )

    def _step(self, b: int, meta: AttnMetadata) -> torch.Tensor:
        n = b * self.q_len
        return self.model.logits(self.model(self.input_ids[:n], self.positions[:n], self.kv_layers, meta))

    @torch.inference_mode()
    def capture(self) -> None:
        backend = self.model.backend
        held = backend.decode_workspace
        if self.workspace is not None:
            backend.decode_workspace = self.workspace
        try:
            pool = torch.cuda.graph_pool_handle()
            for b in reversed(self.sizes):
                self._load([], b)  # valid padding everywhere before the warm-up passes
                meta = self._meta(b)
                for _ in range(2):
                    self._step(b, meta)
                torch.cuda.synchronize()
                g = torch.cuda.CUDAGraph()
                with torch.cuda.graph(g, pool=pool):
                    logits = self._step(b, meta)
                self.graphs[b] = (g, logits, meta)  # meta's tensors (the tile table) must outlive the graph
            torch.cuda.synchronize()
        finally:
            backend.decode_workspace = held

    def padded_size(self, n: int) -> int:
        return self.sizes[bisect.bisect_left(self.sizes, n)]

    def _load(self, seqs, b: int) -> None:
        """Stages the last q tokens of every sequence (token, position, the
        slot table[p // bs] * bs + p % bs, context len(s), the block table)
        and the padding rows (token 0 at positions 0..q - 1 of the scratch
        block, context q) in pinned host memory, then copies each buffer in
        one go (the contract of nimbus/spec/engine.py:114-139)."""
        q, bs, n = self.q_len, self.block_size, len(seqs)
        if self._staged is not None:
            self._staged.synchronize()  # the previous call's copies have read the pinned rows
        rows, ctx, tables = self._host.numpy(), self._host_ctx.numpy(), self._host_tables.numpy()
        tables[:b] = 0
        for i, s in enumerate(seqs):
            if len(s) < q:
                raise ValueError(f"sequence {i} holds {len(s)} tokens, fewer than the {q} it must feed")
            if len(s.block_table) > tables.shape[1]:
                raise ValueError("a block table is wider than max_model_len allows")
            tables[i, :len(s.block_table)] = s.block_table
            ctx[i] = len(s)
            rows[0, i * q:(i + 1) * q] = s.token_ids[len(s) - q:]
        pos = (ctx[:n, None].astype(np.int64) - q + np.arange(q)[None, :]).reshape(-1)
        widths = np.repeat(np.fromiter((len(s.block_table) for s in seqs), dtype=np.int64, count=n), q)
        short = np.flatnonzero(pos // bs >= widths)
        if short.size:
            # (as DecodeGraphs._load: nimbus/spec/engine.py:117-128 raises IndexError on block_table[p // bs])
            i = int(short[0]) // q
            raise IndexError(f"sequence {i} has {len(seqs[i].block_table)} blocks, too few for position "
                             f"{int(pos[short[0]])}")
        rows[1, :n * q] = pos
        rows[2, :n * q] = tables[np.repeat(np.arange(n), q), pos // bs].astype(np.int64) * bs + pos % bs
        pad = np.arange(q, dtype=np.int64)
        rows[0, n * q:b * q] = 0
        rows[1, n * q:b * q] = np.tile(pad, b - n)
        rows[2, n * q:b * q] = np.tile(self.scratch_block * bs + pad, b - n)
        ctx[n:b] = q
        tables[n:b, 0] = self.scratch_block
        for dst, src in ((self.input_ids, self._host[0]), (self.positions, self._host[1]),
                         (self.slots, self._host[2])):
            dst[:b * q].copy_(src[:b * q], non_blocking=True)
        self.ctx[:b].copy_(self._host_ctx[:b], non_blocking=True)
        self.tables[:b].copy_(self._host_tables[:b], non_blocking=True)
        self._staged = torch.cuda.Event()
        self._staged.record()

    @torch.inference_mode()
    def run(self, seqs) -> torch.Tensor:
        """The verification pass for seqs (each feeding its last q tokens);
        returns their logits [len(seqs) * q, vocab] (fp32, a view of the
        graph's output, valid until the next replay)."""
        n = len(seqs)
        if not 0 < n <= self.max_batch:
            raise ValueError(f"batch {n} outside 1..{self.max_batch}")
        b = self.padded_size(n)
        self._load(seqs, b)
        g, logits, _ = self.graphs[b]
        g.replay()
        return logits[:n * self.q_len]
