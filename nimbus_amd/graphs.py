"""Decode attention replayed from hipGraphs at padded batch sizes.

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
"""

from __future__ import annotations

import bisect

import torch

from nimbus_amd.kernels.paged_attention import decode_workspace_bytes, new_decode_workspace
from nimbus_amd.model.attention import AttentionBackend, AttnMetadata

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
