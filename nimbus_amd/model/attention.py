"""Attention over a paged KV cache: the drop-in seam for Nimbus's model.

Mirrors nimbus/model/attention.py:24-95. A forward pass processes one flat
batch: the first `num_prefill_tokens` tokens belong to prefill sequences
(several tokens each, possibly continuing a cached prefix), the rest are
decode tokens, one per sequence (nimbus/runner.py:33-96 builds it). Every
token's K/V is first written into the cache at slot_mapping[t]; attention
then reads each sequence's K/V back through its block table.

The backend here runs the HIP kernels of libnimbus_attn.so and nothing else:
there is no PyTorch or CPU fallback inside it.
"""

from __future__ import annotations

from dataclasses import dataclass

import torch

from nimbus_amd.kernels import cache_ops, paged_attention, prefill_attention


@dataclass
class AttnMetadata:
    """Field for field the reference's AttnMetadata (model/attention.py:24-50)."""

    slot_mapping: torch.Tensor  # [T] int64
    num_prefill_tokens: int
    # Prefill sequences (P of them)
    prefill_query_start: torch.Tensor  # [P+1] int32, offsets into the flat batch
    prefill_context_lens: torch.Tensor  # [P] int32, cached + new tokens
    prefill_block_tables: torch.Tensor  # [P, max_blocks] int32
    # Decode sequences (D of them)
    decode_context_lens: torch.Tensor  # [D] int32, including the new token
    decode_block_tables: torch.Tensor  # [D, max_blocks] int32
    max_decode_context: int
    # Host copies, so nothing on the host waits for the GPU
    prefill_query_start_host: list[int]
    prefill_context_lens_host: list[int]
    # Tile table, built once per step and reused by every layer (here it may
    # also be a prefill_attention.PrefillPieces plan)
    prefill_programs: tuple[torch.Tensor, torch.Tensor] | None = None
    # Fixed decode launch grid of the reference's graph capture (accepted, unused:
    # the grid here is pinned by max_decode_context)
    decode_partitions: int | None = None
    # Not in the reference: which prefill kernel serves this step ("tile" or
    # "verify", see prefill_attention.verify_queries), decided once per step
    # by the backend like the tile table.
    prefill_kernel: str | None = None

    @property
    def num_prefills(self) -> int:
        return len(self.prefill_context_lens_host)

    @property
    def num_decodes(self) -> int:
        return int(self.decode_context_lens.shape[0])


class AttentionBackend:
    """HIP paged attention behind the reference's backend interface
    (model/attention.py:53-95).

    The reference chooses between Triton and its PyTorch oracle with
    `use_triton`; this backend is the GPU path only, so `use_hip=False` is
    rejected rather than silently served by a CPU implementation.
    """

    def __init__(self, use_hip: bool = True, decode_workspace: torch.Tensor | None = None):
        """decode_workspace (not in the reference): a workspace (page prefix
        sum + split partials, see paged_decode_attention) for this backend's
        decode and verify-form prefill calls instead of the per-stream cached
        one; a graph capture passes its own, sized for its largest batch."""
        if not use_hip:
            raise ValueError("nimbus_amd's AttentionBackend is the HIP path only; use Nimbus's reference "
                             "backend for CPU execution")
        self.use_hip = True
        self.decode_workspace = decode_workspace
        self._decode = paged_attention.paged_decode_attention
        self._prefill = prefill_attention.paged_prefill_attention
        self._build_programs = prefill_attention.build_programs

    def _prefill_workspace(self, meta: AttnMetadata, q: torch.Tensor, block_size: int) -> torch.Tensor | None:
        """This backend's workspace for a prefill call in the verify form
        (the decode kernels) when it holds what the call needs, else None: the
        call then takes the per-stream cached workspace (a PrefillPieces plan
        takes the pieces' own cached one)."""
        ws = self.decode_workspace
        if ws is None or meta.prefill_kernel != "verify":
            return None
        h, d = q.shape[1], q.shape[2]
        need = paged_attention.verify_workspace_bytes(meta.num_prefills, meta.prefill_query_start_host[1], h, d,
                                                      meta.prefill_block_tables.shape[1] * block_size)
        return ws if ws.numel() * ws.element_size() >= need else None

    def forward(
        self,
        q: torch.Tensor,  # [T, H, D]
        k: torch.Tensor,  # [T, KV, D]
        v: torch.Tensor,
        k_cache: torch.Tensor,  # [num_blocks, block_size, KV, D]
        v_cache: torch.Tensor,
        meta: AttnMetadata,
        scale: float,
        kv_written: bool = False,
    ) -> torch.Tensor:
        """write_kv, then prefill on q[:p], then decode on q[p:] (the order of
        model/attention.py:78-94). Both kernels write straight into their
        slice of the output instead of copying a temporary into it.
        kv_written (not in the reference): the caller has already written k
        and v into the cache slots (cache_ops.rope_write_kv), so the write
        is skipped."""
        if not kv_written:
            cache_ops.write_kv(k, v, k_cache, v_cache, meta.slot_mapping)
        out = torch.empty_like(q)
        p = meta.num_prefill_tokens
        if p:
            if meta.prefill_kernel is None:
                nq = prefill_attention.verify_queries(meta.prefill_query_start_host, q.shape[1], k_cache.shape[2])
                meta.prefill_kernel = "verify" if nq else "tile"
            if meta.prefill_programs is None and meta.prefill_kernel == "tile":
                # Heavy tiles' key ranges cut into pieces when the tiles alone
                # would not fill the chip, else the cost-ordered tile table
                # (always the table for shapes the general kernel runs).
                pieces = None
                if paged_attention.tuned_shape(k_cache.shape[1], q.shape[2]):
                    pieces = prefill_attention.plan_pieces(meta.prefill_query_start_host,
                                                           meta.prefill_context_lens_host, q.shape[1],
                                                           k_cache.shape[2], q.device)
                meta.prefill_programs = pieces or self._build_programs(meta.prefill_query_start_host, q.device,
                                                                       meta.prefill_context_lens_host)
            self._prefill(
                q[:p], k_cache, v_cache, meta.prefill_query_start, meta.prefill_context_lens,
                meta.prefill_block_tables, scale, meta.prefill_query_start_host,
                meta.prefill_context_lens_host, meta.prefill_programs, out=out[:p],
                workspace=self._prefill_workspace(meta, q, k_cache.shape[1]), kernel=meta.prefill_kernel,
            )
        if meta.num_decodes:
            self._decode(
                q[p:], k_cache, v_cache, meta.decode_context_lens, meta.decode_block_tables,
                meta.max_decode_context, scale, num_partitions=meta.decode_partitions, out=out[p:],
                workspace=self.decode_workspace,
            )
        return out
