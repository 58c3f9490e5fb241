"""Flattening a scheduled batch into one forward pass.

Mirrors nimbus/runner.py:1-96 (StepInput, prepare): prefill sequences first,
then one-token decodes, each token's slot = block_table[p // bs] * bs +
p % bs, and the host copies of the prefill offsets and context lengths the
backend needs. `Sequence` here carries only what prepare and the decode
graphs read (nimbus/sequence.py:34-90's token_ids, num_computed,
block_table, output_ids); the reference's own Sequence objects work as well.
"""

from __future__ import annotations

from dataclasses import dataclass, field

import torch

from nimbus_amd.model.attention import AttnMetadata


@dataclass
class Sequence:
    seq_id: int
    prompt_ids: list[int]
    block_table: list[int] = field(default_factory=list)
    num_computed: int = 0

    def __post_init__(self):
        if not self.prompt_ids:
            raise ValueError("empty prompt")
        self.token_ids: list[int] = list(self.prompt_ids)
        self.output_ids: list[int] = []

    def __len__(self) -> int:
        return len(self.token_ids)

    def append(self, token: int) -> None:
        self.output_ids.append(token)
        self.token_ids.append(token)


@dataclass
class StepInput:
    input_ids: torch.Tensor  # [T]
    positions: torch.Tensor  # [T]
    meta: AttnMetadata
    sample_rows: torch.Tensor  # rows whose logits are sampled (sequences that finish their pending tokens)
    sample_seqs: list


def _pad_tables(tables: list[list[int]], device) -> torch.Tensor:
    width = max((len(t) for t in tables), default=1) or 1
    out = torch.zeros((len(tables), width), dtype=torch.int32)
    for i, t in enumerate(tables):
        if t:
            out[i, :len(t)] = torch.tensor(t, dtype=torch.int32)
    return out.to(device, non_blocking=True)


def prepare(batch: list[tuple[object, int]], block_size: int, device) -> StepInput:
    """batch: (sequence, tokens to feed) pairs, prefills first
    (nimbus/runner.py:33-96). A sequence feeding one token that completes
    its pending work (and has a cached prefix) is a decode; anything else is
    a prefill, possibly continuing a cached prefix."""
    ids: list[int] = []
    pos: list[int] = []
    slots: list[int] = []
    pf_start, pf_ctx, pf_tables = [0], [], []
    dc_ctx, dc_tables = [], []
    sample_rows, sample_seqs = [], []
    seen_decode = False
    for seq, n in batch:
        start = seq.num_computed
        end = start + n
        if end > len(seq):
            raise ValueError(f"sequence {seq.seq_id} cannot feed {n} tokens")
        bt = seq.block_table
        if len(bt) * block_size < end:
            raise ValueError(f"sequence {seq.seq_id} has too few blocks for {end} tokens")
        ids.extend(seq.token_ids[start:end])
        pos.extend(range(start, end))
        slots.extend(bt[p // block_size] * block_size + p % block_size for p in range(start, end))
        if n == 1 and end == len(seq) and start > 0:
            seen_decode = True
            dc_ctx.append(end)
            dc_tables.append(bt)
        else:
            if seen_decode:
                raise ValueError("prefill sequences must come before decodes")
            pf_start.append(pf_start[-1] + n)
            pf_ctx.append(end)
            pf_tables.append(bt)
        if end == len(seq):
            sample_rows.append(len(ids) - 1)
            sample_seqs.append(seq)

    def dev(x, dt=torch.int32):
        return torch.tensor(x, dtype=dt).to(device, non_blocking=True)

    meta = AttnMetadata(
        slot_mapping=dev(slots, torch.int64), num_prefill_tokens=pf_start[-1],
        prefill_query_start=dev(pf_start), prefill_context_lens=dev(pf_ctx),
        prefill_block_tables=_pad_tables(pf_tables, device), decode_context_lens=dev(dc_ctx),
        decode_block_tables=_pad_tables(dc_tables, device), max_decode_context=max(dc_ctx, default=0),
        prefill_query_start_host=pf_start, prefill_context_lens_host=pf_ctx)
    return StepInput(input_ids=dev(ids, torch.int64), positions=dev(pos, torch.int64), meta=meta,
                     sample_rows=dev(sample_rows, torch.int64), sample_seqs=sample_seqs)
