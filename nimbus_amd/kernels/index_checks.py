"""Opt-in host-side checks of the index inputs (slots, block tables).

The kernels never fault on a bad index: a slot outside the cache is skipped
by the slot write, and a page id outside the pool reads page 0. The
reference's torch path (index_copy_ and cache[table] gathers,
nimbus/kernels/reference.py:14-34) raises instead. With NIMBUS_CHECK_INDICES=1
in the environment (or set_enabled(True)) the Python entry points check their
index inputs before launch and raise IndexError, as the reference would.
The check reads the indices back to the host (a device sync), so it is off by
default and skipped while a stream is being captured into a graph.
"""

from __future__ import annotations

import os

import torch

_enabled = os.environ.get("NIMBUS_CHECK_INDICES", "0") not in ("", "0")


def set_enabled(on: bool) -> None:
    global _enabled
    _enabled = bool(on)


def enabled() -> bool:
    """True when checks are on and the current stream is not capturing."""
    if not _enabled:
        return False
    return not (torch.cuda.is_available() and torch.cuda.is_current_stream_capturing())


def check_slots(slot_mapping: torch.Tensor, num_slots: int) -> None:
    """Every slot must address a row of the flat [num_blocks * block_size] cache."""
    s = slot_mapping.cpu()
    if s.numel() and (int(s.min()) < 0 or int(s.max()) >= num_slots):
        bad = int(((s < 0) | (s >= num_slots)).nonzero()[0, 0])
        raise IndexError(f"slot_mapping[{bad}] = {int(s[bad])} is outside the cache's {num_slots} slots")


def check_tables(block_tables: torch.Tensor, context_lens: torch.Tensor, num_blocks: int, block_size: int) -> None:
    """Each row's first ceil(context / block_size) entries must be page ids of
    the pool, and the table must be wide enough for them. Entries past a row's
    context are padding and are not read, so they are not checked."""
    bt = block_tables.cpu().long()
    ctx = context_lens.cpu().long()
    if ctx.numel() and int(ctx.min()) < 0:
        raise IndexError("negative context length")
    pages = (ctx + block_size - 1) // block_size
    if pages.numel() and int(pages.max()) > bt.shape[1]:
        row = int(torch.argmax(pages))
        raise IndexError(f"row {row} needs {int(pages[row])} pages but the block table is {bt.shape[1]} wide")
    used = torch.arange(bt.shape[1])[None, :] < pages[:, None]
    bad = used & ((bt < 0) | (bt >= num_blocks))
    if bad.any():
        r, c = (int(x) for x in bad.nonzero()[0])
        raise IndexError(f"block_tables[{r}, {c}] = {int(bt[r, c])} is outside the pool of {num_blocks} blocks")
