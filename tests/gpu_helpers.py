"""Helpers for the GPU parity tests: run the CPU oracle on exactly the pages
a batch uses (so multi-GB pools never leave the GPU) and print the case
before each GPU step."""

from __future__ import annotations

import sys

import torch

from oracle import reference


def announce(msg: str) -> None:
    print(f"[gpu-case] {msg}", flush=True)
    sys.stdout.flush()


def compact(k_cache, v_cache, block_tables, ctx_lens_host):
    """Copies the pages the rows use to small CPU caches; returns
    (k, v, tables) with tables renumbered into them (zero padded)."""
    rows, lens = [], []
    for b, c in enumerate(ctx_lens_host):
        n = -(-int(c) // 16)
        rows.append(block_tables[b, :n].long())
        lens.append(n)
    used = torch.cat(rows) if rows else torch.zeros(0, dtype=torch.long, device=block_tables.device)
    kc = k_cache[used].cpu()
    vc = v_cache[used].cpu()
    width = max(lens) if lens else 1
    tables = torch.zeros(len(lens), max(width, 1), dtype=torch.int32)
    off = 0
    for b, n in enumerate(lens):
        tables[b, :n] = torch.arange(off, off + n, dtype=torch.int32)
        off += n
    return kc, vc, tables


def oracle_decode(q, k_cache, v_cache, ctx_lens_host, block_tables, scale, batched=False):
    kc, vc, tables = compact(k_cache, v_cache, block_tables, ctx_lens_host)
    qc = q.cpu()
    if batched:
        ctx = torch.tensor(ctx_lens_host, dtype=torch.int32)
        return reference.paged_decode_attention(qc, kc, vc, ctx, tables, max(ctx_lens_host), scale)
    return reference.decode_attention_rows(qc, kc, vc, list(ctx_lens_host), tables, scale)


def oracle_prefill(q, k_cache, v_cache, qs_host, ctx_host, block_tables, scale):
    kc, vc, tables = compact(k_cache, v_cache, block_tables, ctx_host)
    return reference.paged_prefill_attention(q.cpu(), kc, vc, torch.tensor(qs_host, dtype=torch.int32),
                                             torch.tensor(ctx_host, dtype=torch.int32), tables, scale, qs_host,
                                             ctx_host)
