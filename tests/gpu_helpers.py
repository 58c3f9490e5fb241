"""Helpers for the GPU parity tests: run the CPU oracle on exactly the pages
a batch uses (so multi-GB pools never leave the GPU) and print the case
before each GPU step.

The oracle runs the reference's ops (nimbus/kernels/reference.py:14-96) on
the same inputs upcast exactly to float32 by default: that is the reference
attention with fp32 accumulation, the bar the kernels are held to. torch's
CPU scaled_dot_product_attention in bfloat16 keeps bf16 intermediates and
lands up to ~8.6e-3 from the float64 answer by itself (more than the 2e-3 +
1e-2|ref| tolerance), so an in-dtype CPU oracle cannot serve as the bf16
checker; `in_dtype=True` runs it anyway, for the fp16 reference-matrix tests
that mirror Nimbus's own.
"""

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
    bs = k_cache.shape[1]
    for b, c in enumerate(ctx_lens_host):
        n = -(-int(c) // bs)
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


def _prec(x, in_dtype):
    return x if in_dtype else x.float()


def oracle_decode(q, k_cache, v_cache, ctx_lens_host, block_tables, scale, batched=False, in_dtype=False):
    kc, vc, tables = compact(k_cache, v_cache, block_tables, ctx_lens_host)
    qc, kc, vc = (_prec(x, in_dtype) for x in (q.cpu(), kc, vc))
    if batched:
        ctx = torch.tensor(ctx_lens_host, dtype=torch.int32)
        return reference.paged_decode_attention(qc, kc, vc, ctx, tables, max(ctx_lens_host), scale)
    return reference.decode_attention_rows(qc, kc, vc, list(ctx_lens_host), tables, scale)


def oracle_prefill(q, k_cache, v_cache, qs_host, ctx_host, block_tables, scale, in_dtype=False):
    kc, vc, tables = compact(k_cache, v_cache, block_tables, ctx_host)
    qc, kc, vc = (_prec(x, in_dtype) for x in (q.cpu(), kc, vc))
    return reference.paged_prefill_attention(qc, kc, vc, torch.tensor(qs_host, dtype=torch.int32),
                                             torch.tensor(ctx_host, dtype=torch.int32), tables, scale, qs_host,
                                             ctx_host)
