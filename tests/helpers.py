"""Shared test helpers: seeded paged inputs (the reference's own generators,
tests/test_kernels.py:11-30 of Nimbus, restated) and the tolerance check."""

from __future__ import annotations

import random

import numpy as np
import torch

# Output tolerance of the hot path: |got - ref| <= ATOL + RTOL * |ref|
# (fp16/bf16 outputs, fp32 accumulation).
ATOL = 2e-3
RTOL = 1e-2


def scattered_cache(num_blocks, block_size, kv, d, seed=0, dtype=torch.float16, device="cpu"):
    g = torch.Generator(device=device).manual_seed(seed)
    k = torch.randn(num_blocks, block_size, kv, d, generator=g, device=device, dtype=torch.float32).to(dtype)
    v = torch.randn(num_blocks, block_size, kv, d, generator=g, device=device, dtype=torch.float32).to(dtype)
    return k, v


def random_tables(ctx_lens, block_size, num_blocks, seed=0, device="cpu"):
    """Consecutive slices of a seeded permutation of the pool, zero padded."""
    rng = random.Random(seed)
    perm = rng.sample(range(num_blocks), num_blocks)
    tables, i = [], 0
    for c in ctx_lens:
        nb = (c + block_size - 1) // block_size
        tables.append(perm[i:i + nb])
        i += nb
    width = max(len(t) for t in tables)
    bt = torch.zeros(len(tables), width, dtype=torch.int32)
    for r, t in enumerate(tables):
        bt[r, :len(t)] = torch.tensor(t, dtype=torch.int32)
    return bt.to(device)


def query_starts(q_lens):
    qs = [0]
    for n in q_lens:
        qs.append(qs[-1] + n)
    return qs


def max_violation(got, want, atol=ATOL, rtol=RTOL) -> float:
    """max over elements of |got - want| - (atol + rtol |want|); <= 0 passes."""
    g = torch.as_tensor(np.asarray(got, dtype=np.float64)) if not torch.is_tensor(got) else got.double().cpu()
    w = torch.as_tensor(np.asarray(want, dtype=np.float64)) if not torch.is_tensor(want) else want.double().cpu()
    return float(((g - w).abs() - (atol + rtol * w.abs())).max())


def assert_within(got, want, atol=ATOL, rtol=RTOL, what=""):
    viol = max_violation(got, want, atol, rtol)
    g = got.double().cpu() if torch.is_tensor(got) else torch.as_tensor(np.asarray(got, dtype=np.float64))
    w = want.double().cpu() if torch.is_tensor(want) else torch.as_tensor(np.asarray(want, dtype=np.float64))
    assert torch.isfinite(g).all(), f"{what}: non-finite output"
    assert viol <= 0, f"{what}: max-abs {float((g - w).abs().max()):.3e} exceeds {atol} + {rtol}*|ref| by {viol:.3e}"
