"""Writes the known-answer fixtures in tests/golden/*.npz.

    python tests/golden/make_golden.py

Inputs are seeded fp16/bf16 tensors stored as raw 16-bit patterns (int16);
expected outputs come from oracle/closed_form.py in float64, so the fixtures
do not depend on torch's SDPA. Nothing from Nimbus itself is imported or run
(it has no golden vectors of its own; its kernel tests compare against its
PyTorch oracle on seeded inputs, tests/test_kernels.py:33-75).

Shapes follow the reference tests and the two model shapes of the benchmark
configurations (TinyLlama H=32/KV=4/D=64 fp16, Llama-3-8B H=32/KV=8/D=128
bf16), kept small: pools hold just the pages the tables use.
"""

from __future__ import annotations

import os
import sys

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))

from oracle import closed_form  # noqa: E402

BS = 16
DTYPES = {"float16": torch.float16, "bfloat16": torch.bfloat16}


def _bits(t: torch.Tensor) -> np.ndarray:
    return t.contiguous().view(torch.int16).numpy()


def _tables(ctx_lens, pool, rng):
    perm = rng.permutation(pool)
    tables, i = [], 0
    for c in ctx_lens:
        n = -(-c // BS)
        tables.append(perm[i:i + n])
        i += n
    width = max(len(t) for t in tables)
    bt = np.zeros((len(ctx_lens), width), dtype=np.int32)
    for r, t in enumerate(tables):
        bt[r, :len(t)] = t
    return bt


def _cache(pool, kv, d, dtype, gen, scale=1.0):
    shape = (pool, BS, kv, d)
    return ((torch.randn(shape, generator=gen) * scale).to(dtype), (torch.randn(shape, generator=gen) * scale).to(dtype))


def decode_case(name, heads, kv, d, dtype, ctx_lens, seed, kv_scale=1.0):
    rng = np.random.default_rng(seed)
    pool = sum(-(-c // BS) for c in ctx_lens) + 3
    gen = torch.Generator().manual_seed(seed)
    k, v = _cache(pool, kv, d, DTYPES[dtype], gen, kv_scale)
    q = torch.randn(len(ctx_lens), heads, d, generator=gen).to(DTYPES[dtype])
    bt = _tables(ctx_lens, pool, rng)
    ctx = np.asarray(ctx_lens, dtype=np.int32)
    scale = d ** -0.5
    out = closed_form.decode(q, k, v, ctx, bt, scale).astype(np.float32)
    np.savez_compressed(os.path.join(HERE, f"{name}.npz"), kind="decode", dtype=dtype, q=_bits(q), k_cache=_bits(k),
             v_cache=_bits(v), context_lens=ctx, block_tables=bt, scale=np.float64(scale), out=out)


def prefill_case(name, heads, kv, d, dtype, seqs, seed):
    rng = np.random.default_rng(seed)
    ctx_lens = [c for _, c in seqs]
    pool = sum(-(-c // BS) for c in ctx_lens) + 3
    gen = torch.Generator().manual_seed(seed)
    k, v = _cache(pool, kv, d, DTYPES[dtype], gen)
    qs = [0]
    for ql, _ in seqs:
        qs.append(qs[-1] + ql)
    q = torch.randn(qs[-1], heads, d, generator=gen).to(DTYPES[dtype])
    bt = _tables(ctx_lens, pool, rng)
    scale = d ** -0.5
    out = closed_form.prefill(q, k, v, qs, ctx_lens, bt, scale).astype(np.float32)
    np.savez_compressed(os.path.join(HERE, f"{name}.npz"), kind="prefill", dtype=dtype, q=_bits(q), k_cache=_bits(k),
             v_cache=_bits(v), query_start=np.asarray(qs, dtype=np.int32),
             context_lens=np.asarray(ctx_lens, dtype=np.int32), block_tables=bt, scale=np.float64(scale), out=out)


def write_kv_case(name, kv, d, dtype, n_tokens, pool, seed):
    gen = torch.Generator().manual_seed(seed)
    k_cache, v_cache = _cache(pool, kv, d, DTYPES[dtype], gen)
    k = torch.randn(n_tokens, kv, d, generator=gen).to(DTYPES[dtype])
    v = torch.randn(n_tokens, kv, d, generator=gen).to(DTYPES[dtype])
    slots = torch.randperm(pool * BS, generator=gen)[:n_tokens].to(torch.int64)
    kc, vc = closed_form.write_kv(_bits(k), _bits(v), _bits(k_cache), _bits(v_cache), slots)
    np.savez_compressed(os.path.join(HERE, f"{name}.npz"), kind="write_kv", dtype=dtype, k=_bits(k), v=_bits(v),
             k_cache=_bits(k_cache), v_cache=_bits(v_cache), slot_mapping=slots.numpy(), k_cache_out=kc,
             v_cache_out=vc)


def main():
    decode_case("decode_tinyllama_fp16", 32, 4, 64, "float16", [1, 17, 64, 100, 255], seed=10)
    decode_case("decode_llama3_bf16", 32, 8, 128, "bfloat16", [1, 33, 100], seed=11, kv_scale=0.5)
    decode_case("decode_split_fp16", 8, 2, 64, "float16", [1100, 520, 33], seed=12)
    prefill_case("prefill_tinyllama_fp16", 32, 4, 64, "float16", [(5, 5), (64, 64), (3, 40), (9, 70)], seed=13)
    prefill_case("prefill_llama3_bf16", 32, 8, 128, "bfloat16", [(1, 1), (20, 60)], seed=14)
    write_kv_case("write_kv_bf16", 8, 128, "bfloat16", 37, 3, seed=15)
    write_kv_case("write_kv_fp16", 4, 64, "float16", 50, 8, seed=16)


if __name__ == "__main__":
    main()
