"""float64 NumPy brute force of the paged-attention mathematics (and of the
RMSNorm and the int8 weight-only product beside it).

TEST INFRASTRUCTURE ONLY (see oracle/__init__.py).

Written from the definition, not from torch: for every sequence and query
head h, with kv head h // (H // KV),

    o = sum_t softmax_t(scale * q . k_t) v_t

over the keys the query may see. Pages are resolved one token at a time
(token t lives in block_table[t // bs], row t % bs), which is the slot rule
of nimbus/runner.py:61. This pins oracle/reference.py, which goes through
torch's gather and SDPA instead.
"""

from __future__ import annotations

import numpy as np


def _np(x):
    if hasattr(x, "detach"):
        x = x.detach().cpu()
        if str(x.dtype) in ("torch.bfloat16", "torch.float16"):
            x = x.float()
        x = x.numpy()
    return np.asarray(x)


def token_rows(cache, table, n_tokens):
    """[n_tokens, KV, D] float64: token t from page table[t // bs], row t % bs."""
    cache = _np(cache)
    table = _np(table)
    bs = cache.shape[1]
    t = np.arange(n_tokens)
    return cache[table[t // bs].astype(np.int64), t % bs].astype(np.float64)


def attend(q_rows, keys, values, scale, visible):
    """q_rows [M, H, D]; keys/values [S, KV, D]; visible [M, S] bool.

    Returns [M, H, D] float64. Rows with no visible key give 0 (the prefill
    kernel's l == 0 guard, prefill_attention.py:76); the reference's domain
    never produces such rows.
    """
    m, h, d = q_rows.shape
    kv = keys.shape[1]
    g = h // kv
    out = np.zeros((m, h, d), dtype=np.float64)
    for head in range(h):
        kh = head // g
        s = (q_rows[:, head, :] @ keys[:, kh, :].T) * scale  # [M, S]
        s = np.where(visible, s, -np.inf)
        mx = s.max(axis=1, keepdims=True)
        mx = np.where(np.isfinite(mx), mx, 0.0)
        p = np.exp(s - mx)
        den = p.sum(axis=1, keepdims=True)
        out[:, head, :] = (p @ values[:, kh, :]) / np.where(den == 0, 1.0, den)
    return out


def decode(q, k_cache, v_cache, context_lens, block_tables, scale):
    """[B, H, D] float64 decode attention; row b sees tokens 0..ctx_b-1."""
    q = _np(q).astype(np.float64)
    ctx = _np(context_lens).astype(np.int64)
    tables = _np(block_tables)
    out = np.zeros(q.shape, dtype=np.float64)
    for b in range(q.shape[0]):
        c = int(ctx[b])
        keys = token_rows(k_cache, tables[b], c)
        vals = token_rows(v_cache, tables[b], c)
        out[b] = attend(q[b][None], keys, vals, scale, np.ones((1, c), dtype=bool))[0]
    return out


def prefill(q, k_cache, v_cache, query_start_host, context_lens_host, block_tables, scale):
    """[Tp, H, D] float64 causal varlen attention over cached prefixes.

    Query j of sequence i (q_len = qs[i+1]-qs[i], context c) is at absolute
    position c - q_len + j and sees keys 0..c - q_len + j.
    """
    q = _np(q).astype(np.float64)
    tables = _np(block_tables)
    out = np.zeros(q.shape, dtype=np.float64)
    for i, c in enumerate(context_lens_host):
        s, e = query_start_host[i], query_start_host[i + 1]
        q_len = e - s
        keys = token_rows(k_cache, tables[i], c)
        vals = token_rows(v_cache, tables[i], c)
        qpos = c - q_len + np.arange(q_len)
        visible = np.arange(c)[None, :] <= qpos[:, None]
        out[s:e] = attend(q[s:e], keys, vals, scale, visible)
    return out


def write_kv(k, v, k_cache, v_cache, slot_mapping):
    """NumPy scatter: returns new (k_cache, v_cache) arrays with flat slot
    slot_mapping[t] = (block * bs + offset) holding token t's rows."""
    kc = _np(k_cache).copy()
    vc = _np(v_cache).copy()
    nb, bs, kv, d = kc.shape
    slots = _np(slot_mapping).astype(np.int64)
    kc.reshape(nb * bs, kv, d)[slots] = _np(k)
    vc.reshape(nb * bs, kv, d)[slots] = _np(v)
    return kc, vc


def rms_norm(x, weight, eps):
    """float64 RMSNorm from the definition: w * x / sqrt(mean(x^2) + eps), per row."""
    xf = _np(x).astype(np.float64)
    w = _np(weight).astype(np.float64)
    return w * xf / np.sqrt(np.mean(xf * xf, axis=-1, keepdims=True) + eps)


def int8_matmul(x, q, scale):
    """float64 weight-only int8 product from the definition:
    y[i, j] = sum_k x[i, k] q[j, k] * scale[j]."""
    xf = _np(x).astype(np.float64)
    qf = _np(q).astype(np.float64)
    s = _np(scale).astype(np.float64)
    return (xf @ qf.T) * s[None, :]
