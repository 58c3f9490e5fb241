"""CPU restatement of Nimbus's PyTorch reference attention (the test oracle).

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and
bench.py's cpu_baseline leg, never by the product package.

Each function follows one function of the reference, op for op:

  write_kv                nimbus/kernels/reference.py:14-23
  gather_kv               nimbus/kernels/reference.py:26-34
  paged_prefill_attention nimbus/kernels/reference.py:37-68
  paged_decode_attention  nimbus/kernels/reference.py:71-96
  decode_attention_rows   same mathematics as :71-96, one sequence at a time,
                          for batches whose padded gather does not fit in host
                          memory (config 5: ~34 GB batched)
  rms_norm                nimbus/kernels/reference.py:99-104
  add_rms_norm            nimbus/kernels/reference.py:107-112
  quantize_weight         nimbus/quant/int8.py:20-25
  dequantize_weight       nimbus/quant/int8.py:28-29
  int8_matmul             the expected value of nimbus's kernel test
                          (tests/test_quant.py:65): fp32 product of x and the
                          int8 weights, times the fp32 scale, rounded once

Pinned by tests/test_oracle.py against oracle.closed_form (float64 brute force)
and against special cases with textbook answers (ctx=1 gives v_0; one-hot
scores select one row of V; uniform scores average V; the slot write is a
NumPy scatter; a constant row normalises to +-1; the residual add is NumPy's
element-type addition; quantized weights round-trip within half a step and
the int8 product of small integers is exact).
"""

from __future__ import annotations

import torch
import torch.nn.functional as F


def write_kv(k, v, k_cache, v_cache, slot_mapping) -> None:
    """Scatter token rows into the flat slot view of the caches.

    Follows nimbus/kernels/reference.py:14-23: the cache [NB, bs, KV, D] is
    viewed as [NB*bs, KV, D] and row slot_mapping[t] receives k[t] (and v[t]).
    """
    kv_heads, head_dim = k_cache.shape[2], k_cache.shape[3]
    k_cache.view(-1, kv_heads, head_dim).index_copy_(0, slot_mapping, k)
    v_cache.view(-1, kv_heads, head_dim).index_copy_(0, slot_mapping, v)


def gather_kv(cache, block_table, length: int):
    """First `length` tokens of one sequence, [length, KV, D].

    Follows nimbus/kernels/reference.py:26-34: pages block_table[:nb] in table
    order, flattened, truncated to `length`.
    """
    block_size = cache.shape[1]
    n_pages = -(-length // block_size)
    return cache[block_table[:n_pages].long()].flatten(0, 1)[:length]


def paged_prefill_attention(q, k_cache, v_cache, query_start, context_lens, block_tables, scale,
                            query_start_host, context_lens_host, programs=None):
    """Causal attention of each sequence's newest q_len tokens over its cache.

    Follows nimbus/kernels/reference.py:37-68. Query j of a sequence with
    context c sits at absolute position c - q_len + j and sees keys
    0..c - q_len + j. q_len == c uses SDPA's is_causal; otherwise an explicit
    kpos <= qpos mask. `programs` is accepted and unused, as in the reference.
    """
    out = torch.empty_like(q)
    for i, ctx in enumerate(context_lens_host):
        s, e = query_start_host[i], query_start_host[i + 1]
        q_len = e - s
        qi = q[s:e].transpose(0, 1).unsqueeze(0)
        ki = gather_kv(k_cache, block_tables[i], ctx).transpose(0, 1).unsqueeze(0)
        vi = gather_kv(v_cache, block_tables[i], ctx).transpose(0, 1).unsqueeze(0)
        if q_len == ctx:
            o = F.scaled_dot_product_attention(qi, ki, vi, is_causal=True, scale=scale, enable_gqa=True)
        else:
            qpos = torch.arange(ctx - q_len, ctx, device=q.device)[:, None]
            kpos = torch.arange(ctx, device=q.device)[None, :]
            o = F.scaled_dot_product_attention(qi, ki, vi, attn_mask=kpos <= qpos, scale=scale,
                                               enable_gqa=True)
        out[s:e] = o[0].transpose(0, 1)
    return out


def paged_decode_attention(q, k_cache, v_cache, context_lens, block_tables, max_context: int, scale: float):
    """One query per sequence over its first context_lens[b] cached tokens.

    Follows nimbus/kernels/reference.py:71-96: gathers every row's pages up to
    ceil(max_context/bs) into a padded [B, S, KV, D] tensor and masks key
    positions >= context_lens[b].
    """
    batch = q.shape[0]
    block_size = k_cache.shape[1]
    n_pages = -(-max_context // block_size)
    tables = block_tables[:, :n_pages].long()
    k = k_cache[tables].flatten(1, 2)
    v = v_cache[tables].flatten(1, 2)
    span = k.shape[1]
    mask = torch.arange(span, device=q.device)[None, :] < context_lens[:, None]
    o = F.scaled_dot_product_attention(q.unsqueeze(2), k.transpose(1, 2), v.transpose(1, 2),
                                       attn_mask=mask[:, None, None, :], scale=scale, enable_gqa=True)
    return o.view(batch, q.shape[1], q.shape[2])


def decode_attention_rows(q, k_cache, v_cache, context_lens_host, block_tables, scale: float):
    """paged_decode_attention computed one sequence at a time.

    Same mathematics as nimbus/kernels/reference.py:71-96 (each row attends to
    its first ctx tokens, gathered through its block table), but the gather is
    per row, so host memory holds one sequence's K/V at a time instead of the
    padded batch. Used for the long-context configuration and as the CPU
    baseline's bounded sample.
    """
    out = torch.empty_like(q)
    for b, ctx in enumerate(context_lens_host):
        kb = gather_kv(k_cache, block_tables[b], ctx).transpose(0, 1).unsqueeze(0)
        vb = gather_kv(v_cache, block_tables[b], ctx).transpose(0, 1).unsqueeze(0)
        o = F.scaled_dot_product_attention(q[b][None, :, None, :], kb, vb, scale=scale, enable_gqa=True)
        out[b] = o[0, :, 0, :]
    return out


def rms_norm(x, weight, eps: float):
    """HuggingFace LlamaRMSNorm order of operations.

    Follows nimbus/kernels/reference.py:99-104: normalise in float32, cast
    back to x's dtype, then multiply by the weight in that dtype.
    """
    dtype = x.dtype
    xf = x.float()
    xf = xf * torch.rsqrt(xf.pow(2).mean(-1, keepdim=True) + eps)
    return weight * xf.to(dtype)


def add_rms_norm(x, residual, weight, eps: float):
    """residual + x in the model dtype, then rms_norm of it; returns (norm, residual).

    Follows nimbus/kernels/reference.py:107-112.
    """
    residual = residual + x
    return rms_norm(residual, weight, eps), residual


def quantize_weight(w):
    """Symmetric per-output-channel int8 quantization.

    Follows nimbus/quant/int8.py:20-25: scale = max|row| / 127 (rows of
    zeros get 1e-8 / 127), q = clamp(round(w / scale), -127, 127); the scale
    is returned in w's dtype.
    """
    wf = w.float()
    scale = wf.abs().amax(dim=1).clamp_min(1e-8) / 127.0
    q = torch.round(wf / scale[:, None]).clamp_(-127, 127).to(torch.int8)
    return q, scale.to(w.dtype)


def dequantize_weight(q, scale):
    """nimbus/quant/int8.py:28-29: q in the scale's dtype times the row scale."""
    return q.to(scale.dtype) * scale[:, None]


def int8_matmul(x, q, scale):
    """y = dtype(fp32(x @ q^T) * fp32(scale)): the value nimbus's own kernel
    test expects (tests/test_quant.py:65), in x's dtype."""
    return (x.float() @ q.float().T * scale.float()).to(x.dtype)
