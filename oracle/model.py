"""CPU restatement of Nimbus's Llama forward (the model-level test oracle).

TEST INFRASTRUCTURE ONLY: imported by tests/, never by the product package.

Follows nimbus/model/llama.py op for op, in float32 on the CPU, over the
oracle's own attention, cache write and norms (oracle/reference.py):

  rope_inv_freq / rope_tables   llama.py:21-47
  rotate                        llama.py:49-58 (x cos + rotate_half(x) sin)
  forward                       llama.py:88-153 (embed, pre-norm blocks with
                                the residual add fused into the next norm,
                                fused qkv and gate_up projections, final norm)
  logits                        llama.py:155-157

`weights` is a state dict with the module names of LlamaModel (fp32 CPU
tensors); `cfg` any object with ModelConfig's fields.

Pinned by tests/test_oracle_model.py against HuggingFace transformers'
LlamaForCausalLM on the same weights (the check nimbus's own
tests/test_model.py makes), for plain and Llama 3.1-scaled RoPE.
"""

from __future__ import annotations

import math

import torch
import torch.nn.functional as F

from oracle import reference


def rope_inv_freq(cfg) -> torch.Tensor:
    d = cfg.head_dim
    inv = 1.0 / (cfg.rope_theta ** (torch.arange(0, d, 2, dtype=torch.int64).float() / d))
    sc = cfg.rope_scaling
    if sc is None:
        return inv
    wavelen = 2 * math.pi / inv
    low_wl = sc.original_max_position / sc.low_freq_factor
    high_wl = sc.original_max_position / sc.high_freq_factor
    scaled = torch.where(wavelen > low_wl, inv / sc.factor, inv)
    smooth = (sc.original_max_position / wavelen - sc.low_freq_factor) / (sc.high_freq_factor - sc.low_freq_factor)
    smoothed = (1 - smooth) * scaled / sc.factor + smooth * scaled
    medium = ~(wavelen < high_wl) & ~(wavelen > low_wl)
    return torch.where(medium, smoothed, scaled)


def rope_tables(cfg, max_position: int):
    freqs = torch.arange(max_position, dtype=torch.float32)[:, None] * rope_inv_freq(cfg)[None, :]
    emb = torch.cat([freqs, freqs], dim=-1)
    return emb.cos(), emb.sin()


def rotate(x, cos, sin):
    """x [T, heads, D]; cos / sin [T, D] (already gathered by position)."""
    h = x.shape[-1] // 2
    rot = torch.cat([-x[..., h:], x[..., :h]], dim=-1)
    return x * cos[:, None, :] + rot * sin[:, None, :]


def forward(weights, cfg, input_ids, positions, kv_caches, meta, max_position: int):
    """Final hidden states [T, hidden]; writes the new K/V into kv_caches.
    meta: an AttnMetadata with CPU tensors."""
    w = weights
    H, KV, D = cfg.num_heads, cfg.num_kv_heads, cfg.head_dim
    cos_t, sin_t = rope_tables(cfg, max_position)
    cos, sin = cos_t[positions], sin_t[positions]
    x = w["embed_tokens.weight"][input_ids]
    t = x.shape[0]
    residual = None
    p = meta.num_prefill_tokens
    for i, (kc, vc) in enumerate(kv_caches):
        pre = f"layers.{i}."
        if residual is None:
            residual = x
            h = reference.rms_norm(x, w[pre + "input_layernorm.weight"], cfg.rms_norm_eps)
        else:
            h, residual = reference.add_rms_norm(x, residual, w[pre + "input_layernorm.weight"], cfg.rms_norm_eps)
        qkv = h @ w[pre + "self_attn.qkv_proj.weight"].T
        q, k, v = qkv.split([H * D, KV * D, KV * D], dim=-1)
        q, k = rotate(q.view(t, H, D), cos, sin), rotate(k.reshape(t, KV, D), cos, sin)
        v = v.reshape(t, KV, D)
        reference.write_kv(k, v, kc, vc, meta.slot_mapping)
        o = torch.empty(t, H, D)
        scale = D ** -0.5
        if p:
            o[:p] = reference.paged_prefill_attention(
                q[:p], kc, vc, meta.prefill_query_start, meta.prefill_context_lens, meta.prefill_block_tables,
                scale, meta.prefill_query_start_host, meta.prefill_context_lens_host)
        if t > p:
            o[p:] = reference.paged_decode_attention(q[p:], kc, vc, meta.decode_context_lens,
                                                     meta.decode_block_tables, meta.max_decode_context, scale)
        h = o.view(t, H * D) @ w[pre + "self_attn.o_proj.weight"].T
        h, residual = reference.add_rms_norm(h, residual, w[pre + "post_attention_layernorm.weight"],
                                             cfg.rms_norm_eps)
        gate, up = (h @ w[pre + "mlp.gate_up_proj.weight"].T).split(cfg.intermediate_size, dim=-1)
        x = (F.silu(gate) * up) @ w[pre + "mlp.down_proj.weight"].T
    x, _ = reference.add_rms_norm(x, residual, w["norm.weight"], cfg.rms_norm_eps)
    return x


def logits(weights, hidden):
    return (hidden @ weights["lm_head.weight"].T).float()
