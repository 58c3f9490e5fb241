"""CPU: the model-level oracle against HuggingFace transformers' Llama.

nimbus's tests/test_model.py checks its model against HF's
LlamaForCausalLM; here the same check pins oracle/model.py (the CPU fp32
restatement the GPU model is tested against): identical weights, one
sequence, HF without a cache vs the oracle through the paged cache, plain
and Llama 3.1-scaled RoPE, then a decode step over the cached prefix.
Also: the RoPE frequency rule against HF's rope initialisation, and a
planted mistake (rotating the wrong halves) that the comparison catches.
"""

from __future__ import annotations

import pytest
import torch

from nimbus_amd.model.attention import AttnMetadata
from nimbus_amd.model.config import ModelConfig, RopeScaling
from oracle import model as omodel

transformers = pytest.importorskip("transformers")


def _cfg(scaling=None):
    return ModelConfig(vocab_size=300, hidden_size=128, intermediate_size=256, num_layers=2, num_heads=4,
                       num_kv_heads=2, head_dim=32, rms_norm_eps=1e-5, rope_theta=10000.0, max_position=256,
                       rope_scaling=scaling)


def _weights(cfg, seed=0):
    g = torch.Generator().manual_seed(seed)
    H, KV, D, hid, inter = cfg.num_heads, cfg.num_kv_heads, cfg.head_dim, cfg.hidden_size, cfg.intermediate_size
    r = lambda *s: torch.randn(*s, generator=g) * 0.05  # noqa: E731
    w = {"embed_tokens.weight": r(cfg.vocab_size, hid), "norm.weight": 1 + r(hid),
         "lm_head.weight": r(cfg.vocab_size, hid)}
    for i in range(cfg.num_layers):
        p = f"layers.{i}."
        w[p + "input_layernorm.weight"] = 1 + r(hid)
        w[p + "post_attention_layernorm.weight"] = 1 + r(hid)
        w[p + "self_attn.qkv_proj.weight"] = r((H + 2 * KV) * D, hid)
        w[p + "self_attn.o_proj.weight"] = r(hid, H * D)
        w[p + "mlp.gate_up_proj.weight"] = r(2 * inter, hid)
        w[p + "mlp.down_proj.weight"] = r(hid, inter)
    return w


def _hf(cfg, w):
    from transformers import LlamaConfig, LlamaForCausalLM

    rope = None
    if cfg.rope_scaling is not None:
        sc = cfg.rope_scaling
        rope = {"rope_type": "llama3", "factor": sc.factor, "low_freq_factor": sc.low_freq_factor,
                "high_freq_factor": sc.high_freq_factor, "original_max_position_embeddings": sc.original_max_position}
    hc = LlamaConfig(vocab_size=cfg.vocab_size, hidden_size=cfg.hidden_size,
                     intermediate_size=cfg.intermediate_size, num_hidden_layers=cfg.num_layers,
                     num_attention_heads=cfg.num_heads, num_key_value_heads=cfg.num_kv_heads,
                     head_dim=cfg.head_dim, rms_norm_eps=cfg.rms_norm_eps, rope_theta=cfg.rope_theta,
                     max_position_embeddings=cfg.max_position, rope_scaling=rope, tie_word_embeddings=False,
                     attention_bias=False, mlp_bias=False)
    m = LlamaForCausalLM(hc).eval()
    H, KV, D, inter = cfg.num_heads, cfg.num_kv_heads, cfg.head_dim, cfg.intermediate_size
    sd = {"model.embed_tokens.weight": w["embed_tokens.weight"], "model.norm.weight": w["norm.weight"],
          "lm_head.weight": w["lm_head.weight"]}
    for i in range(cfg.num_layers):
        p, hp = f"layers.{i}.", f"model.layers.{i}."
        q, k, v = w[p + "self_attn.qkv_proj.weight"].split([H * D, KV * D, KV * D])
        gate, up = w[p + "mlp.gate_up_proj.weight"].split(inter)
        sd.update({hp + "self_attn.q_proj.weight": q, hp + "self_attn.k_proj.weight": k,
                   hp + "self_attn.v_proj.weight": v, hp + "self_attn.o_proj.weight": w[p + "self_attn.o_proj.weight"],
                   hp + "mlp.gate_proj.weight": gate, hp + "mlp.up_proj.weight": up,
                   hp + "mlp.down_proj.weight": w[p + "mlp.down_proj.weight"],
                   hp + "input_layernorm.weight": w[p + "input_layernorm.weight"],
                   hp + "post_attention_layernorm.weight": w[p + "post_attention_layernorm.weight"]})
    m.load_state_dict(sd)
    return m


def _oracle_run(cfg, w, ids, n_prefill):
    """Prefill ids[:n_prefill] then decode the rest one token at a time through
    the paged cache; returns the logits of every position fed."""
    bs, nb = 16, 8
    table = torch.tensor([[5, 2, 7, 0, 3, 6, 1, 4]], dtype=torch.int32)[:, : -(-len(ids) // bs)]
    caches = [(torch.zeros(nb, bs, cfg.num_kv_heads, cfg.head_dim), torch.zeros(nb, bs, cfg.num_kv_heads,
                                                                                    cfg.head_dim))
              for _ in range(cfg.num_layers)]
    slot = lambda p: int(table[0, p // bs]) * bs + p % bs  # noqa: E731
    empty = torch.zeros(0, dtype=torch.int32)
    meta = AttnMetadata(
        slot_mapping=torch.tensor([slot(p) for p in range(n_prefill)]), num_prefill_tokens=n_prefill,
        prefill_query_start=torch.tensor([0, n_prefill], dtype=torch.int32),
        prefill_context_lens=torch.tensor([n_prefill], dtype=torch.int32), prefill_block_tables=table,
        decode_context_lens=empty, decode_block_tables=empty.view(0, 1), max_decode_context=0,
        prefill_query_start_host=[0, n_prefill], prefill_context_lens_host=[n_prefill])
    out = [omodel.logits(w, omodel.forward(w, cfg, torch.tensor(ids[:n_prefill]), torch.arange(n_prefill), caches,
                                           meta, cfg.max_position))]
    for p in range(n_prefill, len(ids)):
        meta = AttnMetadata(
            slot_mapping=torch.tensor([slot(p)]), num_prefill_tokens=0,
            prefill_query_start=torch.zeros(1, dtype=torch.int32), prefill_context_lens=empty,
            prefill_block_tables=empty.view(0, 1), decode_context_lens=torch.tensor([p + 1], dtype=torch.int32),
            decode_block_tables=table, max_decode_context=p + 1, prefill_query_start_host=[0],
            prefill_context_lens_host=[])
        out.append(omodel.logits(w, omodel.forward(w, cfg, torch.tensor([ids[p]]), torch.tensor([p]), caches, meta,
                                                   cfg.max_position)))
    return torch.cat(out)


@pytest.mark.parametrize("scaling", [None, RopeScaling(8.0, 1.0, 4.0, 64)])
def test_oracle_model_matches_hf_llama(scaling):
    cfg = _cfg(scaling)
    w = _weights(cfg, seed=1)
    ids = [int(i) for i in torch.randint(0, cfg.vocab_size, (90,), generator=torch.Generator().manual_seed(2))]
    with torch.no_grad():
        want = _hf(cfg, w)(torch.tensor([ids])).logits[0]
    got = _oracle_run(cfg, w, ids, 70)  # 70 prefilled across 5 pages, then 20 decodes
    torch.testing.assert_close(got, want, atol=2e-5, rtol=2e-4)


def test_rope_frequencies_match_hf():
    from transformers import LlamaConfig
    from transformers.modeling_rope_utils import ROPE_INIT_FUNCTIONS

    cfg = ModelConfig(vocab_size=10, hidden_size=512, intermediate_size=8, num_layers=1, num_heads=4,
                      num_kv_heads=4, head_dim=128, rms_norm_eps=1e-5, rope_theta=500000.0, max_position=8192,
                      rope_scaling=RopeScaling(8.0, 1.0, 4.0, 8192))
    hc = LlamaConfig(hidden_size=512, num_attention_heads=4, head_dim=128, rope_theta=500000.0,
                     max_position_embeddings=8192,
                     rope_scaling={"rope_type": "llama3", "factor": 8.0, "low_freq_factor": 1.0,
                                   "high_freq_factor": 4.0, "original_max_position_embeddings": 8192})
    want, _ = ROPE_INIT_FUNCTIONS["llama3"](hc, "cpu")
    torch.testing.assert_close(omodel.rope_inv_freq(cfg), want.float(), atol=0, rtol=1e-6)


def test_planted_rope_mistake_is_caught():
    cfg = _cfg()
    w = _weights(cfg, seed=3)
    ids = list(range(3, 40))
    with torch.no_grad():
        want = _hf(cfg, w)(torch.tensor([ids])).logits[0]
    good = omodel.rotate
    try:
        omodel.rotate = lambda x, c, s: x * c[:, None, :] + torch.cat([x[..., :x.shape[-1] // 2],  # noqa: E731
                                                                      -x[..., x.shape[-1] // 2:]], -1) * s[:, None, :]
        bad = _oracle_run(cfg, w, ids, len(ids))
    finally:
        omodel.rotate = good
    assert (bad - want).abs().max() > 1e-2
