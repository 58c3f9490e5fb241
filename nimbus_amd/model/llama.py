"""Llama-family decoder (TinyLlama, Llama 2/3) over a flat, paged batch.

Mirrors nimbus/model/llama.py:1-158 module for module, with the same
parameter names (embed_tokens, layers.i.{input_layernorm, self_attn.qkv_proj,
self_attn.o_proj, post_attention_layernorm, mlp.gate_up_proj,
mlp.down_proj}, norm, lm_head), so a state dict built for Nimbus loads here.
What runs is this build's GPU path: the HIP RMSNorm / fused add + RMSNorm,
the HIP rotary embedding applied in place to the q and k heads of the fused
qkv projection in the same launch that writes the KV cache, the paged
attention backend, the HIP SiLU gate, and the
projections as torch (hipBLASLt) matmuls or, after quant.quantize_model,
the HIP INT8 matmul. Numerics follow the reference's: RoPE tables in fp32
rounded to the model dtype, RMSNorm in fp32, everything else in the model
dtype, logits in fp32.
"""

from __future__ import annotations

import math

import torch
from torch import nn

from nimbus_amd.kernels import cache_ops
from nimbus_amd.kernels.elementwise import rope_, silu_mul
from nimbus_amd.kernels.int8_matmul import SplitPartials
from nimbus_amd.kernels.rmsnorm import add_rms_norm, add_rms_norm_partials, rms_norm
from nimbus_amd.model.attention import AttentionBackend, AttnMetadata
from nimbus_amd.model.config import ModelConfig


def rope_inv_freq(cfg: ModelConfig) -> torch.Tensor:
    """Inverse RoPE frequencies, with Llama 3.1 scaling when configured
    (nimbus/model/llama.py:21-34): wavelengths above
    original_max_position / low_freq_factor are slowed by `factor`, those
    below original_max_position / high_freq_factor kept, the band between
    interpolated."""
    d = cfg.head_dim
    inv = 1.0 / (cfg.rope_theta ** (torch.arange(0, d, 2, dtype=torch.int64).float() / d))
    sc = cfg.rope_scaling
    if sc is None:
        return inv
    wavelen = 2 * math.pi / inv
    low_wl = sc.original_max_position / sc.low_freq_factor
    high_wl = sc.original_max_position / sc.high_freq_factor
    slowed = torch.where(wavelen > low_wl, inv / sc.factor, inv)
    t = (sc.original_max_position / wavelen - sc.low_freq_factor) / (sc.high_freq_factor - sc.low_freq_factor)
    blended = (1 - t) * slowed / sc.factor + t * slowed
    in_band = (wavelen >= high_wl) & (wavelen <= low_wl)
    return torch.where(in_band, blended, slowed)


class Rotary(nn.Module):
    """fp32 cos / sin tables [max_position, head_dim] (angles repeated over
    both halves, nimbus/model/llama.py:37-47)."""

    def __init__(self, cfg: ModelConfig, max_position: int):
        super().__init__()
        inv = rope_inv_freq(cfg)
        ang = torch.arange(max_position, dtype=torch.float32)[:, None] * inv[None, :]
        ang = torch.cat([ang, ang], dim=-1)
        self.register_buffer("cos", ang.cos(), persistent=False)
        self.register_buffer("sin", ang.sin(), persistent=False)
        self.head_dim = cfg.head_dim

    def apply_(self, x: torch.Tensor, heads: int, positions: torch.Tensor) -> torch.Tensor:
        """Rotates the first `heads` heads of every row of x [T, ...] in place."""
        return rope_(x, heads, self.head_dim, positions, self.cos, self.sin)

    def forward(self, q: torch.Tensor, k: torch.Tensor, positions: torch.Tensor):
        """Reference signature (llama.py:49-53): rotated copies of q [T, H, D]
        and k [T, KV, D]."""
        q2 = q.contiguous().clone().view(q.shape[0], -1)
        k2 = k.contiguous().clone().view(k.shape[0], -1)
        self.apply_(q2, q.shape[1], positions)
        self.apply_(k2, k.shape[1], positions)
        return q2.view_as(q), k2.view_as(k)


class RMSNorm(nn.Module):
    """nimbus/model/llama.py:61-77 on the HIP kernel. `fused` is accepted
    for the reference signature; the HIP kernel is what runs."""

    def __init__(self, dim: int, eps: float, fused=None):
        super().__init__()
        self.weight = nn.Parameter(torch.empty(dim))
        self.eps = eps
        del fused

    def forward(self, x, residual: torch.Tensor | None = None):
        if residual is None:
            return rms_norm(x, self.weight, self.eps)
        if isinstance(x, SplitPartials):  # an INT8 projection's output, still in its split-K partials
            return add_rms_norm_partials(x, residual, self.weight, self.eps)
        return add_rms_norm(x, residual, self.weight, self.eps)


class Attention(nn.Module):
    def __init__(self, cfg: ModelConfig, backend: AttentionBackend):
        super().__init__()
        self.h, self.kv, self.d = cfg.num_heads, cfg.num_kv_heads, cfg.head_dim
        self.qkv_proj = nn.Linear(cfg.hidden_size, (self.h + 2 * self.kv) * self.d, bias=False)
        self.o_proj = nn.Linear(self.h * self.d, cfg.hidden_size, bias=False)
        self.scale = self.d ** -0.5
        self.backend = backend

    def forward(self, x, positions, rotary: Rotary, k_cache, v_cache, meta: AttnMetadata, deferred: bool = False):
        """nimbus/model/llama.py:88-98. One launch rotates the q and k heads
        of each qkv row in place and writes the k and v heads into the cache
        (the backend's first step, nimbus/model/attention.py:78), so the
        backend is told the cache already holds them; q goes to it as a
        strided view (no copy). deferred: an INT8 o_proj may return its
        split-K partials for the next norm to fold in."""
        t = x.shape[0]
        hd, kvd = self.h * self.d, self.kv * self.d
        qkv = self.qkv_proj(x)
        cache_ops.rope_write_kv(qkv, self.h, self.kv, self.d, positions, rotary.cos, rotary.sin, k_cache, v_cache,
                                meta.slot_mapping)
        q = qkv[:, :hd].view(t, self.h, self.d)
        k = qkv[:, hd:hd + kvd].view(t, self.kv, self.d)
        v = qkv[:, hd + kvd:].view(t, self.kv, self.d)
        o = self.backend.forward(q, k, v, k_cache, v_cache, meta, self.scale, kv_written=True)
        proj = getattr(self.o_proj, "forward_deferred", None) if deferred else None
        return proj(o.view(t, hd)) if proj is not None else self.o_proj(o.view(t, hd))


class MLP(nn.Module):
    def __init__(self, cfg: ModelConfig):
        super().__init__()
        self.inter = cfg.intermediate_size
        self.gate_up_proj = nn.Linear(cfg.hidden_size, 2 * self.inter, bias=False)
        self.down_proj = nn.Linear(self.inter, cfg.hidden_size, bias=False)

    def forward(self, x, deferred: bool = False):
        # An INT8 gate_up projection runs with the SiLU gate in its epilogue
        # (one launch and no [M, 2I] output; the two steps' bits under the
        # same launch plan).
        fused = getattr(self.gate_up_proj, "forward_silu", None)
        h = fused(x) if fused is not None else None
        if h is None:
            h = silu_mul(self.gate_up_proj(x))
        # deferred: an INT8 down_proj may return its split-K partials for the
        # next norm to fold in
        proj = getattr(self.down_proj, "forward_deferred", None) if deferred else None
        return proj(h) if proj is not None else self.down_proj(h)


class DecoderLayer(nn.Module):
    def __init__(self, cfg: ModelConfig, backend: AttentionBackend, fused_norm=None):
        super().__init__()
        self.input_layernorm = RMSNorm(cfg.hidden_size, cfg.rms_norm_eps, fused_norm)
        self.self_attn = Attention(cfg, backend)
        self.post_attention_layernorm = RMSNorm(cfg.hidden_size, cfg.rms_norm_eps, fused_norm)
        self.mlp = MLP(cfg)

    def forward(self, x, residual, positions, rotary, k_cache, v_cache, meta):
        """Pre-norm residual block with the residual add fused into the next
        norm (nimbus/model/llama.py:115-124)."""
        if residual is None:
            residual = x
            h = self.input_layernorm(x)
        else:
            h, residual = self.input_layernorm(x, residual)
        # (the projections into the two norms may hand over an INT8 output
        # still in split-K partials; the norm folds them in)
        h = self.self_attn(h, positions, rotary, k_cache, v_cache, meta, deferred=True)
        h, residual = self.post_attention_layernorm(h, residual)
        return self.mlp(h, deferred=True), residual


class LlamaModel(nn.Module):
    def __init__(self, cfg: ModelConfig, backend: AttentionBackend | None = None, max_position: int | None = None,
                 fused_norm=None):
        super().__init__()
        self.cfg = cfg
        backend = backend or AttentionBackend()
        self.embed_tokens = nn.Embedding(cfg.vocab_size, cfg.hidden_size)
        self.layers = nn.ModuleList(DecoderLayer(cfg, backend, fused_norm) for _ in range(cfg.num_layers))
        self.norm = RMSNorm(cfg.hidden_size, cfg.rms_norm_eps, fused_norm)
        self.lm_head = nn.Linear(cfg.hidden_size, cfg.vocab_size, bias=False)
        self.rotary = Rotary(cfg, max_position or cfg.max_position)

    @property
    def backend(self) -> AttentionBackend:
        return self.layers[0].self_attn.backend

    @torch.inference_mode()
    def forward(self, input_ids: torch.Tensor, positions: torch.Tensor,
                kv_caches: list[tuple[torch.Tensor, torch.Tensor]], meta: AttnMetadata) -> torch.Tensor:
        """Final hidden states [T, hidden] (nimbus/model/llama.py:138-153)."""
        x = self.embed_tokens(input_ids)
        residual = None
        for layer, (kc, vc) in zip(self.layers, kv_caches):
            x, residual = layer(x, residual, positions, self.rotary, kc, vc, meta)
        x, _ = self.norm(x, residual)
        return x

    @torch.inference_mode()
    def logits(self, hidden: torch.Tensor) -> torch.Tensor:
        return self.lm_head(hidden).float()


@torch.no_grad()
def init_random_(model: LlamaModel, seed: int = 0, std: float = 0.02) -> LlamaModel:
    """Synthetic weights (no checkpoint is loaded in this build): N(0, std)
    projections and embeddings, unit norm weights, drawn on the model's
    device from a seeded generator."""
    dev = next(model.parameters()).device
    g = torch.Generator(device=dev).manual_seed(seed)
    for name, p in model.named_parameters():
        if name.endswith("layernorm.weight") or name == "norm.weight":
            p.fill_(1.0)
        else:
            p.copy_(torch.randn(p.shape, generator=g, device=dev, dtype=torch.float32).mul_(std).to(p.dtype))
    return model


def build_model(cfg: ModelConfig, dtype: torch.dtype = torch.bfloat16, device="cuda", seed: int = 0,
                backend: AttentionBackend | None = None, max_position: int | None = None) -> LlamaModel:
    """A LlamaModel of cfg's shape with init_random_ weights, in dtype on
    device. Parameters are allocated once, in dtype (no fp32 copy of the
    model is ever made); the rotary tables are built in fp32 on device, as
    the reference's loader does (nimbus/model/weights.py:80-91)."""
    with torch.device("meta"):
        model = LlamaModel(cfg, backend, max_position=1)
    for module in model.modules():
        for name, p in list(module._parameters.items()):
            if p is not None:
                module._parameters[name] = nn.Parameter(torch.empty(p.shape, dtype=dtype, device=device),
                                                        requires_grad=False)
    model.rotary = Rotary(cfg, max_position or cfg.max_position).to(device)
    return init_random_(model.eval(), seed)
