"""INT8 weight-only quantization (symmetric, per output channel).

The number format of nimbus/quant/int8.py:20-29: each weight row gets the
scale max|row| / 127 and is stored as round(w / scale) in int8; activations
stay in the model dtype and the scale is applied after the product
(x @ (w_q * s)^T == (x @ w_q^T) * s). Int8Linear runs the HIP kernel
(kernels/int8_matmul.py); the quantizer itself is host-side set-up run once
per weight, in PyTorch on whatever device the weight lives.
"""

from __future__ import annotations

import torch
from torch import nn

from nimbus_amd.kernels.int8_matmul import (int8_matmul_packed, int8_matmul_packed_deferred, int8_matmul_packed_silu,
                                             pack_int8_weight, unpack_int8_weight)


def quantize_weight(w: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """w: [N, K] float -> (int8 [N, K], scale [N] in w's dtype)
    (nimbus/quant/int8.py:20-25)."""
    wf = w.float()
    scale = wf.abs().amax(dim=1).clamp_min(1e-8) / 127.0
    q = torch.round(wf / scale[:, None]).clamp_(-127, 127).to(torch.int8)
    return q, scale.to(w.dtype)


def dequantize_weight(q: torch.Tensor, scale: torch.Tensor) -> torch.Tensor:
    """(nimbus/quant/int8.py:28-29)"""
    return q.to(scale.dtype) * scale[:, None]


class Int8Linear(nn.Module):
    """nimbus/quant/int8.py:32-47 with the HIP kernel. The reference keeps a
    PyTorch path behind use_triton=False; this module is the GPU path only,
    so use_hip=False is refused rather than served on the CPU.

    The quantized weight is kept in the kernel's tile order
    (`weight_packed`, packed once here); `weight_q` gives it back as the
    reference's int8 [out, in] for inspection."""

    def __init__(self, linear: nn.Linear, use_hip: bool = True):
        super().__init__()
        if not use_hip:
            raise ValueError("nimbus_amd's Int8Linear is the HIP path only")
        if linear.bias is not None:
            raise ValueError("the decoder projections have no bias")
        q, s = quantize_weight(linear.weight.data)
        self.register_buffer("weight_packed", pack_int8_weight(q))
        self.register_buffer("scale", s)
        self.in_features, self.out_features = linear.in_features, linear.out_features

    @property
    def weight_q(self) -> torch.Tensor:
        return unpack_int8_weight(self.weight_packed, self.out_features, self.in_features)

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        return int8_matmul_packed(x, self.weight_packed, self.scale, self.out_features, self.in_features)

    def forward_deferred(self, x: torch.Tensor):
        """self(x), or where the tuned launch plan splits K its unreduced
        partials (kernels.int8_matmul.SplitPartials), for the decoder layer's
        residual add + RMSNorm to fold in (the same bits, one launch fewer)."""
        return int8_matmul_packed_deferred(x, self.weight_packed, self.scale, self.out_features, self.in_features)

    def forward_silu(self, x: torch.Tensor) -> torch.Tensor | None:
        """silu_mul(self(x)) in one launch, for the MLP's gate_up projection
        (gate rows first): bit for bit under the same launch plan, within
        rounding where the two tune different ones; None when out_features
        is not a multiple of 32 (the caller then runs the two steps)."""
        if self.out_features % 32 != 0:
            return None
        return int8_matmul_packed_silu(x, self.weight_packed, self.scale, self.out_features, self.in_features)


# Attribute names of the decoder's projections (nimbus/model/llama.py): the
# layers whose weights are quantized. Embeddings, norms and the LM head keep
# the model dtype, as in the reference (quant/int8.py:50-65).
PROJECTIONS = frozenset({"qkv_proj", "o_proj", "gate_up_proj", "down_proj"})


@torch.no_grad()
def quantize_model(model: nn.Module, use_hip: bool = True) -> nn.Module:
    """Swaps each plain nn.Linear registered under one of PROJECTIONS for an
    Int8Linear built from it, in place; returns the model."""
    swaps = [(owner, name, child) for owner in model.modules() for name, child in owner.named_children()
             if name in PROJECTIONS and type(child) is nn.Linear]
    for owner, name, child in swaps:
        owner.add_module(name, Int8Linear(child, use_hip))
    return model


def weight_bytes(model: nn.Module) -> int:
    """Bytes of the tensors a forward pass reads from the model (parameters
    and buffers), each storage counted once: tied weights once, the int8
    projections at one byte an element."""
    sizes: dict[int, int] = {}
    for t in (*model.parameters(), *model.buffers()):
        if t.is_meta:
            continue
        key = t.untyped_storage().data_ptr()
        sizes[key] = max(sizes.get(key, 0), t.untyped_storage().nbytes())
    return sum(sizes.values())
