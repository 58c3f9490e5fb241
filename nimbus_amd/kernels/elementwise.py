"""Rotary embedding and the SiLU gate of the Llama decoder on the GPU.

rope_ is Rotary.forward of nimbus/model/llama.py:37-57 applied in place to
the q and k heads of the fused qkv projection, bit for bit the reference's
dtype arithmetic; silu_mul is MLP.forward's F.silu(gate) * up
(llama.py:100-103). Both run csrc/elementwise.hip.
"""

from __future__ import annotations

import torch

from nimbus_amd import _lib


def rope_(x: torch.Tensor, heads: int, head_dim: int, positions: torch.Tensor, cos: torch.Tensor,
          sin: torch.Tensor) -> torch.Tensor:
    """x: [T, >= heads * head_dim] rows (unit last stride); the first
    heads * head_dim elements of row t are rotated by row positions[t] of
    the fp32 tables cos / sin [max_position, head_dim]. In place; returns x."""
    if x.dim() != 2 or x.stride(-1) != 1 or x.shape[1] < heads * head_dim:
        raise ValueError("x must be [T, >= heads * head_dim] with unit last stride")
    if positions.dtype != torch.int64 or positions.shape != (x.shape[0],):
        raise ValueError("positions must be int64 [T]")
    if (cos.dtype != torch.float32 or sin.dtype != torch.float32 or sin.shape != cos.shape
            or cos.shape[1] < head_dim or not (cos.is_contiguous() and sin.is_contiguous())):
        raise ValueError("cos / sin must be contiguous fp32 [max_position, >= head_dim]")
    if not (x.is_cuda and positions.is_cuda and cos.is_cuda and sin.is_cuda):
        raise ValueError("rope_ runs on the GPU only")
    if x.shape[0] == 0:
        return x
    rc = _lib.load().nimbus_rope(x.data_ptr(), x.stride(0), x.shape[0], heads, head_dim,
                                 positions.contiguous().data_ptr(), cos.data_ptr(), sin.data_ptr(),
                                 cos.stride(0), cos.shape[0], _lib.dtype_code(x.dtype), _lib.stream_of(x))
    _lib.check(rc, "nimbus_rope")
    return x


def silu_mul(x: torch.Tensor, out: torch.Tensor | None = None) -> torch.Tensor:
    """x: [..., 2 I] = [gate | up] -> silu(gate) * up [..., I]."""
    two_i = x.shape[-1]
    if two_i % 16 != 0:
        raise NotImplementedError("the gate and up halves must be multiples of 8")
    if not x.is_cuda:
        raise ValueError("silu_mul runs on the GPU only")
    inter = two_i // 2
    x2 = x.reshape(-1, two_i)
    if x2.stride(-1) != 1 or x2.stride(0) % 8 != 0:
        x2 = x2.contiguous()
    y = torch.empty(x2.shape[0], inter, dtype=x.dtype, device=x.device) if out is None else out
    if x2.shape[0]:
        rc = _lib.load().nimbus_silu_mul(x2.data_ptr(), x2.stride(0), y.data_ptr(), y.stride(0), x2.shape[0], inter,
                                         _lib.dtype_code(x.dtype), _lib.stream_of(x))
        _lib.check(rc, "nimbus_silu_mul")
    return y.view(*x.shape[:-1], inter) if out is None else y


def greedy_step(logits: torch.Tensor, input_ids: torch.Tensor, positions: torch.Tensor, context_lens: torch.Tensor,
                slots: torch.Tensor, block_tables: torch.Tensor, block_size: int, active: torch.Tensor,
                ctx_start: torch.Tensor, tokens: torch.Tensor | None, scratch_slot: int) -> None:
    """One on-device link of a greedy chain (nimbus/cuda_graph.py:104-115):
    argmax of each row of logits [b, vocab] (fp32) -> input_ids, recorded in
    tokens [b, max_steps] at context_lens - ctx_start for active rows, whose
    positions / context_lens / slots then advance. All tensors are device
    buffers the caller owns (int64 ids, positions, slots, tokens; int32
    context lengths, tables, active, ctx_start)."""
    b = logits.shape[0]
    if logits.dtype != torch.float32 or logits.stride(-1) != 1:
        raise ValueError("logits must be fp32 with unit last stride")
    for t, dt in ((input_ids, torch.int64), (positions, torch.int64), (slots, torch.int64),
                  (context_lens, torch.int32), (active, torch.int32), (ctx_start, torch.int32),
                  (block_tables, torch.int32)):
        if t.dtype != dt or t.shape[0] < b or not t.is_cuda:
            raise ValueError("greedy_step buffers: wrong dtype, device or length")
    if block_tables.stride(1) != 1:
        raise ValueError("block_tables needs unit column stride")
    steps = 0 if tokens is None else tokens.shape[1]
    rc = _lib.load().nimbus_greedy_step(
        logits.data_ptr(), logits.stride(0), b, logits.shape[1], input_ids.data_ptr(), positions.data_ptr(),
        context_lens.data_ptr(), slots.data_ptr(), block_tables.data_ptr(), block_tables.stride(0),
        block_tables.shape[1], block_size, active.data_ptr(), ctx_start.data_ptr(),
        tokens.data_ptr() if tokens is not None else None, steps, scratch_slot, _lib.stream_of(logits))
    _lib.check(rc, "nimbus_greedy_step")
