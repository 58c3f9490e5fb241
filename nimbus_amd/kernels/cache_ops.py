"""KV slot write on the GPU.

Drop-in for nimbus/kernels/reference.py:14-23 (`write_kv`), which Nimbus calls
on every backend before attention (nimbus/model/attention.py:78), and
rope_write_kv, which a decoder layer uses to apply its rotary embedding
(nimbus/model/llama.py:88-98) and write the cache in one launch.
"""

from __future__ import annotations

import torch

from nimbus_amd import _lib
from nimbus_amd.kernels import index_checks


def write_kv(
    k: torch.Tensor,  # [T, KV, D]
    v: torch.Tensor,
    k_cache: torch.Tensor,  # [num_blocks, block_size, KV, D]
    v_cache: torch.Tensor,
    slot_mapping: torch.Tensor,  # [T] int64
) -> None:
    """k_cache.view(-1, KV, D)[slot_mapping[t]] = k[t] (and v), bit for bit.

    Same contract as the reference's two index_copy_ calls: the caches must be
    viewable flat (contiguous); k and v may be strided in their first two
    dims (a slice of a fused qkv projection). Slots outside the cache are
    skipped rather than written, unless index checks are on
    (index_checks: NIMBUS_CHECK_INDICES=1), which raise IndexError first.
    """
    if k.shape != v.shape or k.dim() != 3:
        raise ValueError(f"k {tuple(k.shape)} and v {tuple(v.shape)} must both be [T, KV, D]")
    if k_cache.shape != v_cache.shape or k_cache.dim() != 4:
        raise ValueError("k_cache and v_cache must both be [num_blocks, block_size, KV, D]")
    t, kv, d = k.shape
    if (kv, d) != tuple(k_cache.shape[2:]):
        raise ValueError(f"k rows {(kv, d)} do not match the cache's {tuple(k_cache.shape[2:])}")
    if slot_mapping.shape != (t,) or slot_mapping.dtype != torch.int64:
        raise ValueError("slot_mapping must be int64 [T]")
    if not (k_cache.is_contiguous() and v_cache.is_contiguous()):
        raise ValueError("caches must be contiguous (they are written through a flat slot view)")
    if not (k.dtype == v.dtype == k_cache.dtype == v_cache.dtype):
        raise ValueError("k, v and the caches must share one dtype")
    if not (k.is_cuda and k_cache.is_cuda and slot_mapping.is_cuda):
        raise ValueError("write_kv runs on the GPU only")
    if t == 0:
        return
    if index_checks.enabled():
        index_checks.check_slots(slot_mapping, k_cache.shape[0] * k_cache.shape[1])
    if k.stride(-1) != 1:
        k = k.contiguous()
    if v.stride(-1) != 1:
        v = v.contiguous()
    slot_mapping = slot_mapping.contiguous()
    lib = _lib.load()
    rc = lib.nimbus_write_kv(
        k.data_ptr(), v.data_ptr(), k_cache.data_ptr(), v_cache.data_ptr(), slot_mapping.data_ptr(),
        t, kv, d, k.stride(0), k.stride(1), v.stride(0), v.stride(1),
        k_cache.shape[0] * k_cache.shape[1], _lib.dtype_code(k.dtype), _lib.stream_of(k))
    _lib.check(rc, "nimbus_write_kv")


def rope_write_kv(
    qkv: torch.Tensor,  # [T, >= (H + 2 KV) * D]: q heads, k heads, v heads
    heads: int,
    kv_heads: int,
    head_dim: int,
    positions: torch.Tensor,  # [T] int64
    cos: torch.Tensor,  # [max_position, >= D] fp32
    sin: torch.Tensor,
    k_cache: torch.Tensor,  # [num_blocks, block_size, KV, D]
    v_cache: torch.Tensor,
    slot_mapping: torch.Tensor,  # [T] int64
) -> None:
    """The rotary embedding of the q and k heads of the fused qkv rows, in
    place, then write_kv of their k and v heads: the same results, bit for
    bit, as elementwise.rope_(qkv, heads + kv_heads, ...) followed by
    write_kv(k, v, ...), in one launch."""
    if qkv.dim() != 2 or qkv.stride(-1) != 1 or qkv.shape[1] < (heads + 2 * kv_heads) * head_dim:
        raise ValueError("qkv must be [T, >= (heads + 2 kv_heads) * head_dim] with unit last stride")
    t = qkv.shape[0]
    if positions.dtype != torch.int64 or positions.shape != (t,):
        raise ValueError("positions must be int64 [T]")
    if slot_mapping.dtype != torch.int64 or slot_mapping.shape != (t,):
        raise ValueError("slot_mapping must be int64 [T]")
    if (cos.dtype != torch.float32 or sin.dtype != torch.float32 or sin.shape != cos.shape
            or cos.shape[1] < head_dim or not (cos.is_contiguous() and sin.is_contiguous())):
        raise ValueError("cos / sin must be contiguous fp32 [max_position, >= head_dim]")
    if k_cache.shape != v_cache.shape or k_cache.dim() != 4 or tuple(k_cache.shape[2:]) != (kv_heads, head_dim):
        raise ValueError("k_cache and v_cache must both be [num_blocks, block_size, kv_heads, head_dim]")
    if not (k_cache.is_contiguous() and v_cache.is_contiguous()):
        raise ValueError("caches must be contiguous (they are written through a flat slot view)")
    if not (qkv.dtype == k_cache.dtype == v_cache.dtype):
        raise ValueError("qkv and the caches must share one dtype")
    if not (qkv.is_cuda and positions.is_cuda and cos.is_cuda and k_cache.is_cuda and slot_mapping.is_cuda):
        raise ValueError("rope_write_kv runs on the GPU only")
    if t == 0:
        return
    if index_checks.enabled():
        index_checks.check_slots(slot_mapping, k_cache.shape[0] * k_cache.shape[1])
    rc = _lib.load().nimbus_rope_write_kv(
        qkv.data_ptr(), qkv.stride(0), t, heads, kv_heads, head_dim, positions.contiguous().data_ptr(),
        cos.data_ptr(), sin.data_ptr(), cos.stride(0), cos.shape[0], k_cache.data_ptr(), v_cache.data_ptr(),
        slot_mapping.contiguous().data_ptr(), k_cache.shape[0] * k_cache.shape[1], _lib.dtype_code(qkv.dtype),
        _lib.stream_of(qkv))
    _lib.check(rc, "nimbus_rope_write_kv")
