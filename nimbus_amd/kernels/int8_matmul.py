"""INT8 weight-only matmul on the GPU.

Drop-in for nimbus/kernels/int8_matmul.py:50-64 (`int8_matmul(x, w_q,
scale)`), computed by int8_matmul_kernel in csrc/int8_matmul.hip:
y = dtype(fp32(x @ w_q^T) * scale), the weights streamed from HBM once as
int8 and widened exactly in registers. fp16 (the reference's dtype) and
bf16 activations.
"""

from __future__ import annotations

import torch

from nimbus_amd import _lib
from nimbus_amd.kernels.paged_attention import _cached_workspace


def int8_matmul_workspace_bytes(m: int, n: int, k: int) -> int:
    return int(_lib.load().nimbus_int8_matmul_workspace_bytes(m, n, k))


def int8_matmul(x: torch.Tensor, w_q: torch.Tensor, scale: torch.Tensor, out: torch.Tensor | None = None,
                workspace: torch.Tensor | None = None) -> torch.Tensor:
    """x: [..., K] fp16/bf16; w_q: [N, K] int8; scale: [N] in x's dtype.
    Returns [..., N] in x's dtype.

    Not in the reference signature: `out` ([M, N] view with unit last
    stride) receives the result; `workspace` is a caller-owned uint8 buffer
    of at least int8_matmul_workspace_bytes(M, N, K) for the split-K partial
    sums (by default one cached per device and stream is used).
    """
    if w_q.dtype != torch.int8 or w_q.dim() != 2:
        raise ValueError("w_q must be int8 [N, K]")
    n, k = w_q.shape
    if x.shape[-1] != k:
        raise ValueError(f"x [..., {x.shape[-1]}] does not match w_q [{n}, {k}]")
    if x.dtype not in (torch.float16, torch.bfloat16):
        raise NotImplementedError("fp16 or bf16 activations")
    if scale.shape != (n,) or scale.dtype != x.dtype:
        raise ValueError(f"scale must be [{n}] in x's dtype")
    if not (x.is_cuda and w_q.is_cuda and scale.is_cuda):
        raise ValueError("int8_matmul runs on the GPU only")
    if n % 4 != 0 or k % 16 != 0:
        raise NotImplementedError(f"N {n} must be a multiple of 4 and K {k} of 16")
    shape = x.shape
    x2 = x.reshape(-1, k)
    if x2.stride(-1) != 1 or x2.stride(0) % 8 != 0 or x2.data_ptr() % 16 != 0:
        x2 = x2.contiguous()
    if w_q.stride(-1) != 1 or w_q.stride(0) % 16 != 0 or w_q.data_ptr() % 16 != 0:
        w_q = w_q.contiguous()
    scale = scale.contiguous()
    m = x2.shape[0]
    if out is None:
        y = torch.empty((m, n), dtype=x.dtype, device=x.device)
    else:
        if out.shape != (m, n) or out.dtype != x.dtype or out.stride(-1) != 1:
            raise ValueError(f"out must be [{m}, {n}] in x's dtype with unit last stride")
        y = out
    if m == 0:
        return y.view(*shape[:-1], n)
    lib = _lib.load()
    need = lib.nimbus_int8_matmul_workspace_bytes(m, n, k)
    if workspace is not None:
        if workspace.numel() * workspace.element_size() < need or not workspace.is_cuda:
            raise ValueError(f"workspace smaller than the {need} bytes this call needs")
        ws = workspace
    else:
        ws = _cached_workspace(need, x.device) if need > 0 else None
    rc = lib.nimbus_int8_matmul(
        x2.data_ptr(), x2.stride(0), w_q.data_ptr(), w_q.stride(0), scale.data_ptr(), y.data_ptr(), y.stride(0),
        m, n, k, ws.data_ptr() if ws is not None else None,
        ws.numel() * ws.element_size() if ws is not None else 0, _lib.dtype_code(x.dtype), _lib.stream_of(x))
    _lib.check(rc, "nimbus_int8_matmul")
    return y.view(*shape[:-1], n) if out is None else y
