"""Fused residual add + RMSNorm on the GPU.

Drop-in for nimbus/kernels/rmsnorm.py:53-59 (`rms_norm`, `add_rms_norm`), the
optional fused norms of nimbus/model/llama.py:61-77, computed by
add_rms_norm_kernel in csrc/rmsnorm.hip with the numerics of
nimbus/kernels/reference.py:99-112: the residual add in the model dtype, the
normalisation in float32, the cast back, then the weight multiply in the
model dtype.
"""

from __future__ import annotations

import torch

from nimbus_amd import _lib

# Rows the chunked kernel takes (a multiple of 8 elements, at most MAX_COLS);
# any other length runs the library's general kernel.
MAX_COLS = 8192


def _launch(x: torch.Tensor, residual: torch.Tensor | None, weight: torch.Tensor, eps: float):
    n = x.shape[-1]
    if weight.shape != (n,):
        raise ValueError(f"weight {tuple(weight.shape)} does not match rows of {n}")
    if x.dtype not in (torch.float16, torch.bfloat16) or weight.dtype != x.dtype:
        raise NotImplementedError("fp16 or bf16 x and weight of one dtype")
    if residual is not None and (residual.shape != x.shape or residual.dtype != x.dtype):
        raise ValueError("residual must match x's shape and dtype")
    if not (x.is_cuda and weight.is_cuda and (residual is None or residual.is_cuda)):
        raise ValueError("rms_norm runs on the GPU only")
    x2 = x.reshape(-1, n)
    if x2.stride(-1) != 1:
        x2 = x2.contiguous()
    weight = weight.contiguous()
    out = torch.empty(x2.shape, dtype=x.dtype, device=x.device)
    if residual is not None:
        r2 = residual.reshape(-1, n)
        if r2.stride(-1) != 1:
            r2 = r2.contiguous()
        res_out = torch.empty_like(out)
    else:
        r2 = res_out = None
    rows = x2.shape[0]
    if rows:
        lib = _lib.load()
        rc = lib.nimbus_add_rms_norm(
            x2.data_ptr(), x2.stride(0), r2.data_ptr() if r2 is not None else None, r2.stride(0) if r2 is not None else 0,
            weight.data_ptr(), out.data_ptr(), out.stride(0), res_out.data_ptr() if res_out is not None else None,
            res_out.stride(0) if res_out is not None else 0, rows, n, float(eps), _lib.dtype_code(x.dtype),
            _lib.stream_of(x))
        _lib.check(rc, "nimbus_add_rms_norm")
    return out.view(x.shape), (res_out.view(x.shape) if res_out is not None else None)


def rms_norm(x: torch.Tensor, weight: torch.Tensor, eps: float) -> torch.Tensor:
    """weight * dtype(x * rsqrt(mean(x^2, -1) + eps)), normalised in float32."""
    return _launch(x, None, weight, eps)[0]


def add_rms_norm(x: torch.Tensor, residual: torch.Tensor, weight: torch.Tensor, eps: float):
    """residual += x; returns (rms_norm(residual), residual). Does not modify inputs."""
    return _launch(x, residual, weight, eps)
