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
    # (An eager call of a small norm is bound by this function's host time, so
    # it avoids reshapes, views and allocations that a 2-D input does not need.)
    n = x.shape[-1]
    dt = x.dtype
    if weight.shape != (n,):
        raise ValueError(f"weight {tuple(weight.shape)} does not match rows of {n}")
    if (dt is not torch.float16 and dt is not torch.bfloat16) or weight.dtype != dt:
        raise NotImplementedError("fp16 or bf16 x and weight of one dtype")
    if residual is not None and (residual.shape != x.shape or residual.dtype != dt):
        raise ValueError("residual must match x's shape and dtype")
    if not (x.is_cuda and weight.is_cuda and (residual is None or residual.is_cuda)):
        raise ValueError("rms_norm runs on the GPU only")
    flat = x.dim() == 2
    x2 = x if flat else x.reshape(-1, n)
    if x2.stride(-1) != 1:
        x2 = x2.contiguous()
    if weight.stride(0) != 1:
        weight = weight.contiguous()
    out = torch.empty_like(x2, memory_format=torch.contiguous_format)
    if residual is not None:
        r2 = residual if flat else residual.reshape(-1, n)
        if r2.stride(-1) != 1:
            r2 = r2.contiguous()
        res_out = torch.empty_like(out)
        r_ptr, r_st, ro_ptr, ro_st = r2.data_ptr(), r2.stride(0), res_out.data_ptr(), res_out.stride(0)
    else:
        res_out = None
        r_ptr, r_st, ro_ptr, ro_st = None, 0, None, 0
    rows = x2.shape[0]
    if rows:
        rc = _lib.load().nimbus_add_rms_norm(
            x2.data_ptr(), x2.stride(0), r_ptr, r_st, weight.data_ptr(), out.data_ptr(), out.stride(0), ro_ptr, ro_st,
            rows, n, float(eps), _lib.NIMBUS_BFLOAT16 if dt is torch.bfloat16 else _lib.NIMBUS_FLOAT16,
            _lib.stream_of(x))
        if rc:
            _lib.check(rc, "nimbus_add_rms_norm")
    if flat:
        return out, res_out
    return out.view(x.shape), (res_out.view(x.shape) if res_out is not None else None)


def rms_norm(x: torch.Tensor, weight: torch.Tensor, eps: float) -> torch.Tensor:
    """weight * dtype(x * rsqrt(mean(x^2, -1) + eps)), normalised in float32."""
    return _launch(x, None, weight, eps)[0]


def add_rms_norm(x: torch.Tensor, residual: torch.Tensor, weight: torch.Tensor, eps: float):
    """residual += x; returns (rms_norm(residual), residual). Does not modify inputs."""
    return _launch(x, residual, weight, eps)


def add_rms_norm_partials(p, residual: torch.Tensor, weight: torch.Tensor, eps: float):
    """add_rms_norm(h, residual, weight, eps) where h is the INT8 projection
    output that p (kernels.int8_matmul.SplitPartials) stands for: one launch
    folds its split-K partials in as the reducing launch would, then adds and
    normalises; the same bits as the two launches. Returns (out, residual)."""
    splits, m, n = p.partials.shape
    if residual.shape != p.shape or residual.dtype != p.dtype or weight.shape != (n,) or weight.dtype != p.dtype:
        raise ValueError(f"residual {tuple(residual.shape)} / weight {tuple(weight.shape)} do not match {p.shape}")
    if weight.stride(0) != 1:
        weight = weight.contiguous()
    r2 = residual.reshape(m, n)
    if r2.stride(-1) != 1:
        r2 = r2.contiguous()
    out = torch.empty((m, n), dtype=p.dtype, device=residual.device)
    rout = torch.empty_like(out)
    lib = _lib.load()
    rc = lib.nimbus_add_rms_norm_partials(p.partials.data_ptr(), splits, p.scale.data_ptr(), r2.data_ptr(),
                                          r2.stride(0), weight.data_ptr(), out.data_ptr(), n, rout.data_ptr(), n,
                                          m, n, float(eps), _lib.dtype_code(p.dtype), _lib.stream_of(residual))
    _lib.check(rc, "nimbus_add_rms_norm_partials")
    return out.view(p.shape), rout.view(p.shape)
