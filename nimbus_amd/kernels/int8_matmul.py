"""INT8 weight-only matmul on the GPU.

Drop-in for nimbus/kernels/int8_matmul.py:50-64 (`int8_matmul(x, w_q,
scale)`), computed by int8_matmul_kernel in csrc/int8_matmul.hip:
y = dtype(fp32(x @ w_q^T) * scale), the weights streamed from HBM once as
int8 and widened exactly in registers. fp16 (the reference's dtype) and
bf16 activations.

pack_int8_weight / int8_matmul_packed are the same product on weights
stored in MFMA tile order (1 KB per 16 rows x 64 columns, in the order the
kernel's lanes load them), which Int8Linear builds once per layer: each
wave then streams its weights contiguously instead of 64 bytes per row.
"""

from __future__ import annotations

from dataclasses import dataclass

import torch

from nimbus_amd import _lib
from nimbus_amd.kernels.paged_attention import _cached_workspace

# The split-K partials' workspaces (a family apart from the decode ones).
_INT8_WORKSPACES: dict = {}


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
        ws = _cached_workspace(need, x.device, _INT8_WORKSPACES) if need > 0 else None
    rc = lib.nimbus_int8_matmul(
        x2.data_ptr(), x2.stride(0), w_q.data_ptr(), w_q.stride(0), scale.data_ptr(), y.data_ptr(), y.stride(0),
        m, n, k, ws.data_ptr() if ws is not None else None,
        ws.numel() * ws.element_size() if ws is not None else 0, _lib.dtype_code(x.dtype), _lib.stream_of(x))
    _lib.check(rc, "nimbus_int8_matmul")
    return y.view(*shape[:-1], n) if out is None else y


def pack_int8_weight(w_q: torch.Tensor) -> torch.Tensor:
    """int8 [N, K] -> the tile-order layout of nimbus_int8_matmul_packed
    (uint8-free int8 tensor of nimbus_int8_packed_weight_bytes(N, K) bytes,
    shape [ceil(N/16), ceil(K/64), 1024])."""
    if w_q.dtype != torch.int8 or w_q.dim() != 2 or w_q.stride(-1) != 1 or not w_q.is_cuda:
        raise ValueError("w_q must be a CUDA int8 [N, K] with unit last stride")
    n, k = w_q.shape
    out = torch.empty(-(-n // 16), -(-k // 64), 1024, dtype=torch.int8, device=w_q.device)
    rc = _lib.load().nimbus_int8_pack_weight(w_q.data_ptr(), w_q.stride(0), n, k, out.data_ptr(),
                                             _lib.stream_of(w_q))
    _lib.check(rc, "nimbus_int8_pack_weight")
    return out


def unpack_int8_weight(packed: torch.Tensor, n: int, k: int) -> torch.Tensor:
    """The inverse of pack_int8_weight (for inspection): int8 [N, K]."""
    nb, kc = packed.shape[0], packed.shape[1]
    t = packed.view(nb, kc, 4, 16, 16)  # block, chunk, lane group (16 columns), row in block, byte
    return t.permute(0, 3, 1, 2, 4).reshape(nb * 16, kc * 64)[:n, :k].contiguous()


# Launch plans (token tile, k slices, K splits, row blocks per wave) tuned per (M bucket, N, K,
# dtype, device), as nimbus/kernels/int8_matmul.py:16-24 autotunes its
# Triton configs per M bucket. Tuning times every candidate plan on the
# call's own inputs, eagerly, the first time a key is seen; a call being
# captured into a graph never tunes and uses the tuned plan or the
# library's default. Set AUTOTUNE = False to always use the default.
AUTOTUNE = True
_TUNED: dict[tuple, tuple[int, int, int, int] | None] = {}
_TUNE_BYTES = 600e6  # weight copies the timing rotates over (beyond the 256 MB Infinity Cache)


def m_bucket(m: int) -> int:
    """Size class of M (nimbus/kernels/int8_matmul.py:58-59)."""
    return 1 << max(4, (m - 1).bit_length()) if m <= 256 else 512


def _candidate_plans(m: int, n: int, k: int) -> list[tuple[int, int, int, int]]:
    nb = -(-n // 16)
    plans = []
    for bm in (16, 32, 64, 128):
        if bm > 16 and m <= bm // 2:
            continue  # a smaller tile covers M
        for ks in (1, 2, 4, 8):
            if ks * bm > 128:
                continue
            for rw in (1, 2):
                if rw > 1 and m <= 16:
                    continue  # two row blocks per x read pay only when x is read for many tokens
                tiles = -(-nb // (8 // ks * rw)) * -(-m // bm)
                for splits in (1, 2, 3, 4, 6, 8, 12, 16):
                    if splits > 1 and k < 4 * 64 * ks * splits:
                        continue
                    if 64 <= tiles * splits <= 768:
                        plans.append((bm, ks, splits, rw))
    return plans


def _tune(x2, w_packed, scale, y, n, k, lib) -> tuple[int, int, int, int] | None:
    m = x2.shape[0]
    plans = _candidate_plans(m, n, k)
    if len(plans) < 2:
        return None
    need = max(lib.nimbus_int8_matmul_packed_plan_workspace_bytes(m, n, k, *p) for p in plans)
    ws = torch.empty(max(need, 256), dtype=torch.uint8, device=x2.device)
    copies = [w_packed] + [w_packed.clone() for _ in range(max(0, int(_TUNE_BYTES // w_packed.numel()) - 1))]
    stream = torch.cuda.current_stream(x2.device)
    dt = _lib.dtype_code(x2.dtype)

    def run(plan, w):
        rc = lib.nimbus_int8_matmul_packed_plan(x2.data_ptr(), x2.stride(0), w.data_ptr(), scale.data_ptr(),
                                                y.data_ptr(), y.stride(0), m, n, k, *plan, ws.data_ptr(),
                                                ws.numel(), dt, stream.cuda_stream)
        _lib.check(rc, "nimbus_int8_matmul_packed_plan")

    best, best_t = None, float("inf")
    for plan in plans:
        run(plan, copies[0])
        start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        start.record(stream)
        for rep in range(2):
            for w in copies:
                run(plan, w)
        end.record(stream)
        end.synchronize()
        t = start.elapsed_time(end)
        if t < best_t:
            best, best_t = plan, t
    return best


def int8_matmul_packed_workspace_bytes(m: int, n: int, k: int) -> int:
    """Workspace that serves int8_matmul_packed at this shape whichever plan
    tuning picks (the largest over the candidates and the default)."""
    lib = _lib.load()
    need = lib.nimbus_int8_matmul_packed_workspace_bytes(m, n, k)
    for plan in _candidate_plans(m, n, k):
        need = max(need, lib.nimbus_int8_matmul_packed_plan_workspace_bytes(m, n, k, *plan))
    return int(need)


def int8_matmul_packed(x: torch.Tensor, w_packed: torch.Tensor, scale: torch.Tensor, n: int, k: int,
                       out: torch.Tensor | None = None, workspace: torch.Tensor | None = None) -> torch.Tensor:
    """int8_matmul with w_packed = pack_int8_weight(w_q) for w_q [n, k],
    with the launch plan tuned for this shape (see AUTOTUNE)."""
    if w_packed.dtype != torch.int8 or w_packed.shape != (-(-n // 16), -(-k // 64), 1024):
        raise ValueError("w_packed must be pack_int8_weight's layout for [n, k]")
    if x.shape[-1] != k:
        raise ValueError(f"x [..., {x.shape[-1]}] does not match k {k}")
    if x.dtype not in (torch.float16, torch.bfloat16):
        raise NotImplementedError("fp16 or bf16 activations")
    if scale.shape != (n,) or scale.dtype != x.dtype:
        raise ValueError(f"scale must be [{n}] in x's dtype")
    if not (x.is_cuda and w_packed.is_cuda and scale.is_cuda):
        raise ValueError("int8_matmul_packed runs on the GPU only")
    shape = x.shape
    x2 = x.reshape(-1, k)
    if x2.stride(-1) != 1 or x2.stride(0) % 8 != 0 or x2.data_ptr() % 16 != 0:
        x2 = x2.contiguous()
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
    scale = scale.contiguous()
    key = (m_bucket(m), n, k, x.dtype, x.device.index)
    # (plans are the tiled kernel's: shapes it does not take run the general kernel untuned)
    if key not in _TUNED and AUTOTUNE and n % 4 == 0 and k % 8 == 0 and not torch.cuda.is_current_stream_capturing():
        _TUNED[key] = _tune(x2, w_packed, scale, y, n, k, lib)
    plan = _TUNED.get(key)
    if plan is not None and lib.nimbus_int8_matmul_packed_plan_workspace_bytes(m, n, k, *plan) < 0:
        plan = None
    if plan is None:
        need = lib.nimbus_int8_matmul_packed_workspace_bytes(m, n, k)
    else:
        need = lib.nimbus_int8_matmul_packed_plan_workspace_bytes(m, n, k, *plan)
    if workspace is not None:
        if workspace.numel() * workspace.element_size() < need or not workspace.is_cuda:
            raise ValueError(f"workspace smaller than the {need} bytes this call needs")
        ws = workspace
    else:
        ws = _cached_workspace(need, x.device, _INT8_WORKSPACES) if need > 0 else None
    ws_ptr = ws.data_ptr() if ws is not None else None
    ws_bytes = ws.numel() * ws.element_size() if ws is not None else 0
    if plan is None:
        rc = lib.nimbus_int8_matmul_packed(
            x2.data_ptr(), x2.stride(0), w_packed.data_ptr(), scale.data_ptr(), y.data_ptr(), y.stride(0), m, n, k,
            ws_ptr, ws_bytes, _lib.dtype_code(x.dtype), _lib.stream_of(x))
    else:
        rc = lib.nimbus_int8_matmul_packed_plan(
            x2.data_ptr(), x2.stride(0), w_packed.data_ptr(), scale.data_ptr(), y.data_ptr(), y.stride(0), m, n, k,
            *plan, ws_ptr, ws_bytes, _lib.dtype_code(x.dtype), _lib.stream_of(x))
    _lib.check(rc, "nimbus_int8_matmul_packed")
    return y.view(*shape[:-1], n) if out is None else y


def _silu_plans(m: int, n: int, k: int) -> list[tuple[int, int, int]]:
    """Candidate plans (bm, ks, rows per wave) of the fused gate_up + SiLU
    launch: the single-split plans whose row-block groups pair up (ks <= 4)."""
    return sorted({(bm, ks, rw) for bm, ks, splits, rw in _candidate_plans(m, n, k) if splits == 1 and ks <= 4})


_SILU_TUNED: dict[tuple, tuple[int, int, int] | None] = {}


def _tune_silu(x2, w_packed, scale, y, n, k, lib) -> tuple[int, int, int] | None:
    m = x2.shape[0]
    plans = _silu_plans(m, n, k)
    if len(plans) < 2:
        return plans[0] if plans else None
    copies = [w_packed] + [w_packed.clone() for _ in range(max(0, int(_TUNE_BYTES // w_packed.numel()) - 1))]
    stream = torch.cuda.current_stream(x2.device)
    dt = _lib.dtype_code(x2.dtype)

    def run(plan, w):
        rc = lib.nimbus_int8_matmul_packed_silu(x2.data_ptr(), x2.stride(0), w.data_ptr(), scale.data_ptr(),
                                                y.data_ptr(), y.stride(0), m, n, k, *plan, dt, stream.cuda_stream)
        _lib.check(rc, "nimbus_int8_matmul_packed_silu")

    best, best_t = None, float("inf")
    for plan in plans:
        run(plan, copies[0])
        start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        start.record(stream)
        for rep in range(2):
            for w in copies:
                run(plan, w)
        end.record(stream)
        end.synchronize()
        t = start.elapsed_time(end)
        if t < best_t:
            best, best_t = plan, t
    return best


def int8_matmul_packed_silu(x: torch.Tensor, w_packed: torch.Tensor, scale: torch.Tensor, n: int, k: int,
                            out: torch.Tensor | None = None) -> torch.Tensor:
    """silu_mul(int8_matmul_packed(x, w_packed, scale, n, k)) in one launch
    (the MLP's gate_up projection and SiLU gate, nimbus/model/llama.py:
    100-103): [..., n / 2]. n a multiple of 32 (gate rows first, then up
    rows). Under one launch plan the result is the two steps' bit for bit;
    the plan is tuned per shape as int8_matmul_packed's is, but apart from
    it, so where the two pick plans with other k slices the sums over K
    differ in fp32 order (results within rounding)."""
    if w_packed.dtype != torch.int8 or w_packed.shape != (-(-n // 16), -(-k // 64), 1024):
        raise ValueError("w_packed must be pack_int8_weight's layout for [n, k]")
    if n % 32 != 0:
        raise NotImplementedError("the fused gate needs n a multiple of 32")
    if x.shape[-1] != k:
        raise ValueError(f"x [..., {x.shape[-1]}] does not match k {k}")
    if x.dtype not in (torch.float16, torch.bfloat16):
        raise NotImplementedError("fp16 or bf16 activations")
    if scale.shape != (n,) or scale.dtype != x.dtype:
        raise ValueError(f"scale must be [{n}] in x's dtype")
    if not (x.is_cuda and w_packed.is_cuda and scale.is_cuda):
        raise ValueError("int8_matmul_packed_silu runs on the GPU only")
    shape = x.shape
    x2 = x.reshape(-1, k)
    if x2.stride(-1) != 1 or x2.stride(0) % 8 != 0 or x2.data_ptr() % 16 != 0:
        x2 = x2.contiguous()
    m = x2.shape[0]
    h = n // 2
    if out is None:
        y = torch.empty((m, h), dtype=x.dtype, device=x.device)
    else:
        if out.shape != (m, h) or out.dtype != x.dtype or out.stride(-1) != 1:
            raise ValueError(f"out must be [{m}, {h}] in x's dtype with unit last stride")
        y = out
    if m == 0:
        return y.view(*shape[:-1], h)
    lib = _lib.load()
    scale = scale.contiguous()
    key = (m_bucket(m), n, k, x.dtype, x.device.index)
    if key not in _SILU_TUNED and AUTOTUNE and not torch.cuda.is_current_stream_capturing():
        _SILU_TUNED[key] = _tune_silu(x2, w_packed, scale, y, n, k, lib)
    plan = _SILU_TUNED.get(key) or (0, 1, 1)
    rc = lib.nimbus_int8_matmul_packed_silu(x2.data_ptr(), x2.stride(0), w_packed.data_ptr(), scale.data_ptr(),
                                            y.data_ptr(), y.stride(0), m, n, k, *plan, _lib.dtype_code(x.dtype),
                                            _lib.stream_of(x))
    _lib.check(rc, "nimbus_int8_matmul_packed_silu")
    return y.view(*shape[:-1], h) if out is None else y


# Set False to have int8_matmul_packed_deferred always reduce (for comparisons).
DEFER_SPLITS = True


@dataclass
class SplitPartials:
    """An INT8 projection's output left in its split-K partials: partials
    [splits, m, n] fp32 (a view of the per-stream INT8 workspace, valid until
    the next INT8 call on the stream), the channel scale, and the output's
    shape and dtype. add_rms_norm_partials folds it in, bit for bit as the
    reducing launch would have formed the output."""

    partials: torch.Tensor
    scale: torch.Tensor
    shape: tuple
    dtype: torch.dtype


def int8_matmul_packed_deferred(x: torch.Tensor, w_packed: torch.Tensor, scale: torch.Tensor, n: int,
                                k: int) -> torch.Tensor | SplitPartials:
    """int8_matmul_packed(x, w_packed, scale, n, k), except that where its
    tuned plan splits K the output is returned as its unreduced partials
    (SplitPartials) for the residual add + RMSNorm that reads it next, which
    saves the reducing launch. n a multiple of 8 and at most 8192 (the rows
    that norm takes); otherwise, or when the plan does not split, a tensor."""
    m = x.numel() // max(x.shape[-1], 1) if x.dim() else 0
    if (not DEFER_SPLITS or n % 8 != 0 or n > 8192 or m == 0 or x.dim() < 1 or x.shape[-1] != k
            or x.dtype not in (torch.float16, torch.bfloat16)):
        return int8_matmul_packed(x, w_packed, scale, n, k)
    x2 = x.reshape(-1, k)
    key = (m_bucket(m), n, k, x.dtype, x.device.index)
    if key not in _TUNED:
        return int8_matmul_packed(x, w_packed, scale, n, k)  # (tunes: the next call takes the tuned plan)
    plan = _TUNED[key]
    lib = _lib.load()
    need = lib.nimbus_int8_matmul_packed_plan_workspace_bytes(m, n, k, *plan) if plan is not None else 0
    if need <= 0:
        return int8_matmul_packed(x, w_packed, scale, n, k)
    if x2.stride(-1) != 1 or x2.stride(0) % 8 != 0 or x2.data_ptr() % 16 != 0:
        x2 = x2.contiguous()
    ws = _cached_workspace(need, x.device, _INT8_WORKSPACES)
    rc = lib.nimbus_int8_matmul_packed_partials(x2.data_ptr(), x2.stride(0), w_packed.data_ptr(), m, n, k, *plan,
                                                ws.data_ptr(), ws.numel() * ws.element_size(),
                                                _lib.dtype_code(x.dtype), _lib.stream_of(x))
    _lib.check(rc, "nimbus_int8_matmul_packed_partials")
    splits = need // (m * n * 4)
    part = ws.view(torch.uint8)[:need].view(torch.float32).view(splits, m, n)
    return SplitPartials(part, scale.contiguous(), tuple(x.shape[:-1]) + (n,), x.dtype)
