"""Paged decode attention (one query token per sequence) on the GPU.

Drop-in for nimbus/kernels/paged_attention.py:101-146: same signature, same
result (within fp16/bf16 rounding of the reference attention), computed by
paged_decode_kernel + paged_decode_merge_kernel in csrc/paged_decode.hip.

The batch's 16-token pages are split evenly over a fixed number of waves per
kv-head group, so the work is balanced whatever the mix of context lengths
and long contexts spread over many waves at any batch size. The launch grid
is a function of (batch, KV heads, max_context, device) only; inside a
captured graph the caller fixes max_context (Nimbus's DecodeGraphs passes
max_model_len, cuda_graph.py:52-63) and the same graph serves any context
lengths up to it.
"""

from __future__ import annotations

import torch

from nimbus_amd import _lib
from nimbus_amd.kernels import index_checks

PAGE = 16  # tokens per KV-cache block of the tuned kernels (other sizes run the general kernel)


def tuned_shape(block_size: int, head_dim: int) -> bool:
    """Whether the tuned kernels take this page size and head dim; other
    shapes run the general kernel, which has no prefill pieces or stream-K
    form."""
    return block_size == PAGE and head_dim in (64, 128)


def decode_workspace_bytes(batch: int, heads: int, head_dim: int, max_context: int) -> int:
    return int(_lib.load().nimbus_paged_decode_workspace_bytes(batch, heads, head_dim, max_context))


# Workspace sizes by (batch, heads, head dim, max_context): a pure function of
# the shape, asked once per shape instead of once per call.
_WS_BYTES: dict[tuple[int, int, int, int], int] = {}


def _decode_ws_bytes(lib, b: int, h: int, d: int, max_context: int) -> int:
    key = (b, h, d, max_context)
    n = _WS_BYTES.get(key)
    if n is None:
        n = _WS_BYTES[key] = int(lib.nimbus_paged_decode_workspace_bytes(b, h, d, max_context))
    return n


# Workspaces cached per (device, stream), grown on demand, so a call does not
# allocate. Buffers that were outgrown stay alive: a captured graph may still
# use them.
_WORKSPACES: dict[tuple[int, int], torch.Tensor] = {}
_OUTGROWN: list[torch.Tensor] = []


def new_decode_workspace(nbytes: int, device) -> torch.Tensor:
    """A workspace of at least nbytes for decode calls (no initialisation needed)."""
    return torch.empty(max(int(nbytes), 256), dtype=torch.uint8, device=device)


def _cached_workspace(nbytes: int, device: torch.device, cache: dict | None = None) -> torch.Tensor:
    """A workspace per (device, stream), grown on demand; `cache` keeps
    another family of them (the prefill pieces' and the INT8 matmul's), so a
    call of one family never grows or reuses another's buffer."""
    cache = _WORKSPACES if cache is None else cache
    index = device.index if device.index is not None else torch.cuda.current_device()
    key = (index, torch._C._cuda_getCurrentRawStream(index))
    ws = cache.get(key)
    if ws is None or ws.numel() < nbytes:
        if ws is not None:
            _OUTGROWN.append(ws)
        ws = new_decode_workspace(max(nbytes, 1 << 20), device)
        cache[key] = ws
    return ws


def _check_cache(k_cache: torch.Tensor, v_cache: torch.Tensor) -> None:
    if k_cache.dim() != 4 or k_cache.shape != v_cache.shape:
        raise ValueError("k_cache and v_cache must both be [num_blocks, block_size, KV, D]")
    kst = k_cache.stride()
    if kst != v_cache.stride():
        raise ValueError("v_cache must share k_cache's strides")
    if kst[3] != 1:
        raise ValueError("caches need unit stride in the head dim")
    if k_cache.dtype != v_cache.dtype:
        raise ValueError("k_cache and v_cache must share one dtype")
    if not (k_cache.is_cuda and v_cache.is_cuda):
        raise ValueError("the paged-attention kernels run on the GPU only")


def paged_decode_attention(
    q: torch.Tensor,  # [B, H, D]
    k_cache: torch.Tensor,  # [num_blocks, block_size, KV, D]
    v_cache: torch.Tensor,
    context_lens: torch.Tensor,  # [B] int32
    block_tables: torch.Tensor,  # [B, max_blocks] int32
    max_context: int,
    scale: float,
    num_partitions: int | None = None,
    out: torch.Tensor | None = None,
    workspace: torch.Tensor | None = None,
    _entry: str = "nimbus_paged_decode",
) -> torch.Tensor:
    """out[b, h] = softmax(scale * q[b, h] . K^T) V over sequence b's first
    context_lens[b] cached tokens (kv head h // (H // KV)).

    max_context must be >= every context length (the reference relies on the
    same bound for its grid and gather width). num_partitions is accepted for
    signature compatibility with the Triton wrapper, whose graph capture uses
    it to pin the grid; here the grid is already pinned by max_context, so
    the value is not used.
    `out` (optional, not in the reference signature) receives the result in
    place, e.g. a slice of the backend's flat output. `workspace` (optional)
    is a caller-owned uint8 buffer of at least decode_workspace_bytes() (the
    page prefix sum and the pieces of split sequences; nothing in it survives
    the call). By default a workspace cached per (device, stream) is used, so
    concurrent calls must run on different streams. `_entry` selects one
    pass of the C ABI (nimbus_paged_decode_pages / _merge) for timing
    the passes separately; the default runs both.
    """
    del num_partitions
    if q.dim() != 3:
        raise ValueError(f"q must be [B, H, D], got {tuple(q.shape)}")
    b, h, d = q.shape
    _check_cache(k_cache, v_cache)
    kv = k_cache.shape[2]
    if k_cache.shape[3] != d or h % kv != 0:
        raise ValueError(f"q {tuple(q.shape)} does not fit caches {tuple(k_cache.shape)}")
    if q.dtype != k_cache.dtype:
        raise ValueError("q and the caches must share one dtype")
    if out is None:
        out = torch.empty_like(q)
    elif out.shape != q.shape or out.dtype != q.dtype or out.stride(-1) != 1:
        raise ValueError("out must match q's shape and dtype with unit last stride")
    if b == 0:
        return out
    if context_lens.dtype != torch.int32 or block_tables.dtype != torch.int32:
        raise ValueError("context_lens and block_tables must be int32")
    if context_lens.shape != (b,) or block_tables.dim() != 2 or block_tables.shape[0] != b:
        raise ValueError("context_lens must be [B] and block_tables [B, max_blocks]")
    if q.stride(-1) != 1:
        q = q.contiguous()
    context_lens = context_lens.contiguous()
    if block_tables.stride(1) != 1:
        block_tables = block_tables.contiguous()
    if index_checks.enabled():
        index_checks.check_tables(block_tables, context_lens, k_cache.shape[0], k_cache.shape[1])
    lib = _lib.load()
    max_context = int(max_context)
    need = _decode_ws_bytes(lib, b, h, d, max_context)
    if workspace is not None:
        if workspace.numel() * workspace.element_size() < need or not workspace.is_cuda:
            raise ValueError(f"workspace smaller than the {need} bytes this call needs")
        ws = workspace
    else:
        ws = _cached_workspace(need, q.device)
    qst, cst, ost = q.stride(), k_cache.stride(), out.stride()
    rc = getattr(lib, _entry)(
        q.data_ptr(), qst[0], qst[1], k_cache.data_ptr(), v_cache.data_ptr(), k_cache.shape[0], cst[0], cst[1],
        cst[2], block_tables.data_ptr(), block_tables.stride(0), block_tables.shape[1], context_lens.data_ptr(),
        out.data_ptr(), ost[0], ost[1], ws.data_ptr(), ws.nbytes, b, h, kv, d, k_cache.shape[1], max_context,
        float(scale), _lib.dtype_code(q.dtype), _lib.stream_of(q))
    _lib.check(rc, _entry)
    return out


MAX_VERIFY_QUERIES = 16  # queries per sequence nimbus_paged_verify takes


def verify_workspace_bytes(batch: int, queries_per_seq: int, heads: int, head_dim: int, max_context: int) -> int:
    return int(_lib.load().nimbus_paged_verify_workspace_bytes(batch, queries_per_seq, heads, head_dim,
                                                                max_context))


def paged_verify_attention(
    q: torch.Tensor,  # [B * nq, H, D], sequence b's queries in rows b * nq .. b * nq + nq - 1
    k_cache: torch.Tensor,
    v_cache: torch.Tensor,
    context_lens: torch.Tensor,  # [B] int32, including the nq new tokens
    block_tables: torch.Tensor,  # [B, max_blocks] int32
    queries_per_seq: int,
    max_context: int,
    scale: float,
    out: torch.Tensor | None = None,
    workspace: torch.Tensor | None = None,
) -> torch.Tensor:
    """Causal attention of each sequence's newest queries_per_seq tokens over
    its paged cache (nimbus_paged_verify): what paged_prefill_attention
    computes for query_start = arange(B + 1) * queries_per_seq, with the
    page-split decode kernels reading each K/V page once for all the queries.

    Query j of sequence b sits at position context_lens[b] - nq + j and sees
    keys up to it. max_context bounds every context length, as for decode;
    the launch grid depends on it and on the shapes only. `workspace`: as
    for paged_decode_attention, at least verify_workspace_bytes().
    """
    nq = int(queries_per_seq)
    if q.dim() != 3:
        raise ValueError(f"q must be [B * nq, H, D], got {tuple(q.shape)}")
    t, h, d = q.shape
    _check_cache(k_cache, v_cache)
    kv = k_cache.shape[2]
    if k_cache.shape[3] != d or h % kv != 0:
        raise ValueError(f"q {tuple(q.shape)} does not fit caches {tuple(k_cache.shape)}")
    if q.dtype != k_cache.dtype:
        raise ValueError("q and the caches must share one dtype")
    if not 1 <= nq <= MAX_VERIFY_QUERIES:
        raise ValueError(f"queries_per_seq must be in 1..{MAX_VERIFY_QUERIES}, got {nq}")
    if context_lens.dtype != torch.int32 or block_tables.dtype != torch.int32:
        raise ValueError("context_lens and block_tables must be int32")
    b = context_lens.shape[0]
    if context_lens.dim() != 1 or t != b * nq or block_tables.dim() != 2 or block_tables.shape[0] != b:
        raise ValueError(f"q must hold {nq} rows per sequence of context_lens [B], block_tables [B, max_blocks]")
    if out is None:
        out = torch.empty_like(q)
    elif out.shape != q.shape or out.dtype != q.dtype or out.stride(-1) != 1:
        raise ValueError("out must match q's shape and dtype with unit last stride")
    if b == 0:
        return out
    if q.stride(-1) != 1:
        q = q.contiguous()
    context_lens = context_lens.contiguous()
    if block_tables.stride(1) != 1:
        block_tables = block_tables.contiguous()
    if index_checks.enabled():
        index_checks.check_tables(block_tables, context_lens, k_cache.shape[0], k_cache.shape[1])
    lib = _lib.load()
    need = lib.nimbus_paged_verify_workspace_bytes(b, nq, h, d, int(max_context))
    if workspace is not None:
        if workspace.numel() * workspace.element_size() < need or not workspace.is_cuda:
            raise ValueError(f"workspace smaller than the {need} bytes this call needs")
        ws = workspace
    else:
        ws = _cached_workspace(need, q.device)
    rc = lib.nimbus_paged_verify(
        nq, q.data_ptr(), q.stride(0), q.stride(1), k_cache.data_ptr(), v_cache.data_ptr(), k_cache.shape[0],
        k_cache.stride(0), k_cache.stride(1), k_cache.stride(2), block_tables.data_ptr(), block_tables.stride(0),
        block_tables.shape[1], context_lens.data_ptr(), out.data_ptr(), out.stride(0), out.stride(1),
        ws.data_ptr(), ws.numel() * ws.element_size(), b, h, kv, d, k_cache.shape[1], int(max_context), float(scale),
        _lib.dtype_code(q.dtype), _lib.stream_of(q))
    _lib.check(rc, "nimbus_paged_verify")
    return out


def paged_decode_attention_noalloc(
    q: torch.Tensor,  # [B, H, D], unit last stride
    k_cache: torch.Tensor,
    v_cache: torch.Tensor,
    context_lens: torch.Tensor,  # [B] int32, contiguous
    block_tables: torch.Tensor,  # [B, max_blocks] int32, unit stride along a row
    max_context: int,
    scale: float,
    out: torch.Tensor,  # [B, H, D], unit last stride
) -> torch.Tensor:
    """paged_decode_attention without any device allocation, for callers
    that cannot allocate (nimbus_paged_decode_noalloc): the workspace is a
    device array inside the library, one per device, shared by every call
    on it, so calls that overlap on one device (several streams) race.
    Inputs must already be in the layout the kernels read and `out` must be
    given: nothing is copied or allocated here. A call needing more
    workspace than the array holds (_lib.NOALLOC_SCRATCH_BYTES; config 3
    needs ~35 MB of its 64 MiB) raises ValueError without launching."""
    if q.dim() != 3 or out.shape != q.shape or out.dtype != q.dtype:
        raise ValueError("q and out must both be [B, H, D] of one dtype")
    b, h, d = q.shape
    _check_cache(k_cache, v_cache)
    kv = k_cache.shape[2]
    if k_cache.shape[3] != d or h % kv != 0 or q.dtype != k_cache.dtype:
        raise ValueError(f"q {tuple(q.shape)} {q.dtype} does not fit caches {tuple(k_cache.shape)}")
    if q.stride(-1) != 1 or out.stride(-1) != 1 or not context_lens.is_contiguous() or block_tables.stride(1) != 1:
        raise ValueError("q/out need unit last stride, context_lens contiguity and block-table rows unit stride "
                         "(the allocation-free call copies nothing)")
    if context_lens.dtype != torch.int32 or block_tables.dtype != torch.int32:
        raise ValueError("context_lens and block_tables must be int32")
    if context_lens.shape != (b,) or block_tables.dim() != 2 or block_tables.shape[0] != b:
        raise ValueError("context_lens must be [B] and block_tables [B, max_blocks]")
    if b == 0:
        return out
    lib = _lib.load()
    rc = lib.nimbus_paged_decode_noalloc(
        q.data_ptr(), q.stride(0), q.stride(1), k_cache.data_ptr(), v_cache.data_ptr(), k_cache.shape[0],
        k_cache.stride(0), k_cache.stride(1), k_cache.stride(2), block_tables.data_ptr(), block_tables.stride(0),
        block_tables.shape[1], context_lens.data_ptr(), out.data_ptr(), out.stride(0), out.stride(1), b, h, kv, d,
        k_cache.shape[1], int(max_context), float(scale), _lib.dtype_code(q.dtype), _lib.stream_of(q))
    _lib.check(rc, "nimbus_paged_decode_noalloc")
    return out
