"""Causal varlen paged prefill attention on the GPU.

Drop-in for nimbus/kernels/prefill_attention.py:81-119 (`build_programs` and
`paged_prefill_attention`), computed by paged_prefill_kernel in
csrc/paged_prefill.hip. A sequence's queries are its newest q_len tokens;
query j sits at absolute position ctx - q_len + j. This covers fresh prompts
(q_len == ctx), chunked prefill over a cached prefix and speculative
verification of several draft tokens.

A batch in which every sequence has the same short q_len (speculative
verification: k + 1 tokens each, nimbus/spec/engine.py:84-96) runs instead
on the page-split decode kernels through nimbus_paged_verify, which read
each K/V page once for all of a sequence's queries; the tile kernel would
spend a 64-row tile on a handful of queries.
"""

from __future__ import annotations

from dataclasses import dataclass

import numpy as np
import torch

from nimbus_amd import _lib
from nimbus_amd.kernels import index_checks
from nimbus_amd.kernels.paged_attention import (MAX_VERIFY_QUERIES, _cached_workspace, _check_cache,
                                                paged_verify_attention)

BLOCK_M = 64  # query positions per tile-table entry (NIMBUS_PREFILL_TILE)
# Tiles whose workgroups all fit the chip at once: a GQA tile is typically 16
# workgroups (kv-head groups x sub-tiles), and 256 CUs hold two each.
PAIRED_TILES = 32
# Tables up to this many tiles (about two rounds of workgroups) go strictly
# heaviest tile first, so the few that start late are the lightest.
LPT_TILES = 64
# The verify form takes a batch while a sequence's queries times the heads of
# a kv group fit this many MFMA columns: each 16 columns more read every K/V
# page once more.
VERIFY_MAX_COLUMNS = 32
MAX_VERIFY_SEQUENCES = 4096  # the decode kernels' batch limit


def verify_queries(query_start_host: list[int], num_heads: int, num_kv_heads: int) -> int:
    """q_len if every sequence of the batch has the same q_len and the verify
    form takes it (see VERIFY_MAX_COLUMNS), else 0."""
    n = len(query_start_host) - 1
    if not 1 <= n <= MAX_VERIFY_SEQUENCES or query_start_host[0] != 0:
        return 0
    nq = query_start_host[1]
    if not 1 <= nq <= MAX_VERIFY_QUERIES or query_start_host[-1] != n * nq:
        return 0
    if nq * (num_heads // num_kv_heads) > VERIFY_MAX_COLUMNS:
        return 0
    if n > 1 and not np.all(np.diff(np.asarray(query_start_host, dtype=np.int64)) == nq):
        return 0
    return nq


def build_programs(query_start_host: list[int], device,
                   context_lens_host: list[int] | None = None) -> tuple[torch.Tensor, torch.Tensor]:
    """(sequence index, first query offset) for every BLOCK_M query tile.

    Without context_lens_host this is the table of
    nimbus/kernels/prefill_attention.py:81-90, in the same order, built with
    NumPy instead of a Python loop and moved to the device in one copy.
    Nimbus's backend builds it once per step and reuses it in every layer
    (model/attention.py:82-83).

    With context_lens_host (not in the reference signature; the backend
    passes it) the same entries are ordered for the MI355X launch. A tile's
    cost is the keys its last query sees. Sequences go heaviest first (by
    the sum of their tiles' costs), each sequence's tiles together and
    heaviest first: tiles of one sequence read the same K/V pages, so
    keeping them adjacent keeps them resident together and their pages in
    L2, and a longer table ends on light tiles. A table short enough that
    all its workgroups start at once (at most PAIRED_TILES tiles) has its
    second half reversed instead, so that workgroups launched half a grid
    apart, which share a CU, pair a heavy tile with a light one. A table of
    up to LPT_TILES tiles, whose last workgroups wait for a free slot, goes
    strictly heaviest tile first (measured 6% faster than sequence order on
    config 2's 36 tiles), so the late starters are the light ones.
    """
    qs = np.asarray(query_start_host, dtype=np.int64)
    lens = np.diff(qs) if qs.size > 1 else np.zeros(0, dtype=np.int64)
    tiles = (lens + BLOCK_M - 1) // BLOCK_M
    seqs = np.repeat(np.arange(lens.size, dtype=np.int64), tiles)
    first = np.repeat(np.cumsum(tiles) - tiles, tiles)
    starts = (np.arange(seqs.size) - first) * BLOCK_M
    if context_lens_host is not None and seqs.size > 1:
        ctx = np.asarray(context_lens_host, dtype=np.int64)
        cost = np.minimum(ctx[seqs], ctx[seqs] - lens[seqs] + starts + BLOCK_M)
        seq_cost = np.bincount(seqs, weights=cost, minlength=lens.size)[seqs]
        if PAIRED_TILES < seqs.size <= LPT_TILES:
            order = np.lexsort((starts, seqs, -cost))  # last key is the primary one
        else:
            order = np.lexsort((-cost, seqs, -seq_cost))
        if order.size <= PAIRED_TILES:
            half = (order.size + 1) // 2
            order = np.concatenate([order[:half], order[half:][::-1]])
        seqs, starts = seqs[order], starts[order]
    t = _to_device(np.stack([seqs, starts]).astype(np.int32), device)
    return t[0], t[1]


def _to_device(arr: np.ndarray, device) -> torch.Tensor:
    """arr on the device through pinned host memory (an asynchronous copy;
    torch's pinned-memory cache keeps the host block until the copy is done).
    A copy from pageable memory would wait for the host-side staging."""
    if torch.device(device).type != "cuda":
        return torch.from_numpy(arr).to(device)
    host = torch.empty(arr.shape, dtype=torch.from_numpy(arr[:0]).dtype, pin_memory=True)
    host.numpy()[...] = arr
    return host.to(device, non_blocking=True)


# The last tile table built for a call without one: (key, table). Eager callers
# that pass programs=None with the same host lists (every layer of a step)
# reuse it instead of building and copying it again.
_LAST_TABLE: list = [None, None]


KEY_BLOCK = 64  # keys per block of the prefill kernel's walk
RESIDENT_WORKGROUPS = 512  # prefill workgroups a gfx950 part holds at once (256 CUs x 2)


@dataclass
class PrefillPieces:
    """A tile table whose heavy tiles' key ranges are cut into pieces
    (nimbus_paged_prefill_pieces): pieces [n, 5] and merges [m, 4] int32 on
    the device, and the workspace slots the split pieces use."""

    pieces: torch.Tensor
    merges: torch.Tensor
    num_slots: int


def _units_per_tile(num_heads: int, num_kv_heads: int) -> int:
    g = num_heads // num_kv_heads
    gs = 8 if g % 8 == 0 else 4 if g % 4 == 0 else 2 if g % 2 == 0 else 1
    pos = min(128 // gs, BLOCK_M)
    return (BLOCK_M // pos) * num_kv_heads * (g // gs)


def plan_pieces(query_start_host: list[int], context_lens_host: list[int], num_heads: int, num_kv_heads: int,
                device, resident: int = RESIDENT_WORKGROUPS) -> PrefillPieces | None:
    """Key-range pieces for a batch with fewer tiles than the chip holds at
    once (a short chunk over a long cached prefix, say), so that idle CUs
    take part of the heavy tiles' key walks; None otherwise, or when
    splitting would not shorten the walk. (With the chip full, two tiles per
    CU and the cost order pairing heavy with light already balance the work,
    and pieces only add partial writes and a merge: measured slower.)

    A tile's cost is the key blocks its last query sees. With H tiles held
    on the chip at once, pieces aim at S = max(4, ceil(total blocks / H))
    blocks: a tile of more than 1.25 S blocks is cut into ceil(blocks / S)
    near-equal ranges. Pieces go heaviest first."""
    qs = np.asarray(query_start_host, dtype=np.int64)
    if qs.size < 2:
        return None
    lens = np.diff(qs)
    tiles = (lens + BLOCK_M - 1) // BLOCK_M
    seqs = np.repeat(np.arange(lens.size, dtype=np.int64), tiles)
    if seqs.size == 0:
        return None
    first = np.repeat(np.cumsum(tiles) - tiles, tiles)
    starts = (np.arange(seqs.size) - first) * BLOCK_M
    ctx = np.asarray(context_lens_host, dtype=np.int64)
    keys = np.maximum(np.minimum(ctx[seqs], ctx[seqs] - lens[seqs] + starts + BLOCK_M), 0)
    blocks = (keys + KEY_BLOCK - 1) // KEY_BLOCK
    hold = max(1, resident // _units_per_tile(num_heads, num_kv_heads))
    if seqs.size >= hold:
        return None  # the tiles fill the chip: two per CU, heavy paired with light, keep it busy already
    s = max(4, -(-int(blocks.sum()) // hold))
    if blocks.max() <= 1.25 * s:
        return None
    rows, merges, slot = [], [], 0
    for sq, m0, nb in zip(seqs.tolist(), starts.tolist(), blocks.tolist()):
        k = -(-nb // s) if nb > 1.25 * s else 1
        if k == 1:
            rows.append((nb, sq, m0, 0, 2**31 - 1, -1))
            continue
        edges = [round(i * nb / k) for i in range(k + 1)]
        merges.append((sq, m0, slot, k))
        for i in range(k):
            rows.append((edges[i + 1] - edges[i], sq, m0, edges[i], edges[i + 1], slot + i))
        slot += k
    rows.sort(key=lambda r: -r[0])
    table = np.asarray([r[1:] for r in rows], dtype=np.int32)
    t = _to_device(table, device)
    mt = _to_device(np.asarray(merges, dtype=np.int32).reshape(-1, 4), device)
    return PrefillPieces(t, mt, slot)


@dataclass
class PrefillStream:
    """A stream-K plan (nimbus_paged_prefill_stream): the batch's (unit, key
    block) work laid end to end per kv-head group and cut into `num_shares`
    equal contiguous shares, one workgroup each, every workgroup resident at
    once. share_start [num_shares + 1] and pieces [n, 8] int32 live on the
    device; the plan holds for the head shape it was made for."""

    share_start: torch.Tensor
    pieces: torch.Tensor
    num_shares: int
    num_heads: int
    num_kv_heads: int


SK_FIELDS = 8  # int32 per piece record: seq, m0, kb0, kb1, slot, fix_lo, fix_hi, 0
MIN_SHARE_BLOCKS = 2  # a share covers at least this many key blocks, unless units alone need more shares
_CUS: dict[int, int] = {}


def _resident_workgroups(device) -> int:
    """Prefill workgroups the device holds at once: two per CU."""
    dev = torch.device(device)
    if dev.type != "cuda":
        return RESIDENT_WORKGROUPS
    index = dev.index if dev.index is not None else torch.cuda.current_device()
    if index not in _CUS:
        _CUS[index] = torch.cuda.get_device_properties(index).multi_processor_count
    return 2 * _CUS[index]


def stream_units(query_start_host: list[int], context_lens_host: list[int], num_heads: int, num_kv_heads: int):
    """The units of one kv-head group in stream order (sequence, then query
    position): (sequence, first query, key blocks) arrays, and the number of
    kv-head groups. A unit is POS = min(128 / GS, 64) query positions of GS
    query heads (the kernel's 128 rows); its key blocks are the 64-key blocks
    its last query sees."""
    g = num_heads // num_kv_heads
    gs = 8 if g % 8 == 0 else 4 if g % 4 == 0 else 2 if g % 2 == 0 else 1
    pos = min(128 // gs, BLOCK_M)
    qs = np.asarray(query_start_host, dtype=np.int64)
    lens = np.diff(qs) if qs.size > 1 else np.zeros(0, dtype=np.int64)
    ctx = np.asarray(context_lens_host, dtype=np.int64)
    nu = (np.maximum(lens, 0) + pos - 1) // pos
    useq = np.repeat(np.arange(lens.size, dtype=np.int64), nu)
    um0 = (np.arange(useq.size) - np.repeat(np.cumsum(nu) - nu, nu)) * pos
    kv_end = np.clip(np.minimum(ctx[useq], ctx[useq] - lens[useq] + um0 + pos), 0, None)
    return useq, um0, (kv_end + KEY_BLOCK - 1) // KEY_BLOCK, num_kv_heads * (g // gs)


def plan_stream(query_start_host: list[int], context_lens_host: list[int], num_heads: int, num_kv_heads: int,
                device, resident: int | None = None, min_share: int = MIN_SHARE_BLOCKS) -> PrefillStream | None:
    """Stream-K plan of a prefill batch; None when it has no queries.

    Per kv-head group, the units' key blocks are laid end to end (a unit
    with none counts one) and cut into S equal contiguous shares, S = the
    workgroups the chip holds at once per group, fewer for a short batch
    (shares of at least MIN_SHARE_BLOCKS blocks, but at least one share per
    unit). Workgroup (share j, group g) is grid index j * groups + g, so a
    group keeps its XCDs and their L2 as in the tile grid. A unit inside one
    share is written whole. A unit cut by share boundaries is finished by the
    share holding its last blocks (the fixer), which folds in the (O, m, l)
    pieces the lower shares wrote (contributors); every wait is therefore on
    a lower-numbered workgroup, dispatched earlier. Each share runs its
    pieces last-first: its contributor piece (the head of the unit it shares
    with the next share) first, so that piece is ready long before its fixer
    asks for it, and its fixer piece last."""
    useq, um0, nb, kvg = stream_units(query_start_host, context_lens_host, num_heads, num_kv_heads)
    n = useq.size
    if n == 0:
        return None
    cost = np.maximum(nb, 1)
    total = int(cost.sum())
    held = (resident or _resident_workgroups(device)) // kvg
    if held < 1:
        raise ValueError("the device holds fewer workgroups than one per kv-head group")
    shares = max(1, min(held, max(n, -(-total // min_share))))
    bounds = (np.arange(shares + 1, dtype=np.int64) * total) // shares
    ustart = np.cumsum(cost) - cost
    j0 = np.searchsorted(bounds, ustart, side="right") - 1
    j1 = np.searchsorted(bounds, ustart + cost - 1, side="right") - 1
    npc = j1 - j0 + 1
    pu = np.repeat(np.arange(n), npc)                              # unit of each piece
    pj = np.repeat(j0, npc) + (np.arange(pu.size) - np.repeat(np.cumsum(npc) - npc, npc))  # its share
    kb0 = np.maximum(bounds[pj], ustart[pu]) - ustart[pu]
    kb1 = np.minimum(bounds[pj + 1], ustart[pu] + cost[pu]) - ustart[pu]
    first, last = pj == j0[pu], pj == j1[pu]
    kb0[first] = 0
    kb1[last] = 2**31 - 1
    split = npc[pu] > 1
    slot = np.where(split & ~last, pj, -1)
    fix_lo = np.where(split & last, j0[pu], 0)
    fix_hi = np.where(split & last, j1[pu], 0)
    order = np.lexsort((-pu, pj))  # by share, then last piece first
    rec = np.zeros((pu.size, SK_FIELDS), dtype=np.int32)
    for col, arr in enumerate((useq[pu], um0[pu], kb0, kb1, slot, fix_lo, fix_hi)):
        rec[:, col] = arr[order]
    start = np.zeros(shares + 1, dtype=np.int32)
    start[1:] = np.cumsum(np.bincount(pj, minlength=shares))
    return PrefillStream(_to_device(start, device), _to_device(rec, device), shares, num_heads, num_kv_heads)


def stream_workspace_bytes(num_shares: int, heads: int, kv_heads: int, head_dim: int) -> int:
    """Workspace bytes of a PrefillStream plan of num_shares shares."""
    return int(_lib.load().nimbus_paged_prefill_stream_workspace_bytes(num_shares, heads, kv_heads, head_dim))


# Stream-K workspaces per (device, stream), zeroed when allocated: the plan's
# flags must start at zero, and every call that completes leaves them zero.
# Outgrown ones stay alive (a captured graph may still use them).
_STREAM_WORKSPACES: dict[tuple[int, int], torch.Tensor] = {}
_STREAM_OUTGROWN: list[torch.Tensor] = []


def new_stream_workspace(nbytes: int, device) -> torch.Tensor:
    """A zeroed workspace for nimbus_paged_prefill_stream calls of up to nbytes."""
    return torch.zeros(max(int(nbytes), 256), dtype=torch.uint8, device=device)


def _stream_workspace(nbytes: int, device: torch.device) -> torch.Tensor:
    index = device.index if device.index is not None else torch.cuda.current_device()
    key = (index, torch._C._cuda_getCurrentRawStream(index))
    ws = _STREAM_WORKSPACES.get(key)
    if ws is None or ws.numel() < nbytes:
        if ws is not None:
            _STREAM_OUTGROWN.append(ws)
        ws = _STREAM_WORKSPACES[key] = new_stream_workspace(max(nbytes, 8 << 20), device)
    return ws


def stream_error(workspace: torch.Tensor, num_shares: int, heads: int, kv_heads: int) -> int:
    """The error word of a stream-K workspace (nonzero once a fix-up wait gave
    up: the plan was inconsistent); reads the device."""
    off = int(_lib.load().nimbus_paged_prefill_stream_flag_bytes(num_shares, heads, kv_heads)) - 256
    return int(workspace[off:off + 4].view(torch.int32).item())


_PIECES_WORKSPACES: dict = {}  # the pieces plans' workspaces (a family apart from the decode ones)


def pieces_workspace_bytes(num_slots: int, heads: int, head_dim: int) -> int:
    """Workspace bytes of a PrefillPieces plan with num_slots split slots."""
    return int(_lib.load().nimbus_paged_prefill_pieces_workspace_bytes(num_slots, heads, head_dim))


def paged_prefill_attention(
    q: torch.Tensor,  # [Tp, H, D]
    k_cache: torch.Tensor,
    v_cache: torch.Tensor,
    query_start: torch.Tensor,  # [P+1] int32
    context_lens: torch.Tensor,  # [P] int32
    block_tables: torch.Tensor,  # [P, max_blocks] int32
    scale: float,
    query_start_host: list[int],
    context_lens_host: list[int],
    programs: tuple[torch.Tensor, torch.Tensor] | None = None,
    out: torch.Tensor | None = None,
    workspace: torch.Tensor | None = None,
    kernel: str = "auto",
) -> torch.Tensor:
    """Causal attention of each sequence's newest tokens over its paged cache.

    The cache must already hold the new tokens' K/V (write_kv runs first, as
    in nimbus/model/attention.py:78). `programs` is build_programs' tile table
    (built here when None), or a PrefillPieces plan (plan_pieces) that cuts
    heavy tiles' key ranges. Not in the reference signature: `out` receives
    the result in place; `kernel` is "auto" (the verify form when
    verify_queries() takes the batch, else the tile kernel), "tile" or
    "verify"; `workspace` is the verify form's or the pieces' (by default
    the per-stream cached one).

    The verify form bounds context lengths by the block-table width (16
    tokens a column), not by context_lens_host: Nimbus's verify graphs pass
    placeholder host context lengths (spec/engine.py:94).
    """
    if kernel not in ("auto", "tile", "verify"):
        raise ValueError(f"kernel must be 'auto', 'tile' or 'verify', got {kernel!r}")
    if q.dim() != 3:
        raise ValueError(f"q must be [Tp, H, D], got {tuple(q.shape)}")
    t, h, d = q.shape
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
    if t == 0 or len(query_start_host) < 2:
        return out
    for x, name in ((query_start, "query_start"), (context_lens, "context_lens"), (block_tables, "block_tables")):
        if x.dtype != torch.int32:
            raise ValueError(f"{name} must be int32")
    if block_tables.dim() != 2 or block_tables.shape[0] != len(query_start_host) - 1:
        raise ValueError("block_tables must be [P, max_blocks]")
    nq = verify_queries(query_start_host, h, kv) if kernel != "tile" else 0
    if kernel == "verify" and nq == 0:
        raise ValueError("the verify form needs 1..16 queries in every sequence, fitting "
                         f"{VERIFY_MAX_COLUMNS} columns per kv group")
    if nq:
        return paged_verify_attention(q, k_cache, v_cache, context_lens, block_tables, nq,
                                      block_tables.shape[1] * k_cache.shape[1], scale, out=out, workspace=workspace)
    if index_checks.enabled():
        index_checks.check_tables(block_tables, context_lens, k_cache.shape[0], k_cache.shape[1])
    if programs is None:
        key = (q.device, tuple(query_start_host), tuple(context_lens_host))
        if _LAST_TABLE[0] != key or torch.cuda.is_current_stream_capturing():
            _LAST_TABLE[1] = build_programs(query_start_host, q.device, context_lens_host)
            _LAST_TABLE[0] = key
        programs = _LAST_TABLE[1]
    if q.stride(-1) != 1:
        q = q.contiguous()
    if block_tables.stride(1) != 1:
        block_tables = block_tables.contiguous()
    query_start = query_start.contiguous()
    context_lens = context_lens.contiguous()
    lib = _lib.load()
    common = (q.data_ptr(), q.stride(0), q.stride(1), k_cache.data_ptr(), v_cache.data_ptr(), k_cache.shape[0],
              k_cache.stride(0), k_cache.stride(1), k_cache.stride(2), block_tables.data_ptr(),
              block_tables.stride(0), block_tables.shape[1], query_start.data_ptr(), context_lens.data_ptr())
    tail = (out.data_ptr(), out.stride(0), out.stride(1), h, kv, d, k_cache.shape[1], float(scale),
            _lib.dtype_code(q.dtype), _lib.stream_of(q))
    if isinstance(programs, PrefillStream):
        if (programs.num_heads, programs.num_kv_heads) != (h, kv):
            raise ValueError("the stream plan was made for another head shape")
        need = lib.nimbus_paged_prefill_stream_workspace_bytes(programs.num_shares, h, kv, d)
        if workspace is not None:
            if workspace.nbytes < need or not workspace.is_cuda:
                raise ValueError(f"workspace smaller than the {need} bytes this call needs")
            ws = workspace
        else:
            ws = _stream_workspace(need, q.device)
        rc = lib.nimbus_paged_prefill_stream(*common, programs.share_start.data_ptr(), programs.pieces.data_ptr(),
                                             programs.num_shares, ws.data_ptr(), ws.nbytes, *tail)
        _lib.check(rc, "nimbus_paged_prefill_stream")
        return out
    if isinstance(programs, PrefillPieces):
        need = lib.nimbus_paged_prefill_pieces_workspace_bytes(programs.num_slots, h, d)
        if workspace is not None:
            if workspace.numel() * workspace.element_size() < need or not workspace.is_cuda:
                raise ValueError(f"workspace smaller than the {need} bytes this call needs")
            ws = workspace
        else:
            ws = _cached_workspace(need, q.device, _PIECES_WORKSPACES)
        rc = lib.nimbus_paged_prefill_pieces(
            *common, programs.pieces.data_ptr(), programs.pieces.shape[0], programs.merges.data_ptr(),
            programs.merges.shape[0], programs.num_slots, ws.data_ptr(), ws.numel() * ws.element_size(), *tail)
        _lib.check(rc, "nimbus_paged_prefill_pieces")
        return out
    prog_seq, prog_m = programs
    if prog_seq.numel() == 0:
        return out
    rc = lib.nimbus_paged_prefill(*common, prog_seq.data_ptr(), prog_m.data_ptr(), prog_seq.numel(), *tail)
    _lib.check(rc, "nimbus_paged_prefill")
    return out
