#!/usr/bin/env python3
"""Benchmark of the paged-attention hot path on one MI355X.

    python bench.py [--steps K] [--warmup W] [--all] [--no-cpu-baseline]

Prints ONE JSON line. Configs 1-5 are nimbus_amd.workloads' five numbered
configurations. The headline is config 3: Llama-3-8B-shaped
paged decode attention (B=64, H=32, KV=8, D=128, bf16, contexts log-uniform
in [128, 8192], K/V pages scattered over a pool 1.2x the pages needed).
A step is one paged_decode_attention call on inputs already resident in HBM.

value        algorithmic bytes of one call / wall time per step (GB/s):
             every visible K and V row once, q and out once, the page ids and
             context lengths (nimbus_amd.workloads.decode_bytes)
roofline     the whole decode call (paged_decode_kernel, the page pass, then
             paged_decode_merge_kernel, the split merge), K calls back to back
             between one HIP event pair on the launch stream: algorithmic
             bytes / mean time per call, against 8 TB/s
             (`kernel_us_event_pairs`: the mean with an event pair around
             each call, which adds its dispatch latency); `page_pass` gives
             the page pass alone the same way; `traffic` is the HBM bytes per
             call (both kernels) that rocprofv3 FETCH_SIZE + WRITE_SIZE
             counted on this workload (profiles/decode_llama3_traffic.json,
             scaled by the plain-copy calibration), null when absent or
             measured on other decode sources (a sha256 of them is kept)
cpu_baseline the CPU oracle (restated nimbus/kernels/reference.py:71-96,
             batched exact form) on this host's cores, same inputs; `entries`
             adds config 4's prefill part through the prefill oracle
             (reference.py:37-68) and config 5 through the per-row decode
             form, each a bounded sample
reference_shapes the reference's own kernel micro-bench shapes
             (bench/kernels.py:54-74: TinyLlama heads, fp16) beside its
             published numbers (other hardware)
prefill      config 4's prefill part (4 chunks of 512 over cached
             prefixes of up to 1024): causal FLOPs / mean time per call of K
             back-to-back calls, against the 2.5 PFLOP/s dense bf16 MFMA peak
prefill_scaling the same prefill kernel on two larger workloads (not among
             configs 1-5): one 8192-token prompt, and 64 chunks of 512 over
             2048-token cached prefixes; at most 20 timed calls each
mixed_step   the whole config-4 step: slot write of 2,108 tokens + prefill
             (eager) + the 60 decodes replayed from a hipGraph padded to 64;
             `write_kv` is the slot write of all 2,108 tokens alone (k and v
             rows read and written + slots, against 8 TB/s)
verify       speculative verification's attention (16 sequences x 5 tokens)
             replayed from a hipGraph, with the decode kernel on the same
             contexts beside it; `attention_us_graph` and
             `decode_same_contexts_us_graph` compare the two attention calls
             alone (no slot write), each as back-to-back calls in a hipGraph
add_rms_norm the fused residual add + RMSNorm at three model shapes:
             algorithmic bytes (x and residual read, residual and output
             written, weight once) / mean kernel time, against 8 TB/s
decode_step  a whole Llama-3-8B-shaped decode step (random weights, config 3's
             64 sequences): eager, graph replay and on-device greedy chain,
             bf16 and INT8 projections; bytes (weights + K/V) / step time
int8_matmul  the INT8 weight-only matmul at Llama-3-8B decode projections
             (and Nimbus's own TinyLlama bench shape): algorithmic bytes
             (int8 weights, x, y, scales) / mean kernel time, against 8 TB/s,
             beside torch's dense matmul on the dequantized weights

other_configs configs 1, 2 and 5 in compact form (at most 50
             timed calls each); they run before the headline, which is
             thereby measured with the GPU's clocks settled (config 3's calls
             run 2-7% slower over the first ~150 calls of a fresh process)

Between timed calls the K/V pool rotates over enough copies (>= 1.5 GB) that
the 256 MB Infinity Cache cannot serve one call's pages to the next.

--all also times every config (1-5) (--all-out PATH writes the full rows as JSON).
"""

from __future__ import annotations

import argparse
import json
import math
import os
import statistics
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

METRIC = "paged-decode HBM GB/s & µs/call @Llama-3-8B shape; prefill TFLOP/s"
HBM_PEAK_GBS = 8000.0
MFMA_BF16_PEAK_TFLOPS = 2500.0
ROTATE_BYTES = 1.5e9


def parse(argv=None):
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--all", action="store_true", help="also time every config (1-5)")
    ap.add_argument("--all-out", default=None, metavar="PATH", help="with --all: also write the full rows as JSON")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-prefill", action="store_true")
    ap.add_argument("--decode-only", action="store_true",
                    help="the headline, then the other decode configs (1 and 5) only: for kernel traces")
    ap.add_argument("--cpu-seconds", type=float, default=25.0, help="bound on the CPU baseline's timed work")
    ap.add_argument("--copy-calibration", type=int, default=0, metavar="MIB",
                    help="also run a plain device copy of MIB MiB 5 times (the reference kernel for scaling "
                         "rocprofv3 FETCH_SIZE/WRITE_SIZE readings to bytes)")
    return ap.parse_args(argv)


def copy_calibration(mib):
    """A plain copy kernel of known size: reads and writes mib MiB per launch."""
    import torch

    src = torch.empty(mib << 20, dtype=torch.uint8, device="cuda").random_(0, 255)
    dst = torch.empty_like(src)
    torch.cuda.synchronize()
    for _ in range(5):
        dst.copy_(src)
    torch.cuda.synchronize()
    log(f"copy calibration: 5 copies of {mib} MiB ({mib * 1024} KiB read and written per launch)")
    del src, dst


def log(msg):
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


TRAFFIC_RECORD = os.path.join(ROOT, "profiles", "decode_llama3_traffic.json")
# The files the decode kernels' code comes from (the public header and the
# internal one only add declarations and constants those kernels do not use).
DECODE_SOURCES = ("nimbus_amd/csrc/paged_decode.hip", "nimbus_amd/csrc/common.h")


def decode_source_hash():
    """sha256 over the sources the decode kernels are compiled from, so a
    traffic record measured on other code is recognised as stale."""
    import hashlib

    h = hashlib.sha256()
    for rel in DECODE_SOURCES:
        with open(os.path.join(ROOT, rel), "rb") as f:
            h.update(rel.encode() + b"\0" + f.read())
    return h.hexdigest()


def measured_traffic(algorithmic_bytes):
    """HBM bytes of one decode call (page pass + merge pass) on this workload
    as rocprofv3 counted them (FETCH_SIZE + WRITE_SIZE per dispatch, scaled
    by the plain-copy calibration), from the committed record; None when the
    record is absent, was measured on another workload, or on other decode
    sources than the ones built here."""
    try:
        with open(TRAFFIC_RECORD) as f:
            rec = json.load(f)
    except (OSError, ValueError):
        return None
    if rec.get("algorithmic_bytes") != algorithmic_bytes or rec.get("source_sha256") != decode_source_hash():
        return None
    return rec.get("traffic_bytes")


# ---------------------------------------------------------------- timing helpers

def region_us(fn, steps, stream):
    """Runs fn(i) for i < steps back to back between one HIP event pair on
    `stream`; returns the mean time per call in microseconds (each launch's
    duration plus the gap to the next one, as a stream of calls sees it)."""
    import torch

    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record(stream)
    for i in range(steps):
        fn(i)
    end.record(stream)
    torch.cuda.synchronize()
    return start.elapsed_time(end) * 1e3 / steps


def warm_up(fn, calls, min_seconds=0.05):
    """Runs fn(i) `calls` times, then keeps calling it until the GPU has been
    busy with it for min_seconds: the clocks reach their steady state under a
    heavy kernel only after some tens of milliseconds (an 8192-token prefill
    runs 786 us per call in its first 10 calls and 508 us from the 50th on), so
    a count of calls alone leaves long kernels timed on a cold chip."""
    import torch

    for i in range(calls):
        fn(i)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    i = calls
    while time.perf_counter() - t0 < min_seconds:
        for _ in range(8):
            fn(i)
            i += 1
        torch.cuda.synchronize()


def event_times_us(fn, steps, stream):
    """Runs fn(i) for i < steps with a HIP event pair around each call on
    `stream`; returns the per-call durations in microseconds."""
    import torch

    evs = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(steps)]
    for i in range(steps):
        evs[i][0].record(stream)
        fn(i)
        evs[i][1].record(stream)
    torch.cuda.synchronize()
    return [a.elapsed_time(b) * 1e3 for a, b in evs]


def graph_us(fn, calls, stream, reps=7):
    """Captures fn(i) for i < calls into one hipGraph, replays it (3 untimed,
    then `reps` timed replays, one HIP event pair each on `stream`) and returns
    the median time per call in microseconds: the device's time per call with
    no host launch cost between calls, as a serving loop replays decode."""
    import torch

    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        for i in range(calls):
            fn(i)
    for _ in range(3):
        g.replay()
    torch.cuda.synchronize()
    times = []
    for _ in range(reps):
        start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        start.record(stream)
        g.replay()
        end.record(stream)
        torch.cuda.synchronize()
        times.append(start.elapsed_time(end) * 1e3 / calls)
    del g
    return statistics.median(times)


def rotated_pools(batch, min_bytes=ROTATE_BYTES):
    """Copies of (q, k_cache, v_cache) so that consecutive calls read
    distinct memory; the first copy is the batch's own."""
    pool_bytes = 2 * batch.k_cache.numel() * batch.k_cache.element_size()
    n = max(2, math.ceil(min_bytes / pool_bytes))
    pools = [(batch.q, batch.k_cache, batch.v_cache)]
    for _ in range(n - 1):
        pools.append((batch.q.clone(), batch.k_cache.clone(), batch.v_cache.clone()))
    return pools


# ---------------------------------------------------------------- decode

def time_decode(batch, steps, warmup, wall=True):
    import torch

    from nimbus_amd import workloads
    from nimbus_amd.kernels.paged_attention import (decode_workspace_bytes, new_decode_workspace,
                                                    paged_decode_attention)

    p = batch.num_prefills
    t0 = batch.num_prefill_tokens
    ctx_lens = batch.decode_context_host()
    ctx = batch.context_lens[p:]
    bt = batch.block_tables[p:]
    maxc = max(ctx_lens)
    b = len(ctx_lens)
    h, d = batch.q.shape[1], batch.q.shape[2]
    kv = batch.k_cache.shape[2]
    pools = rotated_pools(batch)
    out = torch.empty_like(batch.q[t0:])
    ws = new_decode_workspace(decode_workspace_bytes(b, h, d, maxc), batch.q.device)
    stream = torch.cuda.current_stream()

    def call(i, entry="nimbus_paged_decode"):
        q, kc, vc = pools[i % len(pools)]
        paged_decode_attention(q[t0:], kc, vc, ctx, bt, maxc, batch.scale, out=out, workspace=ws, _entry=entry)

    # (time-based: the first timed section of a process would otherwise meet cold clocks and first-launch costs)
    warm_up(call, warmup)
    warm_up(lambda i: call(i, "nimbus_paged_decode_pages"), 2)
    res = {}
    if wall:
        torch.cuda.synchronize()
        w0 = time.perf_counter()
        for i in range(steps):
            call(i)
        torch.cuda.synchronize()
        res["ms_per_step"] = (time.perf_counter() - w0) * 1e3 / steps
    res["call_us"] = region_us(call, steps, stream)
    res["page_pass_us"] = region_us(lambda i: call(i, "nimbus_paged_decode_pages"), steps, stream)
    # the same with an event pair around each call (adds each launch's own dispatch latency)
    res["call_us_event_pairs"] = statistics.mean(event_times_us(call, steps, stream))
    res["page_pass_us_event_pairs"] = statistics.mean(event_times_us(lambda i: call(i, "nimbus_paged_decode_pages"),
                                                                     steps, stream))
    # the merge pass's share of a call (timed alone, a 5 us launch is bound by the host's launch rate)
    res["merge_us"] = res["call_us"] - res["page_pass_us"]
    # back-to-back calls replayed from one hipGraph (cycling the pools): no host launch cost
    res["call_us_graph"] = graph_us(call, max(len(pools), min(12, steps)), stream)
    res["bytes"] = workloads.decode_bytes(ctx_lens, h, kv, d, batch.q.element_size())
    res["pools"] = len(pools)
    res["batch"] = b
    res["sum_ctx"] = sum(ctx_lens)
    return res


def _cpu_model():
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return ""


def _timed_reps(fn, seconds, reps=3):
    """One warm-up call, then up to `reps` timed calls within `seconds`;
    returns (median seconds, timed reps)."""
    t = time.perf_counter()
    fn()
    first = time.perf_counter() - t
    times = []
    budget = time.perf_counter() + seconds
    while len(times) < reps and time.perf_counter() + first < budget:
        t = time.perf_counter()
        fn()
        times.append(time.perf_counter() - t)
    if not times:
        times = [first]
    return statistics.median(times), len(times)


def cpu_decode_baseline(batch, seconds):
    """The CPU oracle (batched exact form of nimbus/kernels/reference.py:71-96)
    on CPU copies of the same inputs, in their dtype: one warm-up, then up to
    3 timed reps within `seconds`."""
    import torch

    from nimbus_amd import workloads
    from oracle import reference

    p = batch.num_prefills
    t0 = batch.num_prefill_tokens
    ctx_lens = batch.decode_context_host()
    q = batch.q[t0:].cpu()
    kc, vc = batch.k_cache.cpu(), batch.v_cache.cpu()
    ctx = batch.context_lens[p:].cpu()
    bt = batch.block_tables[p:].cpu()
    maxc = max(ctx_lens)
    h, d, kv = q.shape[1], q.shape[2], kc.shape[2]
    med, n = _timed_reps(lambda: reference.paged_decode_attention(q, kc, vc, ctx, bt, maxc, batch.scale), seconds)
    nbytes = workloads.decode_bytes(ctx_lens, h, kv, d, q.element_size())
    return {
        "value": nbytes / med / 1e9,
        "unit": "GB/s",
        "cores": torch.get_num_threads(),
        "kind": "port",
        "sample": (f"config 3: the whole llama3_decode batch (B={len(ctx_lens)}, sum ctx {sum(ctx_lens)}) through the "
                   f"batched CPU oracle, median of {n} reps after 1 warm-up: {med * 1e3:.1f} ms/call; "
                   f"host {_cpu_model()}, os.cpu_count()={os.cpu_count()}"),
    }


def cpu_prefill_baseline(batch, seconds):
    """The CPU oracle of paged prefill (nimbus/kernels/reference.py:37-68) on
    CPU copies of config 4's prefill part, in their dtype."""
    import torch

    from nimbus_amd import workloads
    from oracle import reference

    pa = batch.prefill_args()
    q, kc, vc = pa[0].cpu(), batch.k_cache.cpu(), batch.v_cache.cpu()
    qs, ctx, bt = pa[3].cpu(), pa[4].cpu(), pa[5].cpu()
    med, n = _timed_reps(lambda: reference.paged_prefill_attention(q, kc, vc, qs, ctx, bt, batch.scale, pa[7], pa[8]),
                         seconds)
    seqs = batch.seqs[:batch.num_prefills]
    flops = workloads.prefill_flops(seqs, q.shape[1], q.shape[2])
    return {
        "value": flops / med / 1e12,
        "unit": "TFLOP/s",
        "cores": torch.get_num_threads(),
        "kind": "port",
        "sample": (f"config 4's prefill part (4 chunks of 512 on prefixes {[c - ql for c, ql in seqs]}, "
                   f"{flops / 1e9:.2f} GFLOP causal) through the CPU oracle, median of {n} reps after 1 warm-up: "
                   f"{med * 1e3:.1f} ms/call"),
    }


def cpu_long_decode_baseline(batch, seconds):
    """The per-row form of the decode oracle (oracle/reference.py's
    decode_attention_rows: the math of nimbus/kernels/reference.py:71-96 one
    sequence at a time; the batched form would gather a [256, 32768, 8, 128]
    tensor) on config 5, row by row in batch order until `seconds`
    of oracle time are spent: bytes of the rows done / their oracle time.
    Each row's pages are copied to the host before its timed call."""
    import torch

    from nimbus_amd import workloads
    from oracle import reference

    p = batch.num_prefills
    t0 = batch.num_prefill_tokens
    ctx_lens = batch.decode_context_host()
    q_all = batch.q[t0:]
    bt = batch.block_tables[p:]
    h, d, kv = q_all.shape[1], q_all.shape[2], batch.k_cache.shape[2]
    spent, done = 0.0, []
    for b, c in enumerate(ctx_lens):
        n = -(-c // 16)
        pages = bt[b, :n].long()
        kc, vc = batch.k_cache[pages].cpu(), batch.v_cache[pages].cpu()
        q = q_all[b:b + 1].cpu()
        table = torch.arange(n, dtype=torch.int32)[None]
        t = time.perf_counter()
        reference.decode_attention_rows(q, kc, vc, [c], table, batch.scale)
        spent += time.perf_counter() - t
        done.append(c)
        if spent >= seconds:
            break
    nbytes = workloads.decode_bytes(done, h, kv, d, q_all.element_size())
    return {
        "value": nbytes / spent / 1e9,
        "unit": "GB/s",
        "cores": torch.get_num_threads(),
        "kind": "port",
        "sample": (f"config 5, per-row form: the first {len(done)} of {len(ctx_lens)} rows in batch order "
                   f"(sum ctx {sum(done)} of {sum(ctx_lens)}), one oracle call per row, "
                   f"{spent:.1f} s of oracle time"),
    }


# ---------------------------------------------------------------- prefill and the mixed step

def time_prefill(batch, steps, warmup):
    import torch

    from nimbus_amd import workloads
    from nimbus_amd.kernels.prefill_attention import build_programs, paged_prefill_attention

    args = batch.prefill_args()
    progs = build_programs(args[7], batch.q.device, args[8])
    out = torch.empty_like(args[0])

    def call(i):
        paged_prefill_attention(*args, progs, out=out)

    warm_up(call, warmup)
    us = region_us(call, steps, torch.cuda.current_stream())
    us_pairs = statistics.mean(event_times_us(call, steps, torch.cuda.current_stream()))
    seqs = batch.seqs[:batch.num_prefills]
    h, d = batch.q.shape[1], batch.q.shape[2]
    flops = workloads.prefill_flops(seqs, h, d)
    nbytes = workloads.prefill_bytes(seqs, h, batch.k_cache.shape[2], d, batch.q.element_size())
    return {"us_per_call": us, "us_per_call_event_pairs": us_pairs, "flops": flops, "tflops": flops / us / 1e6,
            "bytes": nbytes, "tiles": int(progs[0].numel())}


def prefill_scaling(steps, warmup):
    """The config-4 prefill kernel (Llama-3-8B heads, bf16) where the chip is
    not bound by one unit's chain of key blocks: one 8192-token prompt, and
    64 chunks of 512 on 2048-token cached prefixes."""
    import torch

    from nimbus_amd import workloads

    rows = []
    for label, seqs in (("one 8192-token prompt", [(8192, 8192)]),
                        ("64 chunks of 512 on 2048-token prefixes", [(2048 + 512, 512)] * 64)):
        b = workloads.build_batch(seqs, heads=32, kv_heads=8, head_dim=128, dtype=torch.bfloat16, device="cuda",
                                  seed=5)
        r = time_prefill(b, steps, warmup)
        rows.append({"workload": label, "us_per_call": r["us_per_call"], "flops": r["flops"],
                     "tflops": r["tflops"], "frac_mfma_peak": r["tflops"] / MFMA_BF16_PEAK_TFLOPS})
        del b
        torch.cuda.empty_cache()
    return rows


def time_mixed_step(batch, steps, warmup):
    """write_kv for every token + prefill (eager) + decode via hipGraph at padded 64."""
    import torch

    from nimbus_amd import workloads
    from nimbus_amd.graphs import DecodeAttentionGraphs
    from nimbus_amd.kernels.cache_ops import write_kv
    from nimbus_amd.kernels.paged_attention import paged_decode_attention
    from nimbus_amd.kernels.prefill_attention import build_programs, paged_prefill_attention

    nb = batch.k_cache.shape[0]
    kc = torch.cat([batch.k_cache, torch.zeros_like(batch.k_cache[:1])])  # + scratch block
    vc = torch.cat([batch.v_cache, torch.zeros_like(batch.v_cache[:1])])
    graphs = DecodeAttentionGraphs(kc, vc, num_heads=batch.q.shape[1], scale=batch.scale, max_model_len=8192,
                                   max_batch=64, scratch_block=nb)
    graphs.capture()
    pa = batch.prefill_args()
    progs = build_programs(pa[7], batch.q.device, pa[8])
    p_tok = batch.num_prefill_tokens
    da = batch.decode_args()
    out = torch.empty_like(batch.q)
    # The decode graph does its own slot write for its tokens; the eager write covers the prefill tokens.
    gb = graphs.load(da[0], batch.k[p_tok:], batch.v[p_tok:], batch.slot_mapping[p_tok:], da[3], da[4])

    def step(i):
        write_kv(batch.k[:p_tok], batch.v[:p_tok], kc, vc, batch.slot_mapping[:p_tok])
        paged_prefill_attention(pa[0], kc, vc, pa[3], pa[4], pa[5], pa[6], pa[7], pa[8], progs, out=out[:p_tok])
        graphs.replay(gb)

    for i in range(warmup):
        step(i)
    us = event_times_us(step, steps, torch.cuda.current_stream())
    replay_us = event_times_us(lambda i: graphs.replay(gb), steps, torch.cuda.current_stream())
    # The slot write alone (all 2,108 tokens of the step), 32 calls back to back in a hipGraph (eager calls
    # would time the host wrapper): algorithmic bytes = k and v rows read and written + the int64 slots.
    def write_all():
        write_kv(batch.k, batch.v, kc, vc, batch.slot_mapping)

    with torch.inference_mode():  # as the decode graphs were captured (their generator state is an inference tensor)
        w_us = _graph_us([write_all] * 32, steps, warmup)
    kvh, d = batch.k.shape[1], batch.k.shape[2]
    w_bytes = workloads.write_kv_bytes(int(batch.k.shape[0]), kvh, d, batch.k.element_size())
    # The decode part apart from its tokens' slot write: the padded-64 decode call on the graphs' static
    # buffers (max_context pinned at max_model_len, as captured), 16 calls back to back in a hipGraph; and the
    # 64 slot writes alone the same way. Bytes: the 60 real decodes' algorithmic bytes (padding rows excluded).
    dq, dctx, dbt = graphs.q[:gb], graphs.ctx[:gb], graphs.tables[:gb]
    dout = torch.empty_like(dq)

    def decode_only():
        paged_decode_attention(dq, kc, vc, dctx, dbt, graphs.max_model_len, batch.scale, out=dout,
                               workspace=graphs.workspace)

    def decode_write():
        write_kv(graphs.k[:gb], graphs.v[:gb], kc, vc, graphs.slots[:gb])

    with torch.inference_mode():
        d_us = _graph_us([decode_only] * 16, steps, warmup)
        dw_us = _graph_us([decode_write] * 32, steps, warmup)
    h = batch.q.shape[1]
    d_bytes = workloads.decode_bytes(batch.decode_context_host(), h, kvh, d, batch.q.element_size())
    return {"step_us": statistics.mean(us), "decode_graph_replay_us": statistics.mean(replay_us),
            "padded_batch": gb, "tokens": int(batch.q.shape[0]),
            "decode": {"bytes": d_bytes, "sum_ctx": int(sum(batch.decode_context_host())), "us_per_call_graph": d_us,
                       "GBps": d_bytes / d_us / 1e3, "frac_hbm_peak": d_bytes / d_us / 1e3 / HBM_PEAK_GBS,
                       "slot_write_us": dw_us,
                       "replay_GBps": d_bytes / statistics.mean(replay_us) / 1e3},
            "write_kv": {"us_per_call": w_us, "bytes": w_bytes, "GBps": w_bytes / w_us / 1e3,
                         "frac_hbm_peak": w_bytes / w_us / 1e3 / HBM_PEAK_GBS}}


# ---------------------------------------------------------------- speculative verification

def time_verify(steps, warmup, n=16, k=4):
    """Speculative verification's attention (nimbus/spec/engine.py:60-150):
    n sequences of k + 1 new tokens on Llama-3-8B-shaped contexts (log-uniform
    128..8192), slot write + prefill replayed from a hipGraph, once as the
    prefill call routes it (its verify form) and once pinned to the tile
    kernel (the reference's route). Bytes: every visible K/V row once per kv
    head, the new tokens' K/V written and q/out. The paged decode call on the
    same contexts (one token each) is timed beside it as the bandwidth
    reference."""
    import torch

    from nimbus_amd import workloads
    from nimbus_amd.graphs import VerifyAttentionGraphs
    from nimbus_amd.kernels.paged_attention import (decode_workspace_bytes, new_decode_workspace,
                                                    paged_decode_attention, paged_verify_attention,
                                                    verify_workspace_bytes)

    q_len = k + 1
    ctx = workloads.llama3_decode_lens(seed=7, batch=n)
    b = workloads.build_batch([(c, q_len) for c in ctx], heads=32, kv_heads=8, head_dim=128,
                              dtype=torch.bfloat16, device="cuda", seed=7, pool_factor=1.2, write_first=False)
    nb = b.k_cache.shape[0]
    kc = torch.cat([b.k_cache, torch.zeros_like(b.k_cache[:1])])
    vc = torch.cat([b.v_cache, torch.zeros_like(b.v_cache[:1])])
    pa = b.prefill_args()
    times = {}
    for kernel in ("auto", "tile"):
        graphs = VerifyAttentionGraphs(kc, vc, num_heads=32, scale=b.scale, max_model_len=8192, max_batch=n, k=k,
                                       scratch_block=nb, kernel=kernel)
        graphs.capture()
        gb = graphs.load(b.q, b.k, b.v, b.slot_mapping, pa[4], b.block_tables)
        for _ in range(warmup):
            graphs.replay(gb)
        times[kernel] = statistics.mean(event_times_us(lambda i: graphs.replay(gb), steps,
                                                       torch.cuda.current_stream()))
        del graphs
    us = times["auto"]
    kv_bytes = sum(ctx) * 2 * 8 * 128 * 2
    nbytes = kv_bytes + 2 * n * q_len * 32 * 128 * 2 + 2 * n * q_len * 8 * 128 * 2 * 2
    # the decode kernel over the same contexts
    qd = torch.randn(n, 32, 128, device="cuda").bfloat16()
    ws = new_decode_workspace(decode_workspace_bytes(n, 32, 128, max(ctx)), torch.device("cuda"))
    outd = torch.empty_like(qd)
    for _ in range(warmup):
        paged_decode_attention(qd, kc, vc, pa[4], b.block_tables, max(ctx), b.scale, out=outd, workspace=ws)
    def decode_call(i):
        paged_decode_attention(qd, kc, vc, pa[4], b.block_tables, max(ctx), b.scale, out=outd, workspace=ws)

    dus = statistics.mean(event_times_us(decode_call, steps, torch.cuda.current_stream()))
    # Like for like: the verify attention call alone (no slot write) and the
    # decode call, each captured back to back in a hipGraph.
    wsv = new_decode_workspace(verify_workspace_bytes(n, q_len, 32, 128, 8192), torch.device("cuda"))
    outv = torch.empty_like(b.q)

    def verify_call(i):
        paged_verify_attention(b.q, kc, vc, pa[4], b.block_tables, q_len, 8192, b.scale, out=outv, workspace=wsv)

    warm_up(verify_call, warmup)
    stream = torch.cuda.current_stream()
    vg = graph_us(verify_call, 12, stream)
    dg = graph_us(decode_call, 12, stream)
    return {"workload": f"{n} sequences x {q_len} tokens (k={k}), Llama-3-8B shape, contexts log-uniform "
                        f"[128, 8192] (sum {sum(ctx)})", "us_per_replay": us, "bytes": nbytes,
            "GBps": nbytes / us / 1e3, "tile_kernel_us_per_replay": times["tile"], "decode_same_contexts_us": dus,
            "decode_same_contexts_GBps": (kv_bytes + 2 * n * 32 * 128 * 2) / dus / 1e3,
            "attention_us_graph": vg, "decode_same_contexts_us_graph": dg, "attention_over_decode": vg / dg}


# ---------------------------------------------------------------- fused residual add + RMSNorm

NORM_SHAPES = (
    ("tinyllama: 2048 tokens x 2048, fp16 (Nimbus's own bench shape)", 2048, 2048, "float16"),
    ("llama3 config-4 step: 2108 tokens x 4096, bf16", 2108, 4096, "bfloat16"),
    ("llama3 decode: 64 tokens x 4096, bf16", 64, 4096, "bfloat16"),
)


def time_add_rms_norm(steps, warmup):
    """add_rms_norm at the model shapes: algorithmic bytes (read x and the
    residual, write the new residual and the output, the weight once) per
    kernel time, against HBM peak. The calls are captured back to back in a
    hipGraph (one per pool of inputs, the pools covering >= 256 MB so the
    Infinity Cache does not hold a call's rows) and the graph is replayed, so
    the time is the kernels', not the Python launch path's."""
    import torch

    from nimbus_amd.kernels.rmsnorm import add_rms_norm

    res = []
    for name, rows, cols, dt in NORM_SHAPES:
        dtype = getattr(torch, dt)
        nbytes = 4 * rows * cols * 2 + cols * 2
        n_pools = max(8, int(math.ceil(256e6 / (2 * rows * cols * 2))))
        g = torch.Generator(device="cuda").manual_seed(rows)
        pools = [(torch.randn(rows, cols, generator=g, device="cuda").to(dtype),
                  torch.randn(rows, cols, generator=g, device="cuda").to(dtype)) for _ in range(n_pools)]
        w = torch.randn(cols, generator=g, device="cuda").to(dtype)
        for x, r in pools[:2]:
            add_rms_norm(x, r, w, 1e-5)  # load the library, warm the caches
        torch.cuda.synchronize()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            for x, r in pools:
                add_rms_norm(x, r, w, 1e-5)
        for i in range(warmup):
            graph.replay()
        per_replay = statistics.mean(event_times_us(lambda i: graph.replay(), max(3, steps // 10),
                                                    torch.cuda.current_stream()))
        us = per_replay / n_pools
        res.append({"shape": name, "rows": rows, "cols": cols, "dtype": dt, "us_per_call": us, "bytes": nbytes,
                    "GBps": nbytes / us / 1e3, "frac_hbm_peak": nbytes / us / 1e3 / HBM_PEAK_GBS,
                    "calls_per_replay": n_pools})
        del graph, pools
    return res


# ---------------------------------------------------------------- INT8 weight-only matmul

INT8_SHAPES = (
    # name, tokens, out channels N, in channels K, dtype
    ("llama3 qkv_proj, 64 tokens (config-3 decode batch)", 64, 6144, 4096, "bfloat16"),
    ("llama3 o_proj, 64 tokens", 64, 4096, 4096, "bfloat16"),
    ("llama3 gate_up_proj, 64 tokens", 64, 28672, 4096, "bfloat16"),
    ("llama3 down_proj, 64 tokens", 64, 4096, 14336, "bfloat16"),
    ("llama3 gate_up_proj, 1 token", 1, 28672, 4096, "bfloat16"),
    ("tinyllama gate_up_proj, 16 tokens, fp16 (Nimbus's kernel bench shape)", 16, 11264, 2048, "float16"),
)


def _graph_us(calls, steps, warmup):
    """Mean time of one call of `calls` (a list of thunks) captured back to
    back in one hipGraph and replayed."""
    import torch

    for c in calls[:2]:
        c()
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        for c in calls:
            c()
    for _ in range(warmup):
        graph.replay()
    per = statistics.mean(event_times_us(lambda i: graph.replay(), max(3, steps // 10), torch.cuda.current_stream()))
    del graph
    return per / len(calls)


def time_int8_matmul(steps, warmup):
    """The INT8 matmul at decode shapes on the tile-order weights Int8Linear
    keeps (int8_matmul_packed; the row-major int8_matmul timed beside it):
    algorithmic bytes (the int8 weights, x, y and the scales once) per
    kernel time, against 8 TB/s, and beside it
    torch's dense matmul (hipBLASLt) on the same weights dequantized to the
    activation dtype, the comparison of Nimbus's own kernel bench
    (int8 vs fp16 cuBLAS). Calls run back to back in a hipGraph over
    weight copies totalling >= 1 GB, so no call finds its weights in the
    256 MB Infinity Cache."""
    import torch

    from nimbus_amd.kernels.int8_matmul import (int8_matmul, int8_matmul_packed, int8_matmul_packed_workspace_bytes,
                                                int8_matmul_workspace_bytes, pack_int8_weight)
    from nimbus_amd.quant import dequantize_weight, quantize_weight

    res = []
    for name, m, n, k, dt in INT8_SHAPES:
        dtype = getattr(torch, dt)
        n_pools = max(4, int(math.ceil(1e9 / (n * k))))
        g = torch.Generator(device="cuda").manual_seed(n + k)
        pools = [quantize_weight((torch.randn(n, k, generator=g, device="cuda") * 0.02).to(dtype))
                 for _ in range(n_pools)]
        x = torch.randn(m, k, generator=g, device="cuda").to(dtype)
        out = torch.empty(m, n, dtype=dtype, device="cuda")
        ws = torch.empty(max(256, int8_matmul_workspace_bytes(m, n, k), int8_matmul_packed_workspace_bytes(m, n, k)),
                         dtype=torch.uint8, device="cuda")
        row_us = _graph_us([lambda q=q, s=s: int8_matmul(x, q, s, out=out, workspace=ws) for q, s in pools],
                           steps, warmup)
        packed = [(pack_int8_weight(q), s) for q, s in pools]
        us = _graph_us([lambda p=p, s=s: int8_matmul_packed(x, p, s, n, k, out=out, workspace=ws) for p, s in packed],
                       steps, warmup)
        del packed
        nbytes = n * k + 2 * m * k + 2 * m * n + 2 * n
        dense = [dequantize_weight(q, s) for q, s in pools[:max(2, n_pools // 2)]]  # 2 bytes a weight
        dus = _graph_us([lambda d=d: torch.matmul(x, d.T, out=out) for d in dense], steps, warmup)
        res.append({"shape": name, "m": m, "n": n, "k": k, "dtype": dt, "us_per_call": us, "bytes": nbytes,
                    "GBps": nbytes / us / 1e3, "frac_hbm_peak": nbytes / us / 1e3 / HBM_PEAK_GBS,
                    "row_major_us_per_call": row_us, "dense_matmul_us": dus, "speedup_vs_dense": dus / us,
                    "calls_per_replay": n_pools})
        del pools, dense
    return res


# ---------------------------------------------------------------- whole-model decode step

def time_decode_step(steps, warmup, chain=16):
    """One decode step of a Llama-3-8B-shaped model (32 layers, random bf16
    weights) for the 64 sequences of config 3 (contexts
    log-uniform [128, 8192]), through DecodeGraphs: eager, one graph replay
    per step, and greedy_chain (step graph + on-device token pick, no host
    round trip); then the same with the decoder projections quantized to
    INT8. Bytes per step: every weight once (int8 projections after
    quantization) + every layer's visible K/V rows + the new K/V rows.
    Each run also replays the target's whole verification pass for the
    same 64 sequences (VerifyGraphs, k = 4 drafts: 5 query tokens per
    sequence, 320 in all)."""
    import random

    import torch

    from nimbus_amd import workloads
    from nimbus_amd.graphs import DecodeGraphs, VerifyGraphs
    from nimbus_amd.model.config import LLAMA3_8B as cfg
    from nimbus_amd.model.llama import build_model
    from nimbus_amd.quant import quantize_model, weight_bytes
    from nimbus_amd.workloads import SeqState, flat_step

    bs = 16
    ctx = workloads.llama3_decode_lens(seed=0, batch=64)
    max_len = 8192 + 2 * chain + 64
    model = build_model(cfg, torch.bfloat16, "cuda", seed=0, max_position=max_len)
    rng = random.Random(0)
    need = sum(-(-(c + 2 * chain + 8) // bs) for c in ctx)
    pool = rng.sample(range(need + 64), need + 64)
    shape = (need + 65, bs, cfg.num_kv_heads, cfg.head_dim)  # the last block is the scratch block
    g = torch.Generator(device="cuda").manual_seed(1)
    caches = [(torch.randn(shape, generator=g, device="cuda").mul_(0.5).bfloat16(),
               torch.randn(shape, generator=g, device="cuda").mul_(0.5).bfloat16()) for _ in range(cfg.num_layers)]
    seqs = []
    for c in ctx:
        seqs.append(SeqState([rng.randrange(cfg.vocab_size) for _ in range(c)],
                             [pool.pop() for _ in range(-(-(c + 2 * chain + 8) // bs))], c - 1))
    kv_bytes = sum(ctx) * cfg.num_layers * 2 * cfg.num_kv_heads * cfg.head_dim * 2

    def measure(label):
        wb = weight_bytes(model)
        graphs = DecodeGraphs(model, caches, bs, max_len, 64, need + 64, cfg.num_kv_heads, "cuda", max_chain=chain)
        graphs.capture()
        batch = [(s, 1) for s in seqs]
        for _ in range(warmup):
            st = flat_step(batch, "cuda", bs)
            model.logits(model(st.input_ids, st.positions, caches, st.meta))
        torch.cuda.synchronize()
        n = max(3, steps // 10)
        t0 = time.perf_counter()
        for _ in range(n):
            st = flat_step(batch, "cuda", bs)
            model.logits(model(st.input_ids, st.positions, caches, st.meta))
        torch.cuda.synchronize()
        eager_ms = (time.perf_counter() - t0) * 1e3 / n
        for _ in range(warmup):
            graphs.run(seqs)
        replay_ms = statistics.mean(event_times_us(lambda i: graphs.run(seqs), n, torch.cuda.current_stream())) / 1e3
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        graphs.greedy_chain(seqs, chain)
        torch.cuda.synchronize()
        chain_ms = (time.perf_counter() - t0) * 1e3 / chain
        nbytes = wb + kv_bytes + 64 * cfg.num_layers * 2 * cfg.num_kv_heads * cfg.head_dim * 2
        del graphs
        verify = VerifyGraphs(model, caches, bs, max_len, 64, 4, need + 64, "cuda")
        verify.capture()
        for _ in range(warmup):
            verify.run(seqs)
        verify_ms = statistics.mean(event_times_us(lambda i: verify.run(seqs), n,
                                                   torch.cuda.current_stream())) / 1e3
        del verify
        return {"weights": label, "weight_bytes": wb, "bytes_per_step": nbytes, "eager_ms": eager_ms,
                "graph_replay_ms": replay_ms, "greedy_chain_ms_per_step": chain_ms,
                "tokens_per_s": 64 / (chain_ms * 1e-3), "GBps": nbytes / (chain_ms * 1e-3) / 1e9,
                "frac_hbm_peak": nbytes / (chain_ms * 1e-3) / 1e9 / HBM_PEAK_GBS,
                "verify_pass_ms": verify_ms, "verify_query_tokens": 64 * 5,
                "verify_query_tokens_per_s": 64 * 5 / (verify_ms * 1e-3)}

    res = {"workload": "Llama-3-8B shape (random weights), 64 decode sequences of config 3 "
                       f"(sum ctx {sum(ctx)}), chains of {chain} greedy steps",
           "runs": [measure("bf16")]}
    quantize_model(model)
    res["runs"].append(measure("int8 projections (bf16 embeddings and head)"))
    del model, caches
    torch.cuda.empty_cache()
    return res


# ---------------------------------------------------------------- the reference's own micro-bench shapes

# Published on an RTX 4050 Laptop GPU (results/kernels.json:15-71 of the reference, triton_us), for the table's
# other column; not a target (other hardware).
REFERENCE_PUBLISHED_US = {
    "paged_decode_attention batch=1 ctx=512": 26.2, "paged_decode_attention batch=1 ctx=2048": 39.9,
    "paged_decode_attention batch=16 ctx=512": 98.3, "paged_decode_attention batch=64 ctx=512": 348.3,
    "paged_decode_attention batch=64 ctx=1024": 626.7, "paged_prefill_attention seqs=1 len=512": 118.9,
    "paged_prefill_attention seqs=4 len=512": 383.4, "paged_prefill_attention seqs=16 len=128": 203.4,
    # results/kernels.json:72-176: add_rms_norm (fp16, hidden 2048) and the INT8 matmul (TinyLlama projections)
    "add_rms_norm rows=1 hidden=2048": 10.0, "add_rms_norm rows=64 hidden=2048": 15.5,
    "add_rms_norm rows=2048 hidden=2048": 273.0,
    "int8_matmul qkv_proj M=1 N=2560 K=2048": 65.6, "int8_matmul qkv_proj M=16 N=2560 K=2048": 65.4,
    "int8_matmul qkv_proj M=64 N=2560 K=2048": 73.8, "int8_matmul qkv_proj M=512 N=2560 K=2048": 358.6,
    "int8_matmul gate_up_proj M=1 N=11264 K=2048": 239.7, "int8_matmul gate_up_proj M=16 N=11264 K=2048": 240.0,
    "int8_matmul gate_up_proj M=64 N=11264 K=2048": 264.8, "int8_matmul gate_up_proj M=512 N=11264 K=2048": 1540.4,
    "int8_matmul down_proj M=1 N=2048 K=5632": 126.6, "int8_matmul down_proj M=16 N=2048 K=5632": 128.6,
    "int8_matmul down_proj M=64 N=2048 K=5632": 163.8, "int8_matmul down_proj M=512 N=2048 K=5632": 795.6,
}


def reference_shapes(reps=200, warmup=25):
    """The shapes of the reference's kernel micro-bench (bench/kernels.py:54-91):
    TinyLlama heads (H=32, KV=4, D=64), fp16, pages a seeded permutation of
    a pool of (pages needed + 8) blocks; decode at (batch, ctx) in {(1,512),
    (1,2048), (16,512), (64,512), (64,1024)}, fresh prefill of (seqs, len) in
    {(1,512), (4,512), (16,128)}; add_rms_norm of {1, 64, 2048} rows of 2048;
    the INT8 matmul at TinyLlama's qkv (2560 x 2048), gate_up (11264 x 2048)
    and down (2048 x 5632) projections for M in {1, 16, 64, 512}, on the
    tile-order weights Int8Linear keeps, beside torch's fp16 matmul of the
    dequantized weights (the reference's cuBLAS column). Each call is timed
    alone between a HIP event pair through the Python entry point (as
    triton.testing.do_bench does), median of `reps`. The inputs are at most
    a few tens of MB, so they sit in the Infinity Cache: GB/s here is
    effective, not HBM."""
    import torch

    from nimbus_amd import workloads
    from nimbus_amd.kernels.paged_attention import paged_decode_attention
    from nimbus_amd.kernels.prefill_attention import paged_prefill_attention

    rows = []
    stream = torch.cuda.current_stream()
    for b, ctx in ((1, 512), (1, 2048), (16, 512), (64, 512), (64, 1024)):
        batch = workloads.build_batch([(ctx, 1)] * b, heads=32, kv_heads=4, head_dim=64, dtype=torch.float16,
                                      device="cuda", seed=0, pool_blocks=b * -(-ctx // 16) + 8,
                                      contiguous_slices=True, write_first=False)
        a = batch.decode_args()
        out = torch.empty_like(a[0])
        fn = lambda i: paged_decode_attention(*a, out=out)  # noqa: E731
        for i in range(warmup):
            fn(i)
        us = statistics.median(event_times_us(fn, reps, stream))
        nbytes = workloads.decode_bytes([ctx] * b, 32, 4, 64, 2)
        name = f"paged_decode_attention batch={b} ctx={ctx}"
        rows.append({"kernel": name, "us": us, "GBps_effective": nbytes / us / 1e3,
                     "reference_published_us": REFERENCE_PUBLISHED_US[name]})
    for n, ql in ((1, 512), (4, 512), (16, 128)):
        batch = workloads.build_batch([(ql, ql)] * n, heads=32, kv_heads=4, head_dim=64, dtype=torch.float16,
                                      device="cuda", seed=0, pool_blocks=n * -(-ql // 16) + 8,
                                      contiguous_slices=True)
        a = batch.prefill_args()
        out = torch.empty_like(a[0])
        fn = lambda i: paged_prefill_attention(*a, out=out)  # noqa: E731
        for i in range(warmup):
            fn(i)
        us = statistics.median(event_times_us(fn, reps, stream))
        flops = workloads.prefill_flops([(ql, ql)] * n, 32, 64)
        name = f"paged_prefill_attention seqs={n} len={ql}"
        rows.append({"kernel": name, "us": us, "TFLOPs": flops / us / 1e6,
                     "frac_mfma_peak": flops / us / 1e6 / MFMA_BF16_PEAK_TFLOPS,
                     "reference_published_us": REFERENCE_PUBLISHED_US[name]})
    from nimbus_amd.kernels.int8_matmul import int8_matmul_packed, pack_int8_weight
    from nimbus_amd.kernels.rmsnorm import add_rms_norm
    from nimbus_amd.quant import dequantize_weight, quantize_weight

    def median_us(fn):
        for i in range(warmup):
            fn(i)
        return statistics.median(event_times_us(fn, reps, stream))

    g = torch.Generator(device="cuda").manual_seed(0)
    for m in (1, 64, 2048):
        x = torch.randn(m, 2048, generator=g, device="cuda").half()
        r = torch.randn(m, 2048, generator=g, device="cuda").half()
        w = torch.randn(2048, generator=g, device="cuda").half()
        us = median_us(lambda i: add_rms_norm(x, r, w, 1e-5))
        nbytes = 4 * m * 2048 * 2 + 2048 * 2
        name = f"add_rms_norm rows={m} hidden=2048"
        rows.append({"kernel": name, "us": us, "GBps_effective": nbytes / us / 1e3,
                     "reference_published_us": REFERENCE_PUBLISHED_US[name]})
    for proj, n, k in (("qkv_proj", 2560, 2048), ("gate_up_proj", 11264, 2048), ("down_proj", 2048, 5632)):
        wq, sc = quantize_weight(torch.randn(n, k, generator=g, device="cuda").half() * 0.02)
        packed = pack_int8_weight(wq)
        dense = dequantize_weight(wq, sc)
        for m in (1, 16, 64, 512):
            x = torch.randn(m, k, generator=g, device="cuda").half()
            us = median_us(lambda i: int8_matmul_packed(x, packed, sc, n, k))
            dense_us = median_us(lambda i: torch.matmul(x, dense.T))
            nbytes = n * k + 2 * m * k + 2 * m * n + 2 * n
            name = f"int8_matmul {proj} M={m} N={n} K={k}"
            rows.append({"kernel": name, "us": us, "GBps_effective": nbytes / us / 1e3,
                         "torch_fp16_matmul_us": dense_us, "reference_published_us": REFERENCE_PUBLISHED_US[name]})
    return {"note": "reference_published_us: the reference's Triton kernels on an RTX 4050 Laptop GPU "
                    "(results/kernels.json), other hardware", "rows": rows}


# ---------------------------------------------------------------- configs 1, 2 and 5

def other_configs(steps, warmup, prefill=True):
    """configs 1 (TinyLlama decode), 2 (TinyLlama varlen prefill)
    and 5 (long-context decode, ~40 GB pool) in compact form: µs per call of
    back-to-back calls (decode: also replayed from a hipGraph, which drops the
    ~15 µs of host work per eager call that bounds config 1), GB/s or TFLOP/s
    and the roofline fraction."""
    import torch

    from nimbus_amd import workloads

    rows = {}
    for cfg, name in ((1, "tinyllama_decode"), (5, "llama3_long_decode")):
        log(f"config {cfg} ({name})")
        b = workloads.CONFIGS[name]("cuda")
        r = time_decode(b, steps, warmup, wall=False)
        rows[f"config{cfg}"] = {
            "workload": name, "batch": r["batch"], "sum_ctx": r["sum_ctx"], "bytes": r["bytes"],
            "us_per_call": r["call_us"], "us_per_call_graph": r["call_us_graph"], "page_pass_us": r["page_pass_us"],
            "GBps_call": r["bytes"] / r["call_us"] / 1e3,
            "GBps_call_graph": r["bytes"] / r["call_us_graph"] / 1e3,
            "frac_hbm_peak_call": r["bytes"] / r["call_us"] / 1e3 / HBM_PEAK_GBS,
            "frac_hbm_peak_page_pass": r["bytes"] / r["page_pass_us"] / 1e3 / HBM_PEAK_GBS,
        }
        del b
        torch.cuda.empty_cache()
    if not prefill:
        return rows
    log("config 2 (tinyllama_prefill)")
    b = workloads.CONFIGS["tinyllama_prefill"]("cuda")
    r = time_prefill(b, steps, warmup)
    rows["config2"] = {"workload": "tinyllama_prefill", "us_per_call": r["us_per_call"], "flops": r["flops"],
                       "tflops": r["tflops"], "frac_mfma_peak": r["tflops"] / MFMA_BF16_PEAK_TFLOPS}
    del b
    torch.cuda.empty_cache()
    return rows


# ---------------------------------------------------------------- --all

def all_configs(steps, warmup, out_path=None):
    import torch

    from nimbus_amd import workloads

    rows = {}
    for name in ("tinyllama_decode", "llama3_decode", "llama3_long_decode"):
        log(f"config {name}")
        b = workloads.CONFIGS[name]("cuda")
        r = time_decode(b, steps, warmup, wall=False)
        r["GBps_call"] = r["bytes"] / r["call_us"] / 1e3
        r["GBps_page_pass"] = r["bytes"] / r["page_pass_us"] / 1e3
        r["frac_hbm_peak_page_pass"] = r["GBps_page_pass"] / HBM_PEAK_GBS
        rows[name] = r
        del b
        torch.cuda.empty_cache()
    for name in ("tinyllama_prefill", "llama3_mixed"):
        log(f"config {name}")
        b = workloads.CONFIGS[name]("cuda")
        r = time_prefill(b, steps, warmup)
        r["frac_mfma_peak"] = r["tflops"] / MFMA_BF16_PEAK_TFLOPS
        if name == "llama3_mixed":
            r["mixed_step"] = time_mixed_step(b, steps, warmup)
        rows[name] = r
        del b
        torch.cuda.empty_cache()
    if out_path:
        with open(out_path, "w") as f:
            json.dump(rows, f, indent=1)
    for k, v in rows.items():
        log(f"{k}: " + ", ".join(f"{a}={b:.4g}" if isinstance(b, float) else f"{a}={b}" for a, b in v.items()
                                 if not isinstance(b, dict)))
    return rows


# ---------------------------------------------------------------- main

def config_summary(result):
    """One compact entry per config: µs per call and the roofline
    fraction (HBM for decode, dense MFMA for prefill)."""
    def r4(x):
        return None if x is None else round(float(x), 4)

    out = {}
    other = result.get("other_configs") or {}
    c1 = other.get("config1")
    if c1:
        out["config1_decode"] = {"us_graph": r4(c1["us_per_call_graph"]), "us_eager": r4(c1["us_per_call"]),
                                 "frac_hbm": r4(c1["bytes"] / c1["us_per_call_graph"] / 1e3 / HBM_PEAK_GBS)}
    c2 = other.get("config2")
    if c2:
        out["config2_prefill"] = {"us": r4(c2["us_per_call"]), "frac_mfma": r4(c2["frac_mfma_peak"])}
    rl = result["roofline"]
    out["config3_decode"] = {"us": r4(rl["kernel_us"]), "us_graph": r4(rl["kernel_us_graph"]), "frac_hbm": r4(rl["frac"])}
    if "prefill" in result:
        out["config4_prefill"] = {"us": r4(result["prefill"]["us_per_call"]),
                                  "frac_mfma": r4(result["prefill"]["frac_mfma_peak"])}
    ms = result.get("mixed_step")
    if ms:
        out["config4_decode"] = {"us_graph": r4(ms["decode"]["us_per_call_graph"]),
                                 "frac_hbm": r4(ms["decode"]["frac_hbm_peak"]),
                                 "slot_write_us": r4(ms["decode"]["slot_write_us"]),
                                 "step_us": r4(ms["step_us"])}
    c5 = other.get("config5")
    if c5:
        out["config5_decode"] = {"us": r4(c5["us_per_call"]), "us_graph": r4(c5["us_per_call_graph"]),
                                 "frac_hbm": r4(c5["frac_hbm_peak_call"])}
    for row in result.get("prefill_scaling") or []:
        if row["workload"].startswith("one 8192"):
            out["prompt8192_prefill"] = {"us": r4(row["us_per_call"]), "frac_mfma": r4(row["frac_mfma_peak"])}
    v = result.get("verify")
    if v:
        out["verify_attention"] = {"us_graph": r4(v["attention_us_graph"]),
                                   "decode_us_graph": r4(v["decode_same_contexts_us_graph"]),
                                   "over_decode": r4(v["attention_over_decode"])}
    return out


def main(argv=None):
    args = parse(argv)
    if args.gpus != 1:
        print(f"bench.py measures one GPU only (asked for --gpus {args.gpus}); this build has no multi-GPU path: "
              "run with --gpus 1", file=sys.stderr)
        sys.exit(2)
    import torch

    from nimbus_amd import _lib, workloads

    if not torch.cuda.is_available():
        print("bench.py needs a GPU", file=sys.stderr)
        sys.exit(1)
    _lib.load()
    torch.manual_seed(0)

    if args.copy_calibration:
        copy_calibration(args.copy_calibration)
    # The other configurations run first: timed per call from a fresh process,
    # config 3's decode runs 2-7% slower over its first ~150 calls (the GPU's
    # clocks settling), so the headline is measured after other GPU work.
    other = None
    if not args.no_prefill or args.decode_only:
        other = other_configs(min(args.steps, 50), args.warmup, prefill=not args.decode_only)
    log("building llama3_decode (config 3)")
    batch = workloads.llama3_decode("cuda")
    dec = time_decode(batch, args.steps, args.warmup)
    log(f"decode: {dec}")
    call_gbs = dec["bytes"] / dec["call_us"] / 1e3
    part_gbs = dec["bytes"] / dec["page_pass_us"] / 1e3
    result = {
        "metric": METRIC,
        "value": dec["bytes"] / (dec["ms_per_step"] * 1e-3) / 1e9,
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": dec["ms_per_step"],
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (seeded N(0,1) q, 0.5*N(0,1) K/V, shuffled page tables)",
        "config": {
            "workload": "llama3_decode: config 3, Llama-3-8B-shaped paged decode attention",
            "batch": dec["batch"], "heads": 32, "kv_heads": 8, "head_dim": 128, "block_size": 16,
            "context": "log-uniform [128, 8192], seed 0", "sum_ctx": dec["sum_ctx"],
            "bytes_per_call": dec["bytes"], "pool_rotation": dec["pools"], "parallelism": "none (1 GPU)",
        },
        "us_per_call": dec["call_us"],
        "roofline": {
            "kernel": "paged_decode_kernel + paged_decode_merge_kernel (the whole decode call)",
            "bound": "hbm",
            "achieved": call_gbs,
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": call_gbs / HBM_PEAK_GBS,
            "traffic": measured_traffic(dec["bytes"]),
            "kernel_us": dec["call_us"],
            "kernel_us_event_pairs": dec["call_us_event_pairs"],
            "kernel_us_graph": dec["call_us_graph"],
            "page_pass": {"kernel": "paged_decode_kernel", "us": dec["page_pass_us"],
                          "us_event_pairs": dec["page_pass_us_event_pairs"], "achieved": part_gbs,
                          "frac": part_gbs / HBM_PEAK_GBS},
            "merge_pass_share_us": dec["merge_us"],
        },
    }
    if other is not None:
        result["other_configs"] = other
    if args.decode_only:
        args.no_prefill = True
    if not args.no_prefill:
        log("building llama3_mixed (config 4)")
        mixed = workloads.llama3_mixed("cuda")
        pre = time_prefill(mixed, args.steps, args.warmup)
        pre["frac_mfma_peak"] = pre["tflops"] / MFMA_BF16_PEAK_TFLOPS
        result["prefill"] = {"workload": "llama3_mixed prefill part (4 x 512 new on prefix U[0,1024])", **pre,
                             "peak_tflops": MFMA_BF16_PEAK_TFLOPS}
        result["mixed_step"] = time_mixed_step(mixed, args.steps, args.warmup)
        log(f"prefill: {result['prefill']}  mixed: {result['mixed_step']}")
        del mixed
        result["prefill_scaling"] = prefill_scaling(min(args.steps, 20), min(args.warmup, 3))
        log(f"prefill_scaling: {result['prefill_scaling']}")
    if not args.no_prefill:
        log("speculative verify")
        result["verify"] = time_verify(args.steps, args.warmup)
        log(f"verify: {result['verify']}")
        log("add_rms_norm")
        result["add_rms_norm"] = time_add_rms_norm(args.steps, args.warmup)
        log(f"add_rms_norm: {result['add_rms_norm']}")
        log("int8_matmul")
        result["int8_matmul"] = time_int8_matmul(args.steps, args.warmup)
        log(f"int8_matmul: {result['int8_matmul']}")
        log("decode_step (whole model)")
        result["decode_step"] = time_decode_step(args.steps, args.warmup)
        log(f"decode_step: {result['decode_step']}")
    if not args.no_prefill:
        log("reference_shapes")
        result["reference_shapes"] = reference_shapes()
        log(f"reference_shapes: {result['reference_shapes']}")
    if args.all:
        result["configs"] = {k: {a: b for a, b in v.items() if not isinstance(b, dict)}
                             for k, v in all_configs(args.steps, args.warmup, args.all_out).items()}
    if not args.no_cpu_baseline:
        log("CPU baseline (oracle on host cores)")
        base = cpu_decode_baseline(batch, args.cpu_seconds)
        entries = [dict(base, config="config 3 (headline), batched form")]
        del batch
        torch.cuda.empty_cache()
        if not args.no_prefill:
            mixed = workloads.llama3_mixed("cuda")
            entries.append(dict(cpu_prefill_baseline(mixed, args.cpu_seconds), config="config 4 prefill part"))
            del mixed
            torch.cuda.empty_cache()
            long_b = workloads.llama3_long_decode("cuda")
            entries.append(dict(cpu_long_decode_baseline(long_b, args.cpu_seconds), config="config 5, per-row form"))
            del long_b
            torch.cuda.empty_cache()
        result["cpu_baseline"] = dict(base, entries=entries)
    # Last on the line (and repeated on stderr after it), where a reader of the output's tail finds it: one
    # figure per config and its share of the roofline.
    result["summary"] = summary = config_summary(result)
    print(json.dumps(result), flush=True)
    for k, v in summary.items():
        log(f"summary {k}: {v}")


if __name__ == "__main__":
    main()
