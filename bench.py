#!/usr/bin/env python3
"""Paged-decode benchmark on one MI355X.

Workload (one "step"): the decode attention of a random-init Qwen3-0.6B layer
stack -- 16 Q / 8 KV heads, head_dim 128, bf16, block 16 -- for 32 sequences
with contexts U[128, 2048] over a 16384-block pool per layer. A step is one
partition plan plus 28 independent layer calls, each one launch that appends
the 32 new K/V rows and runs paged decode attention over that layer's own
cache (28 distinct 1.07 GB caches, so nothing is served from the 256 MB
last-level cache). The step is captured in a hipGraph and replayed; inputs
are resident in HBM before timing.

Prints one JSON line: value = whole-step algorithmic HBM bytes / step time
(GB/s), the roofline of the decode launch and a CPU-oracle baseline. The same
line carries the other half of the metric: decode tok/s (and output tok/s) of
the engine workload -- random-init Qwen3-0.6B serving 64 requests x 128
prompt ids -> 16 greedy tokens -- in ``config.decode_tok_s``, with the same
engine's decode on the host CPU (a KV-cached paged float32 forward under the
same scheduler) in ``cpu_baseline_engine`` / ``config.cpu_decode_tok_s``.
"""

from __future__ import annotations

import argparse
import json
import math
import os
import platform
import statistics
import sys
import time

import numpy as np

HBM_PEAK_GBS = 8000.0
MFMA_BF16_PEAK_TFLOPS = 2500.0


def capture_graph(graph, pool=None, stream=None):
    """The product's garbage-collector-safe graph capture (microinfer_amd.runner)."""
    from microinfer_amd.runner import capture_graph as capture

    return capture(graph, pool, stream)


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def cpu_model() -> str:
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return platform.processor() or "unknown"


def blas_threads() -> int:
    try:
        from threadpoolctl import threadpool_info

        counts = [p.get("num_threads", 1) for p in threadpool_info() if p.get("user_api") == "blas"]
        return max(counts) if counts else 1
    except Exception:  # pragma: no cover - informational only
        return 1


def warm_up(torch, run, args) -> None:
    """The W untimed warmup steps, continued (still untimed) until at least
    --warmup-seconds have passed: the GPU's clocks take about a second of
    sustained work to settle, and a timed region that starts cold measures
    the ramp instead of the kernels."""
    t_end = time.perf_counter() + args.warmup_seconds
    for _ in range(args.warmup):
        run()
    torch.cuda.synchronize()
    while time.perf_counter() < t_end:
        run()
        torch.cuda.synchronize()


def build_decode_state(torch, layers: int, layout: str):
    from microinfer_amd.workloads import QWEN3_06B, make_decode_batch
    from microinfer_amd.worker.kv_cache import KVCache

    batch = make_decode_batch(num_seqs=32, ctx_lo=128, ctx_hi=2048, pool_blocks=16384,
                              draw_pools=False, **QWEN3_06B)
    dev = torch.device("cuda", 0)
    dtype = torch.bfloat16
    cache = KVCache(layers, 16384, 16, 8, 128, dtype=dtype, device=dev, layout=layout)
    gen = torch.Generator(device=dev).manual_seed(0)
    for layer in range(layers):
        cache.keys[layer].copy_(torch.randn(cache.keys[layer].shape, generator=gen, device=dev))
        cache.values[layer].copy_(torch.randn(cache.values[layer].shape, generator=gen, device=dev))
    query = torch.empty((layers, 32, 16, 128), dtype=dtype, device=dev)
    query[0].copy_(torch.from_numpy(batch.query))
    query[1:].copy_(torch.randn(query[1:].shape, generator=gen, device=dev))
    new_k = torch.randn((layers, 32, 8, 128), generator=gen, device=dev).to(dtype)
    new_v = torch.randn((layers, 32, 8, 128), generator=gen, device=dev).to(dtype)
    return dict(
        batch=batch,
        cache=cache,
        views=[cache.layer(i) for i in range(layers)],
        query=query,
        new_k=new_k,
        new_v=new_v,
        tables=torch.tensor(batch.block_tables, device=dev),
        lens=torch.tensor(batch.context_lens, device=dev),
        slots=torch.tensor(batch.slots, device=dev),
    )


PROFILES = os.path.join(os.path.dirname(os.path.abspath(__file__)), "profiles")
DECODE_TRAFFIC = os.path.join(PROFILES, "paged_decode_traffic_qwen3-0.6b_b32.json")
PREFILL_TRAFFIC = os.path.join(PROFILES, "paged_prefill_traffic_qwen3-8b_mixed.json")
QK_TRAFFIC = os.path.join(PROFILES, "qk_norm_rope_traffic_qwen3-8b_mixed.json")
GREEDY_TRAFFIC = os.path.join(PROFILES, "greedy_argmax_traffic_qwen3-vocab_b32.json")
APPEND_TRAFFIC = os.path.join(PROFILES, "kv_append_traffic_qwen3-8b_mixed.json")
GATHER_TRAFFIC = os.path.join(PROFILES, "gather_kv_traffic_qwen3-8b_mixed.json")
LONG_DECODE_TRAFFIC = os.path.join(PROFILES, "paged_decode_long_traffic_qwen3-8b.json")


def measured_traffic(path: str):
    """HBM bytes per launch from a committed FETCH_SIZE / WRITE_SIZE summary
    (calibrated against a copy kernel), or None when that profile is absent."""
    try:
        with open(path) as f:
            return int(json.load(f)["traffic_bytes_per_launch"])
    except (OSError, KeyError, ValueError):
        return None


def copy_calibration(torch, mib: int) -> None:
    """One plain device-to-device copy of ``mib`` MiB (reads and writes that many)."""
    src = torch.empty(mib << 20, dtype=torch.uint8, device="cuda")
    dst = torch.empty_like(src)
    dst.copy_(src)
    torch.cuda.synchronize()
    log(f"calibration copy of {mib} MiB done")


def cpu_baseline(torch, state, samples: int = 5):
    """Oracle (numpy restatement of the reference CPU path) on layer 0's call."""
    from microinfer_amd.workloads import decode_bytes
    from oracle import kv_append, paged_attention_reference

    batch = state["batch"]
    view = state["views"][0]
    tables = batch.block_tables
    contexts = [int(c) for c in batch.context_lens]
    used = sorted({int(b) for r, c in enumerate(contexts) for b in tables[r, : (c + 15) // 16]})
    remap = {b: i for i, b in enumerate(used)}
    small_tables = np.full_like(tables, -1)
    for r, c in enumerate(contexts):
        for j in range((c + 15) // 16):
            small_tables[r, j] = remap[int(tables[r, j])]
    index = torch.tensor(used, dtype=torch.long, device=view.keys.device)
    # bf16 caches widen exactly to f32; the oracle accumulates in f32 as the
    # reference does for half inputs (layer/paged_attention.py:38-40).
    host_k = view.keys.index_select(0, index).float().cpu().numpy()
    host_v = view.values.index_select(0, index).float().cpu().numpy()
    q = state["query"][0].float().cpu().numpy()
    nk = state["new_k"][0].float().cpu().numpy()
    nv = state["new_v"][0].float().cpu().numpy()
    slots = np.array([small_tables[r, (c - 1) // 16] * 16 + (c - 1) % 16
                      for r, c in enumerate(contexts)])
    cu = list(range(len(contexts) + 1))
    scale = 1 / math.sqrt(128)

    def one_call():
        kv_append(host_k, host_v, slots, nk, nv)
        return paged_attention_reference(q, host_k, host_v, small_tables, contexts, cu, scale=scale)

    one_call()  # warm-up
    times = []
    for _ in range(samples):
        t0 = time.perf_counter()
        one_call()
        times.append(time.perf_counter() - t0)
    per_call = statistics.median(times)
    nbytes = decode_bytes(contexts, num_q_heads=16, num_kv_heads=8, head_dim=128, elem_bytes=2,
                          block_size=16)
    return {
        "value": round(nbytes / per_call / 1e9, 3),
        "unit": "GB/s",
        "cores": blas_threads(),
        "kind": "port",
        "sample": (f"1 layer call (KV append of 32 rows + decode over {sum(contexts)} cached "
                   f"tokens, 0.6B shape) x {samples} runs after 1 warm-up, median "
                   f"{per_call * 1e3:.1f} ms; numpy/BLAS on {os.cpu_count()} host CPUs "
                   f"({cpu_model()})"),
    }


def prefill_cpu_baseline(torch, batch, q, cache, samples: int = 3):
    """Oracle on a bounded sample of the mixed batch: 2 prefill chunks + the decode rows."""
    from microinfer_amd.workloads import prefill_flops
    from oracle import paged_attention_reference

    rows = [0, 1] + list(range(8, len(batch.q_lens)))
    tables = batch.block_tables[rows]
    contexts = [int(batch.context_lens[r]) for r in rows]
    used = sorted({int(b) for i, c in enumerate(contexts) for b in tables[i, : (c + 15) // 16]})
    remap = {b: i for i, b in enumerate(used)}
    small = np.full_like(tables, -1)
    for i, c in enumerate(contexts):
        for j in range((c + 15) // 16):
            small[i, j] = remap[int(tables[i, j])]
    index = torch.tensor(used, dtype=torch.long, device=cache.keys[0].device)
    host_k = cache.keys[0].index_select(0, index).float().cpu().numpy()
    host_v = cache.values[0].index_select(0, index).float().cpu().numpy()
    q_rows = np.concatenate([np.arange(batch.cu_seqlens_q[r], batch.cu_seqlens_q[r + 1]) for r in rows])
    host_q = q[torch.tensor(q_rows, device=q.device)].float().cpu().numpy()
    q_lens = [int(batch.q_lens[r]) for r in rows]
    cu = np.concatenate([[0], np.cumsum(q_lens)]).tolist()
    scale = 1 / math.sqrt(128)
    paged_attention_reference(host_q, host_k, host_v, small, contexts, cu, scale=scale)
    times = []
    for _ in range(samples):
        t0 = time.perf_counter()
        paged_attention_reference(host_q, host_k, host_v, small, contexts, cu, scale=scale)
        times.append(time.perf_counter() - t0)
    per_call = statistics.median(times)
    flops = prefill_flops(q_lens, contexts, num_q_heads=32, head_dim=128)
    return {
        "value": round(flops / per_call / 1e12, 4),
        "unit": "TFLOP/s",
        "cores": blas_threads(),
        "kind": "port",
        "sample": (f"2 of the 8 prefill chunks + the 24 decode rows ({flops / 1e9:.1f} GFLOP), "
                   f"x {samples} runs after 1 warm-up, median {per_call * 1e3:.0f} ms; "
                   f"numpy/BLAS on {os.cpu_count()} host CPUs ({cpu_model()})"),
    }


def measured_bf16_gemm_peak(torch, n: int = 8192, runs: int = 20) -> dict:
    """Dense bf16 GEMM rate of the library (hipBLASLt through torch.matmul).

    An n x n x n product, timed with HIP events after warm-up, is the
    measured counterpart of the vendor's dense bf16 MFMA figure: the prefill
    line's `frac` divides by the vendor peak, and this number says how much
    of that peak a library GEMM reaches on the same box.
    """
    dev = torch.device("cuda", 0)
    a = torch.randn((n, n), device=dev, dtype=torch.bfloat16)
    b = torch.randn((n, n), device=dev, dtype=torch.bfloat16)
    c = torch.empty((n, n), device=dev, dtype=torch.bfloat16)
    for _ in range(5):
        torch.matmul(a, b, out=c)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    while time.perf_counter() - t0 < 1.0:  # clocks settle under sustained load
        torch.matmul(a, b, out=c)
        torch.cuda.synchronize()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record()
    for _ in range(runs):
        torch.matmul(a, b, out=c)
    end.record()
    torch.cuda.synchronize()
    ms = start.elapsed_time(end) / runs
    tflops = 2.0 * n**3 / (ms * 1e-3) / 1e12
    del a, b, c
    return {"tflops": round(tflops, 1), "shape": f"{n}x{n}x{n} bf16, torch.matmul (hipBLASLt)",
            "us": round(ms * 1e3, 1)}


# Launches per prefill step that share one launch plan: Qwen3-8B's 36 layers.
PREFILL_LAYERS = 36


def prefill_state(torch, layout: str) -> dict:
    """The mixed chunked-prefill batch on the device (8B shape, pool 65536)."""
    from microinfer_amd.layer.hip_paged_attention import hip_paged_prefill, prefill_plan
    from microinfer_amd.workloads import make_mixed_prefill_batch, prefill_flops
    from microinfer_amd.worker.kv_cache import KVCache

    batch = make_mixed_prefill_batch()
    dev = torch.device("cuda", 0)
    log("allocating the 8B-shape cache (65536 blocks)")
    cache = KVCache(1, batch.pool_blocks, 16, 8, 128, dtype=torch.bfloat16, device=dev,
                    layout=layout)
    gen = torch.Generator(device=dev).manual_seed(0)
    cache.keys[0].copy_(torch.randn(cache.keys[0].shape, generator=gen, device=dev))
    cache.values[0].copy_(torch.randn(cache.values[0].shape, generator=gen, device=dev))
    total_q = int(batch.q_lens.sum())
    q = torch.randn((total_q, 32, 128), generator=gen, device=dev).to(torch.bfloat16)
    tables = torch.tensor(batch.block_tables, device=dev)
    cu_q = torch.tensor(batch.cu_seqlens_q, device=dev)
    cu_k = torch.tensor(batch.cu_seqlens_k, device=dev)
    max_q = int(batch.q_lens.max())
    scale = 1 / math.sqrt(128)

    def step(planned=True):
        # One call without a shared plan (it plans for itself only when
        # short of items) or, planned=False, always unplanned; the
        # output is allocated by the call (from the graph's pool when
        # captured).
        return hip_paged_prefill(q, cache.keys[0], cache.values[0], cu_q, cu_k, tables,
                                 max_seqlen_q=max_q, scale=scale, planned=planned)

    def layers_step():
        # The engine's pattern: one launch plan per step, shared by the
        # launches of every layer.
        plan = prefill_plan(cu_q, cu_k, num_tokens=total_q, num_q_heads=32, num_kv_heads=8,
                            head_dim=128, dtype=q.dtype, block_size=16,
                            block_table_width=tables.shape[1])
        for _ in range(PREFILL_LAYERS):
            hip_paged_prefill(q, cache.keys[0], cache.values[0], cu_q, cu_k, tables,
                              max_seqlen_q=max_q, scale=scale, plan=plan)

    flops = prefill_flops(batch.q_lens, batch.context_lens, num_q_heads=32, head_dim=128)
    return dict(batch=batch, cache=cache, q=q, gen=gen, step=step, layers_step=layers_step,
                flops=flops, total_q=total_q, dev=dev)


def time_launches(torch, run, args, steps: int) -> float:
    """Milliseconds per ``run()`` after the warm-up, HIP events on the
    current stream (the stream every launch goes to)."""
    warm_up(torch, run, args)
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record()
    for _ in range(steps):
        run()
    end.record()
    torch.cuda.synchronize()
    return start.elapsed_time(end) / steps


def run_prefill(args) -> int:
    """Mixed chunked prefill (8B shape): one varlen launch per step."""
    import torch

    from microinfer_amd.layer.hip_paged_attention import hip_paged_prefill
    from microinfer_amd.workloads import prefill_flops

    st = prefill_state(torch, args.layout)
    batch, cache, q, gen, step, dev = (st[k] for k in ("batch", "cache", "q", "gen", "step",
                                                        "dev"))
    total_q = st["total_q"]
    scale = 1 / math.sqrt(128)
    step()
    torch.cuda.synchronize()
    # A step is the plan plus one launch per layer (PREFILL_LAYERS), launched
    # eagerly back to back: the launches queue behind each other and the
    # events time the kernels; a graph replay would add its own gap (--graph
    # measures that). The figure is per launch.
    if args.graph:
        graph = torch.cuda.CUDAGraph()
        with capture_graph(graph):
            st["layers_step"]()
        run = graph.replay
    else:
        run = st["layers_step"]
    ms = time_launches(torch, run, args, max(1, args.steps // 5)) / PREFILL_LAYERS
    single_ms = unplanned_ms = None
    if not args.planned_only:
        single_ms = time_launches(torch, step, args, args.steps)
        unplanned_ms = time_launches(torch, lambda: step(planned=False), args, args.steps)
        log(f"single call (no shared plan): {single_ms * 1e3:.1f} us, unplanned launch: "
            f"{unplanned_ms * 1e3:.1f} us")
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    if args.copy_calibration_mib:
        copy_calibration(torch, args.copy_calibration_mib)
    flops = st["flops"]
    tflops = flops / (ms * 1e-3) / 1e12
    log(f"{ms * 1e3:.1f} us per launch, {tflops:.1f} TFLOP/s")
    # Beside it, the no-prefix (direct) prefill on contiguous K/V: 8 prompts
    # of 512 tokens, the same kernel without a block table.
    d_lens = np.full(8, 512, dtype=np.int32)
    d_cu = torch.tensor(np.concatenate([[0], np.cumsum(d_lens)]).astype(np.int32), device=dev)
    d_rows = int(d_lens.sum())
    dq = torch.randn((d_rows, 32, 128), generator=gen, device=dev).to(torch.bfloat16)
    dk = torch.randn((d_rows, 8, 128), generator=gen, device=dev).to(torch.bfloat16)
    dv = torch.randn((d_rows, 8, 128), generator=gen, device=dev).to(torch.bfloat16)
    from microinfer_amd.layer.hip_paged_attention import prefill_plan

    def direct():
        plan = prefill_plan(d_cu, d_cu, num_tokens=d_rows, num_q_heads=32, num_kv_heads=8,
                            head_dim=128, dtype=dq.dtype, num_kv_rows=d_rows, paged=False)
        for _ in range(PREFILL_LAYERS):
            hip_paged_prefill(dq, dk, dv, d_cu, d_cu, None, max_seqlen_q=512, scale=scale,
                              plan=plan)

    for _ in range(max(1, args.warmup)):
        direct()
    start.record()
    for _ in range(max(1, args.steps // 5)):
        direct()
    end.record()
    torch.cuda.synchronize()
    d_ms = start.elapsed_time(end) / max(1, args.steps // 5) / PREFILL_LAYERS
    d_flops = prefill_flops(d_lens, d_lens, num_q_heads=32, head_dim=128)
    log(f"direct prefill: {d_ms * 1e3:.1f} us per launch, {d_flops / d_ms / 1e9:.1f} TFLOP/s")
    result = {
        "metric": "paged chunked-prefill attention TFLOP/s (% of bf16 dense MFMA peak)",
        "value": round(tflops, 2),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "warmup_seconds": args.warmup_seconds,
        "ms_per_step": round(ms, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic: seeded N(0,1) Q/K/V, random block tables with shared prefix blocks",
        "config": {
            "workload": ("mixed chunked prefill, Qwen3-8B attention (32 Q / 8 KV heads, "
                         "head_dim 128), bf16, block 16, pool 65536 blocks: 8 chunks of 512 "
                         "rows on prefixes U[0,3072] (first 1024 tokens shared) + 24 decode "
                         "rows with contexts U[256,2048] (seed 0); a step is one launch plan "
                         f"and {PREFILL_LAYERS} varlen launches sharing it (Qwen3-8B's layers), "
                         + ("hipGraph replay" if args.graph else "launched eagerly back to back")
                         + "; the figure is per launch"),
            "query_rows": total_q,
            "launches_per_plan": PREFILL_LAYERS,
            "single_call_us": round(single_ms * 1e3, 3) if single_ms else None,
            "single_call": ("one call without a shared plan: it plans for itself only when it "
                            "has fewer (query block, KV head) items than two per CU (this "
                            "batch has more, so it runs unplanned)"),
            "unplanned_us": round(unplanned_ms * 1e3, 3) if unplanned_ms else None,
            "unplanned": "mi_paged_prefill: one workgroup per (query block, KV head), no plan",
            "flops_per_launch": flops,
            "kv_layout": args.layout,
            "direct_prefill_us": round(d_ms * 1e3, 3),
            "direct_prefill_tflops": round(d_flops / d_ms / 1e9, 2),
            "direct_prefill": ("no-prefix prefill of 8 prompts x 512 tokens on contiguous K/V "
                               f"(no block table), same heads; one plan per {PREFILL_LAYERS} "
                               "launches, per launch"),
        },
        "roofline": {
            "bound": "mfma",
            "achieved": round(tflops, 2),
            "peak": MFMA_BF16_PEAK_TFLOPS,
            "unit": "TFLOP/s",
            "frac": round(tflops / MFMA_BF16_PEAK_TFLOPS, 4),
            "traffic": measured_traffic(PREFILL_TRAFFIC),
            "kernel": "paged_prefill_mfma_kernel",
            "flops_per_launch": flops,
            "us_per_launch": round(ms * 1e3, 3),
            "peak_source": "vendor dense bf16 MFMA figure (2.5 PFLOP/s); peak_measured "
                           "is a library GEMM on the same box",
        },
    }
    log("timing a dense bf16 library GEMM for the measured peak")
    gemm = measured_bf16_gemm_peak(torch)
    result["roofline"]["peak_measured"] = gemm["tflops"]
    result["roofline"]["peak_measured_detail"] = gemm
    result["roofline"]["frac_of_measured"] = round(tflops / gemm["tflops"], 4)
    if not args.no_cpu_baseline:
        log("timing the CPU oracle on a sample of the batch")
        result["cpu_baseline"] = prefill_cpu_baseline(torch, batch, q, cache)
    print(json.dumps(result), flush=True)
    return 0


class _DecodeSeq:
    """The attributes of a scheduled sequence that the metadata build reads."""

    __slots__ = ("token_ids", "last_token", "block_table", "num_cached_tokens",
                 "num_scheduled_tokens")

    def __init__(self, token_ids, block_table):
        self.token_ids = token_ids
        self.last_token = token_ids[-1]
        self.block_table = block_table
        self.num_cached_tokens = len(token_ids) - 1
        self.num_scheduled_tokens = 1

    def __len__(self):
        return len(self.token_ids)

    def __getitem__(self, key):
        return self.token_ids[key]


def run_step_metadata(args) -> int:
    """Decode-step metadata of the 0.6B engine shape: 64 running requests
    (128-token prompts, up to 16 generated tokens), pool 4096 blocks + the pad
    block, block 16, written into the 64-row graph bucket at table width 4097."""
    import torch

    from microinfer_amd import _lib
    from microinfer_amd.runner import StepMetadataBuilder

    dev = torch.device("cuda", 0)
    num_blocks, block_size, batch, prompt, gen_tokens = 4096, 16, 64, 128, 16
    width = num_blocks + 1
    rng = np.random.default_rng(0)
    perm = rng.permutation(num_blocks).tolist()
    steps = []  # one list of sequences per decode step, built before timing
    for t in range(gen_tokens):
        seqs = []
        for r in range(batch):
            length = prompt + 1 + t
            blocks = perm[r * 10:r * 10 + (length + block_size - 1) // block_size]
            seqs.append(_DecodeSeq(rng.integers(0, 151936, length).tolist(), blocks))
        steps.append(seqs)
    builder = StepMetadataBuilder(block_size, dev, pad_block_id=num_blocks)
    buffers = builder.pad_buffers(batch, width)

    def run(k, sync):
        for i in range(k):
            builder.fill_decode(buffers, steps[i % gen_tokens], rows=batch)
            if sync:  # an engine reads the step's tokens back before the next step
                torch.cuda.synchronize()

    run(args.warmup, True)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    run(args.steps, True)
    us_per_step = (time.perf_counter() - t0) / args.steps * 1e6
    t0 = time.perf_counter()
    run(args.steps, False)
    host_us = (time.perf_counter() - t0) / args.steps * 1e6
    torch.cuda.synchronize()
    log(f"{us_per_step:.1f} us per synchronised step, {host_us:.1f} us host per pipelined step")

    # Kernel alone, timed with events on the stream it is launched on (the
    # compact description of the last step is still in the builder's upload).
    lib = _lib.load()
    seqs = steps[-1]
    lengths = np.array([len(s) for s in seqs], dtype=np.int32)
    counts = np.array([len(s.block_table) for s in seqs], dtype=np.int32)
    offsets = np.concatenate([[0], np.cumsum(counts)]).astype(np.int32)
    blocks = np.concatenate([s.block_table for s in seqs]).astype(np.int32)
    compact = torch.tensor(np.concatenate([np.arange(batch + 1, dtype=np.int32), lengths - 1,
                                           offsets, blocks]), device=dev)
    tokens = torch.tensor([s.last_token for s in seqs], dtype=torch.int64, device=dev)
    cu_q, starts = compact[:batch + 1], compact[batch + 1:2 * batch + 1]
    d_offsets, d_blocks = compact[2 * batch + 1:3 * batch + 2], compact[3 * batch + 2:]
    stream = _lib.stream_handle(dev)

    def launch():
        _lib.check(lib.mi_step_metadata(
            cu_q.data_ptr(), starts.data_ptr(), d_offsets.data_ptr(), d_blocks.data_ptr(),
            tokens.data_ptr(), batch, batch, batch, block_size, num_blocks,
            buffers.block_tables.data_ptr(), width, width, buffers.context_lens.data_ptr(),
            buffers.slot_mapping.data_ptr(), buffers.positions.data_ptr(),
            buffers.input_ids.data_ptr(), stream), "mi_step_metadata")

    for _ in range(args.warmup):
        launch()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record()
    for _ in range(args.steps):
        launch()
    end.record()
    torch.cuda.synchronize()
    kernel_us = start.elapsed_time(end) / args.steps * 1e3
    # Algorithmic bytes: the table and four per-row outputs written, the
    # compact description read.
    nbytes = batch * width * 4 + batch * (8 + 8 + 4 + 4) + compact.numel() * 4 + batch * 8
    achieved = nbytes / (kernel_us * 1e-6) / 1e9
    result = {
        "metric": "decode step metadata build us/step (64-row graph bucket, table width 4097)",
        "value": round(us_per_step, 2),
        "unit": "us/step",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "warmup_seconds": args.warmup_seconds,
        "ms_per_step": round(us_per_step / 1e3, 5),
        "higher_is_better": False,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int32",
        "data": "synthetic: 64 decode sequences, random token ids and disjoint block tables",
        "config": {
            "workload": ("decode-step metadata for the Qwen3-0.6B engine run: 64 requests, "
                         "contexts 129-144, block 16, pool 4096 + 1 pad block, bucket 64 at "
                         "width 4097; host packing + one pinned upload + one expansion launch "
                         "per step"),
            "host_us_per_step_pipelined": round(host_us, 2),
            "timing": "each timed step ends with a device synchronisation, as an engine "
                      "step does when it reads its sampled tokens",
        },
        "roofline": {
            "bound": "hbm",
            "achieved": round(achieved, 1),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBS, 4),
            "traffic": None,
            "kernel": "step_metadata_kernel",
            "bytes_per_launch": nbytes,
            "us_per_launch": round(kernel_us, 3),
        },
    }
    if not args.no_cpu_baseline:
        result["cpu_baseline"] = step_metadata_cpu_baseline(torch, steps, builder, batch,
                                                           width, num_blocks, dev)
    print(json.dumps(result), flush=True)
    return 0


def step_metadata_cpu_baseline(torch, steps, builder, batch, width, num_blocks, dev,
                               samples: int = 200):
    """The reference's host build: every row filled on the CPU (the oracle's
    restatement of runner.py:160-176, :561-576) and the five arrays, the
    table at full width, copied to the device from pinned memory."""
    from oracle.step_metadata import decode_rows

    pinned = {}
    device = {}

    def one(seqs):
        rows = decode_rows(seqs, builder.block_size, rows=batch, width=width,
                           pad_block=num_blocks)
        for key, array in rows.items():
            if key not in pinned:
                pinned[key] = torch.empty(array.shape, dtype=torch.from_numpy(array).dtype,
                                          pin_memory=True)
                device[key] = torch.empty_like(pinned[key], device=dev)
            pinned[key].numpy()[...] = array
            device[key].copy_(pinned[key], non_blocking=True)
        torch.cuda.synchronize()

    one(steps[0])
    t0 = time.perf_counter()
    for i in range(samples):
        one(steps[i % len(steps)])
    per = (time.perf_counter() - t0) / samples
    return {
        "value": round(per * 1e6, 2),
        "unit": "us/step",
        "cores": 1,
        "kind": "port",
        "sample": (f"{samples} decode steps of the same workload: rows filled on the host by "
                   "the oracle's restatement of the runner, then 5 pinned copies "
                   f"including the full-width table, synchronised each step ({cpu_model()})"),
    }


def _qk_norm_rope_inputs(torch, dev, tokens, hq, hkv, d, num_blocks, block_size, seed):
    from microinfer_amd.layer.hip_qk_norm_rope import rope_tables

    gen = torch.Generator(device=dev).manual_seed(seed)
    qkv = torch.randn((tokens, (hq + 2 * hkv) * d), generator=gen, device=dev).to(torch.bfloat16)
    qw = (1 + 0.1 * torch.randn(d, generator=gen, device=dev)).to(torch.bfloat16)
    kw = (1 + 0.1 * torch.randn(d, generator=gen, device=dev)).to(torch.bfloat16)
    cos, sin = rope_tables(40960, d, 1_000_000.0, device=dev)
    rng = np.random.default_rng(seed)
    positions = torch.tensor(rng.integers(0, 40960, tokens), dtype=torch.int64, device=dev)
    slots = torch.tensor(rng.permutation(num_blocks * block_size)[:tokens], dtype=torch.int32,
                         device=dev)
    return qkv, qw, kw, cos, sin, positions, slots


def run_qk_norm_rope(args) -> int:
    """Fused Q/K RMSNorm + RoPE + KV append for the 4120 tokens of the mixed
    chunked-prefill step (Qwen3-8B heads: 32 Q / 8 KV, head_dim 128, bf16,
    pool 65536 blocks of 16), one launch per step; the 0.6B decode step (32
    tokens, 16 / 8 heads) is timed beside it (launch-bound)."""
    import torch

    from microinfer_amd.layer.hip_qk_norm_rope import qk_norm_rope_append

    dev = torch.device("cuda", 0)
    tokens, hq, hkv, d, num_blocks, block_size = 4120, 32, 8, 128, 65536, 16
    kc = torch.zeros((num_blocks, block_size, hkv, d), dtype=torch.bfloat16, device=dev)
    vc = torch.zeros_like(kc)
    qkv, qw, kw, cos, sin, positions, slots = _qk_norm_rope_inputs(
        torch, dev, tokens, hq, hkv, d, num_blocks, block_size, 0)

    def step(x, n_q, n_kv, pos, slot):
        return qk_norm_rope_append(x, q_weight=qw, k_weight=kw, eps=1e-6, cos_table=cos,
                                   sin_table=sin, positions=pos, num_q_heads=n_q,
                                   num_kv_heads=n_kv, head_dim=d, slot_mapping=slot,
                                   key_cache=kc[:, :, :n_kv], value_cache=vc[:, :, :n_kv])

    def timed(fn, k):
        start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        start.record()
        for _ in range(k):
            fn()
        end.record()
        torch.cuda.synchronize()
        return start.elapsed_time(end) / k * 1e3

    run = lambda: step(qkv, hq, hkv, positions, slots)  # noqa: E731
    warm_up(torch, run, args)
    us = timed(run, args.steps)
    # Algorithmic bytes: the fused rows read, Q written, K and V cache rows
    # written, the cos/sin rows gathered, positions and slots read.
    es = 2
    nbytes = (tokens * (hq + 2 * hkv) * d * es + tokens * hq * d * es
              + tokens * 2 * hkv * d * es + tokens * d * 4 + tokens * 12)
    achieved = nbytes / (us * 1e-6) / 1e9
    # The 0.6B decode step: 28 layer launches of 32 tokens, replayed from a
    # hipGraph so the time is the launches', not the Python wrapper's.
    small = _qk_norm_rope_inputs(torch, dev, 32, 16, 8, d, num_blocks, block_size, 1)
    dec = lambda: step(small[0], 16, 8, small[5], small[6])  # noqa: E731
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        dec()
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with capture_graph(graph):
        for _ in range(28):
            dec()
    for _ in range(args.warmup):
        graph.replay()
    dec_us = timed(graph.replay, args.steps) / 28
    log(f"{us:.2f} us per 4120-token launch ({achieved:.0f} GB/s), "
        f"{dec_us:.2f} us per 32-token decode launch")
    result = {
        "metric": "fused QK RMSNorm + RoPE + KV append HBM GB/s (% peak)",
        "value": round(achieved, 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "warmup_seconds": args.warmup_seconds,
        "ms_per_step": round(us / 1e3, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic: seeded N(0,1) fused QKV rows, random positions < 40960, "
                "distinct random slots",
        "config": {
            "workload": ("Q/K RMSNorm + RoPE (split-half, base 1e6) + KV append of the 4120 "
                         "tokens of the mixed chunked-prefill step, Qwen3-8B heads (32 Q / "
                         "8 KV, head_dim 128), bf16, pool 65536 blocks of 16, one launch"),
            "tokens": tokens,
            "decode_launch_us": round(dec_us, 3),
            "decode_launch": ("Qwen3-0.6B heads (16 Q / 8 KV), 32 tokens: 28 launches "
                              "replayed from a hipGraph, time per launch (launch-bound)"),
        },
        "roofline": {
            "bound": "hbm",
            "achieved": round(achieved, 1),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBS, 4),
            "traffic": measured_traffic(QK_TRAFFIC),
            "kernel": "qk_norm_rope_kernel",
            "bytes_per_launch": nbytes,
            "us_per_launch": round(us, 3),
        },
    }
    if not args.no_cpu_baseline:
        result["cpu_baseline"] = qk_norm_rope_cpu_baseline(torch, qkv, qw, kw, cos, sin,
                                                           positions, slots, hq, hkv, d)
    print(json.dumps(result), flush=True)
    return 0


def qk_norm_rope_cpu_baseline(torch, qkv, qw, kw, cos, sin, positions, slots, hq, hkv, d,
                              sample: int = 1024, runs: int = 5):
    """The oracle's restatement on the host over the first ``sample`` tokens."""
    from oracle import qk_norm_rope as ref

    x = qkv[:sample].float().cpu().numpy()
    w_q, w_k = qw.float().cpu().numpy(), kw.float().cpu().numpy()
    c, s_ = cos.cpu().numpy(), sin.cpu().numpy()
    pos = positions[:sample].cpu().numpy()
    slot = slots[:sample].cpu().numpy() % (64 * 16)
    kc = np.zeros((64, 16, hkv, d), dtype=np.float32)
    vc = np.zeros_like(kc)
    times = []
    for i in range(runs + 1):
        t0 = time.perf_counter()
        ref.qk_norm_rope_append(x, w_q, w_k, 1e-6, c, s_, pos, slot, kc, vc, num_q_heads=hq,
                                num_kv_heads=hkv, head_dim=d, interleaved=False, dtype="bf16")
        if i:
            times.append(time.perf_counter() - t0)
    sec = statistics.median(times)
    nbytes = (sample * (hq + 2 * hkv) * d * 2 + sample * hq * d * 2 + sample * 2 * hkv * d * 2
              + sample * d * 4 + sample * 12)
    return {
        "value": round(nbytes / sec / 1e9, 3),
        "unit": "GB/s",
        "cores": blas_threads(),
        "kind": "port",
        "sample": f"{sample} of the 4120 tokens (same bytes formula), x {runs} runs after 1 "
                  f"warm-up, median {sec * 1e3:.1f} ms; numpy on the host CPU ({cpu_model()})",
    }


def run_greedy(args) -> int:
    """Greedy selection over the logits of the 0.6B decode step: 32 rows of
    the Qwen3 vocabulary (151936), bf16, one launch (the argmax the decode
    graph captures). torch.argmax on the same rows is timed beside it."""
    import torch

    from microinfer_amd.layer.hip_sampler import greedy_argmax

    dev = torch.device("cuda", 0)
    rows, vocab = 32, 151936
    gen = torch.Generator(device=dev).manual_seed(0)
    logits = torch.randn((rows, vocab), generator=gen, device=dev).to(torch.bfloat16)
    out = torch.empty(rows, dtype=torch.int64, device=dev)

    def timed(fn, k):
        start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        start.record()
        for _ in range(k):
            fn()
        end.record()
        torch.cuda.synchronize()
        return start.elapsed_time(end) / k * 1e3

    run = lambda: greedy_argmax(logits, out=out)  # noqa: E731
    warm_up(torch, run, args)
    eager_us = timed(run, args.steps)
    # The decode graph replays the launch with no host work around it: time
    # 20 back-to-back launches captured in a hipGraph (after one call on the
    # capture stream, which creates that stream's zeroed row state).
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        run()
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with capture_graph(graph, stream=side):
        for _ in range(20):
            run()
    for _ in range(args.warmup):
        graph.replay()
    us = timed(graph.replay, args.steps) / 20
    ref = lambda: torch.argmax(logits, dim=-1)  # noqa: E731
    for _ in range(args.warmup):
        ref()
    torch_us = timed(ref, args.steps)
    assert torch.equal(out, torch.argmax(logits, dim=-1))
    nbytes = rows * vocab * 2 + rows * 8  # logits read, tokens written
    achieved = nbytes / (us * 1e-6) / 1e9
    log(f"{us:.2f} us per launch in a graph ({achieved:.0f} GB/s), {eager_us:.2f} us per eager "
        f"call; torch.argmax {torch_us:.2f} us")
    result = {
        "metric": "greedy argmax over decode logits HBM GB/s (% peak)",
        "value": round(achieved, 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "warmup_seconds": args.warmup_seconds,
        "ms_per_step": round(us / 1e3, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic: seeded N(0,1) logits",
        "config": {
            "workload": ("greedy token selection (argmax, first index of the maximum) over "
                         "32 rows x 151936 bf16 logits, the 0.6B decode step's batch, one "
                         "launch"),
            "rows": rows,
            "vocab": vocab,
            "timing": "20 launches replayed from a hipGraph, time per launch",
            "eager_call_us": round(eager_us, 3),
            "torch_argmax_us": round(torch_us, 3),
        },
        "roofline": {
            "bound": "hbm",
            "achieved": round(achieved, 1),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBS, 4),
            "traffic": measured_traffic(GREEDY_TRAFFIC),
            "kernel": "greedy_argmax_kernel",
            "bytes_per_launch": nbytes,
            "us_per_launch": round(us, 3),
        },
    }
    if not args.no_cpu_baseline:
        result["cpu_baseline"] = greedy_cpu_baseline(logits, nbytes)
    print(json.dumps(result), flush=True)
    return 0


def greedy_cpu_baseline(logits, nbytes, runs: int = 5):
    """The oracle's restatement on the host over all 32 rows."""
    from oracle.greedy import greedy_argmax as ref

    host = logits.float().cpu().numpy()
    times = []
    for i in range(runs + 1):
        t0 = time.perf_counter()
        ref(host)
        if i:
            times.append(time.perf_counter() - t0)
    sec = statistics.median(times)
    return {
        "value": round(nbytes / sec / 1e9, 3),
        "unit": "GB/s",
        "cores": 1,
        "kind": "port",
        "sample": f"all 32 rows (same bytes formula, bf16 logits widened once before timing), "
                  f"x {runs} runs after 1 warm-up, median {sec * 1e3:.1f} ms; numpy on the "
                  f"host CPU ({cpu_model()})",
    }


def measure_engine(batches: int, warmup: int) -> dict:
    """The engine workload (``microinfer_amd.workloads``: random-init
    Qwen3-0.6B, bf16, 64 requests x 128 uniform-random prompt ids arriving
    together, 16 greedy tokens each, block 16, 4096 blocks, hipGraph decode,
    mixed batches): ``batches`` batches run to completion after ``warmup``
    untimed ones, fresh prompts each time.

    Output tok/s = output tokens / wall time of the batches
    (microinfer bench/online.py:81-91 semantics); decode tok/s = tokens of
    decode-only steps / the time of those steps."""
    import torch

    from microinfer_amd.engine.blockmanager import BlockManager
    from microinfer_amd.engine.llm_engine import LLMEngine
    from microinfer_amd.engine.model import QwenConfig, Qwen3Model
    from microinfer_amd.engine.model_runner import ModelRunner
    from microinfer_amd.engine.scheduler import Scheduler
    from microinfer_amd.engine.sequence import Sequence
    from microinfer_amd.workloads import (ENGINE_BLOCK_SIZE, ENGINE_NUM_BLOCKS,
                                          ENGINE_OUTPUT_LEN, ENGINE_REQUESTS, engine_config,
                                          engine_prompts, engine_sampling)

    config = engine_config()
    log("building random-init Qwen3-0.6B for the engine workload")
    model = Qwen3Model(QwenConfig(), dtype=torch.bfloat16, device="cuda", seed=0)
    runner = ModelRunner(model, config, num_blocks=ENGINE_NUM_BLOCKS,
                         block_size=ENGINE_BLOCK_SIZE)
    manager = BlockManager(ENGINE_NUM_BLOCKS, ENGINE_BLOCK_SIZE)
    engine = LLMEngine(Scheduler(config, manager), runner)
    params = engine_sampling()

    def one_batch(seed):
        seqs = [Sequence(p, params) for p in engine_prompts(seed, model.config.vocab_size)]
        for seq in seqs:
            engine.add_request(seq)
        decode_s, decode_tokens, steps = 0.0, 0, 0
        torch.cuda.synchronize()
        start = time.perf_counter()
        while not engine.is_finished():
            t0 = time.perf_counter()
            _, num_tokens = engine.step()  # returns host token ids: synchronised
            if num_tokens < 0:
                decode_s += time.perf_counter() - t0
                decode_tokens -= num_tokens
            steps += 1
        wall = time.perf_counter() - start
        assert all(len(s.completion_token_ids) == ENGINE_OUTPUT_LEN for s in seqs)
        manager.reset_prefix_cache()
        return wall, decode_s, decode_tokens, steps

    for i in range(max(1, warmup)):
        one_batch(1000 + i)
    walls, decodes, dec_tokens, steps = [], [], 0, 0
    for i in range(batches):
        wall, dec_s, dec_tok, n = one_batch(i)
        walls.append(wall)
        decodes.append(dec_s)
        dec_tokens += dec_tok
        steps += n
    output_tps = ENGINE_REQUESTS * ENGINE_OUTPUT_LEN * batches / sum(walls)
    decode_tps = dec_tokens / sum(decodes)
    decode_steps = dec_tokens / ENGINE_REQUESTS
    decode_step_us = sum(decodes) / decode_steps * 1e6 if dec_tokens else 0.0
    log(f"engine: {output_tps:.0f} output tok/s over {batches} batches "
        f"({statistics.mean(walls) * 1e3:.1f} ms each), decode {decode_tps:.0f} tok/s, "
        f"{decode_step_us:.0f} us per decode step")
    return dict(model=model, output_tps=output_tps, decode_tps=decode_tps,
                decode_step_us=decode_step_us, wall_ms=statistics.mean(walls) * 1e3,
                steps_per_batch=steps / batches, batches=batches, warmup=max(1, warmup))


def engine_step_bytes(c, requests: int, mean_ctx: float) -> int:
    """Bytes a full decode step streams: every weight once (28 layers of QKV,
    output, gate/up and down products, the norms, the untied vocabulary
    product) plus the batch's K/V."""
    per_layer = ((c.num_q_head + 2 * c.num_kv_head) * c.head_dim * c.hidden_dim
                 + c.hidden_dim * c.num_q_head * c.head_dim
                 + 3 * c.MLP_inter_dim * c.hidden_dim + 2 * c.hidden_dim + 2 * c.head_dim)
    weight_bytes = 2 * (c.num_hidden_layer * per_layer + c.vocab_size * c.hidden_dim
                        + c.hidden_dim)
    kv_bytes = 2 * 2 * c.num_hidden_layer * requests * mean_ctx * c.num_kv_head * c.head_dim
    return int(weight_bytes + kv_bytes)


def run_engine(args) -> int:
    """The engine workload; a bench step is one batch run to completion."""
    from microinfer_amd.workloads import ENGINE_OUTPUT_LEN, ENGINE_PROMPT_LEN, ENGINE_REQUESTS

    e = measure_engine(args.steps, args.warmup)
    step_bytes = engine_step_bytes(e["model"].config, ENGINE_REQUESTS,
                                   ENGINE_PROMPT_LEN + ENGINE_OUTPUT_LEN / 2)
    us = e["decode_step_us"]
    achieved = step_bytes / (us * 1e-6) / 1e9 if us else 0.0
    result = {
        "metric": "engine output tokens/s (random-init Qwen3-0.6B, 64 x 128-token prompts, "
                  "16 greedy outputs)",
        "value": round(e["output_tps"], 1),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": e["warmup"],
        "ms_per_step": round(e["wall_ms"], 3),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic: random-init weights N(0, 0.02) (seed 0), uniform-random prompt ids",
        "config": {
            "workload": ENGINE_WORKLOAD_TEXT + "; a bench step is one batch to completion",
            "decode_tokens_per_s": round(e["decode_tps"], 1),
            "decode_step_us": round(us, 1),
            "engine_steps_per_batch": e["steps_per_batch"],
        },
        "roofline": {
            "bound": "hbm",
            "achieved": round(achieved, 1),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBS, 4),
            "traffic": None,
            "kernel": "decode step (hipGraph replay: 28 layers of GEMMs, fused Q/K norm + "
                      "RoPE + append, paged decode; vocabulary projection; argmax), host "
                      "time included",
            "bytes_per_launch": step_bytes,
            "us_per_launch": round(us, 1),
        },
    }
    if not args.no_cpu_baseline:
        result["cpu_baseline"] = engine_cpu_baseline(e["model"])
    print(json.dumps(result), flush=True)
    return 0


ENGINE_WORKLOAD_TEXT = (
    "engine: random-init Qwen3-0.6B (bf16, weights N(0, 0.02), seed 0), 64 requests x 128 "
    "uniform-random prompt ids arriving together, greedy, 16 output tokens (EOS ignored), "
    "block 16, 4096 blocks, hipGraph decode, mixed batches, max_num_seqs 64, "
    "max_num_batched_tokens 4096, max_num_prefill_tokens 512")


def engine_cpu_baseline(model, decode_steps: int = 5) -> dict:
    """The same engine on the host: the product's Scheduler and BlockManager
    drive a KV-cached paged float32 forward (oracle/qwen3_paged_host.py:
    numpy GEMMs, the oracle's Q/K norm + RoPE + append into a paged cache and
    its paged attention) over the workload's first batch; the prefill steps
    run untimed, then ``decode_steps`` batch-64 decode steps are timed."""
    from microinfer_amd.engine.blockmanager import BlockManager
    from microinfer_amd.engine.llm_engine import LLMEngine
    from microinfer_amd.engine.scheduler import Scheduler
    from microinfer_amd.engine.sequence import Sequence
    from microinfer_amd.workloads import (ENGINE_BLOCK_SIZE, ENGINE_NUM_BLOCKS, engine_config,
                                          engine_prompts, engine_sampling)
    from oracle.qwen3_paged_host import HostPagedRunner

    log("CPU baseline: host paged engine over the workload's first batch")
    runner = HostPagedRunner(model.host_weights(), model.config, ENGINE_NUM_BLOCKS,
                             ENGINE_BLOCK_SIZE)
    engine = LLMEngine(Scheduler(engine_config(), BlockManager(ENGINE_NUM_BLOCKS,
                                                                ENGINE_BLOCK_SIZE)), runner)
    for prompt in engine_prompts(0, model.config.vocab_size):
        engine.add_request(Sequence(prompt, engine_sampling()))
    t0 = time.perf_counter()
    prefill_s, prefill_steps = 0.0, 0
    while True:  # prompt and mixed steps until the first decode-only step
        t = time.perf_counter()
        _, num_tokens = engine.step()
        if num_tokens < 0:
            break
        prefill_s += time.perf_counter() - t
        prefill_steps += 1
    times, tokens = [], 0
    for _ in range(decode_steps):
        t = time.perf_counter()
        _, num_tokens = engine.step()
        times.append(time.perf_counter() - t)
        tokens -= num_tokens
    total = time.perf_counter() - t0
    return {
        "value": round(tokens / sum(times), 2),
        "unit": "decode tokens/s",
        "cores": blas_threads(),
        "kind": "port",
        "sample": (f"first batch of the engine workload: {prefill_steps} prompt/mixed steps "
                   f"untimed ({prefill_s:.1f} s), then {decode_steps} decode steps of "
                   f"{tokens // decode_steps} rows timed ({sum(times):.2f} s); float32 numpy "
                   f"KV-cached paged forward (oracle.qwen3_paged_host) under the product's "
                   f"Scheduler/BlockManager, {total:.1f} s in all, on the host CPU "
                   f"({cpu_model()}, os.cpu_count()={os.cpu_count()})"),
    }


def _graph_time(torch, fn, launches: int, replays: int, warmup: int) -> float:
    """Microseconds per launch of ``fn`` (which makes ``launches`` launches)
    replayed from a hipGraph after one call on the capture stream."""
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        fn()
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with capture_graph(graph, stream=side):
        fn()
    for _ in range(max(1, warmup)):
        graph.replay()
    torch.cuda.synchronize()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record()
    for _ in range(replays):
        graph.replay()
    end.record()
    torch.cuda.synchronize()
    return start.elapsed_time(end) / replays / launches * 1e3


def _hbm_line(metric, achieved, us, nbytes, kernel, args, data, config, cpu=None,
              traffic=None):
    result = {
        "metric": metric,
        "value": round(achieved, 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(us / 1e3, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": data,
        "config": config,
        "roofline": {
            "bound": "hbm",
            "achieved": round(achieved, 1),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBS, 4),
            "traffic": traffic,
            "kernel": kernel,
            "bytes_per_launch": int(nbytes),
            "us_per_launch": round(us, 3),
        },
    }
    if cpu is not None:
        result["cpu_baseline"] = cpu
    print(json.dumps(result), flush=True)
    return 0


def _median_time(fn, runs: int = 5) -> float:
    fn()
    times = []
    for _ in range(runs):
        t0 = time.perf_counter()
        fn()
        times.append(time.perf_counter() - t0)
    return statistics.median(times)


def run_append(args) -> int:
    """KV append of the mixed chunked-prefill step's 4120 tokens (Qwen3-8B KV
    heads: 8 x 128, bf16) into a 65536-block pool at distinct random slots;
    20 launches replayed from a hipGraph. The 0.6B decode step's 32-row
    append is timed beside it (launch-bound)."""
    import torch

    from microinfer_amd.worker.kv_cache import KVCache

    dev = torch.device("cuda", 0)
    tokens, hkv, d, num_blocks, bs = 4120, 8, 128, 65536, 16
    cache = KVCache(1, num_blocks, bs, hkv, d, dtype=torch.bfloat16, device=dev)
    view = cache.layer(0)
    rng = np.random.default_rng(0)
    slots = rng.permutation(num_blocks * bs)[:tokens].astype(np.int32)
    slot_t = torch.tensor(slots, device=dev)
    gen = torch.Generator(device=dev).manual_seed(0)
    keys = torch.randn((tokens, hkv, d), generator=gen, device=dev).to(torch.bfloat16)
    values = torch.randn((tokens, hkv, d), generator=gen, device=dev).to(torch.bfloat16)
    launches = 20

    def many():
        for _ in range(launches):
            view.write_slots(slot_t, keys, values)

    us = _graph_time(torch, many, launches, args.steps, args.warmup)
    small = slot_t[:32].contiguous()
    small_us = _graph_time(torch, lambda: [view.write_slots(small, keys[:32], values[:32])
                                           for _ in range(launches)], launches, args.steps,
                           args.warmup)
    nbytes = 2 * 2 * tokens * hkv * d * 2 + 4 * tokens  # K and V rows read + written, slots
    achieved = nbytes / (us * 1e-6) / 1e9
    log(f"{us:.2f} us per 4120-row append ({achieved:.0f} GB/s), {small_us:.2f} us per 32-row")
    cpu = None
    if not args.no_cpu_baseline:
        from oracle import kv_append

        host_k = np.zeros((4096, bs, hkv, d), dtype=np.float32)
        host_v = np.zeros_like(host_k)
        k32, v32 = keys.float().cpu().numpy(), values.float().cpu().numpy()
        host_slots = slots % (4096 * bs)
        sec = _median_time(lambda: kv_append(host_k, host_v, host_slots, k32, v32))
        cpu = {"value": round(nbytes / sec / 1e9, 3), "unit": "GB/s", "cores": 1,
               "kind": "port",
               "sample": f"all 4120 rows into a 4096-block host pool (same bytes formula), "
                         f"median of 5 after 1 warm-up, {sec * 1e3:.1f} ms; numpy on the host "
                         f"CPU ({cpu_model()})"}
    return _hbm_line(
        "KV append HBM GB/s (% peak)", achieved, us, nbytes, "kv_append_kernel", args,
        "synthetic: seeded N(0,1) K/V rows, distinct random slots",
        {"workload": ("KV append of 4120 tokens (the mixed chunked-prefill step), 8 KV heads x "
                      "128, bf16, head-major pool of 65536 blocks of 16, distinct random slots; "
                      "20 launches replayed from a hipGraph, time per launch"),
         "tokens": tokens, "decode_append_us": round(small_us, 3),
         "decode_append": "32 rows (the 0.6B decode step), same pool, launch-bound"}, cpu,
        measured_traffic(APPEND_TRAFFIC))


def run_gather(args) -> int:
    """Block-table gather of every request of the mixed chunked-prefill step
    (8 chunks on prefixes U[0,3072] + 24 decode rows, Qwen3-8B KV heads,
    bf16) into contiguous varlen K/V, one launch."""
    import torch

    from microinfer_amd.layer.hip_paged_attention import hip_gather_kv
    from microinfer_amd.workloads import make_mixed_prefill_batch

    dev = torch.device("cuda", 0)
    batch = make_mixed_prefill_batch()
    hkv, d, bs = 8, 128, batch.block_size
    shape = (batch.pool_blocks, bs, hkv, d)
    gen = torch.Generator(device=dev).manual_seed(0)
    kc = torch.randn(shape, generator=gen, device=dev).to(torch.bfloat16)
    vc = torch.randn(shape, generator=gen, device=dev).to(torch.bfloat16)
    tables = torch.tensor(batch.block_tables, device=dev)
    contexts = [int(c) for c in batch.context_lens]
    total = sum(contexts)
    # The kernel path: cu_seqlens_k already on the device (gather_paged_kv,
    # the reference-shaped entry, builds it from host contexts each call).
    cu_k = torch.tensor(batch.cu_seqlens_k, device=dev)
    run = lambda: hip_gather_kv(kc, vc, tables, cu_k, total)  # noqa: E731
    warm_up(torch, run, args)
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record()
    for _ in range(args.steps):
        run()
    end.record()
    torch.cuda.synchronize()
    us = start.elapsed_time(end) / args.steps * 1e3
    nbytes = 2 * 2 * total * hkv * d * 2 + 4 * sum(-(-c // bs) for c in contexts)
    achieved = nbytes / (us * 1e-6) / 1e9
    log(f"{us:.2f} us per gather of {total} rows ({achieved:.0f} GB/s)")
    cpu = None
    if not args.no_cpu_baseline:
        from oracle import gather_paged_kv as ref_gather

        sample = 4
        used = sorted({int(b) for r in range(sample)
                       for b in batch.block_tables[r, :-(-contexts[r] // bs)]})
        remap = {b: i for i, b in enumerate(used)}
        small = np.full((sample, batch.block_tables.shape[1]), -1, dtype=np.int32)
        for r in range(sample):
            for j in range(-(-contexts[r] // bs)):
                small[r, j] = remap[int(batch.block_tables[r, j])]
        idx = torch.tensor(used, device=dev)
        hk = kc.index_select(0, idx).float().cpu().numpy()
        hv = vc.index_select(0, idx).float().cpu().numpy()
        sec = _median_time(lambda: ref_gather(hk, hv, small, contexts[:sample], bs))
        sample_bytes = 2 * 2 * sum(contexts[:sample]) * hkv * d * 2
        cpu = {"value": round(sample_bytes / sec / 1e9, 3), "unit": "GB/s", "cores": 1,
               "kind": "port",
               "sample": f"the first {sample} requests ({sum(contexts[:sample])} rows, same "
                         f"bytes formula), median of 5 after 1 warm-up, {sec * 1e3:.1f} ms; "
                         f"numpy on the host CPU ({cpu_model()})"}
    return _hbm_line(
        "paged KV gather HBM GB/s (% peak)", achieved, us, nbytes, "gather_kv_kernel", args,
        "synthetic: seeded N(0,1) pools, mixed-step block tables with shared prefix blocks",
        {"workload": ("gather of all 32 requests of the mixed chunked-prefill step (8 x 512 "
                      "chunks on prefixes U[0,3072] + 24 decode rows, U[256,2048]) into "
                      "contiguous K/V, 8 KV heads x 128, bf16, pool 65536 blocks of 16, one "
                      "launch"), "rows": total}, cpu, measured_traffic(GATHER_TRAFFIC))


LONG_DECODE_CASES = ((1, 4096), (1, 16384), (1, 32768), (4, 4096), (4, 16384), (4, 32768))


def time_long_decode(torch, args, which):
    """Per-launch time of long-context decode cases ``(rows, ctx)`` (8B heads,
    pool 65536 in the ``--layout`` cache): each case replays launches over
    distinct blocks from a hipGraph. Returns (cache, kc, vc, perm, gen,
    {"RxC": (us, algorithmic bytes)})."""
    from microinfer_amd.layer.hip_paged_attention import decode_plan, hip_paged_decode
    from microinfer_amd.worker.kv_cache import KVCache

    dev = torch.device("cuda", 0)
    hq, hkv, d, bs, num_blocks = 32, 8, 128, 16, 65536
    gen = torch.Generator(device=dev).manual_seed(0)
    # The product's cache (the --layout physical layout), logical [N, B, Hkv, D] views.
    cache = KVCache(1, num_blocks, bs, hkv, d, dtype=torch.bfloat16, device=dev,
                    layout=args.layout)
    kc, vc = cache.keys[0], cache.values[0]
    for pool in (kc, vc):
        pool.copy_(torch.randn(pool.shape, generator=gen, device=dev))
    rng = np.random.default_rng(0)
    perm = torch.tensor(rng.permutation(num_blocks).astype(np.int32), device=dev)
    cases = {}
    for rows, ctx in which:
        nb = ctx // bs
        launches = min(28, num_blocks // (rows * nb))
        q = torch.randn((launches, rows, hq, d), generator=gen, device=dev).to(torch.bfloat16)
        tables = [perm[i * rows * nb:(i + 1) * rows * nb].reshape(rows, nb).contiguous()
                  for i in range(launches)]
        lens = torch.full((rows,), ctx, dtype=torch.int32, device=dev)

        def many(q=q, tables=tables, lens=lens, launches=launches, nb=nb):
            # One partition plan per step, shared by every layer's launch.
            plan = decode_plan(lens, num_kv_heads=hkv, block_size=bs, block_table_width=nb)
            for i in range(launches):
                hip_paged_decode(q[i], kc, vc, tables[i], lens, plan=plan)

        us = _graph_time(torch, many, launches, max(1, args.steps // 5), args.warmup)
        nbytes = rows * ctx * hkv * d * 2 * 2 + 2 * rows * hq * d * 2 + rows * nb * 4 + 8 * rows
        cases[f"{rows}x{ctx}"] = (us, nbytes)
        log(f"{rows} x {ctx}: {us:.2f} us per launch, {nbytes / us / 1e3:.0f} GB/s")
    return cache, kc, vc, perm, gen, cases


def run_long_decode(args) -> int:
    """Long-context decode (Qwen3-8B heads: 32 Q / 8 KV, head_dim 128, bf16,
    pool 65536 blocks of 16): 1 or 4 sequences of 4096 / 16384 / 32768
    tokens, split into partitions merged in the same launch. Each case
    replays launches over distinct blocks (more bytes than the last-level
    cache holds) from a hipGraph; ``value`` is the 4 x 32768 case."""
    import torch

    cache, kc, vc, perm, gen, cases = time_long_decode(torch, args, LONG_DECODE_CASES)
    hq, hkv, d, bs, dev = 32, 8, 128, 16, kc.device
    us, nbytes = cases["4x32768"]
    achieved = nbytes / (us * 1e-6) / 1e9
    cpu = None
    if not args.no_cpu_baseline:
        from oracle import paged_attention_reference

        nb = 4096 // bs
        idx = perm[:nb].long()
        hk = kc.index_select(0, idx).float().cpu().numpy()
        hv = vc.index_select(0, idx).float().cpu().numpy()
        q1 = torch.randn((1, hq, d), generator=gen, device=dev).to(torch.bfloat16).float()
        q1 = q1.cpu().numpy()
        table = np.arange(nb, dtype=np.int32)[None]
        sec = _median_time(lambda: paged_attention_reference(q1, hk, hv, table, [4096], [0, 1],
                                                             scale=1 / math.sqrt(d)))
        sample_bytes = cases["1x4096"][1]
        cpu = {"value": round(sample_bytes / sec / 1e9, 3), "unit": "GB/s",
               "cores": blas_threads(), "kind": "port",
               "sample": f"1 x 4096 (same bytes formula), median of 5 after 1 warm-up, "
                         f"{sec * 1e3:.1f} ms; numpy/BLAS on the host CPU ({cpu_model()})"}
    config = {"workload": ("long-context split decode, Qwen3-8B heads (32 Q / 8 KV, head_dim "
                           "128), bf16, pool 65536 blocks of 16; value: 4 sequences x 32768 "
                           "tokens, one launch (partitions merged in the launch)"),
              "cases_us": {k: round(v[0], 2) for k, v in cases.items()},
              "cases_gbs": {k: round(v[1] / v[0] / 1e3, 1) for k, v in cases.items()},
              "kv_layout": args.layout,
              "note": "1 x 4096 (16.8 MB) is launch-latency-bound"}
    return _hbm_line("long-context paged decode HBM GB/s (% peak)", achieved, us, nbytes,
                     "paged_decode_mfma_kernel (split + in-launch merge)", args,
                     "synthetic: seeded N(0,1) Q and pools, random distinct block tables",
                     config, cpu, measured_traffic(LONG_DECODE_TRAFFIC))


def main() -> int:
    parser = argparse.ArgumentParser(description=__doc__)
    parser.add_argument("--gpus", type=int, default=1)
    parser.add_argument("--steps", type=int, default=50)
    parser.add_argument("--warmup", type=int, default=5)
    parser.add_argument("--warmup-seconds", type=float, default=1.0,
                        help="keep running untimed warmup steps until this long has passed")
    parser.add_argument("--layers", type=int, default=28)
    parser.add_argument("--layout", default="paired",
                        choices=["paired", "head_major", "token_major"])
    parser.add_argument("--no-cpu-baseline", action="store_true")
    parser.add_argument("--planned-only", action="store_true",
                        help="prefill: time only the launches that share one plan per step "
                             "(no self-planning or unplanned calls of the same kernel), e.g. "
                             "for kernel profiling")
    parser.add_argument("--no-engine", action="store_true",
                        help="decode: leave out the engine half of the line (decode tok/s of "
                             "the Qwen3-0.6B engine workload), e.g. for kernel profiling")
    parser.add_argument("--workload", default="decode",
                        choices=["decode", "prefill", "step-metadata", "qk-norm-rope",
                                 "greedy", "engine", "append", "gather", "long-decode"],
                        help="decode: the headline paged-decode line; prefill: the mixed "
                             "chunked-prefill (MFMA) line; step-metadata: the decode step's "
                             "device-built metadata; qk-norm-rope: the fused Q/K RMSNorm + "
                             "RoPE + KV append; greedy: the argmax over decode logits; "
                             "engine: random-init Qwen3-0.6B served by the engine; append, "
                             "gather, long-decode: the KV append, the block-table gather and "
                             "long-context split decode")
    parser.add_argument("--no-graph", action="store_true",
                        help="decode: launch the step eagerly (for per-dispatch counter runs)")
    parser.add_argument("--graph", action="store_true",
                        help="prefill: replay the one-launch step from a hipGraph")
    parser.add_argument("--copy-calibration-mib", type=int, default=0,
                        help="after timing, run one device copy of this many MiB (the "
                             "known-size kernel that scales FETCH_SIZE / WRITE_SIZE)")
    args = parser.parse_args()
    if args.gpus != 1:
        print("bench.py measures one GPU only: there is no multi-GPU path (paged "
              "attention shards by request or by KV head with no exchange between GPUs, "
              "so each GPU runs this same single-GPU launch on its share).",
              file=sys.stderr)
        return 2

    sys.path.insert(0, os.path.dirname(os.path.abspath(__file__)))
    standalone = {"qk-norm-rope": run_qk_norm_rope, "greedy": run_greedy,
                  "engine": run_engine, "append": run_append, "gather": run_gather,
                  "long-decode": run_long_decode}
    if args.workload in standalone:
        rc = standalone[args.workload](args)
        if args.copy_calibration_mib:
            import torch

            copy_calibration(torch, args.copy_calibration_mib)
        return rc
    if args.workload == "prefill":
        return run_prefill(args)
    if args.workload == "step-metadata":
        return run_step_metadata(args)

    result = measure_decode(args)
    if args.no_engine:
        print(json.dumps(result), flush=True)
        return 0
    import torch

    torch.cuda.synchronize()
    torch.cuda.empty_cache()  # the 28 decode caches (30 GB) are gone
    # The other workloads' figures, measured before the engine run so that
    # they, like their standalone runs, follow only the decode timing.
    extras = other_workloads(torch, args)
    torch.cuda.synchronize()
    torch.cuda.empty_cache()
    # The other half of the headline metric: decode tok/s of the engine
    # workload, with its host counterpart beside it.
    e = measure_engine(ENGINE_BATCHES, 1)
    cfg = result["config"]
    cfg["decode_tok_s"] = round(e["decode_tps"], 1)
    cfg["engine_output_tok_s"] = round(e["output_tps"], 1)
    cfg["engine_decode_step_us"] = round(e["decode_step_us"], 1)
    cfg["engine_workload"] = (ENGINE_WORKLOAD_TEXT + f"; {ENGINE_BATCHES} batches timed after "
                              "1 untimed, fresh prompts each")
    if not args.no_cpu_baseline:
        cpu = engine_cpu_baseline(e["model"])
        cfg["cpu_decode_tok_s"] = cpu["value"]
        result["cpu_baseline_engine"] = cpu
    del e
    result.update(extras)
    print(json.dumps(result), flush=True)
    return 0


ENGINE_BATCHES = 3
DEFAULT_LONG_CASES = ((4, 32768), (1, 32768), (1, 16384))


def other_workloads(torch, args) -> dict:
    """The other workloads' figures, as extra keys of the default line: the
    mixed chunked prefill (MFMA roofline), long-context split decode and the
    small fp32 decode with its CPU oracle beside it."""
    from microinfer_amd.workloads import QWEN3_06B, decode_bytes, make_decode_batch

    out = {}
    st = prefill_state(torch, args.layout)
    st["step"]()
    torch.cuda.synchronize()
    ms = time_launches(torch, st["layers_step"], args, 4) / PREFILL_LAYERS
    single_ms = time_launches(torch, st["step"], args, 20)
    tflops = st["flops"] / (ms * 1e-3) / 1e12
    log(f"mixed prefill: {ms * 1e3:.1f} us per launch, {tflops:.1f} TFLOP/s "
        f"(single call without a shared plan {single_ms * 1e3:.1f} us)")
    out["prefill"] = {
        "workload": ("mixed chunked prefill, Qwen3-8B attention (32 Q / 8 KV heads), bf16, "
                     "block 16, pool 65536: 8 chunks of 512 rows on prefixes U[0,3072] "
                     "(first 1024 tokens shared) + 24 decode rows, contexts U[256,2048], "
                     f"seed 0; one launch plan per {PREFILL_LAYERS} varlen launches (eager, "
                     "back to back, 4 steps timed), per launch"),
        "tflops": round(tflops, 2), "us_per_launch": round(ms * 1e3, 3),
        "single_call_us": round(single_ms * 1e3, 3),
        "flops_per_launch": st["flops"], "peak_tflops": MFMA_BF16_PEAK_TFLOPS,
        "frac": round(tflops / MFMA_BF16_PEAK_TFLOPS, 4),
        "kernel": "paged_prefill_mfma_kernel"}
    del st
    torch.cuda.empty_cache()

    cache, kc, vc, perm, gen, cases = time_long_decode(torch, args, DEFAULT_LONG_CASES)
    out["long_decode"] = {
        "workload": ("split decode, Qwen3-8B heads (32 Q / 8 KV), bf16, pool 65536, hipGraph "
                     "replay of launches over distinct blocks (plan included)"),
        "cases": {k: {"us_per_launch": round(us, 2), "gbs": round(b / us / 1e3, 1),
                      "frac": round(b / us / 1e3 / HBM_PEAK_GBS, 4)}
                  for k, (us, b) in cases.items()}}
    del cache, kc, vc, perm
    torch.cuda.empty_cache()

    # The reference's CPU-runnable case: fp32, 0.6B shape, pool 1024, 8
    # sequences with contexts U[64, 512], one append + decode layer call.
    out["small_fp32_decode"] = small_fp32_decode(torch, args, make_decode_batch, QWEN3_06B,
                                                 decode_bytes)
    return out


def small_fp32_decode(torch, args, make_decode_batch, shape, decode_bytes) -> dict:
    from microinfer_amd.layer.hip_paged_attention import hip_paged_decode
    from microinfer_amd.worker.kv_cache import KVCache

    batch = make_decode_batch(num_seqs=8, ctx_lo=64, ctx_hi=512, pool_blocks=1024, **shape)
    dev = torch.device("cuda", 0)
    cache = KVCache(1, 1024, 16, 8, 128, dtype=torch.float32, device=dev, layout=args.layout)
    cache.keys[0].copy_(torch.from_numpy(batch.key_pool))
    cache.values[0].copy_(torch.from_numpy(batch.value_pool))
    q = torch.from_numpy(batch.query).to(dev)
    nk = torch.from_numpy(batch.new_keys).to(dev)
    nv = torch.from_numpy(batch.new_values).to(dev)
    tables = torch.tensor(batch.block_tables, device=dev)
    lens = torch.tensor(batch.context_lens, device=dev)
    scale = 1 / math.sqrt(128)

    def call():
        return hip_paged_decode(q, cache.keys[0], cache.values[0], tables, lens, scale=scale,
                                new_keys=nk, new_values=nv)

    ms = time_launches(torch, call, args, 50)
    contexts = [int(c) for c in batch.context_lens]
    nbytes = decode_bytes(contexts, num_q_heads=16, num_kv_heads=8, head_dim=128, elem_bytes=4,
                          block_size=16)
    line = {"workload": ("KV append + paged decode, fp32, Qwen3-0.6B attention (16 Q / 8 KV), "
                         "block 16, pool 1024, 8 sequences, contexts U[64,512] (seed 0), one "
                         "layer call (eager, 50 timed)"),
            "bytes_per_call": nbytes, "us_per_call": round(ms * 1e3, 3),
            "gbs": round(nbytes / (ms * 1e-3) / 1e9, 2)}
    if not args.no_cpu_baseline:
        from oracle import kv_append, paged_attention_reference

        hk, hv = batch.key_pool.copy(), batch.value_pool.copy()
        slots = np.asarray(batch.slots)

        def one_call():
            kv_append(hk, hv, slots, batch.new_keys, batch.new_values)
            return paged_attention_reference(batch.query, hk, hv, batch.block_tables,
                                             contexts, list(range(9)), scale=scale)

        sec = _median_time(one_call)
        line["cpu_baseline"] = {
            "value": round(nbytes / sec / 1e9, 3), "unit": "GB/s", "cores": blas_threads(),
            "kind": "port",
            "sample": (f"the same layer call (append + decode over {sum(contexts)} tokens) x 5 "
                       f"after 1 warm-up, median {sec * 1e3:.2f} ms; numpy/BLAS on the host "
                       f"({cpu_model()})")}
    log(f"small fp32 decode: {ms * 1e3:.1f} us per call")
    return line


def measure_decode(args) -> dict:
    """The headline paged-decode line (without the engine half)."""
    import torch

    from microinfer_amd.layer.hip_paged_attention import decode_plan, hip_paged_decode
    from microinfer_amd.workloads import decode_bytes

    log("allocating 28-layer caches")
    state = build_decode_state(torch, args.layers, args.layout)
    views, query, tables, lens = (state[k] for k in ("views", "query", "tables", "lens"))
    new_k, new_v = state["new_k"], state["new_v"]
    scale = 1 / math.sqrt(128)
    outputs = []

    def step():
        # One partition plan per step, shared by the 28 layers (as the
        # engine's AttentionMetadata does); each layer call appends its new
        # rows and attends in one launch.
        plan = decode_plan(lens, num_kv_heads=8, block_size=16,
                           block_table_width=tables.shape[1])
        outputs.clear()
        for layer, view in enumerate(views):
            outputs.append(hip_paged_decode(query[layer], view.keys, view.values, tables, lens,
                                            scale=scale, plan=plan, new_keys=new_k[layer],
                                            new_values=new_v[layer]))

    step()
    torch.cuda.synchronize()
    if args.no_graph:
        run = step
    else:
        log("capturing the decode step in a hipGraph")
        # One eager step on the capture stream first: the library keeps a
        # zeroed arrival-counter array per stream, and allocating it here
        # keeps its zero fill out of the graph.
        capture_stream = torch.cuda.Stream()
        capture_stream.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(capture_stream):
            step()
        torch.cuda.synchronize()
        graph = torch.cuda.CUDAGraph()
        with capture_graph(graph, stream=capture_stream):
            step()
        torch.cuda.synchronize()
        run = graph.replay

    warm_up(torch, run, args)
    # Events on torch's current stream, which is the stream every launch of
    # the step goes to (the library reads it at call time).
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    log(f"timing {args.steps} steps")
    t0 = time.perf_counter()
    start.record()
    for _ in range(args.steps):
        run()
    end.record()
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    ms_per_step = start.elapsed_time(end) / args.steps
    if args.copy_calibration_mib:
        copy_calibration(torch, args.copy_calibration_mib)

    contexts = state["batch"].context_lens
    layer_bytes = decode_bytes(contexts, num_q_heads=16, num_kv_heads=8, head_dim=128,
                               elem_bytes=2, block_size=16)
    step_bytes = layer_bytes * args.layers
    gbs = step_bytes / (ms_per_step * 1e-3) / 1e9
    layer_us = ms_per_step * 1e3 / args.layers
    log(f"{ms_per_step:.3f} ms/step, {layer_us:.2f} us/layer call, {gbs:.1f} GB/s "
        f"(wall {wall:.2f} s)")

    result = {
        "metric": "paged-decode HBM GB/s (% peak) + decode tok/s, random-init Qwen3-0.6B b64",
        "value": round(gbs, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "warmup_seconds": args.warmup_seconds,
        "ms_per_step": round(ms_per_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic: seeded N(0,1) Q/K/V, random non-overlapping block tables",
        "config": {
            "workload": ("paged decode + KV append, Qwen3-0.6B attention (16 Q / 8 KV heads, "
                         "head_dim 128), bf16, block 16, pool 16384 blocks per layer, "
                         "32 sequences, contexts U[128,2048] (seed 0), 28 independent layer "
                         "caches, " + ("launched eagerly" if args.no_graph else "hipGraph replay")),
            "layers": args.layers,
            "sum_context_tokens": int(np.sum(contexts)),
            "kv_layout": args.layout,
            "pct_hbm_peak": round(100 * gbs / HBM_PEAK_GBS, 2),
            "decode_tok_s": None,
        },
        "roofline": {
            "bound": "hbm",
            "achieved": round(gbs, 2),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(gbs / HBM_PEAK_GBS, 4),
            "traffic": measured_traffic(DECODE_TRAFFIC),
            "traffic_source": ("profiles/paged_decode_traffic_qwen3-0.6b_b32.json: rocprofv3 "
                               "FETCH_SIZE + WRITE_SIZE counter runs of this workload, "
                               "copy-calibrated; read from the file, not measured in this run"),
            "kernel": "paged_decode_mfma_kernel (fused append + decode + split merge)",
            "bytes_per_launch": layer_bytes,
            "us_per_launch": round(layer_us, 3),
            "timing": "HIP events around the timed steps / (steps x layers); includes the "
                      "per-step plan kernel and inter-launch gaps",
        },
    }
    if not args.no_cpu_baseline:
        log("timing the CPU oracle on layer 0")
        result["cpu_baseline"] = cpu_baseline(torch, state)
    return result


if __name__ == "__main__":
    sys.exit(main())
