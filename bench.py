"""Benchmark of liteinfer's `paged` attention path on one MI355X.

A step is one layer's share of a decode step at BASELINE config 2
(Llama-3-8B geometry: 32/8 heads, head_dim 128, bf16, block 16, batch 64,
contexts uniform in [512, 8192], pool of 65,536 blocks with seeded shuffled
block tables): the slot-write of each sequence's new K/V at its newest
position, then paged decode over it, as one call (`paged_decode` with
`new_key` / `new_value`: one launch of the head-grouped decode kernel, which
stores the new rows and folds them, then the combine of split contexts),
captured in a HIP graph and replayed K times between two synchronisations.
The reference's order (slot-write launch, then decode) is timed beside it,
eagerly. Inputs are synthetic N(0, 1) and resident in HBM before the clock
starts.

`value` is algorithmic bytes per step / step time, in GB/s: every context
token's K and V rows for all KV heads plus its int64 slot index, the queries
and outputs, and the slot-write's reads and writes. `roofline` rates the
launch (timed with HIP events on the stream it runs on) against MI355X's
8 TB/s. Config 3's packed
prefill (TFLOP/s of visible causal pairs; also its 8 chunks alone, its 56
one-query rows alone in GB/s, and 8 chunks of 2048 queries over 8192 cached
keys) and config 4's long-context decode are reported beside it, each also
over an fp8 (e4m3) KV pool, and so is the fused RoPE + slot-write at config 3's
packed pass and config 2's decode step, with the reference's separate torch
ops timed on the same inputs, and config 5: `LLM.generate` of 256 requests x
256 greedy tokens over a random-initialised Llama-3-8B-architecture model
(output tokens per second, liteinfer_amd/engine/e2e.py). `reference_a40_shapes`
times this build's calls on the shapes of the reference's own published
benchmark tables (Llama-3.2-1B geometry), beside its A40 figures.
`cpu_baseline` times the dense eager attention (oracle/baseline.py) in fp32 on
this host's cores over a bounded sample of the same step.

    python bench.py [--steps K] [--warmup W] [--gpus 1]
"""

from __future__ import annotations

import argparse
import json
import os
import statistics
import sys
import time
from pathlib import Path

import numpy as np
import torch

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

from liteinfer_amd import _native  # noqa: E402
from liteinfer_amd.attention import PagedKV, paged_attention  # noqa: E402
from liteinfer_amd.cache.kv_cache import scatter_into  # noqa: E402
from liteinfer_amd.paged_kernels import kv_scatter, paged_decode  # noqa: E402
from liteinfer_amd.engine.runner import graph_capture  # noqa: E402
from liteinfer_amd.workloads import LLAMA_3_2_1B, c3_shapes, decode_step, packed_step  # noqa: E402

METRIC = "paged-decode HBM GB/s (% of peak); prefill attn TFLOP/s; e2e output tok/s"
HBM_PEAK_GBS = 8000.0
BF16_PEAK_TFLOPS = 2500.0
TRAFFIC_FILE = ROOT / "profiles" / "decode_c2_traffic.json"
# Untimed calls before each secondary workload's timed ones: enough for the
# clocks to settle after the previous workload (a few ms of work).
SECONDARY_WARMUP = 20
PREFILL_WARMUP_S = 0.15


def decode_bytes(ctxs, geo, elem=2, kv_elem=None) -> int:
    """K and V rows of every context token for all KV heads, its int64 slot, q in and out.

    kv_elem: bytes per pool element when the pool's type differs from q's (1 for an fp8 pool).
    """
    tokens = sum(ctxs)
    kv = elem if kv_elem is None else kv_elem
    return tokens * (2 * geo.num_kv_heads * geo.head_dim * kv + 8) + 2 * len(ctxs) * geo.num_heads * geo.head_dim * elem


def to_fp8_pool(step):
    """The step with its pools quantised to fp8 (e4m3, scales 1) by the slot-write kernel."""
    kp = torch.empty(step.key_pool.shape, dtype=torch.float8_e4m3fn, device=step.key_pool.device)
    vp = torch.empty_like(kp)
    every = torch.arange(kp.shape[0], device=kp.device).view(1, -1)
    kv_scatter(kp, vp, every, step.key_pool.unsqueeze(0).transpose(1, 2), step.value_pool.unsqueeze(0).transpose(1, 2))
    step.key_pool, step.value_pool = kp, vp
    return step


def scatter_bytes(tokens, geo, elem=2) -> int:
    """Read the new K and V rows, write them into the pool, read the int64 slots."""
    return tokens * (4 * geo.num_kv_heads * geo.head_dim * elem + 8)


def prefill_flops(qlens, ctxs, geo) -> int:
    """4 * heads * head_dim flops per visible (query, key) pair (QK^T and PV)."""
    pairs = sum(q * (c - q) + q * (q + 1) // 2 for q, c in zip(qlens, ctxs))
    return 4 * geo.num_heads * geo.head_dim * pairs


def _time_decode(step, steps, warmup):
    geo = step.geometry
    kv = PagedKV(step.key_pool, step.value_pool, step.slot_table, step.context_lens)
    q = step.query.unsqueeze(2)

    def one():
        scatter_into(step.key_pool, step.value_pool, step.write_slots, step.new_k, step.new_v)
        return paged_attention(q, kv, geo.scaling, geo.groups)

    for _ in range(warmup):
        one()
    stream = torch.cuda.current_stream()
    marks = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(steps)]
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for a, b in marks:
        scatter_into(step.key_pool, step.value_pool, step.write_slots, step.new_k, step.new_v)
        a.record(stream)
        paged_attention(q, kv, geo.scaling, geo.groups)
        b.record(stream)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    decode_ms = [a.elapsed_time(b) for a, b in marks]
    return wall, decode_ms


def _fused_step_call(step):
    """Config 2's layer step as one call: the newest K/V rows written and the
    decode over them (paged_decode with new_key / new_value)."""
    geo = step.geometry
    new_k, new_v = step.new_k.squeeze(2), step.new_v.squeeze(2)
    return lambda: paged_decode(step.query, step.key_pool, step.value_pool, step.slot_table, step.context_lens,
                                geo.scaling, geo.groups, new_key=new_k, new_value=new_v)


def _time_step(step, steps, warmup):
    """Config 2's step, timed two ways.

    Wall clock: one step captured in a HIP graph (its launches, as the
    engine replays a layer's decode), then `steps` replays back to back
    between two synchronisations; the reference's own layer timings replay a
    graph the same way. Events: each of `steps` eager calls bracketed by HIP
    events on the stream it runs on. Returns (wall seconds, event ms list).
    """
    one = _fused_step_call(step)
    for _ in range(warmup):
        one()
    stream = torch.cuda.current_stream()
    marks = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(steps)]
    torch.cuda.synchronize()
    for a, b in marks:
        a.record(stream)
        one()
        b.record(stream)
    torch.cuda.synchronize()
    event_ms = [a.elapsed_time(b) for a, b in marks]

    side = torch.cuda.Stream()
    side.wait_stream(stream)
    with torch.cuda.stream(side):
        one()
    stream.wait_stream(side)
    graph = torch.cuda.CUDAGraph()
    with graph_capture(graph):
        one()
    for _ in range(warmup):
        graph.replay()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        graph.replay()
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    del graph
    return wall, event_ms


def _time_prefill(step, steps, warmup):
    geo = step.geometry
    kv = PagedKV(step.key_pool, step.value_pool, step.slot_table, step.context_lens,
                 query_start_loc=step.query_start_loc, max_query_len=step.max_query_len,
                 host_context_lens=tuple(step.host_context_lens), host_query_lens=tuple(step.host_query_lens))
    q = step.query.transpose(0, 1).unsqueeze(0)
    scatter_into(step.key_pool, step.value_pool, step.write_slots, step.new_k, step.new_v)
    # Warm up for `warmup` calls and at least PREFILL_WARMUP_S of them: after
    # the memory-bound decode phases the matrix-bound prefill runs up to ~15%
    # slower for its first ~90 ms while the clock settles (a kernel trace of
    # config 3's calls, averaged by hundreds: 330, 303, 307, 291, 289, 289,
    # 288 us), so the figure is the sustained rate a busy server sees.
    done, t0 = 0, time.perf_counter()
    while done < warmup or time.perf_counter() - t0 < PREFILL_WARMUP_S:
        for _ in range(10):
            paged_attention(q, kv, geo.scaling, geo.groups)
        done += 10
        torch.cuda.synchronize()
    stream = torch.cuda.current_stream()
    marks = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(steps)]
    torch.cuda.synchronize()
    for a, b in marks:
        a.record(stream)
        paged_attention(q, kv, geo.scaling, geo.groups)
        b.record(stream)
    torch.cuda.synchronize()
    return [a.elapsed_time(b) for a, b in marks]


def graph_replay_us(fn, replays: int = 100, repeats: int = 5, calls: int = 1) -> float:
    """Per-call microseconds of `fn` captured `calls` times into one HIP graph.

    `replays` back-to-back replays are bracketed by HIP events; the best of
    `repeats` such runs is kept (the reference's own method for its layer
    timings). A replay costs the host ~16 us to launch on this stack, so a
    call shorter than that needs `calls` > 1 (as a model step's graph holds
    every layer's call) for its own time to show.
    """
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for _ in range(3):
            fn()
    torch.cuda.current_stream().wait_stream(side)
    graph = torch.cuda.CUDAGraph()
    with graph_capture(graph):
        for _ in range(calls):
            fn()
    graph.replay()
    torch.cuda.synchronize()
    best = float("inf")
    for _ in range(repeats):
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a.record()
        for _ in range(replays):
            graph.replay()
        b.record()
        torch.cuda.synchronize()
        best = min(best, a.elapsed_time(b) * 1e3 / (replays * calls))
    del graph
    return best


def _decode_call(step):
    kv = PagedKV(step.key_pool, step.value_pool, step.slot_table, step.context_lens)
    q = step.query.unsqueeze(2)
    geo = step.geometry
    return lambda: paged_attention(q, kv, geo.scaling, geo.groups)


def _prefill_call(step):
    geo = step.geometry
    kv = PagedKV(step.key_pool, step.value_pool, step.slot_table, step.context_lens,
                 query_start_loc=step.query_start_loc, max_query_len=step.max_query_len,
                 host_context_lens=tuple(step.host_context_lens), host_query_lens=tuple(step.host_query_lens))
    q = step.query.transpose(0, 1).unsqueeze(0)
    return lambda: paged_attention(q, kv, geo.scaling, geo.groups)


def _graph_hbm(entry: dict, fn, nbytes: int) -> dict:
    us = graph_replay_us(fn)
    entry["graph_replay_us"] = round(us, 2)
    entry["graph_replay_frac_hbm"] = round(nbytes / (us * 1e-6) / 1e9 / HBM_PEAK_GBS, 4)
    return entry


def _graph_mfma(entry: dict, fn, flops: int) -> dict:
    us = graph_replay_us(fn)
    entry["graph_replay_us"] = round(us, 2)
    entry["graph_replay_frac_bf16_peak"] = round(flops / (us * 1e-6) / 1e12 / BF16_PEAK_TFLOPS, 4)
    return entry


def _time_rope(batch, tokens, geo, iters=50, num_slots=1 << 20, seed=0):
    """Fused RoPE + slot-write vs the reference's separate torch ops (rotary, permute, index_put_)."""
    from liteinfer_amd.rope import apply_rotary_pos_emb, rope_kv_write
    from liteinfer_amd.cache.kv_cache import tokens_first

    g = torch.Generator(device="cuda").manual_seed(seed)
    hq, hkv, d = geo.num_heads, geo.num_kv_heads, geo.head_dim
    proj = lambda h: torch.randn(batch, tokens, h, d, generator=g, device="cuda").to(torch.bfloat16).transpose(1, 2)
    q, k, v = proj(hq), proj(hkv), proj(hkv)
    pos = torch.randint(0, 8192, (batch, tokens), generator=g, device="cuda").float()
    inv = 1.0 / (500000.0 ** (torch.arange(0, d, 2, device="cuda").float() / d))
    emb = torch.cat((pos[..., None] * inv, pos[..., None] * inv), dim=-1)
    cos, sin = emb.cos().to(torch.bfloat16), emb.sin().to(torch.bfloat16)
    kp = torch.zeros(num_slots, hkv, d, dtype=torch.bfloat16, device="cuda")
    vp = torch.zeros_like(kp)
    slots = torch.randperm(num_slots, generator=torch.Generator().manual_seed(seed))[: batch * tokens].view(1, -1).cuda()

    def unfused():
        q_embed, k_embed = apply_rotary_pos_emb(q, k, cos, sin)
        flat = slots.reshape(-1)
        kp[flat] = tokens_first(k_embed)
        vp[flat] = tokens_first(v)
        return q_embed

    def timed(fn):
        for _ in range(5):
            fn()
        stream = torch.cuda.current_stream()
        marks = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(iters)]
        torch.cuda.synchronize()
        for a, b in marks:
            a.record(stream)
            fn()
            b.record(stream)
        torch.cuda.synchronize()
        return statistics.mean(a.elapsed_time(b) for a, b in marks) * 1e3

    def graph_timed(fn, calls=20):
        """Per-call GPU time of `calls` back-to-back calls captured in one graph (no host launch cost)."""
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):
            for _ in range(3):
                fn()
        torch.cuda.current_stream().wait_stream(side)
        graph = torch.cuda.CUDAGraph()
        with graph_capture(graph):
            for _ in range(calls):
                fn()
        graph.replay()
        torch.cuda.synchronize()
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        reps = max(1, iters // 10)
        a.record()
        for _ in range(reps):
            graph.replay()
        b.record()
        torch.cuda.synchronize()
        return a.elapsed_time(b) * 1e3 / (reps * calls)

    fused_us = timed(lambda: rope_kv_write(q, k, v, cos, sin, slots, kp, vp))
    fused_graph_us = graph_timed(lambda: rope_kv_write(q, k, v, cos, sin, slots, kp, vp))
    unfused_us = timed(unfused)
    n = batch * tokens
    nbytes = n * (2 * 2 * hq * d + 2 * 2 * 2 * hkv * d + 2 * 2 * d + 8)
    return {
        "tokens": n,
        "avg_us": round(fused_us, 2),
        "GB/s": round(nbytes / (fused_us * 1e-6) / 1e9, 1),
        "frac_hbm": round(nbytes / (fused_us * 1e-6) / 1e9 / HBM_PEAK_GBS, 4),
        "algorithmic_bytes": nbytes,
        "graph_replay_us": round(fused_graph_us, 2),
        "graph_replay_frac_hbm": round(nbytes / (fused_graph_us * 1e-6) / 1e9 / HBM_PEAK_GBS, 4),
        "unfused_torch_ops_us": round(unfused_us, 2),
    }


def _cpu_model() -> str:
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def _median_of(fn, calls: int = 5) -> float:
    """Median wall seconds of `calls` calls after one untimed warm-up."""
    fn()
    times = []
    for _ in range(calls):
        t0 = time.perf_counter()
        fn()
        times.append(time.perf_counter() - t0)
    return statistics.median(times)


def _host_rows(step, rows: int, width: int):
    """The fp32 host copy of the pool rows the first `rows` sequences read, and their local table."""
    table = step.slot_table[:rows, :width]
    uniq, inverse = torch.unique(table, return_inverse=True)
    return step.key_pool[uniq].float().cpu(), step.value_pool[uniq].float().cpu(), inverse.cpu()


def _cpu_decode(step, budget_s: float) -> dict:
    """eager and sdpa medians over as many of the step's sequences as fit the time budget."""
    from oracle import baseline

    geo = step.geometry
    n = step.batch
    while True:
        ctxs = step.host_context_lens[:n]
        kp, vp, local = _host_rows(step, n, max(ctxs))
        q = step.query[:n].float().cpu()
        ctx_t = torch.tensor(ctxs)
        run = lambda kind: baseline.decode(kind, q, kp, vp, local, ctx_t, geo.scaling, geo.groups)
        t0 = time.perf_counter()
        run("eager")
        first = time.perf_counter() - t0
        # 6 eager + 6 sdpa calls follow; halve the sample until they fit.
        if n == 1 or 12 * first <= budget_s:
            break
        n = max(1, n // 2)
        del kp, vp, local, q
    eager = _median_of(lambda: run("eager"))
    sdpa = _median_of(lambda: run("sdpa"))
    nbytes = decode_bytes(ctxs, geo)
    return {
        "sequences": f"{n} of {step.batch}",
        "context_tokens": sum(ctxs),
        "eager_ms": round(eager * 1e3, 2),
        "sdpa_ms": round(sdpa * 1e3, 2),
        "eager_GB/s": round(nbytes / eager / 1e9, 3),
        "sdpa_GB/s": round(nbytes / sdpa / 1e9, 3),
    }


def _cpu_packed(step, budget_s: float) -> dict:
    """eager and sdpa medians over config 3's whole packed pass (sequence by sequence, as the reference)."""
    from oracle import baseline

    geo = step.geometry
    kp, vp, local = _host_rows(step, len(step.host_query_lens), step.slot_table.shape[1])
    q = step.query.float().cpu()
    ctx_t = step.context_lens.cpu()
    qlens = list(step.host_query_lens)
    run = lambda kind: baseline.packed(kind, q, kp, vp, local, ctx_t, qlens, geo.scaling, geo.groups)
    eager = _median_of(lambda: run("eager"))
    sdpa = _median_of(lambda: run("sdpa"))
    flops = prefill_flops(step.host_query_lens, step.host_context_lens, geo)
    return {
        "sequences": f"all {len(qlens)} (8 chunks + 56 one-query rows)",
        "query_tokens": sum(qlens),
        "eager_ms": round(eager * 1e3, 2),
        "sdpa_ms": round(sdpa * 1e3, 2),
        "eager_TFLOP/s": round(flops / eager / 1e12, 4),
        "sdpa_TFLOP/s": round(flops / sdpa / 1e12, 4),
    }


def cpu_baseline(seed: int = 0, device: str = "cuda", budget_s: float = 20.0, gpu_ms: dict | None = None) -> dict:
    """The reference's dense eager and sdpa attention (fp32 torch, every host core) per config.

    Config 2 and 4 decode steps (all sequences, or the largest halving of the
    batch whose 12 calls fit `budget_s`) and config 3's packed pass; each the
    median of 5 calls after a warm-up. `value` is config 2's eager rate.
    """
    cores = len(os.sched_getaffinity(0))
    torch.set_num_threads(cores)
    configs = {}
    step = decode_step("c2", seed=seed, device=device)
    configs["c2"] = _cpu_decode(step, budget_s)
    del step
    step = packed_step("c3", seed=seed, device=device)
    configs["c3"] = _cpu_packed(step, budget_s)
    del step
    step = decode_step("c4", seed=seed, device=device)
    configs["c4"] = _cpu_decode(step, budget_s)
    del step
    for name, ms in (gpu_ms or {}).items():
        if name in configs:
            configs[name]["gpu_paged_ms_full_config"] = ms
    c2 = configs["c2"]
    return {
        "value": c2["eager_GB/s"],
        "unit": "GB/s",
        "cores": cores,
        "kind": "port",
        "cpu_model": _cpu_model(),
        "sample": (f"dense eager attention (oracle/baseline.py, fp32 torch on {cores} threads) over config 2's "
                   f"decode step, {c2['sequences']} sequences ({c2['context_tokens']} context tokens): median of "
                   f"5 calls = {c2['eager_ms']} ms; sdpa {c2['sdpa_ms']} ms; configs 3 and 4 in `configs`"),
        "configs": configs,
    }


# The reference's own per-call timings (NVIDIA A40, Llama-3.2-1B attention
# geometry: 32 query / 8 KV heads, head_dim 64, bf16, block 16; captured
# CUDA graph, best of 5), docs/benchmarks.md of the reference: decode per
# attention call (:418-423), decode per layer at batch 1 (:1222-1228; the
# better of its unsplit and 21-split figures), chunks over a cached prefix
# and mixed passes (:1373-1391), whole prompts (:1418-1426). Each row:
# (name, kind, spec, A40 microseconds).
REFERENCE_A40_SHAPES = [
    ("decode B=1 ctx 190", "decode", [190], 47.0),
    ("decode B=32 ctx 190", "decode", [190] * 32, 38.0),
    ("decode B=32 ctx 1024", "decode", [1024] * 32, 131.0),
    ("decode B=32 ctx 2048", "decode", [2048] * 32, 253.0),
    ("decode B=1 ctx 128", "decode", [128], 4.2),
    ("decode B=1 ctx 1024", "decode", [1024], 5.8),
    ("decode B=1 ctx 4096", "decode", [4096], 21.0),
    ("decode B=1 ctx 16384", "decode", [16384], 64.6),
    ("chunk 64 over 0", "packed", ([(64, 0)], []), 10.2),
    ("chunk 64 over 4096", "packed", ([(64, 4096)], []), 144.8),
    ("chunk 64 over 15000", "packed", ([(64, 15000)], []), 492.0),
    ("chunk 512 over 0", "packed", ([(512, 0)], []), 32.6),
    ("chunk 512 over 4096", "packed", ([(512, 4096)], []), 272.6),
    ("chunk 512 over 15000", "packed", ([(512, 15000)], []), 945.3),
    ("chunk 2048 over 0", "packed", ([(2048, 0)], []), 227.2),
    ("chunk 2048 over 2048", "packed", ([(2048, 2048)], []), 629.2),
    ("chunk 2048 over 8192", "packed", ([(2048, 8192)], []), 1939.1),
    ("chunk 512 over 4096 beside 7 prompts of 64", "packed", ([(512, 4096)] + [(64, 0)] * 7, []), 274.9),
    ("31 one-token rows over 2000 beside a 256 chunk", "packed", ([(256, 0)], [2000] * 31), 264.6),
    ("prompts 1 x 4096", "packed", ([(4096, 0)], []), 802.8),
    ("prompts 32 x 18", "packed", ([(18, 0)] * 32, []), 19.8),
    ("prompts 32 x 128", "packed", ([(128, 0)] * 32, []), 130.4),
    ("prompts 8 x 512", "packed", ([(512, 0)] * 8, []), 160.1),
]


def _reference_shapes(seed: int) -> list:
    """This build's call time on the reference's own benchmark shapes, beside the reference's A40 figure.

    Same geometry and method as the reference's tables (Llama-3.2-1B attention
    geometry; calls captured in a graph, best of 5 runs: 20 calls per graph,
    20 replays, so that the ~16 us a graph launch costs the host here is not
    what a short call measures);
    the fraction is of this GPU's roofline (8 TB/s for decode, 2.5 PF/s bf16
    for packed passes). Other hardware: a ratio of platforms, not of kernels.
    """
    out = []
    for name, kind, spec, a40_us in REFERENCE_A40_SHAPES:
        if kind == "decode":
            step = decode_step("custom", seed=seed, context_lens=spec, geometry=LLAMA_3_2_1B)
            us = graph_replay_us(_decode_call(step), replays=20, calls=20)
            work = decode_bytes(step.host_context_lens, step.geometry)
            frac = {"frac_hbm": round(work / (us * 1e-6) / 1e9 / HBM_PEAK_GBS, 4)}
        else:
            chunks, rows = spec
            step = packed_step("custom", seed=seed, chunks=chunks, decode_contexts=rows, geometry=LLAMA_3_2_1B,
                               num_blocks=8192)
            us = graph_replay_us(_prefill_call(step), replays=20, calls=20)
            flops = prefill_flops(step.host_query_lens, step.host_context_lens, step.geometry)
            frac = {"frac_bf16_peak": round(flops / (us * 1e-6) / 1e12 / BF16_PEAK_TFLOPS, 4)}
        out.append({"shape": name, "us": round(us, 2), "reference_a40_us": a40_us,
                    "a40_over_this": round(a40_us / us, 2), **frac})
        del step
    torch.cuda.empty_cache()
    return out


def _traffic():
    if TRAFFIC_FILE.exists():
        try:
            return json.loads(TRAFFIC_FILE.read_text()).get("hbm_bytes_per_launch")
        except (OSError, ValueError):
            return None
    return None


def _only_prefill(workload: str, seed: int, steps: int, warmup: int) -> int:
    """One packed prefill workload alone: config 3 (bf16 or fp8 pool), its 8 chunks, or 8 chunks of 2048 over 8192."""
    if workload == "c3":
        step = packed_step("c3", seed=seed)
    elif workload == "c3_fp8":
        step = to_fp8_pool(packed_step("c3", seed=seed))
    elif workload == "c3_chunks":
        chunks, _ = c3_shapes(seed)
        step = packed_step("custom", seed=seed, chunks=chunks, decode_contexts=[])
    else:
        step = packed_step("custom", seed=seed, chunks=[(2048, 8192)] * 8, decode_contexts=[])
    avg = statistics.mean(_time_prefill(step, steps, warmup))
    flops = prefill_flops(step.host_query_lens, step.host_context_lens, step.geometry)
    print(json.dumps({"workload": workload, "avg_us": round(avg * 1e3, 2),
                      "TFLOP/s": round(flops / (avg * 1e-3) / 1e12, 2),
                      "frac_bf16_peak": round(flops / (avg * 1e-3) / 1e12 / BF16_PEAK_TFLOPS, 4)}), flush=True)
    return 0


def _copy_calibration() -> None:
    """Three 1 GiB device-to-device copies: a kernel of known traffic for rocprofv3's counters."""
    src = torch.empty(1 << 30, dtype=torch.uint8, device="cuda").fill_(1)
    dst = torch.empty_like(src)
    for _ in range(3):
        dst.copy_(src)
    torch.cuda.synchronize()
    del src, dst


def _only_step(seed: int, steps: int, warmup: int) -> int:
    """Config 2's fused step alone (eager calls, then graph replays), for profiling."""
    step = decode_step("c2", seed=seed)
    geo = step.geometry
    wall, step_ms = _time_step(step, steps, warmup)
    d_bytes = decode_bytes(step.host_context_lens, geo)
    w_bytes = 4 * step.batch * geo.num_kv_heads * geo.head_dim * 2
    avg = statistics.mean(step_ms)
    print(json.dumps({"workload": "c2_step", "avg_launch_us": round(avg * 1e3, 2),
                      "ms_per_step_graph": round(wall / steps * 1e3, 5),
                      "algorithmic_bytes_per_launch": d_bytes + w_bytes,
                      "frac_hbm": round((d_bytes + w_bytes) / (avg * 1e-3) / 1e9 / HBM_PEAK_GBS, 4)}), flush=True)
    return 0


def main() -> int:
    parser = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    parser.add_argument("--gpus", type=int, default=1)
    parser.add_argument("--steps", type=int, default=200)
    parser.add_argument("--warmup", type=int, default=20)
    parser.add_argument("--seed", type=int, default=0)
    parser.add_argument("--no-cpu-baseline", action="store_true")
    parser.add_argument("--no-secondary", action="store_true", help="skip configs 3 and 4")
    parser.add_argument("--no-e2e", action="store_true", help="skip config 5 (end-to-end generate)")
    parser.add_argument("--copy-calibration", action="store_true",
                        help="first run three 1 GiB device-to-device copies (a reference kernel of known "
                             "size for rocprofv3 FETCH_SIZE / WRITE_SIZE calibration)")
    parser.add_argument("--only-prefill", choices=["c3", "c3_fp8", "c3_chunks", "long"],
                        help="time only this packed prefill pass (for profiling) and print its line")
    parser.add_argument("--only-step", action="store_true",
                        help="time only config 2's fused decode step (for profiling) and print its line")
    parser.add_argument("--no-reference-shapes", action="store_true",
                        help="skip the reference's own benchmark shapes (Llama-3.2-1B geometry)")
    parser.add_argument("--only-reference-shapes", action="store_true",
                        help="time only the reference's own benchmark shapes (Llama-3.2-1B geometry) and print them")
    args = parser.parse_args()

    if args.only_reference_shapes and args.gpus == 1:
        _native.load()
        for row in _reference_shapes(args.seed):
            print(json.dumps(row), flush=True)
        return 0
    if args.only_prefill and args.gpus == 1:
        return _only_prefill(args.only_prefill, args.seed, args.steps, args.warmup)
    if args.only_step and args.gpus == 1:
        if args.copy_calibration:
            _copy_calibration()
        return _only_step(args.seed, args.steps, args.warmup)
    if args.gpus != 1:
        print("bench.py measures one GPU: this build's paged path has no multi-GPU component "
              "(decode shards by sequence or KV head with no exchange inside attention); run with --gpus 1.",
              file=sys.stderr)
        return 2
    if not torch.cuda.is_available():
        print("bench.py needs a ROCm GPU", file=sys.stderr)
        return 2
    _native.load()
    torch.cuda.set_device(0)
    if args.copy_calibration:
        _copy_calibration()

    step = decode_step("c2", seed=args.seed)
    geo = step.geometry
    wall, step_ms = _time_step(step, args.steps, args.warmup)
    ms_per_step = wall / args.steps * 1e3
    d_bytes = decode_bytes(step.host_context_lens, geo)
    s_bytes = scatter_bytes(step.batch, geo)
    # the launch's own bytes: the decode's plus the newest rows read and stored
    w_bytes = 4 * step.batch * geo.num_kv_heads * geo.head_dim * 2
    value = (d_bytes + s_bytes) / (ms_per_step * 1e-3) / 1e9
    step_avg_ms = statistics.mean(step_ms)
    achieved = (d_bytes + w_bytes) / (step_avg_ms * 1e-3) / 1e9
    step_graph_us = graph_replay_us(_fused_step_call(step))
    # The same step as the reference runs it: the slot-write, then the decode.
    unfused_wall, decode_ms = _time_decode(step, args.steps, args.warmup)
    decode_avg_ms = statistics.mean(decode_ms)

    result = {
        "metric": METRIC,
        "value": round(value, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic N(0,1) q/K/V, seeded shuffled block tables",
        "config": {
            "workload": "c2: one layer's decode step (slot-write of the newest K/V + paged decode, one launch), "
                        "Llama-3-8B attention geometry",
            "batch": step.batch,
            "context_tokens": sum(step.host_context_lens),
            "context_range": [min(step.host_context_lens), max(step.host_context_lens)],
            "num_heads": geo.num_heads,
            "num_kv_heads": geo.num_kv_heads,
            "head_dim": geo.head_dim,
            "block_size": 16,
            "pool_blocks": 65536,
            "parallelism": "single GPU",
        },
        "roofline": {
            "kernel": "paged decode step call: decode_grouped (newest-row write + split decode) then combine_balanced",
            "bound": "hbm",
            "achieved": round(achieved, 1),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBS, 4),
            "traffic": _traffic(),
            "algorithmic_bytes_per_launch": d_bytes + w_bytes,
            "avg_launch_us": round(step_avg_ms * 1e3, 2),
            "graph_replay": {
                "avg_launch_us": round(step_graph_us, 2),
                "achieved": round((d_bytes + w_bytes) / (step_graph_us * 1e-6) / 1e9, 1),
                "frac": round((d_bytes + w_bytes) / (step_graph_us * 1e-6) / 1e9 / HBM_PEAK_GBS, 4),
                "method": "one step captured in a HIP graph; 100 replays between HIP events, best of 5",
            },
        },
        "c2_step_two_launches": {
            "what": "the reference's order, eager: slot-write launch (kv_scatter), then the decode call; "
                    "ms_per_step by wall clock over the eager calls",
            "ms_per_step": round(unfused_wall / args.steps * 1e3, 5),
            "decode_call_us": round(decode_avg_ms * 1e3, 2),
            "decode_frac_hbm": round(d_bytes / (decode_avg_ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
        },
    }

    if not args.no_secondary:
        secondary = {}
        del step
        torch.cuda.empty_cache()
        c4 = decode_step("c4", seed=args.seed)
        _, c4_ms = _time_decode(c4, max(10, args.steps // 4), SECONDARY_WARMUP)
        c4_bytes = decode_bytes(c4.host_context_lens, c4.geometry)
        c4_avg = statistics.mean(c4_ms)
        secondary["decode_c4"] = {
            "avg_us": round(c4_avg * 1e3, 2),
            "GB/s": round(c4_bytes / (c4_avg * 1e-3) / 1e9, 1),
            "frac_hbm": round(c4_bytes / (c4_avg * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
            "context_tokens": sum(c4.host_context_lens),
        }
        _graph_hbm(secondary["decode_c4"], _decode_call(c4), c4_bytes)
        # The same decode steps over an fp8 (e4m3) pool: half the K/V bytes.
        c4 = to_fp8_pool(c4)
        _, c4_ms8 = _time_decode(c4, max(10, args.steps // 4), SECONDARY_WARMUP)
        c4_bytes8 = decode_bytes(c4.host_context_lens, c4.geometry, kv_elem=1)
        c4_avg8 = statistics.mean(c4_ms8)
        secondary["decode_c4_fp8_kv"] = {
            "avg_us": round(c4_avg8 * 1e3, 2),
            "GB/s": round(c4_bytes8 / (c4_avg8 * 1e-3) / 1e9, 1),
            "frac_hbm": round(c4_bytes8 / (c4_avg8 * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
            "speedup_vs_bf16_kv": round(c4_avg / c4_avg8, 3),
        }
        _graph_hbm(secondary["decode_c4_fp8_kv"], _decode_call(c4), c4_bytes8)
        del c4
        torch.cuda.empty_cache()
        c2 = to_fp8_pool(decode_step("c2", seed=args.seed))
        _, c2_ms8 = _time_decode(c2, max(10, args.steps // 4), SECONDARY_WARMUP)
        c2_bytes8 = decode_bytes(c2.host_context_lens, c2.geometry, kv_elem=1)
        c2_avg8 = statistics.mean(c2_ms8)
        secondary["decode_c2_fp8_kv"] = {
            "avg_us": round(c2_avg8 * 1e3, 2),
            "GB/s": round(c2_bytes8 / (c2_avg8 * 1e-3) / 1e9, 1),
            "frac_hbm": round(c2_bytes8 / (c2_avg8 * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
            "speedup_vs_bf16_kv": round(decode_avg_ms / c2_avg8, 3),
        }
        _graph_hbm(secondary["decode_c2_fp8_kv"], _decode_call(c2), c2_bytes8)
        del c2
        torch.cuda.empty_cache()
        c3 = packed_step("c3", seed=args.seed)
        c3_ms = _time_prefill(c3, max(10, args.steps // 4), SECONDARY_WARMUP)
        c3_avg = statistics.mean(c3_ms)
        flops = prefill_flops(c3.host_query_lens, c3.host_context_lens, c3.geometry)
        secondary["prefill_c3"] = {
            "avg_us": round(c3_avg * 1e3, 2),
            "TFLOP/s": round(flops / (c3_avg * 1e-3) / 1e12, 2),
            "frac_bf16_peak": round(flops / (c3_avg * 1e-3) / 1e12 / BF16_PEAK_TFLOPS, 4),
            "visible_pair_flops": flops,
            "query_tokens": sum(c3.host_query_lens),
        }
        _graph_mfma(secondary["prefill_c3"], _prefill_call(c3), flops)
        geo3, c3_tokens = c3.geometry, sum(c3.host_query_lens)
        c3 = to_fp8_pool(c3)
        c3_avg8 = statistics.mean(_time_prefill(c3, max(10, args.steps // 4), SECONDARY_WARMUP))
        secondary["prefill_c3_fp8_kv"] = {
            "avg_us": round(c3_avg8 * 1e3, 2),
            "TFLOP/s": round(flops / (c3_avg8 * 1e-3) / 1e12, 2),
            "frac_bf16_peak": round(flops / (c3_avg8 * 1e-3) / 1e12 / BF16_PEAK_TFLOPS, 4),
        }
        _graph_mfma(secondary["prefill_c3_fp8_kv"], _prefill_call(c3), flops)
        del c3
        torch.cuda.empty_cache()
        # Config 3's two kinds of work on their own: the 8 chunks (MFMA-bound)
        # and the 56 one-query rows (HBM-bound), each as a packed pass.
        chunks, rows = c3_shapes(args.seed)
        part = packed_step("custom", seed=args.seed, chunks=chunks, decode_contexts=[])
        part_avg = statistics.mean(_time_prefill(part, max(10, args.steps // 4), SECONDARY_WARMUP))
        part_flops = prefill_flops(part.host_query_lens, part.host_context_lens, part.geometry)
        secondary["prefill_c3_chunks"] = {
            "avg_us": round(part_avg * 1e3, 2),
            "TFLOP/s": round(part_flops / (part_avg * 1e-3) / 1e12, 2),
            "frac_bf16_peak": round(part_flops / (part_avg * 1e-3) / 1e12 / BF16_PEAK_TFLOPS, 4),
        }
        _graph_mfma(secondary["prefill_c3_chunks"], _prefill_call(part), part_flops)
        del part
        torch.cuda.empty_cache()
        part = packed_step("custom", seed=args.seed, chunks=[], decode_contexts=rows)
        part_avg = statistics.mean(_time_prefill(part, max(10, args.steps // 4), SECONDARY_WARMUP))
        part_bytes = decode_bytes(part.host_context_lens, part.geometry)
        secondary["c3_decode_rows"] = {
            "avg_us": round(part_avg * 1e3, 2),
            "GB/s": round(part_bytes / (part_avg * 1e-3) / 1e9, 1),
            "frac_hbm": round(part_bytes / (part_avg * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
        }
        _graph_hbm(secondary["c3_decode_rows"], _prefill_call(part), part_bytes)
        del part
        torch.cuda.empty_cache()
        # Long chunks: 8 chunks of 2048 queries over 8192 cached keys.
        part = packed_step("custom", seed=args.seed, chunks=[(2048, 8192)] * 8, decode_contexts=[])
        part_avg = statistics.mean(_time_prefill(part, max(10, args.steps // 20), 5))
        part_flops = prefill_flops(part.host_query_lens, part.host_context_lens, part.geometry)
        secondary["prefill_8x2048_over_8192"] = {
            "avg_us": round(part_avg * 1e3, 2),
            "TFLOP/s": round(part_flops / (part_avg * 1e-3) / 1e12, 2),
            "frac_bf16_peak": round(part_flops / (part_avg * 1e-3) / 1e12 / BF16_PEAK_TFLOPS, 4),
        }
        _graph_mfma(secondary["prefill_8x2048_over_8192"], _prefill_call(part), part_flops)
        del part
        torch.cuda.empty_cache()
        secondary["rope_kv_write_c3"] = _time_rope(1, c3_tokens, geo3)
        secondary["rope_kv_write_c2"] = _time_rope(64, 1, geo3)
        if not args.no_reference_shapes:
            secondary["reference_a40_shapes"] = _reference_shapes(args.seed)
        result["secondary"] = secondary
        torch.cuda.empty_cache()
        step = None

    if not args.no_secondary and not args.no_e2e:
        from liteinfer_amd.engine import e2e

        result.setdefault("secondary", {})["e2e_c5"] = e2e.run(seed=args.seed)
        torch.cuda.empty_cache()
        result["secondary"]["e2e_c5_fp8_kv"] = e2e.run(seed=args.seed, cache_quant="fp8")
        torch.cuda.empty_cache()

    if not args.no_cpu_baseline:
        gpu_ms = {"c2": round(decode_avg_ms, 4)}
        for name, key in (("c3", "prefill_c3"), ("c4", "decode_c4")):
            if key in result.get("secondary", {}):
                gpu_ms[name] = round(result["secondary"][key]["avg_us"] / 1e3, 4)
        result["cpu_baseline"] = cpu_baseline(args.seed, gpu_ms=gpu_ms)

    print(json.dumps(result))
    return 0


if __name__ == "__main__":
    sys.exit(main())
