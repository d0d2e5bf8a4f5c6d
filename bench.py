"""Benchmark of the paged decode hot path on one MI355X.

Workload (the metric's configuration): batched one-token paged decode attention, batch 64,
32 query / 4 KV heads, head dim 64, fp16 KV with N(0,1) values, context lengths drawn
uniformly from 1..2048 (partial last blocks included), fragmented block tables carved from
a random permutation of an 8192-block pool, repeated over the pool's 22 layers. A step is
one pass over the 22 layers (one pc_paged_decode_attn call per layer: one kernel over
balanced bins of the batch's blocks, sequences cut at a bin edge merged inside it), with
inputs resident in HBM; the 22 layer planes (1.48 GB of KV per step) exceed the 256 MB Infinity
Cache, so the bytes come from HBM.

Printed as one JSON line: value = algorithmic HBM bytes per step x steps / wall time
(GB/s), plus decode tokens/s, the roofline of the attention call (algorithmic bytes per
call over the average call duration in the timed region; HBM traffic per call from the
committed rocprofv3 counter summary), and the CPU baseline (the oracle's op-for-op restatement of the reference's
torch CPU path, timed on a bounded sample on this host's cores).

    python bench.py [--steps K] [--warmup W] [--gpus 1]
"""

from __future__ import annotations

import argparse
import json
import os
import sys
import time

import numpy as np
import torch
from typing import Sequence
from torch import Tensor

ROOT = os.path.dirname(os.path.abspath(__file__))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

from pagedcore_amd import _hip  # noqa: E402
from tests import workloads  # noqa: E402
from tests.support import fragmented_decode_cache  # noqa: E402

LAYERS = 22
PEAK_HBM_GBPS = 8000.0


def attention_bytes(lengths: np.ndarray) -> int:
    """Algorithmic HBM bytes of one attention launch: K+V of every cached token
    (4 kv heads x 64 x 2 B x 2), Q read + O written (fp16), block-table entries and
    context lengths (int32). Split-K workspace traffic is excluded."""
    batch = int(lengths.shape[0])
    kv = int(lengths.astype(np.int64).sum()) * 1024
    qo = batch * 32 * 64 * 2 * 2
    tables = int(((lengths.astype(np.int64) + 15) // 16).sum()) * 4 + batch * 4
    return kv + qo + tables


class DecodeLayers:
    """Device buffers and raw C-ABI launches for the 22-layer decode step."""

    def __init__(self, w: workloads.BatchedDecode, device: torch.device, seed: int) -> None:
        gen = torch.Generator(device=device).manual_seed(seed)
        self.w = w
        self.device = device
        self.pool = torch.randn((LAYERS, 2, w.num_blocks, 16, 4, 64), dtype=torch.float16, device=device, generator=gen)
        self.queries = torch.randn((LAYERS, w.batch, 32, 64), dtype=torch.float16, device=device, generator=gen)
        self.out = torch.empty_like(self.queries)
        self.tables = torch.from_numpy(w.tables).to(device)
        self.lens = torch.from_numpy(w.lengths).to(device)
        self.lib = _hip.load()
        self.max_blocks = int(w.tables.shape[1])
        nbytes = int(self.lib.pc_attn_workspace_bytes(w.batch, self.max_blocks))
        self.workspace = torch.zeros(max(nbytes, 256), dtype=torch.uint8, device=device)
        # One decode plan per step, shared by the 22 layers (built from the host lengths,
        # like the block tables).
        self.plan = torch.from_numpy(_hip.decode_plan(w.lengths, w.tables)).to(device)

    def launch(self, layer: int, stream: int) -> None:
        status = self.lib.pc_paged_decode_attn(
            self.out[layer].data_ptr(), self.queries[layer].data_ptr(), self.pool.data_ptr(), self.w.num_blocks,
            layer, self.lens.data_ptr(), self.w.batch, self.max_blocks, self.plan.data_ptr(), self.plan.shape[0],
            self.workspace.data_ptr(), stream,
        )
        if status:
            raise RuntimeError(self.lib.pc_last_error().decode())

    def step(self) -> None:
        stream = torch.cuda.current_stream(self.device).cuda_stream
        for layer in range(LAYERS):
            self.launch(layer, stream)


def run_decode(steps: int, warmup: int, use_graph: bool = True) -> dict:
    """Times `steps` 22-layer decode steps of the batch-64 workload; returns the figures."""
    device = torch.device("cuda:0")
    w = workloads.batched_decode(batch=64, num_blocks=8192)
    layers = DecodeLayers(w, device, seed=1234)
    bytes_per_launch = attention_bytes(w.lengths)
    for _ in range(warmup):
        layers.step()
    torch.cuda.synchronize(device)
    eager_out = layers.out.clone()

    replay = layers.step
    if use_graph:
        graph = _captured(layers.step, device)
        for _ in range(3):
            layers.out.fill_(float("nan"))
            graph.replay()
            torch.cuda.synchronize(device)
            if not torch.equal(layers.out, eager_out):
                print("graph replay differs from eager launches; timing eager launches", file=sys.stderr)
                use_graph = False
                break
        if use_graph:
            replay = graph.replay

    torch.cuda.synchronize(device)
    start = torch.cuda.Event(enable_timing=True)
    stop = torch.cuda.Event(enable_timing=True)
    start.record()
    for _ in range(steps):
        replay()
    stop.record()
    torch.cuda.synchronize(device)
    total_ms = start.elapsed_time(stop)
    if not torch.equal(layers.out, eager_out):
        raise RuntimeError("timed steps produced different outputs than the warmup")
    _check_faults(layers.workspace, "attention")
    # A second, separate pass times each step alone (its own pair of events) for the median
    # the measurement plan asks for; `value` stays the whole timed region above.
    events = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(steps)]
    for begin, end in events:
        begin.record()
        replay()
        end.record()
    torch.cuda.synchronize(device)
    per_step = sorted(begin.elapsed_time(end) for begin, end in events)
    # The timed region holds steps x 22 pc_paged_decode_attn calls back to back on one
    # stream (one kernel launch each, no host work in between when replayed as a graph), so
    # its HIP-event time divided by the call count is the average call duration (launch
    # gaps included); rocprofv3's average kernel duration is that less the gap.
    launch_ms = total_ms / (steps * LAYERS)
    return {
        "layers": layers,
        "w": w,
        "bytes_per_launch": bytes_per_launch,
        "total_ms": total_ms,
        "ms_per_step": total_ms / steps,
        "gbps": bytes_per_launch * LAYERS * steps / (total_ms / 1e3) / 1e9,
        "tokens_per_s": w.batch * steps / (total_ms / 1e3),
        "launch_ms": launch_ms,
        "launch_gbps": bytes_per_launch / (launch_ms / 1e3) / 1e9,
        "graph": use_graph,
        "bins": int((layers.plan[:, 0] > 0).sum().item()),
        "step_ms_median": per_step[len(per_step) // 2],
        "step_ms_min": per_step[0],
        "step_ms_max": per_step[-1],
    }


def _timed(replay, steps: int, device: torch.device) -> float:
    """Milliseconds of `steps` calls of replay() between two HIP events on the current stream."""
    torch.cuda.synchronize(device)
    start = torch.cuda.Event(enable_timing=True)
    stop = torch.cuda.Event(enable_timing=True)
    start.record()
    for _ in range(steps):
        replay()
    stop.record()
    torch.cuda.synchronize(device)
    return start.elapsed_time(stop)


def _check_faults(workspace: Tensor, where: str) -> None:
    """Refuse to report a figure from runs whose attention recorded a device fault (a merge
    that timed out or saw another XCD's flag, a block id outside the pool)."""
    faults = int(_hip.fault_word(workspace).item())
    if faults:
        raise RuntimeError(f"{where}: paged attention recorded device fault word {faults:#x}")


def _captured(fn, device: torch.device) -> torch.cuda.CUDAGraph:
    """fn's launches as a graph, captured without emptying torch's allocator cache (the
    decoder's capture_graph: a cache released to the driver slows the next seconds'
    bandwidth-bound kernels)."""
    from pagedcore_amd.decoder import capture_graph

    return capture_graph(fn, device)[0]


def cpu_long_context_baseline(pool: Tensor, queries: Tensor, new_kv: Tensor, w: workloads.BatchedDecode,
                              seconds: float) -> dict:
    """The oracle's ports of the reference's per-row decode work on the CPU, per sequence of
    one layer: write_decode_layer's copies of the new token (kv_cache.py:242-245) and one
    paged_attention call over its 2048 tokens (attention.py:14-53, as decoder.py:182-190
    calls it), on all host threads. Sequences are taken in order (cycling the 22 layers)
    for about `seconds`; the per-step figure scales the mean per-sequence time to the
    batch x 22 layers. Copying the sampled blocks to host memory is not timed."""
    from oracle import paged_reference as ref

    cores = len(os.sched_getaffinity(0))
    torch.set_num_threads(cores)
    done, elapsed, row = 0, 0.0, 0
    while elapsed < seconds:
        layer, b = divmod(row, w.batch)
        layer %= LAYERS
        length = int(w.lengths[b])
        table = [int(x) for x in w.tables[b, : (length + 15) // 16]]
        index = torch.tensor(table, dtype=torch.long, device=pool.device)
        sub = torch.empty((LAYERS, 2, len(table), 16, 4, 64), dtype=torch.float16)
        sub[layer] = pool[layer].index_select(1, index).cpu()
        host = sub.view(torch.int16).numpy().view(np.uint16)
        key = new_kv[0, layer, b].cpu().view(torch.int16).numpy().view(np.uint16)
        value = new_kv[1, layer, b].cpu().view(torch.int16).numpy().view(np.uint16)
        query = queries[layer, b].reshape(1, 32, 1, 64).cpu()
        local = list(range(len(table)))
        start = time.perf_counter()
        ref.reference_write_decode(host, layer, local, length, key, value)
        ref.reference_paged_attention(query, sub, layer, local, length)
        elapsed += time.perf_counter() - start
        done += 1
        row += 1
    per_row = elapsed / done
    step_s = per_row * w.batch * LAYERS
    per_step_bytes = (attention_bytes(w.lengths) + w.batch * 1024 * 2) * LAYERS
    return {
        "value": round(per_step_bytes / step_s / 1e9, 4),
        "unit": "GB/s",
        "cores": cores,
        "kind": "port",
        "sample": f"{done} sequence-layers of the same workload (append of the new token + one reference paged_attention "
        f"call over 2048 tokens each), {elapsed:.1f} s on {cores} threads, {per_row * 1e3:.2f} ms per sequence-layer; "
        f"scaled to {w.batch} sequences x 22 layers: {step_s:.2f} s per step, {w.batch / step_s:.2f} decode tokens/s",
    }


def run_long_context(steps: int, warmup: int, cpu_seconds: float = 0.0) -> dict:
    """Long-context, high-occupancy decode: batch 256, every sequence at 2047 cached tokens
    (128 blocks), a fully shuffled 40000-block pool, 22 layers. Per layer the step appends
    each sequence's new token (slot 2047) and runs attention over 2048 tokens, replayed as
    one graph: timed as one fused launch (pc_kv_append_paged_decode_attn) and, for
    comparison, as the pair pc_kv_append + pc_paged_decode_attn, each on its own copy of the
    same pool. The two give the same bits (checked here): the outputs, and the whole pools
    after every step either leg ran, so a new row stored anywhere but its slot shows."""
    device = torch.device("cuda:0")
    w = workloads.batched_decode(batch=256, num_blocks=40000, fixed_length=2048, seed=20261204)
    gen = torch.Generator(device=device).manual_seed(4321)
    base = torch.randn((LAYERS, 2, w.num_blocks, 16, 4, 64), dtype=torch.float16, device=device, generator=gen)
    queries = torch.randn((LAYERS, w.batch, 32, 64), dtype=torch.float16, device=device, generator=gen)
    new_kv = torch.randn((2, LAYERS, w.batch, 4, 64), dtype=torch.float16, device=device, generator=gen)
    out = torch.empty_like(queries)
    lib = _hip.load()
    max_blocks = int(w.tables.shape[1])
    lens = torch.from_numpy(w.lengths).to(device)
    plan = torch.from_numpy(_hip.decode_plan(w.lengths, w.tables)).to(device)
    workspace = torch.zeros(int(lib.pc_attn_workspace_bytes(w.batch, max_blocks)), dtype=torch.uint8, device=device)
    slots = torch.from_numpy(w.tables[:, max_blocks - 1].astype(np.int64) * 16 + 15).to(device)
    assert int(slots.max()) < w.num_blocks * 16

    pools = {"pair": base.clone(), "fused": base}

    def pair_step() -> None:
        pool = pools["pair"]
        stream = torch.cuda.current_stream(device).cuda_stream
        for layer in range(LAYERS):
            status = lib.pc_kv_append(
                pool.data_ptr(), w.num_blocks, layer, 1, new_kv[0, layer].data_ptr(), 0, 256,
                new_kv[1, layer].data_ptr(), 0, 256, slots.data_ptr(), w.batch, stream,
            )
            status = status or lib.pc_paged_decode_attn(
                out[layer].data_ptr(), queries[layer].data_ptr(), pool.data_ptr(), w.num_blocks, layer,
                lens.data_ptr(), w.batch, max_blocks, plan.data_ptr(), plan.shape[0], workspace.data_ptr(), stream,
            )
            if status:
                raise RuntimeError(lib.pc_last_error().decode())

    def fused_step() -> None:
        pool = pools["fused"]
        stream = torch.cuda.current_stream(device).cuda_stream
        for layer in range(LAYERS):
            status = lib.pc_kv_append_paged_decode_attn(
                out[layer].data_ptr(), queries[layer].data_ptr(), pool.data_ptr(), w.num_blocks, layer,
                lens.data_ptr(), w.batch, max_blocks, plan.data_ptr(), plan.shape[0], new_kv[0, layer].data_ptr(),
                new_kv[1, layer].data_ptr(), workspace.data_ptr(), stream,
            )
            if status:
                raise RuntimeError(lib.pc_last_error().decode())

    timings, outputs = {}, {}
    for name, step in (("pair", pair_step), ("fused", fused_step)):
        for _ in range(warmup):
            step()
        torch.cuda.synchronize(device)
        eager_out = out.clone()
        graph = _captured(step, device)
        graph.replay()
        torch.cuda.synchronize(device)
        if not torch.equal(out, eager_out):
            raise RuntimeError(f"{name}: graph replay differs from eager launches")
        outputs[name] = eager_out
        timings[name] = _timed(graph.replay, steps, device)
        del graph
    if not torch.equal(outputs["pair"].view(torch.int16), outputs["fused"].view(torch.int16)):
        raise RuntimeError("fused append + attention differs from pc_kv_append + pc_paged_decode_attn")
    if not torch.equal(pools["pair"].view(torch.int16), pools["fused"].view(torch.int16)):
        raise RuntimeError("the fused call's pool differs from the pool pc_kv_append wrote")
    _check_faults(workspace, "long_context_b256")
    del pools["pair"]
    pool = pools["fused"]
    total_ms = timings["fused"]
    attn = attention_bytes(w.lengths)
    append = w.batch * 1024 * 2  # read the new K/V rows, write them to their slots
    per_step = (attn + append) * LAYERS
    result = {
        "workload": "batch 256, every sequence 2047 cached + 1 appended (128 blocks), 40000-block shuffled pool, "
        "22 layers; per layer one pc_kv_append_paged_decode_attn (append of the 256 new tokens fused with "
        "attention), replayed as one graph",
        "ms_per_step": round(total_ms / steps, 4),
        "gbps": round(per_step * steps / (total_ms / 1e3) / 1e9, 2),
        "hbm_fraction": round(per_step * steps / (total_ms / 1e3) / 1e9 / PEAK_HBM_GBPS, 4),
        "decode_tokens_per_s": round(w.batch * steps / (total_ms / 1e3), 1),
        "bytes_per_layer": attn + append,
        "us_per_layer": round(total_ms / steps / LAYERS * 1e3, 3),
        "unfused_us_per_layer": round(timings["pair"] / steps / LAYERS * 1e3, 3),
    }
    if cpu_seconds > 0:
        result["cpu_baseline"] = cpu_long_context_baseline(pool, queries, new_kv, w, cpu_seconds)
    return result


def cpu_append_baseline(w: workloads.PromptAppend, table: Sequence[int], seconds: float) -> dict:
    """The oracle's port of KVAllocator.append's chunked copies (kv_cache.py:161-172): the
    same 2048-token prompt (K and V of 22 layers) in the same 128 chunk copies per kind, one
    thread (numpy slice copies, as the reference's CPU tensor copies), repeated for about
    `seconds` after one untimed append that faults the pages in. The host pool holds just
    the prompt's 128 blocks, in table order (a 1.4 GB host pool would only add page
    faults). The allocator's Python bookkeeping is not included."""
    from oracle import paged_reference as ref

    key, value = (a.view(np.uint16) for a in w.prompt_kv())
    pool = np.zeros((LAYERS, 2, len(table), 16, 4, 64), dtype=np.uint16)
    compact = list(range(len(table)))
    ref.reference_append(pool, compact, 0, key, value)
    done, elapsed = 0, 0.0
    while elapsed < seconds:
        start = time.perf_counter()
        ref.reference_append(pool, compact, 0, key, value)
        elapsed += time.perf_counter() - start
        done += 1
    nbytes = 2 * 2 * LAYERS * w.prompt_tokens * 256 * 2
    return {
        "value": round(nbytes * done / elapsed / 1e9, 4),
        "unit": "GB/s",
        "cores": 1,
        "kind": "port",
        "sample": f"{done} whole appends of the same 2048-token prompt (128 blocks), {elapsed:.1f} s on one thread; "
        f"{elapsed / done * 1e3:.2f} ms per append",
    }


def cpu_single_decode_baseline(pool: Tensor, query: Tensor, table: Sequence[int], seconds: float) -> dict:
    """Latency of the oracle's port of the reference's paged_attention (attention.py:14-53)
    on the single-sequence case, on this host's cores: one call per iteration, repeated for
    about `seconds` after one untimed call (copying the pool to host memory is not timed)."""
    from oracle import paged_reference as ref

    cores = len(os.sched_getaffinity(0))
    torch.set_num_threads(cores)
    host_pool, host_query = pool.cpu(), query.reshape(1, 32, 1, 64).cpu()
    ref.reference_paged_attention(host_query, host_pool, 0, list(table), 128)
    done, elapsed = 0, 0.0
    while elapsed < seconds:
        start = time.perf_counter()
        ref.reference_paged_attention(host_query, host_pool, 0, list(table), 128)
        elapsed += time.perf_counter() - start
        done += 1
    return {
        "value": round(elapsed / done * 1e6, 2),
        "unit": "us per call",
        "cores": cores,
        "kind": "port",
        "sample": f"{done} calls on the same 128-token sequence, {elapsed:.1f} s on {cores} threads",
    }


def run_single_decode(calls: int = 200, cpu_seconds: float = 0.0) -> dict:
    """The single-sequence decode case: one query [1, 32, 64] over 128 cached tokens (8
    blocks of a random table in a NaN-poisoned 64-block pool), one layer. Latency-bound
    (139 KB of K/V, Q and O), so it is reported as the average duration of one
    pc_paged_decode_attn call, `calls` calls replayed back to back as one graph."""
    device = torch.device("cuda:0")
    gen = torch.Generator(device=device).manual_seed(1)
    pool = torch.full((LAYERS, 2, 64, 16, 4, 64), float("nan"), dtype=torch.float16, device=device)
    table = torch.randperm(64, generator=torch.Generator().manual_seed(1))[:8].to(torch.int32)
    lengths = np.array([128], dtype=np.int32)
    for i, block in enumerate(table.tolist()):
        pool[:, :, block] = torch.randn((LAYERS, 2, 16, 4, 64), dtype=torch.float16, device=device, generator=gen)
    query = torch.randn((1, 32, 64), dtype=torch.float16, device=device, generator=gen)
    out = torch.empty_like(query)
    lib = _hip.load()
    plan = torch.from_numpy(_hip.decode_plan(lengths, table.numpy()[None])).to(device)
    lens = torch.from_numpy(lengths).to(device)
    workspace = torch.zeros(int(lib.pc_attn_workspace_bytes(1, 8)), dtype=torch.uint8, device=device)

    def call() -> None:
        status = lib.pc_paged_decode_attn(
            out.data_ptr(), query.data_ptr(), pool.data_ptr(), 64, 0, lens.data_ptr(), 1, 8, plan.data_ptr(),
            plan.shape[0], workspace.data_ptr(), torch.cuda.current_stream(device).cuda_stream,
        )
        if status:
            raise RuntimeError(lib.pc_last_error().decode())

    call()
    torch.cuda.synchronize(device)
    if not torch.isfinite(out).all():
        raise RuntimeError("single decode produced non-finite output")

    def calls_fn() -> None:
        for _ in range(calls):
            call()

    graph = _captured(calls_fn, device)
    graph.replay()
    total_ms = _timed(graph.replay, 1, device)
    nbytes = attention_bytes(lengths)
    us = total_ms / calls * 1e3
    result = {
        "workload": "one sequence, 128 cached tokens on a random 8-block table of a 64-block pool, one layer",
        "us_per_call": round(us, 3),
        "bytes_per_call": int(nbytes),
        "gbps": round(nbytes / (us / 1e6) / 1e9, 2),
    }
    if cpu_seconds > 0:
        result["cpu_baseline"] = cpu_single_decode_baseline(pool, query, table.tolist(), cpu_seconds)
    return result


def run_prompt_append(steps: int, cpu_seconds: float = 0.0) -> dict:
    """Prompt KV append: one 2048-token prompt's K and V (22 layers, N(0, 1) fp16) into a
    4096-block pool whose free list is in seeded random order with 30% of it held by 10
    filler requests, so the prompt's 128 blocks are scattered. The allocator's append is
    called once (its slot mapping); the timed region replays that one pc_kv_append launch
    (all 22 layers x 2048 tokens) as a graph of `steps` launches."""
    from pagedcore_amd.engine_types import KVReservation, RequestId
    from pagedcore_amd.kv_cache import KVAllocator

    device = torch.device("cuda:0")
    w = workloads.prompt_append()
    pool = torch.zeros((LAYERS, 2, w.num_blocks, 16, 4, 64), dtype=torch.float16, device=device)
    allocator = KVAllocator(pool)
    allocator._free_blocks[:] = w.free_order  # the seeded allocator's free-list order
    for index in range(len(w.filler_blocks)):
        request = RequestId(f"filler{index}")
        allocator.create(KVReservation(request, w.filler_blocks[index]))
        allocator.append(request, *(torch.from_numpy(a).to(device) for a in w.filler_kv(index)))
    key, value = (torch.from_numpy(a).to(device) for a in w.prompt_kv())
    prompt = RequestId("prompt")
    allocator.create(KVReservation(prompt, 128))
    torch.cuda.synchronize(device)
    start = time.perf_counter()
    allocator.append(prompt, key, value)
    torch.cuda.synchronize(device)
    api_ms = (time.perf_counter() - start) * 1e3
    table = np.asarray(allocator.block_table(prompt), dtype=np.int64)
    positions = np.arange(w.prompt_tokens)
    slots = torch.from_numpy(table[positions // 16] * 16 + positions % 16).to(device)
    scattered = int(np.sum(np.diff(table) != 1))

    def launches() -> None:
        for _ in range(steps):
            _hip.kv_append(pool, 0, key, value, slots)

    graph = _captured(launches, device)
    total_ms = _timed(graph.replay, 1, device)
    nbytes = 2 * 2 * LAYERS * w.prompt_tokens * 256 * 2  # K and V, read once and written once
    us = total_ms / steps * 1e3
    result = {
        "workload": "2048-token prompt x 22 layers (K and V [22,2048,4,64] fp16) into a 4096-block pool, 30% held by "
        f"10 filler requests, free list in seeded random order ({scattered} discontinuities in the 128-block table)",
        "us_per_append": round(us, 3),
        "gbps": round(nbytes / (us / 1e6) / 1e9, 2),
        "hbm_fraction": round(nbytes / (us / 1e6) / 1e9 / PEAK_HBM_GBPS, 4),
        "bytes_per_append": nbytes,
        "allocator_append_ms": round(api_ms, 3),
    }
    if cpu_seconds > 0:
        result["cpu_baseline"] = cpu_append_baseline(w, [int(b) for b in table], cpu_seconds)
    return result


def run_prefill(steps: int) -> dict:
    """Paged prefill of one 2048-token prompt through the full TinyLlama-architecture model
    (random N(0, 0.02) fp16 weights): prefill_paged = 22 x (RMSNorm, QKV GEMM, RoPE + KV write
    into the staged slots, causal prompt attention, o_proj, add + RMSNorm, gate/up GEMM,
    SwiGLU, down GEMM, add + RMSNorm), LM head over all positions, one publish. Timed end to
    end per prompt (the request is released and re-admitted between prompts, untimed),
    plus the prompt attention kernel alone on the same shapes."""
    from pagedcore_amd import decoder as dec
    from pagedcore_amd.engine_types import KVReservation, RequestId
    from pagedcore_amd.kv_cache import KVAllocator

    device = torch.device("cuda:0")
    tokens = 2048
    weights = dec.random_weights(device=device, seed=20261206)
    pool = torch.empty((LAYERS, 2, 160, 16, 4, 64), dtype=torch.float16, device=device)
    allocator = KVAllocator(pool)
    gen = torch.Generator(device=device).manual_seed(6)
    ids = torch.randint(0, 32000, (1, tokens), device=device, generator=gen)
    request = RequestId("prompt")
    total = 0.0
    for index in range(steps + 1):
        allocator.create(KVReservation(request, tokens // 16))
        torch.cuda.synchronize(device)
        start = time.perf_counter()
        dec.prefill_paged(ids, weights, allocator, request)
        torch.cuda.synchronize(device)
        if index > 0:  # the first prompt warms up the GEMM libraries
            total += time.perf_counter() - start
        allocator.release_all(request)
    ms = total / steps * 1e3

    query = torch.randn((tokens, 32, 64), dtype=torch.float16, device=device, generator=gen)
    key = torch.randn((tokens, 4, 64), dtype=torch.float16, device=device, generator=gen)
    value = torch.randn((tokens, 4, 64), dtype=torch.float16, device=device, generator=gen)
    out = torch.empty_like(query)
    graph = _captured(lambda: [_hip.prefill_attention(out, query, key, value) for _ in range(10)], device)
    attn_us = _timed(graph.replay, 3, device) / 30 * 1e3
    flops = tokens * (tokens + 1) // 2 * 32 * 64 * 2 * 2
    return {
        "workload": "paged prefill of one 2048-token prompt, TinyLlama-architecture random N(0,0.02) fp16 weights, "
        "22 layers, RoPE + KV write fused into the staged append, causal prompt attention kernel",
        "ms_per_prompt": round(ms, 3),
        "prompt_tokens_per_s": round(tokens / (ms / 1e3), 1),
        "prompt_attention_us_per_layer": round(attn_us, 2),
        "prompt_attention_tflops": round(flops / (attn_us / 1e6) / 1e12, 2),
    }


def run_serving(requests: int = 128, max_active: int = 64) -> dict:
    """Continuous batching through DecodeWorker on the full TinyLlama-architecture model:
    `requests` prompts of U{128..1024} tokens, 64 new tokens each (ignore_eos, so every
    request runs to its length), at most `max_active` active, one admission (prefill) per
    iteration, FIFO; every decode step replays one DecodeGraph of `max_active` rows (a
    smaller batch is padded: the step's GEMMs stream the same weights at any row count up
    to 128, so padding costs little), and every prefill replays the PrefillGraph of the
    smallest multiple of 128 positions that holds the prompt. The graphs are captured
    before the timed region; timed from the first iteration until the queue drains."""
    from pagedcore_amd import decoder as dec
    from pagedcore_amd.engine_types import RequestId
    from pagedcore_amd.kv_cache import KVAllocator
    from pagedcore_amd.worker import DecodeWorker, GenerationRequest

    device = torch.device("cuda:0")
    rng = workloads.rng(20261207)
    weights = dec.random_weights(device=device, seed=20261207)
    lengths = rng.integers(128, 1025, size=requests)
    new_tokens = 64
    blocks = max_active * -(-(1024 + new_tokens) // 16) + 64
    allocator = KVAllocator(torch.empty((LAYERS, 2, blocks, 16, 4, 64), dtype=torch.float16, device=device))
    prompt_sizes = tuple(range(128, 1025, 128))
    worker = DecodeWorker(weights, allocator, max_active=max_active, graph_batch=max_active, prefill_graph_tokens=prompt_sizes)
    worker.capture_graphs()  # at start-up, before the timed run
    for index, length in enumerate(lengths):
        prompt = tuple(int(t) for t in rng.integers(3, 32000, size=int(length)))
        worker.submit(GenerationRequest(RequestId(f"req{index}"), prompt, new_tokens, ignore_eos=True))
    iterations, emitted, batch_sum = 0, 0, 0
    torch.cuda.synchronize(device)
    start = time.perf_counter()
    while not worker.idle:
        emitted += len(worker.step())
        batch_sum += sum(1 for _ in worker.active_ids)
        iterations += 1
    torch.cuda.synchronize(device)
    seconds = time.perf_counter() - start
    results = worker.results
    assert len(results) == requests and all(len(r.greedy_ids) == new_tokens for r in results.values())
    return {
        "workload": f"continuous batching: {requests} requests, prompts U{{128..1024}}, {new_tokens} new tokens each, "
        f"max {max_active} active, TinyLlama-architecture random weights; one prefill per iteration, every "
        f"decode step replays a {max_active}-row DecodeGraph (padded when fewer are active), every prefill a PrefillGraph "
        "of the smallest multiple of 128 positions holding the prompt (graphs captured before timing)",
        "seconds": round(seconds, 3),
        "generated_tokens_per_s": round(requests * new_tokens / seconds, 1),
        "prompt_tokens": int(lengths.sum()),
        "iterations": iterations,
        "mean_active": round(batch_sum / iterations, 2),
    }


def run_decode_step(steps: int, warmup: int) -> dict:
    """Full TinyLlama-architecture greedy decode step, batch 128, random N(0, 0.02) fp16
    weights, contexts uniform in 256..(2048 - steps - warmup - 1) pre-filled with N(0, 1)
    K/V in a fragmented pool; one step = embedding, 22 x (RMSNorm, QKV GEMM, RoPE + KV
    append, paged attention, o_proj, RMSNorm, gate/up GEMM, SwiGLU, down GEMM), final norm,
    LM head, argmax, through DecodeGraph (host bookkeeping + one graph replay per step).
    The attention + append share replays the same 22 x (pc_rope_kv_append +
    pc_paged_decode_attn) launches over the same inputs as a graph of their own (the
    appended rows go to a scratch pool so the cache is not disturbed)."""
    from pagedcore_amd import decoder as dec

    device = torch.device("cuda:0")
    batch = 128
    rng = workloads.rng(20261205)
    top = 2048 - steps - warmup - 1
    lengths = rng.integers(256, top + 1, size=batch)
    weights = dec.random_weights(device=device, seed=20261205)
    # Appends of up to 256 tokens, requests in a fresh random order each round: every
    # request's blocks end up interleaved with the others' (a fragmented pool).
    allocator, requests = fragmented_decode_cache(device, batch, lengths, steps + warmup + 1, seed=5)
    pool = allocator.pool
    num_blocks = int(pool.shape[2])
    gen = torch.Generator(device=device).manual_seed(5)
    graph = dec.DecodeGraph(weights, allocator, batch)
    ids = torch.randint(0, 32000, (batch, 1), device=device, generator=gen)
    state = {"ids": ids}

    def step() -> None:
        state["ids"] = graph.step(state["ids"], requests).argmax(-1)

    for _ in range(warmup):
        step()
    total_ms = _timed(step, steps, device)
    context = int(np.sum([allocator.cached_length(r) for r in requests]))

    # attention + append alone, same launches and inputs
    scratch = torch.empty((LAYERS, 2, (batch + 15) // 16, 16, 4, 64), dtype=torch.float16, device=device)
    scratch_slots = torch.arange(batch, dtype=torch.int64, device=device)
    qkv = torch.randn((batch, 2560), dtype=torch.float16, device=device, generator=gen)
    query = torch.empty((batch, 32, 64), dtype=torch.float16, device=device)
    attention = torch.empty_like(query)

    def attention_and_append() -> None:
        for layer in range(LAYERS):
            _hip.rope_kv_append(query, qkv, graph._inputs64[2], graph._table, pool=scratch, layer=layer, slot_mapping=scratch_slots)
            _hip.planned_decode_attention(attention, query, pool, layer, graph._lens, graph._plan, dec.MAX_BLOCKS, graph._workspace)

    attention_and_append()
    part = _captured(attention_and_append, device)
    part_ms = _timed(part.replay, steps, device)
    _check_faults(graph._workspace, "decode_step_b128")  # the fault word is sticky: covers every step above
    kv_bytes = context * 1024 * LAYERS
    weight_bytes = sum(t.numel() * 2 for layer in weights.layers for t in (dec._fused(layer).qkv, layer.o_proj, dec._fused(layer).gate_up, layer.down_proj))
    weight_bytes += weights.lm_head.numel() * 2
    return {
        "workload": f"TinyLlama-architecture decode step, batch {batch}, random N(0,0.02) fp16 weights, contexts "
        f"U{{256..{top}}} in a fragmented {num_blocks}-block pool, 22 layers, greedy argmax; DecodeGraph replay",
        "ms_per_step": round(total_ms / steps, 4),
        "decode_tokens_per_s": round(batch * steps / (total_ms / 1e3), 1),
        "attention_append_ms_per_step": round(part_ms / steps, 4),
        "attention_append_share": round(part_ms / total_ms, 4),
        "weights_bytes": weight_bytes,
        "kv_bytes_per_step": kv_bytes,
        "gbps_weights_plus_kv": round((weight_bytes + kv_bytes) / (total_ms / steps / 1e3) / 1e9, 2),
    }


def cpu_baseline(layers: DecodeLayers, seconds: float) -> dict:
    """The oracle's op-for-op restatement of the reference torch CPU path
    (attention.py:14-53, one call per sequence as in decoder.py:182-190), run over whole
    layers of the same workload -- cycling through the 22 layers again if needed -- until
    ~`seconds` of CPU work, on all of this host's cores. Only the attention calls are timed
    (copying each layer's blocks to host memory is not)."""
    from oracle import paged_reference as ref

    cores = len(os.sched_getaffinity(0))
    torch.set_num_threads(cores)
    w = layers.w
    host_tables = [w.tables[b, : (int(w.lengths[b]) + 15) // 16].tolist() for b in range(w.batch)]
    used = sorted({blk for table in host_tables for blk in table})
    remap = {blk: i for i, blk in enumerate(used)}
    index = torch.tensor(used, dtype=torch.long, device=layers.device)
    local_tables = [[remap[x] for x in table] for table in host_tables]
    done_bytes, done_layers, elapsed = 0, 0, 0.0
    while elapsed < seconds:
        layer = done_layers % LAYERS
        sub = torch.empty((LAYERS, 2, len(used), 16, 4, 64), dtype=torch.float16)
        sub[layer] = layers.pool[layer].index_select(1, index).cpu()
        queries = layers.queries[layer].reshape(w.batch, 1, 32, 1, 64).cpu()
        start = time.perf_counter()
        for b in range(w.batch):
            ref.reference_paged_attention(queries[b], sub, layer, local_tables[b], int(w.lengths[b]))
        elapsed += time.perf_counter() - start
        done_bytes += attention_bytes(w.lengths)
        done_layers += 1
    return {
        "value": round(done_bytes / elapsed / 1e9, 4),
        "unit": "GB/s",
        "cores": cores,
        "kind": "port",
        "sample": f"{done_layers} layer passes (cycling through the 22 layers) x all {w.batch} sequences of the "
        f"same workload, one reference paged_attention call per sequence, {elapsed:.1f} s of CPU time on "
        f"{cores} threads; decode tokens/s at that rate {w.batch * done_layers / LAYERS / elapsed:.2f}",
    }


def cpu_bookkeeping_baseline(layers: DecodeLayers, seconds: float) -> dict:
    """The secondary CPU number: the reference's per-row decode work including its
    allocator bookkeeping, on the same workload. Per sequence and layer, as its decode loop
    runs it (decoder.py:180-194): write_decode_layer (kv_cache.py:221-246: one
    _assert_accounting, then the new token's K/V copies) and paged_attention
    (attention.py:14-53, whose two iter_layer_blocks traversals each run _assert_accounting,
    kv_cache.py:248-270). _assert_accounting is the oracle's restatement of
    kv_cache.py:314-357 over this workload's state: 64 requests holding their tables in the
    8192-block pool, the rest free. Sequences are taken in order, cycling the layers, for
    about `seconds`; the step figure scales the mean per-sequence time to 64 x 22."""
    from oracle import paged_reference as ref

    cores = len(os.sched_getaffinity(0))
    torch.set_num_threads(cores)
    w = layers.w
    tables = [tuple(int(x) for x in w.tables[b, : (int(w.lengths[b]) + 15) // 16]) for b in range(w.batch)]
    sequences = {f"seq{b}": ref.SequenceRecord(f"seq{b}", 128, int(w.lengths[b]), tables[b]) for b in range(w.batch)}
    owners = {block: f"seq{b}" for b in range(w.batch) for block in tables[b]}
    free = [block for block in range(w.num_blocks - 1, -1, -1) if block not in owners]
    assert ref.reference_assert_accounting(sequences, free, owners, w.num_blocks)[2] == len(owners)
    gen = torch.Generator().manual_seed(3)
    done, elapsed, row = 0, 0.0, 0
    while elapsed < seconds:
        layer, b = divmod(row, w.batch)
        layer %= LAYERS
        length = int(w.lengths[b])
        index = torch.tensor(tables[b], dtype=torch.long, device=layers.device)
        sub = torch.empty((LAYERS, 2, len(tables[b]), 16, 4, 64), dtype=torch.float16)
        sub[layer] = layers.pool[layer].index_select(1, index).cpu()
        host = sub.view(torch.int16).numpy().view(np.uint16)
        new_kv = torch.randn((2, 4, 64), generator=gen).half().view(torch.int16).numpy().view(np.uint16)
        query = layers.queries[layer, b].reshape(1, 32, 1, 64).cpu()
        local = list(range(len(tables[b])))
        start = time.perf_counter()
        ref.reference_assert_accounting(sequences, free, owners, w.num_blocks)  # write_decode_layer
        ref.reference_write_decode(host, layer, local, length, new_kv[0], new_kv[1])
        ref.reference_assert_accounting(sequences, free, owners, w.num_blocks)  # first traversal
        ref.reference_assert_accounting(sequences, free, owners, w.num_blocks)  # second traversal
        ref.reference_paged_attention(query, sub, layer, local, length)
        elapsed += time.perf_counter() - start
        done += 1
        row += 1
    per_row = elapsed / done
    step_s = per_row * w.batch * LAYERS
    return {
        "value": round(attention_bytes(w.lengths) * LAYERS / step_s / 1e9, 4),
        "unit": "GB/s",
        "cores": cores,
        "kind": "port",
        "sample": f"{done} sequence-layers of the same workload, each: write_decode_layer's accounting check and "
        f"K/V copies, then paged_attention with its two accounting checks, {elapsed:.1f} s on {cores} threads, "
        f"{per_row * 1e3:.2f} ms per sequence-layer; scaled to {w.batch} sequences x 22 layers: {step_s:.2f} s per "
        f"step, {w.batch / step_s:.2f} decode tokens/s (GB/s over the attention's algorithmic bytes)",
    }


TRAFFIC_FILE = os.path.join(ROOT, "profiles", "paged_decode_attention_b64_hbm_traffic.txt")
EXTRA_CPU_SECONDS = 3.0  # CPU baseline sample of each extra workload that has one


ATTENTION_SOURCES = ("pagedcore_hip.hip", "pc_device.h", "pc_internal.h")


def kernel_source_hash() -> str:
    """sha256 (first 16 hex digits) of the sources the attention kernels are compiled from
    (csrc/pagedcore_hip.hip and the device headers it includes, in that order): the key
    under which the attention call's counter summary is valid."""
    import hashlib

    folder = os.path.join(ROOT, "pagedcore_amd", "csrc")
    digest = hashlib.sha256()
    for name in ATTENTION_SOURCES:
        with open(os.path.join(folder, name), "rb") as handle:
            digest.update(name.encode() + b"\0" + handle.read())
    return digest.hexdigest()[:16]


def measured_traffic() -> int | None:
    """HBM bytes per attention call from the committed rocprofv3 FETCH_SIZE / WRITE_SIZE
    summary, scaled by the plain-copy calibration recorded there; None unless that summary
    was made from exactly these kernel sources (its source_sha256 equals
    kernel_source_hash())."""
    try:
        with open(TRAFFIC_FILE) as handle:
            fields = dict(
                line.split(":", 1) for line in handle.read().splitlines() if line.count(":") >= 1 and not line.startswith(" ")
            )
    except OSError:
        return None
    fields = {k.strip(): v.strip() for k, v in fields.items()}
    try:
        same = fields["source_sha256"] == kernel_source_hash()
        return int(fields["traffic_bytes_per_call"]) if same else None
    except (KeyError, ValueError):
        return None


def calibration_copy(mib: int, device: torch.device) -> None:
    """One plain device-to-device copy of `mib` MiB (torch's elementwise copy kernel),
    outside any timed region: under rocprofv3 --pmc its FETCH_SIZE / WRITE_SIZE give the
    counters' scale for a known number of bytes."""
    src = torch.ones(mib * 2**20 // 4, dtype=torch.float32, device=device)
    dst = torch.empty_like(src)
    torch.cuda.synchronize(device)
    dst.copy_(src)
    torch.cuda.synchronize(device)
    del src, dst


def run_extra(selected: set, steps: int, cpu_seconds: float = 0.0) -> dict:
    """The workloads beside the headline, each reported as its own object (with a CPU
    baseline of about `cpu_seconds` where the workload has one; 0 = none).

    Device memory a workload frees stays in torch's cache for the next one: returning it to
    the driver (torch.cuda.empty_cache) and allocating again slows the next workload's
    bandwidth-bound kernels for several seconds (measured: the decode step ran 1.97 ms
    instead of 1.92 right after an empty_cache, and 1.92 after 10 idle seconds or with no
    empty_cache in between)."""
    extra = {}
    if "single_decode" in selected:
        extra["single_decode_c1"] = run_single_decode(cpu_seconds=cpu_seconds)
        print(f"single decode: {extra['single_decode_c1']}", file=sys.stderr, flush=True)
    if "prompt_append" in selected:
        extra["prompt_append"] = run_prompt_append(max(10, steps), cpu_seconds)
        print(f"prompt append: {extra['prompt_append']}", file=sys.stderr, flush=True)
    if "long_context" in selected:
        extra["long_context_b256"] = run_long_context(max(5, steps // 5), 2, cpu_seconds)
        print(f"long context: {extra['long_context_b256']}", file=sys.stderr, flush=True)
    if "decode_step" in selected:
        # ten untimed steps: the first replays of a fresh process run about 4 % slower
        extra["decode_step_b128"] = run_decode_step(max(10, steps // 2), 10)
        print(f"decode step: {extra['decode_step_b128']}", file=sys.stderr, flush=True)
    if "prefill" in selected:
        extra["prefill_2048"] = run_prefill(5)
        print(f"prefill: {extra['prefill_2048']}", file=sys.stderr, flush=True)
    if "serving" in selected:
        extra["serving"] = run_serving()
        print(f"serving: {extra['serving']}", file=sys.stderr, flush=True)
    return extra


def main() -> int:
    parser = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    parser.add_argument("--gpus", type=int, default=1)
    parser.add_argument("--steps", type=int, default=50)
    parser.add_argument("--warmup", type=int, default=5)
    parser.add_argument("--cpu-seconds", type=float, default=15.0)
    parser.add_argument("--no-cpu-baseline", action="store_true")
    parser.add_argument("--no-graph", action="store_true", help="launch from Python instead of replaying a HIP graph")
    parser.add_argument("--workloads", default="attention,single_decode,prompt_append,long_context,prefill,decode_step,serving",
                        help="comma list: attention (the headline; without it only the others run, as a diagnostic line), single_decode "
                        "(one 128-token sequence: call latency), prompt_append (2048-token prompt into a "
                        "fragmented pool), long_context (batch 256 x 2048, append + attention), prefill (one 2048-token "
                        "prompt through the model), decode_step (full TinyLlama-architecture step, batch 128), serving "
                        "(continuous batching of 128 requests)")
    parser.add_argument("--calibrate-copy-mib", type=int, default=0,
                        help="run one plain copy of this many MiB first (counter calibration under rocprofv3 --pmc)")
    args = parser.parse_args()
    if args.gpus != 1:
        print(
            f"bench.py measures one GPU: the paged decode path is per-GPU (sequences shard across "
            f"GPUs with no exchange), so --gpus {args.gpus} is not run",
            file=sys.stderr,
        )
        return 2

    torch.cuda.set_device(0)
    if args.calibrate_copy_mib > 0:
        calibration_copy(args.calibrate_copy_mib, torch.device("cuda:0"))
    selected = {name.strip() for name in args.workloads.split(",")}
    unknown = selected - {"attention", "single_decode", "prompt_append", "long_context", "prefill", "decode_step", "serving"}
    if unknown:
        print(f"unknown workloads {sorted(unknown)}", file=sys.stderr)
        return 2
    if "attention" not in selected:
        # Diagnostic run of the other workloads alone (e.g. to profile one of them); the
        # headline line needs the attention workload.
        extra = run_extra(selected, args.steps, 0.0 if args.no_cpu_baseline else EXTRA_CPU_SECONDS)
        print(json.dumps({"diagnostic": True, **extra}), flush=True)
        return 0
    r = run_decode(args.steps, args.warmup, use_graph=not args.no_graph)
    w, layers = r["w"], r["layers"]
    print(
        f"workload: batch {w.batch}, sum of lengths {int(w.lengths.sum())}, {r['bytes_per_launch'] / 1e6:.1f} MB per layer; "
        f"step {r['ms_per_step']:.3f} ms ({'graph' if r['graph'] else 'eager'}), {r['gbps']:.0f} GB/s, "
        f"{r['tokens_per_s']:.0f} tok/s; one attention call {r['launch_ms'] * 1e3:.1f} us ({r['launch_gbps']:.0f} GB/s)",
        file=sys.stderr,
        flush=True,
    )

    baseline = None
    if not args.no_cpu_baseline:
        baseline = cpu_baseline(layers, args.cpu_seconds)
        baseline["with_allocator_bookkeeping"] = cpu_bookkeeping_baseline(layers, EXTRA_CPU_SECONDS)
        print(f"cpu baseline: {baseline}", file=sys.stderr, flush=True)
    del layers, r["layers"]  # its memory stays cached for the next workloads (see run_extra)
    extra = run_extra(selected, args.steps, 0.0 if args.no_cpu_baseline else EXTRA_CPU_SECONDS)

    record = {
        "metric": "paged-decode attn HBM GB/s (% of ~8 TB/s peak) + decode tok/s, batch 64 ctx<=2048",
        "value": round(r["gbps"], 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(r["ms_per_step"], 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic",
        "config": {
            "workload": "batched one-token paged decode attention, batch 64, ctx U{1..2048}, 22 layers, "
            "32q/4kv heads, d64, fp16 KV, 8192-block pool",
            "batch": w.batch,
            "layers": LAYERS,
            "pool_blocks": w.num_blocks,
            "sum_context_tokens": int(w.lengths.sum()),
            "attention_bins": int(r["bins"]),
            "split_k_merge": "in_kernel (flags, same XCD)",
            "kv_dtype": "f16",
            "launch": "hip_graph" if r["graph"] else "eager",
        },
        "hbm_fraction": round(r["gbps"] / PEAK_HBM_GBPS, 4),
        "attention_only_decode_tokens_per_s": round(r["tokens_per_s"], 1),
        "step_ms_median": round(r["step_ms_median"], 4),
        "step_ms_min": round(r["step_ms_min"], 4),
        "step_ms_max": round(r["step_ms_max"], 4),
        "roofline": {
            "bound": "hbm",
            "kernel": "pc_paged_decode_attn: paged_decode_bin_kernel<false>",
            "achieved": round(r["launch_gbps"], 2),
            "peak": PEAK_HBM_GBPS,
            "unit": "GB/s",
            "frac": round(r["launch_gbps"] / PEAK_HBM_GBPS, 4),
            "traffic": measured_traffic(),
            "avg_call_us": round(r["launch_ms"] * 1e3, 3),
            "bytes_per_launch": r["bytes_per_launch"],
        },
        "cpu_baseline": baseline,
        **extra,
    }
    print(json.dumps(record), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
