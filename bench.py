"""Benchmark of the paged decode hot path on one MI355X.

Workload (the metric's configuration): batched one-token paged decode attention, batch 64,
32 query / 4 KV heads, head dim 64, fp16 KV with N(0,1) values, context lengths drawn
uniformly from 1..2048 (partial last blocks included), fragmented block tables carved from
a random permutation of an 8192-block pool, repeated over the pool's 22 layers. A step is
one pass over the 22 layers (partition kernel + split-K reduce per layer), with inputs
resident in HBM; the 22 layer planes (1.48 GB of KV per step) exceed the 256 MB Infinity
Cache, so the bytes come from HBM.

Printed as one JSON line: value = algorithmic HBM bytes per step x steps / wall time
(GB/s), plus decode tokens/s, the roofline of the partition kernel (per-launch HIP-event
timing), and the CPU baseline (the oracle's op-for-op restatement of the reference's
torch CPU path, timed on a bounded sample on this host's cores).

    python bench.py [--steps K] [--warmup W] [--gpus 1]
"""

from __future__ import annotations

import argparse
import ctypes
import json
import os
import sys
import time

import numpy as np
import torch

ROOT = os.path.dirname(os.path.abspath(__file__))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

from pagedcore_amd import _hip, workloads  # noqa: E402

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

    def __init__(self, w: workloads.BatchedDecode, device: torch.device, partition_blocks: int, seed: int) -> None:
        gen = torch.Generator(device=device).manual_seed(seed)
        self.w = w
        self.device = device
        self.pool = torch.randn((LAYERS, 2, w.num_blocks, 16, 4, 64), dtype=torch.float16, device=device, generator=gen)
        self.queries = torch.randn((LAYERS, w.batch, 32, 64), dtype=torch.float16, device=device, generator=gen)
        self.out = torch.empty_like(self.queries)
        self.tables = torch.from_numpy(w.tables).to(device)
        self.lens = torch.from_numpy(w.lengths).to(device)
        self.parts = partition_blocks
        self.lib = _hip.load()
        max_blocks = int(w.tables.shape[1])
        floats = int(self.lib.pc_attn_workspace_floats(w.batch, max_blocks, partition_blocks))
        self.workspace = torch.empty(floats, dtype=torch.float32, device=device)
        max_parts = (max_blocks + partition_blocks - 1) // partition_blocks
        self.ws_out = self.workspace.data_ptr()
        self.ws_ml = self.ws_out + w.batch * 32 * max_parts * 64 * 4
        self.max_blocks = max_blocks

    def _args(self, layer: int, stream: int):
        return (
            self.out[layer].data_ptr(), self.queries[layer].data_ptr(), self.pool.data_ptr(), self.w.num_blocks,
            layer, self.tables.data_ptr(), self.max_blocks, self.lens.data_ptr(), self.w.batch, self.parts,
            self.ws_out, self.ws_ml, stream,
        )

    def step(self) -> None:
        stream = torch.cuda.current_stream(self.device).cuda_stream
        for layer in range(LAYERS):
            status = self.lib.pc_paged_decode_attn(*self._args(layer, stream))
            if status:
                raise RuntimeError(self.lib.pc_last_error().decode())

    def timed_kernels(self, steps: int) -> tuple[float, float]:
        """Mean duration (ms) of the partition kernel and of the reduce kernel, from HIP
        events recorded around each launch on the launch stream."""
        stream = torch.cuda.current_stream(self.device)
        handle = stream.cuda_stream
        part_ms, red_ms = [], []
        for _ in range(steps):
            marks = []
            for layer in range(LAYERS):
                e0, e1, e2 = (torch.cuda.Event(enable_timing=True) for _ in range(3))
                e0.record(stream)
                self.lib.pc_paged_decode_attn_partitions(*self._args(layer, handle))
                e1.record(stream)
                self.lib.pc_paged_decode_attn_reduce(
                    self.out[layer].data_ptr(), self.lens.data_ptr(), self.w.batch, self.max_blocks, self.parts,
                    self.ws_out, self.ws_ml, handle,
                )
                e2.record(stream)
                marks.append((e0, e1, e2))
            torch.cuda.synchronize(self.device)
            for e0, e1, e2 in marks:
                part_ms.append(e0.elapsed_time(e1))
                red_ms.append(e1.elapsed_time(e2))
        return float(np.mean(part_ms)), float(np.mean(red_ms))


def cpu_baseline(layers: DecodeLayers, seconds: float) -> dict:
    """The oracle's restatement of the reference torch CPU path (attention.py:14-53), run
    row by row on layer 0 until ~`seconds` of CPU work, on all of this host's cores."""
    from oracle import paged_reference as ref

    cores = len(os.sched_getaffinity(0))
    torch.set_num_threads(cores)
    w = layers.w
    layer = 0
    done_bytes, done_rows, elapsed = 0, 0, 0.0
    order = np.random.Generator(np.random.PCG64(5)).permutation(w.batch)
    for b in order:
        length = int(w.lengths[b])
        table = w.tables[b, : (length + 15) // 16]
        blocks = torch.from_numpy(table.astype(np.int64)).to(layers.device)
        sub = torch.empty((LAYERS, 2, len(table), 16, 4, 64), dtype=torch.float16)
        sub[layer] = layers.pool[layer].index_select(1, blocks).cpu()
        query = layers.queries[layer, b].reshape(1, 32, 1, 64).cpu()
        start = time.perf_counter()
        ref.reference_paged_attention(query, sub, layer, list(range(len(table))), length)
        elapsed += time.perf_counter() - start
        done_bytes += attention_bytes(np.array([length], dtype=np.int32))
        done_rows += 1
        if elapsed >= seconds:
            break
    return {
        "value": round(done_bytes / elapsed / 1e9, 4),
        "unit": "GB/s",
        "cores": cores,
        "kind": "port",
        "sample": f"{done_rows} of {w.batch} sequences of layer 0 (sum of lengths "
        f"{int(sum(int(w.lengths[b]) for b in order[:done_rows]))} tokens), one reference paged_attention call each, "
        f"{elapsed:.1f} s; tok/s equivalent {done_rows / elapsed / LAYERS:.2f}",
    }


def main() -> int:
    parser = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    parser.add_argument("--gpus", type=int, default=1)
    parser.add_argument("--steps", type=int, default=50)
    parser.add_argument("--warmup", type=int, default=5)
    parser.add_argument("--partition-blocks", type=int, default=None)
    parser.add_argument("--cpu-seconds", type=float, default=15.0)
    parser.add_argument("--no-cpu-baseline", action="store_true")
    parser.add_argument("--no-graph", action="store_true", help="launch from Python instead of replaying a HIP graph")
    args = parser.parse_args()
    if args.gpus != 1:
        print(
            f"bench.py measures one GPU: the paged decode path is per-GPU (sequences shard across "
            f"GPUs with no exchange), so --gpus {args.gpus} is not run",
            file=sys.stderr,
        )
        return 2

    device = torch.device("cuda:0")
    torch.cuda.set_device(device)
    parts = args.partition_blocks or _hip.default_partition_blocks()
    w = workloads.batched_decode(batch=64, num_blocks=8192)
    layers = DecodeLayers(w, device, parts, seed=1234)
    bytes_per_launch = attention_bytes(w.lengths)
    bytes_per_step = bytes_per_launch * LAYERS
    print(f"workload: batch {w.batch}, sum of lengths {int(w.lengths.sum())}, {bytes_per_launch / 1e6:.1f} MB per layer", file=sys.stderr, flush=True)

    for _ in range(args.warmup):
        layers.step()
    torch.cuda.synchronize(device)
    eager_out = layers.out.clone()

    use_graph = not args.no_graph
    replay = layers.step
    if use_graph:
        side = torch.cuda.Stream(device=device)
        side.wait_stream(torch.cuda.current_stream(device))
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.stream(side):
            with torch.cuda.graph(graph, stream=side):
                layers.step()
        torch.cuda.current_stream(device).wait_stream(side)
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
    for _ in range(args.steps):
        replay()
    stop.record()
    torch.cuda.synchronize(device)
    total_ms = start.elapsed_time(stop)
    if not torch.equal(layers.out, eager_out):
        raise RuntimeError("timed steps produced different outputs than the warmup")
    ms_per_step = total_ms / args.steps
    gbps = bytes_per_step * args.steps / (total_ms / 1e3) / 1e9
    tokens_per_s = w.batch * args.steps / (total_ms / 1e3)

    part_ms, red_ms = layers.timed_kernels(steps=5)
    achieved = bytes_per_launch / (part_ms / 1e3) / 1e9
    print(
        f"step {ms_per_step:.3f} ms ({'graph' if use_graph else 'eager'}), {gbps:.0f} GB/s, {tokens_per_s:.0f} tok/s; "
        f"partition kernel {part_ms * 1e3:.1f} us ({achieved:.0f} GB/s), reduce {red_ms * 1e3:.1f} us",
        file=sys.stderr,
        flush=True,
    )

    baseline = None
    if not args.no_cpu_baseline:
        baseline = cpu_baseline(layers, args.cpu_seconds)

    record = {
        "metric": "paged-decode attn HBM GB/s (% of ~8 TB/s peak) + decode tok/s, batch 64 ctx<=2048",
        "value": round(gbps, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 4),
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
            "partition_blocks": parts,
            "kv_dtype": "f16",
            "launch": "hip_graph" if use_graph else "eager",
        },
        "hbm_fraction": round(gbps / PEAK_HBM_GBPS, 4),
        "decode_tokens_per_s": round(tokens_per_s, 1),
        "roofline": {
            "bound": "hbm",
            "kernel": "paged_decode_partition_kernel",
            "achieved": round(achieved, 2),
            "peak": PEAK_HBM_GBPS,
            "unit": "GB/s",
            "frac": round(achieved / PEAK_HBM_GBPS, 4),
            "traffic": None,
            "avg_launch_us": round(part_ms * 1e3, 3),
            "bytes_per_launch": bytes_per_launch,
            "reduce_avg_launch_us": round(red_ms * 1e3, 3),
        },
        "cpu_baseline": baseline,
    }
    print(json.dumps(record), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
