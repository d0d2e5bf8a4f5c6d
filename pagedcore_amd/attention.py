"""Block-table paged decode attention on the GPU.

``paged_attention`` is the reference's entry point (src/pagedcore/attention.py:14-53) with
the same signature, checks, error types and output contract: FP16 [1, 32, 1, 64], q head h
attends kv head h // 8, scores scaled by 1/8, fp32 softmax over every cached token of the
layer (staged decode tokens included once their layer is written), fp32 weighted sum,
one final fp16 rounding, autocast ignored. The two page traversals of the reference are
replaced by one launch of the HIP paged-attention kernels, which walk the block table on
the device; nothing larger than the output is materialised from the pool.

Both entry points fail closed on a device-side failure of the launch (a cut sequence's
merge that timed out or saw another XCD's flag, a block id outside the pool): they read
the workspace's fault word after the launch, which synchronizes, and raise
AttentionFaultError (a RuntimeError) instead of returning NaN rows.

``paged_attention_batch`` is the batched form the decode loop needs (one launch for all
rows of a layer). The reference's ``eager_rounding=True`` path replays HF fp16 rounding for
forensic comparisons; it is not part of the serving path and is rejected here.
"""

from __future__ import annotations

from typing import Sequence, Tuple

import torch
from torch import Tensor

from pagedcore_amd import _hip
from pagedcore_amd.engine_types import RequestId
from pagedcore_amd.kv_cache import LAYERS, KVAllocator

Q_HEADS = 32
HEAD_DIM = 64


def _check_layer(layer_index: int) -> None:
    if type(layer_index) is not int or not 0 <= layer_index < LAYERS:
        raise ValueError("layer_index must identify one of the 22 decoder layers")


def attend_rows(
    query: Tensor,
    allocator: KVAllocator,
    request_ids: Sequence[RequestId],
    layer_index: int,
) -> Tuple[Tensor, Tensor]:
    """One launch of paged attention for already validated rows; returns the output and
    the workspace whose fault word the caller must check (check_attention_faults) before
    it trusts the output. Nothing synchronizes."""
    tables, lengths = allocator.gather_block_tables(request_ids, layer_index=layer_index)
    pool = allocator.pool
    if pool.device != query.device:
        raise ValueError("query and KV cache must be on the same device")
    if not query.is_cuda:
        raise RuntimeError("paged attention runs on the GPU: the KV pool and query must be on a CUDA device")
    batch = len(request_ids)
    q = query.reshape(batch, Q_HEADS, HEAD_DIM)
    if not q.is_contiguous():
        q = q.contiguous()
    out = torch.empty((batch, Q_HEADS, 1, HEAD_DIM), dtype=torch.float16, device=query.device)
    plan = allocator.decode_plan(request_ids, layer_index=layer_index)
    workspace = _hip.paged_decode_attention(out, q, pool, layer_index, tables, lengths, plan=plan)
    return out, workspace


def _checked(query, allocator, request_ids, layer_index, where) -> Tensor:
    out, workspace = attend_rows(query, allocator, request_ids, layer_index)
    _hip.check_attention_faults(workspace, where)
    return out


@torch.inference_mode()
def paged_attention(
    query: Tensor,
    allocator: KVAllocator,
    request_id: RequestId,
    *,
    layer_index: int,
    eager_rounding: bool = False,
) -> Tensor:
    """Decode attention of one FP16 [1, 32, 1, 64] query over the request's cached pages."""
    if query.shape != (1, Q_HEADS, 1, HEAD_DIM) or query.dtype != torch.float16:
        raise ValueError("query must be FP16 [1, 32, 1, 64]")
    _check_layer(layer_index)
    if eager_rounding:
        raise ValueError("eager_rounding replays HF fp16 rounding and is not part of the GPU path")
    return _checked(query, allocator, (request_id,), layer_index, "paged_attention")


@torch.inference_mode()
def paged_attention_batch(
    query: Tensor,
    allocator: KVAllocator,
    request_ids: Sequence[RequestId],
    *,
    layer_index: int,
) -> Tensor:
    """Decode attention for FP16 [B, 32, 1, 64] queries; row b attends request_ids[b]."""
    batch = len(request_ids)
    if batch < 1 or query.shape != (batch, Q_HEADS, 1, HEAD_DIM) or query.dtype != torch.float16:
        raise ValueError("query must be FP16 [batch, 32, 1, 64] matching request IDs")
    if len(set(request_ids)) != batch:
        raise ValueError("attention requires distinct request IDs")
    _check_layer(layer_index)
    return _checked(query, allocator, tuple(request_ids), layer_index, "paged_attention_batch")
