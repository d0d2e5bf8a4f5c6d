"""CPU restatement of the reference paged KV path — test infrastructure only.

See oracle/__init__.py for scope and pinning. Everything here runs on the CPU with torch
or numpy; nothing touches the GPU.
"""

from __future__ import annotations

from dataclasses import dataclass, field
from typing import Dict, List, Sequence, Tuple

import numpy as np
import torch
from torch import Tensor

LAYERS = 22
BLOCK_TOKENS = 16
KV_HEADS = 4
Q_HEADS = 32
HEAD_DIM = 64
SCORE_BUFFER = 2048  # the reference's bounded [4, 8, 2048] fp32 score buffer

# fp16 NaN bit pattern that torch.full(..., nan, dtype=float16) writes.
NAN_F16_BITS = 0x7E00


# ---------------------------------------------------------------------------------------
# Attention
# ---------------------------------------------------------------------------------------


def pages_of(pool: Tensor, layer: int, blocks: Sequence[int], length: int) -> List[Tuple[Tensor, Tensor]]:
    """(K, V) views [valid, 4, 64] of each logical block, as the reference's
    KVAllocator.iter_layer_blocks yields them (kv_cache.py:264-270)."""
    pages = []
    for logical, physical in enumerate(blocks):
        valid = min(BLOCK_TOKENS, length - logical * BLOCK_TOKENS)
        pages.append((pool[layer, 0, physical, :valid], pool[layer, 1, physical, :valid]))
    return pages


def reference_paged_attention(query: Tensor, pool: Tensor, layer: int, blocks: Sequence[int], length: int) -> Tensor:
    """Default paged_attention of the reference, op for op (attention.py:31-53).

    query fp16 [1, 32, 1, 64]; pool fp16 CPU [22, 2, N, 16, 4, 64]. Scores are fp32
    matmuls of the grouped query against each page, scaled by 64**-0.5 (attention.py:41-43);
    one global fp32 softmax over all cached tokens (:46); a second page traversal
    accumulates fp32 probability-weighted values (:47-52); one final fp16 cast (:53).
    """
    if length < 1 or length > SCORE_BUFFER:
        raise ValueError("length must be in [1, 2048]")
    pages = pages_of(pool, layer, blocks, length)
    with torch.autocast(device_type="cpu", enabled=False):
        grouped = query.reshape(KV_HEADS, Q_HEADS // KV_HEADS, HEAD_DIM).float()
        scores = torch.empty((KV_HEADS, Q_HEADS // KV_HEADS, SCORE_BUFFER), dtype=torch.float32)
        filled = 0
        for key, _ in pages:
            stop = filled + key.shape[0]
            scores[..., filled:stop] = torch.matmul(grouped, key.permute(1, 2, 0).float()) * (HEAD_DIM**-0.5)
            filled = stop
        probabilities = scores[..., :filled].softmax(dim=-1)
        output = torch.zeros_like(grouped)
        start = 0
        for _, value in pages:
            stop = start + value.shape[0]
            output.add_(torch.matmul(probabilities[..., start:stop], value.transpose(0, 1).float()))
            start = stop
        return output.reshape(1, Q_HEADS, 1, HEAD_DIM).half()


def reference_paged_attention_batch(
    queries: Tensor, pool: Tensor, layer: int, tables: Sequence[Sequence[int]], lengths: Sequence[int]
) -> Tensor:
    """reference_paged_attention for each row of fp16 [B, 32, 1, 64] (the reference's
    decode loop calls it once per row, decoder.py:182-190)."""
    rows = [
        reference_paged_attention(queries[b : b + 1], pool, layer, tables[b], lengths[b])
        for b in range(queries.shape[0])
    ]
    return torch.cat(rows)


def dense_attention_fp64(query: Tensor, key: Tensor, value: Tensor) -> Tensor:
    """Independent full-history FP64 attention (the reference tests' oracle,
    tests/unit/test_attention.py:173-179 and tests/gpu/test_attention_cuda.py:83-90).

    query [1, 32, 1, 64] (or [32, 64]); key/value [tokens, 4, 64]. Returns float64
    [32, 64]; q head h reads kv head h // 8; scale 1/8; all tokens visible.
    """
    q = query.detach().cpu().double().reshape(Q_HEADS, HEAD_DIM)
    k = key.detach().cpu().double()
    v = value.detach().cpu().double()
    heads = []
    for head in range(Q_HEADS):
        scores = q[head] @ k[:, head // 8].T / 8
        heads.append(scores.softmax(dim=-1) @ v[:, head // 8])
    return torch.stack(heads)


def gather_history(pool: Tensor, layer: int, blocks: Sequence[int], length: int) -> Tuple[Tensor, Tensor]:
    """Contiguous K, V [length, 4, 64] of a paged sequence (oracle-side only)."""
    pages = pages_of(pool, layer, blocks, length)
    return torch.cat([k for k, _ in pages]), torch.cat([v for _, v in pages])


# ---------------------------------------------------------------------------------------
# Append
# ---------------------------------------------------------------------------------------


def slot_positions(blocks: Sequence[int], start: int, count: int) -> List[Tuple[int, int]]:
    """(physical block, slot) of positions start .. start+count-1 (kv_cache.py:163-165)."""
    out = []
    for position in range(start, start + count):
        logical, slot = divmod(position, BLOCK_TOKENS)
        out.append((blocks[logical], slot))
    return out


def reference_append(pool: np.ndarray, blocks: Sequence[int], start: int, key: np.ndarray, value: np.ndarray) -> None:
    """KVAllocator.append's writes (kv_cache.py:161-172), in its chunk order.

    pool: uint16 view [22, 2, N, 16, 4, 64]; key/value: uint16 [22, T, 4, 64] (raw fp16
    bits, so equality is bit-exact). Positions start .. start+T-1 go to
    pool[:, kind, blocks[p // 16], p % 16] in chunks that never cross a block.
    """
    tokens = key.shape[1]
    offset = 0
    while offset < tokens:
        logical, slot = divmod(start + offset, BLOCK_TOKENS)
        count = min(BLOCK_TOKENS - slot, tokens - offset)
        physical = blocks[logical]
        pool[:, 0, physical, slot : slot + count] = key[:, offset : offset + count]
        pool[:, 1, physical, slot : slot + count] = value[:, offset : offset + count]
        offset += count


def reference_write_decode(
    pool: np.ndarray, layer: int, blocks: Sequence[int], length: int, key: np.ndarray, value: np.ndarray
) -> None:
    """KVAllocator.write_decode_layer's writes (kv_cache.py:242-245): the staged token at
    position length-1 of layer `layer`; key/value uint16 [4, 64]."""
    logical, slot = divmod(length - 1, BLOCK_TOKENS)
    pool[layer, 0, blocks[logical], slot] = key
    pool[layer, 1, blocks[logical], slot] = value


def f16_bits(tensor: Tensor) -> np.ndarray:
    """Raw fp16 bits of a CPU tensor as uint16."""
    return tensor.detach().cpu().contiguous().view(torch.int16).numpy().view(np.uint16)


# ---------------------------------------------------------------------------------------
# Allocator bookkeeping
# ---------------------------------------------------------------------------------------


@dataclass(frozen=True)
class SequenceRecord:
    """One request's bookkeeping as the reference allocator keeps it: its reservation's
    request id and block credits, its cached length and its block table."""

    request_id: str
    credits: int
    length: int
    blocks: tuple


def reference_assert_accounting(
    sequences: Dict[str, SequenceRecord], free_blocks: List[int], block_owners: Dict[int, str], total_blocks: int
) -> Tuple[int, int, int, int, int, int]:
    """KVAllocator._assert_accounting (kv_cache.py:314-357), check for check and in the same
    order, with the same messages; returns CapacityCounts' fields (total, free, owned,
    reserved, active slots, live cached token slots). O(pool blocks) per call: it builds the
    full set of block ids each time, which is the reference's per-call host cost."""
    for request_id, sequence in sequences.items():
        if (
            sequence.request_id != request_id
            or type(sequence.length) is not int
            or not 0 <= sequence.length <= 2048
            or type(sequence.blocks) is not tuple
            or len(sequence.blocks) != (sequence.length + 15) // 16
            or not len(sequence.blocks) <= sequence.credits <= 128
        ):
            raise RuntimeError("corrupt KV block table or reservation")
    assigned = [block for sequence in sequences.values() for block in sequence.blocks]
    if any(type(block) is not int or not 0 <= block < total_blocks for block in free_blocks + assigned):
        raise RuntimeError("invalid physical KV block")
    owned = set(assigned)
    free = set(free_blocks)
    if len(assigned) != len(owned):
        raise RuntimeError("physical KV blocks must have unique owners")
    if len(free_blocks) != len(free):
        raise RuntimeError("free KV blocks must be unique")
    if not free.isdisjoint(owned):
        raise RuntimeError("owned KV blocks must not be free")
    if free | owned != set(range(total_blocks)):
        raise RuntimeError("KV blocks must cover the pool")
    owners = {block: request_id for request_id, sequence in sequences.items() for block in sequence.blocks}
    if owners != block_owners:
        raise RuntimeError("KV blocks are not owned by the recorded requests")
    return (
        total_blocks,
        len(free_blocks),
        len(assigned),
        sum(sequence.credits for sequence in sequences.values()),
        len(sequences),
        sum(sequence.length for sequence in sequences.values()),
    )


# ---------------------------------------------------------------------------------------
# Block choice
# ---------------------------------------------------------------------------------------


@dataclass
class LifoFreeList:
    """The reference allocator's free-list rules, restated (kv_cache.py:86,158,197-201,297).

    The list starts as [N-1, ..., 1, 0] so block 0 is handed out first; an append takes
    the last `k` entries in reverse (`reversed(free[-k:])`); a decode step borrows
    free[-1], free[-2], ... in request order and removes them on commit; a release pushes
    the request's blocks in reverse, so its first block is the next one handed out.
    """

    free: List[int]
    tables: Dict[str, List[int]] = field(default_factory=dict)

    @classmethod
    def fresh(cls, blocks: int) -> "LifoFreeList":
        return cls(list(reversed(range(blocks))))

    def take(self, request: str, count: int) -> List[int]:
        if count > len(self.free):
            raise RuntimeError("insufficient free blocks")
        new = list(reversed(self.free[-count:])) if count else []
        if count:
            del self.free[-count:]
        self.tables.setdefault(request, []).extend(new)
        return new

    def grow_to(self, request: str, tokens: int) -> List[int]:
        """Blocks newly needed for `request` to hold `tokens` positions."""
        have = len(self.tables.get(request, []))
        need = (tokens + BLOCK_TOKENS - 1) // BLOCK_TOKENS
        return self.take(request, max(0, need - have))

    def decode_step(self, lengths: Dict[str, int]) -> Dict[str, List[int]]:
        """One staged token per request (in dict order); returns each request's table."""
        borrowed = 0
        for request, length in lengths.items():
            if length % BLOCK_TOKENS == 0:
                borrowed += 1
                self.tables.setdefault(request, []).append(self.free[-borrowed])
        if borrowed:
            del self.free[-borrowed:]
        return {request: self.tables[request] for request in lengths}

    def release(self, request: str) -> None:
        blocks = self.tables.pop(request)
        self.free.extend(reversed(blocks))
