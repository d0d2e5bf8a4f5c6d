"""Seeded synthetic inputs in the shapes the hot path is measured on.

No product logic lives here: these builders only produce query/KV values, context lengths
and block tables (numpy PCG64 streams, so every run and machine regenerates the same
bytes) for the tests, the golden-fixture script and bench.py.

  single_decode   one 128-token sequence, one layer, 8-entry random table of a 64-block pool
  prompt_append   one 2048-token prompt x 22 layers into a 4096-block pool, 30% of it
                  pre-occupied by filler requests, free list in seeded random order
  batched_decode  B sequences, lengths U{lo..hi}, fragmented tables carved from one
                  random permutation of the pool's blocks
"""

from __future__ import annotations

from dataclasses import dataclass
from typing import List

import numpy as np

LAYERS = 22
BLOCK_TOKENS = 16
KV_HEADS = 4
Q_HEADS = 32
HEAD_DIM = 64


def rng(seed: int) -> np.random.Generator:
    return np.random.Generator(np.random.PCG64(seed))


def normal_f16(gen: np.random.Generator, shape) -> np.ndarray:
    """N(0, 1) values rounded to fp16."""
    return gen.standard_normal(size=shape, dtype=np.float32).astype(np.float16)


@dataclass
class SingleDecode:
    query: np.ndarray  # fp16 [1, 32, 1, 64]
    key: np.ndarray  # fp16 [128, 4, 64]
    value: np.ndarray
    table: List[int]  # 8 physical blocks
    layer: int
    num_blocks: int


def single_decode(seed: int = 20261201) -> SingleDecode:
    gen = rng(seed)
    query = normal_f16(gen, (1, Q_HEADS, 1, HEAD_DIM))
    key = normal_f16(gen, (128, KV_HEADS, HEAD_DIM))
    value = normal_f16(gen, (128, KV_HEADS, HEAD_DIM))
    table = gen.permutation(64)[:8].tolist()
    return SingleDecode(query, key, value, [int(b) for b in table], layer=13, num_blocks=64)


@dataclass
class PromptAppend:
    num_blocks: int
    free_order: List[int]  # the allocator's free list (last entry is handed out first)
    filler_blocks: List[int]  # blocks owned by each filler request
    prompt_tokens: int
    seed: int

    def filler_kv(self, index: int) -> tuple[np.ndarray, np.ndarray]:
        tokens = self.filler_blocks[index] * BLOCK_TOKENS
        key = np.full((LAYERS, tokens, KV_HEADS, HEAD_DIM), index + 1, dtype=np.float16)
        return key, -key

    def prompt_kv(self) -> tuple[np.ndarray, np.ndarray]:
        gen = rng(self.seed + 1)
        shape = (LAYERS, self.prompt_tokens, KV_HEADS, HEAD_DIM)
        return normal_f16(gen, shape), normal_f16(gen, shape)


def prompt_append(seed: int = 20261202, num_blocks: int = 4096, occupied_fraction: float = 0.3) -> PromptAppend:
    gen = rng(seed)
    free_order = [int(b) for b in gen.permutation(num_blocks)]
    occupied = int(round(num_blocks * occupied_fraction))
    fillers = 10
    sizes = [occupied // fillers + (1 if i < occupied % fillers else 0) for i in range(fillers)]
    return PromptAppend(num_blocks, free_order, sizes, 2048, seed)


@dataclass
class BatchedDecode:
    lengths: np.ndarray  # int32 [B]
    tables: np.ndarray  # int32 [B, max_blocks], unused entries 0
    num_blocks: int
    seed: int

    @property
    def batch(self) -> int:
        return int(self.lengths.shape[0])

    def queries(self, layer: int) -> np.ndarray:
        """fp16 [B, 32, 64] N(0, 1) queries of one layer."""
        return normal_f16(rng(self.seed * 1000 + 7 + layer), (self.batch, Q_HEADS, HEAD_DIM))


def batched_decode(
    batch: int = 64,
    lo: int = 1,
    hi: int = 2048,
    num_blocks: int = 8192,
    seed: int = 20261203,
    fixed_length: int | None = None,
) -> BatchedDecode:
    """Lengths U{lo..hi} (or all `fixed_length`); sequence b's table is the next
    ceil(L_b/16) entries of one random permutation of the pool's blocks."""
    gen = rng(seed)
    if fixed_length is not None:
        lengths = np.full(batch, fixed_length, dtype=np.int32)
    else:
        lengths = gen.integers(lo, hi + 1, size=batch, dtype=np.int32)
    need = (lengths + BLOCK_TOKENS - 1) // BLOCK_TOKENS
    if int(need.sum()) > num_blocks:
        raise ValueError("pool too small for the batch")
    perm = gen.permutation(num_blocks).astype(np.int32)
    width = int(need.max())
    tables = np.zeros((batch, width), dtype=np.int32)
    offset = 0
    for b in range(batch):
        tables[b, : need[b]] = perm[offset : offset + need[b]]
        offset += int(need[b])
    return BatchedDecode(lengths, tables, num_blocks, seed)
