"""Shared test helpers (not product code)."""

from __future__ import annotations

from typing import Optional, Sequence

import numpy as np
import torch
from torch import Tensor

from pagedcore_amd.engine_types import KVReservation, RequestId
from pagedcore_amd.kv_cache import KVAllocator


class CpuCopyWriter:
    """Test double for the allocator's KV writer on CPU pools.

    Performs the same pool writes as the HIP kernel with tensor indexing, and can fail on
    its N-th call to exercise the allocator's rollback (the GPU path's single launch per
    call makes "fail at call N" the natural injection point).
    """

    def __init__(self, fail_at: Optional[int] = None) -> None:
        self.calls = 0
        self.fail_at = fail_at

    def append(self, pool: Tensor, layer_begin: int, key: Tensor, value: Tensor, slots: Sequence[int]) -> None:
        self.calls += 1
        if self.fail_at is not None and self.calls == self.fail_at:
            raise RuntimeError("injected copy failure")
        slots = torch.as_tensor(np.asarray(slots, dtype=np.int64))
        blocks, offsets = slots // 16, slots % 16
        layers = slice(layer_begin, layer_begin + key.shape[0])
        pool[layers, 0, blocks, offsets] = key
        pool[layers, 1, blocks, offsets] = value

    def rope_append(self, *args) -> None:
        raise RuntimeError("the CPU test writer does not rotate")


def cpu_allocator(pool: Tensor, writer: Optional[CpuCopyWriter] = None) -> KVAllocator:
    return KVAllocator(pool, kv_writer=writer if writer is not None else CpuCopyWriter())


def kv_values(tokens: int, start: int = 0, device: str | torch.device = "cpu") -> tuple[Tensor, Tensor]:
    """Distinct, exactly representable K/V [22, tokens, 4, 64] (V = -K - 1)."""
    key = torch.arange(22 * tokens * 4 * 64, dtype=torch.float32).reshape(22, tokens, 4, 64)
    key = (key / 256 + start).half().to(device)
    return key, -key - 1


def cached(allocator: KVAllocator, key: Tensor, value: Tensor, name: str = "attention") -> RequestId:
    """Create a request holding exactly key/value's tokens."""
    request = RequestId(name)
    allocator.create(KVReservation(request, (key.shape[1] + 15) // 16))
    allocator.append(request, key, value)
    return request


def fragmented_decode_cache(
    device: torch.device, batch: int, lengths: "np.ndarray", spare_tokens: int, seed: int
) -> tuple[KVAllocator, tuple[RequestId, ...]]:
    """The decode-step workload's cache: `batch` requests holding `lengths` tokens of N(0, 1)
    K/V in a pool sized to their blocks plus `spare_tokens` more positions each (and 256
    free blocks), filled by appends of up to 256 tokens with the requests in a fresh random
    order each round, so every request's blocks interleave with the others'."""
    rng = np.random.default_rng(seed)
    need = int(((lengths + spare_tokens + 15) // 16).sum())
    pool = torch.empty((22, 2, need + 256, 16, 4, 64), dtype=torch.float16, device=device)
    allocator = KVAllocator(pool)
    requests = tuple(RequestId(f"seq{i}") for i in range(batch))
    for request, length in zip(requests, lengths):
        allocator.create(KVReservation(request, min(128, int((length + spare_tokens + 15) // 16))))
    gen = torch.Generator(device=device).manual_seed(seed)
    filled = np.zeros(batch, dtype=np.int64)
    while (filled < lengths).any():
        for row in rng.permutation(batch):
            count = int(min(256, lengths[row] - filled[row]))
            if count > 0:
                key = torch.randn((22, count, 4, 64), dtype=torch.float16, device=device, generator=gen)
                value = torch.randn((22, count, 4, 64), dtype=torch.float16, device=device, generator=gen)
                allocator.append(requests[row], key, value)
                filled[row] += count
    return allocator, requests
