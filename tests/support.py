"""Shared test helpers (not product code)."""

from __future__ import annotations

from typing import Optional, Sequence

import numpy as np
import torch
from torch import Tensor
from torch.multiprocessing.reductions import StorageWeakRef
from torch.utils._python_dispatch import TorchDispatchMode
from torch.utils._pytree import tree_leaves

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


ATOL = 2e-3  # max-abs bound on fp16 attention outputs; no relative term


def assert_max_abs(got, expected, what: str = "", atol: float = ATOL, rtol: float = 0.0) -> float:
    """max |got - expected| <= atol (elementwise, in float64); both must be finite. Returns
    the error. rtol > 0 is only for the reference's own cases with a bound tighter than
    2e-3 (atol + rtol * |expected| there, as its assert_close), and the 2e-3 max-abs bound
    holds as well."""
    got64 = got.detach().cpu().double()
    expected64 = expected.detach().cpu().double().reshape(got64.shape)
    assert torch.isfinite(got64).all(), f"{what}: non-finite output"
    assert torch.isfinite(expected64).all(), f"{what}: non-finite expectation"
    difference = (got64 - expected64).abs()
    error = difference.max().item() if got64.numel() else 0.0
    assert error <= ATOL, f"{what}: max |got - expected| = {error:.3e} > {ATOL:.1e}"
    excess = (difference - (atol + rtol * expected64.abs())).max().item() if got64.numel() else 0.0
    assert excess <= 0, f"{what}: max |got - expected| = {error:.3e} exceeds atol {atol:.1e} + rtol {rtol:.1e} * |expected|"
    return error


class PoolPageGuard(TorchDispatchMode):
    """Dispatch mode asserting that no torch op derives more than one KV page from the pool.

    The invariant of the reference's paged decode (a request's history is read page by page,
    never gathered into a dense buffer; reference tests/conftest.py:45-80 checks it the same
    way for its torch path). An op reads KV when one of its tensor inputs shares storage
    with the pool or with a tensor already derived from it; each tensor it returns must then
    be a view of the pool or live in a storage of at most one page of one kind (16 tokens x 4
    kv heads x 64 dims), whatever its own shape (a small view of a big buffer is the big
    buffer). Matrix products reduce K to scores and V to outputs, so their results are not
    tracked further. `kv_ops` counts the ops that read KV.
    """

    PAGE_ELEMENTS = 16 * 4 * 64
    REDUCTIONS = ("aten.mm", "aten.bmm", "aten.matmul", "aten.baddbmm", "aten.addmm")

    def __init__(self, pool: Tensor) -> None:
        super().__init__()
        self._pool = StorageWeakRef(pool.untyped_storage())
        self._derived = {self._pool}
        self.kv_ops = 0

    def __torch_dispatch__(self, func, types, args=(), kwargs=None):
        tensors_in = [t for t in tree_leaves((args, kwargs or {})) if isinstance(t, Tensor)]
        reads_kv = any(StorageWeakRef(t.untyped_storage()) in self._derived for t in tensors_in)
        result = func(*args, **(kwargs or {}))
        if reads_kv:
            self.kv_ops += 1
            reduces = str(func.overloadpacket) in self.REDUCTIONS
            for out in (t for t in tree_leaves(result) if isinstance(t, Tensor)):
                identity = StorageWeakRef(out.untyped_storage())
                if identity == self._pool:
                    continue  # a borrowed view of the pool
                limit = self.PAGE_ELEMENTS * out.element_size()
                assert out.untyped_storage().nbytes() <= limit, (
                    f"{func} derived {out.untyped_storage().nbytes()} bytes of KV history "
                    f"(shape {tuple(out.shape)}); one page is {limit} bytes"
                )
                if not reduces:
                    self._derived.add(identity)
        return result


# Attention workspace layout (include/pagedcore_hip.h): a 256-byte header whose first int32
# is the fault word, then partial slots of 2176 bytes with the part's ready flag at byte 2112.
WORKSPACE_HEADER, SLOT_BYTES, FLAG_OFFSET = 256, 2176, 2112


def workspace_flags(workspace: Tensor) -> Tensor:
    """The ready flag (int32) of every partial slot of an attention workspace."""
    slots = (workspace.numel() - WORKSPACE_HEADER) // SLOT_BYTES
    body = workspace[WORKSPACE_HEADER : WORKSPACE_HEADER + slots * SLOT_BYTES].view(slots, SLOT_BYTES)
    return body[:, FLAG_OFFSET : FLAG_OFFSET + 4].contiguous().view(torch.int32).reshape(slots)


def flags_clear(workspace: Tensor) -> bool:
    """Every partial slot's flag is zero: the state each call must leave for the next."""
    return not workspace_flags(workspace).any().item()


def fault_word(workspace: Tensor) -> int:
    """The workspace's fault word (synchronizes)."""
    return int(workspace[:4].view(torch.int32).item())


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
