"""The KV pool and allocator on the MI355X: the reference's GPU storage spec
(tests/gpu/test_kv_pool_cuda.py:11-93) re-expressed for gfx950. A real allocate_kv_pool
with its layout; pointer stability and no hidden device allocation across writes, appends
and reads; an append that fails after validation publishes nothing; stream ownership."""

from __future__ import annotations

import pytest
import torch

from pagedcore_amd import kv_cache
from pagedcore_amd.config import PagedCoreConfig
from pagedcore_amd.engine_types import CapacityCounts, KVReservation, RequestId
from pagedcore_amd.kv_cache import KVAllocator, allocate_kv_pool

pytestmark = pytest.mark.gpu


def _require_gfx950(device):
    name = torch.cuda.get_device_properties(device).gcnArchName
    assert name.startswith("gfx950"), f"requires an MI355X (gfx950), found {name}"


def test_kv_pool_storage_on_gfx950(device):
    """tests/gpu/test_kv_pool_cuda.py:11-34: 1 MiB holds two whole 352 KiB blocks."""
    _require_gfx950(device)
    pool = allocate_kv_pool(PagedCoreConfig(kv_pool_mib=1))
    assert pool.shape == (22, 2, 2, 16, 4, 64)
    assert pool.dtype == torch.float16
    assert pool.device == torch.device("cuda:0")
    assert pool.is_contiguous()
    assert not pool.requires_grad
    pointer = pool.untyped_storage().data_ptr()
    allocated = torch.cuda.memory_allocated(0)
    for slot in range(16):
        pool[:, 0, 0, slot].fill_(slot)
        pool[:, 1, 1, slot].fill_(slot + 16)
    torch.cuda.synchronize(0)
    assert pool.untyped_storage().data_ptr() == pointer
    assert torch.cuda.memory_allocated(0) == allocated
    assert torch.all(pool[:, 0, 0, 15] == 15).item()
    assert torch.all(pool[:, 1, 1, 0] == 16).item()
    assert torch.all(pool[:, 1, 1, 15] == 31).item()


def test_kv_pool_sizes_whole_blocks_and_checks_the_margin(device):
    """The configured MiB round down to whole blocks; a pool plus margin beyond free
    memory is refused before anything is allocated."""
    _require_gfx950(device)
    pool = allocate_kv_pool(PagedCoreConfig(kv_pool_mib=100, workspace_margin_mib=1))
    assert pool.shape[2] == 100 * 2**20 // (22 * 2 * 16 * 4 * 64 * 2) == 290
    del pool
    free, total = torch.cuda.mem_get_info(device)
    allocated = torch.cuda.memory_allocated(0)
    too_big = PagedCoreConfig(kv_pool_mib=total // 2**20 + 1, workspace_margin_mib=1)
    with pytest.raises(RuntimeError, match="do not fit in GPU memory"):
        allocate_kv_pool(too_big)
    assert torch.cuda.memory_allocated(0) == allocated
    with pytest.raises(ValueError, match="CUDA device"):
        allocate_kv_pool(PagedCoreConfig(kv_pool_mib=1), device="cpu")


def test_kv_allocator_storage_and_stream_ownership_on_gfx950(device, monkeypatch):
    """tests/gpu/test_kv_pool_cuda.py:37-93 on the HIP path: a failed append (the write is
    the single pc_kv_append launch; the failure is injected there) leaves counts, length
    and table unchanged; the retried append lands; read_block views share the pool's
    storage; no call allocates device memory; another stream is refused everywhere."""
    _require_gfx950(device)
    pool = allocate_kv_pool(PagedCoreConfig(kv_pool_mib=1))
    allocator = KVAllocator(pool)
    a, b = RequestId("a"), RequestId("b")
    key = torch.arange(17, dtype=torch.float16, device=device)[None, :, None, None].expand(22, 17, 4, 64)
    value = -key - 1
    other_stream = torch.cuda.Stream(device=pool.device)
    pointer = pool.untyped_storage().data_ptr()

    allocator.create(KVReservation(a, 2))
    assert allocator.capacity() == CapacityCounts(2, 2, 0, 2, 1, 0)
    allocator.append(a, key[:, :16], value[:, :16])
    torch.cuda.synchronize(device)
    allocated = torch.cuda.memory_allocated(0)
    before = allocator.capacity()
    original = kv_cache._hip.kv_append

    def failing(*args, **kwargs):
        raise RuntimeError("injected copy failure")

    with monkeypatch.context() as patch:
        patch.setattr(kv_cache._hip, "kv_append", failing)
        with pytest.raises(RuntimeError, match="injected copy failure"):
            allocator.append(a, key[:, 16:], value[:, 16:])
    assert kv_cache._hip.kv_append is original
    assert allocator.capacity() == before
    assert allocator.cached_length(a) == 16
    assert len(allocator.block_table(a)) == 1
    allocator.append(a, key[:, 16:], value[:, 16:])
    assert allocator.cached_length(a) == 17
    assert len(allocator.block_table(a)) == 2
    assert allocator.capacity() == CapacityCounts(2, 0, 2, 2, 1, 17)
    actual_key, actual_value = allocator.read_block(a, 1)
    assert actual_key.shape == actual_value.shape == (22, 1, 4, 64)
    assert actual_key.untyped_storage().data_ptr() == pointer
    assert actual_value.untyped_storage().data_ptr() == pointer
    torch.testing.assert_close(actual_key, key[:, 16:], atol=0, rtol=0)
    torch.testing.assert_close(actual_value, value[:, 16:], atol=0, rtol=0)

    with torch.cuda.stream(other_stream):
        for operation in (
            allocator.capacity,
            lambda: allocator.append(a, key[:, :1], value[:, :1]),
            lambda: allocator.read_block(a, 0),
            lambda: allocator.release_all(a),
        ):
            with pytest.raises(RuntimeError, match="owning CUDA stream"):
                operation()

    allocator.release_all(a)
    assert allocator.capacity() == CapacityCounts(2, 2, 0, 0, 0, 0)
    with pytest.raises(KeyError):
        allocator.release_all(a)
    assert allocator.capacity() == CapacityCounts(2, 2, 0, 0, 0, 0)
    allocator.create(KVReservation(b, 1))
    allocator.append(b, key[:, :1], value[:, :1])
    actual_key, actual_value = allocator.read_block(b, 0)
    assert actual_key.shape == actual_value.shape == (22, 1, 4, 64)
    assert pool.untyped_storage().data_ptr() == pointer
    torch.testing.assert_close(actual_key, key[:, :1], atol=0, rtol=0)
    torch.testing.assert_close(actual_value, value[:, :1], atol=0, rtol=0)
    allocator.release_all(b)
    assert allocator.capacity() == CapacityCounts(2, 2, 0, 0, 0, 0)
    torch.cuda.synchronize(device)
    # nothing stays allocated on the device (each append's slot mapping is a temporary)
    assert torch.cuda.memory_allocated(0) == allocated
