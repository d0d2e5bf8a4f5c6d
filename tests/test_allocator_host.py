"""Allocator host logic on CPU pools (no GPU): block choice, accounting, reservations,
staged decode, ownership, corruption detection and rollback.

Re-expresses the reference's allocator tests (tests/unit/test_kv_cache.py,
tests/unit/test_kv_cache_properties.py) against this package. CPU pools move bytes with
the CpuCopyWriter test double; the GPU tests repeat the data checks on the HIP path.
"""

from __future__ import annotations

from concurrent.futures import ThreadPoolExecutor
from contextlib import nullcontext
from dataclasses import replace
from math import ceil
from typing import Any
from unittest.mock import Mock

import numpy as np
import pytest
import torch
from hypothesis import settings
from hypothesis import strategies as st
from hypothesis.stateful import RuleBasedStateMachine, invariant, precondition, rule, run_state_machine_as_test

from oracle import paged_reference as ref
from pagedcore_amd.config import PagedCoreConfig
from pagedcore_amd.engine_types import CapacityCounts, KVReservation, RequestId
from pagedcore_amd.kv_cache import LAYERS, KVAllocator, allocate_kv_pool
from tests.support import CpuCopyWriter, cpu_allocator, kv_values


@pytest.fixture
def cuda_memory(monkeypatch: pytest.MonkeyPatch) -> Mock:
    monkeypatch.setattr(torch.cuda, "is_available", lambda: True)
    memory = Mock(return_value=(16 * 2**30, 16 * 2**30))
    monkeypatch.setattr(torch.cuda, "mem_get_info", memory)
    return memory


# --- pool allocation (reference tests/unit/test_kv_cache.py:24-124) -----------------------


@pytest.mark.parametrize("pool_mib", [1, 8192])
def test_pool_uses_one_fp16_allocation_with_whole_blocks(monkeypatch, cuda_memory, pool_mib):
    empty = torch.empty
    allocation = Mock(side_effect=lambda shape, **kwargs: empty(shape, dtype=kwargs["dtype"], device="meta"))
    monkeypatch.setattr(torch, "empty", allocation)
    pool = allocate_kv_pool(PagedCoreConfig(kv_pool_mib=pool_mib))
    blocks = 2 if pool_mib == 1 else 23831
    allocation.assert_called_once_with((22, 2, blocks, 16, 4, 64), dtype=torch.float16, device=torch.device("cuda:0"))
    assert pool.shape == (22, 2, blocks, 16, 4, 64) and pool.is_contiguous()
    used = pool.numel() * pool.element_size()
    assert used <= pool_mib * 2**20 < used + 352 * 1024
    assert cuda_memory.call_count == 2


@pytest.mark.parametrize("device", ["cpu", "meta"])
def test_pool_rejects_non_cuda_devices(monkeypatch, device):
    allocation = Mock()
    monkeypatch.setattr(torch, "empty", allocation)
    with pytest.raises(ValueError, match="requires a CUDA device"):
        allocate_kv_pool(PagedCoreConfig(), device=device)
    allocation.assert_not_called()


def test_pool_rejects_unavailable_runtime(monkeypatch):
    monkeypatch.setattr(torch.cuda, "is_available", lambda: False)
    with pytest.raises(RuntimeError, match="available CUDA runtime"):
        allocate_kv_pool(PagedCoreConfig())


def test_pool_memory_checks_before_and_after(monkeypatch, cuda_memory):
    config = PagedCoreConfig(kv_pool_mib=1, workspace_margin_mib=1)
    cuda_memory.return_value = (2 * 2**20 - 1, 16 * 2**30)
    allocation = Mock(return_value=torch.empty(0))
    monkeypatch.setattr(torch, "empty", allocation)
    with pytest.raises(RuntimeError, match="do not fit"):
        allocate_kv_pool(config)
    allocation.assert_not_called()
    cuda_memory.side_effect = [(2 * 2**20, 16 * 2**30), (2**20 - 1, 16 * 2**30)]
    with pytest.raises(RuntimeError, match="leaves less than"):
        allocate_kv_pool(config)
    allocation.assert_called_once()


@pytest.mark.parametrize("invalid", ["shape", "dtype", "empty", "strides", "grad"])
def test_allocator_rejects_incompatible_pool_storage(invalid):
    pool = torch.empty((22, 2, 1, 16, 4, 64), dtype=torch.float16)
    if invalid == "shape":
        pool = pool[:1]
    elif invalid == "dtype":
        pool = pool.float()
    elif invalid == "empty":
        pool = pool[:, :, :0]
    elif invalid == "strides":
        pool = torch.empty((22, 2, 1, 16, 4, 128), dtype=torch.float16)[..., ::2]
    else:
        pool.requires_grad_(True)
    with pytest.raises(ValueError, match="KV pool must be contiguous FP16"):
        KVAllocator(pool, kv_writer=CpuCopyWriter())


# --- block choice and token mapping --------------------------------------------------------


@pytest.mark.parametrize("tokens,blocks,last_slots", [(1, 1, 1), (15, 1, 15), (16, 1, 16), (17, 2, 1), (32, 2, 16), (33, 3, 1)])
def test_maps_tokens_and_limits_reads_to_valid_slots(tokens, blocks, last_slots):
    pool = torch.full((22, 2, 4, 16, 4, 64), torch.nan, dtype=torch.float16)
    allocator = cpu_allocator(pool)
    request = RequestId("a")
    allocator.create(KVReservation(request, blocks))
    assert allocator.block_table(request) == () and allocator.cached_length(request) == 0
    key, value = kv_values(tokens)
    allocator.append(request, key, value)
    table = allocator.block_table(request)
    assert len(table) == blocks and allocator.cached_length(request) == tokens
    for index, physical in enumerate(table):
        slots = last_slots if index == blocks - 1 else 16
        actual_key, actual_value = allocator.read_block(request, index)
        assert actual_key.shape == (22, slots, 4, 64)
        assert actual_key.untyped_storage().data_ptr() == pool.untyped_storage().data_ptr()
        expected = slice(index * 16, index * 16 + slots)
        assert torch.equal(actual_key, key[:, expected]) and torch.equal(actual_value, value[:, expected])
        if slots < 16:
            assert torch.isnan(pool[:, :, physical, slots:]).all()


def test_fragmented_appends_follow_the_lifo_tables():
    allocator = cpu_allocator(torch.full((22, 2, 4, 16, 4, 64), torch.nan, dtype=torch.float16))
    a, b = RequestId("a"), RequestId("b")
    allocator.create(KVReservation(a, 3))
    allocator.create(KVReservation(b, 1))
    key, value = kv_values(33)
    allocator.append(a, key[:, :15], value[:, :15])
    first = allocator.block_table(a)
    allocator.append(b, *kv_values(16, start=2000))
    allocator.append(a, key[:, 15:16], value[:, 15:16])
    assert allocator.block_table(a) == first
    allocator.append(a, key[:, 16:17], value[:, 16:17])
    assert allocator.read_block(a, 1)[0].shape[1] == 1
    allocator.append(a, key[:, 17:], value[:, 17:])
    assert allocator.block_table(a) == (0, 2, 3) and allocator.block_table(b) == (1,)
    for index, expected in enumerate((slice(0, 16), slice(16, 32), slice(32, 33))):
        assert torch.equal(allocator.read_block(a, index)[0], key[:, expected])


def test_release_reuses_the_released_first_block():
    allocator = cpu_allocator(torch.empty((22, 2, 6, 16, 4, 64), dtype=torch.float16))
    for name in ("released_first", "retained", "released_last"):
        request = RequestId(name)
        allocator.create(KVReservation(request, 1))
        allocator.append(request, *kv_values(16))
    allocator.release_all(RequestId("released_first"))
    allocator.release_all(RequestId("released_last"))
    prompt = RequestId("prompt")
    allocator.create(KVReservation(prompt, 4))
    allocator.append(prompt, *kv_values(49))
    assert allocator.block_table(prompt) == (2, 0, 3, 4)  # reference tests/unit/test_decoder.py:465


def test_reservation_limit_preserves_history():
    allocator = cpu_allocator(torch.empty((22, 2, 2, 16, 4, 64), dtype=torch.float16))
    a, b = RequestId("a"), RequestId("b")
    allocator.create(KVReservation(a, 1))
    allocator.create(KVReservation(b, 1))
    key, value = kv_values(17)
    allocator.append(a, key[:, :15], value[:, :15])
    allocator.append(b, *kv_values(16))
    before = allocator.capacity()
    with pytest.raises(RuntimeError, match="exceeds request reservation"):
        allocator.append(a, key[:, 15:], value[:, 15:])
    assert allocator.capacity() == before and allocator.cached_length(a) == 15
    allocator.append(a, key[:, 15:16], value[:, 15:16])
    allocator.release_all(b)
    with pytest.raises(RuntimeError, match="exceeds request reservation"):
        allocator.append(a, key[:, 16:], value[:, 16:])


def test_duplicate_registration_and_empty_release():
    allocator = cpu_allocator(torch.empty((22, 2, 1, 16, 4, 64), dtype=torch.float16))
    request = RequestId("a")
    allocator.create(KVReservation(request, 1))
    with pytest.raises(ValueError, match="already has a KV cache"):
        allocator.create(KVReservation(request, 1))
    allocator.release_all(request)
    assert allocator.capacity() == CapacityCounts(1, 1, 0, 0, 0, 0)


@pytest.mark.parametrize("index", [-1, 1, True, 0.0])
def test_rejects_invalid_logical_blocks(index: Any):
    allocator = cpu_allocator(torch.empty((22, 2, 1, 16, 4, 64), dtype=torch.float16))
    request = RequestId("a")
    allocator.create(KVReservation(request, 1))
    with pytest.raises(ValueError, match="logical block"):
        allocator.read_block(request, 0)
    allocator.append(request, *kv_values(1))
    with pytest.raises(ValueError, match="logical block"):
        allocator.read_block(request, index)


@pytest.mark.parametrize("invalid", ["shape", "dtype", "device", "empty"])
def test_rejects_invalid_appends_before_assigning_blocks(invalid):
    writer = CpuCopyWriter()
    allocator = cpu_allocator(torch.empty((22, 2, 1, 16, 4, 64), dtype=torch.float16), writer)
    request = RequestId("a")
    allocator.create(KVReservation(request, 1))
    key, value = kv_values(1)
    if invalid == "shape":
        value = value[:1]
    elif invalid == "dtype":
        value = value.float()
    elif invalid == "device":
        value = value.to("meta")
    else:
        key, value = key[:, :0], value[:, :0]
    with pytest.raises(ValueError, match="K and V must share"):
        allocator.append(request, key, value)
    assert writer.calls == 0 and allocator.block_table(request) == ()


def test_rejects_context_overflow_before_writing():
    allocator = cpu_allocator(torch.empty((22, 2, 128, 16, 4, 64), dtype=torch.float16))
    request = RequestId("a")
    allocator.create(KVReservation(request, 128))
    allocator.append(request, *kv_values(2048))
    last = [t.clone() for t in allocator.read_block(request, 127)]
    with pytest.raises(ValueError, match="2048"):
        allocator.append(request, *kv_values(1))
    assert allocator.cached_length(request) == 2048
    assert all(torch.equal(a, b) for a, b in zip(allocator.read_block(request, 127), last))


# --- staged decode (reference tests/unit/test_kv_cache.py:344-410) -------------------------


def test_decode_exposes_only_written_layers_and_commits_together():
    pool = torch.full((22, 2, 4, 16, 4, 64), torch.nan, dtype=torch.float16)
    allocator = cpu_allocator(pool)
    requests = (RequestId("first"), RequestId("second"))
    for request in requests:
        allocator.create(KVReservation(request, 2))
        allocator.append(request, *kv_values(16))
    counts = allocator.capacity()
    tables = [allocator.block_table(request) for request in requests]
    key, value = kv_values(1, start=100)
    with allocator.append_decode(requests):
        with pytest.raises(RuntimeError, match="unwritten"):
            list(allocator.iter_layer_blocks(requests[0], layer_index=0))
        with pytest.raises(RuntimeError, match="unwritten"):
            allocator.gather_block_tables(requests, layer_index=0)
        for operation in (
            lambda: allocator.create(KVReservation(RequestId("other"), 1)),
            lambda: allocator.append(requests[0], key, value),
            lambda: allocator.release_all(requests[0]),
            lambda: allocator.append_decode(requests).__enter__(),
        ):
            with pytest.raises(RuntimeError, match="staged decode"):
                operation()
        for layer in range(22):
            if layer % 2:
                allocator.write_decode_layers(requests, layer, key[layer, 0][None].expand(2, 4, 64).contiguous(), value[layer, 0][None].expand(2, 4, 64).contiguous())
            else:
                for request in requests:
                    allocator.write_decode_layer(request, layer, key[layer, 0], value[layer, 0])
            for request in requests:
                pages = list(allocator.iter_layer_blocks(request, layer_index=layer))
                assert len(pages) == 2
                assert torch.equal(pages[1][0], key[layer]) and torch.equal(pages[1][1], value[layer])
                assert allocator.cached_length(request) == 16
                assert allocator.capacity() == counts
        for request, table in zip(requests, tables):
            assert allocator.block_table(request) == table
    assert allocator.capacity() == CapacityCounts(4, 0, 4, 4, 2, 34)
    lifo = ref.LifoFreeList.fresh(4)
    lifo.grow_to("first", 16)
    lifo.grow_to("second", 16)
    expected = lifo.decode_step({"first": 16, "second": 16})
    assert allocator.block_table(requests[0]) == tuple(expected["first"])
    assert allocator.block_table(requests[1]) == tuple(expected["second"])
    for request in requests:
        assert allocator.cached_length(request) == 17
        allocator.release_all(request)
    assert allocator.capacity() == CapacityCounts(4, 4, 0, 0, 0, 0)


@pytest.mark.parametrize("fault", ["incomplete", "order", "shape", "dtype", "device", "batched_order", "batched_duplicate"])
def test_decode_rejects_incomplete_or_invalid_layer_writes(fault):
    allocator = cpu_allocator(torch.zeros(22, 2, 2, 16, 4, 64, dtype=torch.float16))
    request = RequestId("request")
    allocator.create(KVReservation(request, 2))
    allocator.append(request, *kv_values(16))
    counts = allocator.capacity()
    key = torch.zeros(4, 64, dtype=torch.float16)
    value = key.clone()
    if fault == "shape":
        key = key[0]
    elif fault == "dtype":
        value = value.float()
    elif fault == "device":
        key = key.to("meta")
    error = RuntimeError if fault == "incomplete" else ValueError
    with pytest.raises(error), allocator.append_decode((request,)):
        if fault == "batched_order":
            allocator.write_decode_layers((request,), 1, key[None], value[None])
        elif fault == "batched_duplicate":
            allocator.write_decode_layers((request, request), 0, key[None].repeat(2, 1, 1), value[None].repeat(2, 1, 1))
        else:
            allocator.write_decode_layer(request, 1 if fault == "order" else 0, key, value)
    assert allocator.capacity() == counts and allocator.cached_length(request) == 16
    allocator.release_all(request)
    assert allocator.capacity() == CapacityCounts(2, 2, 0, 0, 0, 0)


# --- ownership and threads -----------------------------------------------------------------


def test_layer_iterator_checks_worker_on_every_page():
    allocator = cpu_allocator(torch.empty(22, 2, 2, 16, 4, 64, dtype=torch.float16))
    request = RequestId("request")
    allocator.create(KVReservation(request, 2))
    allocator.append(request, *kv_values(17))
    pages = allocator.iter_layer_blocks(request, layer_index=0)
    next(pages)
    with ThreadPoolExecutor(max_workers=1) as executor, pytest.raises(RuntimeError, match="owning model worker"):
        executor.submit(next, pages).result()


def test_rejects_access_from_another_thread():
    allocator = cpu_allocator(torch.empty((22, 2, 1, 16, 4, 64), dtype=torch.float16))
    request = RequestId("a")
    allocator.create(KVReservation(request, 1))
    key, value = kv_values(1)
    with ThreadPoolExecutor(max_workers=1) as executor:
        for operation, args in (
            (allocator.create, (KVReservation(RequestId("b"), 1),)),
            (allocator.capacity, ()),
            (allocator.append, (request, key, value)),
            (allocator.read_block, (request, 0)),
            (allocator.block_table, (request,)),
            (allocator.cached_length, (request,)),
            (allocator.release_all, (request,)),
            (allocator.write_decode_layer, (request, 0, key[0, 0], value[0, 0])),
            (lambda: allocator.gather_block_tables((request,), layer_index=0), ()),
            (lambda: allocator.append_decode((request,)).__enter__(), ()),
            (lambda: next(allocator.iter_layer_blocks(request, layer_index=0)), ()),
        ):
            future = executor.submit(operation, *args)
            with pytest.raises(RuntimeError, match="owning model worker"):
                future.result()
    assert allocator.block_table(request) == ()


# --- accounting (reference tests/unit/test_kv_cache.py:453-570) ----------------------------


def test_accounts_for_reserved_owned_and_live_capacity():
    allocator = cpu_allocator(torch.empty((22, 2, 8, 16, 4, 64), dtype=torch.float16))
    a, b = RequestId("a"), RequestId("b")
    assert allocator.capacity() == CapacityCounts(8, 8, 0, 0, 0, 0)
    allocator.create(KVReservation(a, 3))
    assert allocator.capacity() == CapacityCounts(8, 8, 0, 3, 1, 0)
    allocator.create(KVReservation(b, 2))
    key, value = kv_values(33)
    allocator.append(a, key[:, :15], value[:, :15])
    assert allocator.capacity() == CapacityCounts(8, 7, 1, 5, 2, 15)
    allocator.append(b, *kv_values(16, start=2000))
    assert allocator.capacity() == CapacityCounts(8, 6, 2, 5, 2, 31)
    allocator.append(a, key[:, 15:16], value[:, 15:16])
    assert allocator.capacity() == CapacityCounts(8, 6, 2, 5, 2, 32)
    allocator.append(a, key[:, 16:17], value[:, 16:17])
    assert allocator.capacity() == CapacityCounts(8, 5, 3, 5, 2, 33)
    allocator.append(a, key[:, 17:], value[:, 17:])
    assert allocator.capacity() == CapacityCounts(8, 4, 4, 5, 2, 49)
    allocator.release_all(a)
    assert allocator.capacity() == CapacityCounts(8, 7, 1, 2, 1, 16)
    allocator.release_all(b)
    assert allocator.capacity() == CapacityCounts(8, 8, 0, 0, 0, 0)


def test_reservations_use_unpromised_capacity():
    allocator = cpu_allocator(torch.empty((22, 2, 3, 16, 4, 64), dtype=torch.float16))
    a, b = RequestId("a"), RequestId("b")
    allocator.create(KVReservation(a, 3))
    with pytest.raises(RuntimeError, match="insufficient unreserved blocks"):
        allocator.create(KVReservation(b, 1))
    with pytest.raises(KeyError):
        allocator.block_table(b)
    allocator.append(a, *kv_values(17))
    assert allocator.capacity() == CapacityCounts(3, 1, 2, 3, 1, 17)
    allocator.release_all(a)
    allocator.create(KVReservation(b, 1))
    assert allocator.capacity() == CapacityCounts(3, 3, 0, 1, 1, 0)


def test_pending_requests_hold_no_resources():
    allocator = cpu_allocator(torch.empty((22, 2, 3, 16, 4, 64), dtype=torch.float16))
    pending = KVReservation(RequestId("pending"), 3)
    key, value = kv_values(1)
    for operation in (
        lambda: allocator.block_table(pending.request_id),
        lambda: allocator.cached_length(pending.request_id),
        lambda: allocator.append(pending.request_id, key, value),
        lambda: allocator.release_all(pending.request_id),
    ):
        with pytest.raises(KeyError):
            operation()
    assert allocator.capacity() == CapacityCounts(3, 3, 0, 0, 0, 0)


@pytest.mark.parametrize(("blocks", "credits", "message"), [(2, 3, "total KV pool capacity"), (129, 129, "KV context capacity")])
def test_rejects_impossible_reservations(blocks, credits, message):
    allocator = cpu_allocator(torch.empty((22, 2, blocks, 16, 4, 64), dtype=torch.float16))
    with pytest.raises(ValueError, match=message):
        allocator.create(KVReservation(RequestId("impossible"), credits))


def test_reservation_record_validation():
    for credits in (0, -1, True, 1.0):
        with pytest.raises(ValueError):
            KVReservation(RequestId("x"), credits)
    with pytest.raises(ValueError):
        CapacityCounts(4, 3, 0, 0, 0, 0)
    with pytest.raises(ValueError):
        CapacityCounts(4, 2, 2, 1, 1, 0)


# --- corruption detection (reference tests/unit/test_kv_cache.py:572-676) ------------------


@pytest.mark.parametrize("operation", ["read", "append", "release", "gather"])
@pytest.mark.parametrize("corruption", ["duplicate", "foreign", "free", "negative", "outside", "boolean", "float", "short", "length"])
def test_rejects_corrupt_tables_before_access_or_mutation(corruption, operation):
    pool = torch.full((22, 2, 4, 16, 4, 64), -999, dtype=torch.float16)
    writer = CpuCopyWriter()
    allocator = cpu_allocator(pool, writer)
    a, b = RequestId("a"), RequestId("b")
    allocator.create(KVReservation(a, 3))
    allocator.create(KVReservation(b, 1))
    allocator.append(a, *kv_values(17))
    allocator.append(b, *kv_values(1, start=2000))
    before = allocator.capacity()
    original = allocator._sequences[a]
    first, last = original.blocks
    tables = {
        "duplicate": (first, first),
        "foreign": (allocator.block_table(b)[0], last),
        "free": (allocator._free_blocks[-1], last),
        "negative": (-1, last),
        "outside": (4, last),
        "boolean": (True, last),
        "float": (float(first), last),
        "short": (first,),
        "length": original.blocks,
    }
    allocator._sequences[a] = replace(original, blocks=tables[corruption], length=16 if corruption == "length" else 17)
    sequences = allocator._sequences.copy()
    free = allocator._free_blocks.copy()
    contents = pool.clone()
    calls = writer.calls
    with pytest.raises(RuntimeError, match="KV"):
        if operation == "read":
            allocator.read_block(a, 0)
        elif operation == "append":
            allocator.append(a, *kv_values(1))
        elif operation == "gather":
            allocator.gather_block_tables((a,), layer_index=0)
        else:
            allocator.release_all(a)
    assert allocator._sequences == sequences and allocator._free_blocks == free
    assert torch.equal(pool, contents) and writer.calls == calls
    allocator._sequences[a] = original
    assert allocator.capacity() == before


@pytest.mark.parametrize("corruption", ["duplicate", "missing", "owned", "invalid"])
def test_rejects_corrupt_free_lists_before_release(corruption):
    allocator = cpu_allocator(torch.empty((22, 2, 3, 16, 4, 64), dtype=torch.float16))
    request = RequestId("a")
    allocator.create(KVReservation(request, 1))
    allocator.append(request, *kv_values(1))
    if corruption == "duplicate":
        allocator._free_blocks.append(allocator._free_blocks[-1])
    elif corruption == "missing":
        allocator._free_blocks.pop()
    elif corruption == "owned":
        allocator._free_blocks[-1] = allocator.block_table(request)[0]
    else:
        allocator._free_blocks[-1] = -1
    free = allocator._free_blocks.copy()
    with pytest.raises(RuntimeError, match="KV"):
        allocator.release_all(request)
    assert allocator._free_blocks == free


def test_detects_swapped_tables_through_owners():
    allocator = cpu_allocator(torch.full((22, 2, 4, 16, 4, 64), -999, dtype=torch.float16))
    a, b = RequestId("a"), RequestId("b")
    allocator.create(KVReservation(a, 2))
    allocator.create(KVReservation(b, 2))
    allocator.append(a, *kv_values(1))
    allocator.append(b, *kv_values(1, start=2000))
    first, second = allocator._sequences[a], allocator._sequences[b]
    allocator._sequences[a] = replace(first, blocks=second.blocks)
    allocator._sequences[b] = replace(second, blocks=first.blocks)
    with pytest.raises(RuntimeError, match="owned"):
        allocator.read_block(a, 0)


# --- failure injection at the write (reference tests/unit/test_kv_cache.py:679-738) --------


@pytest.mark.parametrize("initial_tokens", [0, 15, 16, 17])
def test_write_failure_preserves_history_and_allows_cleanup_and_reuse(initial_tokens):
    writer = CpuCopyWriter()
    allocator = cpu_allocator(torch.empty((22, 2, 4, 16, 4, 64), dtype=torch.float16), writer)
    a, b, c = RequestId("a"), RequestId("b"), RequestId("c")
    allocator.create(KVReservation(a, 3))
    allocator.create(KVReservation(b, 1))
    key, value = kv_values(initial_tokens)
    if initial_tokens:
        allocator.append(a, key, value)
    other_key, other_value = kv_values(1, start=2000)
    allocator.append(b, other_key, other_value)
    before = allocator.capacity()
    table = allocator.block_table(a)
    writer.fail_at = writer.calls + 1
    with pytest.raises(RuntimeError, match="injected copy failure"):
        allocator.append(a, *kv_values(18, start=100))
    assert allocator.capacity() == before and allocator.block_table(a) == table
    assert allocator.cached_length(a) == initial_tokens
    for logical in range(len(table)):
        assert torch.equal(allocator.read_block(a, logical)[0], key[:, logical * 16 : logical * 16 + 16])
    assert torch.equal(allocator.read_block(b, 0)[0], other_key)
    allocator.release_all(a)
    assert allocator.capacity() == CapacityCounts(4, 3, 1, 1, 1, 1)
    allocator.create(KVReservation(c, 3))
    fresh_key, fresh_value = kv_values(48, start=-100)
    allocator.append(c, fresh_key, fresh_value)
    for logical in range(3):
        assert torch.equal(allocator.read_block(c, logical)[1], fresh_value[:, logical * 16 : logical * 16 + 16])


def test_decode_write_failure_discards_the_staged_step():
    writer = CpuCopyWriter()
    allocator = cpu_allocator(torch.zeros(22, 2, 4, 16, 4, 64, dtype=torch.float16), writer)
    requests = (RequestId("x"), RequestId("y"))
    for request, tokens in zip(requests, (15, 16)):
        allocator.create(KVReservation(request, 2))
        allocator.append(request, *kv_values(tokens))
    counts = allocator.capacity()
    tables = [allocator.block_table(request) for request in requests]
    writer.fail_at = writer.calls + 4
    key = torch.ones(2, 4, 64, dtype=torch.float16)
    with pytest.raises(RuntimeError, match="injected copy failure"), allocator.append_decode(requests):
        for layer in range(22):
            allocator.write_decode_layers(requests, layer, key, -key)
    assert allocator.capacity() == counts
    assert [allocator.block_table(request) for request in requests] == tables
    with allocator.append_decode(requests):
        for layer in range(22):
            allocator.write_decode_layers(requests, layer, key, -key)
    assert [allocator.cached_length(request) for request in requests] == [16, 17]


@pytest.mark.parametrize("batched", [False, True])
def test_corruption_planted_mid_step_raises_at_the_next_layer_write(batched):
    """The reference checks the accounting on every write_decode_layer
    (src/pagedcore/kv_cache.py:227): a duplicate free block planted between two layer
    writes raises at the next write, and nothing of the step is published."""
    writer = CpuCopyWriter()
    allocator = cpu_allocator(torch.zeros(22, 2, 4, 16, 4, 64, dtype=torch.float16), writer)
    request = RequestId("x")
    allocator.create(KVReservation(request, 2))
    allocator.append(request, *kv_values(16))
    owned = allocator.block_table(request)[0]
    key = torch.ones(1, 4, 64, dtype=torch.float16)
    with pytest.raises(RuntimeError, match="owned KV blocks must not be free"):
        with allocator.append_decode((request,)):
            for layer in range(22):
                if layer == 3:
                    allocator._free_blocks.append(owned)
                if batched:
                    allocator.write_decode_layers((request,), layer, key, -key)
                else:
                    allocator.write_decode_layer(request, layer, key[0], -key[0])
    assert writer.calls == 1 + 3  # the prompt append and layers 0..2; layer 3 raised first
    assert allocator._decode_appends is None
    allocator._free_blocks.pop()
    assert allocator.cached_length(request) == 16


# --- device tables ---------------------------------------------------------------------------


def test_gather_block_tables_follows_staged_tables_and_caches_per_state():
    allocator = cpu_allocator(torch.zeros(22, 2, 8, 16, 4, 64, dtype=torch.float16))
    requests = (RequestId("p"), RequestId("q"))
    for request, tokens in zip(requests, (16, 40)):
        allocator.create(KVReservation(request, 3))
        allocator.append(request, *kv_values(tokens))
    tables, lengths = allocator.gather_block_tables(requests, layer_index=5)
    assert tables.dtype == torch.int32 and tables.shape == (2, 3)
    assert tables[0, :1].tolist() == list(allocator.block_table(requests[0]))
    assert tables[1].tolist() == list(allocator.block_table(requests[1]))
    assert lengths.tolist() == [16, 40]
    with allocator.append_decode(requests):
        allocator.write_decode_layers(requests, 0, torch.zeros(2, 4, 64, dtype=torch.float16), torch.zeros(2, 4, 64, dtype=torch.float16))
        staged, staged_lengths = allocator.gather_block_tables(requests, layer_index=0)
        assert staged_lengths.tolist() == [17, 41]
        assert staged[0, :2].tolist() == [allocator.block_table(requests[0])[0], allocator._free_blocks[-1]]
        again = allocator.gather_block_tables(requests, layer_index=0)
        assert again[0] is staged  # the 22 layers of a step share one table upload
        # the cached lookup still refuses a layer that is not written yet
        with pytest.raises(RuntimeError, match="unwritten"):
            allocator.gather_block_tables(requests, layer_index=1)
        with pytest.raises(RuntimeError, match="unwritten"):
            allocator.gather_block_tables(requests[::-1], layer_index=3)
        for layer in range(1, 22):
            allocator.write_decode_layers(requests, layer, torch.zeros(2, 4, 64, dtype=torch.float16), torch.zeros(2, 4, 64, dtype=torch.float16))
            assert allocator.gather_block_tables(requests, layer_index=layer)[0] is staged
    committed, committed_lengths = allocator.gather_block_tables(requests, layer_index=0)
    assert committed_lengths.tolist() == [17, 41]
    assert committed[0, :2].tolist() == list(allocator.block_table(requests[0]))


# --- randomized model (reference tests/unit/test_kv_cache_properties.py) -------------------


def _tagged_kv(tokens: list[int]):
    key = torch.tensor(tokens, dtype=torch.float16)[None, :, None, None].expand(22, -1, 4, 64)
    return key, -key - 1


class _AllocatorMachine(RuleBasedStateMachine):
    def __init__(self, blocks: int) -> None:
        super().__init__()
        self.pool = torch.full((22, 2, blocks, 16, 4, 64), torch.nan, dtype=torch.float16)
        self.writer = CpuCopyWriter()
        self.allocator = cpu_allocator(self.pool, self.writer)
        self.total = blocks
        self.free = set(range(blocks))
        self.requests: dict[RequestId, dict] = {}
        self.next_token = 0

    @rule(slot=st.integers(0, 3), credits=st.integers(1, 9))
    def create(self, slot, credits):
        request = RequestId(str(slot))
        reservation = KVReservation(request, credits)
        if request in self.requests:
            with pytest.raises(ValueError, match="already has a KV cache"):
                self.allocator.create(reservation)
        elif credits > self.total:
            with pytest.raises(ValueError, match="total KV pool capacity"):
                self.allocator.create(reservation)
        elif credits + sum(r["credits"] for r in self.requests.values()) > self.total:
            with pytest.raises(RuntimeError, match="insufficient unreserved blocks"):
                self.allocator.create(reservation)
        else:
            self.allocator.create(reservation)
            self.requests[request] = {"credits": credits, "tokens": [], "blocks": ()}

    @precondition(lambda self: bool(self.requests))
    @rule(data=st.data(), tokens=st.sampled_from((1, 2, 15, 16, 17, 31, 32, 33)), fail=st.booleans())
    def append(self, data, tokens, fail):
        request = data.draw(st.sampled_from(tuple(self.requests)), label="request")
        expected = self.requests[request]
        tags = list(range(self.next_token, self.next_token + tokens))
        self.next_token += tokens
        key, value = _tagged_kv(tags)
        length = len(expected["tokens"]) + tokens
        if length > expected["credits"] * 16:
            with pytest.raises(RuntimeError, match="exceeds request reservation"):
                self.allocator.append(request, key, value)
            return
        if fail:
            self.writer.fail_at = self.writer.calls + 1
            with pytest.raises(RuntimeError, match="injected copy failure"):
                self.allocator.append(request, key, value)
            self.writer.fail_at = None
            return
        self.allocator.append(request, key, value)
        table = self.allocator.block_table(request)
        assert len(table) == ceil(length / 16) and table[: len(expected["blocks"])] == expected["blocks"]
        added = table[len(expected["blocks"]) :]
        assert set(added) <= self.free
        self.free.difference_update(added)
        expected["blocks"] = table
        expected["tokens"].extend(tags)

    @precondition(lambda self: bool(self.requests))
    @rule(data=st.data(), tokens=st.sampled_from((1, 16, 17, 40)), complete=st.booleans())
    def append_prompt(self, data, tokens, complete):
        """The staged prompt append (the fused prefill path): the caller writes each layer's
        K/V to the staged slots; published only when all 22 layers were recorded."""
        request = data.draw(st.sampled_from(tuple(self.requests)), label="request")
        expected = self.requests[request]
        length = len(expected["tokens"]) + tokens
        if length > expected["credits"] * 16:
            with pytest.raises(RuntimeError, match="exceeds request reservation"):
                with self.allocator.append_prompt(request, tokens):
                    pass
            return
        tags = list(range(self.next_token, self.next_token + tokens))
        self.next_token += tokens
        key, value = _tagged_kv(tags)
        with pytest.raises(RuntimeError, match="every cache layer") if not complete else nullcontext():
            with self.allocator.append_prompt(request, tokens) as staged:
                block, offset = staged.slot_mapping // 16, staged.slot_mapping % 16
                for layer in range(LAYERS if complete else LAYERS - 1):
                    self.pool[layer, 0, block, offset] = key[layer]
                    self.pool[layer, 1, block, offset] = value[layer]
                    staged.record_layer(layer)
        if not complete:
            return
        table = self.allocator.block_table(request)
        assert set(table[len(expected["blocks"]) :]) <= self.free
        self.free.difference_update(table[len(expected["blocks"]) :])
        expected["blocks"] = table
        expected["tokens"].extend(tags)

    @rule(slot=st.integers(0, 3))
    def release(self, slot):
        request = RequestId(str(slot))
        if request not in self.requests:
            with pytest.raises(KeyError):
                self.allocator.release_all(request)
        else:
            self.allocator.release_all(request)
            self.free.update(self.requests.pop(request)["blocks"])

    @invariant()
    def matches_model(self):
        owned = sum(ceil(len(r["tokens"]) / 16) for r in self.requests.values())
        reserved = sum(r["credits"] for r in self.requests.values())
        live = sum(len(r["tokens"]) for r in self.requests.values())
        assert self.allocator.capacity() == CapacityCounts(self.total, self.total - owned, owned, reserved, len(self.requests), live)
        # the counts kept across the allocator's own mutations equal a full rescan
        assert self.allocator._full_accounting() == self.allocator.capacity()
        assert set(self.allocator._free_blocks) == self.free
        for request, r in self.requests.items():
            assert self.allocator.block_table(request) == r["blocks"]
            for logical in range(len(r["blocks"])):
                key, value = _tagged_kv(r["tokens"][logical * 16 : (logical + 1) * 16])
                actual_key, actual_value = self.allocator.read_block(request, logical)
                assert torch.equal(actual_key, key) and torch.equal(actual_value, value)


@pytest.mark.parametrize("blocks", [1, 2, 4, 8])
def test_randomized_operations_match_an_independent_model(blocks):
    run_state_machine_as_test(
        lambda: _AllocatorMachine(blocks),
        settings=settings(max_examples=40, stateful_step_count=30, deadline=None, derandomize=True, database=None),
    )


# --- staged prompt append (the fused prefill write path) ----------------------------------


def _twin_allocators():
    """Two allocators in the same state, one request 'p' with 5 cached tokens and a
    blocker 'b' holding the block after it, so new blocks come from the free-list tail."""
    allocators = []
    for _ in range(2):
        allocator = cpu_allocator(torch.zeros((22, 2, 8, 16, 4, 64), dtype=torch.float16))
        allocator.create(KVReservation(RequestId("p"), 4))
        allocator.append(RequestId("p"), *kv_values(5))
        allocator.create(KVReservation(RequestId("b"), 1))
        allocator.append(RequestId("b"), *kv_values(3))
        allocators.append(allocator)
    return allocators


def test_staged_prompt_append_takes_the_blocks_append_would_and_publishes_after_all_layers():
    staged_alloc, plain = _twin_allocators()
    request = RequestId("p")
    plain.append(request, *kv_values(30, start=7))
    with staged_alloc.append_prompt(request, 30) as staged:
        assert staged.tokens == 30
        assert staged.positions.tolist() == list(range(5, 35))
        # nothing published while staged; other mutations are refused
        assert staged_alloc.cached_length(request) == 5
        with pytest.raises(RuntimeError, match="staged prompt append"):
            staged_alloc.release_all(RequestId("b"))
        for layer in range(22):
            staged.record_layer(layer)
    assert staged_alloc.block_table(request) == plain.block_table(request)
    assert staged_alloc.capacity() == plain.capacity()
    table = plain.block_table(request)
    expected = [table[p // 16] * 16 + p % 16 for p in range(5, 35)]
    assert staged.slots.dtype == np.int64 and staged.slots.tolist() == expected  # the host copy
    assert staged.slot_mapping.tolist() == expected  # the device copy, uploaded on first use


def test_staged_prompt_append_discards_on_error_and_requires_every_layer():
    allocator, _ = _twin_allocators()
    request = RequestId("p")
    counts, table, free = allocator.capacity(), allocator.block_table(request), list(allocator._free_blocks)
    with pytest.raises(RuntimeError, match="injected"):
        with allocator.append_prompt(request, 20) as staged:
            staged.record_layer(0)
            raise RuntimeError("injected")
    with pytest.raises(RuntimeError, match="every cache layer"):
        with allocator.append_prompt(request, 20) as staged:
            for layer in range(21):
                staged.record_layer(layer)
    with pytest.raises(ValueError, match="once in order"):
        with allocator.append_prompt(request, 20) as staged:
            staged.record_layer(1)
    assert allocator.capacity() == counts and allocator.block_table(request) == table
    assert list(allocator._free_blocks) == free and allocator.cached_length(request) == 5
    allocator.release_all(RequestId("b"))  # mutations work again after the staging ended


@pytest.mark.parametrize(
    "tokens,error,needle",
    [(0, ValueError, "positive"), (2044, ValueError, "2048"), (60, RuntimeError, "reservation"), (2.0, ValueError, "positive")],
)
def test_staged_prompt_append_checks_before_staging(tokens, error, needle):
    allocator, _ = _twin_allocators()
    counts = allocator.capacity()
    with pytest.raises(error, match=needle):
        with allocator.append_prompt(RequestId("p"), tokens):
            pass
    assert allocator.capacity() == counts and allocator._prompt_append is None
    with pytest.raises(KeyError):
        with allocator.append_prompt(RequestId("unknown"), 3):
            pass


def test_cached_lengths_checks_once_and_raises_for_an_unknown_request():
    allocator = cpu_allocator(torch.zeros((22, 2, 8, 16, 4, 64), dtype=torch.float16))
    for name, tokens in (("a", 5), ("b", 17)):
        allocator.create(KVReservation(RequestId(name), 2))
        allocator.append(RequestId(name), *kv_values(tokens))
    assert allocator.cached_lengths((RequestId("b"), RequestId("a"))) == (17, 5)
    assert allocator.cached_lengths(()) == ()
    with pytest.raises(KeyError):
        allocator.cached_lengths((RequestId("a"), RequestId("missing")))


def test_staged_decode_view_matches_each_staged_sequence():
    """The host view of a staged decode step (tables, lengths, new-token slots and
    positions) row by row, including a request whose new token takes a fresh block and
    zero padding to a wider table."""
    allocator = cpu_allocator(torch.zeros((22, 2, 16, 16, 4, 64), dtype=torch.float16))
    names = {"a": 5, "b": 16, "c": 33, "d": 1}  # b's new token starts its second block
    for name, tokens in names.items():
        allocator.create(KVReservation(RequestId(name), 4))
        allocator.append(RequestId(name), *kv_values(tokens))
    order = (RequestId("c"), RequestId("b"), RequestId("d"), RequestId("a"))
    with allocator.append_decode(order):
        staged = allocator.staged_decode(order, width=6)
        with pytest.raises(ValueError, match="wider"):
            allocator.staged_decode(order, width=2)
        for row, rid in enumerate(order):
            length = names[rid] + 1
            blocks = allocator._decode_appends[rid].sequence.blocks
            assert len(blocks) == (length + 15) // 16
            assert staged.lengths[row] == length and staged.positions[row] == length - 1
            assert staged.tables[row].tolist() == list(blocks) + [0] * (6 - len(blocks))
            assert staged.slots[row] == blocks[(length - 1) // 16] * 16 + (length - 1) % 16
        assert staged.tables.dtype == np.int32 and staged.lengths.dtype == np.int32
        assert staged.slots.dtype == np.int64 and staged.positions.dtype == np.int64
        for layer in range(22):
            kv = torch.zeros(len(order), 4, 64, dtype=torch.float16)
            allocator.write_decode_layers(order, layer, kv, kv)
