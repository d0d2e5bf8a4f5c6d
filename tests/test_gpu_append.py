"""KV append on the GPU: bit-exact against the oracle's restatement of the reference append.

Covers the prompt-append workload (2048 tokens x 22 layers into a 30%-occupied 4096-block
pool, checked against the committed golden digest), the reference allocator tests' token
mapping and fragmentation cases on a GPU pool, strided and misaligned sources, the decode
writes, stream ownership and rollback of a failed launch.
"""

from __future__ import annotations

import hashlib
import json
import os
import sys

import numpy as np
import pytest
import torch

from oracle import paged_reference as ref
from pagedcore_amd import _hip
from tests import workloads
from pagedcore_amd.engine_types import CapacityCounts, KVReservation, RequestId
from pagedcore_amd.kv_cache import HipKVWriter, KVAllocator
from tests.support import kv_values

pytestmark = pytest.mark.gpu


def _say(*parts) -> None:
    print(*parts, flush=True)
    sys.stdout.flush()


def _bits(tensor: torch.Tensor) -> np.ndarray:
    return tensor.detach().cpu().contiguous().view(torch.int16).numpy().view(np.uint16)


def _digest(array: np.ndarray) -> str:
    return hashlib.blake2b(np.ascontiguousarray(array).view(np.uint8), digest_size=32).hexdigest()


def test_prompt_append_into_fragmented_pool_matches_golden_bytes(device):
    """2048-token prompt x 22 layers into a 4096-block pool whose free list is in seeded
    random order with 30% of it held by 10 filler requests: the whole pool (NaN-poisoned
    beforehand) must equal the golden digest and the oracle's pool bit for bit."""
    _say("prompt append golden")
    golden_path = os.path.join(os.path.dirname(__file__), "golden", "config2_prompt_append.json")
    with open(golden_path) as handle:
        golden = json.load(handle)
    w = workloads.prompt_append()
    key_np, value_np = w.prompt_kv()
    assert _digest(key_np.view(np.uint16)) == golden["prompt_key_blake2b"]
    assert _digest(value_np.view(np.uint16)) == golden["prompt_value_blake2b"]

    pool = torch.full((22, 2, w.num_blocks, 16, 4, 64), float("nan"), dtype=torch.float16, device=device)
    allocator = KVAllocator(pool)
    allocator._free_blocks = list(w.free_order)  # the seeded allocator: same free set, random order
    for index in range(len(w.filler_blocks)):
        key, value = (torch.from_numpy(a).to(device) for a in w.filler_kv(index))
        request = RequestId(f"filler{index}")
        allocator.create(KVReservation(request, w.filler_blocks[index]))
        allocator.append(request, key, value)
    prompt = RequestId("prompt")
    allocator.create(KVReservation(prompt, 128))
    allocator.append(prompt, torch.from_numpy(key_np).to(device), torch.from_numpy(value_np).to(device))
    torch.cuda.synchronize()
    assert list(allocator.block_table(prompt)) == golden["prompt_table"]
    counts = allocator.capacity()
    assert counts.owned_blocks == sum(w.filler_blocks) + 128
    actual = _bits(pool)
    assert _digest(actual) == golden["pool_blake2b"]


@pytest.mark.parametrize(
    "tokens,blocks,last_slots",
    [(1, 1, 1), (15, 1, 15), (16, 1, 16), (17, 2, 1), (32, 2, 16), (33, 3, 1)],
)
def test_token_mapping_and_poison_outside_valid_slots(device, tokens, blocks, last_slots):
    # reference tests/unit/test_kv_cache.py:150-183 on a GPU pool.
    pool = torch.full((22, 2, 4, 16, 4, 64), float("nan"), dtype=torch.float16, device=device)
    allocator = KVAllocator(pool)
    request = RequestId("a")
    allocator.create(KVReservation(request, blocks))
    key, value = kv_values(tokens, device=device)
    allocator.append(request, key, value)
    table = allocator.block_table(request)
    assert len(table) == blocks and len(set(table)) == blocks
    assert allocator.cached_length(request) == tokens
    for index, physical in enumerate(table):
        slots = last_slots if index == blocks - 1 else 16
        actual_key, actual_value = allocator.read_block(request, index)
        assert actual_key.shape == actual_value.shape == (22, slots, 4, 64)
        expected = slice(index * 16, index * 16 + slots)
        assert torch.equal(actual_key, key[:, expected])
        assert torch.equal(actual_value, value[:, expected])
        if slots < 16:
            assert torch.isnan(pool[:, :, physical, slots:]).all()
    for physical in set(range(4)) - set(table):
        assert torch.isnan(pool[:, :, physical]).all()


def test_fragmented_appends_match_the_oracle_pool(device):
    # reference tests/unit/test_kv_cache.py:186-213 plus a whole-pool bit comparison.
    pool = torch.full((22, 2, 4, 16, 4, 64), float("nan"), dtype=torch.float16, device=device)
    allocator = KVAllocator(pool)
    a, b = RequestId("a"), RequestId("b")
    allocator.create(KVReservation(a, 3))
    allocator.create(KVReservation(b, 1))
    key, value = kv_values(33, device=device)
    other_key, other_value = kv_values(16, start=2000, device=device)
    expected = np.full((22, 2, 4, 16, 4, 64), ref.NAN_F16_BITS, dtype=np.uint16)
    lifo = ref.LifoFreeList.fresh(4)
    steps = [(a, 0, 15), (b, None, None), (a, 15, 16), (a, 16, 17), (a, 17, 33)]
    for request, start, stop in steps:
        if request == b:
            allocator.append(b, other_key, other_value)
            ref.reference_append(expected, lifo.grow_to("b", 16), 0, _bits(other_key), _bits(other_value))
            continue
        allocator.append(a, key[:, start:stop], value[:, start:stop])
        lifo.grow_to("a", stop)
        ref.reference_append(expected, lifo.tables["a"], start, _bits(key[:, start:stop]), _bits(value[:, start:stop]))
    assert allocator.block_table(a) == (0, 2, 3) == tuple(lifo.tables["a"])
    assert allocator.block_table(b) == (1,)
    assert np.array_equal(_bits(pool), expected)


def test_release_and_reuse_never_expose_stale_slots(device):
    # reference tests/unit/test_kv_cache.py:216-250.
    pool = torch.empty((22, 2, 3, 16, 4, 64), dtype=torch.float16, device=device)
    pointer = pool.untyped_storage().data_ptr()
    allocator = KVAllocator(pool)
    a, b, c = RequestId("a"), RequestId("b"), RequestId("c")
    allocator.create(KVReservation(a, 2))
    allocator.create(KVReservation(b, 1))
    allocator.append(a, *kv_values(17, device=device))
    allocator.append(b, *kv_values(16, start=2000, device=device))
    released = allocator.block_table(a)
    allocator.release_all(a)
    allocator.create(KVReservation(c, 1))
    key, value = kv_values(1, start=-100, device=device)
    allocator.append(c, key, value)
    assert allocator.block_table(c)[0] in released
    actual_key, actual_value = allocator.read_block(c, 0)
    assert torch.equal(actual_key, key) and torch.equal(actual_value, value)
    expected_key, expected_value = kv_values(16, start=2000, device=device)
    actual_key, actual_value = allocator.read_block(b, 0)
    assert torch.equal(actual_key, expected_key) and torch.equal(actual_value, expected_value)
    allocator.release_all(b)
    allocator.release_all(c)
    allocator.create(KVReservation(a, 3))
    allocator.append(a, *kv_values(48, device=device))
    assert set(allocator.block_table(a)) == {0, 1, 2}
    assert pool.untyped_storage().data_ptr() == pointer


@pytest.mark.parametrize("layout", ["transposed", "layer_sliced", "misaligned"])
def test_strided_and_misaligned_sources_copy_exactly(device, layout):
    """Sources that are views (the decoder stacks transposed per-layer K/V) or whose rows are
    not 16-byte aligned take the strided / word paths and still copy bit-exactly."""
    tokens = 37
    base_key, base_value = kv_values(tokens, device=device)
    if layout == "transposed":
        key = base_key.transpose(0, 1).contiguous().transpose(0, 1)  # token-major storage
        value = base_value.transpose(0, 1).contiguous().transpose(0, 1)
    elif layout == "layer_sliced":
        key = torch.empty(22, 2 * tokens, 4, 64, dtype=torch.float16, device=device)[:, ::2]
        value = torch.empty(22, 2 * tokens, 4, 64, dtype=torch.float16, device=device)[:, ::2]
        key.copy_(base_key)  # token stride of two rows
        value.copy_(base_value)
    else:
        flat_key = torch.empty(base_key.numel() + 1, dtype=torch.float16, device=device)
        flat_value = torch.empty(base_value.numel() + 1, dtype=torch.float16, device=device)
        flat_key[1:] = base_key.flatten()
        flat_value[1:] = base_value.flatten()
        key = flat_key[1:].view(base_key.shape)  # 2-byte offset: rows not 16 B aligned
        value = flat_value[1:].view(base_value.shape)
    pool = torch.full((22, 2, 5, 16, 4, 64), float("nan"), dtype=torch.float16, device=device)
    allocator = KVAllocator(pool)
    request = RequestId("strided")
    allocator.create(KVReservation(request, 3))
    allocator.append(request, key, value)
    expected = np.full(pool.shape, ref.NAN_F16_BITS, dtype=np.uint16)
    ref.reference_append(expected, list(allocator.block_table(request)), 0, _bits(base_key), _bits(base_value))
    assert np.array_equal(_bits(pool), expected)


def test_decode_writes_match_the_oracle(device):
    """Staged decode: single-row and batched writes of all 22 layers land exactly where the
    reference's write_decode_layer puts them; the commit publishes the new lengths."""
    pool = torch.full((22, 2, 9, 16, 4, 64), float("nan"), dtype=torch.float16, device=device)
    allocator = KVAllocator(pool)
    requests = (RequestId("p"), RequestId("q"), RequestId("r"))
    lengths = {"p": 16, "q": 5, "r": 32}
    for request in requests:
        allocator.create(KVReservation(request, 3))
        allocator.append(request, *kv_values(lengths[request], start=len(request), device=device))
    expected = _bits(pool).copy()
    gen = torch.Generator(device=device).manual_seed(5)
    step_key = torch.randn(22, 3, 4, 64, dtype=torch.float16, device=device, generator=gen)
    step_value = torch.randn(22, 3, 4, 64, dtype=torch.float16, device=device, generator=gen)
    with allocator.append_decode(requests):
        for layer in range(22):
            if layer % 2 == 0:
                allocator.write_decode_layers(requests, layer, step_key[layer], step_value[layer])
            else:
                for row, request in enumerate(requests):
                    allocator.write_decode_layer(request, layer, step_key[layer, row], step_value[layer, row])
    lifo = ref.LifoFreeList.fresh(9)
    for request in requests:
        lifo.grow_to(request, lengths[request])
    tables = lifo.decode_step({request: lengths[request] for request in requests})
    for row, request in enumerate(requests):
        assert allocator.block_table(request) == tuple(tables[request])
        assert allocator.cached_length(request) == lengths[request] + 1
        for layer in range(22):
            ref.reference_write_decode(
                expected, layer, tables[request], lengths[request] + 1,
                _bits(step_key[layer, row]), _bits(step_value[layer, row]),
            )
    assert np.array_equal(_bits(pool), expected)


def test_foreign_stream_is_rejected(device):
    # reference tests/gpu/test_kv_pool_cuda.py:85-93.
    pool = torch.empty((22, 2, 2, 16, 4, 64), dtype=torch.float16, device=device)
    allocator = KVAllocator(pool)
    a = RequestId("a")
    allocator.create(KVReservation(a, 2))
    key, value = kv_values(16, device=device)
    allocator.append(a, key, value)
    other = torch.cuda.Stream(device=device)
    with torch.cuda.stream(other):
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


class _FailingHipWriter(HipKVWriter):
    def __init__(self, fail_at: int) -> None:
        super().__init__()
        self.calls = 0
        self.fail_at = fail_at

    def append(self, pool, layer_begin, key, value, slots) -> None:
        self.calls += 1
        if self.calls == self.fail_at:
            raise RuntimeError("injected copy failure")
        super().append(pool, layer_begin, key, value, slots)


def test_failed_launch_preserves_history_and_allows_retry(device):
    # reference tests/gpu/test_kv_pool_cuda.py:37-110, failure injected at the launch.
    pool = torch.full((22, 2, 2, 16, 4, 64), float("nan"), dtype=torch.float16, device=device)
    writer = _FailingHipWriter(fail_at=2)
    allocator = KVAllocator(pool, kv_writer=writer)
    a = RequestId("a")
    key, value = kv_values(17, device=device)
    allocator.create(KVReservation(a, 2))
    allocator.append(a, key[:, :16], value[:, :16])
    before = allocator.capacity()
    with pytest.raises(RuntimeError, match="injected copy failure"):
        allocator.append(a, key[:, 16:], value[:, 16:])
    assert allocator.capacity() == before
    assert allocator.cached_length(a) == 16 and len(allocator.block_table(a)) == 1
    allocator.append(a, key[:, 16:], value[:, 16:])
    assert allocator.capacity() == CapacityCounts(2, 0, 2, 2, 1, 17)
    actual_key, actual_value = allocator.read_block(a, 1)
    assert torch.equal(actual_key, key[:, 16:]) and torch.equal(actual_value, value[:, 16:])


def test_c_abi_rejects_bad_arguments_before_launching(device):
    lib = _hip.load()
    pool = torch.zeros((22, 2, 2, 16, 4, 64), dtype=torch.float16, device=device)
    key = torch.ones((1, 1, 4, 64), dtype=torch.float16, device=device)
    slots = torch.zeros(1, dtype=torch.int64, device=device)
    stream = torch.cuda.current_stream(device).cuda_stream
    status = lib.pc_kv_append(pool.data_ptr(), 2, 21, 2, key.data_ptr(), 256, 256, key.data_ptr(), 256, 256, slots.data_ptr(), 1, stream)
    assert status == 1 and b"layers" in lib.pc_last_error()
    torch.cuda.synchronize()
    assert torch.count_nonzero(pool) == 0
    slots.fill_(2 * 16)  # one past the last slot: skipped on the device, nothing written
    _hip.kv_append(pool, 0, key, key, slots)
    slots.fill_(-1)
    _hip.kv_append(pool, 0, key, key, slots)
    torch.cuda.synchronize()
    assert torch.count_nonzero(pool) == 0
