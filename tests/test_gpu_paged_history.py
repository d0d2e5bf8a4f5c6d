"""The paged decode path never materialises a request's KV history.

The reference's invariant (its tests/conftest.py:45-80, exercised at
tests/unit/test_decoder.py:242-295): decoding reads each request's history page by page
and never derives a buffer larger than one 16-token page from the pool. Here the history is
read by the HIP kernels straight from the pool, so no torch op touches it at all; two
checks pin that:

  * a dispatch guard (tests.support.PoolPageGuard) around decode_paged, paged_attention_batch
    and a DecodeGraph step fails any torch op that derives more than one page from the pool,
    and catches a planted shortcut that gathers the history with torch ops;
  * the device memory a 22-layer decode step allocates does not grow with the context: the
    peak allocation of a step over 2040-token contexts is within 1 MiB of one over 60-token
    contexts, while one layer's dense K/V history of that batch would be 16 MiB.
"""

from __future__ import annotations

import sys

import pytest
import torch

from pagedcore_amd import attention as attention_module
from pagedcore_amd import decoder
from pagedcore_amd.attention import paged_attention_batch
from pagedcore_amd.engine_types import KVReservation, RequestId
from pagedcore_amd.kv_cache import KVAllocator
from tests.support import PoolPageGuard

pytestmark = pytest.mark.gpu

BATCH = 8


def _say(*parts) -> None:
    print(*parts, flush=True)
    sys.stdout.flush()


@pytest.fixture
def model(device):
    # 22 full-width layers (hidden 2048, 32/4 heads) with a small MLP and vocabulary: the
    # decode step's shape around attention is the real one.
    return decoder.random_weights(device=device, seed=31, vocab=64, intermediate=128)


def _requests(allocator, prefix, length, gen):
    requests = []
    for index in range(BATCH):
        request = RequestId(f"{prefix}{index}")
        allocator.create(KVReservation(request, 128))
        key = torch.randn(22, length, 4, 64, dtype=torch.float16, device=allocator.pool.device, generator=gen)
        value = torch.randn(22, length, 4, 64, dtype=torch.float16, device=allocator.pool.device, generator=gen)
        allocator.append(request, key, value)
        requests.append(request)
    return tuple(requests)


@pytest.fixture
def caches(device):
    """One pool holding BATCH requests at 60 cached tokens and BATCH at 2040."""
    pool = torch.empty((22, 2, 2 * BATCH * 128 + 64, 16, 4, 64), dtype=torch.float16, device=device)
    allocator = KVAllocator(pool)
    gen = torch.Generator(device=device).manual_seed(32)
    return allocator, {60: _requests(allocator, "short", 60, gen), 2040: _requests(allocator, "long", 2040, gen)}


def _ids(device, seed):
    return torch.randint(0, 64, (BATCH, 1), device=device, generator=torch.Generator(device=device).manual_seed(seed))


def test_decode_step_and_batched_attention_derive_no_history(device, model, caches):
    allocator, sets = caches
    requests = sets[2040]
    lengths = [allocator.cached_length(r) for r in requests]
    with PoolPageGuard(allocator.pool) as guard:
        logits = decoder.decode_paged(_ids(device, 1), model, allocator, requests)
        query = torch.randn(BATCH, 32, 1, 64, dtype=torch.float16, device=device)
        out = paged_attention_batch(query, allocator, requests, layer_index=7)
    torch.cuda.synchronize()
    _say("decode step under the page guard: torch ops that read KV", guard.kv_ops)
    assert torch.isfinite(logits).all() and torch.isfinite(out).all()
    assert [allocator.cached_length(r) for r in requests] == [n + 1 for n in lengths]

    graph = decoder.DecodeGraph(model, allocator, BATCH)  # captured outside the guard
    with PoolPageGuard(allocator.pool) as guard:
        graph_logits = graph.step(_ids(device, 2), requests)
    torch.cuda.synchronize()
    graph.check_faults()
    _say("DecodeGraph step under the page guard: torch ops that read KV", guard.kv_ops)
    assert torch.isfinite(graph_logits).all()
    assert [allocator.cached_length(r) for r in requests] == [n + 2 for n in lengths]


def test_the_guard_catches_a_gathered_history(device, model, caches, monkeypatch):
    """Negative control: attention that first gathers the request's K pages with torch ops
    (as a dense-history implementation would) fails under the guard, before the step
    publishes anything."""
    allocator, sets = caches
    requests = sets[60]
    counts = allocator.capacity()
    lengths = [allocator.cached_length(r) for r in requests]
    original = attention_module.attend_rows

    def gathering(query, allocator_, request_ids, layer_index):
        table = torch.tensor(allocator_.block_table(request_ids[0]), device=device)
        allocator_.pool[layer_index, 0].index_select(0, table)  # a dense copy of the history
        return original(query, allocator_, request_ids, layer_index)

    monkeypatch.setattr(decoder, "attend_rows", gathering)
    with pytest.raises(AssertionError, match="derived .* bytes of KV history"):
        with PoolPageGuard(allocator.pool):
            decoder.decode_paged(_ids(device, 3), model, allocator, requests)
    assert allocator.capacity() == counts
    assert [allocator.cached_length(r) for r in requests] == lengths


def test_step_memory_does_not_grow_with_context(device, model, caches):
    allocator, sets = caches
    for requests in sets.values():  # warm-up: library state, cached workspace, RoPE table
        decoder.decode_paged(_ids(device, 4), model, allocator, requests)
    growth = {}
    for context, requests in sets.items():
        torch.cuda.synchronize()
        torch.cuda.reset_peak_memory_stats(device)
        base = torch.cuda.memory_allocated(device)
        decoder.decode_paged(_ids(device, 5), model, allocator, requests)
        torch.cuda.synchronize()
        growth[context] = torch.cuda.max_memory_allocated(device) - base
    dense_layer = BATCH * 2048 * 4 * 64 * 2 * 2  # one layer's K and V history of the batch
    _say("peak allocation of one decode step by context:", growth, "dense history of one layer:", dense_layer)
    assert growth[2040] <= growth[60] + (1 << 20)
    assert growth[2040] < dense_layer
