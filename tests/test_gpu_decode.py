"""A staged decode step through the unchanged allocator API on the GPU: per layer, the
batched KV write then batched paged attention over the staged tables, against the oracle.

This is the shape of the reference decoder's inner loop (src/pagedcore/decoder.py:178-194:
append_decode, write_decode_layer, paged_attention per layer) with one launch per layer
for all rows instead of one per row.
"""

from __future__ import annotations

import pytest
import torch

from oracle import paged_reference as ref
from pagedcore_amd.attention import paged_attention_batch
from pagedcore_amd.engine_types import CapacityCounts, KVReservation, RequestId
from pagedcore_amd.kv_cache import KVAllocator
from tests.support import assert_max_abs

pytestmark = pytest.mark.gpu


def test_staged_decode_step_reads_each_written_layer(device):
    lengths = [1, 15, 16, 17, 49, 255, 1024, 2047]
    pool = torch.full((22, 2, 300, 16, 4, 64), float("nan"), dtype=torch.float16, device=device)
    allocator = KVAllocator(pool)
    gen = torch.Generator(device=device).manual_seed(21)
    requests = tuple(RequestId(f"seq{i}") for i in range(len(lengths)))
    for request, length in zip(requests, lengths):
        allocator.create(KVReservation(request, (length + 1 + 15) // 16))
        key = torch.randn(22, length, 4, 64, dtype=torch.float16, device=device, generator=gen)
        value = torch.randn(22, length, 4, 64, dtype=torch.float16, device=device, generator=gen)
        allocator.append(request, key, value)
    counts = allocator.capacity()
    step_key = torch.randn(22, len(lengths), 4, 64, dtype=torch.float16, device=device, generator=gen)
    step_value = torch.randn(22, len(lengths), 4, 64, dtype=torch.float16, device=device, generator=gen)
    query = torch.randn(22, len(lengths), 32, 1, 64, dtype=torch.float16, device=device, generator=gen)
    outputs = []
    with allocator.append_decode(requests):
        with pytest.raises(RuntimeError, match="unwritten"):
            paged_attention_batch(query[0], allocator, requests, layer_index=0)
        for layer in range(22):
            allocator.write_decode_layers(requests, layer, step_key[layer], step_value[layer])
            outputs.append(paged_attention_batch(query[layer], allocator, requests, layer_index=layer))
            assert allocator.capacity() == counts  # nothing is published before the commit
    torch.cuda.synchronize()
    host_pool = pool.cpu()
    for row, request in enumerate(requests):
        table = list(allocator.block_table(request))
        length = allocator.cached_length(request)
        assert length == lengths[row] + 1
        for layer in (0, 9, 21):
            expected = ref.reference_paged_attention(query[layer, row : row + 1].cpu(), host_pool, layer, table, length)
            assert_max_abs(outputs[layer][row : row + 1], expected, f"row {row} layer {layer}")
    after = allocator.capacity()
    assert after.live_cached_token_slots == counts.live_cached_token_slots + len(lengths)
    for request in requests:
        allocator.release_all(request)
    assert allocator.capacity() == CapacityCounts(300, 300, 0, 0, 0, 0)
