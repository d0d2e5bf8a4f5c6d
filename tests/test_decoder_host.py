"""Host-side behaviour of the batched decoder (no kernel launches): argument checks and
their error types (reference src/pagedcore/decoder.py:113-177), weight stacking, the RoPE
table and the allocator's fused-write checks."""

from __future__ import annotations

import pytest
import torch

from oracle import decoder_reference as dref
from pagedcore_amd import decoder as dec
from pagedcore_amd.engine_types import KVReservation, RequestId
from pagedcore_amd.kv_cache import KVAllocator
from tests.support import CpuCopyWriter


@pytest.fixture(scope="module")
def small():
    weights = dec.random_weights(device="cpu", seed=1, layers=2, vocab=31, intermediate=32)
    return dec.TinyLlamaWeights(weights.embedding, weights.layers * 11, weights.final_norm, weights.lm_head)


def _allocator(lengths=(5,)):
    pool = torch.zeros((22, 2, 8, 16, 4, 64), dtype=torch.float16)
    allocator = KVAllocator(pool, kv_writer=CpuCopyWriter())
    requests = []
    for index, length in enumerate(lengths):
        request = RequestId(f"r{index}")
        allocator.create(KVReservation(request, 2))
        if length:
            allocator.append(request, *[torch.zeros(22, length, 4, 64, dtype=torch.float16)] * 2)
        requests.append(request)
    return allocator, tuple(requests)


def test_random_weights_shapes_and_stacking(small):
    layer = small.layers[0]
    assert small.embedding.shape == small.lm_head.shape == (31, 2048)
    assert layer.q_proj.shape == (2048, 2048) and layer.k_proj.shape == layer.v_proj.shape == (256, 2048)
    assert layer.gate_proj.shape == layer.up_proj.shape == (32, 2048) and layer.down_proj.shape == (2048, 32)
    assert all(t.dtype == torch.float16 for t in (layer.q_proj, layer.input_norm, small.lm_head))
    assert torch.equal(layer.input_norm, torch.ones(2048, dtype=torch.float16))
    fused = dec._fused(layer)
    # views of the stacked storage: no copy
    assert fused.qkv.data_ptr() == layer.q_proj.data_ptr() and fused.qkv.shape == (2560, 2048)
    assert fused.gate_up.data_ptr() == layer.gate_proj.data_ptr() and fused.gate_up.shape == (64, 2048)
    assert torch.equal(fused.qkv[2048:2304], layer.k_proj) and torch.equal(fused.gate_up[32:], layer.up_proj)
    assert dec._fused(layer) is fused


def test_separate_weights_are_concatenated_and_packed(small):
    layer = small.layers[0]
    separate = dec.LayerWeights(**{name: getattr(layer, name).clone() for name in dref._LAYER_FIELDS})
    fused = dec._fused(separate)
    assert fused.qkv.data_ptr() != separate.q_proj.data_ptr()
    assert torch.equal(fused.qkv, dec._fused(layer).qkv)
    packed = dec.pack_weights(dec.TinyLlamaWeights(small.embedding, (separate,) * 22, small.final_norm, small.lm_head))
    assert dec._fused(packed.layers[0]).qkv.data_ptr() == packed.layers[0].q_proj.data_ptr()


def test_rope_table_is_the_reference_expression():
    table = dec.rope_table(torch.device("cpu"))
    cosine, sine = dref.rope_cos_sin(torch.arange(2048)[None], torch.float16)
    assert torch.equal(table[:, 0], cosine[0, 0, :, :32]) and torch.equal(table[:, 1], sine[0, 0, :, :32])
    assert table.is_contiguous() and dec.rope_table(torch.device("cpu")) is table


def test_decode_paged_argument_checks(small):
    allocator, requests = _allocator((5, 7))
    good = torch.tensor([[1], [2]])
    with pytest.raises(ValueError, match=r"int64 \[batch, 1\]"):
        dec.decode_paged(good.int(), small, allocator, requests)
    with pytest.raises(ValueError, match=r"int64 \[batch, 1\]"):
        dec.decode_paged(good[:1], small, allocator, requests)
    with pytest.raises(ValueError, match="22 decoder layers"):
        dec.decode_paged(good, dec.TinyLlamaWeights(small.embedding, small.layers[:2], small.final_norm, small.lm_head), allocator, requests)
    with pytest.raises(KeyError):
        dec.decode_paged(good, small, allocator, (requests[0], RequestId("unknown")))
    counts = allocator.capacity()
    # no CPU fallback: a CPU pool is refused before anything is staged
    with pytest.raises(RuntimeError, match="runs on the GPU"):
        dec.decode_paged(good, small, allocator, requests)
    assert allocator.capacity() == counts and allocator._decode_appends is None
    assert [allocator.cached_length(r) for r in requests] == [5, 7]


def test_prefill_paged_argument_checks(small):
    allocator, (request, empty) = _allocator((5, 0))
    ids = torch.tensor([[1, 2, 3]])
    with pytest.raises(ValueError, match="empty request cache"):
        dec.prefill_paged(ids, small, allocator, request)
    with pytest.raises(ValueError, match=r"int64 \[1, tokens\]"):
        dec.prefill_paged(ids.repeat(2, 1), small, allocator, empty)
    with pytest.raises(ValueError, match="1 to 2048"):
        dec.prefill_paged(torch.zeros(1, 2049, dtype=torch.int64), small, allocator, empty)
    with pytest.raises(ValueError, match="22 decoder layers"):
        dec.prefill_paged(ids, dec.TinyLlamaWeights(small.embedding, small.layers[:3], small.final_norm, small.lm_head), allocator, empty)
    with pytest.raises(KeyError):
        dec.prefill_paged(ids, small, allocator, RequestId("unknown"))
    with pytest.raises(RuntimeError, match="runs on the GPU"):
        dec.prefill_paged(ids, small, allocator, empty)
    assert allocator.cached_length(empty) == 0


def test_fused_decode_write_checks_before_any_write():
    allocator, requests = _allocator((5, 16))
    table = dec.rope_table(torch.device("cpu"))
    qkv = torch.zeros(2, 2560, dtype=torch.float16)
    with pytest.raises(RuntimeError, match="staged append"):
        allocator.write_decode_layers_rotary(requests, 0, qkv, table)
    counts = allocator.capacity()
    with pytest.raises(RuntimeError, match="every cache layer"), allocator.append_decode(requests):
        with pytest.raises(ValueError, match="written once in order"):
            allocator.write_decode_layers_rotary(requests, 1, qkv, table)
        with pytest.raises(ValueError, match="qkv"):
            allocator.write_decode_layers_rotary(requests, 0, qkv[:, :2552], table)
        with pytest.raises(ValueError, match="qkv"):
            allocator.write_decode_layers_rotary(requests, 0, qkv.float(), table)
        with pytest.raises(ValueError, match="rope_table"):
            allocator.write_decode_layers_rotary(requests, 0, qkv, table[:100])
        with pytest.raises(ValueError, match="distinct"):
            allocator.write_decode_layers_rotary((requests[0], requests[0]), 0, qkv, table)
        with pytest.raises(RuntimeError, match="does not rotate"):
            allocator.write_decode_layers_rotary(requests, 0, qkv, table)
        assert all(append.written_layers == 0 for append in allocator._decode_appends.values())
        slots, positions = allocator._decode_slots(requests, [allocator._decode_appends[r] for r in requests])
        # position = cached length before the step; slot = its block * 16 + offset
        assert positions.tolist() == [5, 16]
        assert slots.tolist() == [allocator.block_table(requests[0])[0] * 16 + 5, allocator._decode_appends[requests[1]].sequence.blocks[1] * 16]
    assert allocator.capacity() == counts
