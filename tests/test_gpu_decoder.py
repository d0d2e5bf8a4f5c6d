"""The batched decode step on the GPU: its three elementwise kernels against the oracle's
torch expressions, then decode_paged / prefill_paged against the contiguous CPU forward
(the reference's own expectation, tests/unit/test_decoder.py:114-195: logits within 5e-3,
cached K/V within 2e-3, old slots bit-identical)."""

from __future__ import annotations

from types import SimpleNamespace

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import decoder_reference as dref
from pagedcore_amd import _hip
from pagedcore_amd import decoder as dec
from pagedcore_amd.engine_types import CapacityCounts, KVReservation, RequestId
from pagedcore_amd.kv_cache import KVAllocator

pytestmark = pytest.mark.gpu


def _bits(tensor: torch.Tensor) -> np.ndarray:
    return tensor.detach().cpu().contiguous().view(torch.int16).numpy()


def _ulps(got: torch.Tensor, expected: torch.Tensor) -> int:
    """Largest distance in fp16 units in the last place (same-sign values)."""
    a = _bits(got).astype(np.int32)
    b = _bits(expected).astype(np.int32)
    a = np.where(a < 0, -(a & 0x7FFF), a)
    b = np.where(b < 0, -(b & 0x7FFF), b)
    return int(np.abs(a - b).max()) if a.size else 0


# ---------------------------------------------------------------------------------------
# Kernels
# ---------------------------------------------------------------------------------------


def test_rope_table_matches_the_oracle(device):
    table = dec.rope_table(device).cpu()
    assert table.shape == (2048, 2, 32) and table.dtype == torch.float16
    cosine, sine = dref.rope_cos_sin(torch.arange(2048)[None], torch.float16)
    assert torch.equal(table[:, 0], cosine[0, 0, :, :32]) and torch.equal(table[:, 1], sine[0, 0, :, :32])
    assert torch.equal(cosine[0, 0, :, :32], cosine[0, 0, :, 32:])


@pytest.mark.parametrize("tokens,stride", [(1, 2560), (7, 2560), (300, 2568)])
def test_rope_kv_append_is_bit_exact(device, tokens, stride):
    """Rotated q/k equal the reference rotation (dense.py:56-59) evaluated by torch with the
    same fp16 cos/sin values, bit for bit; K and V land in their slots and nothing else in
    the pool changes."""
    gen = torch.Generator(device=device).manual_seed(tokens)
    qkv = torch.randn(tokens, stride, dtype=torch.float16, device=device, generator=gen)
    positions = torch.randint(0, 2048, (tokens,), device=device, generator=gen)
    positions[0] = 0
    if tokens > 1:
        positions[1] = 2047
    blocks = 40
    pool = torch.full((22, 2, blocks, 16, 4, 64), float("nan"), dtype=torch.float16, device=device)
    slots = torch.randperm(blocks * 16, device=device, generator=gen)[:tokens]
    if tokens > 2:
        slots[2] = -1  # skipped token
    table = dec.rope_table(device)
    query = torch.empty(tokens, 32, 64, dtype=torch.float16, device=device)
    keys = torch.empty(tokens, 4, 64, dtype=torch.float16, device=device)
    values = torch.empty_like(keys)
    _hip.rope_kv_append(query, qkv, positions, table, key_out=keys, value_out=values, pool=pool, layer=5,
                        slot_mapping=slots)
    torch.cuda.synchronize()

    host = qkv.cpu()
    t = table.cpu()[positions.cpu()]  # [tokens, 2, 32]
    cosine = torch.cat((t[:, 0], t[:, 0]), dim=-1)[:, None, :]
    sine = torch.cat((t[:, 1], t[:, 1]), dim=-1)[:, None, :]
    expected_q = dref.rotate(host[:, :2048].reshape(tokens, 32, 64), cosine, sine)
    expected_k = dref.rotate(host[:, 2048:2304].reshape(tokens, 4, 64), cosine, sine)
    expected_v = host[:, 2304:2560].reshape(tokens, 4, 64)
    assert np.array_equal(_bits(query), _bits(expected_q))
    assert np.array_equal(_bits(keys), _bits(expected_k))
    assert np.array_equal(_bits(values), _bits(expected_v))

    host_pool = pool.cpu()
    written = torch.zeros(22, 2, blocks * 16, dtype=torch.bool)
    for token, slot in enumerate(slots.cpu().tolist()):
        if slot < 0:
            continue
        block, offset = divmod(slot, 16)
        assert np.array_equal(_bits(host_pool[5, 0, block, offset]), _bits(expected_k[token]))
        assert np.array_equal(_bits(host_pool[5, 1, block, offset]), _bits(expected_v[token]))
        written[5, :, slot] = True
    untouched = host_pool.view(22, 2, blocks * 16, 256)[~written]
    assert torch.isnan(untouched).all()


def test_rope_kv_append_rejects_bad_arguments_without_a_gpu_launch(device):
    lib = _hip.load()
    q = torch.empty(2, 32, 64, dtype=torch.float16, device=device)
    qkv = torch.empty(2, 2560, dtype=torch.float16, device=device)
    pos = torch.zeros(2, dtype=torch.int64, device=device)
    table = dec.rope_table(device)
    call = lambda **kw: lib.pc_rope_kv_append(  # noqa: E731
        kw.get("q", q.data_ptr()), None, None, qkv.data_ptr(), kw.get("stride", 2560), pos.data_ptr(),
        table.data_ptr(), 2048, kw.get("pool"), 4, kw.get("layer", 0), kw.get("slots"), 2, None,
    )
    assert call(stride=2552) == 1 and b"qkv_stride" in lib.pc_last_error()
    assert call(q=q.data_ptr() + 2) == 1 and b"aligned" in lib.pc_last_error()
    assert call(pool=q.data_ptr()) == 1 and b"both" in lib.pc_last_error()
    assert call(pool=q.data_ptr(), slots=pos.data_ptr(), layer=22) == 1 and b"layer" in lib.pc_last_error()


@pytest.mark.parametrize("rows,width,with_delta", [(1, 2048, False), (7, 2048, True), (3, 8192, True), (5, 520, True), (0, 2048, True)])
def test_add_rms_norm_matches_the_oracle(device, rows, width, with_delta):
    gen = torch.Generator(device=device).manual_seed(rows * 1000 + width)
    hidden = (torch.randn(rows, width, device=device, generator=gen) * 3).half()
    delta = torch.randn(rows, width, device=device, generator=gen).half() if with_delta else None
    weight = (1 + 0.2 * torch.randn(width, device=device, generator=gen)).half()
    out = torch.empty_like(hidden)
    expected_hidden = hidden.cpu() + delta.cpu() if with_delta else hidden.cpu()
    _hip.add_rms_norm(out, hidden, delta, weight)
    torch.cuda.synchronize()
    assert np.array_equal(_bits(hidden), _bits(expected_hidden))  # fp16 residual sum, in place
    expected = dref.rms_norm(expected_hidden, weight.cpu())
    assert _ulps(out, expected) <= 1  # only the fp32 sum order differs


def test_silu_mul_matches_torch(device):
    gen = torch.Generator(device=device).manual_seed(9)
    gate_up = (torch.randn(9, 2 * 5632, device=device, generator=gen) * 4).half()
    out = torch.empty(9, 5632, dtype=torch.float16, device=device)
    _hip.silu_mul(out, gate_up)
    torch.cuda.synchronize()
    host = gate_up.cpu()
    expected = F.silu(host[:, :5632]) * host[:, 5632:]
    assert _ulps(out, expected) <= 1


# ---------------------------------------------------------------------------------------
# Decode step and prefill
#
# Error model. The reference's decoder tolerances (logits 5e-3, K/V 2e-3) compare two paths
# that run the same GEMMs on the same device. Here the expectation is the CPU forward, whose
# fp16 GEMM outputs round differently from hipBLASLt's (fp32 sums in another order); through
# 22 layers that noise reaches the reference's tolerances. So the tests (1) hold the decode
# step to 5e-3 / 2e-3 with the oracle started from the GPU's own cache, as in the
# reference's test, where prefill is exact; (2) hold layer 0 of prefill (no attention noise
# upstream) to 2e-3; and (3) everywhere else require the GPU to be as close to an fp32
# evaluation of the same weights as the reference's own fp16 computation is:
#     max|gpu - fp32| <= 1.25 * max|cpu fp16 - fp32| + 2e-3.
# A real defect (wrong position, norm, head map or slot) misses every one of these by far.
# ---------------------------------------------------------------------------------------


def _synthetic(device):
    """The reference test's synthetic geometry: hidden 2048, 32/4 heads, MLP 32, vocab 31,
    two distinct layers repeated 11 times to fill the pool's 22 layers."""
    small = dec.random_weights(device=device, seed=11, layers=2, vocab=31, intermediate=32, norm_std=0.1)
    return dec.TinyLlamaWeights(small.embedding, small.layers * 11, small.final_norm, small.lm_head)


def _cpu(weights):
    return dref.to_cpu(weights, dec.LayerWeights, dec.TinyLlamaWeights)


def _fp32(host_weights):
    layers = tuple(
        SimpleNamespace(**{name: getattr(layer, name).float() for name in dref._LAYER_FIELDS}) for layer in host_weights.layers
    )
    return SimpleNamespace(
        embedding=host_weights.embedding.float(), layers=layers, final_norm=host_weights.final_norm.float(),
        lm_head=host_weights.lm_head.float(),
    )


def _gap(a, b) -> float:
    return (a.float().cpu() - b.float().cpu()).abs().max().item()


def _as_accurate(gpu, cpu16, fp32) -> None:
    assert _gap(gpu, fp32) <= 1.25 * _gap(cpu16, fp32) + 2e-3, (_gap(gpu, fp32), _gap(cpu16, fp32))


def _pool_cache(allocator, request):
    """The request's cached K/V as the contiguous forward holds them: per layer
    ([1, 4, length, 64], [1, 4, length, 64]) on the CPU."""
    length = allocator.cached_length(request)
    layers = []
    for layer in range(22):
        pair = []
        for kind in range(2):
            rows = torch.cat([allocator.pool[layer, kind, block] for block in allocator.block_table(request)])[:length]
            pair.append(rows.cpu().transpose(0, 1)[None])
        layers.append(tuple(pair))
    return layers


@pytest.mark.parametrize("lengths", [(1, 15, 16, 17, 49)])
def test_prefill_paged_matches_the_contiguous_prefill(device, lengths):
    weights = _synthetic(device)
    host_weights = _cpu(weights)
    exact = _fp32(host_weights)
    pool = torch.full((22, 2, 16, 16, 4, 64), float("nan"), dtype=torch.float16, device=device)
    allocator = KVAllocator(pool)
    for row, length in enumerate(lengths):
        request = RequestId(str(row))
        allocator.create(KVReservation(request, (length + 15) // 16))
        ids = (torch.arange(length)[None] + length) % 31
        expected_logits, cache = dref.prefill(ids, host_weights)
        exact_logits, exact_cache = dref.forward(ids, exact)
        before = pool.cpu()
        logits = dec.prefill_paged(ids.to(device), weights, allocator, request)
        assert logits.shape == (1, length, 31) and logits.dtype == torch.float16
        torch.testing.assert_close(logits.cpu(), expected_logits, atol=5e-3, rtol=5e-3)
        _as_accurate(logits, expected_logits, exact_logits)
        assert allocator.cached_length(request) == length
        got = _pool_cache(allocator, request)
        for layer in range(22):
            for kind in range(2):
                if layer == 0:
                    torch.testing.assert_close(got[0][kind], cache[0][kind], atol=2e-3, rtol=2e-3)
                _as_accurate(got[layer][kind], cache[layer][kind], exact_cache[layer][kind])
        # slots past the prompt and blocks of no request keep their poison
        after = pool.cpu()
        table = allocator.block_table(request)
        tail = length - (len(table) - 1) * 16
        assert torch.isnan(after[:, :, table[-1], tail:]).all()
        others = [b for b in range(16) if b not in table]
        assert torch.equal(after[:, :, others].isnan(), before[:, :, others].isnan())


@pytest.mark.parametrize("lengths", [(15,), (1, 15, 16, 17, 49)])
def test_decode_paged_matches_the_contiguous_fp32_decode(device, lengths):
    """tests/unit/test_decoder.py:114-195: two steps (the second in reverse request order);
    per row the logits within 5e-3 and the new K/V within 2e-3 of decode(fp32_attention=True)
    started from the same cache; old slots bit-identical; accounting as the reference."""
    weights = _synthetic(device)
    host_weights = _cpu(weights)
    pool = torch.full((22, 2, 16, 16, 4, 64), float("nan"), dtype=torch.float16, device=device)
    allocator = KVAllocator(pool)
    requests = tuple(RequestId(str(row)) for row in range(len(lengths)))
    for request, length in zip(requests, lengths):
        allocator.create(KVReservation(request, (length + 2 + 15) // 16))
        dec.prefill_paged(((torch.arange(length)[None] + length) % 31).to(device), weights, allocator, request)
    pointer = pool.untyped_storage().data_ptr()
    counts = allocator.capacity()
    for step in range(2):
        order = requests if step == 0 else requests[::-1]
        tokens = torch.tensor([[2 + step + int(request)] for request in order])
        caches = {request: _pool_cache(allocator, request) for request in order}
        expected = [dref.decode_fp32(tokens[row : row + 1], caches[request], host_weights) for row, request in enumerate(order)]
        before = pool.cpu()
        logits = dec.decode_paged(tokens.to(device), weights, allocator, order)
        torch.cuda.synchronize()
        assert logits.shape == (len(order), 1, 31) and logits.dtype == torch.float16
        assert torch.isfinite(logits).all()
        for row, request in enumerate(order):
            expected_logits, cache = expected[row]
            old_length = caches[request][0][0].shape[2]
            torch.testing.assert_close(logits[row : row + 1].cpu(), expected_logits, atol=5e-3, rtol=5e-3)
            assert allocator.cached_length(request) == old_length + 1
            got = _pool_cache(allocator, request)
            for layer in range(22):
                for kind in range(2):
                    # old positions untouched, the new one within 2e-3
                    assert torch.equal(got[layer][kind][:, :, :old_length], caches[request][layer][kind])
                    torch.testing.assert_close(
                        got[layer][kind][:, :, old_length], cache[layer][kind][:, :, old_length], atol=2e-3, rtol=2e-3
                    )
            table = allocator.block_table(request)
            block, slot = divmod(old_length, 16)
            after = pool.cpu()
            # the rest of the new token's block is still the poison it held before
            assert torch.equal(after[:, :, table[block], slot + 1 :].isnan(), before[:, :, table[block], slot + 1 :].isnan())
        current = allocator.capacity()
        assert current.live_cached_token_slots == sum(lengths) + len(order) * (step + 1)
        assert current.reserved_blocks == counts.reserved_blocks
        assert current.active_slots == len(order)
        assert pool.untyped_storage().data_ptr() == pointer
    for request in requests:
        allocator.release_all(request)
    assert allocator.capacity() == CapacityCounts(16, 16, 0, 0, 0, 0)


def test_full_size_decode_is_as_accurate_as_the_reference_computation(device):
    """22 distinct full-size layers (MLP 5632, vocab 32000, random N(0, 0.02) weights, norm
    weights 1 + N(0, 0.1)): prefill and decode logits are as close to the fp32 evaluation
    as the CPU fp16 forward is, and the greedy token agrees wherever the fp32 top-2 margin
    exceeds that noise."""
    weights = dec.random_weights(device=device, seed=5, norm_std=0.1)
    host_weights = _cpu(weights)
    exact = _fp32(host_weights)
    lengths = (3, 17, 40)
    pool = torch.full((22, 2, 12, 16, 4, 64), float("nan"), dtype=torch.float16, device=device)
    allocator = KVAllocator(pool)
    requests = tuple(RequestId(f"full{row}") for row in range(len(lengths)))
    gen = torch.Generator().manual_seed(2)
    for request, length in zip(requests, lengths):
        allocator.create(KVReservation(request, (length + 1 + 15) // 16))
        ids = torch.randint(0, 32000, (1, length), generator=gen)
        logits = dec.prefill_paged(ids.to(device), weights, allocator, request)
        _as_accurate(logits, dref.prefill(ids, host_weights)[0], dref.forward(ids, exact)[0])
    tokens = torch.randint(0, 32000, (len(lengths), 1), generator=gen)
    caches = {request: _pool_cache(allocator, request) for request in requests}
    logits = dec.decode_paged(tokens.to(device), weights, allocator, requests)
    for row, request in enumerate(requests):
        cpu16 = dref.decode_fp32(tokens[row : row + 1], caches[request], host_weights)[0]
        fp32 = dref.forward(tokens[row : row + 1], exact, [(k.float(), v.float()) for k, v in caches[request]], fp32_attention=True)[0]
        _as_accurate(logits[row : row + 1], cpu16, fp32)
        top = fp32.flatten().topk(2).values
        if float(top[0] - top[1]) > 4 * _gap(cpu16, fp32):
            assert int(logits[row].argmax()) == int(fp32.argmax())


def test_decode_paged_rows_do_not_depend_on_batch_composition(device):
    """tests/unit/test_decoder.py:198-239: decoding requests together or one at a time gives
    bit-identical logits and cached K/V (the GEMM kernels chosen for these row counts sum
    each output in the same order)."""
    weights = _synthetic(device)
    requests = tuple(RequestId(str(row)) for row in range(3))
    pools = [torch.full((22, 2, 12, 16, 4, 64), float("nan"), dtype=torch.float16, device=device) for _ in range(2)]
    separate, batched = (KVAllocator(pool) for pool in pools)
    for request, length in zip(requests, (1, 16, 49)):
        ids = (torch.arange(length)[None] % 31).to(device)
        for allocator in (separate, batched):
            allocator.create(KVReservation(request, (length + 18) // 16))
            dec.prefill_paged(ids, weights, allocator, request)
    for step in range(3):
        order = requests if step % 2 == 0 else requests[::-1]
        tokens = torch.tensor([[3 + int(request) + step] for request in order], device=device)
        expected = torch.cat([dec.decode_paged(tokens[row : row + 1], weights, separate, (request,)) for row, request in enumerate(order)])
        actual = dec.decode_paged(tokens, weights, batched, order)
        torch.testing.assert_close(actual, expected, atol=0, rtol=0)
        assert torch.equal(actual.argmax(-1), expected.argmax(-1))
        assert batched.capacity() == separate.capacity()
        for request in order:
            assert batched.cached_length(request) == separate.cached_length(request)
            for block in range(len(batched.block_table(request))):
                for actual_kv, expected_kv in zip(batched.read_block(request, block), separate.read_block(request, block)):
                    torch.testing.assert_close(actual_kv, expected_kv, atol=0, rtol=0)


@pytest.mark.parametrize("failure", ["raised", "device fault"])
def test_decode_paged_failure_discards_the_step(device, monkeypatch, failure):
    """A failure inside the step (attention of layer 3 raising, or reporting a device fault
    through its workspace's fault word, forced from the host here, which the step reads
    before it commits) leaves lengths, tables, counts and every published slot unchanged,
    and the step can be retried (tests/unit/test_decoder.py:298-360). The device fault
    surfaces as AttentionFaultError and leaves the workspace zeroed."""
    weights = _synthetic(device)
    pool = torch.full((22, 2, 6, 16, 4, 64), float("nan"), dtype=torch.float16, device=device)
    allocator = KVAllocator(pool)
    requests = (RequestId("first"), RequestId("second"))
    for request, length in zip(requests, (15, 16)):
        allocator.create(KVReservation(request, 2))
        dec.prefill_paged((torch.arange(length)[None] % 31).to(device), weights, allocator, request)
    counts = allocator.capacity()
    tables = [allocator.block_table(request) for request in requests]
    published = pool.clone()
    calls = 0
    original = dec.attend_rows
    faulted = []

    def failing(*args, **kwargs):
        nonlocal calls
        calls += 1
        if calls == 4:
            if failure == "raised":
                raise RuntimeError("injected decode failure")
            out, workspace = original(*args, **kwargs)
            _hip.fault_word(workspace).fill_(_hip.FAULT_FOREIGN_XCD)  # as a merge would record it
            faulted.append(workspace)
            return out, workspace
        return original(*args, **kwargs)

    tokens = torch.tensor([[3], [4]], device=device)
    monkeypatch.setattr(dec, "attend_rows", failing)
    expected = (RuntimeError, "injected") if failure == "raised" else (_hip.AttentionFaultError, "another XCD")
    with pytest.raises(expected[0], match=expected[1]):
        dec.decode_paged(tokens, weights, allocator, requests)
    monkeypatch.setattr(dec, "attend_rows", original)
    for workspace in faulted:
        assert not workspace.any().item()  # zeroed by the fault check
    assert allocator.capacity() == counts
    assert [allocator.block_table(request) for request in requests] == tables
    for request, length in zip(requests, (15, 16)):
        assert allocator.cached_length(request) == length
        for logical, physical in enumerate(allocator.block_table(request)):
            valid = min(16, length - logical * 16)
            assert torch.equal(pool[:, :, physical, :valid].cpu(), published[:, :, physical, :valid].cpu())
    logits = dec.decode_paged(tokens, weights, allocator, requests)
    assert torch.isfinite(logits).all()
    assert [allocator.cached_length(request) for request in requests] == [16, 17]


def test_decode_graph_replays_equal_decode_paged(device):
    """DecodeGraph (one captured HIP graph per step) against eager decode_paged on a twin
    pool: bit-identical logits and pool bytes over several steps, with the request order
    changing and a request replaced between steps, eager GPU work and synchronizations in
    between replays."""
    weights = _synthetic(device)
    lengths = (1, 15, 16, 17, 49, 200, 2040)
    pools = [torch.full((22, 2, 176, 16, 4, 64), float("nan"), dtype=torch.float16, device=device) for _ in range(2)]
    eager, graphed = (KVAllocator(pool) for pool in pools)
    requests = [RequestId(f"g{row}") for row in range(len(lengths))]

    def admit(request, length):
        ids = ((torch.arange(length)[None] * 3 + length) % 31).to(device)
        for allocator in (eager, graphed):
            allocator.create(KVReservation(request, (length + 6 + 15) // 16))
            dec.prefill_paged(ids, weights, allocator, request)

    for request, length in zip(requests, lengths):
        admit(request, length)
    graph = dec.DecodeGraph(weights, graphed, batch=len(lengths))
    with pytest.raises(ValueError, match="batches of 1 to 7"):
        graph.step(torch.zeros((8, 1), dtype=torch.int64, device=device), tuple(RequestId(f"x{i}") for i in range(8)))
    for step in range(5):
        if step == 3:  # replace a request between steps
            for allocator in (eager, graphed):
                allocator.release_all(requests[2])
            requests[2] = RequestId("late")
            admit(requests[2], 33)
        order = tuple(requests) if step % 2 == 0 else tuple(reversed(requests))
        tokens = torch.tensor([[(5 * step + row) % 31] for row in range(len(order))], device=device)
        expected = dec.decode_paged(tokens, weights, eager, order)
        got = graph.step(tokens, order)
        torch.cuda.synchronize()
        assert torch.equal(got, expected)
        assert torch.equal(pools[0].view(torch.int16), pools[1].view(torch.int16))
        assert graphed.capacity() == eager.capacity()
        assert [graphed.cached_length(r) for r in order] == [eager.cached_length(r) for r in order]
        torch.randn(1000, device=device).sum().item()  # unrelated eager work between replays


def test_decode_graph_pads_smaller_batches(device):
    """A DecodeGraph of 6 rows stepping 1, 4, 6 and 3 requests against eager decode_paged on
    a twin pool: the padding rows write nothing (every pool byte outside the real rows'
    new slots, NaN poison included, stays identical) and the real rows' logits and new K/V
    agree within the reference's tolerances (the GEMMs run at 6 rows instead of the batch
    size), with the same greedy tokens and the same allocator state."""
    weights = _synthetic(device)
    lengths = (3, 16, 40, 77, 130, 200)
    pools = [torch.full((22, 2, 80, 16, 4, 64), float("nan"), dtype=torch.float16, device=device) for _ in range(2)]
    eager, graphed = (KVAllocator(pool) for pool in pools)
    requests = [RequestId(f"p{row}") for row in range(len(lengths))]
    for request, length in zip(requests, lengths):
        ids = ((torch.arange(length)[None] * 7 + length) % 31).to(device)
        for allocator in (eager, graphed):
            allocator.create(KVReservation(request, (length + 4 + 15) // 16))
            dec.prefill_paged(ids, weights, allocator, request)
    graph = dec.DecodeGraph(weights, graphed, batch=6)
    for step, rows in enumerate((1, 4, 6, 3)):
        order = tuple(requests[(step + row) % 6] for row in range(rows))
        tokens = torch.tensor([[(3 * step + row) % 31] for row in range(rows)], device=device)
        before = pools[1].clone()
        expected = dec.decode_paged(tokens, weights, eager, order)
        got = graph.step(tokens, order)
        torch.cuda.synchronize()
        assert got.shape == expected.shape == (rows, 1, 31)
        torch.testing.assert_close(got, expected, atol=5e-3, rtol=5e-3)
        assert torch.equal(got.argmax(-1), expected.argmax(-1))
        assert graphed.capacity() == eager.capacity()
        written = torch.zeros(pools[1].shape[2:4], dtype=torch.bool, device=device)
        for request in order:
            length = graphed.cached_length(request)
            assert length == eager.cached_length(request)
            assert graphed.block_table(request) == eager.block_table(request)
            block, slot = divmod(length - 1, 16)
            written[graphed.block_table(request)[block], slot] = True
        untouched = ~written
        assert torch.equal(pools[1][:, :, untouched].view(torch.int16), before[:, :, untouched].view(torch.int16))
        torch.testing.assert_close(pools[1][:, :, written], pools[0][:, :, written], atol=2e-3, rtol=2e-3)
        torch.randn(1000, device=device).sum().item()  # unrelated eager work between replays


def test_prefill_graph_matches_prefill_paged(device):
    """A 128-position PrefillGraph against prefill_paged on a twin pool for prompts of 1, 16,
    37, 100 and 128 positions: the same tables, lengths and counts, and every pool byte
    outside the prompt's slots (NaN poison included) untouched. The last position's
    logits and the cached K/V meet the bars prefill_paged's own test applies against the
    oracle (its GEMMs run at 128 rows, so the two paths differ by rounding): logits within
    5e-3, layer-0 K/V within 2e-3, every layer as accurate as the CPU fp16 forward
    against fp32. Errors leave nothing staged."""
    weights = _synthetic(device)
    host_weights = _cpu(weights)
    exact = _fp32(host_weights)
    pools = [torch.full((22, 2, 40, 16, 4, 64), float("nan"), dtype=torch.float16, device=device) for _ in range(2)]
    eager, graphed = (KVAllocator(pool) for pool in pools)
    graph = dec.PrefillGraph(weights, graphed, 128)
    for index, length in enumerate((1, 16, 37, 100, 128)):
        request = RequestId(f"q{index}")
        for allocator in (eager, graphed):
            allocator.create(KVReservation(request, (length + 15) // 16))
        ids = (torch.arange(length)[None] * 5 + index) % 31
        expected_logits, cache = dref.prefill(ids, host_weights)
        exact_logits, exact_cache = dref.forward(ids, exact)
        before = pools[1].clone()
        eager_logits = dec.prefill_paged(ids.to(device), weights, eager, request)
        got = graph.step(ids.to(device), request)
        torch.cuda.synchronize()
        assert got.shape == (1, 1, 31) and got.dtype == torch.float16
        torch.testing.assert_close(got.cpu(), expected_logits[:, -1:], atol=5e-3, rtol=5e-3)
        _as_accurate(got, expected_logits[:, -1:], exact_logits[:, -1:])
        torch.testing.assert_close(got[0, 0], eager_logits[0, -1], atol=5e-3, rtol=5e-3)
        assert graphed.capacity() == eager.capacity()
        assert graphed.cached_length(request) == eager.cached_length(request) == length
        assert graphed.block_table(request) == eager.block_table(request)
        cached = _pool_cache(graphed, request)
        for layer in range(22):
            for kind in range(2):
                if layer == 0:
                    torch.testing.assert_close(cached[0][kind], cache[0][kind], atol=2e-3, rtol=2e-3)
                _as_accurate(cached[layer][kind], cache[layer][kind], exact_cache[layer][kind])
        written = torch.zeros(pools[1].shape[2:4], dtype=torch.bool, device=device)
        for position in range(length):
            block, slot = divmod(position, 16)
            written[graphed.block_table(request)[block], slot] = True
        assert torch.equal(pools[1][:, :, ~written].view(torch.int16), before[:, :, ~written].view(torch.int16))
        torch.randn(1000, device=device).sum().item()  # unrelated eager work between replays
    counts = graphed.capacity()
    graphed.create(KVReservation(RequestId("long"), 9))
    with pytest.raises(ValueError, match="1 to 128 positions"):
        graph.step(torch.zeros((1, 129), dtype=torch.int64, device=device), RequestId("long"))
    with pytest.raises(ValueError, match="empty request cache"):
        graph.step(torch.zeros((1, 4), dtype=torch.int64, device=device), RequestId("q1"))
    graphed.create(KVReservation(RequestId("small"), 1))
    with pytest.raises(RuntimeError, match="reservation"):
        graph.step(torch.zeros((1, 17), dtype=torch.int64, device=device), RequestId("small"))
    assert graphed.cached_length(RequestId("long")) == graphed.cached_length(RequestId("small")) == 0
    assert graphed.capacity().owned_blocks == counts.owned_blocks


def test_capture_graph_replays_and_reports_the_callables_error(device):
    """decoder.capture_graph (the graphs' capture, which leaves torch's allocator cache
    alone): a capture whose callable raises reports that error and leaves the stream usable;
    a normal capture's outputs are refreshed by every replay, with eager work in between."""
    def failing():
        torch.empty(4, device=device).fill_(1.0)  # a launch inside the capture
        raise ValueError("inside the capture")

    with pytest.raises(ValueError, match="inside the capture"):
        dec.capture_graph(failing, device)
    source = torch.zeros(4, device=device)
    graph, out = dec.capture_graph(lambda: source * 2 + 1, device)
    for value in (1.0, 5.0, -3.0):
        source.fill_(value)
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, torch.full((4,), 2 * value + 1, device=device))
        torch.randn(1000, device=device).sum().item()  # unrelated eager work between replays


def test_graph_greedy_paths_equal_step_argmax(device):
    """PrefillGraph.greedy and DecodeGraph.greedy (host ids in, each row's argmax out) on
    one pool against step() followed by argmax on a twin pool: the same selected ids, the
    same pool bytes and allocator state, over prompts of several lengths and decode steps
    of 2, 5 and 3 rows (padding) with one row's id taken from the device, eager GPU work
    between replays. Bad ids are rejected before anything is staged."""
    weights = _synthetic(device)
    pools = [torch.full((22, 2, 60, 16, 4, 64), float("nan"), dtype=torch.float16, device=device) for _ in range(2)]
    by_step, by_greedy = (KVAllocator(pool) for pool in pools)
    prefills = [dec.PrefillGraph(weights, allocator, 64) for allocator in (by_step, by_greedy)]
    requests = [RequestId(f"s{index}") for index in range(5)]
    first = {}
    for index, (request, length) in enumerate(zip(requests, (1, 9, 16, 40, 64))):
        for allocator in (by_step, by_greedy):
            allocator.create(KVReservation(request, (length + 8 + 15) // 16))
        prompt = (np.arange(length, dtype=np.int64) * 7 + index) % 31
        logits = prefills[0].step(torch.from_numpy(prompt).view(1, -1).to(device), request)
        token = prefills[1].greedy(prompt, request)
        torch.cuda.synchronize()
        assert token.dtype == torch.int64 and token.ndim == 0
        assert int(token) == int(logits[0, 0].argmax())
        first[request] = token
        torch.randn(1000, device=device).sum().item()  # unrelated eager work between replays
    assert torch.equal(pools[0].view(torch.int16), pools[1].view(torch.int16))
    assert by_step.capacity() == by_greedy.capacity()
    spare = RequestId("spare")
    by_greedy.create(KVReservation(spare, 1))
    with pytest.raises(ValueError, match="vocabulary"):
        prefills[1].greedy(np.array([3, 31], dtype=np.int64), spare)
    with pytest.raises(ValueError, match="int64"):
        prefills[1].greedy(np.array([3, 4], dtype=np.int32), spare)
    assert by_greedy.cached_length(spare) == 0
    by_greedy.release_all(spare)

    decodes = [dec.DecodeGraph(weights, allocator, 5) for allocator in (by_step, by_greedy)]
    for step, rows in enumerate((2, 5, 3)):
        order = tuple(requests[(step + row) % 5] for row in range(rows))
        ids = np.array([(4 * step + row) % 31 for row in range(rows)], dtype=np.int64)
        row = rows - 1  # this row's id comes from the device: its prefill's selection
        tokens = torch.from_numpy(ids.copy()).view(-1, 1).to(device)
        tokens[row, 0] = first[order[row]]
        expected = decodes[0].step(tokens, order)[:, -1].argmax(-1)
        got = decodes[1].greedy(ids, order, (row, first[order[row]]))
        torch.cuda.synchronize()
        decodes[0].check_faults()
        decodes[1].check_faults()
        assert got.dtype == torch.int64 and got.shape == (rows,)
        assert torch.equal(got, expected)
        assert torch.equal(pools[0].view(torch.int16), pools[1].view(torch.int16))
        assert by_step.capacity() == by_greedy.capacity()
        assert [by_greedy.cached_length(r) for r in order] == [by_step.cached_length(r) for r in order]
        torch.randn(1000, device=device).sum().item()
    lengths = [by_greedy.cached_length(r) for r in requests]
    for bad, match in (
        (np.array([0, 31], dtype=np.int64), "vocabulary"),
        (np.array([0, 1, 2], dtype=np.int64), "matching request IDs"),
        (np.array([0, 1], dtype=np.int32), "matching request IDs"),
    ):
        with pytest.raises(ValueError, match=match):
            decodes[1].greedy(bad, tuple(requests[:2]))
    with pytest.raises(ValueError, match="outside the batch"):
        decodes[1].greedy(np.array([0, 1], dtype=np.int64), tuple(requests[:2]), (2, first[requests[0]]))
    assert [by_greedy.cached_length(r) for r in requests] == lengths


# ---------------------------------------------------------------------------------------
# Prompt attention (pc_prefill_attention)
# ---------------------------------------------------------------------------------------


def _causal_fp64(query, key, value):
    """FP64 causal GQA attention: query [T, 32, 64], key/value [T, 4, 64] -> [T, 32, 64]."""
    q = query.double().cpu().transpose(0, 1)  # [32, T, 64]
    k = key.double().cpu().repeat_interleave(8, dim=1).transpose(0, 1)
    v = value.double().cpu().repeat_interleave(8, dim=1).transpose(0, 1)
    scores = q @ k.transpose(1, 2) / 8
    tokens = query.shape[0]
    scores = scores.masked_fill(~torch.ones(tokens, tokens, dtype=torch.bool).tril(), float("-inf"))
    return (scores.softmax(-1) @ v).transpose(0, 1)


@pytest.mark.parametrize("tokens", [1, 15, 16, 17, 64, 65, 100, 333, 1000, 2048])
def test_prefill_attention_matches_fp32_and_fp64(device, tokens):
    """Against the reference's fp32 dense attention (dense.py:91-99, causal) and FP64, both
    within 2e-3; positions past the prompt are never written."""
    gen = torch.Generator(device=device).manual_seed(tokens)
    query = torch.randn(tokens, 32, 64, dtype=torch.float16, device=device, generator=gen)
    key = torch.randn(tokens, 4, 64, dtype=torch.float16, device=device, generator=gen)
    value = torch.randn(tokens, 4, 64, dtype=torch.float16, device=device, generator=gen)
    out = torch.full((tokens + 16, 32, 64), 7.0, dtype=torch.float16, device=device)
    _hip.prefill_attention(out[:tokens], query, key, value)
    torch.cuda.synchronize()
    got = out[:tokens].cpu()
    assert torch.all(out[tokens:].cpu() == 7.0)
    allowed = torch.ones(tokens, tokens, dtype=torch.bool).tril()[None, None]
    expected = dref.dense_attention_fp32(
        query.cpu().transpose(0, 1)[None], key.cpu().transpose(0, 1)[None], value.cpu().transpose(0, 1)[None], allowed
    )[0].transpose(0, 1)
    torch.testing.assert_close(got, expected, atol=2e-3, rtol=2e-3)
    torch.testing.assert_close(got.double(), _causal_fp64(query, key, value), atol=2e-3, rtol=2e-3)


def test_prefill_attention_sharp_and_known_answers(device):
    """Scores of +-1000 scale (the running max must follow them exactly), V = c gives c, and
    position 0 returns v[0] (one visible key)."""
    gen = torch.Generator(device=device).manual_seed(9)
    tokens = 70
    query = (torch.randn(tokens, 32, 64, device=device, generator=gen) * 30).half()
    key = (torch.randn(tokens, 4, 64, device=device, generator=gen) * 30).half()
    value = torch.randn(tokens, 4, 64, dtype=torch.float16, device=device, generator=gen)
    out = torch.empty(tokens, 32, 64, dtype=torch.float16, device=device)
    _hip.prefill_attention(out, query, key, value)
    torch.cuda.synchronize()
    assert torch.isfinite(out).all()
    torch.testing.assert_close(out.cpu().double(), _causal_fp64(query, key, value), atol=2e-3, rtol=2e-3)
    torch.testing.assert_close(out[0].cpu(), value[0].cpu().repeat_interleave(8, dim=0), atol=0, rtol=0)
    constant = torch.full_like(value, 0.375)
    _hip.prefill_attention(out, query, key, constant)
    torch.cuda.synchronize()
    assert torch.all(out.cpu() == 0.375)


def test_prefill_attention_rejects_bad_arguments(device):
    lib = _hip.load()
    buf = torch.empty(64, dtype=torch.float16, device=device)
    assert lib.pc_prefill_attention(buf.data_ptr(), buf.data_ptr(), buf.data_ptr(), buf.data_ptr(), -1, None) == 1
    assert b"tokens" in lib.pc_last_error()
    assert lib.pc_prefill_attention(buf.data_ptr() + 2, buf.data_ptr(), buf.data_ptr(), buf.data_ptr(), 1, None) == 1
    assert b"aligned" in lib.pc_last_error()
    assert lib.pc_prefill_attention(None, None, None, None, 0, None) == 0


def test_prefill_paged_failure_publishes_nothing_and_allows_retry(device, monkeypatch):
    """A failure inside the prefill forward (here: the prompt attention of layer 5) leaves
    the request empty and the counts unchanged; the slots it wrote belong to free blocks
    only, and a retry publishes the same table as an undisturbed prefill."""
    weights = _synthetic(device)
    pools = [torch.full((22, 2, 10, 16, 4, 64), float("nan"), dtype=torch.float16, device=device) for _ in range(2)]
    failing, clean = (KVAllocator(pool) for pool in pools)
    ids = (torch.arange(40)[None] % 31).to(device)
    for allocator in (failing, clean):
        allocator.create(KVReservation(RequestId("p"), 3))
        allocator.create(KVReservation(RequestId("other"), 1))
        dec.prefill_paged(ids[:, :9], weights, allocator, RequestId("other"))
    counts = failing.capacity()
    other = pools[0][:, :, failing.block_table(RequestId("other"))[0]].clone()
    calls = 0
    original = _hip.prefill_attention

    def fail_at_layer_five(*args):
        nonlocal calls
        calls += 1
        if calls == 6:
            raise RuntimeError("injected prefill failure")
        return original(*args)

    monkeypatch.setattr(_hip, "prefill_attention", fail_at_layer_five)
    with pytest.raises(RuntimeError, match="injected"):
        dec.prefill_paged(ids, weights, failing, RequestId("p"))
    monkeypatch.setattr(_hip, "prefill_attention", original)
    assert failing.capacity() == counts
    assert failing.cached_length(RequestId("p")) == 0 and failing.block_table(RequestId("p")) == ()
    assert torch.equal(pools[0][:, :, failing.block_table(RequestId("other"))[0]].view(torch.int16), other.view(torch.int16))
    retried = dec.prefill_paged(ids, weights, failing, RequestId("p"))
    expected = dec.prefill_paged(ids, weights, clean, RequestId("p"))
    assert torch.equal(retried, expected)
    assert failing.block_table(RequestId("p")) == clean.block_table(RequestId("p"))
    for logical in range(3):
        for a_kv, b_kv in zip(failing.read_block(RequestId("p"), logical), clean.read_block(RequestId("p"), logical)):
            assert torch.equal(a_kv.view(torch.int16), b_kv.view(torch.int16))


def _generate_alone(weights, request, device):
    """Greedy generation of one request by itself: prefill_paged, then decode_paged one
    token at a time (the single-request loop of reference src/pagedcore/decoder.py:88-100)."""
    from pagedcore_amd.worker import FinishReason

    pool = torch.full((22, 2, 24, 16, 4, 64), float("nan"), dtype=torch.float16, device=device)
    allocator = KVAllocator(pool)
    allocator.create(KVReservation(request.request_id, request.block_credits))
    logits = dec.prefill_paged(torch.tensor([list(request.input_ids)], device=device), weights, allocator, request.request_id)
    selected = [int(logits[0, -1].argmax())]
    while True:
        if selected[-1] == 2 and not request.ignore_eos:
            return tuple(selected), FinishReason.EOS
        if len(selected) == request.max_new_tokens:
            return tuple(selected), FinishReason.LENGTH
        logits = dec.decode_paged(torch.tensor([[selected[-1]]], device=device), weights, allocator, (request.request_id,))
        selected.append(int(logits[0, -1].argmax()))


@pytest.mark.parametrize("graph_batch, prompt_graphs", [(None, ()), (3, ()), ((2, 4), (16, 48))])
def test_worker_streams_equal_each_request_generated_alone(device, graph_batch, prompt_graphs):
    """Continuous batching (requests joining and leaving the decode batch every few steps)
    gives every request exactly the tokens it gets when generated by itself."""
    from pagedcore_amd.worker import DecodeWorker, GenerationRequest

    weights = _synthetic(device)
    pool = torch.full((22, 2, 48, 16, 4, 64), float("nan"), dtype=torch.float16, device=device)
    allocator = KVAllocator(pool)
    worker = DecodeWorker(weights, allocator, max_active=3, graph_batch=graph_batch, prefill_graph_tokens=prompt_graphs)
    gen = torch.Generator().manual_seed(13)
    requests = []
    for index in range(7):
        prompt = tuple(int(t) for t in torch.randint(3, 31, (int(torch.randint(1, 40, (1,), generator=gen)),), generator=gen))
        requests.append(GenerationRequest(RequestId(f"w{index}"), prompt, int(torch.randint(1, 12, (1,), generator=gen)),
                                          ignore_eos=index % 2 == 0))
        worker.submit(requests[-1])
    results = worker.run(max_steps=500)
    for request in requests:
        ids, reason = _generate_alone(weights, request, device)
        got = results[request.request_id]
        assert got.greedy_ids == ids and got.finish_reason == reason, request.request_id
    counts = allocator.capacity()
    assert counts.owned_blocks == 0 and counts.reserved_blocks == 0 and counts.active_slots == 0


# ---------------------------------------------------------------------------------------
# Reference decoder cases re-expressed on the GPU path
# ---------------------------------------------------------------------------------------


@pytest.mark.parametrize("use_graph", [False, True])
def test_decode_at_the_last_context_position(device, use_graph):
    """tests/unit/test_decoder.py:359-378: 2047 cached positions; decode writes position 2047
    (block 127, slot 15) and the logits match the contiguous fp32 decode (new K/V: layer 0
    within 2e-3, every layer as accurate as the CPU fp16 forward against fp32); the next
    decode is refused with ValueError and changes nothing (counts, length, pool bytes)."""
    weights = _synthetic(device)
    host_weights = _cpu(weights)
    pool = torch.zeros(22, 2, 128, 16, 4, 64, dtype=torch.float16, device=device)
    allocator = KVAllocator(pool)
    request = RequestId("last")
    allocator.create(KVReservation(request, 128))
    gen = torch.Generator(device=device).manual_seed(4)
    history = torch.randn(22, 2047, 4, 64, dtype=torch.float16, device=device, generator=gen)
    allocator.append(request, history, -history)
    cache = _pool_cache(allocator, request)
    step = dec.DecodeGraph(weights, allocator, 1).step if use_graph else (
        lambda ids, rids: dec.decode_paged(ids, weights, allocator, rids))
    logits = step(torch.tensor([[3]], device=device), (request,))
    torch.cuda.synchronize()
    assert logits.shape == (1, 1, 31) and torch.isfinite(logits).all()
    assert allocator.cached_length(request) == 2048
    expected, new_cache = dref.decode_fp32(torch.tensor([[3]]), cache, host_weights)
    _, exact_cache = dref.forward(
        torch.tensor([[3]]), _fp32(host_weights), [(k.float(), v.float()) for k, v in cache], fp32_attention=True
    )
    torch.testing.assert_close(logits.cpu(), expected, atol=5e-3, rtol=5e-3)
    block = allocator.block_table(request)[127]
    got = _pool_cache(allocator, request)
    for layer in range(22):
        for kind in range(2):
            assert torch.equal(got[layer][kind][:, :, :2047], cache[layer][kind])
            new = got[layer][kind][:, :, 2047]
            if layer == 0:  # no upstream GEMM or attention noise: the reference's 2e-3
                torch.testing.assert_close(new, new_cache[0][kind][:, :, 2047], atol=2e-3, rtol=0)
            _as_accurate(new, new_cache[layer][kind][:, :, 2047], exact_cache[layer][kind][:, :, 2047])
    assert torch.isfinite(pool[:, :, block, 15]).all()
    counts = allocator.capacity()
    before = pool.clone()
    with pytest.raises(ValueError, match="2047"):
        step(torch.tensor([[5]], device=device), (request,))
    assert allocator.capacity() == counts
    assert allocator.cached_length(request) == 2048
    assert torch.equal(pool.view(torch.int16), before.view(torch.int16))


@pytest.mark.parametrize("tokens", [1, 15, 16, 17, 49])
def test_prefill_writes_absolute_positions_to_reused_fragmented_pages(device, tokens):
    """tests/unit/test_decoder.py:440-493: three one-block requests hold sentinel K/V, the
    first and last are released, and the prompt then gets the table (2, 0, 3, 4): its
    positions land in reused, out-of-order blocks. Logits against the contiguous prefill,
    layer-0 K/V within 2e-3 (every layer as accurate as the CPU fp16 forward), the
    reference's counts, NaN poison kept in the tail slots, and every other block (the
    retained sentinel and the free blocks' old bytes) unchanged."""
    weights = _synthetic(device)
    host_weights = _cpu(weights)
    exact = _fp32(host_weights)
    pool = torch.full((22, 2, 6, 16, 4, 64), float("nan"), dtype=torch.float16, device=device)
    allocator = KVAllocator(pool)
    for name in ("released_first", "retained", "released_last"):
        request = RequestId(name)
        allocator.create(KVReservation(request, 1))
        key = torch.full((22, 16, 4, 64), -100.0, dtype=torch.float16, device=device)
        allocator.append(request, key, -key)
    allocator.release_all(RequestId("released_first"))
    allocator.release_all(RequestId("released_last"))
    request = RequestId("prompt")
    blocks = (tokens + 15) // 16
    allocator.create(KVReservation(request, blocks))
    before = pool.clone()
    pointer = pool.untyped_storage().data_ptr()
    ids = torch.arange(tokens)[None] % 31
    expected_logits, expected_cache = dref.prefill(ids, host_weights)
    exact_logits, exact_cache = dref.forward(ids, exact)

    logits = dec.prefill_paged(ids.to(device), weights, allocator, request)
    torch.cuda.synchronize()

    torch.testing.assert_close(logits.cpu(), expected_logits, atol=5e-3, rtol=5e-3)
    _as_accurate(logits, expected_logits, exact_logits)
    assert logits.dtype == torch.float16 and not logits.requires_grad
    assert pool.untyped_storage().data_ptr() == pointer
    assert allocator.block_table(request) == (2, 0, 3, 4)[:blocks]
    assert allocator.cached_length(request) == tokens
    assert allocator.capacity() == CapacityCounts(6, 5 - blocks, blocks + 1, blocks + 1, 2, tokens + 16)
    got = _pool_cache(allocator, request)
    for layer in range(22):
        for kind in range(2):
            if layer == 0:
                torch.testing.assert_close(got[0][kind], expected_cache[0][kind], atol=2e-3, rtol=0)
            _as_accurate(got[layer][kind], expected_cache[layer][kind], exact_cache[layer][kind])
    for logical, physical in enumerate(allocator.block_table(request)):
        valid = min(16, tokens - logical * 16)
        assert torch.equal(pool[:, :, physical, valid:].view(torch.int16), before[:, :, physical, valid:].view(torch.int16))
    for physical in set(range(6)) - set(allocator.block_table(request)):
        assert torch.equal(pool[:, :, physical].view(torch.int16), before[:, :, physical].view(torch.int16))
    allocator.release_all(request)
    allocator.release_all(RequestId("retained"))
    assert allocator.capacity() == CapacityCounts(6, 6, 0, 0, 0, 0)


def test_decode_step_b128_at_the_bench_workload(device):
    """The full decode-step workload (tests/unit/test_decoder.py:114-195 at scale): 22
    distinct full-size layers (MLP 5632, vocab 32000, N(0, 0.02) weights), batch 128,
    contexts U{256..2034} of N(0, 1) K/V in a fragmented pool, as the benchmark builds it.
    One DecodeGraph step, then one eager decode_paged step. For ten rows per step (the
    shortest and longest, a row whose new token opens a fresh block, one filling the last
    slot of a block, and random rows) the logits are as close to an fp32 evaluation as the
    CPU fp16 forward is (started from the GPU's own cache; error model below), layer 0's
    new K/V is within 2e-3 of the oracle, and the greedy token agrees wherever the fp32
    top-2 margin exceeds that noise. Every row: finite logits, one more cached position,
    old slots unchanged."""
    from tests.support import fragmented_decode_cache

    batch = 128
    rng = np.random.default_rng(20261205)
    lengths = rng.integers(256, 2035, size=batch)
    lengths[:4] = [256, 2034, 1024, 1039]  # shortest, longest, fresh block next, last slot next
    weights = dec.random_weights(device=device, seed=20261205)
    host_weights = _cpu(weights)
    exact = _fp32(host_weights)
    allocator, requests = fragmented_decode_cache(device, batch, lengths, 4, seed=5)
    pool = allocator.pool
    scattered = sum(int(np.sum(np.diff(allocator.block_table(r)) != 1)) for r in requests)
    assert scattered > batch  # the tables really are fragmented
    graph = dec.DecodeGraph(weights, allocator, batch)
    checked = [0, 1, 2, 3] + [int(b) for b in rng.choice(np.arange(4, batch), size=6, replace=False)]
    tokens = torch.from_numpy(rng.integers(0, 32000, size=(batch, 1))).to(device)
    errors, kv_gaps, argmax = [], [], []
    for name, step in (("graph", graph.step), ("eager", lambda ids, rids: dec.decode_paged(ids, weights, allocator, rids))):
        old_lengths = [allocator.cached_length(r) for r in requests]
        caches = {b: _pool_cache(allocator, requests[b]) for b in checked}
        before = pool.clone()
        logits = step(tokens, requests)
        torch.cuda.synchronize()
        assert logits.shape == (batch, 1, 32000) and torch.isfinite(logits).all(), name
        written = torch.zeros(pool.shape[2:4], dtype=torch.bool, device=device)
        for b, request in enumerate(requests):
            assert allocator.cached_length(request) == old_lengths[b] + 1
            block, slot = divmod(old_lengths[b], 16)
            written[allocator.block_table(request)[block], slot] = True
        assert torch.equal(pool[:, :, ~written].view(torch.int16), before[:, :, ~written].view(torch.int16)), name
        del before
        for b in checked:
            request = requests[b]
            cpu16, new_cache = dref.decode_fp32(tokens[b : b + 1].cpu(), caches[b], host_weights)
            fp32 = dref.forward(
                tokens[b : b + 1].cpu(), exact, [(k.float(), v.float()) for k, v in caches[b]], fp32_attention=True
            )[0]
            gpu_err = (logits[b : b + 1].float().cpu() - fp32.float()).abs()
            cpu_err = (cpu16.float() - fp32.float()).abs()
            errors.append(
                (name, b, float(gpu_err.max()), float(cpu_err.max()), float(gpu_err.pow(2).mean().sqrt()),
                 float(cpu_err.pow(2).mean().sqrt()))
            )
            print(
                f"  {name} row {b} len {old_lengths[b]}: max |gpu - fp32| {errors[-1][2]:.4f} |cpu16 - fp32| "
                f"{errors[-1][3]:.4f}  rms {errors[-1][4]:.5f} / {errors[-1][5]:.5f}",
                flush=True,
            )
            got = _pool_cache(allocator, request)
            for kind in range(2):
                kv_gaps.append(_gap(got[0][kind][:, :, old_lengths[b]], new_cache[0][kind][:, :, old_lengths[b]]))
            top = fp32.flatten().topk(2).values
            if float(top[0] - top[1]) > 4 * _gap(cpu16, fp32):
                argmax.append((name, b, int(logits[b].argmax()), int(fp32.argmax())))
        print(f"decode step b128 ({name}): {len(checked)} rows checked against the oracle", flush=True)
        tokens = logits.argmax(-1)
    print(f"  layer-0 new K/V: max |gpu - oracle| {max(kv_gaps):.2e}", flush=True)
    # Error model at this size: the GPU and the CPU fp16 forwards both round 22 layers of
    # fp16 GEMM outputs, so their errors against fp32 have the same distribution; each row's
    # RMS over the 32000 logits is a stable statistic of it, while one row's maximum is an
    # extreme value that scatters by tens of percent between two equally accurate
    # computations. So: every row's RMS error within 1.25x the CPU's, and every row's
    # maximum within 1.25x the largest CPU maximum over the checked rows, plus 2e-3.
    cpu_worst = max(e[3] for e in errors)
    for name, b, gpu_max, _, gpu_rms, cpu_rms in errors:
        assert gpu_rms <= 1.25 * cpu_rms, (name, b, gpu_rms, cpu_rms)
        assert gpu_max <= 1.25 * cpu_worst + 2e-3, (name, b, gpu_max, cpu_worst)
    assert max(kv_gaps) <= 2e-3
    assert all(got == want for _, _, got, want in argmax), argmax
    assert len(argmax) >= 4  # the argmax condition is not vacuous


def _worker_stream_matches_generate(request, result, host_weights, tie: float = 1e-2) -> int:
    """The worker's greedy stream against the oracle's generate (reference
    src/pagedcore/decoder.py:70-100). Equal streams and finish reasons pass. A stream may
    leave the oracle's only at a near-tie: the oracle's own logits at that step, on the
    common prefix, have a top-2 gap within `tie` (twice the 5e-3 logits tolerance) and the
    worker chose the runner-up; from there on each worker token must be the oracle's
    choice (or a near-tie runner-up) given the worker's own prefix. Returns the tie count."""
    ids = torch.tensor([list(request.input_ids)])
    greedy, emitted, reason = dref.generate(
        ids, host_weights, max_new_tokens=request.max_new_tokens, ignore_eos=request.ignore_eos
    )
    got = result.greedy_ids
    if got == greedy:
        assert result.emitted_ids == emitted and result.finish_reason.value == reason
        return 0
    sequence = torch.cat([ids, torch.tensor([list(got[:-1])], dtype=torch.int64)], dim=1)
    logits = dref.prefill(sequence, host_weights)[0][0, ids.shape[1] - 1 :].float()
    ties = 0
    for position, token in enumerate(got):
        values, indices = logits[position].topk(2)
        if token == int(indices[0]):
            continue
        assert token == int(indices[1]) and float(values[0] - values[1]) <= tie, (request.request_id, position)
        ties += 1
    stops = got[-1] == 2 and not request.ignore_eos
    assert result.finish_reason.value == ("eos" if stops else "length")
    assert stops or len(got) == request.max_new_tokens
    assert 2 not in got[:-1] or request.ignore_eos
    return ties


@pytest.mark.parametrize("graph_batch, prompt_graphs", [(None, ()), (3, ()), ((2, 4), (16, 48))])
def test_worker_streams_match_the_oracle_generate(device, graph_batch, prompt_graphs):
    """Continuous batching (requests joining and leaving the decode batch every few steps,
    eager or through padded decode/prefill graphs): every request's tokens and finish
    reason are those of the oracle's single-sequence greedy generate."""
    from pagedcore_amd.worker import DecodeWorker, GenerationRequest

    weights = _synthetic(device)
    host_weights = _cpu(weights)
    pool = torch.full((22, 2, 48, 16, 4, 64), float("nan"), dtype=torch.float16, device=device)
    allocator = KVAllocator(pool)
    worker = DecodeWorker(weights, allocator, max_active=3, graph_batch=graph_batch, prefill_graph_tokens=prompt_graphs)
    gen = torch.Generator().manual_seed(13)
    requests = []
    for index in range(7):
        prompt = tuple(int(t) for t in torch.randint(3, 31, (int(torch.randint(1, 40, (1,), generator=gen)),), generator=gen))
        requests.append(GenerationRequest(RequestId(f"w{index}"), prompt, int(torch.randint(1, 12, (1,), generator=gen)),
                                          ignore_eos=index % 2 == 0))
        worker.submit(requests[-1])
    results = worker.run(max_steps=500)
    ties = sum(_worker_stream_matches_generate(r, results[r.request_id], host_weights) for r in requests)
    print(f"worker vs oracle generate: {len(requests)} requests, {ties} near-tie choices", flush=True)
    counts = allocator.capacity()
    assert counts.owned_blocks == 0 and counts.reserved_blocks == 0 and counts.active_slots == 0


@pytest.mark.parametrize("batch,expect_library_gemm", [(128, True), (130, False)])
def test_decode_paged_projection_path_by_batch_size(device, monkeypatch, batch, expect_library_gemm):
    """Up to 128 rows the step's projections run on pc_gemm_m128 (split-K partials summed by
    the RoPE / residual kernels, SwiGLU fused); above that on F.linear. Both paths match the
    contiguous fp32 decode (tests/unit/test_decoder.py:114-195 tolerances) on sampled rows."""
    weights = _synthetic(device)
    host_weights = _cpu(weights)
    contexts = [3, 16, 17]
    pool = torch.full((22, 2, 3 * batch, 16, 4, 64), float("nan"), dtype=torch.float16, device=device)
    allocator = KVAllocator(pool)
    requests = tuple(RequestId(str(row)) for row in range(batch))
    for row, request in enumerate(requests):
        length = contexts[row % 3]
        allocator.create(KVReservation(request, 3))
        dec.prefill_paged(((torch.arange(length)[None] + row) % 31).to(device), weights, allocator, request)
    calls = []
    original = _hip.gemm_m128

    def counting(*args, **kwargs):
        calls.append(kwargs.get("epilogue", _hip.GEMM_PARTIALS))
        return original(*args, **kwargs)

    monkeypatch.setattr(_hip, "gemm_m128", counting)
    tokens = torch.tensor([[(5 * row) % 31] for row in range(batch)])
    sample = [0, 1, 2, batch // 2, batch - 1]
    expected = {row: dref.decode_fp32(tokens[row : row + 1], _pool_cache(allocator, requests[row]), host_weights)
                for row in sample}
    logits = dec.decode_paged(tokens.to(device), weights, allocator, requests)
    torch.cuda.synchronize()
    if expect_library_gemm:
        # per layer q|k|v, o_proj and gate|up (the synthetic MLP width 32 keeps down, whose
        # K of 32 is not a multiple of 64, on F.linear)
        assert calls.count(_hip.GEMM_PARTIALS) == 2 * 22 and calls.count(_hip.GEMM_SWIGLU) == 22
    else:
        assert calls == []
    assert torch.isfinite(logits).all()
    for row in sample:
        torch.testing.assert_close(logits[row : row + 1].cpu(), expected[row][0], atol=5e-3, rtol=5e-3)
