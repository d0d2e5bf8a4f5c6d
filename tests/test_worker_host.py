"""The continuous-batching worker's scheduling on the CPU (no GPU): FIFO admission under
the active-slot and KV-credit limits, one token per request per iteration, EOS and length
semantics (reference src/pagedcore/decoder.py:61-100), cleanup timing and cancellation.
The model is replaced by scripted prefill/decode functions that keep the allocator's real
bookkeeping (appends and staged decode writes through the CPU test writer)."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from pagedcore_amd.engine_types import RequestId
from pagedcore_amd.worker import DecodeWorker, FinishReason, GenerationRequest, GreedyResult
from tests.support import cpu_allocator

VOCAB = 40


class ScriptedModel:
    """Token chosen for request r at its n-th selection: script[r][n] (default 10 + n)."""

    def __init__(self, script=None):
        self.script = script or {}
        self.decode_batches = []
        self.prefills = []

    def _logits(self, rid, n):
        token = self.script.get(rid, {}).get(n, 10 + n)
        logits = torch.zeros(VOCAB)
        logits[token] = 1.0
        return logits

    def prefill(self, ids, weights, allocator, rid):
        tokens = ids.shape[1]
        kv = torch.zeros(22, tokens, 4, 64, dtype=torch.float16)
        allocator.append(rid, kv, kv)
        self.prefills.append(rid)
        return torch.stack([self._logits(rid, 0)] * tokens)[None]

    def decode(self, tokens, weights, allocator, rids):
        self.decode_batches.append(rids)
        with allocator.append_decode(rids):
            kv = torch.zeros(len(rids), 4, 64, dtype=torch.float16)
            for layer in range(22):
                allocator.write_decode_layers(rids, layer, kv, kv)
            out = []
            for rid in rids:
                # staged length = prompt + tokens selected so far: this is selection number n
                n = allocator._decode_appends[rid].sequence.length - len(self.prompts[rid])
                out.append(self._logits(rid, n))
        return torch.stack(out)[:, None]


def _worker(model, blocks=32, max_active=2):
    allocator = cpu_allocator(torch.zeros((22, 2, blocks, 16, 4, 64), dtype=torch.float16))
    return DecodeWorker(None, allocator, max_active=max_active, prefill=model.prefill, decode=model.decode), allocator


def _request(name, prompt=5, new=4, **kw):
    return GenerationRequest(RequestId(name), tuple(range(1, prompt + 1)), new, **kw)


def _greedy_decode(step, ids, rids, device_token):
    """A fake decode graph's greedy(): its step() over the host ids (with device_token's
    row replaced), argmax of each row."""
    assert ids.dtype == np.int64 and ids.shape == (len(rids),)
    tokens = torch.from_numpy(ids.copy()).view(-1, 1)
    if device_token is not None:
        row, token = device_token
        tokens[row, 0] = token
    return step(tokens, rids)[:, -1].argmax(dim=-1)


def _submit(worker, model, requests):
    model.prompts = {r.request_id: r.input_ids for r in requests}
    for r in requests:
        worker.submit(r)


def test_fifo_admission_one_per_iteration_and_active_limit():
    model = ScriptedModel()
    worker, allocator = _worker(model, max_active=2)
    requests = [_request(f"r{i}", new=3) for i in range(4)]
    _submit(worker, model, requests)
    worker.step()
    assert worker.active_ids == ("r0",) and model.decode_batches == [("r0",)]
    worker.step()  # r0 selects its 3rd token and finishes; the active limit holds r2
    assert worker.active_ids == ("r0", "r1") and model.decode_batches[-1] == ("r0", "r1")
    assert worker.pending_ids == ("r2", "r3") and "r0" not in worker.results
    worker.step()  # cleanup frees r0's slot first, then r2 is admitted
    assert worker.active_ids == ("r1", "r2") and worker.pending_ids == ("r3",)
    assert worker.results["r0"].greedy_ids == (10, 11, 12)
    results = worker.run(max_steps=50)
    assert model.prefills == ["r0", "r1", "r2", "r3"]
    for r in requests:
        assert results[r.request_id] == GreedyResult((10, 11, 12), (10, 11, 12), FinishReason.LENGTH)
    assert allocator.capacity().owned_blocks == 0 and allocator.capacity().reserved_blocks == 0


def test_each_request_selects_one_token_per_iteration_and_finishes_at_its_length():
    model = ScriptedModel()
    worker, _ = _worker(model, max_active=4)
    _submit(worker, model, [_request("a", new=1), _request("b", new=2)])
    emitted = worker.step()
    assert emitted == [("a", 10)]  # a's only token comes from prefill; it is not decoded
    assert model.decode_batches == []
    emitted = worker.step()  # a cleaned up; b prefilled and decoded in the same iteration
    assert emitted == [("b", 10), ("b", 11)]
    assert model.decode_batches == [("b",)]
    results = worker.run()
    assert results["a"].greedy_ids == (10,) and results["b"].greedy_ids == (10, 11)


def test_eos_is_selected_but_not_emitted_and_wins_at_the_limit():
    model = ScriptedModel({RequestId("stop"): {2: 2}, RequestId("limit"): {2: 2}, RequestId("keep"): {1: 2}})
    worker, _ = _worker(model, max_active=3)
    _submit(worker, model, [_request("stop", new=5), _request("limit", new=3), _request("keep", new=3, ignore_eos=True)])
    results = worker.run()
    assert results["stop"] == GreedyResult((10, 11, 2), (10, 11), FinishReason.EOS)
    assert results["limit"] == GreedyResult((10, 11, 2), (10, 11), FinishReason.EOS)
    assert results["keep"] == GreedyResult((10, 2, 12), (10, 2, 12), FinishReason.LENGTH)


def test_kv_credits_block_the_queue_head_and_release_comes_at_the_next_cleanup():
    model = ScriptedModel()
    # 6 blocks; "big" needs 5 credits (70 tokens + 4), "small" needs 1
    worker, allocator = _worker(model, blocks=6, max_active=4)
    _submit(worker, model, [_request("first", prompt=20, new=4), _request("big", prompt=70, new=4), _request("small", prompt=3, new=2)])
    worker.step()
    assert worker.active_ids == ("first",)
    worker.step()
    # big does not fit beside first's 2 credits; small waits behind it (strict FIFO)
    assert worker.pending_ids == ("big", "small")
    steps = 0
    while "first" not in worker.results:
        worker.step()
        steps += 1
    assert worker.active_ids == ("big",) and allocator.capacity().reserved_blocks == 5
    results = worker.run()
    assert set(results) == {"first", "big", "small"}


def test_cancellation_and_validation():
    model = ScriptedModel()
    worker, allocator = _worker(model, max_active=1)
    _submit(worker, model, [_request("a", new=10), _request("b", new=10)])
    worker.step()
    worker.cancel(RequestId("b"))
    worker.cancel(RequestId("a"))
    worker.step()
    assert worker.idle and worker.results == {}
    assert allocator.capacity().owned_blocks == 0
    with pytest.raises(KeyError):
        worker.cancel(RequestId("unknown"))
    with pytest.raises(ValueError, match="unique"):
        worker.submit(_request("a"))
    with pytest.raises(ValueError, match="total KV pool"):
        worker.submit(GenerationRequest(RequestId("huge"), tuple(range(600)), 10))
    with pytest.raises(ValueError, match="2048"):
        GenerationRequest(RequestId("x"), tuple(range(2000)), 100)
    with pytest.raises(ValueError, match="1 to 256"):
        GenerationRequest(RequestId("x"), (1,), 0)
    with pytest.raises(ValueError, match="nonempty"):
        GenerationRequest(RequestId("x"), (), 5)


def test_token_ids_past_the_vocabulary_are_rejected_on_the_host():
    """An id at or above the embedding's row count never reaches the GPU: submit refuses
    it, with the vocabulary taken from the weights or given explicitly."""
    model = ScriptedModel()
    allocator = cpu_allocator(torch.zeros((22, 2, 32, 16, 4, 64), dtype=torch.float16))

    class Weights:
        embedding = torch.zeros(VOCAB, 8)

    worker = DecodeWorker(Weights(), allocator, prefill=model.prefill, decode=model.decode)
    with pytest.raises(ValueError, match="vocabulary size 40"):
        worker.submit(GenerationRequest(RequestId("big"), (1, VOCAB), 3))
    assert worker.idle
    worker.submit(GenerationRequest(RequestId("ok"), (1, VOCAB - 1), 3))
    explicit = DecodeWorker(None, allocator, vocab_size=7, prefill=model.prefill, decode=model.decode)
    with pytest.raises(ValueError, match="vocabulary size 7"):
        explicit.submit(GenerationRequest(RequestId("big"), (7,), 3))
    with pytest.raises(ValueError, match="vocab_size"):
        DecodeWorker(None, allocator, vocab_size=0)


def test_failed_prefill_releases_the_request_and_later_steps_continue():
    """A prefill that raises during admission drops the request from the active set and
    returns its credits; the error reaches the caller, and the next iterations admit and
    decode the requests behind it."""
    model = ScriptedModel()
    worker, allocator = _worker(model, max_active=2)
    requests = [_request("ok0", new=3), _request("bad", new=3), _request("ok1", new=3)]
    _submit(worker, model, requests)
    original = model.prefill

    def failing(ids, weights, alloc, rid):
        if rid == "bad":
            original(ids, weights, alloc, rid)  # publishes its prompt, then fails
            raise RuntimeError("injected prefill failure")
        return original(ids, weights, alloc, rid)

    worker._prefill = failing
    worker.step()
    with pytest.raises(RuntimeError, match="injected prefill failure"):
        worker.step()
    assert worker.active_ids == ("ok0",)
    counts = allocator.capacity()
    assert counts.active_slots == 1 and counts.reserved_blocks == requests[0].block_credits
    results = worker.run(max_steps=10)
    assert set(results) == {"ok0", "ok1"}
    assert all(r.finish_reason is FinishReason.LENGTH and len(r.greedy_ids) == 3 for r in results.values())
    assert allocator.capacity().owned_blocks == 0


def test_decode_steps_replay_the_smallest_graph_that_holds_the_batch(monkeypatch):
    """With graph sizes (4, 2) a step of n requests replays the graph of the smallest size
    >= n, captured once on first use; a step larger than every size runs decode_paged."""
    from pagedcore_amd import decoder

    model = ScriptedModel()
    made, used = [], []

    class RecordingGraph:
        def __init__(self, weights, allocator, batch):
            made.append(batch)
            self.batch, self.allocator = batch, allocator

        def step(self, tokens, rids):
            assert len(rids) <= self.batch
            used.append((self.batch, len(rids)))
            return model.decode(tokens, None, self.allocator, rids)

        def greedy(self, ids, rids, device_token=None):
            return _greedy_decode(self.step, ids, rids, device_token)

        def check_faults(self):
            pass

    monkeypatch.setattr(decoder, "DecodeGraph", RecordingGraph)
    allocator = cpu_allocator(torch.zeros((22, 2, 32, 16, 4, 64), dtype=torch.float16))
    worker = DecodeWorker(None, allocator, max_active=5, prefill=model.prefill, decode=model.decode, graph_batch=(4, 2))
    _submit(worker, model, [_request(f"r{i}", new=8) for i in range(5)])
    for _ in range(6):
        worker.step()
    # one admission per iteration: batches of 1, 2, 3, 4, 5, 5
    assert used == [(2, 1), (2, 2), (4, 3), (4, 4)]
    assert [len(batch) for batch in model.decode_batches] == [1, 2, 3, 4, 5, 5]
    assert made == [2, 4]
    worker.capture_graphs()
    assert made == [2, 4]  # already captured
    results = worker.run()
    assert all(results[f"r{i}"].greedy_ids == tuple(range(10, 18)) for i in range(5))
    captured = []
    monkeypatch.setattr(decoder, "DecodeGraph", lambda weights, allocator, batch: captured.append(batch))
    DecodeWorker(None, allocator, prefill=model.prefill, decode=model.decode, graph_batch=(8, 1, 8)).capture_graphs()
    assert captured == [1, 8]
    for bad in (0, (2, 0), True, (3.0,)):
        with pytest.raises(ValueError, match="graph batch sizes"):
            DecodeWorker(None, allocator, prefill=model.prefill, decode=model.decode, graph_batch=bad)


def test_admissions_replay_the_smallest_prefill_graph_that_holds_the_prompt(monkeypatch):
    """With prefill graph sizes (8, 32) a prompt of T positions replays the PrefillGraph of
    the smallest size >= T (captured once); a longer prompt runs the prefill function."""
    from pagedcore_amd import decoder

    model = ScriptedModel()
    made, used = [], []

    class RecordingPrefillGraph:
        def __init__(self, weights, allocator, tokens):
            made.append(tokens)
            self.tokens, self.allocator = tokens, allocator

        def step(self, ids, rid):
            assert ids.shape[1] <= self.tokens
            used.append((self.tokens, ids.shape[1]))
            return model.prefill(ids, None, self.allocator, rid)[:, -1:]

        def greedy(self, prompt, rid):
            assert prompt.dtype == np.int64 and prompt.ndim == 1
            return self.step(torch.from_numpy(prompt.copy()).view(1, -1), rid)[0, -1].argmax()

    monkeypatch.setattr(decoder, "PrefillGraph", RecordingPrefillGraph)
    allocator = cpu_allocator(torch.zeros((22, 2, 32, 16, 4, 64), dtype=torch.float16))
    worker = DecodeWorker(None, allocator, max_active=4, prefill=model.prefill, decode=model.decode,
                          prefill_graph_tokens=[32, 8])
    requests = [_request("a", prompt=8), _request("b", prompt=9), _request("c", prompt=40), _request("d", prompt=3)]
    _submit(worker, model, requests)
    results = worker.run()
    assert used == [(8, 8), (32, 9), (8, 3)]
    assert model.prefills == ["a", "b", "c", "d"]  # c (40 positions) ran the prefill function
    assert made == [8, 32]
    assert all(results[r.request_id].greedy_ids == (10, 11, 12, 13) for r in requests)
    captured = []
    monkeypatch.setattr(decoder, "PrefillGraph", lambda weights, allocator, tokens: captured.append(tokens))
    DecodeWorker(None, allocator, prefill=model.prefill, decode=model.decode, prefill_graph_tokens=(64, 2048)).capture_graphs()
    assert captured == [64, 2048]
    for bad in ((0,), (2049,), (True,), (16.0,)):
        with pytest.raises(ValueError, match="prefill graph sizes"):
            DecodeWorker(None, allocator, prefill=model.prefill, decode=model.decode, prefill_graph_tokens=bad)


@pytest.mark.parametrize("where", ["graph", "eager"])
def test_a_device_fault_stops_the_worker_before_it_emits(monkeypatch, where):
    """A decode step whose paged attention reports a device fault (DecodeGraph.check_faults
    after the tokens are fetched, or decode_paged's own check) raises AttentionFaultError
    before any of that step's tokens is emitted; the worker then stops: every later step()
    raises RuntimeError and nothing more is prefilled or decoded (fail closed)."""
    from pagedcore_amd import decoder
    from pagedcore_amd._hip import FAULT_MERGE_TIMEOUT, AttentionFaultError

    model = ScriptedModel()
    steps = []

    def faulty_decode(tokens, weights, allocator, rids):
        steps.append(len(rids))
        logits = model.decode(tokens, weights, allocator, rids)
        if len(steps) == 3 and where == "eager":
            raise AttentionFaultError(FAULT_MERGE_TIMEOUT, "decode_paged")
        return logits

    class FaultyGraph:
        def __init__(self, weights, allocator, batch):
            self.allocator = allocator

        def step(self, tokens, rids):
            return faulty_decode(tokens, None, self.allocator, rids)

        def greedy(self, ids, rids, device_token=None):
            return _greedy_decode(self.step, ids, rids, device_token)

        def check_faults(self):
            if len(steps) == 3:
                raise AttentionFaultError(FAULT_MERGE_TIMEOUT, "DecodeGraph.step")

    monkeypatch.setattr(decoder, "DecodeGraph", FaultyGraph)
    allocator = cpu_allocator(torch.zeros((22, 2, 32, 16, 4, 64), dtype=torch.float16))
    worker = DecodeWorker(None, allocator, max_active=3, prefill=model.prefill, decode=faulty_decode,
                          graph_batch=(4,) if where == "graph" else None)
    _submit(worker, model, [_request(f"r{i}", new=8) for i in range(4)])
    emitted = worker.step() + worker.step()
    assert len(emitted) == 2 + 3  # r0's prefill and decode tokens; r1's prefill token, both decode tokens
    with pytest.raises(AttentionFaultError, match="bounded wait"):
        worker.step()
    assert worker.fault is not None and worker.fault.faults == FAULT_MERGE_TIMEOUT
    prefills = list(model.prefills)
    for _ in range(2):
        with pytest.raises(RuntimeError, match="stopped after a device fault"):
            worker.step()
    assert len(steps) == 3 and model.prefills == prefills  # nothing launched after the fault
    # no token of the faulted step was selected: each request holds its prefill token and
    # the decode tokens of the steps before the fault
    assert {rid: len(state.selected) for rid, state in worker._active.items()} == {"r0": 3, "r1": 2, "r2": 1}
