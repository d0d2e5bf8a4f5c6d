"""Continuous-batching greedy decode worker over the paged KV path.

The reference plans this loop but does not build it (its docs/DESIGN.md:348-357, "Scheduler
iteration"); its single-request greedy semantics are src/pagedcore/decoder.py:61-100
(GreedyResult, generate). One call of DecodeWorker.step is one iteration of that plan:

  1. clean up: release the KV blocks, credits and active slot of requests that finished
     (or were cancelled) in the previous iteration; drop cancelled requests still waiting;
  2. admit at most one request, strictly first-in first-out: if an active slot is free and
     the request's KV credits fit the unreserved pool, reserve, prefill (prefill_paged,
     or the replay of a captured PrefillGraph) and select its first token; otherwise it keeps waiting (head-of-line blocking, as
     planned);
  3. decode: every active unfinished request, the newly admitted one included, in one
     batched decode step (decode_paged, or the replay of a captured DecodeGraph of the
     smallest configured size that holds the batch);
  4. emit: each request selects at most one token per iteration. A selected EOS stops the
     request (unless ignore_eos) and is excluded from the emitted ids; reaching
     max_new_tokens stops it with reason LENGTH, EOS taking precedence at the limit.

Everything runs on the allocator's worker thread and stream, so a release is ordered after
every launch that read the released blocks (the reference's stream-ordered reuse rule,
docs/DESIGN.md:282).

The host waits for the GPU once per iteration. The admitted request's first token is
selected on the device (argmax of the prefill's last logits) and fed to the decode step
from device memory, and its host-side selection happens after the step, with the decode's
tokens, in the order of the plan (the prefill token first): the decode step's host work
then runs while the GPU executes the prefill. Only when that token can end the request
early, an EOS with ignore_eos off, does the host wait for it before forming the batch, as
the batch must not hold a finished request. Inputs go to the device through pinned memory
without blocking (with the captured graphs, each replay's ids, slots and plan in one or two
copies), the graphs hand back each row's argmax rather than a copy of the logits, and the
selected ids come back by asynchronous copies into one pinned buffer (the first token's
enqueued right after its prefill) and one event wait.

A device-side failure fails closed (the reference's rule for unsafe device failures,
docs/DESIGN.md:178,255,282): when a decode step's paged attention reports a fault (its
workspace's fault word, read right after the step's tokens are fetched and before any is
emitted), the iteration raises AttentionFaultError and the worker stops: every later step()
raises RuntimeError, and nothing more is launched.
"""

from __future__ import annotations

from collections import deque
from dataclasses import dataclass, field
from enum import Enum
from typing import Callable, Deque, Dict, List, Optional, Sequence, Tuple, Union

import numpy as np
import torch
from torch import Tensor

from pagedcore_amd._hip import AttentionFaultError
from pagedcore_amd.engine_types import KVReservation, RequestId
from pagedcore_amd.kv_cache import BLOCK_TOKENS, CONTEXT_LIMIT, KVAllocator

EOS_TOKEN_ID = 2
MAX_NEW_TOKENS = 256  # reference src/pagedcore/config.py:31 (and generate's bound, decoder.py:79)


class FinishReason(str, Enum):
    """Why a request stopped (reference src/pagedcore/engine_types.py:63-65)."""

    EOS = "eos"
    LENGTH = "length"


@dataclass(frozen=True)
class GenerationRequest:
    """A prompt to complete greedily: up to max_new_tokens selected tokens."""

    request_id: RequestId
    input_ids: Tuple[int, ...]
    max_new_tokens: int = 128
    ignore_eos: bool = False

    def __post_init__(self) -> None:
        if not self.input_ids or any(type(t) is not int or t < 0 for t in self.input_ids):
            raise ValueError("input_ids must be a nonempty sequence of token ids")
        if type(self.max_new_tokens) is not int or not 1 <= self.max_new_tokens <= MAX_NEW_TOKENS:
            raise ValueError("max_new_tokens must be an integer from 1 to 256")
        if type(self.ignore_eos) is not bool:
            raise ValueError("ignore_eos must be a boolean")
        if len(self.input_ids) + self.max_new_tokens > CONTEXT_LIMIT:
            raise ValueError("prompt tokens plus requested output must not exceed 2048")

    @property
    def block_credits(self) -> int:
        """KV blocks the request can ever own: its prompt and every token it may decode."""
        return -(-(len(self.input_ids) + self.max_new_tokens) // BLOCK_TOKENS)


@dataclass(frozen=True)
class GreedyResult:
    """Selected ids; a stopping EOS is selected but excluded from emitted ids
    (reference src/pagedcore/decoder.py:61-67)."""

    greedy_ids: Tuple[int, ...]
    emitted_ids: Tuple[int, ...]
    finish_reason: FinishReason


@dataclass
class _Active:
    request: GenerationRequest
    selected: List[int] = field(default_factory=list)
    finish: Optional[FinishReason] = None


PrefillFn = Callable[[Tensor, object, KVAllocator, RequestId], Tensor]
DecodeFn = Callable[[Tensor, object, KVAllocator, Tuple[RequestId, ...]], Tensor]


class DecodeWorker:
    """The scheduler iteration of the module docstring over one allocator and model.

    `prefill` and `decode` default to the paged model (prefill_paged, decode_paged); tests
    substitute them. `graph_batch` (one size or several) names the batch sizes that get a
    captured DecodeGraph: a decode step of n requests replays the graph of the smallest
    such size >= n (padding rows write nothing and their logits are dropped), captured on
    first use or all at once by capture_graphs(); a step larger than every size runs
    decode_paged. `prefill_graph_tokens` does the same for admissions: a prompt of T
    positions replays the PrefillGraph of the smallest size >= T (it computes the last
    position's logits only, all the selection needs); longer prompts run prefill_paged.
    `vocab_size` (default: rows of `weights.embedding`, when the weights have one) bounds
    the token ids submit() accepts. A prefill that raises during admission releases the
    request's reservation and drops it from the active set before the error propagates.
    """

    def __init__(
        self,
        weights: object,
        allocator: KVAllocator,
        *,
        max_active: int = 32,
        eos_token_id: int = EOS_TOKEN_ID,
        prefill: Optional[PrefillFn] = None,
        decode: Optional[DecodeFn] = None,
        graph_batch: Union[None, int, Sequence[int]] = None,
        prefill_graph_tokens: Sequence[int] = (),
        vocab_size: Optional[int] = None,
    ) -> None:
        if type(max_active) is not int or max_active < 1:
            raise ValueError("max_active must be a positive integer")
        if vocab_size is None:
            embedding = getattr(weights, "embedding", None)
            vocab_size = None if embedding is None else int(embedding.shape[0])
        if vocab_size is not None and (type(vocab_size) is not int or vocab_size < 1):
            raise ValueError("vocab_size must be a positive integer")
        sizes = () if graph_batch is None else (graph_batch,) if isinstance(graph_batch, int) else tuple(graph_batch)
        if any(type(size) is not int or size < 1 for size in sizes):
            raise ValueError("graph batch sizes must be positive integers")
        prompt_sizes = tuple(prefill_graph_tokens)
        if any(type(size) is not int or not 1 <= size <= CONTEXT_LIMIT for size in prompt_sizes):
            raise ValueError("prefill graph sizes must be integers from 1 to 2048")
        if prefill is None or decode is None:
            from pagedcore_amd import decoder

            prefill = prefill or decoder.prefill_paged
            decode = decode or decoder.decode_paged
        self._weights = weights
        self._vocab = vocab_size
        self._allocator = allocator
        self._max_active = max_active
        self._eos = eos_token_id
        self._prefill = prefill
        self._decode = decode
        self._graph_sizes = tuple(sorted(set(sizes)))
        self._graphs: Dict[int, object] = {}
        self._prompt_sizes = tuple(sorted(set(prompt_sizes)))
        self._prefill_graphs: Dict[int, object] = {}
        # Waiting requests, each with its prompt as an int64 array (converted once, at
        # submit, off the iteration's critical path).
        self._pending: Deque[Tuple[GenerationRequest, np.ndarray]] = deque()
        self._active: Dict[RequestId, _Active] = {}
        self._cancelled: set = set()
        self._results: Dict[RequestId, GreedyResult] = {}
        self._known: set = set()
        self._fault: Optional[AttentionFaultError] = None
        self._host_tokens: Optional[Tensor] = None  # pinned read-back buffer of selected ids
        self._read_back_end = 0  # ids copied into it this iteration

    # -- queue -----------------------------------------------------------------------------

    def submit(self, request: GenerationRequest) -> None:
        """Queue a request. Token ids are checked against the model's vocabulary here, on
        the host: an id past the embedding table would be an out-of-bounds device read."""
        if request.request_id in self._known:
            raise ValueError("request IDs must be unique")
        if self._vocab is not None and max(request.input_ids) >= self._vocab:
            raise ValueError(f"input_ids must be below the vocabulary size {self._vocab}")
        if request.block_credits > self._allocator.pool.shape[2]:
            raise ValueError("request exceeds total KV pool capacity")
        self._known.add(request.request_id)
        self._pending.append((request, np.fromiter(request.input_ids, dtype=np.int64, count=len(request.input_ids))))

    def cancel(self, request_id: RequestId) -> None:
        """Stop a waiting or active request; its resources go at the next cleanup."""
        if request_id not in self._known:
            raise KeyError(request_id)
        self._cancelled.add(request_id)

    @property
    def idle(self) -> bool:
        return not self._pending and not self._active

    @property
    def active_ids(self) -> Tuple[RequestId, ...]:
        return tuple(self._active)

    @property
    def pending_ids(self) -> Tuple[RequestId, ...]:
        return tuple(r.request_id for r, _ in self._pending)

    @property
    def results(self) -> Dict[RequestId, GreedyResult]:
        return dict(self._results)

    # -- one iteration -----------------------------------------------------------------------

    @property
    def fault(self) -> Optional[AttentionFaultError]:
        """The device fault that stopped the worker, or None."""
        return self._fault

    def step(self) -> List[Tuple[RequestId, int]]:
        """Run one scheduler iteration; returns the (request, token) pairs emitted."""
        if self._fault is not None:
            raise RuntimeError("the decode worker stopped after a device fault") from self._fault
        try:
            return self._iterate()
        except AttentionFaultError as error:
            self._fault = error
            raise

    def _iterate(self) -> List[Tuple[RequestId, int]]:
        self._cleanup()
        self._read_back_end = 0
        emitted: List[Tuple[RequestId, int]] = []
        first = self._admit_one()  # (admitted request, its first token on the device)
        if first is not None:
            request = self._active[first[0]].request
            if request.max_new_tokens > 1 and not request.ignore_eos:
                # an EOS would finish it now, and a finished request must not be decoded
                self._select(first[0], int(first[1]), emitted)
                first = None
        # A request admitted with one token to select is finished by that token.
        batch = tuple(
            rid
            for rid, state in self._active.items()
            if state.finish is None and (first is None or rid != first[0] or state.request.max_new_tokens > 1)
        )
        chosen: List[Tensor] = []
        if first is not None:
            chosen.append(self._read_back(first[1].view(1)))  # enqueued before the decode step
        graph = None
        if batch:
            selected, graph = self._decode_batch(batch, first)
            chosen.append(self._read_back(selected))
        values = self._fetch(chosen)
        if graph is not None:
            graph.check_faults()  # decode_paged checks inside its step
        if first is not None:
            self._select(first[0], values[0], emitted)
            values = values[1:]
        for rid, token in zip(batch, values):
            self._select(rid, token, emitted)
        return emitted

    def _batch_tokens(self, batch: Tuple[RequestId, ...]) -> Tensor:
        """int64 [len(batch), 1] on the pool's device: each request's last selected token (0
        for one whose first token is still on the device), uploaded through pinned memory."""
        host = torch.tensor(
            [[self._active[rid].selected[-1] if self._active[rid].selected else 0] for rid in batch], dtype=torch.int64
        )
        device = self._device()
        if device.type != "cuda":
            return host.to(device)
        return host.pin_memory().to(device, non_blocking=True)

    def _read_back(self, values: Tensor) -> Tensor:
        """Enqueue the copy of selected ids (an int64 vector on the pool's device) into the
        pinned read-back buffer, after the ids already copied this iteration; returns the
        host tensor _fetch reads. The buffer is reused every iteration, and _fetch waits for
        the copies before anything reads it."""
        if values.device.type != "cuda":
            return values
        if self._host_tokens is None:
            self._host_tokens = torch.empty(self._max_active + 1, dtype=torch.int64, pin_memory=True)
        start = self._read_back_end
        end = start + values.numel()
        if end > self._host_tokens.numel():
            raise RuntimeError("more selected ids than the read-back buffer holds")
        self._host_tokens[start:end].copy_(values, non_blocking=True)
        self._read_back_end = end
        return self._host_tokens[start:end]

    def _fetch(self, chosen: List[Tensor]) -> List[int]:
        """The ids of this iteration's _read_back calls, in order, after one wait on an
        event recorded behind their copies (other streams keep running)."""
        if self._read_back_end:
            done = torch.cuda.Event()
            done.record()
            done.synchronize()
        return [int(v) for part in chosen for v in part.tolist()]

    def run(self, max_steps: Optional[int] = None) -> Dict[RequestId, GreedyResult]:
        """Iterate until every submitted request finished (and was cleaned up)."""
        steps = 0
        while not self.idle:
            if max_steps is not None and steps >= max_steps:
                raise RuntimeError("worker did not drain within max_steps")
            self.step()
            steps += 1
        return self.results

    # -- internals --------------------------------------------------------------------------

    def _device(self) -> torch.device:
        return self._allocator.pool.device

    def _cleanup(self) -> None:
        for rid in [rid for rid, state in self._active.items() if state.finish is not None or rid in self._cancelled]:
            state = self._active.pop(rid)
            self._allocator.release_all(rid)
            if state.finish is not None:
                self._results[rid] = self._result(state)
        if self._cancelled:
            self._pending = deque(item for item in self._pending if item[0].request_id not in self._cancelled)

    def _admit_one(self) -> Optional[Tuple[RequestId, Tensor]]:
        """Admit and prefill the queue head if it fits; returns it with its first token
        still on the device (argmax of the prompt's last logits), or None."""
        if not self._pending or len(self._active) >= self._max_active:
            return None
        request, prompt = self._pending[0]
        counts = self._allocator.capacity()
        if request.block_credits > counts.total_blocks - counts.reserved_blocks:
            return None  # waits (strict FIFO: nothing behind it is admitted first)
        self._pending.popleft()
        rid = request.request_id
        self._allocator.create(KVReservation(rid, request.block_credits))
        self._active[rid] = _Active(request)
        try:
            size = next((size for size in self._prompt_sizes if size >= len(prompt)), None)
            if size is not None:
                token = self._prefill_graph_for(size).greedy(prompt, rid)
            else:
                device = self._device()
                ids = torch.tensor(prompt, dtype=torch.int64).view(1, -1)
                ids = ids.pin_memory().to(device, non_blocking=True) if device.type == "cuda" else ids.to(device)
                token = self._prefill(ids, self._weights, self._allocator, rid)[0, -1].argmax()
        except BaseException:
            # A failed admission leaves nothing behind: the request leaves the active set
            # and its reservation (with any blocks a partial prefill published) is
            # released, so later iterations decode the others and the credits return.
            self._active.pop(rid, None)
            self._allocator.release_all(rid)
            raise
        return rid, token

    def _graph_for(self, size: int):
        graph = self._graphs.get(size)
        if graph is None:
            from pagedcore_amd.decoder import DecodeGraph

            graph = self._graphs[size] = DecodeGraph(self._weights, self._allocator, size)
        return graph

    def _prefill_graph_for(self, size: int):
        graph = self._prefill_graphs.get(size)
        if graph is None:
            from pagedcore_amd.decoder import PrefillGraph

            graph = self._prefill_graphs[size] = PrefillGraph(self._weights, self._allocator, size)
        return graph

    def capture_graphs(self) -> None:
        """Capture the DecodeGraph and PrefillGraph of every configured size now (each
        capture runs one eager forward with no pool writes), instead of at first use."""
        for size in self._graph_sizes:
            self._graph_for(size)
        for size in self._prompt_sizes:
            self._prefill_graph_for(size)

    def _decode_batch(self, batch: Tuple[RequestId, ...], first: Optional[Tuple[RequestId, Tensor]]):
        """The step's selected ids (int64 [len(batch)] on the device), and the DecodeGraph
        that ran it (None for eager decoding). Each request's input is its last selected
        id; `first`'s is still on the device (the prefill's selection, fed device to
        device)."""
        row = batch.index(first[0]) if first is not None and first[0] in batch else None
        size = next((size for size in self._graph_sizes if size >= len(batch)), None)
        if size is not None:
            graph = self._graph_for(size)
            ids = np.fromiter(
                (self._active[rid].selected[-1] if self._active[rid].selected else 0 for rid in batch),
                dtype=np.int64,
                count=len(batch),
            )
            return graph.greedy(ids, batch, None if row is None else (row, first[1])), graph
        tokens = self._batch_tokens(batch)
        if row is not None:
            tokens[row, 0] = first[1]
        return self._decode(tokens, self._weights, self._allocator, batch)[:, -1].argmax(dim=-1), None

    def _select(self, rid: RequestId, token: int, emitted: List[Tuple[RequestId, int]]) -> None:
        state = self._active[rid]
        state.selected.append(token)
        request = state.request
        if token == self._eos and not request.ignore_eos:
            state.finish = FinishReason.EOS  # selected, never emitted
        else:
            emitted.append((rid, token))
            if len(state.selected) == request.max_new_tokens:
                state.finish = FinishReason.LENGTH

    @staticmethod
    def _result(state: _Active) -> GreedyResult:
        ids = tuple(state.selected)
        emitted = ids[:-1] if state.finish is FinishReason.EOS else ids
        return GreedyResult(ids, emitted, state.finish)
