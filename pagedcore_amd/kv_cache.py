"""KV pool, reservation-aware block allocator and the staged block gather.

Drop-in for the reference's src/pagedcore/kv_cache.py: the pool layout, the allocator's
public methods, its LIFO block choice, error types/messages and its publish-after-write /
staged-decode semantics are the same. What changes is where the bytes move: every write
into the pool is one launch of the HIP `pc_kv_append` kernel (all layers and tokens of a
call at once) instead of a Python loop of `Tensor.copy_` calls, and attention reads the
pool through device block tables built here (`gather_block_tables`) instead of a page
generator.

Additions to the reference API (additive, for batched callers):
  * ``write_decode_layers`` writes one layer of a staged decode step for many requests in
    one launch;
  * ``gather_block_tables`` returns the device block table and context lengths that the
    attention kernel walks, with the same staged-layer rules as ``iter_layer_blocks``;
  * ``KVAllocator(pool, kv_writer=...)`` lets host-logic tests substitute the writer.
"""

from __future__ import annotations

from collections.abc import Iterator
from contextlib import contextmanager
from dataclasses import dataclass
from itertools import chain
from threading import current_thread
from typing import Dict, Optional, Protocol, Sequence, Tuple

import numpy as np
import torch
from torch import Tensor

from pagedcore_amd import _hip
from pagedcore_amd.config import PagedCoreConfig
from pagedcore_amd.engine_types import BlockId, BlockTable, CapacityCounts, KVReservation, RequestId

LAYERS = 22
BLOCK_TOKENS = 16
KV_HEADS = 4
HEAD_DIM = 64
CONTEXT_LIMIT = 2048
QKV_COLUMNS = (32 + 2 * KV_HEADS) * HEAD_DIM  # 2560: one token's q | k | v projections
MAX_BLOCKS_PER_REQUEST = CONTEXT_LIMIT // BLOCK_TOKENS  # 128


def allocate_kv_pool(config: PagedCoreConfig, *, device: str | torch.device = "cuda:0") -> Tensor:
    """Allocate the fp16 pool [22, 2, blocks, 16, 4, 64] once; keep it for the worker's life.

    Same sizing and memory checks as the reference (src/pagedcore/kv_cache.py:17-47):
    whole 352 KiB blocks within ``kv_pool_mib``, free memory for pool + margin checked
    before, margin re-checked after. Storage is uninitialised.
    """
    target = torch.device(device)
    if target.type != "cuda":
        raise ValueError("KV pool requires a CUDA device")
    if not torch.cuda.is_available():
        raise RuntimeError("KV pool requires an available CUDA runtime")

    pool_bytes = config.kv_pool_mib * 2**20
    margin_bytes = config.workspace_margin_mib * 2**20
    block_bytes = LAYERS * 2 * config.block_tokens * KV_HEADS * HEAD_DIM * 2
    num_blocks = pool_bytes // block_bytes
    free_bytes, _ = torch.cuda.mem_get_info(target)
    if free_bytes < pool_bytes + margin_bytes:
        raise RuntimeError("configured KV pool and workspace margin do not fit in GPU memory")

    pool = torch.empty(
        (LAYERS, 2, num_blocks, config.block_tokens, KV_HEADS, HEAD_DIM),
        dtype=torch.float16,
        device=target,
    )
    if torch.cuda.mem_get_info(target)[0] < margin_bytes:
        del pool
        raise RuntimeError("KV pool allocation leaves less than the configured workspace margin")
    return pool


class KVWriter(Protocol):
    """Moves token rows into the pool: pool[layer_begin + l, 0/1, s // 16, s % 16] = K/V[l, t]."""

    def append(
        self, pool: Tensor, layer_begin: int, key: Tensor, value: Tensor, slots: Sequence[int]
    ) -> None: ...

    def rope_append(
        self, pool: Tensor, layer: int, qkv: Tensor, rope_table: Tensor, positions: Tensor, slots: Tensor,
        query_out: Tensor,
    ) -> None:
        """RoPE on each row's query and key at `positions`; rotated key and value to
        pool[layer, 0/1, slot // 16, slot % 16]; rotated queries to query_out [B, 32, 1, 64]."""
        ...


class HipKVWriter:
    """The GPU data path: one `pc_kv_append` launch per call, on the current stream."""

    def __init__(self) -> None:
        _hip.load()  # fail at construction, not at the first write

    def append(
        self, pool: Tensor, layer_begin: int, key: Tensor, value: Tensor, slots: Sequence[int]
    ) -> None:
        if isinstance(slots, Tensor):
            slot_mapping = slots
        else:
            slot_mapping = torch.as_tensor(np.asarray(slots, dtype=np.int64)).to(pool.device)
        _hip.kv_append(pool, layer_begin, key, value, slot_mapping)

    def rope_append(
        self, pool: Tensor, layer: int, qkv: Tensor, rope_table: Tensor, positions: Tensor, slots: Tensor,
        query_out: Tensor,
    ) -> None:
        if qkv.ndim == 3:  # fp32 split-K partial sums of the projection
            _hip.rope_kv_append_parts(query_out, qkv, positions, rope_table, pool=pool, layer=layer, slot_mapping=slots)
        else:
            _hip.rope_kv_append(query_out, qkv, positions, rope_table, pool=pool, layer=layer, slot_mapping=slots)


class _HostOnlyWriter:
    """Stand-in for CPU pools: bookkeeping works, moving KV bytes does not."""

    def append(self, pool: Tensor, layer_begin: int, key: Tensor, value: Tensor, slots: Sequence[int]) -> None:
        raise RuntimeError(
            "KV writes run on the GPU: this allocator's pool is on the CPU and has no KV writer"
        )

    def rope_append(self, *args) -> None:
        raise RuntimeError(
            "KV writes run on the GPU: this allocator's pool is on the CPU and has no KV writer"
        )


@dataclass(eq=False)
class StagedPrompt:
    """A prompt append staged by KVAllocator.append_prompt: the caller writes each layer's
    K/V to `slot_mapping` itself and records it with record_layer, in layer order.

    `slots` holds the slot mapping on the host; `slot_mapping` and `positions` are its
    device copies, uploaded together on first use (a caller that stages its inputs itself,
    such as a graph replay, reads `slots` and uploads nothing here)."""

    request_id: RequestId
    tokens: int
    slots: np.ndarray  # int64 [tokens]: block * 16 + offset of each new position
    start: int  # the first new position (the cached length before the append)
    device: torch.device
    written_layers: int = 0
    _uploaded: Optional[Tensor] = None

    def _device_rows(self) -> Tensor:
        if self._uploaded is None:
            positions = np.arange(self.start, self.start + self.tokens, dtype=np.int64)
            self._uploaded = _upload(np.stack([self.slots, positions]), self.device)
        return self._uploaded

    @property
    def slot_mapping(self) -> Tensor:
        """int64 [tokens] on the pool's device: block * 16 + offset of each new position."""
        return self._device_rows()[0]

    @property
    def positions(self) -> Tensor:
        """int64 [tokens] on the pool's device: the new positions (start .. + tokens - 1)."""
        return self._device_rows()[1]

    def record_layer(self, layer_index: int) -> None:
        if type(layer_index) is not int or layer_index != self.written_layers or layer_index >= LAYERS:
            raise ValueError("prompt cache layers must be written once in order")
        self.written_layers += 1


@dataclass(frozen=True)
class StagedDecode:
    """Host arrays of a staged decode step (KVAllocator.staged_decode)."""

    slots: np.ndarray  # int64 [B]: block * 16 + offset of each request's new position
    positions: np.ndarray  # int64 [B]: that position (the cached length before the step)
    lengths: np.ndarray  # int32 [B]: staged lengths (cached length + 1)
    tables: np.ndarray  # int32 [B, width]: staged block tables in logical order, zero padded


@dataclass(slots=True)
class _DecodeBatch:
    """Device block tables and lengths of one batch of requests, plus their host copies
    and the decode plan built from them (on first use). `appends` are the staged appends
    of the batch's requests when it was built: a later lookup of the same allocator state
    only has to check that their layer is written."""

    tables: Tensor
    lengths: Tensor
    host_tables: np.ndarray
    host_lengths: np.ndarray
    appends: Tuple["_TokenAppend", ...] = ()
    plan: Optional[Tensor] = None


@dataclass(frozen=True, slots=True)
class _SequenceCache:
    reservation: KVReservation
    blocks: BlockTable = ()
    length: int = 0


@dataclass(slots=True)
class _TokenAppend:
    sequence: _SequenceCache
    written_layers: int = 0


def _counting(base: type, names: Tuple[str, ...]) -> type:
    """Subclass of list/dict whose mutating methods bump a `mutations` counter, so the
    accounting check can tell in O(1) whether a container changed since it was verified."""

    def wrap(name: str):
        method = getattr(base, name)

        def counted(self, *args, **kwargs):
            self.mutations += 1
            return method(self, *args, **kwargs)

        counted.__name__ = name
        return counted

    namespace = {name: wrap(name) for name in names}
    namespace["__slots__"] = ("mutations",)

    def __init__(self, *args, **kwargs):
        base.__init__(self, *args, **kwargs)
        self.mutations = 0

    namespace["__init__"] = __init__
    return type(f"_Counting{base.__name__.title()}", (base,), namespace)


_CountingList = _counting(
    list,
    ("__setitem__", "__delitem__", "__iadd__", "__imul__", "append", "extend", "insert", "pop", "remove",
     "clear", "sort", "reverse"),
)
_CountingDict = _counting(
    dict, ("__setitem__", "__delitem__", "__ior__", "pop", "popitem", "clear", "update", "setdefault")
)


def _upload(array: np.ndarray, device: torch.device) -> Tensor:
    """A host array on `device`. For a GPU the copy goes through pinned memory and is
    enqueued on the current stream without blocking the host (a copy from pageable memory
    would wait for the stream to drain); torch keeps the pinned buffer until the copy has
    run, and every consumer is ordered after it on the same stream."""
    tensor = torch.from_numpy(np.ascontiguousarray(array))
    if device.type != "cuda":
        return tensor.to(device)
    return tensor.pin_memory().to(device, non_blocking=True)


def _slot_mapping(blocks: BlockTable, start: int, count: int) -> np.ndarray:
    """Pool slot (block * 16 + offset) of positions start .. start + count - 1."""
    positions = np.arange(start, start + count, dtype=np.int64)
    table = np.asarray(blocks, dtype=np.int64)
    return table[positions // BLOCK_TOKENS] * BLOCK_TOKENS + positions % BLOCK_TOKENS


class KVAllocator:
    """Assign blocks within an existing pool; construct and use on the model worker.

    CUDA work stays on the stream current at construction. Block reads borrow pool
    storage: treat them as read-only and do not keep them past an append or release.
    CPU pools support the bookkeeping (tests); their KV writes need an explicit writer.
    """

    def __init__(self, pool: Tensor, *, kv_writer: Optional[KVWriter] = None) -> None:
        if (
            pool.ndim != 6
            or pool.shape[:2] != (LAYERS, 2)
            or pool.shape[2] < 1
            or pool.shape[3:] != (BLOCK_TOKENS, KV_HEADS, HEAD_DIM)
            or pool.dtype != torch.float16
            or pool.device.type not in ("cpu", "cuda")
            or not pool.is_contiguous()
            or pool.requires_grad
        ):
            raise ValueError("KV pool must be contiguous FP16 [22, 2, blocks, 16, 4, 64] storage")
        if kv_writer is None:
            kv_writer = HipKVWriter() if pool.is_cuda else _HostOnlyWriter()
        self._pool = pool
        self._writer = kv_writer
        self._worker = current_thread()
        self._stream = torch.cuda.current_stream(pool.device) if pool.is_cuda else None
        self._stream_handle = self._stream.cuda_stream if self._stream is not None else None
        self._free_blocks = _CountingList(BlockId(index) for index in reversed(range(pool.shape[2])))
        self._sequences: Dict[RequestId, _SequenceCache] = _CountingDict()
        # Tables are checked against the owners recorded when blocks are assigned.
        self._block_owners: Dict[BlockId, RequestId] = _CountingDict()
        # (container identities and mutation counts, counts) of the last verified state.
        self._verified: Optional[Tuple[tuple, CapacityCounts]] = None
        self._decode_appends: Optional[Dict[RequestId, _TokenAppend]] = None
        self._prompt_append: Optional[StagedPrompt] = None
        # Bumped whenever a table or length may change; keys the device-table cache.
        self._version = 0
        self._table_cache: Dict[tuple, _DecodeBatch] = {}
        self._decode_slot_cache: Dict[Tuple[RequestId, ...], Tuple[Tensor, Tensor]] = {}

    @property
    def pool(self) -> Tensor:
        return self._pool

    def create(self, reservation: KVReservation) -> None:
        """Grant credits at admission without assigning physical blocks."""
        self._check_mutation()
        request_id = reservation.request_id
        if request_id in self._sequences:
            raise ValueError("request already has a KV cache")
        counts = self.capacity()
        if reservation.maximum_block_credits > counts.total_blocks:
            raise ValueError("reservation exceeds total KV pool capacity")
        if reservation.maximum_block_credits > MAX_BLOCKS_PER_REQUEST:
            raise ValueError("reservation exceeds KV context capacity")
        if reservation.maximum_block_credits > counts.total_blocks - counts.reserved_blocks:
            raise RuntimeError("KV pool has insufficient unreserved blocks")
        before = self._verified_counts()
        self._sequences[request_id] = _SequenceCache(reservation)
        self._touch()
        credits = reservation.maximum_block_credits
        self._recount(
            before if type(credits) is int and 0 < credits <= MAX_BLOCKS_PER_REQUEST else None,
            reserved=credits,
            active=1,
        )

    def capacity(self) -> CapacityCounts:
        """Snapshot ownership and credits, including requests awaiting cleanup."""
        self._check_worker()
        return self._assert_accounting()

    def block_table(self, request_id: RequestId) -> BlockTable:
        self._check_worker()
        self._assert_accounting()
        return self._sequences[request_id].blocks

    def cached_length(self, request_id: RequestId) -> int:
        self._check_worker()
        self._assert_accounting()
        return self._sequences[request_id].length

    def cached_lengths(self, request_ids: Sequence[RequestId]) -> Tuple[int, ...]:
        """cached_length of each request, with the worker and accounting checks done once
        for the batch; KeyError for the first unknown request."""
        self._check_worker()
        self._assert_accounting()
        sequences = self._sequences
        return tuple(sequences[request_id].length for request_id in request_ids)

    @torch.inference_mode()
    def append(self, request_id: RequestId, key: Tensor, value: Tensor) -> None:
        """Append rotated K and unrotated V, each FP16 [22, tokens, 4, 64].

        All checks run before the launch; the new length and blocks are published only
        after the launch was accepted, so a failed write leaves ownership and the valid
        positions unchanged (unpublished slots may be dirty).
        """
        self._check_mutation()
        self._assert_accounting()
        sequence = self._sequences[request_id]
        if (
            key.ndim != 4
            or key.shape[0] != LAYERS
            or key.shape[1] < 1
            or key.shape[2:] != (KV_HEADS, HEAD_DIM)
            or value.shape != key.shape
            or key.dtype != torch.float16
            or value.dtype != torch.float16
            or key.device != self._pool.device
            or value.device != self._pool.device
        ):
            raise ValueError("K and V must share FP16 [22, tokens, 4, 64] on the pool device")
        length = sequence.length + key.shape[1]
        if length > CONTEXT_LIMIT:
            raise ValueError("KV cache must not exceed 2048 token positions")
        required = (length + BLOCK_TOKENS - 1) // BLOCK_TOKENS
        if required > sequence.reservation.maximum_block_credits:
            raise RuntimeError("KV append exceeds request reservation")
        additional = required - len(sequence.blocks)
        if additional > len(self._free_blocks):
            raise RuntimeError("KV pool has insufficient free blocks")
        new_blocks = tuple(reversed(self._free_blocks[-additional:])) if additional else ()
        blocks = sequence.blocks + new_blocks

        self._writer.append(self._pool, 0, key, value, _slot_mapping(blocks, sequence.length, key.shape[1]))

        # Publish valid positions only after the K and V writes have been issued.
        before = self._verified_counts()
        if additional:
            del self._free_blocks[-additional:]
        self._block_owners.update((block, request_id) for block in new_blocks)
        self._sequences[request_id] = _SequenceCache(sequence.reservation, blocks, length)
        self._touch()
        self._recount(before, moved=additional, tokens=key.shape[1])

    @contextmanager
    def append_prompt(self, request_id: RequestId, tokens: int) -> Iterator[StagedPrompt]:
        """Stage an append of `tokens` positions whose K/V the caller writes itself, layer
        by layer (the fused prefill path: RoPE writes each layer's rotated K and V straight
        into the slots append would fill).

        The checks are append's (src/pagedcore/kv_cache.py:137-157), run before anything is
        staged; the new blocks are the ones append would take (the free-list tail), only
        borrowed while staged. The append is published when the block exits normally with
        all 22 layers recorded; any exception discards it (the borrowed blocks stay free;
        their slots may be dirty, as after a failed append). Other mutations raise meanwhile.
        """
        self._check_mutation()
        self._assert_accounting()
        sequence = self._sequences[request_id]
        if type(tokens) is not int or tokens < 1:
            raise ValueError("a prompt append needs a positive integer token count")
        length = sequence.length + tokens
        if length > CONTEXT_LIMIT:
            raise ValueError("KV cache must not exceed 2048 token positions")
        required = (length + BLOCK_TOKENS - 1) // BLOCK_TOKENS
        if required > sequence.reservation.maximum_block_credits:
            raise RuntimeError("KV append exceeds request reservation")
        additional = required - len(sequence.blocks)
        if additional > len(self._free_blocks):
            raise RuntimeError("KV pool has insufficient free blocks")
        new_blocks = tuple(reversed(self._free_blocks[-additional:])) if additional else ()
        blocks = sequence.blocks + new_blocks
        staged = StagedPrompt(request_id, tokens, _slot_mapping(blocks, sequence.length, tokens), sequence.length,
                              self._pool.device)
        self._prompt_append = staged
        self._touch()
        try:
            yield staged
            if staged.written_layers != LAYERS:
                raise RuntimeError("prompt append must write every cache layer before committing")
            before = self._verified_counts()
            if self._sequences.get(request_id) is not sequence:
                before = None  # replaced from outside while staged: check everything
            if additional:
                del self._free_blocks[-additional:]
            self._block_owners.update((block, request_id) for block in new_blocks)
            self._sequences[request_id] = _SequenceCache(sequence.reservation, blocks, length)
            self._recount(before, moved=additional, tokens=tokens)
        finally:
            self._prompt_append = None
            self._touch()

    @contextmanager
    def append_decode(self, request_ids: Tuple[RequestId, ...]) -> Iterator[None]:
        """Stage one token per request; commit only if all 22 layers were written.

        Blocks for requests at a 16-token boundary are borrowed from the free-list tail in
        request order and only removed from it on commit; any exception discards the
        staged state (reference src/pagedcore/kv_cache.py:181-219).
        """
        self._check_mutation()
        self._assert_accounting()
        if not request_ids or len(set(request_ids)) != len(request_ids):
            raise ValueError("decode requires nonempty, distinct request IDs")
        appends: Dict[RequestId, _TokenAppend] = {}
        additional = 0
        for request_id in request_ids:
            sequence = self._sequences[request_id]
            if not 1 <= sequence.length < CONTEXT_LIMIT:
                raise ValueError("decode requires 1 to 2047 cached token positions")
            length = sequence.length + 1
            blocks = sequence.blocks
            if (length + BLOCK_TOKENS - 1) // BLOCK_TOKENS > sequence.reservation.maximum_block_credits:
                raise RuntimeError("KV append exceeds request reservation")
            if sequence.length % BLOCK_TOKENS == 0:
                additional += 1
                if additional > len(self._free_blocks):
                    raise RuntimeError("KV pool has insufficient free blocks")
                blocks += (self._free_blocks[-additional],)
            appends[request_id] = _TokenAppend(_SequenceCache(sequence.reservation, blocks, length))

        # Block other mutations while free-list entries are borrowed for staged writes.
        self._decode_appends = appends
        self._touch()
        try:
            yield
            if any(append.written_layers != LAYERS for append in appends.values()):
                raise RuntimeError("decode must write every cache layer before committing")
            before = self._verified_counts()
            if additional:
                del self._free_blocks[-additional:]
            for request_id, append in appends.items():
                original = self._sequences[request_id]
                for block in append.sequence.blocks[len(original.blocks) :]:
                    self._block_owners[block] = request_id
                self._sequences[request_id] = append.sequence
            if before is None:
                self._assert_accounting()
            else:
                # The state was verified when the step began and nothing changed it since:
                # the commit only moves `additional` verified free blocks (distinct, in
                # range, unowned) to the requests that staged them and lengthens each
                # staged request by one position within its credits (checked at staging),
                # so every invariant still holds and the counts move by exactly that.
                self._remember(
                    CapacityCounts(
                        total_blocks=before.total_blocks,
                        free_blocks=before.free_blocks - additional,
                        owned_blocks=before.owned_blocks + additional,
                        reserved_blocks=before.reserved_blocks,
                        active_slots=before.active_slots,
                        live_cached_token_slots=before.live_cached_token_slots + len(appends),
                    )
                )
        finally:
            self._decode_appends = None
            self._touch()

    @torch.inference_mode()
    def write_decode_layer(
        self, request_id: RequestId, layer_index: int, key: Tensor, value: Tensor
    ) -> None:
        """Write one token's rotated K / unrotated V, FP16 [4, 64], in layer order."""
        self._check_worker()
        self._check_staged_state()
        if self._decode_appends is None:
            raise RuntimeError("decode writes require a staged append")
        append = self._decode_appends[request_id]
        if type(layer_index) is not int or not 0 <= layer_index < LAYERS:
            raise ValueError("layer_index must identify one of the 22 decoder layers")
        if layer_index != append.written_layers:
            raise ValueError("decode cache layers must be written once in order")
        if any(
            tensor.shape != (KV_HEADS, HEAD_DIM)
            or tensor.dtype != torch.float16
            or tensor.device != self._pool.device
            for tensor in (key, value)
        ):
            raise ValueError("K and V must share FP16 [4, 64] on the pool device")
        logical_block, slot = divmod(append.sequence.length - 1, BLOCK_TOKENS)
        block = append.sequence.blocks[logical_block]
        self._writer.append(self._pool, layer_index, key[None, None], value[None, None], [block * BLOCK_TOKENS + slot])
        append.written_layers += 1

    @torch.inference_mode()
    def write_decode_layers(
        self,
        request_ids: Tuple[RequestId, ...],
        layer_index: int,
        key: Tensor,
        value: Tensor,
    ) -> None:
        """Batched write_decode_layer: row b of FP16 [B, 4, 64] K/V goes to request_ids[b].

        Every row is checked before the single launch; written layers advance together.
        """
        self._check_worker()
        self._check_staged_state()
        if self._decode_appends is None:
            raise RuntimeError("decode writes require a staged append")
        if not request_ids or len(set(request_ids)) != len(request_ids):
            raise ValueError("decode requires nonempty, distinct request IDs")
        appends = [self._decode_appends[request_id] for request_id in request_ids]
        if type(layer_index) is not int or not 0 <= layer_index < LAYERS:
            raise ValueError("layer_index must identify one of the 22 decoder layers")
        if any(layer_index != append.written_layers for append in appends):
            raise ValueError("decode cache layers must be written once in order")
        if any(
            tensor.shape != (len(request_ids), KV_HEADS, HEAD_DIM)
            or tensor.dtype != torch.float16
            or tensor.device != self._pool.device
            for tensor in (key, value)
        ):
            raise ValueError("K and V must share FP16 [batch, 4, 64] on the pool device")
        slots, _ = self._decode_slots(request_ids, appends)
        self._writer.append(self._pool, layer_index, key[None], value[None], slots)
        for append in appends:
            append.written_layers += 1

    @torch.inference_mode()
    def write_decode_layers_rotary(
        self,
        request_ids: Tuple[RequestId, ...],
        layer_index: int,
        qkv: Tensor,
        rope_table: Tensor,
    ) -> Tensor:
        """Fused RoPE + write_decode_layers, the batched decoder's per-layer write.

        qkv: FP16 [B, >= 2560] on the pool device, unit column stride: row b holds the
        query (32 x 64), key (4 x 64) and value (4 x 64) projections of request_ids[b]'s
        new token; or the same projections as contiguous FP32 split-K partial sums
        [splits, B, 2560] (pc_gemm_m128's output), rounded to FP16 once. rope_table: FP16 [rope positions, 2, 32] cos/sin table. Row b's query and
        key are rotated at the request's position (its cached length before this step, as
        the reference decoder passes it to apply_rope, src/pagedcore/decoder.py:173-186);
        the rotated key and the unrotated value go to the staged slot of this layer, like
        write_decode_layer. Returns the rotated queries, FP16 [B, 32, 1, 64]. Same checks,
        errors and layer-order rules as write_decode_layers; one launch for all rows.
        """
        self._check_worker()
        self._check_staged_state()
        if self._decode_appends is None:
            raise RuntimeError("decode writes require a staged append")
        if not request_ids or len(set(request_ids)) != len(request_ids):
            raise ValueError("decode requires nonempty, distinct request IDs")
        appends = [self._decode_appends[request_id] for request_id in request_ids]
        if type(layer_index) is not int or not 0 <= layer_index < LAYERS:
            raise ValueError("layer_index must identify one of the 22 decoder layers")
        if any(layer_index != append.written_layers for append in appends):
            raise ValueError("decode cache layers must be written once in order")
        if qkv.ndim == 3:
            if (
                qkv.shape[1:] != (len(request_ids), QKV_COLUMNS)
                or not 1 <= qkv.shape[0] <= 64
                or qkv.dtype != torch.float32
                or not qkv.is_contiguous()
                or qkv.device != self._pool.device
            ):
                raise ValueError("qkv partial sums must be contiguous FP32 [splits, batch, 2560] on the pool device")
        elif (
            qkv.ndim != 2
            or qkv.shape[0] != len(request_ids)
            or qkv.shape[1] < QKV_COLUMNS
            or qkv.stride(1) != 1
            or qkv.dtype != torch.float16
            or qkv.device != self._pool.device
        ):
            raise ValueError("qkv must be FP16 [batch, >= 2560] rows on the pool device")
        if (
            rope_table.ndim != 3
            or rope_table.shape[1:] != (2, HEAD_DIM // 2)
            or rope_table.shape[0] < CONTEXT_LIMIT
            or rope_table.dtype != torch.float16
            or rope_table.device != self._pool.device
            or not rope_table.is_contiguous()
        ):
            raise ValueError("rope_table must be contiguous FP16 [>= 2048, 2, 32] on the pool device")
        slots, positions = self._decode_slots(request_ids, appends)
        query = torch.empty((len(request_ids), 32, 1, HEAD_DIM), dtype=torch.float16, device=self._pool.device)
        self._writer.rope_append(self._pool, layer_index, qkv, rope_table, positions, slots, query)
        for append in appends:
            append.written_layers += 1
        return query

    def _decode_slots(self, request_ids: Tuple[RequestId, ...], appends: Sequence[_TokenAppend]):
        """(slot, position) of each staged token: slot = block * 16 + offset of position
        length - 1; device int64 tensors cached for the decode step on GPU pools."""
        cached = self._decode_slot_cache.get(request_ids)
        if cached is not None:
            return cached
        slots = np.empty(len(appends), dtype=np.int64)
        positions = np.empty(len(appends), dtype=np.int64)
        for row, append in enumerate(appends):
            position = append.sequence.length - 1
            logical_block, slot = divmod(position, BLOCK_TOKENS)
            slots[row] = append.sequence.blocks[logical_block] * BLOCK_TOKENS + slot
            positions[row] = position
        if not self._pool.is_cuda:
            return slots, positions
        both = _upload(np.stack([slots, positions]), self._pool.device)
        result = (both[0], both[1])
        self._decode_slot_cache[request_ids] = result
        return result

    def staged_decode(self, request_ids: Sequence[RequestId], *, width: Optional[int] = None) -> "StagedDecode":
        """Host view of the staged decode step, for callers that enqueue the step's KV
        writes and reads themselves (a captured HIP graph replayed on this allocator's
        stream): per row, the slot and position of the request's new token, its staged
        length and its staged block table (zero padded to `width`, default the widest).

        Pair with record_decode_writes once the writes are enqueued.
        """
        self._check_worker()
        self._check_staged_state()
        if self._decode_appends is None:
            raise RuntimeError("decode writes require a staged append")
        if not request_ids or len(set(request_ids)) != len(request_ids):
            raise ValueError("decode requires nonempty, distinct request IDs")
        appends = [self._decode_appends[request_id] for request_id in request_ids]
        sequences = [append.sequence for append in appends]
        widest = max(len(sequence.blocks) for sequence in sequences)
        if width is None:
            width = widest
        elif widest > width:
            raise ValueError("staged block tables are wider than the requested width")
        counts = np.fromiter((len(sequence.blocks) for sequence in sequences), dtype=np.int64, count=len(sequences))
        flat = np.fromiter(chain.from_iterable(sequence.blocks for sequence in sequences), dtype=np.int32, count=int(counts.sum()))
        tables = np.zeros((len(sequences), width), dtype=np.int32)
        tables[np.arange(width) < counts[:, None]] = flat  # row-major: each row's blocks in order
        lengths = np.fromiter((sequence.length for sequence in sequences), dtype=np.int32, count=len(sequences))
        positions = lengths.astype(np.int64) - 1
        # the new position's slot: block (position // 16) of the row's table, offset position % 16
        rows = np.arange(len(sequences))
        slots = tables[rows, positions // BLOCK_TOKENS].astype(np.int64) * BLOCK_TOKENS + positions % BLOCK_TOKENS
        return StagedDecode(slots, positions, lengths, tables)

    def record_decode_writes(self, request_ids: Sequence[RequestId], layers: int = LAYERS) -> None:
        """Record that the caller has enqueued, on this allocator's stream, the staged
        token's K/V writes of layers [0, layers) for every request (each layer's write
        ahead of any read of that layer), as write_decode_layers would have. Layers are
        still written once and in order: every request must be at layer 0."""
        self._check_worker()
        self._check_staged_state()
        if self._decode_appends is None:
            raise RuntimeError("decode writes require a staged append")
        if not request_ids or len(set(request_ids)) != len(request_ids):
            raise ValueError("decode requires nonempty, distinct request IDs")
        appends = [self._decode_appends[request_id] for request_id in request_ids]
        if type(layers) is not int or not 0 < layers <= LAYERS:
            raise ValueError("layers must count 1 to 22 decoder layers")
        if any(append.written_layers != 0 for append in appends):
            raise ValueError("decode cache layers must be written once in order")
        for append in appends:
            append.written_layers = layers

    def iter_layer_blocks(
        self, request_id: RequestId, *, layer_index: int
    ) -> Iterator[Tuple[Tensor, Tensor]]:
        """Borrow valid [slots, 4, 64] pages, including a completed staged layer."""
        sequence = self._layer_sequence(request_id, layer_index)
        for logical_block, physical_block in enumerate(sequence.blocks):
            self._check_worker()
            valid = min(BLOCK_TOKENS, sequence.length - logical_block * BLOCK_TOKENS)
            yield (
                self._pool[layer_index, 0, physical_block, :valid],
                self._pool[layer_index, 1, physical_block, :valid],
            )

    def _layer_sequence(self, request_id: RequestId, layer_index: int) -> _SequenceCache:
        """The table/length attention must read for a layer (the staged gather rules).

        Same checks and order as the reference's iter_layer_blocks
        (src/pagedcore/kv_cache.py:252-263): worker, accounting, layer index, unknown
        request (KeyError), unwritten staged layer (RuntimeError), empty cache (ValueError).
        """
        self._check_worker()
        self._check_staged_state((request_id,))
        if type(layer_index) is not int or not 0 <= layer_index < LAYERS:
            raise ValueError("layer_index must identify one of the 22 decoder layers")
        return self._staged_sequence(request_id, layer_index)

    def _staged_sequence(self, request_id: RequestId, layer_index: int) -> _SequenceCache:
        sequence = self._sequences[request_id]
        if self._decode_appends is not None and request_id in self._decode_appends:
            append = self._decode_appends[request_id]
            if layer_index >= append.written_layers:
                raise RuntimeError("cannot read an unwritten decode layer")
            sequence = append.sequence
        if sequence.length == 0:
            raise ValueError("attention requires a nonempty cache")
        return sequence

    def gather_block_tables(
        self, request_ids: Sequence[RequestId], *, layer_index: int
    ) -> Tuple[Tensor, Tensor]:
        """Device block tables int32 [B, W] and context lengths int32 [B] for a layer.

        Row b lists request_ids[b]'s physical blocks in logical order (staged tables for
        requests whose staged layer is written); W is the longest table in the batch.
        Cached per allocator state, so the 22 layers of a decode step share one upload.
        """
        batch = self._gather(request_ids, layer_index)
        return batch.tables, batch.lengths

    def decode_plan(self, request_ids: Sequence[RequestId], *, layer_index: int) -> Tensor:
        """Device decode plan (pc_attn_plan rows: balanced bins of the batch's blocks) for the
        batch that gather_block_tables returns, built once per allocator state from the host
        tables, so the 22 layers of a decode step share it."""
        batch = self._gather(request_ids, layer_index)
        if batch.plan is None:
            plan = _hip.decode_plan(batch.host_lengths, batch.host_tables)
            batch.plan = _upload(plan, self._pool.device)
        return batch.plan

    def _gather(self, request_ids: Sequence[RequestId], layer_index: int) -> _DecodeBatch:
        if not request_ids:
            raise ValueError("attention requires at least one request")
        self._check_worker()
        self._check_staged_state(request_ids)
        if type(layer_index) is not int or not 0 <= layer_index < LAYERS:
            raise ValueError("layer_index must identify one of the 22 decoder layers")
        staged = self._decode_appends is not None
        key = (self._version, tuple(request_ids), staged)
        cached = self._table_cache.get(key)
        # Same allocator state and requests: the requests exist and are nonempty, so only
        # the written-layer check of the staged ones can fail; if it would, the full
        # per-request checks below raise in the reference's order.
        if cached is not None and all(layer_index < append.written_layers for append in cached.appends):
            return cached
        sequences = [self._staged_sequence(request_id, layer_index) for request_id in request_ids]
        if cached is not None:
            return cached
        width = max(len(sequence.blocks) for sequence in sequences)
        tables = np.zeros((len(sequences), width), dtype=np.int32)
        lengths = np.empty(len(sequences), dtype=np.int32)
        for row, sequence in enumerate(sequences):
            tables[row, : len(sequence.blocks)] = sequence.blocks
            lengths[row] = sequence.length
        appends = self._decode_appends or {}
        result = _DecodeBatch(
            _upload(tables, self._pool.device),
            _upload(lengths, self._pool.device),
            tables,
            lengths,
            tuple(appends[request_id] for request_id in request_ids if request_id in appends),
        )
        if len(self._table_cache) > 64:
            self._table_cache.clear()
        self._table_cache[key] = result
        return result

    def read_block(self, request_id: RequestId, logical_block: int) -> Tuple[Tensor, Tensor]:
        """Borrow K/V views [22, valid slots, 4, 64] for one logical block."""
        self._check_worker()
        self._assert_accounting()
        sequence = self._sequences[request_id]
        if type(logical_block) is not int or not 0 <= logical_block < len(sequence.blocks):
            raise ValueError("logical block must identify a cached block")
        physical_block = sequence.blocks[logical_block]
        valid = min(BLOCK_TOKENS, sequence.length - logical_block * BLOCK_TOKENS)
        return (
            self._pool[:, 0, physical_block, :valid],
            self._pool[:, 1, physical_block, :valid],
        )

    def release_all(self, request_id: RequestId) -> None:
        """Release once on the worker stream; unknown/released requests raise KeyError."""
        self._check_mutation()
        self._assert_accounting()
        before = self._verified_counts()
        sequence = self._sequences.pop(request_id)
        for block in sequence.blocks:
            del self._block_owners[block]
        self._free_blocks.extend(reversed(sequence.blocks))
        self._touch()
        self._recount(
            before,
            moved=-len(sequence.blocks),
            tokens=-sequence.length,
            reserved=-sequence.reservation.maximum_block_credits,
            active=-1,
        )

    def _touch(self) -> None:
        self._version += 1
        self._table_cache.clear()
        self._decode_slot_cache.clear()

    def _check_staged_state(self, request_ids: Optional[Sequence[RequestId]] = None) -> None:
        """Accounting check of the per-layer calls of a decode step: _assert_accounting on
        every call, inside a staged decode as well, as the reference's write_decode_layer
        does (src/pagedcore/kv_cache.py:231). A corruption planted between two layer
        writes therefore raises at the next write, before anything is published. The
        check is memoised on the bookkeeping containers' mutation counts, so an
        unchanged state costs a key comparison, not a pool scan. `request_ids` is
        accepted for the callers' symmetry and does not change the check."""
        del request_ids
        self._assert_accounting()

    def _check_mutation(self) -> None:
        self._check_worker()
        if self._decode_appends is not None:
            raise RuntimeError("KV mutation is not allowed during a staged decode append")
        if self._prompt_append is not None:
            raise RuntimeError("KV mutation is not allowed during a staged prompt append")

    def _check_worker(self) -> None:
        if current_thread() is not self._worker:
            raise RuntimeError("KV allocator must be used by its owning model worker")
        if self._stream is not None and _hip.current_stream_handle(self._pool.device) != self._stream_handle:
            raise RuntimeError("KV allocator must use its owning CUDA stream")

    def _state_key(self) -> Optional[tuple]:
        """Identity and mutation count of each bookkeeping container (None if one of them
        is not a counting container, e.g. replaced from outside: then nothing is cached)."""
        containers = (self._free_blocks, self._sequences, self._block_owners)
        if not all(isinstance(c, (_CountingList, _CountingDict)) for c in containers):
            return None
        return tuple((id(c), c.mutations) for c in containers)

    def _verified_counts(self) -> Optional[CapacityCounts]:
        """The counts of the last full check if no container changed since, else None."""
        key = self._state_key()
        if key is not None and self._verified is not None and self._verified[0] == key:
            return self._verified[1]
        return None

    def _remember(self, counts: CapacityCounts) -> None:
        key = self._state_key()
        self._verified = None if key is None else (key, counts)

    def _recount(
        self, before: Optional[CapacityCounts], *, moved: int = 0, tokens: int = 0, reserved: int = 0, active: int = 0
    ) -> None:
        """Accounting after one of this allocator's own mutations. `before` is the verified
        state it started from (None: not verified, or changed from outside since): then the
        full check runs, as the reference does after every mutation. Otherwise the mutation
        was one of the few this class makes, each of which keeps every invariant by
        construction from a verified state (blocks leave the free-list tail for the request
        that was checked to hold the credits, a released request's verified blocks return
        to the free list, a new request starts empty within its checked credits), so the
        counts move by exactly `moved` blocks from free to owned (negative: back), `tokens`
        cached positions, `reserved` credits and `active` slots, and are remembered as
        verified without rescanning the pool."""
        if before is None:
            self._assert_accounting()
            return
        self._remember(
            CapacityCounts(
                total_blocks=before.total_blocks,
                free_blocks=before.free_blocks - moved,
                owned_blocks=before.owned_blocks + moved,
                reserved_blocks=before.reserved_blocks + reserved,
                active_slots=before.active_slots + active,
                live_cached_token_slots=before.live_cached_token_slots + tokens,
            )
        )

    def _assert_accounting(self) -> CapacityCounts:
        """Full ownership invariants (reference src/pagedcore/kv_cache.py:314-357).

        Same checks and messages. The check is a pure function of the three bookkeeping
        containers, which count their own mutations: when none changed since the last
        full check passed, its counts are returned without rescanning the pool (any
        change, including one made from outside through the containers' methods, forces
        the full scan). The per-block type/range scans run as C-level set and min/max
        passes rather than a Python loop.
        """
        cached = self._verified_counts()
        if cached is not None:
            return cached
        counts = self._full_accounting()
        self._remember(counts)
        return counts

    def _full_accounting(self) -> CapacityCounts:
        total = self._pool.shape[2]
        for request_id, sequence in self._sequences.items():
            if (
                sequence.reservation.request_id != request_id
                or type(sequence.length) is not int
                or not 0 <= sequence.length <= CONTEXT_LIMIT
                or type(sequence.blocks) is not tuple
                or len(sequence.blocks) != (sequence.length + BLOCK_TOKENS - 1) // BLOCK_TOKENS
                or not len(sequence.blocks) <= sequence.reservation.maximum_block_credits <= MAX_BLOCKS_PER_REQUEST
            ):
                raise RuntimeError("corrupt KV block table or reservation")
        assigned = [block for sequence in self._sequences.values() for block in sequence.blocks]
        free_list = self._free_blocks
        if free_list or assigned:
            types = set(map(type, chain(free_list, assigned)))
            if types != {int} or min(chain(free_list, assigned)) < 0 or max(chain(free_list, assigned)) >= total:
                raise RuntimeError("invalid physical KV block")
        owned = set(assigned)
        free = set(free_list)
        if len(assigned) != len(owned):
            raise RuntimeError("physical KV blocks must have unique owners")
        if len(free_list) != len(free):
            raise RuntimeError("free KV blocks must be unique")
        if not free.isdisjoint(owned):
            raise RuntimeError("owned KV blocks must not be free")
        if len(free) + len(owned) != total:
            raise RuntimeError("KV blocks must cover the pool")
        owners = {
            block: request_id for request_id, sequence in self._sequences.items() for block in sequence.blocks
        }
        if owners != self._block_owners:
            raise RuntimeError("KV blocks are not owned by the recorded requests")
        return CapacityCounts(
            total_blocks=total,
            free_blocks=len(free_list),
            owned_blocks=len(assigned),
            reserved_blocks=sum(sequence.reservation.maximum_block_credits for sequence in self._sequences.values()),
            active_slots=len(self._sequences),
            live_cached_token_slots=sum(sequence.length for sequence in self._sequences.values()),
        )
