"""Batched TinyLlama decode step and paged prefill over the paged KV pool.

Drop-in for the paged callers of the reference decoder: ``decode_paged``
(src/pagedcore/decoder.py:156-199) and ``prefill_paged`` (:113-135) keep their signatures,
argument checks, error types, staged-append semantics and output shapes. The weights
mirror src/pagedcore/weights.py:51-69 field for field.

What changes is the shape of the work. The reference decodes row by row ("single-request
shapes", decoder.py:183) with about twenty tiny launches per row and layer. Here one
decode step is one batch-wide pass per layer:

  x      = RMSNorm(embedding[ids])                           pc_add_rms_norm
  per layer:
    qkv  = x @ [Wq; Wk; Wv]^T                                 GEMM: fp32 split-K partials
    q    = RoPE(q); RoPE(k) and v -> the staged pool slots     pc_rope_kv_append(_parts)
    a    = paged attention(q) over the request's blocks        pc_paged_decode_attn
    h   += a @ Wo^T;  x = RMSNorm(h)                           GEMM partials, pc_add_rms_norm(_parts)
    m    = silu(x @ Wgate^T) * (x @ Wup^T)                     one GEMM on [Wgate; Wup], SwiGLU epilogue
    h   += m @ Wdown^T; x = RMSNorm_next(h)                    GEMM partials, pc_add_rms_norm(_parts)
  logits = x @ Wlm^T                                          GEMM (hipBLASLt via torch)

The projections run on pc_gemm_m128 at up to 128 rows (the split-K partial sums are added
and rounded to fp16 once by the kernel that consumes them) and on F.linear (hipBLASLt)
otherwise, with pc_silu_mul for the SwiGLU. Every elementwise kernel rounds to fp16 where
the reference's torch expression does (see the kernels' comments), so a row's result
differs from the reference only by fp32 summation order inside the GEMMs, the norms and the
attention.
"""

from __future__ import annotations

import weakref
from dataclasses import dataclass
from typing import Callable, Dict, Optional, Sequence, Tuple, TypeVar

import numpy as np
import torch
import torch.nn.functional as F
from torch import Tensor

from pagedcore_amd import _hip
from pagedcore_amd.attention import attend_rows
from pagedcore_amd.engine_types import RequestId
from pagedcore_amd.kv_cache import CONTEXT_LIMIT, HEAD_DIM, KV_HEADS, LAYERS, KVAllocator

T = TypeVar("T")

Q_HEADS = 32
HIDDEN = Q_HEADS * HEAD_DIM  # 2048
KV_WIDTH = KV_HEADS * HEAD_DIM  # 256
QKV_WIDTH = HIDDEN + 2 * KV_WIDTH  # 2560
INTERMEDIATE = 5632
VOCAB = 32000
RMS_EPS = 1e-5
ROPE_THETA = 10000.0


@dataclass(frozen=True, eq=False)
class LayerWeights:
    """One decoder layer's fp16 weights (reference src/pagedcore/weights.py:51-61)."""

    input_norm: Tensor  # [2048]
    q_proj: Tensor  # [2048, 2048]
    k_proj: Tensor  # [256, 2048]
    v_proj: Tensor  # [256, 2048]
    o_proj: Tensor  # [2048, 2048]
    post_attention_norm: Tensor  # [2048]
    gate_proj: Tensor  # [intermediate, 2048]
    up_proj: Tensor  # [intermediate, 2048]
    down_proj: Tensor  # [2048, intermediate]


@dataclass(frozen=True, eq=False)
class TinyLlamaWeights:
    """Embedding, layers, final norm and untied LM head (reference weights.py:64-69)."""

    embedding: Tensor  # [vocab, 2048]
    layers: Tuple[LayerWeights, ...]
    final_norm: Tensor  # [2048]
    lm_head: Tensor  # [vocab, 2048]


# ---------------------------------------------------------------------------------------
# Weights
# ---------------------------------------------------------------------------------------


def _rows_view(parts: Sequence[Tensor]) -> Optional[Tensor]:
    """The [sum of rows, columns] tensor that `parts` already form in memory, if they are
    contiguous row blocks laid end to end in one storage; else None."""
    first = parts[0]
    expected = first.data_ptr()
    for part in parts:
        if (
            part.dim() != 2
            or not part.is_contiguous()
            or part.shape[1] != first.shape[1]
            or part.dtype != first.dtype
            or part.device != first.device
            or part.untyped_storage().data_ptr() != first.untyped_storage().data_ptr()
            or part.data_ptr() != expected
        ):
            return None
        expected += part.numel() * part.element_size()
    rows = sum(part.shape[0] for part in parts)
    return first.new_empty(0).set_(first.untyped_storage(), first.storage_offset(), (rows, first.shape[1]), (first.shape[1], 1))


@dataclass(frozen=True)
class _FusedLayer:
    qkv: Tensor  # [2560, 2048]: q_proj | k_proj | v_proj rows
    gate_up: Tensor  # [2 * intermediate, 2048]: gate_proj | up_proj rows


_fused_cache: "weakref.WeakKeyDictionary[LayerWeights, _FusedLayer]" = weakref.WeakKeyDictionary()


def _fused(layer: LayerWeights) -> _FusedLayer:
    """The layer's stacked projection matrices: views when the weights were allocated
    stacked (random_weights, pack_weights), else one concatenated copy kept per layer."""
    cached = _fused_cache.get(layer)
    if cached is None:
        qkv = _rows_view((layer.q_proj, layer.k_proj, layer.v_proj))
        gate_up = _rows_view((layer.gate_proj, layer.up_proj))
        cached = _FusedLayer(
            qkv if qkv is not None else torch.cat((layer.q_proj, layer.k_proj, layer.v_proj)),
            gate_up if gate_up is not None else torch.cat((layer.gate_proj, layer.up_proj)),
        )
        _fused_cache[layer] = cached
    return cached


def _layer_from_stacks(input_norm, qkv, o_proj, post_norm, gate_up, down_proj) -> LayerWeights:
    intermediate = gate_up.shape[0] // 2
    return LayerWeights(
        input_norm=input_norm,
        q_proj=qkv[:HIDDEN],
        k_proj=qkv[HIDDEN : HIDDEN + KV_WIDTH],
        v_proj=qkv[HIDDEN + KV_WIDTH :],
        o_proj=o_proj,
        post_attention_norm=post_norm,
        gate_proj=gate_up[:intermediate],
        up_proj=gate_up[intermediate:],
        down_proj=down_proj,
    )


def random_weights(
    *,
    device: str | torch.device = "cuda:0",
    seed: int = 0,
    std: float = 0.02,
    norm_std: float = 0.0,
    layers: int = LAYERS,
    vocab: int = VOCAB,
    intermediate: int = INTERMEDIATE,
) -> TinyLlamaWeights:
    """Random-init fp16 TinyLlama-architecture weights: every projection, the embedding and
    the LM head N(0, std); norm weights 1 + N(0, norm_std) (1 exactly by default, as a
    freshly initialised Llama). Projections are allocated stacked (q|k|v, gate|up), so
    the decoder's fused GEMMs use them without a copy."""
    device = torch.device(device)
    gen = torch.Generator(device=device).manual_seed(seed)

    def normal(*shape: int) -> Tensor:
        return torch.empty(shape, dtype=torch.float16, device=device).normal_(0.0, std, generator=gen)

    def norm() -> Tensor:
        weight = torch.ones(HIDDEN, dtype=torch.float16, device=device)
        if norm_std:
            weight.add_(torch.empty_like(weight).normal_(0.0, norm_std, generator=gen))
        return weight

    built = []
    for _ in range(layers):
        built.append(
            _layer_from_stacks(
                norm(), normal(QKV_WIDTH, HIDDEN), normal(HIDDEN, HIDDEN), norm(), normal(2 * intermediate, HIDDEN),
                normal(HIDDEN, intermediate),
            )
        )
    return TinyLlamaWeights(normal(vocab, HIDDEN), tuple(built), norm(), normal(vocab, HIDDEN))


def pack_weights(weights: TinyLlamaWeights) -> TinyLlamaWeights:
    """A copy whose q/k/v and gate/up projections are stacked in memory (for weights loaded
    as separate tensors), so decode runs its fused GEMMs without per-call concatenation."""
    layers = []
    for layer in weights.layers:
        layers.append(
            _layer_from_stacks(
                layer.input_norm,
                torch.cat((layer.q_proj, layer.k_proj, layer.v_proj)),
                layer.o_proj,
                layer.post_attention_norm,
                torch.cat((layer.gate_proj, layer.up_proj)),
                layer.down_proj,
            )
        )
    return TinyLlamaWeights(weights.embedding, tuple(layers), weights.final_norm, weights.lm_head)


# ---------------------------------------------------------------------------------------
# RoPE table
# ---------------------------------------------------------------------------------------

_rope_tables: Dict[torch.device, Tensor] = {}


def rope_table(device: torch.device) -> Tensor:
    """FP16 [2048, 2, 32]: cos, then sin, of position * inv_freq[j] for every position.

    Computed with the reference's own torch expressions (src/pagedcore/dense.py:47-54):
    inv_freq = 1 / 10000^(arange(0, 64, 2) / 64) in fp32, angles = position * inv_freq in
    fp32, cos/sin in fp32 rounded to fp16; the reference's cat((angles, angles)) repeats
    the 32 values, so one copy per position is kept. The table is evaluated on the CPU and
    copied to `device`: the GPU's fp32 pow gives inverse frequencies an ulp away from the
    CPU's for some j, which the late positions (angles up to 2047 rad) amplify enough to
    move fp16-rounded cos/sin entries; the CPU values are the ones the reference's CPU
    tests pin.
    """
    device = torch.device(device)
    table = _rope_tables.get(device)
    if table is None:
        with torch.autocast(device_type="cpu", enabled=False):
            inverse = 1.0 / (ROPE_THETA ** (torch.arange(0, HEAD_DIM, 2).float() / HEAD_DIM))
            angles = torch.arange(CONTEXT_LIMIT).float().unsqueeze(-1) * inverse
            table = torch.stack((angles.cos().half(), angles.sin().half()), dim=1).contiguous().to(device)
        _rope_tables[device] = table
    return table


# ---------------------------------------------------------------------------------------
# Decode
# ---------------------------------------------------------------------------------------


def _check_weights(weights: TinyLlamaWeights, what: str) -> None:
    if len(weights.layers) != LAYERS:
        raise ValueError(f"paged {what} requires 22 decoder layers")


# Decode steps of up to GEMM_M128_ROWS rows run their q|k|v, o_proj, gate|up and down
# projections on pc_gemm_m128: q|k|v, o_proj and down as fp32 split-K partial sums (summed
# and rounded once by the RoPE / residual-add consumers), gate|up with the SwiGLU epilogue.
# Shapes the kernel does not take (more rows, K not a multiple of 64, ...) use F.linear.
# Split counts measured on the batch-128 step: q|k|v at 2 (160 workgroups of 32-row tiles,
# half the partials of 4) 1.930 vs 1.950 ms; o_proj at 2 or 8 and down at 4 or 16 no better.
GEMM_M128_ROWS = 128
QKV_SPLITS = 2
O_PROJ_SPLITS = 4
DOWN_SPLITS = 8


def _linear_parts(x: Tensor, weight: Tensor, preferred_splits: int) -> Tensor:
    """x @ weight.T: fp32 split-K partial sums [splits, rows, n] from pc_gemm_m128 (the most
    splits up to preferred_splits whose K ranges are multiples of 64), or the fp16 product
    [rows, n] of F.linear when the shape does not fit that kernel."""
    rows, k = x.shape
    n = weight.shape[0]
    if rows <= GEMM_M128_ROWS and n % 32 == 0 and x.is_contiguous() and weight.is_contiguous():
        splits = preferred_splits
        while splits >= 1:
            if k % (64 * splits) == 0:
                parts = torch.empty((splits, rows, n), dtype=torch.float32, device=x.device)
                _hip.gemm_m128(parts, x, weight, splits=splits)
                return parts
            splits //= 2
    return F.linear(x, weight)


def _swiglu(x: Tensor, gate_up: Tensor) -> Tensor:
    """fp16(fp16(silu(x @ gate.T)) * fp16(x @ up.T)) for the stacked [gate | up] weight:
    one pc_gemm_m128 launch with the SwiGLU epilogue, or F.linear + pc_silu_mul."""
    rows, k = x.shape
    n = gate_up.shape[0]
    activated = torch.empty((rows, n // 2), dtype=torch.float16, device=x.device)
    if rows <= GEMM_M128_ROWS and n % 64 == 0 and k % 64 == 0 and x.is_contiguous() and gate_up.is_contiguous():
        _hip.gemm_m128(activated, x, gate_up, epilogue=_hip.GEMM_SWIGLU)
    else:
        _hip.silu_mul(activated, F.linear(x, gate_up))
    return activated


def _add_rms_norm(x: Tensor, hidden: Tensor, delta: Tensor, weight: Tensor) -> None:
    """hidden += delta; x = RMSNorm(hidden) * weight, for an fp16 delta or fp32 partial sums."""
    if delta.ndim == 3:
        _hip.add_rms_norm_parts(x, hidden, delta, weight, RMS_EPS)
    else:
        _hip.add_rms_norm(x, hidden, delta, weight, RMS_EPS)


def _attention_block(
    x: Tensor, hidden: Tensor, layer: LayerWeights, fused: _FusedLayer, following_norm: Tensor, attend
) -> None:
    """One decoder layer around its attention, in place on (x, hidden): q|k|v projection,
    attend(qkv) -> attention [rows, 2048] (RoPE, KV write and paged attention, supplied by
    the caller; qkv fp16 [rows, 2560] or fp32 partial sums [splits, rows, 2560]), o_proj +
    residual + RMSNorm, SwiGLU MLP + residual + the next RMSNorm (reference
    src/pagedcore/decoder.py:173-193)."""
    attention = attend(_linear_parts(x, fused.qkv, QKV_SPLITS))
    _add_rms_norm(x, hidden, _linear_parts(attention, layer.o_proj, O_PROJ_SPLITS), layer.post_attention_norm)
    activated = _swiglu(x, fused.gate_up)
    _add_rms_norm(x, hidden, _linear_parts(activated, layer.down_proj, DOWN_SPLITS), following_norm)


def _check_gpu(allocator: KVAllocator, weights: TinyLlamaWeights, what: str) -> None:
    """The kernels run on the GPU only: fail before any staging when the pool or the
    weights live elsewhere (there is no CPU fallback)."""
    if not allocator.pool.is_cuda or weights.embedding.device != allocator.pool.device:
        raise RuntimeError(f"paged {what} runs on the GPU: the KV pool and the weights must share a CUDA device")


@torch.inference_mode()
def decode_paged(
    input_ids: Tensor,
    weights: TinyLlamaWeights,
    allocator: KVAllocator,
    request_ids: Tuple[RequestId, ...],
) -> Tensor:
    """One greedy-decode step for a batch: input_ids int64 [B, 1] (row b: the new token of
    request_ids[b], at position = its cached length); returns fp16 logits [B, 1, vocab].

    Each request gains one cached position on success; on any exception the staged step
    is discarded and no request changes (reference src/pagedcore/decoder.py:156-199). A
    device-side attention failure counts as one: the step reads the attention workspaces'
    fault words before it commits (one synchronization per step) and raises
    AttentionFaultError instead of returning logits computed from NaN rows.
    """
    request_ids = tuple(request_ids)
    if input_ids.dtype != torch.int64 or input_ids.ndim != 2 or input_ids.shape != (len(request_ids), 1):
        raise ValueError("input_ids must be int64 [batch, 1] matching request IDs")
    if input_ids.device != weights.embedding.device:
        raise ValueError("input_ids and weights must be on the same device")
    _check_weights(weights, "decode")
    allocator.cached_lengths(request_ids)  # KeyError for an unknown request, as the reference
    _check_gpu(allocator, weights, "decode")
    with allocator.append_decode(request_ids):
        table = rope_table(allocator.pool.device)
        hidden = F.embedding(input_ids[:, 0], weights.embedding)  # [B, 2048]
        x = torch.empty_like(hidden)
        _hip.add_rms_norm(x, hidden, None, weights.layers[0].input_norm, RMS_EPS)
        batch = len(request_ids)
        workspaces: Dict[int, Tensor] = {}
        for index, layer in enumerate(weights.layers):

            def attend(qkv: Tensor, index: int = index) -> Tensor:
                query = allocator.write_decode_layers_rotary(request_ids, index, qkv, table)
                out, workspace = attend_rows(query, allocator, request_ids, index)
                workspaces[workspace.data_ptr()] = workspace
                return out.view(batch, HIDDEN)

            following = weights.layers[index + 1].input_norm if index + 1 < LAYERS else weights.final_norm
            _attention_block(x, hidden, layer, _fused(layer), following, attend)
        logits = F.linear(x, weights.lm_head)
        for workspace in workspaces.values():
            _hip.check_attention_faults(workspace, "decode_paged")
    return logits.unsqueeze(1)


# ---------------------------------------------------------------------------------------
# Decode as one replayed HIP graph
# ---------------------------------------------------------------------------------------

MAX_BLOCKS = CONTEXT_LIMIT // 16  # 128: the widest block table of a request


def capture_graph(fn: Callable[[], T], device: torch.device) -> Tuple[torch.cuda.CUDAGraph, T]:
    """Capture fn()'s launches as a HIP graph on a side stream; returns the graph and fn()'s
    result (its tensors are the graph's static outputs). The current stream is synchronized
    before and after.

    Unlike the torch.cuda.graph context manager this leaves torch's allocator cache alone:
    that manager empties the cache, returning every cached block to the driver, and in the
    seconds after such a release bandwidth-bound kernels of the process run slower
    (measured: the batch-128 decode step at 1.98 ms instead of 1.93 ms when its capture
    released 29 GB another workload had cached, and at 1.92 ms again after 10 idle seconds).
    """
    stream = torch.cuda.current_stream(device)
    torch.cuda.synchronize(device)
    side = torch.cuda.Stream(device=device)
    side.wait_stream(stream)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.stream(side):
        graph.capture_begin()
        try:
            result = fn()
        except BaseException:
            try:
                graph.capture_end()
            except RuntimeError:
                pass  # the capture is abandoned; fn's error is the one to report
            raise
        graph.capture_end()
    stream.wait_stream(side)
    torch.cuda.synchronize(device)
    return graph, result


class DecodeGraph:
    """decode_paged for batches of up to a fixed size, captured once as a HIP graph and replayed.

    A decode step is about 200 launches (9 per layer); issued one by one from Python they
    cost more host time than the GPU needs to run them. Here the step's device work is
    captured once, with every per-step input in static device buffers: token ids, the
    staged token's slot and position of each row, the staged context lengths, and the
    decode plan at its full capacity (pc_attn_plan_capacity rows for the batch and
    128-block tables; the attention kernel launches one workgroup per row and empty rows
    exit at once). Per step the host does the allocator's staged-append bookkeeping, builds
    the plan into a pinned buffer, uploads the rows in use (and the empty rows that replace
    a longer previous plan) with two asynchronous copies and replays the graph; nothing
    synchronizes. step() takes the token ids from the device and returns a copy of the
    logits; greedy() takes them from the host, in the first of the two copies, and returns
    only each row's argmax (what a greedy loop reads back).

    Device faults fail closed. After each replay the attention workspace's fault word is
    copied to pinned memory. check_faults() raises AttentionFaultError if the last step's
    attention failed on the device (call it after reading the step's logits, as
    DecodeWorker does), and every step first waits for the step two before it and raises
    if that step failed, before staging anything. On a raise the workspace is zeroed.

    Same checks, errors and staged-append semantics as decode_paged for any 1 to `batch`
    requests (any requests, in any order, step to step). A batch of exactly `batch`
    requests runs the kernels decode_paged runs, at the same shapes, so its logits and
    cache bytes equal decode_paged's. A smaller batch is padded to `batch` rows: a padding
    row has no slot (it writes nothing to the pool) and context length 0 (no attention
    work, its output row is never written), and its logits are dropped. The GEMMs then run
    at `batch` rows, so the real rows' results may differ from decode_paged's at the
    smaller row count in the last bits, as between any two GEMM shapes.
    """

    def __init__(self, weights: TinyLlamaWeights, allocator: KVAllocator, batch: int) -> None:
        _check_weights(weights, "decode")
        if type(batch) is not int or batch < 1:
            raise ValueError("batch must be a positive integer")
        _check_gpu(allocator, weights, "decode")
        device = allocator.pool.device
        self.batch = batch
        self._weights = weights
        self._allocator = allocator
        self._table = rope_table(device)
        fields = int(_hip.load().pc_attn_plan_record_ints())
        self._capacity = _hip.plan_capacity(batch, MAX_BLOCKS)
        # Static graph inputs: int64 [3, B] = token ids, slots, positions; int32
        # [lens_span + capacity * fields] = context lengths (padded to 256 B, which keeps
        # the plan records aligned), then the plan records.
        self._lens_span = (batch + 63) // 64 * 64
        self._inputs64 = torch.zeros((3, batch), dtype=torch.int64, device=device)
        self._inputs64[1].fill_(-1)  # no slot: warm-up and capture write nothing to the pool
        self._inputs32 = torch.zeros(self._lens_span + self._capacity * fields, dtype=torch.int32, device=device)
        self._lens = self._inputs32[:batch]
        self._plan = self._inputs32[self._lens_span :].view(self._capacity, fields)
        self._fields = fields
        self._workspace = torch.zeros(max(256, _hip.workspace_bytes(batch, MAX_BLOCKS)), dtype=torch.uint8, device=device)
        # Two pinned staging buffers used in turn, each with a pinned copy of the fault word
        # after its step; an event marks when that step has finished, so a buffer is not
        # refilled while its upload may still be pending and its fault copy is complete.
        self._host = [
            (
                torch.empty((3, batch), dtype=torch.int64, pin_memory=True),
                torch.zeros(self._lens_span + self._capacity * fields, dtype=torch.int32, pin_memory=True),
            )
            for _ in range(2)
        ]
        self._fault_host = [torch.zeros(1, dtype=torch.int32, pin_memory=True) for _ in range(2)]
        self._finished: list = [None, None]
        self._last_turn: Optional[int] = None
        self._host_rows = [0, 0]  # plan rows a pinned buffer may hold non-empty
        self._device_rows = 0  # plan rows the device buffer may hold non-empty
        self._turn = 0

        self._forward()  # eager warm-up: library initialisation and GEMM selection happen outside the capture
        self._graph, self._logits = capture_graph(self._forward, device)

    def _forward(self) -> Tensor:
        """The step's device work over the static inputs (eager, or under capture)."""
        weights = self._weights
        pool = self._allocator.pool
        batch = self.batch
        ids, slots, positions = self._inputs64
        hidden = F.embedding(ids, weights.embedding)
        x = torch.empty_like(hidden)
        _hip.add_rms_norm(x, hidden, None, weights.layers[0].input_norm, RMS_EPS)
        query = torch.empty((batch, Q_HEADS, HEAD_DIM), dtype=torch.float16, device=pool.device)
        attention = torch.empty_like(query)
        for index, layer in enumerate(weights.layers):

            def attend(qkv: Tensor, index: int = index) -> Tensor:
                if qkv.ndim == 3:
                    _hip.rope_kv_append_parts(query, qkv, positions, self._table, pool=pool, layer=index, slot_mapping=slots)
                else:
                    _hip.rope_kv_append(query, qkv, positions, self._table, pool=pool, layer=index, slot_mapping=slots)
                _hip.planned_decode_attention(attention, query, pool, index, self._lens, self._plan, MAX_BLOCKS, self._workspace)
                return attention.view(batch, HIDDEN)

            following = weights.layers[index + 1].input_norm if index + 1 < LAYERS else weights.final_norm
            _attention_block(x, hidden, layer, _fused(layer), following, attend)
        return F.linear(x, weights.lm_head)

    def _take_faults(self, turn: int) -> None:
        """Wait for the step that last used staging buffer `turn` and fail closed if its copy
        of the workspace's fault word is nonzero (each copy is checked once)."""
        finished = self._finished[turn]
        if finished is None:
            return
        finished.synchronize()
        self._finished[turn] = None
        _hip.raise_for_faults(int(self._fault_host[turn][0]), self._workspace, "DecodeGraph.step")

    def check_faults(self) -> None:
        """Raise AttentionFaultError if the last step's attention failed on the device. Waits
        for that step (a caller that already read its logits has waited for it)."""
        if self._last_turn is not None:
            self._take_faults(self._last_turn)

    @torch.inference_mode()
    def step(self, input_ids: Tensor, request_ids: Tuple[RequestId, ...]) -> Tensor:
        """decode_paged(input_ids, weights, allocator, request_ids) by graph replay, for 1 to
        `batch` requests. Returns fresh fp16 logits [len(request_ids), 1, vocab]; the caller
        checks them with check_faults() once it has synchronized."""
        request_ids = tuple(request_ids)
        if input_ids.dtype != torch.int64 or input_ids.ndim != 2 or input_ids.shape != (len(request_ids), 1):
            raise ValueError("input_ids must be int64 [batch, 1] matching request IDs")
        if input_ids.device != self._weights.embedding.device:
            raise ValueError("input_ids and weights must be on the same device")
        rows = self._replay(request_ids, None, input_ids[:, 0], None)
        return self._logits[:rows].clone().unsqueeze(1)

    @torch.inference_mode()
    def greedy(
        self, token_ids: np.ndarray, request_ids: Tuple[RequestId, ...], device_token: Optional[Tuple[int, Tensor]] = None
    ) -> Tensor:
        """The same step for a greedy caller: the input ids come from the host (int64
        [len(request_ids)], each below the vocabulary size), uploaded with the slots and
        positions in one copy, except that `device_token` = (row, 0-dim int64 device
        tensor) supplies row's id from device memory. Returns int64 [len(request_ids)] on
        the device: the argmax of each row's logits, computed from the graph's own logits
        buffer (no copy of the logits); check_faults() as for step()."""
        request_ids = tuple(request_ids)
        ids = np.asarray(token_ids)
        if ids.dtype != np.int64 or ids.shape != (len(request_ids),):
            raise ValueError("token_ids must be int64 [batch] matching request IDs")
        if ids.size and (int(ids.min()) < 0 or int(ids.max()) >= self._weights.embedding.shape[0]):
            raise ValueError("token ids must be below the vocabulary size")
        if device_token is not None:
            row, token = device_token
            if type(row) is not int or not 0 <= row < len(request_ids):
                raise ValueError("device_token row outside the batch")
            if token.dtype != torch.int64 or token.numel() != 1 or token.device != self._weights.embedding.device:
                raise ValueError("device_token must be one int64 id on the weights' device")
        rows = self._replay(request_ids, ids, None, device_token)
        return self._logits[:rows].argmax(-1)

    def _replay(
        self,
        request_ids: Tuple[RequestId, ...],
        host_ids: Optional[np.ndarray],
        device_ids: Optional[Tensor],
        device_token: Optional[Tuple[int, Tensor]],
    ) -> int:
        """Stage the step (allocator bookkeeping, pinned inputs, the plan) and replay the
        graph; the ids come from `host_ids` (then `device_token` may replace one) or from
        the device vector `device_ids`. Returns the number of real rows."""
        rows = len(request_ids)
        if not 1 <= rows <= self.batch:
            raise ValueError(f"this decode graph runs batches of 1 to {self.batch} requests")
        allocator = self._allocator
        allocator.cached_lengths(request_ids)  # KeyError for an unknown request
        with allocator.append_decode(request_ids):
            staged = allocator.staged_decode(request_ids, width=MAX_BLOCKS)
            turn = self._turn
            self._take_faults(turn)
            self._turn ^= 1
            host64, host32 = self._host[turn]
            h64 = host64.numpy()
            h32 = host32.numpy()
            if host_ids is not None:
                h64[0, :rows] = host_ids
                h64[0, rows:] = 0  # padding rows: a valid id, whose logits are dropped
            h64[1, :rows] = staged.slots
            h64[1, rows:] = -1  # padding rows: no slot, position 0, context length 0
            h64[2, :rows] = staged.positions
            h64[2, rows:] = 0
            h32[:rows] = staged.lengths
            h32[rows : self.batch] = 0
            count = _hip.decode_plan_into(
                staged.lengths, staged.tables, h32[self._lens_span :].reshape(self._capacity, -1), self._host_rows[turn]
            )
            self._host_rows[turn] = count
            upload = self._lens_span + max(count, self._device_rows) * self._fields
            self._device_rows = count
            if host_ids is not None:
                self._inputs64.copy_(host64, non_blocking=True)
                if device_token is not None:
                    self._inputs64[0, device_token[0]].copy_(device_token[1].reshape(()))
            else:
                self._inputs64[1:].copy_(host64[1:], non_blocking=True)
                self._inputs64[0, :rows].copy_(device_ids)
            self._inputs32[:upload].copy_(host32[:upload], non_blocking=True)
            self._graph.replay()
            self._fault_host[turn].copy_(_hip.fault_word(self._workspace), non_blocking=True)
            finished = torch.cuda.Event()
            finished.record()
            self._finished[turn] = finished
            self._last_turn = turn
            allocator.record_decode_writes(request_ids, LAYERS)
        return rows


# ---------------------------------------------------------------------------------------
# Prefill
# ---------------------------------------------------------------------------------------


@torch.inference_mode()
def prefill_paged(
    input_ids: Tensor,
    weights: TinyLlamaWeights,
    allocator: KVAllocator,
    request_id: RequestId,
) -> Tensor:
    """Prefill one admitted, empty request from int64 [1, T] prompt ids; returns fp16
    logits [1, T, vocab]. Only K is rotated (reference src/pagedcore/decoder.py:113-135).

    The K/V write is fused into the forward: per layer, pc_rope_kv_append rotates Q and K
    and writes the rotated K and the V straight into the slots the append takes (staged
    through KVAllocator.append_prompt), besides the contiguous copy the prompt's attention
    reads. The append is published only after the whole forward succeeded, as the
    reference publishes its one append after the forward.
    """
    if allocator.cached_length(request_id) != 0:
        raise ValueError("paged prefill requires an empty request cache")
    _check_weights(weights, "prefill")
    if input_ids.dtype != torch.int64 or input_ids.ndim != 2 or input_ids.shape[0] != 1:
        raise ValueError("input_ids must be int64 [1, tokens]")
    if input_ids.device != weights.embedding.device:
        raise ValueError("input_ids and weights must be on the same device")
    tokens = input_ids.shape[1]
    if tokens < 1 or tokens > CONTEXT_LIMIT:
        raise ValueError("forward requires 1 to 2048 total cached token positions")
    _check_gpu(allocator, weights, "prefill")
    table = rope_table(input_ids.device)
    with allocator.append_prompt(request_id, tokens) as staged:
        x = _prefill_forward(input_ids[0], staged.positions, staged.slot_mapping, weights, allocator.pool, table,
                             staged.record_layer)
        logits = F.linear(x, weights.lm_head)
    return logits.unsqueeze(0)


def _prefill_forward(ids: Tensor, positions: Tensor, slots: Tensor, weights: TinyLlamaWeights, pool: Tensor,
                     table: Tensor, on_layer=None) -> Tensor:
    """The prompt's forward over T = len(ids) rows: per layer, pc_rope_kv_append writes the
    rotated K and the V to `slots` (negative: not written) and to the contiguous copies
    the prompt's attention reads; returns the final-normed hidden states [T, 2048].
    `on_layer(index)` runs after each layer's cache write is enqueued."""
    tokens = ids.shape[0]
    device = ids.device
    hidden = F.embedding(ids, weights.embedding)  # [T, 2048]
    x = torch.empty_like(hidden)
    _hip.add_rms_norm(x, hidden, None, weights.layers[0].input_norm, RMS_EPS)
    key = torch.empty((tokens, KV_HEADS, HEAD_DIM), dtype=torch.float16, device=device)
    value = torch.empty_like(key)
    query = torch.empty((tokens, Q_HEADS, HEAD_DIM), dtype=torch.float16, device=device)
    attended = torch.empty_like(query)
    for index, layer in enumerate(weights.layers):
        fused = _fused(layer)
        qkv = F.linear(x, fused.qkv)
        _hip.rope_kv_append(query, qkv, positions, table, key_out=key, value_out=value, pool=pool, layer=index,
                            slot_mapping=slots)
        if on_layer is not None:
            on_layer(index)
        _hip.prefill_attention(attended, query, key, value)
        projected = F.linear(attended.view(tokens, HIDDEN), layer.o_proj)
        _hip.add_rms_norm(x, hidden, projected, layer.post_attention_norm, RMS_EPS)
        gate_up = F.linear(x, fused.gate_up)
        activated = torch.empty((tokens, gate_up.shape[1] // 2), dtype=torch.float16, device=device)
        _hip.silu_mul(activated, gate_up)
        down = F.linear(activated, layer.down_proj)
        following = weights.layers[index + 1].input_norm if index + 1 < LAYERS else weights.final_norm
        _hip.add_rms_norm(x, hidden, down, following, RMS_EPS)
    return x


class PrefillGraph:
    """prefill_paged for prompts of 1 to `tokens` positions, captured once as a HIP graph
    and replayed, returning only the logits of the prompt's last position (what greedy
    generation selects from).

    prefill_paged issues about 200 launches from Python (about 2.6 ms of host time at any
    prompt length), so short prompts are host-bound. Here the forward is captured at
    `tokens` rows over static inputs: token ids, slot mapping and the index of the last
    real row (positions are 0 .. tokens - 1: the cache is empty). A shorter prompt is
    padded at the end; causal attention keeps every real row blind to the padding rows
    after it, and a padding row's slot is -1, so it writes nothing to the pool. Per call
    the host stages the append (KVAllocator.append_prompt, same checks, errors and
    publish-after-forward semantics as prefill_paged), uploads the inputs into the static
    buffers with one copy from pinned memory (the ids from the device for step(), from the
    host, in the same copy, for greedy()) and replays the graph; nothing synchronizes.

    The GEMMs run at `tokens` rows, and the LM head on the last row alone, so logits and
    cache bytes may differ from prefill_paged's in the last bits, as between any two GEMM
    shapes.
    """

    def __init__(self, weights: TinyLlamaWeights, allocator: KVAllocator, tokens: int) -> None:
        _check_weights(weights, "prefill")
        if type(tokens) is not int or not 1 <= tokens <= CONTEXT_LIMIT:
            raise ValueError("a prefill graph holds 1 to 2048 prompt positions")
        _check_gpu(allocator, weights, "prefill")
        device = allocator.pool.device
        self.tokens = tokens
        self._weights = weights
        self._allocator = allocator
        self._table = rope_table(device)
        # Static inputs: int64 [4, tokens] = token ids, slots, positions, and (row 3,
        # element 0) the last real row's index.
        self._inputs = torch.zeros((4, tokens), dtype=torch.int64, device=device)
        self._inputs[1].fill_(-1)  # warm-up and capture write nothing to the pool
        self._inputs[2].copy_(torch.arange(tokens, device=device))
        self._inputs[3, 0] = tokens - 1
        # Two pinned staging buffers of the same layout used in turn; an event recorded
        # after a buffer's upload marks when it may be refilled.
        self._host = [self._inputs.cpu().pin_memory() for _ in range(2)]
        self._uploaded: list = [None, None]
        self._turn = 0
        self._forward()  # eager warm-up: library initialisation and GEMM selection outside the capture
        self._graph, self._logits = capture_graph(self._forward, device)

    def _forward(self) -> Tensor:
        ids, slots, positions, last = self._inputs
        x = _prefill_forward(ids, positions, slots, self._weights, self._allocator.pool, self._table)
        return F.linear(x.index_select(0, last[:1]), self._weights.lm_head)  # [1, vocab]

    def _check_empty(self, request_id: RequestId) -> None:
        if self._allocator.cached_length(request_id) != 0:
            raise ValueError("paged prefill requires an empty request cache")

    def _check_rows(self, rows: int) -> None:
        if not 1 <= rows <= self.tokens:
            raise ValueError(f"this prefill graph holds prompts of 1 to {self.tokens} positions")

    def _replay(self, request_id: RequestId, rows: int, host_ids: Optional[np.ndarray],
                device_ids: Optional[Tensor]) -> None:
        """Stage the append, upload the slots (and the host ids, when given) with the last
        row's index in one copy from a pinned buffer, and replay the graph."""
        with self._allocator.append_prompt(request_id, rows) as staged:
            turn = self._turn
            self._turn ^= 1
            if self._uploaded[turn] is not None:
                self._uploaded[turn].synchronize()  # its previous upload has run
            host = self._host[turn].numpy()
            if host_ids is not None:
                host[0, :rows] = host_ids  # rows past the prompt keep earlier valid ids
            host[1, :rows] = staged.slots
            host[1, rows:] = -1  # padding rows write nothing to the pool
            host[3, 0] = rows - 1
            if host_ids is not None:
                self._inputs.copy_(self._host[turn], non_blocking=True)
            else:
                self._inputs[1:].copy_(self._host[turn][1:], non_blocking=True)
                self._inputs[0, :rows].copy_(device_ids)
            uploaded = torch.cuda.Event()
            uploaded.record()
            self._uploaded[turn] = uploaded
            self._graph.replay()
            for index in range(LAYERS):
                staged.record_layer(index)

    @torch.inference_mode()
    def step(self, input_ids: Tensor, request_id: RequestId) -> Tensor:
        """prefill_paged(input_ids, weights, allocator, request_id) by graph replay for a
        prompt of 1 to `tokens` positions; returns fresh fp16 logits [1, 1, vocab] of the
        prompt's last position."""
        self._check_empty(request_id)
        if input_ids.dtype != torch.int64 or input_ids.ndim != 2 or input_ids.shape[0] != 1:
            raise ValueError("input_ids must be int64 [1, tokens]")
        if input_ids.device != self._weights.embedding.device:
            raise ValueError("input_ids and weights must be on the same device")
        rows = input_ids.shape[1]
        self._check_rows(rows)
        self._replay(request_id, rows, None, input_ids[0])
        return self._logits.clone().unsqueeze(0)

    @torch.inference_mode()
    def greedy(self, prompt_ids: np.ndarray, request_id: RequestId) -> Tensor:
        """The same prefill for a greedy caller, from host token ids (int64 [tokens], each
        below the vocabulary size) uploaded with the slots in one copy. Returns the argmax
        of the last position's logits as a 0-dim int64 device tensor (the greedy first
        token), computed from the graph's own logits buffer."""
        self._check_empty(request_id)
        ids = np.asarray(prompt_ids)
        if ids.dtype != np.int64 or ids.ndim != 1:
            raise ValueError("prompt_ids must be int64 [tokens]")
        rows = ids.shape[0]
        self._check_rows(rows)
        if int(ids.min()) < 0 or int(ids.max()) >= self._weights.embedding.shape[0]:
            raise ValueError("token ids must be below the vocabulary size")
        self._replay(request_id, rows, ids, None)
        return self._logits[0].argmax()
