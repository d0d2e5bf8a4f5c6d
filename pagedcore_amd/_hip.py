"""ctypes binding of libpagedcore_hip.so, the C ABI declared in include/pagedcore_hip.h.

The library is loaded after torch, so its libamdhip64.so.7 dependency resolves to the HIP
runtime torch already mapped (same soname): one runtime, and torch's streams and device
pointers are valid in every call. There is no fallback: if the library is missing or
fails to load, every entry point raises HipExtensionError.
"""

from __future__ import annotations

import ctypes
import os
import threading
from typing import Dict, Optional, Tuple

import numpy as np
import torch
from torch import Tensor

ABI_VERSION = 13
LIBRARY_NAME = "libpagedcore_hip.so"

_lock = threading.Lock()
_library: Optional[ctypes.CDLL] = None

_p = ctypes.c_void_p
_i32 = ctypes.c_int32
_i64 = ctypes.c_int64


class HipExtensionError(RuntimeError):
    """The HIP library is missing, failed to load, or rejected a call."""


# Attention workspace header (include/pagedcore_hip.h): the fault word, an int32 at byte 0
# that the kernel ORs these bits into and never clears.
WORKSPACE_HEADER_BYTES = 256
FAULT_MERGE_TIMEOUT = 1
FAULT_FOREIGN_XCD = 2
FAULT_BLOCK_ID = 4
_FAULT_TEXT = (
    (FAULT_MERGE_TIMEOUT, "a cut sequence's part was not flagged within the bounded wait"),
    (FAULT_FOREIGN_XCD, "a cut sequence's part was flagged on another XCD"),
    (FAULT_BLOCK_ID, "a block id outside the pool"),
)


class AttentionFaultError(HipExtensionError):
    """Paged attention failed on the device: the fault word of its workspace is nonzero.

    The rows it names are NaN, and every output computed on that workspace since the word
    was last cleared counts as failed. The workspace has been zeroed (flags and fault word)
    when this is raised, so it can be used again; continuing to serve is the caller's
    decision (DecodeWorker stops)."""

    def __init__(self, faults: int, where: str) -> None:
        text = "; ".join(name for bit, name in _FAULT_TEXT if faults & bit) or "unknown fault"
        super().__init__(f"{where}: paged attention failed on the device (fault word {faults:#x}: {text})")
        self.faults = faults


def fault_word(workspace: Tensor) -> Tensor:
    """The attention workspace's fault word as an int32 [1] view (device memory)."""
    return workspace[:4].view(torch.int32)


def raise_for_faults(faults: int, workspace: Tensor, where: str) -> None:
    """Fail closed on a nonzero fault word read from `workspace`: zero the workspace (a fill
    kernel on the current stream, never under graph capture) and raise AttentionFaultError."""
    if faults:
        workspace.zero_()
        raise AttentionFaultError(int(faults), where)


def check_attention_faults(workspace: Tensor, where: str) -> None:
    """Read the workspace's fault word (synchronizing with the current stream) and fail
    closed if it is nonzero."""
    raise_for_faults(int(fault_word(workspace).item()), workspace, where)


def library_path() -> str:
    return os.path.join(os.path.dirname(os.path.abspath(__file__)), LIBRARY_NAME)


def _declare(lib: ctypes.CDLL) -> None:
    lib.pc_abi_version.restype = ctypes.c_int
    lib.pc_abi_version.argtypes = []
    lib.pc_last_error.restype = ctypes.c_char_p
    lib.pc_last_error.argtypes = []
    lib.pc_attn_workspace_bytes.restype = _i64
    lib.pc_attn_workspace_bytes.argtypes = [_i32, _i32]
    lib.pc_kv_append.restype = ctypes.c_int
    lib.pc_kv_append.argtypes = [_p, _i64, _i32, _i32, _p, _i64, _i64, _p, _i64, _i64, _p, _i64, _p]
    lib.pc_paged_decode_attn.restype = ctypes.c_int
    lib.pc_paged_decode_attn.argtypes = [_p, _p, _p, _i64, _i32, _p, _i32, _i32, _p, _i32, _p, _p]
    lib.pc_kv_append_paged_decode_attn.restype = ctypes.c_int
    lib.pc_kv_append_paged_decode_attn.argtypes = [_p, _p, _p, _i64, _i32, _p, _i32, _i32, _p, _i32, _p, _p, _p, _p]
    lib.pc_paged_decode_attn_noalloc.restype = ctypes.c_int
    lib.pc_paged_decode_attn_noalloc.argtypes = [_p, _p, _p, _i64, _i32, _p, _i32, _i32, _p, _i32, _p]
    lib.pc_attn_plan.restype = _i32
    lib.pc_attn_plan.argtypes = [_p, _p, _i32, _i32, _p, _i64]
    lib.pc_attn_plan_record_ints.restype = _i32
    lib.pc_attn_plan_record_ints.argtypes = []
    lib.pc_attn_plan_capacity.restype = _i64
    lib.pc_attn_plan_capacity.argtypes = [_i32, _i32]
    lib.pc_rope_kv_append.restype = ctypes.c_int
    lib.pc_rope_kv_append.argtypes = [_p, _p, _p, _p, _i64, _p, _p, _i32, _p, _i64, _i32, _p, _i64, _p]
    lib.pc_add_rms_norm.restype = ctypes.c_int
    lib.pc_add_rms_norm.argtypes = [_p, _p, _p, _p, _i64, _i32, ctypes.c_float, _p]
    lib.pc_silu_mul.restype = ctypes.c_int
    lib.pc_silu_mul.argtypes = [_p, _p, _i64, _i32, _p]
    lib.pc_prefill_attention.restype = ctypes.c_int
    lib.pc_prefill_attention.argtypes = [_p, _p, _p, _p, _i32, _p]
    lib.pc_rope_kv_append_parts.restype = ctypes.c_int
    lib.pc_rope_kv_append_parts.argtypes = [_p, _p, _p, _p, _i32, _p, _p, _i32, _p, _i64, _i32, _p, _i64, _p]
    lib.pc_add_rms_norm_parts.restype = ctypes.c_int
    lib.pc_add_rms_norm_parts.argtypes = [_p, _p, _p, _i32, _p, _i64, _i32, ctypes.c_float, _p]
    lib.pc_gemm_m128.restype = ctypes.c_int
    lib.pc_gemm_m128.argtypes = [_p, _p, _p, _i32, _i32, _i32, _i32, _i32, _p]


def load() -> ctypes.CDLL:
    """Load (once) and return the library; raise HipExtensionError if it is unusable."""
    global _library
    if _library is not None:
        return _library
    with _lock:
        if _library is None:
            path = library_path()
            if not os.path.exists(path):
                raise HipExtensionError(
                    f"{path} is not built: run `python -c 'import __graft_entry__ as g; g.build()'`"
                    " (hipcc --offload-arch=gfx950) before using the GPU path"
                )
            try:
                lib = ctypes.CDLL(path)
            except OSError as error:
                raise HipExtensionError(f"cannot load {path}: {error}") from error
            _declare(lib)
            version = lib.pc_abi_version()
            if version != ABI_VERSION:
                raise HipExtensionError(f"{path} has ABI {version}, expected {ABI_VERSION}")
            _library = lib
    return _library


def _check(lib: ctypes.CDLL, name: str, status: int) -> None:
    if status != 0:
        message = lib.pc_last_error().decode(errors="replace")
        raise HipExtensionError(f"{name} failed ({status}): {message}")


_raw_stream = getattr(torch._C, "_cuda_getCurrentRawStream", None)


def current_stream_handle(device: torch.device) -> int:
    """The hipStream_t of the current stream of `device`, as an integer. Uses torch's raw
    accessor when present (no Stream object per call: the decode step asks about 300 times),
    else torch.cuda.current_stream."""
    index = device.index if device.index is not None else torch.cuda.current_device()
    if _raw_stream is not None:
        return int(_raw_stream(index))
    return torch.cuda.current_stream(index).cuda_stream


def _stream(device: torch.device) -> int:
    return current_stream_handle(device)


def kv_append(pool: Tensor, layer_begin: int, key: Tensor, value: Tensor, slot_mapping: Tensor) -> None:
    """pool[layer_begin + l, 0/1, slot // 16, slot % 16] = key/value[l, t] for slot = slot_mapping[t].

    key/value: fp16 [layers, tokens, 4, 64] on the pool's device; layer and token strides
    are free, each [4, 64] row must be contiguous. slot_mapping: int64 [tokens] on the
    device. Enqueued on the current stream of the pool's device.
    """
    lib = load()
    rows = []
    for tensor in (key, value):
        if tensor.stride(3) != 1 or tensor.stride(2) != 64:
            tensor = tensor.contiguous()
        rows.append(tensor)
    key, value = rows
    status = lib.pc_kv_append(
        pool.data_ptr(),
        pool.shape[2],
        layer_begin,
        key.shape[0],
        key.data_ptr(),
        key.stride(0),
        key.stride(1),
        value.data_ptr(),
        value.stride(0),
        value.stride(1),
        slot_mapping.data_ptr(),
        slot_mapping.shape[0],
        _stream(pool.device),
    )
    _check(lib, "pc_kv_append", status)


_workspaces: Dict[Tuple[int, int], Tensor] = {}


def _stream_key(device: torch.device) -> Tuple[int, int]:
    return (device.index if device.index is not None else torch.cuda.current_device(), _stream(device))


def attention_workspace(device: torch.device, nbytes: int) -> Tensor:
    """Split-K partial scratch for the current stream of `device`, grown on demand.

    Zero-initialized: the part flags and the fault word in it must start at zero, and every
    call leaves the flags so (a fault is cleared by raise_for_faults). Reuse is safe because
    every call that uses it is ordered on that one stream.
    """
    key = _stream_key(device)
    workspace = _workspaces.get(key)
    if workspace is None or workspace.numel() < nbytes:
        workspace = torch.zeros(max(nbytes, 256), dtype=torch.uint8, device=device)
        _workspaces[key] = workspace
    return workspace


def workspace_bytes(batch: int, max_blocks: int) -> int:
    return int(load().pc_attn_workspace_bytes(batch, max_blocks))


def plan_capacity(batch: int, max_blocks: int) -> int:
    """Plan rows pc_attn_plan may write for this shape (its pc_attn_plan_capacity)."""
    capacity = int(load().pc_attn_plan_capacity(batch, max_blocks))
    if capacity < 0:
        raise HipExtensionError(f"invalid attention shape batch={batch} max_blocks={max_blocks}")
    return capacity


def decode_plan_into(context_lens: np.ndarray, block_tables: np.ndarray, plan: np.ndarray,
                     clear_to: Optional[int] = None) -> int:
    """pc_attn_plan into the caller's C-contiguous int32 [capacity, row ints] array
    (capacity >= plan_capacity of the shape). Rows past the returned count are made empty
    padding rows up to `clear_to` (default: the whole array); a caller that knows how many
    rows an earlier plan left in the array passes that count, and the whole array is then
    a valid plan of `capacity` rows."""
    lib = load()
    lens = np.ascontiguousarray(context_lens, dtype=np.int32)
    tables = np.ascontiguousarray(block_tables, dtype=np.int32)
    if tables.ndim != 2 or tables.shape[0] != lens.shape[0]:
        raise HipExtensionError("block_tables must be [batch, max_blocks] matching context_lens")
    if plan.dtype != np.int32 or plan.ndim != 2 or plan.shape[1] != int(lib.pc_attn_plan_record_ints()) or not plan.flags.c_contiguous:
        raise HipExtensionError("plan must be a C-contiguous int32 [capacity, record ints] array")
    count = int(lib.pc_attn_plan(lens.ctypes.data, tables.ctypes.data, lens.shape[0], tables.shape[1], plan.ctypes.data, plan.shape[0]))
    if count < 0:
        _check(lib, "pc_attn_plan", -count)
    end = plan.shape[0] if clear_to is None else min(max(clear_to, count), plan.shape[0])
    plan[count:end] = 0
    return count


def decode_plan(context_lens: np.ndarray, block_tables: np.ndarray) -> np.ndarray:
    """Host decode plan: int32 [rows, pc_attn_plan_record_ints()] from pc_attn_plan, built
    from HOST copies of the lengths [batch] and block tables [batch, max_blocks]."""
    lib = load()
    lens = np.ascontiguousarray(context_lens, dtype=np.int32)
    tables = np.ascontiguousarray(block_tables, dtype=np.int32)
    batch = int(lens.shape[0])
    if tables.ndim != 2 or tables.shape[0] != batch:
        raise HipExtensionError("block_tables must be [batch, max_blocks] matching context_lens")
    max_blocks = int(tables.shape[1])
    fields = int(lib.pc_attn_plan_record_ints())
    capacity = int(lib.pc_attn_plan_capacity(batch, max_blocks))
    if capacity < 0:
        _check(lib, "pc_attn_plan_capacity", 1)
    plan = np.empty((max(capacity, 1), fields), dtype=np.int32)
    count = int(lib.pc_attn_plan(lens.ctypes.data, tables.ctypes.data, batch, max_blocks, plan.ctypes.data, capacity))
    if count < 0:
        _check(lib, "pc_attn_plan", -count)
    return plan[:count]


def paged_decode_attention(
    out: Tensor,
    query: Tensor,
    pool: Tensor,
    layer: int,
    block_tables: Tensor,
    context_lens: Tensor,
    *,
    plan: Optional[Tensor] = None,
    workspace: Optional[Tensor] = None,
) -> Tensor:
    """out[b] = paged decode attention of query[b] over layer `layer` of the pool.

    out/query: fp16 [batch, 32, 64] contiguous; block_tables: int32 [batch, max_blocks];
    context_lens: int32 [batch] contiguous. All on the pool's device. `plan`: the
    decode_plan() rows for the same lengths and tables as a contiguous int32 device tensor
    (None: built here from host copies, which synchronizes). `workspace` (uint8, zero before
    its first use; every call leaves its flags so) defaults to the per-stream cached buffer.
    Returns the workspace used, whose fault word (fault_word) the caller checks once it
    synchronizes.
    """
    lib = load()
    batch, max_blocks = block_tables.shape
    nbytes = int(lib.pc_attn_workspace_bytes(batch, max_blocks))
    if nbytes <= 0:
        raise HipExtensionError(f"invalid attention shape batch={batch} max_blocks={max_blocks}")
    if workspace is None:
        workspace = attention_workspace(pool.device, nbytes)
    if plan is None:
        plan = torch.from_numpy(decode_plan(context_lens.cpu().numpy(), block_tables.cpu().numpy())).to(pool.device)
    planned_decode_attention(out, query, pool, layer, context_lens, plan, max_blocks, workspace)
    return workspace


def planned_decode_attention(
    out: Tensor, query: Tensor, pool: Tensor, layer: int, context_lens: Tensor, plan: Tensor, max_blocks: int,
    workspace: Tensor, *, new_key: Optional[Tensor] = None, new_value: Optional[Tensor] = None,
) -> None:
    """pc_paged_decode_attn with a ready device plan (decode_plan() rows, possibly padded
    with empty rows) for a batch of context_lens.shape[0] rows whose tables are at most
    max_blocks wide; workspace of workspace_bytes(batch, max_blocks) bytes, zero before its
    first use (every call leaves its flags so; a device fault sets its fault word, which
    the caller checks: check_attention_faults).

    With new_key and new_value (fp16 [batch, 4, 64] contiguous, the token at position
    context_lens[b] - 1 of each sequence) the call is pc_kv_append_paged_decode_attn: the
    rows are appended to layer `layer` of the pool in the same launch, with the results of
    kv_append followed by attention."""
    lib = load()
    batch = int(context_lens.shape[0])
    nbytes = int(lib.pc_attn_workspace_bytes(batch, max_blocks))
    if nbytes <= 0:
        raise HipExtensionError(f"invalid attention shape batch={batch} max_blocks={max_blocks}")
    if workspace.numel() * workspace.element_size() < nbytes:
        raise HipExtensionError(f"workspace needs {nbytes} bytes")
    if (
        plan.dtype != torch.int32
        or plan.dim() != 2
        or plan.shape[1] != int(lib.pc_attn_plan_record_ints())
        or not plan.is_contiguous()
    ):
        raise HipExtensionError("plan must be a contiguous int32 decode_plan() array")
    args = (out.data_ptr(), query.data_ptr(), pool.data_ptr(), pool.shape[2], layer, context_lens.data_ptr(), batch,
            max_blocks, plan.data_ptr(), int(plan.shape[0]))
    if new_key is None and new_value is None:
        status = lib.pc_paged_decode_attn(*args, workspace.data_ptr(), _stream(pool.device))
        _check(lib, "pc_paged_decode_attn", status)
        return
    for name, rows in (("new_key", new_key), ("new_value", new_value)):
        if (
            rows is None
            or rows.dtype != torch.float16
            or tuple(rows.shape) != (batch, 4, 64)
            or not rows.is_contiguous()
            or rows.device != pool.device
        ):
            raise HipExtensionError(f"{name} must be a contiguous fp16 [{batch}, 4, 64] tensor on the pool's device")
    status = lib.pc_kv_append_paged_decode_attn(
        *args, new_key.data_ptr(), new_value.data_ptr(), workspace.data_ptr(), _stream(pool.device)
    )
    _check(lib, "pc_kv_append_paged_decode_attn", status)


def _ptr(tensor: Optional[Tensor]) -> Optional[int]:
    return None if tensor is None else tensor.data_ptr()


def rope_kv_append(
    query_out: Tensor,
    qkv: Tensor,
    positions: Tensor,
    rope_table: Tensor,
    *,
    key_out: Optional[Tensor] = None,
    value_out: Optional[Tensor] = None,
    pool: Optional[Tensor] = None,
    layer: int = 0,
    slot_mapping: Optional[Tensor] = None,
) -> None:
    """RoPE on each token's query and key; the rotated key and the value optionally go to
    key_out/value_out and to pool[layer, 0/1, slot // 16, slot % 16].

    qkv: fp16 [tokens, >= 2560] with unit column stride (q | k | v columns); positions:
    int64 [tokens]; rope_table: fp16 [positions, 2, 32]; query_out: fp16 [tokens, 32, 64];
    key_out/value_out: fp16 [tokens, 4, 64]; slot_mapping: int64 [tokens]. All contiguous
    except qkv's row stride, on one device; enqueued on its current stream. Positions are
    not read back here: callers check them on the host.
    """
    lib = load()
    if qkv.dim() != 2 or qkv.stride(1) != 1:
        raise HipExtensionError("qkv must be [tokens, columns] with unit column stride")
    status = lib.pc_rope_kv_append(
        query_out.data_ptr(),
        _ptr(key_out),
        _ptr(value_out),
        qkv.data_ptr(),
        qkv.stride(0),
        positions.data_ptr(),
        rope_table.data_ptr(),
        rope_table.shape[0],
        _ptr(pool),
        pool.shape[2] if pool is not None else 0,
        layer,
        _ptr(slot_mapping),
        qkv.shape[0],
        _stream(qkv.device),
    )
    _check(lib, "pc_rope_kv_append", status)


def rope_kv_append_parts(
    query_out: Tensor,
    qkv_parts: Tensor,
    positions: Tensor,
    rope_table: Tensor,
    *,
    key_out: Optional[Tensor] = None,
    value_out: Optional[Tensor] = None,
    pool: Optional[Tensor] = None,
    layer: int = 0,
    slot_mapping: Optional[Tensor] = None,
) -> None:
    """rope_kv_append with the q | k | v row given as split-K partial sums: qkv_parts
    contiguous fp32 [splits, tokens, 2560] (gemm_m128's partials), rounded to fp16 once."""
    lib = load()
    if qkv_parts.dim() != 3 or qkv_parts.dtype != torch.float32 or not qkv_parts.is_contiguous():
        raise HipExtensionError("qkv_parts must be contiguous fp32 [splits, tokens, 2560]")
    status = lib.pc_rope_kv_append_parts(
        query_out.data_ptr(),
        _ptr(key_out),
        _ptr(value_out),
        qkv_parts.data_ptr(),
        qkv_parts.shape[0],
        positions.data_ptr(),
        rope_table.data_ptr(),
        rope_table.shape[0],
        _ptr(pool),
        pool.shape[2] if pool is not None else 0,
        layer,
        _ptr(slot_mapping),
        qkv_parts.shape[1],
        _stream(qkv_parts.device),
    )
    _check(lib, "pc_rope_kv_append_parts", status)


def add_rms_norm_parts(out: Tensor, hidden: Tensor, delta_parts: Tensor, weight: Tensor, eps: float = 1e-5) -> None:
    """add_rms_norm with delta given as split-K partial sums: delta_parts contiguous fp32
    [splits, rows, width]; hidden = fp16(hidden + fp16(sum of the splits))."""
    lib = load()
    if delta_parts.dim() != 3 or delta_parts.shape[1:] != hidden.shape or delta_parts.dtype != torch.float32:
        raise HipExtensionError("delta_parts must be fp32 [splits, rows, width] matching hidden")
    if not delta_parts.is_contiguous():
        raise HipExtensionError("delta_parts must be contiguous")
    status = lib.pc_add_rms_norm_parts(
        out.data_ptr(), hidden.data_ptr(), delta_parts.data_ptr(), delta_parts.shape[0], weight.data_ptr(),
        hidden.shape[0], hidden.shape[1], eps, _stream(hidden.device),
    )
    _check(lib, "pc_add_rms_norm_parts", status)


GEMM_PARTIALS, GEMM_HALF, GEMM_SWIGLU = 0, 1, 2


def gemm_m128(out: Tensor, x: Tensor, w: Tensor, *, splits: int = 1, epilogue: int = GEMM_PARTIALS) -> None:
    """Decode-step projection x @ w.T for up to 128 rows of x (pc_gemm_m128): x fp16 [m, k],
    w fp16 [n, k], both contiguous. out: fp32 [splits, m, n] (GEMM_PARTIALS), fp16 [m, n]
    (GEMM_HALF) or fp16 [m, n // 2] (GEMM_SWIGLU, w the stacked [gate | up] weight)."""
    lib = load()
    m, k = x.shape
    n = w.shape[0]
    expected = {
        GEMM_PARTIALS: ((splits, m, n), torch.float32),
        GEMM_HALF: ((m, n), torch.float16),
        GEMM_SWIGLU: ((m, n // 2), torch.float16),
    }.get(epilogue)
    if expected is None:
        raise HipExtensionError(f"unknown GEMM epilogue {epilogue}")
    if x.dtype != torch.float16 or w.dtype != torch.float16 or w.shape[1] != k:
        raise HipExtensionError("x and w must be fp16 [m, k] and [n, k]")
    if tuple(out.shape) != expected[0] or out.dtype != expected[1]:
        raise HipExtensionError(f"out must be {expected[1]} {list(expected[0])}")
    if not (x.is_contiguous() and w.is_contiguous() and out.is_contiguous()):
        raise HipExtensionError("x, w and out must be contiguous")
    status = lib.pc_gemm_m128(out.data_ptr(), x.data_ptr(), w.data_ptr(), m, n, k, splits, epilogue, _stream(x.device))
    _check(lib, "pc_gemm_m128", status)


def add_rms_norm(out: Tensor, hidden: Tensor, delta: Optional[Tensor], weight: Tensor, eps: float = 1e-5) -> None:
    """hidden += delta (fp16, in place, when delta is given); out = RMSNorm(hidden) * weight.
    hidden/delta/out: contiguous fp16 [rows, width]; weight fp16 [width]."""
    lib = load()
    status = lib.pc_add_rms_norm(
        out.data_ptr(), hidden.data_ptr(), _ptr(delta), weight.data_ptr(), hidden.shape[0], hidden.shape[1], eps,
        _stream(hidden.device),
    )
    _check(lib, "pc_add_rms_norm", status)


def silu_mul(out: Tensor, gate_up: Tensor) -> None:
    """out = fp16(fp16(silu(gate)) * up) for gate_up = [gate | up], contiguous fp16 [rows, 2 * width]."""
    lib = load()
    status = lib.pc_silu_mul(out.data_ptr(), gate_up.data_ptr(), out.shape[0], out.shape[1], _stream(out.device))
    _check(lib, "pc_silu_mul", status)


def prefill_attention(out: Tensor, query: Tensor, key: Tensor, value: Tensor) -> None:
    """Causal attention of one prompt: out/query contiguous fp16 [T, 32, 64], key/value
    contiguous fp16 [T, 4, 64], on one device; enqueued on its current stream."""
    lib = load()
    tokens = int(query.shape[0])
    if (
        query.shape != (tokens, 32, 64)
        or out.shape != query.shape
        or key.shape != (tokens, 4, 64)
        or value.shape != key.shape
        or not all(t.is_contiguous() and t.dtype == torch.float16 for t in (out, query, key, value))
    ):
        raise HipExtensionError("prefill attention needs contiguous fp16 [T, 32, 64] query/out and [T, 4, 64] K/V")
    status = lib.pc_prefill_attention(
        out.data_ptr(), query.data_ptr(), key.data_ptr(), value.data_ptr(), tokens, _stream(query.device)
    )
    _check(lib, "pc_prefill_attention", status)
