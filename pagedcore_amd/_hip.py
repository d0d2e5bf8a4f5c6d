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

import torch
from torch import Tensor

ABI_VERSION = 1
LIBRARY_NAME = "libpagedcore_hip.so"

_lock = threading.Lock()
_library: Optional[ctypes.CDLL] = None

_p = ctypes.c_void_p
_i32 = ctypes.c_int32
_i64 = ctypes.c_int64


class HipExtensionError(RuntimeError):
    """The HIP library is missing, failed to load, or rejected a call."""


def library_path() -> str:
    return os.path.join(os.path.dirname(os.path.abspath(__file__)), LIBRARY_NAME)


def _declare(lib: ctypes.CDLL) -> None:
    lib.pc_abi_version.restype = ctypes.c_int
    lib.pc_abi_version.argtypes = []
    lib.pc_last_error.restype = ctypes.c_char_p
    lib.pc_last_error.argtypes = []
    lib.pc_attn_default_partition_blocks.restype = _i32
    lib.pc_attn_default_partition_blocks.argtypes = []
    lib.pc_attn_workspace_floats.restype = _i64
    lib.pc_attn_workspace_floats.argtypes = [_i32, _i32, _i32]
    lib.pc_kv_append.restype = ctypes.c_int
    lib.pc_kv_append.argtypes = [_p, _i64, _i32, _i32, _p, _i64, _i64, _p, _i64, _i64, _p, _i64, _p]
    attn = [_p, _p, _p, _i64, _i32, _p, _i32, _p, _i32, _i32, _p, _p, _p]
    for name in ("pc_paged_decode_attn", "pc_paged_decode_attn_partitions"):
        fn = getattr(lib, name)
        fn.restype = ctypes.c_int
        fn.argtypes = attn
    lib.pc_paged_decode_attn_reduce.restype = ctypes.c_int
    lib.pc_paged_decode_attn_reduce.argtypes = [_p, _p, _i32, _i32, _i32, _p, _p, _p]


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


def _stream(device: torch.device) -> int:
    return torch.cuda.current_stream(device).cuda_stream


def default_partition_blocks() -> int:
    return int(load().pc_attn_default_partition_blocks())


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


def attention_workspace(device: torch.device, floats: int) -> Tensor:
    """Split-K scratch for the current stream of `device`, grown on demand and reused.

    Reuse is safe because every call that uses it is ordered on that one stream.
    """
    key = (device.index if device.index is not None else torch.cuda.current_device(), _stream(device))
    workspace = _workspaces.get(key)
    if workspace is None or workspace.numel() < floats:
        workspace = torch.empty(max(floats, 1), dtype=torch.float32, device=device)
        _workspaces[key] = workspace
    return workspace


def paged_decode_attention(
    out: Tensor,
    query: Tensor,
    pool: Tensor,
    layer: int,
    block_tables: Tensor,
    context_lens: Tensor,
    *,
    partition_blocks: Optional[int] = None,
    workspace: Optional[Tensor] = None,
) -> None:
    """out[b] = paged decode attention of query[b] over layer `layer` of the pool.

    out/query: fp16 [batch, 32, 64] contiguous; block_tables: int32 [batch, max_blocks]
    contiguous; context_lens: int32 [batch]. All on the pool's device.
    """
    lib = load()
    batch, max_blocks = block_tables.shape
    parts = partition_blocks if partition_blocks is not None else default_partition_blocks()
    floats = int(lib.pc_attn_workspace_floats(batch, max_blocks, parts))
    if floats <= 0:
        raise HipExtensionError(f"invalid attention shape batch={batch} max_blocks={max_blocks} partition={parts}")
    if workspace is None:
        workspace = attention_workspace(pool.device, floats)
    elif workspace.numel() < floats or workspace.dtype != torch.float32:
        raise HipExtensionError(f"workspace needs {floats} fp32 elements")
    max_parts = (max_blocks + parts - 1) // parts
    ws_out = workspace.data_ptr()
    ws_ml = ws_out + batch * 32 * max_parts * 64 * 4
    status = lib.pc_paged_decode_attn(
        out.data_ptr(),
        query.data_ptr(),
        pool.data_ptr(),
        pool.shape[2],
        layer,
        block_tables.data_ptr(),
        max_blocks,
        context_lens.data_ptr(),
        batch,
        parts,
        ws_out,
        ws_ml,
        _stream(pool.device),
    )
    _check(lib, "pc_paged_decode_attn", status)
