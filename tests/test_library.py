"""The C-ABI library: loads without a GPU, exports every symbol include/pagedcore_hip.h
declares, and rejects invalid arguments before anything would be launched."""

from __future__ import annotations

import ctypes
import os
import re

import pytest

from pagedcore_amd import _hip

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _declared_symbols() -> list[str]:
    with open(os.path.join(ROOT, "include", "pagedcore_hip.h")) as handle:
        text = handle.read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(pc_[a-z0-9_]+)\s*\(", text)))


def test_library_exports_every_declared_symbol():
    lib = _hip.load()
    names = _declared_symbols()
    assert "pc_kv_append" in names and "pc_paged_decode_attn" in names
    for name in names:
        assert hasattr(lib, name), name
    assert lib.pc_abi_version() == _hip.ABI_VERSION


def test_workspace_size_formula():
    lib = _hip.load()
    # 64 sequences x 32 heads x ceil(128/32) partitions x (64 outputs + max + sum)
    assert lib.pc_attn_workspace_floats(64, 128, 32) == 64 * 32 * 4 * 66
    assert lib.pc_attn_workspace_floats(1, 8, 4) == 32 * 2 * 66
    assert lib.pc_attn_workspace_floats(1, 8, 6) == 0  # partition size must be a multiple of 4


@pytest.mark.parametrize(
    "args,needle",
    [
        ((None, 1, 0, 1, None, 0, 0, None, 0, 0, None, 1, None), b"null pointer"),
        ((16, 0, 0, 1, 16, 0, 0, 16, 0, 0, 16, 1, None), b"num_blocks"),
        ((16, 4, 21, 2, 16, 0, 0, 16, 0, 0, 16, 1, None), b"layers"),
        ((16, 4, 0, 1, 16, 0, 0, 16, 0, 0, 16, -1, None), b"negative"),
        ((8, 4, 0, 1, 16, 0, 0, 16, 0, 0, 16, 1, None), b"aligned"),
    ],
)
def test_append_rejects_invalid_arguments_without_a_gpu(args, needle):
    lib = _hip.load()
    assert lib.pc_kv_append(*args) == 1
    assert needle in lib.pc_last_error()


@pytest.mark.parametrize(
    "overrides,needle",
    [
        ({"layer": 22}, b"layer"),
        ({"batch": -1}, b"batch"),
        ({"max_blocks": 0}, b"max_blocks"),
        ({"parts": 6}, b"partition_blocks"),
        ({"parts": 256}, b"partition_blocks"),
        ({"ws": None}, b"workspace"),
        ({"query": 8}, b"aligned"),
    ],
)
def test_attention_rejects_invalid_arguments_without_a_gpu(overrides, needle):
    lib = _hip.load()
    a = {"out": 16, "query": 16, "pool": 16, "blocks": 10, "layer": 0, "tables": 16, "max_blocks": 128,
         "lens": 16, "batch": 1, "parts": 32, "ws": 16}
    a.update(overrides)
    status = lib.pc_paged_decode_attn(
        a["out"], a["query"], a["pool"], a["blocks"], a["layer"], a["tables"], a["max_blocks"], a["lens"],
        a["batch"], a["parts"], a["ws"], a["ws"], None,
    )
    assert status == 1
    assert needle in lib.pc_last_error()


def test_missing_library_fails_loudly(monkeypatch, tmp_path):
    monkeypatch.setattr(_hip, "_library", None)
    monkeypatch.setattr(_hip, "library_path", lambda: str(tmp_path / "missing.so"))
    with pytest.raises(_hip.HipExtensionError, match="not built"):
        _hip.load()


def test_gpu_pool_allocator_requires_the_library(monkeypatch, tmp_path):
    """A GPU pool never falls back to a CPU path: constructing its allocator without the
    HIP library raises (checked here on a meta tensor standing in for device storage)."""
    import torch

    from pagedcore_amd import kv_cache

    monkeypatch.setattr(_hip, "_library", None)
    monkeypatch.setattr(_hip, "library_path", lambda: str(tmp_path / "missing.so"))
    with pytest.raises(_hip.HipExtensionError):
        kv_cache.HipKVWriter()
    pool = torch.empty((22, 2, 1, 16, 4, 64), dtype=torch.float16)
    allocator = kv_cache.KVAllocator(pool)  # CPU pool: bookkeeping only
    from pagedcore_amd.engine_types import KVReservation, RequestId

    allocator.create(KVReservation(RequestId("a"), 1))
    with pytest.raises(RuntimeError, match="KV writes run on the GPU"):
        allocator.append(RequestId("a"), *[torch.zeros(22, 1, 4, 64, dtype=torch.float16)] * 2)
    assert allocator.cached_length(RequestId("a")) == 0
