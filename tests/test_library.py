"""The C-ABI library: loads without a GPU, exports every symbol include/pagedcore_hip.h
declares, and rejects invalid arguments before anything would be launched."""

from __future__ import annotations

import ctypes
import os
import re

import numpy as np
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
    # partials: 64 sequences x ceil(128/4) items x 32 q heads x 64 floats, then the
    # (max, sum) pairs; 256 B aligned regions
    out = 64 * 32 * 32 * 64 * 4
    ml = 64 * 32 * 32 * 2 * 4
    assert lib.pc_attn_workspace_bytes(64, 128, 4) == out + ml
    assert lib.pc_attn_workspace_bytes(1, 8, 4) == 2 * 32 * 64 * 4 + 512
    assert lib.pc_attn_workspace_bytes(1, 9, 8) == lib.pc_attn_workspace_bytes(1, 8, 4)
    for bad in (0, 3, 5, 16, 64):  # items hold 1, 2, 4 or 8 blocks
        assert lib.pc_attn_workspace_bytes(1, 8, bad) == 0


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
        ({"parts": 0}, b"partition_blocks"),
        ({"parts": 3}, b"partition_blocks"),
        ({"parts": 16}, b"partition_blocks"),
        ({"ws": None}, b"workspace"),
        ({"ws": 272}, b"aligned"),
        ({"query": 8}, b"aligned"),
        ({"out": 260}, b"aligned"),
        ({"flags": 6}, b"flags"),
        ({"tickets": None}, b"tickets"),
        ({"tickets": 258}, b"aligned"),
        ({"blocks": 2**31}, b"num_blocks"),
        ({"items": 258}, b"aligned"),
        ({"items": 256, "nitems": -1}, b"num_work_items"),
        ({"items": 256, "nitems": 17}, b"num_work_items"),  # batch 1 x 16 items
    ],
)
def test_attention_rejects_invalid_arguments_without_a_gpu(overrides, needle):
    lib = _hip.load()
    a = {"out": 256, "query": 256, "pool": 256, "blocks": 10, "layer": 0, "tables": 256, "max_blocks": 128,
         "lens": 256, "batch": 1, "parts": 8, "items": None, "nitems": 0, "ws": 256, "tickets": 256, "flags": 0}
    a.update(overrides)
    status = lib.pc_paged_decode_attn(
        a["out"], a["query"], a["pool"], a["blocks"], a["layer"], a["tables"], a["max_blocks"], a["lens"],
        a["batch"], a["parts"], a["items"], a["nitems"], a["ws"], a["tickets"], a["flags"], None,
    )
    assert status == 1
    assert needle in lib.pc_last_error()


def _plan_by_enumeration(lengths, tables, partition_blocks):
    """The plan records written out directly: {row, item, length, 0 (closer flag, set by
    the caller), block ids padded with 0 to a multiple of 4}."""
    fields = 4 + -(-partition_blocks // 4) * 4
    rows = []
    for b, length in enumerate(lengths):
        if length <= 0:
            continue
        blocks = min(-(-int(length) // 16), tables.shape[1])
        for item in range(-(-blocks // partition_blocks)):
            ids = [int(tables[b, i]) for i in range(item * partition_blocks, min((item + 1) * partition_blocks, blocks))]
            record = [b, item, int(length), 0] + ids
            rows.append(tuple(record + [0] * (fields - len(record))))
    return rows


@pytest.mark.parametrize("partition_blocks", [1, 2, 4, 8])
def test_decode_plan_lists_every_partition_once(partition_blocks):
    """pc_attn_plan (host code) against a direct enumeration, on ragged lengths including
    zero-length rows, exact block multiples and lengths clamped by the table width."""
    rng = np.random.default_rng(partition_blocks)
    lengths = rng.integers(0, 2049, size=97).astype(np.int32)
    lengths[:6] = [0, 1, 16, 17, 2048, 5000]  # 5000 tokens exceed the 128-block width: clamped
    tables = rng.integers(0, 50000, size=(97, 128)).astype(np.int32)
    plan = _hip.plan_work_items(lengths, tables, partition_blocks)
    assert plan.dtype == np.int32 and plan.shape[1] == _hip.load().pc_attn_plan_record_ints(partition_blocks)
    records = [tuple(r) for r in plan.tolist()]
    expected = _plan_by_enumeration(lengths, tables, partition_blocks)
    # the closer flag marks the last item of every multi-item sequence
    items_of = {}
    for r in expected:
        items_of[r[0]] = items_of.get(r[0], 0) + 1
    expected = [r[:3] + (1 if items_of[r[0]] > 1 and r[1] == items_of[r[0]] - 1 else 0,) + r[4:] for r in expected]
    assert sorted(records) == sorted(expected)
    # dispatch order: every closer after every other item; within each group, items with
    # more blocks first, sequence-major among equals
    flags = [r[3] for r in records]
    assert flags == sorted(flags)
    for flag in (0, 1):
        group = [r for r in records if r[3] == flag]
        counts = [min(min(-(-r[2] // 16), 128) - r[1] * partition_blocks, partition_blocks) for r in group]
        assert counts == sorted(counts, reverse=True)
        for count in set(counts):
            rows = [(r[0], r[1]) for r, c in zip(group, counts) if c == count]
            assert rows == sorted(rows)


def test_decode_plan_rejects_bad_arguments():
    lib = _hip.load()
    lens = np.array([100, 200], dtype=np.int32)
    tables = np.zeros((2, 16), dtype=np.int32)
    items = np.zeros((2, 8), dtype=np.int32)
    plan = lib.pc_attn_plan
    assert plan(lens.ctypes.data, tables.ctypes.data, 2, 16, 4, items.ctypes.data, 2) == -1  # needs 2 + 4 records
    assert b"capacity" in lib.pc_last_error()
    assert plan(lens.ctypes.data, tables.ctypes.data, 2, 16, 0, items.ctypes.data, 2) == -1
    assert b"partition_blocks" in lib.pc_last_error()
    assert plan(None, tables.ctypes.data, 2, 16, 4, items.ctypes.data, 2) == -1
    assert plan(lens.ctypes.data, None, 2, 16, 4, items.ctypes.data, 2) == -1
    assert b"null" in lib.pc_last_error()
    assert lib.pc_attn_plan_capacity(2, 16, 4) == 8
    assert lib.pc_attn_plan_capacity(2, 16, 6) == -1
    assert [lib.pc_attn_plan_record_ints(w) for w in (1, 2, 4, 8)] == [8, 8, 8, 12]
    assert lib.pc_attn_plan_record_ints(3) == -1
    assert plan(None, None, 0, 16, 4, None, 0) == 0  # empty batch: nothing to plan


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
