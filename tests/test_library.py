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
    # one fp32 partial per (sequence, kv head, 9-block work item): O [8 q heads][64] then
    # (max, sum) of the 8 q heads
    part = (8 * 64 + 16) * 4
    assert lib.pc_attn_workspace_bytes(64, 128) == 64 * 4 * 15 * part
    assert lib.pc_attn_workspace_bytes(1, 9) == 4 * part
    assert lib.pc_attn_workspace_bytes(1, 10) == 4 * 2 * part
    assert lib.pc_attn_workspace_bytes(0, 128) == 0
    for batch, blocks in ((-1, 8), (1, 0), (1, 65537)):
        assert lib.pc_attn_workspace_bytes(batch, blocks) == 0


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
        ({"plan": None}, b"null pointer"),
        ({"lens": None}, b"null pointer"),
        ({"ws": None}, b"workspace"),
        ({"ws": 272}, b"aligned"),
        ({"query": 8}, b"aligned"),
        ({"out": 260}, b"aligned"),
        ({"plan": 260}, b"aligned"),
        ({"blocks": 2**31}, b"num_blocks"),
        ({"nrec": -1}, b"num_records"),
        ({"nrec": (1 + 8) * 15 + 1}, b"num_records"),  # batch 1, 128 blocks: 15 items per sequence
    ],
)
def test_attention_rejects_invalid_arguments_without_a_gpu(overrides, needle):
    lib = _hip.load()
    a = {"out": 256, "query": 256, "pool": 256, "blocks": 10, "layer": 0, "lens": 256, "batch": 1,
         "max_blocks": 128, "plan": 256, "nrec": 1, "ws": 256}
    a.update(overrides)
    status = lib.pc_paged_decode_attn(
        a["out"], a["query"], a["pool"], a["blocks"], a["layer"], a["lens"], a["batch"], a["max_blocks"],
        a["plan"], a["nrec"], a["ws"], None,
    )
    assert status == 1
    assert needle in lib.pc_last_error()


def _items_by_enumeration(lengths, tables):
    """Every (sequence, item) record written out directly: {row, item, length, items of the
    row, the item's 9 block ids (past the row's last block: its last id), 0, 0, 0}."""
    records = {}
    for b, length in enumerate(lengths):
        if length <= 0:
            continue
        blocks = min(-(-int(length) // 16), tables.shape[1])
        items = -(-blocks // 9)
        for item in range(items):
            ids = [int(tables[b, min(item * 9 + i, blocks - 1)]) for i in range(9)]
            records[(b, item)] = tuple([b, item, int(length), items] + ids + [0, 0, 0])
    return records


def test_decode_plan_lists_every_item_once_on_one_bin_per_sequence():
    """pc_attn_plan (host code) against a direct enumeration, on ragged lengths including
    zero-length rows, exact block multiples and the full 128-block table width: every
    item appears once, the items of a sequence share record index modulo 8 (one XCD), the
    8 bins' item counts differ by at most one sequence's items, padding records are empty,
    and longer sequences are dealt first."""
    rng = np.random.default_rng(5)
    lengths = rng.integers(0, 2049, size=97).astype(np.int32)
    lengths[:6] = [0, 1, 16, 17, 2048, 2047]
    tables = rng.integers(0, 50000, size=(97, 128)).astype(np.int32)
    plan = _hip.decode_plan(lengths, tables)
    lib = _hip.load()
    assert plan.dtype == np.int32 and plan.shape[1] == lib.pc_attn_plan_record_ints() == 16
    assert plan.shape[0] % 8 == 0 and plan.shape[0] <= lib.pc_attn_plan_capacity(97, 128)
    expected = _items_by_enumeration(lengths, tables)
    live = [tuple(r) for r in plan.tolist() if r[0] >= 0]
    assert sorted(live) == sorted(expected.values())
    for r in plan.tolist():
        if r[0] < 0:
            assert r == [-1] + [0] * 15
    bin_of = {}
    for index, r in enumerate(plan.tolist()):
        if r[0] >= 0:
            assert bin_of.setdefault(r[0], index % 8) == index % 8, "items of a sequence on two bins"
    per_bin = [sum(1 for index, r in enumerate(plan.tolist()) if r[0] >= 0 and index % 8 == x) for x in range(8)]
    assert max(per_bin) - min(per_bin) <= 15
    first_seen = {}
    for index, r in enumerate(plan.tolist()):
        if r[0] >= 0:
            first_seen.setdefault(r[0], index // 8)
    # within a bin, rows appear in order of decreasing length
    for x in range(8):
        rows = sorted((first_seen[b], b) for b in bin_of if bin_of[b] == x)
        lens = [lengths[b] for _, b in rows]
        assert lens == sorted(lens, reverse=True)


def test_decode_plan_rejects_bad_arguments():
    lib = _hip.load()
    lens = np.array([100, 200], dtype=np.int32)
    tables = np.zeros((2, 16), dtype=np.int32)
    records = np.zeros((64, 16), dtype=np.int32)
    plan = lib.pc_attn_plan
    assert plan(lens.ctypes.data, tables.ctypes.data, 2, 16, records.ctypes.data, 8) == -1  # needs 16 records
    assert b"capacity" in lib.pc_last_error()
    assert plan(lens.ctypes.data, tables.ctypes.data, 2, 16, records.ctypes.data, 16) == 16
    assert plan(lens.ctypes.data, tables.ctypes.data, 2, 0, records.ctypes.data, 64) == -1
    assert b"max_blocks" in lib.pc_last_error()
    assert plan(None, tables.ctypes.data, 2, 16, records.ctypes.data, 64) == -1
    assert plan(lens.ctypes.data, None, 2, 16, records.ctypes.data, 64) == -1
    assert b"null" in lib.pc_last_error()
    assert lib.pc_attn_plan_capacity(2, 16) == (2 + 8) * 2
    assert lib.pc_attn_plan_capacity(2, 0) == -1
    assert plan(None, None, 0, 16, None, 0) == 0  # empty batch: nothing to plan
    # a context longer than its table (16 tokens per entry) is refused, not clamped, and the
    # check does not overflow near INT32_MAX
    for too_long in (16 * 16 + 1, 2**31 - 1):
        lens[1] = too_long
        assert plan(lens.ctypes.data, tables.ctypes.data, 2, 16, records.ctypes.data, 64) == -1
        assert b"exceeds its 16-block table" in lib.pc_last_error()
    lens[1] = 16 * 16
    assert plan(lens.ctypes.data, tables.ctypes.data, 2, 16, records.ctypes.data, 64) == 16


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


def test_noalloc_attention_refuses_oversize_shapes_before_any_hip_call():
    """The allocation-free entry point checks the shape against its 32 MiB device array
    first, so the refusal needs no GPU (nothing else is touched)."""
    lib = _hip.load()
    assert lib.pc_attn_workspace_bytes(512, 128) > 32 << 20
    status = lib.pc_paged_decode_attn_noalloc(None, None, None, 8, 0, None, 512, 128, None, 1, None)
    assert status == 1 and b"allocation-free entry point holds" in lib.pc_last_error()
    assert lib.pc_paged_decode_attn_noalloc(None, None, None, 8, 0, None, 1, 0, None, 1, None) == 1
    assert b"max_blocks" in lib.pc_last_error()


@pytest.mark.parametrize(
    "overrides,needle",
    [
        ({"out": None}, b"null pointer"),
        ({"m": 0}, b"m = 0"),
        ({"m": 129}, b"m = 129"),
        ({"k": 2048, "splits": 3}, b"not divisible"),
        ({"k": 96}, b"multiple of 64"),
        ({"n": 48}, b"multiple of 32"),
        ({"epilogue": 1, "splits": 2}, b"one split"),
        ({"epilogue": 2, "splits": 2}, b"one split"),
        ({"epilogue": 2, "n": 96, "splits": 1}, b"multiple of 64"),
        ({"epilogue": 7}, b"unknown epilogue"),
        ({"x": 264}, b"aligned"),
        ({"n": 1 << 20, "k": 1 << 12}, b"too large"),
    ],
)
def test_gemm_rejects_invalid_arguments_without_a_gpu(overrides, needle):
    """pc_gemm_m128 validates shapes, splits, epilogue and alignment before any HIP call."""
    lib = _hip.load()
    a = {"out": 256, "x": 256, "w": 256, "m": 128, "n": 2048, "k": 2048, "splits": 4, "epilogue": 0}
    a.update(overrides)
    status = lib.pc_gemm_m128(a["out"], a["x"], a["w"], a["m"], a["n"], a["k"], a["splits"], a["epilogue"], None)
    assert status == 1
    assert needle in lib.pc_last_error()


def test_split_k_consumers_reject_invalid_arguments_without_a_gpu():
    lib = _hip.load()
    assert lib.pc_add_rms_norm_parts(256, 256, None, 1, 256, 4, 2048, 1e-5, None) == 1
    assert b"null pointer" in lib.pc_last_error()
    assert lib.pc_add_rms_norm_parts(256, 256, 256, 0, 256, 4, 2048, 1e-5, None) == 1
    assert b"splits" in lib.pc_last_error()
    assert lib.pc_add_rms_norm_parts(256, 256, 264, 2, 256, 4, 2048, 1e-5, None) == 1
    assert b"aligned" in lib.pc_last_error()
    assert lib.pc_add_rms_norm_parts(256, 256, 256, 2, 256, 4, 2049, 1e-5, None) == 1
    assert b"width" in lib.pc_last_error()
    assert lib.pc_rope_kv_append_parts(256, None, None, None, 4, 256, 256, 2048, None, 0, 0, None, 3, None) == 1
    assert b"null pointer" in lib.pc_last_error()
    assert lib.pc_rope_kv_append_parts(256, None, None, 256, 65, 256, 256, 2048, None, 0, 0, None, 3, None) == 1
    assert b"splits" in lib.pc_last_error()
    assert lib.pc_rope_kv_append_parts(256, None, None, 256, 4, 256, 256, 2048, 256, 0, 0, None, 3, None) == 1
    assert b"both" in lib.pc_last_error()
