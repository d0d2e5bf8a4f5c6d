"""The C-ABI library: loads without a GPU, exports every symbol include/pagedcore_hip.h
declares, and rejects invalid arguments before anything would be launched."""

from __future__ import annotations

import ctypes
import os
import re

import numpy as np
import pytest
from hypothesis import given, settings
from hypothesis import strategies as st

from pagedcore_amd import _hip
from tests.bin_plan import ROW, check_decode_plan

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


def _slots_bound(batch, max_blocks):
    """Partial slots a plan of the shape can need: at most one per bin (only a bin's last
    segment can be a part that is not its sequence's last), and the bins number at most 256
    plus one per 256 blocks, 2 per group for rounding, and one early close per 3 sequences."""
    total = batch * max_blocks
    return 256 + -(-total // 256) + 16 + (batch + 2) // 3


def test_workspace_and_capacity_formulas():
    lib = _hip.load()
    # a 256-byte header (the fault word), then one partial slot per (cut part, kv head): fp32
    # O of 8 q heads x 64 dims (2 KiB), then (max, sum) of the 8 q heads, then the part's
    # ready flag, padded to 17 128-byte lines
    slot = 2048 + 64 + 64
    assert slot == 2176 and _hip.WORKSPACE_HEADER_BYTES == 256
    for batch, blocks in ((64, 128), (1, 9), (1, 10), (256, 128), (97, 128), (0, 128)):
        assert lib.pc_attn_workspace_bytes(batch, blocks) == 256 + _slots_bound(batch, blocks) * 4 * slot
        group = max(256, -(-batch * blocks // 256)) + 1 + (batch + 2) // 3 + 1
        assert lib.pc_attn_plan_capacity(batch, blocks) == 8 * group
    assert lib.pc_attn_workspace_bytes(64, 128) < 3 << 20  # a few MiB, independent of context length
    for batch, blocks in ((-1, 8), (1, 0), (1, 65537)):
        assert lib.pc_attn_workspace_bytes(batch, blocks) == 0
        assert lib.pc_attn_plan_capacity(batch, blocks) == -1


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
        ({"nrec": 8 * (256 + 1 + 1 + 1) + 1}, b"num_records"),  # batch 1, 128 blocks: capacity + 1
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


@pytest.mark.parametrize(
    "overrides,needle",
    [
        ({"key": None}, b"null pointer"),
        ({"value": None}, b"null pointer"),
        ({"key": 264}, b"new_key/new_value must be 16-byte aligned"),
        ({"value": 258}, b"new_key/new_value must be 16-byte aligned"),
        ({"layer": -1}, b"layer"),
        ({"ws": None}, b"workspace"),
        ({"nrec": 8 * (256 + 1 + 1 + 1) + 1}, b"num_records"),
    ],
)
def test_fused_append_attention_rejects_invalid_arguments_without_a_gpu(overrides, needle):
    """pc_kv_append_paged_decode_attn checks its rows, then everything pc_paged_decode_attn
    checks, before any HIP call."""
    lib = _hip.load()
    a = {"out": 256, "query": 256, "pool": 256, "blocks": 10, "layer": 0, "lens": 256, "batch": 1,
         "max_blocks": 128, "plan": 256, "nrec": 1, "key": 512, "value": 768, "ws": 256}
    a.update(overrides)
    status = lib.pc_kv_append_paged_decode_attn(
        a["out"], a["query"], a["pool"], a["blocks"], a["layer"], a["lens"], a["batch"], a["max_blocks"],
        a["plan"], a["nrec"], a["key"], a["value"], a["ws"], None,
    )
    assert status == 1
    assert needle in lib.pc_last_error()


def _plan_and_check(lengths, tables, num_blocks):
    lib = _hip.load()
    plan = _hip.decode_plan(lengths, tables)
    assert plan.dtype == np.int32 and plan.shape[1] == lib.pc_attn_plan_record_ints() == ROW
    assert plan.shape[0] <= lib.pc_attn_plan_capacity(len(lengths), tables.shape[1])
    workspace = lib.pc_attn_workspace_bytes(len(lengths), tables.shape[1])
    return plan, check_decode_plan(plan, lengths, tables, num_blocks, workspace)


def test_decode_plan_covers_every_block_once_in_balanced_bins():
    """pc_attn_plan (host code) on ragged lengths including zero-length rows, exact block
    multiples and the full 128-block table width: every block of every sequence appears
    once, in order, with its table id; a cut sequence's parts sit in one group (one XCD) at
    rows first bin + 8 k; only a bin's first and last segments are cut parts; partial slots
    lie inside the workspace and do not overlap; the bins' block counts are balanced."""
    rng = np.random.default_rng(5)
    lengths = rng.integers(0, 2049, size=97).astype(np.int32)
    lengths[:6] = [0, 1, 16, 17, 2048, 2047]
    tables = rng.integers(0, 50000, size=(97, 128)).astype(np.int32)
    plan, stats = _plan_and_check(lengths, tables, 50000)
    # 256 bins of about 24 blocks (one per CU), and an early close or two where a bin
    # would hold more than 4 sequences
    assert 256 <= stats["rows"] <= 8 * 34 and stats["cut"] > 0
    blocks = plan[:, 1][plan[:, 0] > 0]
    nominal = -(-int(plan[:, 1].sum()) // 256)
    assert blocks.max() <= nominal + 1


@pytest.mark.parametrize(
    "name,lengths,max_blocks",
    [
        ("one token", [1], 8),
        ("one long sequence", [2048 * 16], 2048),
        ("many short sequences", [16] * 1000 + [1] * 24, 4),
        ("short and long", [17] * 300 + [2048] * 8, 128),
        ("long-context batch", [2048] * 256, 128),
        ("all empty", [0] * 7, 16),
        ("maximum table", [65536 * 16, 3, 0], 65536),
    ],
)
def test_decode_plan_edge_shapes(name, lengths, max_blocks):
    """Shapes that stress the planner's bounds: a single block, one sequence cut over many
    bins, more sequences than 4 per bin allows (early closes), a mix, a batch of whole
    sequences, an empty batch and the maximum table width; every plan passes the full check
    and fits the advertised capacity and workspace."""
    lengths = np.asarray(lengths, dtype=np.int32)
    rng = np.random.default_rng(len(lengths))
    tables = rng.integers(0, 1 << 20, size=(len(lengths), max_blocks)).astype(np.int32)
    plan, stats = _plan_and_check(lengths, tables, 1 << 20)
    if lengths.max() == 0:
        assert plan.shape[0] == 0
    else:
        assert plan.shape[0] % 8 == 0 and stats["rows"] == plan.shape[0]


@settings(max_examples=60, deadline=None, derandomize=True)
@given(
    batch=st.integers(1, 300),
    top=st.integers(1, 2048),
    zeros=st.floats(0.0, 0.5),
    seed=st.integers(0, 2**31 - 1),
)
def test_decode_plan_random_batches_pass_the_full_check(batch, top, zeros, seed):
    """Random ragged batches (1 to 300 sequences, lengths up to `top`, a share of empty
    rows): every plan passes the full check of what the kernel reads and writes, and fits
    the advertised capacity and workspace."""
    rng = np.random.default_rng(seed)
    lengths = rng.integers(1, top + 1, size=batch).astype(np.int32)
    lengths[rng.random(batch) < zeros] = 0
    max_blocks = max(1, (int(lengths.max()) + 15) // 16)
    tables = rng.integers(0, 1 << 20, size=(batch, max_blocks)).astype(np.int32)
    plan, stats = _plan_and_check(lengths, tables, 1 << 20)
    assert (plan.shape[0] == 0) == (lengths.max() == 0)


def test_decode_plan_rejects_bad_arguments():
    lib = _hip.load()
    lens = np.array([100, 200], dtype=np.int32)
    tables = np.zeros((2, 16), dtype=np.int32)
    records = np.zeros((64, ROW), dtype=np.int32)
    plan = lib.pc_attn_plan
    # 7 + 13 blocks: 2 bins (8 blocks or more each, one whole sequence in each), in two
    # groups; one row per group, so 8 rows
    assert plan(lens.ctypes.data, tables.ctypes.data, 2, 16, records.ctypes.data, 7) == -1
    assert b"capacity" in lib.pc_last_error()
    assert plan(lens.ctypes.data, tables.ctypes.data, 2, 16, records.ctypes.data, 8) == 8
    assert plan(lens.ctypes.data, tables.ctypes.data, 2, 0, records.ctypes.data, 64) == -1
    assert b"max_blocks" in lib.pc_last_error()
    assert plan(None, tables.ctypes.data, 2, 16, records.ctypes.data, 64) == -1
    assert plan(lens.ctypes.data, None, 2, 16, records.ctypes.data, 64) == -1
    assert b"null" in lib.pc_last_error()
    assert lib.pc_attn_plan_capacity(2, 16) == 8 * (256 + 1 + 1 + 1)
    assert lib.pc_attn_plan_capacity(2, 0) == -1
    assert plan(None, None, 0, 16, None, 0) == 0  # empty batch: nothing to plan
    # a context longer than its table (16 tokens per entry) is refused, not clamped, and the
    # check does not overflow near INT32_MAX
    for too_long in (16 * 16 + 1, 2**31 - 1):
        lens[1] = too_long
        assert plan(lens.ctypes.data, tables.ctypes.data, 2, 16, records.ctypes.data, 64) == -1
        assert b"exceeds its 16-block table" in lib.pc_last_error()
    lens[1] = 16 * 16
    assert plan(lens.ctypes.data, tables.ctypes.data, 2, 16, records.ctypes.data, 64) == 8


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
    assert lib.pc_attn_workspace_bytes(8192, 128) > 32 << 20
    assert lib.pc_attn_workspace_bytes(4096, 128) <= 32 << 20
    status = lib.pc_paged_decode_attn_noalloc(None, None, None, 8, 0, None, 8192, 128, None, 1, None)
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
