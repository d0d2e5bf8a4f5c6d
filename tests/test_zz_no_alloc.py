"""pc_paged_decode_attn_noalloc, the allocation-free variant of pc_paged_decode_attn: its
split-K partials live in the library's own per-GPU device array instead of a caller
workspace. Through the C ABI, against the workspace entry point on the same inputs (same
kernels, so the bits must match), on two calls in a row with the second one smaller, and
its refusal of shapes beyond the array. Runs alone in a fresh process and after the other
tests (the array keeps the previous call's contents, which must not matter)."""

from __future__ import annotations

import sys

import numpy as np
import pytest
import torch

from oracle import paged_reference as ref
from pagedcore_amd import _hip
from tests import workloads
from tests.support import fault_word, flags_clear

pytestmark = pytest.mark.gpu

SCRATCH_BYTES = 32 << 20  # PC_ATTN_NOALLOC_SCRATCH_BYTES


def _say(*parts) -> None:
    print(*parts, flush=True)
    sys.stdout.flush()


def _inputs(device, batch, hi, num_blocks, seed, layer):
    w = workloads.batched_decode(batch=batch, lo=1, hi=hi, num_blocks=num_blocks, seed=seed)
    gen = torch.Generator(device=device).manual_seed(seed)
    pool = torch.randn((22, 2, num_blocks, 16, 4, 64), dtype=torch.float16, device=device, generator=gen)
    queries = torch.from_numpy(w.queries(layer)).to(device)
    plan = torch.from_numpy(_hip.decode_plan(w.lengths, w.tables)).to(device)
    lens = torch.from_numpy(w.lengths).to(device)
    return w, pool, queries, plan, lens


def _call(lib, name, out, queries, pool, layer, lens, w, plan, *workspace):
    stream = torch.cuda.current_stream(out.device).cuda_stream
    status = getattr(lib, name)(
        out.data_ptr(), queries.data_ptr(), pool.data_ptr(), pool.shape[2], layer, lens.data_ptr(), w.batch,
        int(w.tables.shape[1]), plan.data_ptr(), int(plan.shape[0]), *workspace, stream,
    )
    assert status == 0, lib.pc_last_error().decode()


def test_noalloc_entry_point_matches_the_workspace_entry_point(device):
    lib = _hip.load()
    # First call: batch 64 over the full 2048-token range (long rows cut over several bins,
    # their parts merged through the array); second call: a smaller batch with shorter
    # tables, so the array still holds the first call's partials in places the second call
    # does not write.
    for batch, hi, num_blocks, seed, layer in ((64, 2048, 8192, 61, 4), (9, 500, 1024, 62, 17)):
        _say("no-alloc call", batch, hi)
        w, pool, queries, plan, lens = _inputs(device, batch, hi, num_blocks, seed, layer)
        nbytes = int(lib.pc_attn_workspace_bytes(w.batch, int(w.tables.shape[1])))
        assert 0 < nbytes <= SCRATCH_BYTES
        workspace = torch.zeros((nbytes,), dtype=torch.uint8, device=device)
        expected = torch.full_like(queries, float("nan"))
        _call(lib, "pc_paged_decode_attn", expected, queries, pool, layer, lens, w, plan, workspace.data_ptr())
        got = torch.full_like(queries, float("nan"))
        torch.cuda.synchronize(device)
        # Nothing is allocated: neither through torch's caching allocator nor by the library
        # itself (hipMalloc / hipMallocAsync would lower the device's free bytes).
        allocated = torch.cuda.memory_allocated(device)
        free_before = torch.cuda.mem_get_info(device)[0]
        _call(lib, "pc_paged_decode_attn_noalloc", got, queries, pool, layer, lens, w, plan)
        torch.cuda.synchronize(device)
        free_after = torch.cuda.mem_get_info(device)[0]
        assert torch.cuda.memory_allocated(device) == allocated
        assert free_after == free_before, (free_before, free_after)
        assert torch.equal(got.view(torch.int16), expected.view(torch.int16))
        # the workspace call left every part flag at zero again (the next call relies on it)
        # and recorded no fault
        assert flags_clear(workspace) and fault_word(workspace) == 0
        # and both within 2e-3 of FP64 on a few rows (the kernels' own parity bar)
        for b in (0, w.batch // 2, w.batch - 1):
            length = int(w.lengths[b])
            table = w.tables[b, : (length + 15) // 16].tolist()
            sub = torch.zeros((22, 2, len(table), 16, 4, 64), dtype=torch.float16)
            sub[layer] = pool[layer].index_select(1, torch.tensor(table, device=device)).cpu()
            fp64 = ref.dense_attention_fp64(
                queries[b : b + 1].reshape(1, 32, 1, 64).cpu(), *ref.gather_history(sub, layer, list(range(len(table))), length)
            )
            error = (got[b].cpu().double() - fp64.reshape(32, 64)).abs().max().item()
            assert error <= 2e-3, (batch, b, error)


def test_noalloc_entry_point_refuses_shapes_beyond_its_array(device):
    lib = _hip.load()
    # batch 8192 with 128-block tables needs 61.8 MB of partial slots: refused before any launch
    assert lib.pc_attn_workspace_bytes(8192, 128) > SCRATCH_BYTES
    out = torch.empty(16, dtype=torch.float16, device=device)
    status = lib.pc_paged_decode_attn_noalloc(
        out.data_ptr(), out.data_ptr(), out.data_ptr(), 8, 0, out.data_ptr(), 8192, 128, out.data_ptr(), 1,
        torch.cuda.current_stream(device).cuda_stream,
    )
    assert status == 1
    assert b"allocation-free entry point holds" in lib.pc_last_error()
    assert lib.pc_attn_workspace_bytes(256, 128) <= SCRATCH_BYTES  # the long-context batch fits
