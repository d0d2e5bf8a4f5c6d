"""pc_kv_append_paged_decode_attn on the GPU: one launch that appends each sequence's newest
token and attends over it, against the two launches it replaces.

The decode step of the reference writes the new key and value (KVAllocator.write_decode_layer,
reference src/pagedcore/kv_cache.py:221-246) and then runs paged_attention over the history
that now holds them (reference src/pagedcore/decoder.py:187-190). The fused call must give
the same bits as pc_kv_append of those slots followed by pc_paged_decode_attn: the whole
pool (every layer, every row) and every output row compared with torch.equal. The unfused
pair is itself held to the oracle and to FP64 by the attention tests; one case here also
checks the fused rows against FP64 directly, within the 2e-3 max-abs bound.
"""

from __future__ import annotations

import sys

import numpy as np
import pytest
import torch

from pagedcore_amd import _hip
from tests import workloads
from tests.bin_plan import check_decode_plan, regrouped_plan
from tests.support import fault_word, flags_clear, workspace_flags

pytestmark = pytest.mark.gpu

ATOL = 2e-3


def _say(*parts) -> None:
    print(*parts, flush=True)
    sys.stdout.flush()


def _tables(lengths, num_blocks, seed):
    need = [(int(x) + 15) // 16 for x in lengths]
    perm = np.random.default_rng(seed).permutation(num_blocks).astype(np.int32)
    tables = np.zeros((len(lengths), max(max(need), 1)), dtype=np.int32)
    offset = 0
    for b, n in enumerate(need):
        tables[b, :n] = perm[offset : offset + n]
        offset += n
    return tables


def _slots(lengths, tables):
    """The pool slot of each sequence's newest token (position length - 1), -1 for an empty
    sequence: what pc_kv_append is given in the unfused pair."""
    slots = np.full(len(lengths), -1, dtype=np.int64)
    for b, n in enumerate(lengths):
        if n > 0:
            slots[b] = int(tables[b, (n - 1) // 16]) * 16 + (n - 1) % 16
    return slots




def _fp64_rows(pool, layer, tables, lengths, queries):
    out = torch.empty((len(lengths), 32, 64), dtype=torch.float64)
    for b, n in enumerate(lengths):
        width = (int(n) + 15) // 16
        ids = torch.as_tensor(tables[b, :width].astype(np.int64), device=pool.device)
        k = pool[layer, 0].index_select(0, ids).cpu().reshape(width * 16, 4, 64)[:n].permute(1, 0, 2).double()
        v = pool[layer, 1].index_select(0, ids).cpu().reshape(width * 16, 4, 64)[:n].permute(1, 0, 2).double()
        q = queries[b].cpu().double().reshape(4, 8, 64)
        scores = torch.matmul(q, k.transpose(-1, -2).contiguous()) / 8.0
        out[b] = torch.matmul(torch.softmax(scores, dim=-1), v).reshape(32, 64)
    return out


def _both_ways(device, lengths, tables, num_blocks, layer, seed, plan=None, check_plan=True):
    """(pool, out) of the unfused pair and of the fused call, from the same inputs, plus the
    fused call's workspace and the queries. check_plan: the plan covers every block once
    with ids inside the pool (off for tables that hold an id outside it on purpose)."""
    lengths = np.asarray(lengths, dtype=np.int32)
    batch = len(lengths)
    gen = torch.Generator(device=device).manual_seed(seed)
    pool = torch.randn((22, 2, num_blocks, 16, 4, 64), dtype=torch.float16, device=device, generator=gen)
    queries = torch.randn((batch, 32, 64), dtype=torch.float16, device=device, generator=gen)
    new_key = torch.randn((batch, 4, 64), dtype=torch.float16, device=device, generator=gen)
    new_value = torch.randn((batch, 4, 64), dtype=torch.float16, device=device, generator=gen)
    if plan is None:
        plan = _hip.decode_plan(lengths, tables)
    if check_plan:
        check_decode_plan(plan, lengths, tables, num_blocks, _hip.workspace_bytes(batch, tables.shape[1]))
    plan_d = torch.from_numpy(np.ascontiguousarray(plan)).to(device)
    lens_d = torch.from_numpy(lengths).to(device)
    nbytes = _hip.workspace_bytes(batch, tables.shape[1])

    pool_a = pool.clone()
    out_a = torch.full_like(queries, float("nan"))
    ws_a = torch.zeros(nbytes, dtype=torch.uint8, device=device)
    _hip.kv_append(pool_a, layer, new_key[None], new_value[None], torch.from_numpy(_slots(lengths, tables)).to(device))
    _hip.planned_decode_attention(out_a, queries, pool_a, layer, lens_d, plan_d, tables.shape[1], ws_a)

    pool_b = pool
    out_b = torch.full_like(queries, float("nan"))
    ws_b = torch.zeros(nbytes, dtype=torch.uint8, device=device)
    _hip.planned_decode_attention(out_b, queries, pool_b, layer, lens_d, plan_d, tables.shape[1], ws_b,
                                  new_key=new_key, new_value=new_value)
    torch.cuda.synchronize()
    return (pool_a, out_a), (pool_b, out_b), ws_b, queries


def _where(x, y, dims):
    """Count and the first few index tuples (over the leading `dims` axes) where x and y
    differ bitwise."""
    diff = (x.view(torch.int16) != y.view(torch.int16)).reshape(*x.shape[:dims], -1).any(-1)
    at = diff.nonzero().tolist()
    return len(at), at[:8]


def _assert_same(a, b, what):
    (pool_a, out_a), (pool_b, out_b) = a, b
    count, first = _where(pool_a, pool_b, 5)
    assert count == 0, f"{what}: pools differ at {count} (layer, kind, block, slot, head) rows, first {first}"
    count, first = _where(out_a, out_b, 2)
    assert count == 0, f"{what}: outputs differ at {count} (sequence, q head) rows, first {first}"


CASES = {
    # batch 64, lengths U{1..2048}: one to four sequences per bin, every last block patched
    "batch 64": (lambda: workloads.batched_decode(batch=64, num_blocks=8192, seed=91), None),
    # block boundaries: the new token at slot 0, 1, 14, 15 of its block, and empty rows
    "block boundaries": ([0, 1, 2, 15, 16, 17, 31, 32, 33, 47, 48, 0, 1000, 2047, 2048], 600),
    # sequences cut over many bins: the new token sits in the merging bin's last block
    "cut sequences": ([20000, 1, 5000, 16, 17, 8191], 2400),
    # 1000 short sequences: four segments per bin, each one ending at its sequence's last block
    "many short": (None, 3000),
}


@pytest.mark.parametrize("case", list(CASES))
def test_fused_append_matches_append_then_attention(device, case):
    """Whole pool and every output row bit-identical to pc_kv_append + pc_paged_decode_attn;
    the part flags end at zero."""
    _say("fused append + attention:", case)
    source, num_blocks = CASES[case]
    if case == "batch 64":
        w = source()
        lengths, tables, num_blocks = w.lengths, w.tables, w.num_blocks
    elif case == "many short":
        lengths = np.random.default_rng(92).integers(1, 49, size=1000).astype(np.int32)
        tables = _tables(lengths, num_blocks, 93)
    else:
        lengths = np.asarray(source, dtype=np.int32)
        tables = _tables(lengths, num_blocks, 94)
    a, b, workspace, queries = _both_ways(device, lengths, tables, num_blocks, layer=9, seed=95)
    _assert_same(a, b, case)
    assert flags_clear(workspace)
    nonempty = np.flatnonzero(np.asarray(lengths) > 0)
    assert torch.isfinite(b[1][torch.from_numpy(nonempty).to(device)]).all()


def test_fused_rows_match_fp64_after_append(device):
    """The fused call's outputs against FP64 attention over the appended history (the new
    token's row included), within 2e-3, for tokens on both sides of a block boundary."""
    lengths = np.asarray([1, 15, 16, 17, 33, 500, 2048, 2047], dtype=np.int32)
    tables = _tables(lengths, 400, 96)
    _, (pool, out), _, queries = _both_ways(device, lengths, tables, 400, layer=21, seed=97)
    expected = _fp64_rows(pool, 21, tables, lengths, queries)
    error = (out.cpu().double() - expected).abs().max().item()
    _say(f"fused rows vs fp64: max error {error:.2e}")
    assert error <= ATOL


def test_long_context_b256_fused_at_full_size(device):
    """The long-context workload exactly as the benchmark times it: batch 256, every sequence
    2047 cached tokens + the new one (128 blocks each) in a fully shuffled 40000-block pool
    (7.2e9 elements), the new rows appended by the fused call (pc_kv_append_paged_decode_attn)
    on one copy of the pool and by pc_kv_append + pc_paged_decode_attn on another. Layer 21,
    so the fused call's pool stores land at element offsets above 2^31. Both pools are
    bit-equal (every layer, every block, every slot), all 256 output rows are bit-equal, and
    every fused row is within 2e-3 of FP64 attention over the appended history."""
    w = workloads.batched_decode(batch=256, num_blocks=40000, fixed_length=2048, seed=20261204)
    layer = 21
    slots = _slots(w.lengths, w.tables)
    assert (slots // 16 == w.tables[:, 127]).all() and (slots % 16 == 15).all()
    assert ((2 * layer + 1) * w.num_blocks + int(w.tables[:, 127].max())) * 4096 > 2**31
    _say("b256 x 2048 fused at full size, layer", layer)
    a, b, workspace, queries = _both_ways(device, w.lengths, w.tables, w.num_blocks, layer=layer, seed=100)
    _assert_same(a, b, "b256 x 2048")
    assert flags_clear(workspace) and fault_word(workspace) == 0
    (pool, out) = b
    del a
    expected = _fp64_rows(pool, layer, w.tables, w.lengths, queries)
    error = (out.cpu().double() - expected).abs().max().item()
    _say(f"b256 fused rows vs fp64: max error {error:.2e}")
    assert error <= ATOL


def test_fused_append_with_regrouped_bins(device):
    """The plan's groups of bins moved to other XCDs: the same bits as the unfused pair."""
    w = workloads.batched_decode(batch=64, num_blocks=8192, seed=98)
    plan = regrouped_plan(_hip.decode_plan(w.lengths, w.tables), np.random.default_rng(4).permutation(8))
    a, b, workspace, _ = _both_ways(device, w.lengths, w.tables, w.num_blocks, layer=0, seed=99, plan=plan)
    _assert_same(a, b, "regrouped")
    assert flags_clear(workspace)


@pytest.mark.parametrize("where", ["last block", "earlier block"])
def test_out_of_pool_block_id(device, where):
    """An id outside the pool in a table: that row is NaN in both paths; in its last block
    the new token is not written (pc_kv_append skips the slot too); elsewhere it is. Pools
    and the other rows stay bit-identical."""
    lengths = np.asarray([300, 40, 1000, 17], dtype=np.int32)
    num_blocks = 200
    tables = _tables(lengths, num_blocks, 100)
    row = 2
    col = (int(lengths[row]) - 1) // 16 if where == "last block" else 3
    tables[row, col] = num_blocks + 5
    a, b, _, _ = _both_ways(device, lengths, tables, num_blocks, layer=4, seed=101, check_plan=False)
    assert torch.isnan(b[1][row]).all()
    keep = [r for r in range(len(lengths)) if r != row]
    assert torch.equal(a[1][keep].view(torch.int16), b[1][keep].view(torch.int16))
    assert torch.equal(a[0].view(torch.int16), b[0].view(torch.int16))


def test_fused_call_appends_in_place_over_a_decode_run(device):
    """Five decode steps of one layer: each step's fused call appends at the next position
    and attends; after the run the pool and the last outputs match five unfused steps."""
    lengths0 = np.asarray([14, 31, 1, 250], dtype=np.int32)
    num_blocks = 64
    tables = _tables(lengths0 + 5, num_blocks, 102)
    gen = torch.Generator(device=device).manual_seed(103)
    pool0 = torch.randn((22, 2, num_blocks, 16, 4, 64), dtype=torch.float16, device=device, generator=gen)
    pools = {"fused": pool0.clone(), "pair": pool0.clone()}
    outs = {}
    nbytes = _hip.workspace_bytes(len(lengths0), tables.shape[1])
    workspaces = {k: torch.zeros(nbytes, dtype=torch.uint8, device=device) for k in pools}
    for step in range(5):
        lengths = lengths0 + 1 + step
        queries = torch.randn((4, 32, 64), dtype=torch.float16, device=device, generator=gen)
        key = torch.randn((4, 4, 64), dtype=torch.float16, device=device, generator=gen)
        value = torch.randn((4, 4, 64), dtype=torch.float16, device=device, generator=gen)
        plan = torch.from_numpy(_hip.decode_plan(lengths, tables)).to(device)
        lens = torch.from_numpy(lengths).to(device)
        for kind, pool in pools.items():
            out = torch.empty_like(queries)
            if kind == "pair":
                _hip.kv_append(pool, 6, key[None], value[None], torch.from_numpy(_slots(lengths, tables)).to(device))
                _hip.planned_decode_attention(out, queries, pool, 6, lens, plan, tables.shape[1], workspaces[kind])
            else:
                _hip.planned_decode_attention(out, queries, pool, 6, lens, plan, tables.shape[1], workspaces[kind],
                                              new_key=key, new_value=value)
            outs[kind] = out
        torch.cuda.synchronize()
        assert torch.equal(outs["fused"].view(torch.int16), outs["pair"].view(torch.int16)), f"step {step}"
    assert torch.equal(pools["fused"].view(torch.int16), pools["pair"].view(torch.int16))


def test_fused_call_in_a_graph_replays_as_eager(device):
    """The fused call captured in a HIP graph: three replays, with eager fused calls and
    synchronizations between them, each give the eager call's pool and outputs."""
    w = workloads.batched_decode(batch=32, num_blocks=4096, seed=104)
    gen = torch.Generator(device=device).manual_seed(105)
    pool = torch.randn((22, 2, w.num_blocks, 16, 4, 64), dtype=torch.float16, device=device, generator=gen)
    queries = torch.randn((w.batch, 32, 64), dtype=torch.float16, device=device, generator=gen)
    key = torch.randn((w.batch, 4, 64), dtype=torch.float16, device=device, generator=gen)
    value = torch.randn((w.batch, 4, 64), dtype=torch.float16, device=device, generator=gen)
    plan = torch.from_numpy(_hip.decode_plan(w.lengths, w.tables)).to(device)
    lens = torch.from_numpy(w.lengths).to(device)
    width = w.tables.shape[1]
    workspace = torch.zeros(_hip.workspace_bytes(w.batch, width), dtype=torch.uint8, device=device)
    out = torch.empty_like(queries)

    def call():
        _hip.planned_decode_attention(out, queries, pool, 3, lens, plan, width, workspace, new_key=key, new_value=value)

    call()
    torch.cuda.synchronize()
    eager_out, eager_pool = out.clone(), pool.clone()
    side = torch.cuda.Stream(device=device)
    side.wait_stream(torch.cuda.current_stream(device))
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.stream(side):
        with torch.cuda.graph(graph, stream=side):
            call()
    torch.cuda.current_stream(device).wait_stream(side)
    for replay in range(3):
        out.fill_(float("nan"))
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out.view(torch.int16), eager_out.view(torch.int16)), f"replay {replay}"
        assert torch.equal(pool.view(torch.int16), eager_pool.view(torch.int16)), f"replay {replay}"
        assert flags_clear(workspace)
        call()  # eager work between replays
        torch.cuda.synchronize()


@pytest.mark.parametrize("fault", ["missing earlier part", "slots outside the workspace", "sequence outside the batch"])
def test_fused_call_with_malformed_plans_writes_only_planned_rows(device, fault):
    """The malformed plans of the attention tests, through the fused call: outputs of the
    rows the fault does not touch keep the intact plan's bits, and the pool differs from
    the intact plan's result at most in the new-token rows of the touched sequences, each
    of which holds either its old bits or the new row (never anything else, nowhere else)."""
    from tests.test_gpu_attention import _spans

    w = workloads.batched_decode(batch=64, num_blocks=8192, seed=86)
    plan = _hip.decode_plan(w.lengths, w.tables)
    spans = _spans(plan)
    bad_plan = plan.copy()
    if fault == "missing earlier part":
        row = spans[min(spans)][0][0]
        bad_plan[row] = 0
        spoiled = {int(x) for x in plan[row, 8 : 8 + 8 * int(plan[row, 0]) : 8]}
    elif fault == "slots outside the workspace":
        b = min(spans)
        for row, s, _, _, _ in spans[b].values():
            bad_plan[row, 8 + 8 * s + 7] = 1 << 30
        spoiled = {b}
    else:
        b = next(int(plan[r, 8 + 8 * s]) for r in range(plan.shape[0]) for s in range(int(plan[r, 0]))
                 if plan[r, 8 + 8 * s + 6] == 1)
        for r in range(plan.shape[0]):
            for s in range(int(plan[r, 0])):
                if plan[r, 8 + 8 * s] == b:
                    bad_plan[r, 8 + 8 * s] = w.batch + 5
        spoiled = {b}
    _say("fused call, malformed plan:", fault, "spoiled rows", sorted(spoiled))
    gen = torch.Generator(device=device).manual_seed(106)
    pool = torch.randn((22, 2, w.num_blocks, 16, 4, 64), dtype=torch.float16, device=device, generator=gen)
    queries = torch.randn((w.batch, 32, 64), dtype=torch.float16, device=device, generator=gen)
    key = torch.randn((w.batch, 4, 64), dtype=torch.float16, device=device, generator=gen)
    value = torch.randn((w.batch, 4, 64), dtype=torch.float16, device=device, generator=gen)
    lens = torch.from_numpy(w.lengths).to(device)
    width = w.tables.shape[1]
    results = []
    for p in (plan, bad_plan):
        target = pool.clone()
        out = torch.full_like(queries, 7.0)
        workspace = torch.zeros(_hip.workspace_bytes(w.batch, width), dtype=torch.uint8, device=device)
        _hip.planned_decode_attention(out, queries, target, 8, lens, torch.from_numpy(p).to(device), width, workspace,
                                      new_key=key, new_value=value)
        torch.cuda.synchronize()
        assert flags_clear(workspace)
        results.append((target, out))
    (good_pool, good), (bad_pool, bad) = results
    others = [x for x in range(w.batch) if x not in spoiled]
    assert torch.equal(bad[others].view(torch.int16), good[others].view(torch.int16))
    slots = _slots(w.lengths, w.tables)
    for x in sorted(spoiled):
        block, offset = divmod(int(slots[x]), 16)
        for kind, new in ((0, key[x]), (1, value[x])):
            got = bad_pool[8, kind, block, offset].view(torch.int16)
            assert torch.equal(got, new.view(torch.int16)) or torch.equal(got, pool[8, kind, block, offset].view(torch.int16))
            bad_pool[8, kind, block, offset] = good_pool[8, kind, block, offset]
    assert torch.equal(bad_pool.view(torch.int16), good_pool.view(torch.int16))
