"""Paged decode attention on the GPU vs the CPU oracle and the FP64 dense oracle.

The reference's attention tests (tests/unit/test_attention.py, tests/gpu/test_attention_cuda.py)
re-run against the HIP path through the unchanged Python API, plus the batched shapes the
hot path is measured on. Tolerance: max |gpu - expected| <= 2e-3 on the fp16 outputs with
no relative term (the parity bound of this path; the reference's own tests use assert_close with
atol = rtol = 2e-3, which is looser), against both the op-for-op oracle (an fp16 output)
and FP64 dense attention (compared unrounded); tighter where the reference uses a tighter
bound. Each check prints the largest error it saw.
"""

from __future__ import annotations

import os
import sys

import numpy as np
import pytest
import torch

from oracle import paged_reference as ref
from pagedcore_amd import _hip
from tests import workloads
from tests.bin_plan import check_decode_plan, regrouped_plan
from tests.support import ATOL, assert_max_abs, fault_word, flags_clear, workspace_flags
from pagedcore_amd.attention import paged_attention, paged_attention_batch
from pagedcore_amd.engine_types import CapacityCounts, KVReservation, RequestId
from pagedcore_amd.kv_cache import KVAllocator

pytestmark = pytest.mark.gpu

def _say(*parts) -> None:
    print(*parts, flush=True)
    sys.stdout.flush()


class Worst:
    """Largest oracle / FP64 errors seen by one test, printed at its end."""

    def __init__(self, name: str) -> None:
        self.name, self.oracle, self.fp64 = name, 0.0, 0.0

    def check(self, got, oracle, fp64, what: str) -> None:
        if oracle is not None:
            self.oracle = max(self.oracle, assert_max_abs(got, oracle, f"{what} vs oracle"))
        self.fp64 = max(self.fp64, assert_max_abs(got, fp64, f"{what} vs fp64"))

    def report(self) -> None:
        _say(f"{self.name}: max |gpu - oracle| = {self.oracle:.2e}, max |gpu - fp64| = {self.fp64:.2e} (bound {ATOL:.0e})")


def test_device_is_gfx950_and_one_hip_runtime_is_mapped(device):
    name = torch.cuda.get_device_properties(device).gcnArchName
    _say("device", torch.cuda.get_device_name(device), name)
    assert name.startswith("gfx950")
    _hip.load()
    with open("/proc/self/maps") as maps:
        runtimes = {line.split()[-1] for line in maps if "libamdhip64" in line}
    assert len(runtimes) == 1, runtimes
    with open("/proc/self/maps") as maps:
        assert any(_hip.LIBRARY_NAME in line for line in maps)


def _fp64(query, key, value):
    return ref.dense_attention_fp64(query, key, value).reshape(1, 32, 1, 64)


def _check(query, key, value, *, layer, atol=ATOL, rtol=0.0, exact=None):
    """The reference GPU harness (tests/gpu/test_attention_cuda.py:93-145) on the HIP path:
    a NaN-poisoned pool with a retained sentinel request between released ones, so the
    request's table is fragmented; checks FP64 and oracle agreement, autocast invariance,
    untouched pool, unchanged table/length/accounting."""
    device = query.device
    tokens = key.shape[1]
    blocks = (tokens + 15) // 16
    pool = torch.full((22, 2, blocks + 3, 16, 4, 64), float("nan"), dtype=torch.float16, device=device)
    allocator = KVAllocator(pool)
    for name in ("first", "retained", "last"):
        request = RequestId(name)
        allocator.create(KVReservation(request, 1))
        sentinel = torch.full((22, 16, 4, 64), -100.0, dtype=torch.float16, device=device)
        allocator.append(request, sentinel, -sentinel)
    allocator.release_all(RequestId("first"))
    allocator.release_all(RequestId("last"))
    request = RequestId("attention")
    allocator.create(KVReservation(request, blocks))
    allocator.append(request, key, value)
    table = allocator.block_table(request)
    if blocks > 1:
        assert table != tuple(range(table[0], table[0] + blocks))
    before = pool.clone()
    counts = allocator.capacity()

    actual = paged_attention(query, allocator, request, layer_index=layer)
    with torch.autocast("cuda", dtype=torch.float16):
        autocast_actual = paged_attention(query, allocator, request, layer_index=layer)
    torch.cuda.synchronize(device)

    assert actual.device == query.device and actual.dtype == torch.float16
    assert actual.shape == (1, 32, 1, 64) and not actual.requires_grad
    assert torch.isfinite(actual).all()
    expected = _fp64(query.detach().cpu(), key[layer].cpu(), value[layer].cpu())
    oracle = ref.reference_paged_attention(query.detach().cpu(), pool.cpu(), layer, list(table), tokens)
    worst = Worst(f"{tokens} tokens, layer {layer}")
    worst.oracle = assert_max_abs(actual, oracle, "vs oracle", atol, rtol)
    worst.fp64 = assert_max_abs(actual, expected, "vs fp64", atol, rtol)
    worst.report()
    if exact is not None:
        assert torch.equal(actual.cpu(), torch.full_like(actual.cpu(), exact) if not callable(exact) else exact())
    assert torch.equal(autocast_actual, actual)
    torch.testing.assert_close(pool, before, atol=0, rtol=0, equal_nan=True)
    assert allocator.block_table(request) == table
    assert allocator.cached_length(request) == tokens
    assert allocator.capacity() == counts
    allocator.release_all(request)
    allocator.release_all(RequestId("retained"))
    assert allocator.capacity() == CapacityCounts(blocks + 3, blocks + 3, 0, 0, 0, 0)
    return actual


@pytest.mark.parametrize("tokens,layer", [(1, 0), (15, 21), (16, 7), (17, 0), (49, 21), (2048, 11)])
def test_cache_boundaries_match_fp64_and_oracle(device, tokens, layer):
    _say("boundaries", tokens, layer)
    gen = torch.Generator(device=device).manual_seed(tokens)
    key = torch.randn(22, tokens, 4, 64, dtype=torch.float16, device=device, generator=gen)
    value = torch.randn(22, tokens, 4, 64, dtype=torch.float16, device=device, generator=gen)
    query = torch.randn(1, 32, 1, 128, dtype=torch.float16, device=device, generator=gen)
    _check(query[..., ::2].requires_grad_(), key, value, layer=layer)


def test_eight_query_heads_map_to_each_kv_head(device):
    key = torch.zeros(22, 33, 4, 64, dtype=torch.float16, device=device)
    values = 100 * torch.arange(4, device=device)[None, :] + torch.arange(33, device=device)[:, None]
    value = values[None, :, :, None].expand(22, 33, 4, 64).half()
    out = _check(torch.zeros(1, 32, 1, 64, dtype=torch.float16, device=device), key, value, layer=21)
    for head in range(32):
        assert torch.equal(out[0, head, 0].cpu(), torch.full((64,), 100 * (head // 8) + 16).half())


def test_tiny_probabilities_survive_until_value_accumulation(device):
    key = torch.zeros(22, 17, 4, 64, dtype=torch.float16, device=device)
    key[:, :, :, 0], key[:, 0, :, 0] = -160, 0
    value = torch.full_like(key, 65504)
    value[:, 0] = 0
    query = torch.zeros(1, 32, 1, 64, dtype=torch.float16, device=device)
    query[..., 0] = 1
    # tests/unit/test_attention.py:224-242 bounds this case by atol=1e-6, rtol=2e-3 (the
    # output is about 2.2e-3, where one fp16 ulp is 1.9e-6)
    out = _check(query, key, value, layer=0, atol=1e-6, rtol=2e-3)
    assert (out > 0).all()


def test_rounds_only_after_value_cancellation_across_pages(device):
    key = torch.zeros(22, 32, 4, 64, dtype=torch.float16, device=device)
    value = torch.zeros_like(key)
    value[:, 0], value[:, 1], value[:, 16] = 32768, 8, -32768
    _check(torch.zeros(1, 32, 1, 64, dtype=torch.float16, device=device), key, value, layer=0, exact=0.25)


def test_normalizes_all_scores_before_value_products(device):
    # tests/unit/test_attention.py:182-221 (tables (0, 2) on a 3-block pool): exactly 3.
    pool = torch.full((22, 2, 3, 16, 4, 64), float("nan"), dtype=torch.float16, device=device)
    allocator = KVAllocator(pool)
    key = torch.zeros(22, 17, 4, 64, dtype=torch.float16, device=device)
    value = torch.zeros_like(key)
    value[:, :16], value[:, 16:] = 2, 19
    request, blocker = RequestId("normalized"), RequestId("blocker")
    allocator.create(KVReservation(request, 2))
    allocator.append(request, key[:, :16], value[:, :16])
    allocator.create(KVReservation(blocker, 1))
    allocator.append(blocker, key[:, :16], torch.full_like(key[:, :16], 1000))
    allocator.append(request, key[:, 16:], value[:, 16:])
    assert allocator.block_table(request) == (0, 2)
    before, counts = pool.clone(), allocator.capacity()
    with torch.autocast("cuda", dtype=torch.bfloat16):
        actual = paged_attention(torch.zeros(1, 32, 1, 64, dtype=torch.float16, device=device), allocator, request, layer_index=0)
    assert torch.equal(actual.cpu(), torch.full((1, 32, 1, 64), 3, dtype=torch.float16))
    torch.testing.assert_close(pool, before, atol=0, rtol=0, equal_nan=True)
    assert allocator.capacity() == counts


@pytest.mark.parametrize("reverse", [False, True])
@pytest.mark.parametrize("query_scale", [1.0, 1000.0])
def test_large_block_scores_rescale_softmax(device, reverse, query_scale):
    key = torch.full((22, 49, 4, 64), -1000.0, dtype=torch.float16, device=device)
    key[:, 16:32] = 0
    key[:, 32:] = 1000
    value = torch.randn(key.shape, dtype=torch.float16, device=device, generator=torch.Generator(device=device).manual_seed(9))
    if reverse:
        key, value = key.flip(1), value.flip(1)
    query = torch.full((1, 32, 1, 64), query_scale, dtype=torch.float16, device=device)
    _check(query, key, value, layer=0)


@pytest.mark.parametrize("state", ["unknown", "empty", "released"])
def test_rejects_requests_without_cached_tokens(device, state):
    allocator = KVAllocator(torch.empty(22, 2, 1, 16, 4, 64, dtype=torch.float16, device=device))
    request = RequestId("missing")
    if state != "unknown":
        allocator.create(KVReservation(request, 1))
    if state == "released":
        allocator.release_all(request)
    before = allocator.capacity()
    with pytest.raises(ValueError if state == "empty" else KeyError):
        paged_attention(torch.zeros(1, 32, 1, 64, dtype=torch.float16, device=device), allocator, request, layer_index=0)
    assert allocator.capacity() == before


def _upload_single_decode(device):
    w = workloads.single_decode()
    pool = torch.full((22, 2, w.num_blocks, 16, 4, 64), float("nan"), dtype=torch.float16)
    for logical, physical in enumerate(w.table):
        pool[w.layer, 0, physical] = torch.from_numpy(w.key[logical * 16 : logical * 16 + 16])
        pool[w.layer, 1, physical] = torch.from_numpy(w.value[logical * 16 : logical * 16 + 16])
    return w, pool.to(device)


def test_config1_golden_through_the_c_abi(device):
    """Single-sequence 128-token decode over a seeded random table of a 64-block pool, via
    the raw C ABI; the committed FP64 output is the reference answer."""
    golden = np.load(os.path.join(os.path.dirname(__file__), "golden", "config1_single_decode.npz"))
    w, pool = _upload_single_decode(device)
    assert np.array_equal(golden["query"], w.query.view(np.uint16))
    assert np.array_equal(golden["key"], w.key.view(np.uint16))
    assert golden["table"].tolist() == w.table
    query = torch.from_numpy(w.query).to(device).reshape(1, 32, 64)
    out = torch.empty(1, 32, 64, dtype=torch.float16, device=device)
    tables = torch.tensor([w.table], dtype=torch.int32, device=device)
    lens = torch.tensor([128], dtype=torch.int32, device=device)
    out.fill_(float("nan"))
    _hip.paged_decode_attention(out, query, pool, w.layer, tables, lens)
    torch.cuda.synchronize()
    expected = torch.from_numpy(golden["expected_fp64"]).reshape(1, 32, 64)
    worst = Worst("config 1 golden")
    worst.check(out, None, expected, "config 1")
    worst.report()


def _random_pool(device, num_blocks, seed):
    gen = torch.Generator(device=device).manual_seed(seed)
    return torch.randn((22, 2, num_blocks, 16, 4, 64), dtype=torch.float16, device=device, generator=gen)


def _oracle_rows(pool, layer, w, queries, rows):
    """Oracle outputs for selected rows, reading only those rows' blocks from the GPU."""
    out = {}
    for b in rows:
        length = int(w.lengths[b])
        table = w.tables[b, : (length + 15) // 16].tolist()
        blocks = torch.tensor(table, dtype=torch.long, device=pool.device)
        sub = torch.zeros((22, 2, len(table), 16, 4, 64), dtype=torch.float16)
        sub[layer] = pool[layer].index_select(1, blocks).cpu()
        q = queries[b : b + 1].reshape(1, 32, 1, 64).cpu()
        out[b] = (
            ref.reference_paged_attention(q, sub, layer, list(range(len(table))), length),
            ref.dense_attention_fp64(q, *ref.gather_history(sub, layer, list(range(len(table))), length)).reshape(
                1, 32, 1, 64
            ),
        )
    return out


def _shuffled_plan(w, seed):
    """The decode plan with its 8 groups of bins moved to other groups in a random order:
    every bin runs on another XCD and in another dispatch position; the answer must not
    change."""
    plan = _hip.decode_plan(w.lengths, w.tables)
    return regrouped_plan(plan, np.random.default_rng(seed).permutation(8))


@pytest.mark.parametrize("order", ["binned", "shuffled"])
def test_batched_decode_b64_matches_oracle(device, order):
    """Batch 64, lengths U{1..2048}, fragmented tables over an 8192-block pool; every row
    against the oracle restatement and FP64, with the plan as built and with its groups of
    bins moved to other XCDs."""
    _say("batched b64 plan", order)
    w = workloads.batched_decode(batch=64, num_blocks=8192)
    pool = _random_pool(device, w.num_blocks, 11)
    layer = 5
    queries = torch.from_numpy(w.queries(layer)).to(device)
    out = torch.full_like(queries, float("nan"))
    plan = _hip.decode_plan(w.lengths, w.tables) if order == "binned" else _shuffled_plan(w, 3)
    _hip.paged_decode_attention(
        out, queries, pool, layer, torch.from_numpy(w.tables).to(device), torch.from_numpy(w.lengths).to(device),
        plan=torch.from_numpy(plan).to(device),
    )
    torch.cuda.synchronize()
    expected = _oracle_rows(pool, layer, w, queries, range(w.batch))
    worst = Worst(f"batch 64 ({order} plan)")
    for b, (oracle, fp64) in expected.items():
        worst.check(out[b : b + 1].reshape(1, 32, 1, 64), oracle, fp64, f"row {b} len {w.lengths[b]}")
    worst.report()


def test_block_and_bin_boundaries_match_oracle(device):
    """Lengths on both sides of 16-token block boundaries and of multiples of 9 blocks, a
    single token and a single block, in one ragged batch over a shuffled pool: the plan cuts
    the long rows across bins (parts merged in the kernel) and puts short rows several to a
    bin; every row against the oracle and FP64."""
    lengths = np.array([143, 144, 145, 287, 288, 289, 1151, 1152, 1153, 1295, 1296, 1297, 2047, 2048, 1, 16],
                       dtype=np.int32)
    _say("block and bin boundaries", lengths.tolist())
    need = (lengths + 15) // 16
    num_blocks = 1024
    perm = np.random.default_rng(77).permutation(num_blocks).astype(np.int32)
    tables = np.zeros((len(lengths), int(need.max())), dtype=np.int32)
    offset = 0
    for b, n in enumerate(need):
        tables[b, :n] = perm[offset : offset + n]
        offset += int(n)
    w = workloads.BatchedDecode(lengths, tables, num_blocks, 77)
    pool = _random_pool(device, num_blocks, 13)
    layer = 9
    queries = torch.from_numpy(w.queries(layer)).to(device)
    out = torch.full_like(queries, float("nan"))
    _hip.paged_decode_attention(out, queries, pool, layer, torch.from_numpy(tables).to(device),
                                torch.from_numpy(lengths).to(device))
    torch.cuda.synchronize()
    stats = check_decode_plan(_hip.decode_plan(lengths, tables), lengths, tables, num_blocks,
                              _hip.workspace_bytes(len(lengths), tables.shape[1]))
    assert stats["cut"] > 0
    worst = Worst("block and bin boundaries")
    for b, (oracle, fp64) in _oracle_rows(pool, layer, w, queries, range(len(lengths))).items():
        worst.check(out[b : b + 1].reshape(1, 32, 1, 64), oracle, fp64, f"row {b} len {lengths[b]}")
    worst.report()


@pytest.mark.parametrize("seed", [101, 202, 303, 404])
def test_random_batches_through_the_allocator_match_fp64(device, seed):
    """Random batch sizes (1-200) and lengths (1-2048) appended through the allocator into
    one NaN-poisoned pool, attended with paged_attention_batch at a random layer: every row
    within 2e-3 of FP64 over the request's gathered history."""
    rng = np.random.default_rng(seed)
    batch = int(rng.integers(1, 201))
    lengths = rng.integers(1, 2049, size=batch)
    blocks = int(((lengths + 15) // 16).sum()) + 8
    _say("random batch", seed, batch, int(lengths.sum()))
    gen = torch.Generator(device=device).manual_seed(seed)
    pool = torch.full((22, 2, blocks, 16, 4, 64), float("nan"), dtype=torch.float16, device=device)
    allocator = KVAllocator(pool)
    requests = tuple(RequestId(f"s{seed}-{b}") for b in range(batch))
    for request, length in zip(requests, lengths):
        allocator.create(KVReservation(request, int((length + 15) // 16)))
        key = torch.randn(22, int(length), 4, 64, dtype=torch.float16, device=device, generator=gen)
        value = torch.randn(22, int(length), 4, 64, dtype=torch.float16, device=device, generator=gen)
        allocator.append(request, key, value)
    layer = int(rng.integers(0, 22))
    query = torch.randn(batch, 32, 1, 64, dtype=torch.float16, device=device, generator=gen)
    out = paged_attention_batch(query, allocator, requests, layer_index=layer)
    torch.cuda.synchronize()
    worst = Worst(f"random batch seed {seed}")
    for b, request in enumerate(requests):
        table = list(allocator.block_table(request))
        index = torch.tensor(table, dtype=torch.long, device=device)
        sub = torch.zeros((22, 2, len(table), 16, 4, 64), dtype=torch.float16)
        sub[layer] = pool[layer].index_select(1, index).cpu()
        history = ref.gather_history(sub, layer, list(range(len(table))), int(lengths[b]))
        fp64 = ref.dense_attention_fp64(query[b : b + 1].cpu(), *history).reshape(1, 32, 1, 64)
        worst.check(out[b : b + 1], None, fp64, f"seed {seed} row {b} len {lengths[b]}")
    worst.report()


def _fp64_all_rows(pool, layer, tables, lengths, queries, chunk=32):
    """FP64 dense attention of every row over its gathered history (rows batched, the
    history masked past each row's length): [batch, 32, 64] float64 on the CPU."""
    batch = queries.shape[0]
    out = torch.empty((batch, 32, 64), dtype=torch.float64)
    for lo in range(0, batch, chunk):
        hi = min(batch, lo + chunk)
        lens = torch.as_tensor(np.asarray(lengths[lo:hi], dtype=np.int64))
        width = int((lens.max() + 15) // 16)
        ids = torch.as_tensor(np.asarray(tables[lo:hi, :width], dtype=np.int64)).clamp(0, pool.shape[2] - 1)
        k, v = (pool[layer, kind].index_select(0, ids.reshape(-1).to(pool.device)).cpu() for kind in (0, 1))
        k = k.reshape(hi - lo, width * 16, 4, 64).permute(0, 2, 1, 3).double()  # [rows, 4, T, 64]
        v = v.reshape(hi - lo, width * 16, 4, 64).permute(0, 2, 1, 3).double()
        q = queries[lo:hi].cpu().double().reshape(hi - lo, 4, 8, 64)
        scores = torch.matmul(q, k.transpose(-1, -2).contiguous()) / 8.0  # [rows, 4, 8, T]
        mask = torch.arange(width * 16)[None, :] >= lens[:, None]
        scores.masked_fill_(mask[:, None, None, :], float("-inf"))
        out[lo:hi] = torch.matmul(torch.softmax(scores, dim=-1), v).reshape(hi - lo, 32, 64)
    return out


def test_long_context_b256_full_length(device):
    """The long-context workload as one step of one layer: batch 256, each sequence 2047
    cached tokens on 128 blocks of a fully shuffled 40000-block pool; pc_kv_append writes
    every sequence's new token (slot 2047), then attention runs over 2048 tokens (one bin
    of 128 blocks per sequence). The appended rows are bit-exact, every row is within 2e-3
    of FP64, sampled rows within 2e-3 of the op-for-op oracle, and regrouped bins give the
    same bits."""
    _say("b256 long context: append + attention")
    w = workloads.batched_decode(batch=256, num_blocks=40000, fixed_length=2048, seed=44)
    pool = _random_pool(device, w.num_blocks, 12)
    layer = 21
    gen = torch.Generator(device=device).manual_seed(21)
    new_key = torch.randn((1, w.batch, 4, 64), dtype=torch.float16, device=device, generator=gen)
    new_value = torch.randn((1, w.batch, 4, 64), dtype=torch.float16, device=device, generator=gen)
    last = torch.from_numpy(w.tables[:, 127].astype(np.int64))
    slots = (last * 16 + 15).to(device)
    before = pool[layer, :, last.to(device)].clone()  # [2, 256, 16, 4, 64]
    _hip.kv_append(pool, layer, new_key, new_value, slots)
    after = pool[layer, :, last.to(device)]
    torch.cuda.synchronize()
    assert torch.equal(after[0, :, 15].view(torch.int16), new_key[0].view(torch.int16))
    assert torch.equal(after[1, :, 15].view(torch.int16), new_value[0].view(torch.int16))
    assert torch.equal(after[:, :, :15].view(torch.int16), before[:, :, :15].view(torch.int16))

    queries = torch.from_numpy(w.queries(layer)).to(device)
    tables = torch.from_numpy(w.tables).to(device)
    lens = torch.from_numpy(w.lengths).to(device)
    results = {}
    for order in ("binned", "shuffled"):
        plan = _hip.decode_plan(w.lengths, w.tables) if order == "binned" else _shuffled_plan(w, 5)
        out = torch.full_like(queries, float("nan"))
        _hip.paged_decode_attention(out, queries, pool, layer, tables, lens, plan=torch.from_numpy(plan).to(device))
        results[order] = out
    torch.cuda.synchronize()
    assert torch.equal(results["binned"], results["shuffled"])
    got = results["binned"]
    worst = Worst("b256 x 2048 after append")
    fp64 = _fp64_all_rows(pool, layer, w.tables, w.lengths, queries)
    for b in range(w.batch):
        worst.check(got[b], None, fp64[b], f"row {b}")
    for b, (oracle, _) in _oracle_rows(pool, layer, w, queries, [0, 1, 63, 64, 127, 128, 200, 255]).items():
        worst.oracle = max(worst.oracle, assert_max_abs(got[b : b + 1].reshape(1, 32, 1, 64), oracle, f"row {b} vs oracle"))
    worst.report()


def test_plan_order_and_graph_replays_are_invisible(device):
    """Ragged lengths with empty, one-token, block-boundary and full rows: the output is the
    same bits for the plan as built, for its groups of bins in reverse XCD order, and for
    every replay of a captured HIP graph (with eager calls in between), and matches the
    oracle."""
    _say("plan order and graph replays")
    w = workloads.batched_decode(batch=64, num_blocks=8192, seed=49)
    lengths = w.lengths.copy()
    lengths[:6] = [1, 16, 17, 144, 145, 2048]
    lengths[6] = 0  # no cached token: the row is not written
    pool = _random_pool(device, w.num_blocks, 18)
    queries = torch.from_numpy(w.queries(9)).to(device)
    tables = torch.from_numpy(w.tables).to(device)
    lens = torch.from_numpy(lengths).to(device)
    plan = _hip.decode_plan(lengths, w.tables)
    first = torch.full_like(queries, 7.0)
    _hip.paged_decode_attention(first, queries, pool, 9, tables, lens, plan=torch.from_numpy(plan).to(device))
    reversed_out = torch.full_like(queries, 7.0)
    _hip.paged_decode_attention(
        reversed_out, queries, pool, 9, tables, lens, plan=torch.from_numpy(regrouped_plan(plan, list(range(7, -1, -1)))).to(device)
    )
    torch.cuda.synchronize()
    assert torch.equal(first, reversed_out)
    assert torch.equal(first[6], torch.full_like(first[6], 7.0))  # untouched
    live = [b for b in range(64) if b != 6]
    assert not torch.isnan(first[live]).any()
    device_plan = torch.from_numpy(plan).to(device)
    graph_out = torch.empty_like(queries)
    side = torch.cuda.Stream(device=device)
    side.wait_stream(torch.cuda.current_stream(device))
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.stream(side), torch.cuda.graph(graph, stream=side):
        _hip.paged_decode_attention(graph_out, queries, pool, 9, tables, lens, plan=device_plan)
    torch.cuda.current_stream(device).wait_stream(side)
    for _ in range(3):
        graph_out.fill_(float("nan"))
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(graph_out[live], first[live])
        eager = torch.empty_like(queries)
        _hip.paged_decode_attention(eager, queries, pool, 9, tables, lens, plan=device_plan)
        torch.cuda.synchronize()
        assert torch.equal(eager[live], first[live])
    w.lengths = lengths
    worst = Worst("plan order and graph replays")
    for b, (oracle, fp64) in _oracle_rows(pool, 9, w, queries, [0, 1, 2, 3, 4, 5, 40]).items():
        worst.check(first[b : b + 1].reshape(1, 32, 1, 64), oracle, fp64, f"row {b}")
    worst.report()


def test_cached_scratch_survives_changing_shapes(device):
    """Calls of different batch sizes and table widths share the cached per-stream scratch;
    each must still match the oracle."""
    pool = _random_pool(device, 1024, 17)
    for batch, hi, layer in ((3, 300, 1), (9, 1000, 2), (2, 2048, 3), (9, 900, 4)):
        w = workloads.batched_decode(batch=batch, lo=20, hi=hi, num_blocks=1024, seed=batch + hi)
        queries = torch.from_numpy(w.queries(layer)).to(device)
        out = torch.full_like(queries, float("nan"))
        _hip.paged_decode_attention(
            out, queries, pool, layer, torch.from_numpy(w.tables).to(device), torch.from_numpy(w.lengths).to(device)
        )
        torch.cuda.synchronize()
        worst = Worst(f"scratch reuse batch {batch} hi {hi}")
        for b, (oracle, fp64) in _oracle_rows(pool, layer, w, queries, range(batch)).items():
            worst.check(out[b : b + 1].reshape(1, 32, 1, 64), oracle, fp64, f"row {b}")
        worst.report()


def test_constant_values_return_the_constant(device):
    """Size-independent property at full batch: V == c everywhere gives c for any scores."""
    w = workloads.batched_decode(batch=64, num_blocks=8192, seed=45)
    pool = _random_pool(device, w.num_blocks, 13)
    pool[:, 1] = 0.375
    queries = torch.from_numpy(w.queries(0)).to(device)
    out = torch.empty_like(queries)
    _hip.paged_decode_attention(
        out, queries, pool, 0, torch.from_numpy(w.tables).to(device), torch.from_numpy(w.lengths).to(device)
    )
    torch.cuda.synchronize()
    assert torch.equal(out, torch.full_like(out, 0.375))


def test_block_table_indirection_is_invisible(device):
    """Moving a sequence's blocks to other physical ids (and permuting its table to match)
    gives bit-identical output."""
    w = workloads.batched_decode(batch=8, num_blocks=2048, seed=46)
    pool = _random_pool(device, w.num_blocks, 14)
    queries = torch.from_numpy(w.queries(3)).to(device)
    tables = torch.from_numpy(w.tables).to(device)
    lens = torch.from_numpy(w.lengths).to(device)
    first = torch.empty_like(queries)
    _hip.paged_decode_attention(first, queries, pool, 3, tables, lens)
    perm = torch.randperm(w.num_blocks, device=device)
    moved = torch.empty_like(pool)
    moved[:, :, perm] = pool  # block i now lives at perm[i]
    second = torch.empty_like(queries)
    _hip.paged_decode_attention(second, queries, moved, 3, perm[tables.long()].int(), lens)
    torch.cuda.synchronize()
    assert torch.equal(first, second)


def test_out_of_range_block_id_poisons_only_its_row(device):
    """A table entry outside the pool never reads out of bounds: that row's output is NaN,
    the other rows are unaffected, and the fault is recorded in the workspace's fault word:
    the fault check raises AttentionFaultError and clears the workspace."""
    w = workloads.batched_decode(batch=4, num_blocks=512, lo=40, hi=300, seed=47)
    pool = _random_pool(device, w.num_blocks, 15)
    queries = torch.from_numpy(w.queries(0)).to(device)
    tables = torch.from_numpy(w.tables).to(device)
    lens = torch.from_numpy(w.lengths).to(device)
    good = torch.empty_like(queries)
    workspace = _hip.paged_decode_attention(good, queries, pool, 0, tables, lens)
    assert fault_word(workspace) == 0
    broken = tables.clone()
    broken[2, 1] = w.num_blocks + 7
    bad = torch.empty_like(queries)
    assert _hip.paged_decode_attention(bad, queries, pool, 0, broken, lens) is workspace
    torch.cuda.synchronize()
    assert torch.isnan(bad[2]).all()
    for b in (0, 1, 3):
        assert torch.equal(bad[b], good[b])
    assert fault_word(workspace) == _hip.FAULT_BLOCK_ID
    with pytest.raises(_hip.AttentionFaultError, match="outside the pool"):
        _hip.check_attention_faults(workspace, "test")
    assert fault_word(workspace) == 0 and flags_clear(workspace)


def _one_token_cache(device):
    pool = torch.full((22, 2, 4, 16, 4, 64), float("nan"), dtype=torch.float16, device=device)
    allocator = KVAllocator(pool)
    request = RequestId("one")
    allocator.create(KVReservation(request, 1))
    key = torch.zeros(22, 1, 4, 64, dtype=torch.float16, device=device)
    allocator.append(request, key, key)
    return allocator, request


@pytest.mark.parametrize(
    "shape,dtype",
    [((2, 32, 1, 64), torch.float16), ((1, 31, 1, 64), torch.float16), ((1, 32, 2, 64), torch.float16),
     ((1, 32, 1, 63), torch.float16), ((1, 32, 1, 64), torch.float32)],
)
@pytest.mark.parametrize("api", ["paged_attention", "paged_attention_batch"])
def test_rejects_invalid_queries(device, shape, dtype, api):
    """The reference's query checks (tests/unit/test_attention.py:353-368) on a gfx950 pool,
    through both entry points: ValueError("query must be FP16 ..."), raised before any launch,
    with the allocator's counts, table and length unchanged."""
    allocator, request = _one_token_cache(device)
    before = (allocator.capacity(), allocator.block_table(request), allocator.cached_length(request))
    query = torch.zeros(shape, dtype=dtype, device=device)
    with pytest.raises(ValueError, match="query must be FP16"):
        if api == "paged_attention":
            paged_attention(query, allocator, request, layer_index=0)
        else:
            paged_attention_batch(query, allocator, (request,), layer_index=0)
    assert (allocator.capacity(), allocator.block_table(request), allocator.cached_length(request)) == before


@pytest.mark.parametrize("layer", [-1, 22, True, 1.0])
@pytest.mark.parametrize("api", ["paged_attention", "paged_attention_batch"])
def test_rejects_invalid_layers(device, layer, api):
    """tests/unit/test_attention.py:371-376 on a gfx950 pool: a layer index that is not an
    int in [0, 22) (bool and float included) raises ValueError naming layer_index."""
    allocator, request = _one_token_cache(device)
    before = allocator.capacity()
    query = torch.zeros(1, 32, 1, 64, dtype=torch.float16, device=device)
    with pytest.raises(ValueError, match="layer_index"):
        if api == "paged_attention":
            paged_attention(query, allocator, request, layer_index=layer)
        else:
            paged_attention_batch(query, allocator, (request,), layer_index=layer)
    assert allocator.capacity() == before


@pytest.mark.parametrize("api", ["paged_attention", "paged_attention_batch"])
def test_rejects_a_query_on_another_device(device, api):
    """tests/unit/test_attention.py:379-384 on a gfx950 pool: a host query (the pool is on
    the GPU) raises ValueError("... same device"), with the counts unchanged; the same
    query on the pool's device then succeeds."""
    allocator, request = _one_token_cache(device)
    before = allocator.capacity()
    for query in (torch.zeros(1, 32, 1, 64, dtype=torch.float16),
                  torch.empty(1, 32, 1, 64, dtype=torch.float16, device="meta")):
        with pytest.raises(ValueError, match="same device"):
            if api == "paged_attention":
                paged_attention(query, allocator, request, layer_index=0)
            else:
                paged_attention_batch(query, allocator, (request,), layer_index=0)
        assert allocator.capacity() == before
    good = torch.zeros(1, 32, 1, 64, dtype=torch.float16, device=device)
    out = paged_attention(good, allocator, request, layer_index=0)
    assert out.device == good.device and torch.equal(out, torch.zeros_like(out))  # V = 0 everywhere


def test_batched_api_matches_single_request_api(device):
    pool = torch.full((22, 2, 40, 16, 4, 64), float("nan"), dtype=torch.float16, device=device)
    allocator = KVAllocator(pool)
    gen = torch.Generator(device=device).manual_seed(3)
    requests = []
    for index, tokens in enumerate((1, 16, 17, 100, 300)):
        key = torch.randn(22, tokens, 4, 64, dtype=torch.float16, device=device, generator=gen)
        value = torch.randn(22, tokens, 4, 64, dtype=torch.float16, device=device, generator=gen)
        request = RequestId(f"r{index}")
        allocator.create(KVReservation(request, (tokens + 15) // 16))
        allocator.append(request, key, value)
        requests.append(request)
    query = torch.randn(5, 32, 1, 64, dtype=torch.float16, device=device, generator=gen)
    batched = paged_attention_batch(query, allocator, requests, layer_index=4)
    for row, request in enumerate(requests):
        single = paged_attention(query[row : row + 1], allocator, request, layer_index=4)
        assert torch.equal(single, batched[row : row + 1])




def _permuted_tables(lengths, num_blocks, seed):
    need = [(int(x) + 15) // 16 for x in lengths]
    perm = np.random.default_rng(seed).permutation(num_blocks).astype(np.int32)
    tables = np.zeros((len(lengths), max(max(need), 1)), dtype=np.int32)
    offset = 0
    for b, n in enumerate(need):
        tables[b, :n] = perm[offset : offset + n]
        offset += n
    return tables


@pytest.mark.parametrize(
    "lengths,num_blocks",
    [
        ([32768 - 5], 2100),  # one sequence: 256 bins of one group, merged from 256 parts
        ([20000, 1, 5000, 16, 17, 8191], 2400),
    ],
    ids=["one-sequence", "mixed"],
)
def test_long_sequences_cut_over_many_bins(device, lengths, num_blocks):
    """Sequences far longer than a bin: every part but the last goes through the workspace
    and the last bin folds up to 255 of them. Every row within 2e-3 of FP64, two calls on
    the same workspace give the same bits, and both leave the part flags at zero."""
    lengths = np.asarray(lengths, dtype=np.int32)
    _say("long sequences", lengths.tolist())
    tables = _permuted_tables(lengths, num_blocks, 81)
    stats = check_decode_plan(_hip.decode_plan(lengths, tables), lengths, tables, num_blocks,
                              _hip.workspace_bytes(len(lengths), tables.shape[1]))
    assert stats["cut"] >= 1
    pool = _random_pool(device, num_blocks, 19)
    layer = 13
    gen = torch.Generator(device=device).manual_seed(7)
    queries = torch.randn((len(lengths), 32, 64), dtype=torch.float16, device=device, generator=gen)
    workspace = torch.zeros(_hip.workspace_bytes(len(lengths), tables.shape[1]), dtype=torch.uint8, device=device)
    outs = []
    for _ in range(2):
        out = torch.full_like(queries, float("nan"))
        _hip.paged_decode_attention(out, queries, pool, layer, torch.from_numpy(tables).to(device),
                                    torch.from_numpy(lengths).to(device), workspace=workspace)
        torch.cuda.synchronize()
        assert flags_clear(workspace)
        outs.append(out)
    assert torch.equal(outs[0], outs[1])
    worst = Worst(f"long sequences {lengths.tolist()}")
    fp64 = _fp64_all_rows(pool, layer, tables, lengths, queries, chunk=1)
    for b in range(len(lengths)):
        worst.check(outs[0][b], None, fp64[b], f"row {b} len {lengths[b]}")
    worst.report()


def test_many_short_sequences_close_bins_early(device):
    """1000 sequences of 1..48 tokens: a bin closes at 4 sequences before its nominal end,
    so the plan has more bins than CUs. Every row within 2e-3 of FP64, sampled rows of the
    oracle."""
    rng = np.random.default_rng(82)
    lengths = rng.integers(1, 49, size=1000).astype(np.int32)
    lengths[:4] = [1, 16, 17, 48]
    num_blocks = 3000
    tables = _permuted_tables(lengths, num_blocks, 83)
    plan = _hip.decode_plan(lengths, tables)
    stats = check_decode_plan(plan, lengths, tables, num_blocks, _hip.workspace_bytes(len(lengths), tables.shape[1]))
    assert stats["rows"] > 256 and (plan[:, 0] == 4).sum() > 0
    _say("many short sequences", stats)
    pool = _random_pool(device, num_blocks, 20)
    w = workloads.BatchedDecode(lengths, tables, num_blocks, 84)
    queries = torch.from_numpy(w.queries(2)).to(device)
    out = torch.full_like(queries, float("nan"))
    _hip.paged_decode_attention(out, queries, pool, 2, torch.from_numpy(tables).to(device),
                                torch.from_numpy(lengths).to(device), plan=torch.from_numpy(plan).to(device))
    torch.cuda.synchronize()
    worst = Worst("1000 short sequences")
    fp64 = _fp64_all_rows(pool, 2, tables, lengths, queries)
    for b in range(len(lengths)):
        worst.check(out[b], None, fp64[b], f"row {b} len {lengths[b]}")
    for b, (oracle, _) in _oracle_rows(pool, 2, w, queries, [0, 1, 2, 3, 500, 999]).items():
        worst.oracle = max(worst.oracle, assert_max_abs(out[b : b + 1].reshape(1, 32, 1, 64), oracle, f"row {b} vs oracle"))
    worst.report()


@pytest.mark.parametrize("where", ["first part", "middle part", "last part"])
def test_bad_block_in_a_cut_sequence_poisons_only_its_row(device, where):
    """An out-of-pool id in one part of a sequence cut over three or more bins: the merged
    row is NaN, every other row (including those sharing its bins) keeps its bits, and the
    part flags end at zero."""
    w = workloads.batched_decode(batch=64, num_blocks=8192, seed=85)
    plan = _hip.decode_plan(w.lengths, w.tables)
    spans = {}
    for r in range(plan.shape[0]):
        for s in range(int(plan[r, 0])):
            b, _, j0, n, _, kidx, nspan, _ = (int(v) for v in plan[r, 8 + 8 * s : 16 + 8 * s])
            if nspan >= 3:
                spans.setdefault(b, {})[kidx] = (j0, n, nspan)
    assert spans, "the workload cuts no sequence over three bins"
    b = min(spans)
    nspan = spans[b][0][2]
    kidx = {"first part": 0, "middle part": 1, "last part": nspan - 1}[where]
    j0, n, _ = spans[b][kidx]
    _say("bad block in", where, "of row", b, "parts", nspan, "block", j0 + n // 2)
    pool = _random_pool(device, w.num_blocks, 21)
    queries = torch.from_numpy(w.queries(6)).to(device)
    lens = torch.from_numpy(w.lengths).to(device)
    workspace = torch.zeros(_hip.workspace_bytes(w.batch, w.tables.shape[1]), dtype=torch.uint8, device=device)
    good = torch.empty_like(queries)
    _hip.paged_decode_attention(good, queries, pool, 6, torch.from_numpy(w.tables).to(device), lens, workspace=workspace)
    assert fault_word(workspace) == 0
    broken = w.tables.copy()
    broken[b, j0 + n // 2] = w.num_blocks + 3
    bad = torch.empty_like(queries)
    _hip.paged_decode_attention(bad, queries, pool, 6, torch.from_numpy(broken).to(device), lens, workspace=workspace)
    torch.cuda.synchronize()
    assert torch.isnan(bad[b]).all()
    others = [x for x in range(w.batch) if x != b]
    assert torch.equal(bad[others], good[others])
    assert not torch.isnan(good).any()
    assert flags_clear(workspace)
    assert fault_word(workspace) == _hip.FAULT_BLOCK_ID


def _spans(plan):
    """{sequence: {part: (row, segment index, first block, blocks, parts)}} of a plan's cut
    sequences."""
    spans = {}
    for r in range(plan.shape[0]):
        for s in range(int(plan[r, 0])):
            b, _, j0, n, _, kidx, nspan, _ = (int(v) for v in plan[r, 8 + 8 * s : 16 + 8 * s])
            if nspan > 1:
                spans.setdefault(b, {})[kidx] = (r, s, j0, n, nspan)
    return spans


@pytest.mark.parametrize(
    "fault", ["missing earlier part", "missing merging part", "slots outside the workspace", "sequence outside the batch"]
)
def test_malformed_plans_stay_in_bounds_and_spoil_only_their_rows(device, fault):
    """Plans that do not match the batch: a cut sequence whose earlier part's row was
    dropped (its merge waits out its bounded spin, writes NaN and records
    PC_ATTN_FAULT_MERGE_TIMEOUT, which the fault check turns into AttentionFaultError), a cut
    sequence whose merging row was dropped (its earlier parts' flags stay raised; the row is
    never written), a cut sequence whose partial slots point past the workspace (neither
    stored nor merged: its row is left alone), a complete sequence relabelled past the batch
    (not written). Every other row keeps the bits of the intact plan. The part flags end at
    zero, except those of the dropped merge: a later call with a new plan on the same
    workspace ignores them (they carry the old plan's epoch) and gives the intact plan's bits."""
    w = workloads.batched_decode(batch=64, num_blocks=8192, seed=86)
    plan = _hip.decode_plan(w.lengths, w.tables)
    spans = _spans(plan)
    assert spans
    pool = _random_pool(device, w.num_blocks, 22)
    queries = torch.from_numpy(w.queries(8)).to(device)
    lens = torch.from_numpy(w.lengths).to(device)
    tables = torch.from_numpy(w.tables).to(device)
    workspace = torch.zeros(_hip.workspace_bytes(w.batch, w.tables.shape[1]), dtype=torch.uint8, device=device)
    good = torch.full_like(queries, 7.0)
    _hip.paged_decode_attention(good, queries, pool, 8, tables, lens, workspace=workspace)
    bad_plan = plan.copy()
    merger_dropped = set()
    if fault == "missing earlier part":
        b = min(spans)
        row = spans[b][0][0]
        bad_plan[row] = 0  # the whole bin is dropped: every sequence it touches is spoiled
        spoiled = {int(x) for x in plan[row, 8 : 8 + 8 * int(plan[row, 0]) : 8]}
        nan_rows = {x for x in spoiled if x in spans}
    elif fault == "missing merging part":
        # a sequence whose merging bin holds no earlier part of another sequence, so that no
        # merge times out and the flags it leaves raised meet the next call
        def merging_row(x):
            return spans[x][max(spans[x])][0]

        def ends_with_earlier_part(row):
            last = 8 + 8 * (int(plan[row, 0]) - 1)
            return plan[row, last + 6] > 1 and plan[row, last + 5] < plan[row, last + 6] - 1

        b = min((x for x in spans if not ends_with_earlier_part(merging_row(x))), default=min(spans))
        row = merging_row(b)  # the bin holding the sequence's last part
        bad_plan[row] = 0
        spoiled = {int(x) for x in plan[row, 8 : 8 + 8 * int(plan[row, 0]) : 8]}
        # sequences whose merging part was in the dropped bin: their earlier parts stay flagged
        merger_dropped = {x for x in spoiled if x in spans and spans[x][max(spans[x])][0] == row}
        assert b in merger_dropped
        # an earlier part of another sequence in the dropped bin makes that sequence's merge time out
        nan_rows = {x for x in spoiled if x in spans and x not in merger_dropped}
    elif fault == "slots outside the workspace":
        b = min(spans)
        for row, s, _, _, _ in spans[b].values():
            bad_plan[row, 8 + 8 * s + 7] = 1 << 30
        spoiled, nan_rows = {b}, set()
    else:
        complete = [int(plan[r, 8 + 8 * s]) for r in range(plan.shape[0]) for s in range(int(plan[r, 0]))
                    if plan[r, 8 + 8 * s + 6] == 1]
        assert complete, "the workload has no sequence complete within one bin"
        b = complete[0]
        for r in range(plan.shape[0]):
            for s in range(int(plan[r, 0])):
                if plan[r, 8 + 8 * s] == b:
                    bad_plan[r, 8 + 8 * s] = w.batch + 5
        spoiled, nan_rows = {b}, set()
    _say("malformed plan:", fault, "spoiled rows", sorted(spoiled))
    bad = torch.full_like(queries, 7.0)
    _hip.paged_decode_attention(bad, queries, pool, 8, tables, lens, plan=torch.from_numpy(bad_plan).to(device),
                                workspace=workspace)
    torch.cuda.synchronize()
    others = [x for x in range(w.batch) if x not in spoiled]
    assert torch.equal(bad[others], good[others])
    for x in nan_rows:
        assert torch.isnan(bad[x]).all(), x
    for x in spoiled - nan_rows if fault != "missing earlier part" else ():
        assert torch.equal(bad[x], torch.full_like(bad[x], 7.0)), x  # never written
    raised = int((workspace_flags(workspace) != 0).sum().item())
    if merger_dropped:
        assert raised > 0, "the dropped merge's earlier parts should still be flagged"
        _say("flags left raised by the dropped merge:", raised)
    else:
        assert raised == 0
    expected_fault = _hip.FAULT_MERGE_TIMEOUT if nan_rows else 0
    assert fault_word(workspace) == expected_fault
    if expected_fault:
        with pytest.raises(_hip.AttentionFaultError, match="bounded wait"):
            _hip.check_attention_faults(workspace, "test")
        assert fault_word(workspace) == 0 and flags_clear(workspace)  # zeroed whole
    if merger_dropped:
        # a new plan (new epoch) of the same batch on the same workspace: the old flags are not taken
        again = torch.full_like(queries, 7.0)
        _hip.paged_decode_attention(again, queries, pool, 8, tables, lens, workspace=workspace)
        torch.cuda.synchronize()
        assert torch.equal(again, good)
        assert fault_word(workspace) == 0
    assert flags_clear(workspace)


@pytest.mark.parametrize("stale", ["earlier epoch", "other layer"])
def test_stale_raised_flags_are_not_taken(device, stale):
    """Flags left raised in the workspace by an earlier call (planted here from the host in
    every partial slot, with garbage partials: an earlier plan's epoch, or this plan's epoch
    and another layer, with every XCD id) are never taken for this call's parts: the output
    equals a call on a clean workspace bit for bit, no fault is recorded, and every flag ends
    at zero."""
    w = workloads.batched_decode(batch=64, num_blocks=8192, seed=87)
    plan = _hip.decode_plan(w.lengths, w.tables)
    assert _spans(plan)
    epoch, layer = int(plan[0, 2]), 5
    pool = _random_pool(device, w.num_blocks, 23)
    queries = torch.from_numpy(w.queries(layer)).to(device)
    lens = torch.from_numpy(w.lengths).to(device)
    tables = torch.from_numpy(w.tables).to(device)
    device_plan = torch.from_numpy(plan).to(device)
    nbytes = _hip.workspace_bytes(w.batch, w.tables.shape[1])
    clean = torch.zeros(nbytes, dtype=torch.uint8, device=device)
    expected = torch.full_like(queries, 7.0)
    _hip.paged_decode_attention(expected, queries, pool, layer, tables, lens, plan=device_plan, workspace=clean)
    planted = torch.randint(0, 256, (nbytes,), dtype=torch.uint8, device=device,
                            generator=torch.Generator(device=device).manual_seed(88))
    planted[:256] = 0  # the fault word starts clear
    slots = (nbytes - 256) // 2176
    if stale == "earlier epoch":
        key = (((epoch - 1) & ((1 << 22) - 1)) << 9) | (layer << 4)
    else:
        key = (epoch << 9) | (((layer + 1) % 22) << 4)
    xcc = torch.arange(slots, dtype=torch.int32, device=device) % 8 + 1
    flags = (key | xcc).view(torch.uint8).view(slots, 4)
    planted[256 : 256 + slots * 2176].view(slots, 2176)[:, 2112:2116] = flags
    assert (workspace_flags(planted) != 0).all()
    got = torch.full_like(queries, 7.0)
    _hip.paged_decode_attention(got, queries, pool, layer, tables, lens, plan=device_plan, workspace=planted)
    torch.cuda.synchronize()
    assert torch.equal(got.view(torch.int16), expected.view(torch.int16))
    assert fault_word(planted) == 0 and fault_word(clean) == 0
    # the slots the plan uses were consumed and lowered; the others keep their planted flags
    used = check_decode_plan(plan, w.lengths, w.tables, w.num_blocks, nbytes)["slots"]
    assert int((workspace_flags(planted) == 0).sum().item()) == used * 4
