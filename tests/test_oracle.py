"""Pins the CPU oracle before anything is checked against it.

Each check below comes from the reference's own tests (known answers and FP64 agreement,
cited per test) or from mathematics (closed forms, brute force). The last group plants
plausible mistakes in the oracle and shows the checks catch them.
"""

from __future__ import annotations

import math

import numpy as np
import pytest
import torch

from oracle import paged_reference as ref

pytestmark = []


def _pool_with(key: torch.Tensor, value: torch.Tensor, blocks, layer: int = 0, spare: int = 1):
    """NaN-poisoned CPU pool holding key/value [tokens, 4, 64] at `blocks` of `layer`."""
    n = max(blocks) + 1 + spare
    pool = torch.full((22, 2, n, 16, 4, 64), float("nan"), dtype=torch.float16)
    for logical, physical in enumerate(blocks):
        chunk = slice(logical * 16, min(key.shape[0], logical * 16 + 16))
        valid = chunk.stop - chunk.start
        pool[layer, 0, physical, :valid] = key[chunk]
        pool[layer, 1, physical, :valid] = value[chunk]
    return pool


def _attend(query, key, value, blocks=None, layer=0, attention=ref.reference_paged_attention):
    blocks = blocks if blocks is not None else list(range((key.shape[0] + 15) // 16))
    pool = _pool_with(key, value, blocks, layer)
    return attention(query, pool, layer, blocks, key.shape[0]), pool


def _fp64_half(query, key, value):
    return ref.dense_attention_fp64(query, key, value).reshape(1, 32, 1, 64).half()


# --- FP64 oracle: closed forms and brute force ------------------------------------------


def test_fp64_oracle_zero_query_gives_mean_of_values():
    gen = torch.Generator().manual_seed(1)
    key = torch.randn(37, 4, 64, generator=gen).half()
    value = torch.randn(37, 4, 64, generator=gen).half()
    out = ref.dense_attention_fp64(torch.zeros(1, 32, 1, 64), key, value)
    expected = value.double().mean(dim=0)  # [4, 64]
    for head in range(32):
        torch.testing.assert_close(out[head], expected[head // 8], atol=1e-14, rtol=0)


def test_fp64_oracle_dominant_key_selects_its_value():
    key = torch.zeros(5, 4, 64, dtype=torch.float16)
    key[3, :, 0] = 100.0  # score 100*q0/8 dominates by e^-125 relative
    value = torch.arange(5 * 4 * 64, dtype=torch.float32).reshape(5, 4, 64).half()
    query = torch.zeros(1, 32, 1, 64, dtype=torch.float16)
    query[..., 0] = 10.0
    out = ref.dense_attention_fp64(query, key, value)
    for head in range(32):
        torch.testing.assert_close(out[head], value[3, head // 8].double(), atol=1e-9, rtol=0)


def test_fp64_oracle_matches_pure_python_brute_force():
    gen = torch.Generator().manual_seed(2)
    key = torch.randn(3, 4, 64, generator=gen).half()
    value = torch.randn(3, 4, 64, generator=gen).half()
    query = torch.randn(1, 32, 1, 64, generator=gen).half()
    out = ref.dense_attention_fp64(query, key, value)
    q = query.reshape(32, 64).tolist()
    k = key.tolist()
    v = value.tolist()
    for head in (0, 7, 8, 31):
        group = head // 8
        scores = [sum(q[head][d] * k[t][group][d] for d in range(64)) / 8 for t in range(3)]
        top = max(scores)
        weights = [math.exp(s - top) for s in scores]
        total = sum(weights)
        for d in (0, 13, 63):
            expected = sum(weights[t] * v[t][group][d] for t in range(3)) / total
            assert abs(out[head, d].item() - expected) < 1e-12


# --- Paged restatement: the reference tests' known answers -------------------------------


def test_normalizes_all_scores_before_page_value_products():
    # tests/unit/test_attention.py:182-221: q = 0, V = 2 on a full page and 19 on one
    # token of the next page (tables (0, 2)); every weight is 1/17, the output exactly 3.
    key = torch.zeros(17, 4, 64, dtype=torch.float16)
    value = torch.zeros_like(key)
    value[:16], value[16:] = 2, 19
    out, pool = _attend(torch.zeros(1, 32, 1, 64, dtype=torch.float16), key, value, blocks=[0, 2])
    before = pool.clone()
    assert torch.equal(out, torch.full_like(out, 3))
    torch.testing.assert_close(pool, before, atol=0, rtol=0, equal_nan=True)


def test_maps_eight_query_heads_to_each_kv_head():
    # tests/unit/test_attention.py:281-302: V[:, h] = 100 h + t over 33 tokens, q = 0.
    key = torch.zeros(33, 4, 64, dtype=torch.float16)
    value = torch.zeros_like(key)
    for head in range(4):
        value[:, head] = (100 * head + torch.arange(33))[:, None]
    out, _ = _attend(torch.zeros(1, 32, 1, 64, dtype=torch.float16), key, value, layer=21)
    for head in range(32):
        assert torch.equal(out[0, head, 0], torch.full((64,), 100 * (head // 8) + 16).half())


def test_rounds_only_after_value_cancellation_across_pages():
    # tests/unit/test_attention.py:245-259: exactly 0.25.
    key = torch.zeros(32, 4, 64, dtype=torch.float16)
    value = torch.zeros_like(key)
    value[0], value[1], value[16] = 32768, 8, -32768
    out, _ = _attend(torch.zeros(1, 32, 1, 64, dtype=torch.float16), key, value)
    assert torch.equal(out, torch.full_like(out, 0.25))


def test_retains_tiny_probabilities_until_value_accumulation():
    # tests/unit/test_attention.py:224-242.
    key = torch.zeros(17, 4, 64, dtype=torch.float16)
    key[:, :, 0] = -160
    key[0, :, 0] = 0
    value = torch.full_like(key, 65504)
    value[0] = 0
    query = torch.zeros(1, 32, 1, 64, dtype=torch.float16)
    query[..., 0] = 1
    out, _ = _attend(query, key, value)
    assert (out > 0).all()
    torch.testing.assert_close(out, _fp64_half(query, key, value), atol=1e-6, rtol=2e-3)


@pytest.mark.parametrize("tokens,layer", [(1, 0), (15, 21), (16, 7), (17, 0), (49, 21), (2048, 11)])
def test_matches_fp64_at_cache_boundaries(tokens, layer):
    # tests/unit/test_attention.py:262-278.
    gen = torch.Generator().manual_seed(tokens)
    key = torch.randn(tokens, 4, 64, generator=gen).half()
    value = torch.randn(tokens, 4, 64, generator=gen).half()
    query = torch.randn(1, 32, 1, 128, generator=gen).half()[..., ::2]
    blocks = torch.randperm((tokens + 15) // 16 + 3, generator=gen)[: (tokens + 15) // 16].tolist()
    out, _ = _attend(query, key, value, blocks=blocks, layer=layer)
    torch.testing.assert_close(out, _fp64_half(query, key, value), atol=2e-3, rtol=2e-3)


@pytest.mark.parametrize("reverse", [False, True])
@pytest.mark.parametrize("query_scale", [1.0, 1000.0])
def test_rescales_softmax_across_large_block_scores(reverse, query_scale):
    # tests/unit/test_attention.py:305-322.
    key = torch.full((49, 4, 64), -1000.0, dtype=torch.float16)
    key[16:32] = 0
    key[32:] = 1000
    value = torch.randn_like(key)
    if reverse:
        key, value = key.flip(0), value.flip(0)
    query = torch.full((1, 32, 1, 64), query_scale, dtype=torch.float16)
    out, _ = _attend(query, key, value)
    assert torch.isfinite(out).all()
    torch.testing.assert_close(out, _fp64_half(query, key, value), atol=2e-3, rtol=2e-3)


def test_ignores_autocast():
    # tests/unit/test_attention.py:325-335.
    gen = torch.Generator().manual_seed(3)
    key = torch.randn(49, 4, 64, generator=gen).half()
    value = torch.randn(49, 4, 64, generator=gen).half()
    query = torch.randn(1, 32, 1, 64, generator=gen).half()
    plain, _ = _attend(query, key, value)
    with torch.autocast("cpu", dtype=torch.bfloat16):
        auto, _ = _attend(query, key, value)
    assert torch.equal(plain, auto)


def test_config1_golden_fixture():
    """Single-sequence 128-token layer on a seeded random 8-entry table of a 64-block pool:
    the committed FP64 output pins the restatement at 2e-3 (tests/golden/make_golden.py)."""
    data = np.load(_golden("config1_single_decode.npz"))
    query = torch.from_numpy(data["query"].view(np.float16)).reshape(1, 32, 1, 64)
    key = torch.from_numpy(data["key"].view(np.float16))
    value = torch.from_numpy(data["value"].view(np.float16))
    blocks = data["table"].tolist()
    expected = torch.from_numpy(data["expected_fp64"])
    torch.testing.assert_close(ref.dense_attention_fp64(query, key, value), expected, atol=0, rtol=0)
    out, _ = _attend(query, key, value, blocks=blocks, layer=int(data["layer"]))
    torch.testing.assert_close(out, expected.reshape(1, 32, 1, 64).half(), atol=2e-3, rtol=2e-3)


def _golden(name: str) -> str:
    import os

    return os.path.join(os.path.dirname(__file__), "golden", name)


# --- Append and block choice --------------------------------------------------------------


def _kv_bits(tokens: int, start: int = 0):
    key = torch.arange(22 * tokens * 4 * 64, dtype=torch.float32).reshape(22, tokens, 4, 64)
    key = (key / 256 + start).half()
    return ref.f16_bits(key), ref.f16_bits(-key - 1)


def test_append_satisfies_the_slot_closed_form_and_leaves_other_slots():
    pool = np.full((22, 2, 6, 16, 4, 64), ref.NAN_F16_BITS, dtype=np.uint16)
    blocks = [4, 1, 3]
    key, value = _kv_bits(40)
    ref.reference_append(pool, blocks, 0, key[:, :15], value[:, :15])
    ref.reference_append(pool, blocks, 15, key[:, 15:], value[:, 15:])
    touched = np.zeros((6, 16), dtype=bool)
    for p in range(40):
        block, slot = blocks[p // 16], p % 16
        assert np.array_equal(pool[:, 0, block, slot], key[:, p])
        assert np.array_equal(pool[:, 1, block, slot], value[:, p])
        touched[block, slot] = True
    assert (pool[:, :, ~touched] == ref.NAN_F16_BITS).all()


def test_free_list_reproduces_the_reference_tables():
    # tests/unit/test_kv_cache.py:186-205: a appends 15, b 16, a 1, a 1, a 16 tokens.
    lifo = ref.LifoFreeList.fresh(4)
    lifo.grow_to("a", 15)
    lifo.grow_to("b", 16)
    lifo.grow_to("a", 16)
    lifo.grow_to("a", 17)
    lifo.grow_to("a", 33)
    assert lifo.tables == {"a": [0, 2, 3], "b": [1]}

    # tests/unit/test_decoder.py:439-465: three one-block requests, release first and last,
    # then a prompt of up to 49 tokens gets (2, 0, 3, 4).
    lifo = ref.LifoFreeList.fresh(6)
    for name in ("released_first", "retained", "released_last"):
        lifo.grow_to(name, 16)
    lifo.release("released_first")
    lifo.release("released_last")
    assert lifo.grow_to("prompt", 49) == [2, 0, 3, 4]

    # tests/unit/test_attention.py:182-197: request 16 tokens, blocker 16, request +1 -> (0, 2).
    lifo = ref.LifoFreeList.fresh(3)
    lifo.grow_to("normalized", 16)
    lifo.grow_to("blocker", 16)
    lifo.grow_to("normalized", 17)
    assert lifo.tables["normalized"] == [0, 2]


def test_decode_step_borrows_the_free_tail_in_request_order():
    # tests/unit/test_kv_cache.py:344-382: two 16-token requests on a 4-block pool each take
    # one block in the staged step; the pool ends fully owned (CapacityCounts(4,0,4,4,2,34)).
    lifo = ref.LifoFreeList.fresh(4)
    lifo.grow_to("first", 16)
    lifo.grow_to("second", 16)
    tables = lifo.decode_step({"first": 16, "second": 16})
    assert tables == {"first": [0, 2], "second": [1, 3]}
    assert lifo.free == []


# --- Planted mistakes: the checks above must catch them -----------------------------------


def _wrong_head_mapping(query, pool, layer, blocks, length):
    # q head h -> kv head h % 4 instead of h // 8
    q = query.reshape(32, 64)
    q = q.reshape(8, 4, 64).transpose(0, 1).reshape(1, 32, 1, 64)
    return ref.reference_paged_attention(q, pool, layer, blocks, length)


def _missing_scale(query, pool, layer, blocks, length):
    return ref.reference_paged_attention((query.float() * 8).half(), pool, layer, blocks, length)


def _transposed_page(query, pool, layer, blocks, length):
    flipped = pool.clone()
    flipped[layer, 0] = pool[layer, 0].flip(1)  # tokens of each key page reversed
    return ref.reference_paged_attention(query, flipped, layer, blocks, length)


@pytest.mark.parametrize("mistake", [_wrong_head_mapping, _missing_scale, _transposed_page])
def test_planted_attention_mistakes_are_caught(mistake):
    gen = torch.Generator().manual_seed(5)
    key = torch.randn(33, 4, 64, generator=gen).half()
    value = torch.randn(33, 4, 64, generator=gen).half()
    query = torch.randn(1, 32, 1, 64, generator=gen).half()
    expected = _fp64_half(query, key, value)
    correct, _ = _attend(query, key, value)
    assert torch.allclose(correct.float(), expected.float(), atol=2e-3, rtol=2e-3)
    wrong, _ = _attend(query, key, value, attention=mistake)
    assert not torch.allclose(wrong.float(), expected.float(), atol=2e-3, rtol=2e-3)


def test_planted_fifo_free_list_is_caught():
    lifo = ref.LifoFreeList(list(range(4)))  # FIFO order: hands out 3, 2, ... first
    lifo.grow_to("a", 15)
    lifo.grow_to("b", 16)
    lifo.grow_to("a", 33)
    assert lifo.tables != {"a": [0, 2, 3], "b": [1]}


# --- The decode write (kv_cache.py:242-245) ------------------------------------------------


def _write_decode_changes(write, length, layer=7, num_blocks=9):
    """Flat pool indices a decode write changes, for a seeded pool and a 130-entry table
    (enough entries past the sequence that a misplaced write still lands in the pool)."""
    rng = np.random.default_rng(length)
    pool = rng.integers(0, 0x7C00, size=(22, 2, num_blocks, 16, 4, 64), dtype=np.uint16)
    before = pool.copy()
    blocks = [int(b) for b in rng.integers(0, num_blocks, size=130)]
    key = rng.integers(0x7C00, 0x7E00, size=(4, 64), dtype=np.uint16)  # values not in the pool
    value = key ^ 0x0100
    write(pool, layer, blocks, length, key, value)
    changed = np.flatnonzero(pool != before)
    return pool, blocks, key, value, changed


@pytest.mark.parametrize("length", [1, 15, 16, 17, 32, 33, 2047, 2048])
def test_write_decode_satisfies_the_element_closed_form(length):
    """The staged token of a length-L sequence goes to position L - 1: element
    (((layer * 2 + kind) * N + blocks[(L - 1) // 16]) * 16 + (L - 1) % 16) * 256 + h * 64 + d
    of the flat pool for kind 0 (key) and 1 (value), and nothing else changes."""
    layer, num_blocks = 7, 9
    pool, blocks, key, value, changed = _write_decode_changes(ref.reference_write_decode, length, layer, num_blocks)
    block = blocks[(length - 1) // 16]
    slot = (length - 1) % 16
    expected = []
    for kind in (0, 1):
        base = (((layer * 2 + kind) * num_blocks + block) * 16 + slot) * 256
        expected.extend(range(base, base + 256))
    flat = pool.reshape(-1)
    assert np.array_equal(flat[np.asarray(expected[:256])], key.reshape(-1))
    assert np.array_equal(flat[np.asarray(expected[256:])], value.reshape(-1))
    assert set(changed.tolist()) <= set(expected)  # a byte equal to its old value may not show


@pytest.mark.parametrize("shift", [-1, 1])
def test_planted_write_decode_off_by_one_is_caught(shift):
    """Writing position L or L - 2 instead of L - 1 fails the closed form at every length."""

    def planted(pool, layer, blocks, length, key, value):
        ref.reference_write_decode(pool, layer, blocks, length + shift, key, value)

    for length in (2, 16, 17, 33):
        with pytest.raises(AssertionError):
            layer, num_blocks = 7, 9
            pool, blocks, key, value, changed = _write_decode_changes(planted, length, layer, num_blocks)
            block, slot = blocks[(length - 1) // 16], (length - 1) % 16
            base = (((layer * 2) * num_blocks + block) * 16 + slot) * 256
            assert np.array_equal(pool.reshape(-1)[base : base + 256], key.reshape(-1))


# --- Allocator bookkeeping (kv_cache.py:314-357) ----------------------------------------------


class _Model:
    """Bookkeeping driven through the restated LIFO rules, checked by the restated
    _assert_accounting after each step."""

    def __init__(self, total):
        self.total = total
        self.lifo = ref.LifoFreeList.fresh(total)
        self.sequences, self.owners = {}, {}

    def create(self, rid, credits):
        self.sequences[rid] = ref.SequenceRecord(rid, credits, 0, ())

    def append(self, rid, tokens):
        old = self.sequences[rid]
        new = self.lifo.grow_to(rid, old.length + tokens)
        for block in new:
            self.owners[block] = rid
        self.sequences[rid] = ref.SequenceRecord(rid, old.credits, old.length + tokens, old.blocks + tuple(new))

    def release(self, rid):
        for block in self.sequences.pop(rid).blocks:
            del self.owners[block]
        self.lifo.release(rid)

    def counts(self):
        return ref.reference_assert_accounting(self.sequences, self.lifo.free, self.owners, self.total)


def test_accounting_reproduces_the_reference_counts():
    # tests/unit/test_kv_cache.py:453-483
    m = _Model(8)
    assert m.counts() == (8, 8, 0, 0, 0, 0)
    m.create("a", 3)
    assert m.counts() == (8, 8, 0, 3, 1, 0)
    m.create("b", 2)
    assert m.counts() == (8, 8, 0, 5, 2, 0)
    for rid, tokens, expected in (
        ("a", 15, (8, 7, 1, 5, 2, 15)),
        ("b", 16, (8, 6, 2, 5, 2, 31)),
        ("a", 1, (8, 6, 2, 5, 2, 32)),
        ("a", 1, (8, 5, 3, 5, 2, 33)),
        ("a", 16, (8, 4, 4, 5, 2, 49)),
    ):
        m.append(rid, tokens)
        assert m.counts() == expected
    m.release("a")
    assert m.counts() == (8, 7, 1, 2, 1, 16)
    m.release("b")
    assert m.counts() == (8, 8, 0, 0, 0, 0)
    # tests/unit/test_kv_cache.py:344-382: a staged decode step that borrows one block for
    # each of two 16-token requests leaves the pool fully owned, 34 live slots
    m = _Model(4)
    for rid in ("first", "second"):
        m.create(rid, 2)
        m.append(rid, 16)
    tables = m.lifo.decode_step({"first": 16, "second": 16})
    for rid in ("first", "second"):
        m.sequences[rid] = ref.SequenceRecord(rid, 2, 17, tuple(tables[rid]))
        for block in tables[rid]:
            m.owners[block] = rid
    assert m.counts() == (4, 0, 4, 4, 2, 34)


def _corrupted(kind):
    m = _Model(6)
    m.create("a", 3)
    m.append("a", 17)
    m.create("b", 1)
    m.append("b", 5)
    a = m.sequences["a"]
    if kind == "table":
        m.sequences["a"] = ref.SequenceRecord("a", 3, 40, a.blocks)  # 40 tokens need 3 blocks
    elif kind == "credits":
        m.sequences["a"] = ref.SequenceRecord("a", 1, 17, a.blocks)
    elif kind == "invalid":
        m.lifo.free[0] = 6
    elif kind == "shared":
        m.sequences["b"] = ref.SequenceRecord("b", 1, 5, (a.blocks[0],))
    elif kind == "duplicate_free":
        m.lifo.free.append(m.lifo.free[0])
    elif kind == "owned_free":
        m.lifo.free.append(a.blocks[1])
        m.lifo.free.remove(m.lifo.free[0])
    elif kind == "missing":
        m.lifo.free.pop()
    elif kind == "owner":
        m.owners[a.blocks[0]] = "b"
    return m


@pytest.mark.parametrize(
    "kind,message",
    [
        ("table", "corrupt KV block table or reservation"),
        ("credits", "corrupt KV block table or reservation"),
        ("invalid", "invalid physical KV block"),
        ("shared", "physical KV blocks must have unique owners"),
        ("duplicate_free", "free KV blocks must be unique"),
        ("owned_free", "owned KV blocks must not be free"),
        ("missing", "KV blocks must cover the pool"),
        ("owner", "KV blocks are not owned by the recorded requests"),
    ],
)
def test_accounting_raises_the_reference_message_for_each_corruption(kind, message):
    assert _corrupted("none").counts() == (6, 3, 3, 4, 2, 22)
    with pytest.raises(RuntimeError, match=message):
        _corrupted(kind).counts()


@pytest.mark.parametrize("kind", ["missing", "duplicate_free"])
def test_planted_accounting_mistake_is_caught(monkeypatch, kind):
    """An accounting check that derives the free set from the owned blocks instead of
    reading the free list returns counts for a lost or duplicated free block; the
    corruption cases above tell the two apart."""
    original = ref.reference_assert_accounting

    def blind_to_free_list(sequences, free_blocks, block_owners, total_blocks):
        owned = {b for s in sequences.values() for b in s.blocks}
        return original(sequences, [b for b in range(total_blocks) if b not in owned], block_owners, total_blocks)

    with pytest.raises(RuntimeError):
        _corrupted(kind).counts()
    monkeypatch.setattr(ref, "reference_assert_accounting", blind_to_free_list)
    assert _corrupted(kind).counts()[0] == 6  # no error: the planted check misses the corruption
