"""Size-independent properties of the paged decode attention that hold bit for bit, checked
at the benchmark's full sizes (batch 64 over U{1..2048} on an 8192-block pool, and batch
256 x 2048 on a 40,000-block pool), where the oracle would take minutes per row:

- doubling V (one layer's V plane, in place) doubles every output exactly: softmax weights
  do not depend on V, the fp16 products with V, the fp32 sums, the split-K partials and
  their merge all scale by 2 without rounding, and fp16(2x) = 2 fp16(x) for results in the
  normal range (an fp16 subnormal result may differ by its last unit, 2^-24);
- swapping two kv heads' K and V in the pool, together with their two groups of eight
  query heads, swaps the corresponding output heads exactly (each kv head is computed by
  its own wave with the same arithmetic, and the plan does not depend on heads);
- doubling the queries and halving the keys (none of them subnormal after halving) changes
  no score and so no output bit;
- for the fused append + attention launch, doubling V and the new value rows doubles the
  outputs and the written V rows and leaves the K rows as they were;
- the first three also for the causal prompt attention kernel (pc_prefill_attention).

The reference computes each head independently (src/pagedcore/attention.py:31-53), so these
hold for it up to its own rounding; here they pin the index arithmetic of the head mapping
and the exactness of the split-K merge on the full workloads.
"""

from __future__ import annotations

import sys

import pytest
import torch

from pagedcore_amd import _hip
from tests import workloads

pytestmark = pytest.mark.gpu

SUBNORMAL = 2.0**-14  # smallest normal fp16 magnitude
WORKLOADS = {
    "batch64": dict(batch=64, num_blocks=8192, seed=61),
    "batch256x2048": dict(batch=256, num_blocks=40000, fixed_length=2048, seed=62),
}


def _say(*parts) -> None:
    print("[exact]", *parts, file=sys.stderr, flush=True)


@pytest.fixture
def device():
    if not torch.cuda.is_available():
        pytest.skip("needs a GPU")
    return torch.device("cuda:0")


def _setup(device, name):
    w = workloads.batched_decode(**WORKLOADS[name])
    gen = torch.Generator(device=device).manual_seed(w.seed)
    pool = torch.randn((22, 2, w.num_blocks, 16, 4, 64), dtype=torch.float16, device=device, generator=gen)
    layer = 7
    queries = torch.from_numpy(w.queries(layer)).to(device)
    tables = torch.from_numpy(w.tables).to(device)
    lens = torch.from_numpy(w.lengths).to(device)
    plan = torch.from_numpy(_hip.decode_plan(w.lengths, w.tables)).to(device)
    return w, pool, layer, queries, tables, lens, plan


def _attend(pool, layer, queries, tables, lens, plan):
    out = torch.full_like(queries, float("nan"))
    workspace = _hip.paged_decode_attention(out, queries, pool, layer, tables, lens, plan=plan)
    torch.cuda.synchronize()
    _hip.check_attention_faults(workspace, "exact properties")
    return out


@pytest.mark.parametrize("name", list(WORKLOADS))
def test_doubling_v_doubles_every_output_exactly(device, name):
    _say("doubling V", name)
    w, pool, layer, queries, tables, lens, plan = _setup(device, name)
    out = _attend(pool, layer, queries, tables, lens, plan)
    pool[layer, 1].mul_(2)  # exact in fp16 for N(0, 1) values
    doubled = _attend(pool, layer, queries, tables, lens, plan)
    assert not torch.isnan(out).any()
    expected = out * 2  # exact: no fp16 output is near the overflow threshold
    normal = out.abs() >= SUBNORMAL
    assert torch.equal(doubled[normal], expected[normal]), "a normal-range output is not exactly doubled"
    tiny = (doubled[~normal].float() - expected[~normal].float()).abs()
    assert tiny.numel() == 0 or float(tiny.max()) <= 2.0**-24
    _say(name, "rows", w.batch, "subnormal outputs", int((~normal).sum()))


@pytest.mark.parametrize("name", list(WORKLOADS))
@pytest.mark.parametrize("heads", [(0, 3), (1, 2)])
def test_swapping_kv_heads_swaps_output_heads_exactly(device, name, heads):
    _say("swapping kv heads", heads, name)
    h1, h2 = heads
    w, pool, layer, queries, tables, lens, plan = _setup(device, name)
    out = _attend(pool, layer, queries, tables, lens, plan)
    order = list(range(4))
    order[h1], order[h2] = h2, h1
    pool[layer] = pool[layer][..., order, :].clone()
    qorder = [8 * order[g] + i for g in range(4) for i in range(8)]
    swapped = _attend(pool, layer, queries[:, qorder].contiguous(), tables, lens, plan)
    assert torch.equal(swapped, out[:, qorder])


@pytest.mark.parametrize("name", list(WORKLOADS))
def test_doubling_q_and_halving_k_changes_no_bit(device, name):
    """(2q)(k/2) = qk exactly when no k is an fp16 subnormal after halving: the scores, and
    so every output bit, are those of the unscaled call (pins the Q and K paths)."""
    _say("2q, k/2", name)
    w, pool, layer, queries, tables, lens, plan = _setup(device, name)
    key = pool[layer, 0]
    floor = torch.where(key < 0, -(2.0**-13), 2.0**-13).to(torch.float16)
    key.copy_(torch.where(key.abs() < 2.0**-13, floor, key))  # halving keeps every k normal
    out = _attend(pool, layer, queries, tables, lens, plan)
    key.mul_(0.5)
    scaled = _attend(pool, layer, queries * 2, tables, lens, plan)
    assert not torch.isnan(out).any()
    assert torch.equal(scaled, out)


@pytest.mark.parametrize("name", list(WORKLOADS))
def test_fused_append_doubling_v_doubles_outputs_and_written_rows(device, name):
    """The same for pc_kv_append_paged_decode_attn (the kernel the batch-256 figure times):
    doubling the pool's V plane and the new value rows doubles every output and every
    written V row, and the written K rows are unchanged."""
    _say("fused doubling V", name)
    w, pool, layer, queries, tables, lens, plan = _setup(device, name)
    gen = torch.Generator(device=device).manual_seed(w.seed + 1)
    new_key = torch.randn((w.batch, 4, 64), dtype=torch.float16, device=device, generator=gen)
    new_value = torch.randn((w.batch, 4, 64), dtype=torch.float16, device=device, generator=gen)
    twin = pool.clone()
    twin[layer, 1].mul_(2)
    outs = []
    for p, v in ((pool, new_value), (twin, new_value * 2)):
        out = torch.full_like(queries, float("nan"))
        workspace = torch.zeros(_hip.workspace_bytes(w.batch, w.tables.shape[1]), dtype=torch.uint8, device=device)
        _hip.planned_decode_attention(out, queries, p, layer, lens, plan, w.tables.shape[1], workspace,
                                      new_key=new_key, new_value=v)
        torch.cuda.synchronize()
        _hip.check_attention_faults(workspace, "fused exact properties")
        outs.append(out)
    assert not torch.isnan(outs[0]).any()
    normal = outs[0].abs() >= SUBNORMAL
    assert torch.equal(outs[1][normal], (outs[0] * 2)[normal])
    tiny = (outs[1][~normal].float() - (outs[0] * 2)[~normal].float()).abs()
    assert tiny.numel() == 0 or float(tiny.max()) <= 2.0**-24
    assert torch.equal(twin[layer, 0], pool[layer, 0])  # K planes, new rows included
    assert torch.equal(twin[layer, 1], pool[layer, 1] * 2)  # V planes, new rows included


# --- the prompt attention kernel (pc_prefill_attention) -----------------------------------


def _prompt(device, tokens, seed):
    gen = torch.Generator(device=device).manual_seed(seed)
    q = torch.randn((tokens, 32, 64), dtype=torch.float16, device=device, generator=gen)
    k = torch.randn((tokens, 4, 64), dtype=torch.float16, device=device, generator=gen)
    v = torch.randn((tokens, 4, 64), dtype=torch.float16, device=device, generator=gen)
    return q, k, v


def _prefill(q, k, v):
    out = torch.full_like(q, float("nan"))
    _hip.prefill_attention(out, q, k, v)
    torch.cuda.synchronize()
    return out


@pytest.mark.parametrize("tokens", [333, 2048])
def test_prompt_attention_exact_properties(device, tokens):
    """For the causal prompt kernel (P is rounded to fp16 before its product with V, the
    rest fp32): doubling V doubles the outputs, swapping two kv heads with their query
    heads swaps the output heads, and 2q with k/2 changes no bit."""
    _say("prompt attention exact properties", tokens)
    q, k, v = _prompt(device, tokens, 70 + tokens)
    floor = torch.where(k < 0, -(2.0**-13), 2.0**-13).to(torch.float16)
    k = torch.where(k.abs() < 2.0**-13, floor, k).contiguous()
    out = _prefill(q, k, v)
    assert not torch.isnan(out).any()
    doubled = _prefill(q, k, (v * 2).contiguous())
    normal = out.abs() >= SUBNORMAL
    assert torch.equal(doubled[normal], (out * 2)[normal])
    tiny = (doubled[~normal].float() - (out * 2)[~normal].float()).abs()
    assert tiny.numel() == 0 or float(tiny.max()) <= 2.0**-24
    order = [3, 1, 2, 0]
    qorder = [8 * order[g] + i for g in range(4) for i in range(8)]
    swapped = _prefill(q[:, qorder].contiguous(), k[:, order].contiguous(), v[:, order].contiguous())
    assert torch.equal(swapped, out[:, qorder])
    scaled = _prefill((q * 2).contiguous(), (k * 0.5).contiguous(), v)
    assert torch.equal(scaled, out)
