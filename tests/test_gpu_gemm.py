"""pc_gemm_m128 (the decode step's projections at up to 128 rows) and the split-K consumers.

The GEMM is compared with an fp32 torch product of the same fp16 inputs (fp32 accumulation
in both; only the summation order differs), split by split so that a wrong K range cannot
hide in the total. The fp16 and SwiGLU epilogues are checked against the fp16 rounding of
that product and against pc_silu_mul applied to the library's own fp16 projections. The
split-K consumers are checked bit for bit against the fp16 path fed fp16(sum of the parts),
summed in the same split order.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from pagedcore_amd import _hip
from pagedcore_amd import decoder as dec

pytestmark = pytest.mark.gpu

# (m, n, k, splits): the decode step's q|k|v, o_proj and down projections at batch 128 and
# 64 (the serving graph), and ragged row counts.
PARTIAL_SHAPES = [
    (128, 2560, 2048, 4),
    (128, 2048, 2048, 4),
    (128, 2048, 5632, 8),
    (64, 2560, 2048, 4),
    (37, 2048, 2048, 4),
    (1, 2048, 5632, 8),
    (128, 11264, 2048, 1),
]


def _inputs(device, m, n, k, seed):
    gen = torch.Generator(device=device).manual_seed(seed)
    x = (torch.randn((m, k), device=device, generator=gen) * 0.5).half()
    w = (torch.randn((n, k), device=device, generator=gen) * 0.02).half()
    return x, w


def _bits(t: torch.Tensor) -> np.ndarray:
    return t.detach().cpu().contiguous().view(torch.int16).numpy()


@pytest.mark.parametrize("m,n,k,splits", PARTIAL_SHAPES)
def test_gemm_partials_match_fp32_split_by_split(device, m, n, k, splits):
    x, w = _inputs(device, m, n, k, seed=m + n + k + splits)
    out = torch.full((splits, m, n), float("nan"), dtype=torch.float32, device=device)
    _hip.gemm_m128(out, x, w, splits=splits, epilogue=_hip.GEMM_PARTIALS)
    torch.cuda.synchronize()
    span = k // splits
    worst = 0.0
    for s in range(splits):
        part = x[:, s * span : (s + 1) * span].float() @ w[:, s * span : (s + 1) * span].float().t()
        err = (out[s] - part).abs().max().item()
        scale = part.abs().max().item()
        worst = max(worst, err / scale)
        # fp32 accumulation of the same products in another order: a few ulp of the sums.
        assert err <= 2e-6 * scale + 1e-7, (s, err, scale)
    print(f"m {m} n {n} k {k} splits {splits}: max error / max |part| {worst:.2e}")


@pytest.mark.parametrize("m,n,k", [(128, 11264, 2048), (128, 2048, 2048), (5, 2048, 2048)])
def test_gemm_half_rounds_the_fp32_product(device, m, n, k):
    x, w = _inputs(device, m, n, k, seed=7 + m)
    out = torch.empty((m, n), dtype=torch.float16, device=device)
    _hip.gemm_m128(out, x, w, splits=1, epilogue=_hip.GEMM_HALF)
    exact = x.float() @ w.float().t()
    torch.cuda.synchronize()
    # fp16(Y), Y the fp32 partial-sum path of the same kernel, bit for bit; and Y differs
    # from the exact product by the summation order only: within a half fp16 ulp plus the
    # fp32 accumulation error (absolute, a few 1e-7 of the largest sums: it dominates where
    # the sum cancels to a tiny value).
    parts = torch.empty((1, m, n), dtype=torch.float32, device=device)
    _hip.gemm_m128(parts, x, w, splits=1, epilogue=_hip.GEMM_PARTIALS)
    torch.cuda.synchronize()
    assert np.array_equal(_bits(out), _bits(parts[0].half()))
    ulp = torch.finfo(torch.float16).eps * exact.abs().clamp_min(2.0**-14)
    slack = 2e-6 * exact.abs().max().item()
    assert ((out.float() - exact).abs() <= ulp + slack).all()
    assert (out == exact.half()).float().mean().item() > 0.99


@pytest.mark.parametrize("m", [128, 64, 3])
def test_gemm_swiglu_equals_silu_mul_of_the_fp16_projections(device, m):
    """The SwiGLU epilogue on the stacked [gate | up] weight equals pc_silu_mul applied to
    the fp16 projections of the same kernel configuration, bit for bit (the projections
    themselves are checked against fp32 in test_gemm_half_rounds_the_fp32_product)."""
    width = 5632
    x, w = _inputs(device, m, 2 * width, 2048, seed=11 + m)
    fused = torch.empty((m, width), dtype=torch.float16, device=device)
    _hip.gemm_m128(fused, x, w, splits=1, epilogue=_hip.GEMM_SWIGLU)
    projected = torch.empty((m, 2 * width), dtype=torch.float16, device=device)
    _hip.gemm_m128(projected, x, w, splits=1, epilogue=_hip.GEMM_HALF)
    separate = torch.empty_like(fused)
    _hip.silu_mul(separate, projected)
    torch.cuda.synchronize()
    assert np.array_equal(_bits(fused), _bits(separate))
    # and the reference expression (dense.py:102-104, torch's silu) on those projections
    # within two ulp of the product (silu's own last bit may differ from x / (1 + e^-x)).
    gate, up = projected[:, :width].float(), projected[:, width:].float()
    expected = (torch.nn.functional.silu(gate).half().float() * up).half().float()
    ulp = torch.finfo(torch.float16).eps * expected.abs().clamp_min(2.0**-14)
    assert ((fused.float() - expected).abs() <= 2 * ulp + 2.0**-24).all()


def _sum_in_split_order(parts: torch.Tensor) -> torch.Tensor:
    total = parts[0].clone()
    for s in range(1, parts.shape[0]):
        total = total + parts[s]
    return total.half()


@pytest.mark.parametrize("rows,splits", [(128, 4), (64, 8), (3, 1), (128, 16), (7, 64)])
def test_add_rms_norm_parts_equals_the_fp16_path(device, rows, splits):
    gen = torch.Generator(device=device).manual_seed(rows * splits)
    width = 2048
    parts = torch.randn((splits, rows, width), device=device, generator=gen) * 0.3
    hidden = torch.randn((rows, width), device=device, generator=gen).half()
    weight = (1 + 0.1 * torch.randn(width, device=device, generator=gen)).half()
    h1, h2 = hidden.clone(), hidden.clone()
    out1 = torch.empty_like(hidden)
    out2 = torch.empty_like(hidden)
    _hip.add_rms_norm(out1, h1, _sum_in_split_order(parts), weight, dec.RMS_EPS)
    _hip.add_rms_norm_parts(out2, h2, parts, weight, dec.RMS_EPS)
    torch.cuda.synchronize()
    assert np.array_equal(_bits(h1), _bits(h2))
    assert np.array_equal(_bits(out1), _bits(out2))


@pytest.mark.parametrize("tokens,splits", [(128, 4), (5, 8), (128, 16), (3, 64)])
def test_rope_kv_append_parts_equals_the_fp16_path(device, tokens, splits):
    gen = torch.Generator(device=device).manual_seed(tokens + splits)
    parts = torch.randn((splits, tokens, 2560), device=device, generator=gen) * 0.5
    positions = torch.randint(0, 2048, (tokens,), device=device, generator=gen)
    blocks = 20
    slots = torch.randperm(blocks * 16, device=device, generator=gen)[:tokens]
    table = dec.rope_table(device)
    results = []
    for use_parts in (False, True):
        pool = torch.full((22, 2, blocks, 16, 4, 64), float("nan"), dtype=torch.float16, device=device)
        query = torch.empty(tokens, 32, 64, dtype=torch.float16, device=device)
        keys = torch.empty(tokens, 4, 64, dtype=torch.float16, device=device)
        values = torch.empty_like(keys)
        common = dict(key_out=keys, value_out=values, pool=pool, layer=3, slot_mapping=slots)
        if use_parts:
            _hip.rope_kv_append_parts(query, parts, positions, table, **common)
        else:
            _hip.rope_kv_append(query, _sum_in_split_order(parts), positions, table, **common)
        torch.cuda.synchronize()
        results.append((query, keys, values, pool))
    for a, b in zip(*results):
        assert np.array_equal(_bits(a), _bits(b))


# --- exact properties at the decode step's shapes ------------------------------------------


@pytest.mark.parametrize("m,n,k,splits", [s for s in PARTIAL_SHAPES if s[0] == 128])
def test_gemm_partials_permute_and_scale_exactly(device, m, n, k, splits):
    """Permuting the activation rows permutes the partials' rows, permuting the weight rows
    permutes their columns, and doubling the weight doubles them, all bit for bit: every
    output element is the same sequence of MFMA sums wherever its row and column sit in
    the tiles, and a power-of-two scale rounds nothing."""
    x, w = _inputs(device, m, n, k, seed=7 * n + k)
    gen = torch.Generator(device="cpu").manual_seed(n + splits)
    rows, cols = torch.randperm(m, generator=gen).to(device), torch.randperm(n, generator=gen).to(device)

    def run(xx, ww):
        out = torch.full((splits, m, n), float("nan"), dtype=torch.float32, device=device)
        _hip.gemm_m128(out, xx.contiguous(), ww.contiguous(), splits=splits, epilogue=_hip.GEMM_PARTIALS)
        torch.cuda.synchronize()
        return out

    base = run(x, w)
    assert not torch.isnan(base).any()
    assert torch.equal(run(x[rows], w), base[:, rows])
    assert torch.equal(run(x, w[cols]), base[:, :, cols])
    assert torch.equal(run(x, w * 2), base * 2)


def test_gemm_swiglu_permutes_exactly(device):
    """The SwiGLU epilogue (output column c from gate row c and up row half + c): the same
    permutation of the gate rows and of the up rows permutes the output columns, and
    permuting the activation rows permutes the output rows, bit for bit."""
    m, n, k = 128, 11264, 2048
    half = n // 2
    x, w = _inputs(device, m, n, k, seed=91)
    gen = torch.Generator(device="cpu").manual_seed(92)
    rows, cols = torch.randperm(m, generator=gen).to(device), torch.randperm(half, generator=gen).to(device)

    def run(xx, ww):
        out = torch.full((m, half), float("nan"), dtype=torch.float16, device=device)
        _hip.gemm_m128(out, xx.contiguous(), ww.contiguous(), epilogue=_hip.GEMM_SWIGLU)
        torch.cuda.synchronize()
        return out

    base = run(x, w)
    assert not torch.isnan(base).any()
    assert torch.equal(run(x[rows], w), base[rows])
    permuted = torch.cat((w[:half][cols], w[half:][cols]))
    assert torch.equal(run(x, permuted), base[:, cols])
