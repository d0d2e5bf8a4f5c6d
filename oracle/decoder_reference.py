"""CPU restatement of the reference's TinyLlama forward — test infrastructure only.

Op for op with src/pagedcore/dense.py and the contiguous forward of
src/pagedcore/decoder.py:202-240, in torch on the CPU, so that the GPU decode step and
paged prefill can be checked against "the contiguous FP32 decode" the reference's own
paged-decode test uses as its expectation (tests/unit/test_decoder.py:144-164:
decode(..., fp32_attention=True), logits within 5e-3, cached K/V within 2e-3), and the
greedy loop of generate (src/pagedcore/decoder.py:70-100) as the expectation of the
continuous-batching worker.

Weights are any object with the reference's field names (embedding, layers, final_norm,
lm_head; per layer input_norm, q_proj, k_proj, v_proj, o_proj, post_attention_norm,
gate_proj, up_proj, down_proj), as fp16 CPU tensors.

Pinning (tests/test_oracle_decoder.py): prefill logits against the transformers Llama
implementation on the reference test's synthetic configuration (the reference's own check,
tests/unit/test_decoder.py:78-105, atol=rtol=5e-3); decode logits against the same model's
full-sequence logits; closed forms for RoPE (position 0 is the identity, a rotation keeps
each (d, d+32) pair's norm, the fp32 rotation makes q.k depend only on the position
difference) and for RMSNorm (constant rows); planted mistakes (K not rotated, V rotated,
the rotate-half sign flipped, the 8-head grouping transposed) fail the transformers check;
generate's stream against a transformers greedy loop, and its stopping rules (EOS
selected but not emitted, EOS winning at the limit, ignore_eos, the number of decode
calls) against scripted logits, with planted rule mistakes that those cases catch.
"""

from __future__ import annotations

from typing import List, Optional, Sequence, Tuple

import torch
import torch.nn.functional as F
from torch import Tensor

Q_HEADS = 32
KV_HEADS = 4
HEAD_DIM = 64
GROUP = Q_HEADS // KV_HEADS
EPS = 1e-5
THETA = 10000.0

KVCache = List[Tuple[Tensor, Tensor]]  # per layer: rotated K, V, each [1, 4, tokens, 64]


def rms_norm(hidden: Tensor, weight: Tensor) -> Tensor:
    """dense.py:17-21: fp32 normalisation, rounded to the hidden dtype, then times the fp16
    weight (an fp16 product)."""
    as_float = hidden.float()
    inverse_rms = torch.rsqrt(as_float.square().mean(dim=-1, keepdim=True) + EPS)
    return weight * (as_float * inverse_rms).to(hidden.dtype)


def project_qkv(hidden: Tensor, layer) -> Tuple[Tensor, Tensor, Tensor]:
    """dense.py:24-30: [batch, tokens, 2048] -> q [b, 32, t, 64], k and v [b, 4, t, 64]."""
    batch, tokens, _ = hidden.shape

    def heads(weight: Tensor, count: int) -> Tensor:
        return F.linear(hidden, weight).view(batch, tokens, count, HEAD_DIM).transpose(1, 2)

    return heads(layer.q_proj, Q_HEADS), heads(layer.k_proj, KV_HEADS), heads(layer.v_proj, KV_HEADS)


def rope_cos_sin(positions: Tensor, dtype: torch.dtype) -> Tuple[Tensor, Tensor]:
    """dense.py:46-54: fp32 frequencies and angles, cos/sin rounded to the query dtype,
    [batch, 1, tokens, 64] (the 32 angles repeated)."""
    with torch.autocast(device_type="cpu", enabled=False):
        inverse = 1.0 / (THETA ** (torch.arange(0, HEAD_DIM, 2).float() / HEAD_DIM))
        angles = positions.float().unsqueeze(-1) * inverse
        angles = torch.cat((angles, angles), dim=-1)
        return angles.cos().to(dtype).unsqueeze(1), angles.sin().to(dtype).unsqueeze(1)


def rotate(tensor: Tensor, cosine: Tensor, sine: Tensor) -> Tensor:
    """dense.py:56-59: x * cos + cat(-x2, x1) * sin, each op in the tensor's dtype."""
    half = tensor.shape[-1] // 2
    swapped = torch.cat((-tensor[..., half:], tensor[..., :half]), dim=-1)
    return tensor * cosine + swapped * sine


def apply_rope(query: Tensor, key: Tensor, positions: Tensor) -> Tuple[Tensor, Tensor]:
    """dense.py:33-61: rotate Q and K at int64 [batch or 1, tokens] positions."""
    cosine, sine = rope_cos_sin(positions, query.dtype)
    return rotate(query, cosine, sine), rotate(key, cosine, sine)


def repeat_kv(tensor: Tensor) -> Tensor:
    """dense.py:64-66: kv head g serves query heads 8g .. 8g + 7."""
    return tensor.repeat_interleave(GROUP, dim=1)


def dense_attention(query: Tensor, key: Tensor, value: Tensor, allowed: Tensor) -> Tensor:
    """dense.py:69-81 (prefill and the default decode): fp16 scores * 1/8, masked with the
    fp16 minimum, fp32 softmax rounded to fp16, fp16 product."""
    scores = torch.matmul(query, repeat_kv(key).transpose(-2, -1)) * (HEAD_DIM**-0.5)
    scores = scores.masked_fill(~allowed, torch.finfo(query.dtype).min)
    weights = F.softmax(scores, dim=-1, dtype=torch.float32).to(query.dtype)
    return torch.matmul(weights, repeat_kv(value))


def dense_attention_fp32(query: Tensor, key: Tensor, value: Tensor, allowed: Tensor) -> Tensor:
    """dense.py:91-99 (the paging reference): everything in fp32, one final rounding."""
    with torch.autocast(device_type="cpu", enabled=False):
        scores = torch.matmul(query.float(), repeat_kv(key).float().transpose(-2, -1))
        scores = (scores * (HEAD_DIM**-0.5)).masked_fill(~allowed, -torch.inf)
        return torch.matmul(scores.softmax(dim=-1), repeat_kv(value).float()).to(query.dtype)


def output_projection(attention: Tensor, layer) -> Tensor:
    """dense.py:84-88: heads merged in head order, then o_proj."""
    batch, _, tokens, _ = attention.shape
    return F.linear(attention.transpose(1, 2).reshape(batch, tokens, Q_HEADS * HEAD_DIM), layer.o_proj)


def swiglu(hidden: Tensor, layer) -> Tensor:
    """dense.py:102-104."""
    return F.linear(F.silu(F.linear(hidden, layer.gate_proj)) * F.linear(hidden, layer.up_proj), layer.down_proj)


def final_logits(hidden: Tensor, weights) -> Tensor:
    """dense.py:107-109."""
    return F.linear(rms_norm(hidden, weights.final_norm), weights.lm_head)


def forward(
    input_ids: Tensor, weights, cache: Optional[KVCache] = None, *, fp32_attention: bool = False
) -> Tuple[Tensor, KVCache]:
    """decoder.py:202-240: the contiguous forward of one sequence, int64 [1, tokens], at
    positions cache length .. cache length + tokens - 1; returns fp16 logits
    [1, tokens, vocab] and the new cache (old K/V concatenated with this call's)."""
    offset = 0 if cache is None else cache[0][0].shape[2]
    tokens = input_ids.shape[1]
    positions = torch.arange(offset, offset + tokens)[None]
    allowed = (torch.arange(offset + tokens)[None, :] <= positions[0, :, None])[None, None]
    attend = dense_attention_fp32 if fp32_attention else dense_attention
    hidden = F.embedding(input_ids, weights.embedding)
    layers: KVCache = []
    for index, layer in enumerate(weights.layers):
        query, key, value = project_qkv(rms_norm(hidden, layer.input_norm), layer)
        query, key = apply_rope(query, key, positions)
        if cache is not None:
            key = torch.cat((cache[index][0], key), dim=2)
            value = torch.cat((cache[index][1], value), dim=2)
        layers.append((key, value))
        hidden = hidden + output_projection(attend(query, key, value, allowed), layer)
        hidden = hidden + swiglu(rms_norm(hidden, layer.post_attention_norm), layer)
    return final_logits(hidden, weights), layers


@torch.inference_mode()
def prefill(input_ids: Tensor, weights) -> Tuple[Tensor, KVCache]:
    """decoder.py:103-110: the prompt's logits and cache (fp16 dense attention)."""
    return forward(input_ids, weights)


@torch.inference_mode()
def decode_fp32(input_ids: Tensor, cache: KVCache, weights) -> Tuple[Tensor, KVCache]:
    """decoder.py:138-153 with fp32_attention=True: one token [1, 1] after the cache."""
    return forward(input_ids, weights, cache, fp32_attention=True)


@torch.inference_mode()
def decode(input_ids: Tensor, cache: KVCache, weights) -> Tuple[Tensor, KVCache]:
    """decoder.py:138-153 with fp32_attention=False (what generate uses): one token [1, 1]
    after the cache, fp16 dense attention."""
    return forward(input_ids, weights, cache)


EOS_TOKEN_ID = 2  # reference src/pagedcore/decoder.py:94


@torch.inference_mode()
def generate(input_ids: Tensor, weights, *, max_new_tokens: int = 128, ignore_eos: bool = False):
    """decoder.py:70-100: single-sequence greedy generation with the contiguous cache.

    Returns (greedy_ids, emitted_ids, finish_reason) with finish_reason "eos" or "length".
    The token of step s is the argmax of the last position's logits; it is selected before
    the stop test, so a stopping EOS is in greedy_ids and not in emitted_ids, and EOS wins
    when it is selected at the output limit; decode runs only while another token is due
    (max_new_tokens - 1 decode calls at most)."""
    if type(max_new_tokens) is not int or not 1 <= max_new_tokens <= 256:
        raise ValueError("max_new_tokens must be an integer from 1 to 256")
    if type(ignore_eos) is not bool:
        raise ValueError("ignore_eos must be a boolean")
    if input_ids.ndim != 2 or input_ids.shape[0] != 1:
        raise ValueError("input_ids must be int64 [1, tokens]")
    if input_ids.shape[1] + max_new_tokens > 2048:
        raise ValueError("prompt tokens plus requested output must not exceed 2048")
    logits, cache = prefill(input_ids, weights)
    selected: List[int] = []
    for step in range(max_new_tokens):
        token = logits[:, -1:].argmax(dim=-1)
        selected.append(int(token.item()))
        if selected[-1] == EOS_TOKEN_ID and not ignore_eos:
            return tuple(selected), tuple(selected[:-1]), "eos"
        if step + 1 < max_new_tokens:
            logits, cache = decode(token, cache, weights)
    return tuple(selected), tuple(selected), "length"


def pool_layout(cache: KVCache) -> Tuple[Tensor, Tensor]:
    """The cache as the allocator stores it: K and V [layers, tokens, 4, 64]
    (decoder.py:132-133)."""
    key = torch.stack([k[0].transpose(0, 1) for k, _ in cache])
    value = torch.stack([v[0].transpose(0, 1) for _, v in cache])
    return key, value


def to_cpu(weights, cls_layer, cls_weights):
    """A CPU copy of GPU weights (same dataclasses)."""
    layers = tuple(cls_layer(**{name: getattr(layer, name).cpu() for name in _LAYER_FIELDS}) for layer in weights.layers)
    return cls_weights(weights.embedding.cpu(), layers, weights.final_norm.cpu(), weights.lm_head.cpu())


_LAYER_FIELDS: Sequence[str] = (
    "input_norm",
    "q_proj",
    "k_proj",
    "v_proj",
    "o_proj",
    "post_attention_norm",
    "gate_proj",
    "up_proj",
    "down_proj",
)
