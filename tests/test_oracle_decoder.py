"""Pins the CPU decoder oracle (oracle/decoder_reference.py) before it is trusted as the
expectation of the GPU decode step: against the transformers Llama implementation on the
reference tests' synthetic configuration (tests/unit/test_decoder.py:32-105), against
closed forms, and with planted mistakes that those checks must catch."""

from __future__ import annotations

import math
from types import SimpleNamespace

import pytest
import torch

from oracle import decoder_reference as dref

FIELDS = dref._LAYER_FIELDS


@pytest.fixture(scope="module")
def synthetic():
    """The reference test's synthetic Llama (head geometry of TinyLlama, 2 layers, MLP 32,
    vocab 31, seed 0), with norm weights perturbed so the norm scale is exercised too."""
    transformers = pytest.importorskip("transformers")
    from transformers.models.llama.modeling_llama import LlamaRotaryEmbedding

    config = transformers.LlamaConfig(
        vocab_size=31,
        hidden_size=2048,
        intermediate_size=32,
        num_hidden_layers=2,
        num_attention_heads=32,
        num_key_value_heads=4,
        head_dim=64,
        max_position_embeddings=2048,
        rms_norm_eps=1e-5,
        rope_theta=10000.0,
        tie_word_embeddings=False,
        attention_dropout=0.0,
    )
    config._attn_implementation = "eager"
    with torch.random.fork_rng(devices=[]):
        torch.manual_seed(0)
        model = transformers.LlamaForCausalLM(config).half().eval()
        with torch.no_grad():
            for layer in model.model.layers:
                layer.input_layernorm.weight.add_(0.1 * torch.randn(2048).half())
                layer.post_attention_layernorm.weight.add_(0.1 * torch.randn(2048).half())
            model.model.norm.weight.add_(0.1 * torch.randn(2048).half())
    # .half() also rounded the rotary buffers; RoPE frequencies stay fp32 (as the reference test does).
    model.model.rotary_emb = LlamaRotaryEmbedding(config)
    layers = tuple(
        SimpleNamespace(
            input_norm=layer.input_layernorm.weight.detach(),
            q_proj=layer.self_attn.q_proj.weight.detach(),
            k_proj=layer.self_attn.k_proj.weight.detach(),
            v_proj=layer.self_attn.v_proj.weight.detach(),
            o_proj=layer.self_attn.o_proj.weight.detach(),
            post_attention_norm=layer.post_attention_layernorm.weight.detach(),
            gate_proj=layer.mlp.gate_proj.weight.detach(),
            up_proj=layer.mlp.up_proj.weight.detach(),
            down_proj=layer.mlp.down_proj.weight.detach(),
        )
        for layer in model.model.layers
    )
    weights = SimpleNamespace(
        embedding=model.model.embed_tokens.weight.detach(),
        layers=layers,
        final_norm=model.model.norm.weight.detach(),
        lm_head=model.lm_head.weight.detach(),
    )
    return model, weights


def _hf_logits(model, ids):
    with torch.inference_mode():
        return model(ids, use_cache=False).logits


@pytest.mark.parametrize("tokens", [1, 15, 16, 17, 49])
def test_prefill_matches_transformers(synthetic, tokens):
    model, weights = synthetic
    ids = torch.arange(tokens)[None] % 31
    logits, cache = dref.prefill(ids, weights)
    assert logits.dtype == torch.float16 and logits.shape == (1, tokens, 31)
    torch.testing.assert_close(logits, _hf_logits(model, ids), atol=5e-3, rtol=5e-3)
    assert len(cache) == 2
    for key, value in cache:
        assert key.shape == value.shape == (1, 4, tokens, 64)


@pytest.mark.parametrize("tokens", [1, 16, 40])
def test_fp32_decode_matches_transformers_full_sequence(synthetic, tokens):
    """decode_fp32 after a prefill gives the next position's logits of the full sequence."""
    model, weights = synthetic
    ids = (torch.arange(tokens + 1)[None] * 7 + 3) % 31
    _, cache = dref.prefill(ids[:, :tokens], weights)
    logits, new_cache = dref.decode_fp32(ids[:, tokens:], cache, weights)
    assert logits.shape == (1, 1, 31)
    torch.testing.assert_close(logits[0, 0], _hf_logits(model, ids)[0, -1], atol=5e-3, rtol=5e-3)
    assert new_cache[1][0].shape == (1, 4, tokens + 1, 64)
    # the old positions are carried over exactly; the new one is appended
    torch.testing.assert_close(new_cache[0][0][:, :, :tokens], cache[0][0], atol=0, rtol=0)


def test_cache_holds_rotated_keys_and_unrotated_values(synthetic):
    """tests/unit/test_decoder.py:97-105: layer 0's cache equals RoPE(K) and V exactly."""
    _, weights = synthetic
    ids = torch.arange(9)[None] % 31
    _, cache = dref.prefill(ids, weights)
    hidden = weights.embedding[ids]
    _, key, value = dref.project_qkv(dref.rms_norm(hidden, weights.layers[0].input_norm), weights.layers[0])
    _, rotated = dref.apply_rope(torch.zeros(1, 32, 9, 64, dtype=torch.float16), key, torch.arange(9)[None])
    torch.testing.assert_close(cache[0][0], rotated, atol=0, rtol=0)
    torch.testing.assert_close(cache[0][1], value, atol=0, rtol=0)
    assert not torch.equal(rotated[:, :, 1:], key[:, :, 1:])


def test_rope_closed_forms():
    gen = torch.Generator().manual_seed(3)
    x = torch.randn(1, 4, 6, 64, generator=gen)
    # position 0: cos = 1, sin = 0 exactly, so the rotation is the identity
    same, _ = dref.apply_rope(x.half(), x.half(), torch.zeros(1, 6, dtype=torch.int64))
    torch.testing.assert_close(same, x.half(), atol=0, rtol=0)
    # fp32: each (d, d + 32) pair keeps its norm
    positions = torch.tensor([[0, 1, 5, 100, 1000, 2047]])
    rotated, _ = dref.apply_rope(x, x, positions)
    pair = x[..., :32] ** 2 + x[..., 32:] ** 2
    rotated_pair = rotated[..., :32] ** 2 + rotated[..., 32:] ** 2
    torch.testing.assert_close(rotated_pair, pair, atol=1e-5, rtol=1e-5)
    # e_0 at position 1 (frequency 1 rad): cos 1 in dim 0, sin 1 in dim 32
    unit = torch.zeros(1, 1, 1, 64)
    unit[..., 0] = 1.0
    turned, _ = dref.apply_rope(unit, unit, torch.tensor([[1]]))
    expected = torch.zeros(64)
    expected[0], expected[32] = math.cos(1.0), math.sin(1.0)
    torch.testing.assert_close(turned.flatten(), expected, atol=1e-6, rtol=0)
    # fp32: q(m) . k(n) depends only on m - n
    q = torch.randn(1, 1, 1, 64, generator=gen)
    k = torch.randn(1, 1, 1, 64, generator=gen)

    def score(m, n):
        qm, _ = dref.apply_rope(q, q, torch.tensor([[m]]))
        kn, _ = dref.apply_rope(k, k, torch.tensor([[n]]))
        return float((qm * kn).sum())

    assert abs(score(10, 3) - score(507, 500)) < 1e-4
    assert abs(score(10, 3) - score(3, 10)) > 1e-3  # not symmetric: the sign of m - n matters


def test_rms_norm_closed_forms():
    weight = torch.linspace(0.5, 2.0, 2048).half()
    for c in (2.0, -0.75, 1e-3):
        row = torch.full((1, 2048), c, dtype=torch.float16)
        exact = float(row[0, 0]) / math.sqrt(float(row[0, 0]) ** 2 + 1e-5)
        expected = weight * torch.tensor(exact).half()
        torch.testing.assert_close(dref.rms_norm(row, weight)[0], expected, atol=0, rtol=0)
    # scale invariance up to eps: x and 4x normalise to the same row
    gen = torch.Generator().manual_seed(1)
    x = torch.randn(3, 2048, generator=gen).half()
    torch.testing.assert_close(dref.rms_norm(x, weight), dref.rms_norm(x * 4, weight), atol=2e-3, rtol=2e-3)


@pytest.mark.parametrize("mistake", ["key_not_rotated", "value_rotated", "rotate_sign", "head_grouping"])
def test_planted_mistakes_fail_the_transformers_check(synthetic, mistake, monkeypatch):
    model, weights = synthetic
    ids = torch.arange(17)[None] % 31
    expected = _hf_logits(model, ids)
    apply_rope, rotate, repeat_kv = dref.apply_rope, dref.rotate, dref.repeat_kv
    if mistake == "key_not_rotated":
        monkeypatch.setattr(dref, "apply_rope", lambda q, k, p: (apply_rope(q, k, p)[0], k))
    elif mistake == "value_rotated":
        project = dref.project_qkv

        def rotated_value(hidden, layer):
            q, k, v = project(hidden, layer)
            return q, k, apply_rope(v, v, torch.arange(v.shape[2])[None])[1]

        monkeypatch.setattr(dref, "project_qkv", rotated_value)
    elif mistake == "rotate_sign":
        monkeypatch.setattr(dref, "rotate", lambda t, c, s: rotate(t, c, -s))
    else:
        monkeypatch.setattr(dref, "repeat_kv", lambda t: repeat_kv(t).view(t.shape[0], 8, 4, *t.shape[2:]).transpose(1, 2).reshape(t.shape[0], 32, *t.shape[2:]))
    logits, _ = dref.prefill(ids, weights)
    assert not torch.allclose(logits, expected, atol=5e-3, rtol=5e-3)


# ---------------------------------------------------------------------------------------
# generate (reference src/pagedcore/decoder.py:70-100)
# ---------------------------------------------------------------------------------------


def _hf_greedy(model, ids, max_new_tokens, ignore_eos):
    """A greedy loop over the transformers model (full recompute each step) with the
    reference's stopping rules."""
    selected = []
    sequence = ids
    for step in range(max_new_tokens):
        token = int(_hf_logits(model, sequence)[0, -1].argmax())
        selected.append(token)
        if token == 2 and not ignore_eos:
            return tuple(selected), "eos"
        sequence = torch.cat([sequence, torch.tensor([[token]])], dim=1)
    return tuple(selected), "length"


@pytest.mark.parametrize("seed", [0, 1, 2, 3])
def test_generate_matches_a_transformers_greedy_loop(synthetic, seed):
    """The oracle's generate (prefill, then one fp16 decode per further token) selects the
    same tokens as greedy selection over the transformers model's full-sequence logits."""
    model, weights = synthetic
    gen = torch.Generator().manual_seed(seed)
    ids = torch.randint(3, 31, (1, int(torch.randint(1, 30, (1,), generator=gen))), generator=gen)
    greedy, emitted, reason = dref.generate(ids, weights, max_new_tokens=12, ignore_eos=seed % 2 == 0)
    expected, expected_reason = _hf_greedy(model, ids, 12, seed % 2 == 0)
    assert greedy == expected and reason == expected_reason
    assert emitted == (greedy[:-1] if reason == "eos" else greedy)


class _Scripted:
    """prefill / decode stand-ins whose last-position logits select script[n] at the n-th
    selection (the other positions favour another token, so reading the wrong position
    shows)."""

    def __init__(self, script, vocab=8):
        self.script, self.vocab, self.decodes = list(script), vocab, 0

    def _logits(self, n, positions):
        logits = torch.zeros(1, positions, self.vocab, dtype=torch.float16)
        logits[0, :, (self.script[n] + 1) % self.vocab] = 1.0
        logits[0, -1] = 0.0
        logits[0, -1, self.script[n]] = 1.0
        return logits

    def prefill(self, ids, weights):
        return self._logits(0, ids.shape[1]), [ids.shape[1]]

    def decode(self, token, cache, weights):
        self.decodes += 1
        # the cache counts the forward calls so far; this call feeds the last selection
        assert token.shape == (1, 1) and int(token) == self.script[len(cache) - 1]
        return self._logits(len(cache), 1), cache + [len(cache)]


@pytest.mark.parametrize(
    "script,max_new,ignore_eos,expected",
    [
        # EOS mid-stream: selected, not emitted; no decode after it
        ((5, 6, 2, 7), 4, False, ((5, 6, 2), (5, 6), "eos", 2)),
        # EOS selected exactly at the limit still wins
        ((5, 6, 2), 3, False, ((5, 6, 2), (5, 6), "eos", 2)),
        # ignore_eos keeps going through EOS to the limit
        ((5, 2, 6), 3, True, ((5, 2, 6), (5, 2, 6), "length", 2)),
        # one token: prefill only, no decode
        ((7,), 1, False, ((7,), (7,), "length", 0)),
        # EOS as the very first token
        ((2, 5), 2, False, ((2,), (), "eos", 0)),
    ],
)
def test_generate_stopping_rules_on_scripted_logits(monkeypatch, script, max_new, ignore_eos, expected):
    scripted = _Scripted(script)
    monkeypatch.setattr(dref, "prefill", scripted.prefill)
    monkeypatch.setattr(dref, "decode", scripted.decode)
    greedy, emitted, reason = dref.generate(torch.tensor([[1, 3, 4]]), None, max_new_tokens=max_new, ignore_eos=ignore_eos)
    assert (greedy, emitted, reason, scripted.decodes) == expected


def test_generate_validates_like_the_reference():
    ids = torch.tensor([[1, 2]])
    for kwargs, needle in (
        (dict(max_new_tokens=0), "1 to 256"),
        (dict(max_new_tokens=257), "1 to 256"),
        (dict(max_new_tokens=True), "1 to 256"),
        (dict(ignore_eos=1), "boolean"),
    ):
        with pytest.raises(ValueError, match=needle):
            dref.generate(ids, None, **kwargs)
    with pytest.raises(ValueError, match=r"\[1, tokens\]"):
        dref.generate(torch.tensor([[1], [2]]), None)
    with pytest.raises(ValueError, match="2048"):
        dref.generate(torch.zeros((1, 1950), dtype=torch.int64), None, max_new_tokens=100)


@pytest.mark.parametrize("mistake", ["eos_id", "first_position"])
def test_planted_generate_mistakes_fail_the_scripted_cases(monkeypatch, mistake):
    """A wrong EOS id, or selecting from the first position instead of the last, changes the
    scripted streams above."""
    scripted = _Scripted((5, 6, 2, 7))
    prefill = scripted.prefill
    monkeypatch.setattr(dref, "decode", scripted.decode)
    if mistake == "eos_id":
        monkeypatch.setattr(dref, "EOS_TOKEN_ID", 3)
        monkeypatch.setattr(dref, "prefill", prefill)
    else:
        monkeypatch.setattr(dref, "prefill", lambda ids, w: (prefill(ids, w)[0][:, :1].flip(1), prefill(ids, w)[1]))
    try:
        result = dref.generate(torch.tensor([[1, 3, 4]]), None, max_new_tokens=4)
    except AssertionError:
        return  # the scripted decode saw a token it did not select
    assert result != ((5, 6, 2), (5, 6), "eos")
