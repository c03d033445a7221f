"""Pins the CPU decoder-shell oracle (oracle/decoder_shell.py) to the installed
transformers Qwen3 implementation, and to closed forms. CPU only.

The reference runs its packed linears inside the Transformers model shell
(src/nanoquant/runtime/transformers_generation.py:84-114), so
``Qwen3ForCausalLM`` with the packed linears' dense reconstructions as weights
is the reference decoder. Planted mistakes in the oracle must break the match.
"""

from __future__ import annotations

import pytest
import torch

from nanoquant_amd import synthetic as syn
from nanoquant_amd.runtime.decoder_shell import DecoderShellConfig
from oracle import decoder_shell as ods
from oracle.nq_oracle import dense_forward, operands_from_state, relative_l2

transformers = pytest.importorskip("transformers")

GEOMETRY = DecoderShellConfig(layers=2, hidden=64, intermediate=160, q_heads=4, kv_heads=2, head_dim=32, vocab=97)
PROMPT = torch.tensor([5, 17, 3, 88, 41, 0, 63, 29, 70])
DECODE_STEPS = 4


def oracle_weights(weights) -> ods.ShellWeights:
    return ods.ShellWeights(
        weights.embed,
        weights.lm_head,
        weights.final_norm,
        [
            ods.LayerWeights(
                layer.input_norm, layer.post_norm, layer.q_norm, layer.k_norm,
                {role: operands_from_state(state) for role, state in layer.linears.items()},
            )
            for layer in weights.layers
        ],
    )


def geometry(config: DecoderShellConfig) -> ods.ShellGeometry:
    return ods.ShellGeometry(config.layers, config.hidden, config.intermediate, config.q_heads, config.kv_heads,
                             config.head_dim, config.vocab, config.eps, config.rope_theta)


def hf_model(config: DecoderShellConfig, weights):
    from transformers import Qwen3Config, Qwen3ForCausalLM

    hf_config = Qwen3Config(
        vocab_size=config.vocab, hidden_size=config.hidden, intermediate_size=config.intermediate,
        num_hidden_layers=config.layers, num_attention_heads=config.q_heads, num_key_value_heads=config.kv_heads,
        head_dim=config.head_dim, rms_norm_eps=config.eps, rope_theta=config.rope_theta,
        tie_word_embeddings=False, max_position_embeddings=256, attention_bias=False,
    )
    hf_config._attn_implementation = "eager"
    model = Qwen3ForCausalLM(hf_config).float().eval()

    def dense(state) -> torch.Tensor:
        op = operands_from_state(state)
        eye = torch.eye(op.in_features, dtype=torch.float64)
        return dense_forward(op, eye).T.float()

    with torch.no_grad():
        model.model.embed_tokens.weight.copy_(weights.embed.float())
        model.lm_head.weight.copy_(weights.lm_head.float())
        model.model.norm.weight.copy_(weights.final_norm.float())
        for block, layer in zip(model.model.layers, weights.layers):
            block.input_layernorm.weight.copy_(layer.input_norm.float())
            block.post_attention_layernorm.weight.copy_(layer.post_norm.float())
            block.self_attn.q_norm.weight.copy_(layer.q_norm.float())
            block.self_attn.k_norm.weight.copy_(layer.k_norm.float())
            for role in ("q_proj", "k_proj", "v_proj", "o_proj"):
                getattr(block.self_attn, role).weight.copy_(dense(layer.linears[role]))
            for role in ("gate_proj", "up_proj", "down_proj"):
                getattr(block.mlp, role).weight.copy_(dense(layer.linears[role]))
    return model


def hf_logits(model, prompt: torch.Tensor, steps: int) -> tuple[list[torch.Tensor], list[int]]:
    """Prefill logits of every prompt row, then the greedy decode steps' logits."""

    with torch.no_grad():
        out = model(input_ids=prompt[None], use_cache=True)
        rows = [out.logits[0]]
        cache = out.past_key_values
        tokens = []
        last = out.logits[0, -1]
        for _ in range(steps):
            token = int(torch.argmax(last))
            tokens.append(token)
            out = model(input_ids=torch.tensor([[token]]), past_key_values=cache, use_cache=True)
            cache = out.past_key_values
            last = out.logits[0, -1]
            rows.append(out.logits[0])
    return rows, tokens


def oracle_logits(decoder: ods.OracleDecoder, prompt: torch.Tensor, tokens: list[int]) -> list[torch.Tensor]:
    decoder.reset()
    rows = [decoder.forward(prompt, 0)]
    position = prompt.numel()
    for token in tokens:
        rows.append(decoder.forward(torch.tensor([token]), position))
        position += 1
    return rows


@pytest.fixture(scope="module")
def setup():
    torch.manual_seed(0)
    weights = syn.synthetic_decoder(GEOMETRY, seed=syn.BASE_SEED + 50, random_norms=True)
    model = hf_model(GEOMETRY, weights)
    reference, tokens = hf_logits(model, PROMPT, DECODE_STEPS)
    return weights, reference, tokens


def compare(decoder: ods.OracleDecoder, reference, tokens) -> float:
    got = oracle_logits(decoder, PROMPT, tokens)
    return max(relative_l2(a, b) for a, b in zip(got, reference))


def test_oracle_matches_transformers_qwen3(setup):
    weights, reference, tokens = setup
    decoder = ods.OracleDecoder(geometry(GEOMETRY), oracle_weights(weights), max_positions=64)
    assert compare(decoder, reference, tokens) < 1e-5
    greedy, _ = decoder.greedy(PROMPT, DECODE_STEPS)
    assert greedy == tokens


@pytest.mark.parametrize("mistake", ["rope_sign", "no_causal_mask", "norm_weight_dropped", "kv_group_order",
                                     "no_qk_norm", "silu_on_up"])
def test_planted_mistakes_break_the_match(setup, monkeypatch, mistake):
    weights, reference, tokens = setup
    ow = oracle_weights(weights)
    if mistake == "rope_sign":
        def bad_rope(x, cos, sin):
            half = x.shape[-1] // 2
            c = torch.cat((cos, cos), dim=-1)[:, None, :]
            s = torch.cat((sin, sin), dim=-1)[:, None, :]
            return x * c + torch.cat((x[..., half:], -x[..., :half]), dim=-1) * s
        monkeypatch.setattr(ods, "apply_rope", bad_rope)
    elif mistake == "no_causal_mask":
        def no_mask(self, layer, q, start):
            g = self.g
            keys = self.k_cache[layer].repeat_interleave(g.q_heads // g.kv_heads, dim=0)
            values = self.v_cache[layer].repeat_interleave(g.q_heads // g.kv_heads, dim=0)
            scores = torch.einsum("thd,hld->htl", q, keys) * (g.head_dim**-0.5)
            return torch.einsum("htl,hld->thd", torch.softmax(scores, dim=-1), values)
        monkeypatch.setattr(ods.OracleDecoder, "_attention", no_mask)
    elif mistake == "norm_weight_dropped":
        real = ods.rms_norm
        monkeypatch.setattr(ods, "rms_norm", lambda x, w, eps: real(x, torch.ones_like(w), eps))
    elif mistake == "kv_group_order":
        def tiled(self, layer, q, start):
            g = self.g
            group = g.q_heads // g.kv_heads
            keys = self.k_cache[layer].repeat(group, 1, 1)  # head h -> kv h % kv_heads
            values = self.v_cache[layer].repeat(group, 1, 1)
            t = q.shape[0]
            scores = torch.einsum("thd,hld->htl", q, keys) * (g.head_dim**-0.5)
            allowed = torch.arange(keys.shape[1])[None, :] <= (start + torch.arange(t))[:, None]
            scores = scores.masked_fill(~allowed[None], float("-inf"))
            return torch.einsum("htl,hld->thd", torch.softmax(scores, dim=-1), values)
        monkeypatch.setattr(ods.OracleDecoder, "_attention", tiled)
    elif mistake == "no_qk_norm":
        for layer in ow.layers:
            layer.q_norm = None
            layer.k_norm = None
    elif mistake == "silu_on_up":
        for layer in ow.layers:
            layer.linears["gate_proj"], layer.linears["up_proj"] = layer.linears["up_proj"], layer.linears["gate_proj"]
    decoder = ods.OracleDecoder(geometry(GEOMETRY), ow, max_positions=64)
    assert compare(decoder, reference, tokens) > 1e-3


def test_closed_forms():
    # RMSNorm of a constant row c is w * sign(c) (up to eps).
    x = torch.full((1, 16), 3.0)
    w = torch.linspace(0.5, 2.0, 16)
    assert torch.allclose(ods.rms_norm(x, w, 1e-6), w, rtol=1e-6)
    # RoPE at position 0 is the identity; at any position it preserves norms.
    cos, sin = ods.rope_tables(32, 1e6, 8)
    v = torch.randn(8, 3, 32)
    assert torch.equal(ods.apply_rope(v[:1], cos[:1], sin[:1]), v[:1])
    assert torch.allclose(ods.apply_rope(v, cos, sin).norm(dim=-1), v.norm(dim=-1), rtol=1e-5)
    # inv_freq[i] = theta^(-2i/D): first is 1, ratio between neighbours constant.
    inv = ods.inv_freq(32, 1e6)
    assert inv[0] == 1.0 and torch.allclose(inv[1:] / inv[:-1], torch.full((15,), 1e6 ** (-2 / 32)), rtol=1e-5)
