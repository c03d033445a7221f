"""CPU oracle for the batch-1 decoder shell around the packed linears — TEST
INFRASTRUCTURE ONLY.

This module checks the product and is never part of it: only ``tests/``,
``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of ``bench.py`` may
import it.

The reference runs its packed linears inside the Transformers model shell
(src/nanoquant/runtime/transformers_generation.py:84-114, one
``PreparedLinear`` per projection), so the decoder algorithm is that of the
installed transformers 5.15.0 Qwen3 model, restated here in fp32 torch on the
CPU with the packed linears evaluated by the oracle's
``CpuPackedForward`` (the reference's ``PackedReferenceBackend``):

* RMSNorm ``w * (x * rsqrt(mean(x^2) + eps))`` (modeling_qwen3.py
  ``Qwen3RMSNorm``), applied before attention and MLP, per head to q and k,
  and after the last layer;
* default RoPE: ``inv_freq = 1 / theta^(arange(0, D, 2) / D)``, angle
  ``position * inv_freq`` in fp32, rotate-half form
  ``x * cos + rotate_half(x) * sin`` (``Qwen3RotaryEmbedding``,
  ``apply_rotary_pos_emb``);
* grouped-query causal attention, scaling ``D^-0.5``, softmax in fp32
  (``eager_attention_forward``, ``repeat_kv``);
* ``down(silu(gate(x)) * up(x))`` (``Qwen3MLP``); residual adds around both
  blocks (``Qwen3DecoderLayer``); untied ``lm_head`` on the final norm;
* greedy selection ``argmax`` (src/nanoquant/runtime/generation.py:240-246).

Pinning: tests/test_decoder_shell_oracle.py runs the installed transformers
``Qwen3ForCausalLM`` (eager attention, fp32, KV cache) on a small geometry with
the packed linears' dense reconstructions as its weights and requires this
restatement to agree on prefill and decode logits; plus closed forms (RMSNorm
of a constant row, RoPE at position 0 is the identity, a single cache row
gives attention output = v, softmax rows sum to one).

Optional rounding points (``activation_dtype``, ``cache_dtype``) round the
linear inputs and the KV cache the way a bf16 shell does, so the GPU shell can
also be compared at its deployed precision.
"""

from __future__ import annotations

from dataclasses import dataclass, field

import torch
from torch.nn import functional as F

from oracle.nq_oracle import CpuPackedForward, PackedOperands

ROLES = ("q_proj", "k_proj", "v_proj", "o_proj", "gate_proj", "up_proj", "down_proj")


@dataclass(frozen=True)
class ShellGeometry:
    layers: int
    hidden: int
    intermediate: int
    q_heads: int
    kv_heads: int
    head_dim: int
    vocab: int
    eps: float = 1e-6
    rope_theta: float = 1_000_000.0


@dataclass
class LayerWeights:
    input_norm: torch.Tensor
    post_norm: torch.Tensor
    q_norm: torch.Tensor | None
    k_norm: torch.Tensor | None
    linears: dict[str, PackedOperands]


@dataclass
class ShellWeights:
    embed: torch.Tensor  # [vocab, hidden]
    lm_head: torch.Tensor  # [vocab, hidden]
    final_norm: torch.Tensor  # [hidden]
    layers: list[LayerWeights] = field(default_factory=list)


def inv_freq(head_dim: int, theta: float) -> torch.Tensor:
    return 1.0 / (theta ** (torch.arange(0, head_dim, 2, dtype=torch.float) / head_dim))


def rope_tables(head_dim: int, theta: float, positions: int) -> tuple[torch.Tensor, torch.Tensor]:
    """cos/sin ``[positions, head_dim / 2]`` fp32 of ``position * inv_freq``."""

    freqs = torch.arange(positions, dtype=torch.float)[:, None] * inv_freq(head_dim, theta)[None, :]
    return freqs.cos(), freqs.sin()


def rms_norm(x: torch.Tensor, weight: torch.Tensor, eps: float) -> torch.Tensor:
    x32 = x.float()
    variance = x32.pow(2).mean(-1, keepdim=True)
    return weight.float() * (x32 * torch.rsqrt(variance + eps))


def apply_rope(x: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor) -> torch.Tensor:
    """x ``[T, heads, D]``; cos/sin ``[T, D/2]``."""

    half = x.shape[-1] // 2
    c = torch.cat((cos, cos), dim=-1)[:, None, :]
    s = torch.cat((sin, sin), dim=-1)[:, None, :]
    rotated = torch.cat((-x[..., half:], x[..., :half]), dim=-1)
    return x * c + rotated * s


def _round(x: torch.Tensor, dtype: torch.dtype) -> torch.Tensor:
    return x if dtype == torch.float32 else x.to(dtype).float()


class OracleDecoder:
    """fp32 CPU decoder with a KV cache; ``forward(ids, start)`` returns the
    logits of every input row (positions ``start .. start + T - 1``)."""

    def __init__(
        self,
        geometry: ShellGeometry,
        weights: ShellWeights,
        *,
        max_positions: int,
        activation_dtype: torch.dtype = torch.float32,
        cache_dtype: torch.dtype = torch.float32,
    ) -> None:
        self.g = geometry
        self.w = weights
        self.max_positions = max_positions
        self.activation_dtype = activation_dtype
        self.cache_dtype = cache_dtype
        self.linears = [
            {role: CpuPackedForward(layer.linears[role]) for role in ROLES} for layer in weights.layers
        ]
        self.cos, self.sin = rope_tables(geometry.head_dim, geometry.rope_theta, max_positions)
        self.reset()

    def reset(self) -> None:
        g = self.g
        shape = (g.kv_heads, 0, g.head_dim)
        self.k_cache = [torch.zeros(shape) for _ in range(g.layers)]
        self.v_cache = [torch.zeros(shape) for _ in range(g.layers)]

    def _attention(self, layer: int, q: torch.Tensor, start: int) -> torch.Tensor:
        g = self.g
        group = g.q_heads // g.kv_heads
        keys = self.k_cache[layer].repeat_interleave(group, dim=0)  # [Hq, L, D]
        values = self.v_cache[layer].repeat_interleave(group, dim=0)
        t = q.shape[0]
        scores = torch.einsum("thd,hld->htl", q, keys) * (g.head_dim**-0.5)
        length = keys.shape[1]
        allowed = torch.arange(length)[None, :] <= (start + torch.arange(t))[:, None]
        scores = scores.masked_fill(~allowed[None, :, :], float("-inf"))
        probs = torch.softmax(scores, dim=-1)
        return torch.einsum("htl,hld->thd", probs, values)

    def forward(self, ids: torch.Tensor, start: int) -> torch.Tensor:
        g, w = self.g, self.w
        t = ids.numel()
        if start + t > self.max_positions:
            raise ValueError("oracle decoder cache overflow")
        act = self.activation_dtype
        h = w.embed[ids.long()].float()
        cos, sin = self.cos[start : start + t], self.sin[start : start + t]
        for i, layer in enumerate(w.layers):
            lin = self.linears[i]
            x = _round(rms_norm(h, layer.input_norm, g.eps), act)
            q = lin["q_proj"](x).view(t, g.q_heads, g.head_dim)
            k = lin["k_proj"](x).view(t, g.kv_heads, g.head_dim)
            v = lin["v_proj"](x).view(t, g.kv_heads, g.head_dim)
            if layer.q_norm is not None:
                q = rms_norm(q, layer.q_norm, g.eps)
            if layer.k_norm is not None:
                k = rms_norm(k, layer.k_norm, g.eps)
            q = apply_rope(q, cos, sin)
            k = _round(apply_rope(k, cos, sin), self.cache_dtype)
            v = _round(v, self.cache_dtype)
            self.k_cache[i] = torch.cat((self.k_cache[i], k.transpose(0, 1)), dim=1)
            self.v_cache[i] = torch.cat((self.v_cache[i], v.transpose(0, 1)), dim=1)
            attn = _round(self._attention(i, q, start).reshape(t, -1), act)
            h = h + lin["o_proj"](attn)
            x = _round(rms_norm(h, layer.post_norm, g.eps), act)
            mlp_in = _round(F.silu(lin["gate_proj"](x)) * lin["up_proj"](x), act)
            h = h + lin["down_proj"](mlp_in)
        x = rms_norm(h, w.final_norm, g.eps)
        return x @ w.lm_head.float().T

    def greedy(self, prompt: torch.Tensor, new_tokens: int) -> tuple[list[int], list[torch.Tensor]]:
        """Greedy continuation: the generated ids and the logits each was taken from."""

        self.reset()
        logits = self.forward(prompt, 0)[-1]
        tokens, history = [], []
        position = prompt.numel()
        for step in range(new_tokens):
            history.append(logits)
            token = int(torch.argmax(logits))
            tokens.append(token)
            if step + 1 == new_tokens:
                break
            logits = self.forward(torch.tensor([token]), position)[-1]
            position += 1
        return tokens, history
