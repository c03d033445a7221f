"""Synthetic packed layers and model shapes for parity tests and benchmarks.

Signs are i.i.d. Bernoulli(0.5) bits written straight into packed words (pad
bits cleared, as the layout requires), scales are fp16 ``exp(N(0, 0.25^2))``,
activations are bf16 ``N(0, 1)``. Shapes follow the Gemma-3, Qwen3-8B and
Llama-3-8B projections at a chosen bits-per-weight, with
``rank = round(bpw * m * n / (m + n))``.
"""

from __future__ import annotations

import math
from dataclasses import dataclass

import torch

from nanoquant_amd.runtime.backend import QuantizedLinearSpec
from nanoquant_amd.runtime.packed import PACKED_LAYOUT_VERSION, PackedLayerState
from nanoquant_amd.runtime.row_sidecar import OutputRowSidecar, RowSidecarLayerState

BASE_SEED = 20260715


@dataclass(frozen=True)
class LinearShape:
    name: str
    in_features: int
    out_features: int
    rank: int

    @property
    def weight_bytes(self) -> int:
        """Sign words plus fp16 scales: 4*r*wc(in) + 4*out*wc(r) + 2*(in+r+out)."""

        wc = lambda c: -(-c // 32)  # noqa: E731
        return (
            4 * self.rank * wc(self.in_features)
            + 4 * self.out_features * wc(self.rank)
            + 2 * (self.in_features + self.rank + self.out_features)
        )

    @property
    def flops_per_token(self) -> int:
        return 2 * self.rank * (self.in_features + self.out_features)


def rank_for(in_features: int, out_features: int, bpw: float = 1.0) -> int:
    return int(round(bpw * in_features * out_features / (in_features + out_features)))


def qwen3_8b_layer(layer: int = 0, bpw: float = 1.0) -> list[LinearShape]:
    """The seven projections of a Qwen3-8B decoder layer (hidden 4096,
    intermediate 12288, 32 q / 8 kv heads x 128)."""

    hidden, inter, kv = 4096, 12288, 1024
    dims = (
        ("self_attn.q_proj", hidden, hidden),
        ("self_attn.k_proj", hidden, kv),
        ("self_attn.v_proj", hidden, kv),
        ("self_attn.o_proj", hidden, hidden),
        ("mlp.gate_proj", hidden, inter),
        ("mlp.up_proj", hidden, inter),
        ("mlp.down_proj", inter, hidden),
    )
    return [
        LinearShape(f"blocks.{layer}.{name}", i, o, rank_for(i, o, bpw)) for name, i, o in dims
    ]


def llama3_8b_layer(layer: int = 0, bpw: float = 0.8) -> list[LinearShape]:
    """Llama-3-8B projections (hidden 4096, intermediate 14336, kv dim 1024)."""

    hidden, inter, kv = 4096, 14336, 1024
    dims = (
        ("self_attn.q_proj", hidden, hidden),
        ("self_attn.k_proj", hidden, kv),
        ("self_attn.v_proj", hidden, kv),
        ("self_attn.o_proj", hidden, hidden),
        ("mlp.gate_proj", hidden, inter),
        ("mlp.up_proj", hidden, inter),
        ("mlp.down_proj", inter, hidden),
    )
    return [
        LinearShape(f"blocks.{layer}.{name}", i, o, rank_for(i, o, bpw)) for name, i, o in dims
    ]


def gemma3_1b_gate() -> LinearShape:
    return LinearShape("blocks.0.mlp.gate_proj", 1152, 6912, 768)


def gemma3_4b_down() -> LinearShape:
    return LinearShape("blocks.0.mlp.down_proj", 10240, 2560, 1536)


def _random_words(rows: int, cols: int, g: torch.Generator, device: torch.device) -> torch.Tensor:
    words = torch.randint(
        -(2**31), 2**31, (rows, -(-cols // 32)), generator=g, dtype=torch.int64, device=device
    ).to(torch.int32)
    tail = cols % 32
    if tail:
        words[:, -1] &= (1 << tail) - 1
    return words.contiguous()


def _lognormal(n: int, g: torch.Generator, device: torch.device, dtype: torch.dtype) -> torch.Tensor:
    return torch.exp(0.25 * torch.randn(n, generator=g, device=device)).to(dtype)


def synthetic_packed_layer(
    shape: LinearShape,
    *,
    seed: int,
    scale_dtype: torch.dtype = torch.float16,
    salient: int = 0,
    salient_dtype: torch.dtype | None = None,
    bias: bool = False,
    device: str | torch.device = "cpu",
) -> PackedLayerState:
    """A random packed layer; with ``salient > 0`` the salient input columns are
    sorted unique indices and ``scale_pre`` is zeroed there (layout invariant)."""

    device = torch.device(device)
    g = torch.Generator(device=device).manual_seed(seed)
    right = _random_words(shape.rank, shape.in_features, g, device)
    left = _random_words(shape.out_features, shape.rank, g, device)
    s_in = _lognormal(shape.in_features, g, device, scale_dtype)
    s_mid = _lognormal(shape.rank, g, device, scale_dtype)
    s_out = _lognormal(shape.out_features, g, device, scale_dtype)
    indices = values = scales = None
    value_dtype = None
    if salient:
        value_dtype = salient_dtype or torch.int8
        perm = torch.randperm(shape.in_features, generator=g, device=device)[:salient]
        indices = torch.sort(perm).values.to(torch.int32)
        s_in[indices.long()] = 0
        if value_dtype == torch.int8:
            values = torch.randint(
                -127, 128, (shape.out_features, salient), generator=g, device=device
            ).to(torch.int8)
            scales = (_lognormal(salient, g, device, torch.float32) / 127).to(scale_dtype)
        else:
            values = torch.randn(shape.out_features, salient, generator=g, device=device).to(
                value_dtype
            )
    bias_t = torch.randn(shape.out_features, generator=g, device=device).to(scale_dtype) if bias else None
    spec = QuantizedLinearSpec(
        shape.name,
        "nanoquant-v1",
        shape.in_features,
        shape.out_features,
        shape.rank,
        "float32",
        str(scale_dtype).removeprefix("torch."),
        outlier_count=salient,
        outlier_value_dtype=None if not salient else str(value_dtype).removeprefix("torch."),
        has_outlier_scales=bool(salient) and value_dtype == torch.int8,
        has_bias=bias,
    )
    return PackedLayerState(
        spec,
        PACKED_LAYOUT_VERSION,
        left,
        right,
        s_in,
        s_mid,
        s_out,
        bias_t,
        indices,
        values,
        scales,
    )


def synthetic_row_sidecar(
    base: PackedLayerState, rows: int, *, seed: int
) -> RowSidecarLayerState:
    """``rows`` output rows (sorted, unique) stored as dense int8 in [-127, 127]
    with fp16 per-row scales ``lognormal(0, 0.25) / 127``."""

    device = base.left_words.device
    spec = base.spec
    g = torch.Generator(device=device).manual_seed(seed)
    idx = torch.sort(torch.randperm(spec.out_features, generator=g, device=device)[:rows]).values
    values = torch.randint(-127, 128, (rows, spec.in_features), generator=g, device=device).to(
        torch.int8
    )
    scales = (_lognormal(rows, g, device, torch.float32) / 127).to(base.scale_pre.dtype)
    return RowSidecarLayerState(base, OutputRowSidecar(idx.to(torch.int32), values, scales))


def synthetic_activations(
    tokens: int, in_features: int, *, seed: int, dtype: torch.dtype = torch.bfloat16,
    device: str | torch.device = "cpu",
) -> torch.Tensor:
    g = torch.Generator(device=torch.device(device)).manual_seed(seed)
    return torch.randn(tokens, in_features, generator=g, device=torch.device(device)).to(dtype)


def bits_per_weight(shape: LinearShape) -> float:
    return 8.0 * shape.weight_bytes / (shape.in_features * shape.out_features)


def model_weight_bytes(shapes: list[LinearShape]) -> int:
    return int(math.fsum(s.weight_bytes for s in shapes))


def synthetic_decoder(
    config,
    *,
    seed: int = BASE_SEED + 5,
    device: str | torch.device = "cpu",
    bpw: float = 1.0,
    random_norms: bool = False,
):
    """A random-init decoder of ``config`` (a ``DecoderShellConfig``): every
    projection a packed linear at ``bpw`` (rank ``round(bpw*m*n/(m+n))``),
    embeddings and untied ``lm_head`` bf16 ``N(0, 0.02)``, norm weights ones
    (the Transformers initialisation) or, with ``random_norms``,
    ``1 + 0.1 N(0, 1)`` so that tests see every weight applied."""

    from nanoquant_amd.runtime.decoder_shell import ROLES, DecoderLayerWeights, DecoderShellWeights

    device = torch.device(device)
    g = torch.Generator(device=device).manual_seed(seed)
    dims = config.linear_dims()

    def dense(rows: int, cols: int) -> torch.Tensor:
        return (0.02 * torch.randn(rows, cols, generator=g, device=device)).to(torch.bfloat16)

    def norm(n: int) -> torch.Tensor:
        if not random_norms:
            return torch.ones(n, dtype=torch.float32, device=device)
        return 1.0 + 0.1 * torch.randn(n, generator=g, device=device)

    embed = dense(config.vocab, config.hidden)
    lm_head = dense(config.vocab, config.hidden)
    final_norm = norm(config.hidden)
    layers = []
    for layer in range(config.layers):
        linears = {}
        for r, role in enumerate(ROLES):
            i, o = dims[role]
            prefix = "self_attn" if r < 4 else "mlp"
            shape = LinearShape(f"blocks.{layer}.{prefix}.{role}", i, o, rank_for(i, o, bpw))
            linears[role] = synthetic_packed_layer(shape, seed=seed + 1000 * (layer + 1) + r, device=device)
        layers.append(
            DecoderLayerWeights(norm(config.hidden), norm(config.hidden), norm(config.head_dim),
                                norm(config.head_dim), linears)
        )
    return DecoderShellWeights(embed, lm_head, final_norm, layers)
