"""Batch-1 decoder shell (Qwen3 geometry) around the packed linears, on gfx950.

The reference decodes a packed model by running the Transformers model shell
with one ``PreparedLinear`` per projection and capturing the one-token step in
a CUDA graph (``TransformersGenerationModel``,
src/nanoquant/runtime/transformers_generation.py:37-260), driven by the
generation engine's ``GenerationModel.forward_step`` protocol
(src/nanoquant/runtime/generation.py:28-41). ``PackedDecoder`` is that model
shell built from this library's kernels instead:

* every projection is a packed linear on ``HipPackedBackend`` — Q/K/V and
  gate/up run as one batched call each: the decode stages for up to 16
  tokens, the MFMA prefill phases for a longer prompt;
* embedding, residual add + RMSNorm, q/k RMSNorm + RoPE + KV append,
  grouped-query attention (for a decode token one kernel per 64-row cache
  block, then a merge), SiLU product, the bf16 output projection and greedy
  selection are the HIP kernels of ``include/nqamd_shell.h``;
* a decode token folds the norms, the SiLU product and the residual adds into
  the packed calls (``linear_batch_fused``): 10 launches per layer (12 without
  the fused calls), 9 when the attention's merge also folds into the O
  projection's input (by default for caches of up to FOLD_MAX_BLOCKS blocks);
  the embedding writes the row statistics the first layer's folded norm reads,
  so a step is the layers, the embedding, the final norm, the output
  projection and the greedy selection;
* the KV cache is one device tensor per layer ``[kv_heads, max_positions,
  head_dim]``, and the token position lives in device memory, so one HIP graph
  of the whole one-token step replays for every position with no host
  synchronisation; ``generate_greedy`` replays a graph of STEPS_PER_GRAPH
  consecutive steps (the one-step graph for the remainder), keeps the chosen
  tokens on the device and synchronises once at the end.

``forward_step`` implements the reference's ``GenerationModel`` protocol for
batch 1 (a prompt without padding), returning ``[1, 1, vocab]`` fp32 logits
and itself as the cache handle.
"""

from __future__ import annotations

from dataclasses import dataclass, field
from typing import NamedTuple

import torch

from nanoquant_amd.runtime import shell_ops as ops
from nanoquant_amd.runtime.backend import PreparedLayer
from nanoquant_amd.runtime.hip_backend import HipPackedBackend
from nanoquant_amd.runtime.packed import PackedLayerState

ROLES = ("q_proj", "k_proj", "v_proj", "o_proj", "gate_proj", "up_proj", "down_proj")

# Cache blocks (64 rows each) up to which a decode token folds the attention's
# merge into the O projection by default. Measured on the 36-layer Qwen3-8B
# geometry, fused one-token steps with a bf16 cache, folded against unfolded:
# 571.5 / 554.7 tok/s at 10 blocks, 566.1 / 553.4 at 11, 560.2 / 551.6 at 13,
# 558.5 / 550.9 at 14, 555.9 / 550.6 at 15, 555.5 / 551.0 at 16, the most
# blocks the folded input holds.
FOLD_MAX_BLOCKS = 16

# Decode steps captured in one graph for greedy generation (the remainder
# replays the one-step graph). Each graph launch leaves a gap before its first
# kernel; measured on the same model and cache, tok/s with 1 / 2 / 4 / 8 / 16
# steps per graph: 570.6 / 572.2 / 572.1 / 573.0 / 572.9.
STEPS_PER_GRAPH = 8


class DecodeStep(NamedTuple):
    """Result of ``PackedDecoder.forward_step``: logits ``[1, 1, vocab]`` and the
    cache handle (the decoder itself, which owns its KV cache)."""

    logits: torch.Tensor
    cache: object | None


class DecoderShellError(ValueError):
    """A request the decoder shell does not support (batch > 1, padding, cache overflow)."""


@dataclass(frozen=True)
class DecoderShellConfig:
    layers: int = 36
    hidden: int = 4096
    intermediate: int = 12288
    q_heads: int = 32
    kv_heads: int = 8
    head_dim: int = 128
    vocab: int = 151936
    eps: float = 1e-6
    rope_theta: float = 1_000_000.0
    qk_norm: bool = True

    @staticmethod
    def qwen3_8b() -> "DecoderShellConfig":
        return DecoderShellConfig()

    def linear_dims(self) -> dict[str, tuple[int, int]]:
        """(in, out) of each projection role."""

        q, kv = self.q_heads * self.head_dim, self.kv_heads * self.head_dim
        return {
            "q_proj": (self.hidden, q),
            "k_proj": (self.hidden, kv),
            "v_proj": (self.hidden, kv),
            "o_proj": (q, self.hidden),
            "gate_proj": (self.hidden, self.intermediate),
            "up_proj": (self.hidden, self.intermediate),
            "down_proj": (self.intermediate, self.hidden),
        }


@dataclass
class DecoderLayerWeights:
    input_norm: torch.Tensor
    post_norm: torch.Tensor
    q_norm: torch.Tensor | None
    k_norm: torch.Tensor | None
    linears: dict[str, PackedLayerState]


@dataclass
class DecoderShellWeights:
    embed: torch.Tensor  # [vocab, hidden] bf16
    lm_head: torch.Tensor  # [vocab, hidden] bf16
    final_norm: torch.Tensor  # [hidden]
    layers: list[DecoderLayerWeights] = field(default_factory=list)


# Transformers names of the dense tensors of a Qwen3 checkpoint.
QWEN3_DENSE_NAMES = {
    "embed": "model.embed_tokens.weight",
    "lm_head": "lm_head.weight",
    "final_norm": "model.norm.weight",
    "input_norm": "model.layers.{layer}.input_layernorm.weight",
    "post_norm": "model.layers.{layer}.post_attention_layernorm.weight",
    "q_norm": "model.layers.{layer}.self_attn.q_norm.weight",
    "k_norm": "model.layers.{layer}.self_attn.k_norm.weight",
}
PACKED_LAYER_NAME = "blocks.{layer}.{module}.{role}"


def load_decoder_weights(
    artifact,
    dense: dict[str, torch.Tensor],
    config: DecoderShellConfig,
    *,
    device: torch.device | str = "cpu",
    layer_name: str = PACKED_LAYER_NAME,
    dense_names: dict[str, str] = QWEN3_DENSE_NAMES,
) -> DecoderShellWeights:
    """Decoder weights from a packed artifact (every projection, via
    ``OpenPackedArtifact.load_layer``) and the checkpoint's dense tensors
    (embeddings, norms, ``lm_head``; a missing ``lm_head`` means tied
    embeddings). Packed layer names follow `layer_name` with ``module`` =
    ``self_attn`` / ``mlp``."""

    def get(key: str, **fmt) -> torch.Tensor:
        name = dense_names[key].format(**fmt)
        if name not in dense:
            raise KeyError(f"dense tensor missing from the checkpoint: {name}")
        return dense[name].to(device)

    embed = get("embed")
    lm_head = dense[dense_names["lm_head"]].to(device) if dense_names["lm_head"] in dense else embed
    if tuple(embed.shape) != (config.vocab, config.hidden) or tuple(lm_head.shape) != (config.vocab, config.hidden):
        raise DecoderShellError("embedding / lm_head shapes do not match the configuration")
    dims = config.linear_dims()
    layers = []
    for layer in range(config.layers):
        linears = {}
        for i, role in enumerate(ROLES):
            state = artifact.load_layer(layer_name.format(layer=layer, module="self_attn" if i < 4 else "mlp",
                                                          role=role), device)
            if (state.spec.in_features, state.spec.out_features) != dims[role]:
                raise DecoderShellError(f"packed layer {state.spec.name} does not match the configuration")
            linears[role] = state
        qn = get("q_norm", layer=layer) if config.qk_norm else None
        kn = get("k_norm", layer=layer) if config.qk_norm else None
        layers.append(DecoderLayerWeights(get("input_norm", layer=layer), get("post_norm", layer=layer), qn, kn,
                                          linears))
    return DecoderShellWeights(embed, lm_head, get("final_norm"), layers)


def dense_tensors(weights: DecoderShellWeights, dense_names: dict[str, str] = QWEN3_DENSE_NAMES) -> dict[str, torch.Tensor]:
    """The dense tensors of `weights` under checkpoint names (inverse of the
    dense part of ``load_decoder_weights``)."""

    out = {dense_names["embed"]: weights.embed, dense_names["lm_head"]: weights.lm_head,
           dense_names["final_norm"]: weights.final_norm}
    for i, layer in enumerate(weights.layers):
        out[dense_names["input_norm"].format(layer=i)] = layer.input_norm
        out[dense_names["post_norm"].format(layer=i)] = layer.post_norm
        if layer.q_norm is not None:
            out[dense_names["q_norm"].format(layer=i)] = layer.q_norm
            out[dense_names["k_norm"].format(layer=i)] = layer.k_norm
    return out


def rope_tables(head_dim: int, theta: float, positions: int) -> tuple[torch.Tensor, torch.Tensor]:
    """cos/sin ``[positions, head_dim / 2]`` fp32 of ``position * inv_freq`` with
    ``inv_freq = 1 / theta^(arange(0, D, 2) / D)``, computed on the host in fp32
    like the Transformers default rotary embedding."""

    inv = 1.0 / (theta ** (torch.arange(0, head_dim, 2, dtype=torch.float) / head_dim))
    freqs = torch.arange(positions, dtype=torch.float)[:, None] * inv[None, :]
    return freqs.cos(), freqs.sin()


@dataclass
class _Buffers:
    """Activations of one forward over `tokens` rows (fixed addresses for graphs)."""

    tokens: int
    residual: torch.Tensor
    xn: torch.Tensor
    q: torch.Tensor
    k: torch.Tensor
    v: torch.Tensor
    q_rot: torch.Tensor
    attn: torch.Tensor
    o: torch.Tensor
    gate: torch.Tensor
    up: torch.Tensor
    act: torch.Tensor
    down: torch.Tensor
    final: torch.Tensor
    attn_ws: torch.Tensor
    o_slots: torch.Tensor      # fused decode: sums of residual^2 per 16 rows after the o-projection
    down_slots: torch.Tensor   # ... and after the down-projection


class PackedDecoder:
    """Batch-1 decoder over prepared packed linears; see the module docstring."""

    def __init__(
        self,
        config: DecoderShellConfig,
        weights: DecoderShellWeights,
        *,
        device: torch.device | str = "cuda",
        max_positions: int = 640,
        backend: HipPackedBackend | None = None,
        activation_dtype: torch.dtype = torch.bfloat16,
        cache_dtype: torch.dtype = torch.bfloat16,
        history_capacity: int = 4096,
        fuse_decode: bool = True,
        fold_attention_merge: bool | None = None,
    ) -> None:
        self.config = c = config
        self.device = torch.device(device)
        if self.device.type != "cuda":
            raise DecoderShellError("the packed decoder shell runs on a HIP device")
        if len(weights.layers) != c.layers:
            raise DecoderShellError("weights do not match the configured layer count")
        if c.q_heads % c.kv_heads or c.head_dim not in (64, 128, 256):
            raise DecoderShellError("unsupported attention geometry")
        if activation_dtype not in (torch.bfloat16, torch.float16, torch.float32):
            raise DecoderShellError("activation dtype must be BF16, F16 or F32")
        self.max_positions = int(max_positions)
        self.activation_dtype = activation_dtype
        self.cache_dtype = cache_dtype
        # The prompt pass's errors reach every later token through the KV cache
        # and compound over the layers. With fp32 activations it takes split
        # prefill operands (an fp16 value and its fp16 remainder, about 22
        # bits); with 16-bit activations, which the shell rounds to 8 (bf16) or
        # 11 (fp16) bits before every linear, one fp16 operand (11 bits) adds
        # less than that rounding and halves the prompt's MFMA work.
        operands = "split" if activation_dtype == torch.float32 else "fp16"
        self.backend = backend or HipPackedBackend(prefill_operands=operands)
        dev = self.device
        self.embed = weights.embed.to(dev, torch.bfloat16).contiguous()
        self.lm_head = weights.lm_head.to(dev, torch.bfloat16).contiguous()
        self.final_norm = weights.final_norm.to(dev).contiguous()
        self.layers: list[dict[str, PreparedLayer]] = []
        self.norms: list[tuple[torch.Tensor, torch.Tensor, torch.Tensor | None, torch.Tensor | None]] = []
        for layer in weights.layers:
            self.layers.append({role: self.backend.prepare(layer.linears[role], dev) for role in ROLES})
            qn = None if layer.q_norm is None or not c.qk_norm else layer.q_norm.to(dev).contiguous()
            kn = None if layer.k_norm is None or not c.qk_norm else layer.k_norm.to(dev).contiguous()
            self.norms.append((layer.input_norm.to(dev).contiguous(), layer.post_norm.to(dev).contiguous(), qn, kn))
        # One-token steps fold the RMSNorms, the SiLU product and the residual
        # adds into the packed calls (nq_linear_batch_fused) when every layer
        # allows it: fp16 scales, no sidecars, hidden a multiple of 64 up to 16384.
        self.fuse_decode = bool(fuse_decode) and self._fusable(weights)
        self.col_scales: list[tuple[torch.Tensor, ...]] = []
        if self.fuse_decode:
            for prepared, (in_norm, post_norm, _qn, _kn) in zip(self.layers, self.norms):
                self.col_scales.append(tuple(
                    self.backend.norm_column_scale(prepared[role], norm)
                    for role, norm in (("q_proj", in_norm), ("k_proj", in_norm), ("v_proj", in_norm),
                                       ("gate_proj", post_norm), ("up_proj", post_norm))))
        # One-token steps with the fused calls can also fold the attention's
        # second pass (the merge of its cache blocks) into the O projection's
        # input (input_kind="attention"): one launch fewer per layer, but every
        # O workgroup then reads all blocks' partials (blocks x 8 KB of fp16
        # outputs at 4096 columns). None chooses by the cache length: folded up
        # to FOLD_MAX_BLOCKS blocks, where the saved launch outweighs the reads.
        # The folded merge reads each block's output in fp16: by default only
        # with a 16-bit cache, whose values the attention output already carries.
        blocks = -(-self.max_positions // 64)
        fold = (blocks <= FOLD_MAX_BLOCKS and cache_dtype != torch.float32 if fold_attention_merge is None
                else bool(fold_attention_merge))
        self.fold_attention_merge = (
            fold and self.fuse_decode
            and ops.decode_attention_partials_supported(c.q_heads, c.kv_heads, c.head_dim, cache_dtype)
            and c.q_heads * c.head_dim <= 4096 and blocks <= 16 and (c.q_heads * blocks) % 2 == 0)
        cache_shape = (c.layers, c.kv_heads, self.max_positions, c.head_dim)
        self.k_cache = torch.zeros(cache_shape, dtype=cache_dtype, device=dev)
        self.v_cache = torch.zeros(cache_shape, dtype=cache_dtype, device=dev)
        cos, sin = rope_tables(c.head_dim, c.rope_theta, self.max_positions)
        self.cos, self.sin = cos.to(dev), sin.to(dev)
        self.scaling = c.head_dim**-0.5
        self.position = torch.zeros(1, dtype=torch.int32, device=dev)
        self.step = torch.zeros(1, dtype=torch.int32, device=dev)
        self.ids = torch.zeros(1, dtype=torch.int64, device=dev)
        self.history = torch.zeros(history_capacity, dtype=torch.int64, device=dev)
        self.logits = torch.empty(c.vocab, dtype=torch.float32, device=dev)
        self.proj_ws = torch.empty(ops.output_projection_workspace_bytes(c.vocab, c.hidden), dtype=torch.uint8, device=dev)
        self._decode_bufs: _Buffers | None = None
        self._graphs: dict[int, torch.cuda.CUDAGraph] = {}
        self.host_position = 0

    def _fusable(self, weights: DecoderShellWeights) -> bool:
        c = self.config
        if c.hidden % 64 or c.hidden > 16384:
            return False
        for layer in weights.layers:
            for state in layer.linears.values():
                if state.scale_pre.dtype != torch.float16 or state.scale_mid.dtype != torch.float16 \
                        or state.scale_post.dtype != torch.float16:
                    return False
                if state.outlier_indices is not None or state.patch_left is not None \
                        or getattr(state, "row_indices", None) is not None:
                    return False
        return True

    # -- buffers -----------------------------------------------------------------
    def _buffers(self, tokens: int) -> _Buffers:
        c, dev, act = self.config, self.device, self.activation_dtype
        q_width, kv_width = c.q_heads * c.head_dim, c.kv_heads * c.head_dim

        def f32(*shape):
            return torch.empty(shape, dtype=torch.float32, device=dev)

        def a(*shape):
            return torch.empty(shape, dtype=act, device=dev)

        return _Buffers(
            tokens, f32(tokens, c.hidden), a(tokens, c.hidden), f32(tokens, q_width), f32(tokens, kv_width),
            f32(tokens, kv_width), f32(tokens, c.q_heads, c.head_dim), a(tokens, q_width), f32(tokens, c.hidden),
            f32(tokens, c.intermediate), f32(tokens, c.intermediate), a(tokens, c.intermediate),
            f32(tokens, c.hidden), f32(tokens, c.hidden),
            torch.empty(
                ops.decode_attention_workspace_bytes(c.q_heads, c.kv_heads, c.head_dim, self.cache_dtype,
                                                     self.max_positions)
                if tokens == 1 else ops.attention_workspace_bytes(tokens, c.q_heads, c.head_dim, self.max_positions),
                dtype=torch.uint8, device=dev),
            f32(-(-c.hidden // 16)), f32(-(-c.hidden // 16)),
        )

    # -- one forward -----------------------------------------------------------------
    def _linears(self, xs: list[torch.Tensor], layers: list[PreparedLayer], outs: list[torch.Tensor], tokens: int) -> None:
        self.backend.linear_batch(xs, layers, outs=outs)

    def _forward(self, ids: torch.Tensor, b: _Buffers) -> None:
        """Embedding .. final norm for `b.tokens` rows at positions position[0] + t,
        then the logits and argmax partials of the last row."""

        c, t = self.config, b.tokens
        fused = t == 1 and self.fuse_decode
        # The fused step's first layer reads the embedding's row sums of squares
        # as later layers read the down projection's.
        ops.launch_embedding(ids, self.embed, out=b.residual, slots=b.down_slots.view(1, -1) if fused else None)
        for i, prepared in enumerate(self.layers):
            in_norm, post_norm, qn, kn = self.norms[i]
            qkv = [prepared["q_proj"], prepared["k_proj"], prepared["v_proj"]]
            if fused:
                # residual holds the embedding or the previous down projection (its epilogue)
                self.backend.linear_batch_fused([b.residual[0]] * 3, qkv, input_kind="rmsnorm", eps=c.eps,
                                                col_scales=list(self.col_scales[i][:3]), norm_slots=b.down_slots,
                                                outs=[b.q[0], b.k[0], b.v[0]])
            else:
                ops.launch_add_rmsnorm(b.residual, in_norm, c.eps, delta=b.down if i else None, out=b.xn)
                self._linears([b.xn] * 3, qkv, [b.q, b.k, b.v], t)
            if t == 1 and fused and self.fold_attention_merge:
                ops.launch_decode_attention_partials(
                    b.q, b.k, b.v, q_heads=c.q_heads, kv_heads=c.kv_heads, head_dim=c.head_dim, q_norm=qn,
                    k_norm=kn, eps=c.eps, cos=self.cos, sin=self.sin, position=self.position,
                    k_cache=self.k_cache[i], v_cache=self.v_cache[i], scaling=self.scaling, workspace=b.attn_ws,
                )
            elif t == 1:
                ops.launch_decode_attention(
                    b.q, b.k, b.v, q_heads=c.q_heads, kv_heads=c.kv_heads, head_dim=c.head_dim, q_norm=qn,
                    k_norm=kn, eps=c.eps, cos=self.cos, sin=self.sin, position=self.position,
                    k_cache=self.k_cache[i], v_cache=self.v_cache[i], scaling=self.scaling, out=b.attn,
                    workspace=b.attn_ws,
                )
            else:
                ops.launch_qk_norm_rope_cache(
                    b.q, b.k, b.v, q_heads=c.q_heads, kv_heads=c.kv_heads, head_dim=c.head_dim, q_norm=qn,
                    k_norm=kn, eps=c.eps, cos=self.cos, sin=self.sin, position=self.position,
                    k_cache=self.k_cache[i], v_cache=self.v_cache[i], q_out=b.q_rot,
                )
                ops.launch_attention(b.q_rot, self.k_cache[i], self.v_cache[i], position=self.position,
                                     scaling=self.scaling, out=b.attn, workspace=b.attn_ws)
            if fused:
                if self.fold_attention_merge:
                    self.backend.linear_batch_fused(
                        [b.attn_ws], [prepared["o_proj"]], input_kind="attention",
                        attention_position=self.position, attention_head_dim=c.head_dim,
                        attention_max_positions=self.max_positions, residuals=[b.residual[0]],
                        out_slots=[b.o_slots])
                else:
                    self.backend.linear_batch_fused([b.attn.view(-1)], [prepared["o_proj"]],
                                                    residuals=[b.residual[0]], out_slots=[b.o_slots])
                # gate and up in one workgroup per output tile: the epilogue writes
                # silu(gate) * up in the activation dtype, the down projection's input
                self.backend.linear_batch_fused([b.residual[0]] * 2, [prepared["gate_proj"], prepared["up_proj"]],
                                                input_kind="rmsnorm", eps=c.eps,
                                                col_scales=list(self.col_scales[i][3:]), norm_slots=b.o_slots,
                                                output_kind="silu_product", outs=[b.act[0]],
                                                output_dtype=self.activation_dtype)
                self.backend.linear_batch_fused([b.act[0]], [prepared["down_proj"]], residuals=[b.residual[0]],
                                                out_slots=[b.down_slots])
                continue
            self._linears([b.attn], [prepared["o_proj"]], [b.o], t)
            ops.launch_add_rmsnorm(b.residual, post_norm, c.eps, delta=b.o, out=b.xn)
            self._linears([b.xn] * 2, [prepared["gate_proj"], prepared["up_proj"]], [b.gate, b.up], t)
            ops.launch_silu_mul(b.gate, b.up, out=b.act)
            self._linears([b.act], [prepared["down_proj"]], [b.down], t)
        ops.launch_add_rmsnorm(b.residual, self.final_norm, c.eps, delta=None if fused else b.down, out=b.final)
        ops.launch_output_projection(b.final[t - 1], self.lm_head, logits=self.logits, workspace=self.proj_ws)

    def _decode_body(self) -> None:
        assert self._decode_bufs is not None
        self._forward(self.ids, self._decode_bufs)
        ops.launch_greedy_select(self.proj_ws, self.config.vocab, self.config.hidden, token_out=self.ids,
                                 history=self.history, step=self.step, position=self.position)

    def _decode_graph(self, steps: int = 1) -> torch.cuda.CUDAGraph:
        """Capture `steps` consecutive one-token steps once (each step reads
        the token, position and step counters the previous one advanced on the
        device). A warm-up run precedes the first capture (it allocates the
        packed calls' workspaces); it writes the cache row at the current
        position, which the step that follows rewrites, and its changes to the
        token, step and position counters are undone."""

        if steps not in self._graphs:
            saved = (self.position.clone(), self.step.clone(), self.ids.clone())
            if self._decode_bufs is None or not self._graphs:
                self._decode_bufs = self._decode_bufs or self._buffers(1)
                side = torch.cuda.Stream(self.device)
                side.wait_stream(torch.cuda.current_stream(self.device))
                with torch.cuda.stream(side):
                    self._decode_body()  # warm-up: allocates the packed-call workspaces
                torch.cuda.current_stream(self.device).wait_stream(side)
                self._restore(saved)
            graph = torch.cuda.CUDAGraph()
            with torch.cuda.graph(graph):
                for _ in range(steps):
                    self._decode_body()
            self._restore(saved)
            self._graphs[steps] = graph
        return self._graphs[steps]

    def _restore(self, saved: tuple[torch.Tensor, torch.Tensor, torch.Tensor]) -> None:
        self.position.copy_(saved[0])
        self.step.copy_(saved[1])
        self.ids.copy_(saved[2])

    # -- public API ------------------------------------------------------------------
    def reset(self) -> None:
        """Forget the sequence (the cache rows are overwritten as positions are reused)."""

        self.position.zero_()
        self.step.zero_()
        self.host_position = 0

    def prefill(self, prompt: torch.Tensor, *, start: int = 0) -> torch.Tensor:
        """Run `prompt` (int64 ids) at positions start..; returns the last row's
        logits (fp32 [vocab], the decoder's own buffer) and leaves the greedy
        partials in the workspace."""

        ids = prompt.reshape(-1).to(self.device, torch.int64).contiguous()
        t = ids.numel()
        if t < 1 or start + t > self.max_positions:
            raise DecoderShellError("prompt does not fit the KV cache")
        self.position.fill_(start)
        self._forward(ids, self._buffers(t))
        self.position.fill_(start + t)
        self.host_position = start + t
        return self.logits

    def generate_greedy(
        self, prompt: torch.Tensor, max_new_tokens: int, *, use_graph: bool = True, timings: dict | None = None
    ) -> torch.Tensor:
        """Greedy continuation of one prompt: prefill, then `max_new_tokens - 1`
        captured one-token steps, replayed STEPS_PER_GRAPH at a time from one
        graph and the remainder from the one-step graph (`use_graph=False`:
        eager launches). Tokens stay on the device; the
        only synchronisation is the caller's read of the result. With a
        `timings` dict, device events bracket the prefill and the decode steps
        and their milliseconds are stored under "prefill_ms" / "decode_ms"
        (this synchronises once at the end)."""

        if max_new_tokens < 1 or max_new_tokens > self.history.numel():
            raise DecoderShellError("max_new_tokens outside the history capacity")
        t = int(prompt.numel())
        if t + max_new_tokens - 1 > self.max_positions:
            raise DecoderShellError("prompt plus generated tokens exceed the KV cache")
        steps = max_new_tokens - 1
        graph = self._decode_graph() if use_graph else None
        multi = self._decode_graph(STEPS_PER_GRAPH) if use_graph and steps >= STEPS_PER_GRAPH else None
        if not use_graph:
            self._decode_bufs = self._decode_bufs or self._buffers(1)
        events = [torch.cuda.Event(enable_timing=True) for _ in range(3)] if timings is not None else None
        self.reset()
        if events:
            events[0].record()
        self.prefill(prompt)
        ops.launch_greedy_select(self.proj_ws, self.config.vocab, self.config.hidden, token_out=self.ids,
                                 history=self.history, step=self.step)
        if events:
            events[1].record()
        if graph is None:
            for _ in range(steps):
                self._decode_body()
        else:
            for _ in range(steps // STEPS_PER_GRAPH if multi is not None else 0):
                multi.replay()
            for _ in range(steps % STEPS_PER_GRAPH if multi is not None else steps):
                graph.replay()
        if events:
            events[2].record()
            events[2].synchronize()
            timings["prefill_ms"] = events[0].elapsed_time(events[1])
            timings["decode_ms"] = events[1].elapsed_time(events[2])
        self.host_position = t + max_new_tokens - 1
        return self.history[:max_new_tokens].clone()

    def forward_step(
        self,
        *,
        input_ids: torch.Tensor,
        attention_mask: torch.Tensor,
        position_ids: torch.Tensor,
        cache_position: torch.Tensor,
        cache: object | None,
        max_cache_length: int,
        workload: str,
        deterministic: bool,
    ):
        """``GenerationModel.forward_step`` (src/nanoquant/runtime/generation.py:28-41)
        for batch 1, so the reference's generation engine can drive this shell:
        prefill rows run eagerly, a one-token decode step replays the captured
        graph. Positions come from `cache_position` (device), so no host
        synchronisation is needed. Returns a ``DecodeStep`` (the engine reads
        its ``logits`` and ``cache``)."""

        if input_ids.ndim != 2 or input_ids.shape[0] != 1:
            raise DecoderShellError("the packed decoder shell serves batch 1")
        if not deterministic:
            raise DecoderShellError("the packed decoder shell is deterministic only")
        if max_cache_length > self.max_positions:
            raise DecoderShellError("max_cache_length exceeds the decoder's KV cache")
        if attention_mask.ndim != 2 or attention_mask.shape[0] != 1:
            raise DecoderShellError("attention mask must be [1, width] for the batch-1 shell")
        t = input_ids.shape[1]
        if cache is None:
            self.reset()
        self.position.copy_(cache_position.reshape(-1)[:1])
        if workload == "decode" and t == 1:
            self.ids.copy_(input_ids.reshape(1))
            self._decode_graph().replay()
        else:
            if bool((~attention_mask.bool()).any()):
                raise DecoderShellError("padded prompts are not supported by the batch-1 shell")
            self._forward(input_ids.reshape(-1).contiguous(), self._buffers(t))
        return DecodeStep(self.logits.clone().view(1, 1, -1), self)
