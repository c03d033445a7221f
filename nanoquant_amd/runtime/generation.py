"""Deterministic autoregressive generation engine (the reference runtime's API).

Same types, fields, error codes and stopping semantics as the reference's
engine (src/nanoquant/runtime/generation.py:14-425), so a model shell written
for either runs under either: ``GenerationModel.forward_step`` returns a
``GenerationStep`` with ``[batch, 1, vocab]`` logits and an opaque cache
handle; ``generate`` prefills (optionally in chunks), then selects one token
per row per step on the device (greedy ``argmax`` or seeded sampling with
temperature / top-k / top-p), tracks EOS and stop sequences per row, and
synchronises with the host only every ``stopping_check_interval`` steps and
once at the end.

With ``PackedDecoder`` (batch 1) every decode step is one HIP-graph replay.
"""

from __future__ import annotations

import math
from collections.abc import Sequence
from dataclasses import dataclass
from typing import Literal, Protocol, runtime_checkable

import torch


class GenerationError(ValueError):
    """A generation request or a model result that breaks the runtime contract."""


@dataclass(frozen=True, slots=True)
class GenerationStep:
    logits: torch.Tensor
    cache: object | None


@runtime_checkable
class GenerationModel(Protocol):
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
    ) -> GenerationStep: ...


@dataclass(frozen=True, slots=True)
class SamplingConfig:
    mode: Literal["greedy", "sample"] = "greedy"
    temperature: float = 1.0
    top_k: int | None = None
    top_p: float | None = None
    seed: int | None = None

    def __post_init__(self) -> None:
        fail = lambda why: GenerationError(f"NQ-GEN-SAMPLING {why}")  # noqa: E731
        if self.mode not in ("greedy", "sample"):
            raise fail(f"unsupported sampling mode: {self.mode}")
        if not (math.isfinite(self.temperature) and self.temperature > 0):
            raise fail("temperature must be finite and positive")
        if self.top_k is not None and self.top_k <= 0:
            raise fail("top_k must be positive when configured")
        if self.top_p is not None and not (math.isfinite(self.top_p) and 0 < self.top_p <= 1):
            raise fail("top_p must be in (0, 1]")
        if self.seed is not None and self.seed < 0:
            raise fail("seed must be non-negative")
        sampling_only = (self.temperature != 1.0, self.top_k is not None, self.top_p is not None,
                         self.seed is not None)
        if self.mode == "greedy" and any(sampling_only):
            raise fail("greedy mode does not accept sampling-only settings")
        if self.mode == "sample" and self.seed is None:
            raise fail("deterministic sampling requires an explicit seed")


@dataclass(frozen=True, slots=True)
class GenerationRequest:
    input_ids: torch.Tensor
    attention_mask: torch.Tensor
    max_new_tokens: int
    eos_token_ids: tuple[int, ...]
    pad_token_id: int
    deterministic: bool = True
    stop_token_sequences: tuple[tuple[int, ...], ...] = ()
    sampling: SamplingConfig = SamplingConfig()
    stopping_check_interval: int = 1
    prefill_chunk_size: int | None = None


@dataclass(frozen=True, slots=True)
class GenerationResult:
    token_ids: torch.Tensor
    lengths: tuple[int, ...]
    stop_reasons: tuple[str, ...]
    prefill_forward_count: int
    decode_forward_count: int
    maximum_cache_length: int
    stopping_sync_count: int
    terminal_sync_count: int


def batch_prompts(
    prompts: Sequence[Sequence[int]], *, pad_token_id: int, device: torch.device | str | None = None
) -> tuple[torch.Tensor, torch.Tensor]:
    """Left-padded ``[batch, width]`` ids and boolean mask (the last column is
    valid for every row)."""

    if pad_token_id < 0:
        raise GenerationError("NQ-GEN-TOKEN-ID the pad token ID must be non-negative")
    rows = [[int(token) for token in prompt] for prompt in prompts]
    if not rows:
        raise GenerationError("NQ-GEN-EMPTY prompt batches must be non-empty")
    if any(len(row) == 0 for row in rows):
        raise GenerationError("NQ-GEN-EMPTY every prompt row must contain at least one token")
    if any(token < 0 for row in rows for token in row):
        raise GenerationError("NQ-GEN-TOKEN-ID prompt token IDs must be non-negative")
    width = max(len(row) for row in rows)
    ids = torch.full((len(rows), width), pad_token_id, dtype=torch.long)
    mask = torch.zeros((len(rows), width), dtype=torch.bool)
    for i, row in enumerate(rows):
        ids[i, width - len(row):] = torch.tensor(row, dtype=torch.long)
        mask[i, width - len(row):] = True
    return ids.to(device), mask.to(device)


def _validated_mask(request: GenerationRequest) -> torch.Tensor:
    ids, mask = request.input_ids, request.attention_mask
    if ids.ndim != 2 or mask.ndim != 2 or ids.shape != mask.shape:
        raise GenerationError("NQ-GEN-SHAPE input IDs and attention mask must have one equal 2D shape")
    if ids.dtype != torch.long:
        raise GenerationError("NQ-GEN-TOKEN-DTYPE input IDs must use torch.long")
    if ids.device != mask.device:
        raise GenerationError("NQ-GEN-DEVICE input IDs and attention mask must share a device")
    if ids.shape[0] <= 0 or ids.shape[1] <= 0:
        raise GenerationError("NQ-GEN-EMPTY prompt batches and prompt widths must be non-empty")
    if request.max_new_tokens <= 0:
        raise GenerationError("NQ-GEN-LIMIT max_new_tokens must be positive")
    eos = request.eos_token_ids
    if not eos or len(set(eos)) != len(eos):
        raise GenerationError("NQ-GEN-EOS EOS token IDs must be non-empty and unique")
    if request.pad_token_id < 0 or min(eos) < 0:
        raise GenerationError("NQ-GEN-TOKEN-ID pad and EOS token IDs must be non-negative")
    if bool((ids < 0).any()):
        raise GenerationError("NQ-GEN-TOKEN-ID prompt token IDs must be non-negative")
    stops = request.stop_token_sequences
    if len(set(stops)) != len(stops):
        raise GenerationError("NQ-GEN-STOP stop token sequences must be unique")
    if any(len(seq) == 0 for seq in stops):
        raise GenerationError("NQ-GEN-STOP stop token sequences must be non-empty")
    if any(token < 0 for seq in stops for token in seq):
        raise GenerationError("NQ-GEN-TOKEN-ID stop token IDs must be non-negative")
    if not request.deterministic:
        raise GenerationError("NQ-GEN-MODE the generation engine requires deterministic model execution")
    if request.stopping_check_interval <= 0:
        raise GenerationError("NQ-GEN-SYNC stopping_check_interval must be positive")
    chunk = request.prefill_chunk_size
    if chunk is not None and (type(chunk) is not int or chunk <= 0):
        raise GenerationError("NQ-GEN-PREFILL prefill_chunk_size must be positive when configured")
    as_bool = mask.bool()
    if not bool((mask == as_bool).all()):
        raise GenerationError("NQ-GEN-MASK attention mask values must be boolean or zero/one")
    if bool((as_bool.sum(dim=1) == 0).any()):
        raise GenerationError("NQ-GEN-EMPTY every prompt row must contain at least one token")
    if not bool(as_bool[:, -1].all()):
        raise GenerationError("NQ-GEN-PADDING prompt batches must use left padding")
    if as_bool.shape[1] > 1 and bool((as_bool[:, :-1] & ~as_bool[:, 1:]).any()):
        raise GenerationError("NQ-GEN-PADDING attention masks must be contiguous left padding")
    return as_bool


def _check_step(step: GenerationStep, batch: int, workload: str, device: torch.device) -> None:
    logits = step.logits
    if logits.ndim != 3 or logits.shape[0] != batch or logits.shape[1] != 1:
        raise GenerationError(f"NQ-GEN-LOGITS runtime {workload} must return logits shaped [batch, 1, vocabulary]")
    if logits.shape[2] <= 0 or not logits.dtype.is_floating_point:
        raise GenerationError("NQ-GEN-LOGITS model logits must have a floating vocabulary dimension")
    if logits.device != device:
        raise GenerationError(f"NQ-GEN-DEVICE runtime {workload} logits must remain on {device}")


def select_tokens(logits: torch.Tensor, config: SamplingConfig, generator: torch.Generator | None) -> torch.Tensor:
    """Greedy ``argmax`` (lowest index on ties), or a seeded draw from the
    temperature-scaled distribution restricted to the top-k and to the smallest
    prefix of descending probability whose mass reaches top-p."""

    if config.mode == "greedy":
        return torch.argmax(logits, dim=-1)
    scaled = logits.float() / config.temperature
    if config.top_k is not None:
        kth = torch.topk(scaled, min(config.top_k, scaled.shape[-1]), dim=-1).values[..., -1:]
        scaled = scaled.masked_fill(scaled < kth, -torch.inf)
    if config.top_p is not None and config.top_p < 1:
        ordered, order = torch.sort(scaled, descending=True, dim=-1)
        mass = torch.softmax(ordered, dim=-1).cumsum(dim=-1)
        drop = torch.zeros_like(mass, dtype=torch.bool)
        drop[..., 1:] = mass[..., :-1] > config.top_p  # keep the token that crosses top-p
        ordered = ordered.masked_fill(drop, -torch.inf)
        scaled = torch.full_like(scaled, -torch.inf).scatter(-1, order, ordered)
    return torch.multinomial(torch.softmax(scaled, dim=-1), 1, generator=generator).squeeze(-1)


def generate(request: GenerationRequest, model: GenerationModel) -> GenerationResult:
    mask = _validated_mask(request)
    ids = request.input_ids
    device = ids.device
    batch, width = ids.shape
    total = width + request.max_new_tokens
    positions = torch.arange(width, dtype=torch.long, device=device).expand(batch, -1).clone()
    positions.masked_fill_(~mask, 0)
    prompt_cache_positions = torch.arange(width, dtype=torch.long, device=device)
    decode_cache_positions = torch.arange(width, total, dtype=torch.long, device=device)
    full_mask = torch.zeros((batch, total), dtype=torch.bool, device=device)
    full_mask[:, :width] = mask
    eos = torch.tensor(request.eos_token_ids, dtype=torch.long, device=device)
    stops = tuple(torch.tensor(seq, dtype=torch.long, device=device) for seq in request.stop_token_sequences)
    generator = None
    if request.sampling.mode == "sample":
        generator = torch.Generator(device=device)
        generator.manual_seed(request.sampling.seed)

    with torch.inference_mode():
        chunk = request.prefill_chunk_size or width
        cache: object | None = None
        step: GenerationStep | None = None
        prefill_count = 0
        for begin in range(0, width, chunk):
            end = min(begin + chunk, width)
            step = model.forward_step(
                input_ids=ids[:, begin:end], attention_mask=full_mask[:, :end],
                position_ids=positions[:, begin:end], cache_position=prompt_cache_positions[begin:end],
                cache=cache, max_cache_length=total, workload="prefill", deterministic=request.deterministic,
            )
            _check_step(step, batch, "prefill", device)
            cache = step.cache
            prefill_count += 1
        assert step is not None

        out = torch.full((batch, request.max_new_tokens), request.pad_token_id, dtype=torch.long, device=device)
        lengths = torch.zeros(batch, dtype=torch.long, device=device)
        finished = torch.zeros(batch, dtype=torch.bool, device=device)
        by_eos = torch.zeros_like(finished)
        by_stop = torch.zeros_like(finished)
        decode_count = syncs = 0
        for index in range(request.max_new_tokens):
            chosen = select_tokens(step.logits[:, -1, :], request.sampling, generator)
            live = ~finished
            out[:, index] = torch.where(live, chosen, request.pad_token_id)
            lengths += live.long()
            hit_eos = live & (chosen[:, None] == eos[None, :]).any(dim=1)
            hit_stop = torch.zeros_like(finished)
            for seq in stops:
                n = seq.numel()
                if n <= index + 1:
                    hit_stop |= (out[:, index + 1 - n: index + 1] == seq[None, :]).all(dim=1)
            hit_stop &= live & ~hit_eos
            by_eos |= hit_eos
            by_stop |= hit_stop
            finished |= hit_eos | hit_stop
            if index + 1 == request.max_new_tokens:
                break
            if (index + 1) % request.stopping_check_interval == 0:
                syncs += 1
                if bool(finished.all()):
                    break
            if cache is None:
                raise GenerationError("NQ-GEN-CACHE model prefill returned no cache for decode")
            live = ~finished
            full_mask[:, width + index] = live
            step = model.forward_step(
                input_ids=torch.where(live, chosen, request.pad_token_id)[:, None],
                attention_mask=full_mask[:, : width + index + 1],
                position_ids=torch.where(live, width + index, 0)[:, None],
                cache_position=decode_cache_positions[index: index + 1],
                cache=cache, max_cache_length=total, workload="decode", deterministic=request.deterministic,
            )
            _check_step(step, batch, "decode", device)
            cache = step.cache
            decode_count += 1

    summary = torch.stack((lengths, by_eos.long(), by_stop.long()), dim=1).cpu().tolist()
    reasons = tuple("eos" if e else "stop_sequence" if s else "max_new_tokens" for _, e, s in summary)
    return GenerationResult(out, tuple(int(row[0]) for row in summary), reasons, prefill_count, decode_count,
                            total, syncs, 1)
