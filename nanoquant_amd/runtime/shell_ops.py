"""Launch wrappers of the decoder-shell kernels (``include/nqamd_shell.h``).

Each function validates its tensors the way the reference's launch helpers do
(src/nanoquant/runtime/cuda_kernels.py:493-544,644-815: ``ValueError`` for a
wrong dtype, device, geometry or layout), then enqueues the HIP kernel on the
current stream. Outputs and workspaces come from torch's caching allocator
unless the caller passes them, so every call can be captured in a HIP graph.
Token positions are device int32 tensors (``position[0]`` = cache row of the
first token) so a captured step replays at every position.
"""

from __future__ import annotations

import torch

from nanoquant_amd.runtime import _native

_FLOAT = (torch.float32, torch.float16, torch.bfloat16)


def _check_device(name: str, device: torch.device, *tensors: torch.Tensor | None) -> None:
    if device.type != "cuda":
        raise ValueError(f"{name} requires CUDA/HIP tensors")
    for tensor in tensors:
        if tensor is None:
            continue
        if tensor.device != device:
            raise ValueError(f"{name} inputs must share one device")
        if not tensor.is_contiguous():
            raise ValueError(f"{name} requires contiguous tensors")


def _check_float(name: str, *tensors: torch.Tensor | None) -> None:
    for tensor in tensors:
        if tensor is not None and tensor.dtype not in _FLOAT:
            raise ValueError(f"{name} tensor dtype {tensor.dtype} is not F32/F16/BF16")


def _position(name: str, position: torch.Tensor, device: torch.device) -> None:
    if position.dtype != torch.int32 or position.numel() < 1 or position.device != device:
        raise ValueError(f"{name} position must be a device int32 tensor")


def _stream(device: torch.device) -> int:
    return _native.current_stream_handle(device)


def _ptr(t: torch.Tensor | None) -> int | None:
    return None if t is None else t.data_ptr()


def launch_embedding(
    ids: torch.Tensor, table: torch.Tensor, *, scale: torch.Tensor | None = None, out: torch.Tensor | None = None,
    slots: torch.Tensor | None = None,
) -> torch.Tensor:
    """fp32 rows ``table[ids]`` (``* scale``). Mirrors ``launch_bfloat16_embedding``
    (src/nanoquant/runtime/cuda_kernels.py:644-681) for any float table. With
    ``slots`` (fp32 ``[*ids, hidden / 16]``) it also writes each row's sums of
    squares per 16 columns, the statistics a ``rmsnorm`` input kind of
    ``linear_batch_fused`` reads."""

    if ids.dtype != torch.int64 or table.ndim != 2:
        raise ValueError("embedding requires int64 ids and a 2-D table")
    _check_float("embedding", table)
    _check_device("embedding", ids.device, ids, table, scale, out)
    if scale is not None and (scale.dtype != torch.float32 or scale.numel() != 1):
        raise ValueError("embedding scale must be one fp32 value")
    vocab, hidden = table.shape
    if out is None:
        out = torch.empty((*ids.shape, hidden), dtype=torch.float32, device=ids.device)
    elif out.dtype != torch.float32 or tuple(out.shape) != (*ids.shape, hidden):
        raise ValueError("embedding output must be fp32 [*ids, hidden]")
    if slots is None:
        status = _native.load().nq_embedding(
            ids.data_ptr(), ids.numel(), table.data_ptr(), _native.dtype_code(table.dtype), vocab, hidden,
            _ptr(scale), out.data_ptr(), _stream(ids.device),
        )
        _native.check("nq_embedding", status)
        return out
    _check_device("embedding", ids.device, slots)
    if hidden % 16 or slots.dtype != torch.float32 or tuple(slots.shape) != (*ids.shape, hidden // 16) \
            or not slots.is_contiguous():
        raise ValueError("embedding slots must be contiguous fp32 [*ids, hidden / 16] (hidden % 16 == 0)")
    status = _native.load().nq_embedding_slots(
        ids.data_ptr(), ids.numel(), table.data_ptr(), _native.dtype_code(table.dtype), vocab, hidden,
        _ptr(scale), out.data_ptr(), slots.data_ptr(), _stream(ids.device),
    )
    _native.check("nq_embedding_slots", status)
    return out


def launch_add_rmsnorm(
    residual: torch.Tensor,
    weight: torch.Tensor,
    eps: float,
    *,
    delta: torch.Tensor | None = None,
    out: torch.Tensor | None = None,
    out_dtype: torch.dtype = torch.bfloat16,
) -> torch.Tensor:
    """``residual += delta`` (in place, optional), then
    ``out = weight * (residual * rsqrt(mean(residual^2) + eps))`` per row."""

    if residual.dtype != torch.float32:
        raise ValueError("rmsnorm residual must be fp32")
    _check_float("rmsnorm", weight, delta)
    _check_device("rmsnorm", residual.device, residual, weight, delta, out)
    hidden = residual.shape[-1]
    if weight.numel() != hidden or (delta is not None and delta.shape != residual.shape):
        raise ValueError("rmsnorm geometry is incompatible")
    if out is None:
        out = torch.empty(residual.shape, dtype=out_dtype, device=residual.device)
    elif out.shape != residual.shape or out.dtype not in _FLOAT:
        raise ValueError("rmsnorm output geometry is incompatible")
    rows = residual.numel() // hidden
    status = _native.load().nq_add_rmsnorm(
        residual.data_ptr(), _ptr(delta), _native.dtype_code(delta.dtype) if delta is not None else 0,
        weight.data_ptr(), _native.dtype_code(weight.dtype), float(eps), rows, hidden, out.data_ptr(),
        _native.dtype_code(out.dtype), _stream(residual.device),
    )
    _native.check("nq_add_rmsnorm", status)
    return out


def launch_qk_norm_rope_cache(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    *,
    q_heads: int,
    kv_heads: int,
    head_dim: int,
    q_norm: torch.Tensor | None,
    k_norm: torch.Tensor | None,
    eps: float,
    cos: torch.Tensor,
    sin: torch.Tensor,
    position: torch.Tensor,
    k_cache: torch.Tensor,
    v_cache: torch.Tensor,
    q_out: torch.Tensor | None = None,
) -> torch.Tensor:
    """Per-head RMSNorm + RoPE of q and k, KV-cache append; returns the rotated q
    (fp32 ``[tokens, q_heads, head_dim]``). Mirrors ``launch_decode_rope`` and
    ``launch_cache_prefix_update`` (src/nanoquant/runtime/cuda_kernels.py:715-815)."""

    device = q.device
    tokens = q.numel() // (q_heads * head_dim)
    for name, t, heads in (("q", q, q_heads), ("k", k, kv_heads), ("v", v, kv_heads)):
        if t.dtype != torch.float32 or t.numel() != tokens * heads * head_dim:
            raise ValueError(f"{name} must be fp32 [tokens, {heads} * {head_dim}]")
    if (q_norm is None) != (k_norm is None):
        raise ValueError("q_norm and k_norm must be given together")
    if q_norm is not None and (q_norm.numel() != head_dim or k_norm.numel() != head_dim or q_norm.dtype != k_norm.dtype):
        raise ValueError("q/k norm weights must be [head_dim] of one dtype")
    _check_float("qk norm", q_norm, k_norm, k_cache)
    _check_device("qk rope", device, q, k, v, q_norm, k_norm, cos, sin, position, k_cache, v_cache, q_out)
    _position("qk rope", position, device)
    max_positions = k_cache.shape[-2]
    expected = (kv_heads, max_positions, head_dim)
    if tuple(k_cache.shape) != expected or v_cache.shape != k_cache.shape or v_cache.dtype != k_cache.dtype:
        raise ValueError("KV cache must be [kv_heads, max_positions, head_dim] for K and V")
    if cos.dtype != torch.float32 or sin.dtype != torch.float32 or tuple(cos.shape) != (max_positions, head_dim // 2) or sin.shape != cos.shape:
        raise ValueError("RoPE tables must be fp32 [max_positions, head_dim / 2]")
    if q_out is None:
        q_out = torch.empty((tokens, q_heads, head_dim), dtype=torch.float32, device=device)
    elif q_out.dtype != torch.float32 or q_out.numel() != tokens * q_heads * head_dim:
        raise ValueError("q_out must be fp32 [tokens, q_heads, head_dim]")
    status = _native.load().nq_qk_norm_rope_cache(
        q.data_ptr(), k.data_ptr(), v.data_ptr(), tokens, q_heads, kv_heads, head_dim, _ptr(q_norm),
        _ptr(k_norm), _native.dtype_code(q_norm.dtype) if q_norm is not None else 0, float(eps),
        cos.data_ptr(), sin.data_ptr(), position.data_ptr(), max_positions, q_out.data_ptr(),
        k_cache.data_ptr(), v_cache.data_ptr(), _native.dtype_code(k_cache.dtype), _stream(device),
    )
    _native.check("nq_qk_norm_rope_cache", status)
    return q_out


def attention_workspace_bytes(tokens: int, q_heads: int, head_dim: int, max_positions: int) -> int:
    return int(_native.load().nq_attention_workspace_bytes(tokens, q_heads, head_dim, max_positions))


def launch_attention(
    q: torch.Tensor,
    k_cache: torch.Tensor,
    v_cache: torch.Tensor,
    *,
    position: torch.Tensor,
    scaling: float,
    out: torch.Tensor | None = None,
    out_dtype: torch.dtype = torch.bfloat16,
    workspace: torch.Tensor | None = None,
) -> torch.Tensor:
    """Causal grouped-query attention of ``q`` (fp32 ``[tokens, q_heads, D]``) over
    cache rows ``[0, position + t]``. Mirrors ``launch_decode_attention``
    (src/nanoquant/runtime/cuda_kernels.py:493-544) for any GQA geometry."""

    device = q.device
    if q.dtype != torch.float32 or q.ndim != 3:
        raise ValueError("attention query must be fp32 [tokens, q_heads, head_dim]")
    tokens, q_heads, head_dim = q.shape
    kv_heads, max_positions = k_cache.shape[0], k_cache.shape[1]
    if k_cache.ndim != 3 or k_cache.shape[2] != head_dim or v_cache.shape != k_cache.shape or v_cache.dtype != k_cache.dtype:
        raise ValueError("attention cache geometry is incompatible")
    _check_float("attention", k_cache)
    _check_device("attention", device, q, k_cache, v_cache, position, out, workspace)
    _position("attention", position, device)
    if out is None:
        out = torch.empty((tokens, q_heads * head_dim), dtype=out_dtype, device=device)
    elif out.numel() != tokens * q_heads * head_dim or out.dtype not in _FLOAT:
        raise ValueError("attention output geometry is incompatible")
    need = attention_workspace_bytes(tokens, q_heads, head_dim, max_positions)
    if need < 0:
        raise ValueError("attention geometry was rejected")
    if workspace is None:
        workspace = torch.empty(need, dtype=torch.uint8, device=device)
    status = _native.load().nq_attention(
        q.data_ptr(), k_cache.data_ptr(), v_cache.data_ptr(), _native.dtype_code(k_cache.dtype), tokens, q_heads,
        kv_heads, head_dim, position.data_ptr(), max_positions, float(scaling), out.data_ptr(),
        _native.dtype_code(out.dtype), workspace.data_ptr(), workspace.numel() * workspace.element_size(),
        _stream(device),
    )
    _native.check("nq_attention", status)
    return out


def decode_attention_workspace_bytes(q_heads: int, kv_heads: int, head_dim: int, cache_dtype: torch.dtype,
                                     max_positions: int) -> int:
    return int(_native.load().nq_decode_attention_workspace_bytes(
        q_heads, kv_heads, head_dim, _native.dtype_code(cache_dtype), max_positions))


def _decode_attention_checks(q, k, v, q_heads, kv_heads, head_dim, q_norm, k_norm, cos, sin, position, k_cache,
                             v_cache, out, workspace) -> tuple[int, torch.Tensor]:
    """Validate one-token attention operands; returns (max_positions, workspace)."""

    device = q.device
    for name, t, heads in (("q", q, q_heads), ("k", k, kv_heads), ("v", v, kv_heads)):
        if t.dtype != torch.float32 or t.numel() != heads * head_dim:
            raise ValueError(f"{name} must be fp32 [{heads} * {head_dim}] (one token)")
    if (q_norm is None) != (k_norm is None):
        raise ValueError("q_norm and k_norm must be given together")
    if q_norm is not None and (q_norm.numel() != head_dim or k_norm.numel() != head_dim or q_norm.dtype != k_norm.dtype):
        raise ValueError("q/k norm weights must be [head_dim] of one dtype")
    _check_float("decode attention", q_norm, k_norm, k_cache)
    _check_device("decode attention", device, q, k, v, q_norm, k_norm, cos, sin, position, k_cache, v_cache, out,
                  workspace)
    _position("decode attention", position, device)
    max_positions = k_cache.shape[-2]
    if tuple(k_cache.shape) != (kv_heads, max_positions, head_dim) or v_cache.shape != k_cache.shape or v_cache.dtype != k_cache.dtype:
        raise ValueError("KV cache must be [kv_heads, max_positions, head_dim] for K and V")
    if cos.dtype != torch.float32 or tuple(cos.shape) != (max_positions, head_dim // 2) or sin.shape != cos.shape:
        raise ValueError("RoPE tables must be fp32 [max_positions, head_dim / 2]")
    need = decode_attention_workspace_bytes(q_heads, kv_heads, head_dim, k_cache.dtype, max_positions)
    if need < 0:
        raise ValueError("decode attention geometry was rejected")
    if workspace is None:
        workspace = torch.empty(need, dtype=torch.uint8, device=device)
    return max_positions, workspace


def launch_decode_attention(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    *,
    q_heads: int,
    kv_heads: int,
    head_dim: int,
    q_norm: torch.Tensor | None,
    k_norm: torch.Tensor | None,
    eps: float,
    cos: torch.Tensor,
    sin: torch.Tensor,
    position: torch.Tensor,
    k_cache: torch.Tensor,
    v_cache: torch.Tensor,
    scaling: float,
    out: torch.Tensor | None = None,
    out_dtype: torch.dtype = torch.bfloat16,
    workspace: torch.Tensor | None = None,
) -> torch.Tensor:
    """One decode token: q/k RMSNorm + RoPE, KV append at ``position`` and
    causal GQA attention, fused into one kernel where the geometry allows."""

    device = q.device
    max_positions, workspace = _decode_attention_checks(q, k, v, q_heads, kv_heads, head_dim, q_norm, k_norm, cos,
                                                        sin, position, k_cache, v_cache, out, workspace)
    if out is None:
        out = torch.empty(q_heads * head_dim, dtype=out_dtype, device=device)
    elif out.numel() != q_heads * head_dim or out.dtype not in _FLOAT:
        raise ValueError("decode attention output geometry is incompatible")
    status = _native.load().nq_decode_attention(
        q.data_ptr(), k.data_ptr(), v.data_ptr(), q_heads, kv_heads, head_dim, _ptr(q_norm), _ptr(k_norm),
        _native.dtype_code(q_norm.dtype) if q_norm is not None else 0, float(eps), cos.data_ptr(), sin.data_ptr(),
        position.data_ptr(), max_positions, k_cache.data_ptr(), v_cache.data_ptr(),
        _native.dtype_code(k_cache.dtype), float(scaling), out.data_ptr(), _native.dtype_code(out.dtype),
        workspace.data_ptr(), workspace.numel() * workspace.element_size(), _stream(device),
    )
    _native.check("nq_decode_attention", status)
    return out


def decode_attention_partials_supported(q_heads: int, kv_heads: int, head_dim: int, cache_dtype: torch.dtype) -> bool:
    """Whether one-token attention runs as pass 1 + merge (the form whose
    partials ``launch_decode_attention_partials`` leaves in the workspace):
    head_dim * cache element bytes <= 256 and 1, 2, 4 or 8 q heads per kv head."""

    if q_heads <= 0 or kv_heads <= 0 or q_heads % kv_heads:
        return False
    element = 4 if cache_dtype == torch.float32 else 2
    return head_dim in (64, 128, 256) and head_dim * element <= 256 and q_heads // kv_heads in (1, 2, 4, 8)


def launch_decode_attention_partials(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    *,
    q_heads: int,
    kv_heads: int,
    head_dim: int,
    q_norm: torch.Tensor | None,
    k_norm: torch.Tensor | None,
    eps: float,
    cos: torch.Tensor,
    sin: torch.Tensor,
    position: torch.Tensor,
    k_cache: torch.Tensor,
    v_cache: torch.Tensor,
    scaling: float,
    workspace: torch.Tensor | None = None,
) -> torch.Tensor:
    """Pass 1 of ``launch_decode_attention`` alone (nq_decode_attention_partials):
    returns the workspace, which holds every cache block's partial (max, sum,
    acc) for a projection with ``input_kind="attention"`` to merge."""

    device = q.device
    max_positions, workspace = _decode_attention_checks(q, k, v, q_heads, kv_heads, head_dim, q_norm, k_norm, cos,
                                                        sin, position, k_cache, v_cache, None, workspace)
    status = _native.load().nq_decode_attention_partials(
        q.data_ptr(), k.data_ptr(), v.data_ptr(), q_heads, kv_heads, head_dim, _ptr(q_norm), _ptr(k_norm),
        _native.dtype_code(q_norm.dtype) if q_norm is not None else 0, float(eps), cos.data_ptr(), sin.data_ptr(),
        position.data_ptr(), max_positions, k_cache.data_ptr(), v_cache.data_ptr(),
        _native.dtype_code(k_cache.dtype), float(scaling),
        workspace.data_ptr(), workspace.numel() * workspace.element_size(), _stream(device),
    )
    _native.check("nq_decode_attention_partials", status)
    return workspace


def launch_silu_mul(
    gate: torch.Tensor, up: torch.Tensor, *, out: torch.Tensor | None = None, out_dtype: torch.dtype = torch.bfloat16
) -> torch.Tensor:
    """``silu(gate) * up`` (fp32 inputs)."""

    if gate.dtype != torch.float32 or up.dtype != torch.float32 or gate.shape != up.shape:
        raise ValueError("silu_mul requires fp32 gate and up of one shape")
    _check_device("silu_mul", gate.device, gate, up, out)
    if out is None:
        out = torch.empty(gate.shape, dtype=out_dtype, device=gate.device)
    elif out.shape != gate.shape or out.dtype not in _FLOAT:
        raise ValueError("silu_mul output geometry is incompatible")
    status = _native.load().nq_silu_mul(
        gate.data_ptr(), up.data_ptr(), gate.numel(), out.data_ptr(), _native.dtype_code(out.dtype),
        _stream(gate.device),
    )
    _native.check("nq_silu_mul", status)
    return out


def output_projection_workspace_bytes(vocab: int, hidden: int) -> int:
    return int(_native.load().nq_output_projection_workspace_bytes(vocab, hidden))


def launch_output_projection(
    x: torch.Tensor,
    weight: torch.Tensor,
    *,
    logits: torch.Tensor | None = None,
    workspace: torch.Tensor | None = None,
) -> tuple[torch.Tensor, torch.Tensor]:
    """fp32 logits of one token through a bf16 ``[vocab, hidden]`` matrix; also
    returns the workspace holding the argmax partials for
    ``launch_greedy_select``. Mirrors ``launch_bfloat16_output_projection``
    (src/nanoquant/runtime/cuda_kernels.py:684-712) for one token."""

    if weight.dtype != torch.bfloat16 or weight.ndim != 2:
        raise ValueError("output projection requires a bf16 [vocab, hidden] matrix")
    if x.dtype not in (torch.float32, torch.bfloat16) or x.numel() != weight.shape[1]:
        raise ValueError("output projection input must be one F32/BF16 row of width hidden")
    _check_device("output projection", x.device, x, weight, logits, workspace)
    vocab, hidden = weight.shape
    if logits is None:
        logits = torch.empty(vocab, dtype=torch.float32, device=x.device)
    elif logits.dtype != torch.float32 or logits.numel() != vocab:
        raise ValueError("logits must be fp32 [vocab]")
    need = output_projection_workspace_bytes(vocab, hidden)
    if need < 0:
        raise ValueError("output projection geometry was rejected")
    if workspace is None:
        workspace = torch.empty(need, dtype=torch.uint8, device=x.device)
    status = _native.load().nq_output_projection(
        x.data_ptr(), _native.dtype_code(x.dtype), weight.data_ptr(), vocab, hidden, logits.data_ptr(),
        workspace.data_ptr(), workspace.numel() * workspace.element_size(), _stream(x.device),
    )
    _native.check("nq_output_projection", status)
    return logits, workspace


def launch_greedy_select(
    workspace: torch.Tensor,
    vocab: int,
    hidden: int,
    *,
    token_out: torch.Tensor,
    history: torch.Tensor | None = None,
    step: torch.Tensor | None = None,
    position: torch.Tensor | None = None,
) -> torch.Tensor:
    """Greedy token (lowest index among equal maxima, like ``torch.argmax``) from
    the partials of ``launch_output_projection``, written to ``token_out[0]``;
    optionally appended to ``history`` at ``step`` and advancing ``position``."""

    device = workspace.device
    if token_out.dtype != torch.int64 or token_out.numel() < 1:
        raise ValueError("token_out must be an int64 tensor")
    if (history is None) != (step is None):
        raise ValueError("history and step must be given together")
    if history is not None and (history.dtype != torch.int64 or step.dtype != torch.int32):
        raise ValueError("history must be int64 and step int32")
    if position is not None:
        _position("greedy select", position, device)
    _check_device("greedy select", device, workspace, token_out, history, step, position)
    status = _native.load().nq_greedy_select(
        workspace.data_ptr(), vocab, hidden, token_out.data_ptr(), _ptr(history),
        0 if history is None else history.numel(), _ptr(step), _ptr(position), _stream(device),
    )
    _native.check("nq_greedy_select", status)
    return token_out
