"""HIP backend for the packed binary low-rank linear on MI355X (gfx950).

Drop-in for the reference's GPU packed backend ``CudaPackedBackend``
(src/nanoquant/runtime/cuda_backend.py:151-278): same protocol, capability
declaration, error convention (misuse raises ``ValueError``/``TypeError``;
capability gaps are returned as ``SupportResult.rejected`` codes) and the same
fp32 output boundary. ``linear`` validates, allocates the output and workspace
from torch's caching allocator and enqueues the HIP kernels on torch's current
stream through the C ABI; it never synchronises, transfers or unpacks.
"""

from __future__ import annotations

import ctypes
from dataclasses import MISSING, dataclass, field, fields, replace

import torch

from nanoquant_amd.runtime import _native
from nanoquant_amd.runtime.codecs import MixedVLayerState, ProductCodebookLayerState, device_packed_state
from nanoquant_amd.runtime.backend import (
    BackendCapabilities,
    DeviceLike,
    PreparedLayer,
    QuantizedLinearSpec,
    RuntimeLayerState,
    SupportResult,
    WorkloadSpec,
    evaluate_capabilities,
)
from nanoquant_amd.runtime.logical import canonical_torch_dtype
from nanoquant_amd.runtime.packed import PACKED_LAYOUT_VERSION, PackedLayerState
from nanoquant_amd.runtime.row_sidecar import RowSidecarLayerState

HIP_PACKED_BACKEND_NAME = "rocm-packed-hip"
HIP_PACKED_BACKEND_VERSION = "1"
_FLOAT_DTYPES = ("float16", "bfloat16", "float32")
_REQUIRED_ARCH = "gfx950"


@dataclass(frozen=True, slots=True)
class _HipPackedPayload:
    device: torch.device
    left_words: torch.Tensor
    right_words: torch.Tensor
    scale_pre: torch.Tensor
    scale_mid: torch.Tensor
    scale_post: torch.Tensor
    bias: torch.Tensor | None
    outlier_indices: torch.Tensor | None
    outlier_values: torch.Tensor | None
    outlier_scales: torch.Tensor | None
    patch_left: torch.Tensor | None
    patch_right: torch.Tensor | None
    row_indices: torch.Tensor | None
    row_values: torch.Tensor | None
    row_scales: torch.Tensor | None
    tiles: torch.Tensor | None
    desc: _native.LinearDesc = field(repr=False)


def _to_device(tensor: torch.Tensor | None, device: torch.device) -> torch.Tensor | None:
    return None if tensor is None else tensor.to(device=device).contiguous()


_OWN_STATES = (RowSidecarLayerState, PackedLayerState, MixedVLayerState, ProductCodebookLayerState)
# Tried in this order; no state kind carries all the required fields of another.
_ADOPTABLE_STATES = (MixedVLayerState, ProductCodebookLayerState, PackedLayerState)


def adopt_layer_state(state: object) -> RuntimeLayerState:
    """This package's state object for ``state``.

    The reference planner prepares layers with its own ``PackedLayerState``,
    ``MixedVLayerState`` and ``ProductCodebookLayerState``
    (src/nanoquant/runtime/planning.py:273-299 -> backend.prepare), whose
    classes this package does not import. A state is recognised by the
    reference's field names (src/nanoquant/runtime/packed.py:231-244,
    mixed_v.py:169-187, product_codebook.py:147-164) and rebuilt as the
    matching class here, which re-checks every invariant. The caller's ``spec``
    object is kept, so ``PreparedLayer.spec`` compares equal to the state's
    spec as the reference planner requires (planning.py:255-256). Objects
    lacking a kind's required fields raise ``TypeError``."""

    if isinstance(state, _OWN_STATES):
        return state
    for cls in _ADOPTABLE_STATES:
        names = fields(cls)
        required = [f.name for f in names if f.default is MISSING]
        if all(hasattr(state, name) for name in required):
            return cls(**{f.name: getattr(state, f.name, None) for f in names})
    raise TypeError("HIP packed backend requires PackedLayerState, RowSidecarLayerState, MixedVLayerState "
                    "or ProductCodebookLayerState (or an object with their fields)")


def _device_arch(index: int) -> str:
    return str(getattr(torch.cuda.get_device_properties(index), "gcnArchName", ""))


def _describe(
    p: _HipPackedPayload, spec: QuantizedLinearSpec, desc: _native.LinearDesc
) -> None:
    """Fill the C descriptor with the payload's device pointers."""

    ptr = _native.pointer
    desc.in_features = spec.in_features
    desc.out_features = spec.out_features
    desc.rank = spec.rank
    desc.right_words = ptr(p.right_words)
    desc.left_words = ptr(p.left_words)
    desc.scale_pre = ptr(p.scale_pre)
    desc.scale_mid = ptr(p.scale_mid)
    desc.scale_post = ptr(p.scale_post)
    desc.scale_dtype = _native.dtype_code(p.scale_pre.dtype)
    if p.bias is not None:
        desc.bias = ptr(p.bias)
        desc.bias_dtype = _native.dtype_code(p.bias.dtype)
    if p.outlier_indices is not None and p.outlier_values is not None:
        desc.salient_count = int(p.outlier_indices.numel())
        desc.salient_indices = ptr(p.outlier_indices)
        desc.salient_values = ptr(p.outlier_values)
        desc.salient_dtype = _native.dtype_code(p.outlier_values.dtype)
        desc.salient_scales = ptr(p.outlier_scales)
    if p.patch_left is not None and p.patch_right is not None:
        desc.patch_rank = int(p.patch_left.shape[1])
        desc.patch_left = ptr(p.patch_left)
        desc.patch_right = ptr(p.patch_right)
        desc.patch_dtype = _native.dtype_code(p.patch_left.dtype)
    if p.row_indices is not None:
        desc.row_count = int(p.row_indices.numel())
        desc.row_indices = ptr(p.row_indices)
        desc.row_values = ptr(p.row_values)
        desc.row_scales = ptr(p.row_scales)


_DECODE_LAUNCH = {"split": _native.NQ_DECODE_SPLIT, "fused": _native.NQ_DECODE_FUSED}
_PREFILL_OPERANDS = {"fp16": _native.NQ_PREFILL_FP16, "split": _native.NQ_PREFILL_FP16_SPLIT}


class HipPackedBackend:
    """gfx950 HIP kernels behind the reference backend protocol."""

    name = HIP_PACKED_BACKEND_NAME
    version = HIP_PACKED_BACKEND_VERSION
    packed_layout = PACKED_LAYOUT_VERSION

    def __init__(self, *, tiled_decode: bool = True, decode_launch: str = "split",
                 prefill_operands: str = "fp16") -> None:
        """``tiled_decode`` prepares the MFMA tile layout (decode and prefill
        kernels); without it every call takes the canonical-word fp32 path.
        ``decode_launch``: ``"split"`` runs the two decode stages as two
        kernels, ``"fused"`` as one kernel with an in-kernel grid handoff.
        ``prefill_operands`` (above 16 tokens): ``"fp16"`` rounds the prefill
        GEMMs' activations and rank intermediate to fp16 (about 3e-4 rel-L2
        per linear); ``"split"`` carries each as an fp16 value plus an fp16
        remainder (about 1e-6), at twice the MFMA work, for callers whose
        errors compound through many layers."""

        if decode_launch not in _DECODE_LAUNCH:
            raise ValueError(f"decode_launch must be one of {sorted(_DECODE_LAUNCH)}")
        if prefill_operands not in _PREFILL_OPERANDS:
            raise ValueError(f"prefill_operands must be one of {sorted(_PREFILL_OPERANDS)}")
        self._tiled_decode = tiled_decode
        self._decode_launch = _DECODE_LAUNCH[decode_launch]
        self._prefill_operands = _PREFILL_OPERANDS[prefill_operands]

    def capabilities(self) -> BackendCapabilities:
        return BackendCapabilities(
            logical_formats=("nanoquant-v1",),
            device_types=("cuda",),
            input_dtypes=_FLOAT_DTYPES,
            factor_dtypes=_FLOAT_DTYPES,
            scale_dtypes=_FLOAT_DTYPES,
            outlier_value_dtypes=(*_FLOAT_DTYPES, "int8"),
            workload_kinds=("prefill", "decode"),
            supports_bias=True,
            supports_outliers=True,
            supports_deterministic=True,
            patch_value_dtypes=_FLOAT_DTYPES,
        )

    def supports(self, op: QuantizedLinearSpec, workload: WorkloadSpec) -> SupportResult:
        result = evaluate_capabilities(self.capabilities(), op, workload)
        if not result.supported:
            return result
        if not _native.library_available():
            return SupportResult.rejected(
                "NQ-INF-HIP-KERNEL", "the HIP library libnqamd.so is not built"
            )
        if not torch.cuda.is_available():
            return SupportResult.rejected(
                "NQ-INF-DEVICE-UNAVAILABLE", "CUDA is not available in this runtime"
            )
        arch = _device_arch(torch.cuda.current_device())
        if not arch.startswith(_REQUIRED_ARCH):
            return SupportResult.rejected(
                "NQ-INF-HIP-ARCH", f"device architecture {arch!r} is not {_REQUIRED_ARCH}"
            )
        return result

    def prepare(self, state: RuntimeLayerState, device: DeviceLike) -> PreparedLayer:
        """Copy a layer to the device once and build its tile layout. Compact
        right factors (mixed-V, product codebook) are expanded on the device, as
        the reference backend does for mixed-V (src/nanoquant/runtime/cuda_backend.py:199-241)."""

        state = adopt_layer_state(state)
        target = torch.device(device)
        if target.type != "cuda":
            raise ValueError("HIP packed backend preparation requires a CUDA (HIP) device")
        if not torch.cuda.is_available():
            raise RuntimeError("CUDA is not available in this runtime")
        if target.index is None:
            target = torch.device("cuda", torch.cuda.current_device())
        if isinstance(state, RowSidecarLayerState):
            packed, rows = state.base, state.rows
        elif isinstance(state, PackedLayerState):
            packed, rows = state, None
        else:
            with torch.cuda.device(target):
                packed, rows = device_packed_state(state, target), None
        lib = _native.load()
        payload = _HipPackedPayload(
            target,
            _to_device(packed.left_words, target),
            _to_device(packed.right_words, target),
            _to_device(packed.scale_pre, target),
            _to_device(packed.scale_mid, target),
            _to_device(packed.scale_post, target),
            _to_device(packed.bias, target),
            _to_device(packed.outlier_indices, target),
            _to_device(packed.outlier_values, target),
            _to_device(packed.outlier_scales, target),
            _to_device(packed.patch_left, target),
            _to_device(packed.patch_right, target),
            None if rows is None else _to_device(rows.indices, target),
            None if rows is None else _to_device(rows.values, target),
            None if rows is None else _to_device(rows.scales, target),
            None,
            _native.LinearDesc(),
        )
        _describe(payload, packed.spec, payload.desc)
        payload.desc.decode_launch = self._decode_launch
        payload.desc.prefill_operands = self._prefill_operands
        spec = packed.spec
        size = int(lib.nq_tiles_bytes(spec.in_features, spec.out_features, spec.rank))
        if self._tiled_decode and size > 0:
            tiles = torch.empty(size, dtype=torch.uint8, device=target)
            with torch.cuda.device(target):
                _native.check(
                    "nq_prepare_tiles",
                    lib.nq_prepare_tiles(
                        ctypes.byref(payload.desc),
                        tiles.data_ptr(),
                        size,
                        _native.current_stream_handle(target),
                    ),
                )
            payload = replace(payload, tiles=tiles)
            payload.desc.tiles = tiles.data_ptr()
            payload.desc.tiles_bytes = size
        return PreparedLayer(self.name, self.version, packed.spec, payload)

    def with_decode_launch(self, layer: PreparedLayer, decode_launch: str) -> PreparedLayer:
        """The same prepared layer (device tensors shared, no copies) with another
        decode launch structure. Layers sharing tiles must not run concurrently."""

        payload = self._payload(layer)
        if decode_launch not in _DECODE_LAUNCH:
            raise ValueError(f"decode_launch must be one of {sorted(_DECODE_LAUNCH)}")
        desc = _native.LinearDesc.from_buffer_copy(payload.desc)
        desc.decode_launch = _DECODE_LAUNCH[decode_launch]
        return PreparedLayer(layer.backend_name, layer.backend_version, layer.spec, replace(payload, desc=desc))

    def fused_launch_timed_out(self, layer: PreparedLayer) -> bool:
        """True when a fused decode launch of this layer ever gave up waiting for
        its stage-1 results (the sticky flag in the tiles header). Such a launch
        stored NaN for the outputs of the workgroups that gave up, so a caller
        that cannot check every call still sees the failure. Reads the flag
        after synchronising the device: a diagnostic, not for the token loop."""

        payload = self._payload(layer)
        if payload.tiles is None:
            return False
        torch.cuda.synchronize(payload.device)
        misc = int(_native.load().nq_tiles_header_bytes()) // 4 - 64
        return int(payload.tiles.view(torch.int32)[misc].item()) != 0

    def _payload(self, layer: PreparedLayer) -> _HipPackedPayload:
        if (layer.backend_name, layer.backend_version) != (self.name, self.version):
            raise ValueError("prepared runtime layer belongs to a different backend")
        if not isinstance(layer.payload, _HipPackedPayload):
            raise TypeError("prepared runtime layer has an invalid HIP packed payload")
        return layer.payload

    def linear(self, value: torch.Tensor, layer: PreparedLayer) -> torch.Tensor:
        return self.linear_into(value, layer, output_dtype=torch.float32)

    def linear_batch(
        self,
        values: list[torch.Tensor] | tuple[torch.Tensor, ...],
        layers: list[PreparedLayer] | tuple[PreparedLayer, ...],
        *,
        output_dtype: torch.dtype = torch.float32,
        outs: list[torch.Tensor] | None = None,
    ) -> list[torch.Tensor]:
        """Run up to 8 prepared layers with one launch per kernel phase: the
        decode kernels for 1-16 token slots, the prefill row pass, sign GEMMs
        and reductions above that.

        Generalises the reference's grouped Q/K/V and gate/up projection
        (src/nanoquant/runtime/cuda_backend.py:65-144): members may have distinct
        inputs and any rank; inputs may be the same tensor."""

        if len(values) != len(layers) or not 1 <= len(layers) <= 8:
            raise ValueError("HIP packed batch needs 1-8 layers with one input each")
        if len({id(layer) for layer in layers}) != len(layers):
            raise ValueError("HIP packed batch members must be distinct prepared layers")
        payloads = [self._payload(layer) for layer in layers]
        if any(p.tiles is None for p in payloads):
            raise ValueError("HIP packed batch requires layers prepared with tiled decode")
        tokens = {v.numel() // layer.spec.in_features for v, layer in zip(values, layers)}
        dtypes = {v.dtype for v in values}
        if len(tokens) != 1 or len(dtypes) != 1:
            raise ValueError("HIP packed batch members must share token count and input dtype")
        (count,) = tokens
        for value, layer, payload in zip(values, layers, payloads):
            _check_value(value, layer.spec, payload.device)
        if output_dtype not in (torch.float32, torch.bfloat16, torch.float16):
            raise ValueError(f"HIP packed output dtype is unsupported: {output_dtype}")
        device = payloads[0].device
        if outs is None:
            outs = [
                torch.empty((*v.shape[:-1], layer.spec.out_features), dtype=output_dtype, device=device)
                for v, layer in zip(values, layers)
            ]
        for out, value, layer in zip(outs, values, layers):
            shape = (*value.shape[:-1], layer.spec.out_features)
            if tuple(out.shape) != shape or out.dtype != output_dtype or not out.is_contiguous():
                raise ValueError("HIP packed output tensor shape, dtype or layout differs")
        lib = _native.load()
        n = len(layers)
        sizes = [int(lib.nq_linear_workspace_bytes(ctypes.byref(p.desc), count)) for p in payloads]
        if min(sizes) < 0:
            raise ValueError("HIP packed layer descriptor was rejected")
        workspaces = [torch.empty(max(b, 1), dtype=torch.uint8, device=device) for b in sizes]
        desc_ptrs = (ctypes.POINTER(_native.LinearDesc) * n)(*[ctypes.pointer(p.desc) for p in payloads])
        x_ptrs = (ctypes.c_void_p * n)(*[v.data_ptr() for v in values])
        y_ptrs = (ctypes.c_void_p * n)(*[o.data_ptr() for o in outs])
        w_ptrs = (ctypes.c_void_p * n)(*[w.data_ptr() for w in workspaces])
        w_sizes = (ctypes.c_int64 * n)(*sizes)
        status = lib.nq_linear_batch(
            desc_ptrs, n, x_ptrs, _native.dtype_code(values[0].dtype), count, y_ptrs,
            _native.dtype_code(output_dtype), w_ptrs, w_sizes, _native.current_stream_handle(device),
        )
        _native.check("nq_linear_batch", status)
        return list(outs)

    def norm_column_scale(self, layer: PreparedLayer, norm_weight: torch.Tensor) -> torch.Tensor:
        """fp32 column scale norm_weight * s_in of a prepared layer: the
        RMSNorm weight folded into the linear for ``linear_batch_fused``."""

        payload = self._payload(layer)
        weight = norm_weight.to(device=payload.device, dtype=torch.float32).reshape(-1)
        if weight.numel() != layer.spec.in_features:
            raise ValueError("norm weight width differs from the layer's input features")
        return (weight * payload.scale_pre.to(torch.float32)).contiguous()

    def linear_batch_fused(
        self,
        values: list[torch.Tensor] | tuple[torch.Tensor, ...],
        layers: list[PreparedLayer] | tuple[PreparedLayer, ...],
        *,
        input_kind: str = "plain",
        eps: float = 1e-6,
        col_scales: list[torch.Tensor] | None = None,
        norm_slots: torch.Tensor | None = None,
        ups: list[torch.Tensor] | None = None,
        residuals: list[torch.Tensor] | None = None,
        out_slots: list[torch.Tensor] | None = None,
        outs: list[torch.Tensor] | None = None,
        output_dtype: torch.dtype = torch.float32,
        output_kind: str = "plain",
        attention_position: torch.Tensor | None = None,
        attention_head_dim: int = 0,
        attention_max_positions: int = 0,
    ) -> list[torch.Tensor] | None:
        """One decode token through 1-8 prepared layers with the decoder's
        neighbouring element-wise work fused in (nq_linear_batch_fused):

        * ``input_kind="rmsnorm"``: each value is the fp32 residual h; member i
          sees RMSNorm(h) * w through ``col_scales[i]`` (``norm_column_scale``)
          and the per-16-row-tile sums of h^2 in ``norm_slots``;
        * ``input_kind="silu_gate"``: each value is the fp32 gate, ``ups[i]`` the
          fp32 up; member i sees silu(gate) * up;
        * ``input_kind="attention"``: each value is the workspace that
          ``shell_ops.launch_decode_attention_partials`` filled for a cache of
          ``attention_max_positions`` rows; member i sees the attention output
          (heads of ``attention_head_dim``) merged from the partials of the
          cache blocks up to ``attention_position`` (int32 on the device), the
          attention's second pass;
        * ``residuals`` / ``out_slots``: member i adds its output to
          ``residuals[i]`` (fp32) and writes the tile sums of the new residual's
          squares to ``out_slots[i]`` instead of producing an output tensor;
        * ``output_kind="silu_product"``: two members of equal geometry (gate
          and up) produce ONE output, ``silu(y_0) * y_1`` in ``output_dtype``
          (returned as a one-element list), which a following projection reads
          as a plain input.

        No reference counterpart: the reference runs these element-wise steps as
        separate torch operations (src/nanoquant/runtime/torch_model.py:493-505,
        625-660)."""

        kinds = {"plain": _native.INPUT_PLAIN, "rmsnorm": _native.INPUT_RMSNORM,
                 "silu_gate": _native.INPUT_SILU_GATE, "attention": _native.INPUT_ATTENTION}
        if input_kind not in kinds:
            raise ValueError(f"unknown fused input kind {input_kind!r}")
        out_kinds = {"plain": _native.OUTPUT_PLAIN, "silu_product": _native.OUTPUT_SILU_PRODUCT}
        if output_kind not in out_kinds:
            raise ValueError(f"unknown fused output kind {output_kind!r}")
        n = len(layers)
        if len(values) != n or not 1 <= n <= 8:
            raise ValueError("HIP fused batch needs 1-8 layers with one input each")
        if output_kind == "silu_product" and n != 2:
            raise ValueError("silu_product takes two members of the same output width")
        if len({id(layer) for layer in layers}) != n:
            raise ValueError("HIP fused batch members must be distinct prepared layers")
        payloads = [self._payload(layer) for layer in layers]
        if any(p.tiles is None for p in payloads):
            raise ValueError("HIP fused batch requires layers prepared with tiled decode")
        device = payloads[0].device
        if input_kind == "attention":
            hd, rows = int(attention_head_dim), int(attention_max_positions)
            if hd not in (64, 128, 256) or rows <= 0:
                raise ValueError("attention input needs head_dim 64, 128 or 256 and a positive cache length")
            if (attention_position is None or attention_position.device != device
                    or attention_position.dtype != torch.int32 or attention_position.numel() < 1):
                raise ValueError("attention input needs the int32 device position")
            blocks = -(-rows // 64)
            for value, layer in zip(values, layers):
                heads, rem = divmod(layer.spec.in_features, hd)
                if rem or value.device != device or not value.is_contiguous():
                    raise ValueError("attention input: in_features must be heads * head_dim, one contiguous workspace")
                if value.numel() * value.element_size() < (2 + hd) * heads * blocks * 4:
                    raise ValueError("attention input workspace is smaller than the partials it holds")
        else:
            for value, layer in zip(values, layers):
                _check_value(value, layer.spec, device)
                if value.numel() != layer.spec.in_features:
                    raise ValueError("HIP fused batch runs exactly one token")
            if input_kind != "plain" and any(v.dtype != torch.float32 for v in values):
                raise ValueError("HIP fused rmsnorm / silu_gate inputs are fp32")
            if len({v.dtype for v in values}) != 1:
                raise ValueError("HIP fused batch members must share the input dtype")

        def vec(t: torch.Tensor | None, length: int, what: str) -> torch.Tensor:
            if (t is None or t.device != device or t.dtype != torch.float32 or not t.is_contiguous()
                    or t.numel() != length):
                raise ValueError(f"HIP fused {what} must be a contiguous fp32 device vector of {length}")
            return t

        def ptrs(items: list[torch.Tensor] | None):
            return None if items is None else (ctypes.c_void_p * n)(*[t.data_ptr() for t in items])

        fusion = _native.DecodeFusion()
        fusion.input_kind = kinds[input_kind]
        fusion.output_kind = out_kinds[output_kind]
        fusion.eps = float(eps)
        keep: list = []
        if input_kind == "attention":
            fusion.attn_position = attention_position.data_ptr()
            fusion.attn_head_dim = int(attention_head_dim)
            fusion.attn_max_positions = int(attention_max_positions)
        if input_kind == "rmsnorm":
            if col_scales is None or len(col_scales) != n:
                raise ValueError("rmsnorm input needs one column scale per member")
            for t, layer in zip(col_scales, layers):
                vec(t, layer.spec.in_features, "column scale")
            in_features = {layer.spec.in_features for layer in layers}
            if len(in_features) != 1:
                raise ValueError("rmsnorm members share one residual width")
            slots = -(-in_features.pop() // 16)
            vec(norm_slots, slots, "norm slots")
            arr = ptrs(col_scales)
            keep.append(arr)
            fusion.col_scales = ctypes.cast(arr, ctypes.POINTER(ctypes.c_void_p))
            fusion.norm_slots = norm_slots.data_ptr()
            fusion.norm_slot_count = slots
        elif input_kind == "silu_gate":
            if ups is None or len(ups) != n:
                raise ValueError("silu_gate input needs one up tensor per member")
            for t, layer in zip(ups, layers):
                vec(t.reshape(-1) if t is not None else None, layer.spec.in_features, "up")
            arr = ptrs(ups)
            keep.append(arr)
            fusion.ups = ctypes.cast(arr, ctypes.POINTER(ctypes.c_void_p))
        if residuals is not None:
            if out_slots is None or len(residuals) != n or len(out_slots) != n:
                raise ValueError("residual epilogue needs one residual and one slot vector per member")
            for r, sl, layer in zip(residuals, out_slots, layers):
                vec(r.reshape(-1), layer.spec.out_features, "residual")
                vec(sl, -(-layer.spec.out_features // 16), "output slots")
            ra, sa = ptrs(residuals), ptrs(out_slots)
            keep += [ra, sa]
            fusion.residuals = ctypes.cast(ra, ctypes.POINTER(ctypes.c_void_p))
            fusion.out_slots = ctypes.cast(sa, ctypes.POINTER(ctypes.c_void_p))
            outs = None
        elif output_kind == "silu_product":
            if n != 2 or layers[0].spec.out_features != layers[1].spec.out_features:
                raise ValueError("silu_product takes two members of the same output width")
            if output_dtype not in (torch.float32, torch.bfloat16, torch.float16):
                raise ValueError(f"HIP packed output dtype is unsupported: {output_dtype}")
            width = layers[0].spec.out_features
            if outs is None:
                outs = [torch.empty(width, dtype=output_dtype, device=device)]
            if (len(outs) != 1 or outs[0].numel() != width or outs[0].dtype != output_dtype
                    or not outs[0].is_contiguous() or outs[0].device != device):
                raise ValueError("silu_product writes one contiguous output of the members' width")
        else:
            if output_dtype not in (torch.float32, torch.bfloat16, torch.float16):
                raise ValueError(f"HIP packed output dtype is unsupported: {output_dtype}")
            lead = [() if input_kind == "attention" else tuple(v.shape[:-1]) for v in values]
            if outs is None:
                outs = [torch.empty((*ld, layer.spec.out_features), dtype=output_dtype, device=device)
                        for ld, layer in zip(lead, layers)]
            for out, ld, layer in zip(outs, lead, layers):
                if (tuple(out.shape) != (*ld, layer.spec.out_features) or out.dtype != output_dtype
                        or not out.is_contiguous()):
                    raise ValueError("HIP packed output tensor shape, dtype or layout differs")
        lib = _native.load()
        sizes = [int(lib.nq_linear_workspace_bytes(ctypes.byref(p.desc), 1)) for p in payloads]
        if min(sizes) < 0:
            raise ValueError("HIP packed layer descriptor was rejected")
        workspaces = [torch.empty(max(b, 1), dtype=torch.uint8, device=device) for b in sizes]
        desc_ptrs = (ctypes.POINTER(_native.LinearDesc) * n)(*[ctypes.pointer(p.desc) for p in payloads])
        x_ptrs = (ctypes.c_void_p * n)(*[v.data_ptr() for v in values])
        if output_kind == "silu_product":
            y_ptrs = (ctypes.c_void_p * n)(outs[0].data_ptr(), 0)
        else:
            y_ptrs = (ctypes.c_void_p * n)(*[(o.data_ptr() if outs is not None else 0) for o in (outs or values)])
        w_ptrs = (ctypes.c_void_p * n)(*[w.data_ptr() for w in workspaces])
        w_sizes = (ctypes.c_int64 * n)(*sizes)
        status = lib.nq_linear_batch_fused(
            desc_ptrs, n, x_ptrs,
            _native.dtype_code(torch.float32 if input_kind == "attention" else values[0].dtype), y_ptrs,
            _native.dtype_code(output_dtype),
            w_ptrs, w_sizes, ctypes.byref(fusion), _native.current_stream_handle(device),
        )
        _native.check("nq_linear_batch_fused", status)
        return None if outs is None else list(outs)

    def linear_into(
        self,
        value: torch.Tensor,
        layer: PreparedLayer,
        *,
        output_dtype: torch.dtype = torch.float32,
        out: torch.Tensor | None = None,
    ) -> torch.Tensor:
        """``linear`` with an explicit output dtype (fp32 boundary by default;
        bf16/f16 stores fuse the cast) and an optional preallocated output."""

        payload = self._payload(layer)
        spec = layer.spec
        _check_value(value, spec, payload.device)
        if output_dtype not in (torch.float32, torch.bfloat16, torch.float16):
            raise ValueError(f"HIP packed output dtype is unsupported: {output_dtype}")
        tokens = value.numel() // spec.in_features
        shape = (*value.shape[:-1], spec.out_features)
        if out is None:
            out = torch.empty(shape, dtype=output_dtype, device=value.device)
        elif tuple(out.shape) != shape or out.dtype != output_dtype or not out.is_contiguous():
            raise ValueError("HIP packed output tensor shape, dtype or layout differs")
        lib = _native.load()
        desc = payload.desc
        ws_bytes = int(lib.nq_linear_workspace_bytes(ctypes.byref(desc), tokens))
        if ws_bytes < 0:
            raise ValueError("HIP packed layer descriptor was rejected")
        workspace = torch.empty(max(ws_bytes, 1), dtype=torch.uint8, device=value.device)
        status = lib.nq_linear(
            ctypes.byref(desc),
            value.data_ptr(),
            _native.dtype_code(value.dtype),
            tokens,
            out.data_ptr(),
            _native.dtype_code(output_dtype),
            workspace.data_ptr(),
            ws_bytes,
            _native.current_stream_handle(value.device),
        )
        _native.check("nq_linear", status)
        return out


@dataclass(frozen=True, slots=True)
class HipProjectionGroup:
    """Prepared layers that read the same input (Q/K/V, gate/up), run as one
    decode launch pair. Holds the layers themselves: no device copies."""

    device: torch.device
    layers: tuple[PreparedLayer, ...]
    ranks: tuple[int, ...]
    output_features: tuple[int, ...]


def prepare_hip_projection_group(layers: tuple[PreparedLayer, ...]) -> HipProjectionGroup | None:
    """Group prepared HIP layers that share one input, or None when they cannot
    share a launch: fewer than 2 or more than 8 layers, a layer that is not a
    tiled HIP layer, repeated layers, or different devices or input widths.

    Same name, argument and None-for-incompatible contract as the reference's
    prepare_cuda_projection_group (src/nanoquant/runtime/cuda_backend.py:65-120),
    without its restrictions (ranks and output widths that are multiples of 8,
    salient columns required, no bias or salient scales): the launch takes any
    rank, such as Qwen3 k/v's 819, and every sidecar."""

    layers = tuple(layers)
    if not 2 <= len(layers) <= 8 or len({id(layer) for layer in layers}) != len(layers):
        return None
    keys = {(layer.backend_name, layer.backend_version) for layer in layers}
    if keys != {(HIP_PACKED_BACKEND_NAME, HIP_PACKED_BACKEND_VERSION)}:
        return None
    payloads = [layer.payload for layer in layers]
    if not all(isinstance(p, _HipPackedPayload) and p.tiles is not None for p in payloads):
        return None
    if len({p.device for p in payloads}) != 1 or len({layer.spec.in_features for layer in layers}) != 1:
        return None
    if len({p.desc.decode_launch for p in payloads}) != 1:
        return None
    return HipProjectionGroup(
        payloads[0].device,
        layers,
        tuple(layer.spec.rank for layer in layers),
        tuple(layer.spec.out_features for layer in layers),
    )


def grouped_hip_projection(value: torch.Tensor, group: HipProjectionGroup) -> tuple[torch.Tensor, ...]:
    """Every layer of `group` applied to `value` ([..., in], f16/bf16/f32): fp32
    outputs ``[..., out_i]`` in group order, as grouped_cuda_projection returns
    (src/nanoquant/runtime/cuda_backend.py:123-144). The whole group shares
    one launch per kernel phase (nq_linear_batch): the decode stages for 1-16
    tokens, the prefill phases above that."""

    if value.device != group.device:
        raise ValueError("grouped HIP projection input uses a different device")
    backend = HipPackedBackend()
    return tuple(backend.linear_batch([value] * len(group.layers), list(group.layers)))


def _check_value(value: torch.Tensor, spec: QuantizedLinearSpec, device: torch.device) -> None:
    if value.device != device:
        raise ValueError("HIP packed input and prepared layer must use the same device")
    if canonical_torch_dtype(value.dtype) not in _FLOAT_DTYPES:
        raise ValueError(f"HIP packed input dtype is unsupported: {value.dtype}")
    if value.ndim == 0 or value.shape[-1] != spec.in_features:
        raise ValueError("HIP packed input feature dimension differs from the layer")
    if value.numel() == 0:
        raise ValueError("HIP packed input must contain at least one token")
    if not value.is_contiguous():
        raise ValueError("HIP packed input must be contiguous")
    if value.requires_grad:
        raise ValueError("HIP packed runtime does not support autograd")


def unpack_sign_matrix_device(
    words: torch.Tensor,
    rows: int,
    columns: int,
    *,
    dtype: torch.dtype = torch.float32,
) -> torch.Tensor:
    """Bit-exact HIP unpack of device sign words to dense +/-1
    (device form of src/nanoquant/runtime/packed.py:204-218)."""

    if words.device.type != "cuda":
        raise ValueError("device unpack requires words on a HIP device")
    stride = -(-columns // 32)
    if words.dtype != torch.int32 or tuple(words.shape) != (rows, stride) or not words.is_contiguous():
        raise ValueError(
            f"packed sign matrix must be contiguous int32 with shape {(rows, stride)}, got "
            f"{words.dtype} {tuple(words.shape)}"
        )
    out = torch.empty(rows, columns, dtype=dtype, device=words.device)
    lib = _native.load()
    bad = torch.empty(1, dtype=torch.int32, device=words.device)
    stream = _native.current_stream_handle(words.device)
    _native.check(
        "nq_count_bad_padding",
        lib.nq_count_bad_padding(words.data_ptr(), rows, columns, stride, bad.data_ptr(), stream),
    )
    if int(bad.item()) != 0:
        raise ValueError("packed sign matrix has a non-zero padding bit")
    _native.check(
        "nq_unpack_signs",
        lib.nq_unpack_signs(
            words.data_ptr(), rows, columns, stride, _native.dtype_code(dtype), out.data_ptr(), stream
        ),
    )
    return out
