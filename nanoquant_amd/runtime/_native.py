"""ctypes binding of the C ABI in ``include/nqamd.h``.

The library is loaded from ``nanoquant_amd/_lib/libnqamd.so`` (built in-tree by
``nanoquant_amd.build``). There is no fallback: a missing library raises
``NativeLibraryError`` at the first call that needs it.
"""

from __future__ import annotations

import ctypes
from pathlib import Path

import torch

LIBRARY_PATH = Path(__file__).resolve().parent.parent / "_lib" / "libnqamd.so"

NQ_OK = 0
NQ_ERR_ARGUMENT = -1
NQ_ERR_DTYPE = -2
NQ_ERR_SHAPE = -3
NQ_ERR_ALIGNMENT = -4
NQ_ERR_WORKSPACE = -5
NQ_ERR_LAUNCH = -6
NQ_ERR_DEVICE = -7
NQ_ERR_UNSUPPORTED = -8
NQ_ERR_SCRATCH = -9
NQ_STATIC_SCRATCH_BYTES = 4 << 20

NQ_DECODE_SPLIT = 0
NQ_DECODE_FUSED = 1
# nq_prefill_operands
NQ_PREFILL_FP16 = 0
NQ_PREFILL_FP16_SPLIT = 1

DTYPE_CODES: dict[torch.dtype, int] = {
    torch.float32: 0,
    torch.float16: 1,
    torch.bfloat16: 2,
    torch.int8: 3,
    torch.int32: 4,
}

# Every symbol include/nqamd.h and include/nqamd_shell.h declare; tests check
# the library exports them all.
EXPORTED_SYMBOLS = (
    "nq_abi_version",
    "nq_status_string",
    "nq_query_device",
    "nq_unpack_signs",
    "nq_count_bad_padding",
    "nq_tiles_header_bytes",
    "nq_tiles_bytes",
    "nq_prepare_tiles",
    "nq_linear_workspace_bytes",
    "nq_linear",
    "nq_linear_static",
    "nq_read_stream",
    "nq_linear_batch",
    "nq_linear_batch_fused",
    "nq_decode_mixed_v_words",
    "nq_decode_product_codebook_words",
    "nq_transpose_signs",
    "nq_embedding",
    "nq_embedding_slots",
    "nq_add_rmsnorm",
    "nq_qk_norm_rope_cache",
    "nq_attention_workspace_bytes",
    "nq_attention",
    "nq_decode_attention_workspace_bytes",
    "nq_decode_attention",
    "nq_decode_attention_partials",
    "nq_silu_mul",
    "nq_output_projection_workspace_bytes",
    "nq_output_projection",
    "nq_greedy_select",
)


class NativeLibraryError(RuntimeError):
    """The HIP library is missing or failed to load."""


class NativeCallError(RuntimeError):
    """A C-ABI call returned a non-zero nq_status."""

    def __init__(self, function: str, status: int, message: str) -> None:
        super().__init__(f"{function} failed with status {status}: {message}")
        self.function = function
        self.status = status


class DeviceCaps(ctypes.Structure):
    _fields_ = [
        ("arch", ctypes.c_char * 64),
        ("compute_units", ctypes.c_int32),
        ("wavefront_size", ctypes.c_int32),
        ("lds_bytes_per_block", ctypes.c_int64),
        ("global_mem_bytes", ctypes.c_int64),
        ("clock_khz", ctypes.c_int32),
        ("memory_clock_khz", ctypes.c_int32),
        ("memory_bus_width_bits", ctypes.c_int32),
        ("is_gfx950", ctypes.c_int32),
    ]


class LinearDesc(ctypes.Structure):
    _fields_ = [
        ("in_features", ctypes.c_int64),
        ("out_features", ctypes.c_int64),
        ("rank", ctypes.c_int64),
        ("right_words", ctypes.c_void_p),
        ("left_words", ctypes.c_void_p),
        ("scale_pre", ctypes.c_void_p),
        ("scale_mid", ctypes.c_void_p),
        ("scale_post", ctypes.c_void_p),
        ("scale_dtype", ctypes.c_int32),
        ("bias_dtype", ctypes.c_int32),
        ("bias", ctypes.c_void_p),
        ("salient_count", ctypes.c_int64),
        ("salient_indices", ctypes.c_void_p),
        ("salient_values", ctypes.c_void_p),
        ("salient_dtype", ctypes.c_int32),
        ("salient_scales", ctypes.c_void_p),
        ("patch_rank", ctypes.c_int64),
        ("patch_left", ctypes.c_void_p),
        ("patch_right", ctypes.c_void_p),
        ("patch_dtype", ctypes.c_int32),
        ("row_count", ctypes.c_int64),
        ("row_indices", ctypes.c_void_p),
        ("row_values", ctypes.c_void_p),
        ("row_scales", ctypes.c_void_p),
        ("tiles", ctypes.c_void_p),
        ("tiles_bytes", ctypes.c_int64),
        ("decode_launch", ctypes.c_int32),
        ("prefill_operands", ctypes.c_int32),
    ]


# nq_input_kind
INPUT_PLAIN, INPUT_RMSNORM, INPUT_SILU_GATE, INPUT_ATTENTION = 0, 1, 2, 3
# nq_output_kind
OUTPUT_PLAIN, OUTPUT_SILU_PRODUCT = 0, 1


class DecodeFusion(ctypes.Structure):
    """nq_decode_fusion (include/nqamd.h)."""

    _fields_ = [
        ("input_kind", ctypes.c_int32),
        ("eps", ctypes.c_float),
        ("col_scales", ctypes.POINTER(ctypes.c_void_p)),
        ("norm_slots", ctypes.c_void_p),
        ("norm_slot_count", ctypes.c_int64),
        ("ups", ctypes.POINTER(ctypes.c_void_p)),
        ("residuals", ctypes.POINTER(ctypes.c_void_p)),
        ("out_slots", ctypes.POINTER(ctypes.c_void_p)),
        ("output_kind", ctypes.c_int32),
        ("attn_position", ctypes.c_void_p),
        ("attn_head_dim", ctypes.c_int32),
        ("attn_max_positions", ctypes.c_int64),
    ]


_LIB: ctypes.CDLL | None = None


def library_available() -> bool:
    return LIBRARY_PATH.exists()


def _declare(lib: ctypes.CDLL) -> None:
    c_int, c_i64, vp = ctypes.c_int, ctypes.c_int64, ctypes.c_void_p
    i32, f32 = ctypes.c_int32, ctypes.c_float
    desc_p = ctypes.POINTER(LinearDesc)
    table = {
        "nq_abi_version": (c_int, []),
        "nq_status_string": (ctypes.c_char_p, [c_int]),
        "nq_query_device": (c_int, [c_int, ctypes.POINTER(DeviceCaps)]),
        "nq_unpack_signs": (c_int, [vp, c_i64, c_i64, c_i64, ctypes.c_int32, vp, vp]),
        "nq_count_bad_padding": (c_int, [vp, c_i64, c_i64, c_i64, vp, vp]),
        "nq_tiles_header_bytes": (c_i64, []),
        "nq_tiles_bytes": (c_i64, [c_i64, c_i64, c_i64]),
        "nq_prepare_tiles": (c_int, [desc_p, vp, c_i64, vp]),
        "nq_linear_workspace_bytes": (c_i64, [desc_p, c_i64]),
        "nq_linear": (
            c_int,
            [desc_p, vp, ctypes.c_int32, c_i64, vp, ctypes.c_int32, vp, c_i64, vp],
        ),
        "nq_linear_static": (c_int, [desc_p, vp, ctypes.c_int32, c_i64, vp, ctypes.c_int32, vp]),
        "nq_read_stream": (c_int, [vp, c_i64, vp, c_i64, vp]),
        "nq_linear_batch": (
            c_int,
            [ctypes.POINTER(desc_p), ctypes.c_int32, ctypes.POINTER(vp), ctypes.c_int32, c_i64,
             ctypes.POINTER(vp), ctypes.c_int32, ctypes.POINTER(vp), ctypes.POINTER(c_i64), vp],
        ),
        "nq_linear_batch_fused": (
            c_int,
            [ctypes.POINTER(desc_p), ctypes.c_int32, ctypes.POINTER(vp), ctypes.c_int32, ctypes.POINTER(vp),
             ctypes.c_int32, ctypes.POINTER(vp), ctypes.POINTER(c_i64), ctypes.POINTER(DecodeFusion), vp],
        ),
        "nq_decode_mixed_v_words": (c_int, [vp, c_i64, vp, c_i64, vp, c_i64, c_i64, vp, vp, vp]),
        "nq_decode_product_codebook_words": (c_int, [vp, c_i64, vp, c_i64, vp, vp, c_i64, c_i64, vp, vp]),
        "nq_transpose_signs": (c_int, [vp, c_i64, c_i64, vp, vp]),
        "nq_embedding": (c_int, [vp, c_i64, vp, i32, c_i64, c_i64, vp, vp, vp]),
        "nq_embedding_slots": (c_int, [vp, c_i64, vp, i32, c_i64, c_i64, vp, vp, vp, vp]),
        "nq_add_rmsnorm": (c_int, [vp, vp, i32, vp, i32, f32, c_i64, c_i64, vp, i32, vp]),
        "nq_qk_norm_rope_cache": (
            c_int,
            [vp, vp, vp, c_i64, i32, i32, i32, vp, vp, i32, f32, vp, vp, vp, c_i64, vp, vp, vp, i32, vp],
        ),
        "nq_attention_workspace_bytes": (c_i64, [c_i64, i32, i32, c_i64]),
        "nq_attention": (
            c_int, [vp, vp, vp, i32, c_i64, i32, i32, i32, vp, c_i64, f32, vp, i32, vp, c_i64, vp],
        ),
        "nq_decode_attention_workspace_bytes": (c_i64, [i32, i32, i32, i32, c_i64]),
        "nq_decode_attention": (
            c_int,
            [vp, vp, vp, i32, i32, i32, vp, vp, i32, f32, vp, vp, vp, c_i64, vp, vp, i32, f32, vp, i32, vp,
             c_i64, vp],
        ),
        "nq_decode_attention_partials": (
            c_int,
            [vp, vp, vp, i32, i32, i32, vp, vp, i32, f32, vp, vp, vp, c_i64, vp, vp, i32, f32, vp, c_i64, vp],
        ),
        "nq_silu_mul": (c_int, [vp, vp, c_i64, vp, i32, vp]),
        "nq_output_projection_workspace_bytes": (c_i64, [c_i64, c_i64]),
        "nq_output_projection": (c_int, [vp, i32, vp, c_i64, c_i64, vp, vp, c_i64, vp]),
        "nq_greedy_select": (c_int, [vp, c_i64, c_i64, vp, vp, c_i64, vp, vp, vp]),
    }
    for name, (restype, argtypes) in table.items():
        fn = getattr(lib, name)
        fn.restype = restype
        fn.argtypes = argtypes


def load() -> ctypes.CDLL:
    """Load (once) and return the HIP library; raise if it is not built."""

    global _LIB
    if _LIB is None:
        if not LIBRARY_PATH.exists():
            raise NativeLibraryError(
                f"HIP library not built: {LIBRARY_PATH} (run python -m nanoquant_amd.build)"
            )
        try:
            lib = ctypes.CDLL(str(LIBRARY_PATH))
        except OSError as error:
            raise NativeLibraryError(f"cannot load {LIBRARY_PATH}: {error}") from error
        _declare(lib)
        _LIB = lib
    return _LIB


def status_text(status: int) -> str:
    raw = load().nq_status_string(status)
    return raw.decode() if raw else "unknown status"


def check(function: str, status: int) -> None:
    if status != NQ_OK:
        raise NativeCallError(function, status, status_text(status))


def dtype_code(dtype: torch.dtype) -> int:
    if dtype not in DTYPE_CODES:
        raise ValueError(f"dtype {dtype} has no C-ABI code")
    return DTYPE_CODES[dtype]


def current_stream_handle(device: torch.device) -> int:
    return torch.cuda.current_stream(device).cuda_stream


def query_device(index: int) -> DeviceCaps:
    caps = DeviceCaps()
    check("nq_query_device", load().nq_query_device(index, ctypes.byref(caps)))
    return caps


def pointer(tensor: torch.Tensor | None) -> int | None:
    return None if tensor is None else tensor.data_ptr()
