"""ctypes wrapper over the C oracle (test infrastructure only)."""

from __future__ import annotations

import ctypes

import numpy as np

from oracle.build_oracle import LIBRARY, build

_LIB = None


def lib() -> ctypes.CDLL:
    global _LIB
    if _LIB is None:
        if not LIBRARY.exists():
            build()
        handle = ctypes.CDLL(str(LIBRARY))
        vp, i64 = ctypes.c_void_p, ctypes.c_int64
        handle.oracle_bad_padding_rows.restype = i64
        handle.oracle_bad_padding_rows.argtypes = [vp, i64, i64]
        handle.oracle_unpack.restype = ctypes.c_int
        handle.oracle_unpack.argtypes = [vp, i64, i64, vp]
        handle.oracle_pack.restype = None
        handle.oracle_pack.argtypes = [vp, i64, i64, vp]
        handle.oracle_linear_f64.restype = None
        handle.oracle_linear_f64.argtypes = [i64, i64, i64, vp, vp, vp, vp, vp, vp, i64, vp, vp,
                                             vp, i64, vp, vp]
        _LIB = handle
    return _LIB


def _ptr(a: np.ndarray | None) -> int | None:
    return None if a is None else a.ctypes.data


def unpack(words: np.ndarray, rows: int, cols: int) -> np.ndarray:
    words = np.ascontiguousarray(words, dtype=np.int32)
    out = np.empty((rows, cols), dtype=np.int8)
    if lib().oracle_unpack(_ptr(words), rows, cols, _ptr(out)) != 0:
        raise ValueError("packed sign matrix has a non-zero padding bit")
    return out


def pack(signs: np.ndarray) -> np.ndarray:
    signs = np.ascontiguousarray(signs, dtype=np.int8)
    rows, cols = signs.shape
    words = np.empty((rows, (cols + 31) // 32), dtype=np.int32)
    lib().oracle_pack(_ptr(signs), rows, cols, _ptr(words))
    return words


def linear_f64(in_f, out_f, rank, left_words, right_words, s_pre, s_mid, s_out, x,
               bias=None, idx=None, sal=None) -> np.ndarray:
    f64 = lambda a: None if a is None else np.ascontiguousarray(a, dtype=np.float64)  # noqa: E731
    x = f64(x).reshape(-1, in_f)
    tokens = x.shape[0]
    k = 0 if idx is None else int(len(idx))
    idx_a = None if idx is None else np.ascontiguousarray(idx, dtype=np.int32)
    y = np.empty((tokens, out_f), dtype=np.float64)
    scratch = np.empty(rank, dtype=np.float64)
    lw = np.ascontiguousarray(left_words, dtype=np.int32)
    rw = np.ascontiguousarray(right_words, dtype=np.int32)
    arrays = [f64(s_pre), f64(s_mid), f64(s_out), f64(bias), f64(sal)]
    lib().oracle_linear_f64(in_f, out_f, rank, _ptr(lw), _ptr(rw), _ptr(arrays[0]),
                            _ptr(arrays[1]), _ptr(arrays[2]), _ptr(arrays[3]), k, _ptr(idx_a),
                            _ptr(arrays[4]), _ptr(x), tokens, _ptr(y), _ptr(scratch))
    return y
