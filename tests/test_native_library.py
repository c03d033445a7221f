"""The C-ABI library loads and exports every entry point include/nqamd.h declares.
No compute call is made here (no GPU needed)."""

from __future__ import annotations

import ctypes
import re
from pathlib import Path

from nanoquant_amd.runtime import _native

HEADER = Path(__file__).resolve().parent.parent / "include" / "nqamd.h"


def _declared_functions() -> set[str]:
    text = re.sub(r"/\*.*?\*/", "", HEADER.read_text(), flags=re.S)
    return set(re.findall(r"\b(nq_[a-z0-9_]+)\s*\(", text))


def test_header_and_binding_agree():
    assert _declared_functions() == set(_native.EXPORTED_SYMBOLS)


def test_library_exports_every_declared_symbol():
    lib = _native.load()
    for name in _declared_functions():
        assert hasattr(lib, name), name


def test_host_only_entry_points():
    lib = _native.load()
    assert lib.nq_abi_version() == 2
    assert _native.status_text(-5).startswith("workspace smaller")
    # Argument validation happens before any device work.
    desc = _native.LinearDesc()
    assert lib.nq_linear_workspace_bytes(ctypes.byref(desc), 1) == -1
    assert lib.nq_linear(ctypes.byref(desc), None, 0, 1, None, 0, None, 0, None) == _native.NQ_ERR_SHAPE
    assert lib.nq_unpack_signs(None, 1, 1, 1, 0, None, None) == _native.NQ_ERR_ARGUMENT
