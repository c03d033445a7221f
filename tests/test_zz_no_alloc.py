"""nq_linear_static, the allocation-free entry point, against nq_linear.

Both run the same kernels; the static one takes its workspace from the
library's per-device static scratch array instead of an argument. Calls run
back to back with shrinking inputs, so stale scratch contents from a larger
call would show up in a smaller one. Bar: bit-identical to nq_linear.
"""

from __future__ import annotations

import ctypes

import pytest
import torch

from nanoquant_amd import synthetic as syn
from nanoquant_amd.runtime import HipPackedBackend, _native

pytestmark = [
    pytest.mark.gpu,
    pytest.mark.skipif(not torch.cuda.is_available(), reason="needs a HIP device"),
]


def _say(*parts) -> None:
    print("[case]", *parts, flush=True)


def _call(layer, x: torch.Tensor, *, static: bool) -> tuple[int, torch.Tensor]:
    lib = _native.load()
    desc = layer.payload.desc
    tokens = x.shape[0]
    y = torch.full((tokens, layer.spec.out_features), -7.0, dtype=torch.float32, device=x.device)
    stream = _native.current_stream_handle(x.device)
    code = _native.dtype_code(x.dtype)
    if static:
        status = lib.nq_linear_static(ctypes.byref(desc), x.data_ptr(), code, tokens, y.data_ptr(), 0, stream)
    else:
        size = int(lib.nq_linear_workspace_bytes(ctypes.byref(desc), tokens))
        ws = torch.empty(size, dtype=torch.uint8, device=x.device)
        status = lib.nq_linear(ctypes.byref(desc), x.data_ptr(), code, tokens, y.data_ptr(), 0, ws.data_ptr(),
                               size, stream)
    torch.cuda.synchronize()
    return status, y


def test_static_entry_point_matches_nq_linear_on_shrinking_calls():
    backend = HipPackedBackend()
    qwen, llama = syn.qwen3_8b_layer(), syn.llama3_8b_layer()
    # (shape, tokens): a prefill call (2.5 MiB of workspace), then decode calls
    # with less and less workspace; every call fits the 4 MiB array.
    cases = [(qwen[0], 17), (qwen[4], 16), (llama[6], 4), (qwen[1], 1)]
    lib = _native.load()
    for i, (shape, tokens) in enumerate(cases):
        _say("static", shape.name, tokens)
        state = syn.synthetic_packed_layer(shape, seed=syn.BASE_SEED + 300 + i, salient=2, bias=True)
        layer = backend.prepare(state, "cuda")
        need = int(lib.nq_linear_workspace_bytes(ctypes.byref(layer.payload.desc), tokens))
        assert 0 < need <= _native.NQ_STATIC_SCRATCH_BYTES
        x = syn.synthetic_activations(tokens, shape.in_features, seed=300 + i, device="cuda")
        st_ref, ref = _call(layer, x, static=False)
        st, got = _call(layer, x, static=True)
        assert st_ref == _native.NQ_OK and st == _native.NQ_OK, (st_ref, st)
        assert torch.isfinite(ref).all()
        assert torch.equal(got, ref), (shape.name, tokens)
        # A second static call on the same input gives the same bits.
        _, again = _call(layer, x, static=True)
        assert torch.equal(again, ref)


def test_static_entry_point_rejects_calls_beyond_its_scratch():
    backend = HipPackedBackend()
    shape = syn.qwen3_8b_layer()[4]  # gate 4096 -> 12288 r3072 at 64 tokens: 16.6 MiB
    layer = backend.prepare(syn.synthetic_packed_layer(shape, seed=syn.BASE_SEED + 310), "cuda")
    x = syn.synthetic_activations(64, shape.in_features, seed=310, device="cuda")
    status, y = _call(layer, x, static=True)
    assert status == _native.NQ_ERR_SCRATCH
    assert "static scratch" in _native.status_text(status)
    assert bool((y == -7.0).all())  # nothing was launched
