"""Fused one-token decode calls (nq_linear_batch_fused) against the oracle's
fp32 forward of the same element-wise chain: the RMSNorm-folded residual
input, the SiLU-gated input and the residual epilogue with its per-tile sums
of squares; the attention input (the decode attention's merge folded into the
O projection) against the attention's own merge followed by a plain call; and
the fused decoder against the unfused one."""

from __future__ import annotations

import sys

import pytest
import torch

from nanoquant_amd import synthetic as syn
from nanoquant_amd.runtime import DecoderShellConfig, HipPackedBackend, PackedDecoder
from nanoquant_amd.runtime import shell_ops as ops
from nanoquant_amd.runtime._native import NativeCallError
from oracle import decoder_shell as ods
from oracle import nq_oracle as orc

pytestmark = [
    pytest.mark.gpu,
    pytest.mark.skipif(not torch.cuda.is_available(), reason="needs a HIP device"),
]

REL_L2 = 2e-3  # against the fp32 reference forward
EPS = 1e-6


def _say(*parts) -> None:
    print("[case]", *parts, flush=True)
    sys.stdout.flush()


def _tile_sums(h: torch.Tensor) -> torch.Tensor:
    """Sums of squares per 16 rows (fp64), the layout the residual epilogue writes."""

    h = h.double().reshape(-1)
    h = torch.nn.functional.pad(h, (0, (-h.numel()) % 16))
    return h.view(-1, 16).pow(2).sum(1)


def _rmsnorm(h: torch.Tensor, w: torch.Tensor) -> torch.Tensor:
    h = h.double()
    return (h / torch.sqrt(h.pow(2).mean() + EPS) * w.double()).float()


def _layers(backend, shapes, seed):
    states = [syn.synthetic_packed_layer(s, seed=seed + i) for i, s in enumerate(shapes)]
    return states, [backend.prepare(st, "cuda") for st in states]


@pytest.mark.parametrize("roles", [(0, 1, 2), (4, 5)])
def test_rmsnorm_input_matches_oracle(roles):
    backend = HipPackedBackend()
    shapes = [syn.qwen3_8b_layer()[r] for r in roles]
    _say("rmsnorm input", [s.name for s in shapes])
    states, layers = _layers(backend, shapes, syn.BASE_SEED + 300)
    g = torch.Generator().manual_seed(5)
    h = 3 * torch.randn(4096, generator=g)
    w = 1 + 0.1 * torch.randn(4096, generator=g)
    slots = _tile_sums(h).float().cuda()
    cols = [backend.norm_column_scale(layer, w.cuda()) for layer in layers]
    kwargs = dict(input_kind="rmsnorm", eps=EPS, col_scales=cols, norm_slots=slots)
    outs = backend.linear_batch_fused([h.cuda()] * len(layers), layers, **kwargs)
    again = backend.linear_batch_fused([h.cuda()] * len(layers), layers, **kwargs)
    xn = _rmsnorm(h, w)
    unfused = backend.linear_batch([xn.cuda()] * len(layers), layers)
    for state, y, y2, yu in zip(states, outs, again, unfused):
        expected = orc.packed_forward(orc.operands_from_state(state), xn[None])[0]
        err = orc.relative_l2(y, expected)
        assert err <= REL_L2, (state.spec.name, err)
        assert orc.relative_l2(y, yu) <= 2e-4, state.spec.name  # same arithmetic up to rounding
        assert torch.equal(y, y2)
        print(f"  {state.spec.name} rel_l2={err:.2e}", flush=True)


def test_silu_gate_input_matches_oracle():
    backend = HipPackedBackend()
    shape = syn.qwen3_8b_layer()[6]
    _say("silu gate input", shape.name)
    (state,), (layer,) = _layers(backend, [shape], syn.BASE_SEED + 310)
    g = torch.Generator().manual_seed(6)
    gate = 2 * torch.randn(12288, generator=g)
    up = torch.randn(12288, generator=g)
    (y,) = backend.linear_batch_fused([gate.cuda()], [layer], input_kind="silu_gate", ups=[up.cuda()])
    act = (gate.double() * torch.sigmoid(gate.double()) * up.double()).float()
    expected = orc.packed_forward(orc.operands_from_state(state), act[None])[0]
    err = orc.relative_l2(y, expected)
    assert err <= REL_L2, err
    print(f"  rel_l2={err:.2e}", flush=True)


@pytest.mark.parametrize("out_dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("input_kind", ["rmsnorm", "plain"])
def test_silu_product_output_matches_oracle(input_kind, out_dtype):
    """gate/up in one workgroup per output tile, the epilogue storing
    silu(gate) * up: against the oracle's fp32 gate and up, and equal to the
    two outputs of the same fused call computed separately."""

    backend = HipPackedBackend()
    shapes = [syn.qwen3_8b_layer()[r] for r in (4, 5)]
    _say("silu product", input_kind, out_dtype)
    states, layers = _layers(backend, shapes, syn.BASE_SEED + 330)
    g = torch.Generator().manual_seed(9)
    h = 3 * torch.randn(4096, generator=g)
    w = 1 + 0.1 * torch.randn(4096, generator=g)
    if input_kind == "rmsnorm":
        kwargs = dict(input_kind="rmsnorm", eps=EPS, col_scales=[backend.norm_column_scale(lay, w.cuda())
                                                                 for lay in layers],
                      norm_slots=_tile_sums(h).float().cuda())
        value, xn = h.cuda(), _rmsnorm(h, w)
    else:
        kwargs = {}
        value = syn.synthetic_activations(1, 4096, seed=9, device="cuda")[0]
        xn = value.float().cpu()
    (prod,) = backend.linear_batch_fused([value] * 2, layers, output_kind="silu_product", output_dtype=out_dtype,
                                         **kwargs)
    gate, up = backend.linear_batch_fused([value] * 2, layers, **kwargs)
    assert prod.dtype == out_dtype and prod.shape == (12288,)
    separate = torch.nn.functional.silu(gate.double()) * up.double()
    ref = [orc.packed_forward(orc.operands_from_state(st), xn[None])[0].double() for st in states]
    expected = (torch.nn.functional.silu(ref[0]) * ref[1]).float()
    tol = REL_L2 if out_dtype == torch.float32 else 5e-3  # bf16 rounding of the product: 2^-9
    err = orc.relative_l2(prod.float(), expected)
    assert err <= tol, err
    assert orc.relative_l2(prod.float(), separate.float()) <= (1e-5 if out_dtype == torch.float32 else 5e-3)
    print(f"  rel_l2={err:.2e}", flush=True)
    with pytest.raises(ValueError, match="two members"):
        backend.linear_batch_fused([value], layers[:1], output_kind="silu_product", **kwargs)


@pytest.mark.parametrize("role", [3, 6])
def test_residual_epilogue_adds_and_writes_tile_sums(role):
    backend = HipPackedBackend()
    shape = syn.qwen3_8b_layer()[role]
    _say("residual epilogue", shape.name)
    (state,), (layer,) = _layers(backend, [shape], syn.BASE_SEED + 320)
    x = syn.synthetic_activations(1, shape.in_features, seed=7)[0]
    r0 = 4 * torch.randn(shape.out_features, generator=torch.Generator().manual_seed(8))
    r = r0.cuda()
    slots = torch.full((-(-shape.out_features // 16),), -1.0, device="cuda")
    kind = "plain" if role == 3 else "silu_gate"
    ups = None if role == 3 else [torch.ones(shape.in_features, device="cuda")]
    value = x.cuda() if role == 3 else x.float().cuda()
    ret = backend.linear_batch_fused([value], [layer], input_kind=kind, ups=ups, residuals=[r], out_slots=[slots])
    assert ret is None
    act = x.float() if role == 3 else (x.double() * torch.sigmoid(x.double())).float()
    expected = orc.packed_forward(orc.operands_from_state(state), act[None])[0]
    err = orc.relative_l2((r.cpu() - r0), expected)
    assert err <= REL_L2, err
    assert torch.allclose(slots.cpu().double(), _tile_sums(r.cpu()), rtol=1e-5, atol=1e-3)


def test_fused_calls_reject_what_they_do_not_cover():
    backend = HipPackedBackend()
    shape = syn.qwen3_8b_layer()[0]
    state = syn.synthetic_packed_layer(shape, seed=syn.BASE_SEED + 330, salient=4)
    layer = backend.prepare(state, "cuda")
    h = torch.randn(4096, device="cuda")
    col = backend.norm_column_scale(layer, torch.ones(4096, device="cuda"))
    slots = _tile_sums(h).float().cuda()
    with pytest.raises(NativeCallError):  # salient columns read the raw input
        backend.linear_batch_fused([h], [layer], input_kind="rmsnorm", col_scales=[col], norm_slots=slots)
    with pytest.raises(ValueError):  # one token only
        backend.linear_batch_fused([torch.randn(2, 4096, device="cuda")], [layer])


def _attention_operands(max_pos, p, cache_dtype, seed, q_heads=32, kv_heads=8, head_dim=128):
    g = torch.Generator().manual_seed(seed)
    q = (3 * torch.randn(q_heads * head_dim, generator=g)).cuda()
    k = (3 * torch.randn(kv_heads * head_dim, generator=g)).cuda()
    v = torch.randn(kv_heads * head_dim, generator=g).cuda()
    cos, sin = ods.rope_tables(head_dim, 1e6, max_pos)
    caches = [torch.randn(kv_heads, max_pos, head_dim, generator=g).to(cache_dtype) for _ in range(2)]
    common = dict(q_heads=q_heads, kv_heads=kv_heads, head_dim=head_dim,
                  q_norm=(1 + 0.1 * torch.randn(head_dim, generator=g)).cuda(),
                  k_norm=(1 + 0.1 * torch.randn(head_dim, generator=g)).cuda(), eps=EPS, cos=cos.cuda(),
                  sin=sin.cuda(), position=torch.tensor([p], dtype=torch.int32, device="cuda"),
                  scaling=head_dim**-0.5)
    return q, k, v, caches, common


@pytest.mark.parametrize(
    "max_pos,p,cache_dtype,kv_heads,head_dim",
    [
        (640, 639, torch.bfloat16, 8, 128),  # 10 blocks (up-to-12 kind), last row; MFMA pass 1
        (640, 0, torch.bfloat16, 8, 128),    # one live block
        (512, 300, torch.float16, 8, 128),   # 8 blocks (up-to-8 kind)
        (768, 767, torch.bfloat16, 8, 128),  # 12 blocks (up-to-12 kind, every slot)
        (832, 777, torch.bfloat16, 8, 128),  # 13 blocks (up-to-16 kind)
        (1024, 1023, torch.bfloat16, 8, 128),  # 16 blocks
        (100, 64, torch.float16, 8, 128),    # 2 blocks, first row of the second
        (20, 7, torch.bfloat16, 8, 128),     # 1 block
        (640, 640, torch.bfloat16, 8, 128),  # position outside the cache: zero input
        (640, 639, torch.float32, 32, 64),   # head dim 64, fp32 cache, two q heads per kv head
        (130, 70, torch.bfloat16, 64, 64),   # head dim 64, one q head per kv head
        (512, 511, torch.float16, 16, 64),   # head dim 64, four q heads per kv head
    ],
)
def test_attention_input_equals_merge_then_plain_call(max_pos, p, cache_dtype, kv_heads, head_dim):
    # The folded input merges the blocks' fp16 outputs (acc / sum), the merge
    # kernel their fp32 accumulators: the O projection's results agree to the
    # fp16 rounding of a block output (unit roundoff 2^-11), within the 2e-3
    # bar; the appended cache rows are identical (the same pass 1), and so is a
    # zero input (for the MFMA pass 1 and for the other one-pass geometries).
    backend = HipPackedBackend()
    shape = syn.qwen3_8b_layer()[3]
    q_heads = shape.in_features // head_dim
    _say("attention input", max_pos, p, cache_dtype, f"{q_heads}/{kv_heads} x {head_dim}")
    (state,), (layer,) = _layers(backend, [shape], syn.BASE_SEED + 350)
    q, k, v, caches, common = _attention_operands(max_pos, p, cache_dtype, 11, q_heads, kv_heads, head_dim)
    r0 = 4 * torch.randn(4096, generator=torch.Generator().manual_seed(12))
    results = []
    for fold in (False, True):
        kc, vc = (c.cuda() for c in caches)
        r = r0.cuda()
        slots = torch.full((256,), -1.0, device="cuda")
        if fold:
            ws = ops.launch_decode_attention_partials(q, k, v, k_cache=kc, v_cache=vc, **common)
            ret = backend.linear_batch_fused([ws], [layer], input_kind="attention",
                                             attention_position=common["position"], attention_head_dim=head_dim,
                                             attention_max_positions=max_pos, residuals=[r], out_slots=[slots])
            assert ret is None
        else:
            attn = ops.launch_decode_attention(q, k, v, k_cache=kc, v_cache=vc, out_dtype=torch.float32, **common)
            backend.linear_batch_fused([attn], [layer], residuals=[r], out_slots=[slots])
            expected = orc.packed_forward(orc.operands_from_state(state), attn.cpu()[None])[0]
            err = orc.relative_l2(r.cpu() - r0, expected)
            assert err <= REL_L2, err
        results.append((r, slots, kc, vc))
    (r_m, s_m, kc_m, vc_m), (r_f, s_f, kc_f, vc_f) = results
    assert torch.equal(kc_m, kc_f) and torch.equal(vc_m, vc_f)
    if p >= max_pos:
        assert torch.equal(r_f.cpu(), r0) and torch.equal(r_m.cpu(), r0)  # zero input, no bias
        return
    err = orc.relative_l2(r_f.cpu() - r0, r_m.cpu() - r0)
    _say("folded against merged, rel-L2", f"{err:.2e}")
    assert err <= REL_L2, err
    assert orc.relative_l2(s_f.cpu(), s_m.cpu()) <= REL_L2


def test_attention_input_rejects_what_it_does_not_cover():
    backend = HipPackedBackend()
    (state,), (layer,) = _layers(backend, [syn.qwen3_8b_layer()[3]], syn.BASE_SEED + 351)
    q, k, v, caches, common = _attention_operands(1100, 5, torch.bfloat16, 13)
    kc, vc = (c.cuda() for c in caches)
    ws = ops.launch_decode_attention_partials(q, k, v, k_cache=kc, v_cache=vc, **common)
    kwargs = dict(input_kind="attention", attention_position=common["position"], attention_head_dim=128)
    with pytest.raises(NativeCallError):  # 18 cache blocks: more than one register pass holds
        backend.linear_batch_fused([ws], [layer], attention_max_positions=1100, **kwargs)
    with pytest.raises(ValueError):  # workspace smaller than the partials of the cache length
        backend.linear_batch_fused([ws[:1024]], [layer], attention_max_positions=1100, **kwargs)
    with pytest.raises(ValueError):  # head_dim must divide in_features and be 64, 128 or 256
        backend.linear_batch_fused([ws], [layer], input_kind="attention", attention_position=common["position"],
                                   attention_head_dim=96, attention_max_positions=1100)
    # head_dim 256 with a 16-bit cache is the unfused form: no partials to leave
    g = torch.Generator().manual_seed(14)
    kc2 = torch.randn(2, 64, 256, generator=g).to(torch.bfloat16).cuda()
    cos, sin = ods.rope_tables(256, 1e6, 64)
    with pytest.raises(NativeCallError):
        ops.launch_decode_attention_partials(
            torch.randn(8 * 256).cuda(), torch.randn(2 * 256).cuda(), torch.randn(2 * 256).cuda(), q_heads=8,
            kv_heads=2, head_dim=256, q_norm=None, k_norm=None, eps=EPS, cos=cos.cuda(), sin=sin.cuda(),
            position=torch.tensor([3], dtype=torch.int32, device="cuda"), k_cache=kc2, v_cache=kc2.clone(),
            scaling=256**-0.5)


SMALL = DecoderShellConfig(layers=3, hidden=256, intermediate=768, q_heads=4, kv_heads=2, head_dim=64, vocab=1000)


@pytest.mark.parametrize("cache", [torch.float32, torch.bfloat16])
def test_folded_attention_decoder_matches_unfolded(cache):
    # 130 cache rows: three blocks; the unfolded decoder rounds the attention
    # output to the activation dtype (fp32 here), the folded one merges the
    # blocks' fp16 outputs: logits agree to that rounding, and so do the tokens.
    weights = syn.synthetic_decoder(SMALL, seed=syn.BASE_SEED + 345, random_norms=True)
    prompt = torch.randint(0, SMALL.vocab, (70,), generator=torch.Generator().manual_seed(10)).cuda()
    runs = {}
    for fold in (True, False):
        decoder = PackedDecoder(SMALL, weights, device="cuda", max_positions=130, activation_dtype=torch.float32,
                                cache_dtype=cache, fold_attention_merge=fold)
        assert decoder.fuse_decode and decoder.fold_attention_merge == fold
        runs[fold] = decoder.generate_greedy(prompt, 40).tolist()
        decoder.reset()
        decoder.prefill(prompt)
        bufs = decoder._decode_bufs or decoder._buffers(1)
        decoder._decode_bufs = bufs
        logits = []
        for token in runs[fold][:8]:
            decoder.ids.fill_(token)
            decoder._forward(decoder.ids, bufs)
            decoder.position += 1
            logits.append(decoder.logits.clone())
        runs[(fold, "logits")] = logits
    for a, b in zip(runs[(True, "logits")], runs[(False, "logits")]):
        err = orc.relative_l2(a, b)
        _say("folded decoder logits against unfolded, rel-L2", f"{err:.2e}")
        assert err <= 2e-3
    assert runs[True][:8] == runs[False][:8]


@pytest.mark.parametrize("act", [torch.float32, torch.bfloat16])
def test_fused_decoder_matches_unfused(act):
    weights = syn.synthetic_decoder(SMALL, seed=syn.BASE_SEED + 340, random_norms=True)
    prompt = torch.randint(0, SMALL.vocab, (20,), generator=torch.Generator().manual_seed(9)).cuda()
    runs = {}
    for fuse in (True, False):
        decoder = PackedDecoder(SMALL, weights, device="cuda", max_positions=64, activation_dtype=act,
                                cache_dtype=torch.float32, fuse_decode=fuse)
        assert decoder.fuse_decode == fuse
        logits = []
        tokens = decoder.generate_greedy(prompt, 8, use_graph=False)
        runs[fuse] = tokens.tolist()
        decoder.reset()
        decoder.prefill(prompt)
        bufs = decoder._decode_bufs or decoder._buffers(1)
        decoder._decode_bufs = bufs
        for token in runs[fuse][:4]:
            decoder.ids.fill_(token)
            decoder._forward(decoder.ids, bufs)
            decoder.position += 1
            logits.append(decoder.logits.clone())
        runs[(fuse, "logits")] = logits
    tol = 2e-3 if act == torch.float32 else 2e-2
    for a, b in zip(runs[(True, "logits")], runs[(False, "logits")]):
        assert orc.relative_l2(a, b) <= tol
    assert runs[True][:3] == runs[False][:3]
