"""The registered torch operators (w8a8.torch_ops) on the GPU: torch.library.opcheck on each (schema,
fake implementation against the real kernel, no hidden aliasing), one function of them compiled
with fullgraph=True (so no graph break anywhere) giving the eager result bit for bit, and the tiny
HF Gemma 4 with every decoder layer compiled the way the reference compiles its layers
(gemma_npu.py:255-265: torch.compile(layer.forward, dynamic=True) for prefill rows, the eager
forward for decode rows) giving the eager model's logits.  The compiler backend is aot_eager: it
traces with dynamo and AOTAutograd as inductor does, without generating kernels of its own."""
import copy

import pytest
import torch

from hf_tiny import build, rel_err

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _weights(N, K, seed, interleave=0):
    from w8a8 import ops
    g = torch.Generator(device=DEV).manual_seed(seed)
    w = torch.randint(-127, 128, (N, K), generator=g, dtype=torch.int8, device=DEV)
    sw = torch.rand(N, generator=g, device=DEV) * 0.015 + 0.005
    return w, sw, ops.pack_weight(w, "nk", interleave, sw=sw)


def test_opcheck_every_operator():
    from w8a8 import ops, torch_ops  # noqa: F401
    g = torch.Generator(device=DEV).manual_seed(1)
    x = torch.randn(40, 256, generator=g, device=DEV).to(torch.bfloat16)
    w, sw, pw = _weights(512, 256, 2)
    torch.library.opcheck(torch.ops.w8a8.linear.default, (x, pw.data, sw, 512, 256, 0, "none", None, None, 1e-6))
    _, swg, pwg = _weights(512, 256, 3, interleave=256)
    torch.library.opcheck(torch.ops.w8a8.linear.default, (x, pwg.data, swg, 512, 256, 256, "gelu", None, None, 1e-6))
    a = torch.randint(-127, 128, (40, 256), generator=g, dtype=torch.int8, device=DEV)
    c = torch.empty((40, 512), dtype=torch.int32, device=DEV)
    torch.library.opcheck(torch.ops.w8a8.mm_i8.default, (a, pw.data, 512, 256, c))
    gw = ops.pack_gemv_weight(w)
    torch.library.opcheck(torch.ops.w8a8.gemv.default, (x[:4].contiguous(), gw.data, 512, 256, sw.to(torch.bfloat16)))
    nw = (torch.rand(256, generator=g, device=DEV) + 0.5).to(torch.bfloat16)
    torch.library.opcheck(torch.ops.w8a8.rms_norm.default, (x, nw, 1e-6))
    # a transposed (non-contiguous) input: the real op and the fake both return contiguous rows
    xt = torch.randn(256, 40, generator=g, device=DEV).to(torch.bfloat16).t()
    torch.library.opcheck(torch.ops.w8a8.rms_norm.default, (xt, nw, 1e-6))
    yt = torch.ops.w8a8.rms_norm(xt, nw, 1e-6)
    assert yt.is_contiguous() and torch.equal(yt, torch.ops.w8a8.rms_norm(xt.contiguous(), nw, 1e-6))
    q = torch.randn(4, 24, 128, generator=g, device=DEV).to(torch.bfloat16)
    k = torch.randn(1, 24, 128, generator=g, device=DEV).to(torch.bfloat16)
    v = torch.randn(1, 24, 128, generator=g, device=DEV).to(torch.bfloat16)
    torch.library.opcheck(torch.ops.w8a8.attention.default, (q, k, v, 0, 8, 0.1))
    torch.library.opcheck(torch.ops.w8a8.attention_decode.default, (q[:, -1].contiguous(), k, v, 23, 0, 0.1))


@torch.inference_mode()
def test_fullgraph_compile_matches_eager():
    """rmsnorm -> [gate; up] GEMM with the GELU epilogue -> down GEMM with the residual epilogue ->
    int32 GEMM, compiled as one graph: bit for bit the eager calls."""
    from w8a8 import ops, torch_ops
    g = torch.Generator(device=DEV).manual_seed(5)
    x = torch.randn(300, 256, generator=g, device=DEV).to(torch.bfloat16)
    nw = (torch.rand(256, generator=g, device=DEV) + 0.5).to(torch.bfloat16)
    _, _, gu = _weights(1024, 256, 6, interleave=512)
    _, _, down = _weights(256, 512, 7)
    _, _, w32 = _weights(128, 256, 8)
    a8 = torch.randint(-127, 128, (300, 256), generator=g, dtype=torch.int8, device=DEV)

    def block(x, a8):
        h = torch_ops.rms_norm(x, nw, 1e-6)
        act = torch_ops.linear(h, gu, epilogue="gelu")
        y = torch_ops.linear(act, down, epilogue="residual", residual=x)
        c = torch.empty((a8.shape[0], 128), dtype=torch.int32, device=a8.device)
        torch.ops.w8a8.mm_i8(a8, w32.data, 128, 256, c)
        return y, c

    want_y, want_c = block(x, a8)
    compiled = torch.compile(block, fullgraph=True, backend="aot_eager")
    got_y, got_c = compiled(x, a8)
    assert torch.equal(got_y, want_y)
    assert torch.equal(got_c, want_c)
    ref_c = torch.empty_like(want_c)
    ops.gemm_i32(a8, w32, ref_c)
    assert torch.equal(got_c, ref_c)


@torch.inference_mode()
def test_hf_layers_compiled_like_the_reference():
    """Every decoder layer compiled as the reference compiles it: the prefill logits equal the eager
    model's bit for bit (the compiled graph calls the same kernels on the same inputs, and aot_eager
    runs HF's own torch ops unfused), each layer's [q; k; v] GEMM runs once per attention call in the
    compiled forward too (the input-identity check that hands its columns to q, k and v survives
    tracing), and decode after the compiled prefill matches the eager model's."""
    from w8a8 import hf, ops
    torch._dynamo.reset()
    # one compiled forward per layer, each with its own hooks to guard on (gemma_npu.py:260 raises the
    # same limit)
    torch._dynamo.config.cache_size_limit = 256
    base = build(seed=23).to(torch.bfloat16).to(DEV)
    eager_model = copy.deepcopy(base)
    hf.to_gpu(eager_model)
    model = copy.deepcopy(base)
    hf.to_gpu(model)
    for layer in hf.language_model(model).layers:
        eager = layer.forward
        compiled = torch.compile(eager, dynamic=True, backend="aot_eager")
        layer.forward = (lambda e, c: lambda hidden_states, *a, **k:
                         (c if hidden_states.shape[1] > 16 else e)(hidden_states, *a, **k))(eager, compiled)
    # count GEMM launches per [q; k; v] weight at run time: both the eager helper and the registered
    # operator's implementation end in ops.linear_bf16
    qkv = {roles["qkv"].packed.data.data_ptr(): i for i, roles in enumerate(model.layer_gemms)}
    calls = {}
    real = ops.linear_bf16

    def counted(x, w, *a, **k):
        i = qkv.get(w.data.data_ptr())
        if i is not None:
            calls[i] = calls.get(i, 0) + 1
        return real(x, w, *a, **k)
    ids = torch.randint(0, 512, (1, 40), generator=torch.Generator().manual_seed(24)).to(DEV)
    want = eager_model(input_ids=ids, use_cache=True)
    ops.linear_bf16 = counted
    try:
        got = model(input_ids=ids, use_cache=True)
    finally:
        ops.linear_bf16 = real
    assert calls == {i: 1 for i in range(len(model.layer_gemms))}, f"[q; k; v] GEMMs per layer: {calls}"
    e = rel_err(got.logits[0], want.logits[0])
    print(f"prefill logits, compiled layers vs eager: max relative error {e:.2e}")
    assert torch.equal(got.logits, want.logits)
    nxt = want.logits[0, -1].argmax().view(1, 1)
    want1 = eager_model(input_ids=nxt, past_key_values=want.past_key_values, use_cache=True)
    got1 = model(input_ids=nxt, past_key_values=got.past_key_values, use_cache=True)
    e1 = rel_err(got1.logits[0, -1], want1.logits[0, -1])
    print(f"decode logits after the compiled prefill: relative error {e1:.2e}")
    assert torch.equal(got1.logits, want1.logits)
