"""HF transformers' Gemma 4 text decoder driven unchanged on top of the engine (w8a8.hf.to_gpu).

A small random-init Gemma 4 with every feature of E2B's decoder -- sliding and full layers
(head_dim 128 / 256), 4 query heads on 1 KV head, KV-shared layers, double-wide MLPs, per-layer
inputs -- runs its prefill (W8A8 GEMMs, prefill attention) and its decode loop (int8 GEMVs, decode
attention) on the GPU.  The reference is the same HF model on the CPU in float32 with the same
per-channel int8 weights dequantized (what the engine's weights mean), torch's sdpa as attention.
The W8A8 prefill also rounds activations to int8 per token, so its logits differ by that
quantisation noise: bounded here by the relative error of each logits row (for scale: the same
model in bf16 on the CPU is 2-3% from float32, and the int8 weights alone move it 4-7%); decode
(weight-only GEMV) is tighter.
"""
import copy

import pytest
import torch

from hf_tiny import build, dequantized_reference, rel_err

pytestmark = pytest.mark.gpu
DEV = "cuda"


@torch.inference_mode()
def test_prefill_and_decode_loop():
    from w8a8 import hf
    base = build()
    ref = dequantized_reference(base)
    ours = copy.deepcopy(base).to(torch.bfloat16).to(DEV)
    gemms = hf.to_gpu(ours)
    assert len(gemms) == 10 * 6 + 2  # six groups per layer, the PLE model projection, the LM head
    T = 40
    ids = torch.randint(0, 512, (1, T), generator=torch.Generator().manual_seed(1))

    out_ref = ref(input_ids=ids, use_cache=True)
    out = ours(input_ids=ids.to(DEV), use_cache=True)
    e_pre = rel_err(out.logits[0], out_ref.logits[0])
    print(f"prefill: max relative logits error {e_pre:.4f}")
    assert e_pre < 0.10

    past_ref, past = out_ref.past_key_values, out.past_key_values
    nxt = out_ref.logits[0, -1].argmax().view(1, 1)
    for step in range(6):  # teacher-forced: both models get the reference's greedy token
        o_ref = ref(input_ids=nxt, past_key_values=past_ref, use_cache=True)
        o = ours(input_ids=nxt.to(DEV), past_key_values=past, use_cache=True)
        e = rel_err(o.logits[0, -1], o_ref.logits[0, -1])
        print(f"decode step {step} (position {T + step}): relative logits error {e:.4f}")
        assert e < 0.05
        past_ref, past = o_ref.past_key_values, o.past_key_values
        nxt = o_ref.logits[0, -1].argmax().view(1, 1)


@torch.inference_mode()
def test_decode_past_the_window():
    """Decode continues past the sliding window (16 here), where HF's sliding cache keeps only the
    last window of keys; one call per token, the unchanged HF loop."""
    from w8a8 import hf
    base = build(seed=3)
    ref = dequantized_reference(base)
    ours = copy.deepcopy(base).to(torch.bfloat16).to(DEV)
    hf.to_gpu(ours)
    ids = torch.randint(0, 512, (1, 5), generator=torch.Generator().manual_seed(2))
    o_ref = ref(input_ids=ids, use_cache=True)
    o = ours(input_ids=ids.to(DEV), use_cache=True)
    past_ref, past = o_ref.past_key_values, o.past_key_values
    worst = 0.0
    for step in range(24):
        nxt = o_ref.logits[0, -1].argmax().view(1, 1)
        o_ref = ref(input_ids=nxt, past_key_values=past_ref, use_cache=True)
        o = ours(input_ids=nxt.to(DEV), past_key_values=past, use_cache=True)
        worst = max(worst, rel_err(o.logits[0, -1], o_ref.logits[0, -1]))
        past_ref, past = o_ref.past_key_values, o.past_key_values
    print(f"decode to position 29: max relative logits error {worst:.4f}")
    assert worst < 0.05


@torch.inference_mode()
def test_gpu_rmsnorm_matches_the_module():
    """GpuRMSNorm (the row kernel) against HF's Gemma4RMSNorm on the same bf16 rows, with and without
    a weight, on decoder-shaped inputs (hidden rows, per-head rows, one decode row): within one bf16
    ulp everywhere, bit for bit on nearly all elements (the sum of squares is added in another
    order than torch's mean)."""
    from transformers.models.gemma4.modeling_gemma4 import Gemma4RMSNorm
    from w8a8 import hf
    g = torch.Generator().manual_seed(21)
    for shape, with_scale in (((1, 40, 256), True), ((1, 40, 4, 128), True), ((1, 1, 4, 256), False),
                              ((1, 1, 1536), True), ((3, 7, 64), True)):
        N = shape[-1]
        norm = Gemma4RMSNorm(N, eps=1e-6, with_scale=with_scale)
        if with_scale:
            with torch.no_grad():
                norm.weight.copy_(torch.rand(N, generator=g) + 0.5)
        norm = norm.to(torch.bfloat16).to(DEV)
        x = (torch.randn(shape, generator=g) * 3).to(torch.bfloat16).to(DEV)
        want = norm(x)
        got = hf.GpuRMSNorm(norm)(x)
        assert got.shape == want.shape and got.dtype == torch.bfloat16
        gi = got.view(torch.int16).int().cpu()
        wi = want.view(torch.int16).int().cpu()
        assert (gi - wi).abs().max().item() <= 1, f"{shape}: more than one bf16 ulp apart"
        assert (gi == wi).float().mean().item() > 0.97, f"{shape}: too few bit-exact elements"
    f32 = torch.randn(2, 8, 64, device=DEV)
    assert torch.equal(hf.GpuRMSNorm(Gemma4RMSNorm(64).to(DEV))(f32), Gemma4RMSNorm(64).to(DEV)(f32))


@torch.inference_mode()
def test_gpu_mlp_matches_the_module_path():
    """GpuMLP (GELU-tanh * up in the gate/up GEMM's epilogue) against the same MLP run through the
    engine's separate gate/up GEMM and HF's activation and product: the same bf16 gate and up feed
    the same arithmetic, so the activations agree to one bf16 ulp (torch's tanh against the
    epilogue's exp2 form) and mostly bit for bit; after the down GEMM's per-token quant the MLP
    outputs agree to quantisation noise.  Decode rows take the module's own path, bit for bit."""
    from w8a8 import hf, ops
    ours = copy.deepcopy(build(seed=17)).to(torch.bfloat16).to(DEV)
    hf.to_gpu(ours)
    mlp = ours.model.layers[6].mlp
    assert isinstance(mlp, hf.GpuMLP) and mlp.fused
    g = torch.Generator().manual_seed(18)
    for rows in (40, 300, 3):
        x = torch.randn(1, rows, 256, generator=g).to(torch.bfloat16).to(DEV)
        got = mlp(x)
        want = mlp.orig(x)
        assert got.shape == want.shape == (1, rows, 256)
        if rows < 16:
            assert torch.equal(got, want)
            continue
        x2 = x.reshape(rows, 256)
        a_fused = ops.linear_bf16(x2, mlp.gate_up.packed_gelu, epilogue="gelu")
        o = mlp.orig
        a_ref = o.act_fn(o.gate_proj(x2)) * o.up_proj(x2)
        ai, ri = a_fused.view(torch.int16).int().cpu(), a_ref.view(torch.int16).int().cpu()
        assert (ai - ri).abs().max().item() <= 1
        assert (ai == ri).float().mean().item() > 0.99
        assert rel_err(got[0], want[0]) < 2e-2


@torch.inference_mode()
def test_projection_groups_run_once_per_call():
    """The [q; k; v] weight runs once per attention call and its columns are handed to the three
    projections (w8a8.hf.share_input), nothing stays parked after the call, and the plain GEMM
    packing of a [gate; up] weight is never made when the MLP takes the fused GELU epilogue."""
    from w8a8 import hf
    ours = copy.deepcopy(build(seed=19)).to(torch.bfloat16).to(DEV)
    hf.to_gpu(ours)
    calls = {}
    for i, roles in enumerate(ours.layer_gemms):
        w = roles["qkv"]
        orig = w.apply

        def counted(x2d, orig=orig, i=i):
            calls[i] = calls.get(i, 0) + 1
            return orig(x2d)
        w.apply = counted
    ids = torch.randint(0, 512, (1, 24), generator=torch.Generator().manual_seed(20))
    out = ours(input_ids=ids.to(DEV), use_cache=True)
    assert calls == {i: 1 for i in range(len(ours.layer_gemms))}
    nxt = out.logits[0, -1].argmax().view(1, 1)
    ours(input_ids=nxt, past_key_values=out.past_key_values, use_cache=True)
    assert calls == {i: 2 for i in range(len(ours.layer_gemms))}
    for layer in ours.model.layers:
        for name in ("q_proj", "k_proj", "v_proj"):
            proj = getattr(layer.self_attn, name, None)
            if isinstance(proj, hf.QuantizedLinear):
                assert proj.parked is None
        assert layer.mlp.gate_up._packed is None
