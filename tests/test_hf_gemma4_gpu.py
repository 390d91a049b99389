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

pytestmark = pytest.mark.gpu
DEV = "cuda"


def tiny_config(window=16):
    from transformers.models.gemma4.configuration_gemma4 import Gemma4TextConfig
    return Gemma4TextConfig(vocab_size=512, hidden_size=256, intermediate_size=512, num_hidden_layers=10,
                            num_attention_heads=4, num_key_value_heads=1, head_dim=128, global_head_dim=256,
                            sliding_window=window, layer_types=(["sliding_attention"] * 4 + ["full_attention"]) * 2,
                            num_kv_shared_layers=4, use_double_wide_mlp=True, vocab_size_per_layer_input=512,
                            hidden_size_per_layer_input=64)


def build(seed=0):
    from transformers.models.gemma4.modeling_gemma4 import Gemma4ForCausalLM
    torch.manual_seed(seed)
    m = Gemma4ForCausalLM(tiny_config()).eval()
    with torch.no_grad():
        for p in m.parameters():  # larger weights than the 0.02 init, so the layers do visible work
            if p.dim() == 2:
                p.mul_(4.0)
        # q / k norm weights of head_dim^-1/4 keep the (scale 1.0) scores near unit variance, as a
        # trained model's small norm weights do; with the init's 1.0 the softmax is nearly one-hot
        # and bf16 rounding alone moves the logits by tens of percent
        for layer in m.model.layers:
            a = layer.self_attn
            a.q_norm.weight.fill_(a.head_dim ** -0.25)
            if getattr(a, "k_norm", None) is not None:
                a.k_norm.weight.fill_(a.head_dim ** -0.25)
    return m


def dequantized_reference(model):
    """CPU float32 copy whose linears hold the per-channel int8 weights times their scales."""
    ref = copy.deepcopy(model).float()
    with torch.no_grad():
        for mod in ref.modules():
            if isinstance(mod, torch.nn.Linear):
                w = mod.weight
                s = w.abs().amax(1, keepdim=True).clamp(min=1e-8) / 127
                mod.weight.copy_(torch.round(w / s).clamp(-127, 127) * s)
    ref.config._attn_implementation = "sdpa"
    return ref


def rel_err(a, b):
    a, b = a.float().cpu(), b.float().cpu()
    return ((a - b).norm(dim=-1) / b.norm(dim=-1)).max().item()


@torch.inference_mode()
def test_prefill_and_decode_loop():
    from w8a8 import hf
    base = build()
    ref = dequantized_reference(base)
    ours = copy.deepcopy(base).to(torch.bfloat16).to(DEV)
    gemms = hf.to_gpu(ours)
    assert len(gemms) == 10 * 6 + 1
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
