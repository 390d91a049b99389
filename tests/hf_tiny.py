"""A small random-init Gemma 4 (HF transformers' own model code) with every feature of E2B's text
decoder, and its float32 CPU reference, for the GPU tests that drive the whole model."""
import copy

import torch


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
