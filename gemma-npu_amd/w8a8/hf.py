"""HF transformers' Gemma 4 text decoder on the GPU with this engine underneath.

The reference swaps the decoder's linears for grouped W8A8 GEMMs (`to_npu`, gemma_npu.py:208-241,
with `NPUGemm`, gemma_npu.py:57-152, and `Slice`, gemma_npu.py:175-193), the LM head for an int8
GEMV (`Int8Head`, gemma_npu.py:159-172), and registers its attention as "local_sdpa"
(gemma_npu.py:253, local_attn.py:110-111).  `to_gpu` does the same on a model whose weights are on
the GPU:

    model = AutoModelForCausalLM.from_pretrained(...).to("cuda")      # or a random-init config
    hf.to_gpu(model)
    out = model(input_ids=ids, use_cache=True, logits_to_keep=1)      # prefill: W8A8 GEMMs
    out = model(input_ids=nxt, past_key_values=out.past_key_values)   # decode: int8 GEMVs

Groups as the reference forms them: [q; k; v] (q only on KV-shared layers), o, [gate; up], down,
the per-layer-input gate and projection, and the per-layer model projection.  Rows < 16 (decode)
take the weight-only int8 GEMV with bf16 scales (gemma_npu.py:120-121); more rows take per-token
quant -> int8 GEMM -> dequant (gemma_npu.py:123-152).  Unlike the reference, the small PLE gate and
projection stay on the GPU too.  Every RMSNorm module of the text decoder becomes one launch of the
engine's row kernel (GpuRMSNorm), and for prefill rows each MLP's GELU-tanh * up runs in the gate/up
GEMM's epilogue (GpuMLP); the other HF modules around them (RoPE, residuals, the KV cache, the decode
loop) run unchanged, as torch ops on the GPU.
"""
import torch

from . import attention, ops

DECODE_ROWS = 16  # rows below this go to the GEMV (gemma_npu.py:120)


class GpuGemm(torch.nn.Module):
    """One group of linears sharing an input, as one weight [sum of N, K] (gemma_npu.py:57-84):
    per-channel int8 quantisation (absmax / 127), packed for the GEMM (fp32 scales) and for the
    GEMV (bf16 scales, the reference's decode copy w_cpu / sw_cpu, gemma_npu.py:81-82)."""

    def __init__(self, linears, gelu_pair=False):
        super().__init__()
        w = torch.cat([l.weight.detach() for l in linears], 0)
        if w.device.type != "cuda":
            raise ValueError("to_gpu: move the model to the GPU first")
        self.N, self.K = w.shape
        self.sizes = [l.out_features for l in linears]
        self.dtype = w.dtype
        q, sw = ops.quant_rows(w.float().contiguous())
        self.sw = sw
        self.packed = ops.pack_weight(q, "nk", sw=sw)
        # [gate; up]: a second copy packed for the GEMM's fused gelu(gate) * up epilogue, which the
        # whole-prompt pipeline uses in place of the int32 result and k_gelu
        self.packed_gelu = ops.pack_weight(q, "nk", self.N // 2, sw=sw) if gelu_pair else None
        self.gemv_w = ops.pack_gemv_weight(q)
        self.sw_bf16 = sw.to(torch.bfloat16)
        self.pending = None

    def matmul(self, x2d):
        x2d = x2d.to(torch.bfloat16).contiguous()
        if x2d.shape[0] < DECODE_ROWS:
            y = ops.gemv_bf16(x2d, self.gemv_w, self.sw_bf16)
        else:
            y = ops.linear_bf16(x2d, self.packed)
        return y.to(self.dtype)


class Slice(torch.nn.Module):
    """Stands in for one linear of a GpuGemm group (gemma_npu.py:175-193): the first slice called
    computes the whole group, its siblings reuse the result for the same input tensor."""

    def __init__(self, gemm, index, in_features, out_features):
        super().__init__()
        self.gemm, self.index = gemm, index
        self.in_features, self.out_features = in_features, out_features

    def forward(self, x):
        g = self.gemm
        shape = x.shape[:-1]
        if self.index == 0 or g.pending is None or g.pending[0] is not x:
            y = g.matmul(x.reshape(-1, x.shape[-1]))
            parts = torch.split(y, g.sizes, dim=-1) if len(g.sizes) > 1 else (y,)
            g.pending = (x, parts)
        out = g.pending[1][self.index]
        if self.index == len(g.sizes) - 1:
            g.pending = None
        return out.reshape(*shape, -1)


class Int8Head(torch.nn.Module):
    """The LM head as a weight-only int8 GEMV (gemma_npu.py:159-172), 16 rows per launch."""

    def __init__(self, linear):
        super().__init__()
        q, sw = ops.quant_rows(linear.weight.detach().float().contiguous())
        self.w = ops.pack_gemv_weight(q)
        self.sw = sw.to(torch.bfloat16)
        self.in_features, self.out_features = linear.in_features, linear.out_features

    def forward(self, x):
        shape = x.shape[:-1]
        x2d = x.reshape(-1, x.shape[-1]).to(torch.bfloat16).contiguous()
        outs = [ops.gemv_bf16(x2d[r:r + DECODE_ROWS], self.w, self.sw) for r in range(0, x2d.shape[0], DECODE_ROWS)]
        y = outs[0] if len(outs) == 1 else torch.cat(outs, 0)
        return y.reshape(*shape, -1)


class GpuRMSNorm(torch.nn.Module):
    """HF Gemma 4's RMSNorm on bf16 GPU rows through the engine's row kernel
    (w8a8_rms_residual_bf16 without a residual): x * (mean(x^2) + eps)^-0.5 * w in fp32, rounded to
    bf16 once, as the module computes it (the reference's decode runs these modules around every
    decoder layer, gemma_npu.py:278-300).  One launch instead of the module's ~6 elementwise and
    reduction launches.  Inputs the kernel does not take (not bf16, rows not a multiple of 8 or
    above 12288 elements) go to the model's own module."""

    def __init__(self, norm):
        super().__init__()
        self.orig = norm
        self.eps = float(norm.eps)
        w = getattr(norm, "weight", None) if getattr(norm, "with_scale", True) else None
        self.weight = w

    def forward(self, x):
        N = x.shape[-1]
        w = self.weight
        if (x.dtype != torch.bfloat16 or x.device.type != "cuda" or N % 8 or N > 12288 or x.numel() == 0
                or (w is not None and (w.dtype != torch.bfloat16 or w.device != x.device))):
            return self.orig(x)
        x2 = x.reshape(-1, N)
        if not x2.is_contiguous() or x2.data_ptr() % 16:
            x2 = x2.clone(memory_format=torch.contiguous_format)
        return ops.rms_residual(x2, None, w, self.eps).reshape(x.shape)


class GpuMLP(torch.nn.Module):
    """Gemma 4's MLP, down(gelu_tanh(gate(x)) * up(x)), with the activation and product fused into
    the gate/up GEMM's epilogue for prefill rows: the epilogue computes bf16(bf16(gelu_tanh(gate)) * up)
    on the bf16 gate and up the unfused GEMM would have written (k_gelu's arithmetic, pipeline.py:
    102-107), so the [T, 2I] gate/up result never goes to HBM.  Decode rows (< 16) and activations
    other than GELU-tanh keep the module's own steps."""

    def __init__(self, mlp, gate_up, down):
        super().__init__()
        self.orig = mlp
        self.gate_up, self.down = gate_up, down
        self.fused = (getattr(mlp.config, "hidden_activation", None) == "gelu_pytorch_tanh"
                      and gate_up.packed_gelu is not None)

    def forward(self, x):
        x2 = x.reshape(-1, x.shape[-1])
        if not self.fused or x2.shape[0] < DECODE_ROWS:
            return self.orig(x)
        a = ops.linear_bf16(x2.to(torch.bfloat16).contiguous(), self.gate_up.packed_gelu, epilogue="gelu")
        return self.down.matmul(a).reshape(*x.shape[:-1], -1)


def language_model(model):
    """The text decoder of a Gemma 4 causal LM (multimodal or text-only)."""
    m = model.model
    return m.language_model if hasattr(m, "language_model") else m


def register_attention():
    """Registers attention.local_sdpa as HF's "local_sdpa" (local_attn.py:110-111)."""
    from transformers import AttentionInterface
    from transformers.masking_utils import ALL_MASK_ATTENTION_FUNCTIONS, sdpa_mask
    AttentionInterface.register("local_sdpa", attention.local_sdpa)
    ALL_MASK_ATTENTION_FUNCTIONS.register("local_sdpa", sdpa_mask)


def to_gpu(model):
    """Swap the text decoder's linears for GPU W8A8 groups, the LM head for the int8 GEMV head, and
    the attention for local_sdpa (gemma_npu.py:208-241, 253).  Returns the groups; model.layer_gemms
    holds each layer's groups by name ("qkv", "o", "gate_up", "down", "ple_gate", "ple_proj") for
    w8a8.pipeline.Prefill."""
    lm = language_model(model)
    groups = []
    per_layer = []  # (layer index, group key) of each group, as the reference's layer_gemms keys
    for li, layer in enumerate(lm.layers):
        a, mlp = layer.self_attn, layer.mlp
        qkv = [a.q_proj]
        if not a.is_kv_shared_layer:
            qkv += [a.k_proj] + ([a.v_proj] if a.v_proj is not None else [])
        groups += [(a, ["q_proj", "k_proj", "v_proj"][: len(qkv)], qkv),
                   (a, ["o_proj"], [a.o_proj]),
                   (mlp, ["gate_proj", "up_proj"], [mlp.gate_proj, mlp.up_proj]),
                   (mlp, ["down_proj"], [mlp.down_proj])]
        per_layer += [(li, "qkv"), (li, "o"), (li, "gate_up"), (li, "down")]
        if getattr(layer, "per_layer_input_gate", None) is not None:
            groups += [(layer, ["per_layer_input_gate"], [layer.per_layer_input_gate]),
                       (layer, ["per_layer_projection"], [layer.per_layer_projection])]
            per_layer += [(li, "ple_gate"), (li, "ple_proj")]
    if getattr(lm, "per_layer_model_projection", None) is not None:
        groups.append((lm, ["per_layer_model_projection"], [lm.per_layer_model_projection]))
    gemms = []
    for parent, names, linears in groups:
        g = GpuGemm(linears, gelu_pair=names == ["gate_proj", "up_proj"])
        g.name = "+".join(names)
        gemms.append(g)
        for i, (name, l) in enumerate(zip(names, linears)):
            setattr(parent, name, Slice(g, i, l.in_features, l.out_features))
    # the per-layer groups by name, for the whole-prompt pipeline (gemma_npu.py:238-239)
    model.layer_gemms = [{} for _ in lm.layers]
    for (li, key), g in zip(per_layer, gemms):
        model.layer_gemms[li][key] = g
    # the MLPs with the GELU-tanh * up step in the gate/up GEMM's epilogue for prefill rows
    for li, layer in enumerate(lm.layers):
        G = model.layer_gemms[li]
        if "gate_up" in G and "down" in G:
            layer.mlp = GpuMLP(layer.mlp, G["gate_up"], G["down"])
    # every RMSNorm of the text decoder on the row kernel
    for parent in list(lm.modules()):
        for name, child in list(parent.named_children()):
            if type(child).__name__ == "Gemma4RMSNorm":
                setattr(parent, name, GpuRMSNorm(child))
    # tied to the input embedding, so this is a new int8 copy, not a swap
    model.lm_head = Int8Head(model.lm_head)
    register_attention()
    lm.set_attn_implementation("local_sdpa")
    return gemms
