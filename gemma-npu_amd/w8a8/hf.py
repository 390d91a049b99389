"""HF transformers' Gemma 4 text decoder on the GPU with this engine underneath.

What the reference does to the model on its NPU path -- its linears become grouped W8A8 GEMMs
(gemma_npu.py:57-152, 175-241), the LM head an int8 GEMV (gemma_npu.py:159-172), attention the
registered "local_sdpa" (gemma_npu.py:253, local_attn.py:110-111) -- `to_gpu` does on a model whose
weights are on the GPU:

    model = AutoModelForCausalLM.from_pretrained(...).to("cuda")      # or a random-init config
    hf.to_gpu(model)
    out = model(input_ids=ids, use_cache=True, logits_to_keep=1)      # prefill: W8A8 GEMMs
    out = model(input_ids=nxt, past_key_values=out.past_key_values)   # decode: int8 GEMVs

Linears that read the same input share one quantized weight ([q; k; v] -- q alone on KV-shared
layers --, [gate; up]), as the reference groups them (gemma_npu.py:213-224); o, down, the per-layer
input gate and projection and the per-layer model projection are groups of one.  Each original
linear is replaced by a QuantizedLinear, a view of its group's output columns.  The group's
output is computed once per input:
  * attention: a forward pre-hook on the attention module runs the [q; k; v] GEMM on the module's
    hidden states and parks each projection's columns on it; the projections return them, and a
    forward hook drops them when the module returns;
  * MLP: GpuMLP runs the [gate; up] weight in one launch itself -- for prefill rows with
    gelu_tanh(gate) * up in the GEMM's epilogue (k_gelu's arithmetic, pipeline.py:102-107), for
    decode rows as one GEMV followed by the module's own activation.
Rows < 16 (decode) take the weight-only int8 GEMV with bf16 scales (gemma_npu.py:120-121), more
rows per-token quant -> int8 GEMM -> dequant (gemma_npu.py:123-152).  Every RMSNorm module becomes
one launch of the engine's row kernel (GpuRMSNorm).  RoPE, residuals, the KV cache and the decode
loop stay HF's own torch ops on the GPU.  Under torch.compile (the reference compiles each layer's
forward, gemma_npu.py:255-265) these modules call the engine through its registered torch operators
(w8a8.torch_ops), which the compiler traces instead of breaking the graph.
"""
import torch

from . import attention, ops, torch_ops

DECODE_ROWS = 16  # rows below this go to the GEMV (gemma_npu.py:120)


class QuantizedWeight:
    """The weights of linears that read one input, stacked along N into [sum N_i, K] and quantized
    per output channel once (absmax / 127, gemma_npu.py:68-69).

    Kept in the forms its callers read: `packed` (the GEMM's fragment layout, fp32 scales `sw`) for
    prefill rows, `gemv_w` / `sw_bf16` (the GEMV's layout and bf16 scales, the reference's decode copy,
    gemma_npu.py:81-82) for decode rows, and for a [gate; up] pair `packed_gelu`, packed for the GEMM's
    fused GELU epilogue.  With gemm=False only the GEMV form exists (the LM head) and every row goes
    through it, 16 rows per launch.  The plain GEMM packing of a [gate; up] pair is made on first
    use, by permuting the tiles of `packed_gelu`: the fused path does not need it, and no int8
    copy is kept for it."""

    def __init__(self, weights, gemm=True, gelu_pair=False):
        w = torch.cat([t.detach() for t in weights], 0)
        if w.device.type != "cuda":
            raise ValueError("to_gpu: move the model to the GPU first")
        self.N, self.K = w.shape
        self.sizes = [t.shape[0] for t in weights]
        self.dtype = w.dtype
        q, sw = ops.quant_rows(w.float().contiguous())
        del w
        self.sw, self.sw_bf16 = sw, sw.to(torch.bfloat16)
        self.gemv_w = ops.pack_gemv_weight(q)
        self.has_gemm = bool(gemm)
        self._packed = ops.pack_weight(q, "nk", sw=sw) if (gemm and not gelu_pair) else None
        self.packed_gelu = ops.pack_weight(q, "nk", self.N // 2, sw=sw) if (gemm and gelu_pair) else None
        self.name = ""

    @property
    def packed(self):
        if self._packed is None:
            if not self.has_gemm:
                raise AttributeError("this weight is kept for the GEMV only")
            self._packed = ops.unpair_packed(self.packed_gelu)
        return self._packed

    def apply(self, x2d):
        """y [rows, N] in the model's dtype for rows x2d [rows, K]."""
        x2d = x2d.to(torch.bfloat16).contiguous()
        rows = x2d.shape[0]
        if rows < DECODE_ROWS:
            y = torch_ops.gemv(x2d, self.gemv_w, self.sw_bf16)
        elif self.has_gemm:
            y = torch_ops.linear(x2d, self.packed)
        else:
            y = torch.empty((rows, self.N), dtype=torch.bfloat16, device=x2d.device)
            for r in range(0, rows, DECODE_ROWS):
                torch_ops.gemv(x2d[r:r + DECODE_ROWS], self.gemv_w, self.sw_bf16, y[r:r + DECODE_ROWS])
        return y.to(self.dtype)


class QuantizedLinear(torch.nn.Module):
    """One original linear: output columns [c0, c1) of a QuantizedWeight.  Returns the columns
    parked on it for this very input if there are any (a group computed once for its members),
    otherwise runs the group and keeps its own columns."""

    def __init__(self, weight, c0=0, c1=None):
        super().__init__()
        self.weight_q = weight
        self.c0, self.c1 = c0, weight.N if c1 is None else c1
        self.in_features, self.out_features = weight.K, self.c1 - self.c0
        self.parked = None  # (input tensor, its output columns)

    def forward(self, x):
        p = self.parked
        if p is not None and p[0] is x:
            return p[1]
        y = self.weight_q.apply(x.reshape(-1, x.shape[-1]))
        if self.c0 != 0 or self.c1 != self.weight_q.N:
            y = y[:, self.c0:self.c1]
        return y.reshape(*x.shape[:-1], self.out_features)


def _column_views(weight, names):
    """QuantizedLinear views of a group's members, in stacking order, by name."""
    views, c = {}, 0
    for name, n in zip(names, weight.sizes):
        views[name] = QuantizedLinear(weight, c, c + n)
        c += n
    return views


def share_input(module, weight, views):
    """Run `weight` once per forward of `module` on its hidden states and park each view's columns
    on it for the duration of that forward (the views are the module's projections of that input)."""
    sizes = [v.out_features for v in views]

    def before(mod, args, kwargs):
        hs = kwargs.get("hidden_states", args[0] if args else None)
        if hs is None or hs.shape[-1] != weight.K:
            return None
        y = weight.apply(hs.reshape(-1, weight.K))
        for v, part in zip(views, torch.split(y, sizes, dim=-1)):
            v.parked = (hs, part.reshape(*hs.shape[:-1], v.out_features))
        return None

    def after(mod, args, kwargs, output):
        for v in views:
            v.parked = None
        return None

    module.register_forward_pre_hook(before, with_kwargs=True)
    module.register_forward_hook(after, with_kwargs=True)


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
        if torch_ops.tracing():
            return torch_ops.rms_norm(x2, w, self.eps).reshape(x.shape)
        if not x2.is_contiguous() or x2.data_ptr() % 16:
            x2 = x2.clone(memory_format=torch.contiguous_format)
        return torch_ops.rms_norm(x2, w, self.eps).reshape(x.shape)


class GpuMLP(torch.nn.Module):
    """Gemma 4's MLP, down(act(gate(x)) * up(x)), with gate and up from one launch of their stacked
    weight.  Prefill rows with the GELU-tanh activation take the GEMM's GELU epilogue, which computes
    bf16(bf16(gelu_tanh(gate)) * up) on the bf16 gate and up the plain GEMM would have written (k_gelu's
    arithmetic, pipeline.py:102-107), so the [T, 2I] result never goes to HBM.  Decode rows take one
    GEMV for [gate; up] and the module's own activation and product on its columns."""

    def __init__(self, mlp, gate_up, down):
        super().__init__()
        self.orig = mlp
        self.gate_up, self.down = gate_up, down
        self.act = mlp.act_fn
        self.fused = (getattr(mlp.config, "hidden_activation", None) == "gelu_pytorch_tanh"
                      and gate_up.packed_gelu is not None)

    def forward(self, x):
        x2 = x.reshape(-1, x.shape[-1])
        I = self.gate_up.N // 2
        if self.fused and x2.shape[0] >= DECODE_ROWS:
            a = torch_ops.linear(x2.to(torch.bfloat16).contiguous(), self.gate_up.packed_gelu, epilogue="gelu")
            a = a.to(self.gate_up.dtype)
        else:
            y = self.gate_up.apply(x2)
            a = self.act(y[:, :I]) * y[:, I:]
        return self.down.apply(a).reshape(*x.shape[:-1], -1)


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


def _single(module, name):
    """Replace module.<name> (a linear) by a QuantizedLinear over its own quantized weight."""
    w = QuantizedWeight([getattr(module, name).weight])
    w.name = name
    setattr(module, name, QuantizedLinear(w))
    return w


def _convert_layer(layer):
    """One decoder layer's linears and MLP on the engine; returns its weights by pipeline role."""
    attn, mlp = layer.self_attn, layer.mlp
    names = ["q_proj"]
    if not attn.is_kv_shared_layer:
        names += [n for n in ("k_proj", "v_proj") if getattr(attn, n, None) is not None]
    qkv = QuantizedWeight([getattr(attn, n).weight for n in names])
    qkv.name = "+".join(names)
    views = _column_views(qkv, names)
    for n, v in views.items():
        setattr(attn, n, v)
    share_input(attn, qkv, [views[n] for n in names])
    roles = {"qkv": qkv, "o": _single(attn, "o_proj")}

    gate_up = QuantizedWeight([mlp.gate_proj.weight, mlp.up_proj.weight], gelu_pair=True)
    gate_up.name = "gate_proj+up_proj"
    for n, v in _column_views(gate_up, ["gate_proj", "up_proj"]).items():
        setattr(mlp, n, v)
    down = _single(mlp, "down_proj")
    layer.mlp = GpuMLP(mlp, gate_up, down)
    roles.update(gate_up=gate_up, down=down)
    if getattr(layer, "per_layer_input_gate", None) is not None:
        roles["ple_gate"] = _single(layer, "per_layer_input_gate")
        roles["ple_proj"] = _single(layer, "per_layer_projection")
    return roles


def to_gpu(model):
    """Put the text decoder's linears, MLPs, RMSNorms and LM head on the engine and its attention on
    local_sdpa (what gemma_npu.py:208-241, 253 does for the NPU).  Returns every quantized weight;
    model.layer_gemms holds each layer's by pipeline role ("qkv", "o", "gate_up", "down", "ple_gate",
    "ple_proj") for w8a8.pipeline.Prefill."""
    lm = language_model(model)
    model.layer_gemms = [_convert_layer(layer) for layer in lm.layers]
    weights = [w for roles in model.layer_gemms for w in roles.values()]
    if getattr(lm, "per_layer_model_projection", None) is not None:
        weights.append(_single(lm, "per_layer_model_projection"))
    for parent in list(lm.modules()):
        for name, child in list(parent.named_children()):
            if type(child).__name__ == "Gemma4RMSNorm":
                setattr(parent, name, GpuRMSNorm(child))
    # the LM head is tied to the input embedding: this is a new int8 copy, kept for the GEMV only
    head = QuantizedWeight([model.lm_head.weight], gemm=False)
    head.name = "lm_head"
    model.lm_head = QuantizedLinear(head)
    weights.append(head)
    register_attention()
    lm.set_attn_implementation("local_sdpa")
    return weights
