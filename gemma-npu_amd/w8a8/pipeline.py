"""The reference's prefill pipeline (pipeline.py:224-339) with every step on the GPU.

    gemms = hf.to_gpu(model)                 # groups + model.layer_gemms (gemma_npu.py:208-241)
    prefill = Prefill(model)                 # pipeline.py:224-231
    logits, cache = prefill(ids)             # pipeline.py:312-339: fp32 last-token logits, DynamicCache
    out = model(input_ids=nxt, past_key_values=cache, use_cache=True)   # HF's decode loop continues

A decoder layer is the reference's step sequence (pipeline.py:244-310): k_in -> qkv GEMM -> k_qkv
-> attention -> k_attn_out -> o GEMM -> k_post_attn -> gate/up GEMM -> k_gelu -> down GEMM ->
k_post_ff -> PLE gate GEMM -> k_ple_gate -> PLE projection GEMM -> k_ple_out.  The GEMMs are the
engine's int32 W8A8 GEMMs on the packed per-channel int8 weights of hf.to_gpu, the steps between
them the fused kernels of w8a8.fused, attention the kernels of w8a8.attention; all of it is issued
on torch's current stream, and activations stay on the device from the embedding to the logits.

The reference cuts the prompt into 512-row micro-batches so that its CPU and NPU work overlap
(pipeline.py:322-330, 341-392).  One GPU gains nothing from that overlap, so by default every
layer runs over the whole prompt at once (row_step=None), which hands the GEMMs their long-M
shapes and attention one call per layer.  row_step=512 runs the reference's micro-batches
instead, each through every layer in prompt order, attending to the keys of the micro-batches
before it (pipeline.py:266-276).  Every step but attention is row-wise, so the two orders differ
only by attention's summation order.

k_gelu's arithmetic -- dequant, bf16(bf16(gelu_tanh(gate)) * up), per-token quant -- also exists as
the GEMM's fused GELU epilogue followed by the quant kernel, which never writes the int32 [T, 2I]
result; with fuse_gelu (the default) the gate/up step takes that form, on the interleaved copy of
the gate/up weight that hf.to_gpu packs for it.  Both forms give the same int8 rows and scales.

The embedding, the per-layer-input (PLE) tables, RoPE tables, the final norm and the logit
softcap are the model's own modules, as in the reference (pipeline.py:318-338); the PLE model
projection inside them and the LM head are the engine's GEMM and GEMV after hf.to_gpu.
"""
import torch

from . import attention, fused, ops
from .hf import language_model


class Prefill:
    """pipeline.py:224-339 on the GPU: Prefill(model)(ids) -> (logits [vocab] fp32, DynamicCache)."""

    def __init__(self, model, layer_gemms=None, row_step=None, fuse_gelu=True):
        self.model = model
        self.lm = language_model(model)
        self.cfg = self.lm.config
        self.layer_gemms = layer_gemms if layer_gemms is not None else getattr(model, "layer_gemms", None)
        if self.layer_gemms is None:
            raise ValueError("Prefill: run w8a8.hf.to_gpu(model) first (it builds model.layer_gemms)")
        if row_step is not None and int(row_step) < 1:
            raise ValueError(f"Prefill: row_step {row_step} must be positive")
        self.row_step = None if row_step is None else int(row_step)
        self.fuse_gelu = bool(fuse_gelu)
        if getattr(self.cfg, "enable_moe_block", False):
            raise NotImplementedError("Prefill: MoE decoder layers are not on the reference's path")
        if not self.cfg.hidden_size_per_layer_input:
            raise NotImplementedError("Prefill: the reference's pipeline needs per-layer inputs (PLE)")
        for i, layer in enumerate(self.lm.layers):
            a = layer.self_attn
            if not a.is_kv_shared_layer and a.v_proj is None:
                raise NotImplementedError(f"Prefill: layer {i} derives v from k (attention_k_eq_v); the "
                                          "reference's k_qkv expects a v projection")
            if set(self.layer_gemms[i]) != {"qkv", "o", "gate_up", "down", "ple_gate", "ple_proj"}:
                raise ValueError(f"Prefill: layer {i} lacks GEMM groups, got {sorted(self.layer_gemms[i])}")

    @staticmethod
    def gemm(g, xq):
        """The int32 GEMM result [T, N] of group g on int8 rows xq (pipeline.py:233-242)."""
        return ops.gemm_i32(xq, g.packed)

    def steps(self, mb, ctx):
        """One micro-batch (s, e, slot) through every layer (pipeline.py:244-310); returns its rows."""
        lm, cfg = self.lm, self.cfg
        s, e, slot = mb
        eps = cfg.rms_norm_eps
        h = ctx["h0"][s:e]
        kv = ctx["kv"]
        for i, layer in enumerate(lm.layers):
            G = self.layer_gemms[i]
            a = layer.self_attn
            lt = cfg.layer_types[i]
            cos, sin = ctx["rope"][lt]
            cos, sin = cos[s:e], sin[s:e]
            H, D = cfg.num_attention_heads, a.head_dim
            KV = cfg.per_layer_config[i].num_key_value_heads
            shared = a.is_kv_shared_layer

            xq, sx = fused.k_in(h, layer.input_layernorm.weight, eps, packed=True)
            acc = self.gemm(G["qkv"], xq)
            q, k, v = fused.k_qkv(acc, sx, G["qkv"].sw, cos, sin, a.q_norm.weight,
                                  None if shared else a.k_norm.weight, eps, H, KV, D, shared)
            if shared:
                k_all, v_all = kv[("shared", lt, slot)]
            else:
                # every earlier micro-batch has run all its layers, so its keys are here
                kv[(i, slot)] = (k, v)
                if slot == 0:
                    k_all, v_all = k, v
                else:
                    prev = [kv[(i, j)] for j in range(slot + 1)]
                    k_all = torch.cat([p[0] for p in prev], 1)
                    v_all = torch.cat([p[1] for p in prev], 1)
                if slot == ctx["last"]:
                    ctx["cache"].update(k_all[None], v_all[None], i)
                if a.store_full_length_kv:
                    kv[("shared", lt, slot)] = (k_all, v_all)
            if a.sliding_window:
                o = attention.sliding_attention(q, k_all, v_all, s, a.sliding_window)
            else:
                o = attention.full_attention(q, k_all, v_all, s)

            xq, sx = fused.k_attn_out(o, packed=True)
            acc = self.gemm(G["o"], xq)
            h, xq, sx = fused.k_post_attn(acc, sx, G["o"].sw, h, layer.post_attention_layernorm.weight,
                                          layer.pre_feedforward_layernorm.weight, eps, packed=True)
            gu = G["gate_up"]
            if self.fuse_gelu and getattr(gu, "packed_gelu", None) is not None:
                # the GEMM's GELU epilogue writes k_gelu's bf16 bf16(gelu(gate)) * up, then its quant
                a_ = ops.gemm_bf16(xq, sx, gu.packed_gelu, epilogue="gelu")
                xq, sx = ops.quant_rows_packed(a_)
            else:
                acc = self.gemm(gu, xq)
                xq, sx = fused.k_gelu(acc, sx, gu.sw, gu.N // 2, packed=True)
            acc = self.gemm(G["down"], xq)
            h, xq, sx = fused.k_post_ff(acc, sx, G["down"].sw, h, layer.post_feedforward_layernorm.weight, eps,
                                        packed=True)
            acc = self.gemm(G["ple_gate"], xq)
            xq, sx = fused.k_ple_gate(acc, sx, G["ple_gate"].sw, ctx["ple"][s:e, i], packed=True)
            acc = self.gemm(G["ple_proj"], xq)
            h = fused.k_ple_out(acc, sx, G["ple_proj"].sw, h, layer.post_per_layer_input_norm.weight,
                                ctx["scalar"][i], eps)
        return h

    @torch.inference_mode()
    def __call__(self, ids, all_hidden=False):
        """ids [1, T] -> (last-token logits [vocab] fp32, DynamicCache) (pipeline.py:312-339).

        With all_hidden, the final-norm hidden states [T, hidden] instead of the logits."""
        from transformers import DynamicCache
        lm, cfg = self.lm, self.cfg
        if ids.dim() != 2 or ids.shape[0] != 1 or ids.shape[1] < 1:
            raise ValueError(f"Prefill: expected ids [1, T], got {tuple(ids.shape)}")
        dev = lm.embed_tokens.weight.device
        ids = ids.to(dev)
        T = ids.shape[1]
        emb = lm.embed_tokens(ids)
        ple = lm.project_per_layer_inputs(emb, lm.get_per_layer_inputs(ids, emb))[0]
        pos = torch.arange(T, device=dev)[None]
        rope = {lt: tuple(t[0] for t in lm.rotary_emb(emb, pos, lt)) for lt in set(cfg.layer_types)}
        cache = DynamicCache(config=cfg)
        step = self.row_step or T
        mbs = [(s, min(s + step, T), j) for j, s in enumerate(range(0, T, step))]
        scalar = [layer.layer_scalar.to(torch.bfloat16) for layer in lm.layers]
        ctx = dict(h0=emb[0], ple=ple, rope=rope, kv={}, cache=cache, last=len(mbs) - 1, scalar=scalar)
        out = [self.steps(mb, ctx) for mb in mbs]
        if all_hidden:
            return lm.norm(torch.cat(out)[None])[0], cache
        h = lm.norm(out[-1][-1:][None])
        logits = self.model.lm_head(h)[0, -1].float()
        cap = cfg.final_logit_softcapping
        if cap:
            logits = torch.tanh(logits / cap) * cap
        return logits, cache
