"""The reference's prefill pipeline (pipeline.py:224-339) with every step on the GPU.

    gemms = hf.to_gpu(model)                 # groups + model.layer_gemms (gemma_npu.py:208-241)
    prefill = Prefill(model)                 # pipeline.py:224-231
    logits, cache = prefill(ids)             # pipeline.py:312-339: fp32 last-token logits, DynamicCache
    out = model(input_ids=nxt, past_key_values=cache, use_cache=True)   # HF's decode loop continues
    run = prefill.capture(T)                 # the same, captured in one HIP graph for T-token prompts
    logits, cache = run(ids)

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
                    ctx["layer_kv"].append((i, k_all, v_all))
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

    def _check_ids(self, ids):
        if ids.dim() != 2 or ids.shape[0] != 1 or ids.shape[1] < 1:
            raise ValueError(f"Prefill: expected ids [1, T], got {tuple(ids.shape)}")
        return ids.to(self.lm.embed_tokens.weight.device)

    def _inputs(self, ids):
        """The model's own embedding, per-layer inputs (PLE) and RoPE tables for ids [1, T]
        (pipeline.py:318-321): (h0 [T, hidden], ple [T, layers, P], {layer type: (cos, sin)})."""
        lm, cfg = self.lm, self.cfg
        T = ids.shape[1]
        emb = lm.embed_tokens(ids)
        ple = lm.project_per_layer_inputs(emb, lm.get_per_layer_inputs(ids, emb))[0]
        pos = torch.arange(T, device=ids.device)[None]
        rope = {lt: tuple(t[0] for t in lm.rotary_emb(emb, pos, lt)) for lt in set(cfg.layer_types)}
        return emb[0], ple, rope

    def _layers(self, h0, ple, rope, scalar):
        """Every layer over the prompt, in micro-batches of row_step rows (all at once by default):
        (the final rows [T, hidden] before the last norm, [(layer, k, v)] of the non-shared layers)."""
        T = h0.shape[0]
        step = self.row_step or T
        mbs = [(s, min(s + step, T), j) for j, s in enumerate(range(0, T, step))]
        ctx = dict(h0=h0, ple=ple, rope=rope, kv={}, layer_kv=[], last=len(mbs) - 1, scalar=scalar)
        out = [self.steps(mb, ctx) for mb in mbs]
        return (out[0] if len(out) == 1 else torch.cat(out)), ctx["layer_kv"]

    def _scalars(self):
        return [layer.layer_scalar.to(torch.bfloat16) for layer in self.lm.layers]

    def _head(self, h_last):
        """Final norm, LM head and logit softcap of the last row (pipeline.py:334-338)."""
        h = self.lm.norm(h_last[None])
        logits = self.model.lm_head(h)[0, -1].float()
        cap = self.cfg.final_logit_softcapping
        if cap:
            logits = torch.tanh(logits / cap) * cap
        return logits

    def _cache(self, layer_kv, copy):
        """A DynamicCache holding each non-shared layer's keys and values (pipeline.py:273-274)."""
        from transformers import DynamicCache
        cache = DynamicCache(config=self.cfg)
        for i, k, v in layer_kv:
            cache.update((k.clone() if copy else k)[None], (v.clone() if copy else v)[None], i)
        return cache

    @torch.inference_mode()
    def __call__(self, ids, all_hidden=False):
        """ids [1, T] -> (last-token logits [vocab] fp32, DynamicCache) (pipeline.py:312-339).

        With all_hidden, the final-norm hidden states [T, hidden] instead of the logits."""
        h0, ple, rope = self._inputs(self._check_ids(ids))
        rows, layer_kv = self._layers(h0, ple, rope, self._scalars())
        if all_hidden:
            return self.lm.norm(rows[None])[0], self._cache(layer_kv, copy=False)
        return self._head(rows[-1:]), self._cache(layer_kv, copy=False)

    @torch.inference_mode()
    def capture(self, T):
        """This prefill for prompts of T tokens, captured once in a HIP graph: returns a callable
        ids [1, T] -> (logits, DynamicCache) that replays it.  The launches of a whole prefill
        (~600 for E2B) then cost one graph launch on the host."""
        return CapturedPrefill(self, int(T))


class CapturedPrefill:
    """Prefill.capture(T): the layers of one prompt length's prefill as a HIP graph.

    The graph holds every layer's launches (GEMMs, fused kernels, attention) over static input
    buffers.  A call runs the model's own embedding and per-layer-input modules eagerly, copies
    their results into those buffers, replays the graph, and runs the final norm, LM head and
    softcap of the last row eagerly; the RoPE tables depend on T only and are computed once.  The
    returned logits and cache hold their own copies, so a later replay does not change them.  An
    eager run on the capture stream before the capture creates every cached workspace outside the
    graph, so the graph allocates and clears nothing itself."""

    def __init__(self, prefill, T):
        if T < 1:
            raise ValueError(f"Prefill.capture: T={T} must be positive")
        self.prefill, self.T = prefill, T
        dev = prefill.lm.embed_tokens.weight.device
        ids = torch.zeros((1, T), dtype=torch.long, device=dev)
        h0, ple, rope = prefill._inputs(ids)
        self.h0, self.ple, self.rope = h0.clone(), ple.clone(), rope
        self.scalar = prefill._scalars()
        self.stream = torch.cuda.Stream(dev)
        self.stream.wait_stream(torch.cuda.current_stream(dev))
        with torch.cuda.stream(self.stream):
            prefill._layers(self.h0, self.ple, self.rope, self.scalar)
        torch.cuda.current_stream(dev).wait_stream(self.stream)
        torch.cuda.synchronize(dev)
        self.graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(self.graph, stream=self.stream):
            self.rows, self.layer_kv = prefill._layers(self.h0, self.ple, self.rope, self.scalar)
        torch.cuda.synchronize(dev)

    @torch.inference_mode()
    def __call__(self, ids):
        p = self.prefill
        ids = p._check_ids(ids)
        if ids.shape[1] != self.T:
            raise ValueError(f"CapturedPrefill: captured for {self.T} tokens, got {ids.shape[1]}")
        h0, ple, _ = p._inputs(ids)
        self.h0.copy_(h0)
        self.ple.copy_(ple)
        self.graph.replay()
        return p._head(self.rows[-1:]), p._cache(self.layer_kv, copy=True)
