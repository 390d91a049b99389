"""The reference's prefill pipeline (pipeline.py:224-339) with every step on the GPU.

    gemms = hf.to_gpu(model)                 # weights + model.layer_gemms (gemma_npu.py:208-241)
    prefill = Prefill(model)
    logits, cache = prefill(ids)             # fp32 last-token logits, DynamicCache (pipeline.py:312-339)
    out = model(input_ids=nxt, past_key_values=cache, use_cache=True)   # HF's decode loop continues
    run = prefill.capture(T)                 # the same, captured in one HIP graph for T-token prompts
    logits, cache = run(ids)

Per decoder layer the arithmetic is the reference's (pipeline.py:244-310): input norm + quant (k_in),
the [q; k; v] GEMM, q/k norm + RoPE (k_qkv), attention, quant of its output (k_attn_out), the o GEMM,
residual + norms + quant (k_post_attn), the gate/up GEMM with GELU-tanh * up and quant (k_gelu),
the down GEMM, residual + norm + quant (k_post_ff), the per-layer-input gate GEMM (k_ple_gate) and
projection GEMM (k_ple_out).  GEMMs are the engine's int32 W8A8 GEMMs on hf.to_gpu's packed weights,
the steps between them w8a8.fused's kernels, attention w8a8.attention's; everything is issued on
torch's current stream and activations stay on the device from the embedding to the logits.

How it is organised here:
  * each layer's weights, norm weights, attention geometry and key/value source are resolved once,
    at construction, into a LayerPlan;
  * keys and values live in a KVStore: one [KV heads, T, head_dim] tensor pair per layer that owns
    keys; a layer that shares keys (KV-shared layers, which read the last earlier layer of their
    attention kind that stores full-length keys) reads its source's pair; rows are written where
    they belong and attention reads the prefix it may see;
  * the prompt runs as one row range through all layers by default (row_step=None): one GPU has no
    CPU work to overlap, and the whole prompt gives the GEMMs their long-M shapes and attention one
    call per layer.  row_step=512 runs the reference's 512-row micro-batch order instead (pipeline.py:
    322-330), each range through every layer in prompt order against the keys of the ranges before
    it.  Every step but attention is row-wise, so the orders differ only by attention's summation
    order.

The gate/up step takes the GEMM's fused GELU epilogue followed by the quant kernel by default
(fuse_gelu): the same int8 rows and scales as k_gelu on the int32 result, without writing the
[T, 2I] int32 result.  Past 1024 rows the other GEMMs write their dequantised bf16 result
(dequant_in_gemm), which the fused kernels after them read in place of the int32 result and its
scales: their first step is that dequant, so every value is the same and the hand-over moves half
the bytes.  The embedding, per-layer-input tables, RoPE tables, final norm and logit
softcap are the model's own modules (pipeline.py:318-338); inside them the per-layer model
projection and the LM head run on the engine after hf.to_gpu.
"""
import time

import torch

from . import attention, fused, ops
from ._lib import lib
from .hf import language_model

ROLES = ("qkv", "o", "gate_up", "down", "ple_gate", "ple_proj")


class LayerPlan:
    """One decoder layer's prefill, resolved once: weights by role, norm weights, attention geometry
    and the layer whose keys and values it attends to (itself unless it shares them)."""

    def __init__(self, index, layer, cfg, weights, kv_source):
        a = layer.self_attn
        self.index = index
        self.weights = weights
        self.kind = cfg.layer_types[index]
        self.window = int(a.sliding_window or 0)
        self.heads = cfg.num_attention_heads
        self.kv_heads = cfg.per_layer_config[index].num_key_value_heads
        self.head_dim = a.head_dim
        self.shares_kv = bool(a.is_kv_shared_layer)
        self.kv_source = kv_source
        self.norm_in = layer.input_layernorm.weight
        self.norm_q = a.q_norm.weight
        self.norm_k = None if self.shares_kv else a.k_norm.weight
        self.norm_post_attn = layer.post_attention_layernorm.weight
        self.norm_pre_ff = layer.pre_feedforward_layernorm.weight
        self.norm_post_ff = layer.post_feedforward_layernorm.weight
        self.norm_post_ple = layer.post_per_layer_input_norm.weight


class KVStore:
    """Keys and values of the prompt, per layer that owns them: [KV heads, T, head_dim] each.  A row
    range is written where it belongs; `visible(layer, end)` is the prefix rows [0, end)."""

    def __init__(self, T):
        self.T = T
        self.kv = {}

    def write(self, layer, start, k, v):
        n = k.shape[1]
        if start == 0 and n == self.T:  # the whole prompt at once: keep the tensors themselves
            self.kv[layer] = (k, v)
            return
        if layer not in self.kv:
            self.kv[layer] = (k.new_empty((k.shape[0], self.T, k.shape[2])),
                              v.new_empty((v.shape[0], self.T, v.shape[2])))
        kb, vb = self.kv[layer]
        kb[:, start:start + n].copy_(k)
        vb[:, start:start + n].copy_(v)

    def visible(self, layer, end):
        kb, vb = self.kv[layer]
        return kb[:, :end], vb[:, :end]

    def to_cache(self, cfg, copy):
        """A DynamicCache with every owning layer's keys and values (what HF's decode loop reads).

        Each layer is left in the state its first `update` would leave (transformers cache_utils:
        DynamicLayer.update keeps the keys and values, DynamicSlidingWindowLayer.update counts the T
        tokens and keeps the last sliding_window - 1 of them) without that update's concatenation
        onto an empty tensor, which copies every layer's keys and values once more.  The layers hold
        the store's own tensors, or copies of what they keep when `copy` is set (buffers that a
        later run overwrites)."""
        from transformers import DynamicCache
        from transformers.cache_utils import DynamicLayer, DynamicSlidingWindowLayer
        cache = DynamicCache(config=cfg)
        for layer in sorted(self.kv):
            k, v = self.kv[layer]
            k, v = k[None], v[None]
            lw = cache.layers[layer]
            if type(lw) not in (DynamicLayer, DynamicSlidingWindowLayer) or lw.is_initialized:
                cache.update(k.clone() if copy else k, v.clone() if copy else v, layer)
                continue
            lw.lazy_initialization(k, v)
            if lw.is_sliding:
                lw.cumulative_length += k.shape[-2]
                if not lw.record_past:
                    k, v = k[:, :, -lw.sliding_window + 1:], v[:, :, -lw.sliding_window + 1:]
            lw.keys, lw.values = (k.clone(), v.clone()) if copy else (k, v)
        return cache


def prompt_inputs(lm, ids, rope_cache=None):
    """The model's own inputs to its decoder layers for ids [1, T]: the token embeddings [T, hidden],
    the per-layer inputs [T, layers, P] and the RoPE (cos, sin) rows [T, head_dim] per attention kind.
    The RoPE rows depend on the prompt length alone (positions 0 .. T-1): with rope_cache (a dict) the
    rows of the last few lengths are kept there and reused instead of recomputed."""
    emb = lm.embed_tokens(ids)
    per_layer = lm.project_per_layer_inputs(emb, lm.get_per_layer_inputs(ids, emb))[0]
    # a dynamic RoPE (its frequencies follow the longest sequence seen) is recomputed every time
    kinds = getattr(lm.rotary_emb, "rope_type", {})
    if any("dynamic" in str(t) for t in (kinds.values() if isinstance(kinds, dict) else [kinds])):
        rope_cache = None
    key = (ids.shape[1], ids.device, emb.dtype)
    rope = rope_cache.get(key) if rope_cache is not None else None
    if rope is None:
        positions = torch.arange(ids.shape[1], device=ids.device)[None]
        rope = {}
        for kind in dict.fromkeys(lm.config.layer_types):
            cos, sin = lm.rotary_emb(emb, positions, kind)
            rope[kind] = (cos[0], sin[0])
        if rope_cache is not None:
            while len(rope_cache) >= 4:
                rope_cache.pop(next(iter(rope_cache)))
            rope_cache[key] = rope
    return emb[0], per_layer, rope


class Prefill:
    """pipeline.py:224-339 on the GPU: Prefill(model)(ids) -> (logits [vocab] fp32, DynamicCache)."""

    def __init__(self, model, layer_gemms=None, row_step=None, fuse_gelu=True, dequant_in_gemm=None):
        self.model = model
        self.lm = language_model(model)
        self.cfg = cfg = self.lm.config
        weights = layer_gemms if layer_gemms is not None else getattr(model, "layer_gemms", None)
        if weights is None:
            raise ValueError("Prefill: run w8a8.hf.to_gpu(model) first (it builds model.layer_gemms)")
        if row_step is not None and int(row_step) < 1:
            raise ValueError(f"Prefill: row_step {row_step} must be positive")
        self.row_step = None if row_step is None else int(row_step)
        self.fuse_gelu = bool(fuse_gelu)
        self.rope_cache = {}  # (T, device, dtype) -> the RoPE rows of positions 0 .. T-1 per attention kind
        # The GEMMs that feed k_qkv / k_post_attn / k_post_ff / k_ple_gate / k_ple_out may write their
        # dequantised bf16 result (the dequant epilogue) instead of int32: those kernels dequantise
        # first, so the results are bit-identical with half the bytes written and read.  True / False
        # force the bf16 / int32 (the reference's NPU output, npu_kernels.py:56) hand-over; None takes
        # bf16 past 1024 rows, where the halved traffic wins (3658-token prompt: 15.7 -> 15.3 ms), and
        # int32 up to there, where the dequant epilogue costs more than it saves (one 512-row layer
        # chain: 103.5 against 107.2 us).
        self.dequant_in_gemm = None if dequant_in_gemm is None else bool(dequant_in_gemm)
        if getattr(cfg, "enable_moe_block", False):
            raise NotImplementedError("Prefill: MoE decoder layers are not on the reference's path")
        if not cfg.hidden_size_per_layer_input:
            raise NotImplementedError("Prefill: the reference's pipeline needs per-layer inputs (PLE)")
        self.plans = []
        full_length = {}  # attention kind -> the last layer so far that stores full-length keys
        for i, layer in enumerate(self.lm.layers):
            a = layer.self_attn
            if not a.is_kv_shared_layer and a.v_proj is None:
                raise NotImplementedError(f"Prefill: layer {i} derives v from k (attention_k_eq_v); the "
                                          "reference's k_qkv expects a v projection")
            if set(weights[i]) != set(ROLES):
                raise ValueError(f"Prefill: layer {i} lacks GEMM groups, got {sorted(weights[i])}")
            kind = cfg.layer_types[i]
            source = full_length[kind] if a.is_kv_shared_layer else i
            if not a.is_kv_shared_layer and a.store_full_length_kv:
                full_length[kind] = i
            self.plans.append(LayerPlan(i, layer, cfg, weights[i], source))
        self.layer_scalars = None

    def _scalars(self):
        if self.layer_scalars is None:
            self.layer_scalars = [layer.layer_scalar.to(torch.bfloat16) for layer in self.lm.layers]
        return self.layer_scalars

    def _layer(self, p, h, start, end, per_layer, rope, store, scalar, xin=None, norm_next=None):
        """Rows [start, end) of the prompt through decoder layer p; returns their new hidden rows.  xin:
        the layer's input rows already normed and quantised (k_in), by the previous layer's last
        launch; with norm_next (the next layer's input-norm weight) that launch also makes the next
        layer's: returns (rows, xq, sx)."""
        eps = self.cfg.rms_norm_eps
        W = p.weights

        bf16_out = self.dequant_in_gemm if self.dequant_in_gemm is not None else end - start > 1024

        def gemm(xq, sx, w):
            """The result of one GEMM as the fused kernel after it reads it."""
            if bf16_out:
                return ops.gemm_bf16(xq, sx, w.packed, w.sw)
            return ops.gemm_i32(xq, w.packed)
        cos, sin = (t[start:end] for t in rope[p.kind])
        xq, sx = fused.k_in(h, p.norm_in, eps, packed=True) if xin is None else xin
        acc = gemm(xq, sx, W["qkv"])
        q, k, v = fused.k_qkv(acc, sx, W["qkv"].sw, cos, sin, p.norm_q, p.norm_k, eps, p.heads, p.kv_heads,
                              p.head_dim, p.shares_kv)
        if not p.shares_kv:
            store.write(p.index, start, k, v)
        keys, values = store.visible(p.kv_source, end)
        # attention with k_attn_out in its epilogue (the two steps where that does not apply)
        xq, sx = attention.attention_quant(q, keys, values, start, p.window, 1.0)
        acc = gemm(xq, sx, W["o"])
        h, xq, sx = fused.k_post_attn(acc, sx, W["o"].sw, h, p.norm_post_attn, p.norm_pre_ff, eps, packed=True)
        gu = W["gate_up"]
        if self.fuse_gelu and getattr(gu, "packed_gelu", None) is not None:
            # the GEMM's GELU epilogue writes k_gelu's bf16 bf16(gelu(gate)) * up, then its quant
            xq, sx = ops.quant_rows_packed(ops.gemm_bf16(xq, sx, gu.packed_gelu, epilogue="gelu"))
        else:
            xq, sx = fused.k_gelu(ops.gemm_i32(xq, gu.packed), sx, gu.sw, gu.N // 2, packed=True)
        acc = gemm(xq, sx, W["down"])
        h, xq, sx = fused.k_post_ff(acc, sx, W["down"].sw, h, p.norm_post_ff, eps, packed=True)
        acc = gemm(xq, sx, W["ple_gate"])
        xq, sx = fused.k_ple_gate(acc, sx, W["ple_gate"].sw, per_layer[start:end, p.index], packed=True)
        acc = gemm(xq, sx, W["ple_proj"])
        return fused.k_ple_out(acc, sx, W["ple_proj"].sw, h, p.norm_post_ple, scalar[p.index], eps, norm_next,
                               packed=True)

    def run_layers(self, h0, per_layer, rope, scalar=None):
        """Every decoder layer over the prompt: (final hidden rows [T, hidden] before the last norm,
        the KVStore of the prompt's keys and values)."""
        scalar = self._scalars() if scalar is None else scalar
        T = h0.shape[0]
        store = KVStore(T)
        step = self.row_step or T
        rows = []
        for start in range(0, T, step):  # prompt order: each range sees the keys of those before it
            end = min(start + step, T)
            h = h0[start:end]
            xin = None
            for i, p in enumerate(self.plans):
                if i + 1 < len(self.plans):
                    h, *xin = self._layer(p, h, start, end, per_layer, rope, store, scalar, xin,
                                          self.plans[i + 1].norm_in)
                else:
                    h = self._layer(p, h, start, end, per_layer, rope, store, scalar, xin)
            rows.append(h)
        return (rows[0] if len(rows) == 1 else torch.cat(rows)), store

    def check_ids(self, ids):
        if ids.dim() != 2 or ids.shape[0] != 1 or ids.shape[1] < 1:
            raise ValueError(f"Prefill: expected ids [1, T], got {tuple(ids.shape)}")
        return ids.to(self.lm.embed_tokens.weight.device)

    def last_token_logits(self, rows):
        """The model's final norm, LM head and logit softcap on the last hidden row (pipeline.py:334-338)."""
        logits = self.model.lm_head(self.lm.norm(rows[-1:][None]))[0, -1].float()
        cap = self.cfg.final_logit_softcapping
        return torch.tanh(logits / cap) * cap if cap else logits

    @torch.inference_mode()
    def __call__(self, ids, all_hidden=False):
        """ids [1, T] -> (last-token logits [vocab] fp32, DynamicCache) (pipeline.py:312-339).

        With all_hidden, the final-norm hidden states [T, hidden] instead of the logits."""
        h0, per_layer, rope = prompt_inputs(self.lm, self.check_ids(ids), self.rope_cache)
        rows, store = self.run_layers(h0, per_layer, rope)
        cache = store.to_cache(self.cfg, copy=False)
        if all_hidden:
            return self.lm.norm(rows[None])[0], cache
        return self.last_token_logits(rows), cache

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
        h0, per_layer, rope = prompt_inputs(prefill.lm, torch.zeros((1, T), dtype=torch.long, device=dev))
        self.h0, self.per_layer, self.rope = h0.clone(), per_layer.clone(), rope
        scalar = prefill._scalars()
        self.stream = torch.cuda.Stream(dev)
        self.stream.wait_stream(torch.cuda.current_stream(dev))
        with torch.cuda.stream(self.stream):
            prefill.run_layers(self.h0, self.per_layer, self.rope, scalar)
        torch.cuda.current_stream(dev).wait_stream(self.stream)
        torch.cuda.synchronize(dev)
        self.graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(self.graph, stream=self.stream):
            self.rows, self.store = prefill.run_layers(self.h0, self.per_layer, self.rope, scalar)
        torch.cuda.synchronize(dev)

    @torch.inference_mode()
    def __call__(self, ids):
        p = self.prefill
        ids = p.check_ids(ids)
        if ids.shape[1] != self.T:
            raise ValueError(f"CapturedPrefill: captured for {self.T} tokens, got {ids.shape[1]}")
        h0, per_layer, _ = prompt_inputs(p.lm, ids)
        self.h0.copy_(h0)
        self.per_layer.copy_(per_layer)
        self.graph.replay()
        return p.last_token_logits(self.rows), self.store.to_cache(p.cfg, copy=True)


class Decoder:
    """Greedy decoding after the prompt, every step on the GPU: the reference's decode loop
    (gemma_npu.py:278-300, HF's model called once per token) as one fixed sequence of launches.

    Per layer, for the one new token: the decode linears on the int8 GEMV with bf16 activations, the
    reference's decode copy of each weight (gemma_npu.py:117-121, 155-156); q / k norms and RoPE
    (k_qkv); the key and value written into the cache at the token's position; the decode attention
    over the cache (local_attn.py:44-83); and the norms, residuals, GELU-tanh products and
    per-layer-input steps of pipeline.py:66-127 without the activation quant, since the next linear
    reads bf16.  Each residual + norm step is the prologue of the GEMV that reads its result (the
    norm is made in that launch, bit for bit the row kernel's), and k_qkv runs inside the attention
    launch, so a layer is eight launches: qkv, two of attention, o, gate/up, down, per-layer gate,
    per-layer projection.  The token, its position and the key / value cache [KV, max_len, head_dim]
    of every layer that owns keys live in device memory, so a step does not depend on host values: capture()
    records one step in a HIP graph and each replay decodes the next token.  The next token is the
    argmax of the last logits (greedy), chosen on the device.

        dec = Decoder(Prefill(model), max_len=4096)
        logits = dec.start(ids)              # the prompt through the prefill; the first new token
        tokens = dec.generate(32)            # 32 greedy steps, graph-replayed
    """

    def __init__(self, prefill, max_len):
        self.pre = prefill
        self.lm, self.cfg = prefill.lm, prefill.cfg
        self.max_len = int(max_len)
        if self.max_len < 2:
            raise ValueError(f"Decoder: max_len {max_len} leaves no room to decode")
        dev = self.lm.embed_tokens.weight.device
        self.device = dev
        self.tok = torch.zeros((1, 1), dtype=torch.long, device=dev)
        self.pos = torch.zeros((1,), dtype=torch.int32, device=dev)      # read by the attention kernel
        self.pos64 = torch.zeros((1,), dtype=torch.long, device=dev)     # for the index operations
        self.emitted = torch.zeros((self.max_len,), dtype=torch.long, device=dev)
        self.zero_index = torch.zeros((1,), dtype=torch.long, device=dev)
        self.n_emitted = torch.zeros((1,), dtype=torch.long, device=dev)
        positions = torch.arange(self.max_len, device=dev)[None]
        probe = torch.zeros((1, self.max_len, self.cfg.hidden_size), dtype=torch.bfloat16, device=dev)
        self.rope = {}
        for kind in dict.fromkeys(self.cfg.layer_types):
            cos, sin = self.lm.rotary_emb(probe, positions, kind)
            self.rope[kind] = (cos[0].contiguous(), sin[0].contiguous())
        del probe
        self.cache = {}
        ws = 1 << 16
        for p in prefill.plans:
            if not p.shares_kv:
                shape = (p.kv_heads, self.max_len, p.head_dim)
                self.cache[p.index] = (torch.zeros(shape, dtype=torch.bfloat16, device=dev),
                                       torch.zeros(shape, dtype=torch.bfloat16, device=dev))
            ws = max(ws, attention.decode_at_workspace_bytes(p.heads, p.kv_heads, self.max_len, p.head_dim,
                                                             p.window))
        self.workspace = torch.empty(ws, dtype=torch.uint8, device=dev)
        # The final norm joins the last layer's per-layer-input norm in one row-kernel launch, with
        # its weight as the model's module applies it (x * (mean(x^2) + eps)^-0.5 * w, or no weight).
        norm = self.lm.norm
        self.final_norm = getattr(norm, "weight", None) if getattr(norm, "with_scale", True) else None
        if float(getattr(norm, "eps", self.cfg.rms_norm_eps)) != float(self.cfg.rms_norm_eps):
            raise ValueError("Decoder: the final norm's eps differs from the layers' rms_norm_eps")
        self.tail_ws = torch.empty(int(lib().w8a8_decode_tail_workspace_bytes(self.cfg.vocab_size)),
                                   dtype=torch.uint8, device=dev)
        # layers whose few key chunks (a sliding window) the o projection merges in its prologue
        self.merge_in_o = {p.index for p in prefill.plans
                           if p.heads // p.kv_heads <= 8 and p.heads * p.head_dim <= 4096
                           and attention.decode_grid_chunks(p.head_dim, self.max_len, p.window) <= 16}
        # the residual stream's norms as the prologue of the linear that reads them (hidden <= 1536)
        self.fuse_norms = self.cfg.hidden_size <= 1536 and self.cfg.hidden_size % 16 == 0
        self.length = None
        self.graph = None

    @torch.inference_mode()
    def start(self, ids):
        """The prompt ids [1, T] through the whole-prompt prefill: fills the key / value cache, sets the
        first new token (the argmax of the returned last-token logits) at position T."""
        ids = self.pre.check_ids(ids)
        T = ids.shape[1]
        if T >= self.max_len:
            raise ValueError(f"Decoder: a {T}-token prompt leaves no room in max_len {self.max_len}")
        h0, per_layer, rope = prompt_inputs(self.lm, ids, self.pre.rope_cache)
        rows, store = self.pre.run_layers(h0, per_layer, rope)
        for layer, (kc, vc) in self.cache.items():
            k, v = store.kv[layer]
            kc[:, :T].copy_(k)
            vc[:, :T].copy_(v)
        logits = self.pre.last_token_logits(rows)
        self.pos.fill_(T)
        self.pos64.fill_(T)
        self.n_emitted.zero_()
        self._emit(logits)
        self.length = T
        return logits

    def _emit(self, logits):
        """The first new token after the prefill, chosen on the device: the argmax becomes the next
        input token and is recorded (the decode steps take theirs in ops.decode_tail).  The argmax
        runs in two single-block stages (per row of a [rows, 512] view, then over the rows' maxima;
        the first index of the maximum, as a flat argmax gives) and the writes are index_copy_
        kernels, so no memset or memcpy is issued."""
        V = logits.shape[0]
        cols = 512 if V % 512 == 0 else V
        grid = logits.view(-1, cols)
        idx = grid.argmax(dim=1)
        row = grid.amax(dim=1).argmax().view(1)
        nxt = row * cols + idx.index_select(0, row)
        self.tok.view(1).index_copy_(0, self.zero_index, nxt)
        self.emitted.index_copy_(0, self.n_emitted, nxt)
        self.n_emitted.add_(1)

    def _head(self, x):
        """The model's head on the token's final-norm row x as HF's decode call computes it (the loop
        this replaces), and the step's end: the LM head GEMV, then in two launches the logit softcap
        in the model's dtype (bf16 ops, then fp32; the prefill pipeline takes it in fp32, as
        pipeline.py:334-338 does), the greedy argmax into the next token and the emitted list, and
        the position advanced.  Returns the fp32 logits."""
        y = self.pre.model.lm_head(x[None])[0, -1]
        return ops.decode_tail(y, self.cfg.final_logit_softcapping, self.pos, self.pos64, self.tok, self.emitted,
                               self.n_emitted, workspace=self.tail_ws)

    def _norm_linear(self, pend, w, act=None, mul=None):
        """The linear w on the residual stream's norm: pend = (y, res, w1, scalar, w2, store) describes
        h = bf16(bf16(res + bf16(rms(y) * w1)) * scalar) and x = bf16(rms(h) * w2) (x = h without w2,
        h = the norm alone without res).  Returns (w's output on x, h or None unless store).  With a
        hidden size of at most 1536 the norm is the GEMV's own prologue (one launch); otherwise the row
        kernel runs first."""
        y, res, w1, scalar, w2, store = pend
        eps = self.cfg.rms_norm_eps
        if self.fuse_norms:
            return ops.gemv_norm_bf16(y, res, w1, eps, w.gemv_w, w.sw_bf16, act=act, w2=w2, norm2=w2 is not None,
                                      scalar=scalar, mul=mul, store_h=store)
        if w2 is not None:
            h, x = ops.rms_residual_norm(y, res, w1, w2, eps, scalar=scalar)
        else:
            h = x = ops.rms_residual(y, res, w1, eps)
        out = (ops.gemv_bf16(x, w.gemv_w, w.sw_bf16) if act is None
               else ops.gemv_act_bf16(x, w.gemv_w, w.sw_bf16, act, mul=mul))
        return out, (h if store else None)

    def _layer(self, p, h, pend, per_layer, scalar, rope, norm_next):
        """Decoder layer p on the token's row at the device-held position: h [1, hidden] is the residual
        stream before the layer's input norm and pend how that norm is made (_norm_linear); rope maps
        the attention kind to its (cos, sin) tables [max_len, head_dim], read at the position.  Returns the
        residual stream and the pending norm after the layer: the next layer's input norm with
        norm_next, else the model's final norm."""
        W = p.weights
        y, hn = self._norm_linear(pend, W["qkv"])
        if hn is not None:
            h = hn
        cos, sin = rope[p.kind]
        eps = self.cfg.rms_norm_eps
        kc, vc = self.cache[p.kv_source]
        if p.heads // p.kv_heads <= 8:
            # k_qkv inside the attention launch (the key and value written at the position there); a
            # sliding window's few key chunks are merged in the o projection's prologue
            merge_in_o = p.index in self.merge_in_o
            o = attention.decode_qkv_at(y, cos, sin, p.norm_q, p.norm_k, eps, p.heads, p.kv_heads, p.head_dim, kc,
                                        vc, self.pos, not p.shares_kv, p.window, 1.0, workspace=self.workspace,
                                        merge=not merge_in_o)
            if merge_in_o:
                y = ops.gemv_attn_merge_bf16(self.workspace, self.pos, p.heads, p.kv_heads, self.max_len, p.head_dim,
                                             p.window, 1.0, W["o"].gemv_w, W["o"].sw_bf16)
        else:
            merge_in_o = False
            cos, sin = cos.index_select(0, self.pos64), sin.index_select(0, self.pos64)
            if p.shares_kv:
                q = fused.k_qkv(y, None, None, cos, sin, p.norm_q, None, eps, p.heads, p.kv_heads, p.head_dim,
                                True)[0]
            else:
                q = fused.k_qkv_cache(y, cos, sin, p.norm_q, p.norm_k, eps, p.heads, p.kv_heads, p.head_dim, kc, vc,
                                      self.pos)
            o = attention.decode_at(q[:, 0], kc, vc, self.pos, p.window, 1.0, workspace=self.workspace)
        if not merge_in_o:
            y = ops.gemv_bf16(o.reshape(1, -1), W["o"].gemv_w, W["o"].sw_bf16)
        g, h = self._norm_linear((y, h, p.norm_post_attn, None, p.norm_pre_ff, True), W["gate_up"], "gelu_pair")
        y = ops.gemv_bf16(g, W["down"].gemv_w, W["down"].sw_bf16)
        g, h = self._norm_linear((y, h, p.norm_post_ff, None, None, True), W["ple_gate"], "gelu_mul",
                                 mul=per_layer[:, p.index])
        y = ops.gemv_bf16(g, W["ple_proj"].gemv_w, W["ple_proj"].sw_bf16)
        return h, (y, h, p.norm_post_ple, scalar[p.index], norm_next, True)

    @torch.inference_mode()
    def step(self):
        """Decode the current token at the current position: its last-position logits [vocab] fp32;
        the argmax becomes the next token and the position advances, all on the device."""
        if self.length is None:
            raise RuntimeError("Decoder: call start(ids) first")
        if self.length >= self.max_len:
            raise RuntimeError(f"Decoder: the cache of {self.max_len} positions is full")
        logits = self._step()
        self.length += 1
        return logits

    def _step(self):
        emb = self.lm.embed_tokens(self.tok)
        per_layer = self.lm.project_per_layer_inputs(emb, self.lm.get_per_layer_inputs(self.tok, emb))[0]
        h = emb[0]
        scalar = self.pre._scalars()
        rope = self.rope  # the attention reads the tables' rows at the position itself
        plans = self.pre.plans
        pend = (h, None, plans[0].norm_in, None, None, False)
        for i, p in enumerate(plans):
            nxt = plans[i + 1].norm_in if i + 1 < len(plans) else self.final_norm
            h, pend = self._layer(p, h, pend, per_layer, scalar, rope, nxt)
        y, res, w1, sc, w2, _ = pend
        _, x = ops.rms_residual_norm(y, res, w1, w2, self.cfg.rms_norm_eps, scalar=sc)
        return self._head(x)

    @torch.inference_mode()
    def capture(self):
        """One decode step recorded in a HIP graph.  Runs one eager step first on the capture stream
        (its logits are returned: it is a real step, and it creates every workspace outside the
        graph), then captures the next step without running it.  replay() then decodes one token per
        call into the static logits tensor `self.graph_logits`."""
        if self.length is None:
            raise RuntimeError("Decoder: call start(ids) first")
        if self.length + 2 > self.max_len:
            raise RuntimeError("Decoder: no room left to capture a step")
        stream = torch.cuda.Stream(self.device)
        stream.wait_stream(torch.cuda.current_stream(self.device))
        with torch.cuda.stream(stream):
            first = self.step()
        torch.cuda.current_stream(self.device).wait_stream(stream)
        torch.cuda.synchronize(self.device)
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, stream=stream):
            self.graph_logits = self._step()
        torch.cuda.synchronize(self.device)
        self.graph = graph
        return first

    def replay(self):
        """One graph-replayed decode step: the static logits tensor, the next token chosen."""
        if self.graph is None:
            raise RuntimeError("Decoder: capture() first")
        if self.length >= self.max_len:
            raise RuntimeError(f"Decoder: the cache of {self.max_len} positions is full")
        self.graph.replay()
        self.length += 1
        return self.graph_logits

    @torch.inference_mode()
    def generate(self, n, graph=True):
        """n more greedy tokens (after start): a list of ints, read once at the end."""
        if self.length is None:
            raise RuntimeError("Decoder: call start(ids) first")
        if self.length + n > self.max_len:
            raise ValueError(f"Decoder: {n} more tokens pass max_len {self.max_len}")
        first = int(self.n_emitted.item())
        if graph:
            if self.graph is None and n >= 2:
                self.capture()
                n -= 1
            for _ in range(n):
                self.replay()
        else:
            for _ in range(n):
                self.step()
        return self.emitted[first:int(self.n_emitted.item())].tolist()


@torch.inference_mode()
def run(model, ids, n_decode, prefill=None):
    """gemma_npu.py:271-296 on the device: prefill (timed) then greedy decode of n_decode tokens;
    returns (ttft seconds, decode tok/s, tokens, last-token logits fp32), as the reference's run().

    With a Prefill (this module's, on the engine's weights) the prompt runs as the whole-prompt prefill
    and the decode as Decoder steps: the second token's step runs eagerly while it is captured in a
    HIP graph (untimed set-up), and the rate is taken over the graph replays of the tokens after it.
    Without one, HF's own forward and decode loop run on the model (the reference's prefill=None
    path).  Times include a device synchronisation, so they cover the GPU work."""
    dev = language_model(model).embed_tokens.weight.device
    if prefill is None:
        torch.cuda.synchronize(dev)
        t = time.perf_counter()
        out = model(input_ids=ids.to(dev), use_cache=True, logits_to_keep=1)
        logits, past = out.logits[0, -1].float(), out.past_key_values
        nxt = logits.argmax().view(1, 1)
        toks = [int(nxt.item())]
        ttft = time.perf_counter() - t
        t = time.perf_counter()
        for _ in range(n_decode - 1):
            out = model(input_ids=nxt, past_key_values=past, use_cache=True, logits_to_keep=1)
            past = out.past_key_values
            nxt = out.logits[0, -1].argmax().view(1, 1)
            toks.append(int(nxt.item()))
        dec = (n_decode - 1) / (time.perf_counter() - t) if n_decode > 1 else 0.0
        return ttft, dec, toks, logits
    T = ids.shape[1]
    decoder = Decoder(prefill, max_len=T + max(n_decode, 2) + 1)
    torch.cuda.synchronize(dev)
    t = time.perf_counter()
    logits = decoder.start(ids)
    torch.cuda.synchronize(dev)
    ttft = time.perf_counter() - t
    dec = 0.0
    if n_decode > 1:
        decoder.capture()
        torch.cuda.synchronize(dev)
        t = time.perf_counter()
        for _ in range(n_decode - 2):
            decoder.replay()
        torch.cuda.synchronize(dev)
        if n_decode > 2:
            dec = (n_decode - 2) / (time.perf_counter() - t)
    return ttft, dec, decoder.emitted[:n_decode].tolist(), logits
