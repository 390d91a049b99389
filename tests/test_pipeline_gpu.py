"""The reference's prefill pipeline with every step on the GPU (w8a8.pipeline.Prefill, after
pipeline.py:224-339): int32 W8A8 GEMMs, the fused kernels between them and prefill attention,
driven over a small random-init Gemma 4 with every feature of E2B's text decoder (sliding and full
layers, KV-shared layers, double-wide MLPs, per-layer inputs; see hf_tiny.py).

Checks:
- the last-token logits against the same HF model run in float32 on the CPU with the engine's
  dequantized int8 weights (the W8A8 activations add per-token quantisation noise, so the bound is
  the one the HF-driven engine meets, test_hf_gemma4_gpu.py), and against that HF-driven engine on
  the GPU, whose linears quantize the same activations;
- the DynamicCache it returns: HF's own decode loop continues from it past the sliding window, token
  for token within the decode bound against the float32 reference;
- the reference's 512-row micro-batch order (row_step) against the whole-prompt order: every step
  but attention is row-wise, so the final hidden rows agree to bf16 noise;
- the fused gate/up route (the GEMM's GELU epilogue, then the quant kernel) against k_gelu on the
  int32 result: the same int8 rows and scales, and the same final hidden rows through the model;
- the GEMMs' dequantised bf16 hand-over to the fused kernels against the int32 one: the same bits;
- determinism, and its refusals (no layer groups, a bad row_step, ids of the wrong shape).
"""
import copy

import pytest
import torch

from hf_tiny import build, dequantized_reference, rel_err

pytestmark = pytest.mark.gpu
DEV = "cuda"


def engine_model(base):
    from w8a8 import hf
    m = copy.deepcopy(base).to(torch.bfloat16).to(DEV)
    hf.to_gpu(m)
    return m


@torch.inference_mode()
@pytest.mark.parametrize("T", [40, 33])
def test_prefill_logits(T):
    from w8a8.pipeline import Prefill
    base = build()
    ref = dequantized_reference(base)
    ours = engine_model(base)
    ids = torch.randint(0, 512, (1, T), generator=torch.Generator().manual_seed(T))
    logits, cache = Prefill(ours)(ids)
    assert logits.shape == (512,) and logits.dtype == torch.float32 and logits.device.type == "cuda"
    want = ref(input_ids=ids, use_cache=True).logits[0, -1]
    e_ref = rel_err(logits, want)
    hf_engine = ours(input_ids=ids.to(DEV), use_cache=True).logits[0, -1]
    e_hf = rel_err(logits, hf_engine)
    print(f"T={T}: pipeline vs float32 reference {e_ref:.4f}, vs HF-driven engine {e_hf:.4f}")
    assert e_ref < 0.10
    assert e_hf < 0.10
    assert cache.get_seq_length() == T


@torch.inference_mode()
def test_decode_continues_from_pipeline_cache():
    """HF's decode loop (the engine's GEMVs and decode attention) runs on the cache the pipeline
    filled; 24 tokens take it past the sliding window of 16."""
    from w8a8.pipeline import Prefill
    base = build(seed=3)
    ref = dequantized_reference(base)
    ours = engine_model(base)
    ids = torch.randint(0, 512, (1, 20), generator=torch.Generator().manual_seed(4))
    _, past = Prefill(ours)(ids)
    o_ref = ref(input_ids=ids, use_cache=True)
    past_ref = o_ref.past_key_values
    worst = 0.0
    for step in range(24):
        nxt = o_ref.logits[0, -1].argmax().view(1, 1)
        o_ref = ref(input_ids=nxt, past_key_values=past_ref, use_cache=True)
        o = ours(input_ids=nxt.to(DEV), past_key_values=past, use_cache=True)
        worst = max(worst, rel_err(o.logits[0, -1], o_ref.logits[0, -1]))
        past_ref, past = o_ref.past_key_values, o.past_key_values
    print(f"decode from the pipeline's cache to position 43: max relative logits error {worst:.4f}")
    assert worst < 0.05


@torch.inference_mode()
def test_micro_batches_match_whole_prompt():
    from w8a8.pipeline import Prefill
    ours = engine_model(build(seed=5))
    ids = torch.randint(0, 512, (1, 45), generator=torch.Generator().manual_seed(6))
    whole, _ = Prefill(ours)(ids, all_hidden=True)
    for step in (16, 7):
        mb, cache = Prefill(ours, row_step=step)(ids, all_hidden=True)
        assert cache.get_seq_length() == 45
        e = rel_err(mb, whole)
        print(f"row_step {step}: max relative row difference {e:.5f}")
        assert e < 2e-2
    logits_w, _ = Prefill(ours)(ids)
    logits_m, _ = Prefill(ours, row_step=16)(ids)
    assert rel_err(logits_m, logits_w) < 2e-2


@torch.inference_mode()
def test_pipeline_is_deterministic():
    from w8a8.pipeline import Prefill
    ours = engine_model(build(seed=7))
    ids = torch.randint(0, 512, (1, 37), generator=torch.Generator().manual_seed(8))
    p = Prefill(ours)
    a, _ = p(ids, all_hidden=True)
    b, _ = p(ids, all_hidden=True)
    assert torch.equal(a, b)


def test_refusals():
    from w8a8.pipeline import Prefill
    base = build(seed=9)
    gpu_plain = copy.deepcopy(base).to(torch.bfloat16).to(DEV)
    with pytest.raises(ValueError, match="to_gpu"):
        Prefill(gpu_plain)
    ours = engine_model(base)
    with pytest.raises(ValueError, match="row_step"):
        Prefill(ours, row_step=0)
    with pytest.raises(ValueError, match=r"ids \[1, T\]"):
        Prefill(ours)(torch.zeros((2, 4), dtype=torch.long))


@torch.inference_mode()
@pytest.mark.parametrize("M,I", [(40, 512), (77, 96), (512, 1536)])
def test_gelu_epilogue_equals_k_gelu(M, I):
    """The fused route of the gate/up step (GELU epilogue, then the quant kernel) gives k_gelu's int8
    rows and scales bit for bit (pipeline.py:102-107)."""
    from w8a8 import fused, ops, workloads
    K = 256
    x = workloads.activations(M, K, seed=M + I).to(DEV)
    w, sw = workloads.weights(2 * I, K, seed=M + I + 1)
    w, sw = w.to(DEV), sw.to(DEV)
    xq, sx = ops.quant_rows_packed(x)
    acc = ops.gemm_i32(xq, ops.pack_weight(w, "nk", sw=sw))
    q1, s1 = fused.k_gelu(acc, sx, sw, I)
    a = ops.gemm_bf16(xq, sx, ops.pack_weight(w, "nk", I, sw=sw), epilogue="gelu")
    q2, s2 = ops.quant_rows(a)
    assert torch.equal(q1, q2) and torch.equal(s1, s2)


@torch.inference_mode()
def test_fused_gelu_route_matches_reference_route():
    """Prefill with the fused gate/up route and with the reference's int32 + k_gelu route: the same
    final hidden rows, bit for bit."""
    from w8a8.pipeline import Prefill
    ours = engine_model(build(seed=11))
    ids = torch.randint(0, 512, (1, 52), generator=torch.Generator().manual_seed(12))
    a, _ = Prefill(ours)(ids, all_hidden=True)
    b, _ = Prefill(ours, fuse_gelu=False)(ids, all_hidden=True)
    assert torch.equal(a, b)


@torch.inference_mode()
def test_dequant_in_gemm_matches_int32_handover():
    """Prefill with the GEMMs writing their dequantised bf16 result (the default) and with the
    reference's int32 hand-over (each fused kernel dequantising first): the same logits, final
    hidden rows and cache, bit for bit."""
    from w8a8.pipeline import Prefill
    ours = engine_model(build(seed=17))
    ids = torch.randint(0, 512, (1, 45), generator=torch.Generator().manual_seed(18))
    a, ca = Prefill(ours, dequant_in_gemm=True)(ids)
    b, cb = Prefill(ours, dequant_in_gemm=False)(ids)
    assert torch.equal(a, b)
    for la, lb in zip(ca.layers, cb.layers):
        if getattr(la, "keys", None) is not None and la.keys.numel():
            assert torch.equal(la.keys, lb.keys) and torch.equal(la.values, lb.values)
    ha, _ = Prefill(ours, dequant_in_gemm=True)(ids, all_hidden=True)
    hb, _ = Prefill(ours)(ids, all_hidden=True)  # 45 rows: the automatic choice is the int32 hand-over
    assert torch.equal(ha, hb)


@torch.inference_mode()
def test_captured_prefill_replays_match_eager():
    """Prefill.capture(T): every replay, with eager work and synchronisations between replays, gives
    the eager prefill's logits and cache bit for bit, and HF's decode loop continues from its cache."""
    from w8a8.pipeline import Prefill
    ours = engine_model(build(seed=13))
    pre = Prefill(ours)
    T = 37
    run = pre.capture(T)
    for seed in (14, 15, 16):
        ids = torch.randint(0, 512, (1, T), generator=torch.Generator().manual_seed(seed))
        want, want_cache = pre(ids)
        torch.cuda.synchronize()
        got, cache = run(ids)
        torch.cuda.synchronize()
        assert torch.equal(got, want), f"replay for seed {seed} differs from the eager prefill"
        assert cache.get_seq_length() == T
        for lw, lg in zip(want_cache.layers, cache.layers):
            if getattr(lw, "keys", None) is not None and getattr(lw, "keys").numel():
                assert torch.equal(lw.keys, lg.keys) and torch.equal(lw.values, lg.values)
        _ = torch.ones(1000, device=DEV).sum().item()  # eager work between replays
    nxt = got.argmax().view(1, 1).to(DEV)
    a = ours(input_ids=nxt, past_key_values=cache, use_cache=True).logits[0, -1]
    b = ours(input_ids=nxt, past_key_values=want_cache, use_cache=True).logits[0, -1]
    assert torch.equal(a, b)
    with pytest.raises(ValueError, match="captured for 37"):
        run(torch.zeros((1, 36), dtype=torch.long))
