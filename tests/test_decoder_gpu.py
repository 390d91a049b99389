"""w8a8.pipeline.Decoder: greedy decoding after the prompt with every step on the GPU (the reference's
decode loop, gemma_npu.py:278-300, as one fixed launch sequence per token), on the small Gemma 4
of hf_tiny.py (sliding and full layers, KV-shared layers, double-wide MLPs, per-layer inputs).

Checks:
- against HF's own decode loop on the engine (w8a8.hf.to_gpu: the same GEMV weights and decode
  attention kernel, HF's torch ops between them), continuing from the same prompt: the same greedy
  tokens for 28 steps, past the sliding window of 16, and the logits within bf16 noise per step;
- a step replayed from the HIP graph gives the eager step's logits and tokens bit for bit, with
  eager work between replays;
- the refusals: no start, a prompt that fills max_len, steps past max_len.
"""
import pytest
import torch

from hf_tiny import build, rel_err
from test_pipeline_gpu import engine_model

pytestmark = pytest.mark.gpu
DEV = "cuda"


@torch.inference_mode()
def test_decoder_matches_hf_decode_loop():
    from w8a8.pipeline import Decoder, Prefill
    ours = engine_model(build(seed=31))
    ids = torch.randint(0, 512, (1, 20), generator=torch.Generator().manual_seed(32))
    first_logits, past = Prefill(ours)(ids)
    dec = Decoder(Prefill(ours), max_len=64)
    logits = dec.start(ids)
    assert torch.equal(logits, first_logits)
    nxt = first_logits.argmax().view(1, 1).to(DEV)
    worst = 0.0
    for step in range(28):
        o = ours(input_ids=nxt, past_key_values=past, use_cache=True)
        want = o.logits[0, -1].float()
        got = dec.step()
        e = rel_err(got, want)
        worst = max(worst, e)
        assert int(got.argmax()) == int(want.argmax()), f"step {step}: the greedy tokens differ"
        past = o.past_key_values
        nxt = want.argmax().view(1, 1)
    print(f"28 decode steps to position 48: max relative logits difference from HF's loop {worst:.5f}")
    assert worst < 2e-2
    assert dec.length == 20 + 28
    assert dec.emitted[:29].tolist() == [int(first_logits.argmax())] + dec.emitted[1:29].tolist()


@torch.inference_mode()
def test_graph_replay_matches_eager_steps():
    from w8a8.pipeline import Decoder, Prefill
    ours = engine_model(build(seed=33))
    ids = torch.randint(0, 512, (1, 13), generator=torch.Generator().manual_seed(34))
    eager = Decoder(Prefill(ours), max_len=48)
    eager.start(ids)
    want = [eager.step().clone() for _ in range(20)]
    replayed = Decoder(Prefill(ours), max_len=48)
    replayed.start(ids)
    got = [replayed.capture().clone()]
    for _ in range(19):
        got.append(replayed.replay().clone())
        torch.cuda.synchronize()
        _ = torch.ones(1000, device=DEV).sum().item()  # eager work between replays
    for i, (g, w) in enumerate(zip(got, want)):
        assert torch.equal(g, w), f"step {i}: the replayed logits differ from the eager step's"
    assert torch.equal(replayed.emitted[:21], eager.emitted[:21])
    toks = replayed.generate(5)
    assert len(toks) == 5 and replayed.length == 13 + 25


def test_decoder_refusals():
    from w8a8.pipeline import Decoder, Prefill
    ours = engine_model(build(seed=35))
    dec = Decoder(Prefill(ours), max_len=16)
    with pytest.raises(RuntimeError, match="start"):
        dec.step()
    with pytest.raises(ValueError, match="max_len"):
        dec.start(torch.zeros((1, 16), dtype=torch.long))
    dec.start(torch.zeros((1, 14), dtype=torch.long))
    dec.step()
    dec.step()
    with pytest.raises(RuntimeError, match="full"):
        dec.step()
    with pytest.raises(ValueError, match="max_len"):
        Decoder(Prefill(ours), max_len=1)


@torch.inference_mode()
def test_norm_prologues_match_the_row_kernels():
    """The residual + norm steps made in the prologue of the GEMV that reads them against the same steps
    as row-kernel launches of their own (hidden sizes above the prologue's 1536 take that route):
    the same logits and tokens bit for bit, eager and graph-replayed."""
    from w8a8.pipeline import Decoder, Prefill
    ours = engine_model(build(seed=37))
    ids = torch.randint(0, 512, (1, 11), generator=torch.Generator().manual_seed(38))
    fused, rows = Decoder(Prefill(ours), max_len=40), Decoder(Prefill(ours), max_len=40)
    assert fused.fuse_norms
    rows.fuse_norms = False
    fused.start(ids)
    rows.start(ids)
    for i in range(10):
        assert torch.equal(fused.step(), rows.step()), f"step {i}"
    assert torch.equal(fused.capture(), rows.capture())
    for i in range(5):
        assert torch.equal(fused.replay(), rows.replay()), f"replay {i}"
    assert torch.equal(fused.emitted, rows.emitted)


@torch.inference_mode()
def test_run_like_the_reference():
    """pipeline.run with gemma_npu.py:271-296's signature and results: (ttft, decode tok/s, tokens,
    last-token logits).  With the engine's Prefill its tokens are a Decoder's (the first the argmax of
    the prefill logits, the rest greedy steps); without one it is HF's forward and decode loop on the
    engine, whose first-token logits agree with the pipeline's within the prefill tolerance."""
    from w8a8.pipeline import Decoder, Prefill, run
    ours = engine_model(build(seed=39))
    ids = torch.randint(0, 512, (1, 17), generator=torch.Generator().manual_seed(40))
    ttft, dec, toks, logits = run(ours, ids, 12, Prefill(ours))
    assert ttft > 0 and dec > 0 and len(toks) == 12
    assert toks[0] == int(logits.argmax())
    ref = Decoder(Prefill(ours), max_len=40)
    ref.start(ids)
    assert toks == [toks[0]] + ref.generate(11, graph=False)
    ttft2, dec2, toks2, logits2 = run(ours, ids, 5)
    assert ttft2 > 0 and dec2 > 0 and len(toks2) == 5 and toks2[0] == int(logits2.argmax())
    assert rel_err(logits, logits2) < 0.1


@pytest.mark.parametrize("cap", [30.0, None])
def test_decode_tail_equals_the_models_softcap_and_argmax(cap):
    """ops.decode_tail (the decode step's end in two launches) against the ops it replaces: the logit
    softcap as the model's bf16 ops compute it, bit for bit; the next token = torch.argmax of those
    logits (the first index of the maximum: a tie planted across candidate workgroups, then a NaN);
    the emitted list, its count and the position advanced by one.  A ragged vocabulary of 262149."""
    from w8a8 import ops
    V = 262144 + 5
    g = torch.Generator(device=DEV).manual_seed(41)
    y = (torch.randn(V, generator=g, device=DEV) * 20).to(torch.bfloat16)
    top = y.float().abs().max().to(torch.bfloat16) * 2
    y[70000] = top
    y[3000] = top  # the same maximum at a smaller index, in another workgroup
    for plant_nan in (False, True):
        if plant_nan:
            y[200000] = float("nan")
        want = (torch.tanh(y / cap) * cap).float() if cap else y.float()
        pos = torch.tensor([7], dtype=torch.int32, device=DEV)
        pos64 = torch.tensor([7], dtype=torch.long, device=DEV)
        tok = torch.zeros((1, 1), dtype=torch.long, device=DEV)
        emitted = torch.zeros(16, dtype=torch.long, device=DEV)
        n = torch.tensor([3], dtype=torch.long, device=DEV)
        got = ops.decode_tail(y, cap, pos, pos64, tok, emitted, n)
        assert torch.equal(got.isnan(), want.isnan())
        assert torch.equal(torch.nan_to_num(got), torch.nan_to_num(want))
        expect = 200000 if plant_nan else 3000
        assert int(want.argmax()) == expect and int(tok) == expect
        assert int(emitted[3]) == expect and int(emitted.sum()) == expect
        assert int(n) == 4 and int(pos) == 8 and int(pos64) == 8
