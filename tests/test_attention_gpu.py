"""GPU parity of prefill attention (w8a8_attention_bf16) against the oracle.

The oracle computes each output in double and rounds it to bf16 once; the GPU rounds the softmax
weights to bf16 for the second product (as the reference's CPU flash kernel does with bf16
inputs) and its output once.  Tolerance per element:

    |o - o_ref| <= 2^-8 * sum_j p_j |v_j| + 1 ulp_bf16(o_ref)

twice the bound of the weight rounding (2^-9 relative per weight) plus the two output roundings.
The same bound is reported for torch's CPU sdpa in bf16 on the same inputs (the routine the
reference calls), so the two can be compared.
"""
import numpy as np
import pytest
import torch
import torch.nn.functional as F

from helpers import f32, to_bits, ulp_bf16

import oracle.oracle as orc
from w8a8 import W8A8Error
from w8a8 import attention as attn

pytestmark = pytest.mark.gpu
DEV = "cuda"


def make(H, KV, Tq, Tk, D, seed, qscale=1.0):
    g = torch.Generator().manual_seed(seed)
    q = (torch.randn(H, Tq, D, generator=g) * qscale).to(torch.bfloat16)
    k = (torch.randn(KV, Tk, D, generator=g) * qscale).to(torch.bfloat16)
    v = torch.randn(KV, Tk, D, generator=g).to(torch.bfloat16)
    return q, k, v


def reference(q, k, v, q_start, window, scale=1.0):
    out, bud, lse = orc.attention(to_bits(q), to_bits(k), to_bits(v), q_start, window, scale, budget=True, lse=True)
    return f32(out), bud, lse


def check(o, ref, bud, what, strict=True):
    """Max |err| / budget; raises if any element is outside the tolerance (strict)."""
    got = f32(to_bits(o))
    tol = 2.0 ** -8 * bud + ulp_bf16(ref)
    err = np.abs(got - ref)
    bad = err > tol
    if strict and bad.any():
        i = tuple(np.argwhere(bad)[0])
        raise AssertionError(f"{what}: {bad.sum()} of {bad.size} outside tolerance; first at {i}: "
                             f"got {got[i]!r} ref {ref[i]!r} budget {bud[i]!r}")
    return float((err / np.maximum(bud, 1e-30)).max())


CASES = [
    # H, KV, Tq, Tk, D, q_start, window, scale, qscale
    (8, 1, 512, 512, 256, 0, 512, 1.0, 1.0),     # sliding layer, first micro-batch
    (8, 1, 512, 1024, 256, 512, 512, 1.0, 0.3),  # sliding layer, second micro-batch
    (8, 1, 300, 400, 256, 100, 512, 1.0, 0.3),   # ragged, q_start not a multiple of 128
    (8, 1, 77, 77, 256, 0, 16, 1.0, 1.0),        # window shorter than a key block
    (8, 1, 256, 256, 512, 0, 0, 1.0, 0.3),       # full layer, head_dim 512
    (8, 1, 256, 768, 512, 512, 0, 1.0, 1.0),     # full layer against earlier keys
    (8, 1, 33, 290, 512, 257, 0, 1.0, 0.3),      # ragged full layer
    (4, 2, 200, 200, 128, 0, 0, 0.0883883, 1.0),  # head_dim 128, 2 KV heads, HF's 1/sqrt(D)
    (6, 2, 130, 190, 128, 60, 50, 1.0, 0.3),     # 3 heads per KV head (rows not a power of 2)
    (2, 2, 64, 64, 256, 0, 0, 1.0, 1.0),         # no grouping (one head per KV head)
    (16, 1, 40, 100, 256, 60, 1, 1.0, 1.0),      # window 1: each query sees only itself
]


@pytest.mark.parametrize("H,KV,Tq,Tk,D,q_start,window,scale,qscale", CASES)
def test_attention_matches_oracle(H, KV, Tq, Tk, D, q_start, window, scale, qscale):
    print(f"attention H={H} KV={KV} Tq={Tq} Tk={Tk} D={D} q_start={q_start} W={window}", flush=True)
    q, k, v = make(H, KV, Tq, Tk, D, seed=Tq + 3 * D + window, qscale=qscale)
    o, lse = attn.attention(q.to(DEV), k.to(DEV), v.to(DEV), q_start, window, scale, return_lse=True)
    ref, bud, lse_ref = reference(q, k, v, q_start, window, scale)
    check(o, ref, bud, "attention")
    assert np.allclose(lse.cpu().numpy(), lse_ref, rtol=1e-5, atol=1e-4), "logsumexp differs"
    if window == 1:
        assert torch.equal(o.cpu(), v[torch.arange(H) // (H // KV), q_start:q_start + Tq]), "window 1"


def test_micro_batches_like_the_reference_pipeline():
    """pipeline.py:281-295: each 512-row micro-batch of a sliding layer attends to keys 0..e, each
    256-row chunk of a full layer to keys 0..s+r1; the chunks are the pipeline's calls.  These calls
    are too few tiles for the CUs, so their keys are split and the parts merged by the second kernel
    (the planner's choice is checked, so the test keeps covering that path)."""
    import ctypes
    from w8a8 import lib
    T = 1300
    merge = ctypes.c_int(-1)
    for args in ((8, 1, 512, 1024, 256, 512, 512), (8, 1, 256, 768, 512, 512, 0)):
        assert lib().w8a8_attention_plan_items(*args, None, ctypes.byref(merge)) > 0 and merge.value == 1, args
    q, k, v = make(8, 1, T, T, 256, seed=1, qscale=0.3)
    qd, kd, vd = q.to(DEV), k.to(DEV), v.to(DEV)
    ref, bud, _ = reference(q, k, v, 0, 512)
    for s in range(0, T, 512):
        e = min(s + 512, T)
        o = attn.sliding_attention(qd[:, s:e], kd[:, :e], vd[:, :e], s, 512)
        check(o, ref[:, s:e], bud[:, s:e], f"sliding micro-batch {s}")
    q, k, v = make(8, 1, T, T, 512, seed=2, qscale=0.3)
    qd, kd, vd = q.to(DEV), k.to(DEV), v.to(DEV)
    ref, bud, _ = reference(q, k, v, 0, 0)
    for s in range(0, T, 512):
        e = min(s + 512, T)
        for r0 in range(0, e - s, 256):
            r1 = min(r0 + 256, e - s)
            o = attn.full_attention(qd[:, s + r0:s + r1], kd[:, :s + r1], vd[:, :s + r1], s + r0)
            check(o, ref[:, s + r0:s + r1], bud[:, s + r0:s + r1], f"full chunk {s + r0}")


@pytest.mark.parametrize("D,window", [(256, 512), (512, 0)])
def test_whole_prompt_3658(D, window):
    """The 3658-token prompt in one call; rows at the start, the middle and the end against the oracle."""
    T = 3658
    print(f"attention whole prompt T={T} D={D} W={window}", flush=True)
    q, k, v = make(8, 1, T, T, D, seed=D, qscale=0.3)
    o = attn.attention(q.to(DEV), k.to(DEV), v.to(DEV), 0, window).cpu()
    for r0 in (0, 1800, T - 40):
        r1 = r0 + 40
        ref, bud, _ = reference(q[:, r0:r1], k[:, :r1], v[:, :r1], r0, window)
        check(o[:, r0:r1], ref, bud, f"rows {r0}..{r1}")


def test_layouts_and_local_sdpa():
    """HF hands local_sdpa query [1, H, T, D] as a transposed view of [1, T, H, D] and wants
    [1, T, H, D] back; strided inputs and outputs give the same bits as contiguous ones."""
    H, KV, T, D = 8, 1, 200, 256
    q, k, v = make(H, KV, T, T, D, seed=7, qscale=0.3)
    qd, kd, vd = q.to(DEV), k.to(DEV), v.to(DEV)
    o = attn.attention(qd, kd, vd, 0, 64)
    q_thd = qd.transpose(0, 1).contiguous()            # [T, H, D]
    out, none = attn.local_sdpa(None, q_thd.transpose(0, 1)[None], kd[None], vd[None], None, scaling=1.0,
                                sliding_window=64)
    assert none is None and out.shape == (1, T, H, D) and out.is_contiguous()
    assert torch.equal(out[0].transpose(0, 1), o)
    full = attn.local_sdpa(None, qd[None], kd[None], vd[None], None, scaling=1.0)[0]
    assert torch.equal(full[0].transpose(0, 1), attn.full_attention(qd, kd, vd, 0))
    # decode: one query at the last position against the cache (local_attn.py:74-83) goes to the
    # split-key decode kernels
    dec = attn.local_sdpa(None, qd[None, :, -1:], kd[None], vd[None], None, scaling=1.0, sliding_window=64)[0]
    assert torch.equal(dec[0, 0], attn.decode(qd[:, -1], kd, vd, T - 1, 64))
    # k / v as column slices of a wider buffer
    kv = torch.cat([kd, vd], 2)
    o2 = attn.attention(qd, kv[:, :, :D], kv[:, :, D:], 0, 64)
    assert torch.equal(o, o2)


def test_split_tiles_and_the_unsplit_entry():
    """Long causal calls split their longest tiles' keys over several workgroups (the workspace
    entry, which attention() uses); the entry without a workspace computes every tile in one
    workgroup.  Both agree with the oracle; the split result is deterministic across calls."""
    from w8a8 import lib
    from w8a8._lib import call
    T, D = 1300, 512
    assert lib().w8a8_attention_workspace_bytes(8, 1, T, T, D, 0, 0) > 0
    q, k, v = make(8, 1, T, T, D, seed=11, qscale=0.3)
    qd, kd, vd = q.to(DEV), k.to(DEV), v.to(DEV)
    a, lse_a = attn.attention(qd, kd, vd, 0, 0, return_lse=True)
    b = attn.attention(qd, kd, vd, 0, 0)
    assert torch.equal(a, b)
    u = torch.empty_like(a)
    lse_u = torch.empty(8, T, dtype=torch.float32, device=DEV)
    call("w8a8_attention_bf16", qd.data_ptr(), T * D, D, kd.data_ptr(), T * D, D, vd.data_ptr(), T * D, D, 8, 1, T, T,
         D, 0, 0, 1.0, u.data_ptr(), T * D, D, lse_u.data_ptr(), torch.cuda.current_stream().cuda_stream)
    rows = list(range(0, 40)) + list(range(T - 200, T))
    ref, bud, lse_ref = reference(q[:, rows[:40]], k[:, :40], v[:, :40], 0, 0)
    check(a[:, :40], ref, bud, "split, first rows")
    check(u[:, :40], ref, bud, "unsplit, first rows")
    ref, bud, lse_ref = reference(q[:, T - 200:], k, v, T - 200, 0)
    check(a[:, T - 200:], ref, bud, "split, last rows")
    check(u[:, T - 200:], ref, bud, "unsplit, last rows")
    assert np.allclose(lse_a[:, T - 200:].cpu().numpy(), lse_ref, rtol=1e-5, atol=1e-4)
    assert np.allclose(lse_u[:, T - 200:].cpu().numpy(), lse_ref, rtol=1e-5, atol=1e-4)


SPLIT_CASES = [
    # H, KV, Tq, Tk, D, q_start: causal calls whose plans split their longest tiles
    (8, 1, 1300, 1300, 256, 0),     # head_dim 256 (attn_fwd_kernel's park and merge)
    (8, 2, 1300, 1300, 256, 0),     # two KV groups interleaved in the launch order
    (4, 2, 1300, 1300, 128, 0),     # head_dim 128, 2 heads per group
    (8, 2, 1300, 1300, 512, 0),     # head_dim 512 (attn_fwd2_kernel), two KV groups
    (8, 1, 256, 1300, 256, 1044),   # a micro-batch at the end of the prompt: every tile split
]


@pytest.mark.parametrize("H,KV,Tq,Tk,D,q_start", SPLIT_CASES)
def test_split_plans_match_oracle(H, KV, Tq, Tk, D, q_start):
    """Split causal calls at head_dims 128 / 256 / 512, with one and two KV groups: the first 40 and
    the last 200 rows against the oracle, the logsumexp of the last rows, and two calls equal."""
    from w8a8 import lib
    assert lib().w8a8_attention_workspace_bytes(H, KV, Tq, Tk, D, q_start, 0) > 0
    q, k, v = make(H, KV, Tq, Tk, D, seed=41 + D + KV, qscale=0.3)
    qd, kd, vd = q.to(DEV), k.to(DEV), v.to(DEV)
    a, lse = attn.attention(qd, kd, vd, q_start, 0, return_lse=True)
    assert torch.equal(a, attn.attention(qd, kd, vd, q_start, 0))
    ref, bud, _ = reference(q[:, :40], k[:, :q_start + 40], v[:, :q_start + 40], q_start, 0)
    check(a[:, :40], ref, bud, "first rows")
    ref, bud, lse_ref = reference(q[:, Tq - 200:], k, v, q_start + Tq - 200, 0)
    check(a[:, Tq - 200:], ref, bud, "last rows")
    assert np.allclose(lse[:, Tq - 200:].cpu().numpy(), lse_ref, rtol=1e-5, atol=1e-4)


def test_split_plan_past_the_order_table():
    """A causal call whose split plan holds more items per KV group than the launch-order table
    (1536): a 20000-token prompt at head_dim 512, 1250 query tiles of which the longest are split.
    Its items then run in plain item order.  The first and last 40 rows against the oracle, and
    two calls equal."""
    import ctypes
    from w8a8 import lib
    H, KV, D = 8, 1, 512
    order = ctypes.c_int(-1)
    T = next((t for t in (20000, 20500, 21000, 19500, 21500, 22000)
              if lib().w8a8_attention_plan_items(H, KV, t, t, D, 0, 0, ctypes.byref(order), None) > 1536
              and lib().w8a8_attention_workspace_bytes(H, KV, t, t, D, 0, 0) > 0), None)
    assert T is not None, "no prompt length in the list plans past the order table"
    lib().w8a8_attention_plan_items(H, KV, T, T, D, 0, 0, ctypes.byref(order), None)
    assert order.value == 0
    print(f"attention T={T} D={D}: {lib().w8a8_attention_plan_items(H, KV, T, T, D, 0, 0, None, None)} items, "
          "item order", flush=True)
    q, k, v = make(H, KV, T, T, D, seed=57, qscale=0.3)
    qd, kd, vd = q.to(DEV), k.to(DEV), v.to(DEV)
    a, lse = attn.attention(qd, kd, vd, 0, 0, return_lse=True)
    assert torch.equal(a, attn.attention(qd, kd, vd, 0, 0))
    ref, bud, _ = reference(q[:, :40], k[:, :40], v[:, :40], 0, 0)
    check(a[:, :40], ref, bud, "first rows")
    ref, bud, lse_ref = reference(q[:, T - 40:], k, v, T - 40, 0)
    check(a[:, T - 40:], ref, bud, "last rows")
    assert np.allclose(lse[:, T - 40:].cpu().numpy(), lse_ref, rtol=1e-5, atol=1e-4)


QUANT_CASES = [
    # H, KV, Tq, Tk, D, q_start, window: attention + k_attn_out in one launch, or the two-step fallback
    (8, 1, 700, 700, 256, 0, 128),     # sliding, whole prompt (one item per tile), ragged Tq
    (8, 1, 1300, 1300, 256, 0, 0),     # causal, head_dim 256, long tiles split and merged in the kernel
    (8, 1, 1300, 1300, 512, 0, 0),     # causal, head_dim 512 (attn_fwd2_kernel), split and merged in the kernel
    (8, 1, 77, 600, 512, 523, 0),      # a few queries past earlier keys
    (4, 1, 300, 300, 128, 0, 64),      # head_dim 128, 4 heads
    (8, 2, 300, 300, 256, 0, 64),      # two KV groups: the two-step form
    (8, 1, 512, 3658, 256, 3146, 512),  # the reference's last sliding micro-batch: parts merged by a second kernel
]


@pytest.mark.parametrize("H,KV,Tq,Tk,D,q_start,window", QUANT_CASES)
def test_attention_quant_equals_attention_then_k_attn_out(H, KV, Tq, Tk, D, q_start, window):
    """attention_quant (k_attn_out, pipeline.py:88-92, in the attention epilogue where it applies):
    the packed int8 rows (padding included) and scales equal k_attn_out on attention's bf16 output, bit
    for bit, whichever form runs; the one-launch form runs exactly where the library says it applies."""
    import ctypes
    from test_gemm_gpu import unpack_act
    from w8a8 import fused, lib
    q, k, v = make(H, KV, Tq, Tk, D, seed=H + Tq + D + window, qscale=0.3)
    qd, kd, vd = q.to(DEV), k.to(DEV), v.to(DEV)
    fused_form = lib().w8a8_attention_quant_supported(H, KV, Tq, Tk, D, q_start, window)
    mk = ctypes.c_int(-1)
    lib().w8a8_attention_plan_items(H, KV, Tq, Tk, D, q_start, window, None, ctypes.byref(mk))
    assert fused_form == (KV == 1 and mk.value == 0)
    xq, sx = attn.attention_quant(qd, kd, vd, q_start, window, 1.0)
    xr, sr = fused.k_attn_out(attn.attention(qd, kd, vd, q_start, window, 1.0), packed=True)
    assert torch.equal(sx, sr)
    got = unpack_act(xq.data.cpu().numpy(), Tq, H * D)
    assert np.array_equal(got[:Tq], unpack_act(xr.data.cpu().numpy(), Tq, H * D)[:Tq])
    assert not got[Tq:].any(), "padding rows must be zero"
    xq2, sx2 = attn.attention_quant(qd, kd, vd, q_start, window, 1.0)
    assert torch.equal(xq2.data, xq.data) and torch.equal(sx2, sx)


def test_split_workspace_shared_across_shapes():
    """Split calls of different shapes share the stream's workspace.  A whole-prompt causal call at
    head_dim 512 (T = 3658: ~190 split tiles), then 256 queries at the end of the prompt (16 split
    tiles), then the first call again: the second plan parks its parts past the same fixed counter
    region, so the first call's counters are still zero and its repeat is bit-identical, finite and
    within the tolerance of the unsplit entry on the last rows (checked against the oracle there)."""
    T, D = 3658, 512
    q, k, v = make(8, 1, T, T, D, seed=31, qscale=0.3)
    qd, kd, vd = q.to(DEV), k.to(DEV), v.to(DEV)
    first = attn.attention(qd, kd, vd, 0, 0)
    qs = T - 256
    mb = attn.attention(qd[:, qs:], kd, vd, qs, 0)
    again = attn.attention(qd, kd, vd, 0, 0)
    assert torch.isfinite(again).all()
    assert torch.equal(again, first)
    assert torch.equal(attn.attention(qd[:, qs:], kd, vd, qs, 0), mb)
    ref, bud, _ = reference(q[:, qs:], k, v, qs, 0)
    check(again[:, qs:], ref, bud, "whole prompt after a micro-batch, last rows")
    check(mb, ref, bud, "micro-batch")


def test_deterministic():
    q, k, v = make(8, 1, 600, 600, 512, seed=3, qscale=0.3)
    qd, kd, vd = q.to(DEV), k.to(DEV), v.to(DEV)
    a = attn.attention(qd, kd, vd, 0, 0)
    b = attn.attention(qd, kd, vd, 0, 0)
    assert torch.equal(a, b)


def test_versus_torch_cpu_flash():
    """Error against the double-precision oracle, relative to the weight-rounding budget, of ours
    (within the tolerance) and, for comparison, of torch's CPU sdpa in bf16 (what the reference
    runs)."""
    H, KV, T, D, W = 8, 1, 384, 256, 128
    q, k, v = make(H, KV, T, T, D, seed=5, qscale=0.3)
    ref, bud, _ = reference(q, k, v, 0, W)
    ours = check(attn.sliding_attention(q.to(DEV), k.to(DEV), v.to(DEV), 0, W), ref, bud, "ours")
    qp = torch.arange(T)[:, None]
    kp = torch.arange(T)[None, :]
    mask = (kp <= qp) & (qp - kp < W)
    cpu = F.scaled_dot_product_attention(q[None], k[None], v[None], attn_mask=mask, scale=1.0, enable_gqa=True)[0]
    theirs = check(cpu, ref, bud, "torch cpu bf16", strict=False)
    print(f"max |err| / budget: ours {ours:.3g}, torch cpu {theirs:.3g}")


def test_errors():
    q, k, v = make(4, 2, 8, 8, 128, seed=0)
    qd, kd, vd = q.to(DEV), k.to(DEV), v.to(DEV)
    with pytest.raises(W8A8Error, match="head_dim"):
        attn.attention(qd[:, :, :64].contiguous(), kd[:, :, :64].contiguous(), vd[:, :, :64].contiguous())
    with pytest.raises(W8A8Error, match="Tk >= q_start"):
        attn.attention(qd, kd, vd, q_start=1)
    with pytest.raises(W8A8Error, match="multiple of KV"):
        attn.attention(qd[:3], kd, vd)
    with pytest.raises(ValueError):
        attn.attention(qd, kd[:, :4], vd)
    with pytest.raises(ValueError):
        attn.sliding_attention(qd, kd, vd, 0, 0)
    # Tq == 0 is a no-op
    assert attn.attention(qd[:, :0], kd, vd).shape == (4, 0, 128)


# ---- decode (local_attn.py:44-83) -------------------------------------------------------------

DECODE_CASES = [
    # H, KV, Tk, D, q_pos, window
    (8, 1, 3658, 512, 3657, 0),     # full layer at the end of the benchmark prompt
    (8, 1, 3658, 256, 3657, 512),   # sliding layer: the last 512 keys
    (8, 1, 1, 256, 0, 0),           # the first token
    (8, 1, 65, 256, 64, 0),         # one key past a 64-key chunk
    (8, 1, 64, 512, 63, 0),         # exactly one chunk
    (8, 1, 500, 256, 300, 0),       # keys past the query position are ignored
    (4, 2, 300, 128, 299, 50),      # 2 KV heads, window not a chunk multiple
    (16, 1, 200, 256, 199, 0),      # 16 heads per KV head
    (6, 2, 130, 128, 129, 7),       # 3 heads per KV head
]


@pytest.mark.parametrize("H,KV,Tk,D,q_pos,window", DECODE_CASES)
def test_decode_matches_oracle(H, KV, Tk, D, q_pos, window):
    print(f"decode H={H} KV={KV} Tk={Tk} D={D} q_pos={q_pos} W={window}", flush=True)
    q, k, v = make(H, KV, 1, Tk, D, seed=Tk + D + window, qscale=0.5)
    o, lse = attn.decode(q[:, 0].to(DEV), k.to(DEV), v.to(DEV), q_pos, window, return_lse=True)
    ref, bud, lse_ref = reference(q, k, v, q_pos, window)
    check(o[:, None], ref, bud, "decode")
    assert np.allclose(lse.cpu().numpy(), lse_ref[:, 0], rtol=1e-5, atol=1e-4), "decode logsumexp differs"


def ragged_cases(seed, n, decode):
    """Seeded ragged attention calls: head groupings, head_dims, prompt lengths, query offsets and
    windows drawn at random (window 0 = full causal)."""
    rng = np.random.default_rng(seed)
    groups = [(8, 1), (4, 2), (6, 2), (16, 1), (2, 2), (12, 3)]
    out = []
    for _ in range(n):
        H, KV = groups[int(rng.integers(len(groups)))]
        D = int(rng.choice([128, 256, 512]))
        Tk = int(rng.integers(1, 700 if D == 512 else 900))
        window = int(rng.choice([0, 0, int(rng.integers(1, 600))]))
        if decode:
            out.append((H, KV, Tk, D, int(rng.integers(0, Tk)), window))
        else:
            q_start = int(rng.integers(0, Tk))
            out.append((H, KV, Tk - q_start, Tk, D, q_start, window))
    return out


@pytest.mark.parametrize("H,KV,Tq,Tk,D,q_start,window", ragged_cases(404, 10, False))
def test_attention_ragged_calls_match_oracle(H, KV, Tq, Tk, D, q_start, window):
    print(f"attention ragged H={H} KV={KV} Tq={Tq} Tk={Tk} D={D} q_start={q_start} W={window}", flush=True)
    q, k, v = make(H, KV, Tq, Tk, D, seed=Tq * 7 + Tk + D, qscale=0.5)
    o, lse = attn.attention(q.to(DEV), k.to(DEV), v.to(DEV), q_start, window, return_lse=True)
    ref, bud, lse_ref = reference(q, k, v, q_start, window)
    check(o, ref, bud, "ragged attention")
    assert np.allclose(lse.cpu().numpy(), lse_ref, rtol=1e-5, atol=1e-4), "ragged attention logsumexp differs"


@pytest.mark.parametrize("H,KV,Tk,D,q_pos,window", ragged_cases(505, 10, True))
def test_decode_ragged_calls_match_oracle(H, KV, Tk, D, q_pos, window):
    test_decode_matches_oracle(H, KV, Tk, D, q_pos, window)


def test_decode_mirror_and_determinism():
    """split_kv_decode takes the reference's shapes ([1, H, 1, D] against [1, 1, T, D]) and
    returns [1, 1, H, D]; repeated calls give the same bits."""
    H, T, D = 8, 1000, 256
    q, k, v = make(H, 1, 1, T, D, seed=21, qscale=0.5)
    qd, kd, vd = q.to(DEV), k.to(DEV), v.to(DEV)
    out = attn.split_kv_decode(qd.transpose(0, 1)[None].transpose(1, 2), kd[None], vd[None], 1.0)
    assert out.shape == (1, 1, H, D)
    a = attn.decode(qd[:, 0], kd, vd)
    assert torch.equal(out[0, 0], a)
    assert torch.equal(attn.decode(qd[:, 0], kd, vd), a)
    # and the result agrees with the prefill kernel's row for the same query within the tolerance
    ref, bud, _ = reference(q, k, v, T - 1, 0)
    check(a[:, None], ref, bud, "decode vs oracle")


def test_decode_errors():
    from w8a8._lib import call
    q, k, v = make(8, 1, 1, 100, 256, seed=0)
    qd, kd, vd = q[:, 0].to(DEV), k.to(DEV), v.to(DEV)
    with pytest.raises(W8A8Error, match="q_pos"):
        attn.decode(qd, kd, vd, q_pos=100)
    q32 = torch.zeros(32, 256, dtype=torch.bfloat16, device=DEV)
    with pytest.raises(W8A8Error, match="16 heads per KV head"):
        attn.decode(q32, kd, vd)
    o = torch.empty(8, 256, dtype=torch.bfloat16, device=DEV)
    ws = torch.empty(64, dtype=torch.uint8, device=DEV)
    with pytest.raises(W8A8Error, match="workspace"):
        call("w8a8_attention_decode_bf16", qd.data_ptr(), 256, kd.data_ptr(), 100 * 256, 256, vd.data_ptr(),
             100 * 256, 256, 8, 1, 100, 256, 99, 0, 1.0, o.data_ptr(), 256, None, ws.data_ptr(), 64,
             torch.cuda.current_stream().cuda_stream)
