"""Pins the oracle's attention (pipeline.py:140-180, local_attn.py:28-38, 71-107).

The oracle loops over each query's visible key range in double precision.  It is checked against
an independent library routine -- torch's scaled_dot_product_attention in float64, heads
repeated for grouped-query attention, given the boolean mask built from the reference's own
window-mask formula (key >= 0, key <= query, query - key < W; local_attn.py:28-38) -- and against
closed forms that a wrong index, window bound or head mapping would break: window 1 returns the
query's own value row, a zero query averages the visible value rows, and the logsumexp of a zero
query is log(number of visible keys).
"""
import numpy as np
import pytest
import torch
import torch.nn.functional as F

import oracle.oracle as orc


def bf16(x):
    return orc.bf16_bits(np.asarray(x, np.float32))


def f32(b):
    return orc.bits_to_f32(b)


def inputs(H, KV, Tq, Tk, D, seed, scale=1.0):
    rng = np.random.default_rng(seed)
    q = bf16(rng.standard_normal((H, Tq, D)) * scale)
    k = bf16(rng.standard_normal((KV, Tk, D)) * scale)
    v = bf16(rng.standard_normal((KV, Tk, D)))
    return q, k, v


def reference_mask(Tq, Tk, q_start, window):
    """local_attn.py:28-38 / pipeline.py:176: key >= 0, key <= query, query - key < W."""
    qp = q_start + torch.arange(Tq)[:, None]
    kp = torch.arange(Tk)[None, :]
    m = (kp >= 0) & (kp <= qp)
    if window:
        m &= (qp - kp) < window
    return m


def torch64(q, k, v, q_start, window, scale):
    H, KV = q.shape[0], k.shape[0]
    qt = torch.from_numpy(f32(q).astype(np.float64))
    kt = torch.from_numpy(f32(k).astype(np.float64)).repeat_interleave(H // KV, 0)
    vt = torch.from_numpy(f32(v).astype(np.float64)).repeat_interleave(H // KV, 0)
    mask = reference_mask(q.shape[1], k.shape[1], q_start, window)
    o = F.scaled_dot_product_attention(qt[None], kt[None], vt[None], attn_mask=mask, scale=scale)[0]
    s = (qt @ kt.transpose(1, 2)) * scale
    lse = torch.logsumexp(s.masked_fill(~mask, float("-inf")), -1)
    return o.numpy(), lse.numpy()


CASES = [
    # H, KV, Tq, Tk, D, q_start, window, scale
    (4, 2, 17, 17, 16, 0, 0, 1.0),
    (4, 2, 9, 30, 16, 21, 0, 1.0),      # a micro-batch after earlier keys (full_attention's merge)
    (8, 1, 24, 40, 32, 16, 5, 1.0),     # sliding window, queries past the first keys
    (8, 1, 33, 33, 32, 0, 8, 0.25),
    (6, 3, 12, 50, 8, 38, 64, 1.0),     # window wider than the keys
    (2, 2, 5, 12, 16, 7, 1, 1.0),       # window 1
]


@pytest.mark.parametrize("H,KV,Tq,Tk,D,q_start,window,scale", CASES)
def test_attention_vs_torch_float64(H, KV, Tq, Tk, D, q_start, window, scale):
    q, k, v = inputs(H, KV, Tq, Tk, D, seed=Tq * 7 + D)
    out, bud, lse = orc.attention(q, k, v, q_start, window, scale, budget=True, lse=True)
    o64, lse64 = torch64(q, k, v, q_start, window, scale)
    ref = bf16(o64)
    # Both sides compute in double; their bf16 roundings agree except at a rounding tie.
    diff = np.abs(f32(out) - f32(ref))
    assert (out != ref).mean() < 1e-3 and diff.max() <= 2.0 ** -7 * np.abs(f32(ref)).max()
    assert np.allclose(lse, lse64, rtol=1e-12, atol=1e-12)
    # budget = sum_j p_j |v_j| >= |o| (fp32 rounding of both aside)
    assert (bud >= np.abs(o64) * (1 - 1e-6) - 1e-30).all()


def test_window_one_is_own_value():
    q, k, v = inputs(4, 1, 10, 25, 16, seed=3)
    out = orc.attention(q, k, v, q_start=15, window=1)
    assert np.array_equal(out, np.repeat(v[:, 15:25][None, 0], 4, axis=0))


def test_zero_query_averages_visible_values():
    H, KV, Tq, Tk, D, q_start, W = 4, 2, 8, 20, 16, 12, 6
    _, k, v = inputs(H, KV, Tq, Tk, D, seed=5)
    q = np.zeros((H, Tq, D), np.uint16)
    out, lse = orc.attention(q, k, v, q_start, W, lse=True)
    vf = f32(v).astype(np.float64)
    for h in range(H):
        g = h // (H // KV)
        for i in range(Tq):
            p = q_start + i
            lo = max(0, p - W + 1)
            mean = vf[g, lo:p + 1].mean(0)
            # equal weights 1/n: the bf16 of the mean, up to the double rounding of 1/n where the
            # mean cancels to ~0
            assert np.allclose(f32(out[h, i]), f32(bf16(mean)), rtol=0, atol=1e-12) or \
                np.array_equal(out[h, i], bf16(mean))
            assert (np.abs(f32(out[h, i]) - mean) <= np.maximum(np.abs(mean) * 2.0 ** -8, 1e-12)).all()
            assert lse[h, i] == pytest.approx(np.log(p + 1 - lo), rel=1e-12)


def test_grouped_heads_use_their_kv_head():
    """Heads 0-1 read KV head 0 and heads 2-3 KV head 1: swapping the KV heads swaps the halves."""
    q, k, v = inputs(4, 2, 6, 6, 16, seed=9)
    a = orc.attention(q, k, v)
    b = orc.attention(q[[2, 3, 0, 1]], k[::-1].copy(), v[::-1].copy())
    assert np.array_equal(a, b[[2, 3, 0, 1]])


def test_causal_ignores_future_keys():
    q, k, v = inputs(2, 1, 5, 12, 16, seed=11)
    a = orc.attention(q, k, v, q_start=3)
    k2, v2 = k.copy(), v.copy()
    k2[:, 8:] = bf16(np.full((1, 4, 16), 7.0))   # positions past the last query (7)
    v2[:, 8:] = bf16(np.full((1, 4, 16), -3.0))
    assert np.array_equal(a, orc.attention(q, k2, v2, q_start=3))
