"""Pins the oracle's restatement of the fused kernels between the GEMMs (pipeline.py:43-127).

Golden vectors come from eager torch ops in the expressions of pipeline.py
(tests/golden/make_golden.py); known answers fix what the golden values leave open: the head
layout of k_qkv, the row layout of k_attn_out, the rotation's direction and pairing, and
exact special cases of the norms.
"""
import os

import numpy as np
import pytest

from helpers import assert_bf16_close, f32

import oracle.oracle as orc

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "w8a8_golden.npz")
EPS = 1e-6


@pytest.fixture(scope="module")
def gold():
    return np.load(GOLDEN)


def assert_quant_close(q, s, q_ref, s_ref, what, min_exact=0.95):
    """int8 rows of values that may differ by one bf16 rounding (reduction order of a norm
    upstream): scales within one bf16 ulp of the row maximum, codes within 1, mostly equal."""
    s, s_ref = np.asarray(s, np.float64), np.asarray(s_ref, np.float64)
    assert (np.abs(s - s_ref) <= s_ref * 2.0 ** -7).all(), f"{what}: scales differ"
    d = np.abs(q.astype(np.int32) - q_ref.astype(np.int32))
    assert d.max() <= 1, f"{what}: int8 codes differ by {d.max()}"
    assert (d == 0).mean() >= min_exact, f"{what}: only {(d == 0).mean():.3f} of the codes agree"


# ---- rope (pipeline.py:60-63) ----------------------------------------------------------------

def test_rope_golden(gold):
    out = orc.rope(gold["rope_x"], gold["rope_cos"], gold["rope_sin"])
    # both products and the sum are single roundings of exact fp32 values: bit-exact
    assert np.array_equal(out, gold["rope_out"])


def test_rope_known_answers():
    rng = np.random.default_rng(11)
    R, D = 4, 16
    x = orc.bf16_bits(rng.standard_normal((R, D)).astype(np.float32))
    one = orc.bf16_bits(np.ones((R, D), np.float32))
    zero = orc.bf16_bits(np.zeros((R, D), np.float32))
    # angle 0: identity
    assert np.array_equal(orc.rope(x, one, zero), x)
    # angle pi/2: rot(x) = cat(-x[D/2:], x[:D/2]), element d paired with d + D/2
    xf = f32(x)
    rot = np.concatenate([-xf[:, D // 2:], xf[:, :D // 2]], axis=1)
    r1 = orc.rope(x, zero, one)
    assert np.array_equal(f32(r1), rot)
    # twice pi/2 is pi: -x
    assert np.array_equal(f32(orc.rope(r1, zero, one)), -xf)
    # the rotation preserves each pair's norm up to bf16 rounding
    c = orc.bf16_bits(np.full((R, D), np.cos(0.3), np.float32))
    s = orc.bf16_bits(np.full((R, D), np.sin(0.3), np.float32))
    r = f32(orc.rope(x, c, s))
    n0 = xf[:, :D // 2] ** 2 + xf[:, D // 2:] ** 2
    n1 = r[:, :D // 2] ** 2 + r[:, D // 2:] ** 2
    assert np.allclose(n0, n1, rtol=2e-2, atol=1e-3)


# ---- rms to bf16 (pipeline.py:43-46) ---------------------------------------------------------

def test_rms_bf16_golden(gold):
    for w, key in ((gold["rmsb_w"], "rmsb_out"), (None, "rmsb_out_now")):
        out = orc.rms_bf16(gold["rmsb_x"], w, EPS)
        assert_bf16_close(f32(out), f32(gold[key]), what=key)
        assert (out == gold[key]).mean() > 0.97


def test_rms_bf16_known_answers():
    # a +-c pattern has mean square c^2: with eps = 0 the result is exactly +-1 (times w)
    x = orc.bf16_bits(np.tile(np.array([3.0, -3.0], np.float32), (2, 8)))
    assert np.array_equal(f32(orc.rms_bf16(x, None, 0.0)), np.tile(np.array([1.0, -1.0], np.float32), (2, 8)))
    w = orc.bf16_bits(np.arange(16, dtype=np.float32) / 4)
    assert np.array_equal(f32(orc.rms_bf16(x, w, 0.0))[0], np.tile([1.0, -1.0], 8) * np.arange(16) / 4)
    # eps enters inside the root: a zero row stays zero, a one-hot row of D gives sqrt(D)
    z = orc.bf16_bits(np.zeros((1, 16), np.float32))
    assert not f32(orc.rms_bf16(z, None, EPS)).any()
    oh = np.zeros((1, 16), np.float32)
    oh[0, 5] = 2.0
    assert f32(orc.rms_bf16(orc.bf16_bits(oh), None, 0.0))[0, 5] == 4.0


# ---- k_in (pipeline.py:66-69) ----------------------------------------------------------------

def test_k_in_golden(gold):
    q, s = orc.k_in(gold["kin_h"], gold["kin_w"], EPS)
    assert_quant_close(q, s, gold["kin_q"], gold["kin_s"], "k_in")


# ---- k_qkv (pipeline.py:72-85) ---------------------------------------------------------------

def test_k_qkv_golden(gold):
    args = [gold[f"kqkv_{n}"] for n in ("acc", "sx", "sw", "cos", "sin", "qw", "kw")]
    q, k, v = orc.k_qkv(*args, EPS, 2, 1, 16, False)
    for got, key in ((q, "kqkv_q"), (k, "kqkv_k"), (v, "kqkv_v")):
        assert got.shape == gold[key].shape
        assert_bf16_close(f32(got), f32(gold[key]), what=key)
        assert (got == gold[key]).mean() > 0.95
    qs, ks, vs = orc.k_qkv(*args, EPS, 2, 1, 16, True)
    assert np.array_equal(qs, q) and ks is qs and vs is qs


def _one_hot_heads(T, H, KV, D):
    """acc whose head j (q heads, then k, then v) holds a single 1 at position j of the head."""
    acc = np.zeros((T, (H + 2 * KV) * D), np.int32)
    for j in range(H + 2 * KV):
        acc[:, j * D + j] = 1
    return acc


def test_k_qkv_head_layout_and_rotation():
    T, H, KV, D = 3, 2, 1, 16
    acc = _one_hot_heads(T, H, KV, D)
    ones = np.ones(T, np.float32)
    sw = np.ones(acc.shape[1], np.float32)
    w = orc.bf16_bits(np.ones(D, np.float32))
    c1 = orc.bf16_bits(np.ones((T, D), np.float32))
    s0 = orc.bf16_bits(np.zeros((T, D), np.float32))
    q, k, v = orc.k_qkv(acc, ones, sw, c1, s0, w, w, 0.0, H, KV, D, False)
    assert q.shape == (H, T, D) and k.shape == (KV, T, D) and v.shape == (KV, T, D)
    root = np.float32(np.sqrt(D))  # rms of a one-hot head
    for j, (arr, i) in enumerate([(q, 0), (q, 1), (k, 0), (v, 0)]):
        want = np.zeros((T, D), np.float32)
        want[:, j] = root
        assert np.array_equal(f32(arr[i]), want), f"head slot {j}"
    # a quarter turn moves element j < D/2 to j + D/2 in q and k, and leaves v alone
    q, k, v = orc.k_qkv(acc, ones, sw, s0, c1, w, w, 0.0, H, KV, D, False)
    for j, arr in ((0, q[0]), (1, q[1]), (2, k[0])):
        want = np.zeros((T, D), np.float32)
        want[:, j + D // 2] = root
        assert np.array_equal(f32(arr), want)
    want = np.zeros((T, D), np.float32)
    want[:, 3] = root
    assert np.array_equal(f32(v[0]), want)


# ---- k_attn_out (pipeline.py:88-92) ----------------------------------------------------------

def test_k_attn_out_golden(gold):
    q, s = orc.k_attn_out(gold["kao_o"])
    assert np.array_equal(q, gold["kao_q"]) and np.array_equal(s, gold["kao_s"])


def test_k_attn_out_row_layout():
    H, T, D = 3, 4, 8
    o = np.zeros((H, T, D), np.float32)
    for h in range(H):
        for t in range(T):
            o[h, t] = (h + 1) * (t + 1)
    q, s = orc.k_attn_out(orc.bf16_bits(o))
    # row t is [head 0 | head 1 | head 2] of token t; the largest head maps to 127
    for t in range(T):
        assert s[t] == np.float32(np.float32(3 * (t + 1)) / np.float32(127))
        assert q[t].tolist() == [42] * D + [85] * D + [127] * D


# ---- k_post_attn / k_post_ff (pipeline.py:95-99, 110-114) ------------------------------------

def test_k_post_attn_golden(gold):
    a = [gold[f"kpa_{n}"] for n in ("acc", "sx", "sw", "res", "w1", "w2")]
    h, q, s = orc.k_post_attn(*a, EPS)
    assert_bf16_close(f32(h), f32(gold["kpa_h"]), what="k_post_attn h")
    assert (h == gold["kpa_h"]).mean() > 0.97
    assert_quant_close(q, s, gold["kpa_q"], gold["kpa_s"], "k_post_attn q")


def test_k_post_ff_golden(gold):
    a = [gold[f"kpa_{n}"] for n in ("acc", "sx", "sw", "res", "w1")]
    h, q, s = orc.k_post_ff(*a, EPS)
    assert_bf16_close(f32(h), f32(gold["kpa_h"]), what="k_post_ff h")
    assert_quant_close(q, s, gold["kpf_q"], gold["kpf_s"], "k_post_ff q")


def test_k_post_attn_second_norm_is_applied():
    # with a second-norm weight of 2 the int8 codes match those of weight 1 (quant is scale
    # invariant) but the scales double: the norm feeds the quant, not h
    rng = np.random.default_rng(12)
    T, N = 4, 32
    acc = rng.integers(-2 ** 20, 2 ** 20, (T, N)).astype(np.int32)
    sx = np.full(T, 1e-3, np.float32)
    sw = np.full(N, 1e-2, np.float32)
    res = orc.bf16_bits(rng.standard_normal((T, N)).astype(np.float32))
    w1 = orc.bf16_bits(np.ones(N, np.float32))
    h1, q1, s1 = orc.k_post_attn(acc, sx, sw, res, w1, w1, EPS)
    h2, q2, s2 = orc.k_post_attn(acc, sx, sw, res, w1, orc.bf16_bits(np.full(N, 2.0, np.float32)), EPS)
    assert np.array_equal(h1, h2) and np.array_equal(q1, q2) and np.array_equal(s2, 2 * s1)
    # and the rms of h has unit mean square, so the quant scale is max|rms(h)| / 127, not max|h| / 127
    hf = f32(h1).astype(np.float64)
    r = hf / np.sqrt((hf ** 2).mean(1, keepdims=True) + EPS)
    assert np.allclose(s1, np.abs(r).max(1) / 127, rtol=1e-2)


# ---- k_gelu / k_ple_gate (pipeline.py:102-107, 117-121) --------------------------------------

def test_k_gelu_golden(gold):
    q, s = orc.k_gelu(gold["kg_acc"], gold["kg_sx"], gold["kg_sw"], 32)
    assert_quant_close(q, s, gold["kg_q"], gold["kg_s"], "k_gelu")


def test_k_ple_gate_golden(gold):
    q, s = orc.k_ple_gate(gold["kpg_acc"], gold["kpg_sx"], gold["kpg_sw"], gold["kpg_ple"])
    assert_quant_close(q, s, gold["kpg_q"], gold["kpg_s"], "k_ple_gate")


def test_k_ple_gate_known_answers():
    # gelu(0) = 0 whatever ple holds; ple = 0 zeroes the row (scale floor 1e-8/127)
    T, N = 2, 16
    acc = np.zeros((T, N), np.int32)
    acc[0] = 1000
    ple = orc.bf16_bits(np.vstack([np.zeros(N, np.float32), np.full(N, 5.0, np.float32)]))
    q, s = orc.k_ple_gate(acc, np.full(T, 1e-2, np.float32), np.ones(N, np.float32), ple)
    assert not q.any()
    assert s[0] == s[1] == np.float32(np.float32(1e-8) / np.float32(127))


# ---- k_ple_out (pipeline.py:124-127) ---------------------------------------------------------

def test_k_ple_out_golden(gold):
    a = [gold[f"kpo_{n}"] for n in ("acc", "sx", "sw", "h", "w")]
    out = orc.k_ple_out(*a, gold["kpo_scalar"][0], EPS)
    assert_bf16_close(f32(out), f32(gold["kpo_out"]), what="k_ple_out")
    assert (out == gold["kpo_out"]).mean() > 0.97


def test_k_ple_out_scalar():
    rng = np.random.default_rng(13)
    T, N = 3, 32
    acc = rng.integers(-2 ** 20, 2 ** 20, (T, N)).astype(np.int32)
    sx, sw = np.full(T, 1e-3, np.float32), np.full(N, 1e-2, np.float32)
    h = orc.bf16_bits(rng.standard_normal((T, N)).astype(np.float32))
    w = orc.bf16_bits(np.ones(N, np.float32))
    one = orc.bf16_bits(np.array([1.0], np.float32))[0]
    two = orc.bf16_bits(np.array([2.0], np.float32))[0]
    base = orc.k_ple_out(acc, sx, sw, h, w, one, EPS)
    # scalar 1 is the residual with the norm alone; scalar 2 doubles it exactly
    assert np.array_equal(base, orc.rms_residual(orc.dequant(acc, sx, sw), h, w, EPS))
    assert np.array_equal(f32(orc.k_ple_out(acc, sx, sw, h, w, two, EPS)), 2 * f32(base))
