"""Pins the C oracle (oracle/w8a8_oracle.c) before anything is checked against it.

Each oracle function is checked three ways, chosen so that a plausible slip (a dropped
term, a wrong rounding mode, a transposed operand, a wrong scale order) fails one of them:
  * golden vectors written by torch's CPU ops, the library the reference runs
    (tests/golden/make_golden.py);
  * known answers worked out by hand (ties to even, zero rows, one-hot rows, extremes);
  * closed forms / invariants on seeded inputs (linearity, transposition, exact sums).
"""
import os

import numpy as np
import pytest
import torch

from helpers import assert_bf16_close, bf16_close, f32, from_bits, to_bits

import oracle.oracle as orc

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "w8a8_golden.npz")


@pytest.fixture(scope="module")
def gold():
    return np.load(GOLDEN)


# ---- int_mm (npu_kernels.py:40-56) ---------------------------------------------------------

@pytest.mark.parametrize("name", ["mm_a", "mm_b", "mm_c"])
def test_int_mm_golden(gold, name):
    c = orc.int_mm(gold[f"{name}_a"], gold[f"{name}_b"])
    assert np.array_equal(c, gold[f"{name}_c"])


def test_int_mm_known_answers():
    K = 64
    a = np.full((3, K), -128, np.int8)
    b = np.full((K, 5), -128, np.int8)
    assert (orc.int_mm(a, b) == 128 * 128 * K).all()
    a[1] = 127
    assert (orc.int_mm(a, b)[1] == -127 * 128 * K).all()
    # one-hot rows of A select rows of B
    rng = np.random.default_rng(0)
    B = rng.integers(-128, 128, (K, 7), dtype=np.int8)
    A = np.zeros((K, K), np.int8)
    A[np.arange(K), np.arange(K)] = 1
    assert np.array_equal(orc.int_mm(A, B), B.astype(np.int32))
    # the largest |acc| the workloads reach: K = 12288, all -128
    K = 12288
    c = orc.int_mm(np.full((1, K), -128, np.int8), np.full((K, 1), -128, np.int8))
    assert c[0, 0] == 128 * 128 * K


def test_int_mm_vs_torch_and_transpose():
    rng = np.random.default_rng(1)
    a = rng.integers(-128, 128, (33, 320), dtype=np.int8)
    b = rng.integers(-128, 128, (320, 40), dtype=np.int8)
    ref = torch._int_mm(torch.from_numpy(a), torch.from_numpy(b)).numpy()
    assert np.array_equal(orc.int_mm(a, b), ref)
    # the [N, K] form is the same product with the weight transposed
    assert np.array_equal(orc.int_mm_nk(a, np.ascontiguousarray(b.T)), ref)


# ---- quant_rows (pipeline.py:49-52) --------------------------------------------------------

def test_quant_golden(gold):
    q, s = orc.quant_rows(gold["quant_x"], "bf16")
    assert np.array_equal(s, gold["quant_s"])
    assert np.array_equal(q, gold["quant_q"])
    q, s = orc.quant_rows(gold["wquant_x"], "f32")
    assert np.array_equal(s, gold["wquant_s"])
    assert np.array_equal(q, gold["wquant_q"])


def test_quant_known_answers():
    # absmax 127 -> scale exactly 1.0; halves round to even; clamp never needed
    row = np.array([127.0, 63.5, 0.5, -127.0, 1.5, 2.5, -2.5, -0.5, 3.0, 0.0], np.float32)
    q, s = orc.quant_rows(orc.bf16_bits(row[None]), "bf16")
    assert s[0] == np.float32(1.0)
    assert q[0].tolist() == [127, 64, 0, -127, 2, 2, -2, 0, 3, 0]
    # zero row: scale is the 1e-8 floor / 127 in fp32, every q is 0
    q, s = orc.quant_rows(np.zeros((1, 16), np.float32), "f32")
    assert s[0] == np.float32(np.float32(1e-8) / np.float32(127)) and not q.any()
    # the absmax element always maps to +-127 exactly
    rng = np.random.default_rng(2)
    x = rng.standard_normal((50, 33)).astype(np.float32)
    q, s = orc.quant_rows(x, "f32")
    am = np.abs(x).argmax(1)
    assert (np.abs(q[np.arange(50), am]) == 127).all()
    assert (np.abs(q) <= 127).all()


def nan_inf_rows():
    """bf16 rows holding NaN and +-Inf next to ordinary and zero rows."""
    nan, inf = float("nan"), float("inf")
    x = torch.randn(6, 48, generator=torch.Generator().manual_seed(3))
    x[1, 5] = nan
    x[2, 7] = inf
    x[3, 0] = -inf
    x[4] = 0.0
    x[5, 9], x[5, 30] = inf, nan
    return x.to(torch.bfloat16)


def test_quant_nan_and_inf_rows_follow_torch():
    """torch.amax propagates NaN (pipeline.py:51): a row holding NaN gets a NaN scale, a row
    holding +-Inf an Inf scale, and both quantise to 0 everywhere (x / NaN and Inf / Inf are NaN,
    which torch's float -> int8 conversion makes 0; finite / Inf is 0).  Checked against the
    reference expression run by torch itself."""
    x = nan_inf_rows()
    xf = x.float()
    s_t = xf.abs().amax(dim=-1, keepdim=True).clamp(min=1e-8) / 127
    q_t = torch.round(xf / s_t).clamp(-127, 127).to(torch.int8)
    q, s = orc.quant_rows(to_bits(x), "bf16")
    s_ref = s_t[:, 0].numpy()
    assert np.array_equal(np.isnan(s), np.isnan(s_ref)) and np.isnan(s[[1, 5]]).all()
    fin = ~np.isnan(s_ref)
    assert np.array_equal(s[fin], s_ref[fin]) and np.isinf(s[[2, 3]]).all()
    assert np.array_equal(q, q_t.numpy())
    assert not q[1:6].any() and q[0].any()


# ---- dequant (pipeline.py:55-57) -----------------------------------------------------------

def test_dequant_golden(gold):
    y = orc.dequant(gold["deq_acc"], gold["deq_sx"], gold["deq_sw"])
    assert np.array_equal(y, gold["deq_y"])


def test_dequant_known_answers():
    acc = np.array([[2 ** 24 + 1, -(2 ** 24 + 3), 7, 0]], np.int32)
    y = f32(orc.dequant(acc, np.ones(1, np.float32), np.ones(4, np.float32)))
    # int32 -> fp32 rounds to nearest even (2^24+1 -> 2^24, 2^24+3 -> 2^24+4), then to bf16
    # (8 significant bits: 2^24+4 -> 2^24)
    assert y[0].tolist() == [2.0 ** 24, -(2.0 ** 24), 7.0, 0.0]
    # scale order: (acc * sx) * sw, not acc * (sx * sw); the two differ at this point
    acc = np.array([[3]], np.int32)
    sx, sw = np.array([1.1], np.float32), np.array([0.7], np.float32)
    ref = np.float32(np.float32(3.0) * sx[0]) * sw[0]
    assert orc.dequant(acc, sx, sw)[0, 0] == orc.bf16_bits(np.array([ref], np.float32))[0]


# ---- gelu_tanh(gate) * up (pipeline.py:106) ------------------------------------------------

def test_gelu_golden(gold):
    a = orc.gelu_mul(gold["gelu_y"])
    assert_bf16_close(f32(a), f32(gold["gelu_out"]), what="gelu_mul vs torch")
    # eager torch rounds the same way almost everywhere
    assert (a == gold["gelu_out"]).mean() > 0.98


def test_gelu_known_answers():
    y = orc.bf16_bits(np.array([[0.0, 8.0, -8.0, 1.0, 2.0, 2.0, 2.0, 3.0]], np.float32))
    a = f32(orc.gelu_mul(y))[0]
    assert a[0] == 0.0                      # gelu(0) = 0
    assert a[1] == 16.0                     # gelu(8) = 8 to bf16 precision, times 2
    assert a[2] == 0.0 or abs(a[2]) < 1e-6  # gelu(-8) ~ -1e-14 -> times 2
    assert abs(a[3] - 0.8412 * 3.0) < 0.02  # gelu_tanh(1) = 0.84119...


# ---- res + rms(y) * w (pipeline.py:43-46, 113) ---------------------------------------------

def test_rms_golden(gold):
    h = orc.rms_residual(gold["rms_y"], gold["rms_res"], gold["rms_w"], float(gold["rms_eps"]))
    assert_bf16_close(f32(h), f32(gold["rms_h"]), what="rms_residual vs torch")


def test_rms_known_answers():
    # constant rows: rms(c) = c / sqrt(c^2 + eps); w = 2 doubles it; res adds
    y = orc.bf16_bits(np.full((2, 64), 3.0, np.float32))
    res = orc.bf16_bits(np.array([[1.0] * 64, [-2.0] * 64], np.float32))
    w = orc.bf16_bits(np.full(64, 2.0, np.float32))
    h = f32(orc.rms_residual(y, res, w, 1e-6))
    assert np.allclose(h[0], 3.0) and np.allclose(h[1], 0.0)
    # without a weight (pipeline.py:46): a +-1 pattern has rms 1
    y = orc.bf16_bits(np.tile(np.array([1.0, -1.0], np.float32), (1, 32)))
    h = f32(orc.rms_residual(y, orc.bf16_bits(np.zeros((1, 64), np.float32)), None, 0.0))
    assert np.array_equal(h[0], np.tile(np.array([1.0, -1.0], np.float32), 32))


def test_add_residual():
    rng = np.random.default_rng(3)
    y = orc.bf16_bits(rng.standard_normal((4, 32)).astype(np.float32))
    r = orc.bf16_bits(rng.standard_normal((4, 32)).astype(np.float32))
    ref = (from_bits(y).float() + from_bits(r).float()).to(torch.bfloat16)
    assert np.array_equal(orc.add_residual(y, r), to_bits(ref))


# ---- weight-only int8 GEMV (gemma_npu.py:155-156) ------------------------------------------

@pytest.mark.parametrize("name", ["gemv_a", "gemv_b", "gemv_c"])
def test_gemv_golden(gold, name):
    x, w = gold[f"{name}_x"], gold[f"{name}_w"]
    yb = orc.gemv(x, w, gold[f"{name}_sb"], "bf16")
    assert_bf16_close(f32(yb), f32(gold[f"{name}_yb"]), what=f"{name} bf16 scales")
    yf = orc.gemv(x, w, gold[f"{name}_sf"], "f32")
    assert_bf16_close(f32(yf), f32(gold[f"{name}_yf"]), what=f"{name} fp32 scales")


def test_gemv_exact_on_integer_activations():
    # integer-valued bf16 activations make every partial sum exact in fp32, so the GEMV must
    # equal bf16(int_mm * s) exactly
    rng = np.random.default_rng(4)
    xi = rng.integers(-8, 9, (3, 192)).astype(np.int8)
    w = rng.integers(-127, 128, (24, 192), dtype=np.int8)
    s = (rng.random(24) * 0.01 + 0.005).astype(np.float32)
    y = orc.gemv(orc.bf16_bits(xi.astype(np.float32)), w, s, "f32")
    acc = orc.int_mm_nk(xi, w).astype(np.float32)
    assert np.array_equal(y, orc.bf16_bits(acc * s[None, :]))


def test_linear_composition():
    """quant -> int_mm -> dequant, composed as NPUGemm.matmul does (gemma_npu.py:127-150),
    against the same chain in torch ops."""
    rng = np.random.default_rng(5)
    x = orc.bf16_bits((rng.standard_normal((9, 128)) * 2).astype(np.float32))
    w = rng.integers(-127, 128, (40, 128), dtype=np.int8)
    sw = (rng.random(40) * 0.015 + 0.005).astype(np.float32)
    out, acc, sx = orc.linear_bf16(x, w, sw)
    xf = from_bits(x).float()
    s = xf.abs().amax(-1).clamp(min=1e-8) / 127
    q = torch.round(xf / s[:, None]).clamp(-127, 127).to(torch.int8)
    ref_acc = torch._int_mm(q, torch.from_numpy(w).t().contiguous())
    ref = (ref_acc.float() * s[:, None] * torch.from_numpy(sw)[None, :]).to(torch.bfloat16)
    assert np.array_equal(acc, ref_acc.numpy())
    assert np.array_equal(out, to_bits(ref))
    assert bf16_close(f32(out), f32(to_bits(ref))).all()
