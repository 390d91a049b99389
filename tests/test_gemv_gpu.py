"""GPU parity of the decode GEMV (torch._weight_int8pack_mm semantics, gemma_npu.py:155-172).

bf16 results agree with the oracle and with torch's CPU op within
max(1e-2 |ref|, 2 ulp, 4 * 2^-24 * sum_k |x w| * |s|): the last term is the fp32 accumulation
error bound, which only matters where the K-long sum cancels to near zero (there the oracle's
sequential sum and torch's own vectorised sum disagree with each other by the same amount).
With integer-valued activations every partial sum is exact, so the result must be
bf16(int32 product * s) bit for bit."""
import os

import numpy as np
import pytest
import torch

from helpers import assert_bf16_close, dot_error_bound, f32, from_bits, to_bits

import oracle.oracle as orc
from w8a8 import ops, workloads

pytestmark = pytest.mark.gpu
DEV = "cuda"
GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "w8a8_golden.npz")


@pytest.mark.parametrize("name", ["gemv_a", "gemv_b", "gemv_c"])
def test_gemv_golden(name):
    d = np.load(GOLDEN)
    x = from_bits(d[f"{name}_x"]).to(DEV)
    w = torch.from_numpy(d[f"{name}_w"]).to(DEV)
    extra = dot_error_bound(f32(d[f"{name}_x"]), d[f"{name}_w"], d[f"{name}_sf"])
    yb = ops.gemv_bf16(x, w, from_bits(d[f"{name}_sb"]).to(DEV))
    assert_bf16_close(f32(to_bits(yb)), f32(d[f"{name}_yb"]), what=f"{name} bf16 scales vs torch", extra=extra)
    yf = ops.gemv_bf16(x, w, torch.from_numpy(d[f"{name}_sf"]).to(DEV))
    assert_bf16_close(f32(to_bits(yf)), f32(d[f"{name}_yf"]), what=f"{name} fp32 scales vs torch", extra=extra)


@pytest.mark.parametrize("M", [1, 4, 16])
@pytest.mark.parametrize("K,N", [(1536, 2560), (2048, 1536), (1536, 12288), (6144, 1536), (80, 40)])
def test_gemv_layer_shapes(M, K, N):
    x = workloads.activations(M, K, seed=M * 31 + K, outliers=False)
    w, sw = workloads.weights(N, K, seed=N + 1)
    s = sw.to(torch.bfloat16)
    y = ops.gemv_bf16(x.to(DEV), w.to(DEV), s.to(DEV))
    extra = dot_error_bound(x.float().numpy(), w.numpy(), s.float().numpy())
    ref = orc.gemv(to_bits(x), w.numpy(), to_bits(s), "bf16")
    got = f32(to_bits(y))
    assert_bf16_close(got, f32(ref), what=f"gemv M{M} K{K} N{N} vs oracle", extra=extra)
    ref_t = torch._weight_int8pack_mm(x, w, s)
    assert_bf16_close(got, f32(to_bits(ref_t)), what=f"gemv M{M} K{K} N{N} vs torch", extra=extra)
    # outside the cancellation zone the plain bf16 bar holds for almost every element
    assert (got == f32(ref)).mean() > 0.97


def test_gemv_exact_on_integer_activations():
    g = torch.Generator().manual_seed(3)
    xi = torch.randint(-8, 9, (5, 1536), generator=g)
    w = torch.randint(-128, 128, (1000, 1536), generator=g, dtype=torch.int8)
    s = torch.rand(1000, generator=g) * 0.01 + 0.005
    y = ops.gemv_bf16(xi.to(torch.bfloat16).to(DEV), w.to(DEV), s.to(DEV))
    acc = (xi.long() @ w.t().long()).float()  # |acc| < 2^24: exact in fp32
    assert torch.equal(y.cpu(), (acc * s[None, :]).to(torch.bfloat16))


def test_gemv_lm_head_m1():
    """The LM head at decode (K=1536, N=262144, M=1) against torch's CPU op."""
    K, N = workloads.LM_HEAD
    x = workloads.activations(1, K, seed=77, outliers=False)
    w, sw = workloads.weights(N, K, seed=78)
    s = sw.to(torch.bfloat16)
    y = ops.gemv_bf16(x.to(DEV), w.to(DEV), s.to(DEV))
    ref = torch._weight_int8pack_mm(x, w, s)
    extra = dot_error_bound(x.float().numpy(), w.numpy(), s.float().numpy())
    assert_bf16_close(f32(to_bits(y)), f32(to_bits(ref)), what="lm head", extra=extra)


def test_gemv_lm_head_m16():
    """The LM head with 16 decode rows (K=1536, N=262144, M=16; BASELINE's largest GEMV row count)
    on the packed weight, N(0,1) activations: every element against torch's CPU op with bf16
    scales (the reference's decode copy, gemma_npu.py:82), and a 4096-column sample against the
    oracle with fp32 scales."""
    K, N = workloads.LM_HEAD
    M = 16
    x = workloads.activations(M, K, seed=79, outliers=False)
    w, sw = workloads.weights(N, K, seed=80)
    s = sw.to(torch.bfloat16)
    wd = w.to(DEV)
    pw = ops.pack_gemv_weight(wd)
    y = ops.gemv_bf16(x.to(DEV), pw, s.to(DEV))
    ref = torch._weight_int8pack_mm(x, w, s)
    # the fp32 accumulation allowance of dot_error_bound, from float64 products on the GPU
    # (|x| w sums are far below 2^53, so the bound itself is exact)
    extra = ((4.0 * 2.0 ** -24) * (x.to(DEV).double().abs() @ wd.double().abs().t())
             * s.to(DEV).double().abs()[None, :]).float().cpu().numpy()
    got = f32(to_bits(y))
    assert_bf16_close(got, f32(to_bits(ref)), what="lm head M16 vs torch", extra=extra)
    assert (got == f32(to_bits(ref))).mean() > 0.97
    cols = torch.randperm(N, generator=torch.Generator().manual_seed(81))[:4096].sort().values
    yf = ops.gemv_bf16(x.to(DEV), pw, sw.to(DEV))
    wc = w[cols].contiguous()
    ref_o = orc.gemv(to_bits(x), wc.numpy(), sw[cols].numpy(), "f32")
    extra_c = dot_error_bound(x.float().numpy(), wc.numpy(), sw[cols].numpy())
    assert_bf16_close(f32(to_bits(yf))[:, cols.numpy()], f32(ref_o), what="lm head M16 fp32 scales vs oracle",
                      extra=extra_c)


def test_gemv_deterministic():
    x = workloads.activations(4, 6144, seed=1, outliers=False).to(DEV)
    w, sw = workloads.weights(1536, 6144, seed=2)
    w, s = w.to(DEV), sw.to(DEV)
    y0 = ops.gemv_bf16(x, w, s)
    for _ in range(3):
        assert torch.equal(ops.gemv_bf16(x, w, s), y0)


# ---- the GEMV fragment layout (w8a8_pack_gemv_weight) -------------------------------------

def _unpack_gemv(packed, N, K):
    """Row-major int8 [N, K] from the GEMV fragment layout: fragment (t, kb) at
    (t * KB + kb) KiB, byte 16*l + b = W[16t + l%16][64kb + 16(l/16) + b]."""
    KB = (K + 63) // 64
    T = (N + 15) // 16
    f = packed.reshape(T, KB, 4, 16, 16)           # t, kb, l/16, l%16, b
    rows = f.transpose(0, 3, 1, 2, 4).reshape(T * 16, KB * 64)
    return rows[:N, :K], rows


@pytest.mark.parametrize("N,K", [(40, 80), (2560, 1536), (1000, 2064)])
def test_pack_gemv_weight_layout(N, K):
    g = torch.Generator().manual_seed(N + K)
    w = torch.randint(-128, 128, (N, K), generator=g, dtype=torch.int8)
    pw = ops.pack_gemv_weight(w.to(DEV))
    assert pw.data.numel() == lib_bytes(N, K)
    rows, full = _unpack_gemv(pw.data.cpu().numpy(), N, K)
    assert np.array_equal(rows, w.numpy())
    assert not full[N:].any() and not full[:, K:].any()


def lib_bytes(N, K):
    from w8a8 import lib
    return lib().w8a8_gemv_packed_bytes(N, K)


@pytest.mark.parametrize("M", [1, 4, 16])
@pytest.mark.parametrize("K,N", [(1536, 2560), (6144, 1536), (80, 40), (2064, 1000), (1536, 65536)])
def test_gemv_packed_matches_row_major(M, K, N):
    """Same products added in the same order: the packed GEMV equals the row-major one bit for
    bit, and the oracle within the GEMV tolerance."""
    x = workloads.activations(M, K, seed=M * 17 + K, outliers=False)
    w, sw = workloads.weights(N, K, seed=N + 3)
    for s in (sw.to(torch.bfloat16), sw):
        y_rm = ops.gemv_bf16(x.to(DEV), w.to(DEV), s.to(DEV))
        y_pk = ops.gemv_bf16(x.to(DEV), ops.pack_gemv_weight(w.to(DEV)), s.to(DEV))
        assert torch.equal(y_rm, y_pk)
    if N * K <= 4_000_000:
        s = sw.to(torch.bfloat16)
        extra = dot_error_bound(x.float().numpy(), w.numpy(), s.float().numpy())
        ref = orc.gemv(to_bits(x), w.numpy(), to_bits(s), "bf16")
        assert_bf16_close(f32(to_bits(y_pk)), f32(ref), what=f"packed gemv M{M} K{K} N{N}", extra=extra)


def ragged_gemv_shapes():
    """Seeded ragged shapes over every row count the GEMV takes and the few-tile, split-K and
    wide launch forms its picker chooses between."""
    rng = np.random.default_rng(77)
    out = []
    for M in range(1, 17):
        N = int(rng.integers(1, 4000))
        K = int(rng.integers(1, 260)) * 16
        out.append((M, N, K))
    return out + [(1, 1, 16), (16, 17, 6160), (3, 40000, 48)]


@pytest.mark.parametrize("M,N,K", ragged_gemv_shapes())
def test_gemv_packed_ragged_shapes_vs_oracle(M, N, K):
    """Packed and row-major GEMV at ragged N and K (K a multiple of 16), both scale types: equal
    to each other bit for bit and to the oracle within the GEMV tolerance."""
    x = workloads.activations(M, K, seed=M * 101 + K, outliers=False)
    g = torch.Generator().manual_seed(N * 3 + K)
    w = torch.randint(-127, 128, (N, K), generator=g, dtype=torch.int8)
    sf = torch.rand(N, generator=g) * 0.015 + 0.005
    print(f"gemv ragged M={M} N={N} K={K}", flush=True)
    pw = ops.pack_gemv_weight(w.to(DEV))
    for s, kind in ((sf.to(torch.bfloat16), "bf16"), (sf, "f32")):
        y = ops.gemv_bf16(x.to(DEV), pw, s.to(DEV))
        assert torch.equal(y, ops.gemv_bf16(x.to(DEV), w.to(DEV), s.to(DEV)))
        extra = dot_error_bound(x.float().numpy(), w.numpy(), s.float().numpy())
        ref = orc.gemv(to_bits(x), w.numpy(), to_bits(s) if kind == "bf16" else s.numpy(), kind)
        assert_bf16_close(f32(to_bits(y)), f32(ref), what=f"ragged gemv M{M} N{N} K{K} {kind} scales",
                          extra=extra)


def test_gemv_packed_lm_head_exact_on_integer_activations():
    """The LM-head shape (K=1536, N=262144) with integer activations: every partial sum is exact,
    so the packed GEMV must equal bf16(int32 product * s)."""
    g = torch.Generator().manual_seed(11)
    K, N = 1536, 262144
    xi = torch.randint(-4, 5, (4, K), generator=g)
    w = torch.randint(-127, 128, (N, K), generator=g, dtype=torch.int8)
    s = torch.rand(N, generator=g) * 0.01 + 0.005
    wd = w.to(DEV)
    y = ops.gemv_bf16(xi.to(torch.bfloat16).to(DEV), ops.pack_gemv_weight(wd), s.to(DEV))
    acc = (xi.to(DEV).double() @ wd.double().t()).float()  # exact integers, |acc| < 2^24
    ref = (acc * s.to(DEV)[None, :]).to(torch.bfloat16)
    assert torch.equal(y, ref)


@pytest.mark.parametrize("M, K, I", [(1, 1536, 6144), (4, 1536, 12288), (16, 256, 1536), (1, 64, 16)])
def test_gemv_gelu_pair_equals_gemv_then_gelu_mul(M, K, I):
    """The GEMV's GELU-pair epilogue on a [gate; up] stacked weight (the decode MLP) against the
    GEMV writing [gate | up] followed by the row kernel's gelu_mul: bit for bit, bf16 and fp32
    scales, including gate / up values around zero and in GELU's saturated range."""
    dev = torch.device("cuda")
    g = torch.Generator(device=dev).manual_seed(M * 1000 + I)
    x = (torch.randn(M, K, generator=g, device=dev) * 2).to(torch.bfloat16)
    w = torch.randint(-127, 128, (2 * I, K), generator=g, dtype=torch.int8, device=dev)
    pw = ops.pack_gemv_weight(w)
    for s in ((torch.rand(2 * I, generator=g, device=dev) * 0.01).to(torch.bfloat16),
              torch.rand(2 * I, generator=g, device=dev) * 0.01):
        want = ops.gelu_mul_bf16(ops.gemv_bf16(x, pw, s))
        got = ops.gemv_act_bf16(x, pw, s, "gelu_pair")
        assert got.shape == (M, I)
        assert torch.equal(got, want)


@pytest.mark.parametrize("M, K, N", [(1, 1536, 256), (3, 1536, 256), (16, 2048, 1536)])
def test_gemv_gelu_mul_equals_gemv_then_gelu_mul(M, K, N):
    """The GEMV's GELU-times-multiplier epilogue (the decode step's per-layer-input gate) against the
    GEMV followed by gelu_mul with the same multiplier rows, strided as the per-layer slice is."""
    dev = torch.device("cuda")
    g = torch.Generator(device=dev).manual_seed(M * 100 + N)
    x = torch.randn(M, K, generator=g, device=dev).to(torch.bfloat16)
    w = torch.randint(-127, 128, (N, K), generator=g, dtype=torch.int8, device=dev)
    pw = ops.pack_gemv_weight(w)
    s = (torch.rand(N, generator=g, device=dev) * 0.01).to(torch.bfloat16)
    table = torch.randn(M, 5, N, generator=g, device=dev).to(torch.bfloat16)
    mul = table[:, 2]
    want = ops.gelu_mul_bf16(ops.gemv_bf16(x, pw, s), mul)
    got = ops.gemv_act_bf16(x, pw, s, "gelu_mul", mul=mul)
    assert torch.equal(got, want)
    with pytest.raises(ValueError, match="needs mul"):
        ops.gemv_act_bf16(x, pw, s, "gelu_mul")


@pytest.mark.parametrize("K, N, act", [(1536, 2560, None), (1536, 2 * 6144, "gelu_pair"), (1536, 256, "gelu_mul"),
                                       (256, 640, None), (1024, 96, "gelu_pair"), (1296, 200, None)])
def test_gemv_norm_equals_row_kernel_then_gemv(K, N, act):
    """The decode GEMV with its input norm made in the same launch (the post-attention, post-MLP and
    per-layer-input norms of the decode step as the next linear's prologue) against the row kernel
    (rms_residual_norm, or rms_residual without the second norm) followed by the GEMV: h and the
    GEMV's output bit for bit, with and without the residual, the per-layer scalar and the second
    norm.  K = 1296 leaves the last k-block partial; K = 256 / 1024 / 1536 take one, two and three
    8-element chunks per lane."""
    dev = torch.device("cuda")
    g = torch.Generator(device=dev).manual_seed(K * 7 + N)
    y = (torch.randn(1, K, generator=g, device=dev) * 3).to(torch.bfloat16)
    res = (torch.randn(1, K, generator=g, device=dev) * 5).to(torch.bfloat16)
    w1 = (torch.rand(K, generator=g, device=dev) + 0.5).to(torch.bfloat16)
    w2 = (torch.rand(K, generator=g, device=dev) * 2).to(torch.bfloat16)
    scalar = torch.tensor([0.75], device=dev).to(torch.bfloat16)
    w = torch.randint(-127, 128, (N, K), generator=g, dtype=torch.int8, device=dev)
    pw = ops.pack_gemv_weight(w)
    s = (torch.rand(N, generator=g, device=dev) * 0.01).to(torch.bfloat16)
    mul = torch.randn(1, 3, N, generator=g, device=dev).to(torch.bfloat16)[:, 1] if act == "gelu_mul" else None
    eps = 1e-6
    for r, sc, norm2 in ((res, None, True), (res, scalar, True), (res, None, False), (None, None, False)):
        if norm2:
            h_ref, x_ref = ops.rms_residual_norm(y, r, w1, w2, eps, scalar=sc)
        else:
            assert sc is None
            h_ref = ops.rms_residual(y, r, w1, eps)
            x_ref = h_ref
        want = ops.gemv_bf16(x_ref, pw, s) if act is None else ops.gemv_act_bf16(x_ref, pw, s, act, mul=mul)
        got, h = ops.gemv_norm_bf16(y, r, w1, eps, pw, s, act=act, w2=w2 if norm2 else None, norm2=norm2,
                                    scalar=sc, mul=mul)
        assert torch.equal(h, h_ref), (r is None, sc is None, norm2)
        assert torch.equal(got, want), (r is None, sc is None, norm2)
    got, h = ops.gemv_norm_bf16(y, res, w1, eps, pw, s, act=act, w2=w2, mul=mul, store_h=False)
    _, x_ref = ops.rms_residual_norm(y, res, w1, w2, eps)
    want = ops.gemv_bf16(x_ref, pw, s) if act is None else ops.gemv_act_bf16(x_ref, pw, s, act, mul=mul)
    assert h is None and torch.equal(got, want)


def test_gemv_norm_refusals():
    """The fused norm + GEMV refuses what its one-wave prologue and concurrent workgroups cannot do:
    more than one row, K above 1536, h overlapping the rows every workgroup reads, the LM head's
    many-tile shape."""
    from w8a8._lib import W8A8Error
    dev = torch.device("cuda")
    K = 1536
    y = torch.randn(1, K, device=dev).to(torch.bfloat16)
    w1 = torch.ones(K, device=dev).to(torch.bfloat16)
    pw = ops.pack_gemv_weight(torch.ones((64, K), dtype=torch.int8, device=dev))
    s = torch.ones(64, device=dev).to(torch.bfloat16)
    with pytest.raises(ValueError, match="one row"):
        ops.gemv_norm_bf16(torch.randn(2, K, device=dev).to(torch.bfloat16), None, w1, 1e-6, pw, s)
    big = ops.pack_gemv_weight(torch.ones((64, 2048), dtype=torch.int8, device=dev))
    y2 = torch.randn(1, 2048, device=dev).to(torch.bfloat16)
    with pytest.raises(W8A8Error, match="above the prologue"):
        ops.gemv_norm_bf16(y2, None, None, 1e-6, big, s)
    buf = torch.zeros(2 * K, dtype=torch.bfloat16, device=dev)
    out = torch.empty(64, dtype=torch.bfloat16, device=dev)
    from w8a8._lib import call
    with pytest.raises(W8A8Error, match="h must not overlap"):
        call("w8a8_gemv_packed_norm_bf16", y.data_ptr(), buf.data_ptr(), w1.data_ptr(), None, 0, None, 1e-6,
             buf.data_ptr() + 64, pw.data.data_ptr(), 64, K, s.data_ptr(), 0, 0, None, out.data_ptr(), None)
    with pytest.raises(W8A8Error, match="out must not overlap"):
        call("w8a8_gemv_packed_norm_bf16", y.data_ptr(), None, w1.data_ptr(), None, 0, None, 1e-6,
             None, pw.data.data_ptr(), 64, K, s.data_ptr(), 0, 0, None, y.data_ptr(), None)
    head = ops.pack_gemv_weight(torch.ones((65536, K), dtype=torch.int8, device=dev))
    with pytest.raises(W8A8Error, match="few-tile"):
        ops.gemv_norm_bf16(y, None, w1, 1e-6, head, torch.ones(65536, device=dev).to(torch.bfloat16))
