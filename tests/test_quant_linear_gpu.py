"""GPU parity of the per-token quant prologue (pipeline.py:49-52), the RMSNorm-residual
epilogue (pipeline.py:110-114) and the whole bf16 -> bf16 linear (gemma_npu.py:117-152)."""
import os

import numpy as np
import pytest
import torch

from helpers import assert_bf16_close, f32, from_bits, to_bits

import oracle.oracle as orc
from w8a8 import ops, workloads

pytestmark = pytest.mark.gpu
DEV = "cuda"
GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "w8a8_golden.npz")


def test_quant_rows_golden_inputs():
    d = np.load(GOLDEN)
    x = from_bits(d["quant_x"]).to(DEV)
    q, s = ops.quant_rows(x)
    assert np.array_equal(s.cpu().numpy(), d["quant_s"])
    assert np.array_equal(q.cpu().numpy(), d["quant_q"])
    wq, ws = ops.quant_rows(torch.from_numpy(d["wquant_x"]).to(DEV))
    assert np.array_equal(ws.cpu().numpy(), d["wquant_s"])
    assert np.array_equal(wq.cpu().numpy(), d["wquant_q"])


@pytest.mark.parametrize("M,K", [(1, 16), (5, 24), (512, 1536), (300, 2048), (64, 6144), (3, 12288)])
def test_quant_rows_bf16_exact(M, K):
    x = workloads.activations(M, K, seed=M + K, row_spread=True)
    q_ref, s_ref = orc.quant_rows(to_bits(x), "bf16")
    q, s = ops.quant_rows(x.to(DEV))
    assert np.array_equal(s.cpu().numpy(), s_ref)
    assert np.array_equal(q.cpu().numpy(), q_ref)


def test_quant_rows_ties_and_zero_rows():
    x = torch.zeros((4, 64))
    x[1, :8] = torch.tensor([127.0, 63.5, 0.5, -127.0, 1.5, 2.5, -2.5, -0.5])
    x[2] = torch.arange(64) - 31.5          # halves everywhere after scaling by 127/32
    x[3, 0] = 1e-30                          # below the 1e-8 floor
    xb = x.to(torch.bfloat16)
    q_ref, s_ref = orc.quant_rows(to_bits(xb), "bf16")
    q, s = ops.quant_rows(xb.to(DEV))
    assert np.array_equal(s.cpu().numpy(), s_ref) and np.array_equal(q.cpu().numpy(), q_ref)
    assert q[1, :8].tolist() == [127, 64, 0, -127, 2, 2, -2, 0]


def _nan_inf_rows(K, dtype=torch.bfloat16):
    nan, inf = float("nan"), float("inf")
    x = torch.randn(6, K, generator=torch.Generator().manual_seed(K))
    x[1, K // 3] = nan
    x[2, K - 1] = inf
    x[3, 0] = -inf
    x[4] = 0.0
    x[5, 1], x[5, K // 2] = inf, nan
    return x.to(dtype)


def _assert_scales(s, s_ref):
    s = s.cpu().numpy()
    assert np.array_equal(np.isnan(s), np.isnan(s_ref)) and np.isnan(s[[1, 5]]).all()
    fin = ~np.isnan(s_ref)
    assert np.array_equal(s[fin], s_ref[fin]) and np.isinf(s[[2, 3]]).all()


@pytest.mark.parametrize("K", [48, 100, 12800])
def test_quant_nan_and_inf_rows_follow_torch(K):
    """Rows holding NaN get a NaN scale and rows holding +-Inf an Inf scale, as torch.amax and
    clamp give them (pipeline.py:51), and both quantise to 0 everywhere, as the oracle (pinned
    against torch's own output on the host) does.  Every quant kernel: the block-per-row kernel
    (K = 48), the wave-per-row kernel without (K = 100) and with (K = 12800) vector loads, their
    packed-layout forms, fp32 rows, and the fused k_in row kernel."""
    x = _nan_inf_rows(K)
    q_ref, s_ref = orc.quant_rows(to_bits(x), "bf16")
    assert not q_ref[1:].any()
    q, s = ops.quant_rows(x.to(DEV))
    _assert_scales(s, s_ref)
    assert np.array_equal(q.cpu().numpy(), q_ref)
    if K % 16 == 0:
        from test_gemm_gpu import unpack_act
        for xd in (x.to(DEV), torch.cat([x, x[:, :1]], 1).to(DEV)[:, :K]):  # vector and odd-stride rows
            pa, sp = ops.quant_rows_packed(xd)
            _assert_scales(sp, s_ref)
            assert np.array_equal(unpack_act(pa.data.cpu().numpy(), 6, K)[:6, :K], q_ref)
    xf = _nan_inf_rows(K, torch.float32)
    qf_ref, sf_ref = orc.quant_rows(xf.numpy(), "f32")
    qf, sf = ops.quant_rows(xf.to(DEV))
    _assert_scales(sf, sf_ref)
    assert np.array_equal(qf.cpu().numpy(), qf_ref) and not qf_ref[1:].any()
    if K % 8 == 0 and K <= 12288:
        from w8a8 import fused
        w = torch.ones(K, dtype=torch.bfloat16)
        qk, sk = fused.k_in(x.to(DEV), w.to(DEV), 1e-6)
        qk_ref, sk_ref = orc.k_in(to_bits(x), to_bits(w), 1e-6)
        sk = sk.cpu().numpy()
        assert np.array_equal(np.isnan(sk), np.isnan(sk_ref)) and np.isnan(sk[[1, 2, 3, 5]]).all()
        assert np.array_equal(qk.cpu().numpy()[1:], qk_ref[1:]) and not qk_ref[1:4].any()


@pytest.mark.parametrize("M,K", [(2048, 1536), (2049, 2048), (3658, 6144), (2056, 12288)])
def test_quant_rows_packed_long_m(M, K):
    """Packed quant at the whole-prompt row counts (the GEMM operand of every long-M linear):
    codes and scales bit-exact against the oracle, NaN / Inf / zero rows among them, row counts
    that are not multiples of 8 or 32, padding rows and columns zero."""
    x = workloads.activations(M, K, seed=M + K, row_spread=True)
    x[:6] = _nan_inf_rows(K)
    q_ref, s_ref = orc.quant_rows(to_bits(x), "bf16")
    from test_gemm_gpu import unpack_act
    pa, s = ops.quant_rows_packed(x.to(DEV))
    _assert_scales(s[:6], s_ref[:6])
    assert np.array_equal(s.cpu().numpy()[6:], s_ref[6:])
    full = unpack_act(pa.data.cpu().numpy(), M, K)
    assert np.array_equal(full[:M, :K], q_ref)
    assert not full[M:].any() and not full[:, K:].any(), "padding must be zero"


def test_quant_rows_f32_weights():
    """Per-output-channel weight quant (gemma_npu.py:68-69) is the same kernel on fp32 rows."""
    g = torch.Generator().manual_seed(9)
    w = torch.randn(300, 1536, generator=g) * 0.02
    q_ref, s_ref = orc.quant_rows(w.numpy(), "f32")
    q, s = ops.quant_rows(w.to(DEV))
    assert np.array_equal(s.cpu().numpy(), s_ref) and np.array_equal(q.cpu().numpy(), q_ref)


def test_quant_rows_strided_input():
    x = workloads.activations(33, 256, seed=3)
    big = torch.zeros((33, 320), dtype=torch.bfloat16)
    big[:, :256] = x
    q_ref, s_ref = orc.quant_rows(to_bits(x), "bf16")
    q, s = ops.quant_rows(big.to(DEV)[:, :256])
    assert np.array_equal(q.cpu().numpy(), q_ref) and np.array_equal(s.cpu().numpy(), s_ref)


@pytest.mark.parametrize("with_w", [True, False])
def test_rms_residual(with_w):
    M, N = 65, 1536
    g = torch.Generator().manual_seed(7)
    y = (torch.randn(M, N, generator=g) * 3).to(torch.bfloat16)
    res = torch.randn(M, N, generator=g).to(torch.bfloat16)
    w = (torch.rand(N, generator=g) + 0.5).to(torch.bfloat16) if with_w else None
    ref = orc.rms_residual(to_bits(y), to_bits(res), to_bits(w) if with_w else None, 1e-6)
    h, q, sq = ops.rms_residual(y.to(DEV), res.to(DEV), w.to(DEV) if with_w else None, 1e-6, quant=True)
    got = to_bits(h)
    # h = res + n: the rounding of n (one bf16 ulp of |n|, from fp32 reduction-order
    # differences in mean(y^2)) carries into h even where res cancels n, so the ulp is taken
    # at max(|h|, |res|, |n|)
    addends = np.maximum(np.abs(f32(to_bits(res))), np.abs(f32(ref) - f32(to_bits(res))))
    assert_bf16_close(f32(got), f32(ref), what="rms_residual", ulp_at=addends)
    assert (got == ref).mean() > 0.99
    # the fused quant of h is the prologue's quant of the h it wrote
    q_ref, s_ref = orc.quant_rows(got, "bf16")
    assert np.array_equal(q.cpu().numpy(), q_ref) and np.array_equal(sq.cpu().numpy(), s_ref)


@pytest.mark.parametrize("group", ["qkv", "o", "gate_up", "down"])
def test_linear_bf16_layer_group(group):
    """One E2B-class layer group at M=512, bf16 in -> bf16 out; int32 path checked through
    the bf16 outputs (exact for none / residual, tolerance for gelu)."""
    K, N, epi = workloads.LAYER_GROUPS[group]
    M = 512
    x = workloads.activations(M, K, seed=100 + K)
    w, sw = workloads.weights(N, K, seed=200 + N)
    res = workloads.activations(M, N, seed=300, outliers=False) if epi == "residual" else None
    interleave = N // 2 if epi == "gelu" else 0
    pw = ops.pack_weight(w.to(DEV), "nk", interleave, sw=sw.to(DEV))
    out = ops.linear_bf16(x.to(DEV), pw, epilogue=epi, residual=None if res is None else res.to(DEV))
    ref, _, _ = orc.linear_bf16(to_bits(x), w.numpy(), sw.numpy(), epilogue=epi,
                                residual=None if res is None else to_bits(res))
    got = to_bits(out)
    if epi == "gelu":
        assert_bf16_close(f32(got), f32(ref), what=group)
        assert (got == ref).mean() > 0.99
    else:
        assert np.array_equal(got, ref)


def test_linear_bf16_residual_rms():
    """The down-projection epilogue as the reference runs it: res + rms(y) * w (pipeline.py:113)."""
    M, K, N = 256, 6144, 1536
    x = workloads.activations(M, K, seed=5)
    w, sw = workloads.weights(N, K, seed=6)
    res = workloads.activations(M, N, seed=7, outliers=False)
    g = torch.Generator().manual_seed(8)
    rw = (torch.rand(N, generator=g) + 0.5).to(torch.bfloat16)
    pw = ops.pack_weight(w.to(DEV), "nk", sw=sw.to(DEV))
    out = ops.linear_bf16(x.to(DEV), pw, epilogue="residual_rms", residual=res.to(DEV), rms_w=rw.to(DEV), eps=1e-6)
    ref, _, _ = orc.linear_bf16(to_bits(x), w.numpy(), sw.numpy(), "residual_rms", to_bits(res), to_bits(rw), 1e-6)
    got = to_bits(out)
    addends = np.maximum(np.abs(f32(to_bits(res))), np.abs(f32(ref) - f32(to_bits(res))))
    assert_bf16_close(f32(got), f32(ref), what="residual_rms", ulp_at=addends)
    assert (got == ref).mean() > 0.99


def test_quant_weight_roundtrip():
    """quant_weight packs the per-channel int8 weight; its GEMM equals the oracle's."""
    g = torch.Generator().manual_seed(12)
    wf = torch.randn(96, 256, generator=g) * 0.05
    pw = ops.quant_weight(wf.to(DEV))
    q_ref, s_ref = orc.quant_rows(wf.numpy(), "f32")
    assert np.array_equal(pw.sw.cpu().numpy(), s_ref)
    a = torch.randint(-127, 128, (40, 256), generator=g, dtype=torch.int8)
    c = ops.gemm_i32(a.to(DEV), pw)
    assert np.array_equal(c.cpu().numpy(), orc.int_mm_nk(a.numpy(), q_ref))


def test_selfcheck_quant_step():
    """The division-free quant step equals the IEEE-division step on the GPU for every bf16
    absmax and every bf16 value not above it (1,065,402,240 pairs)."""
    from w8a8._lib import call
    counts = torch.zeros(2, dtype=torch.int64, device=DEV)
    call("w8a8_selfcheck_quant_step", counts.data_ptr(), torch.cuda.current_stream().cuda_stream)
    bad, pairs = counts.cpu().tolist()
    assert pairs == 1065402240
    assert bad == 0


@pytest.mark.parametrize("I,K", [(32, 64), (96, 208), (6144, 1536)])
def test_unpair_packed_equals_the_plain_packing(I, K):
    """The plain packing derived from a GELU-paired one by permuting its tiles is the packing of
    the same weight made directly, byte for byte, and multiplies to torch._int_mm's result."""
    g = torch.Generator().manual_seed(I + K)
    w = torch.randint(-127, 128, (2 * I, K), generator=g, dtype=torch.int8).to(DEV)
    sw = torch.rand(2 * I, generator=g).to(DEV)
    plain = ops.pack_weight(w, "nk", sw=sw)
    derived = ops.unpair_packed(ops.pack_weight(w, "nk", I, sw=sw))
    assert derived.interleave == 0 and derived.sw is sw
    assert torch.equal(derived.data, plain.data)
    a = torch.randint(-127, 128, (40, K), generator=g, dtype=torch.int8).to(DEV)
    ref = torch._int_mm(a.cpu(), w.cpu().t().contiguous())
    assert torch.equal(ops.gemm_i32(a, derived).cpu(), ref)


def test_unpair_packed_refuses_a_plain_weight():
    w = torch.zeros((64, 64), dtype=torch.int8, device=DEV)
    with pytest.raises(ValueError):
        ops.unpair_packed(ops.pack_weight(w, "nk"))
