"""GPU parity of the fused kernels between the GEMMs (pipeline.py:66-127) against the oracle.

Every stage is compared with the oracle run on the same inputs (the GPU's own inputs to that
stage), so differences cannot compound.  bf16 results: within max(1e-2 |ref|, 2 ulp) and
mostly bit-equal (the row sums of squares are added in another order than the oracle's).  int8
results: the quant step is exact given its bf16 input; where that input passed through a norm
or GELU, codes may differ by 1 and scales by one bf16 ulp of the row maximum.
"""
import numpy as np
import pytest
import torch

from helpers import assert_bf16_close, f32, to_bits

import oracle.oracle as orc
from w8a8 import fused, ops, workloads

pytestmark = pytest.mark.gpu
DEV = "cuda"
EPS = 1e-6


def gen(seed):
    return torch.Generator().manual_seed(seed)


def acc_inputs(T, N, seed, spread=2 ** 20):
    """int32 result, per-token and per-channel scales of magnitude y ~ U(-10, 10)."""
    g = gen(seed)
    acc = torch.randint(-spread, spread, (T, N), generator=g, dtype=torch.int32)
    sx = torch.rand(T, generator=g) * 1e-3 + 5e-4
    sw = torch.rand(N, generator=g) * 0.015 + 0.005
    return acc, sx, sw


def norm_weight(N, seed):
    return (torch.rand(N, generator=gen(seed)) + 0.5).to(torch.bfloat16)


def bf16_rows(T, N, seed, scale=2.0):
    return (torch.randn(T, N, generator=gen(seed)) * scale).to(torch.bfloat16)


def npy(t):
    """CPU numpy of a device tensor (bf16 as bit patterns)."""
    return to_bits(t) if t.dtype == torch.bfloat16 else t.cpu().numpy()


def check_quant(q, s, q_ref, s_ref, what, min_exact=0.99):
    q, s = npy(q), npy(s)
    assert np.all(np.abs(s.astype(np.float64) - s_ref) <= s_ref * 2.0 ** -7), f"{what}: scales differ"
    d = np.abs(q.astype(np.int32) - q_ref.astype(np.int32))
    assert d.max() <= 1, f"{what}: int8 codes differ by {d.max()}"
    assert (d == 0).mean() >= min_exact, f"{what}: {(d == 0).mean():.4f} of the codes agree"


def check_h(h, ref, res, what):
    """h = res + n: the rounding of n carries into h even where res cancels it, so the ulp is
    taken at max(|h|, |res|, |n|)."""
    got = npy(h)
    addends = np.maximum(np.abs(f32(res)), np.abs(f32(ref) - f32(res)))
    assert_bf16_close(f32(got), f32(ref), what=what, ulp_at=addends)
    assert (got == ref).mean() > 0.99, f"{what}: {(got == ref).mean():.4f} bit-equal"


def pair_mag(ref):
    """Magnitude of the rotation pair (d, d +- D/2) of each element of a rotated head.  An output
    x*cos + rot*sin can cancel to far below its addends, so a one-ulp difference in the normed
    input (reduction order) shows up as one ulp of the addends, bounded by the pair's norm."""
    r = f32(ref)
    h = r.shape[-1] // 2
    pair = np.concatenate([r[..., h:], r[..., :h]], axis=-1)
    return np.sqrt(r * r + pair * pair)


def unpacked(xq):
    """Row-major int8 view of a PackedActivation (GEMM A layout, 32x32 fragments)."""
    M, K = xq.M, xq.K
    KF = 2 * ((K + 63) // 64)
    Mp = 32 * ((M + 31) // 32)
    b = xq.data.cpu().numpy()[: (Mp // 32) * KF * 1024].reshape(Mp // 32, KF, 2, 32, 16)
    # byte 16*l + j of fragment (mt, f): row 32 mt + l % 32, k 32 f + 16 (l // 32) + j
    rows = b.transpose(0, 3, 1, 2, 4).reshape(Mp, KF * 32)
    return rows[:M, :K], rows


# ---- k_in ---------------------------------------------------------------------------------

@pytest.mark.parametrize("T", [1, 77, 512])
def test_k_in(T):
    N = 1536
    h = workloads.activations(T, N, seed=10 + T)
    w = norm_weight(N, 11)
    q, s = fused.k_in(h.to(DEV), w.to(DEV), EPS)
    q_ref, s_ref = orc.k_in(to_bits(h), to_bits(w), EPS)
    check_quant(q, s, q_ref, s_ref, "k_in")
    # packed output holds the same codes, zero in the padding
    qp, sp = fused.k_in(h.to(DEV), w.to(DEV), EPS, packed=True)
    rows, full = unpacked(qp)
    assert np.array_equal(rows, npy(q)) and np.array_equal(npy(sp), npy(s))
    assert not full[T:].any() and not full[:, N:].any()


# ---- k_qkv --------------------------------------------------------------------------------

@pytest.mark.parametrize("D,shared", [(256, False), (256, True), (512, False), (128, False)])
def test_k_qkv(D, shared):
    T, H, KV = 77, 8, 1
    slots = H if shared else H + 2 * KV
    acc, sx, sw = acc_inputs(T, slots * D, seed=20 + D)
    pos = torch.arange(T).float()[:, None] + 100.0
    ang = pos * (10000.0 ** (-torch.arange(0, D, 2).float() / D))[None, :]
    ang = torch.cat([ang, ang], dim=-1)
    cos, sin = ang.cos().to(torch.bfloat16), ang.sin().to(torch.bfloat16)
    qw, kw = norm_weight(D, 22), norm_weight(D, 23)
    d = [t.to(DEV) for t in (acc, sx, sw, cos, sin, qw, kw)]
    q, k, v = fused.k_qkv(*d, EPS, H, KV, D, shared)
    rq, rk, rv = orc.k_qkv(acc.numpy(), sx.numpy(), sw.numpy(), to_bits(cos), to_bits(sin), to_bits(qw),
                           to_bits(kw), EPS, H, KV, D, shared)
    assert tuple(q.shape) == (H, T, D)
    pairs = [(q, rq, "q")] if shared else [(q, rq, "q"), (k, rk, "k"), (v, rv, "v")]
    for got, ref, name in pairs:
        got = npy(got)
        assert got.shape == ref.shape
        assert_bf16_close(f32(got), f32(ref), what=f"k_qkv {name}", ulp_at=pair_mag(ref) if name != "v" else None)
        assert (got == ref).mean() > 0.99
    if shared:
        assert k is q and v is q


def test_k_qkv_strided_acc_and_cos():
    """acc as a view of a wider result buffer (ld > N, as gemma_npu.py:115 hands it over) and
    cos / sin as row slices of the whole prompt's tables (pipeline.py:254-255)."""
    T, H, KV, D = 40, 8, 1, 256
    N = (H + 2 * KV) * D
    acc, sx, sw = acc_inputs(T, N + 512, seed=30)
    big = torch.randn(T + 16, D, generator=gen(31)).to(torch.bfloat16)
    cos, sin = big[8:8 + T], big.flip(0)[8:8 + T]
    qw, kw = norm_weight(D, 32), norm_weight(D, 33)
    dacc = acc.to(DEV)[:, :N]
    dbig = big.to(DEV)
    dsin = big.flip(0).to(DEV)
    q, k, v = fused.k_qkv(dacc, sx.to(DEV), sw[:N].to(DEV), dbig[8:8 + T], dsin[8:8 + T], qw.to(DEV),
                          kw.to(DEV), EPS, H, KV, D, False)
    rq, rk, rv = orc.k_qkv(np.ascontiguousarray(acc.numpy()[:, :N]), sx.numpy(), sw[:N].numpy(), to_bits(cos),
                           to_bits(sin), to_bits(qw), to_bits(kw), EPS, H, KV, D, False)
    for got, ref in ((q, rq), (k, rk), (v, rv)):
        assert_bf16_close(f32(npy(got)), f32(ref), what="k_qkv strided", ulp_at=pair_mag(ref))


@pytest.mark.parametrize("D, KV, T", [(256, 1, 1), (512, 1, 1), (128, 2, 3)])
def test_k_qkv_cache_writes_the_cache_rows(D, KV, T):
    """k_qkv_cache (the decode step's form) against k_qkv on the same bf16 rows: the same q, and the
    same k / v written into rows pos .. pos+T-1 of the cache at a position held in device memory,
    every other row untouched; a position outside the cache writes nothing."""
    H, rows = 4 * KV, 40
    N = (H + 2 * KV) * D
    y = (torch.randn(T, N, generator=gen(40 + D)) * 0.5).to(torch.bfloat16).to(DEV)
    ang = torch.rand(T, D, generator=gen(41)) * 6.0
    cos, sin = ang.cos().to(torch.bfloat16).to(DEV), ang.sin().to(torch.bfloat16).to(DEV)
    qw, kw = norm_weight(D, 42).to(DEV), norm_weight(D, 43).to(DEV)
    q0, k0, v0 = fused.k_qkv(y, None, None, cos, sin, qw, kw, EPS, H, KV, D, False)
    fill = torch.randn(KV, rows, D, generator=gen(44)).to(torch.bfloat16).to(DEV)
    for p in (0, 17, rows - T):
        kc, vc = fill.clone(), fill.clone()
        pos = torch.tensor([p], dtype=torch.int32, device=DEV)
        q = fused.k_qkv_cache(y, cos, sin, qw, kw, EPS, H, KV, D, kc, vc, pos)
        assert torch.equal(q, q0)
        assert torch.equal(kc[:, p:p + T], k0) and torch.equal(vc[:, p:p + T], v0)
        keep = torch.ones(rows, dtype=torch.bool)
        keep[p:p + T] = False
        assert torch.equal(kc[:, keep.to(DEV)], fill[:, keep.to(DEV)]) and torch.equal(vc[:, keep.to(DEV)], fill[:, keep.to(DEV)])
    for p in (rows, -T - 1, 1 << 20):
        kc, vc = fill.clone(), fill.clone()
        q = fused.k_qkv_cache(y, cos, sin, qw, kw, EPS, H, KV, D, kc, vc, torch.tensor([p], dtype=torch.int32, device=DEV))
        assert torch.equal(q, q0) and torch.equal(kc, fill) and torch.equal(vc, fill)


# ---- k_attn_out ---------------------------------------------------------------------------

@pytest.mark.parametrize("strided", [False, True])
def test_k_attn_out(strided):
    H, T, D = 8, 77, 256
    o_full = (torch.randn(H, T, D + (64 if strided else 0), generator=gen(40)) * 2).to(torch.bfloat16)
    o = o_full[:, :, :D]
    o_dev = o_full.to(DEV)[:, :, :D]  # sliced on the device: row stride D + 64 when strided
    q, s = fused.k_attn_out(o_dev)
    q_ref, s_ref = orc.k_attn_out(to_bits(o))
    # a quant of bf16 values: exact
    assert np.array_equal(npy(q), q_ref) and np.array_equal(npy(s), s_ref)
    qp, _ = fused.k_attn_out(o_dev, packed=True)
    assert np.array_equal(unpacked(qp)[0], q_ref)


# ---- k_post_attn / k_post_ff ------------------------------------------------------------

@pytest.mark.parametrize("T", [1, 77, 512])
def test_k_post_attn(T):
    N = 1536
    acc, sx, sw = acc_inputs(T, N, seed=50 + T)
    res = bf16_rows(T, N, 51)
    w1, w2 = norm_weight(N, 52), norm_weight(N, 53)
    h, q, s = fused.k_post_attn(acc.to(DEV), sx.to(DEV), sw.to(DEV), res.to(DEV), w1.to(DEV), w2.to(DEV), EPS)
    h_ref, _, _ = orc.k_post_attn(acc.numpy(), sx.numpy(), sw.numpy(), to_bits(res), to_bits(w1), to_bits(w2), EPS)
    check_h(h, h_ref, to_bits(res), "k_post_attn h")
    # the int8 rows are the quant of bf16(rms(h, w_pre_ff)) of the h the kernel wrote
    q_ref, s_ref = orc.quant_rows(orc.rms_bf16(npy(h), to_bits(w2), EPS), "bf16")
    check_quant(q, s, q_ref, s_ref, "k_post_attn q")
    _, qp, sp = fused.k_post_attn(acc.to(DEV), sx.to(DEV), sw.to(DEV), res.to(DEV), w1.to(DEV), w2.to(DEV), EPS,
                                  packed=True)
    assert np.array_equal(unpacked(qp)[0], npy(q)) and np.array_equal(npy(sp), npy(s))


@pytest.mark.parametrize("T", [77, 512])
def test_k_post_ff(T):
    N = 1536
    acc, sx, sw = acc_inputs(T, N, seed=60 + T)
    res = bf16_rows(T, N, 61)
    w = norm_weight(N, 62)
    h, q, s = fused.k_post_ff(acc.to(DEV), sx.to(DEV), sw.to(DEV), res.to(DEV), w.to(DEV), EPS)
    h_ref, _, _ = orc.k_post_ff(acc.numpy(), sx.numpy(), sw.numpy(), to_bits(res), to_bits(w), EPS)
    check_h(h, h_ref, to_bits(res), "k_post_ff h")
    q_ref, s_ref = orc.quant_rows(npy(h), "bf16")
    assert np.array_equal(npy(q), q_ref) and np.array_equal(npy(s), s_ref)


@pytest.mark.parametrize("N", [8, 200, 1000, 2560, 3840, 5000, 12288])
def test_row_kernels_at_other_hidden_sizes(N):
    """k_in, k_post_attn and k_post_ff at hidden sizes other than E2B's 1536 (any multiple of 8 up
    to 12288: other Gemma sizes and ragged widths), against the oracle with the same bars as the
    1536-wide tests."""
    T = 37
    print(f"row kernels N={N}", flush=True)
    h = workloads.activations(T, N, seed=N + 1)
    w = norm_weight(N, N + 2)
    q, s = fused.k_in(h.to(DEV), w.to(DEV), EPS)
    q_ref, s_ref = orc.k_in(to_bits(h), to_bits(w), EPS)
    check_quant(q, s, q_ref, s_ref, f"k_in N={N}", min_exact=0.98)
    qp, sp = fused.k_in(h.to(DEV), w.to(DEV), EPS, packed=True)
    assert np.array_equal(unpacked(qp)[0], npy(q)) and np.array_equal(npy(sp), npy(s))

    acc, sx, sw = acc_inputs(T, N, seed=N + 3)
    res = bf16_rows(T, N, N + 4)
    w1, w2 = norm_weight(N, N + 5), norm_weight(N, N + 6)
    hh, q, s = fused.k_post_attn(acc.to(DEV), sx.to(DEV), sw.to(DEV), res.to(DEV), w1.to(DEV), w2.to(DEV), EPS)
    h_ref, _, _ = orc.k_post_attn(acc.numpy(), sx.numpy(), sw.numpy(), to_bits(res), to_bits(w1), to_bits(w2), EPS)
    check_h(hh, h_ref, to_bits(res), f"k_post_attn h N={N}")
    q_ref, s_ref = orc.quant_rows(orc.rms_bf16(npy(hh), to_bits(w2), EPS), "bf16")
    check_quant(q, s, q_ref, s_ref, f"k_post_attn q N={N}", min_exact=0.98)

    hh, q, s = fused.k_post_ff(acc.to(DEV), sx.to(DEV), sw.to(DEV), res.to(DEV), w1.to(DEV), EPS)
    h_ref, _, _ = orc.k_post_ff(acc.numpy(), sx.numpy(), sw.numpy(), to_bits(res), to_bits(w1), EPS)
    check_h(hh, h_ref, to_bits(res), f"k_post_ff h N={N}")
    q_ref, s_ref = orc.quant_rows(npy(hh), "bf16")
    assert np.array_equal(npy(q), q_ref) and np.array_equal(npy(s), s_ref)


# ---- k_gelu / k_ple_gate ------------------------------------------------------------------

@pytest.mark.parametrize("T,I", [(33, 6144), (5, 256)])
def test_k_gelu(T, I):
    acc, sx, sw = acc_inputs(T, 2 * I, seed=70 + I)
    q, s = fused.k_gelu(acc.to(DEV), sx.to(DEV), sw.to(DEV), I)
    q_ref, s_ref = orc.k_gelu(acc.numpy(), sx.numpy(), sw.numpy(), I)
    check_quant(q, s, q_ref, s_ref, "k_gelu")


def test_k_ple_gate_strided_ple():
    """ple as the reference slices it: ctx['ple'][s:e, i] of a [T, layers, 256] tensor."""
    T, L, P, layer = 77, 35, 256, 17
    acc, sx, sw = acc_inputs(T, P, seed=80)
    ple_all = bf16_rows(T, L * P, 81).reshape(T, L, P)
    ple = ple_all[:, layer]
    q, s = fused.k_ple_gate(acc.to(DEV), sx.to(DEV), sw.to(DEV), ple_all.to(DEV)[:, layer])
    q_ref, s_ref = orc.k_ple_gate(acc.numpy(), sx.numpy(), sw.numpy(), to_bits(ple))
    check_quant(q, s, q_ref, s_ref, "k_ple_gate")


# ---- k_ple_out ----------------------------------------------------------------------------

@pytest.mark.parametrize("T", [77, 512])
def test_k_ple_out(T):
    N = 1536
    acc, sx, sw = acc_inputs(T, N, seed=90 + T)
    h = bf16_rows(T, N, 91)
    w = norm_weight(N, 92)
    scalar = torch.tensor([0.62], dtype=torch.bfloat16)
    out = fused.k_ple_out(acc.to(DEV), sx.to(DEV), sw.to(DEV), h.to(DEV), w.to(DEV), scalar.to(DEV), EPS)
    ref = orc.k_ple_out(acc.numpy(), sx.numpy(), sw.numpy(), to_bits(h), to_bits(w), to_bits(scalar)[0], EPS)
    sc = float(scalar.float())
    got = npy(out)
    ulp_at = np.maximum(np.abs(f32(to_bits(h))) * sc, np.abs(f32(ref)))
    assert_bf16_close(f32(got), f32(ref), what="k_ple_out", ulp_at=ulp_at * 2)
    assert (got == ref).mean() > 0.99


# ---- the dequantised bf16 input (the GEMM's dequant epilogue) gives the same bits ----------

@pytest.mark.parametrize("T", [77, 512])
def test_kernels_on_dequantised_rows_match_int32(T):
    """k_qkv, k_post_attn, k_post_ff, k_ple_gate and k_ple_out fed y = bf16((acc * sx) * sw) -- the
    rows the GEMM's dequant epilogue writes, here from the standalone dequant kernel -- give exactly
    the outputs of the int32 entries on acc, sx, sw, as strided views too."""
    D, H, KV, N, P = 256, 8, 1, 1536, 256

    def dq(acc, sx, sw, pad=0):
        a = acc.to(DEV)
        y = torch.empty((T, a.shape[1] + pad), dtype=torch.bfloat16, device=DEV)[:, :a.shape[1]]
        return ops.dequant_bf16(a, sx.to(DEV), sw.to(DEV), out=y)

    def same(a, b, what):
        for x, y in zip(a if isinstance(a, tuple) else (a,), b if isinstance(b, tuple) else (b,)):
            xs = x.data if hasattr(x, "data") and not isinstance(x, torch.Tensor) else x
            ys = y.data if hasattr(y, "data") and not isinstance(y, torch.Tensor) else y
            assert torch.equal(xs, ys), what

    acc, sx, sw = acc_inputs(T, (H + 2 * KV) * D, seed=100 + T)
    ang = (torch.arange(T).float()[:, None] * 0.01 + torch.arange(D).float()[None, :] * 0.1)
    cos, sin = ang.cos().to(torch.bfloat16).to(DEV), ang.sin().to(torch.bfloat16).to(DEV)
    qw, kw = norm_weight(D, 101).to(DEV), norm_weight(D, 102).to(DEV)
    ref = fused.k_qkv(acc.to(DEV), sx.to(DEV), sw.to(DEV), cos, sin, qw, kw, EPS, H, KV, D, False)
    same(fused.k_qkv(dq(acc, sx, sw, pad=64), None, None, cos, sin, qw, kw, EPS, H, KV, D, False), ref, "k_qkv")
    acc, sx, sw = acc_inputs(T, N, seed=110 + T)
    res, w1, w2 = bf16_rows(T, N, 111).to(DEV), norm_weight(N, 112).to(DEV), norm_weight(N, 113).to(DEV)
    d = (acc.to(DEV), sx.to(DEV), sw.to(DEV))
    for packed in (False, True):
        same(fused.k_post_attn(dq(acc, sx, sw), None, None, res, w1, w2, EPS, packed=packed),
             fused.k_post_attn(*d, res, w1, w2, EPS, packed=packed), "k_post_attn")
        same(fused.k_post_ff(dq(acc, sx, sw, pad=8), None, None, res, w1, EPS, packed=packed),
             fused.k_post_ff(*d, res, w1, EPS, packed=packed), "k_post_ff")
    scalar = torch.tensor([0.62], dtype=torch.bfloat16, device=DEV)
    same(fused.k_ple_out(dq(acc, sx, sw), None, None, res, w1, scalar, EPS),
         fused.k_ple_out(*d, res, w1, scalar, EPS), "k_ple_out")
    acc, sx, sw = acc_inputs(T, P, seed=120 + T)
    ple = bf16_rows(T, 4 * P, 121).to(DEV)[:, P:2 * P]
    same(fused.k_ple_gate(dq(acc, sx, sw), None, None, ple, packed=True),
         fused.k_ple_gate(acc.to(DEV), sx.to(DEV), sw.to(DEV), ple, packed=True), "k_ple_gate")


# ---- a decoder layer's linear path, stage by stage --------------------------------------

def test_layer_chain_stagewise():
    """k_in -> qkv GEMM -> k_qkv -> (q as attention output) -> k_attn_out -> o GEMM -> k_post_attn
    -> gate_up GEMM -> k_gelu -> down GEMM -> k_post_ff -> PLE gate GEMM -> k_ple_gate -> PLE
    projection GEMM -> k_ple_out (pipeline.py:244-310), every stage on the device, each checked
    against the oracle on that stage's device inputs; the GEMMs are exact."""
    T, E, H, KV, D, I, P = 77, 1536, 8, 1, 256, 6144, 256
    shapes = {"qkv": ((H + 2 * KV) * D, E), "o": (E, H * D), "gate_up": (2 * I, E), "down": (E, I),
              "ple_gate": (P, E), "ple_proj": (E, P)}
    W = {}
    for i, (name, (N, K)) in enumerate(shapes.items()):
        w, sw = workloads.weights(N, K, seed=300 + i)
        W[name] = (w.numpy(), sw, ops.pack_weight(w.to(DEV), "nk", sw=sw.to(DEV)))
    nw = {n: norm_weight(E if n not in ("qw", "kw") else D, 400 + i).to(DEV)
          for i, n in enumerate(("in", "qw", "kw", "post", "pre_ff", "post_ff", "post_ple"))}
    h0 = workloads.activations(T, E, seed=310).to(DEV)
    ang = torch.arange(T).float()[:, None] * (10000.0 ** (-torch.arange(0, D, 2).float() / D))[None, :]
    ang = torch.cat([ang, ang], dim=-1)
    cos, sin = ang.cos().to(torch.bfloat16).to(DEV), ang.sin().to(torch.bfloat16).to(DEV)
    ple = bf16_rows(T, P, 311).to(DEV)
    scalar = torch.tensor([0.8], dtype=torch.bfloat16, device=DEV)
    B = lambda t: npy(t)  # noqa: E731

    def gemm(xq, name):
        acc = ops.gemm_i32(xq, W[name][2])
        assert np.array_equal(npy(acc), orc.int_mm_nk(npy(xq), W[name][0])), f"{name} GEMM"
        return acc, W[name][1].to(DEV)

    xq, sx = fused.k_in(h0, nw["in"], EPS)
    check_quant(xq, sx, *orc.k_in(B(h0), B(nw["in"]), EPS), "k_in")
    acc, sw = gemm(xq, "qkv")
    q, k, v = fused.k_qkv(acc, sx, sw, cos, sin, nw["qw"], nw["kw"], EPS, H, KV, D, False)
    for got, ref in zip((q, k, v), orc.k_qkv(B(acc), B(sx), B(sw), B(cos), B(sin), B(nw["qw"]), B(nw["kw"]), EPS,
                                             H, KV, D, False)):
        assert_bf16_close(f32(B(got)), f32(ref), what="chain k_qkv", ulp_at=pair_mag(ref))
    xq, sx = fused.k_attn_out(q)
    q_ref, s_ref = orc.k_attn_out(B(q))
    assert np.array_equal(B(xq), q_ref) and np.array_equal(B(sx), s_ref)
    acc, sw = gemm(xq, "o")
    sa = sx  # the scales of the rows that entered the GEMM
    h, xq, sx = fused.k_post_attn(acc, sa, sw, h0, nw["post"], nw["pre_ff"], EPS)
    h_ref, _, _ = orc.k_post_attn(B(acc), B(sa), B(sw), B(h0), B(nw["post"]), B(nw["pre_ff"]), EPS)
    check_h(h, h_ref, B(h0), "chain k_post_attn")
    check_quant(xq, sx, *orc.quant_rows(orc.rms_bf16(B(h), B(nw["pre_ff"]), EPS), "bf16"), "chain k_post_attn q")
    acc, sw = gemm(xq, "gate_up")
    sa = sx
    xq, sx = fused.k_gelu(acc, sa, sw, I)
    check_quant(xq, sx, *orc.k_gelu(B(acc), B(sa), B(sw), I), "chain k_gelu")
    acc, sw = gemm(xq, "down")
    sa, h_in = sx, h
    h, xq, sx = fused.k_post_ff(acc, sa, sw, h_in, nw["post_ff"], EPS)
    h_ref, _, _ = orc.k_post_ff(B(acc), B(sa), B(sw), B(h_in), B(nw["post_ff"]), EPS)
    check_h(h, h_ref, B(h_in), "chain k_post_ff")
    assert np.array_equal(B(xq), orc.quant_rows(B(h), "bf16")[0])
    acc, sw = gemm(xq, "ple_gate")
    sa = sx
    xq, sx = fused.k_ple_gate(acc, sa, sw, ple)
    check_quant(xq, sx, *orc.k_ple_gate(B(acc), B(sa), B(sw), B(ple)), "chain k_ple_gate")
    acc, sw = gemm(xq, "ple_proj")
    out = fused.k_ple_out(acc, sx, sw, h, nw["post_ple"], scalar, EPS)
    ref = orc.k_ple_out(B(acc), B(sx), B(sw), B(h), B(nw["post_ple"]), B(scalar)[0], EPS)
    ulp_at = np.maximum(np.abs(f32(B(h))), np.abs(f32(ref)))
    assert_bf16_close(f32(B(out)), f32(ref), what="chain k_ple_out", ulp_at=ulp_at)
    assert (B(out) == ref).mean() > 0.99
    assert np.isfinite(f32(B(out))).all()


# ---- k_qkv inside the decode attention ------------------------------------------------------

@pytest.mark.parametrize("D, KV, window", [(256, 1, 512), (512, 1, 0), (256, 2, 0), (128, 1, 64)])
def test_decode_qkv_at_equals_k_qkv_then_decode_at(D, KV, window):
    """attention.decode_qkv_at (k_qkv made inside the split-key decode attention) against
    k_qkv_cache / k_qkv followed by decode_at: the same output and the same cache bit for bit, for a
    layer that owns its keys (the token's key and value written at the device-held position and
    attended to there) and one that reads another layer's cache (q only), at positions in the first
    key chunk, on chunk edges, past the window and at the cache's last row."""
    from w8a8 import attention
    H, rows = 8 * KV, 1100
    y_full = (torch.randn(1, (H + 2 * KV) * D, generator=gen(50 + D)) * 0.7).to(torch.bfloat16).to(DEV)
    ang = torch.rand(1, D, generator=gen(51)) * 6.0
    cos, sin = ang.cos().to(torch.bfloat16).to(DEV), ang.sin().to(torch.bfloat16).to(DEV)
    qw, kw = norm_weight(D, 52).to(DEV), norm_weight(D, 53).to(DEV)
    fill = (torch.randn(KV, rows, D, generator=gen(54)) * 0.7).to(torch.bfloat16).to(DEV)
    fill_v = (torch.randn(KV, rows, D, generator=gen(55))).to(torch.bfloat16).to(DEV)
    tables_c = torch.rand(rows, D, generator=gen(56)).to(torch.bfloat16).to(DEV)
    tables_s = torch.rand(rows, D, generator=gen(57)).to(torch.bfloat16).to(DEV)
    for p in (0, 5, 31, 32, 63, 64, 100, 600, rows - 1):
        pos = torch.tensor([p], dtype=torch.int32, device=DEV)
        for kv_write in (True, False):
            y = y_full if kv_write else y_full[:, :H * D].contiguous()
            kc_ref, vc_ref = fill.clone(), fill_v.clone()
            if kv_write:
                q = fused.k_qkv_cache(y, cos, sin, qw, kw, EPS, H, KV, D, kc_ref, vc_ref, pos)
            else:
                q = fused.k_qkv(y, None, None, cos, sin, qw, None, EPS, H, KV, D, True)[0]
            want = attention.decode_at(q[:, 0], kc_ref, vc_ref, pos, window, 0.75)
            kc, vc = fill.clone(), fill_v.clone()
            got = attention.decode_qkv_at(y, cos, sin, qw, kw, EPS, H, KV, D, kc, vc, pos, kv_write, window, 0.75)
            assert torch.equal(got, want), (p, kv_write)
            assert torch.equal(kc, kc_ref) and torch.equal(vc, vc_ref), (p, kv_write)
            # the RoPE tables [rows, D] read at the position held in pos
            ctab, stab = tables_c.clone(), tables_s.clone()
            ctab[p], stab[p] = cos[0], sin[0]
            kc, vc = fill.clone(), fill_v.clone()
            got = attention.decode_qkv_at(y, ctab, stab, qw, kw, EPS, H, KV, D, kc, vc, pos, kv_write, window, 0.75)
            assert torch.equal(got, want), (p, kv_write, "table")
            assert torch.equal(kc, kc_ref) and torch.equal(vc, vc_ref), (p, kv_write, "table")


@pytest.mark.parametrize("D, window, H, KV", [(256, 512, 8, 1), (512, 512, 8, 1), (128, 64, 4, 1), (256, 128, 16, 2)])
def test_o_projection_merging_the_attention_chunks(D, window, H, KV):
    """ops.gemv_attn_merge_bf16 (the o projection whose prologue merges the decode attention's key
    chunks) after decode_qkv_at(..., merge=False) against the attention with its merge kernel
    followed by the GEMV: the same output bit for bit, at positions with one, several and all 16
    chunks live, on a chunk edge and at the cache's end."""
    from w8a8 import attention
    rows, N = 1100, 1536
    y = (torch.randn(1, (H + 2 * KV) * D, generator=gen(60 + D)) * 0.7).to(torch.bfloat16).to(DEV)
    ang = torch.rand(1, D, generator=gen(61)) * 6.0
    cos, sin = ang.cos().to(torch.bfloat16).to(DEV), ang.sin().to(torch.bfloat16).to(DEV)
    qw, kw = norm_weight(D, 62).to(DEV), norm_weight(D, 63).to(DEV)
    fill = (torch.randn(KV, rows, D, generator=gen(64)) * 0.7).to(torch.bfloat16).to(DEV)
    fill_v = torch.randn(KV, rows, D, generator=gen(65)).to(torch.bfloat16).to(DEV)
    w = torch.randint(-127, 128, (N, H * D), generator=gen(66), dtype=torch.int8).to(DEV)
    pw = ops.pack_gemv_weight(w)
    s = (torch.rand(N, generator=gen(67)) * 0.01).to(torch.bfloat16).to(DEV)
    ws = torch.empty(attention.decode_at_workspace_bytes(H, KV, rows, D, window), dtype=torch.uint8, device=DEV)
    assert attention.decode_grid_chunks(D, rows, window) <= 16
    for p in (0, 40, 63, 64, 300, 700, rows - 1):
        pos = torch.tensor([p], dtype=torch.int32, device=DEV)
        kc, vc = fill.clone(), fill_v.clone()
        o = attention.decode_qkv_at(y, cos, sin, qw, kw, EPS, H, KV, D, kc, vc, pos, True, window, 0.5, workspace=ws)
        want = ops.gemv_bf16(o.reshape(1, -1), pw, s)
        kc2, vc2 = fill.clone(), fill_v.clone()
        assert attention.decode_qkv_at(y, cos, sin, qw, kw, EPS, H, KV, D, kc2, vc2, pos, True, window, 0.5,
                                       workspace=ws, merge=False) is None
        got = ops.gemv_attn_merge_bf16(ws, pos, H, KV, rows, D, window, 0.5, pw, s)
        assert torch.equal(got, want), p
        assert torch.equal(kc2, kc) and torch.equal(vc2, vc), p


@pytest.mark.parametrize("T", [1, 77, 600])
@pytest.mark.parametrize("packed", [False, True])
def test_k_ple_out_with_the_next_k_in(T, packed):
    """k_ple_out with the next layer's input norm and quant in the same launch (the whole-prompt
    prefill's layer boundary) against k_ple_out then k_in: the rows and the int8 rows and scales bit
    for bit, from the int32 GEMM result and from its dequantised bf16 form, row-major and packed."""
    N = 1536
    acc, sx, sw = acc_inputs(T, N, seed=95 + T)
    acc, sx, sw = acc.to(DEV), sx.to(DEV), sw.to(DEV)
    h = bf16_rows(T, N, 96).to(DEV)
    w, w_next = norm_weight(N, 97).to(DEV), norm_weight(N, 98).to(DEV)
    scalar = torch.tensor([0.62], dtype=torch.bfloat16, device=DEV)
    y = ops.dequant_bf16(acc, sx, sw)
    for src in ((acc, sx, sw), (y, None, None)):
        out_ref = fused.k_ple_out(*src, h, w, scalar, EPS)
        xq_ref, sx_ref = fused.k_in(out_ref, w_next, EPS, packed=packed)
        out, xq, sxn = fused.k_ple_out(*src, h, w, scalar, EPS, norm_next=w_next, packed=packed)
        assert torch.equal(out, out_ref)
        assert torch.equal(sxn, sx_ref)
        if packed:
            assert torch.equal(xq.data, xq_ref.data)
        else:
            assert torch.equal(xq, xq_ref)
