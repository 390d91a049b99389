"""GPU parity of the int8 GEMM (npu_kernels.py:40-56) and its fused epilogues, through the
C ABI.  int32 results must be bit-exact against the oracle / torch._int_mm; bf16 epilogues
bit-exact where the arithmetic is exact (dequant, residual add) and within
max(1e-2 |ref|, 2 ulp) where it involves tanh."""
import numpy as np
import pytest
import torch

from helpers import assert_bf16_close, f32, to_bits

import oracle.oracle as orc
from w8a8 import lib, ops, workloads

pytestmark = pytest.mark.gpu
DEV = "cuda"
CONFIGS = list(range(lib().w8a8_gemm_tile_configs()))


def rand_i8(shape, seed, lo=-128, hi=128):
    g = torch.Generator().manual_seed(seed)
    return torch.randint(lo, hi, shape, generator=g, dtype=torch.int8)


def packed_from_nk(w_nk, interleave=0):
    return ops.pack_weight(w_nk.to(DEV), "nk", interleave)


@pytest.mark.parametrize("cfg", CONFIGS)
@pytest.mark.parametrize("M,N,K", [(1, 16, 64), (37, 72, 128), (130, 200, 192), (300, 520, 320),
                                   (64, 48, 80), (257, 33, 1536)])
def test_gemm_i32_vs_oracle(cfg, M, N, K):
    a = rand_i8((M, K), seed=M * 7 + K)
    w = rand_i8((N, K), seed=N * 13 + K)
    ref = orc.int_mm_nk(a.numpy(), w.numpy())
    c = ops.gemm_i32(a.to(DEV), packed_from_nk(w), tile_cfg=cfg)
    got = c.cpu().numpy()
    assert np.array_equal(got, ref), f"mismatches: {(got != ref).sum()}"


def test_gemm_i32_from_kn_layout():
    """The reference's B is [K, N] (npu_kernels.py:46); packing from it gives the same product."""
    a = rand_i8((96, 256), 1)
    b = rand_i8((256, 144), 2)
    w = ops.pack_weight(b.to(DEV), "kn")
    c = ops.gemm_i32(a.to(DEV), w)
    assert torch.equal(c.cpu(), torch._int_mm(a, b))


def test_gemm_i32_extremes():
    K = 12288  # the largest K in the model's double-wide layers: |acc| = 128*128*K < 2^31
    a = torch.full((40, K), -128, dtype=torch.int8)
    w = torch.full((24, K), -128, dtype=torch.int8)
    c = ops.gemm_i32(a.to(DEV), packed_from_nk(w))
    assert (c == 128 * 128 * K).all()
    w[3] = 127
    c = ops.gemm_i32(a.to(DEV), packed_from_nk(w)).cpu()
    assert (c[:, 3] == -128 * 127 * K).all() and (c[:, 0] == 128 * 128 * K).all()


def test_gemm_i32_one_hot_rows_select_weights():
    K, N = 128, 80
    w = rand_i8((N, K), 5)
    a = torch.zeros((K, K), dtype=torch.int8)
    a[torch.arange(K), torch.arange(K)] = 1
    c = ops.gemm_i32(a.to(DEV), packed_from_nk(w)).cpu()
    assert torch.equal(c, w.t().int())


def test_gemm_i32_empty_m():
    w = packed_from_nk(rand_i8((32, 64), 1))
    c = ops.gemm_i32(torch.empty((0, 64), dtype=torch.int8, device=DEV), w)
    assert c.shape == (0, 32)


def test_gemm_i32_strided_views():
    """Row-strided A and C views, as the reference's slot buffers are (gemma_npu.py:104-115)."""
    M, K, N = 50, 128, 96
    a_big = rand_i8((M, K + 64), 3)
    w = rand_i8((N, K), 4)
    c_big = torch.full((M, N + 32), -7, dtype=torch.int32, device=DEV)
    a_view = a_big.to(DEV)[:, :K]
    c_view = c_big[:, :N]
    ops.gemm_i32(a_view, packed_from_nk(w), c_view)
    ref = torch._int_mm(a_big[:, :K].contiguous(), w.t().contiguous())
    assert torch.equal(c_view.cpu(), ref)
    assert (c_big[:, N:] == -7).all(), "wrote past N"


def test_gemm_i32_single_prefill_microbatch():
    """One prefill micro-batch GEMM, M=512 K=1536 N=6144, seed 0: bit-exact vs torch._int_mm."""
    M, K, N = 512, 1536, 6144
    x, w, _ = workloads.single_gemm_inputs(M, K, N, seed=0)
    a, _ = ops.quant_rows(x.to(DEV))
    c = ops.gemm_i32(a, packed_from_nk(w))
    ref = torch._int_mm(a.cpu(), w.t().contiguous())
    assert torch.equal(c.cpu(), ref)


@pytest.mark.parametrize("M", [3658, 4096])
def test_gemm_i32_prefill_m_unpadded_and_padded(M):
    """M=3658 runs unpadded (no 512-row micro-batching); the rows of M=4096 agree."""
    K, N = 2048, 1536
    x = workloads.activations(M, K, seed=11)
    a, _ = ops.quant_rows(x.to(DEV))
    w, _ = workloads.weights(N, K, seed=12)
    c = ops.gemm_i32(a, packed_from_nk(w))
    ref = torch._int_mm(a.cpu(), w.t().contiguous())
    assert torch.equal(c.cpu(), ref)


# ---- bf16 epilogues -------------------------------------------------------------------------

def _inputs(M, K, N, seed):
    x = workloads.activations(M, K, seed)
    w, sw = workloads.weights(N, K, seed + 1)
    q, sx = orc.quant_rows(to_bits(x), "bf16")
    return x, w, sw, q, sx


@pytest.mark.parametrize("cfg", CONFIGS)
def test_gemm_dequant_epilogue_exact(cfg):
    M, K, N = 200, 256, 320
    x, w, sw, q, sx = _inputs(M, K, N, 21)
    ref = orc.dequant(orc.int_mm_nk(q, w.numpy()), sx, sw.numpy())
    out = ops.gemm_bf16(torch.from_numpy(q).to(DEV), torch.from_numpy(sx).to(DEV), packed_from_nk(w),
                        sw.to(DEV), tile_cfg=cfg)
    assert np.array_equal(to_bits(out), ref)


@pytest.mark.parametrize("cfg", CONFIGS)
def test_gemm_residual_epilogue_exact(cfg):
    M, K, N = 130, 192, 256
    x, w, sw, q, sx = _inputs(M, K, N, 31)
    res = workloads.activations(M, N, 32, outliers=False)
    y = orc.dequant(orc.int_mm_nk(q, w.numpy()), sx, sw.numpy())
    ref = orc.add_residual(y, to_bits(res))
    out = ops.gemm_bf16(torch.from_numpy(q).to(DEV), torch.from_numpy(sx).to(DEV), packed_from_nk(w),
                        sw.to(DEV), epilogue="residual", residual=res.to(DEV), tile_cfg=cfg)
    assert np.array_equal(to_bits(out), ref)


@pytest.mark.parametrize("cfg", CONFIGS)
def test_gemm_gelu_epilogue(cfg):
    M, K, I = 150, 256, 192
    x, w, sw, q, sx = _inputs(M, K, 2 * I, 41)
    y = orc.dequant(orc.int_mm_nk(q, w.numpy()), sx, sw.numpy())
    ref = orc.gelu_mul(y)
    out = ops.gemm_bf16(torch.from_numpy(q).to(DEV), torch.from_numpy(sx).to(DEV),
                        packed_from_nk(w, interleave=I), sw.to(DEV), epilogue="gelu", tile_cfg=cfg)
    got = to_bits(out)
    assert_bf16_close(f32(got), f32(ref), what="gelu epilogue")
    assert (got == ref).mean() > 0.99


def _view(rows, cols, dtype, fill):
    """A [rows, cols] view with an odd row stride and an offset of one element into its buffer (no
    vector store fits its rows), and the buffer with the elements outside the view."""
    big = torch.full((rows + 1, cols + 3), fill, dtype=dtype, device=DEV)
    outside = torch.ones(big.shape, dtype=torch.bool)
    outside[1:, 1:cols + 1] = False
    return big[1:, 1:cols + 1], big, outside


@pytest.mark.parametrize("cfg", CONFIGS)
def test_gemm_outputs_in_unaligned_strided_views(cfg):
    """Every configuration's stores into outputs whose rows allow no vector store (odd row stride,
    one element of offset), with ragged N: int32, dequant, residual (also aliasing the output) and
    GELU results exact as above, and nothing written outside the view."""
    M, K, N, I = 77, 192, 100, 96
    x, w, sw, q, sx = _inputs(M, K, N, 51)
    qd, sxd, pw = torch.from_numpy(q).to(DEV), torch.from_numpy(sx).to(DEV), packed_from_nk(w)
    acc = orc.int_mm_nk(q, w.numpy())
    c, big, outside = _view(M, N, torch.int32, -7)
    ops.gemm_i32(qd, pw, c, tile_cfg=cfg)
    assert np.array_equal(c.cpu().numpy(), acc) and (big.cpu()[outside] == -7).all()
    y = orc.dequant(acc, sx, sw.numpy())
    out, big, outside = _view(M, N, torch.bfloat16, 3.0)
    ops.gemm_bf16(qd, sxd, pw, sw.to(DEV), out=out, tile_cfg=cfg)
    assert np.array_equal(to_bits(out), y) and (big.cpu()[outside] == 3.0).all()
    res = workloads.activations(M, N, 52, outliers=False)
    ref = orc.add_residual(y, to_bits(res))
    out, big, outside = _view(M, N, torch.bfloat16, 3.0)
    rv, _, _ = _view(M, N, torch.bfloat16, 0.0)
    rv.copy_(res.to(DEV))
    ops.gemm_bf16(qd, sxd, pw, sw.to(DEV), epilogue="residual", residual=rv, out=out, tile_cfg=cfg)
    assert np.array_equal(to_bits(out), ref) and (big.cpu()[outside] == 3.0).all()
    out.copy_(res.to(DEV))  # the residual aliasing the output
    ops.gemm_bf16(qd, sxd, pw, sw.to(DEV), epilogue="residual", residual=out, out=out, tile_cfg=cfg)
    assert np.array_equal(to_bits(out), ref)
    wg, swg = workloads.weights(2 * I, K, 53)
    yg = orc.dequant(orc.int_mm_nk(q, wg.numpy()), sx, swg.numpy())
    refg = orc.gelu_mul(yg)
    out, big, outside = _view(M, I, torch.bfloat16, 3.0)
    ops.gemm_bf16(qd, sxd, packed_from_nk(wg, interleave=I), swg.to(DEV), epilogue="gelu", out=out,
                  tile_cfg=cfg)
    got = to_bits(out)
    assert_bf16_close(f32(got), f32(refg), what="gelu epilogue, strided output")
    assert (got == refg).mean() > 0.99 and (big.cpu()[outside] == 3.0).all()


def test_gemm_gelu_ragged_tiles():
    """I not a multiple of the 128/256-column block: gate/up tiles straddle the block edge."""
    M, K, I = 70, 128, 96
    x, w, sw, q, sx = _inputs(M, K, 2 * I, 43)
    ref = orc.gelu_mul(orc.dequant(orc.int_mm_nk(q, w.numpy()), sx, sw.numpy()))
    out = ops.gemm_bf16(torch.from_numpy(q).to(DEV), torch.from_numpy(sx).to(DEV),
                        packed_from_nk(w, interleave=I), sw.to(DEV), epilogue="gelu")
    assert_bf16_close(f32(to_bits(out)), f32(ref), what="gelu ragged")


def test_standalone_dequant_exact():
    M, N = 77, 300
    g = torch.Generator().manual_seed(3)
    acc = torch.randint(-(2 ** 30), 2 ** 30, (M, N), generator=g, dtype=torch.int32)
    sx = torch.rand(M, generator=g) * 1e-3
    sw = torch.rand(N, generator=g) * 0.02
    out = ops.dequant_bf16(acc.to(DEV), sx.to(DEV), sw.to(DEV))
    assert np.array_equal(to_bits(out), orc.dequant(acc.numpy(), sx.numpy(), sw.numpy()))


# ---- packed activations ---------------------------------------------------------------------

def unpack_act(packed, M, K):
    """Inverse of the packed activation layout (fragment (mt, j), byte 16*l + b = row
    32*mt + l%32, k 32*j + 16*(l/32) + b), written out independently of the kernels."""
    KF = 2 * ((K + 63) // 64)
    MT = (M + 31) // 32
    arr = packed.reshape(MT, KF, 2, 32, 16)            # [mt][j][h][r][b]
    full = arr.transpose(0, 3, 1, 2, 4).reshape(MT * 32, KF * 32)
    return full


@pytest.mark.parametrize("M,K", [(1, 64), (33, 80), (512, 1536), (100, 2048)])
def test_pack_act_layout(M, K):
    a = rand_i8((M, K), seed=M + K)
    pa = ops.pack_act(a.to(DEV))
    full = unpack_act(pa.data.cpu().numpy(), M, K)
    assert np.array_equal(full[:M, :K], a.numpy())
    assert not full[M:].any() and not full[:, K:].any(), "padding must be zero"


@pytest.mark.parametrize("M,K", [(5, 16), (64, 1536), (77, 6144), (300, 2048)])
def test_quant_rows_packed_vs_oracle(M, K):
    x = workloads.activations(M, K, seed=M * K, row_spread=True)
    q_ref, s_ref = orc.quant_rows(to_bits(x), "bf16")
    pa, s = ops.quant_rows_packed(x.to(DEV))
    full = unpack_act(pa.data.cpu().numpy(), M, K)
    assert np.array_equal(s.cpu().numpy(), s_ref)
    assert np.array_equal(full[:M, :K], q_ref)
    assert not full[M:].any() and not full[:, K:].any()


@pytest.mark.parametrize("cfg", CONFIGS)
@pytest.mark.parametrize("M,N,K", [(1, 16, 64), (37, 72, 128), (300, 520, 320), (257, 33, 1536)])
def test_gemm_i32_packed_a(cfg, M, N, K):
    a = rand_i8((M, K), seed=M * 3 + K)
    w = rand_i8((N, K), seed=N * 5 + K)
    ref = orc.int_mm_nk(a.numpy(), w.numpy())
    c = ops.gemm_i32(ops.pack_act(a.to(DEV)), packed_from_nk(w), tile_cfg=cfg)
    assert np.array_equal(c.cpu().numpy(), ref)


@pytest.mark.parametrize("cfg", CONFIGS)
def test_gemm_bf16_packed_a_epilogues(cfg):
    M, K, I = 150, 256, 192
    x, w, sw, q, sx = _inputs(M, K, 2 * I, 51)
    pa, sx_d = ops.quant_rows_packed(x.to(DEV))
    assert np.array_equal(sx_d.cpu().numpy(), sx)
    y = orc.dequant(orc.int_mm_nk(q, w.numpy()), sx, sw.numpy())
    out = ops.gemm_bf16(pa, sx_d, packed_from_nk(w), sw.to(DEV), tile_cfg=cfg)
    assert np.array_equal(to_bits(out), y)
    g = ops.gemm_bf16(pa, sx_d, packed_from_nk(w, interleave=I), sw.to(DEV), epilogue="gelu", tile_cfg=cfg)
    assert_bf16_close(f32(to_bits(g)), f32(orc.gelu_mul(y)), what="gelu packed A")


# ---- long K ---------------------------------------------------------------------------------

def test_split_k_request_is_refused():
    """No configuration splits K across blocks: a request for it fails before launching."""
    from w8a8 import W8A8Error
    a = rand_i8((64, 256), 1).to(DEV)
    w = packed_from_nk(rand_i8((128, 256), 2))
    with pytest.raises(W8A8Error, match="never split"):
        ops.gemm_i32(a, w, split_k=4)


def test_linear_long_k_layer_shapes():
    """The M=512 micro-batch groups with long K (o: K=2048 N=1536; down: K=6144 N=1536), whose
    64x64 tiles have four waves split the k-steps and add their partials in LDS."""
    for K, N in ((2048, 1536), (6144, 1536)):
        x = workloads.activations(512, K, seed=K)
        w, sw = workloads.weights(N, K, seed=N + K)
        pw = ops.pack_weight(w.to(DEV), "nk", sw=sw.to(DEV))
        out = ops.linear_bf16(x.to(DEV), pw)
        ref, _, _ = orc.linear_bf16(to_bits(x), w.numpy(), sw.numpy())
        assert np.array_equal(to_bits(out), ref)


def test_long_k_repeated_launches_fresh_inputs():
    """Back-to-back launches of the wave split-K tile (M=512, K=6144, N=1536) with a different A each
    time: a partial tile left in LDS or an output written from the wrong launch would show up as a
    wrong product."""
    M, N, K = 512, 1536, 6144
    w = rand_i8((N, K), 71)
    pw = packed_from_nk(w)
    wt = w.t().contiguous()
    assert lib().w8a8_gemm_pick_tile_config(M, N, K, -1) == 3
    outs, refs = [], []
    for it in range(12):
        a = rand_i8((M, K), 100 + it)
        outs.append(ops.gemm_i32(ops.pack_act(a.to(DEV)), pw))
        refs.append(torch._int_mm(a, wt))
    for it, (c, r) in enumerate(zip(outs, refs)):
        assert torch.equal(c.cpu(), r), f"launch {it}"


def test_clock_probe_reads_a_plausible_engine_clock():
    """w8a8_clock_probe (the bench's clock reading): the core-clock / real-time ratio over a window
    is a clock between 0.5 and 3 GHz (MI355X tops out at 2.4 GHz), idle and with GEMMs running on
    another stream, and the window it reports is the one asked for."""
    import ctypes
    import bench
    from w8a8._lib import call
    out = torch.zeros(2, dtype=torch.int64, device=DEV)
    khz = ctypes.c_int(0)
    call("w8a8_clock_probe", out.data_ptr(), 20000, ctypes.byref(khz), torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    cycles, real = out.tolist()
    assert 10_000 <= khz.value <= 1_000_000
    assert 20000 <= real < 20000 + 5000
    idle = cycles / (real / (khz.value * 1e3)) / 1e9
    a = ops.pack_act(rand_i8((512, 1536), seed=1).to(DEV))
    w = packed_from_nk(rand_i8((12288, 1536), seed=2))
    c = torch.empty((512, 12288), dtype=torch.int32, device=DEV)
    busy = bench.clock_during(lambda: ops.gemm_i32(a, w, c=c), torch.device(DEV), launches=40)
    print(f"engine clock: idle {idle:.3f} GHz, under int8 GEMMs {busy:.3f} GHz")
    assert 0.5 < idle < 3.0 and 0.5 < busy < 3.0
