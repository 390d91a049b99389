"""The int8 GEMM (npu_kernels.py:40-56) on the tile the library picks by itself, over seeded random
ragged shapes that cross the picker's rules (M around 1024 and past 8192, K from one k-tile to
12288, N from one 16-column tile to the double-wide gate/up): int32 bit-exact against an fp64
product on the GPU (every product and partial sum is an integer below 2^53, so the fp64 result is
exact), the dequant epilogue bit-exact against bf16((acc.float() * sx) * sw) (pipeline.py:55-57) and
the residual epilogue against that plus the residual in bf16."""
import numpy as np
import pytest
import torch

from w8a8 import ops

pytestmark = pytest.mark.gpu
DEV = "cuda"


def shapes():
    rng = np.random.default_rng(2026)
    out = []
    for lo, hi in ((1, 300), (300, 1100), (1000, 1100), (1100, 4200), (4000, 4200), (8190, 8400)):
        for _ in range(3):
            M = int(rng.integers(lo, hi + 1))
            N = int(rng.integers(1, 820)) * 16
            K = int(rng.choice([64, 128, 1536, 2048, 6144, 12288, int(rng.integers(1, 100)) * 64]))
            out.append((M, N, K))
    out += [(3658, 24576, 1536), (3658, 1536, 12288), (512, 12288, 1536), (17, 16, 64)]
    return out


@pytest.mark.parametrize("M,N,K", shapes())
def test_auto_tile_int32_and_dequant_exact(M, N, K):
    g = torch.Generator(device=DEV).manual_seed(M * 31 + N * 7 + K)
    a = torch.randint(-128, 128, (M, K), generator=g, dtype=torch.int8, device=DEV)
    w = torch.randint(-127, 128, (N, K), generator=g, dtype=torch.int8, device=DEV)
    sx = torch.rand(M, generator=g, device=DEV) * 0.05 + 1e-3
    sw = torch.rand(N, generator=g, device=DEV) * 0.015 + 0.005
    pw = ops.pack_weight(w, "nk", sw=sw)
    print(f"auto tile M={M} N={N} K={K}", flush=True)
    c = ops.gemm_i32(a, pw)
    want = (a.double() @ w.double().T).long()
    assert torch.equal(c.long(), want), f"int32 mismatch at M={M} N={N} K={K}"
    y = ops.gemm_bf16(a, sx, pw)
    ref = ((want.int().float() * sx[:, None]) * sw[None, :]).to(torch.bfloat16)
    assert torch.equal(y.view(torch.int16), ref.view(torch.int16)), f"dequant mismatch at M={M} N={N} K={K}"
    r = torch.randn(M, N, generator=g, device=DEV).to(torch.bfloat16)
    yr = ops.gemm_bf16(a, sx, pw, epilogue="residual", residual=r)
    assert torch.equal(yr.view(torch.int16), (ref + r).view(torch.int16)), f"residual mismatch at M={M} N={N} K={K}"
