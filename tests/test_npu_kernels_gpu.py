"""The drop-in module: npu_kernels.mm_i8(a, b, c) with the reference's call pattern
(npu_kernels.py:59-64; gemma_npu.py:75, 89-115) runs on the HIP GEMM and is exact."""
import pytest
import torch

import npu_kernels
from w8a8 import resident

pytestmark = pytest.mark.gpu


def test_mm_i8_device_tensors_returns_c():
    g = torch.Generator().manual_seed(0)
    a = torch.randint(-128, 128, (512, 1536), generator=g, dtype=torch.int8)
    b = torch.randint(-128, 128, (1536, 1024), generator=g, dtype=torch.int8)
    c = torch.zeros((512, 1024), dtype=torch.int32, device="cuda")
    out = npu_kernels.mm_i8(a.cuda(), b.cuda(), c)
    assert out is c
    assert torch.equal(c.cpu(), torch._int_mm(a, b))


def test_mm_i8_resident_pattern_of_the_reference():
    """NPUGemm: static resident weight [K, N_pad], host slot buffers, 512-row chunks."""
    npu_kernels.use_npu()
    from triton.backends.amd_triton_npu import resident as aliased  # the reference's import
    assert aliased is resident
    K, N, n_pad, T = 1536, 2560, 3072, 700
    g = torch.Generator().manual_seed(1)
    q = torch.randint(-127, 128, (N, K), generator=g, dtype=torch.int8)
    wt = torch.zeros((K, n_pad), dtype=torch.int8)
    wt[:, :N] = q.t()
    w = resident.to_npu(wt, static=True)
    rows = -(-T // npu_kernels.BLOCK_M) * npu_kernels.BLOCK_M
    a_flat = resident.empty(rows * K, dtype=torch.int8)
    c_flat = resident.empty(rows * n_pad, dtype=torch.int32)
    xq = torch.randint(-127, 128, (T, K), generator=g, dtype=torch.int8)
    a_flat[: rows * K].view(rows, K)[:T].copy_(xq)
    a_flat[T * K: rows * K].zero_()
    for r0 in range(0, rows, npu_kernels.BLOCK_M):
        av = a_flat[r0 * K: (r0 + 512) * K].view(512, K)
        cv = c_flat[r0 * n_pad: (r0 + 512) * n_pad].view(512, n_pad)
        npu_kernels.mm_i8(av, w, cv)
    c = c_flat[: rows * n_pad].view(rows, n_pad)[:T, :N]
    assert torch.equal(c, torch._int_mm(xq, q.t().contiguous()))


def test_mm_i8_any_m_no_padding():
    g = torch.Generator().manual_seed(2)
    a = torch.randint(-128, 128, (3658, 128), generator=g, dtype=torch.int8)
    b = torch.randint(-128, 128, (128, 200), generator=g, dtype=torch.int8)
    c = torch.empty((3658, 200), dtype=torch.int32)
    npu_kernels.mm_i8(a, b, c)
    assert torch.equal(c, torch._int_mm(a, b))


def test_mm_i8_rejects_mismatched_shapes():
    a = torch.zeros((4, 64), dtype=torch.int8, device="cuda")
    b = torch.zeros((128, 32), dtype=torch.int8, device="cuda")
    with pytest.raises(ValueError):
        npu_kernels.mm_i8(a, b, torch.zeros((4, 32), dtype=torch.int32, device="cuda"))
    b = torch.zeros((64, 32), dtype=torch.int8, device="cuda")
    with pytest.raises(ValueError):
        npu_kernels.mm_i8(a, b, torch.zeros((4, 31), dtype=torch.int32, device="cuda"))
