"""The real Gemma-4 E2B linear shapes beyond the uniform layer of the workload configs
(KV-shared layers with q only, full-attention layers with 512-wide heads, the double-wide MLP,
the per-layer-embedding gate / projection, N not a multiple of 512): int32 results bit-exact
against torch._int_mm on the CPU (the reference's cpu-int8 GEMM, pipeline.py:237), and the fused
GELU / residual epilogues against the oracle, at a ragged micro-batch and a full one."""
import numpy as np
import pytest
import torch

from helpers import assert_bf16_close, f32, to_bits

import oracle.oracle as orc
from w8a8 import ops, workloads

pytestmark = pytest.mark.gpu
DEV = "cuda"

SHAPES = {
    "q_kv_shared": (1536, 2048),       # KV-shared layer: the q projection alone
    "qkv_full_attn": (1536, 5120),     # 8 heads x 512 + 512 + 512
    "o_full_attn": (4096, 1536),
    "gate_up_double": (1536, 24576),   # double-wide MLP, [gate; up] of 12288 each
    "down_double": (12288, 1536),
    "ple_model_proj": (1536, 8960),    # 35 x 256
    "ple_gate": (1536, 256),
    "ple_proj": (256, 1536),
}


@pytest.mark.parametrize("M", [77, 512])
@pytest.mark.parametrize("name", list(SHAPES))
def test_real_shape_int32_exact(name, M):
    K, N = SHAPES[name]
    x = workloads.activations(M, K, seed=K + M)
    w, _ = workloads.weights(N, K, seed=N + 7)
    q, s = orc.quant_rows(to_bits(x), "bf16")
    c = ops.gemm_i32(torch.from_numpy(q).to(DEV), ops.pack_weight(w.to(DEV), "nk"))
    ref = torch._int_mm(torch.from_numpy(q), w.t().contiguous())
    assert torch.equal(c.cpu(), ref), name


def test_double_wide_gate_up_gelu():
    """gate_up of the double-wide MLP (I = 12288) with the fused GELU epilogue."""
    M, K, I = 77, 1536, 12288
    x = workloads.activations(M, K, seed=21)
    w, sw = workloads.weights(2 * I, K, seed=22)
    pw = ops.pack_weight(w.to(DEV), "nk", I, sw=sw.to(DEV))
    out = ops.linear_bf16(x.to(DEV), pw, epilogue="gelu")
    q, sx = orc.quant_rows(to_bits(x), "bf16")
    acc = torch._int_mm(torch.from_numpy(q), w.t().contiguous()).numpy()
    ref = orc.gelu_mul(orc.dequant(acc, sx, sw.numpy()))
    got = to_bits(out)
    assert_bf16_close(f32(got), f32(ref), what="double-wide gelu")
    assert (got == ref).mean() > 0.99


def test_double_wide_down_residual_rms():
    """down of the double-wide MLP (K = 12288) with the reference's residual + RMSNorm epilogue."""
    M, K, N = 77, 12288, 1536
    x = workloads.activations(M, K, seed=23)
    w, sw = workloads.weights(N, K, seed=24)
    res = workloads.activations(M, N, seed=25, outliers=False)
    g = torch.Generator().manual_seed(26)
    rw = (torch.rand(N, generator=g) + 0.5).to(torch.bfloat16)
    pw = ops.pack_weight(w.to(DEV), "nk", sw=sw.to(DEV))
    out = ops.linear_bf16(x.to(DEV), pw, epilogue="residual_rms", residual=res.to(DEV), rms_w=rw.to(DEV), eps=1e-6)
    q, sx = orc.quant_rows(to_bits(x), "bf16")
    acc = torch._int_mm(torch.from_numpy(q), w.t().contiguous()).numpy()
    ref = orc.rms_residual(orc.dequant(acc, sx, sw.numpy()), to_bits(res), to_bits(rw), 1e-6)
    got = to_bits(out)
    addends = np.maximum(np.abs(f32(to_bits(res))), np.abs(f32(ref) - f32(to_bits(res))))
    assert_bf16_close(f32(got), f32(ref), what="double-wide down", ulp_at=addends)
    assert (got == ref).mean() > 0.99
