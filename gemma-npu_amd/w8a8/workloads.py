"""Shapes and seeded synthetic inputs of the W8A8 workloads (Gemma-4 E2B-class prefill / decode).

Group layout follows the reference's fused linears (gemma_npu.py:213-224): [q; k; v] and
[gate; up] are concatenated along N, so one decoder layer's prefill is four GEMMs, plus the
per-layer-embedding model projection once per prompt.

Inputs are generated on the CPU from torch.Generator seeds so that every run, here or on a
GPU host, sees the same numbers:
  activations  bf16 N(0, 1) with round(0.001 * M * K) distinct entries scaled by 20
               (outliers), optionally each row scaled by 10**U(-2, 2);
  weights      int8 uniform over [-127, 127], fp32 per-channel scales U(0.005, 0.02).
"""
import torch

HIDDEN = 1536
LAYER_GROUPS = {
    # name: (K, N, epilogue); N of gate_up is 2 x 6144 in [gate; up] order.
    "qkv": (1536, 2048 + 256 + 256, "none"),
    "o": (2048, 1536, "none"),
    "gate_up": (1536, 2 * 6144, "gelu"),
    "down": (6144, 1536, "residual"),
}
PLE_PROJ = (1536, 8960, "none")
N_LAYERS = 35
LM_HEAD = (1536, 262144)  # K, N (vocabulary)


def activations(M, K, seed, outliers=True, row_spread=False):
    """bf16 [M, K] on the CPU."""
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(M, K, generator=g)
    if outliers:
        n_out = round(0.001 * M * K)
        if n_out:
            idx = torch.unique(torch.randint(0, M * K, (n_out + n_out // 8 + 16,), generator=g))
            while idx.numel() < n_out:
                idx = torch.unique(torch.cat([idx, torch.randint(0, M * K, (n_out,), generator=g)]))
            idx = idx[torch.randperm(idx.numel(), generator=g)[:n_out]]
            x.view(-1)[idx] *= 20.0
    if row_spread:
        x *= 10.0 ** (torch.rand(M, 1, generator=g) * 4.0 - 2.0)
    return x.to(torch.bfloat16)


def weights(N, K, seed):
    """(int8 [N, K] uniform over [-127, 127], fp32 [N] scales in U(0.005, 0.02)) on the CPU."""
    g = torch.Generator().manual_seed(seed)
    w = torch.randint(-127, 128, (N, K), generator=g, dtype=torch.int8)
    sw = torch.rand(N, generator=g) * 0.015 + 0.005
    return w, sw


def single_gemm_inputs(M=512, K=1536, N=6144, seed=0):
    """The single prefill micro-batch GEMM (M=512, K=1536, N=6144): bf16 activations (with outliers)
    and int8 weights with their scales, both drawn from one seed (0 by default)."""
    x = activations(M, K, seed)
    w, sw = weights(N, K, seed)
    return x, w, sw


def layer_seed(layer, group):
    """Seed of one layer's weight group in the full-prefill sweep (distinct per layer)."""
    return 1000 + 16 * layer + group


def gemm_ops(M, N, K):
    """Algorithmic int8 ops of one GEMM: 2*M*N*K on the real (unpadded) sizes."""
    return 2 * M * N * K


def sweep_shapes():
    """The (K, N) of every GEMM in one prefill: 35 layers x 4 groups + the PLE projection."""
    shapes = []
    for layer in range(N_LAYERS):
        for gi, (name, (K, N, epi)) in enumerate(LAYER_GROUPS.items()):
            shapes.append((name, layer, gi, K, N))
    shapes.append(("ple_proj", -1, 0, PLE_PROJ[0], PLE_PROJ[1]))
    return shapes
