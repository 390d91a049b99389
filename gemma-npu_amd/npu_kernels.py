"""Drop-in for the reference's `npu_kernels` module (npu_kernels.py:1-64), on MI355X.

Same names and call signature:

    mm_i8(a, b, c) -> c        a [M, K] int8, b [K, N] int8, c [M, N] int32; C = A @ B exactly
    use_npu()                  select this process's GPU for the calling thread
    BLOCK_M, BLOCK_N, BLOCK_K  the padding granules the reference's callers read
                               (gemma_npu.py:65, 67, 129); the HIP GEMM itself needs none

`b` is normally the PackedWeight returned by `resident.to_npu(w, static=True)` (the weight
stays resident in HBM in the MFMA layout); a plain int8 [K, N] tensor also works and is
packed on every call.  `a` and `c` may be host tensors (the reference's host-visible
resident buffers) or GPU tensors.

Completion is synchronous, as in the reference: its launch returns when C is ready, and the
worker thread that made it hands C to another thread straight away (pipeline.py:202-216;
gemma_npu.py:99-115).  So when mm_i8 returns, c holds the product and a may be refilled,
whichever thread called it and whatever stream the thread that reads c uses.  A caller that
reads c on the stream that launched it can pass wait=False to skip the final wait; the GEMM
is then ordered on torch's current stream like any other GPU op.

Importing this module also makes `from triton.backends.amd_triton_npu import resident`
resolve to `w8a8.resident`, so gemma_npu.py's NPUGemm runs on it unchanged.
"""
import importlib.util
import os
import sys
import types

import torch

from w8a8 import ops, resident
from w8a8.ops import PackedWeight

BLOCK_M = BLOCK_N = 512
BLOCK_K = 128

_DEVICE_INDEX = int(os.environ.get("W8A8_DEVICE", "0"))


def use_npu():
    """HIP device selection is per host thread, like the reference's per-thread driver
    (npu_kernels.py:20-26): call this first on a thread that launches GEMMs."""
    torch.cuda.set_device(_DEVICE_INDEX)


def _device():
    return torch.device("cuda", _DEVICE_INDEX)


def mm_i8(a, b, c, *, wait=True):
    """c[M, N] = a[M, K] @ b[K, N] (int8 x int8 -> int32, exact).  Returns c.

    Unlike the reference (npu_kernels.py:59-64), any M and N work, and a shape mismatch
    raises instead of truncating to multiples of 512.  With wait=True (the reference's
    contract) c is complete and a is no longer read when this returns.
    """
    if a.dtype != torch.int8 or a.dim() != 2:
        raise TypeError(f"mm_i8: a must be int8 [M, K], got {a.dtype} {tuple(a.shape)}")
    if c.dtype != torch.int32 or c.dim() != 2:
        raise TypeError(f"mm_i8: c must be int32 [M, N], got {c.dtype} {tuple(c.shape)}")
    M, K = a.shape
    if isinstance(b, PackedWeight):
        Kb, N = b.K, b.N
        dev = b.device
    else:
        if b.dtype != torch.int8 or b.dim() != 2:
            raise TypeError(f"mm_i8: b must be int8 [K, N], got {b.dtype} {tuple(b.shape)}")
        Kb, N = b.shape
        dev = b.device if b.is_cuda else (a.device if a.is_cuda else (c.device if c.is_cuda else _device()))
    if Kb != K:
        raise ValueError(f"mm_i8: a is [{M}, {K}] but b is [{Kb}, {N}]")
    if tuple(c.shape) != (M, N):
        raise ValueError(f"mm_i8: c is {tuple(c.shape)}, expected ({M}, {N})")
    if M == 0:
        return c
    w = b if isinstance(b, PackedWeight) else ops.pack_weight(b.to(dev), layout="kn")
    # A host `a` is copied synchronously: the caller may refill its staging rows as soon as
    # mm_i8 returns (gemma_npu.py:94-97, pipeline.py:241), even when c stays on the GPU.
    a_d = a if a.is_cuda else a.to(dev)
    if a_d.stride(1) != 1 or a_d.stride(0) % 16 or a_d.data_ptr() % 16:
        a_d = a_d.contiguous()
    if c.is_cuda and c.stride(1) == 1 and c.stride(0) % 4 == 0 and c.data_ptr() % 16 == 0:
        ops.gemm_i32(a_d, w, c)
    else:
        c_d = torch.empty((M, N), dtype=torch.int32, device=dev)
        ops.gemm_i32(a_d, w, c_d)
        c.copy_(c_d)  # a host c: this copy waits for the GEMM
    if wait and c.is_cuda:
        torch.cuda.current_stream(c.device).synchronize()
    return c


def _install_resident_alias():
    """Register w8a8.resident as triton.backends.amd_triton_npu.resident (gemma_npu.py:60, 88)."""
    name = "triton.backends.amd_triton_npu"
    if name in sys.modules:
        return
    if importlib.util.find_spec("triton") is None:
        for parent in ("triton", "triton.backends"):
            if parent not in sys.modules:
                m = types.ModuleType(parent)
                m.__path__ = []
                sys.modules[parent] = m
    mod = types.ModuleType(name)
    mod.__path__ = []
    mod.resident = resident
    sys.modules[name] = mod
    sys.modules[name + ".resident"] = resident


_install_resident_alias()
