"""Resident memory for the W8A8 engine, in place of Triton-XDNA's `resident` module.

The reference allocates host memory shared with the NPU (gemma_npu.py:75, 89-92):
`to_npu(w, static=True)` uploads a weight once and never syncs it again, `to_npu(t)` and
`empty(n, dtype=)` give host buffers the NPU reads and writes in place.  Here:

  * `to_npu(w, static=True)` packs the int8 [K, N] weight into the GPU-resident MFMA layout
    and returns a `PackedWeight` that `npu_kernels.mm_i8` takes as its `b`;
  * `to_npu(t)` and `empty(n, dtype)` return pinned host tensors (the caller fills and reads
    them on the CPU exactly as before; `mm_i8` moves rows across PCIe), or device tensors
    when `device=` names a GPU, for callers that keep their neighbouring ops on the GPU.
"""
import torch

from . import ops


def _device(device):
    if device is None:
        return torch.device("cuda", torch.cuda.current_device())
    return torch.device(device)


def to_npu(t, static=False, device=None):
    """Static int8 [K, N] weights -> PackedWeight on the GPU; anything else -> a resident copy."""
    if static:
        if t.dtype != torch.int8 or t.dim() != 2:
            raise TypeError(f"static resident weights are int8 [K, N], got {t.dtype} {tuple(t.shape)}")
        dev = _device(device if device is not None else (t.device if t.is_cuda else None))
        return ops.pack_weight(t.to(dev).contiguous(), layout="kn")
    if device is not None and torch.device(device).type == "cuda":
        return t.to(device).contiguous()
    out = torch.empty(t.shape, dtype=t.dtype, pin_memory=True)
    out.copy_(t)
    return out


def empty(n, dtype=torch.int8, device=None):
    """A flat resident buffer of n elements: pinned host memory, or GPU memory if `device` is a GPU."""
    if isinstance(n, (tuple, list)):
        shape = tuple(n)
    else:
        shape = (int(n),)
    if device is not None and torch.device(device).type == "cuda":
        return torch.empty(shape, dtype=dtype, device=device)
    return torch.empty(shape, dtype=dtype, pin_memory=True)
