"""Shared test helpers: bf16 tolerance and tensor <-> numpy conversion."""
import numpy as np
import torch

# bf16 tolerance of the W8A8 path: |y - ref| <= max(REL * |ref|, ULPS * ulp_bf16(ref)).
REL = 1e-2
ULPS = 2


def ulp_bf16(v):
    """One bf16 unit in the last place at |v| (fp32 array in, fp32 array out)."""
    a = np.abs(np.asarray(v, dtype=np.float32))
    e = np.floor(np.log2(np.maximum(a, np.float32(2.0 ** -126))))
    return (2.0 ** (e - 7)).astype(np.float32)


def bf16_close(y, ref, rel=REL, ulps=ULPS):
    """Boolean mask of elements within tolerance; y, ref as fp32 arrays."""
    y = np.asarray(y, dtype=np.float32)
    ref = np.asarray(ref, dtype=np.float32)
    tol = np.maximum(rel * np.abs(ref), ulps * ulp_bf16(ref))
    return np.abs(y - ref) <= tol


def assert_bf16_close(y, ref, rel=REL, ulps=ULPS, what=""):
    ok = bf16_close(y, ref, rel, ulps)
    if not ok.all():
        bad = np.argwhere(~ok)
        i = tuple(bad[0])
        raise AssertionError(
            f"{what}: {len(bad)} of {ok.size} elements outside max({rel}*|ref|, {ulps} ulp); "
            f"first at {i}: got {np.asarray(y)[i]!r}, ref {np.asarray(ref)[i]!r}")


def to_bits(t):
    """bf16 tensor -> uint16 numpy bit patterns."""
    return t.detach().cpu().contiguous().view(torch.int16).numpy().view(np.uint16)


def from_bits(b):
    """uint16 numpy bit patterns -> bf16 CPU tensor."""
    return torch.from_numpy(np.ascontiguousarray(b).view(np.int16)).view(torch.bfloat16)


def f32(bits):
    return (np.asarray(bits, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)
