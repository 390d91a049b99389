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


def bf16_close(y, ref, rel=REL, ulps=ULPS, ulp_at=None, extra=None):
    """Boolean mask of elements within tolerance; y, ref as fp32 arrays.

    ulp_at: magnitudes at which to take the ulp instead of |ref| (for a sum a + b the rounding
            error of each addend is an ulp of that addend, not of the sum: pass max(|a|, |b|)).
    extra:  an additional absolute allowance per element (e.g. the fp32 dot-product error
            bound of a long accumulation, see dot_error_bound).
    """
    y = np.asarray(y, dtype=np.float32)
    ref = np.asarray(ref, dtype=np.float32)
    mag = np.abs(ref) if ulp_at is None else np.maximum(np.abs(ref), np.abs(np.asarray(ulp_at, np.float32)))
    tol = np.maximum(rel * np.abs(ref), ulps * ulp_bf16(mag))
    if extra is not None:
        tol = np.maximum(tol, np.asarray(extra, dtype=np.float32))
    return np.abs(y - ref) <= tol


def dot_error_bound(x, w, s):
    """Absolute error allowance of y = (sum_k x[m,k] w[n,k]) * s[n] accumulated in fp32 in any
    order: 4 * 2^-24 * sum_k |x w| * |s|.  Two fp32 accumulations of the same products (the
    oracle's sequential sum, torch's vectorised one, the MFMA's) may each be off by rounding
    of the running sum, which matters only where the sum cancels to near zero."""
    xa = torch.as_tensor(np.abs(np.asarray(x, np.float32)))
    wa = torch.as_tensor(np.abs(np.asarray(w, np.float32)))
    return (4.0 * 2.0 ** -24) * (xa @ wa.T).numpy() * np.abs(np.asarray(s, np.float32))[None, :]


def assert_bf16_close(y, ref, rel=REL, ulps=ULPS, what="", ulp_at=None, extra=None):
    ok = bf16_close(y, ref, rel, ulps, ulp_at, extra)
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
