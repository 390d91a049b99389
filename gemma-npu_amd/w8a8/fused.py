"""The reference's fused kernels between the GEMMs, on the GPU (pipeline.py:66-127).

Same names, arguments and results as the torch.compile'd CPU functions of the reference's
pipeline, so a caller swaps the module and keeps its code:

    k_in(h, w, eps)                                          -> (xq, sx)      pipeline.py:66-69
    k_qkv(acc, sx, sw, cos, sin, qw, kw, eps, H, KV, D, shared) -> (q, k, v)  pipeline.py:72-85
    k_attn_out(o)                                            -> (xq, sx)      pipeline.py:88-92
    k_post_attn(acc, sx, sw, res, w_post, w_pre_ff, eps)     -> (h, xq, sx)   pipeline.py:95-99
    k_gelu(acc, sx, sw, I)                                   -> (xq, sx)      pipeline.py:102-107
    k_post_ff(acc, sx, sw, res, w_post_ff, eps)              -> (h, xq, sx)   pipeline.py:110-114
    k_ple_gate(acc, sx, sw, ple)                             -> (xq, sx)      pipeline.py:117-121
    k_ple_out(acc, sx, sw, h, w_post_ple, scalar, eps)       -> h             pipeline.py:124-127

acc is the int32 GEMM result [T, N] (rows contiguous, any row stride, as the reference's
strided view of its result buffer), sx fp32 [T] and sw fp32 [N] its scales; activations and
norm weights are bf16.  k_qkv, k_post_attn, k_post_ff, k_ple_gate and k_ple_out also take, as acc,
the dequantised bf16 rows bf16((acc * sx) * sw) that the GEMM's dequant epilogue writes (sx and sw
are then not read and may be None): the kernels' first step is that dequant, so the results are
bit-identical and the GEMM writes half the bytes.  xq is int8 [T, K] row-major, or, with packed=True, a PackedActivation
that the GEMM reads fastest.  q / k / v of k_qkv are contiguous [heads, T, D] tensors holding
the values of the reference's transposed views.  Everything runs on torch's current stream of
the tensors' device; there is no CPU fallback.
"""
import torch

from ._lib import call
from .ops import PackedActivation, _check, _ld, _same_device, _stream, packed_act_bytes


def _vec(t, name, n):
    """A bf16 [n] norm weight, or None."""
    if t is None:
        return None
    _check(t, name, torch.bfloat16, 1)
    if t.shape[0] != n:
        raise ValueError(f"{name}: expected {n} elements, got {t.shape[0]}")
    return t.data_ptr()


def _acc(acc, sx, sw, ncols, dequantised_ok=False):
    """Checks acc (int32 with its scales, or with dequantised_ok the bf16 rows); True if it is bf16."""
    if dequantised_ok and isinstance(acc, torch.Tensor) and acc.dtype == torch.bfloat16:
        _check(acc, "acc", torch.bfloat16)
        if acc.shape[1] < ncols:
            raise ValueError(f"acc {tuple(acc.shape)} does not cover {ncols} columns")
        return True
    _check(acc, "acc", torch.int32)
    _check(sx, "sx", torch.float32, 1)
    _check(sw, "sw", torch.float32, 1)
    if acc.shape[1] < ncols or sx.shape[0] != acc.shape[0] or sw.shape[0] < ncols:
        raise ValueError(f"acc {tuple(acc.shape)} / sx {tuple(sx.shape)} / sw {tuple(sw.shape)} do not cover "
                         f"{ncols} columns")
    return False


def _q_out(M, N, device, packed):
    """(q tensor, ldq, packed flag, result object) for M rows of N int8 values."""
    if packed:
        buf = torch.empty(max(packed_act_bytes(M, N), 1), dtype=torch.int8, device=device)
        return buf, 0, 1, PackedActivation(buf, M, N)
    q = torch.empty((M, N), dtype=torch.int8, device=device)
    return q, N, 0, q


def _rows(t, name, M, N):
    _check(t, name, torch.bfloat16)
    if tuple(t.shape) != (M, N):
        raise ValueError(f"{name}: expected shape {(M, N)}, got {tuple(t.shape)}")
    return t.data_ptr(), _ld(t)


def k_in(h, w, eps, packed=False):
    """input_layernorm -> int8 rows for q/k/v: quant(bf16(rms(h, w)))."""
    _check(h, "h", torch.bfloat16)
    M, N = h.shape
    wp = _vec(w, "w", N)
    q, ldq, qp, xq = _q_out(M, N, h.device, packed)
    sx = torch.empty((M,), dtype=torch.float32, device=h.device)
    _same_device(h, w)
    call("w8a8_k_in", h.data_ptr(), _ld(h), wp, float(eps), M, N, q.data_ptr(), ldq, qp, sx.data_ptr(), _stream(h))
    return xq, sx


def k_qkv(acc, sx, sw, cos, sin, qw, kw, eps, H, KV, D, shared):
    """q/k/v GEMM out -> normed, rotated q [H, T, D], k, v [KV, T, D] (bf16)."""
    H, KV, D = int(H), int(KV), int(D)
    slots = H if shared else H + 2 * KV
    y = _acc(acc, sx, sw, slots * D, dequantised_ok=True)
    T = acc.shape[0]
    for t, name in ((cos, "cos"), (sin, "sin")):
        _check(t, name, torch.bfloat16)
        if t.shape[0] != T or t.shape[1] != D:
            raise ValueError(f"{name}: expected shape {(T, D)}, got {tuple(t.shape)}")
    if cos.stride(0) != sin.stride(0):
        raise ValueError("cos and sin must share a row stride")
    qwp = _vec(qw, "qw", D)
    kwp = None if shared else _vec(kw, "kw", D)
    dev = acc.device
    q = torch.empty((H, T, D), dtype=torch.bfloat16, device=dev)
    k = v = None
    if not shared:
        k = torch.empty((KV, T, D), dtype=torch.bfloat16, device=dev)
        v = torch.empty((KV, T, D), dtype=torch.bfloat16, device=dev)
    if y:
        _same_device(acc, cos, sin, qw, kw)
        call("w8a8_k_qkv_y", acc.data_ptr(), _ld(acc), cos.data_ptr(), sin.data_ptr(), _ld(cos), qwp, kwp,
             float(eps), T, H, KV, D, 1 if shared else 0, q.data_ptr(), None if shared else k.data_ptr(),
             None if shared else v.data_ptr(), _stream(acc))
    else:
        _same_device(acc, sx, sw, cos, sin, qw, kw)
        call("w8a8_k_qkv", acc.data_ptr(), _ld(acc), sx.data_ptr(), sw.data_ptr(), cos.data_ptr(), sin.data_ptr(),
             _ld(cos), qwp, kwp, float(eps), T, H, KV, D, 1 if shared else 0, q.data_ptr(),
             None if shared else k.data_ptr(), None if shared else v.data_ptr(), _stream(acc))
    if shared:
        return q, q, q
    return q, k, v


def k_qkv_cache(y, cos, sin, qw, kw, eps, H, KV, D, k_cache, v_cache, pos):
    """k_qkv on the decode step's bf16 GEMV rows y [T, (H + 2KV) D] (not a KV-shared layer), writing
    the keys and values straight into the cache [KV, rows, D] at rows pos[0] + t (pos: an int32 device
    tensor of one element; rows outside the cache are not written) -> q [H, T, D]."""
    H, KV, D = int(H), int(KV), int(D)
    _check(y, "y", torch.bfloat16)
    T = y.shape[0]
    if y.shape[1] < (H + 2 * KV) * D:
        raise ValueError(f"y {tuple(y.shape)} does not cover {(H + 2 * KV) * D} columns")
    for t, name in ((cos, "cos"), (sin, "sin")):
        _check(t, name, torch.bfloat16)
        if t.shape[0] != T or t.shape[1] != D:
            raise ValueError(f"{name}: expected shape {(T, D)}, got {tuple(t.shape)}")
    if cos.stride(0) != sin.stride(0):
        raise ValueError("cos and sin must share a row stride")
    for t, name in ((k_cache, "k_cache"), (v_cache, "v_cache")):
        if not isinstance(t, torch.Tensor) or t.dtype != torch.bfloat16 or t.dim() != 3 or not t.is_contiguous():
            raise ValueError(f"{name} must be a contiguous bf16 tensor [KV, rows, D]")
        if t.shape[0] != KV or t.shape[2] != D:
            raise ValueError(f"{name}: expected [{KV}, rows, {D}], got {tuple(t.shape)}")
    if k_cache.shape != v_cache.shape:
        raise ValueError("k_cache and v_cache differ in shape")
    if not isinstance(pos, torch.Tensor) or pos.dtype != torch.int32 or pos.numel() != 1:
        raise ValueError("pos must be an int32 tensor of one element")
    q = torch.empty((H, T, D), dtype=torch.bfloat16, device=y.device)
    _same_device(y, cos, sin, qw, kw, k_cache, v_cache, pos)
    call("w8a8_k_qkv_cache_y", y.data_ptr(), _ld(y), cos.data_ptr(), sin.data_ptr(), _ld(cos), _vec(qw, "qw", D),
         _vec(kw, "kw", D), float(eps), T, H, KV, D, q.data_ptr(), k_cache.data_ptr(), v_cache.data_ptr(),
         k_cache.shape[1], pos.data_ptr(), _stream(y))
    return q


def k_attn_out(o, packed=False):
    """attention output [H, T, D] -> int8 rows [T, H*D] for o_proj."""
    _check(o, "o", torch.bfloat16, 3)
    H, T, D = o.shape
    if D > 1 and o.stride(2) != 1:
        raise ValueError(f"o: the last dimension must be contiguous, got strides {o.stride()}")
    q, ldq, qp, xq = _q_out(T, H * D, o.device, packed)
    sx = torch.empty((T,), dtype=torch.float32, device=o.device)
    call("w8a8_k_attn_out", o.data_ptr(), o.stride(0) if H > 1 else D, o.stride(1) if T > 1 else D, H, T, D,
         q.data_ptr(), ldq, qp, sx.data_ptr(), _stream(o))
    return xq, sx


def k_post_attn(acc, sx, sw, res, w_post, w_pre_ff, eps, packed=False):
    """o_proj out -> residual add -> pre-FFN norm -> int8 rows for gate/up: (h, xq, sx)."""
    M, N = res.shape
    y = _acc(acc, sx, sw, N, dequantised_ok=True)
    rp, ldr = _rows(res, "res", M, N)
    h = torch.empty((M, N), dtype=torch.bfloat16, device=res.device)
    q, ldq, qp, xq = _q_out(M, N, res.device, packed)
    sq = torch.empty((M,), dtype=torch.float32, device=res.device)
    tail = (rp, ldr, _vec(w_post, "w_post", N), _vec(w_pre_ff, "w_pre_ff", N), float(eps), M, N, h.data_ptr(), N,
            q.data_ptr(), ldq, qp, sq.data_ptr(), _stream(acc))
    if y:
        _same_device(acc, res, w_post, w_pre_ff)
        call("w8a8_k_post_attn_y", acc.data_ptr(), _ld(acc), *tail)
    else:
        _same_device(acc, sx, sw, res, w_post, w_pre_ff)
        call("w8a8_k_post_attn", acc.data_ptr(), _ld(acc), sx.data_ptr(), sw.data_ptr(), *tail)
    return h, xq, sq


def k_gelu(acc, sx, sw, I, packed=False):
    """gate/up out [T, 2I] -> gelu(gate) * up -> int8 rows for down_proj."""
    I = int(I)
    _acc(acc, sx, sw, 2 * I)
    M = acc.shape[0]
    q, ldq, qp, xq = _q_out(M, I, acc.device, packed)
    sq = torch.empty((M,), dtype=torch.float32, device=acc.device)
    _same_device(acc, sx, sw)
    call("w8a8_k_gelu", acc.data_ptr(), _ld(acc), sx.data_ptr(), sw.data_ptr(), M, I, q.data_ptr(), ldq, qp,
         sq.data_ptr(), _stream(acc))
    return xq, sq


def k_post_ff(acc, sx, sw, res, w_post_ff, eps, packed=False):
    """down_proj out -> residual add -> int8 rows for the PLE gate: (h, xq, sx)."""
    M, N = res.shape
    y = _acc(acc, sx, sw, N, dequantised_ok=True)
    rp, ldr = _rows(res, "res", M, N)
    h = torch.empty((M, N), dtype=torch.bfloat16, device=res.device)
    q, ldq, qp, xq = _q_out(M, N, res.device, packed)
    sq = torch.empty((M,), dtype=torch.float32, device=res.device)
    tail = (rp, ldr, _vec(w_post_ff, "w_post_ff", N), float(eps), M, N, h.data_ptr(), N, q.data_ptr(), ldq, qp,
            sq.data_ptr(), _stream(acc))
    if y:
        _same_device(acc, res, w_post_ff)
        call("w8a8_k_post_ff_y", acc.data_ptr(), _ld(acc), *tail)
    else:
        _same_device(acc, sx, sw, res, w_post_ff)
        call("w8a8_k_post_ff", acc.data_ptr(), _ld(acc), sx.data_ptr(), sw.data_ptr(), *tail)
    return h, xq, sq


def k_ple_gate(acc, sx, sw, ple, packed=False):
    """PLE gate out -> gelu * this layer's per-layer input -> int8 rows."""
    M, N = ple.shape
    y = _acc(acc, sx, sw, N, dequantised_ok=True)
    pp, ldp = _rows(ple, "ple", M, N)
    q, ldq, qp, xq = _q_out(M, N, ple.device, packed)
    sq = torch.empty((M,), dtype=torch.float32, device=ple.device)
    tail = (pp, ldp, M, N, q.data_ptr(), ldq, qp, sq.data_ptr(), _stream(acc))
    if y:
        _same_device(acc, ple)
        call("w8a8_k_ple_gate_y", acc.data_ptr(), _ld(acc), *tail)
    else:
        _same_device(acc, sx, sw, ple)
        call("w8a8_k_ple_gate", acc.data_ptr(), _ld(acc), sx.data_ptr(), sw.data_ptr(), *tail)
    return xq, sq


def k_ple_out(acc, sx, sw, h, w_post_ple, scalar, eps, norm_next=None, packed=False):
    """PLE projection out -> residual add -> layer scalar: bf16(bf16(h + rms(y)) * scalar).

    scalar: a one-element bf16 tensor on the device (the layer scalar), or a Python number,
    which is rounded to bf16 first.  With norm_next (the next layer's input-norm weight) the same
    launch also runs that layer's k_in on the rows it writes: returns (out, xq, sx_next), xq packed
    or row-major as k_in's."""
    M, N = h.shape
    y = _acc(acc, sx, sw, N, dequantised_ok=True)
    hp, ldh = _rows(h, "h", M, N)
    if not isinstance(scalar, torch.Tensor):
        scalar = torch.tensor([float(scalar)], dtype=torch.bfloat16, device=h.device)
    if scalar.dtype != torch.bfloat16 or scalar.numel() != 1 or scalar.device != h.device:
        raise ValueError("k_ple_out: scalar must be one bf16 value on the tensors' device")
    scalar = scalar.reshape(1).contiguous()
    out = torch.empty((M, N), dtype=torch.bfloat16, device=h.device)
    if norm_next is None:
        tail = (hp, ldh, _vec(w_post_ple, "w_post_ple", N), scalar.data_ptr(), float(eps), M, N, out.data_ptr(), N,
                _stream(acc))
        name = "w8a8_k_ple_out"
    else:
        q, ldq, qp, xq = _q_out(M, N, h.device, packed)
        sxn = torch.empty((M,), dtype=torch.float32, device=h.device)
        tail = (hp, ldh, _vec(w_post_ple, "w_post_ple", N), scalar.data_ptr(), _vec(norm_next, "norm_next", N),
                float(eps), M, N, out.data_ptr(), N, q.data_ptr(), ldq, qp, sxn.data_ptr(), _stream(acc))
        name = "w8a8_k_ple_out_k_in"
    if y:
        _same_device(acc, h, w_post_ple, norm_next)
        call(name + "_y", acc.data_ptr(), _ld(acc), *tail)
    else:
        _same_device(acc, sx, sw, h, w_post_ple, norm_next)
        call(name, acc.data_ptr(), _ld(acc), sx.data_ptr(), sw.data_ptr(), *tail)
    return out if norm_next is None else (out, xq, sxn)
