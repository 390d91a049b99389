"""torch-facing wrappers of the libw8a8 C ABI.

Every function takes device tensors on a ROCm GPU, checks dtype / layout on the host, and
launches on torch's current stream for that device.  Results are stream-ordered: they are
ready for any later work on the same stream.  There is no CPU fallback.
"""
import torch

from ._lib import call, lib

EPILOGUES = {"none": 0, "gelu": 1, "residual": 2, "residual_rms": 3}


# torch's current HIP stream of a device as a raw handle.  torch.cuda.current_stream() builds a
# Python Stream object on every call (~2 us); the raw-handle accessor it is built on does not.
_RAW_STREAM = getattr(torch._C, "_cuda_getCurrentRawStream", None)


def current_stream_handle(device):
    """The raw hipStream_t of torch's current stream on `device` (a torch.device or index)."""
    index = device if isinstance(device, int) else device.index
    if index is None:
        index = torch.cuda.current_device()
    if _RAW_STREAM is not None:
        return _RAW_STREAM(index)
    return torch.cuda.current_stream(index).cuda_stream


def _stream(t):
    return current_stream_handle(t.device)


def _check(t, name, dtype, ndim=2):
    if not isinstance(t, torch.Tensor):
        raise TypeError(f"{name}: expected a tensor, got {type(t).__name__}")
    if t.device.type != "cuda":
        raise ValueError(f"{name}: expected a GPU tensor, got device {t.device}")
    if t.dtype != dtype:
        raise TypeError(f"{name}: expected {dtype}, got {t.dtype}")
    if t.dim() != ndim:
        raise ValueError(f"{name}: expected {ndim}-D, got shape {tuple(t.shape)}")
    if ndim == 2 and t.shape[1] > 1 and t.stride(1) != 1:
        raise ValueError(f"{name}: rows must be contiguous (stride(1) == 1), got strides {t.stride()}")
    if ndim == 1 and t.shape[0] > 1 and t.stride(0) != 1:
        raise ValueError(f"{name}: must be contiguous")


def _ld(t):
    return t.stride(0) if t.shape[0] > 1 else max(t.shape[1], 1)


def workspace(device, nbytes):
    """Scratch of at least nbytes on device for one call on the current stream (the linear's packed
    int8 rows and row scales: nothing is kept between calls).  It comes from torch's caching
    allocator, which ties the block to the current stream, so no buffer outlives its stream and no
    stream reuses another's while that one may still be running."""
    return torch.empty(max(int(nbytes), 256), dtype=torch.uint8, device=torch.device(device))


def _same_device(*ts):
    devs = {t.device for t in ts if t is not None}
    if len(devs) > 1:
        raise ValueError(f"tensors on different devices: {sorted(map(str, devs))}")


class PackedWeight:
    """An int8 weight resident on the GPU in the GEMM's MFMA-fragment layout.

    N output channels x K inputs; `interleave` = I > 0 marks a [gate; up] pair (N = 2I)
    packed for the fused GELU epilogue.  `sw` (fp32 [N]) optionally carries the
    per-channel scales that belong to it.
    """

    __slots__ = ("data", "N", "K", "interleave", "sw")

    def __init__(self, data, N, K, interleave=0, sw=None):
        self.data, self.N, self.K, self.interleave, self.sw = data, int(N), int(K), int(interleave), sw

    @property
    def device(self):
        return self.data.device

    @property
    def shape(self):
        """(K, N), the shape of the reference's B operand (npu_kernels.py:46)."""
        return (self.K, self.N)

    def __repr__(self):
        return f"PackedWeight(N={self.N}, K={self.K}, interleave={self.interleave}, device={self.device})"


def packed_weight_bytes(N, K, interleave=0):
    n = lib().w8a8_packed_weight_bytes(N, K, interleave)
    if n < 0:
        raise ValueError(f"invalid packed weight shape N={N} K={K} interleave={interleave}")
    return n


def pack_weight(w, layout="nk", interleave=0, sw=None):
    """int8 weight -> PackedWeight.  layout "nk": w is [N, K] (gemma_npu.py:69);
    "kn": w is [K, N], the reference GEMM's B operand (npu_kernels.py:46)."""
    _check(w, "w", torch.int8)
    if layout == "nk":
        N, K = w.shape
        fn = "w8a8_pack_weight_nk"
    elif layout == "kn":
        K, N = w.shape
        fn = "w8a8_pack_weight_kn"
    else:
        raise ValueError(f"layout must be 'nk' or 'kn', got {layout!r}")
    nbytes = packed_weight_bytes(N, K, interleave)
    data = torch.empty(nbytes, dtype=torch.int8, device=w.device)
    ld = w.stride(0) if w.shape[0] > 1 else w.shape[1]
    call(fn, w.data_ptr(), ld, *((N, K) if layout == "nk" else (K, N)), interleave, data.data_ptr(), _stream(w))
    return PackedWeight(data, N, K, interleave, sw)


def unpair_packed(pw):
    """The plain packing of a [gate; up] PackedWeight packed for the GELU epilogue, without the
    int8 source.  Both layouts store whole 32-channel tiles as contiguous blocks of KF KiB; the
    paired one orders them gate 0, up 0, gate 1, up 1, ..., the plain one gate 0 .. I/32-1 then
    up 0 .. I/32-1, so the plain weight is a permutation of the paired one's blocks."""
    if not isinstance(pw, PackedWeight) or pw.interleave <= 0:
        raise ValueError("unpair_packed: expects a PackedWeight packed with interleave > 0")
    nt = pw.N // 32
    blocks = pw.data.view(nt, -1)
    perm = torch.cat([torch.arange(0, nt, 2), torch.arange(1, nt, 2)]).to(blocks.device)
    return PackedWeight(blocks.index_select(0, perm).reshape(-1), pw.N, pw.K, 0, pw.sw)


def quant_rows(x, q=None, scale=None):
    """Per-row int8 quant of bf16 or fp32 rows (pipeline.py:49-52) -> (q int8 [M,K], scale fp32 [M])."""
    if x.dtype not in (torch.bfloat16, torch.float32):
        raise TypeError(f"quant_rows: x must be bf16 or fp32, got {x.dtype}")
    _check(x, "x", x.dtype)
    M, K = x.shape
    if q is None:
        q = torch.empty((M, K), dtype=torch.int8, device=x.device)
    if scale is None:
        scale = torch.empty((M,), dtype=torch.float32, device=x.device)
    _check(q, "q", torch.int8)
    _check(scale, "scale", torch.float32, 1)
    if tuple(q.shape) != (M, K) or scale.shape[0] != M:
        raise ValueError("quant_rows: output shapes do not match x")
    _same_device(x, q, scale)
    fn = "w8a8_quant_rows_bf16" if x.dtype == torch.bfloat16 else "w8a8_quant_rows_f32"
    call(fn, x.data_ptr(), _ld(x), M, K, q.data_ptr(), _ld(q), scale.data_ptr(), _stream(x))
    return q, scale


def quant_weight(w, layout="nk", interleave=0):
    """Float weight [N, K] -> PackedWeight with per-output-channel fp32 scales
    (absmax/127 per channel, gemma_npu.py:68-69)."""
    if layout != "nk":
        raise ValueError("quant_weight takes a float [N, K] weight")
    q, sw = quant_rows(w.contiguous())
    return pack_weight(q, "nk", interleave, sw=sw)


def _packed(w):
    if not isinstance(w, PackedWeight):
        raise TypeError(f"expected a PackedWeight, got {type(w).__name__}")
    return w


class PackedActivation:
    """int8 activations [M, K] in the GEMM's packed fragment layout (w8a8_packed_act_bytes),
    the fastest form of the A operand."""

    __slots__ = ("data", "M", "K")

    def __init__(self, data, M, K):
        self.data, self.M, self.K = data, int(M), int(K)

    @property
    def device(self):
        return self.data.device

    @property
    def shape(self):
        return (self.M, self.K)


def packed_act_bytes(M, K):
    n = lib().w8a8_packed_act_bytes(M, K)
    if n < 0:
        raise ValueError(f"invalid activation shape M={M} K={K}")
    return n


def pack_act(a, out=None):
    """Row-major int8 A [M, K] -> PackedActivation."""
    _check(a, "a", torch.int8)
    M, K = a.shape
    n = packed_act_bytes(M, K)
    if out is None:
        out = torch.empty(max(n, 1), dtype=torch.int8, device=a.device)
    call("w8a8_pack_act", a.data_ptr(), _ld(a), M, K, out.data_ptr(), _stream(a))
    return PackedActivation(out, M, K)


def quant_rows_packed(x, out=None, scale=None):
    """Per-row int8 quant of bf16 rows straight into the packed layout -> (PackedActivation, scale)."""
    _check(x, "x", torch.bfloat16)
    M, K = x.shape
    n = packed_act_bytes(M, K)
    if out is None:
        out = torch.empty(max(n, 1), dtype=torch.int8, device=x.device)
    if scale is None:
        scale = torch.empty((M,), dtype=torch.float32, device=x.device)
    _same_device(x, out, scale)
    call("w8a8_quant_rows_packed_bf16", x.data_ptr(), _ld(x), M, K, out.data_ptr(), scale.data_ptr(), _stream(x))
    return PackedActivation(out, M, K), scale


def _a_operand(a):
    """(pointer, lda, a_packed, M, K, tensor) of a row-major int8 tensor or a PackedActivation."""
    if isinstance(a, PackedActivation):
        return a.data.data_ptr(), 0, 1, a.M, a.K, a.data
    _check(a, "a", torch.int8)
    return a.data_ptr(), _ld(a), 0, a.shape[0], a.shape[1], a


def gemm_i32(a, w, c=None, tile_cfg=-1, split_k=0):
    """C[M,N] int32 = A[M,K] int8 @ W (exact; npu_kernels.py:40-56).  A is a row-major int8
    tensor or a PackedActivation."""
    w = _packed(w)
    ap, lda, a_packed, M, K, at = _a_operand(a)
    if K != w.K:
        raise ValueError(f"gemm_i32: A has K={K}, weight has K={w.K}")
    if w.interleave:
        raise ValueError("gemm_i32: a gate/up-interleaved weight has no plain int32 column order")
    if c is None:
        c = torch.empty((M, w.N), dtype=torch.int32, device=at.device)
    _check(c, "c", torch.int32)
    if tuple(c.shape) != (M, w.N):
        raise ValueError(f"gemm_i32: C has shape {tuple(c.shape)}, expected {(M, w.N)}")
    _same_device(at, w.data, c)
    call("w8a8_gemm_i32_ex", ap, lda, a_packed, w.data.data_ptr(), M, w.N, K, c.data_ptr(), _ld(c), tile_cfg,
         split_k, None, 0, _stream(at))
    return c


def gemm_bf16(a, sx, w, sw=None, epilogue="none", residual=None, out=None, tile_cfg=-1, split_k=0):
    """GEMM + dequant epilogue -> bf16 (pipeline.py:55-57, 102-107).  A is a row-major int8
    tensor or a PackedActivation."""
    w = _packed(w)
    sw = w.sw if sw is None else sw
    if sw is None:
        raise ValueError("gemm_bf16: no per-channel scales")
    ap, lda, a_packed, M, K, at = _a_operand(a)
    _check(sx, "sx", torch.float32, 1)
    _check(sw, "sw", torch.float32, 1)
    if K != w.K or sx.shape[0] != M or sw.shape[0] != w.N:
        raise ValueError("gemm_bf16: operand shapes do not match")
    epi = EPILOGUES[epilogue]
    if epi == 3:
        raise ValueError("gemm_bf16: use linear_bf16 or rms_residual for the RMSNorm residual")
    ncols = w.interleave if epi == 1 else w.N
    if out is None:
        out = torch.empty((M, ncols), dtype=torch.bfloat16, device=at.device)
    _check(out, "out", torch.bfloat16)
    if tuple(out.shape) != (M, ncols):
        raise ValueError(f"gemm_bf16: out has shape {tuple(out.shape)}, expected {(M, ncols)}")
    rp, ldr = None, 0
    if epi == 2:
        if residual is None:
            raise ValueError("gemm_bf16: residual epilogue without a residual")
        _check(residual, "residual", torch.bfloat16)
        if tuple(residual.shape) != (M, w.N):
            raise ValueError("gemm_bf16: residual shape does not match")
        rp, ldr = residual.data_ptr(), _ld(residual)
    _same_device(at, sx, sw, w.data, out, residual)
    call("w8a8_gemm_bf16_ex", ap, lda, a_packed, sx.data_ptr(), w.data.data_ptr(), sw.data_ptr(), M, w.N, K,
         epi, w.interleave, rp, ldr, out.data_ptr(), _ld(out), tile_cfg, split_k, None, 0, _stream(at))
    return out


def dequant_bf16(acc, sx, sw, out=None):
    """bf16((acc * sx[:,None]) * sw[None,:]) (pipeline.py:55-57)."""
    _check(acc, "acc", torch.int32)
    _check(sx, "sx", torch.float32, 1)
    _check(sw, "sw", torch.float32, 1)
    M, N = acc.shape
    if out is None:
        out = torch.empty((M, N), dtype=torch.bfloat16, device=acc.device)
    _check(out, "out", torch.bfloat16)
    _same_device(acc, sx, sw, out)
    call("w8a8_dequant_bf16", acc.data_ptr(), _ld(acc), sx.data_ptr(), sw.data_ptr(), M, N, out.data_ptr(),
         _ld(out), _stream(acc))
    return out


def rms_residual(y, res, w, eps, out=None, quant=False):
    """h = res + bf16(rms(y) * w)  (k_post_ff, pipeline.py:110-114); with quant=True also
    returns the int8 rows and scales of h.  res=None: h = bf16(rms(y) * w), an RMSNorm."""
    _check(y, "y", torch.bfloat16)
    M, N = y.shape
    if res is not None:
        _check(res, "res", torch.bfloat16)
        if tuple(res.shape) != (M, N):
            raise ValueError("rms_residual: shapes differ")
    wp = None
    if w is not None:
        _check(w, "w", torch.bfloat16, 1)
        wp = w.data_ptr()
    if out is None:
        out = torch.empty((M, N), dtype=torch.bfloat16, device=y.device)
    _check(out, "out", torch.bfloat16)
    q = sq = None
    if quant:
        q = torch.empty((M, N), dtype=torch.int8, device=y.device)
        sq = torch.empty((M,), dtype=torch.float32, device=y.device)
    _same_device(y, res, w, out)
    call("w8a8_rms_residual_bf16", y.data_ptr(), _ld(y), None if res is None else res.data_ptr(),
         0 if res is None else _ld(res), wp, float(eps), M, N,
         out.data_ptr(), _ld(out), q.data_ptr() if quant else None, N if quant else 0,
         sq.data_ptr() if quant else None, _stream(y))
    return (out, q, sq) if quant else out


def gemv_act_bf16(x, w, s, act, mul=None, out=None):
    """gemv_bf16 with its activation in the epilogue (the decode path's MLP and per-layer-input
    gate): act "gelu_pair" -> y [M, N/2] = bf16(bf16(gelu_tanh(g)) * u) for a [gate; up] stacked
    GemvWeight; act "gelu_mul" -> y [M, N] = bf16(bf16(gelu_tanh(g)) * mul).  Bit for bit
    gemv_bf16 followed by gelu_mul_bf16."""
    _check(x, "x", torch.bfloat16)
    if not isinstance(w, GemvWeight):
        raise TypeError("gemv_act_bf16: w must be a packed GemvWeight")
    if s.dtype not in (torch.bfloat16, torch.float32):
        raise TypeError(f"gemv_act_bf16: scales must be bf16 or fp32, got {s.dtype}")
    _check(s, "s", s.dtype, 1)
    code = {"gelu_pair": 1, "gelu_mul": 2}.get(act)
    if code is None:
        raise ValueError(f"gemv_act_bf16: act must be 'gelu_pair' or 'gelu_mul', got {act!r}")
    M, K = x.shape
    if w.K != K or s.shape[0] != w.N:
        raise ValueError("gemv_act_bf16: operand shapes do not match")
    nout = w.N // 2 if code == 1 else w.N
    if code == 2:
        if mul is None:
            raise ValueError("gemv_act_bf16: 'gelu_mul' needs mul")
        _check(mul, "mul", torch.bfloat16)
        if tuple(mul.shape) != (M, w.N):
            raise ValueError(f"gemv_act_bf16: mul {tuple(mul.shape)} does not match ({M}, {w.N})")
    if out is None:
        out = torch.empty((M, nout), dtype=torch.bfloat16, device=x.device)
    _check(out, "out", torch.bfloat16)
    if tuple(out.shape) != (M, nout):
        raise ValueError(f"gemv_act_bf16: out has shape {tuple(out.shape)}, expected {(M, nout)}")
    _same_device(x, w.data, s, mul, out)
    call("w8a8_gemv_packed_act_bf16", x.data_ptr(), _ld(x), M, w.data.data_ptr(), w.N, K, s.data_ptr(),
         1 if s.dtype == torch.float32 else 0, code, None if mul is None else mul.data_ptr(),
         0 if mul is None else _ld(mul), out.data_ptr(), _ld(out), _stream(x))
    return out


def gemv_norm_bf16(y, res, w1, eps, w, s, act=None, w2=None, norm2=True, scalar=None, mul=None, store_h=True):
    """The decode row's GEMV with its input norm made in the same launch: (out, h) with
    h = bf16(bf16(res + bf16(rms(y) * w1)) * scalar) (res None: the norm alone), x = bf16(rms(h) * w2)
    when norm2 (else x = h), and out the GEMV of x (act None), or with act "gelu_pair" / "gelu_mul"
    as gemv_act_bf16.  h and out are bit for bit rms_residual_norm / rms_residual followed by
    gemv_bf16 / gemv_act_bf16; h is None unless store_h.  y, res [1, K]; mul [1, N]."""
    _check(y, "y", torch.bfloat16)
    if not isinstance(w, GemvWeight):
        raise TypeError("gemv_norm_bf16: w must be a packed GemvWeight")
    if s.dtype not in (torch.bfloat16, torch.float32):
        raise TypeError(f"gemv_norm_bf16: scales must be bf16 or fp32, got {s.dtype}")
    _check(s, "s", s.dtype, 1)
    code = {None: 0, "gelu_pair": 1, "gelu_mul": 2}.get(act)
    if code is None:
        raise ValueError(f"gemv_norm_bf16: act must be None, 'gelu_pair' or 'gelu_mul', got {act!r}")
    M, K = y.shape
    if M != 1 or w.K != K or s.shape[0] != w.N:
        raise ValueError(f"gemv_norm_bf16: one row of {w.K} expected, got {tuple(y.shape)}")
    if res is not None:
        _check(res, "res", torch.bfloat16)
        if tuple(res.shape) != (1, K):
            raise ValueError("gemv_norm_bf16: res does not match y")
    for t, name in ((w1, "w1"), (w2, "w2")):
        if t is not None:
            _check(t, name, torch.bfloat16, 1)
    if scalar is not None and (scalar.dtype != torch.bfloat16 or scalar.numel() != 1):
        raise ValueError("gemv_norm_bf16: scalar must be one bf16 value")
    if code == 2:
        if mul is None:
            raise ValueError("gemv_norm_bf16: 'gelu_mul' needs mul")
        _check(mul, "mul", torch.bfloat16)
        if tuple(mul.shape) != (1, w.N):
            raise ValueError(f"gemv_norm_bf16: mul {tuple(mul.shape)} does not match (1, {w.N})")
    nout = w.N // 2 if code == 1 else w.N
    out = torch.empty((1, nout), dtype=torch.bfloat16, device=y.device)
    h = torch.empty((1, K), dtype=torch.bfloat16, device=y.device) if store_h else None
    _same_device(y, res, w1, w2, scalar, w.data, s, mul)
    ptr = lambda t: None if t is None else t.data_ptr()
    call("w8a8_gemv_packed_norm_bf16", y.data_ptr(), ptr(res), ptr(w1), ptr(scalar), 1 if norm2 else 0, ptr(w2),
         float(eps), ptr(h), w.data.data_ptr(), w.N, K, s.data_ptr(), 1 if s.dtype == torch.float32 else 0, code,
         ptr(mul), out.data_ptr(), _stream(y))
    return out, h


def gemv_attn_merge_bf16(workspace, pos, H, KV, Tk, D, window, scale, w, s):
    """The decode step's o projection with the attention's chunk merge as its prologue: the output
    row [1, N] of the GEMV on the token's attention output [H * D], which every workgroup merges
    from the chunk partials that attention.decode_qkv_at(..., merge=False) left in `workspace`
    (the same Tk, window, scale).  Bit for bit the merge kernel followed by gemv_bf16.  At most 16
    key chunks (a sliding window of 512 keys at head_dim 256 takes 8) and H * D <= 4096."""
    if not isinstance(w, GemvWeight):
        raise TypeError("gemv_attn_merge_bf16: w must be a packed GemvWeight")
    if s.dtype not in (torch.bfloat16, torch.float32):
        raise TypeError(f"gemv_attn_merge_bf16: scales must be bf16 or fp32, got {s.dtype}")
    if w.K != H * D or s.shape[0] != w.N:
        raise ValueError(f"gemv_attn_merge_bf16: weight [{w.N}, {w.K}] does not take a row of {H}x{D}")
    if not isinstance(pos, torch.Tensor) or pos.dtype != torch.int32 or pos.numel() != 1:
        raise ValueError("gemv_attn_merge_bf16: pos must be an int32 tensor of one element")
    out = torch.empty((1, w.N), dtype=torch.bfloat16, device=w.data.device)
    _same_device(workspace, pos, w.data, s, out)
    call("w8a8_gemv_packed_attn_merge_bf16", workspace.data_ptr(), pos.data_ptr(), H, KV, Tk, D, int(window),
         float(scale), w.data.data_ptr(), w.N, s.data_ptr(), 1 if s.dtype == torch.float32 else 0, out.data_ptr(),
         _stream(out))
    return out


def decode_tail(y, cap, pos, pos64, tok, emitted, n_emitted, logits=None, workspace=None):
    """The decode step's tail in two launches: y bf16 [V] (the LM head's output) softcapped as the
    model's bf16 ops do it (cap > 0; 0 or None: no softcap) into fp32 logits [V]; the first index of
    their maximum becomes the next token (tok, int64 [1, 1]) and is written at emitted[n_emitted]
    (int64 [max]); n_emitted, pos (int32 [1]) and pos64 (int64 [1]) advance by one.  Returns the
    logits."""
    _check(y, "y", torch.bfloat16, 1)
    V = y.shape[0]
    if logits is None:
        logits = torch.empty(V, dtype=torch.float32, device=y.device)
    _check(logits, "logits", torch.float32, 1)
    for t, name, dt in ((pos, "pos", torch.int32), (pos64, "pos64", torch.int64), (tok, "tok", torch.int64),
                        (emitted, "emitted", torch.int64), (n_emitted, "n_emitted", torch.int64)):
        if not isinstance(t, torch.Tensor) or t.dtype != dt or t.device != y.device or not t.is_contiguous():
            raise ValueError(f"decode_tail: {name} must be a contiguous {dt} tensor on y's device")
    need = int(lib().w8a8_decode_tail_workspace_bytes(V))
    ws = workspace if workspace is not None else torch.empty(need, dtype=torch.uint8, device=y.device)
    call("w8a8_decode_tail", y.data_ptr(), V, float(cap or 0.0), logits.data_ptr(), pos.data_ptr(), pos64.data_ptr(),
         tok.data_ptr(), emitted.data_ptr(), n_emitted.data_ptr(), emitted.numel(), ws.data_ptr(), ws.numel(),
         _stream(y))
    return logits


def rms_residual_norm(y, res, w1, w2, eps, scalar=None):
    """(h, x): h = bf16(bf16(res + bf16(rms(y) * w1)) * scalar) and x = bf16(rms(h) * w2), one launch:
    k_post_attn's two norms (pipeline.py:95-99), or k_ple_out and the next layer's input norm
    (pipeline.py:124-127, 66-69), with bf16 outputs (the decode step).  scalar: a bf16 tensor of
    one element, or None."""
    _check(y, "y", torch.bfloat16)
    _check(res, "res", torch.bfloat16)
    M, N = y.shape
    if tuple(res.shape) != (M, N):
        raise ValueError("rms_residual_norm: shapes differ")
    for t, name in ((w1, "w1"), (w2, "w2")):
        if t is not None:
            _check(t, name, torch.bfloat16, 1)
    if scalar is not None and (scalar.dtype != torch.bfloat16 or scalar.numel() != 1):
        raise ValueError("rms_residual_norm: scalar must be one bf16 value")
    h = torch.empty((M, N), dtype=torch.bfloat16, device=y.device)
    x = torch.empty((M, N), dtype=torch.bfloat16, device=y.device)
    _same_device(y, res, w1, w2, scalar)
    call("w8a8_rms_residual_norm_bf16", y.data_ptr(), _ld(y), res.data_ptr(), _ld(res),
         None if w1 is None else w1.data_ptr(), None if scalar is None else scalar.data_ptr(),
         None if w2 is None else w2.data_ptr(), float(eps), M, N, h.data_ptr(), N, x.data_ptr(), N, _stream(y))
    return h, x


def gelu_mul_bf16(y, mul=None, out=None):
    """bf16(bf16(gelu_tanh(y[:, :N])) * m) as bf16 rows: m = mul [M, N], or y's second half when mul is
    None (y [M, 2N]).  k_gelu's / k_ple_gate's activation (pipeline.py:102-107, 117-121) without the
    quant, for the decode step."""
    _check(y, "y", torch.bfloat16)
    M = y.shape[0]
    if mul is None:
        if y.shape[1] % 2:
            raise ValueError("gelu_mul_bf16: y must hold [gate | up] halves")
        N = y.shape[1] // 2
    else:
        N = y.shape[1]
        _check(mul, "mul", torch.bfloat16)
        if tuple(mul.shape) != (M, N):
            raise ValueError(f"gelu_mul_bf16: mul {tuple(mul.shape)} does not match y {tuple(y.shape)}")
    if out is None:
        out = torch.empty((M, N), dtype=torch.bfloat16, device=y.device)
    _check(out, "out", torch.bfloat16)
    if tuple(out.shape) != (M, N):
        raise ValueError(f"gelu_mul_bf16: out has shape {tuple(out.shape)}, expected {(M, N)}")
    _same_device(y, mul, out)
    call("w8a8_gelu_mul_bf16", y.data_ptr(), _ld(y), None if mul is None else mul.data_ptr(),
         0 if mul is None else _ld(mul), M, N, out.data_ptr(), _ld(out), _stream(y))
    return out


def linear_workspace_bytes(M, N, K):
    return lib().w8a8_linear_workspace_bytes(M, N, K)


def linear_bf16(x, w, sw=None, epilogue="none", residual=None, rms_w=None, eps=1e-6, out=None, ws_arg=None):
    """bf16 x -> per-token quant -> W8A8 GEMM -> dequant epilogue -> bf16 (gemma_npu.py:117-152).
    ws_arg: a uint8 device tensor of at least linear_workspace_bytes(M, N, K) bytes to use as the call's
    scratch instead of a fresh one from torch's caching allocator."""
    w = _packed(w)
    sw = w.sw if sw is None else sw
    if sw is None:
        raise ValueError("linear_bf16: no per-channel scales")
    _check(x, "x", torch.bfloat16)
    _check(sw, "sw", torch.float32, 1)
    M, K = x.shape
    if K != w.K or sw.shape[0] != w.N:
        raise ValueError("linear_bf16: operand shapes do not match")
    epi = EPILOGUES[epilogue]
    ncols = w.interleave if epi == 1 else w.N
    if out is None:
        out = torch.empty((M, ncols), dtype=torch.bfloat16, device=x.device)
    _check(out, "out", torch.bfloat16)
    if tuple(out.shape) != (M, ncols):
        raise ValueError(f"linear_bf16: out has shape {tuple(out.shape)}, expected {(M, ncols)}")
    rp, ldr = None, 0
    if epi in (2, 3):
        if residual is None:
            raise ValueError("linear_bf16: residual epilogue without a residual")
        _check(residual, "residual", torch.bfloat16)
        if tuple(residual.shape) != (M, w.N):
            raise ValueError("linear_bf16: residual shape does not match")
        rp, ldr = residual.data_ptr(), _ld(residual)
    rwp = None
    if rms_w is not None:
        _check(rms_w, "rms_w", torch.bfloat16, 1)
        rwp = rms_w.data_ptr()
    need = linear_workspace_bytes(M, w.N, K)
    ws = workspace(x.device, need) if ws_arg is None else ws_arg
    _same_device(x, sw, w.data, out, residual, rms_w, ws)
    call("w8a8_linear_bf16", x.data_ptr(), _ld(x), w.data.data_ptr(), sw.data_ptr(), M, w.N, K, epi,
         w.interleave, rp, ldr, rwp, float(eps), out.data_ptr(), _ld(out), ws.data_ptr(), ws.numel(), _stream(x))
    return out


class GemvWeight:
    """An int8 weight [N, K] resident in the GEMV fragment layout (w8a8_gemv_packed_bytes): the
    decode copy of a linear's weight (the reference's w_cpu, gemma_npu.py:81)."""

    __slots__ = ("data", "N", "K")

    def __init__(self, data, N, K):
        self.data, self.N, self.K = data, int(N), int(K)

    @property
    def device(self):
        return self.data.device

    @property
    def shape(self):
        """(N, K), the shape of the row-major weight it holds."""
        return (self.N, self.K)


def pack_gemv_weight(w):
    """int8 W [N, K] -> GemvWeight (the layout the GEMV streams fastest)."""
    _check(w, "w", torch.int8)
    N, K = w.shape
    n = lib().w8a8_gemv_packed_bytes(N, K)
    if n < 0:
        raise ValueError(f"invalid weight shape {tuple(w.shape)}")
    out = torch.empty(n, dtype=torch.int8, device=w.device)
    call("w8a8_pack_gemv_weight", w.data_ptr(), _ld(w), N, K, out.data_ptr(), _stream(w))
    return GemvWeight(out, N, K)


def gemv_bf16(x, w, s, out=None):
    """y = bf16((x @ w^T) * s): torch._weight_int8pack_mm semantics (gemma_npu.py:155-156).
    x bf16 [M<=16, K]; w int8 [N, K] or a GemvWeight; s bf16 or fp32 [N]."""
    _check(x, "x", torch.bfloat16)
    packed = isinstance(w, GemvWeight)
    if not packed:
        _check(w, "w", torch.int8)
    if s.dtype not in (torch.bfloat16, torch.float32):
        raise TypeError(f"gemv_bf16: scales must be bf16 or fp32, got {s.dtype}")
    _check(s, "s", s.dtype, 1)
    M, K = x.shape
    N, KW = (w.N, w.K) if packed else w.shape
    if KW != K or s.shape[0] != N:
        raise ValueError("gemv_bf16: operand shapes do not match")
    if out is None:
        out = torch.empty((M, N), dtype=torch.bfloat16, device=x.device)
    _check(out, "out", torch.bfloat16)
    wt = w.data if packed else w
    _same_device(x, wt, s, out)
    if packed:
        call("w8a8_gemv_packed_bf16", x.data_ptr(), _ld(x), M, wt.data_ptr(), N, K, s.data_ptr(),
             1 if s.dtype == torch.float32 else 0, out.data_ptr(), _ld(out), _stream(x))
    else:
        call("w8a8_gemv_bf16", x.data_ptr(), _ld(x), M, w.data_ptr(), _ld(w), N, K, s.data_ptr(),
             1 if s.dtype == torch.float32 else 0, out.data_ptr(), _ld(out), _stream(x))
    return out
