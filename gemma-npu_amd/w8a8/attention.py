"""Prefill attention on the GPU, with the reference's function names (pipeline.py:130-180,
local_attn.py:71-107).

    full_attention(q, k_all, v_all, q_start)        -> o [H, Tq, D]      pipeline.py:140-155
    sliding_attention(q, k_all, v_all, q_start, W)  -> o [H, Tq, D]      pipeline.py:158-180
    local_sdpa(module, query, key, value, mask, ...) -> ([1, T, H, D], None)   local_attn.py:71-107
    split_kv_decode(query, key, value, scale)        -> [1, 1, H, D]      local_attn.py:44-68
    attention(q, k, v, q_start, window, scale)      -> o (and the logsumexp)
    decode(q, k, v, q_pos, window, scale)           -> o [H, D] (and the logsumexp)

q is bf16 [H, Tq, D] at positions q_start.., k_all / v_all bf16 [KV, Tk, D] holding positions
0.. (Tk >= q_start + Tq); any strides with a contiguous last dimension.  Scale 1.0 as Gemma uses.
The query at position p sees keys j <= p, and with a window W only those with p - j < W.  One
kernel launch (w8a8_attention_bf16) on torch's current stream computes the whole masked softmax in
one pass, so the reference's logsumexp merge of a prefix pass and a causal pass (`_merge`,
pipeline.py:133-137) and its 128-query window blocks have no counterpart here; the result is the
same function.  Unlike the reference's sliding_attention, q_start need not be a multiple of 128.
There is no CPU fallback.
"""
import threading

import torch

from ._lib import call, lib
from .ops import _stream, current_stream_handle

_WS = {}
_WS_LOCK = threading.Lock()


def _workspace(device, nbytes):
    """Decode scratch of (device, current stream), grown to at least nbytes (calls on one stream are
    ordered, so they can share it; nothing is kept between calls)."""
    key = (device.index, current_stream_handle(device))
    with _WS_LOCK:
        buf = _WS.get(key)
        if buf is None or buf.numel() < nbytes:
            buf = torch.empty(max(nbytes, 1 << 16), dtype=torch.uint8, device=device)
            _WS[key] = buf
    return buf


_SPLIT_WS = {}


def _split_workspace(device, nbytes):
    """The zero-filled workspace of (device, current stream) for split causal tiles, grown to at
    least nbytes: its counters are zero between calls by the kernel's own contract, so it is only
    cleared when (re)allocated."""
    key = (device.index, current_stream_handle(device))
    with _WS_LOCK:
        buf = _SPLIT_WS.get(key)
        if buf is None or buf.numel() < nbytes:
            buf = torch.zeros(nbytes, dtype=torch.uint8, device=device)
            _SPLIT_WS[key] = buf
    return buf


def _check3(t, name):
    if not isinstance(t, torch.Tensor):
        raise TypeError(f"{name}: expected a tensor, got {type(t).__name__}")
    if t.device.type != "cuda":
        raise ValueError(f"{name}: expected a GPU tensor, got device {t.device}")
    if t.dtype != torch.bfloat16:
        raise TypeError(f"{name}: expected torch.bfloat16, got {t.dtype}")
    if t.dim() != 3:
        raise ValueError(f"{name}: expected [heads, rows, head_dim], got shape {tuple(t.shape)}")
    if t.shape[2] > 1 and t.stride(2) != 1:
        raise ValueError(f"{name}: the last dimension must be contiguous, got strides {t.stride()}")


def _strides(t):
    """(head stride, row stride) in elements; sizes of 1 take the natural stride."""
    H, T, D = t.shape
    rs = t.stride(1) if T > 1 else D
    hs = t.stride(0) if H > 1 else max(T, 1) * rs
    return hs, rs


def attention(q, k, v, q_start=0, window=0, scale=1.0, out=None, return_lse=False):
    """softmax(scale q k^T, causal [+ window]) v per head; grouped-query heads h -> h // (H // KV).

    out: optional bf16 [H, Tq, D] destination (any strides with a contiguous last dimension, e.g.
    a transposed view of a [Tq, H, D] tensor).  With return_lse, also the fp32 [H, Tq] natural-log
    logsumexp of the scaled scores (what torch's flash kernels return beside the output)."""
    _check3(q, "q")
    _check3(k, "k")
    _check3(v, "v")
    H, Tq, D = q.shape
    KV, Tk, Dk = k.shape
    if tuple(v.shape) != (KV, Tk, Dk) or Dk != D:
        raise ValueError(f"q {tuple(q.shape)}, k {tuple(k.shape)}, v {tuple(v.shape)} do not match")
    if len({q.device, k.device, v.device}) != 1:
        raise ValueError("q, k and v must be on one device")
    if out is None:
        out = torch.empty((H, Tq, D), dtype=torch.bfloat16, device=q.device)
    else:
        _check3(out, "out")
        if tuple(out.shape) != (H, Tq, D) or out.device != q.device:
            raise ValueError(f"out: expected shape {(H, Tq, D)} on {q.device}, got {tuple(out.shape)}")
    lse = torch.empty((H, Tq), dtype=torch.float32, device=q.device) if return_lse else None
    qhs, qrs = _strides(q)
    khs, krs = _strides(k)
    vhs, vrs = _strides(v)
    ohs, ors = _strides(out)
    need = lib().w8a8_attention_workspace_bytes(H, KV, Tq, Tk, D, int(q_start), int(window))
    ws = _split_workspace(q.device, need) if need > 0 else None
    call("w8a8_attention_ws_bf16", q.data_ptr(), qhs, qrs, k.data_ptr(), khs, krs, v.data_ptr(), vhs, vrs, H, KV,
         Tq, Tk, D, int(q_start), int(window), float(scale), out.data_ptr(), ohs, ors,
         lse.data_ptr() if return_lse else None, None if ws is None else ws.data_ptr(),
         0 if ws is None else ws.numel(), _stream(q))
    return (out, lse) if return_lse else out


def attention_quant(q, k, v, q_start=0, window=0, scale=1.0):
    """attention(q, k, v, q_start, window, scale) followed by k_attn_out (pipeline.py:88-92): the
    output's per-token int8 rows [Tq, H*D] in the GEMM's packed activation layout, and their fp32
    scales -> (PackedActivation, sx).  With one KV group of at most 16 heads (E2B: 8 heads on one)
    the quantisation runs in the attention launch itself and the bf16 output is never written; other
    calls (more KV groups, or a plan that merges key parts in a second kernel) run the two steps.
    Bit-identical either way."""
    from .fused import k_attn_out
    from .ops import PackedActivation, packed_act_bytes
    _check3(q, "q")
    _check3(k, "k")
    _check3(v, "v")
    H, Tq, D = q.shape
    KV, Tk, Dk = k.shape
    if tuple(v.shape) != (KV, Tk, Dk) or Dk != D:
        raise ValueError(f"q {tuple(q.shape)}, k {tuple(k.shape)}, v {tuple(v.shape)} do not match")
    if len({q.device, k.device, v.device}) != 1:
        raise ValueError("q, k and v must be on one device")
    if Tq == 0 or not lib().w8a8_attention_quant_supported(H, KV, Tq, Tk, D, int(q_start), int(window)):
        return k_attn_out(attention(q, k, v, q_start, window, scale), packed=True)
    packed = torch.empty(packed_act_bytes(Tq, H * D), dtype=torch.int8, device=q.device)
    sx = torch.empty((Tq,), dtype=torch.float32, device=q.device)
    qhs, qrs = _strides(q)
    khs, krs = _strides(k)
    vhs, vrs = _strides(v)
    need = lib().w8a8_attention_workspace_bytes(H, KV, Tq, Tk, D, int(q_start), int(window))
    ws = _split_workspace(q.device, need) if need > 0 else None
    call("w8a8_attention_quant_bf16", q.data_ptr(), qhs, qrs, k.data_ptr(), khs, krs, v.data_ptr(), vhs, vrs, H, KV,
         Tq, Tk, D, int(q_start), int(window), float(scale), packed.data_ptr(), sx.data_ptr(),
         None if ws is None else ws.data_ptr(), 0 if ws is None else ws.numel(), _stream(q))
    return PackedActivation(packed, Tq, H * D), sx


def full_attention(q, k_all, v_all, q_start):
    """q [H, Tq, D] at positions q_start.. ; k/v [KV, q_start + Tq, D] -> [H, Tq, D] (causal, scale 1)."""
    return attention(q, k_all, v_all, q_start, 0, 1.0)


def sliding_attention(q, k_all, v_all, q_start, W):
    """Sliding-window attention for queries at q_start.. against keys 0..q_start+Tq (scale 1)."""
    if int(W) < 1:
        raise ValueError(f"sliding_attention: window {W} must be positive")
    return attention(q, k_all, v_all, q_start, int(W), 1.0)


def decode_workspace_bytes(H, KV, Tk, D, q_pos=None, window=0):
    """Bytes of scratch decode() needs (w8a8_attention_decode_workspace_bytes)."""
    n = lib().w8a8_attention_decode_workspace_bytes(H, KV, Tk, D, Tk - 1 if q_pos is None else int(q_pos),
                                                    int(window))
    if n < 0:
        raise ValueError(f"decode: invalid shape H={H} KV={KV} Tk={Tk} D={D}")
    return n


def decode(q, k, v, q_pos=None, window=0, scale=1.0, out=None, return_lse=False, workspace=None):
    """One query per head at position q_pos (default: the last key) against k / v [KV, Tk, D].

    q: bf16 [H, D] or [H, 1, D]; keys 0..q_pos are visible, with a window W only the last W of them.
    Returns o [H, D] (into `out` if given), and with return_lse the fp32 [H] logsumexp.
    workspace: a device uint8 tensor of at least decode_workspace_bytes(...) (scratch; nothing is kept
    between calls); by default a buffer cached per device and stream."""
    if q.dim() == 3:
        if q.shape[1] != 1:
            raise ValueError(f"decode: expected one query per head, got shape {tuple(q.shape)}")
        q = q[:, 0]
    if not isinstance(q, torch.Tensor) or q.dim() != 2 or q.dtype != torch.bfloat16 or q.device.type != "cuda":
        raise ValueError("decode: q must be a bf16 GPU tensor [H, D]")
    if q.shape[1] > 1 and q.stride(1) != 1:
        raise ValueError("decode: q's last dimension must be contiguous")
    _check3(k, "k")
    _check3(v, "v")
    H, D = q.shape
    KV, Tk, Dk = k.shape
    if tuple(v.shape) != (KV, Tk, Dk) or Dk != D:
        raise ValueError(f"q {tuple(q.shape)}, k {tuple(k.shape)}, v {tuple(v.shape)} do not match")
    if len({q.device, k.device, v.device}) != 1:
        raise ValueError("q, k and v must be on one device")
    pos = Tk - 1 if q_pos is None else int(q_pos)
    if out is None:
        out = torch.empty((H, D), dtype=torch.bfloat16, device=q.device)
    elif out.shape != (H, D) or out.dtype != torch.bfloat16 or (D > 1 and out.stride(1) != 1):
        raise ValueError(f"decode: out must be bf16 [{H}, {D}] with a contiguous last dimension")
    lse = torch.empty((H,), dtype=torch.float32, device=q.device) if return_lse else None
    need = lib().w8a8_attention_decode_workspace_bytes(H, KV, Tk, D, pos, int(window))
    ws = _workspace(q.device, max(need, 0)) if workspace is None else workspace
    khs, krs = _strides(k)
    vhs, vrs = _strides(v)
    call("w8a8_attention_decode_bf16", q.data_ptr(), q.stride(0) if H > 1 else D, k.data_ptr(), khs, krs,
         v.data_ptr(), vhs, vrs, H, KV, Tk, D, pos, int(window), float(scale), out.data_ptr(),
         out.stride(0) if H > 1 else D, lse.data_ptr() if return_lse else None, ws.data_ptr(), ws.numel(),
         _stream(q))
    return (out, lse) if return_lse else out


def decode_grid_chunks(D, Tk, window=0):
    """Key chunks per KV head the decode attention launches for a cache of Tk rows (the last `window`
    keys with a window): 64 keys a chunk, 32 at head_dim 512."""
    chunk = 32 if D >= 512 else 64
    span = window if 0 < window < Tk else Tk
    return (span - 1) // chunk + 1


def decode_at_workspace_bytes(H, KV, Tk, D, window=0):
    """Bytes of scratch decode_at() needs for a key cache of Tk rows."""
    n = lib().w8a8_attention_decode_dev_workspace_bytes(H, KV, Tk, D, int(window))
    if n < 0:
        raise ValueError(f"decode_at: invalid shape H={H} KV={KV} Tk={Tk} D={D} window={window}")
    return n


def decode_at(q, k, v, pos, window=0, scale=1.0, out=None, workspace=None):
    """decode() with the query position read from device memory: pos is an int32 GPU tensor [1]
    holding q_pos, k / v the key and value cache [KV, Tk, D] of capacity Tk > q_pos.  The launch does
    not depend on the position, so a decode step captured in a HIP graph replays at each new one.
    workspace: at least decode_at_workspace_bytes(H, KV, Tk, D, window) bytes (allocate it before a
    capture); by default a buffer cached per device and stream."""
    if q.dim() == 3:
        if q.shape[1] != 1:
            raise ValueError(f"decode_at: expected one query per head, got shape {tuple(q.shape)}")
        q = q[:, 0]
    if not isinstance(q, torch.Tensor) or q.dim() != 2 or q.dtype != torch.bfloat16 or q.device.type != "cuda":
        raise ValueError("decode_at: q must be a bf16 GPU tensor [H, D]")
    if q.shape[1] > 1 and q.stride(1) != 1:
        raise ValueError("decode_at: q's last dimension must be contiguous")
    _check3(k, "k")
    _check3(v, "v")
    if not isinstance(pos, torch.Tensor) or pos.dtype != torch.int32 or pos.numel() != 1 or pos.device != q.device:
        raise ValueError("decode_at: pos must be an int32 tensor of one element on q's device")
    H, D = q.shape
    KV, Tk, Dk = k.shape
    if tuple(v.shape) != (KV, Tk, Dk) or Dk != D:
        raise ValueError(f"q {tuple(q.shape)}, k {tuple(k.shape)}, v {tuple(v.shape)} do not match")
    if len({q.device, k.device, v.device}) != 1:
        raise ValueError("q, k and v must be on one device")
    if out is None:
        out = torch.empty((H, D), dtype=torch.bfloat16, device=q.device)
    elif out.shape != (H, D) or out.dtype != torch.bfloat16 or (D > 1 and out.stride(1) != 1):
        raise ValueError(f"decode_at: out must be bf16 [{H}, {D}] with a contiguous last dimension")
    need = decode_at_workspace_bytes(H, KV, Tk, D, window)
    ws = _workspace(q.device, need) if workspace is None else workspace
    khs, krs = _strides(k)
    vhs, vrs = _strides(v)
    call("w8a8_attention_decode_dev_bf16", q.data_ptr(), q.stride(0) if H > 1 else D, k.data_ptr(), khs, krs,
         v.data_ptr(), vhs, vrs, H, KV, Tk, D, pos.data_ptr(), int(window), float(scale), out.data_ptr(),
         out.stride(0) if H > 1 else D, ws.data_ptr(), ws.numel(), _stream(q))
    return out


def decode_qkv_at(y, cos, sin, qw, kw, eps, H, KV, D, k, v, pos, kv_write, window=0, scale=1.0, out=None,
                  workspace=None, merge=True):
    """k_qkv and decode_at in one launch, for the token's qkv row y [1, (H + 2 KV) D] bf16 ([1, H D] when
    the layer reads another layer's keys): q = RoPE(rms(q head) * qw) per head with cos / sin [1, D]
    (the rows at the position) or tables [rows, D] read at the position held in pos; with kv_write the token's key (rms * kw, RoPE) and value (rms) of each KV
    head are also written into the cache k / v [KV, Tk, D] at the position read from pos (int32 [1])
    and attended to there.  Bit for bit fused.k_qkv_cache (or fused.k_qkv for q alone) followed by
    decode_at.  At most 8 query heads per KV head.  merge=False leaves the chunk partials in the
    workspace for ops.gemv_attn_merge_bf16 (the o projection that merges them) and returns None."""
    for t, name in ((y, "y"), (cos, "cos"), (sin, "sin")):
        if not isinstance(t, torch.Tensor) or t.dtype != torch.bfloat16 or t.device.type != "cuda":
            raise ValueError(f"decode_qkv_at: {name} must be a bf16 GPU tensor")
        if not t.is_contiguous():
            raise ValueError(f"decode_qkv_at: {name} must be contiguous")
    width = (H + (2 * KV if kv_write else 0)) * D
    if y.numel() != width:
        raise ValueError(f"decode_qkv_at: y holds {y.numel()} values, expected {width}")
    if cos.dim() != 2 or cos.shape[1] != D or tuple(sin.shape) != tuple(cos.shape):
        raise ValueError(f"decode_qkv_at: cos / sin must be [rows, {D}]: one row, or a table read at the position")
    for t, name in ((qw, "qw"), (kw, "kw")):
        if t is not None and (t.dtype != torch.bfloat16 or t.numel() != D or not t.is_contiguous()):
            raise ValueError(f"decode_qkv_at: {name} must be a contiguous bf16 [{D}]")
    _check3(k, "k")
    _check3(v, "v")
    if not isinstance(pos, torch.Tensor) or pos.dtype != torch.int32 or pos.numel() != 1 or pos.device != y.device:
        raise ValueError("decode_qkv_at: pos must be an int32 tensor of one element on y's device")
    KVk, Tk, Dk = k.shape
    if KVk != KV or Dk != D or tuple(v.shape) != (KV, Tk, D):
        raise ValueError(f"decode_qkv_at: k {tuple(k.shape)} / v {tuple(v.shape)} do not match KV={KV} D={D}")
    if not merge:
        if workspace is None:
            raise ValueError("decode_qkv_at: merge=False needs the workspace that holds the partials")
        out = None
    elif out is None:
        out = torch.empty((H, D), dtype=torch.bfloat16, device=y.device)
    elif out.shape != (H, D) or out.dtype != torch.bfloat16 or (D > 1 and out.stride(1) != 1):
        raise ValueError(f"decode_qkv_at: out must be bf16 [{H}, {D}] with a contiguous last dimension")
    need = decode_at_workspace_bytes(H, KV, Tk, D, window)
    ws = _workspace(y.device, need) if workspace is None else workspace
    khs, krs = _strides(k)
    vhs, vrs = _strides(v)
    ptr = lambda t: None if t is None else t.data_ptr()
    call("w8a8_attention_decode_qkv_dev_bf16", y.data_ptr(), cos.data_ptr(), sin.data_ptr(), cos.shape[0], ptr(qw), ptr(kw),
         float(eps), k.data_ptr(), khs, krs, v.data_ptr(), vhs, vrs, H, KV, Tk, D, 1 if kv_write else 0,
         pos.data_ptr(), int(window), float(scale), None if out is None else out.data_ptr(),
         D if out is None or H == 1 else out.stride(0), ws.data_ptr(), ws.numel(), _stream(y))
    return out


def split_kv_decode(query, key, value, scale):
    """local_attn.py:44-68: one query per head [1, H, 1, D] against one KV head [1, 1, T, D] ->
    [1, 1, H, D] (the reference's split over up to 16 key chunks and logsumexp merge)."""
    if query.dim() != 4 or query.shape[0] != 1 or query.shape[2] != 1:
        raise ValueError(f"split_kv_decode: expected query [1, H, 1, D], got {tuple(query.shape)}")
    H, D = query.shape[1], query.shape[3]
    out = torch.empty((1, 1, H, D), dtype=torch.bfloat16, device=query.device)
    decode(query[0, :, 0], key[0], value[0], None, 0, scale, out=out[0, 0])
    return out


def local_sdpa(module, query, key, value, attention_mask, dropout=0.0, scaling=None, sliding_window=None,
               **kwargs):
    """The attention interface the reference registers with HF as "local_sdpa", on the GPU.

    query [1, H, T, D], key / value [1, KV, Tk, D] with Tk >= T (the last T positions are the
    queries'); returns ([1, T, H, D] contiguous, None).  Causal, and with sliding_window W only the
    last W keys of each query, which is what HF's mask says for these layers; attention_mask is
    therefore not read.  Decode (T == 1) goes to the split-key decode kernels (one query at position
    Tk - 1)."""
    if dropout:
        raise ValueError("local_sdpa: dropout is not supported")
    if query.dim() != 4 or query.shape[0] != 1 or key.shape[0] != 1 or value.shape[0] != 1:
        raise ValueError("local_sdpa: batch size 1 only")
    _, H, T, D = query.shape
    Tk = key.shape[2]
    if Tk < T:
        raise ValueError(f"local_sdpa: {Tk} keys for {T} queries")
    from . import torch_ops  # the registered operators while torch.compile traces, else the calls above
    scale = float(scaling) if scaling is not None else D ** -0.5
    out = torch.empty((1, T, H, D), dtype=torch.bfloat16, device=query.device)
    if T == 1 and H // key.shape[1] <= 16:
        torch_ops.attention_decode(query[0, :, 0], key[0], value[0], Tk - 1, int(sliding_window or 0), scale,
                                   out=out[0, 0])
    else:
        torch_ops.attention(query[0], key[0], value[0], Tk - T, int(sliding_window or 0), scale,
                            out=out[0].transpose(0, 1))
    return out, None
