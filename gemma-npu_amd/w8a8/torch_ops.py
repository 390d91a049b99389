"""libw8a8's launches as torch custom operators (namespace `w8a8`), so that torch.compile traces
through them.

The reference compiles each decoder layer's forward (gemma_npu.py:255-265) and its NPU calls are
graph breaks there.  Registered with torch.library, with a fake (shape-only) implementation each,
the engine's launches are ordinary nodes of the traced graph:

    torch.ops.w8a8.mm_i8(a, w_data, N, K, c)                 int8 A @ packed W -> int32 C (in place)
    torch.ops.w8a8.linear(x, w_data, sw, N, K, interleave, epilogue, residual, rms_w, eps) -> bf16
    torch.ops.w8a8.gemv(x, w_data, N, K, s) -> bf16          weight-only int8 GEMV (decode rows)
    torch.ops.w8a8.rms_norm(x, w, eps) -> bf16               Gemma RMSNorm on bf16 rows
    torch.ops.w8a8.attention(q, k, v, q_start, window, scale) -> bf16 [H, Tq, D]
    torch.ops.w8a8.attention_decode(q, k, v, q_pos, window, scale) -> bf16 [H, D]

Each takes the tensors a w8a8.ops object holds (PackedWeight.data and its sizes, GemvWeight.data)
because an operator's arguments are tensors and scalars.  Eager callers go straight to w8a8.ops,
without the dispatcher's per-call cost; the helpers at the bottom (linear, gemv, rms_norm,
attention, attention_decode) pick the registered operator only while dynamo traces, which is how
w8a8.hf's modules call the engine.
"""
from typing import Optional

import torch
from torch import Tensor

from . import attention as _attn
from . import ops


@torch.library.custom_op("w8a8::mm_i8", mutates_args=("c",), device_types="cuda")
def mm_i8(a: Tensor, w_data: Tensor, N: int, K: int, c: Tensor) -> None:
    ops.gemm_i32(a, ops.PackedWeight(w_data, N, K), c)


@mm_i8.register_fake
def _mm_i8_fake(a, w_data, N, K, c):
    return None


@torch.library.custom_op("w8a8::linear", mutates_args=(), device_types="cuda")
def linear_op(x: Tensor, w_data: Tensor, sw: Tensor, N: int, K: int, interleave: int, epilogue: str,
              residual: Optional[Tensor], rms_w: Optional[Tensor], eps: float) -> Tensor:
    return ops.linear_bf16(x, ops.PackedWeight(w_data, N, K, interleave), sw, epilogue, residual, rms_w, eps)


@linear_op.register_fake
def _linear_fake(x, w_data, sw, N, K, interleave, epilogue, residual, rms_w, eps):
    return x.new_empty((x.shape[0], interleave if epilogue == "gelu" else N))


@torch.library.custom_op("w8a8::gemv", mutates_args=(), device_types="cuda")
def gemv_op(x: Tensor, w_data: Tensor, N: int, K: int, s: Tensor) -> Tensor:
    return ops.gemv_bf16(x, ops.GemvWeight(w_data, N, K), s)


@gemv_op.register_fake
def _gemv_fake(x, w_data, N, K, s):
    return x.new_empty((x.shape[0], N))


@torch.library.custom_op("w8a8::rms_norm", mutates_args=(), device_types="cuda")
def rms_norm_op(x: Tensor, w: Optional[Tensor], eps: float) -> Tensor:
    if not x.is_contiguous() or x.data_ptr() % 16:  # the row kernel reads 16-byte vectors
        x = x.clone(memory_format=torch.contiguous_format)
    return ops.rms_residual(x, None, w, eps)


@rms_norm_op.register_fake
def _rms_norm_fake(x, w, eps):
    # the real op works on (and returns) a contiguous copy of a strided x
    return x.new_empty(x.shape)


@torch.library.custom_op("w8a8::attention", mutates_args=(), device_types="cuda")
def attention_op(q: Tensor, k: Tensor, v: Tensor, q_start: int, window: int, scale: float) -> Tensor:
    return _attn.attention(q, k, v, q_start, window, scale)


@attention_op.register_fake
def _attention_fake(q, k, v, q_start, window, scale):
    return q.new_empty(q.shape)


@torch.library.custom_op("w8a8::attention_decode", mutates_args=(), device_types="cuda")
def attention_decode_op(q: Tensor, k: Tensor, v: Tensor, q_pos: int, window: int, scale: float) -> Tensor:
    return _attn.decode(q, k, v, q_pos, window, scale)


@attention_decode_op.register_fake
def _attention_decode_fake(q, k, v, q_pos, window, scale):
    return q.new_empty(q.shape)


def tracing():
    return torch.compiler.is_compiling()


def linear(x, w, epilogue="none", residual=None, rms_w=None, eps=1e-6):
    """ops.linear_bf16(x, w, ...) eagerly; the registered operator under torch.compile."""
    if tracing():
        return torch.ops.w8a8.linear(x, w.data, w.sw, w.N, w.K, w.interleave, epilogue, residual, rms_w, eps)
    return ops.linear_bf16(x, w, epilogue=epilogue, residual=residual, rms_w=rms_w, eps=eps)


def gemv(x, w, s, out=None):
    """ops.gemv_bf16(x, w, s) eagerly (into `out` if given); the registered operator under torch.compile."""
    if tracing():
        y = torch.ops.w8a8.gemv(x, w.data, w.N, w.K, s)
        if out is not None:
            out.copy_(y)
            return out
        return y
    return ops.gemv_bf16(x, w, s, out)


def rms_norm(x, w, eps):
    """ops.rms_residual(x, None, w, eps) eagerly; the registered operator under torch.compile."""
    if tracing():
        return torch.ops.w8a8.rms_norm(x, w, eps)
    return ops.rms_residual(x, None, w, eps)


def attention(q, k, v, q_start, window, scale, out=None):
    """attention.attention(...) eagerly (into `out` if given); the registered operator under torch.compile."""
    if tracing():
        y = torch.ops.w8a8.attention(q, k, v, q_start, window, scale)
        if out is not None:
            out.copy_(y)
            return out
        return y
    return _attn.attention(q, k, v, q_start, window, scale, out=out)


def attention_decode(q, k, v, q_pos, window, scale, out=None):
    """attention.decode(...) eagerly (into `out` if given); the registered operator under torch.compile."""
    if tracing():
        y = torch.ops.w8a8.attention_decode(q, k, v, q_pos, window, scale)
        if out is not None:
            out.copy_(y)
            return out
        return y
    return _attn.decode(q, k, v, q_pos, window, scale, out=out)
