"""numpy front end of the C oracle -- TEST INFRASTRUCTURE ONLY.

Only the test suite, the smoke check and the benchmark's CPU-baseline leg use
this module, and only to check results against; the product library never loads it.
Every function takes and returns numpy arrays.  bf16 data is carried as
uint16 bit patterns (see `bf16_bits` / `bits_to_f32`).

Reference file:line for each restated function is given in w8a8_oracle.c.
"""
import ctypes
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "liboracle_w8a8.so")

_lib = None


def build():
    """Compile the C oracle with gcc (oracle/Makefile)."""
    subprocess.run(["make", "-s", "-C", HERE], check=True)


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            build()
        L = ctypes.CDLL(LIB_PATH)
        p, i64, i32, f32 = ctypes.c_void_p, ctypes.c_int64, ctypes.c_int, ctypes.c_float
        L.oracle_int_mm.argtypes = [p, i64, p, i64, p, i64, i64, i64, i64]
        L.oracle_int_mm_nk.argtypes = [p, i64, p, i64, p, i64, i64, i64, i64]
        L.oracle_quant_rows.argtypes = [p, i32, i64, i64, i64, p, i64, p]
        L.oracle_dequant.argtypes = [p, i64, p, p, i64, i64, p, i64]
        L.oracle_gelu_mul.argtypes = [p, i64, i64, i64, p, i64]
        L.oracle_rms_residual.argtypes = [p, i64, p, i64, p, f32, i64, i64, p, i64]
        L.oracle_add_residual.argtypes = [p, i64, p, i64, i64, i64, p, i64]
        L.oracle_gemv.argtypes = [p, i64, i64, p, i64, i64, i64, p, i32, p, i64]
        L.oracle_rms_bf16.argtypes = [p, i64, p, f32, i64, i64, p, i64]
        L.oracle_rope_rows.argtypes = [p, i64, p, p, i64, i64, i64, p, i64]
        L.oracle_attention.argtypes = [p, i64, i64, p, p, i64, i64, i64, i64, i64, i64, i64, i64, i64,
                                       ctypes.c_double, p, i64, i64, p, p]
        L.oracle_f32_to_bf16.argtypes = [f32]
        L.oracle_f32_to_bf16.restype = ctypes.c_uint16
        _lib = L
    return _lib


def _ptr(a):
    return a.ctypes.data_as(ctypes.c_void_p)


def _c(a, dtype):
    a = np.ascontiguousarray(a)
    assert a.dtype == dtype, (a.dtype, dtype)
    return a


# ---- bf16 helpers (bit patterns in uint16) ---------------------------------

def bf16_bits(x):
    """fp32 -> bf16 bit patterns, round to nearest even (torch's .to(bfloat16))."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    u = x.view(np.uint32).astype(np.uint64)
    nan = (u & 0x7FFFFFFF) > 0x7F800000
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    r[nan] = ((u[nan] >> 16) | 0x40).astype(np.uint16)
    return r


def bits_to_f32(h):
    return (np.ascontiguousarray(h, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


# ---- restated reference functions ------------------------------------------

def int_mm(a, b):
    """C = A[M,K] @ B[K,N], int8 -> int32 (npu_kernels.py:40-56)."""
    a, b = _c(a, np.int8), _c(b, np.int8)
    M, K = a.shape
    K2, N = b.shape
    assert K == K2
    c = np.empty((M, N), np.int32)
    lib().oracle_int_mm(_ptr(a), K, _ptr(b), N, _ptr(c), N, M, N, K)
    return c


def int_mm_nk(a, w):
    """C = A[M,K] @ W[N,K]^T, int8 -> int32 (the [N,K] weight layout, gemma_npu.py:69)."""
    a, w = _c(a, np.int8), _c(w, np.int8)
    M, K = a.shape
    N = w.shape[0]
    c = np.empty((M, N), np.int32)
    lib().oracle_int_mm_nk(_ptr(a), K, _ptr(w), K, _ptr(c), N, M, N, K)
    return c


def quant_rows(x, dtype="bf16"):
    """Per-row absmax/127 int8 quant (pipeline.py:49-52). x: uint16 bf16 bits or float32."""
    if dtype == "bf16":
        x = _c(x, np.uint16)
        code = 0
    else:
        x = _c(x, np.float32)
        code = 1
    M, K = x.shape
    q = np.empty((M, K), np.int8)
    s = np.empty((M,), np.float32)
    lib().oracle_quant_rows(_ptr(x), code, K, M, K, _ptr(q), K, _ptr(s))
    return q, s


def dequant(acc, sx, sw):
    """bf16 bits of ((acc*sx)*sw) (pipeline.py:55-57)."""
    acc = _c(acc, np.int32)
    sx, sw = _c(sx, np.float32), _c(sw, np.float32)
    M, N = acc.shape
    out = np.empty((M, N), np.uint16)
    lib().oracle_dequant(_ptr(acc), N, _ptr(sx), _ptr(sw), M, N, _ptr(out), N)
    return out


def gelu_mul(y):
    """bf16 bits of gelu_tanh(y[:, :I]) * y[:, I:] (pipeline.py:106)."""
    y = _c(y, np.uint16)
    M, N2 = y.shape
    I = N2 // 2
    out = np.empty((M, I), np.uint16)
    lib().oracle_gelu_mul(_ptr(y), N2, M, I, _ptr(out), I)
    return out


def rms_residual(y, res, w, eps):
    """bf16 bits of res + bf16(rms(y) * w) (pipeline.py:43-46, 113)."""
    y, res = _c(y, np.uint16), _c(res, np.uint16)
    M, N = y.shape
    wp = None
    if w is not None:
        w = _c(w, np.uint16)
        wp = _ptr(w)
    h = np.empty((M, N), np.uint16)
    lib().oracle_rms_residual(_ptr(y), N, _ptr(res), N, wp, float(eps), M, N, _ptr(h), N)
    return h


def add_residual(y, res):
    """bf16 bits of res + y."""
    y, res = _c(y, np.uint16), _c(res, np.uint16)
    M, N = y.shape
    h = np.empty((M, N), np.uint16)
    lib().oracle_add_residual(_ptr(y), N, _ptr(res), N, M, N, _ptr(h), N)
    return h


def gemv(x, w, s, sdtype="bf16"):
    """bf16 bits of (x @ w^T) * s  (torch._weight_int8pack_mm, gemma_npu.py:155-156).

    x: uint16 bf16 bits [M,K]; w: int8 [N,K]; s: uint16 bf16 bits or float32 [N].
    """
    x, w = _c(x, np.uint16), _c(w, np.int8)
    M, K = x.shape
    N = w.shape[0]
    if sdtype == "bf16":
        s = _c(s, np.uint16)
        code = 0
    else:
        s = _c(s, np.float32)
        code = 1
    y = np.empty((M, N), np.uint16)
    lib().oracle_gemv(_ptr(x), K, M, _ptr(w), K, N, K, _ptr(s), code, _ptr(y), N)
    return y


def linear_bf16(x, wq, sw, epilogue="none", residual=None, rms_w=None, eps=1e-6):
    """The whole W8A8 linear as the reference pipeline composes it.

    x bf16 bits [M,K] -> quant_rows -> int_mm_nk with wq [N,K] -> dequant -> epilogue:
      "none": bf16 y                                    (gemma_npu.py:127-150)
      "gelu": gelu_tanh(y[:, :I]) * y[:, I:]            (pipeline.py:102-107)
      "residual": res + y                               (plain add)
      "residual_rms": res + bf16(rms(y) * rms_w)        (pipeline.py:110-114)
    Returns (out_bits, int32 acc, sx).
    """
    q, sx = quant_rows(x, "bf16")
    acc = int_mm_nk(q, wq)
    y = dequant(acc, sx, sw)
    if epilogue == "none":
        out = y
    elif epilogue == "gelu":
        out = gelu_mul(y)
    elif epilogue == "residual":
        out = add_residual(y, residual)
    elif epilogue == "residual_rms":
        out = rms_residual(y, residual, rms_w, eps)
    else:
        raise ValueError(epilogue)
    return out, acc, sx


# ---- the fused kernels between the GEMMs (pipeline.py:43-127) ---------------------------

def rms_bf16(x, w, eps):
    """bf16 bits of _rms(x, w, eps).to(bfloat16) over the last axis (pipeline.py:43-46)."""
    x = _c(x, np.uint16)
    shape = x.shape
    x2 = x.reshape(-1, shape[-1])
    M, N = x2.shape
    wp = None
    if w is not None:
        w = _c(w, np.uint16)
        wp = _ptr(w)
    out = np.empty((M, N), np.uint16)
    lib().oracle_rms_bf16(_ptr(x2), N, wp, float(eps), M, N, _ptr(out), N)
    return out.reshape(shape)


def rope(x, cos, sin):
    """bf16 bits of _rope(x, cos, sin) on bf16 tensors (pipeline.py:60-63); x [R, D], cos / sin
    [R, D] (row r rotated by row r)."""
    x, cos, sin = _c(x, np.uint16), _c(cos, np.uint16), _c(sin, np.uint16)
    R, D = x.shape
    assert cos.shape == (R, D) and sin.shape == (R, D)
    out = np.empty((R, D), np.uint16)
    lib().oracle_rope_rows(_ptr(x), D, _ptr(cos), _ptr(sin), D, R, D, _ptr(out), D)
    return out


def scale_bf16(x, scalar):
    """bf16 bits of x * scalar on bf16 values (scalar given as bf16 bits)."""
    prod = bits_to_f32(x) * bits_to_f32(np.asarray([scalar], np.uint16))[0]
    return bf16_bits(prod.astype(np.float32))


def k_in(h, w, eps):
    """quant(bf16(rms(h, w)))  (pipeline.py:66-69) -> (q, s)."""
    return quant_rows(rms_bf16(h, w, eps), "bf16")


def k_qkv(acc, sx, sw, cos, sin, qw, kw, eps, H, KV, D, shared):
    """(pipeline.py:72-85) -> q [H, T, D], k, v [KV, T, D] bf16 bits (q, q, q when shared)."""
    y = dequant(acc, sx, sw)
    T = y.shape[0]

    def heads(col0, n, w, rotate):
        x = y[:, col0:col0 + n * D].reshape(T, n, D).transpose(1, 0, 2)      # [n, T, D]
        x = rms_bf16(np.ascontiguousarray(x), w, eps)
        if rotate:
            x = np.stack([rope(x[i], cos, sin) for i in range(n)])
        return x

    q = heads(0, H, qw, True)
    if shared:
        return q, q, q
    k = heads(H * D, KV, kw, True)
    v = heads((H + KV) * D, KV, None, False)
    return q, k, v


def k_attn_out(o):
    """quant of o [H, T, D] read as rows [T, H*D]  (pipeline.py:88-92) -> (q, s)."""
    H, T, D = o.shape
    return quant_rows(np.ascontiguousarray(np.asarray(o).transpose(1, 0, 2).reshape(T, H * D)), "bf16")


def k_post_attn(acc, sx, sw, res, w_post, w_pre_ff, eps):
    """(pipeline.py:95-99) -> (h, q, s)."""
    h = rms_residual(dequant(acc, sx, sw), res, w_post, eps)
    q, s = quant_rows(rms_bf16(h, w_pre_ff, eps), "bf16")
    return h, q, s


def k_gelu(acc, sx, sw, I):
    """(pipeline.py:102-107) on acc [T, 2I] -> (q, s)."""
    y = dequant(acc, sx, sw)
    return quant_rows(gelu_mul(y[:, :2 * I]), "bf16")


def k_post_ff(acc, sx, sw, res, w_post_ff, eps):
    """(pipeline.py:110-114) -> (h, q, s)."""
    h = rms_residual(dequant(acc, sx, sw), res, w_post_ff, eps)
    q, s = quant_rows(h, "bf16")
    return h, q, s


def k_ple_gate(acc, sx, sw, ple):
    """(pipeline.py:117-121) -> (q, s): gelu_mul on [y | ple] is bf16(bf16(gelu(y)) * ple)."""
    y = dequant(acc, sx, sw)
    g = gelu_mul(np.concatenate([y, _c(ple, np.uint16)], axis=1))
    return quant_rows(g, "bf16")


def k_ple_out(acc, sx, sw, h, w_post_ple, scalar, eps):
    """(pipeline.py:124-127) -> bf16 bits of bf16(bf16(h + bf16(rms(y, w))) * scalar)."""
    t = rms_residual(dequant(acc, sx, sw), h, w_post_ple, eps)
    return scale_bf16(t, scalar)


# ---- prefill attention (pipeline.py:141-180, local_attn.py:71-107) --------------------------

def attention(q, k, v, q_start=0, window=0, scale=1.0, budget=False, lse=False):
    """bf16 bits of softmax(scale q k^T, causal [+ window]) v per head (double precision inside).

    q [H, Tq, D], k / v [KV, Tk, D] uint16 bf16 bits; the query at position q_start + i sees keys
    j <= q_start + i, and with window W > 0 only those with q_start + i - j < W.  Returns out, then
    with budget=True sum_j p_j |v_j| per output element (float32 [H, Tq, D]), then with lse=True
    the logsumexp of the scaled scores (float64 [H, Tq])."""
    q, k, v = _c(q, np.uint16), _c(k, np.uint16), _c(v, np.uint16)
    H, Tq, D = q.shape
    KV, Tk, D2 = k.shape
    assert D2 == D and v.shape == k.shape and H % KV == 0 and Tk >= q_start + Tq
    out = np.empty((H, Tq, D), np.uint16)
    bud = np.empty((H, Tq, D), np.float32) if budget else None
    ls = np.empty((H, Tq), np.float64) if lse else None
    lib().oracle_attention(_ptr(q), Tq * D, D, _ptr(k), _ptr(v), Tk * D, D, H, KV, Tq, Tk, D, int(q_start),
                           int(window), float(scale), _ptr(out), Tq * D, D, _ptr(bud) if budget else None,
                           _ptr(ls) if lse else None)
    res = (out,) + ((bud,) if budget else ()) + ((ls,) if lse else ())
    return res if len(res) > 1 else out
