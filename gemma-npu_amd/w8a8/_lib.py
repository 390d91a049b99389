"""Loads libw8a8.so (the C ABI declared in include/w8a8.h) through ctypes.

There is no fallback: if the library is missing or fails to load, every entry point raises.
ctypes releases the GIL for the duration of each foreign call, so launches from a worker
thread overlap with Python work on other threads.
"""
import ctypes
import os
import threading

LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), "libw8a8.so")

W8A8_OK, W8A8_EINVAL, W8A8_EALIGN, W8A8_EHIP, W8A8_ENOTSUP = 0, 1, 2, 3, 4
STATUS_NAMES = {1: "EINVAL", 2: "EALIGN", 3: "EHIP", 4: "ENOTSUP"}

_p = ctypes.c_void_p
_i64 = ctypes.c_int64
_i32 = ctypes.c_int
_f32 = ctypes.c_float

# name -> (restype, argtypes); must match include/w8a8.h.
SIGNATURES = {
    "w8a8_last_error": (ctypes.c_char_p, []),
    "w8a8_abi_version": (_i32, []),
    "w8a8_packed_weight_bytes": (_i64, [_i64, _i64, _i64]),
    "w8a8_pack_weight_kn": (_i32, [_p, _i64, _i64, _i64, _i64, _p, _p]),
    "w8a8_pack_weight_nk": (_i32, [_p, _i64, _i64, _i64, _i64, _p, _p]),
    "w8a8_quant_rows_bf16": (_i32, [_p, _i64, _i64, _i64, _p, _i64, _p, _p]),
    "w8a8_quant_rows_f32": (_i32, [_p, _i64, _i64, _i64, _p, _i64, _p, _p]),
    "w8a8_selfcheck_quant_step": (_i32, [_p, _p]),
    "w8a8_clock_probe": (_i32, [_p, ctypes.c_uint, _p, _p]),
    "w8a8_gemm_i32": (_i32, [_p, _i64, _p, _i64, _i64, _i64, _p, _i64, _p]),
    "w8a8_gemm_tile_configs": (_i32, []),
    "w8a8_gemm_pick_tile_config": (_i32, [_i64, _i64, _i64, _i32]),
    "w8a8_gemm_workspace_bytes": (_i64, [_i64, _i64, _i64, _i32, _i32]),
    "w8a8_gemm_i32_ex": (_i32, [_p, _i64, _i32, _p, _i64, _i64, _i64, _p, _i64, _i32, _i32, _p, _i64, _p]),
    "w8a8_packed_act_bytes": (_i64, [_i64, _i64]),
    "w8a8_pack_act": (_i32, [_p, _i64, _i64, _i64, _p, _p]),
    "w8a8_quant_rows_packed_bf16": (_i32, [_p, _i64, _i64, _i64, _p, _p, _p]),
    "w8a8_gemm_bf16": (_i32, [_p, _i64, _p, _p, _p, _i64, _i64, _i64, _i32, _i64, _p, _i64, _p, _i64, _p]),
    "w8a8_gemm_bf16_ex": (_i32, [_p, _i64, _i32, _p, _p, _p, _i64, _i64, _i64, _i32, _i64, _p, _i64, _p, _i64,
                                 _i32, _i32, _p, _i64, _p]),
    "w8a8_dequant_bf16": (_i32, [_p, _i64, _p, _p, _i64, _i64, _p, _i64, _p]),
    "w8a8_rms_residual_bf16": (_i32, [_p, _i64, _p, _i64, _p, _f32, _i64, _i64, _p, _i64, _p, _i64, _p, _p]),
    "w8a8_k_in": (_i32, [_p, _i64, _p, _f32, _i64, _i64, _p, _i64, _i32, _p, _p]),
    "w8a8_k_qkv": (_i32, [_p, _i64, _p, _p, _p, _p, _i64, _p, _p, _f32, _i64, _i64, _i64, _i64, _i32, _p, _p, _p,
                          _p]),
    "w8a8_k_attn_out": (_i32, [_p, _i64, _i64, _i64, _i64, _i64, _p, _i64, _i32, _p, _p]),
    "w8a8_k_post_attn": (_i32, [_p, _i64, _p, _p, _p, _i64, _p, _p, _f32, _i64, _i64, _p, _i64, _p, _i64, _i32, _p,
                                _p]),
    "w8a8_k_gelu": (_i32, [_p, _i64, _p, _p, _i64, _i64, _p, _i64, _i32, _p, _p]),
    "w8a8_k_post_ff": (_i32, [_p, _i64, _p, _p, _p, _i64, _p, _f32, _i64, _i64, _p, _i64, _p, _i64, _i32, _p, _p]),
    "w8a8_k_ple_gate": (_i32, [_p, _i64, _p, _p, _p, _i64, _i64, _i64, _p, _i64, _i32, _p, _p]),
    "w8a8_k_ple_out": (_i32, [_p, _i64, _p, _p, _p, _i64, _p, _p, _f32, _i64, _i64, _p, _i64, _p]),
    "w8a8_k_qkv_y": (_i32, [_p, _i64, _p, _p, _i64, _p, _p, _f32, _i64, _i64, _i64, _i64, _i32, _p, _p, _p, _p]),
    "w8a8_k_post_attn_y": (_i32, [_p, _i64, _p, _i64, _p, _p, _f32, _i64, _i64, _p, _i64, _p, _i64, _i32, _p, _p]),
    "w8a8_k_post_ff_y": (_i32, [_p, _i64, _p, _i64, _p, _f32, _i64, _i64, _p, _i64, _p, _i64, _i32, _p, _p]),
    "w8a8_k_ple_gate_y": (_i32, [_p, _i64, _p, _i64, _i64, _i64, _p, _i64, _i32, _p, _p]),
    "w8a8_k_ple_out_k_in": (_i32, [_p, _i64, _p, _p, _p, _i64, _p, _p, _p, _f32, _i64, _i64, _p, _i64, _p, _i64, _i32,
                                   _p, _p]),
    "w8a8_k_ple_out_k_in_y": (_i32, [_p, _i64, _p, _i64, _p, _p, _p, _f32, _i64, _i64, _p, _i64, _p, _i64, _i32, _p,
                                     _p]),
    "w8a8_k_ple_out_y": (_i32, [_p, _i64, _p, _i64, _p, _p, _f32, _i64, _i64, _p, _i64, _p]),
    "w8a8_gelu_mul_bf16": (_i32, [_p, _i64, _p, _i64, _i64, _i64, _p, _i64, _p]),
    "w8a8_k_qkv_cache_y": (_i32, [_p, _i64, _p, _p, _i64, _p, _p, _f32, _i64, _i64, _i64, _i64, _p, _p, _p, _i64, _p,
                                   _p]),
    "w8a8_rms_residual_norm_bf16": (_i32, [_p, _i64, _p, _i64, _p, _p, _p, _f32, _i64, _i64, _p, _i64, _p, _i64, _p]),
    "w8a8_linear_workspace_bytes": (_i64, [_i64, _i64, _i64]),
    "w8a8_linear_bf16": (_i32, [_p, _i64, _p, _p, _i64, _i64, _i64, _i32, _i64, _p, _i64, _p, _f32, _p, _i64, _p,
                                _i64, _p]),
    "w8a8_linear_bf16_noalloc": (_i32, [_p, _i64, _p, _p, _i64, _i64, _i64, _i32, _i64, _p, _i64, _p, _f32, _p,
                                        _i64, _p]),
    "w8a8_gemv_bf16": (_i32, [_p, _i64, _i64, _p, _i64, _i64, _i64, _p, _i32, _p, _i64, _p]),
    "w8a8_gemv_packed_bytes": (_i64, [_i64, _i64]),
    "w8a8_pack_gemv_weight": (_i32, [_p, _i64, _i64, _i64, _p, _p]),
    "w8a8_gemv_packed_bf16": (_i32, [_p, _i64, _i64, _p, _i64, _i64, _p, _i32, _p, _i64, _p]),
    "w8a8_gemv_packed_act_bf16": (_i32, [_p, _i64, _i64, _p, _i64, _i64, _p, _i32, _i32, _p, _i64, _p, _i64, _p]),
    "w8a8_gemv_packed_norm_bf16": (_i32, [_p, _p, _p, _p, _i32, _p, _f32, _p, _p, _i64, _i64, _p, _i32, _i32, _p, _p,
                                          _p]),
    "w8a8_attention_bf16": (_i32, [_p, _i64, _i64, _p, _i64, _i64, _p, _i64, _i64, _i64, _i64, _i64, _i64, _i64,
                                   _i64, _i64, _f32, _p, _i64, _i64, _p, _p]),
    "w8a8_attention_workspace_bytes": (_i64, [_i64, _i64, _i64, _i64, _i64, _i64, _i64]),
    "w8a8_attention_plan_items": (_i64, [_i64, _i64, _i64, _i64, _i64, _i64, _i64, _p, _p]),
    "w8a8_attention_ws_bf16": (_i32, [_p, _i64, _i64, _p, _i64, _i64, _p, _i64, _i64, _i64, _i64, _i64, _i64, _i64,
                                      _i64, _i64, _f32, _p, _i64, _i64, _p, _p, _i64, _p]),
    "w8a8_attention_quant_supported": (_i32, [_i64, _i64, _i64, _i64, _i64, _i64, _i64]),
    "w8a8_attention_quant_bf16": (_i32, [_p, _i64, _i64, _p, _i64, _i64, _p, _i64, _i64, _i64, _i64, _i64, _i64,
                                         _i64, _i64, _i64, _f32, _p, _p, _p, _i64, _p]),
    "w8a8_attention_decode_workspace_bytes": (_i64, [_i64, _i64, _i64, _i64, _i64, _i64]),
    "w8a8_attention_decode_dev_workspace_bytes": (_i64, [_i64, _i64, _i64, _i64, _i64]),
    "w8a8_attention_decode_dev_bf16": (_i32, [_p, _i64, _p, _i64, _i64, _p, _i64, _i64, _i64, _i64, _i64, _i64, _p,
                                               _i64, _f32, _p, _i64, _p, _i64, _p]),
    "w8a8_gemv_packed_attn_merge_bf16": (_i32, [_p, _p, _i64, _i64, _i64, _i64, _i64, _f32, _p, _i64, _p, _i32, _p,
                                                 _p]),
    "w8a8_decode_tail_workspace_bytes": (_i64, [_i64]),
    "w8a8_decode_tail": (_i32, [_p, _i64, _f32, _p, _p, _p, _p, _p, _p, _i64, _p, _i64, _p]),
    "w8a8_attention_decode_qkv_dev_bf16": (_i32, [_p, _p, _p, _i64, _p, _p, _f32, _p, _i64, _i64, _p, _i64, _i64, _i64, _i64,
                                                   _i64, _i64, _i32, _p, _i64, _f32, _p, _i64, _p, _i64, _p]),
    "w8a8_attention_decode_bf16": (_i32, [_p, _i64, _p, _i64, _i64, _p, _i64, _i64, _i64, _i64, _i64, _i64, _i64,
                                          _i64, _f32, _p, _i64, _p, _p, _i64, _p]),
}

_lib = None
_lock = threading.Lock()


class W8A8Error(RuntimeError):
    """A libw8a8 call returned a non-zero status."""

    def __init__(self, fn, status, msg):
        super().__init__(f"{fn}: {STATUS_NAMES.get(status, status)}: {msg}")
        self.status = status


def lib():
    """The loaded library with argtypes set; raises if it is not built."""
    global _lib
    if _lib is None:
        with _lock:
            if _lib is None:
                if not os.path.exists(LIB_PATH):
                    raise RuntimeError(
                        f"libw8a8.so not found at {LIB_PATH}: build it with "
                        "`python -m w8a8.build` (from gemma-npu_amd/) or __graft_entry__.build()")
                L = ctypes.CDLL(LIB_PATH)
                for name, (res, args) in SIGNATURES.items():
                    fn = getattr(L, name)
                    fn.restype = res
                    fn.argtypes = args
                _lib = L
    return _lib


def call(name, *args):
    """Call `name`; raise W8A8Error with w8a8_last_error() on a non-zero status."""
    L = lib()
    rc = getattr(L, name)(*args)
    if rc != W8A8_OK:
        msg = L.w8a8_last_error().decode(errors="replace")
        raise W8A8Error(name, rc, msg)
    return rc
