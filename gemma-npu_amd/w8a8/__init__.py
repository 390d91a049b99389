"""W8A8 linear engine for MI355X (gfx950): HIP kernels behind the C ABI in include/w8a8.h.

    from w8a8 import ops          # torch-facing entry points (GEMM, quant, GEMV, linear)
    from w8a8 import fused        # the reference's fused kernels between the GEMMs (k_in ... k_ple_out)
    from w8a8 import attention    # prefill and decode attention (full_attention, sliding_attention, local_sdpa)
    from w8a8 import hf           # HF Gemma 4 on the engine (to_gpu, the reference's to_npu)
    from w8a8.pipeline import Prefill   # the reference's whole-prompt prefill, every step on the GPU
    import npu_kernels            # drop-in for the reference's npu_kernels.mm_i8
"""
from . import attention, fused  # noqa: F401
from ._lib import LIB_PATH, W8A8Error, lib  # noqa: F401
from .ops import (  # noqa: F401
    GemvWeight, PackedActivation, PackedWeight, dequant_bf16, pack_gemv_weight, pack_act, packed_act_bytes, quant_rows_packed, gemm_bf16, gemm_i32, gemv_bf16, linear_bf16, pack_weight, packed_weight_bytes,
    quant_rows, quant_weight, rms_residual,
)
