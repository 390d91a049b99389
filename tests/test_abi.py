"""The C-ABI library: it loads, exports every symbol include/w8a8.h declares, and rejects bad
arguments with a status code and a message before launching anything (no GPU needed)."""
import ctypes
import os
import re

import pytest

from w8a8 import _lib

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "w8a8.h")


def declared_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(w8a8_\w+)\s*\(", text)))


def test_header_declares_the_abi():
    names = declared_functions()
    assert "w8a8_gemm_i32" in names and "w8a8_gemv_bf16" in names
    assert set(names) == set(_lib.SIGNATURES), "ctypes signature table and header disagree"


def test_library_exports_every_declared_symbol():
    L = _lib.lib()
    missing = [n for n in declared_functions() if not hasattr(L, n)]
    assert not missing, f"not exported: {missing}"
    assert L.w8a8_abi_version() == 1
    assert L.w8a8_gemm_tile_configs() == 11


def test_pick_tile_config_is_a_valid_configuration():
    """The automatic choice names a real configuration for every prefill shape, differs between
    one micro-batch and a whole prompt where the tiles do, and rejects invalid shapes."""
    L = _lib.lib()
    n = L.w8a8_gemm_tile_configs()
    shapes = [(1536, 2560), (2048, 1536), (1536, 12288), (6144, 1536), (1536, 8960), (12288, 1536),
              (1536, 24576)]
    for M in (1, 77, 512, 3658, 4096, 16384):
        for K, N in shapes:
            for epi in (-1, 0, 1, 2):
                cfg = L.w8a8_gemm_pick_tile_config(M, N, K, epi)
                assert 0 <= cfg < n, (M, N, K, epi, cfg)
    assert L.w8a8_gemm_pick_tile_config(512, 12288, 1536, 1) != L.w8a8_gemm_pick_tile_config(3658, 12288, 1536, 1)
    # past one micro-batch (256 CUs), N <= 4096: one round of direct-W BMx256 tiles with the smallest BM
    # that fits (96: 7, 128: 5, 160: 8, 192: 9) where it moves fewer bytes per CU than the 64x128
    # tiles (0); then 128x256 with two blocks per CU (6) for the long-K narrow ones; the wide int32
    # gate/up on the pipelined kernel (10)
    assert L.w8a8_gemm_pick_tile_config(3658, 1536, 6144, -1) == 7
    assert L.w8a8_gemm_pick_tile_config(3658, 1536, 2048, -1) == 7
    assert L.w8a8_gemm_pick_tile_config(3658, 2560, 1536, -1) == 8
    assert L.w8a8_gemm_pick_tile_config(4096, 2560, 1536, -1) == 9
    assert L.w8a8_gemm_pick_tile_config(4096, 1536, 6144, -1) == 5
    assert L.w8a8_gemm_pick_tile_config(8192, 1536, 6144, -1) == 6
    assert L.w8a8_gemm_pick_tile_config(16384, 1536, 6144, 2) == 6
    assert L.w8a8_gemm_pick_tile_config(3658, 256, 1536, -1) == 0      # one column tile: 64x128 moves less
    assert L.w8a8_gemm_pick_tile_config(3658, 12288, 1536, -1) == 10
    assert L.w8a8_gemm_pick_tile_config(512, 6144, 1536, -1) == 4      # one round of 64x256 tiles
    assert L.w8a8_gemm_pick_tile_config(512, 8192, 1536, 0) == 4
    assert L.w8a8_gemm_pick_tile_config(512, 4096, 1536, -1) == 2      # 64x128 tiles fit one round
    assert L.w8a8_gemm_pick_tile_config(512, 8960, 1536, -1) == 0      # 64x256 tiles past one round
    assert L.w8a8_gemm_pick_tile_config(768, 6144, 1536, 2) == 0
    assert L.w8a8_gemm_pick_tile_config(3658, 8960, 1536, 0) == 6      # wide, bf16 epilogue
    assert L.w8a8_gemm_pick_tile_config(3658, 5120, 1536, -1) == 6     # 580 128x256 tiles, a full last round
    assert L.w8a8_gemm_pick_tile_config(3072, 6144, 1536, -1) == 0     # 576 tiles: a short last round
    assert L.w8a8_gemm_pick_tile_config(2048, 5120, 1536, 2) == 0      # 320 tiles: likewise
    assert L.w8a8_gemm_pick_tile_config(3658, 256, 256, -1) == 0       # fewer 128x256 tiles than CUs
    assert L.w8a8_gemm_pick_tile_config(0, 64, 64, 0) == -1
    assert L.w8a8_gemm_pick_tile_config(64, 64, 64, 3) == -1
    assert L.w8a8_gemm_pick_tile_config(64, 64, 64, -2) == -1


def test_every_tile_configuration_is_reachable():
    """The library builds exactly the configurations the automatic choice takes: each of them is the
    choice for one of these E2B prefill shapes (M, N, K, epilogue)."""
    L = _lib.lib()
    cases = {0: (3658, 256, 1536, -1), 1: (512, 1536, 1536, 0), 2: (512, 4096, 1536, -1),
             3: (512, 1536, 6144, 2), 4: (512, 12288, 1536, 1), 5: (4096, 1536, 6144, -1),
             6: (8192, 1536, 6144, -1), 7: (3658, 1536, 6144, -1), 8: (3658, 2560, 1536, -1),
             9: (4096, 2560, 1536, -1), 10: (3658, 12288, 1536, -1)}
    assert sorted(cases) == list(range(L.w8a8_gemm_tile_configs()))
    for cfg, (M, N, K, epi) in cases.items():
        assert L.w8a8_gemm_pick_tile_config(M, N, K, epi) == cfg, (cfg, M, N, K, epi)


def test_packed_weight_bytes():
    L = _lib.lib()
    assert L.w8a8_packed_weight_bytes(6144, 1536, 0) == 6144 * 1536
    assert L.w8a8_packed_weight_bytes(2560, 1536, 0) == 2560 * 1536
    assert L.w8a8_packed_weight_bytes(17, 70, 0) == 32 * 128       # padded to 32 channels x 64 k
    assert L.w8a8_packed_weight_bytes(33, 64, 0) == 64 * 64
    assert L.w8a8_packed_weight_bytes(12288, 1536, 6144) == 12288 * 1536
    assert L.w8a8_packed_weight_bytes(12288, 1536, 6000) == -1   # I must be a multiple of 32
    assert L.w8a8_packed_weight_bytes(12288, 1536, 4096) == -1   # N must be 2 I
    assert L.w8a8_packed_weight_bytes(0, 64, 0) == -1


def test_linear_workspace_bytes():
    L = _lib.lib()
    assert L.w8a8_packed_act_bytes(512, 1536) == 512 * 1536
    assert L.w8a8_packed_act_bytes(33, 40) == 64 * 64       # rows to 32, k to 64
    assert L.w8a8_packed_act_bytes(0, 64) == 0
    # no configuration splits K across blocks: the GEMMs need no workspace, and split_k > 1 is refused
    for cfg in range(-1, 11):
        assert L.w8a8_gemm_workspace_bytes(512, 1536, 6144, cfg, 0) == 0
        assert L.w8a8_gemm_workspace_bytes(3658, 12288, 1536, cfg, 1) == 0
    assert L.w8a8_gemm_workspace_bytes(512, 1536, 6144, 3, 4) == -1
    assert L.w8a8_gemm_workspace_bytes(3658, 1536, 6144, 11, 0) == -1      # past the last configuration
    # the linear's scratch: packed int8 rows (to 32 rows, k to 64), then the row scales, 256-aligned
    assert L.w8a8_linear_workspace_bytes(512, 1536, 6144) == 512 * 6144 + 512 * 4
    assert L.w8a8_linear_workspace_bytes(512, 1536, 2048) == 512 * 2048 + 512 * 4
    assert L.w8a8_linear_workspace_bytes(3, 64, 64) == 32 * 64 + 256


def _status(name, *args):
    L = _lib.lib()
    rc = getattr(L, name)(*args)
    return rc, L.w8a8_last_error().decode()


def test_errors_are_reported_without_launching():
    fake = ctypes.c_void_p(0x100000)  # never dereferenced: validation fails first
    rc, msg = _status("w8a8_gemm_i32", None, 64, fake, 4, 8, 64, fake, 8, None)
    assert rc == _lib.W8A8_EINVAL and "null" in msg
    rc, msg = _status("w8a8_gemm_i32", fake, 64, fake, 4, 8, 60, fake, 8, None)
    assert rc == _lib.W8A8_ENOTSUP and "multiple of 16" in msg
    rc, msg = _status("w8a8_gemm_i32", fake, 32, fake, 4, 8, 64, fake, 8, None)
    assert rc == _lib.W8A8_EINVAL and "lda" in msg
    rc, msg = _status("w8a8_gemm_i32", ctypes.c_void_p(0x100001), 64, fake, 4, 8, 64, fake, 8, None)
    assert rc == _lib.W8A8_EALIGN
    rc, msg = _status("w8a8_gemm_i32", fake, 64, fake, 4, 8, 64, fake, 6, None)
    assert rc == _lib.W8A8_EINVAL and "ldc" in msg
    rc, msg = _status("w8a8_gemm_i32_ex", fake, 64, 0, fake, 4, 8, 64, fake, 8, 99, 0, None, 0, None)
    assert rc == _lib.W8A8_EINVAL and "config" in msg
    rc, msg = _status("w8a8_gemm_bf16", fake, 64, fake, fake, fake, 4, 16, 64, 1, 0, None, 0, fake, 16, None)
    assert rc == _lib.W8A8_EINVAL and "interleave" in msg
    rc, msg = _status("w8a8_gemm_bf16", fake, 64, fake, fake, fake, 4, 16, 64, 2, 0, None, 0, fake, 16, None)
    assert rc == _lib.W8A8_EINVAL and "residual" in msg
    rc, msg = _status("w8a8_gemv_bf16", fake, 64, 17, fake, 64, 8, 64, fake, 0, fake, 8, None)
    assert rc == _lib.W8A8_EINVAL and "1..16" in msg
    rc, msg = _status("w8a8_gemv_bf16", fake, 64, 1, fake, 64, 8, 40, fake, 0, fake, 8, None)
    assert rc == _lib.W8A8_ENOTSUP
    rc, msg = _status("w8a8_quant_rows_bf16", fake, 8, 4, 16, fake, 16, fake, None)
    assert rc == _lib.W8A8_EINVAL
    rc, msg = _status("w8a8_pack_weight_nk", fake, 64, 96, 64, 48, fake, None)
    assert rc == _lib.W8A8_EINVAL and "interleave" in msg
    rc, msg = _status("w8a8_rms_residual_bf16", fake, 8, fake, 8, None, 1e-6, 2, 8, fake, 8, fake, 8, None, None)
    assert rc == _lib.W8A8_EINVAL


def test_noalloc_linear_refuses_before_touching_the_device():
    """The allocation-free linear checks its arguments and the size of its fixed scratch before
    any HIP call, so the refusals are decided on the host."""
    fake = ctypes.c_void_p(0x100000)
    rc, msg = _status("w8a8_linear_bf16_noalloc", fake, 6144, fake, fake, 16384, 1536, 6144, 0, 0, None, 0, None,
                      1e-6, fake, 1536, None)
    assert rc == _lib.W8A8_ENOTSUP and "scratch" in msg and "64 MiB" in msg
    rc, msg = _status("w8a8_linear_bf16_noalloc", fake, 100, fake, fake, 4, 64, 100, 0, 0, None, 0, None,
                      1e-6, fake, 64, None)
    assert rc == _lib.W8A8_ENOTSUP and "multiple of 16" in msg
    rc, msg = _status("w8a8_linear_bf16_noalloc", fake, 64, fake, fake, 4, 64, 64, 3, 0, None, 0, None,
                      1e-6, fake, 64, None)
    assert rc == _lib.W8A8_EINVAL and "residual" in msg
    rc, msg = _status("w8a8_linear_bf16_noalloc", fake, 64, fake, fake, 4, 64, 64, 7, 0, None, 0, None,
                      1e-6, fake, 64, None)
    assert rc == _lib.W8A8_EINVAL and "epilogue" in msg


def test_python_layer_raises():
    import torch
    from w8a8 import ops
    with pytest.raises(ValueError, match="GPU tensor"):
        ops.quant_rows(torch.zeros(2, 16, dtype=torch.bfloat16))
    with pytest.raises(TypeError):
        ops.gemm_i32(torch.zeros(2, 16, dtype=torch.int8), object())


def test_attention_workspace_and_errors():
    """Attention workspace sizing (closed forms) and argument errors, all decided on the host."""
    L = _lib.lib()
    part512 = 32 * 512 * 16 + 128 * 16          # one split part of a 128-row tile at head_dim 512: O^T, (m, l)
    part256 = 8 * 64 * (256 // 16 + 1) * 16     # one at head_dim 256: O^T and each thread's (m, l)
    counters = 65536
    # a whole-prompt sliding-window call (229 tiles) and short causal calls need no workspace
    assert L.w8a8_attention_workspace_bytes(8, 1, 3658, 3658, 256, 0, 512) == 0
    assert L.w8a8_attention_workspace_bytes(8, 1, 200, 200, 128, 0, 0) == 0
    # a 512-query sliding-window micro-batch (32 tiles of ~9 key blocks on 256 CUs) splits every tile
    # into the same number of parts, merged by the second kernel
    ws = L.w8a8_attention_workspace_bytes(8, 1, 512, 3658, 256, 3146, 512)
    order, merge = ctypes.c_int(-1), ctypes.c_int(-1)
    items = L.w8a8_attention_plan_items(8, 1, 512, 3658, 256, 3146, 512, ctypes.byref(order), ctypes.byref(merge))
    assert items % 32 == 0 and 2 <= items // 32 <= 16 and merge.value == 1
    assert ws == counters + items * part256
    # 256 queries at the end of the 3658-token prompt, head_dim 512: 16 tiles of ~110 key blocks
    # against a fair share of 7 blocks per CU -> every tile split, into 8 to 16 (the cap) parts,
    # parked after the 64 KiB of arrival counters (at the same offsets for every shape); one round of
    # workgroups, so the merge kernel merges them
    ws = L.w8a8_attention_workspace_bytes(8, 1, 256, 3658, 512, 3402, 0)
    assert (ws - counters) % part512 == 0 and 16 * 8 <= (ws - counters) // part512 <= 16 * 16
    L.w8a8_attention_plan_items(8, 1, 256, 3658, 512, 3402, 0, None, ctypes.byref(merge))
    assert merge.value == 1
    # the whole prompt: more items than CUs, so the last part of each split tile merges it in the
    # kernel while other tiles still run
    ws = L.w8a8_attention_workspace_bytes(8, 1, 3658, 3658, 512, 0, 0)
    assert ws > counters and (ws - counters) % part512 == 0
    L.w8a8_attention_plan_items(8, 1, 3658, 3658, 512, 0, 0, None, ctypes.byref(merge))
    assert merge.value == 0
    assert L.w8a8_attention_workspace_bytes(8, 3, 16, 16, 256, 0, 0) == -1     # H % KV
    assert L.w8a8_attention_workspace_bytes(8, 1, 16, 8, 256, 0, 0) == -1      # Tk < Tq
    assert L.w8a8_attention_workspace_bytes(8, 1, 16, 16, 64, 0, 0) == -1      # head_dim
    # decode: chunks of 64 keys (32 at head_dim 512) over the visible range
    assert L.w8a8_attention_decode_workspace_bytes(8, 1, 3658, 512, 3657, 0) == 115 * 8 * 514 * 4
    assert L.w8a8_attention_decode_workspace_bytes(8, 1, 3658, 256, 3657, 512) == 8 * 8 * 258 * 4
    assert L.w8a8_attention_decode_workspace_bytes(8, 1, 1, 256, 0, 0) == 1 * 8 * 258 * 4
    assert L.w8a8_attention_decode_workspace_bytes(32, 1, 100, 256, 99, 0) == -1   # > 16 heads per KV head
    assert L.w8a8_attention_decode_workspace_bytes(8, 1, 100, 256, 100, 0) == -1   # q_pos past the keys
    fake = ctypes.c_void_p(0x100000)
    rc, msg = _status("w8a8_attention_bf16", fake, 64 * 8, 64, fake, 64 * 8, 64, fake, 64 * 8, 64, 1, 1, 8, 8, 64, 0,
                      0, 1.0, fake, 64 * 8, 64, None, None)
    assert rc == _lib.W8A8_ENOTSUP and "head_dim" in msg
    rc, msg = _status("w8a8_attention_bf16", fake, 256 * 8, 256, fake, 256 * 8, 256, fake, 256 * 8, 256, 1, 1, 8, 4,
                      256, 0, 0, 1.0, fake, 256 * 8, 256, None, None)
    assert rc == _lib.W8A8_EINVAL and "Tk >= q_start" in msg
    rc, msg = _status("w8a8_attention_bf16", fake, 256 * 8, 256, fake, 256 * 8, 256, fake, 256 * 8, 256, 1, 1, 8, 8,
                      256, 0, 0, -1.0, fake, 256 * 8, 256, None, None)
    assert rc == _lib.W8A8_EINVAL and "scale" in msg
    rc, msg = _status("w8a8_attention_bf16", fake, 256 * 8, 260, fake, 256 * 8, 256, fake, 256 * 8, 256, 1, 1, 8, 8,
                      256, 0, 0, 1.0, fake, 256 * 8, 256, None, None)
    assert rc == _lib.W8A8_EALIGN
    rc, msg = _status("w8a8_attention_decode_bf16", fake, 256, fake, 100 * 256, 256, fake, 100 * 256, 256, 8, 1, 100,
                      256, 99, 0, 1.0, fake, 256, None, fake, 16, None)
    assert rc == _lib.W8A8_EINVAL and "workspace" in msg
    rc, msg = _status("w8a8_attention_decode_bf16", fake, 256, fake, 100 * 256, 256, fake, 100 * 256, 256, 8, 1, 100,
                      256, 100, 0, 1.0, fake, 256, None, fake, 1 << 20, None)
    assert rc == _lib.W8A8_EINVAL and "q_pos" in msg


def test_attention_python_layer_raises():
    import torch
    from w8a8 import attention
    with pytest.raises(ValueError, match="GPU tensor"):
        attention.attention(*(torch.zeros(1, 4, 128, dtype=torch.bfloat16) for _ in range(3)))
    with pytest.raises(ValueError, match="batch size 1"):
        attention.local_sdpa(None, torch.zeros(2, 1, 4, 128), torch.zeros(2, 1, 4, 128), torch.zeros(2, 1, 4, 128),
                             None)


def test_clock_probe_rejects_bad_arguments_on_the_host():
    fake = ctypes.c_void_p(0x100000)
    khz = ctypes.c_int(0)
    rc, msg = _status("w8a8_clock_probe", fake, 0, ctypes.byref(khz), None)
    assert rc == _lib.W8A8_EINVAL and "ticks" in msg
    rc, msg = _status("w8a8_clock_probe", fake, 200000000, ctypes.byref(khz), None)
    assert rc == _lib.W8A8_EINVAL and "ticks" in msg
    rc, msg = _status("w8a8_clock_probe", None, 100, ctypes.byref(khz), None)
    assert rc == _lib.W8A8_EINVAL and "null" in msg
