"""Parity at the prefill workloads' own sizes, on the tiles the automatic choice takes there.

Two workloads run GEMMs far longer than the small-shape tests reach:
  * the full-prompt sweep: every prefill linear of a 3658-token prompt (qkv K1536 N2560,
    o K2048 N1536, gate_up K1536 N12288, down K6144 N1536 per layer, and the per-layer-embedding
    model projection K1536 N8960), at M = 3658 unpadded and M = 4096 (whole 512-row
    micro-batches), int8 A -> int32 C (the reference's launches, gemma_npu.py:99-115);
  * the stress case: M = 16384 rows (several prompts concatenated) with per-row magnitudes
    spread over 10^-2 .. 10^2, gate_up with the fused GELU epilogue and down with the residual
    epilogue.
At these sizes the automatic choice takes tile configurations (256-row and direct-W 128x256
tiles, one or two blocks per CU) and 32-bit offsets that a few hundred rows never exercise.

Checks, on the automatic tile choice:
  * int32 C, every element: bit-exact against torch._int_mm on the GPU (an independent exact
    int8 GEMM), and an exact int64 checksum per row and per column that ties C to A and W alone:
    C s == A (W^T s) and r^T C == (r^T A) W^T for random integer r, s;
  * rows sampled over all of M (tile edges, the ragged last tile, random rows): bit-exact
    against the reference's own CPU path, torch._int_mm on the host (pipeline.py:237);
  * bf16 epilogues on the sampled rows against the oracle: the quant prologue and dequant
    bit-exact, GELU (pipeline.py:102-107) within max(1e-2 |ref|, 2 ulp), the residual add
    bit-exact.
"""
import numpy as np
import pytest
import torch

from helpers import assert_bf16_close, f32, to_bits

import oracle.oracle as orc
from w8a8 import lib, ops, workloads

pytestmark = pytest.mark.gpu
DEV = "cuda"

SWEEP = {  # name: (K, N, group index used in the per-layer seed)
    "qkv": (1536, 2560, 0),
    "o": (2048, 1536, 1),
    "gate_up": (1536, 12288, 2),
    "down": (6144, 1536, 3),
    "ple_proj": (1536, 8960, 0),
}


def sample_rows(M, n_random=96, seed=0):
    """Rows at tile boundaries (multiples of 32 / 64 / 128 / 256 and their neighbours), the last
    rows (the ragged last tile), and random rows over all of M."""
    edges = {0, 1, 31, 32, 63, 64, 127, 128, 255, 256, 511, 512, M // 2, M - 1, M - 2, M - 33}
    edges |= {(M // 256) * 256 - 1, (M // 256) * 256, (M // 128) * 128}
    g = np.random.default_rng(seed)
    rows = edges | set(g.choice(M, size=n_random, replace=False).tolist())
    return torch.tensor(sorted(r for r in rows if 0 <= r < M), dtype=torch.long)


def checksums_equal(c, a, w, seed):
    """Exact int64 row and column checksums of C = A W^T with random integer weights in
    [-64, 64], computed on the GPU from A and W alone (no GEMM library involved)."""
    M, N = c.shape
    g = torch.Generator(device=DEV).manual_seed(seed)
    s = torch.randint(-64, 65, (N,), generator=g, device=DEV, dtype=torch.int64)
    r = torch.randint(-64, 65, (M,), generator=g, device=DEV, dtype=torch.int64)
    wl = w.to(torch.int64)
    ws = (wl * s[:, None]).sum(0)   # W^T s: [K]
    ra = torch.zeros(a.shape[1], dtype=torch.int64, device=DEV)
    ok_rows = True
    cs = torch.empty(M, dtype=torch.int64, device=DEV)
    rc = torch.zeros(N, dtype=torch.int64, device=DEV)
    for r0 in range(0, M, 1024):  # bounded int64 temporaries
        cb = c[r0:r0 + 1024].to(torch.int64)
        ab = a[r0:r0 + 1024].to(torch.int64)
        cs[r0:r0 + 1024] = (cb * s[None, :]).sum(1)
        ok_rows &= bool(torch.equal(cs[r0:r0 + 1024], (ab * ws[None, :]).sum(1)))
        rc += (cb * r[r0:r0 + 1024, None]).sum(0)
        ra += (ab * r[r0:r0 + 1024, None]).sum(0)
    ok_cols = torch.equal(rc, (wl * ra[None, :]).sum(1))
    return ok_rows, bool(ok_cols)


def _sweep_inputs(M, K, N, layer, gi):
    """The sweep's A (packed, as timed) and its row-major twin, and one layer's weight."""
    x = workloads.activations(M, K, seed=K).to(DEV)
    pa, _ = ops.quant_rows_packed(x)
    q, _ = ops.quant_rows(x)
    g = torch.Generator(device=DEV).manual_seed(workloads.layer_seed(layer, gi))
    w = torch.randint(-127, 128, (N, K), generator=g, dtype=torch.int8, device=DEV)
    return pa, q, w


@pytest.mark.parametrize("M", [3658, 4096])
@pytest.mark.parametrize("name", list(SWEEP))
def test_sweep_gemm_at_prefill_length(name, M):
    K, N, gi = SWEEP[name]
    layers = (0, 34) if name != "ple_proj" else (-1,)
    cfg = lib().w8a8_gemm_pick_tile_config(M, N, K, -1)
    for layer in layers:
        pa, q, w = _sweep_inputs(M, K, N, layer, gi)
        c = ops.gemm_i32(pa, ops.pack_weight(w, "nk"))
        ref = torch._int_mm(q, w.t())
        assert torch.equal(c, ref), f"{name} M={M} layer {layer} tile {cfg}: {(c != ref).sum().item()} mismatches"
        ok_rows, ok_cols = checksums_equal(c, q, w, seed=layer + 2)
        assert ok_rows and ok_cols, f"{name} M={M} layer {layer}: checksum rows {ok_rows} cols {ok_cols}"
        rows = sample_rows(M, seed=layer + 1)
        host = torch._int_mm(q[rows.to(DEV)].cpu(), w.cpu().t().contiguous())
        assert torch.equal(c[rows.to(DEV)].cpu(), host), f"{name} M={M} layer {layer}: vs host _int_mm"
        print(f"{name} M={M} layer {layer}: tile config {cfg}, bit-exact")
        del pa, q, w, c, ref
    torch.cuda.empty_cache()


@pytest.fixture(scope="module")
def stress_inputs():
    """M = 16384 rows with per-row magnitudes 10^-2 .. 10^2 (the stress workload's activations)."""
    out = {}
    for name in ("gate_up", "down"):
        K, N, _ = workloads.LAYER_GROUPS[name]
        x = workloads.activations(16384, K, seed=9, row_spread=True)
        w, sw = workloads.weights(N, K, seed=10 if name == "gate_up" else 11)
        out[name] = (x, w, sw)
    return out


@pytest.mark.parametrize("name", ["gate_up", "down"])
def test_stress_m16384_int32(name, stress_inputs):
    x, w, sw = stress_inputs[name]
    M, K = x.shape
    N = w.shape[0]
    xd, wd = x.to(DEV), w.to(DEV)
    pa, sx = ops.quant_rows_packed(xd)
    q, sx2 = ops.quant_rows(xd)
    assert torch.equal(sx, sx2)
    rows = sample_rows(M, seed=3)
    q_ref, sx_ref = orc.quant_rows(to_bits(x[rows]), "bf16")
    assert np.array_equal(q[rows.to(DEV)].cpu().numpy(), q_ref), "quant prologue differs from the oracle"
    assert np.array_equal(sx[rows.to(DEV)].cpu().numpy(), sx_ref)
    cfg = lib().w8a8_gemm_pick_tile_config(M, N, K, -1)
    c = ops.gemm_i32(pa, ops.pack_weight(wd, "nk"))
    ref = torch._int_mm(q, wd.t())
    assert torch.equal(c, ref), f"{name} M={M} tile {cfg}: {(c != ref).sum().item()} mismatches"
    ok_rows, ok_cols = checksums_equal(c, q, wd, seed=5)
    assert ok_rows and ok_cols
    host = torch._int_mm(torch.from_numpy(q_ref), w.t().contiguous())
    assert torch.equal(c[rows.to(DEV)].cpu(), host)
    print(f"stress {name}: tile config {cfg}, bit-exact")


def test_stress_m16384_gelu_epilogue(stress_inputs):
    """gate_up + GELU at M = 16384 (the fused epilogue of the stress workload) against the oracle
    on rows sampled over all of M."""
    x, w, sw = stress_inputs["gate_up"]
    M, K = x.shape
    I = w.shape[0] // 2
    xd = x.to(DEV)
    pa, sx = ops.quant_rows_packed(xd)
    pw = ops.pack_weight(w.to(DEV), "nk", interleave=I, sw=sw.to(DEV))
    cfg = lib().w8a8_gemm_pick_tile_config(M, 2 * I, K, 1)
    out = ops.gemm_bf16(pa, sx, pw, epilogue="gelu")
    rows = sample_rows(M, seed=4)
    ref, _, _ = orc.linear_bf16(to_bits(x[rows]), w.numpy(), sw.numpy(), epilogue="gelu")
    got = to_bits(out[rows.to(DEV)])
    assert_bf16_close(f32(got), f32(ref), what=f"gelu M={M} tile {cfg}")
    assert (got == ref).mean() > 0.99
    # the same through the one-call linear (quant prologue + GEMM + epilogue)
    out2 = ops.linear_bf16(xd, pw, epilogue="gelu")
    assert torch.equal(out2, out)
    print(f"stress gate_up+GELU: tile config {cfg}, {(got == ref).mean():.4f} bit-equal")


def test_stress_m16384_residual_epilogue(stress_inputs):
    x, w, sw = stress_inputs["down"]
    M, K = x.shape
    N = w.shape[0]
    res = workloads.activations(M, N, seed=12, outliers=False)
    xd = x.to(DEV)
    pa, sx = ops.quant_rows_packed(xd)
    pw = ops.pack_weight(w.to(DEV), "nk", sw=sw.to(DEV))
    cfg = lib().w8a8_gemm_pick_tile_config(M, N, K, 2)
    out = ops.gemm_bf16(pa, sx, pw, epilogue="residual", residual=res.to(DEV))
    rows = sample_rows(M, seed=6)
    ref, _, _ = orc.linear_bf16(to_bits(x[rows]), w.numpy(), sw.numpy(), epilogue="residual",
                                residual=to_bits(res[rows]))
    assert np.array_equal(to_bits(out[rows.to(DEV)]), ref), f"residual M={M} tile {cfg}"
    # the plain dequant on the same tile, every sampled row bit-exact
    y = ops.gemm_bf16(pa, sx, pw)
    ref_y, _, _ = orc.linear_bf16(to_bits(x[rows]), w.numpy(), sw.numpy())
    assert np.array_equal(to_bits(y[rows.to(DEV)]), ref_y)
    print(f"stress down+residual: tile config {cfg}, bit-exact")


# Past one micro-batch, GEMMs up to N = 4096 take one round of the smallest direct-W BMx256 tile
# (BM = 96, 128, 160, 192) that fits the CUs; the choice changes where ceil(M / BM) * ceil(N / 256)
# crosses the CU count (256 on MI355X), and each side of every such edge is a different tile.
ONE_ROUND_EDGES = [
    (2048, 1536, (1025, 4032, 4033)),             # output projection: 64x128, 96x256, 128x256
    (6144, 1536, (4032, 4033, 5376, 5377)),       # down: 96x256, 128x256, then 160x256
    (1536, 2560, (2400, 2401, 3200, 3201, 4000, 4001, 4800, 4801)),  # qkv: 96/128/160/192 rows, then 64x128
    # one micro-batch: 64x128 one per CU, then one round of direct-W 64x256, then 64x128 three per CU
    (1536, 6144, (256, 384, 640, 704)),
    (1536, 8192, (448, 512, 513)),
]


@pytest.mark.parametrize("K,N,Ms", ONE_ROUND_EDGES, ids=["o", "down", "qkv", "micro_n6144", "micro_n8192"])
def test_one_round_tile_edges(K, N, Ms):
    """int32 C bit-exact against torch._int_mm on both sides of every edge of the one-round tile
    choice, and the bf16 residual epilogue on the chosen tile bit-identical to the 64x128 tile's."""
    g = torch.Generator(device=DEV).manual_seed(K + N)
    w = torch.randint(-127, 128, (N, K), generator=g, dtype=torch.int8, device=DEV)
    _, sw = workloads.weights(N, K, seed=K)
    pw = ops.pack_weight(w, "nk", sw=sw.to(DEV))
    picked = set()
    for M in Ms:
        x = workloads.activations(M, K, seed=M).to(DEV)
        pa, sx = ops.quant_rows_packed(x)
        q, _ = ops.quant_rows(x)
        cfg = lib().w8a8_gemm_pick_tile_config(M, N, K, -1)
        picked.add(cfg)
        c = ops.gemm_i32(pa, pw)
        ref = torch._int_mm(q, w.t())
        assert torch.equal(c, ref), f"K={K} N={N} M={M} tile {cfg}: {(c != ref).sum().item()} mismatches"
        res = workloads.activations(M, N, seed=M + 1, outliers=False).to(DEV)
        y = ops.gemm_bf16(pa, sx, pw, epilogue="residual", residual=res)
        y12 = ops.gemm_bf16(pa, sx, pw, epilogue="residual", residual=res, tile_cfg=0)  # 64x128
        assert torch.equal(y, y12), f"K={K} N={N} M={M}: residual epilogue differs between tiles"
    assert len(picked) >= 2, f"K={K} N={N}: the edges {Ms} gave one tile {picked}"
