"""W8A8 linear engine benchmark on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu] [--no-extra]

A step is one E2B-class decoder layer's prefill linears on one 512-row micro-batch, bf16 in
-> bf16 out, each with its fused quant prologue and dequant epilogue:
  qkv     K=1536 N=2560            (dequant)
  o       K=2048 N=1536            (dequant)
  gate_up K=1536 N=2x6144          (dequant + gelu_tanh(gate) * up)
  down    K=6144 N=1536            (dequant + residual add)
The step's 8 launches (quant-to-packed + GEMM per linear) are issued eagerly on torch's
current stream, one linear_bf16 call per linear as the reference's pipeline calls mm_i8; the
outputs of the timed steps are checked bit for bit against the first run.  `value` is int8
TOP/s over the step's 2*M*N*K ops with inputs resident in HBM.  The JSON line also carries the
roofline of the dominant kernel (the gate_up GEMM, timed live with HIP events on the launch
stream), the host CPU's torch._int_mm on the same GEMMs (the reference's --backend cpu-int8
path, pipeline.py:237), and `extra`: the same step captured in one HIP graph and replayed
(checked bit for bit against the eager run; also 50 steps per graph, which spreads a replay's fixed
launch cost), the full-prefill GEMM sweep at M=3658 / 4096, the M=16384
stress GEMMs, the int32 GEMMs of those shapes against hipBLASLt (torch._int_mm on the same GPU, cold
weights), a decoder layer's whole linear path on the device (the six GEMMs with the fused
norm / RoPE / GELU / residual / quant kernels between them, one HIP graph), and the decode GEMV
bandwidth.
"""
import argparse
import json
import os
import statistics
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "gemma-npu_amd"))
sys.path.insert(0, ROOT)

PEAK_INT8_TOPS = 5000.0   # MI355X dense int8 MFMA, published
PEAK_HBM_GBS = 8000.0     # MI355X HBM3E, published
PEAK_BF16_TFLOPS = 2500.0  # MI355X dense bf16 MFMA, published
# Gemma 4 E2B attention: 8 query heads on 1 KV head; 28 sliding layers (head_dim 256, window 512)
# and 7 full layers (head_dim 512); the reference's benchmark prompt is 3658 tokens.
ATTN_H, ATTN_KV, ATTN_T = 8, 1, 3658
ATTN_LAYERS = {"sliding": (256, 512, 28), "full": (512, 0, 7)}
PMC_SUMMARY = os.path.join(ROOT, "profiles", "gemm_gate_up_m512_traffic.md")


def log(msg):
    print(msg, file=sys.stderr, flush=True)


def event_time_ms(fn, reps, warmup):
    import torch
    for _ in range(warmup):
        fn()
    s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    s.record()
    for _ in range(reps):
        fn()
    e.record()
    e.synchronize()
    return s.elapsed_time(e) / reps


def build_layer(M, dev, seed0=0):
    import torch
    from w8a8 import ops, workloads
    groups = []
    for gi, (name, (K, N, epi)) in enumerate(workloads.LAYER_GROUPS.items()):
        x = workloads.activations(M, K, seed=seed0 + 10 * gi).to(dev)
        w, sw = workloads.weights(N, K, seed=seed0 + 10 * gi + 1)
        pw = ops.pack_weight(w.to(dev), "nk", N // 2 if epi == "gelu" else 0, sw=sw.to(dev))
        ncols = N // 2 if epi == "gelu" else N
        out = torch.empty((M, ncols), dtype=torch.bfloat16, device=dev)
        res = workloads.activations(M, N, seed=seed0 + 10 * gi + 2, outliers=False).to(dev) if epi == "residual" else None
        q, sx = ops.quant_rows_packed(x)
        groups.append(dict(name=name, K=K, N=N, epi=epi, x=x, w=w, pw=pw, out=out, res=res, q=q, sx=sx))
    return groups


def single_gemm(dev, M=512, K=1536, N=6144):
    """The single prefill micro-batch GEMM (M=512 K=1536 N=6144, seed 0: int8 A from the quantized
    activations, int32 out) on the automatic tile: average launch from a 50-launch graph, with the
    output checked bit for bit against the eager launch."""
    import torch
    from w8a8 import lib, ops, workloads
    x, w, _ = workloads.single_gemm_inputs(M, K, N, seed=0)
    a, _ = ops.quant_rows_packed(x.to(dev))
    pw = ops.pack_weight(w.to(dev), "nk")
    c = torch.empty((M, N), dtype=torch.int32, device=dev)
    ops.gemm_i32(a, pw, c)
    first = c.clone()
    ms = graph_time_ms(lambda: ops.gemm_i32(a, pw, c), dev)
    if not torch.equal(c, first):
        raise RuntimeError("graph-replayed single GEMM differs from its eager launch")
    t = workloads.gemm_ops(M, N, K) / (ms * 1e-3) / 1e12
    return {"us": round(ms * 1e3, 2), "tops": round(t, 1), "frac_mfma": round(t / PEAK_INT8_TOPS, 4),
            "tile": tile_name(lib().w8a8_gemm_pick_tile_config(M, N, K, -1)),
            "shape": f"M={M} K={K} N={N}, packed int8 A, int32 out, weights hot"}


def host_slot_gemm(dev, M=512, K=1536, N=6144, reps=50):
    """The same single GEMM through the drop-in `npu_kernels.mm_i8` on the reference's host-side
    resident buffers (gemma_npu.py:89-115): A staged in pinned host memory, C read back into it,
    the weight resident in HBM.  Each synchronous call moves A (M*K bytes) to the GPU and the int32
    C (4*M*N bytes) back over PCIe; this is the boundary's host-buffer rate, not the HBM-resident
    `value`."""
    import time
    import torch
    import npu_kernels
    from w8a8 import ops, resident, workloads
    x, w, _ = workloads.single_gemm_inputs(M, K, N, seed=0)
    a_dev, _ = ops.quant_rows(x.to(dev))
    a = resident.empty((M, K), dtype=torch.int8)
    a.copy_(a_dev.cpu())
    c = resident.empty((M, N), dtype=torch.int32)
    b = resident.to_npu(w.t().contiguous(), static=True, device=dev)
    for _ in range(3):
        npu_kernels.mm_i8(a, b, c)
    ref = c.clone()
    t0 = time.perf_counter()
    for _ in range(reps):
        npu_kernels.mm_i8(a, b, c)
    us = (time.perf_counter() - t0) / reps * 1e6
    if not torch.equal(c, ref):
        raise RuntimeError("host-slot mm_i8 results differ between calls")
    nbytes = M * K + 4 * M * N
    return {"us": round(us, 1), "tops": round(workloads.gemm_ops(M, N, K) / (us * 1e-6) / 1e12, 1),
            "pcie_bytes": nbytes, "pcie_gbs": round(nbytes / (us * 1e-6) / 1e9, 1),
            "what": f"npu_kernels.mm_i8 on pinned host A [{M}, {K}] int8 and C [{M}, {N}] int32 "
                    "(the reference's resident host slots), packed weight in HBM; synchronous calls, wall clock"}


def layer_step(groups, ws=None):
    from w8a8 import ops
    for g in groups:
        ops.linear_bf16(g["x"], g["pw"], epilogue=g["epi"], residual=g["res"], out=g["out"], ws_arg=ws)


def capture(fn, dev):
    """fn's launches captured in one HIP graph (after one warm run on the capture stream)."""
    import torch
    side = torch.cuda.Stream(dev)
    side.wait_stream(torch.cuda.current_stream(dev))
    with torch.cuda.stream(side):
        fn()
    torch.cuda.current_stream(dev).wait_stream(side)
    torch.cuda.synchronize(dev)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        fn()
    torch.cuda.synchronize(dev)
    return graph


def graph_time_ms(fn, dev, launches=50, reps=10):
    """Average duration of fn's launch sequence: `launches` copies captured in one graph,
    replayed `reps` times between HIP events on the current stream."""
    import torch

    def many():
        for _ in range(launches):
            fn()
    graph = capture(many, dev)
    graph.replay()
    s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize(dev)
    s.record()
    for _ in range(reps):
        graph.replay()
    e.record()
    e.synchronize()
    return s.elapsed_time(e) / (reps * launches)


def clock_during(fn, dev, launches=100, window_ms=1.0):
    """Engine clock (GHz) while fn's kernels run: `launches` copies of fn captured in one graph and
    replayed on the current stream, while w8a8_clock_probe's one wave on a second stream (default
    priority) counts core cycles against the real-time counter over `window_ms` inside the replay."""
    import ctypes
    import torch
    from w8a8._lib import call
    out = torch.zeros(2, dtype=torch.int64, device=dev)
    khz = ctypes.c_int(0)
    side = torch.cuda.Stream(dev)
    call("w8a8_clock_probe", out.data_ptr(), 100, ctypes.byref(khz), side.cuda_stream)
    torch.cuda.synchronize(dev)

    def many():
        for _ in range(launches):
            fn()
    graph = capture(many, dev)
    replay_ms = event_time_ms(graph.replay, 1, 1)
    window_ms = min(window_ms, 0.6 * replay_ms)
    ticks = max(1, int(khz.value * window_ms))
    torch.cuda.synchronize(dev)
    graph.replay()
    call("w8a8_clock_probe", out.data_ptr(), ticks, ctypes.byref(khz), side.cuda_stream)
    torch.cuda.synchronize(dev)
    cycles, real = out.tolist()
    return cycles / (real / (khz.value * 1e3)) / 1e9


def read_traffic():
    """HBM bytes per launch of the dominant kernel, from the committed rocprofv3 counter summary
    (FETCH_SIZE + WRITE_SIZE, each calibrated on a 64 MiB copy); None if it is absent."""
    try:
        with open(PMC_SUMMARY) as f:
            for line in f:
                if line.startswith("hbm_bytes_per_launch:"):
                    return int(line.split(":")[1])
    except OSError:
        pass
    return None


def cpu_int_mm_ms(shapes, M, warm=3, reps=5, budget_s=None):
    """Median ms of torch._int_mm (host CPU) per (K, N) shape: `warm` untimed calls, then `reps`
    timed ones, or as many rounds over all shapes as fit in `budget_s` seconds."""
    import torch
    g = torch.Generator().manual_seed(0)
    ops = {}
    for K, N in shapes:
        a = torch.randint(-127, 128, (M, K), generator=g, dtype=torch.int8)
        w = torch.randint(-127, 128, (K, N), generator=g, dtype=torch.int8)
        for _ in range(warm):
            torch._int_mm(a, w)
        ops[(K, N)] = (a, w)
    ts = {s: [] for s in ops}
    t_start = time.perf_counter()
    rounds = 0
    while True:
        for s, (a, w) in ops.items():
            t = time.perf_counter()
            torch._int_mm(a, w)
            ts[s].append(time.perf_counter() - t)
        rounds += 1
        if budget_s is None:
            if rounds >= reps:
                break
        elif time.perf_counter() - t_start >= budget_s and rounds >= 3:
            break
    return {s: statistics.median(v) * 1e3 for s, v in ts.items()}, rounds


TILE_NAMES = {
    0: "gemm_kernel 64x128 tiles, three blocks per CU",
    1: "gemm_kernel 64x64 tiles, two waves",
    2: "gemm_kernel 64x128 tiles, two waves per 32-row sub-tile splitting its k-steps",
    3: "gemm_kernel 64x64 tiles with 4-wave split-K, 512-deep k-tiles",
    4: "gemm_dw_kernel (direct-W) 64x256 tiles, two blocks per CU",
    5: "gemm_dw_kernel (direct-W) 128x256 tiles, W 8 k-steps ahead",
    6: "gemm_dw_kernel (direct-W) 128x256 tiles, two blocks per CU",
    7: "gemm_dw_kernel (direct-W) 96x256 tiles, W 8 k-steps ahead",
    8: "gemm_dw_kernel (direct-W) 160x256 tiles, W 8 k-steps ahead",
    9: "gemm_dw_kernel (direct-W) 192x256 tiles, W 8 k-steps ahead",
    10: "gemm_pipe_kernel (software-pipelined, persistent) 256x256 tiles",
}


def tile_name(cfg):
    return TILE_NAMES.get(cfg, f"tile configuration {cfg}")


def cpu_identity():
    """nproc, the CPU model string and the int8 / bf16 matrix ISA flags of the host (Linux)."""
    model, flags = "unknown", set()
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name") and model == "unknown":
                    model = line.split(":", 1)[1].strip()
                elif line.startswith("flags") and not flags:
                    flags = set(line.split(":", 1)[1].split())
    except OSError:
        pass
    isa = [x for x in ("amx_int8", "amx_bf16", "avx512_vnni", "avx_vnni", "avx512_bf16", "avx512f") if x in flags]
    return {"nproc": os.cpu_count(), "cpu_model": model, "isa": isa}


def cpu_gemv_ms(M, K, N, warm=3, reps=5, seed=5):
    """Median ms of torch._weight_int8pack_mm on the host (the reference's decode linear and int8
    LM head, gemma_npu.py:155-156): x bf16 [M, K], w int8 [N, K], bf16 per-channel scales."""
    import torch
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(M, K, generator=g).to(torch.bfloat16)
    w = torch.randint(-127, 128, (N, K), generator=g, dtype=torch.int8)
    s = (torch.rand(N, generator=g) * 0.015 + 0.005).to(torch.bfloat16)
    for _ in range(warm):
        torch._weight_int8pack_mm(x, w, s)
    ts = []
    for _ in range(reps):
        t = time.perf_counter()
        torch._weight_int8pack_mm(x, w, s)
        ts.append(time.perf_counter() - t)
    return statistics.median(ts) * 1e3


def gemv_layers(dev, reps, cpu=True):
    """Decode GEMVs of one E2B-class layer's linears (qkv, o, gate_up, down) at M = 1 / 4 / 16, int8
    weights in the GEMV fragment layout, bf16 scales as the reference's decode copy (gemma_npu.py:82):
      hot   each shape alone, the same weight replayed from one graph (it stays in the 256 MB MALL);
      cold  one decode token's linears: 35 layers x 4 groups with distinct weights (1.24 GB, five
            times the MALL) back to back, as the decode loop streams them: launched eagerly (Python
            launch overhead included), and captured in one HIP graph.
    Bytes per GEMV = K*N + 2N + 2MK + 2MN; the host leg is torch._weight_int8pack_mm per shape."""
    import torch
    from w8a8 import ops, workloads
    out = {}
    groups = list(workloads.LAYER_GROUPS.items())
    layers = []
    for layer in range(workloads.N_LAYERS):
        row = []
        for gi, (name, (K, N, _)) in enumerate(groups):
            g = torch.Generator(device=dev).manual_seed(workloads.layer_seed(layer, gi))
            w = torch.randint(-127, 128, (N, K), generator=g, dtype=torch.int8, device=dev)
            s = (torch.rand(N, generator=g, device=dev) * 0.015 + 0.005).to(torch.bfloat16)
            row.append((name, K, N, ops.pack_gemv_weight(w), s))
            del w
        layers.append(row)
    for M in (1, 4, 16):
        xs = {K: workloads.activations(M, K, seed=K, outliers=False).to(dev) for _, (K, _, _) in groups}
        ys = {N: torch.empty((M, N), dtype=torch.bfloat16, device=dev) for _, (_, N, _) in groups}
        entry = {}
        for name, K, N, pw, s in layers[0]:
            ms = graph_time_ms(lambda: ops.gemv_bf16(xs[K], pw, s, ys[N]), dev)
            nbytes = K * N + 2 * N + 2 * M * K + 2 * M * N
            e = {"us": round(ms * 1e3, 2), "gbs": round(nbytes / (ms * 1e-3) / 1e9, 1), "bytes": nbytes}
            if cpu:
                cms = cpu_gemv_ms(M, K, N)
                e["cpu_us"] = round(cms * 1e3, 1)
                e["speedup_vs_cpu"] = round(cms / ms, 1)
            entry[name] = e

        def token():
            for row in layers:
                for name, K, N, pw, s in row:
                    ops.gemv_bf16(xs[K], pw, s, ys[N])
        nbytes = sum(K * N + 2 * N + 2 * M * K + 2 * M * N for row in layers for _, K, N, _, _ in row)

        def rate(ms):
            return {"us": round(ms * 1e3, 1), "gemvs": 4 * len(layers), "bytes": nbytes,
                    "gbs": round(nbytes / (ms * 1e-3) / 1e9, 1),
                    "frac_hbm": round(nbytes / (ms * 1e-3) / 1e9 / PEAK_HBM_GBS, 4)}
        ms = event_time_ms(token, reps, 2)
        entry["cold_token_all_layers"] = rate(ms)
        ref = ys[workloads.LAYER_GROUPS["down"][1]].clone()
        graph = capture(token, dev)
        ys[workloads.LAYER_GROUPS["down"][1]].zero_()
        entry["cold_token_graph"] = rate(event_time_ms(graph.replay, reps, 2))
        if not torch.equal(ys[workloads.LAYER_GROUPS["down"][1]], ref):
            raise RuntimeError("the captured token's last GEMV differs from the eager one")
        del graph
        out[f"m{M}"] = entry
        log(f"bench: decode layer GEMVs M={M}: {entry}")
    return out


def sweep(M, dev, reps, epilogues=False):
    """All prefill GEMMs of one prompt: 35 layers x 4 groups + the PLE projection, distinct weights per
    layer.  int8 A -> int32 C (the reference's NPU launches, gemma_npu.py:99-115), or with epilogues
    each group with its epilogue of one E2B-class layer's linears: bf16 out (dequantised with the
    per-token and per-channel scales), gate/up with the GELU product (N/2 bf16 columns), down with
    the residual add."""
    import torch
    from w8a8 import ops, workloads
    shapes = workloads.sweep_shapes()
    epi_of = dict(workloads.LAYER_GROUPS, ple_proj=workloads.PLE_PROJ)
    A = {}
    packed = []
    for name, layer, gi, K, N in shapes:
        if K not in A:
            A[K] = ops.quant_rows_packed(workloads.activations(M, K, seed=K).to(dev))
        g = torch.Generator(device=dev).manual_seed(workloads.layer_seed(layer, gi))
        w = torch.randint(-127, 128, (N, K), generator=g, dtype=torch.int8, device=dev)
        epi = epi_of[name][2] if epilogues else "int32"
        if epilogues:
            sw = torch.rand(N, generator=g, device=dev) * 0.015 + 0.005
            packed.append((K, N, epi, ops.pack_weight(w, "nk", N // 2 if epi == "gelu" else 0, sw=sw)))
        else:
            packed.append((K, N, epi, ops.pack_weight(w, "nk")))
        del w
    if epilogues:
        C = {(N, e): torch.empty((M, N // 2 if e == "gelu" else N), dtype=torch.bfloat16, device=dev)
             for _, N, e, _ in packed}
        R = {N: torch.randn((M, N), device=dev).to(torch.bfloat16) for _, N, e, _ in packed if e == "residual"}
    else:
        C = {N: torch.empty((M, N), dtype=torch.int32, device=dev) for _, _, _, _, N in shapes}

    def run():
        for K, N, epi, pw in packed:
            if epilogues:
                ops.gemm_bf16(A[K][0], A[K][1], pw, epilogue=epi, residual=R.get(N) if epi == "residual" else None,
                              out=C[(N, epi)])
            else:
                ops.gemm_i32(A[K][0], pw, C[N])

    ms = event_time_ms(run, reps, 2)
    total_ops = sum(workloads.gemm_ops(M, N, K) for _, _, _, K, N in shapes)
    wbytes = sum(K * N for _, _, _, K, N in shapes)
    return ms, total_ops, wbytes, [(K, N) for _, _, _, K, N in shapes], run


def vendor_compare(dev, cases=((3658, ("qkv", "o", "gate_up", "down", "ple_proj")),
                               (16384, ("gate_up", "down")))):
    """The int32 GEMM (automatic tile) against hipBLASLt through torch._int_mm on the same GPU, the
    same operands and the same weight temperature: per shape, enough distinct weight copies to pass
    512 MB (more than the 256 MB MALL) are cycled, so both read their weights cold; each side is
    timed twice, alternating, and the faster run kept.  hipBLASLt has no fused epilogues, so the
    comparison is int8 -> int32 on both sides; outputs are compared bit for bit."""
    import torch
    from w8a8 import lib, ops, workloads
    shapes = dict(workloads.LAYER_GROUPS, ple_proj=workloads.PLE_PROJ)
    out = {}
    for M, names in cases:
        for name in names:
            K, N, _ = shapes[name]
            copies = max(2, -(-512 * 2 ** 20 // (K * N)))
            g = torch.Generator(device=dev).manual_seed(77)
            a = torch.randint(-127, 128, (M, K), generator=g, dtype=torch.int8, device=dev)
            ap = ops.pack_act(a)
            ws = [torch.randint(-127, 128, (N, K), generator=g, dtype=torch.int8, device=dev) for _ in range(copies)]
            pws = [ops.pack_weight(w, "nk") for w in ws]
            wts = [w.t() for w in ws]  # [K, N] column-major: hipBLASLt's faster B layout here
            c = torch.empty((M, N), dtype=torch.int32, device=dev)
            it = [0]

            def ours():
                ops.gemm_i32(ap, pws[it[0] % copies], c)
                it[0] += 1

            def theirs():
                torch._int_mm(a, wts[it[0] % copies], out=c)
                it[0] += 1

            n = max(copies, 20)
            t = {"ours": 1e9, "hipblaslt": 1e9}
            for _ in range(2):
                t["ours"] = min(t["ours"], event_time_ms(ours, n, 2))
                t["hipblaslt"] = min(t["hipblaslt"], event_time_ms(theirs, n, 2))
            ref = torch._int_mm(a, wts[0])
            ops.gemm_i32(ap, pws[0], c)
            same = bool(torch.equal(ref, c))
            key = f"m{M}_{name}"
            out[key] = {"K": K, "N": N, "tile": lib().w8a8_gemm_pick_tile_config(M, N, K, -1),
                        "ours_us": round(t["ours"] * 1e3, 1), "hipblaslt_us": round(t["hipblaslt"] * 1e3, 1),
                        "speedup": round(t["hipblaslt"] / t["ours"], 3), "bit_exact": same}
            log(f"bench: vs hipBLASLt {key}: {out[key]}")
            del a, ap, ws, pws, wts, c, ref
            torch.cuda.empty_cache()
    return out


def gemv_bench(M, K, N, dev, reps, seed=5):
    import torch
    from w8a8 import ops, workloads
    x = workloads.activations(M, K, seed=seed, outliers=False).to(dev)
    g = torch.Generator(device=dev).manual_seed(seed)
    w = torch.randint(-127, 128, (N, K), generator=g, dtype=torch.int8, device=dev)
    s = (torch.rand(N, generator=g, device=dev) * 0.015 + 0.005).to(torch.bfloat16)
    y = torch.empty((M, N), dtype=torch.bfloat16, device=dev)
    ms = event_time_ms(lambda: ops.gemv_bf16(x, w, s, y), reps, 3)
    pw = ops.pack_gemv_weight(w)
    del w
    ms_packed = event_time_ms(lambda: ops.gemv_bf16(x, pw, s, y), reps, 3)
    nbytes = K * N + 2 * N + 2 * M * K + 2 * M * N
    return ms, ms_packed, nbytes


def build_chain(M, dev, seed0=500):
    """A decoder layer's whole linear path on the device (pipeline.py:244-310 without the
    attention itself): the six GEMMs of an E2B-class layer and the fused kernels between them.
    The attention output is stood in for by the rotated q heads."""
    import torch
    from w8a8 import ops, workloads
    E, H, KV, D, I, P = workloads.HIDDEN, 8, 1, 256, 6144, 256
    shapes = {"qkv": ((H + 2 * KV) * D, E, 0), "o": (E, H * D, 0), "gate_up": (2 * I, E, I), "down": (E, I, 0),
              "ple_gate": (P, E, 0), "ple_proj": (E, P, 0)}
    c = {"M": M, "H": H, "KV": KV, "D": D, "I": I, "eps": 1e-6, "pw": {}}
    for i, (name, (N, K, inter)) in enumerate(shapes.items()):
        w, sw = workloads.weights(N, K, seed=seed0 + i)
        c["pw"][name] = ops.pack_weight(w.to(dev), "nk", inter, sw=sw.to(dev))
    g = torch.Generator().manual_seed(seed0 + 99)
    c["norm"] = {n: (torch.rand(D if n in ("qw", "kw") else E, generator=g) + 0.5).to(torch.bfloat16).to(dev)
                 for n in ("in", "qw", "kw", "post", "pre_ff", "post_ff", "post_ple")}
    ang = torch.arange(M).float()[:, None] * (10000.0 ** (-torch.arange(0, D, 2).float() / D))[None, :]
    ang = torch.cat([ang, ang], dim=-1)
    c["cos"], c["sin"] = ang.cos().to(torch.bfloat16).to(dev), ang.sin().to(torch.bfloat16).to(dev)
    c["ple"] = workloads.activations(M, P, seed=seed0 + 98, outliers=False).to(dev)
    c["scalar"] = torch.tensor([0.8], dtype=torch.bfloat16, device=dev)
    c["h0"] = workloads.activations(M, E, seed=seed0 + 97).to(dev)
    c["ops"] = sum(workloads.gemm_ops(M, N, K) for N, K, _ in shapes.values())
    c["launches"] = 14
    return c


def chain_step(c, dequant_in_gemm=False):
    """k_in -> qkv -> k_qkv -> k_attn_out -> o -> k_post_attn -> gate_up (GELU epilogue) -> quant
    -> down -> k_post_ff -> ple_gate -> k_ple_gate -> ple_proj -> k_ple_out; returns the new h.  The
    GEMMs before the fused kernels hand over their int32 result (as w8a8.pipeline does at this row
    count), or with dequant_in_gemm their dequantised bf16 result (the same bits)."""
    from w8a8 import fused, ops
    pw, nw, eps = c["pw"], c["norm"], c["eps"]

    def gemm(xq, sx, w):
        return ops.gemm_bf16(xq, sx, w) if dequant_in_gemm else ops.gemm_i32(xq, w)
    xq, sx = fused.k_in(c["h0"], nw["in"], eps, packed=True)
    acc = gemm(xq, sx, pw["qkv"])
    q, k, v = fused.k_qkv(acc, sx, pw["qkv"].sw, c["cos"], c["sin"], nw["qw"], nw["kw"], eps, c["H"], c["KV"],
                          c["D"], False)
    xq, sx = fused.k_attn_out(q, packed=True)
    acc = gemm(xq, sx, pw["o"])
    h, xq, sx = fused.k_post_attn(acc, sx, pw["o"].sw, c["h0"], nw["post"], nw["pre_ff"], eps, packed=True)
    a = ops.gemm_bf16(xq, sx, pw["gate_up"], epilogue="gelu")
    xq, sx = ops.quant_rows_packed(a)
    acc = gemm(xq, sx, pw["down"])
    h, xq, sx = fused.k_post_ff(acc, sx, pw["down"].sw, h, nw["post_ff"], eps, packed=True)
    acc = gemm(xq, sx, pw["ple_gate"])
    xq, sx = fused.k_ple_gate(acc, sx, pw["ple_gate"].sw, c["ple"], packed=True)
    acc = gemm(xq, sx, pw["ple_proj"])
    c["out"] = fused.k_ple_out(acc, sx, pw["ple_proj"].sw, h, nw["post_ple"], c["scalar"], eps)
    return c["out"]


def time_chain(M, dev, reps):
    """(graph-replayed us, eager us) of one chain step; the replay must equal the eager result."""
    import torch
    c = build_chain(M, dev)
    ref = chain_step(c).clone()
    if not torch.equal(chain_step(c, dequant_in_gemm=True), ref):
        raise RuntimeError("the bf16 hand-over gives another layer chain result than the int32 one")
    graph = capture(lambda: chain_step(c), dev)
    c["out"].zero_()
    graph.replay()
    torch.cuda.synchronize()
    if not torch.equal(c["out"], ref):
        raise RuntimeError("captured layer chain differs from eager")
    ms = event_time_ms(graph.replay, reps, 5)
    eager = event_time_ms(lambda: chain_step(c), reps, 5)
    graph16 = capture(lambda: chain_step(c, dequant_in_gemm=True), dev)
    c["bf16_handover_us"] = round(event_time_ms(graph16.replay, reps, 5) * 1e3, 1)
    return ms, eager, c


COPY_BYTES = 64 << 20


def attention_pairs(q_start, Tq, window):
    """(query, key) pairs the masked softmax covers for queries q_start .. q_start + Tq - 1."""
    n = 0
    for i in range(Tq):
        p = q_start + i
        n += p + 1 if window == 0 else min(p + 1, window)
    return n


def attention_inputs(D, T, dev, seed):
    import torch
    g = torch.Generator(device=dev).manual_seed(seed)
    q = (torch.randn(ATTN_H, T, D, generator=g, device=dev) * 0.3).to(torch.bfloat16)
    k = (torch.randn(ATTN_KV, T, D, generator=g, device=dev) * 0.3).to(torch.bfloat16)
    v = torch.randn(ATTN_KV, T, D, generator=g, device=dev).to(torch.bfloat16)
    return q, k, v


def e2b_model(dev):
    """A Gemma 4 E2B-shaped text decoder (HF transformers' own model code), random-init in bf16 on
    the GPU, with the engine underneath (w8a8.hf.to_gpu).  Shapes: hidden 1536, 35 layers (4
    sliding + 1 full, repeated), 8 query heads on 1 KV head, head_dim 256 / 512, window 512, the
    last 20 layers KV-shared with double-wide MLPs, 256-wide per-layer inputs, vocab 262144.  The q /
    k norm weights are head_dim^-1/4, as a trained model's small norm weights keep the (scale 1.0)
    scores near unit variance; with the init's 1.0 the random model's softmax is nearly one-hot and
    any rounding difference grows layer by layer, which would make logit comparisons meaningless."""
    import torch
    from transformers.models.gemma4.configuration_gemma4 import Gemma4TextConfig
    from transformers.models.gemma4.modeling_gemma4 import Gemma4ForCausalLM
    from w8a8 import hf
    cfg = Gemma4TextConfig(vocab_size=262144, hidden_size=1536, intermediate_size=6144, num_hidden_layers=35,
                           num_attention_heads=8, num_key_value_heads=1, head_dim=256, global_head_dim=512,
                           sliding_window=512, layer_types=(["sliding_attention"] * 4 + ["full_attention"]) * 7,
                           num_kv_shared_layers=20, use_double_wide_mlp=True, vocab_size_per_layer_input=262144,
                           hidden_size_per_layer_input=256, final_logit_softcapping=30.0)
    torch.manual_seed(0)
    old = torch.get_default_dtype()
    torch.set_default_dtype(torch.bfloat16)
    try:
        with torch.device(dev):
            model = Gemma4ForCausalLM(cfg).eval()
    finally:
        torch.set_default_dtype(old)
    with torch.no_grad():
        for layer in model.model.layers:
            a = layer.self_attn
            a.q_norm.weight.fill_(a.head_dim ** -0.25)
            if getattr(a, "k_norm", None) is not None:
                a.k_norm.weight.fill_(a.head_dim ** -0.25)
    nparams = sum(p.numel() for p in model.parameters())
    hf.to_gpu(model)
    return model, nparams


def pipeline_prefill_bench(model, ids, hf_logits, reps=3):
    """The reference's prefill pipeline (pipeline.py:224-339) on the GPU, w8a8.pipeline.Prefill, on
    the same model and prompt: whole-prompt layers (the default), the reference's 512-row
    micro-batches, and the whole-prompt layers captured in one HIP graph (Prefill.capture); each the
    median of `reps` timed calls after one warm-up.  Logits are compared with the HF-driven engine's
    (relative L2 difference of the last-token logits); the captured form must equal the eager one."""
    import torch
    from w8a8.pipeline import Prefill
    res = {}
    for name, step in (("whole_prompt", None), ("row_step_512", 512)):
        pre = Prefill(model, row_step=step)
        times = []
        for _ in range(reps + 1):
            torch.cuda.synchronize()
            t = time.perf_counter()
            logits, _ = pre(ids)
            torch.cuda.synchronize()
            times.append(time.perf_counter() - t)
        diff = ((logits - hf_logits).norm() / hf_logits.norm()).item()
        res[name] = {"ms": round(statistics.median(times[1:]) * 1e3, 2), "logits_rel_diff_vs_hf_engine": round(diff, 4)}
        log(f"bench: pipeline prefill {name}: {res[name]}")
    # the layers captured in one HIP graph (Prefill.capture), checked against the eager call on the
    # same prompt: the whole-prompt order is GPU-bound already, the micro-batch order host-bound
    for name, step in (("whole_prompt_graph", None), ("row_step_512_graph", 512)):
        pre = Prefill(model, row_step=step)
        want, _ = pre(ids)
        run = pre.capture(ids.shape[1])
        times = []
        for _ in range(reps + 1):
            torch.cuda.synchronize()
            t = time.perf_counter()
            logits, _ = run(ids)
            torch.cuda.synchronize()
            times.append(time.perf_counter() - t)
        if not torch.equal(logits, want):
            raise RuntimeError(f"captured prefill ({name}) differs from the eager prefill")
        res[name] = {"ms": round(statistics.median(times[1:]) * 1e3, 2), "identical_to_eager": True}
        log(f"bench: pipeline prefill {name}: {res[name]}")
        del run
    res["what"] = ("w8a8.pipeline.Prefill: embedding/PLE/RoPE tables from the model, then per layer k_in, qkv "
                   "GEMM, k_qkv, attention, k_attn_out, o GEMM, k_post_attn, gate/up GEMM, k_gelu, down GEMM, "
                   "k_post_ff, PLE gate GEMM, k_ple_gate, PLE projection GEMM, k_ple_out (int32 GEMMs + fused "
                   "kernels + attention kernels), final norm and the int8 LM head GEMV; returns the logits and "
                   "the filled DynamicCache")
    return res


def native_decode_bench(model, ids, n):
    """w8a8.pipeline.Decoder on the same model and prompt: n greedy steps eagerly and n replayed from
    one HIP graph (one step per replay), each after the whole-prompt prefill; tokens per second from
    the host clock around the steps (one synchronisation at the end).  Its greedy tokens are checked
    against HF's own loop on the engine continuing from the same whole-prompt prefill's cache (the
    first token is the prefill's argmax, then n steps)."""
    import torch
    from w8a8.pipeline import Decoder, Prefill
    T = ids.shape[1]
    logits, past = Prefill(model)(ids)
    nxt = logits.argmax().view(1, 1)
    hf_tokens = [nxt.view(1)]
    for _ in range(n):
        o = model(input_ids=nxt, past_key_values=past, use_cache=True, logits_to_keep=1)
        past, nxt = o.past_key_values, o.logits[0, -1].argmax().view(1, 1)
        hf_tokens.append(nxt.view(1))
    hf_tokens = torch.cat(hf_tokens).tolist()
    del past, o
    # the same steps fed HF's tokens (teacher-forced): logits against HF's loop step by step
    dec = Decoder(Prefill(model), max_len=T + n + 8)
    dec.start(ids)
    worst, agree = 0.0, 0
    logits, past = Prefill(model)(ids)
    nxt = logits.argmax().view(1, 1)
    for _ in range(n):
        o = model(input_ids=nxt, past_key_values=past, use_cache=True, logits_to_keep=1)
        want = o.logits[0, -1].float()
        dec.tok.copy_(nxt)
        got = dec.step()
        worst = max(worst, ((got - want).norm() / want.norm()).item())
        agree += int(int(got.argmax()) == int(want.argmax()))
        past, nxt = o.past_key_values, want.argmax().view(1, 1)
    del dec, past, o
    res = {"vs_hf_loop": {"max_rel_logits_diff": round(worst, 5), "argmax_agree": f"{agree}/{n}",
                          "how": "each step fed HF's token; HF's loop on the same engine from the same prefill"}}
    for name in ("eager", "graph"):
        dec = Decoder(Prefill(model), max_len=T + n + 8)
        dec.start(ids)
        if name == "graph":
            dec.capture()  # one real step, then the capture
            steps = n - 1
            run = dec.replay
        else:
            steps = n
            run = dec.step
        torch.cuda.synchronize()
        t = time.perf_counter()
        for _ in range(steps):
            run()
        torch.cuda.synchronize()
        dt = time.perf_counter() - t
        tokens = dec.emitted[:n + 1].tolist()
        same = next((i for i, (x, y) in enumerate(zip(tokens, hf_tokens)) if x != y), len(tokens))
        res[name] = {"tok_s": round(steps / dt, 1), "ms_per_token": round(dt / steps * 1e3, 3),
                     "leading_tokens_equal_hf_loop": f"{same}/{n + 1}"}
        log(f"bench: native decode {name}: {res[name]}")
        del dec
    res["what"] = ("w8a8.pipeline.Decoder after the whole-prompt prefill: per token and layer the int8 GEMVs with "
                   "bf16 activations, k_qkv, the key / value cache write, the decode attention at a device-held "
                   "position, the residual norms made in the prologue of the GEMV that reads them; greedy argmax on "
                   "the device; the graph form replays one captured step per token")
    return res


def e2e_bench(dev, T=ATTN_T, n_decode=32):
    """The reference's run() (gemma_npu.py:278-300) on the GPU: a timed prefill of T tokens, then
    greedy decode through HF's unchanged loop, one model call per token."""
    import torch
    model, nparams = e2b_model(dev)
    ids = torch.randint(0, 262144, (1, T), generator=torch.Generator().manual_seed(1)).to(dev)
    ttfts = []
    with torch.inference_mode():
        for _ in range(4):  # the first call pays one-time set-up
            torch.cuda.synchronize()
            t = time.perf_counter()
            out = model(input_ids=ids, use_cache=True, logits_to_keep=1)
            torch.cuda.synchronize()
            ttfts.append(time.perf_counter() - t)
        past, nxt = out.past_key_values, out.logits[0, -1].argmax().view(1, 1)
        torch.cuda.synchronize()
        t = time.perf_counter()
        for _ in range(n_decode):
            o = model(input_ids=nxt, past_key_values=past, use_cache=True, logits_to_keep=1)
            past, nxt = o.past_key_values, o.logits[0, -1].argmax().view(1, 1)
            torch.cuda.synchronize()
        dt = time.perf_counter() - t
        del past, o
        native = native_decode_bench(model, ids, n_decode)
        pipe = pipeline_prefill_bench(model, ids, out.logits[0, -1].float())
    del model, out
    return {"prefill_ms": round(statistics.median(ttfts[1:]) * 1e3, 1), "prompt_tokens": T,
            "pipeline_prefill": pipe, "native_decode": native,
            "decode_tok_s": round(n_decode / dt, 1), "decode_ms_per_token": round(dt / n_decode * 1e3, 2),
            "decode_tokens": n_decode, "params": nparams,
            "what": "HF Gemma 4 (transformers' modeling code, unchanged) with E2B's shapes, random-init bf16 weights, "
                    "linears through w8a8.hf.to_gpu (W8A8 GEMM prefill, int8 GEMV decode and LM head), attention "
                    "through local_sdpa (prefill and split-key decode kernels); prefill = median of 3 timed calls "
                    "after one warm-up (logits_to_keep=1); decode = greedy, one model call per token",
            "reference": {"ttft_ms": 2911, "decode_tok_s": 27.4, "source": "README.md:40-45 (NPU backend, 3658 "
                                                                          "prompt tokens, real weights)"}}


def decode_attention_bench(dev, launches=50):
    """Decode attention at the end of the 3658-token prompt: one query per head against the cache
    (full layers) or its last 512 keys (sliding layers), HIP-graph replays of back-to-back calls."""
    import torch
    from w8a8 import attention as attn
    res = {}
    for name, (D, W, layers) in ATTN_LAYERS.items():
        _, k, v = attention_inputs(D, ATTN_T, dev, seed=D + 1)
        q = (torch.randn(ATTN_H, D, generator=torch.Generator(device=dev).manual_seed(7), device=dev) * 0.3).to(
            torch.bfloat16)
        out = torch.empty_like(q)
        ws = torch.empty(attn.decode_workspace_bytes(ATTN_H, ATTN_KV, ATTN_T, D, None, W), dtype=torch.uint8,
                         device=dev)
        ms = graph_time_ms(lambda: attn.decode(q, k, v, ATTN_T - 1, W, out=out, workspace=ws), dev,
                           launches=launches)
        keys = ATTN_T if W == 0 else W
        nbytes = 2 * keys * D * 2 * ATTN_KV
        res[name] = {"us": round(ms * 1e3, 2), "kv_bytes": nbytes, "gbs": round(nbytes / (ms * 1e-3) / 1e9, 1),
                     "head_dim": D, "window": W, "layers": layers}
    res["token_total_us"] = round(sum(r["us"] * r["layers"] for r in res.values()), 1)
    res["what"] = ("one decode token's attention per layer kind (split-key kernel + logsumexp merge, two launches), "
                   "HIP-graph replay; token_total = 28 sliding + 7 full layers")
    return res


def cpu_attention_ms(D, W, T=ATTN_T, rows=512, reps=2):
    """The reference's CPU prefill attention (torch's CPU sdpa, bf16, as pipeline.py:140-180 and
    local_attn.py:91-107 call it) for the last `rows` queries of a T-token prompt: a sliding layer
    as 128-query blocks against the W + 128 keys their window reaches (one batched, masked sdpa);
    a full layer as one causal sdpa over the rows' own keys plus one non-causal sdpa over the
    earlier keys, merged by their logsumexp.  Host threads: torch's default."""
    import torch
    import torch.nn.functional as F
    g = torch.Generator().manual_seed(D)
    q = (torch.randn(ATTN_H, rows, D, generator=g) * 0.3).to(torch.bfloat16)
    k = (torch.randn(ATTN_KV, T, D, generator=g) * 0.3).to(torch.bfloat16)
    v = torch.randn(ATTN_KV, T, D, generator=g).to(torch.bfloat16)
    s = T - rows
    flash = torch.ops.aten._scaled_dot_product_flash_attention_for_cpu

    def sliding():
        B = 128
        nb = rows // B
        qb = q.view(ATTN_H, nb, B, D).transpose(0, 1)
        kw = k[:, s - W: T].unfold(1, W + B, B).permute(1, 0, 3, 2)
        vw = v[:, s - W: T].unfold(1, W + B, B).permute(1, 0, 3, 2)
        qp = s + torch.arange(nb)[:, None, None] * B + torch.arange(B)[None, :, None]
        kp = qp[:, :1, :1] - W + torch.arange(W + B)[None, None, :]
        mask = ((kp >= 0) & (kp <= qp) & (qp - kp < W))[:, None]
        return F.scaled_dot_product_attention(qb, kw, vw, attn_mask=mask, scale=1.0, enable_gqa=True)

    def full():
        kb = k[None, :, s:].expand(1, ATTN_H, rows, D).contiguous()
        vb = v[None, :, s:].expand(1, ATTN_H, rows, D).contiguous()
        ob, lb = flash(q[None], kb, vb, 0.0, True, scale=1.0)
        ka = k[None, :, :s].expand(1, ATTN_H, s, D).contiguous()
        va = v[None, :, :s].expand(1, ATTN_H, s, D).contiguous()
        oa, la = flash(q[None], ka, va, 0.0, False, scale=1.0)
        m = torch.maximum(la, lb)
        w1, w2 = torch.exp(la - m)[..., None], torch.exp(lb - m)[..., None]
        return ((oa.float() * w1 + ob.float() * w2) / (w1 + w2)).to(torch.bfloat16)

    fn = sliding if W else full
    fn()
    times = []
    for _ in range(reps):
        t = time.perf_counter()
        fn()
        times.append(time.perf_counter() - t)
    return min(times) * 1e3


def attention_bench(dev, reps, cpu=True):
    """Prefill attention of the 3658-token prompt: each layer kind in one call over the whole prompt,
    and the reference pipeline's largest per-micro-batch calls (pipeline.py:281-295); with cpu, the
    reference's CPU attention for the same last micro-batch beside them."""
    import torch
    from w8a8 import attention as attn
    T = ATTN_T
    res, total_us = {}, 0.0
    for name, (D, W, layers) in ATTN_LAYERS.items():
        q, k, v = attention_inputs(D, T, dev, seed=D)
        out = torch.empty_like(q)
        ms = event_time_ms(lambda: attn.attention(q, k, v, 0, W, out=out), reps, 3)
        flops = 4.0 * D * ATTN_H * attention_pairs(0, T, W)
        tf = flops / (ms * 1e-3) / 1e12
        e = {"us": round(ms * 1e3, 1), "tflops": round(tf, 1), "frac_mfma_bf16": round(tf / PEAK_BF16_TFLOPS, 4),
             "head_dim": D, "window": W, "layers": layers}
        # the reference's per-micro-batch calls at the end of the prompt: a sliding micro-batch of 512
        # rows, a full-attention chunk of 256 rows (ATTN_ROWS) against every earlier key
        r = 512 if W else 256
        qs = T - r
        ms_mb = event_time_ms(lambda: attn.attention(q[:, qs:], k, v, qs, W, out=out[:, qs:]), reps, 3)
        e["last_micro_batch_us"] = round(ms_mb * 1e3, 1)
        e["last_micro_batch"] = f"{r} queries at position {qs}"
        if cpu:
            cms = cpu_attention_ms(D, W, rows=r)
            e["cpu_last_micro_batch_ms"] = round(cms, 2)
            e["cpu_threads"] = torch.get_num_threads()
            e["speedup_vs_cpu_last_micro_batch"] = round(cms / (ms_mb * 1e3) * 1e3, 1)
        res[name] = e
        total_us += layers * ms * 1e3
        del q, k, v, out
    res["prompt_total_us"] = round(total_us, 1)
    res["what"] = (f"E2B prefill attention at T={T}: H={ATTN_H}, KV={ATTN_KV}; flops = 4 * head_dim * H * "
                   f"visible (query, key) pairs; prompt_total = 28 sliding + 7 full layers")
    return res


def profile_kernel(groups, dev, launches):
    """The dominant kernel alone, plus one plain copy of COPY_BYTES (read COPY_BYTES, write
    COPY_BYTES) whose FETCH_SIZE / WRITE_SIZE readings give the counters' byte scale."""
    import torch
    from w8a8 import ops
    gu = next(g for g in groups if g["name"] == "gate_up")
    src = torch.ones(COPY_BYTES // 4, dtype=torch.float32, device=dev)
    dst = torch.empty_like(src)
    torch.cuda.synchronize()
    dst.copy_(src)
    for _ in range(launches):
        ops.gemm_bf16(gu["q"], gu["sx"], gu["pw"], epilogue="gelu", out=gu["out"])
    torch.cuda.synchronize()
    log(f"bench: profiled {launches} gate_up launches and one {COPY_BYTES >> 20} MiB copy")
    return 0


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--no-cpu", action="store_true", help="skip the host CPU baseline")
    ap.add_argument("--no-extra", action="store_true", help="skip the sweep / stress / GEMV sub-results")
    ap.add_argument("--profile-kernel", action="store_true",
                    help="for counter collection: launch only the dominant GEMM (eager, --steps times) and a "
                         "64 MiB device copy that calibrates the byte counters, then exit")
    ap.add_argument("--profile-gemm", metavar="M,K,N,EPI[,TILE]",
                    help="for counter collection: launch one GEMM of that shape (EPI i32 / none / gelu / residual; "
                         "random data, the automatic tile or configuration TILE) --steps times, then exit")
    ap.add_argument("--profile-gemv", action="store_true",
                    help="for kernel traces / counters: run the packed LM-head GEMV at M=1 (--steps times) and a "
                         "64 MiB device copy that calibrates the byte counters, then exit")
    ap.add_argument("--profile-attention", action="store_true",
                    help="for kernel traces: run the whole-prompt sliding and full attention calls at T=3658 "
                         "(--steps times each) and exit")
    ap.add_argument("--profile-e2e", action="store_true",
                    help="for kernel traces: one prefill of the 3658-token prompt and --steps decode tokens of the "
                         "E2B-shaped HF Gemma 4 on the engine, then exit")
    ap.add_argument("--profile-pipeline", action="store_true",
                    help="for kernel traces: --steps whole-prompt prefills of the 3658-token prompt through "
                         "w8a8.pipeline.Prefill on the E2B-shaped HF Gemma 4, then exit")
    ap.add_argument("--profile-decoder", action="store_true",
                    help="run w8a8.pipeline.Decoder on the E2B-shaped model after a 3658-token prompt: one captured "
                         "step, then --steps graph replays (for rocprofv3)")
    ap.add_argument("--profile-decode", action="store_true",
                    help="for kernel traces: decode attention at the end of the 3658-token prompt for each layer "
                         "kind (--steps calls each, eager) and exit")
    ap.add_argument("--profile-sweep", action="store_true",
                    help="for kernel traces: run the 141-GEMM int32 prefill sweep at M=3658 (--steps + 2 times) "
                         "and exit")
    ap.add_argument("--profile-chain", action="store_true",
                    help="for kernel traces: run the device layer chain (--steps times, eager) and exit")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU; --gpus {args.gpus} is not supported (the W8A8 path runs "
              "per GPU with no cross-GPU exchange)", file=sys.stderr)
        return 2

    import torch
    from w8a8 import lib, ops, workloads

    dev = torch.device("cuda", 0)
    torch.cuda.set_device(dev)
    M = 512
    if args.profile_sweep:
        for Ms in (3658,):
            ms = sweep(Ms, dev, reps=args.steps)[0]
        log(f"bench: ran the 141-GEMM int32 prefill sweep at M=3658 {args.steps} + 2 times, {ms:.3f} ms per timed sweep")
        return 0
    if args.profile_gemv:
        K, N = workloads.LM_HEAD
        x = workloads.activations(1, K, seed=5, outliers=False).to(dev)
        g = torch.Generator(device=dev).manual_seed(5)
        pw = ops.pack_gemv_weight(torch.randint(-127, 128, (N, K), generator=g, dtype=torch.int8, device=dev))
        s = (torch.rand(N, generator=g, device=dev) * 0.015 + 0.005).to(torch.bfloat16)
        y = torch.empty((1, N), dtype=torch.bfloat16, device=dev)
        src = torch.ones(COPY_BYTES // 4, dtype=torch.float32, device=dev)
        dst = torch.empty_like(src)
        torch.cuda.synchronize()
        dst.copy_(src)
        for _ in range(args.steps):
            ops.gemv_bf16(x, pw, s, y)
        torch.cuda.synchronize()
        log(f"bench: ran the packed LM-head GEMV (M=1, K={K}, N={N}) {args.steps} times")
        return 0
    if args.profile_e2e:
        model, _ = e2b_model(dev)
        ids = torch.randint(0, 262144, (1, ATTN_T), generator=torch.Generator().manual_seed(1)).to(dev)
        with torch.inference_mode():
            out = model(input_ids=ids, use_cache=True, logits_to_keep=1)
            past, nxt = out.past_key_values, out.logits[0, -1].argmax().view(1, 1)
            for _ in range(args.steps):
                o = model(input_ids=nxt, past_key_values=past, use_cache=True, logits_to_keep=1)
                past, nxt = o.past_key_values, o.logits[0, -1].argmax().view(1, 1)
        torch.cuda.synchronize()
        log(f"bench: ran the E2B-shaped model: prefill of {ATTN_T} tokens, {args.steps} decode tokens")
        return 0
    if args.profile_gemm:
        fields = args.profile_gemm.split(",")
        Mg, Kg, Ng, epi = int(fields[0]), int(fields[1]), int(fields[2]), fields[3]
        tile = int(fields[4]) if len(fields) > 4 else -1
        if epi not in ("i32", "none", "gelu", "residual"):
            raise SystemExit(f"--profile-gemm: epilogue {epi!r} is not i32, none, gelu or residual")
        x = workloads.activations(Mg, Kg, seed=9).to(dev)
        q, sx = ops.quant_rows_packed(x)
        w, sw = workloads.weights(Ng, Kg, seed=10)
        pw = ops.pack_weight(w.to(dev), "nk", Ng // 2 if epi == "gelu" else 0, sw=sw.to(dev))
        del w
        res = workloads.activations(Mg, Ng, seed=11, outliers=False).to(dev) if epi == "residual" else None
        if epi == "i32":
            out = torch.empty((Mg, Ng), dtype=torch.int32, device=dev)
            for _ in range(args.steps):
                ops.gemm_i32(q, pw, out, tile_cfg=tile)
        else:
            out = torch.empty((Mg, Ng // 2 if epi == "gelu" else Ng), dtype=torch.bfloat16, device=dev)
            for _ in range(args.steps):
                ops.gemm_bf16(q, sx, pw, epilogue=epi, residual=res, out=out, tile_cfg=tile)
        torch.cuda.synchronize()
        log(f"bench: ran the {epi} GEMM M={Mg} K={Kg} N={Ng} (tile {tile}) {args.steps} times")
        return 0
    if args.profile_pipeline:
        from w8a8.pipeline import Prefill
        model, _ = e2b_model(dev)
        ids = torch.randint(0, 262144, (1, ATTN_T), generator=torch.Generator().manual_seed(1)).to(dev)
        pre = Prefill(model)
        for _ in range(args.steps):
            pre(ids)
        torch.cuda.synchronize()
        log(f"bench: ran {args.steps} whole-prompt pipeline prefills of {ATTN_T} tokens on the E2B-shaped model")
        return 0
    if args.profile_decoder:
        from w8a8.pipeline import Decoder, Prefill
        model, _ = e2b_model(dev)
        ids = torch.randint(0, 262144, (1, ATTN_T), generator=torch.Generator().manual_seed(1)).to(dev)
        dec = Decoder(Prefill(model), max_len=ATTN_T + args.steps + 8)
        dec.start(ids)
        dec.capture()
        for _ in range(args.steps):
            dec.replay()
        torch.cuda.synchronize()
        log(f"bench: decoded {args.steps + 1} tokens after a {ATTN_T}-token prompt, {args.steps} of them graph-replayed")
        return 0
    if args.profile_decode:
        from w8a8 import attention as attn
        for name, (D, W, _) in ATTN_LAYERS.items():
            _, k, v = attention_inputs(D, ATTN_T, dev, seed=D + 1)
            q = (torch.randn(ATTN_H, D, generator=torch.Generator(device=dev).manual_seed(7), device=dev) * 0.3).to(
                torch.bfloat16)
            out = torch.empty_like(q)
            for _ in range(args.steps):
                attn.decode(q, k, v, ATTN_T - 1, W, out=out)
            torch.cuda.synchronize()
            log(f"bench: ran {name} decode attention (keys {ATTN_T}, head_dim {D}, window {W}) {args.steps} times")
        return 0
    if args.profile_attention:
        from w8a8 import attention as attn
        for name, (D, W, _) in ATTN_LAYERS.items():
            q, k, v = attention_inputs(D, ATTN_T, dev, seed=D)
            out = torch.empty_like(q)
            for _ in range(args.steps):
                attn.attention(q, k, v, 0, W, out=out)
            torch.cuda.synchronize()
            log(f"bench: ran {name} attention (T={ATTN_T}, head_dim {D}, window {W}) {args.steps} times")
            # the reference pipeline's last micro-batch of this layer kind (as attention_bench)
            qs = ATTN_T - (512 if W else 256)
            for _ in range(args.steps):
                attn.attention(q[:, qs:], k, v, qs, W, out=out[:, qs:])
            torch.cuda.synchronize()
            log(f"bench: ran {name} attention for {ATTN_T - qs} queries at position {qs} {args.steps} times")
        return 0
    if args.profile_chain:
        c = build_chain(M, dev)
        for _ in range(args.steps):
            chain_step(c)
        torch.cuda.synchronize()
        log(f"bench: ran the device layer chain {args.steps} times at M={M}")
        return 0
    log(f"bench: building one E2B layer at M={M}")
    groups = build_layer(M, dev)
    if args.profile_kernel:
        return profile_kernel(groups, dev, args.steps)
    step_ops = sum(workloads.gemm_ops(M, g["N"], g["K"]) for g in groups)
    ws = torch.zeros(max(ops.linear_workspace_bytes(M, g["N"], g["K"]) for g in groups), dtype=torch.uint8,
                     device=dev)

    # eager reference outputs, then the captured step must reproduce them bit for bit
    layer_step(groups, ws)
    eager_out = [g["out"].clone() for g in groups]
    graph = capture(lambda: layer_step(groups, ws), dev)
    for g in groups:
        g["out"].zero_()
    graph.replay()
    torch.cuda.synchronize()
    for g, ref in zip(groups, eager_out):
        if not torch.equal(g["out"], ref):
            raise RuntimeError(f"captured layer step differs from eager for {g['name']}")

    # ---- timed region: K steps bracketed by synchronisation ------------------------------
    # A step is launched the way the reference's pipeline calls the linears (one mm_i8 per
    # linear, eagerly): 4 x (quant prologue + GEMM) on torch's current stream.  The captured
    # replay of the same 8 launches, checked above, is reported beside it.
    for _ in range(args.warmup):
        layer_step(groups, ws)
    torch.cuda.synchronize()
    s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    s.record()
    for _ in range(args.steps):
        layer_step(groups, ws)
    e.record()
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    ms_step = s.elapsed_time(e) / args.steps
    value = step_ops / (ms_step * 1e-3) / 1e12
    log(f"bench: layer step {ms_step * 1e3:.1f} us = {value:.1f} TOP/s (wall {wall:.3f} s)")
    for g, ref in zip(groups, eager_out):
        if not torch.equal(g["out"], ref):
            raise RuntimeError(f"timed layer step output differs from the first run for {g['name']}")
    graph_ms = event_time_ms(graph.replay, args.steps, args.warmup)
    log(f"bench: graph-replayed layer step {graph_ms * 1e3:.1f} us")
    # the same step 50 times in one graph: a replay's fixed launch cost spread over 50 steps
    graph50_ms = graph_time_ms(lambda: layer_step(groups, ws), dev, launches=50, reps=4)
    log(f"bench: layer step from a 50-step graph {graph50_ms * 1e3:.1f} us")

    # ---- dominant kernel: the gate_up GEMM with fused GELU epilogue ----------------------
    gu = next(g for g in groups if g["name"] == "gate_up")
    per_ms = {}
    for g in groups:
        per_ms[g["name"]] = graph_time_ms(
            lambda g=g: ops.gemm_bf16(g["q"], g["sx"], g["pw"], epilogue=g["epi"], residual=g["res"],
                                      out=g["out"]), dev)
    gu_ops = workloads.gemm_ops(M, gu["N"], gu["K"])
    gu_cfg = lib().w8a8_gemm_pick_tile_config(M, gu["N"], gu["K"], 1)
    gu_ms = per_ms["gate_up"]
    achieved = gu_ops / (gu_ms * 1e-3) / 1e12
    traffic = read_traffic()
    clock = clock_during(lambda: ops.gemm_bf16(gu["q"], gu["sx"], gu["pw"], epilogue="gelu", out=gu["out"]), dev)
    peak_at_clock = 256 * 8192 * clock / 1e3  # TOP/s: 256 CUs x 8192 int8 op/clk/CU at the measured clock
    # the step's own roofline: per linear max(t_mfma, t_hbm) over its algorithmic ops and compulsory
    # bytes (bf16 x in, int8 W, fp32 scales, bf16 out, the residual in), summed over the four
    step_floor_us = 0.0
    for g in groups:
        n_out = g["N"] // 2 if g["epi"] == "gelu" else g["N"]
        nbytes = 2 * M * g["K"] + g["K"] * g["N"] + 4 * g["N"] + 2 * M * n_out + (2 * M * g["N"] if g["res"] is not None
                                                                                   else 0)
        step_floor_us += max(workloads.gemm_ops(M, g["N"], g["K"]) / (PEAK_INT8_TOPS * 1e12),
                             nbytes / (PEAK_HBM_GBS * 1e9)) * 1e6
    roofline = {"bound": "mfma", "achieved": round(achieved, 1), "peak": PEAK_INT8_TOPS, "unit": "TFLOP/s",
                "frac": round(achieved / PEAK_INT8_TOPS, 4), "traffic": traffic,
                "traffic_source": f"{os.path.relpath(PMC_SUMMARY, ROOT)}: rocprofv3 FETCH_SIZE + WRITE_SIZE of this "
                                  "kernel, each calibrated on a 64 MiB copy (read from the committed summary, not "
                                  "measured in this run)" if traffic is not None else None,
                "kernel": f"{tile_name(gu_cfg)} gate_up M=512 K=1536 N=12288 with the GELU epilogue, packed A",
                "avg_launch_us": round(gu_ms * 1e3, 2), "clock_ghz": round(clock, 3),
                "frac_at_clock": round(achieved / peak_at_clock, 4),
                "step_roofline_us": round(step_floor_us, 2),
                "step_frac": round(step_floor_us / (ms_step * 1e3), 4)}
    log(f"bench: gate_up runs at {clock:.3f} GHz: {achieved:.0f} TOP/s = {achieved / peak_at_clock:.3f} of the "
        f"MFMA peak at that clock ({peak_at_clock:.0f} TOP/s)")
    log(f"bench: per-GEMM us: " + ", ".join(f"{k} {v * 1e3:.1f}" for k, v in per_ms.items()))

    # ---- host CPU baseline: torch._int_mm on the same four GEMMs -------------------------
    cpu = None
    if not args.no_cpu:
        torch.set_num_threads(os.cpu_count() or 1)
        cm, rounds = cpu_int_mm_ms([(g["K"], g["N"]) for g in groups], M, budget_s=10.0)
        cpu_ms = sum(cm.values())
        cpu = {"value": round(step_ops / (cpu_ms * 1e-3) / 1e12, 3), "unit": "TOP/s",
               "cores": torch.get_num_threads(), "kind": "reference", **cpu_identity(),
               "sample": f"torch._int_mm (the reference's --backend cpu-int8 GEMM, pipeline.py:237) on the same "
                         f"layer's 4 GEMMs at M={M} (int8 in, int32 out): 3 warm-up calls each, then {rounds} "
                         f"rounds over the 4 (~10 s), median per GEMM summed: {cpu_ms:.1f} ms per layer"}
        log(f"bench: cpu _int_mm layer {cpu_ms:.1f} ms")

    extra = {"graph_layer_step_us": round(graph_ms * 1e3, 1),
             "graph_layer_step_us_50_per_replay": round(graph50_ms * 1e3, 1),
             "gemm_us_m512": {k: round(v * 1e3, 2) for k, v in per_ms.items()},
             "single_gemm_m512_int32": single_gemm(dev)}
    log(f"bench: single micro-batch GEMM: {extra['single_gemm_m512_int32']}")
    if not args.no_extra:
        extra["mm_i8_host_slots_m512"] = host_slot_gemm(dev)
        log(f"bench: mm_i8 on host slots: {extra['mm_i8_host_slots_m512']}")
        for Ms in (3658, 4096):
            ms, tops_ops, wbytes, shp, run = sweep(Ms, dev, reps=5)
            tops = tops_ops / (ms * 1e-3) / 1e12
            clk = clock_during(run, dev, launches=2, window_ms=4.0)
            entry = {"ms": round(ms, 3), "gemms": len(shp), "tops": round(tops, 1),
                     "frac_mfma": round(tops / PEAK_INT8_TOPS, 4), "clock_ghz": round(clk, 3),
                     "frac_at_clock": round(tops / (256 * 8192 * clk / 1e3), 4),
                     "weights": f"cold: {wbytes / 1e9:.2f} GB of distinct per-layer weights, int32 out"}
            if not args.no_cpu and Ms == 3658:
                uniq = sorted(set(shp))
                cm, _ = cpu_int_mm_ms(uniq, Ms, warm=3, reps=5)
                cpu_total = sum(cm[s] for s in shp)
                entry["cpu_int_mm_ms"] = round(cpu_total, 1)
                entry["cpu"] = dict(cpu_identity(), threads=torch.get_num_threads(),
                                    sample="torch._int_mm per distinct shape, 3 warm-up calls then the median of 5, "
                                           "summed over the 141 GEMMs")
                entry["speedup_vs_cpu"] = round(cpu_total / ms, 1)
            extra[f"prefill_sweep_m{Ms}"] = entry
            log(f"bench: sweep M={Ms}: {entry}")
            torch.cuda.empty_cache()
            ms, tops_ops, wbytes, shp, run = sweep(Ms, dev, reps=5, epilogues=True)
            tops = tops_ops / (ms * 1e-3) / 1e12
            clk = clock_during(run, dev, launches=2, window_ms=4.0)
            extra[f"prefill_sweep_m{Ms}_epilogues"] = {
                "ms": round(ms, 3), "gemms": len(shp), "tops": round(tops, 1),
                "frac_mfma": round(tops / PEAK_INT8_TOPS, 4), "clock_ghz": round(clk, 3),
                "frac_at_clock": round(tops / (256 * 8192 * clk / 1e3), 4),
                "weights": f"cold: {wbytes / 1e9:.2f} GB of distinct per-layer weights",
                "what": "the same 141 GEMMs with one E2B-class layer's epilogues: bf16 out (qkv, o, PLE projection "
                        "dequantised), gate/up with the GELU product, down with the residual add"}
            log(f"bench: sweep M={Ms} with epilogues: {extra[f'prefill_sweep_m{Ms}_epilogues']}")
            torch.cuda.empty_cache()
        # M=16384 stress: gate_up with fused GELU, down with residual
        for name in ("gate_up", "down"):
            K, N, epi = workloads.LAYER_GROUPS[name]
            Ms = 16384
            x = workloads.activations(Ms, K, seed=9, row_spread=True).to(dev)
            q, sx = ops.quant_rows_packed(x)
            gw = torch.Generator(device=dev).manual_seed(10)
            w = torch.randint(-127, 128, (N, K), generator=gw, dtype=torch.int8, device=dev)
            sw = torch.rand(N, generator=gw, device=dev) * 0.015 + 0.005
            pw = ops.pack_weight(w, "nk", N // 2 if epi == "gelu" else 0, sw=sw)
            res = torch.randn((Ms, N), device=dev).to(torch.bfloat16) if epi == "residual" else None
            out = torch.empty((Ms, N // 2 if epi == "gelu" else N), dtype=torch.bfloat16, device=dev)
            ms = event_time_ms(lambda: ops.gemm_bf16(q, sx, pw, epilogue=epi, residual=res, out=out), 20, 3)
            t = workloads.gemm_ops(Ms, N, K) / (ms * 1e-3) / 1e12
            extra[f"stress_m16384_{name}"] = {"us": round(ms * 1e3, 1), "tops": round(t, 1),
                                              "frac_mfma": round(t / PEAK_INT8_TOPS, 4)}
            log(f"bench: stress {name}: {extra[f'stress_m16384_{name}']}")
            del x, q, w, pw, res, out
        extra["vs_hipblaslt_int32"] = vendor_compare(dev)
        ms, eager, c = time_chain(M, dev, reps=100)
        extra[f"device_layer_chain_m{M}"] = {
            "us": round(ms * 1e3, 1), "eager_us": round(eager * 1e3, 1), "launches": c["launches"],
            "bf16_handover_us": c["bf16_handover_us"],
            "gemm_tops": round(c["ops"] / (ms * 1e-3) / 1e12, 1),
            "what": "k_in, qkv GEMM, k_qkv, k_attn_out, o GEMM, k_post_attn, gate_up GEMM+GELU, quant, down GEMM, "
                    "k_post_ff, PLE gate GEMM, k_ple_gate, PLE proj GEMM, k_ple_out (no attention), one HIP graph; "
                    "the GEMMs hand their int32 result to the fused kernels (bf16_handover_us: their dequantised "
                    "bf16 result instead, the same bits)"}
        log(f"bench: device layer chain M={M}: {extra[f'device_layer_chain_m{M}']}")
        del c
        for Mg in (1, 4, 16):
            K, N = workloads.LM_HEAD
            ms_rm, ms, nbytes = gemv_bench(Mg, K, N, dev, reps=50)
            gbs = nbytes / (ms * 1e-3) / 1e9
            entry = {"us": round(ms * 1e3, 1), "gbs": round(gbs, 1), "frac_hbm": round(gbs / PEAK_HBM_GBS, 4),
                     "weight": "GEMV fragment layout (w8a8_pack_gemv_weight); cold: 403 MB, more than the 256 MB MALL",
                     "row_major_us": round(ms_rm * 1e3, 1),
                     "row_major_gbs": round(nbytes / (ms_rm * 1e-3) / 1e9, 1)}
            if not args.no_cpu:
                cms = cpu_gemv_ms(Mg, K, N)
                entry.update(cpu_us=round(cms * 1e3, 1), cpu_gbs=round(nbytes / (cms * 1e-3) / 1e9, 1),
                             speedup_vs_cpu=round(cms / ms, 1))
            extra[f"gemv_lm_head_m{Mg}"] = entry
            log(f"bench: gemv lm head M={Mg}: {entry}")
        torch.cuda.empty_cache()
        extra["gemv_decode_layers"] = gemv_layers(dev, reps=10, cpu=not args.no_cpu)
        torch.cuda.empty_cache()
        extra["attention_prefill_t3658"] = attention_bench(dev, reps=20, cpu=not args.no_cpu)
        log(f"bench: attention: {extra['attention_prefill_t3658']}")
        torch.cuda.empty_cache()
        extra["decode_attention_t3658"] = decode_attention_bench(dev)
        log(f"bench: decode attention: {extra['decode_attention_t3658']}")
        extra["hf_gemma4_e2b_shape"] = e2e_bench(dev)
        log(f"bench: HF Gemma 4 end to end: {extra['hf_gemma4_e2b_shape']}")
        torch.cuda.empty_cache()

    line = {
        "metric": "W8A8 GEMM int8 TOPS (% of MFMA peak) at M=512/3658; GEMV HBM GB/s",
        "value": round(value, 2), "unit": "TOP/s", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
        "ms_per_step": round(ms_step, 5), "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "int8", "data": "synthetic (seeded N(0,1) bf16 activations with 0.1% x20 outliers, "
                                 "int8 U[-127,127] weights)",
        "config": {"workload": "one E2B-class decoder layer's prefill linears, M=512 micro-batch, bf16 in -> bf16 "
                               "out with fused per-token quant and dequant/GELU/residual epilogues",
                   "M": M, "groups": {g["name"]: [g["K"], g["N"], g["epi"]] for g in groups},
                   "weights": "hot: the step's 31.5 MB of packed weights are reused every step and stay in "
                              "the 256 MB MALL (the sweep's 1.25 GB and the LM head's 403 MB are cold)"},
        "roofline": roofline, "cpu_baseline": cpu, "extra": extra,
    }
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
