"""The bf16 linears captured in a HIP graph, the way a serving loop replays a layer: every
replay must reproduce the eager outputs bit for bit, with eager work and synchronisation
between replays (the captured launches hold no memset nodes and no host-side state)."""
import pytest
import torch

from w8a8 import ops, workloads

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _layer(M):
    groups = []
    for gi, (name, (K, N, epi)) in enumerate(workloads.LAYER_GROUPS.items()):
        x = workloads.activations(M, K, seed=100 + gi).to(DEV)
        w, sw = workloads.weights(N, K, seed=200 + gi)
        inter = N // 2 if epi == "gelu" else 0
        pw = ops.pack_weight(w.to(DEV), "nk", inter, sw=sw.to(DEV))
        res = workloads.activations(M, N, seed=300 + gi, outliers=False).to(DEV) if epi == "residual" else None
        out = torch.empty((M, inter or N), dtype=torch.bfloat16, device=DEV)
        groups.append((x, pw, epi, res, out))
    return groups


def _step(groups, ws):
    for x, pw, epi, res, out in groups:
        ops.linear_bf16(x, pw, epilogue=epi, residual=res, out=out, ws_arg=ws)


@pytest.mark.parametrize("M", [512, 37])
def test_captured_layer_replays_match_eager(M):
    groups = _layer(M)
    ws = torch.zeros(max(ops.linear_workspace_bytes(M, pw.N, pw.K) for _, pw, _, _, _ in groups),
                     dtype=torch.uint8, device=DEV)
    _step(groups, ws)
    torch.cuda.synchronize()
    ref = [g[4].clone() for g in groups]

    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        _step(groups, ws)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        _step(groups, ws)
    torch.cuda.synchronize()

    for rep in range(4):
        for g in groups:
            g[4].fill_(float("nan"))
        # unrelated eager work on the same buffers' stream between replays
        ops.quant_rows(groups[0][0])
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        for i, g in enumerate(groups):
            assert torch.equal(g[4], ref[i]), f"replay {rep}: linear {i} differs from eager"
