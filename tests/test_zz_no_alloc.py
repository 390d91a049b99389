"""w8a8_linear_bf16_noalloc, the whole-linear entry point that allocates nothing (it has no
counterpart in the reference; it serves callers that cannot allocate device memory).  Through
the C ABI it must give the bits w8a8_linear_bf16 (the same linear with a caller workspace)
gives, for every epilogue, on two calls in a row whose second has fewer rows (the shared
scratch keeps the first call's contents), and refuse sizes beyond its scratch."""
import pytest
import torch

from w8a8 import lib, ops, workloads
from w8a8._lib import W8A8_ENOTSUP, W8A8Error, call

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _run(entry, x, pw, epilogue, res=None, rms_w=None, eps=1e-6):
    M, K = x.shape
    N, I = pw.N, pw.interleave
    out = torch.full((M, I if epilogue == 1 else N), float("nan"), dtype=torch.bfloat16, device=DEV)
    stream = torch.cuda.current_stream().cuda_stream
    args = [x.data_ptr(), x.stride(0), pw.data.data_ptr(), pw.sw.data_ptr(), M, N, K, epilogue, I,
            None if res is None else res.data_ptr(), 0 if res is None else res.stride(0),
            None if rms_w is None else rms_w.data_ptr(), eps, out.data_ptr(), out.stride(0)]
    if entry == "w8a8_linear_bf16":
        need = lib().w8a8_linear_workspace_bytes(M, N, K)
        ws = torch.zeros(need, dtype=torch.uint8, device=DEV)
        assert ws.data_ptr() % 256 == 0
        call(entry, *args, ws.data_ptr(), need, stream)
    else:
        call(entry, *args, stream)
    return out


CASES = {  # epilogue code: (K, N, interleave)
    0: (2048, 1536, 0),      # o projection, plain dequant
    1: (1536, 12288, 6144),  # gate_up with the GELU epilogue
    2: (6144, 1536, 0),      # down with the residual add
    3: (6144, 1536, 0),      # down with residual + RMSNorm (pipeline.py:113)
}


@pytest.mark.parametrize("epilogue", sorted(CASES))
def test_noalloc_linear_matches_the_workspace_linear(epilogue):
    K, N, I = CASES[epilogue]
    w, sw = workloads.weights(N, K, seed=40 + epilogue)
    pw = ops.pack_weight(w.to(DEV), "nk", interleave=I, sw=sw.to(DEV))
    rms_w = (torch.rand(N, generator=torch.Generator().manual_seed(3)) + 0.5).to(torch.bfloat16).to(DEV)
    for call_no, M in enumerate((512, 77)):  # the second call has fewer rows
        x = workloads.activations(M, K, seed=50 + 10 * epilogue + call_no).to(DEV)
        res = workloads.activations(M, N, seed=60 + call_no, outliers=False).to(DEV) if epilogue >= 2 else None
        kw = dict(res=res, rms_w=rms_w if epilogue == 3 else None)
        got = _run("w8a8_linear_bf16_noalloc", x, pw, epilogue, **kw)
        ref = _run("w8a8_linear_bf16", x, pw, epilogue, **kw)
        torch.cuda.synchronize()
        assert not torch.isnan(ref).any()
        assert torch.equal(got.view(torch.int16), ref.view(torch.int16)), f"epilogue {epilogue}, call {call_no}, M={M}"


def test_noalloc_linear_refuses_more_than_its_scratch():
    K, N = 6144, 1536
    w, sw = workloads.weights(N, K, seed=7)
    pw = ops.pack_weight(w.to(DEV), "nk", sw=sw.to(DEV))
    x = torch.zeros((16384, K), dtype=torch.bfloat16, device=DEV)  # 96 MiB of packed rows
    with pytest.raises(W8A8Error) as e:
        _run("w8a8_linear_bf16_noalloc", x, pw, 0)
    assert e.value.status == W8A8_ENOTSUP and "scratch" in str(e.value)
    # the largest size that fits still runs, right after the refusal
    x = workloads.activations(8192, K, seed=8).to(DEV)
    got = _run("w8a8_linear_bf16_noalloc", x, pw, 0)
    ref = _run("w8a8_linear_bf16", x, pw, 0)
    assert torch.equal(got.view(torch.int16), ref.view(torch.int16))
