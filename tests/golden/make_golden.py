"""Writes tests/golden/w8a8_golden.npz: small input/output vectors from torch's CPU ops.

The reference ships no golden vectors (its .gitignore drops *.npz), and its arithmetic on
this path is torch's: `torch._int_mm` (pipeline.py:237), `torch._weight_int8pack_mm`
(gemma_npu.py:156), and eager torch element-wise ops in `_quant` / `_deq` / `k_gelu` /
`_rms` (pipeline.py:43-57, 102-114).  This script runs those torch ops (not reference code)
on seeded and hand-picked inputs and stores inputs and outputs, so the C oracle is checked
against the library the reference actually executes.  bf16 arrays are stored as uint16 bit
patterns.

    python tests/golden/make_golden.py
"""
import os

import numpy as np
import torch
import torch.nn.functional as F

OUT = os.path.join(os.path.dirname(os.path.abspath(__file__)), "w8a8_golden.npz")


def bits(t):
    return t.contiguous().view(torch.int16).numpy().view(np.uint16)


def main():
    g = torch.Generator().manual_seed(1234)
    d = {}

    # -- int_mm: torch._int_mm over the full int8 range, ragged shapes --------------------
    for name, (M, K, N) in {"mm_a": (37, 128, 72), "mm_b": (5, 64, 16), "mm_c": (64, 192, 48)}.items():
        a = torch.randint(-128, 128, (M, K), generator=g, dtype=torch.int8)
        b = torch.randint(-128, 128, (K, N), generator=g, dtype=torch.int8)
        d[f"{name}_a"], d[f"{name}_b"] = a.numpy(), b.numpy()
        d[f"{name}_c"] = torch._int_mm(a, b).numpy()

    # -- quant rows (pipeline.py:49-52), torch eager ---------------------------------------
    x = torch.randn(12, 96, generator=g) * 3
    x[0] = 0.0                                    # zero row -> scale 1e-8/127
    x[1, :8] = torch.tensor([127.0, 63.5, 0.5, -127.0, 1.5, 2.5, -2.5, -0.5])  # exact ties
    x[1, 8:] = 0.25
    x[2] = torch.linspace(-1, 1, 96) * 1e-3       # small magnitudes
    x[3] = torch.randn(96, generator=g) * 1e4     # large magnitudes
    x[4, 5] = 200.0                               # one outlier dominates the row
    xb = x.to(torch.bfloat16)
    xf = xb.float()
    s = xf.abs().amax(dim=-1).clamp(min=1e-8) / 127
    q = torch.round(xf / s[:, None]).clamp(-127, 127).to(torch.int8)
    d["quant_x"], d["quant_q"], d["quant_s"] = bits(xb), q.numpy(), s.numpy()
    # fp32 rows, as the per-channel weight quant of gemma_npu.py:68-69 sees them
    wf = torch.randn(10, 80, generator=g) * 0.05
    wf[0] = 0.0
    sw = wf.abs().amax(dim=1).clamp(min=1e-8) / 127
    qw = torch.round(wf / sw[:, None]).clamp(-127, 127).to(torch.int8)
    d["wquant_x"], d["wquant_q"], d["wquant_s"] = wf.numpy(), qw.numpy(), sw.numpy()

    # -- dequant (pipeline.py:55-57) --------------------------------------------------------
    acc = torch.randint(-(2 ** 28), 2 ** 28, (9, 40), generator=g, dtype=torch.int32)
    acc[0, :4] = torch.tensor([2 ** 24 + 1, -(2 ** 24 + 3), 0, 2 ** 27 + 5], dtype=torch.int32)
    sx = torch.rand(9, generator=g) * 0.1 + 1e-3
    swd = torch.rand(40, generator=g) * 0.015 + 0.005
    y = (acc.float() * sx[:, None] * swd[None, :]).to(torch.bfloat16)
    d["deq_acc"], d["deq_sx"], d["deq_sw"], d["deq_y"] = acc.numpy(), sx.numpy(), swd.numpy(), bits(y)

    # -- gelu(gate) * up (pipeline.py:106), eager bf16 ----------------------------------------
    yy = (torch.randn(7, 2 * 48, generator=g) * 3).to(torch.bfloat16)
    I = 48
    a = (F.gelu(yy[:, :I], approximate="tanh") * yy[:, I:]).to(torch.bfloat16)
    d["gelu_y"], d["gelu_out"] = bits(yy), bits(a)

    # -- res + rms(y, w) (pipeline.py:43-46, 113) ------------------------------------------
    eps = 1e-6
    yr = (torch.randn(6, 64, generator=g) * 2).to(torch.bfloat16)
    res = torch.randn(6, 64, generator=g).to(torch.bfloat16)
    wr = (torch.rand(64, generator=g) + 0.5).to(torch.bfloat16)
    v = yr.float()
    rn = v * torch.pow(v.pow(2).mean(-1, keepdim=True) + eps, -0.5)
    h = res + (rn * wr.float()).to(torch.bfloat16)
    d["rms_y"], d["rms_res"], d["rms_w"], d["rms_h"] = bits(yr), bits(res), bits(wr), bits(h)
    d["rms_eps"] = np.float32(eps)

    # -- weight-only int8 GEMV (gemma_npu.py:155-156) -----------------------------------------
    for name, (M, K, N) in {"gemv_a": (1, 256, 48), "gemv_b": (4, 128, 40), "gemv_c": (16, 64, 32)}.items():
        xg = torch.randn(M, K, generator=g).to(torch.bfloat16)
        wg = torch.randint(-127, 128, (N, K), generator=g, dtype=torch.int8)
        sg = (torch.rand(N, generator=g) * 0.015 + 0.005)
        yb = torch._weight_int8pack_mm(xg, wg, sg.to(torch.bfloat16))
        yf = torch._weight_int8pack_mm(xg.float(), wg, sg).to(torch.bfloat16)
        d[f"{name}_x"], d[f"{name}_w"] = bits(xg), wg.numpy()
        d[f"{name}_sb"], d[f"{name}_sf"] = bits(sg.to(torch.bfloat16)), sg.numpy()
        d[f"{name}_yb"], d[f"{name}_yf"] = bits(yb), bits(yf)

    np.savez_compressed(OUT, **d)
    print(f"wrote {OUT}: {len(d)} arrays, {os.path.getsize(OUT)} bytes")


if __name__ == "__main__":
    main()
