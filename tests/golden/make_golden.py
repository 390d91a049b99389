"""Writes tests/golden/w8a8_golden.npz: small input/output vectors from torch's CPU ops.

The reference ships no golden vectors (its .gitignore drops *.npz), and its arithmetic on
this path is torch's: `torch._int_mm` (pipeline.py:237), `torch._weight_int8pack_mm`
(gemma_npu.py:156), and eager torch element-wise ops in `_quant` / `_deq` / `_rope` / `_rms`
and the fused k_* functions (pipeline.py:43-127).  This script runs those torch ops (not reference code)
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

    # -- the fused kernels between the GEMMs (pipeline.py:43-127), eager torch -------------------
    # Written with torch tensor ops in the expressions of pipeline.py; torch's own kernels (its
    # vectorised reductions, bf16 tensor arithmetic and type promotion) compute the values.
    def t_rms(x, w, e):
        x = x.float()
        y = x * torch.pow(x.pow(2).mean(-1, keepdim=True) + e, -0.5)
        return y * w.float() if w is not None else y

    def t_quant(x):
        x = x.float()
        s = x.abs().amax(dim=-1).clamp(min=1e-8) / 127
        return torch.round(x / s[:, None]).clamp(-127, 127).to(torch.int8), s

    def t_deq(acc, sx, sw):
        return (acc.float() * sx[:, None] * sw[None, :]).to(torch.bfloat16)

    def t_rope(x, c, s_):
        h = x.shape[-1] // 2
        rot = torch.cat((-x[..., h:], x[..., :h]), dim=-1)
        return x * c + rot * s_

    def acc_scales(T, N):
        acc = torch.randint(-(2 ** 20), 2 ** 20, (T, N), generator=g, dtype=torch.int32)
        sx = torch.rand(T, generator=g) * 2e-3 + 5e-4
        sw = torch.rand(N, generator=g) * 0.015 + 0.005
        return acc, sx, sw

    # rope on its own, at real angles: inv_freq = 10000^(-2i/D), positions 0..R-1
    R, D = 9, 32
    xr = (torch.randn(R, D, generator=g) * 2).to(torch.bfloat16)
    ang = torch.arange(R).float()[:, None] * (10000.0 ** (-torch.arange(0, D, 2).float() / D))[None, :]
    ang = torch.cat([ang, ang], dim=-1)
    cr, sr = ang.cos().to(torch.bfloat16), ang.sin().to(torch.bfloat16)
    d["rope_x"], d["rope_cos"], d["rope_sin"] = bits(xr), bits(cr), bits(sr)
    d["rope_out"] = bits(t_rope(xr, cr, sr))
    # rms alone, to bf16, with and without a weight
    xn = (torch.randn(6, 48, generator=g) * 4).to(torch.bfloat16)
    wn = (torch.rand(48, generator=g) + 0.5).to(torch.bfloat16)
    d["rmsb_x"], d["rmsb_w"] = bits(xn), bits(wn)
    d["rmsb_out"], d["rmsb_out_now"] = bits(t_rms(xn, wn, eps).to(torch.bfloat16)), bits(t_rms(xn, None, eps).to(torch.bfloat16))

    T, N = 7, 64
    # k_in
    hin = (torch.randn(T, N, generator=g) * 3).to(torch.bfloat16)
    win = (torch.rand(N, generator=g) + 0.5).to(torch.bfloat16)
    q, s = t_quant(t_rms(hin, win, eps).to(torch.bfloat16))
    d["kin_h"], d["kin_w"], d["kin_q"], d["kin_s"] = bits(hin), bits(win), q.numpy(), s.numpy()
    # k_qkv, H=2 query heads, KV=1, D=16, non-shared and shared
    H, KV, Dh = 2, 1, 16
    acc, sx, sw = acc_scales(T, (H + 2 * KV) * Dh)
    ang = torch.arange(T).float()[:, None] * (10000.0 ** (-torch.arange(0, Dh, 2).float() / Dh))[None, :]
    ang = torch.cat([ang, ang], dim=-1)
    cq, sq_ = ang.cos().to(torch.bfloat16), ang.sin().to(torch.bfloat16)
    qw = (torch.rand(Dh, generator=g) + 0.5).to(torch.bfloat16)
    kw = (torch.rand(Dh, generator=g) + 0.5).to(torch.bfloat16)
    y = t_deq(acc, sx, sw)
    qh = y[:, :H * Dh].reshape(T, H, Dh)
    qh = t_rope(t_rms(qh, qw, eps).to(torch.bfloat16), cq[:, None], sq_[:, None]).transpose(0, 1)
    kh = y[:, H * Dh:(H + KV) * Dh].reshape(T, KV, Dh)
    vh = y[:, (H + KV) * Dh:].reshape(T, KV, Dh)
    kh = t_rope(t_rms(kh, kw, eps).to(torch.bfloat16), cq[:, None], sq_[:, None]).transpose(0, 1)
    vh = t_rms(vh, None, eps).to(torch.bfloat16).transpose(0, 1)
    d["kqkv_acc"], d["kqkv_sx"], d["kqkv_sw"] = acc.numpy(), sx.numpy(), sw.numpy()
    d["kqkv_cos"], d["kqkv_sin"], d["kqkv_qw"], d["kqkv_kw"] = bits(cq), bits(sq_), bits(qw), bits(kw)
    d["kqkv_q"], d["kqkv_k"], d["kqkv_v"] = bits(qh), bits(kh), bits(vh)
    # k_attn_out: o [H, T, D]
    o = (torch.randn(H, T, Dh, generator=g) * 2).to(torch.bfloat16)
    q, s = t_quant(o.transpose(0, 1).reshape(T, H * Dh))
    d["kao_o"], d["kao_q"], d["kao_s"] = bits(o), q.numpy(), s.numpy()
    # k_post_attn and k_post_ff
    acc, sx, sw = acc_scales(T, N)
    res = (torch.randn(T, N, generator=g) * 2).to(torch.bfloat16)
    w1 = (torch.rand(N, generator=g) + 0.5).to(torch.bfloat16)
    w2 = (torch.rand(N, generator=g) + 0.5).to(torch.bfloat16)
    hh = res + t_rms(t_deq(acc, sx, sw), w1, eps).to(torch.bfloat16)
    q, s = t_quant(t_rms(hh, w2, eps).to(torch.bfloat16))
    q2, s2 = t_quant(hh)
    d["kpa_acc"], d["kpa_sx"], d["kpa_sw"], d["kpa_res"] = acc.numpy(), sx.numpy(), sw.numpy(), bits(res)
    d["kpa_w1"], d["kpa_w2"], d["kpa_h"], d["kpa_q"], d["kpa_s"] = bits(w1), bits(w2), bits(hh), q.numpy(), s.numpy()
    d["kpf_q"], d["kpf_s"] = q2.numpy(), s2.numpy()
    # k_gelu on an int32 [gate; up] result
    I = 32
    acc, sx, sw = acc_scales(T, 2 * I)
    y = t_deq(acc, sx, sw)
    q, s = t_quant((F.gelu(y[:, :I], approximate="tanh") * y[:, I:]).to(torch.bfloat16))
    d["kg_acc"], d["kg_sx"], d["kg_sw"], d["kg_q"], d["kg_s"] = acc.numpy(), sx.numpy(), sw.numpy(), q.numpy(), s.numpy()
    # k_ple_gate
    Np = 32
    acc, sx, sw = acc_scales(T, Np)
    ple = (torch.randn(T, Np, generator=g) * 2).to(torch.bfloat16)
    q, s = t_quant((F.gelu(t_deq(acc, sx, sw), approximate="tanh") * ple).to(torch.bfloat16))
    d["kpg_acc"], d["kpg_sx"], d["kpg_sw"], d["kpg_ple"] = acc.numpy(), sx.numpy(), sw.numpy(), bits(ple)
    d["kpg_q"], d["kpg_s"] = q.numpy(), s.numpy()
    # k_ple_out
    acc, sx, sw = acc_scales(T, N)
    hp = (torch.randn(T, N, generator=g) * 2).to(torch.bfloat16)
    wp = (torch.rand(N, generator=g) + 0.5).to(torch.bfloat16)
    scalar = torch.tensor([0.7], dtype=torch.bfloat16)
    out = ((hp + t_rms(t_deq(acc, sx, sw), wp, eps).to(torch.bfloat16)) * scalar).to(torch.bfloat16)
    d["kpo_acc"], d["kpo_sx"], d["kpo_sw"], d["kpo_h"], d["kpo_w"] = acc.numpy(), sx.numpy(), sw.numpy(), bits(hp), bits(wp)
    d["kpo_scalar"], d["kpo_out"] = bits(scalar), bits(out)

    np.savez_compressed(OUT, **d)
    print(f"wrote {OUT}: {len(d)} arrays, {os.path.getsize(OUT)} bytes")


if __name__ == "__main__":
    main()
