"""Closed-form known-answer cases shared by the CPU oracle tests and the GPU kernel tests.

Each case restates one of the reference's driver-level known-answer tests
(tests/probe_gpu_no_torch.py) as inputs plus expectations computed by hand with explicit bf16
rounding (oracle.bf16), independent of torch. ``ops`` is any object with the reference's ops
interface (the CPU oracle's TorchOps, or HipOps on the GPU); ``dev`` is where inputs go.
"""
import math

import torch

from oracle.bf16 import r, rms_expected, rope_expected, silu_mul_expected

BF = torch.bfloat16


def _t(vals, dev, shape=None):
    t = torch.tensor(vals, dtype=torch.float32).to(BF)
    return (t.reshape(shape) if shape else t).to(dev)


def case_silu(ops, dev):
    """probe_gpu_no_torch.py:73-98: SiLU x up at both rounding points."""
    gates = [[-4.0, -1.0, 0.0, 1.0, 4.0, 0.5, -0.5, 2.0], [2.5, -3.0, 0.25, -0.25, 1.5, 0.0, 0.0, 0.0]]
    ups = [[1.0, -2.0, 3.0, -4.0, 5.0, -6.0, 7.0, -8.0], [-1.0, 2.0, -3.0, 4.0, -5.0, 0.0, 0.0, 0.0]]
    gu = _t([gates[0] + ups[0], gates[1] + ups[1]], dev)
    out = ops.silu_mul(gu).float().cpu()
    exp = torch.tensor([[silu_mul_expected(r(g), r(u)) for g, u in zip(gr, ur)]
                        for gr, ur in zip(gates, ups)])
    return out, exp


def case_add_rms(ops, dev, eps=1e-6):
    """probe_gpu_no_torch.py:103-153: residual add (bit-exact) then RMSNorm."""
    x = [[0.25, -0.5, 1.0, -1.5, 2.0, -2.5, 0.125], [-0.125, 0.75, -1.25, 1.75, -2.25, 2.75, -0.875]]
    d = [[0.1, 0.2, -0.3, 0.4, -0.5, 0.6, -0.7], [0.7, -0.6, 0.5, -0.4, 0.3, -0.2, -0.1]]
    w = [1.0, 0.75, 1.25, -0.5, 1.5, 0.25, -1.0]
    hn, y = ops.add_rms(_t(x, dev), _t(d, dev), _t(w, dev))
    xb = [[r(v) for v in row] for row in x]
    db = [[r(v) for v in row] for row in d]
    wb = [r(v) for v in w]
    h_exp = torch.tensor([[r(a + b) for a, b in zip(xr, dr)] for xr, dr in zip(xb, db)])
    y_exp = torch.tensor([rms_expected(row.tolist(), wb, eps) for row in h_exp])
    return hn.float().cpu(), h_exp, y.float().cpu(), y_exp


def case_gemv_exact(ops, dev, M=2, N=32, K=64):
    """probe_gpu_no_torch.py:467-527: one-hot activation rows make every output an exact sum of
    two bf16 weights, so the GEMV must match bit for bit."""
    x = torch.zeros(M, K)
    for row in range(M):
        x[row, row] = 1.0
        x[row, 32 + row] = 1.0
    w = torch.zeros(N, K)
    for n in range(N):
        w[n, 0] = (n % 4 + 1) * 0.125
        w[n, 32] = (n % 3 + 1) * 0.0625
        w[n, 1] = -(n % 5 + 1) * 0.125
        w[n, 33] = (n % 2 + 1) * 0.25
    out = ops.linear(x.to(BF).to(dev), w.to(BF).to(dev)).float().cpu()
    exp = torch.tensor([[r(w[n, row].item() + w[n, 32 + row].item()) for n in range(N)]
                        for row in range(M)])
    return out, exp


def case_gate_up_exact(ops, dev, M=2, N=32, K=64):
    """probe_gpu_no_torch.py:576-621: fused gate/up GEMV with SiLU epilogue on exact sums."""
    x = torch.zeros(M, K)
    for row in range(M):
        x[row, row] = 1.0
        x[row, 32 + row] = 1.0
    w = torch.zeros(2 * N, K)
    for n in range(N):
        w[n, 0] = (n % 4 + 1) * 0.125
        w[n, 32] = (n % 3 + 1) * 0.0625
        w[n, 1] = -(n % 5 + 1) * 0.125
        w[n, 33] = (n % 2 + 1) * 0.25
        for row in range(M):
            up = 1.0 if row == 0 else -0.5
            w[N + n, row] = up
            w[N + n, 32 + row] = up
    out = ops.gate_up_silu(x.to(BF).to(dev), w.to(BF).to(dev)).float().cpu()
    exp = torch.tensor([[silu_mul_expected(r(w[n, row].item() + w[n, 32 + row].item()),
                                           r(w[N + n, row].item() + w[N + n, 32 + row].item()))
                         for n in range(N)] for row in range(M)])
    return out, exp


def case_linear_add_norm_exact(ops, dev, eps=1e-6, M=2, N=7, K=64):
    """probe_gpu_no_torch.py:627-688 (restated through the public op): hn = h + bf16(x.W^T) is
    bit-exact on exact sums; y follows the RMSNorm rounding points."""
    x = torch.zeros(M, K)
    for row in range(M):
        x[row, row] = 1.0
        x[row, 32 + row] = 1.0
    w = torch.zeros(N, K)
    for n in range(N):
        for row in range(M):
            w[n, row] = (n + 1) * 0.0625
            w[n, 32 + row] = (1 if n % 2 == 0 else -1) * (row + 1) * 0.03125
    h = torch.tensor([[((c - 3) * 0.25 + row * 0.125) for c in range(N)] for row in range(M)])
    lnw = torch.tensor([0.5 + c * 0.125 for c in range(N)])
    hn, y = ops.linear_add_norm(x.to(BF).to(dev), w.to(BF).to(dev), h.to(BF).to(dev),
                                lnw.to(BF).to(dev))
    lin = [[r(w[n, row].item() + w[n, 32 + row].item()) for n in range(N)] for row in range(M)]
    h_exp = torch.tensor([[r(h[row, n].item() + lin[row][n]) for n in range(N)] for row in range(M)])
    y_exp = torch.tensor([rms_expected(row.tolist(), [r(v) for v in lnw.tolist()], eps)
                          for row in h_exp])
    return hn.float().cpu(), h_exp, y.float().cpu(), y_exp


def rotation_tables(cap, hd, cos_by_pos, sin_by_pos):
    """Rope tables whose row p is the constant cos_by_pos[p] / sin_by_pos[p] (identity 1/0,
    quarter turn 0/1, mixed 0.75/0.25), the probe's rotation special cases."""
    cos = torch.tensor([[cos_by_pos[p] if p < len(cos_by_pos) else 1.0] * hd for p in range(cap)])
    sin = torch.tensor([[sin_by_pos[p] if p < len(sin_by_pos) else 0.0] * hd for p in range(cap)])
    return cos.to(BF), sin.to(BF)


def qkv_decode_expected(qkv_row_vals, h, hd, eps, c, s):
    """Expected q/k head after norm (weights 1) and rotation by the constant (c, s)."""
    vals = qkv_row_vals[h * hd:(h + 1) * hd]
    var = sum(v * v for v in vals) / hd
    normed = [r(r(v / math.sqrt(var + eps)) * 1.0) for v in vals]
    return rope_expected(normed, c, s)


def case_attention_structured(B=2, NKV=2, G=4, HD=128, CAP=128, W=7, pos=(0, 66)):
    """probe_gpu_no_torch.py:333-401: structured q/k/v whose softmax has a closed form; the
    second row crosses a 64-key tile boundary. Returns (q [B,NKV,W,G,HD], kc, vc, pos, expected
    [B*W, NKV*G*HD] float64)."""
    q = torch.zeros(B, NKV, W, G, HD)
    k = torch.zeros(B, NKV, CAP, HD)
    v = torch.zeros(B, NKV, CAP, HD)
    for b in range(B):
        for h in range(NKV):
            base = (b + 1) * (h + 1) * 0.25
            for s in range(W):
                q[b, h, s, :, 0] = 2 * (s + 1)
            for j in range(66 + W):
                k[b, h, j, 0] = 2 * (j % 4 + 1)
                v[b, h, j, :] = (2 * (j % 4) + 1) * base
    exp = torch.zeros(B * W, NKV * G * HD, dtype=torch.float64)
    for b in range(B):
        for h in range(NKV):
            base = (b + 1) * (h + 1) * 0.25
            for s in range(W):
                scores = [4 * (s + 1) * (j % 4 + 1) * HD ** -0.5 for j in range(pos[b] + s + 1)]
                peak = max(scores)
                wts = [math.exp(sc - peak) for sc in scores]
                val = sum(wt * (2 * (j % 4) + 1) * base for j, wt in enumerate(wts)) / sum(wts)
                for g in range(G):
                    exp[b * W + s, (h * G + g) * HD:(h * G + g + 1) * HD] = val
    return q.to(BF), k.to(BF), v.to(BF), torch.tensor(pos, dtype=torch.long), exp
