"""Pin the CPU oracle (oracle.reference) against closed forms: the reference's own driver-level
known-answer cases (tests/probe_gpu_no_torch.py), the textbook rope tables, and fp64 brute force.
These run on the CPU only."""
import math

import pytest
import torch

import known_answers as ka
from oracle import bf16 as B16
from oracle.reference import (TorchOps, attn_reference_fp64, build_rope_tables, fake_engine, rms,
                              rope)

CPU = torch.device("cpu")


@pytest.fixture
def ops():
    return TorchOps(fake_engine(nh=8, nkv=2, hd=128))


def test_bf16_helper_rne():
    # ties to even, and values just above a tie round up
    assert B16.r(1.0 + 2 ** -8) == 1.0
    assert B16.r(1.0 + 3 * 2 ** -8) == 1.0 + 2 ** -6
    assert B16.r(1.0 + 2 ** -8 + 2 ** -20) == 1.0 + 2 ** -7
    for v in (0.1, -3.7, 1e-3, 12345.678):
        assert B16.r(v) == torch.tensor(v).to(torch.bfloat16).item()


def test_silu_known_answer(ops):
    out, exp = ka.case_silu(ops, CPU)
    assert (out - exp).abs().max().item() < 0.05
    # torch's CPU silu rounds at the same points: identical on these values
    assert torch.equal(out, exp)


def test_add_rms_known_answer(ops):
    hn, h_exp, y, y_exp = ka.case_add_rms(ops, CPU)
    assert torch.equal(hn, h_exp)                   # residual add is bit-exact
    assert (y - y_exp).abs().max().item() < 0.02


def test_rms_rounds_before_weight():
    # a dropped bf16 cast before the weight multiply changes this value
    x = torch.tensor([[1.0, 3.0, 5.0, 7.0]], dtype=torch.bfloat16)
    w = torch.tensor([1.0, 1.0 + 2 ** -7, 1.0, 1.0], dtype=torch.bfloat16)
    y = rms(x, w, 1e-6).float()
    exp = B16.rms_expected([1.0, 3.0, 5.0, 7.0], [1.0, 1.0 + 2 ** -7, 1.0, 1.0], 1e-6)
    assert y.tolist()[0] == exp


def test_gemv_exact_sums(ops):
    out, exp = ka.case_gemv_exact(ops, CPU)
    assert torch.equal(out, exp)


def test_gate_up_exact(ops):
    out, exp = ka.case_gate_up_exact(ops, CPU)
    assert (out - exp).abs().max().item() < 0.02


def test_linear_add_norm_exact(ops):
    hn, h_exp, y, y_exp = ka.case_linear_add_norm_exact(ops, CPU)
    assert torch.equal(hn, h_exp)
    assert (y - y_exp).abs().max().item() < 0.02


def test_linear_fp64_bruteforce(ops):
    g = torch.Generator().manual_seed(1)
    x = torch.randn(3, 40, generator=g).to(torch.bfloat16)
    w = torch.randn(24, 40, generator=g).to(torch.bfloat16)
    ref = x.double() @ w.double().T
    out = ops.linear(x, w).double()
    assert ((out - ref).abs() <= 2 ** -7 * ref.abs() + 1e-6).all()


def test_rope_tables_closed_form():
    theta, hd, n = 5e6, 128, 4096
    cos, sin = build_rope_tables(theta, hd, n)
    j = torch.arange(0, hd, 2, dtype=torch.float64)
    inv = 1.0 / theta ** (j / hd)
    ang = torch.outer(torch.arange(n, dtype=torch.float64), torch.cat((inv, inv)))
    # bound: bf16 rounding (half an ulp, 2^-8 relative) plus the fp32 angle error, which grows
    # with the angle (a few fp32 ulps of inv, times the position)
    for got, want in ((cos, ang.cos()), (sin, ang.sin())):
        err = (got.double() - want).abs()
        assert (err <= want.abs() * 2 ** -8 + ang * 8 * 2 ** -24).all()
    # a wrong exponent (j/hd instead of 2j/hd) would fail the bound above by orders of magnitude
    bad = torch.outer(torch.arange(n, dtype=torch.float64), 1.0 / theta ** (torch.arange(0, hd // 2,
                      dtype=torch.float64) / hd)).repeat(1, 2).cos()
    assert ((cos.double() - bad).abs() > bad.abs() * 2 ** -8 + ang * 8 * 2 ** -24).any()
    # duplicated halves (emb = cat(f, f)) and the exact row 0
    assert torch.equal(cos[:, :hd // 2], cos[:, hd // 2:])
    assert torch.equal(cos[0], torch.ones(hd, dtype=torch.bfloat16))
    assert torch.equal(sin[0], torch.zeros(hd, dtype=torch.bfloat16))


def test_rope_tables_match_hf():
    from transformers import Qwen3Config
    from transformers.models.qwen3.modeling_qwen3 import Qwen3RotaryEmbedding
    cfg = Qwen3Config(head_dim=128, rope_theta=5e6, hidden_size=256, num_attention_heads=2,
                      max_position_embeddings=4096)
    rot = Qwen3RotaryEmbedding(cfg)
    x = torch.zeros(1, 1, 128)
    cos_hf, sin_hf = rot(x, torch.arange(2048)[None])
    cos, sin = build_rope_tables(5e6, 128, 2048)
    assert torch.equal(cos_hf[0].to(torch.bfloat16), cos)
    assert torch.equal(sin_hf[0].to(torch.bfloat16), sin)


def test_rope_rotate_half_sign():
    # quarter turn (cos 0, sin 1) maps x -> cat(-x[h:], x[:h]) exactly
    x = torch.arange(1, 9, dtype=torch.float32).to(torch.bfloat16)
    y = rope(x, torch.zeros(8, dtype=torch.bfloat16), torch.ones(8, dtype=torch.bfloat16))
    assert y.tolist() == [-5.0, -6.0, -7.0, -8.0, 1.0, 2.0, 3.0, 4.0]


def test_qkv_post_prefill_last_query_rotations():
    """probe_gpu_no_torch.py:158-246: identity / quarter turn / (0.75, 0.25) at positions 0..2;
    V bit-exact, K rotated per position, q of the last token only, cache tail untouched."""
    B, S, CAP, NH, NKV, HD, EPS = 2, 3, 8, 4, 2, 128, 1e-6
    e = fake_engine(nh=NH, nkv=NKV, hd=HD)
    e.cos, e.sin = ka.rotation_tables(CAP, HD, [1.0, 0.0, 0.75], [0.0, 1.0, 0.25])
    ops = TorchOps(e)
    total = (NH + 2 * NKV) * HD
    qkv = torch.tensor([((i % 31) - 15) / 16 for i in range(B * S * total)]).reshape(B * S, total)
    qkv = qkv.to(torch.bfloat16)

    class L:
        qn = torch.ones(HD, dtype=torch.bfloat16)
        kn = torch.ones(HD, dtype=torch.bfloat16)
    kc = torch.zeros(B, NKV, CAP, HD, dtype=torch.bfloat16)
    vc = torch.zeros_like(kc)
    q = ops.qkv_post(qkv, L, kc, vc, B, S, None, last_query_only=True)
    rc, rs = [1.0, 0.0, 0.75], [0.0, 1.0, 0.25]
    vals = qkv.float()
    for b in range(B):
        for h in range(NH):
            exp = ka.qkv_decode_expected(vals[b * S + S - 1].tolist(), h, HD, EPS, rc[S - 1], rs[S - 1])
            assert (q[b, h, 0].float() - torch.tensor(exp)).abs().max() < 0.03
        for h in range(NKV):
            for s in range(S):
                exp = ka.qkv_decode_expected(vals[b * S + s].tolist(), NH + h, HD, EPS, rc[s], rs[s])
                assert (kc[b, h, s].float() - torch.tensor(exp)).abs().max() < 0.03
                src = qkv[b * S + s, (NH + NKV + h) * HD:(NH + NKV + h + 1) * HD]
                assert torch.equal(vc[b, h, s], src)
        assert not kc[b, :, S:].any() and not vc[b, :, S:].any()


def test_qkv_post_decode_per_row_positions():
    """probe_gpu_no_torch.py:251-328: two rows at positions (2, 4); V bit-exact; K rotated by
    the table row of its own position; q in the [B, NKV, S, G, HD] decode layout."""
    B, CAP, NH, NKV, HD, EPS = 2, 8, 4, 2, 128, 1e-6
    G = NH // NKV
    e = fake_engine(nh=NH, nkv=NKV, hd=HD)
    dcos = [1.0, 1.0, 0.75, 1.0, 0.0, 0.75]
    dsin = [0.0, 0.0, 0.25, 0.0, 1.0, 0.25]
    e.cos, e.sin = ka.rotation_tables(CAP, HD, dcos, dsin)
    ops = TorchOps(e)
    total = (NH + 2 * NKV) * HD
    qkv = torch.tensor([((i % 37) - 18) / 16 for i in range(B * total)]).reshape(B, total)
    qkv = qkv.to(torch.bfloat16)

    class L:
        qn = torch.ones(HD, dtype=torch.bfloat16)
        kn = torch.ones(HD, dtype=torch.bfloat16)
    kc = torch.zeros(B, NKV, CAP, HD, dtype=torch.bfloat16)
    vc = torch.zeros_like(kc)
    pos = torch.tensor([2, 4])
    q = ops.qkv_post_rows(qkv, L, kc, vc, pos)           # [B, NH, 1, HD]
    qd = q.reshape(B, NKV, 1, G, HD)                     # decode layout of the same buffer
    vals = qkv.float()
    for b in range(B):
        p = int(pos[b])
        for h in range(NH):
            exp = ka.qkv_decode_expected(vals[b].tolist(), h, HD, EPS, dcos[p], dsin[p])
            assert (qd[b, h // G, 0, h % G].float() - torch.tensor(exp)).abs().max() < 0.03
        for h in range(NKV):
            exp = ka.qkv_decode_expected(vals[b].tolist(), NH + h, HD, EPS, dcos[p], dsin[p])
            assert (kc[b, h, p].float() - torch.tensor(exp)).abs().max() < 0.03
            assert torch.equal(vc[b, h, p], qkv[b, (NH + NKV + h) * HD:(NH + NKV + h + 1) * HD])
            others = [j for j in range(CAP) if j != p]
            assert not kc[b, h, others].any() and not vc[b, h, others].any()


def test_attention_structured_closed_form():
    """probe_gpu_no_torch.py:333-401 closed form, through the fp64 loop reference and (one
    query token at a time) the oracle's SDPA-based attn_decode."""
    q, kc, vc, pos, exp = ka.case_attention_structured()
    B, NKV, W, G, HD = q.shape
    loop = attn_reference_fp64(q, kc, vc, pos, W, NKV * G, NKV, HD)
    assert (loop - exp).abs().max().item() < 1e-9 + 0.02   # bf16 inputs are exact here
    ops = TorchOps(fake_engine(nh=NKV * G, nkv=NKV, hd=HD))
    for b in range(B):
        for s in range(W):
            o = ops.attn_decode(q[b:b + 1, :, s:s + 1].contiguous(), kc[b:b + 1], vc[b:b + 1],
                                torch.tensor([int(pos[b]) + s]))
            assert (o[0].double() - exp[b * W + s]).abs().max().item() < 0.02


def test_attention_sdpa_vs_fp64_random():
    g = torch.Generator().manual_seed(3)
    NH, NKV, HD, cap = 32, 8, 128, 640
    ops = TorchOps(fake_engine(nh=NH, nkv=NKV, hd=HD))
    for B, posl in ((1, [512]), (4, [512, 300, 0, 17])):
        kc = torch.randn(B, NKV, cap, HD, generator=g).to(torch.bfloat16)
        vc = torch.randn(B, NKV, cap, HD, generator=g).to(torch.bfloat16)
        q = torch.randn(B, NKV, 1, NH // NKV, HD, generator=g).to(torch.bfloat16)
        pos = torch.tensor(posl)
        out = ops.attn_decode_rows(q.reshape(B, NH, 1, HD), kc, vc, pos).double()
        ref = attn_reference_fp64(q, kc, vc, pos, 1, NH, NKV, HD)
        assert (out - ref).abs().max().item() < 0.02


def test_argmax_first_index_on_ties():
    logits = torch.tensor([[1.0, 3.0, 3.0, -1.0], [float("nan"), 2.0, float("nan"), 5.0]])
    assert logits.to(torch.bfloat16).argmax(-1).tolist() == [1, 0]
    assert math.isnan(float("nan"))
