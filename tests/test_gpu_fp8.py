"""fp8 prefill GEMMs (opt-in, ENGINE_FP8=1): the HIP tensorwise quantisation against torch's own
float -> float8_e4m3fn cast on the CPU (bit for bit: scale and every byte, round-to-nearest-even
ties included), the fp8 GEMM against a float64 product of the dequantised operands, and a
prefill through the engine with fp8 QKV and gate/up projections against the bf16 oracle (the
reference's 2.0-logit gate: the path is not bf16-exact by design, engine.py:97-104).
"""
import math
import os

import pytest
import torch

from dryft_amd import synth
from gpu_checks import near_tie
from oracle.reference import OracleEngine

pytestmark = pytest.mark.gpu
F8 = torch.float8_e4m3fn


def _lib():
    from dryft_amd._lib import lib
    return lib()


def _quant(x):
    L = _lib()
    n = x.numel()
    out = torch.empty(n, dtype=F8, device="cuda")
    sc = torch.empty(1, dtype=torch.float32, device="cuda")
    ws = torch.empty(L.dd_fp8_quant_ws_bytes(n) // 4 + 1, dtype=torch.float32, device="cuda")
    assert L.dd_fp8_quant(x.data_ptr(), n, out.data_ptr(), sc.data_ptr(), ws.data_ptr(),
                          torch.cuda.current_stream().cuda_stream) == 0
    return out.view(x.shape), sc


def _torch_quant(x):
    """quant_fp8_tensorwise (fused.py:140-149) on the CPU: amax over |x|, scale amax / 448,
    values x * (448 / amax) cast to float8_e4m3fn."""
    xf = x.float()
    amax = xf.abs().max().clamp(min=1e-6)
    inv = torch.tensor(448.0) / amax
    return (xf * inv).to(F8), (amax / 448.0).reshape(1)


@pytest.mark.parametrize("shape,spread", [((16, 1024), 1.0), ((80, 2560), 30.0), ((1, 8), 1e-4),
                                          ((48, 9728), 1.0)])
def test_quant_matches_torch_cast(cuda, shape, spread):
    g = torch.Generator().manual_seed(shape[0])
    x = (torch.randn(shape, generator=g) * spread).to(torch.bfloat16)
    x.view(-1)[::97] = 0.0
    x.view(-1)[5::131] *= 40                        # outliers set the scale
    q, sc = _quant(x.cuda())
    wq, wsc = _torch_quant(x)
    assert torch.equal(sc.cpu(), wsc)
    assert torch.equal(q.cpu().view(torch.uint8), wq.view(torch.uint8))


def test_quant_rounding_edges(cuda):
    """amax 448 makes the scale exactly 1: the kernel's conversion meets the cast on chosen
    values -- subnormal ties (2^-10 -> 0, 3 * 2^-11 -> 2^-9), the subnormal/normal seam, mantissa
    ties to even (1.0625 -> 1, 1.1875 -> 1.25), rounding up to the largest finite 448, signs."""
    vals = [448.0, 440.0, 432.0, 2 ** -9, 2 ** -10, 3 * 2 ** -11, 2 ** -6, 2 ** -6 * 1.0625,
            2 ** -7 * 1.9375, 1.0625, 1.1875, 1.3125, -0.0, -3.5, -448.0, 0.0, 5 * 2 ** -10,
            7 * 2 ** -10, 15.5, 17.0, 2 ** -12, 0.1]
    x = torch.tensor(vals + [0.0] * (-len(vals) % 8), dtype=torch.bfloat16)
    q, sc = _quant(x.cuda())
    wq, wsc = _torch_quant(x)
    assert float(sc) == 1.0 and torch.equal(sc.cpu(), wsc)
    assert q.cpu().view(torch.uint8).tolist() == wq.view(torch.uint8).tolist()


def test_quant_nan_propagates(cuda):
    """A NaN anywhere in x makes the scale NaN and every quantised value NaN, as torch's amax and
    clamp (the reference's quantisation, fused.py:130-149) propagate it."""
    x = torch.randn(4096, generator=torch.Generator().manual_seed(5)).to(torch.bfloat16)
    x[1234] = float("nan")
    q, sc = _quant(x.cuda())
    assert math.isnan(float(sc))
    assert torch.isnan(q.cpu().float()).all()
    wq, wsc = _torch_quant(x)
    assert math.isnan(float(wsc)) and torch.isnan(wq.float()).all()


def test_fp8_linear_matches_dequantised_product(cuda):
    from dryft_amd.hipops import HipOps
    import types
    e = types.SimpleNamespace(dev=torch.device("cuda"), eps=1e-6, nh=8, nkv=2, hd=128)
    ops = HipOps(e)
    g = torch.Generator().manual_seed(3)
    M, K, N = 64, 2560, 1536
    x = torch.randn(M, K, generator=g).to(torch.bfloat16).cuda()
    w = (torch.randn(N, K, generator=g) * 0.02).to(torch.bfloat16).cuda()
    s = (w.abs().amax().clamp(min=1e-6) / 448.0).float().reshape(1, 1)
    w8 = (w / s).to(F8).contiguous()
    y = ops.fp8_linear(x, w8, s, w)
    xq, xs = _quant(x)
    ref = (xq.double() * float(xs)) @ (w8.double() * float(s)).T
    d = (y.double() - ref).abs().max().item()
    scale = ref.abs().max().item()
    assert d <= 1e-2 * scale, (d, scale)
    # a row count that is not a multiple of 16 takes the bf16 path, as the reference's _fp8_lin
    # does (engine.py:451-454); 48 rows (a multiple) stay on fp8
    assert torch.equal(ops.fp8_linear(x[:5], w8, s, w), ops.linear(x[:5], w))
    assert torch.equal(ops.fp8_linear(x[:37], w8, s, w), ops.linear(x[:37], w))
    y48 = ops.fp8_linear(x[:48], w8, s, w)
    xq48, xs48 = _quant(x[:48].contiguous())
    ref48 = (xq48.double() * float(xs48)) @ (w8.double() * float(s)).T
    assert y48.shape == (48, N) and (y48.double() - ref48).abs().max().item() <= 1e-2 * scale
    bf = torch.nn.functional.linear(x, w)
    print(f"fp8 GEMM: max|y - dequantised fp64| {d:.3g} (scale {scale:.3g}); "
          f"max|y - bf16 linear| {(y - bf).abs().max().item():.3g}")


SMALL = synth.qwen3_config(vocab_size=1024, hidden_size=1024, intermediate_size=512,
                           num_hidden_layers=3, num_attention_heads=4, num_key_value_heads=1,
                           head_dim=128)


def test_engine_fp8_prefill_gate(cuda, monkeypatch):
    """A packed prefill with fp8 QKV and gate/up GEMMs: first-token logits within the 2.0 gate of
    the bf16 oracle, the first token its argmax up to the measured disagreement."""
    from dryft_amd.engine import Engine
    monkeypatch.setenv("ENGINE_FP8", "1")
    w = synth.random_weights(SMALL, seed=4)
    ref = OracleEngine.from_state_dict(SMALL, dict(w))
    eng = Engine.from_state_dict(SMALL, {k: v.cuda() for k, v in w.items()})
    assert eng.fp8 and hasattr(eng.layers[0], "wqkv8")
    g = torch.Generator().manual_seed(9)
    lens = [16, 37, 43]                                   # 96 packed rows: the fp8 GEMMs
    prompts = [torch.randint(0, 1024, (n,), generator=g).tolist() for n in lens]
    st = eng._new_state(len(lens), 128)
    eng._dbg = []
    eng._prefill(prompts, st)
    logits = eng._dbg[-1]
    eng._dbg = None
    for b, p in enumerate(prompts):
        rs = ref.new_state(1, 128)
        ref._dbg = []
        ref.prefill(rs, torch.tensor([p]))
        rl = ref._dbg[-1][0]
        ref._dbg = None
        d = (logits[b] - rl).abs().max().item()
        assert d <= 2.0, (b, d)
        tok = int(st.tok[b])
        gap, tie = near_tie(rl, tok, d)
        assert tok == int(rl.argmax()) or tie, (b, tok, int(rl.argmax()), gap)
        print(f"fp8 prefill prompt {b} (len {lens[b]}): max|logit diff| vs bf16 oracle {d:.4f}")
