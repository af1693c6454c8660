"""Pure-Python bf16 helpers (round to nearest even), for tiny known-answer cases.

These restate the RNE helper of the reference's driver-level probe
(tests/probe_gpu_no_torch.py:42-49) so that closed-form expectations can be written with the
reference's rounding points spelled out by hand. Test infrastructure only.
"""
import math
import struct


def bf16_bits(x):
    """float -> bf16 bit pattern, round to nearest even (finite inputs)."""
    bits = struct.unpack("I", struct.pack("f", x))[0]
    bits += 0x7FFF + ((bits >> 16) & 1)
    return (bits >> 16) & 0xFFFF


def from_bits(b):
    return struct.unpack("f", struct.pack("I", (b & 0xFFFF) << 16))[0]


def r(x):
    """Round a Python float to the nearest bf16 value (returned as a float)."""
    return from_bits(bf16_bits(x))


def f32(x):
    """Round a Python float to fp32."""
    return struct.unpack("f", struct.pack("f", x))[0]


def silu_mul_expected(g, u):
    """bf16(bf16(silu(g)) * u) with g, u already bf16 (fused.py:677-682 rounding points)."""
    return r(r(g / (1.0 + math.exp(-g))) * u)


def rms_expected(row, w, eps):
    """y = bf16(bf16(x * rsqrt(mean(x^2) + eps)) * w) for one row (engine.py:107-110)."""
    var = sum(v * v for v in row) / len(row)
    return [r(r(v / math.sqrt(var + eps)) * wc) for v, wc in zip(row, w)]


def rope_expected(normed, cos, sin):
    """bf16(bf16(x*cos) + bf16(rot(x)*sin)) with rot = cat(-x[h:], x[:h]) (engine.py:113-115)."""
    hd = len(normed)
    h = hd // 2
    out = []
    for d in range(hd):
        partner = -normed[d + h] if d < h else normed[d - h]
        out.append(r(r(normed[d] * cos) + r(partner * sin)))
    return out
