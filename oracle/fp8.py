"""The E4M3 KV-cache format: quantizer, dequantizer and the format's closed form.
TEST INFRASTRUCTURE ONLY.

The reference has no FP8 KV cache (README.md:431 lists it as a roadmap item), so the format is
this build's: OCP FP8 E4M3 (PyTorch's float8_e4m3fn) with one positive scale per cache tensor.
  quantize(x, s)   = (x.float() / s).clamp(-448, 448).to(torch.float8_e4m3fn)   (PyTorch, CPU)
  dequantize(c, s) = c.float() * s
The attention over an E4M3 cache is checked against the fp32 / fp64 oracles run on the
dequantized caches. `e4m3_value` is the format's definition (sign, 4-bit exponent with bias 7,
3-bit mantissa; exponent 0 subnormal; 0x7f / 0xff NaN; no infinities), against which the
tests pin PyTorch's conversion in both directions.
"""

from __future__ import annotations

import math

import torch

FP8 = torch.float8_e4m3fn
FP8_MAX = 448.0


def e4m3_value(code: int) -> float:
    """The real number an E4M3 byte encodes (NaN for 0x7f / 0xff)."""
    sign = -1.0 if code & 0x80 else 1.0
    e, m = (code >> 3) & 0xF, code & 0x7
    if e == 0xF and m == 0x7:
        return math.nan
    if e == 0:
        return sign * (m / 8.0) * 2.0**-6
    return sign * (1.0 + m / 8.0) * 2.0 ** (e - 7)


def quantize(x: torch.Tensor, scale: float) -> torch.Tensor:
    """x (any float dtype, any device) -> float8_e4m3fn on the CPU, as the cache stores it."""
    return (x.detach().cpu().float() / scale).clamp(-FP8_MAX, FP8_MAX).to(FP8)


def dequantize(c: torch.Tensor, scale: float) -> torch.Tensor:
    """float8_e4m3fn -> fp32 values e4m3 * scale (on c's device)."""
    return c.float() * scale
