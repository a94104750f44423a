"""Seeded synthetic tensors that come out the same on the CPU and on the GPU.

Random-init weights for a 1.7B-parameter model take about a minute to draw
with the CPU generator, and the GPU generator's stream differs from the CPU's.
This draws them from a counter-based generator written in plain torch ops
instead: element i of stream s under seed k is a function of (k, s, i) alone,
computed with 64-bit integer mixing (exact on every device) and an f64
Box-Muller transform. The f64 values agree between devices to an ulp or two,
far inside one bf16 step, so the landed bf16 tensors are identical (a
disagreement needs an f64 value within ~1e-16 of a bf16 rounding boundary).
On the GPU the whole model takes well under a second.
"""
from __future__ import annotations

import math

import torch

_M64 = (1 << 64) - 1


def _i64(c: int) -> int:
    """A 64-bit constant as the int64 torch stores."""
    c &= _M64
    return c - (1 << 64) if c >= (1 << 63) else c


_C1 = _i64(0x9E3779B97F4A7C15)
_C2 = _i64(0xBF58476D1CE4E5B9)
_C3 = _i64(0x94D049BB133111EB)
_C4 = _i64(0xD6E8FEB86659FD93)


def _shr(x: torch.Tensor, k: int) -> torch.Tensor:
    """Logical right shift of int64 bit patterns."""
    return (x >> k) & ((1 << (64 - k)) - 1)


def _mix(z: torch.Tensor) -> torch.Tensor:
    """splitmix64's finaliser (wrapping 64-bit arithmetic)."""
    z = (z ^ _shr(z, 30)) * _C2
    z = (z ^ _shr(z, 27)) * _C3
    return z ^ _shr(z, 31)


def normal(shape, seed: int, stream: int, std: float = 1.0, mean: float = 0.0,
           device="cpu", dtype=torch.bfloat16, chunk: int = 1 << 26) -> torch.Tensor:
    """``mean + std * N(0, 1)`` of ``shape``, reproducible across devices."""
    n = 1
    for d in shape:
        n *= int(d)
    out = torch.empty(n, dtype=dtype, device=device)
    base = _mix(torch.tensor([_i64(seed * 0x100000001B3 + stream * 0x9E3779B1)], dtype=torch.int64,
                             device=device))
    two_pi = 2.0 * math.pi
    for s in range(0, n, chunk):
        e = min(n, s + chunk)
        i = torch.arange(s, e, dtype=torch.int64, device=device)
        k1 = _mix(base + i * _C1)
        k2 = _mix(k1 ^ _C4)
        u1 = (_shr(k1, 11) + 1).to(torch.float64) * (2.0 ** -53)   # (0, 1]
        u2 = _shr(k2, 11).to(torch.float64) * (2.0 ** -53)         # [0, 1)
        z = torch.sqrt(-2.0 * torch.log(u1)) * torch.cos(two_pi * u2)
        out[s:e] = (mean + std * z).to(torch.float32).to(dtype)
        del i, k1, k2, u1, u2, z
    return out.view(*shape)
