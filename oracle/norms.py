"""RMSNorm variants (CPU, torch) -- test infrastructure only.

Reference rounding orders:

* ``rms_norm_q`` -- Qwen3RMSNorm / MiniCPMRMSNorm: normalise in f32, land in
  bf16, *then* multiply by the bf16 gamma (bf16 x bf16 -> bf16).
  examples/qwen3_1_7b-tilelang/fast/test_kernels.py:32-38 (t_rms_norm);
  examples/qwen3_1_7b-tilelang/ref_src/model.py:124-136;
  examples/minicpm3_4b-cutedsl/kernels/reference_ops.py:31-39.
* ``rms_norm_1p`` -- Qwen3_5RMSNorm: ``x * rsqrt(mean x^2 + eps) * (1 + gamma)``
  in f32, one landing in bf16.
  examples/qwen3_8_27b_prefill-tilelang/kernels/elementwise.py:5,64;
  src/tilefoundry/ir/hir/nn/rms_norm.py:99-106 (HIR eval rule) with the
  ``gamma + 1.0`` weight of examples/qwen3_8_27b_prefill-tilelang/model.py:344.
* ``add_rms_norm`` -- residual add landing in bf16, then ``rms_norm_q`` of the
  landed sum: examples/qwen3_1_7b-tilelang/fast/test_kernels.py:41-53
  (t_resid_rms_norm) with ``P`` already reduced.

Pinned by (tests/test_oracle.py): the constant-row closed form (a row of one
value c normalises to sign(c), so y == sign(c) * gamma exactly); agreement with
an f64 evaluation to within one bf16 rounding; and a planted-mistake check
(dropping the bf16 landing before gamma changes the result on random rows).
``resid_rms_norm`` is pinned on its own: against its f64 statement (1-8
partials, one ulp), exactly on integer partials (the integer sum; a row summing
to a constant normalises to sign(c) * gamma), and by two hand-worked
known answers that separate its two landings, which fail when the partials are
landed before the sum or when the residual add and the sum land once.
"""
from __future__ import annotations

import torch

BF16 = torch.bfloat16


def rms_norm_q(x: torch.Tensor, gamma: torch.Tensor, eps: float) -> torch.Tensor:
    """``bf16(bf16(x * rsqrt(mean(x^2) + eps)) * gamma)`` over the last axis."""
    x32 = x.float()
    var = (x32 * x32).mean(-1, keepdim=True)
    return (x32 * torch.rsqrt(var + eps)).to(BF16) * gamma.to(BF16)


def rms_norm_1p(x: torch.Tensor, gamma: torch.Tensor, eps: float) -> torch.Tensor:
    """``bf16(x * rsqrt(mean(x^2) + eps) * (1 + gamma))`` in f32."""
    x32 = x.float()
    var = x32.pow(2).mean(-1, keepdim=True)
    return (x32 * torch.rsqrt(var + eps) * (gamma.float() + 1.0)).to(BF16)


def rms_norm(x, gamma, eps, mode: int = 0):
    return rms_norm_q(x, gamma, eps) if mode == 0 else rms_norm_1p(x, gamma, eps)


def add_rms_norm(x, residual, gamma, eps, mode: int = 0):
    """Returns ``(y, residual_out)``: ``residual_out = bf16(x + residual)``."""
    r = (x.to(BF16) + residual.to(BF16))
    return rms_norm(r, gamma, eps, mode), r


def resid_rms_norm(a, partials, gamma, eps):
    """``Hout = A + bf16(sum_s P[s])``; ``Xn = rms_norm_q(Hout)``.

    examples/qwen3_1_7b-tilelang/fast/test_kernels.py:41-53.
    """
    h = a + partials.float().sum(0).to(BF16)
    return h, rms_norm_q(h, gamma, eps)
