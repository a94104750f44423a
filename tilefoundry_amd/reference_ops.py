"""The MiniCPM3 decode operations under the reference's names, on gfx950 kernels.

Mirrors examples/minicpm3_4b-cutedsl/kernels/reference_ops.py (the torch
statement of the interface) and kernels/cute_ops.py (its kernel-backed twin):
flat ``(hidden,)`` activations, every projection weight ``(out, in)`` row-major,
and each function writes the destination it is given (``out=``) or allocates
one when none is -- a step that passes every destination allocates nothing and
can be captured as a HIP graph. Positions and context lengths are one-element
device tensors, read inside the kernels.

Rounding follows the torch statement: the RMSNorm lands in bf16 before the
learned scale; each projection lands in bf16; SwiGLU lands the activation
before the product; ``embed_scaled`` and ``lm_head_gemv`` scale / divide in f32
and land once; ``rope_attend`` rotates in bf16, scales the query in bf16,
keeps scores and weights in f32.

``rope_attend`` needs an f32 workspace for its split partials; it is allocated
once per (device, shape) and kept.
"""
from __future__ import annotations

import torch

from ._lib import C

__all__ = [
    "embed_scaled", "gemv", "gemv_residual", "lm_head_gemv", "rmsnorm",
    "rmsnorm_gemv", "rmsnorm_gemv_pair", "rmsnorm_gemv_swiglu", "rope_attend",
]

BF16 = torch.bfloat16


def _like(ref: torch.Tensor, n: int, out, dtype=None):
    if out is not None:
        return out
    return torch.empty(n, device=ref.device, dtype=dtype or ref.dtype)


def _i32(v, device) -> torch.Tensor:
    if isinstance(v, torch.Tensor) and v.dtype == torch.int32 and v.device == device:
        return v.reshape(1)
    return torch.as_tensor(v, dtype=torch.int32).reshape(1).to(device)


def _bf16_scalar(v, device) -> torch.Tensor:
    if isinstance(v, torch.Tensor) and v.dtype == BF16 and v.device == device:
        return v.reshape(1)
    return torch.as_tensor(v).to(BF16).reshape(1).to(device)


def rmsnorm(x, gamma, eps, out=None):
    """``bf16(bf16(x * rsqrt(mean x^2 + eps)) * gamma)`` (reference_ops.py:31-43)."""
    out = _like(x, x.numel(), out)
    C.rms_norm(x, gamma, out, float(eps), 0)
    return out


def rmsnorm_gemv(x, gamma, w, eps, out=None, plan=None):
    """``rms_norm(x, gamma) @ w.T``, w ``(out, in)`` (reference_ops.py:46-48)."""
    out = _like(x, w.shape[0], out)
    C.rmsnorm_gemv(x, gamma, float(eps), w, out)
    return out


def rmsnorm_gemv_pair(x1, g1, w1, x2, g2, w2, eps, out1=None, out2=None):
    """Two independent ``rmsnorm_gemv`` (reference_ops.py:51-54)."""
    return (rmsnorm_gemv(x1, g1, w1, eps, out1), rmsnorm_gemv(x2, g2, w2, eps, out2))


def gemv(x, w, out=None, plan=None):
    """``x @ w.T`` landed in bf16 (reference_ops.py:57-58)."""
    out = _like(x, w.shape[0], out)
    C.gemv(x, w, out)
    return out


def gemv_residual(x, w, residual, alpha, out=None, plan=None):
    """``residual + bf16(x @ w.T) * alpha``, each step in bf16 (reference_ops.py:61-63)."""
    out = _like(x, w.shape[0], out)
    C.gemv_residual(x, w, residual, _bf16_scalar(alpha, x.device), out)
    return out


def rmsnorm_gemv_swiglu(x, gamma, w_gate, w_up, eps, out=None):
    """``silu(n @ w_gate.T) * (n @ w_up.T)`` for ``n = rms_norm(x, gamma)``
    (reference_ops.py:66-69)."""
    out = _like(x, w_gate.shape[0], out)
    C.rmsnorm_gemv_gate_up(x, gamma, float(eps), w_gate, w_up, out)
    return out


def embed_scaled(table, token, scale, out=None):
    """``table[token] * scale`` landed in bf16; the token id stays on the device
    (reference_ops.py:72-75)."""
    out = _like(table, table.shape[1], out)
    ids = token.reshape(1)
    if ids.dtype != torch.int64:
        ids = ids.to(torch.int64)
    C.embed(table, ids, out, float(scale), None)
    return out


def lm_head_gemv(hidden, w_head, divisor, out=None):
    """``bf16(hidden / divisor) @ w_head.T``, w_head ``(vocab, hidden)``; a divide,
    not a reciprocal multiply (reference_ops.py:78-84)."""
    out = _like(hidden, w_head.shape[0], out)
    C.lm_head_gemv(hidden, w_head, float(divisor), out)
    return out


_WS: dict = {}


def _workspace(device, ns: int, heads: int, v_dim: int):
    key = (device, ns, heads, v_dim)
    ws = _WS.get(key)
    if ws is None:
        n = max(ns, 1)
        ws = (torch.empty(n * heads * v_dim, device=device, dtype=torch.float32),
              torch.empty(n * heads, device=device, dtype=torch.float32),
              torch.empty(n * heads, device=device, dtype=torch.float32))
        _WS[key] = ws
    return ws


def rope_attend(q_up, kv_up, k_rope, cos, sin, pos, k_cache, v_cache, ctx, scale,
                heads, nope, rope, v_dim, attn=None, k_new=None, v_new=None):
    """Rotate, assemble and attend the cache together with this token
    (reference_ops.py:87-130). ``k_cache`` / ``v_cache`` are ``(capacity, heads, .)``
    with their first ``ctx`` rows context; ``pos`` and ``ctx`` are one-element
    device tensors. Returns ``(attn, k_new, v_new)`` flattened."""
    dev = q_up.device
    qk = nope + rope
    attn = _like(q_up, heads * v_dim, attn)
    k_new = _like(q_up, heads * qk, k_new)
    v_new = _like(q_up, heads * v_dim, v_new)
    cap = k_cache.numel() // (heads * qk)
    ns = int(C.rope_attend_splits(cap))
    op, mp, lp = _workspace(dev, ns, heads, v_dim)
    kc = k_cache.reshape(-1) if cap else torch.empty(0, device=dev, dtype=BF16)
    vc = v_cache.reshape(-1) if cap else torch.empty(0, device=dev, dtype=BF16)
    C.rope_attend(q_up.reshape(-1), kv_up.reshape(-1), k_rope.reshape(-1), cos, sin,
                  _i32(pos, dev), kc, vc, _i32(ctx, dev), _bf16_scalar(scale, dev),
                  int(heads), int(nope), int(rope), int(v_dim),
                  op[: ns * heads * v_dim], mp[: ns * heads], lp[: ns * heads],
                  attn, k_new, v_new, None)
    return attn, k_new, v_new
