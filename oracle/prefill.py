"""Causal GQA prefill attention layer (Qwen3.5-family full-attention layer at
Qwen3.8-27B shapes), restated on the CPU -- test infrastructure only.

What each function follows (jingchangshi/TileFoundry):

* ``rope_tables`` -- examples/qwen3_8_27b_prefill-tilelang/model.py:404-417: the plain
  rotary frequencies over the leading ``rot = head_dim * partial_rotary_factor``
  = 64 dims, theta 1e7, ``cat(f, f)``, cos / sin landed in bf16.
* ``qkv`` -- ``Attention.qkv``, model.py:271-303: one projection of width
  ``heads * 2 * head_dim`` holding per head ``[q | gate]``; q and k each get the
  Qwen3.5 RMSNorm (``x * rsqrt(mean x^2 + eps) * (1 + gamma)`` in f32, one bf16
  landing -- the HIR ``rms_norm`` eval rule, src/tilefoundry/ir/hir/nn/rms_norm.py:99-106);
  then rotate-half RoPE on the leading 64 dims with each product and the sum
  landing in bf16; v and the gate pass through.
* ``attention`` -- ``Attention.attention``, model.py:305-324: f32 scores (bf16
  operands, f32 accumulate) times ``head_dim^-1/2``, causal mask, f32 softmax,
  probabilities landed in bf16 for the value product (f32 accumulate, bf16
  result), then ``attn * sigmoid(gate)`` in bf16.
* ``o_proj`` -- model.py:326-333: ``bf16(hidden + bf16(gated @ W_o^T))``.

Weights are ``(out, in)``. Pinned by (tests/test_oracle.py): causal-prefix
invariance (rows before m do not change when later rows do), a one-row prompt
returning ``bf16(v * sigmoid(gate))``, identical keys returning the running
mean of the values, an f64 brute force of the attention on a tiny shape, the
rope tables against the closed form and a planted mistake (a non-causal
softmax changes row 0).
"""
from __future__ import annotations

from dataclasses import dataclass

import torch

from .norms import rms_norm_1p

BF16 = torch.bfloat16


@dataclass(frozen=True)
class PrefillConfig:
    """examples/qwen3_8_27b_prefill-tilelang/config.json (text_config, full attention)."""

    hidden: int = 5120
    heads: int = 24
    kv_heads: int = 4
    head_dim: int = 256
    rot: int = 64            # head_dim * partial_rotary_factor (0.25)
    eps: float = 1e-6
    rope_theta: float = 1.0e7

    @property
    def group(self) -> int:
        return self.heads // self.kv_heads

    @property
    def scale(self) -> float:
        return self.head_dim ** -0.5


def rope_tables(n: int, cfg: PrefillConfig = PrefillConfig()):
    inv = 1.0 / (cfg.rope_theta ** (torch.arange(0, cfg.rot, 2, dtype=torch.int64).float() / cfg.rot))
    freqs = torch.arange(n).float()[:, None] * inv[None, :]
    emb = torch.cat((freqs, freqs), dim=-1)
    return emb.cos().to(BF16), emb.sin().to(BF16)


def rope_partial(x: torch.Tensor, c: torch.Tensor, s: torch.Tensor, rot: int) -> torch.Tensor:
    """Rotate-half on ``x[..., :rot]`` (bf16 products and sum), the rest as is.
    ``c`` / ``s`` broadcast against ``x[..., :rot]``."""
    half = rot // 2
    xr = x[..., :rot]
    xh = torch.cat((-xr[..., half:], xr[..., :half]), dim=-1)
    return torch.cat((xr * c + xh * s, x[..., rot:]), dim=-1)


def proj(x: torch.Tensor, w: torch.Tensor) -> torch.Tensor:
    return (x.float() @ w.float().t()).to(BF16)


def qkv(hn, w_q, w_k, w_v, gamma_q, gamma_k, cos, sin, cfg: PrefillConfig = PrefillConfig()):
    """hn [N, hidden] bf16 -> q, gate [N, heads, D]; k, v [N, kv_heads, D] (bf16)."""
    N, D = hn.shape[0], cfg.head_dim
    qg = proj(hn, w_q).view(N, cfg.heads, 2 * D)
    q = rms_norm_1p(qg[..., :D], gamma_q, cfg.eps)
    gate = qg[..., D:]
    k = rms_norm_1p(proj(hn, w_k).view(N, cfg.kv_heads, D), gamma_k, cfg.eps)
    v = proj(hn, w_v).view(N, cfg.kv_heads, D)
    c, s = cos[:N].view(N, 1, cfg.rot), sin[:N].view(N, 1, cfg.rot)
    return rope_partial(q, c, s, cfg.rot), gate.contiguous(), rope_partial(k, c, s, cfg.rot), v


def attention(q, k, v, gate, cfg: PrefillConfig = PrefillConfig(), heads=None):
    """q, gate [N, heads, D]; k, v [N, kv_heads, D] bf16 -> [N, heads * D] bf16.
    ``heads`` limits the computation to the listed query heads (their columns
    are returned in order, [N, len(heads) * D])."""
    N, H, D = q.shape
    hs = range(H) if heads is None else heads
    causal = torch.ones(N, N, dtype=torch.bool).tril()
    outs = []
    for h in hs:
        g = h // cfg.group
        s = (q[:, h].float() @ k[:, g].float().t()) * cfg.scale
        s = s.masked_fill(~causal, float("-inf"))
        p = torch.softmax(s, dim=-1).to(BF16)
        o = (p.float() @ v[:, g].float()).to(BF16)
        outs.append(o * torch.sigmoid(gate[:, h]))
    return torch.stack(outs, 1).reshape(N, -1)


def attention_rows(q, k, v, gate, rows, heads, cfg: PrefillConfig = PrefillConfig()):
    """:func:`attention` for the listed query rows and heads only: row i (its
    position) attends keys 0..i, in the same operation order. Returns
    ``[len(rows), len(heads), D]`` bf16. For full-length prompts where the
    whole N x N computation would take minutes on the CPU; pinned against
    :func:`attention` on a small prompt (tests/test_oracle.py)."""
    out = torch.empty(len(rows), len(heads), q.shape[-1], dtype=BF16)
    for r, i in enumerate(rows):
        for c, h in enumerate(heads):
            kv = h // cfg.group
            s = (q[i, h].float().unsqueeze(0) @ k[: i + 1, kv].float().t()) * cfg.scale
            p = torch.softmax(s, dim=-1).to(BF16)
            o = (p.float() @ v[: i + 1, kv].float()).to(BF16)
            out[r, c] = o[0] * torch.sigmoid(gate[i, h])
    return out


def o_proj(gated, hidden, w_o):
    """``bf16(hidden + bf16(gated . W_o^T))``: the product lands, then the
    residual add lands (examples/qwen3_8_27b_prefill-tilelang/model.py:326-333).
    Pinned with a non-zero hidden state against its f64 statement and a
    hand-worked known answer that one landing fails (tests/test_oracle.py)."""
    return hidden.to(BF16) + proj(gated, w_o)


def random_layer(cfg: PrefillConfig, seed: int = 0, std: float = 0.02):
    g = torch.Generator().manual_seed(seed)

    def w(*shape):
        return (std * torch.randn(*shape, generator=g)).to(BF16)

    D = cfg.head_dim
    return {
        "w_q": w(cfg.heads * 2 * D, cfg.hidden), "w_k": w(cfg.kv_heads * D, cfg.hidden),
        "w_v": w(cfg.kv_heads * D, cfg.hidden), "w_o": w(cfg.hidden, cfg.heads * D),
        "gamma_q": (0.1 * torch.randn(D, generator=g)).to(BF16),
        "gamma_k": (0.1 * torch.randn(D, generator=g)).to(BF16),
    }
