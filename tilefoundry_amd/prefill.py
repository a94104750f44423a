"""The Qwen3.5 full-attention layer over a whole prompt, in the reference's
signatures, on the gfx950 prefill kernels.

``Attention`` mirrors ``Attention`` of examples/qwen3_8_27b_prefill-tilelang/model.py:263-333
(``qkv``, ``attention``, ``o_proj``; its kernels are kernels/gemm.py:193-300 and
kernels/attention.py:313-438):

* ``qkv`` -- one MFMA GEMM of the normed hidden state against ``[W_q; W_k; W_v]``
  (the q projection holds ``[q | gate]`` per head) into one packed buffer, with
  the head norm and RoPE in its epilogue: per-head RMSNorm with ``(1 + gamma)``
  in f32 landing once, rotate-half RoPE on the leading ``rot`` dims with each
  product and the sum in bf16. ``q``, ``gate``, ``k``, ``v`` come back as
  strided views of that buffer (nothing is copied out).
* ``attention`` -- causal GQA flash attention (f32 scores scaled after the dot,
  online f32 softmax, bf16 weights into P.V) with the output gate
  ``bf16(o) * bf16(sigmoid(gate))``.
* ``o_proj`` -- ``bf16(hidden + bf16(gated @ W_o^T))`` as the GEMM's epilogue.

Weights are ``(out, in)`` (``b_layout="NK"`` in the reference). Token counts are
multiples of 128 (the attention's row block); activations are ``[1, N, .]`` bf16.
"""
from __future__ import annotations

from dataclasses import dataclass

import torch

from ._lib import C

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
    def scale(self) -> float:
        return self.head_dim ** -0.5


def rope_tables(n: int, cfg: PrefillConfig = PrefillConfig(), device=None):
    """cos / sin ``[n, rot]`` bf16 (model.py:404-417): f32 phases over the leading
    ``rot`` dims, ``cat(f, f)``, landed in bf16."""
    inv = 1.0 / (cfg.rope_theta ** (torch.arange(0, cfg.rot, 2, dtype=torch.int64).float() / cfg.rot))
    ph = torch.arange(n).float()[:, None] * inv[None, :]
    ph = torch.cat((ph, ph), dim=-1)
    return ph.cos().to(BF16).to(device), ph.sin().to(BF16).to(device)


class Attention:
    """``Qwen3_5Attention`` over a whole prompt: causal, gated output."""

    def __init__(self, cfg: PrefillConfig = PrefillConfig()):
        self.cfg = cfg
        self._w_qkv = {}

    def _stacked(self, w_q, w_k, w_v):
        key = (w_q.data_ptr(), w_k.data_ptr(), w_v.data_ptr())
        hit = self._w_qkv.get(key)
        if hit is None or hit[0] is not w_q or hit[1] is not w_k or hit[2] is not w_v:
            hit = (w_q, w_k, w_v, torch.cat([w_q, w_k, w_v], 0).contiguous())
            self._w_qkv = {key: hit}
        return hit[3]

    def qkv(self, hn, cos, sin, w_q, w_k, w_v, gamma_q, gamma_k):
        """hn ``[1, N, H]`` -> ``(q, gate [1, N, HQ, D], k, v [1, N, HKV, D])``
        (model.py:271-303)."""
        cfg = self.cfg
        HQ, HKV, D = cfg.heads, cfg.kv_heads, cfg.head_dim
        x = hn.reshape(-1, cfg.hidden)
        N = x.shape[0]
        if N % 128:
            raise ValueError(f"N={N} tokens: the prefill attention takes multiples of 128")
        if cos.shape != (N, cfg.rot) or sin.shape != (N, cfg.rot):
            raise ValueError(f"cos / sin: expected ({N}, {cfg.rot})")
        width = HQ * 2 * D + 2 * HKV * D
        buf = torch.empty(N, width, device=x.device, dtype=BF16)
        C.qkv_norm_rope(x, self._stacked(w_q, w_k, w_v), buf, HQ, HKV, gamma_q, gamma_k, cfg.eps,
                        cos, sin)
        qg = buf[:, : HQ * 2 * D].view(N, HQ, 2 * D)
        k0 = HQ * 2 * D
        k = buf[:, k0: k0 + HKV * D].view(N, HKV, D)
        v = buf[:, k0 + HKV * D:].view(N, HKV, D)
        return (qg[:, :, :D].unsqueeze(0), qg[:, :, D:].unsqueeze(0), k.unsqueeze(0),
                v.unsqueeze(0))

    def attention(self, q, k, v, gate):
        """Causal GQA attention with the output gate -> ``[1, N, HQ * D]``
        (model.py:305-324)."""
        cfg = self.cfg
        N = q.shape[1]
        out = torch.empty(N, cfg.heads * cfg.head_dim, device=q.device, dtype=BF16)
        C.prefill_attention(q[0], k[0], v[0], gate[0], out, cfg.scale)
        return out.unsqueeze(0)

    def o_proj(self, gated, hidden, w_o):
        """``bf16(hidden + bf16(gated @ W_o^T))`` -> ``[1, N, H]`` (model.py:326-333)."""
        cfg = self.cfg
        g = gated.reshape(-1, cfg.heads * cfg.head_dim)
        h = hidden.reshape(-1, cfg.hidden)
        out = torch.empty(g.shape[0], cfg.hidden, device=g.device, dtype=BF16)
        C.gemm_nt(g, w_o, out, h)
        return out.unsqueeze(0)
