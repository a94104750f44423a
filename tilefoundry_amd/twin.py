"""The decode layers in the reference's own signatures, on the gfx950 kernels.

The captured engines (``qwen3.Engine``, ``minicpm3.MLABlock``) are the fast
path; their caches have a fixed capacity and their steps read the position
from device memory. This module exposes the same kernels under the authored
modules' contract instead, so a caller of the reference's layer / root API can
switch over and a parity check can compare function by function:

* ``LayerTwin`` -- ``Qwen3_1_7B_DecoderLayer`` (examples/qwen3_1_7b-tilelang/ref_src/model.py:121-265;
  the reference's runtime twin is fast/twin.py:113-200): ``input_rms_norm``,
  ``self_attention``, ``mlp``, ``decoder_layer``. A prior cache of ``ctx_len``
  positions comes in, this step's own key and value go out.
* ``RootTwin`` -- ``Qwen3_1_7B`` (ref_src/model.py:268-383): ``embed``,
  ``final_rms_norm``, ``lm_head``, ``forward``, ``decode_hidden``,
  ``append_cache``, ``init_caches``, ``prepare_inputs_for_generation``, and the
  ``layers`` list.
* ``MiniCPM3LayerTwin`` -- ``MiniCPM3_4B_DecoderLayer``
  (examples/minicpm3_4b-cutedsl/model.py:187-340; runtime twin
  runtime_model.py:146-250): ``input_rms_norm``, ``mla_attention``, ``mlp``,
  ``decoder_layer`` on the ``reference_ops`` kernels.

Weights: every method takes the weights its authored ``@func`` takes. A matrix
given in the authored ``ConstTensor`` shape ``[1, in, out]`` is read through its
transpose (free when it is a transposed view of an ``(out, in)`` tensor,
otherwise copied once and kept for as long as the caller's tensor lives); a 2-D
matrix is taken as the checkpoint's ``(out, in)`` layout. A twin built with
``weights=`` (checkpoint names, as ``qwen3.hf_names`` lists them) also answers
the activation-only call ``layer(hidden, cos, sin, pos_ids, k_cache, v_cache,
scale)`` the root makes, like a runtime module with its parameters bound.

Departures from the authored HIR, both toward the published model: the
attention scale multiplies the f32 dot (the HIR scales q in bf16 first), and
the softmax weights land in bf16 before the value product -- the order of the
reference's own kernels (fast/kernels.py:343-348,476-479,484-488).
"""
from __future__ import annotations

import weakref

import torch

from ._lib import C
from . import reference_ops as R
from .qwen3 import QWEN3_1_7B, Qwen3Config, hf_names, rope_tables

BF16 = torch.bfloat16
SPLIT = 256  # context slots per attention split in the twins


# ------------------------------------------------------------------ weights
class _Packed:
    """Derived weight layouts, remembered per source tensor (by identity, for as
    long as the source lives)."""

    def __init__(self):
        self._memo: dict = {}

    def get(self, srcs: tuple, build):
        key = tuple(id(t) for t in srcs)
        hit = self._memo.get(key)
        if hit is not None and all(r() is t for r, t in zip(hit[0], srcs)):
            return hit[1]
        val = build()
        memo = self._memo

        def drop(_ref, key=key):
            memo.pop(key, None)

        memo[key] = (tuple(weakref.ref(t, drop) for t in srcs), val)
        return val


_PACKED = _Packed()


def _transposed(w: torch.Tensor, t: torch.Tensor) -> torch.Tensor:
    """``t`` (a transpose of the caller's ``w``) as a contiguous matrix: itself
    when it already is, else a copy kept while ``w`` lives."""
    return t if t.is_contiguous() else _PACKED.get((w,), lambda: t.contiguous())


def out_in(w: torch.Tensor) -> torch.Tensor:
    """A projection matrix as contiguous ``(out, in)``: ``[1, in, out]`` (the
    authored shape) is transposed, 2-D is taken as ``(out, in)``."""
    if w.dim() == 3:
        if w.shape[0] != 1:
            raise ValueError(f"expected a [1, in, out] weight, got {tuple(w.shape)}")
        return _transposed(w, w[0].t())
    if w.dim() != 2:
        raise ValueError(f"expected a 2-D (out, in) or [1, in, out] weight, got {tuple(w.shape)}")
    return w if w.is_contiguous() else _PACKED.get((w,), lambda: w.contiguous())


def _rms_row(hidden, gamma, eps: float) -> torch.Tensor:
    H = gamma.numel()
    out = torch.empty(H, device=hidden.device, dtype=BF16)
    C.rms_norm(_vec(hidden), gamma, out, float(eps), 0)
    return out.reshape(1, 1, H)


def _stacked(*ws: torch.Tensor) -> torch.Tensor:
    """``[w_0; w_1; ...]`` in (out, in) rows: the one matrix a fused projection reads."""
    return _PACKED.get(ws, lambda: torch.cat([out_in(w) for w in ws], 0).contiguous())


def _vec(x: torch.Tensor) -> torch.Tensor:
    return x.reshape(-1) if x.is_contiguous() else x.contiguous().reshape(-1)


def _i32(v, device) -> torch.Tensor:
    if isinstance(v, torch.Tensor) and v.dtype == torch.int32 and v.device == device:
        return v.reshape(-1)[:1]
    return torch.as_tensor(v).reshape(-1)[:1].to(device=device, dtype=torch.int32)


def _scale(scale) -> float:
    return float(scale.reshape(-1)[0]) if isinstance(scale, torch.Tensor) else float(scale)


# -------------------------------------------------------------------- Qwen3
class LayerTwin:
    """One Qwen3 decoder layer in the reference's signatures."""

    _LAYER_NAMES = ("gamma_in", "w_q", "w_k", "w_v", "gamma_q", "gamma_k", "w_o", "gamma_post",
                    "w_gate", "w_up", "w_down")

    def __init__(self, cfg: Qwen3Config = QWEN3_1_7B, weights: dict | None = None):
        self.cfg = cfg
        self._bound = dict(weights) if weights is not None else None

    # ---------------------------------------------------------------- pieces
    def input_rms_norm(self, hidden, gamma_in):
        """``bf16(bf16(x * rsqrt(mean x^2 + eps)) * gamma_in)`` (model.py:123-136)."""
        return _rms_row(hidden, gamma_in, self.cfg.eps)

    def _attend(self, hidden, gamma_in, w_q, w_k, w_v, gamma_q, gamma_k, cos_cache, sin_cache,
                pos_ids, k_cache, v_cache, scale, w_o, residual):
        cfg = self.cfg
        H, HQ, HKV, D = cfg.hidden, cfg.heads, cfg.kv_heads, cfg.head_dim
        dev = hidden.device
        ctx = int(k_cache.shape[1])
        cap = max(SPLIT, -(-(ctx + 1) // SPLIT) * SPLIT)
        ns = cap // SPLIT
        KN = HKV * D
        # the scratch cache: prior context, this step's entry written at slot ctx;
        # zeroed so that slots past the end hold finite values
        kc = torch.zeros(cap, KN, device=dev, dtype=BF16)
        vc = torch.zeros(cap, KN, device=dev, dtype=BF16)
        if ctx:
            kc[:ctx] = k_cache.reshape(ctx, KN)
            vc[:ctx] = v_cache.reshape(ctx, KN)
        write = torch.full((1,), ctx, device=dev, dtype=torch.int32)
        pos = _i32(pos_ids, dev)
        n_qk = (HQ + HKV) * D
        qk = torch.empty(n_qk, device=dev, dtype=BF16)
        C.decode_qkv(_vec(hidden), None, None, None, gamma_in, cfg.eps, _stacked(w_q, w_k, w_v),
                     n_qk, qk, write, vc, None)
        op = torch.empty(ns, HQ, D, device=dev, dtype=torch.float32)
        mp = torch.empty(ns, HQ, device=dev, dtype=torch.float32)
        lp = torch.empty(ns, HQ, device=dev, dtype=torch.float32)
        C.decode_attention(qk, None, gamma_q, gamma_k, cfg.eps, cos_cache, sin_cache, kc, vc, pos,
                           write, HQ, HKV, SPLIT, _scale(scale), op, mp, lp, False, None)
        attn = torch.empty(HQ * D, device=dev, dtype=BF16)
        C.attn_combine(op, mp, lp, attn, write, SPLIT)
        out = torch.empty(H, device=dev, dtype=BF16)
        if residual is None:
            C.gemv(attn, out_in(w_o), out)
        else:
            C.gemv_residual(attn, out_in(w_o), _vec(residual), None, out)
        k_new = kc[ctx].reshape(1, 1, HKV, D).clone()
        v_new = vc[ctx].reshape(1, 1, HKV, D).clone()
        return out.reshape(1, 1, H), k_new, v_new

    def self_attention(self, hidden, gamma_in, w_q, w_k, w_v, gamma_q, gamma_k, cos_cache,
                       sin_cache, pos_ids, k_cache, v_cache, scale, w_o):
        """Input norm + q|k|v + q/k head norm + RoPE + GQA attention over the prior
        cache and this token + o_proj (model.py:138-215). Returns ``(out, k_new,
        v_new)`` with this step's entry ``[1, 1, HKV, D]`` for the caller to append."""
        return self._attend(hidden, gamma_in, w_q, w_k, w_v, gamma_q, gamma_k, cos_cache,
                            sin_cache, pos_ids, k_cache, v_cache, scale, w_o, None)

    def _mlp(self, hidden, gamma_post, w_gate, w_up, w_down, residual):
        cfg = self.cfg
        dev = hidden.device
        act = torch.empty(cfg.inter, device=dev, dtype=BF16)
        C.rmsnorm_gemv_gate_up(_vec(hidden), gamma_post, cfg.eps, out_in(w_gate), out_in(w_up), act)
        out = torch.empty(cfg.hidden, device=dev, dtype=BF16)
        if residual is None:
            C.gemv(act, out_in(w_down), out)
        else:
            C.gemv_residual(act, out_in(w_down), _vec(residual), None, out)
        return out.reshape(1, 1, cfg.hidden)

    def mlp(self, hidden, gamma_post, w_gate, w_up, w_down):
        """Post-attention norm + SwiGLU + down (model.py:217-233), no residual."""
        return self._mlp(hidden, gamma_post, w_gate, w_up, w_down, None)

    def decoder_layer(self, hidden, gamma_in, w_q, w_k, w_v, gamma_q, gamma_k, cos_cache,
                      sin_cache, pos_ids, k_cache, v_cache, scale, w_o, gamma_post, w_gate, w_up,
                      w_down):
        """``h1 = hidden + self_attention(...)``; ``h1 + mlp(h1)`` (model.py:235-265).
        Each residual add is the epilogue of its projection; ``bf16(a + bf16(b))``
        is the same value either way."""
        h1, k_new, v_new = self._attend(hidden, gamma_in, w_q, w_k, w_v, gamma_q, gamma_k,
                                        cos_cache, sin_cache, pos_ids, k_cache, v_cache, scale,
                                        w_o, hidden)
        return self._mlp(h1, gamma_post, w_gate, w_up, w_down, h1), k_new, v_new

    # ---------------------------------------------------------- bound call
    def __call__(self, hidden, cos_cache, sin_cache, pos_ids, k_cache, v_cache, scale):
        """``decoder_layer`` with the bound weights: the activation-only call a
        runtime module answers."""
        if self._bound is None:
            raise TypeError("this LayerTwin has no bound weights; call decoder_layer(...) with them")
        b = self._bound
        return self.decoder_layer(hidden, b["gamma_in"], b["w_q"], b["w_k"], b["w_v"],
                                  b["gamma_q"], b["gamma_k"], cos_cache, sin_cache, pos_ids,
                                  k_cache, v_cache, scale, b["w_o"], b["gamma_post"], b["w_gate"],
                                  b["w_up"], b["w_down"])


def bind_layer(weights: dict, i: int) -> dict:
    """Layer ``i``'s parameters under the authored names, from checkpoint names."""
    names = hf_names(i)
    try:
        return {k: weights[names[k]] for k in LayerTwin._LAYER_NAMES}
    except KeyError as exc:
        raise KeyError(f"layer {i}: checkpoint weight {exc.args[0]} missing") from None


class RootTwin:
    """The layer stack and the step around it (ref_src/model.py:268-383)."""

    def __init__(self, cfg: Qwen3Config = QWEN3_1_7B, weights: dict | None = None, device=None):
        self.cfg = cfg
        self.device = torch.device(device) if device is not None else None
        self.layers = [LayerTwin(cfg, bind_layer(weights, i) if weights is not None else None)
                       for i in range(cfg.layers)]
        self._bound = None
        if weights is not None:
            try:
                emb = weights["model.embed_tokens.weight"]
                self._bound = {"w_embed": emb, "gamma_final": weights["model.norm.weight"],
                               "w_head": weights.get("lm_head.weight", emb)}
            except KeyError as exc:
                raise KeyError(f"checkpoint weight {exc.args[0]} missing") from None
        self._rope = {}

    # ---------------------------------------------------------------- pieces
    def embed(self, w_embed, token_ids):
        """``w_embed[token_ids]`` -> ``[1, 1, H]`` (model.py:275-283)."""
        ids = token_ids.reshape(-1)[:1]
        if ids.dtype != torch.int64:
            ids = ids.to(torch.int64)
        out = torch.empty(self.cfg.hidden, device=w_embed.device, dtype=BF16)
        C.embed(w_embed, ids, out, None, None)
        return out.reshape(1, 1, self.cfg.hidden)

    def final_rms_norm(self, hidden, gamma_final):
        """The norm after the last layer (model.py:285-294)."""
        return _rms_row(hidden, gamma_final, self.cfg.eps)

    def lm_head(self, hidden, w_head):
        """Logits ``[1, V]``: f32 dots landed in bf16 (model.py:296-301). ``w_head``
        is ``[H, V]`` (authored) or the ``(V, H)`` table (tied)."""
        H = self.cfg.hidden
        if w_head.dim() == 2 and w_head.shape[0] == H and w_head.shape[1] != H:
            w = _transposed(w_head, w_head.t())
        else:
            w = out_in(w_head)
        V = w.shape[0]
        dev = hidden.device
        logits = torch.empty(V, device=dev, dtype=torch.float32)
        nb = C.lm_head_blocks(V)
        bv = torch.empty(nb, device=dev, dtype=torch.float32)
        bi = torch.empty(nb, device=dev, dtype=torch.int32)
        C.lm_head_argmax(_vec(hidden), None, 0.0, w, logits, bv, bi)
        return logits.to(BF16).reshape(1, V)

    # ----------------------------------------------------------- orchestration
    def _b(self):
        if self._bound is None:
            raise TypeError("this RootTwin has no bound weights")
        return self._bound

    def forward(self, token_ids, cos_cache, sin_cache, pos_ids, scale, caches):
        """Embed, every layer, final norm, logits; returns ``(logits, entries)``
        with each layer's own fresh ``(k_new, v_new)`` (model.py:303-313)."""
        b = self._b()
        hidden = self.embed(b["w_embed"], token_ids)
        normed, entries = self.decode_hidden(hidden, cos_cache, sin_cache, pos_ids, scale, caches)
        return self.lm_head(normed, b["w_head"]), entries

    def decode_hidden(self, hidden, cos_cache, sin_cache, pos_ids, scale, caches):
        """One step through every layer, then the final norm (model.py:315-333)."""
        if len(caches) != len(self.layers):
            raise ValueError(f"decoder has {len(self.layers)} layers but was given "
                             f"{len(caches)} caches")
        entries = []
        for layer, (k_cache, v_cache) in zip(self.layers, caches):
            hidden, k_new, v_new = layer(hidden, cos_cache, sin_cache, pos_ids, k_cache, v_cache,
                                         scale)
            entries.append((k_new, v_new))
        return self.final_rms_norm(hidden, self._b()["gamma_final"]), tuple(entries)

    def append_cache(self, caches, fresh):
        """Each layer's context with this step's entry after it (model.py:335-348)."""
        return tuple((torch.cat([k, kn], dim=1), torch.cat([v, vn], dim=1))
                     for (k, v), (kn, vn) in zip(caches, fresh))

    def init_caches(self, device=None):
        """Zero-length ``[1, 0, HKV, D]`` caches, one pair per layer (model.py:350-369)."""
        dev = torch.device(device) if device is not None else (self.device or torch.device("cuda"))
        empty = (1, 0, self.cfg.kv_heads, self.cfg.head_dim)
        return tuple((torch.zeros(empty, device=dev, dtype=BF16),
                      torch.zeros(empty, device=dev, dtype=BF16)) for _ in self.layers)

    def _tables(self, dev):
        t = self._rope.get(dev)
        if t is None:
            t = rope_tables(self.cfg.max_pos, self.cfg.head_dim, self.cfg.rope_theta, dev)
            self._rope[dev] = t
        return t

    def prepare_inputs_for_generation(self, input_ids, step, caches, device=None):
        """``(token_ids, cos_cache, sin_cache, pos_ids, scale, caches)`` for one
        step (model.py:371-383): the rope tables over ``max_position_embeddings``,
        the position ``step``, ``scale = bf16(D^-1/2)``."""
        dev = torch.device(device) if device is not None else (self.device or torch.device("cuda"))
        token_ids = input_ids[step].reshape(1).to(device=dev, dtype=torch.int64)
        cos, sin = self._tables(dev)
        pos_ids = torch.tensor([step], device=dev, dtype=torch.int32)
        scale = torch.full((1, 1, 1, 1), self.cfg.head_dim ** -0.5, device=dev, dtype=BF16)
        return token_ids, cos, sin, pos_ids, scale, caches


# ----------------------------------------------------------------- MiniCPM3
class MiniCPM3LayerTwin:
    """One MiniCPM3 MLA decoder layer in the reference's signatures, on the
    ``reference_ops`` kernels (non-absorbed attention over the assembled cache)."""

    def __init__(self, cfg=None, inter: int = 6400):
        from .minicpm3 import MiniCPM3Config  # noqa: PLC0415

        self.cfg = cfg or MiniCPM3Config()
        self.inter = inter

    def input_rms_norm(self, hidden, gamma_in):
        """Input norm, eps = rms_norm_eps (model.py:188-203)."""
        H = self.cfg.hidden
        return R.rmsnorm(_vec(hidden), gamma_in, self.cfg.eps).reshape(1, 1, H)

    def _attend(self, hidden, gamma_in, w_q_a, gamma_q_a, w_q_b, w_kv_a, gamma_kv_a, w_kv_b,
                cos_cache, sin_cache, pos_ids, k_cache, v_cache, scale, w_o, residual, alpha):
        cfg = self.cfg
        H, NH, QL, KL, QK, VD = cfg.hidden, cfg.heads, cfg.q_lora, cfg.kv_lora, cfg.qk_dim, cfg.v_dim
        dev = hidden.device
        lora = R.rmsnorm_gemv(_vec(hidden), gamma_in, _stacked(w_q_a, w_kv_a), cfg.eps)
        q_up, kv_up = R.rmsnorm_gemv_pair(lora[:QL], gamma_q_a, out_in(w_q_b),
                                          lora[QL:QL + KL], gamma_kv_a, out_in(w_kv_b),
                                          cfg.lora_eps)
        ctx = int(k_cache.shape[1]) if k_cache.dim() == 4 else int(k_cache.shape[0])
        ctx_t = torch.full((1,), ctx, device=dev, dtype=torch.int32)
        attn, k_new, v_new = R.rope_attend(
            q_up, kv_up, lora[QL + KL:QL + KL + cfg.rope], cos_cache, sin_cache,
            _i32(pos_ids, dev), k_cache.reshape(-1, NH, QK), v_cache.reshape(-1, NH, VD), ctx_t,
            scale, NH, cfg.nope, cfg.rope, VD)
        if residual is None:
            out = R.gemv(attn, out_in(w_o))
        else:
            out = R.gemv_residual(attn, out_in(w_o), _vec(residual), alpha)
        return out.reshape(1, 1, H), k_new.reshape(1, 1, NH, QK), v_new.reshape(1, 1, NH, VD)

    def mla_attention(self, hidden, gamma_in, w_q_a, gamma_q_a, w_q_b, w_kv_a, gamma_kv_a,
                      w_kv_b, cos_cache, sin_cache, pos_ids, k_cache, v_cache, scale, w_o):
        """Input norm + MLA over the prior cache and this token + o_proj, no
        residual (model.py:205-291). Returns ``(out, k_new [1,1,heads,96],
        v_new [1,1,heads,64])``."""
        return self._attend(hidden, gamma_in, w_q_a, gamma_q_a, w_q_b, w_kv_a, gamma_kv_a, w_kv_b,
                            cos_cache, sin_cache, pos_ids, k_cache, v_cache, scale, w_o, None, None)

    def _mlp(self, hidden, gamma_post, w_gate, w_up, w_down, residual, alpha):
        act = R.rmsnorm_gemv_swiglu(_vec(hidden), gamma_post, out_in(w_gate), out_in(w_up),
                                    self.cfg.eps)
        if residual is None:
            out = R.gemv(act, out_in(w_down))
        else:
            out = R.gemv_residual(act, out_in(w_down), _vec(residual), alpha)
        return out.reshape(1, 1, self.cfg.hidden)

    def mlp(self, hidden, gamma_post, w_gate, w_up, w_down):
        """Post-attention norm + SwiGLU + down, no residual (model.py:293-308)."""
        return self._mlp(hidden, gamma_post, w_gate, w_up, w_down, None, None)

    def decoder_layer(self, hidden, gamma_in, w_q_a, gamma_q_a, w_q_b, w_kv_a, gamma_kv_a, w_kv_b,
                      cos_cache, sin_cache, pos_ids, k_cache, v_cache, scale, w_o, gamma_post,
                      w_gate, w_up, w_down, residual_scale):
        """``h1 = hidden + attn * residual_scale``; ``h1 + mlp(h1) * residual_scale``,
        each residual folded into its projection's epilogue (model.py:310-340)."""
        h1, k_new, v_new = self._attend(hidden, gamma_in, w_q_a, gamma_q_a, w_q_b, w_kv_a,
                                        gamma_kv_a, w_kv_b, cos_cache, sin_cache, pos_ids, k_cache,
                                        v_cache, scale, w_o, hidden, residual_scale)
        return self._mlp(h1, gamma_post, w_gate, w_up, w_down, h1, residual_scale), k_new, v_new
