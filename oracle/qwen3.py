"""Qwen3-1.7B-shaped decode, restated on the CPU -- test infrastructure only.

What each function follows (jingchangshi/TileFoundry):

* ``rope_tables`` -- ``_generation_rope``, examples/qwen3_1_7b-tilelang/ref_src/model.py:106-119
  (inverse frequencies in f32, ``cat(f, f)``, cos / sin landed in bf16).
* ``head_norm`` / ``rope`` -- the torch spelling of ``qk_rope_cache``,
  examples/qwen3_1_7b-tilelang/fast/test_kernels.py:87-92,110-118 (``_rope_ref``,
  ``nrm``): per-head Qwen3RMSNorm, then rotate-half in f32 landing once in bf16.
* ``attend`` -- ``_attn_ref``, examples/qwen3_1_7b-tilelang/fast/test_kernels.py:121-129:
  scores in f32 with the ``1/sqrt(D)`` scale applied after the dot, f32 softmax,
  f32 weighted sum, one landing in bf16. (The authored HIR multiplies the scale
  onto q in bf16 first, ref_src/model.py:182; the kernels and this oracle follow
  the torch spelling, which the reference's f64 arbiter found closer to truth,
  examples/qwen3_1_7b-tilelang/fast/arbitrate.py:22-56.)
* ``proj`` -- every projection ``bf16(x @ W^T)`` with f32 accumulation, the
  evaluator's ``matmul`` rule (src/tilefoundry/ir/hir/nn/matmul.py:183-202).
* ``decoder_layer`` -- ``Qwen3_1_7B_DecoderLayer.decoder_layer``,
  examples/qwen3_1_7b-tilelang/ref_src/model.py:138-265: input norm, q/k/v, q/k
  norm + rope, attention over the prior cache plus this token, o_proj,
  residual; post norm, SwiGLU (``silu`` and the product each landing in bf16,
  fast/kernels.py:237-241), down, residual.
* ``lm_logits`` / ``greedy`` -- f32 logits from the bf16 normed hidden state
  (fast/kernels.py:260-321) and ``torch.argmax`` (lowest index on ties,
  ref_src/generation.py:24-26).
* ``decode`` -- the greedy loop of ref_src/generation.py:41-85 with the cache
  appended each step (ref_src/model.py:335-348).

Weights are ``(out, in)`` -- the checkpoint's own layout (``hf_alias.py``
transposes it for the TileLang engine; the arithmetic is the same).

Pinned by (tests/test_oracle.py): RoPE at position 0 is the identity; the
rotate-half form equals multiplication by e^{i theta} on (x_d, x_{d+D/2}) pairs;
attention over one key returns that key's value, over identical keys the mean
of the values, and matches an f64 brute-force softmax; the projection is exact
on integer-valued inputs; argmax takes the lowest index on planted ties; the
layer keeps causal-prefix invariance (appending a later token does not change
an earlier step's output).
"""
from __future__ import annotations

from dataclasses import dataclass, field

import torch

from .norms import rms_norm_q

BF16 = torch.bfloat16


@dataclass(frozen=True)
class Qwen3Config:
    """Qwen3-1.7B's shape: examples/qwen3_1_7b-tilelang/ref_src/config.json."""

    hidden: int = 2048
    heads: int = 16
    kv_heads: int = 8
    head_dim: int = 128
    inter: int = 6144
    vocab: int = 151936
    layers: int = 28
    eps: float = 1e-6
    rope_theta: float = 1.0e6
    max_pos: int = 40960

    @property
    def scale(self) -> float:
        return self.head_dim ** -0.5


def rope_tables(n: int, head_dim: int, theta: float):
    """cos, sin bf16 ``[n, head_dim]`` (``cat(f, f)`` layout)."""
    inv = 1.0 / (theta ** (torch.arange(0, head_dim, 2, dtype=torch.float32) / head_dim))
    ph = torch.outer(torch.arange(n, dtype=torch.float32), inv)
    ph = torch.cat((ph, ph), dim=-1)
    return ph.cos().to(BF16), ph.sin().to(BF16)


def proj(x: torch.Tensor, w: torch.Tensor) -> torch.Tensor:
    """``bf16(x @ w^T)`` with f32 accumulation; w is ``(out, in)``."""
    return (x.float() @ w.float().t()).to(BF16)


def head_norm(x: torch.Tensor, gamma: torch.Tensor, eps: float) -> torch.Tensor:
    """Qwen3RMSNorm over the last axis (per head)."""
    return rms_norm_q(x, gamma, eps)


def rope(x: torch.Tensor, cos_row: torch.Tensor, sin_row: torch.Tensor) -> torch.Tensor:
    """Rotate-half RoPE of ``x (..., D)`` bf16 at one position; one bf16 landing."""
    D = x.shape[-1]
    xf = x.float()
    half = torch.cat([-xf[..., D // 2:], xf[..., : D // 2]], dim=-1)
    return (xf * cos_row.float() + half * sin_row.float()).to(BF16)


def attend(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, scale: float,
           p_bf16: bool = False) -> torch.Tensor:
    """GQA attention of one position.

    q ``(HQ, D)``, k / v ``(n, HKV, D)`` -> ``(HQ*D,)`` bf16.

    ``p_bf16=False``: f32 throughout (``_attn_ref``,
    examples/qwen3_1_7b-tilelang/fast/test_kernels.py:121-129) -- the per-op bar.
    ``p_bf16=True``: the reference kernel's order (fast/kernels.py:476-501):
    ``e = exp(s - max)`` in f32, ``l = sum(e)`` in f32, the weights landed in bf16
    before the value product, ``o / l`` landed once. This is also Hugging Face's
    own order (bf16 probabilities into P.V); whole-model comparisons use it.
    """
    HQ, D = q.shape
    G = HQ // k.shape[1]
    kk = k.float().repeat_interleave(G, dim=1)
    vv = v.float().repeat_interleave(G, dim=1)
    s = (q.float().unsqueeze(0) * kk).sum(-1) * scale          # (n, HQ)
    if not p_bf16:
        w = torch.softmax(s, dim=0)
        return (w.unsqueeze(-1) * vv).sum(0).to(BF16).reshape(-1)
    e = torch.exp(s - s.max(0).values)
    lsum = e.sum(0)
    o = (e.to(BF16).float().unsqueeze(-1) * vv).sum(0)
    return (o / lsum.unsqueeze(-1)).to(BF16).reshape(-1)


@dataclass
class LayerWeights:
    gamma_in: torch.Tensor
    w_q: torch.Tensor      # (HQ*D, H)
    w_k: torch.Tensor      # (HKV*D, H)
    w_v: torch.Tensor      # (HKV*D, H)
    gamma_q: torch.Tensor
    gamma_k: torch.Tensor
    w_o: torch.Tensor      # (H, HQ*D)
    gamma_post: torch.Tensor
    w_gate: torch.Tensor   # (I, H)
    w_up: torch.Tensor     # (I, H)
    w_down: torch.Tensor   # (H, I)
    f32: dict = field(default_factory=dict, repr=False)

    def w32(self, name: str) -> torch.Tensor:
        """f32 copy of a projection, made once (the oracle's matmuls run in f32)."""
        t = self.f32.get(name)
        if t is None:
            t = getattr(self, name).float()
            self.f32[name] = t
        return t


def _proj(x, lw: LayerWeights, name: str):
    return (x.float() @ lw.w32(name).t()).to(BF16)


def self_attention(h, lw: LayerWeights, cfg: Qwen3Config, cos_row, sin_row, k_cache, v_cache,
                   p_bf16: bool = False):
    """Input norm + attention block for one token. Returns ``(out, k_new, v_new)``.

    h ``(H,)`` bf16; k_cache / v_cache ``(ctx, HKV, D)`` bf16 (prior positions).
    """
    HQ, HKV, D = cfg.heads, cfg.kv_heads, cfg.head_dim
    xn = rms_norm_q(h, lw.gamma_in, cfg.eps)
    q = _proj(xn, lw, "w_q").view(HQ, D)
    k = _proj(xn, lw, "w_k").view(HKV, D)
    v = _proj(xn, lw, "w_v").view(HKV, D)
    q = rope(head_norm(q, lw.gamma_q, cfg.eps), cos_row, sin_row)
    k = rope(head_norm(k, lw.gamma_k, cfg.eps), cos_row, sin_row)
    kk = torch.cat([k_cache, k.unsqueeze(0)], dim=0)
    vv = torch.cat([v_cache, v.unsqueeze(0)], dim=0)
    attn = attend(q, kk, vv, cfg.scale, p_bf16)
    return _proj(attn, lw, "w_o"), k, v


def mlp(h1, lw: LayerWeights, cfg: Qwen3Config):
    xn = rms_norm_q(h1, lw.gamma_post, cfg.eps)
    g = _proj(xn, lw, "w_gate")
    u = _proj(xn, lw, "w_up")
    act = torch.nn.functional.silu(g.float()).to(BF16) * u
    return _proj(act, lw, "w_down")


def decoder_layer(h, lw, cfg, cos_row, sin_row, k_cache, v_cache, p_bf16: bool = False):
    """``h -> (h_out, k_new, v_new)``: attention + residual, mlp + residual."""
    a, k, v = self_attention(h, lw, cfg, cos_row, sin_row, k_cache, v_cache, p_bf16)
    h1 = h + a
    return h1 + mlp(h1, lw, cfg), k, v


def lm_logits(h, gamma_final, w_head32, eps):
    """f32 logits of the final-normed hidden state; ``w_head32`` f32 ``(V, H)``."""
    xn = rms_norm_q(h, gamma_final, eps)
    return xn.float() @ w_head32.t()


def greedy(logits: torch.Tensor) -> int:
    return int(torch.argmax(logits))


@dataclass
class ModelWeights:
    embed: torch.Tensor        # (V, H), tied with the head
    gamma_final: torch.Tensor
    layers: list
    _head32: torch.Tensor | None = None

    def head32(self):
        if self._head32 is None:
            self._head32 = self.embed.float()
        return self._head32


def step(model: ModelWeights, cfg: Qwen3Config, token: int, pos: int, caches, cos, sin,
         p_bf16: bool = False):
    """One decode step of the whole stack; appends to ``caches`` in place.

    Returns the f32 logits."""
    h = model.embed[token].clone()
    for lw, cache in zip(model.layers, caches):
        h, k, v = decoder_layer(h, lw, cfg, cos[pos], sin[pos], cache[0], cache[1], p_bf16)
        cache[0] = torch.cat([cache[0], k.unsqueeze(0)], dim=0)
        cache[1] = torch.cat([cache[1], v.unsqueeze(0)], dim=0)
    return lm_logits(h, model.gamma_final, model.head32(), cfg.eps)


def step_batch(model: ModelWeights, cfg: Qwen3Config, tokens: list[int], positions: list[int],
               caches_b, cos, sin, p_bf16: bool = False):
    """One decode step of ``B`` sequences at once: the same arithmetic as
    :func:`step` for each row (the norms, projections, RoPE and SwiGLU act row by
    row; attention runs per sequence over its own cache), with the projections
    as one ``[B, in]`` matmul. ``caches_b[b]`` is sequence b's per-layer
    ``[k, v]`` list, appended in place. Returns f32 logits ``[B, V]``.

    Pinned against :func:`step` run per sequence (tests/test_oracle.py)."""
    HQ, HKV, D = cfg.heads, cfg.kv_heads, cfg.head_dim
    B = len(tokens)
    h = model.embed[torch.tensor(tokens, dtype=torch.int64)].clone()
    c = cos[torch.tensor(positions, dtype=torch.int64)].unsqueeze(1)
    s = sin[torch.tensor(positions, dtype=torch.int64)].unsqueeze(1)
    for li, lw in enumerate(model.layers):
        xn = rms_norm_q(h, lw.gamma_in, cfg.eps)
        q = rope(head_norm(_proj(xn, lw, "w_q").view(B, HQ, D), lw.gamma_q, cfg.eps), c, s)
        k = rope(head_norm(_proj(xn, lw, "w_k").view(B, HKV, D), lw.gamma_k, cfg.eps), c, s)
        v = _proj(xn, lw, "w_v").view(B, HKV, D)
        outs = []
        for b in range(B):
            cache = caches_b[b][li]
            cache[0] = torch.cat([cache[0], k[b].unsqueeze(0)], dim=0)
            cache[1] = torch.cat([cache[1], v[b].unsqueeze(0)], dim=0)
            outs.append(attend(q[b], cache[0], cache[1], cfg.scale, p_bf16))
        h1 = h + _proj(torch.stack(outs, 0), lw, "w_o")
        h = h1 + mlp(h1, lw, cfg)
    return lm_logits(h, model.gamma_final, model.head32(), cfg.eps)


def empty_caches(cfg: Qwen3Config, n_layers: int):
    z = torch.zeros(0, cfg.kv_heads, cfg.head_dim, dtype=BF16)
    return [[z, z] for _ in range(n_layers)]


def decode(model: ModelWeights, cfg: Qwen3Config, prompt: list[int], max_new: int,
           teacher: list[int] | None = None, record=None, p_bf16: bool = False):
    """Greedy continuation of ``prompt``: ``max_new`` ids.

    With ``teacher``, step i feeds ``teacher[i]`` instead of its own pick (the
    picks are still returned), so a comparison can continue past a divergence.
    ``record`` (a list) receives ``(logits, top1, top2_gap)`` per generated step.
    """
    n = len(prompt) + max_new
    cos, sin = rope_tables(n, cfg.head_dim, cfg.rope_theta)
    caches = empty_caches(cfg, len(model.layers))
    logits = None
    for p, tok in enumerate(prompt):
        logits = step(model, cfg, tok, p, caches, cos, sin, p_bf16)
    out = []
    for i in range(max_new):
        pick = greedy(logits)
        out.append(pick)
        if record is not None:
            top = torch.topk(logits, 2)
            record.append((logits.clone(), pick, float(top.values[0] - top.values[1])))
        if i + 1 == max_new:
            break
        nxt = teacher[i] if teacher is not None else pick
        logits = step(model, cfg, nxt, len(prompt) + i, caches, cos, sin, p_bf16)
    return out


def random_model(cfg: Qwen3Config, seed: int = 0, n_layers: int | None = None,
                 std: float = 0.02) -> ModelWeights:
    """Random-init weights: projections and embedding ~N(0, std), norm scales ~N(1, 0.1).

    Drawn on the CPU from one seeded generator in a fixed order, so the same
    seed gives the same weights on any machine.
    """
    g = torch.Generator().manual_seed(seed)
    L = cfg.layers if n_layers is None else n_layers
    H, HQ, HKV, D, I = cfg.hidden, cfg.heads, cfg.kv_heads, cfg.head_dim, cfg.inter

    def w(*shape):
        return (torch.randn(*shape, generator=g) * std).to(BF16)

    def gam(n):
        return (1.0 + 0.1 * torch.randn(n, generator=g)).to(BF16)

    embed = w(cfg.vocab, H)
    layers = []
    for _ in range(L):
        layers.append(LayerWeights(
            gamma_in=gam(H), w_q=w(HQ * D, H), w_k=w(HKV * D, H), w_v=w(HKV * D, H),
            gamma_q=gam(D), gamma_k=gam(D), w_o=w(H, HQ * D), gamma_post=gam(H),
            w_gate=w(I, H), w_up=w(I, H), w_down=w(H, I)))
    return ModelWeights(embed=embed, gamma_final=gam(H), layers=layers)


def prompt_ids(vocab: int, n: int = 64, seed: int = 0, batch: int = 1) -> list[list[int]]:
    """Uniform-random prompt ids from a seeded generator, one row per sequence."""
    g = torch.Generator().manual_seed(seed)
    return torch.randint(0, vocab, (batch, n), generator=g).tolist()


__all__ = [
    "Qwen3Config", "rope_tables", "proj", "head_norm", "rope", "attend", "LayerWeights",
    "self_attention", "mlp", "decoder_layer", "lm_logits", "greedy", "ModelWeights", "step",
    "step_batch", "empty_caches", "decode", "random_model", "prompt_ids",
]
