"""MiniCPM3-4B decode restated on the CPU: the MLA attention and, at the end of this
file, the whole model (embedding, layers, head) -- test infrastructure only.

What each function follows (jingchangshi/TileFoundry):

* ``rope_tables`` -- ``_generation_rope``, examples/minicpm3_4b-cutedsl/model.py:151-167:
  longrope short factors, ``inv = 1 / (factor * theta^(2i/32))`` in f32,
  ``cat(phases, phases)``, cos / sin landed in bf16. theta = 10000 and
  head_dim = 32 are what ``MiniCPM3Config`` derives from the published
  config.json (``rope_parameters["rope_theta"]``, ``head_dim``).
* ``rope32`` -- the rotation of ``reference_ops.rope_attend``,
  examples/minicpm3_4b-cutedsl/kernels/reference_ops.py:99-109:
  ``x * c + cat(-x[16:], x[:16]) * s`` in bf16 (each product and the sum land).
* ``project`` -- steps 1-4 of ``mla_attention``, examples/minicpm3_4b-cutedsl/model.py:220-250:
  input norm (eps 1e-5), ``q_a`` -> LoRA norm (eps 1e-6) -> ``q_b``; ``kv_a`` ->
  latent ``c`` (LoRA norm, eps 1e-6) and the shared 32-wide rotary key.
* ``attend_reference`` -- the non-absorbed attention of
  ``reference_ops.rope_attend`` (reference_ops.py:87-130) over the cache Hugging
  Face keeps (assembled per-head keys ``[k_nope | k_rope]`` and values, each
  ``bf16(c @ W_kv_b^T)``, model.py:28-38): q scaled in bf16 before an f32 dot,
  f32 softmax, f32 weighted sum, one landing.
* ``attend_absorbed`` -- the same attention over the compressed cache (latent
  ``c`` [256] + rotated rope key [32] per position) with ``W_UK`` absorbed into
  the query and ``W_UV`` applied after the weighted sum: the arithmetic the
  kernels run (``q_lat = bf16(W_UK^T q_nope)``, f32 scores scaled after the
  dot, f32 softmax, optionally bf16 weights into the value sum, f32 latent
  output, ``bf16(W_UV o_lat)``). The reference has no absorbed implementation
  (model.py:28-38 caches assembled K/V); this is pinned to ``attend_reference``
  by the identity ``q_nope . (W_UK c) = (W_UK^T q_nope) . c`` and
  ``sum_j p_j W_UV c_j = W_UV sum_j p_j c_j``.
* ``rope_attend`` -- ``reference_ops.rope_attend`` itself (reference_ops.py:87-130)
  over the assembled cache ``k [cap, heads, 96]``, ``v [cap, heads, 64]`` with
  ``ctx`` context rows and this token's own key and value: the rotary slices
  rotated in bf16, ``q * scale`` in bf16, f32 scores against the context and
  the token, one f32 softmax (a joint max), f32 weighted sum, one landing.
* ``o_proj_residual`` -- ``gemv_residual``, reference_ops.py:63-65:
  ``residual + bf16(x @ W_o^T) * alpha``, each step landing in bf16.

* ``top_p_kept`` -- the token set and probabilities the sampler of
  examples/minicpm3_4b-cutedsl/run.py:29-47 (``_sampler``) draws from:
  softmax of ``logits / T`` in f32, ranked in descending order (a stable sort:
  ties in index order), a token kept while the mass ranked before it is below
  ``top_p``; the draw is proportional to the kept probabilities. Pinned
  (tests/test_oracle.py) by closed forms: one dominant logit keeps that token
  alone, a uniform row keeps the first ceil(top_p V) tokens, and top_p >= 1 keeps
  every token of nonzero probability.

Weights are ``(out, in)``: ``w_kv_b`` rows ``h*128 .. h*128+63`` are head h's
``W_UK`` and rows ``h*128+64 .. h*128+127`` its ``W_UV`` (the ``[k_nope | v]``
split of model.py:247-250).

Pinned by (tests/test_oracle.py): the rope tables against an f64 closed form,
position 0 as the identity and the rotation as complex multiplication on
(x_d, x_{d+16}) pairs; the absorbed attention against the non-absorbed
reference on the same cache (the identity above, within the bf16 bar); a
one-position context returning ``bf16(W_UV c_0)`` per head; an f64 brute force of
the absorbed formula on a tiny shape; and a planted mistake (absorbing with the
value half of ``W_kv_b``) that the identity check catches.
"""
from __future__ import annotations

from dataclasses import dataclass, field

import torch

from .norms import rms_norm_q

BF16 = torch.bfloat16

# examples/minicpm3_4b-cutedsl/config.json rope_scaling.short_factor
SHORT_FACTOR = (
    1.0591234137867171, 1.1241891283591912, 1.2596935748670968, 1.5380380402321725,
    2.093982484148734, 3.1446935121267696, 4.937952647693647, 7.524541999994549,
    10.475458000005451, 13.062047352306353, 14.85530648787323, 15.906017515851266,
    16.461961959767827, 16.740306425132907, 16.87581087164081, 16.940876586213285,
)


@dataclass(frozen=True)
class MLAConfig:
    """MiniCPM3-4B's attention shape (examples/minicpm3_4b-cutedsl/config.json)."""

    hidden: int = 2560
    heads: int = 40
    q_lora: int = 768
    kv_lora: int = 256
    nope: int = 64
    rope: int = 32
    v_dim: int = 64
    eps: float = 1e-5          # input_layernorm (rms_norm_eps)
    lora_eps: float = 1e-6     # MiniCPM3RMSNorm default for the two LoRA norms
    rope_theta: float = 10000.0
    short_factor: tuple = field(default=SHORT_FACTOR)

    @property
    def qk_dim(self) -> int:
        return self.nope + self.rope

    @property
    def scale(self) -> float:
        """``layer.self_attn.scaling`` = qk_head_dim^-1/2, as the bf16 tensor the
        reference passes (model.py:481-489)."""
        return float(torch.tensor(self.qk_dim ** -0.5).to(BF16))


def rope_tables(n: int, cfg: MLAConfig = MLAConfig()):
    """cos, sin bf16 ``[n, rope]``."""
    dim = cfg.rope
    factors = torch.tensor(cfg.short_factor[: dim // 2], dtype=torch.float32)
    inv = 1.0 / (factors * cfg.rope_theta ** (torch.arange(0, dim, 2, dtype=torch.float32) / dim))
    ph = torch.outer(torch.arange(n, dtype=torch.float32), inv)
    ph = torch.cat((ph, ph), dim=-1)
    return ph.cos().to(BF16), ph.sin().to(BF16)


def rope32(x: torch.Tensor, c: torch.Tensor, s: torch.Tensor) -> torch.Tensor:
    """Rotate-half over the last axis in bf16, each product and the sum landing."""
    half = x.shape[-1] // 2
    rot = torch.cat((-x[..., half:], x[..., :half]), dim=-1)
    return (x.to(BF16) * c.to(BF16)) + (rot.to(BF16) * s.to(BF16))


def proj(x: torch.Tensor, w: torch.Tensor) -> torch.Tensor:
    """``bf16(x @ w^T)`` with f32 accumulation; w is ``(out, in)``."""
    return (x.float() @ w.float().t()).to(BF16)


@dataclass
class MLAWeights:
    gamma_in: torch.Tensor   # [hidden]
    w_q_a: torch.Tensor      # [q_lora, hidden]
    gamma_q_a: torch.Tensor  # [q_lora]
    w_q_b: torch.Tensor      # [heads * qk_dim, q_lora]
    w_kv_a: torch.Tensor     # [kv_lora + rope, hidden]
    gamma_kv_a: torch.Tensor  # [kv_lora]
    w_kv_b: torch.Tensor     # [heads * (nope + v_dim), kv_lora]
    w_o: torch.Tensor        # [hidden, heads * v_dim]

    def w_uk(self, cfg: MLAConfig) -> torch.Tensor:
        """``[heads, nope, kv_lora]``."""
        return self.w_kv_b.view(cfg.heads, cfg.nope + cfg.v_dim, cfg.kv_lora)[:, : cfg.nope]

    def w_uv(self, cfg: MLAConfig) -> torch.Tensor:
        """``[heads, v_dim, kv_lora]``."""
        return self.w_kv_b.view(cfg.heads, cfg.nope + cfg.v_dim, cfg.kv_lora)[:, cfg.nope:]


def random_weights(cfg: MLAConfig, seed: int = 0, std: float = 0.02) -> MLAWeights:
    g = torch.Generator().manual_seed(seed)

    def w(*shape):
        return (std * torch.randn(*shape, generator=g)).to(BF16)

    def gam(n):
        return (1.0 + 0.1 * torch.randn(n, generator=g)).to(BF16)

    return MLAWeights(
        gamma_in=gam(cfg.hidden), w_q_a=w(cfg.q_lora, cfg.hidden), gamma_q_a=gam(cfg.q_lora),
        w_q_b=w(cfg.heads * cfg.qk_dim, cfg.q_lora), w_kv_a=w(cfg.kv_lora + cfg.rope, cfg.hidden),
        gamma_kv_a=gam(cfg.kv_lora), w_kv_b=w(cfg.heads * (cfg.nope + cfg.v_dim), cfg.kv_lora),
        w_o=w(cfg.hidden, cfg.heads * cfg.v_dim))


@dataclass
class Projected:
    """One token's projections (model.py:220-250)."""

    q_up: torch.Tensor      # [heads, qk_dim] bf16: [q_nope | q_rope] (q_rope not yet rotated)
    latent: torch.Tensor    # [kv_lora] bf16: the LoRA-normed kv latent c (what the cache holds)
    k_rope: torch.Tensor    # [rope] bf16, rotated at the token's position


def project(hidden: torch.Tensor, wts: MLAWeights, cfg: MLAConfig, pos: int, cos, sin) -> Projected:
    x = rms_norm_q(hidden, wts.gamma_in, cfg.eps)
    q_n = rms_norm_q(proj(x, wts.w_q_a), wts.gamma_q_a, cfg.lora_eps)
    q_up = proj(q_n, wts.w_q_b).view(cfg.heads, cfg.qk_dim)
    comp = proj(x, wts.w_kv_a)
    c = rms_norm_q(comp[: cfg.kv_lora], wts.gamma_kv_a, cfg.lora_eps)
    k_rope = rope32(comp[cfg.kv_lora:], cos[pos], sin[pos])
    return Projected(q_up=q_up, latent=c, k_rope=k_rope)


def attend_reference(q_up, latent_ctx, rope_ctx, wts: MLAWeights, cfg: MLAConfig, pos: int, cos, sin):
    """Non-absorbed attention over ``n`` positions of the compressed cache,
    expanded to the assembled per-head K / V the reference keeps.

    ``latent_ctx`` [n, kv_lora], ``rope_ctx`` [n, rope] (rotated) bf16, the last
    row being this token's own. Returns attn [heads * v_dim] bf16."""
    n = latent_ctx.shape[0]
    H = cfg.heads
    q_rope = rope32(q_up[:, cfg.nope:], cos[pos], sin[pos])
    q_full = torch.cat((q_up[:, : cfg.nope], q_rope), dim=-1)                       # [H, 96]
    kv = proj(latent_ctx, wts.w_kv_b).view(n, H, cfg.nope + cfg.v_dim)               # bf16(c W^T)
    k = torch.cat((kv[:, :, : cfg.nope], rope_ctx.view(n, 1, cfg.rope).expand(n, H, cfg.rope)), -1)
    v = kv[:, :, cfg.nope:]
    qh = (q_full * torch.tensor(cfg.scale).to(BF16)).float()                          # bf16 product
    s = torch.einsum("hd,nhd->hn", qh, k.float())
    e = torch.exp(s - s.amax(-1, keepdim=True))
    weighted = torch.einsum("hn,nhv->hv", e, v.float())
    return (weighted / e.sum(-1, keepdim=True)).reshape(-1).to(BF16)


def rope_attend(q_up, kv_up, k_rope, cos, sin, pos: int, k_cache, v_cache, ctx: int, scale,
                heads: int, nope: int, rope: int, v_dim: int, drop_new: bool = False):
    """Returns ``(attn [heads * v_dim], k_new [heads * (nope + rope)], v_new
    [heads * v_dim])`` bf16. ``k_cache`` [cap, heads, nope + rope] and
    ``v_cache`` [cap, heads, v_dim] hold ``ctx`` context rows; ``scale`` is the
    bf16 factor. ``drop_new`` plants a mistake for the pinning tests (the
    token's own score left out of the softmax)."""
    qk = nope + rope
    c, s = cos[pos], sin[pos]
    q = q_up.view(heads, qk)
    kv = kv_up.view(heads, nope + v_dim)
    q_full = torch.cat((q[:, :nope], rope32(q[:, nope:], c, s)), dim=-1)
    k_rot = rope32(k_rope.view(rope), c, s)
    k_full = torch.cat((kv[:, :nope], k_rot.view(1, rope).expand(heads, rope)), dim=-1)
    v_full = kv[:, nope:]
    qh = (q_full * torch.as_tensor(scale).to(BF16).reshape(())).float()          # bf16 product
    score_new = (qh * k_full.float()).sum(-1)                                     # [H]
    if ctx == 0:
        weighted, total = v_full.float(), torch.ones_like(score_new)
    else:
        kc = k_cache[:ctx].float().permute(1, 0, 2)                               # [H, n, qk]
        vc = v_cache[:ctx].float().permute(1, 0, 2)
        score_ctx = torch.einsum("hd,hnd->hn", qh, kc)
        peak = score_ctx.amax(-1) if drop_new else torch.maximum(score_ctx.amax(-1), score_new)
        p_ctx = torch.exp(score_ctx - peak[:, None])
        p_new = torch.zeros_like(peak) if drop_new else torch.exp(score_new - peak)
        total = p_ctx.sum(-1) + p_new
        weighted = torch.einsum("hn,hnv->hv", p_ctx, vc) + p_new[:, None] * v_full.float()
    out = (weighted / total[:, None]).reshape(-1).to(BF16)
    return out, k_full.reshape(-1).contiguous(), v_full.reshape(-1).contiguous()


def mla_attention(hidden, wts: MLAWeights, cfg: MLAConfig, pos: int, cos, sin, k_cache, v_cache,
                  ctx: int, scale):
    """``mla_attention`` of model.py:205-291 in the ``reference_ops`` spelling
    (runtime_model.py:146-186): input norm -> ``[q_a | kv_a]`` projection ->
    LoRA norms -> ``q_b`` / ``kv_b`` -> ``rope_attend`` over the assembled cache
    -> ``W_o``. Returns ``(out [hidden], k_new, v_new)`` bf16."""
    x = rms_norm_q(hidden, wts.gamma_in, cfg.eps)
    q_a = proj(x, wts.w_q_a)
    comp = proj(x, wts.w_kv_a)
    q_up = proj(rms_norm_q(q_a, wts.gamma_q_a, cfg.lora_eps), wts.w_q_b)
    kv_up = proj(rms_norm_q(comp[: cfg.kv_lora], wts.gamma_kv_a, cfg.lora_eps), wts.w_kv_b)
    attn, k_new, v_new = rope_attend(q_up, kv_up, comp[cfg.kv_lora:], cos, sin, pos, k_cache,
                                     v_cache, ctx, scale, cfg.heads, cfg.nope, cfg.rope, cfg.v_dim)
    return proj(attn, wts.w_o), k_new, v_new


def assembled_cache(latent_ctx, rope_ctx, wts: MLAWeights, cfg: MLAConfig):
    """The per-head cache Hugging Face keeps for a compressed one:
    ``k [n, heads, nope + rope]`` = ``[bf16(c W_UK^T) | k_rope]``, ``v [n, heads,
    v_dim]`` = ``bf16(c W_UV^T)`` (model.py:28-38)."""
    n, H = latent_ctx.shape[0], cfg.heads
    kv = proj(latent_ctx, wts.w_kv_b).view(n, H, cfg.nope + cfg.v_dim)
    k = torch.cat((kv[:, :, : cfg.nope], rope_ctx.view(n, 1, cfg.rope).expand(n, H, cfg.rope)), -1)
    return k.contiguous(), kv[:, :, cfg.nope:].contiguous()


def absorb_query(q_up, wts: MLAWeights, cfg: MLAConfig, pos: int, cos, sin):
    """``[heads, kv_lora + rope]`` bf16: ``bf16(W_UK^T q_nope)`` and the rotated
    q_rope -- the query the absorbed attention scores the compressed cache with."""
    q_lat = torch.einsum("hi,hic->hc", q_up[:, : cfg.nope].float(), wts.w_uk(cfg).float()).to(BF16)
    q_rope = rope32(q_up[:, cfg.nope:], cos[pos], sin[pos])
    return torch.cat((q_lat, q_rope), dim=-1)


def attend_absorbed(q_abs, latent_ctx, rope_ctx, wts: MLAWeights, cfg: MLAConfig, p_bf16: bool = False,
                    return_latent: bool = False):
    """Absorbed attention: ``q_abs`` [heads, kv_lora + rope] bf16 against the
    compressed cache; f32 scores scaled after the dot, f32 softmax, the latent
    weighted sum in f32, then ``bf16(W_UV o_lat)``. Returns attn [heads * v_dim]."""
    kc = torch.cat((latent_ctx, rope_ctx), dim=-1).float()                          # [n, 288]
    s = (q_abs.float() @ kc.t()) * cfg.scale                                        # [H, n]
    m = s.amax(-1, keepdim=True)
    e = torch.exp(s - m)
    l = e.sum(-1, keepdim=True)
    p = e.to(BF16).float() if p_bf16 else e
    o_lat = (p @ latent_ctx.float()) / l                                            # [H, kv_lora]
    out = torch.einsum("hc,hvc->hv", o_lat, wts.w_uv(cfg).float()).to(BF16)
    return (out.reshape(-1), o_lat) if return_latent else out.reshape(-1)


def o_proj_residual(attn, w_o, residual, alpha: float):
    """``bf16(residual + bf16(bf16(attn @ W_o^T) * alpha))``."""
    a = torch.tensor(alpha).to(BF16)
    return residual.to(BF16) + proj(attn, w_o) * a


def random_cache(batch: int, n: int, cfg: MLAConfig, seed: int = 1):
    """Latent ``[batch, n, kv_lora]`` and rope-key ``[batch, n, rope]`` caches ~N(0,1) bf16."""
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(batch, n, cfg.kv_lora, generator=g).to(BF16),
            torch.randn(batch, n, cfg.rope, generator=g).to(BF16))


# ---------------------------------------------------------------- the whole model
# MiniCPM3_4B's root and decoder layer (examples/minicpm3_4b-cutedsl/model.py:320-420),
# decoded one token at a time over the compressed cache:
#   embed           bf16(table[id] * scale_emb)                         (:356-365)
#   decoder_layer   h1 = h + bf16(attn(h) * a); h' = h1 + bf16(mlp(h1) * a),
#                   a = bf16(scale_depth / sqrt(layers))                (:320-344)
#   mlp             down(bf16(silu(gate(xn))) * up(xn)), xn = norm(h1) (reference_ops.py:66-70)
#   final_rms_norm  + lm_head: bf16(bf16(norm(h)) / logits_scaling) @ W_embed^T,
#                   landed in bf16 (:367-392); greedy = lowest-index argmax.
# Pinned (tests/test_oracle.py) against Hugging Face's MiniCPM3ForCausalLM (the
# reference's own third-party arithmetic boundary, transformers installed here)
# built from the same tiny random weights, within the bf16 bar, and by the
# zero-branch closed form (all projections zero: every layer is the identity
# and the logits are the head of the scaled embedding's norm).


@dataclass(frozen=True)
class ModelConfig(MLAConfig):
    """MLAConfig plus the fields of the whole model (examples/minicpm3_4b-cutedsl/config.json)."""

    inter: int = 6400
    vocab: int = 73448
    layers: int = 62
    scale_emb: float = 12.0
    dim_model_base: int = 256
    scale_depth: float = 1.4

    @property
    def logits_scaling(self) -> float:
        return self.hidden / self.dim_model_base

    @property
    def residual_scale(self) -> float:
        """``scale_depth / sqrt(layers)`` as the bf16 scalar the reference passes."""
        import math

        return float(torch.tensor(self.scale_depth / math.sqrt(self.layers)).to(BF16))


@dataclass
class LayerWeights(MLAWeights):
    gamma_post: torch.Tensor = None   # [hidden]
    w_gate: torch.Tensor = None       # [inter, hidden]
    w_up: torch.Tensor = None         # [inter, hidden]
    w_down: torch.Tensor = None       # [hidden, inter]


@dataclass
class ModelWeights:
    embed: torch.Tensor               # [vocab, hidden], tied with the head
    gamma_final: torch.Tensor
    layers: list


def random_model(cfg: ModelConfig, seed: int = 0, std: float = 0.02) -> ModelWeights:
    g = torch.Generator().manual_seed(seed)

    def w(*shape):
        return (std * torch.randn(*shape, generator=g)).to(BF16)

    def gam(n):
        return (1.0 + 0.1 * torch.randn(n, generator=g)).to(BF16)

    layers = []
    for _ in range(cfg.layers):
        a = random_weights(cfg, seed=int(torch.randint(0, 2 ** 31 - 1, (1,), generator=g)), std=std)
        layers.append(LayerWeights(**a.__dict__, gamma_post=gam(cfg.hidden), w_gate=w(cfg.inter, cfg.hidden),
                                   w_up=w(cfg.inter, cfg.hidden), w_down=w(cfg.hidden, cfg.inter)))
    return ModelWeights(embed=w(cfg.vocab, cfg.hidden), gamma_final=gam(cfg.hidden), layers=layers)


def mlp(h1, lw: LayerWeights, cfg: ModelConfig):
    xn = rms_norm_q(h1, lw.gamma_post, cfg.eps)
    act = torch.nn.functional.silu(proj(xn, lw.w_gate).float()).to(BF16) * proj(xn, lw.w_up)
    return proj(act, lw.w_down)


def decode_step(model: ModelWeights, cfg: ModelConfig, token: int, pos: int, caches, cos, sin,
                p_bf16: bool = True):
    """One decode step of the whole model over the compressed caches
    (``caches[i] = [latent [n, kv_lora], rope_k [n, rope]]``, appended in place).
    Returns the logits (f32 holding the bf16 values the reference returns)."""
    a = torch.tensor(cfg.residual_scale).to(BF16)
    h = model.embed[token] * torch.tensor(cfg.scale_emb).to(BF16)
    for lw, cache in zip(model.layers, caches):
        pr = project(h, lw, cfg, pos, cos, sin)
        cache[0] = torch.cat((cache[0], pr.latent.view(1, -1)), 0)
        cache[1] = torch.cat((cache[1], pr.k_rope.view(1, -1)), 0)
        q_abs = absorb_query(pr.q_up, lw, cfg, pos, cos, sin)
        attn = attend_absorbed(q_abs, cache[0], cache[1], lw, cfg, p_bf16=p_bf16)
        h1 = o_proj_residual(attn, lw.w_o, h, cfg.residual_scale)
        h = h1 + mlp(h1, lw, cfg) * a
    xs = rms_norm_q(h, model.gamma_final, cfg.eps) / torch.tensor(cfg.logits_scaling).to(BF16)
    return proj(xs, model.embed).float()


def empty_caches(cfg: ModelConfig, n_layers: int):
    return [[torch.zeros(0, cfg.kv_lora, dtype=BF16), torch.zeros(0, cfg.rope, dtype=BF16)]
            for _ in range(n_layers)]


def greedy(logits: torch.Tensor) -> int:
    return int(torch.argmax(logits))


def decode(model: ModelWeights, cfg: ModelConfig, prompt: list, max_new: int, record=None,
           p_bf16: bool = True, teacher: list | None = None) -> list:
    """Greedy continuation; ``record`` receives ``(logits, pick, top-2 gap)`` per generated step.
    With ``teacher``, step i feeds ``teacher[i]`` instead of its own pick (the
    picks are still returned)."""
    cos, sin = rope_tables(len(prompt) + max_new, cfg)
    caches = empty_caches(cfg, len(model.layers))
    for p, t in enumerate(prompt):
        logits = decode_step(model, cfg, t, p, caches, cos, sin, p_bf16)
    out = []
    for i in range(max_new):
        pick = greedy(logits)
        out.append(pick)
        if record is not None:
            top = torch.topk(logits, 2).values
            record.append((logits.clone(), pick, float(top[0] - top[1])))
        if i + 1 < max_new:
            nxt = teacher[i] if teacher is not None else pick
            logits = decode_step(model, cfg, nxt, len(prompt) + i, caches, cos, sin, p_bf16)
    return out


def top_p_kept(logits: torch.Tensor, temperature: float, top_p: float):
    """``(ids, probs)`` of the tokens the run.py sampler may draw for one row of
    logits, and their probabilities renormalised over the kept set (the
    distribution of its one multinomial draw). Ties are ranked in index order."""
    probs = torch.softmax(logits.reshape(-1).float() / temperature, dim=-1)
    order = torch.sort(probs, descending=True, stable=True).indices
    ranked = probs[order]
    before = torch.cumsum(ranked, dim=-1) - ranked
    keep = before < top_p
    ids = order[keep]
    kept = ranked[keep].double()
    return ids, kept / kept.sum()
