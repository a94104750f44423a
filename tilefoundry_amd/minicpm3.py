"""MiniCPM3-4B-shaped MLA decode attention block on MI355X, absorbed form.

``MLABlock`` runs one attention block of the MiniCPM3 decoder for a batch of
sequences, one token each: input RMSNorm, the q / kv LoRA projections, the
compressed cache append, absorbed multi-head latent attention over the cache,
the value up-projection, o_proj and MiniCPM3's ``scale_depth`` residual --
``MiniCPM3_4B_DecoderLayer.mla_attention`` plus the residual of
``decoder_layer`` (examples/minicpm3_4b-cutedsl/model.py:205-291,337-344), with the
cache holding the 288-wide compressed entry per position (latent c | rotated
rope key) instead of 40 assembled keys and values.

Launch sequence of one step (8 kernels, capturable as one graph):

    rms_norm         input norm (eps 1e-5)                       [B, 2560]
    skinny_gemm      x_n . [W_q_a; W_kv_a]^T -> split-K partials   [ks, B, 1056]
    mla_prep         q_a / kv_c LoRA norms, latent + rope cache append at pos
    mla_qb_absorb    q_up = bf16(q_n . W_q_b^T) per head on MFMA, then
                     q_lat = bf16(W_UK^T q_nope), rotated q_rope   [B, 40, 288]
    mla_attention    split attention over the compressed cache (bf16 MFMA)
    mla_combine_up   split merge, bf16(W_UV o_lat)                  [B, 2560]
    skinny_gemm      attn . W_o^T -> split-K partials              [ks, B, 2560]
    rows_residual    hidden + bf16(bf16(.) * residual_scale)        [B, 2560]

Weights are ``(out, in)`` with Hugging Face names; random-init, cross-device
reproducible (:mod:`synthetic`).
"""
from __future__ import annotations

import math
from dataclasses import dataclass, field

import torch

from . import synthetic
from ._lib import C

BF16 = torch.bfloat16

# examples/minicpm3_4b-cutedsl/config.json rope_scaling.short_factor
SHORT_FACTOR = (
    1.0591234137867171, 1.1241891283591912, 1.2596935748670968, 1.5380380402321725,
    2.093982484148734, 3.1446935121267696, 4.937952647693647, 7.524541999994549,
    10.475458000005451, 13.062047352306353, 14.85530648787323, 15.906017515851266,
    16.461961959767827, 16.740306425132907, 16.87581087164081, 16.940876586213285,
)


@dataclass(frozen=True)
class MiniCPM3Config:
    """examples/minicpm3_4b-cutedsl/config.json."""

    hidden: int = 2560
    heads: int = 40
    q_lora: int = 768
    kv_lora: int = 256
    nope: int = 64
    rope: int = 32
    v_dim: int = 64
    layers: int = 62
    eps: float = 1e-5
    lora_eps: float = 1e-6
    rope_theta: float = 10000.0
    scale_depth: float = 1.4
    short_factor: tuple = field(default=SHORT_FACTOR)
    inter: int = 6400
    vocab: int = 73448
    scale_emb: float = 12.0
    dim_model_base: int = 256
    original_max_pos: int = 32768   # rope_scaling.original_max_position_embeddings

    @property
    def logits_scaling(self) -> float:
        """hidden / dim_model_base: MiniCPM3ForCausalLM divides the final hidden state by it."""
        return self.hidden / self.dim_model_base

    @property
    def qk_dim(self) -> int:
        return self.nope + self.rope

    @property
    def scale(self) -> float:
        """qk_head_dim^-1/2 as the bf16 scalar the reference passes."""
        return float(torch.tensor(self.qk_dim ** -0.5).to(BF16))

    @property
    def residual_scale(self) -> float:
        """scale_depth / sqrt(layers) as a bf16 scalar (model.py:337-344)."""
        return float(torch.tensor(self.scale_depth / math.sqrt(self.layers)).to(BF16))


MINICPM3_4B = MiniCPM3Config()

NAMES = {   # key -> Hugging Face name within layer i
    "gamma_in": "input_layernorm.weight",
    "w_q_a": "self_attn.q_a_proj.weight",
    "gamma_q_a": "self_attn.q_a_layernorm.weight",
    "w_q_b": "self_attn.q_b_proj.weight",
    "w_kv_a": "self_attn.kv_a_proj_with_mqa.weight",
    "gamma_kv_a": "self_attn.kv_a_layernorm.weight",
    "w_kv_b": "self_attn.kv_b_proj.weight",
    "w_o": "self_attn.o_proj.weight",
}


def synthetic_weights(cfg: MiniCPM3Config = MINICPM3_4B, seed: int = 0, device="cpu", layer: int = 0,
                      std: float = 0.02) -> dict[str, torch.Tensor]:
    """One layer's attention weights ``(out, in)`` ~N(0, std), norm scales ~N(1, 0.1), bf16."""
    H, QA, KV, R = cfg.hidden, cfg.q_lora, cfg.kv_lora, cfg.rope
    shapes = {
        "gamma_in": (H,), "w_q_a": (QA, H), "gamma_q_a": (QA,), "w_q_b": (cfg.heads * cfg.qk_dim, QA),
        "w_kv_a": (KV + R, H), "gamma_kv_a": (KV,), "w_kv_b": (cfg.heads * (cfg.nope + cfg.v_dim), KV),
        "w_o": (H, cfg.heads * cfg.v_dim),
    }
    out = {}
    for j, (key, name) in enumerate(NAMES.items()):
        stream = 5000 + 16 * layer + j
        if key.startswith("gamma"):
            out[key] = synthetic.normal(shapes[key], seed, stream, 0.1, 1.0, device=device)
        else:
            out[key] = synthetic.normal(shapes[key], seed, stream, std, device=device)
    return out


def rope_tables(n: int, cfg: MiniCPM3Config, device):
    """``_generation_rope`` (examples/minicpm3_4b-cutedsl/model.py:151-167): longrope
    short factors, f32 phases ``cat(f, f)``, cos / sin landed in bf16."""
    dim = cfg.rope
    factors = torch.tensor(cfg.short_factor[: dim // 2], dtype=torch.float32)
    inv = 1.0 / (factors * cfg.rope_theta ** (torch.arange(0, dim, 2, dtype=torch.float32) / dim))
    ph = torch.outer(torch.arange(n, dtype=torch.float32), inv)
    ph = torch.cat((ph, ph), dim=-1)
    return ph.cos().to(BF16).to(device), ph.sin().to(BF16).to(device)


class MLABlock:
    """The MiniCPM3 attention block for ``batch`` sequences over a compressed
    cache of ``cap`` positions each; ``step`` appends every sequence's entry at
    its own ``pos`` and attends slots ``0..pos``."""

    def __init__(self, cfg: MiniCPM3Config = MINICPM3_4B, *, batch: int = 8, cap: int = 8192,
                 device="cuda:0", weights: dict | None = None, seed: int = 0, split: int = 256,
                 ks_a: int = 5, ks_qb: int = 3, ks_o: int = 5, fuse_qb: bool = True):
        if cfg.kv_lora != 256 or cfg.rope != 32 or cfg.nope != 64 or cfg.v_dim != 64:
            raise ValueError("the MLA kernels are built for kv_lora 256, rope 32, nope 64, value 64")
        if cap % split:
            raise ValueError(f"cap {cap} must be a multiple of split {split}")
        self.cfg, self.batch, self.cap, self.split = cfg, batch, cap, split
        self.device = torch.device(device)
        self.ks = {"a": ks_a, "qb": ks_qb, "o": ks_o}
        self.fuse_qb = fuse_qb   # q_b projection + absorption in one launch (else split-K q_b, then absorb)
        w = synthetic_weights(cfg, seed, self.device) if weights is None else {
            k: v.to(self.device) for k, v in weights.items()}
        self.w = w
        self.w_a = torch.cat((w["w_q_a"], w["w_kv_a"]), 0).contiguous()   # [q_lora + 288, hidden]
        self.cos, self.sin = rope_tables(cap, cfg, self.device)
        self.alpha = cfg.residual_scale
        B, H, dev = batch, cfg.heads, self.device
        f32 = torch.float32

        def z(*shape, dtype=BF16):
            return torch.zeros(*shape, device=dev, dtype=dtype)

        self.ns = cap // split
        self.hidden = z(B, cfg.hidden)
        self.xn = z(B, cfg.hidden)
        self.part_a = z(ks_a, B, cfg.q_lora + cfg.kv_lora + cfg.rope, dtype=f32)
        self.q_n = z(B, cfg.q_lora)
        self.part_qb = z(ks_qb, B, H * cfg.qk_dim, dtype=f32)
        self.q_abs = z(B, H, cfg.kv_lora + cfg.rope)
        self.latent = z(B, cap, cfg.kv_lora)
        self.rope_k = z(B, cap, cfg.rope)
        self.op = z(B, self.ns, H, cfg.kv_lora)
        self.mp = z(B, self.ns, H, dtype=f32)
        self.lp = z(B, self.ns, H, dtype=f32)
        self.attn = z(B, H * cfg.v_dim)
        self.part_o = z(ks_o, B, cfg.hidden, dtype=f32)
        self.out = z(B, cfg.hidden)
        self.pos = z(B, dtype=torch.int32)
        self.err = z(1, dtype=torch.int32)
        self.graph = None

    # ------------------------------------------------------------------ step
    def _step(self):
        cfg, w = self.cfg, self.w
        C.rms_norm(self.hidden, w["gamma_in"], self.xn, cfg.eps, 0)
        C.skinny_gemm(self.xn, self.w_a, self.ks["a"], 0, self.part_a, None, None, None, None)
        C.mla_prep(self.part_a, w["gamma_q_a"], w["gamma_kv_a"], cfg.lora_eps, self.cos, self.sin,
                   self.pos, self.latent, self.rope_k, self.q_n, self.err)
        if self.fuse_qb:
            C.mla_qb_absorb(self.q_n, w["w_q_b"], w["w_kv_b"], self.cos, self.sin, self.pos, self.q_abs, self.err)
        else:
            C.skinny_gemm(self.q_n, w["w_q_b"], self.ks["qb"], 0, self.part_qb, None, None, None, None)
            C.mla_q_absorb(self.part_qb, w["w_kv_b"], self.cos, self.sin, self.pos, self.q_abs, self.err)
        C.mla_attention(self.q_abs, self.latent, self.rope_k, self.pos, self.split, cfg.scale,
                        self.op, self.mp, self.lp, self.err)
        C.mla_combine_up(self.op, self.mp, self.lp, self.pos, self.split, w["w_kv_b"], self.attn)
        C.skinny_gemm(self.attn, w["w_o"], self.ks["o"], 0, self.part_o, None, None, None, None)
        C.rows_residual(self.part_o, self.hidden, self.alpha, self.out)

    def capture(self):
        """Record one step as a graph (inputs: ``hidden``, ``pos``, the caches)."""
        side = torch.cuda.Stream(device=self.device)
        side.wait_stream(torch.cuda.current_stream(self.device))
        with torch.cuda.stream(side):
            self._step()
        torch.cuda.current_stream(self.device).wait_stream(side)
        torch.cuda.synchronize(self.device)
        self.graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(self.graph):
            self._step()
        torch.cuda.synchronize(self.device)

    def run(self):
        if self.graph is not None:
            self.graph.replay()
        else:
            self._step()

    def step(self, hidden: torch.Tensor, pos) -> torch.Tensor:
        """``hidden`` [batch, hidden] bf16; ``pos`` per-sequence slots (list or
        int32 tensor). Returns the block output [batch, hidden] (a view of the
        block's own buffer)."""
        self.hidden.copy_(hidden)
        p = torch.as_tensor(pos, dtype=torch.int32)
        if p.numel() != self.batch or int(p.min()) < 0 or int(p.max()) >= self.cap:
            raise ValueError(f"positions must be {self.batch} slots in [0, {self.cap})")
        self.pos.copy_(p)
        self.err.zero_()
        self.run()
        torch.cuda.synchronize(self.device)
        e = int(self.err.item())
        if e:
            raise RuntimeError(f"mla block: device error code {e}")
        return self.out


# ------------------------------------------------------------ the whole model
MLP_NAMES = {   # key -> Hugging Face name within layer i
    "gamma_post": "post_attention_layernorm.weight",
    "w_gate": "mlp.gate_proj.weight",
    "w_up": "mlp.up_proj.weight",
    "w_down": "mlp.down_proj.weight",
}


def hf_layer_names(i: int) -> dict[str, str]:
    """Key -> published checkpoint name of every weight of layer i."""
    return {k: f"model.layers.{i}.{v}" for k, v in {**NAMES, **MLP_NAMES}.items()}


def synthetic_model_weights(cfg: MiniCPM3Config = MINICPM3_4B, seed: int = 0, device="cpu",
                            std: float = 0.02) -> dict[str, torch.Tensor]:
    """Random-init weights of the whole model under the published names and
    ``(out, in)`` shapes (the embedding doubles as the tied head)."""
    H, I = cfg.hidden, cfg.inter
    out = {"model.embed_tokens.weight": synthetic.normal((cfg.vocab, H), seed, 9000, std, device=device),
           "model.norm.weight": synthetic.normal((H,), seed, 9001, 0.1, 1.0, device=device)}
    for i in range(cfg.layers):
        names = hf_layer_names(i)
        for k, v in synthetic_weights(cfg, seed, device, layer=i, std=std).items():
            out[names[k]] = v
        base = 20000 + 8 * i
        out[names["gamma_post"]] = synthetic.normal((H,), seed, base, 0.1, 1.0, device=device)
        out[names["w_gate"]] = synthetic.normal((I, H), seed, base + 1, std, device=device)
        out[names["w_up"]] = synthetic.normal((I, H), seed, base + 2, std, device=device)
        out[names["w_down"]] = synthetic.normal((H, I), seed, base + 3, std, device=device)
    return out


class TopP:
    """Top-p sampling as the decode step's last kernel (``tfa_top_p_sample_step``):
    the sampler of examples/minicpm3_4b-cutedsl/run.py:29-47 (``_sampler``, the
    published ``generation_config.json``: T = 0.8, top-p 0.8) -- probabilities
    softmax(logits / T), ranked, a token kept while the mass ranked before it is
    below ``top_p``, one draw from the kept mass -- drawn on the device inside the
    captured step, so no host round trip per token. The draws come from a
    counter-based generator of (``seed``, sequence, position): a seed gives the
    same continuation on every run, on any device."""

    def __init__(self, temperature: float = 0.8, top_p: float = 0.8, seed: int = 0):
        if not temperature > 0.0 or not top_p > 0.0:
            raise ValueError(f"temperature {temperature} and top_p {top_p} must be positive")
        self.temperature, self.top_p, self.seed = float(temperature), float(top_p), int(seed)


def sample_top_p(temperature: float = 0.8, top_p: float = 0.8, generator: torch.Generator | None = None,
                 seed: int | None = None) -> TopP:
    """The run.py sampler for ``MiniCPM3Engine.generate(sampler=...)``: a
    :class:`TopP` whose seed is ``seed``, else the generator's seed (run.py's
    ``--seed``), else 0."""
    if seed is None:
        seed = generator.initial_seed() if generator is not None else 0
    return TopP(temperature, top_p, seed)


class MiniCPM3Engine:
    """The whole MiniCPM3 decode model for up to 32 sequences in lockstep, one
    captured step over all of them (examples/minicpm3_4b-cutedsl/model.py:320-420,
    runtime twin runtime_model.py; run.py drives it token by token).

    One step (batch > 1), 10 launches per layer plus 5 -- at one sequence the
    projections run on the bs=1 GEMVs instead, 7 launches per layer (``_step_one``):

        embed            bf16(table[id] * scale_emb), then the first input norm
        -- per layer: the MLA attention block of ``MLABlock`` ----------------
        skinny_gemm [q_a | kv_a], mla_prep, mla_qb_absorb (q_b + absorption),
        mla_attention, mla_combine_up, skinny_gemm o_proj,
        rows_norm_scaled h1 = h + bf16(bf16(o) * a), a = scale_depth / sqrt(layers),
                         and the post-attention norm of h1
        -- the MLP -------------------------------------------------------------
        skinny_gemm      gate|up + SwiGLU (interleaved rows)
        skinny_gemm      down -> split-K partials
        rows_norm_scaled h = h1 + bf16(bf16(down) * a) and the next layer's input
                         norm (rows_residual after the last layer)
        -- the head -------------------------------------------------------------
        rms_norm_div     bf16(bf16(norm(h)) / logits_scaling)             (once)
        skinny_gemm      head, bf16 logits, per-group winners (lowest index on ties)
        batch_sample     greedy pick, next input id, position + 1

    The compressed cache holds 576 bytes per position per layer (latent 256 +
    rotated rope key 32, bf16). ``generate`` takes ``sampler=`` to sample instead
    of taking the greedy pick: a :class:`TopP` (``sample_top_p()``) runs a second
    captured step whose last kernel draws on the device
    (``top_p_sample_step``, no host round trip); any other callable
    ``sampler(logits) -> id`` is called on each sequence's bf16 logits after each
    replay, and its id fed back (one host round trip per step).
    """

    MAX_BATCH = 32

    def __init__(self, cfg: MiniCPM3Config = MINICPM3_4B, *, batch: int = 1, device="cuda:0",
                 max_new: int = 512, prompt_room: int = 512, weights: dict | None = None, seed: int = 0,
                 split: int | None = None, ks_a: int = 5, ks_qb: int = 3, ks_o: int = 5, ks_down: int = 5,
                 capture: bool = True, fuse_qb: bool = True):
        if cfg.kv_lora != 256 or cfg.rope != 32 or cfg.nope != 64 or cfg.v_dim != 64:
            raise ValueError("the MLA kernels are built for kv_lora 256, rope 32, nope 64, value 64")
        if not 1 <= batch <= self.MAX_BATCH:
            raise ValueError(f"batch {batch} not in [1, {self.MAX_BATCH}]")
        self.nsteps = max_new + prompt_room
        # positions per attention split: at small batch the shortest split (32:
        # a three-wave block over one 32-position step) whose split count the
        # merge still takes in one memory round trip (64); 256 (eight-wave
        # blocks over two 128-position steps) once the batch alone fills the
        # device. bs=1, 8 + 512 positions: 128 -> 32 took the step
        # from 322 to 343 tok/s.
        if split is None:
            split = 256
            if batch <= 4:
                split = next((c for c in (32, 64, 128) if -(-self.nsteps // c) <= 64), 128)
        self.cfg, self.batch, self.split = cfg, batch, split
        self.device = torch.device(device)
        self.ks = {"a": ks_a, "qb": ks_qb, "o": ks_o, "down": ks_down}
        self.fuse_qb = fuse_qb   # one sequence: prep + q_b + absorption in one launch (else prep-q GEMV, absorb)
        self.cap = ((self.nsteps + split - 1) // split) * split
        if self.cap > cfg.original_max_pos:
            raise ValueError(f"cache of {self.cap} positions: past original_max_position_embeddings "
                             f"({cfg.original_max_pos}) longrope switches to its long factors, not built here")
        if weights is None:
            weights = synthetic_model_weights(cfg, seed, self.device)
        self._pack(weights)
        del weights
        self.cos, self.sin = rope_tables(self.cap, cfg, self.device)
        self.alpha = cfg.residual_scale
        self.alpha_t = torch.tensor([self.alpha], dtype=BF16, device=self.device)
        self._buffers()
        self.graph = None
        self.graph_sample = None   # the step ending in the device top-p draw, captured on first use
        self.capture = capture
        if capture:
            self._capture()

    @classmethod
    def from_checkpoint(cls, ckpt, *, device="cuda:0", **kw):
        """The engine over a MiniCPM3 checkpoint directory (``config.json`` and
        safetensors shards or ``pytorch_model.bin``, ``checkpoint.load_minicpm3``):
        the model run.py decodes from ``--ckpt`` (examples/minicpm3_4b-cutedsl/run.py:53-116)."""
        from .checkpoint import load_minicpm3

        cfg, wts = load_minicpm3(ckpt, device)
        return cls(cfg, device=device, weights=wts, **kw)

    def _pack(self, wts):
        cfg, dev = self.cfg, self.device

        def get(name):
            return wts[name].to(dev, BF16).contiguous()

        self.embed = get("model.embed_tokens.weight")
        self.gamma_final = get("model.norm.weight")
        self.head = get("lm_head.weight") if "lm_head.weight" in wts else self.embed
        self.layers = []
        for i in range(cfg.layers):
            n = hf_layer_names(i)
            gate, up = get(n["w_gate"]), get(n["w_up"])
            self.layers.append({
                "gamma_in": get(n["gamma_in"]),
                "w_a": torch.cat((get(n["w_q_a"]), get(n["w_kv_a"])), 0).contiguous(),
                "gamma_q_a": get(n["gamma_q_a"]),
                "w_q_b": get(n["w_q_b"]),
                "gamma_kv_a": get(n["gamma_kv_a"]),
                "w_kv_b": get(n["w_kv_b"]),
                "w_o": get(n["w_o"]),
                "gamma_post": get(n["gamma_post"]),
                "w_gu": torch.stack([gate, up], 1).reshape(2 * cfg.inter, cfg.hidden).contiguous(),
                "w_down": get(n["w_down"]),
            })
            del gate, up

    def _buffers(self):
        cfg, B, dev, ks = self.cfg, self.batch, self.device, self.ks
        f32 = torch.float32

        def z(*shape, dtype=BF16):
            return torch.zeros(*shape, device=dev, dtype=dtype)

        H, NH = cfg.hidden, cfg.heads
        self.ns = self.cap // self.split
        self.h = z(B, H)
        self.h1 = z(B, H)
        self.xn = z(B, H)
        self.part_a = z(ks["a"], B, cfg.q_lora + cfg.kv_lora + cfg.rope, dtype=f32)
        self.q_n = z(B, cfg.q_lora)
        self.part_qb = z(ks["qb"], B, NH * cfg.qk_dim, dtype=f32)
        self.q_abs = z(B, NH, cfg.kv_lora + cfg.rope)
        self.latent = z(cfg.layers, B, self.cap, cfg.kv_lora)
        self.rope_k = z(cfg.layers, B, self.cap, cfg.rope)
        self.op = z(B, self.ns, NH, cfg.kv_lora)
        self.mp = z(B, self.ns, NH, dtype=f32)
        self.lp = z(B, self.ns, NH, dtype=f32)
        self.attn = z(B, NH * cfg.v_dim)
        self.part_o = z(ks["o"], B, H, dtype=f32)
        self.act = z(B, cfg.inter)
        self.part_d = z(ks["down"], B, H, dtype=f32)
        self.logits = z(B, cfg.vocab, dtype=f32)
        nb = C.skinny_blocks(cfg.vocab)
        self.bv = z(B, nb, dtype=f32)
        self.bi = z(B, nb, dtype=torch.int32)
        self.pos = z(B, dtype=torch.int32)
        self.ids = z(B, dtype=torch.int64)
        self.inp = z(B, self.nsteps, dtype=torch.int32)
        self.sam = z(B, self.nsteps, dtype=torch.int32)
        self.plen = z(B, dtype=torch.int32)
        self.err = z(1, dtype=torch.int32)
        self.topp = z(2, dtype=f32)                 # temperature, top_p of the sampling step
        self.topp_seed = z(1, dtype=torch.int64)

    def _finish(self, sample: bool):
        """The step's last launch: the greedy pick over the head's block winners,
        or the top-p draw over the bf16 logits."""
        if sample:
            C.top_p_sample_step(self.logits, self.topp, self.topp_seed, self.inp, self.plen, self.ids, self.pos,
                                self.sam, self.err)
        else:
            C.batch_sample_step(self.bv, self.bi, self.inp, self.plen, self.ids, self.pos, self.sam,
                                self.err)

    def _step(self, keep_logits: bool = True, sample: bool = False):
        keep_logits = keep_logits or sample
        if self.batch == 1:
            self._step_one(keep_logits, sample)
            return
        cfg, ks = self.cfg, self.ks
        L = len(self.layers)
        C.embed(self.embed, self.ids, self.h, cfg.scale_emb, self.err)
        C.rms_norm(self.h, self.layers[0]["gamma_in"], self.xn, cfg.eps, 0)
        for i, w in enumerate(self.layers):
            lat, rk = self.latent[i], self.rope_k[i]
            C.skinny_gemm(self.xn, w["w_a"], ks["a"], 0, self.part_a, None, None, None, None)
            C.mla_prep(self.part_a, w["gamma_q_a"], w["gamma_kv_a"], cfg.lora_eps, self.cos, self.sin,
                       self.pos, lat, rk, self.q_n, self.err)
            C.mla_qb_absorb(self.q_n, w["w_q_b"], w["w_kv_b"], self.cos, self.sin, self.pos, self.q_abs, self.err)
            C.mla_attention(self.q_abs, lat, rk, self.pos, self.split, cfg.scale, self.op, self.mp,
                            self.lp, self.err)
            C.mla_combine_up(self.op, self.mp, self.lp, self.pos, self.split, w["w_kv_b"], self.attn)
            C.skinny_gemm(self.attn, w["w_o"], ks["o"], 0, self.part_o, None, None, None, None)
            C.rows_norm_scaled(self.part_o, self.h, self.alpha, self.h1, w["gamma_post"], self.xn, cfg.eps)
            C.skinny_gemm(self.xn, w["w_gu"], 1, 1, None, self.act, None, None, None)
            C.skinny_gemm(self.act, w["w_down"], ks["down"], 0, self.part_d, None, None, None, None)
            if i + 1 < L:   # the residual fused with the next layer's input norm
                C.rows_norm_scaled(self.part_d, self.h1, self.alpha, self.h, self.layers[i + 1]["gamma_in"],
                                   self.xn, cfg.eps)
            else:
                C.rows_residual(self.part_d, self.h1, self.alpha, self.h)
        C.rms_norm_div(self.h, self.gamma_final, self.xn, cfg.eps, cfg.logits_scaling)
        C.skinny_gemm(self.xn, self.head, 1, 3, None, None, self.logits if keep_logits else None,
                      self.bv, self.bi)
        self._finish(sample)

    def _step_one(self, keep_logits: bool = True, sample: bool = False):
        """One sequence: the projections on the bs=1 GEMVs, each with its norm or
        scaled residual fused (7 launches per layer):
        rmsnorm_gemv_f32 [q_a | kv_a] (one f32 split-K partial), mla_prep_qb_absorb
        (q_a lands, LoRA norm, q_b and the absorption per head on MFMA; one block
        lands the latent and the rope key in the caches), mla_attention,
        mla_combine_up, gemv_residual o_proj + scaled residual,
        rmsnorm_gemv_swiglu (post norm + gate|up + SwiGLU), gemv_residual down +
        scaled residual. With ``fuse_qb=False`` the prep and q_b run as
        mla_prep_q_gemv (f32 out) and the absorption as mla_q_absorb (8 launches)."""
        cfg = self.cfg
        h, h1 = self.h[0], self.h1[0]
        part_a, part_qb = self.part_a[:1], self.part_qb[:1]
        C.embed(self.embed, self.ids, self.h, cfg.scale_emb, self.err)
        for i, w in enumerate(self.layers):
            lat, rk = self.latent[i], self.rope_k[i]
            C.rmsnorm_gemv_f32(h, w["gamma_in"], cfg.eps, w["w_a"], part_a.view(-1))
            if self.fuse_qb:
                C.mla_prep_qb_absorb(part_a.view(-1), w["gamma_q_a"], w["gamma_kv_a"], cfg.lora_eps, self.cos,
                                     self.sin, self.pos, lat, rk, w["w_q_b"], w["w_kv_b"], self.q_abs, self.err)
            else:
                C.mla_prep_q_gemv(part_a.view(-1), w["gamma_q_a"], w["gamma_kv_a"], cfg.lora_eps, self.cos,
                                  self.sin, self.pos, lat, rk, w["w_q_b"], part_qb.view(-1), self.err)
                C.mla_q_absorb(part_qb, w["w_kv_b"], self.cos, self.sin, self.pos, self.q_abs, self.err)
            C.mla_attention(self.q_abs, lat, rk, self.pos, self.split, cfg.scale, self.op, self.mp,
                            self.lp, self.err)
            C.mla_combine_up(self.op, self.mp, self.lp, self.pos, self.split, w["w_kv_b"], self.attn)
            C.gemv_residual(self.attn[0], w["w_o"], h, self.alpha_t, h1)
            C.rmsnorm_gemv_swiglu(h1, w["gamma_post"], cfg.eps, w["w_gu"], self.act[0])
            C.gemv_residual(self.act[0], w["w_down"], h1, self.alpha_t, h)
        C.rms_norm_div(self.h, self.gamma_final, self.xn, cfg.eps, cfg.logits_scaling)
        C.skinny_gemm(self.xn, self.head, 1, 3, None, None, self.logits if keep_logits else None,
                      self.bv, self.bi)
        self._finish(sample)

    def _capture(self, sample: bool = False):
        side = torch.cuda.Stream(device=self.device)
        side.wait_stream(torch.cuda.current_stream(self.device))
        self._load([[0]] * self.batch, 1)
        with torch.cuda.stream(side):
            self._step(sample=sample)  # every kernel has run once before capture
        torch.cuda.current_stream(self.device).wait_stream(side)
        torch.cuda.synchronize(self.device)
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            self._step(sample=sample)
        self._load([[0]] * self.batch, 1)
        if sample:
            self.graph_sample = graph
        else:
            self.graph = graph

    def _run_step(self, sample: bool = False):
        if sample:
            if self.capture and self.graph_sample is None:
                self._capture(sample=True)
            if self.graph_sample is not None:
                self.graph_sample.replay()
            else:
                self._step(sample=True)
        elif self.graph is not None:
            self.graph.replay()
        else:
            self._step()

    def _load(self, rows: list[list[int]], plen: int):
        if len(rows) != self.batch:
            raise ValueError(f"{len(rows)} sequences given to an engine of batch {self.batch}")
        if any(len(r) != len(rows[0]) for r in rows):
            raise ValueError("sequences of one batch advance in lockstep: give equal lengths")
        if len(rows[0]) > self.nsteps:
            raise ValueError(f"{len(rows[0])} input ids exceed this engine's {self.nsteps} steps")
        if any(not 0 <= t < self.cfg.vocab for r in rows for t in r):
            raise ValueError(f"token ids out of range [0, {self.cfg.vocab})")
        self.pos.zero_()
        self.sam.zero_()
        self.err.zero_()
        self.inp.zero_()
        self.inp[:, : len(rows[0])] = torch.tensor(rows, dtype=torch.int32, device=self.device)
        self.plen.fill_(plen)
        self.ids.copy_(torch.tensor([r[0] for r in rows], dtype=torch.int64, device=self.device))

    def check_device_errors(self):
        code = int(self.err.item())
        if code:
            raise RuntimeError(f"a decode kernel found an index out of range (code {code})")

    def forced(self, prompts: list[list[int]], teachers: list[list[int]], record_logits: bool = False):
        """Teacher-forced greedy picks: position ``len(prompt) - 1 + i`` of sequence b
        is fed ``teachers[b][i - 1]``. Returns the picks ``[batch][len(teacher) + 1]``
        (and, when asked, the logits ``[batch, vocab]`` of each of those positions)."""
        if len(teachers) != self.batch or any(len(t) != len(teachers[0]) for t in teachers):
            raise ValueError(f"give {self.batch} teacher sequences of equal length")
        rows = [list(p) + list(t) for p, t in zip(prompts, teachers)]
        self._load(rows, len(rows[0]))
        pl = len(prompts[0])
        logits = []
        for p in range(len(rows[0])):
            self._run_step()
            if record_logits and p >= pl - 1:
                logits.append(self.logits.clone())
        torch.cuda.synchronize(self.device)
        self.check_device_errors()
        picks = self.sam[:, pl - 1: len(rows[0])].tolist()
        return (picks, logits) if record_logits else picks

    def generate(self, prompts: list[list[int]], max_new: int, sampler=None):
        """Walk every prompt, then continue each for ``max_new`` tokens, greedy
        (lowest-index argmax over the bf16 logits) or drawn by ``sampler(logits)``.
        Returns ``qwen3.Generated``; timing covers the continuation steps only."""
        from time import perf_counter

        from .qwen3 import Generated

        if not prompts or not prompts[0]:
            raise ValueError("decode needs prompts of at least one token")
        pl = len(prompts[0])
        if pl + max_new > self.nsteps:
            raise ValueError(f"prompt {pl} + {max_new} new exceeds this engine's {self.nsteps} steps")
        device_draw = isinstance(sampler, TopP)
        if device_draw and self.capture and self.graph_sample is None:
            self._capture(sample=True)   # before the load: capturing reloads the buffers
        self._load([list(p) for p in prompts], pl)
        if device_draw:
            self.topp.copy_(torch.tensor([sampler.temperature, sampler.top_p], dtype=torch.float32))
            self.topp_seed.fill_(sampler.seed)
        torch.cuda.synchronize(self.device)
        t0 = perf_counter()
        for _ in range(pl - 1):
            self._run_step(device_draw)
        torch.cuda.synchronize(self.device)
        t1 = perf_counter()
        for s in range(max_new):
            self._run_step(device_draw)
            if sampler is not None and not device_draw:
                p = pl - 1 + s
                picks = [sampler(self.logits[b]) for b in range(self.batch)]
                t = torch.tensor(picks, dtype=torch.int64, device=self.device)
                self.ids.copy_(t)
                self.sam[:, p] = t.to(torch.int32)
        torch.cuda.synchronize(self.device)
        t2 = perf_counter()
        self.check_device_errors()
        out = self.sam[:, pl - 1: pl - 1 + max_new].tolist()
        return Generated(out, t2 - t1, t1 - t0, pl)
