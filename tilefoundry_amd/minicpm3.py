"""MiniCPM3-4B-shaped MLA decode attention block on MI355X, absorbed form.

``MLABlock`` runs one attention block of the MiniCPM3 decoder for a batch of
sequences, one token each: input RMSNorm, the q / kv LoRA projections, the
compressed cache append, absorbed multi-head latent attention over the cache,
the value up-projection, o_proj and MiniCPM3's ``scale_depth`` residual --
``MiniCPM3_4B_DecoderLayer.mla_attention`` plus the residual of
``decoder_layer`` (examples/minicpm3_4b-cutedsl/model.py:205-291,337-344), with the
cache holding the 288-wide compressed entry per position (latent c | rotated
rope key) instead of 40 assembled keys and values.

Launch sequence of one step (9 kernels, capturable as one graph):

    rms_norm         input norm (eps 1e-5)                       [B, 2560]
    skinny_gemm      x_n . [W_q_a; W_kv_a]^T -> split-K partials   [ks, B, 1056]
    mla_prep         q_a / kv_c LoRA norms, latent + rope cache append at pos
    skinny_gemm      q_n . W_q_b^T -> split-K partials             [ks, B, 3840]
    mla_q_absorb     q_lat = bf16(W_UK^T q_nope), rotated q_rope   [B, 40, 288]
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
    """examples/minicpm3_4b-cutedsl/config.json (attention-block fields)."""

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
                 ks_a: int = 5, ks_qb: int = 3, ks_o: int = 5):
        if cfg.kv_lora != 256 or cfg.rope != 32 or cfg.nope != 64 or cfg.v_dim != 64:
            raise ValueError("the MLA kernels are built for kv_lora 256, rope 32, nope 64, value 64")
        if cap % split:
            raise ValueError(f"cap {cap} must be a multiple of split {split}")
        self.cfg, self.batch, self.cap, self.split = cfg, batch, cap, split
        self.device = torch.device(device)
        self.ks = {"a": ks_a, "qb": ks_qb, "o": ks_o}
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
