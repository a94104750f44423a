"""Qwen3-1.7B-shaped greedy decode on the gfx950 kernels: one captured step.

The step entry mirrors the reference engine
(examples/qwen3_1_7b-tilelang/fast/engine.py:69-271): ``Engine(...)`` packs the
weights once, allocates every buffer once, captures one decode step as a HIP
graph and ``generate(prompt_ids, max_new)`` replays it, returning
``Generated(tokens, seconds, prefill_seconds, prompt_steps)``. The cache has a
fixed capacity and the position lives in a one-element device tensor, so one
capture walks the prompt and continues past it with no host round trip: the
last kernel of the step writes the pick, feeds the next prompt id or the pick
back as the next input, and advances the position.

One step is 6 kernels per layer plus two for the head (170 launches for 28
layers; the reference's TileLang step is 228):

    decode_qkv          input norm (embedding gather on layer 0) + q|k|v GEMV;
                        v lands in the cache slot
    decode_attention    q/k head norm + RoPE + K-cache write, then split-KV GQA
                        attention partials
    attn_combine        log-sum-exp merge of the splits
    gemv_residual       o_proj + residual add
    rmsnorm_gemv_swiglu post-attention norm + gate|up GEMV + SwiGLU
    gemv_residual       down_proj + residual add
    lm_head_argmax      final norm + head GEMV + per-block winners
    sample_step         greedy pick, record, next input id, position + 1

No kernel waits on another block of its own launch: on gfx950 a cross-block
hand-off inside a kernel (coherent stores, an atomic, coherent loads) costs
more round trips than a kernel boundary inside a graph.

Weights are kept in the checkpoint's ``(out, in)`` layout: ``q|k|v`` stacked
into one matrix, ``gate`` and ``up`` rows interleaved into another, the head
tied to the embedding table (one 622 MB tensor serves both).
"""
from __future__ import annotations

from dataclasses import dataclass
from time import perf_counter

import torch

from . import synthetic
from ._lib import C

BF16 = torch.bfloat16


@dataclass(frozen=True)
class Qwen3Config:
    """examples/qwen3_1_7b-tilelang/ref_src/config.json."""

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

    @property
    def qkv_rows(self) -> int:
        return (self.heads + 2 * self.kv_heads) * self.head_dim


QWEN3_1_7B = Qwen3Config()


def hf_names(i: int) -> dict[str, str]:
    p = f"model.layers.{i}."
    return {
        "gamma_in": p + "input_layernorm.weight",
        "w_q": p + "self_attn.q_proj.weight",
        "w_k": p + "self_attn.k_proj.weight",
        "w_v": p + "self_attn.v_proj.weight",
        "gamma_q": p + "self_attn.q_norm.weight",
        "gamma_k": p + "self_attn.k_norm.weight",
        "w_o": p + "self_attn.o_proj.weight",
        "gamma_post": p + "post_attention_layernorm.weight",
        "w_gate": p + "mlp.gate_proj.weight",
        "w_up": p + "mlp.up_proj.weight",
        "w_down": p + "mlp.down_proj.weight",
    }


def synthetic_weights(cfg: Qwen3Config = QWEN3_1_7B, seed: int = 0, device="cpu",
                      layers: int | None = None, std: float = 0.02) -> dict[str, torch.Tensor]:
    """Random-init weights under the checkpoint's own names and ``(out, in)`` shapes.

    Projections and the (tied) embedding ~N(0, std), norm scales ~N(1, 0.1), all
    bf16, from :func:`synthetic.normal` -- identical on every device.
    """
    H, HQ, HKV, D, I = cfg.hidden, cfg.heads, cfg.kv_heads, cfg.head_dim, cfg.inter
    L = cfg.layers if layers is None else layers
    shapes = {
        "gamma_in": (H,), "w_q": (HQ * D, H), "w_k": (HKV * D, H), "w_v": (HKV * D, H),
        "gamma_q": (D,), "gamma_k": (D,), "w_o": (H, HQ * D), "gamma_post": (H,),
        "w_gate": (I, H), "w_up": (I, H), "w_down": (H, I),
    }
    out = {
        "model.embed_tokens.weight": synthetic.normal((cfg.vocab, H), seed, 0, std, device=device),
        "model.norm.weight": synthetic.normal((H,), seed, 1, 0.1, 1.0, device=device),
    }
    for i in range(L):
        for j, (key, name) in enumerate(hf_names(i).items()):
            stream = 100 + 16 * i + j
            if key.startswith("gamma"):
                out[name] = synthetic.normal(shapes[key], seed, stream, 0.1, 1.0, device=device)
            else:
                out[name] = synthetic.normal(shapes[key], seed, stream, std, device=device)
    return out


def rope_tables(n: int, head_dim: int, theta: float, device):
    """``_generation_rope`` (examples/qwen3_1_7b-tilelang/ref_src/model.py:106-119):
    f32 phases ``cat(f, f)``, cos / sin landed in bf16, rows 0..n-1."""
    inv = 1.0 / (theta ** (torch.arange(0, head_dim, 2, dtype=torch.float32) / head_dim))
    ph = torch.outer(torch.arange(n, dtype=torch.float32), inv)
    ph = torch.cat((ph, ph), dim=-1)
    return ph.cos().to(BF16).to(device), ph.sin().to(BF16).to(device)


@dataclass(frozen=True)
class Generated:
    """A continuation and the timing of the part that produced it
    (examples/qwen3_1_7b-tilelang/fast/engine.py:55-66)."""

    tokens: list
    seconds: float
    prefill_seconds: float
    prompt_steps: int

    @property
    def tokens_per_second(self) -> float:
        n = len(self.tokens)
        if n and isinstance(self.tokens[0], list):
            n = sum(len(t) for t in self.tokens)
        return n / self.seconds


class DeviceIndexError(RuntimeError):
    """A kernel found a device-resident index (token id, position, slot) out of range."""


class Engine:
    """A Qwen3-shaped model on one GPU and one captured decode step over it (batch 1)."""

    def __init__(self, cfg: Qwen3Config = QWEN3_1_7B, *, device="cuda:0", max_new: int = 2048,
                 prompt_room: int = 512, weights: dict | None = None, seed: int = 0,
                 split: int = 64, capture: bool = True):
        self.cfg = cfg
        self.device = torch.device(device)
        self.split = split
        self.nsteps = max_new + prompt_room
        self.cap = ((self.nsteps + split - 1) // split) * split
        self.ns = self.cap // split
        if weights is None:
            weights = synthetic_weights(cfg, seed, self.device)
        self._pack(weights)
        del weights
        self._buffers()
        self.graph = None
        if capture:
            self._capture()

    # ---------------------------------------------------------------- weights
    def _pack(self, wts):
        cfg, dev = self.cfg, self.device

        def get(name):
            return wts[name].to(dev, BF16).contiguous()

        self.embed = get("model.embed_tokens.weight")
        self.gamma_final = get("model.norm.weight")
        self.layers = []
        for i in range(cfg.layers):
            n = hf_names(i)
            gate, up = get(n["w_gate"]), get(n["w_up"])
            self.layers.append({
                "gamma_in": get(n["gamma_in"]),
                "w_qkv": torch.cat([get(n["w_q"]), get(n["w_k"]), get(n["w_v"])], 0).contiguous(),
                "gamma_q": get(n["gamma_q"]),
                "gamma_k": get(n["gamma_k"]),
                "w_o": get(n["w_o"]),
                "gamma_post": get(n["gamma_post"]),
                # rows (2i, 2i+1) = (gate_i, up_i): one block sees both halves of a pair
                "w_gu": torch.stack([gate, up], 1).reshape(2 * cfg.inter, cfg.hidden).contiguous(),
                "w_down": get(n["w_down"]),
            })
            del gate, up
        self.cos, self.sin = rope_tables(self.cap, cfg.head_dim, cfg.rope_theta, dev)

    # ---------------------------------------------------------------- buffers
    def _buffers(self):
        cfg, dev = self.cfg, self.device
        H, HQ, HKV, D = cfg.hidden, cfg.heads, cfg.kv_heads, cfg.head_dim

        def z(*shape, dtype=BF16):
            return torch.zeros(*shape, device=dev, dtype=dtype)

        self.hid = z(H)
        self.h1 = z(H)
        self.qk = z((HQ + HKV) * D)
        self.attn = z(HQ * D)
        self.act = z(cfg.inter)
        self.op = z(self.ns, HQ, D, dtype=torch.float32)
        self.mp = z(self.ns, HQ, dtype=torch.float32)
        self.lp = z(self.ns, HQ, dtype=torch.float32)
        self.kc = z(cfg.layers, self.cap, HKV * D)
        self.vc = z(cfg.layers, self.cap, HKV * D)
        self.logits = z(cfg.vocab, dtype=torch.float32)
        nb = C.lm_head_blocks(cfg.vocab)
        self.bv = z(nb, dtype=torch.float32)
        self.bi = z(nb, dtype=torch.int32)
        self.pos = z(1, dtype=torch.int32)
        self.ids = z(1, dtype=torch.int64)
        self.inp = z(self.nsteps, dtype=torch.int32)
        self.sam = z(self.nsteps, dtype=torch.int32)
        self.plen = z(1, dtype=torch.int32)
        self.err = z(1, dtype=torch.int32)

    # ------------------------------------------------------------------ step
    def _step(self):
        cfg = self.cfg
        HQ, HKV, D = cfg.heads, cfg.kv_heads, cfg.head_dim
        n_qk = (HQ + HKV) * D
        for i, w in enumerate(self.layers):
            kc, vc = self.kc[i], self.vc[i]
            if i == 0:
                C.decode_qkv(None, self.embed, self.ids, self.hid, w["gamma_in"], cfg.eps,
                             w["w_qkv"], n_qk, self.qk, self.pos, vc, self.err)
            else:
                C.decode_qkv(self.hid, None, None, None, w["gamma_in"], cfg.eps, w["w_qkv"], n_qk,
                             self.qk, self.pos, vc, self.err)
            C.decode_attention(self.qk, w["gamma_q"], w["gamma_k"], cfg.eps, self.cos, self.sin,
                               kc, vc, self.pos, self.pos, HQ, HKV, self.split, cfg.scale,
                               self.op, self.mp, self.lp, False, self.err)
            C.attn_combine(self.op, self.mp, self.lp, self.attn, self.pos, self.split)
            C.gemv_residual(self.attn, w["w_o"], self.hid, None, self.h1)
            C.rmsnorm_gemv_swiglu(self.h1, w["gamma_post"], cfg.eps, w["w_gu"], self.act)
            C.gemv_residual(self.act, w["w_down"], self.h1, None, self.hid)
        C.lm_head_argmax(self.hid, self.gamma_final, cfg.eps, self.embed, self.logits, self.bv,
                         self.bi)
        C.sample_step(self.bv, self.bi, self.inp, self.plen, self.ids, self.pos, self.sam,
                      self.err)

    def _capture(self):
        side = torch.cuda.Stream(device=self.device)
        side.wait_stream(torch.cuda.current_stream(self.device))
        self._load([0], 1)
        with torch.cuda.stream(side):
            self._step()  # one eager step: every kernel has run once before capture
        torch.cuda.current_stream(self.device).wait_stream(side)
        torch.cuda.synchronize(self.device)
        self.graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(self.graph):
            self._step()
        self._reset()

    def _run_step(self):
        if self.graph is not None:
            self.graph.replay()
        else:
            self._step()

    # ------------------------------------------------------------- state
    def _reset(self):
        self.pos.zero_()
        self.sam.zero_()
        self.err.zero_()

    def _load(self, ids: list[int], plen: int):
        if len(ids) > self.nsteps:
            raise ValueError(f"{len(ids)} input ids exceed this engine's {self.nsteps} steps")
        bad = [t for t in ids if not 0 <= t < self.cfg.vocab]
        if bad:
            raise ValueError(f"token ids out of range [0, {self.cfg.vocab}): {bad[:4]}")
        self._reset()
        self.inp.zero_()
        self.inp[: len(ids)] = torch.tensor(ids, dtype=torch.int32, device=self.device)
        self.plen.fill_(plen)
        self.ids.fill_(ids[0])

    def check_device_errors(self):
        code = int(self.err.item())
        if code:
            raise DeviceIndexError(f"a decode kernel found an index out of range (code {code})")

    # ------------------------------------------------------------ generation
    def generate(self, prompt_ids: list[int], max_new: int) -> Generated:
        """Walk ``prompt_ids``, then continue for ``max_new`` tokens.

        Timing covers exactly the steps that produce the continuation: the step at
        ``pos = len(prompt) - 1`` is the first whose pick is kept
        (examples/qwen3_1_7b-tilelang/fast/engine.py:239-271).
        """
        pl = len(prompt_ids)
        if pl < 1:
            raise ValueError("decode needs a prompt of at least one token")
        if pl + max_new > self.nsteps:
            raise ValueError(f"prompt {pl} + {max_new} new exceeds this engine's {self.nsteps} steps")
        self._load(list(prompt_ids), pl)
        torch.cuda.synchronize(self.device)
        t0 = perf_counter()
        for _ in range(pl - 1):
            self._run_step()
        torch.cuda.synchronize(self.device)
        t1 = perf_counter()
        for _ in range(max_new):
            self._run_step()
        torch.cuda.synchronize(self.device)
        t2 = perf_counter()
        self.check_device_errors()
        out = self.sam[pl - 1: pl - 1 + max_new].tolist()
        return Generated(out, t2 - t1, t1 - t0, pl)

    def forced(self, prompt_ids: list[int], teacher: list[int], record_logits: bool = False):
        """Teacher-forced picks: position ``len(prompt) - 1 + i`` is fed ``teacher[i-1]``.

        Returns the model's pick at each of ``len(teacher) + 1`` positions (and
        the f32 logits of each, when asked)."""
        ids = list(prompt_ids) + list(teacher)
        self._load(ids, len(ids))
        pl = len(prompt_ids)
        logits = []
        for p in range(len(ids)):
            self._run_step()
            if record_logits and p >= pl - 1:
                logits.append(self.logits.clone())
        torch.cuda.synchronize(self.device)
        self.check_device_errors()
        picks = self.sam[pl - 1: len(ids)].tolist()
        return (picks, logits) if record_logits else picks

    def logits_for(self, prompt_ids: list[int]) -> torch.Tensor:
        """The f32 logits after consuming every token of ``prompt_ids``."""
        self._load(list(prompt_ids), len(prompt_ids))
        for _ in range(len(prompt_ids)):
            self._run_step()
        torch.cuda.synchronize(self.device)
        self.check_device_errors()
        return self.logits.clone()
