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

(``fuse_o=True`` runs the merge and o_proj as one launch,
``attn_combine_gemv_residual``, bit-identical; every one of its blocks re-reads
the split partials, and the step measured 905 tok/s against 961 apart.)
    rmsnorm_gemv_swiglu post-attention norm + gate|up GEMV + SwiGLU
    gemv_residual       down_proj + residual add
    lm_head_argmax      final norm + head GEMV + per-block winners
    sample_step         greedy pick, record, next input id, position + 1

No kernel waits on another block of its own launch: on gfx950 a cross-block
hand-off inside a kernel (coherent stores, an atomic, coherent loads) costs
more round trips than a kernel boundary inside a graph.

Weights are kept in the checkpoint's ``(out, in)`` layout: ``q|k|v`` stacked
into one matrix, ``gate`` and ``up`` rows interleaved into another, the head
tied to the embedding table (one 622 MB tensor serves both) unless the
checkpoint ships its own ``lm_head.weight``. ``Engine.from_checkpoint(dir)``
reads a published checkpoint directory (``checkpoint.load_qwen3``).
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


def pack_weights(cfg: Qwen3Config, wts: dict, dev):
    """The decode layout of a checkpoint-named weight dict: ``q|k|v`` stacked,
    ``gate``/``up`` rows interleaved (row 2i = gate_i, 2i+1 = up_i, so one tile
    holds both halves of every pair), everything else as stored; the embedding
    table doubles as the head unless the dict holds an untied ``lm_head.weight``.
    Returns ``(embed, gamma_final, layers, head)``."""

    def get(name):
        return wts[name].to(dev, BF16).contiguous()

    embed = get("model.embed_tokens.weight")
    gamma_final = get("model.norm.weight")
    layers = []
    for i in range(cfg.layers):
        n = hf_names(i)
        gate, up = get(n["w_gate"]), get(n["w_up"])
        layers.append({
            "gamma_in": get(n["gamma_in"]),
            "w_qkv": torch.cat([get(n["w_q"]), get(n["w_k"]), get(n["w_v"])], 0).contiguous(),
            "gamma_q": get(n["gamma_q"]),
            "gamma_k": get(n["gamma_k"]),
            "w_o": get(n["w_o"]),
            "gamma_post": get(n["gamma_post"]),
            "w_gu": torch.stack([gate, up], 1).reshape(2 * cfg.inter, cfg.hidden).contiguous(),
            "w_down": get(n["w_down"]),
        })
        del gate, up
    head = get("lm_head.weight") if "lm_head.weight" in wts else embed
    return embed, gamma_final, layers, head


def prefill_caches(cfg: Qwen3Config, embed, layers, kc, vc, cos, sin, ids: torch.Tensor, err):
    """Every layer over whole prompts at once, writing their K/V cache rows.

    ``ids`` int64 ``[B, n]`` on the device: sequence b's tokens at positions
    0..n-1; ``kc`` / ``vc`` per layer ``[B, cap, kv_heads*head_dim]`` (or
    ``[cap, .]`` for B = 1). Afterwards cache rows 0..n-1 hold what n decode
    steps over the same tokens would have written, computed with the same
    rounding points: every projection is an f32 GEMM over all B*n rows
    (``gemm_nt_f32``, its K split into partial slices when few rows would leave
    most CUs idle) whose consumer lands it in bf16 as the decode step lands
    its split-K partials -- ``prefill_qk_rope`` (per-head norm + RoPE + cache
    write), ``rows_norm`` (residual add + norm), ``swiglu_pairs`` -- and the
    attention of every row is one causal launch over the cache
    (``causal_attention``). Only the summation order of the products differs
    from the walk. 11 launches per layer, none per token; the last layer stops
    after its attention (nothing downstream of it reaches a cache).

    This replaces the reference's token-by-token prompt walk
    (examples/qwen3_1_7b-tilelang/fast/engine.py:261-263); it computes
    ref_src/model.py:235-265 (decoder_layer) for every prompt row.
    """
    H, HQ, HKV, D, I = cfg.hidden, cfg.heads, cfg.kv_heads, cfg.head_dim, cfg.inter
    B, n = ids.shape
    R = B * n
    dev = ids.device
    f32 = torch.float32

    def e(*shape, dtype=BF16):
        return torch.empty(*shape, device=dev, dtype=dtype)

    h, h1, xn = e(R, H), e(R, H), e(R, H)
    # each projection's f32 result as split-K partials [ks, R, out] when few
    # rows leave the GEMM's grid too small to fill the CUs; the consumers sum
    # the partials in split order, as the decode step sums its own
    ks = {name: C.gemm_f32_splits(R, nout, nin) for name, nout, nin in (
        ("qkv", cfg.qkv_rows, H), ("o", H, HQ * D), ("gu", 2 * I, H), ("down", H, I))}
    qkv = e(ks["qkv"], R, cfg.qkv_rows, dtype=f32)
    q = e(R, HQ * D)
    attn = e(R, HQ * D)
    o = e(ks["o"], R, H, dtype=f32)
    gu = e(ks["gu"], R, 2 * I, dtype=f32)
    act = e(R, I)
    d = e(ks["down"], R, H, dtype=f32)
    C.rows_norm(embed, ids.reshape(-1), None, None, h, layers[0]["gamma_in"], xn, cfg.eps, err)
    for i, w in enumerate(layers):
        k4 = kc[i].view(B, -1, HKV, D)
        v4 = vc[i].view(B, -1, HKV, D)
        C.gemm_nt_f32(xn, w["w_qkv"], qkv)
        C.prefill_qk_rope(qkv, w["gamma_q"], w["gamma_k"], cfg.eps, cos, sin, B, n, 0,
                          k4.view(B, -1, HKV * D), v4.view(B, -1, HKV * D), q, HQ, HKV)
        if i + 1 == len(layers):
            break
        C.causal_attention(q.view(B, n, HQ, D), k4, v4, attn.view(B, n, HQ * D), cfg.scale)
        C.gemm_nt_f32(attn, w["w_o"], o)
        C.rows_norm(None, None, h, o, h1, w["gamma_post"], xn, cfg.eps, err)
        C.gemm_nt_f32(xn, w["w_gu"], gu)
        C.swiglu_pairs(gu, act)
        C.gemm_nt_f32(act, w["w_down"], d)
        C.rows_norm(None, None, h1, d, h, layers[i + 1]["gamma_in"], xn, cfg.eps, err)


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
                 split: int = 64, capture: bool = True, prompt_prefill: bool = False,
                 fuse_o: bool = False):
        self.cfg = cfg
        self.device = torch.device(device)
        self.split = split
        self.prompt_prefill = prompt_prefill
        self.nsteps = max_new + prompt_room
        self.cap = ((self.nsteps + split - 1) // split) * split
        self.ns = self.cap // split
        # the split merge folded into o_proj: up to 64 splits, 4..16 heads of 128, <= 2560 rows
        fusable = (self.ns <= 64 and cfg.head_dim == 128 and cfg.heads % 4 == 0 and 4 <= cfg.heads <= 16
                   and cfg.hidden <= 2560)
        if fuse_o and not fusable:
            raise ValueError(f"fuse_o needs <= 64 splits (cache {self.cap} / split {split}), 4..16 heads of 128 "
                             f"and hidden <= 2560")
        self.fuse_o = bool(fuse_o)
        if weights is None:
            weights = synthetic_weights(cfg, seed, self.device)
        self._pack(weights)
        del weights
        self._buffers()
        self.graph = None
        if capture:
            self._capture()

    @classmethod
    def from_checkpoint(cls, ckpt, ref_dir=None, *, device="cuda:0", **kw):
        """The reference's ``Engine(ckpt, ref_dir, device=..., max_new=...,
        prompt_room=...)`` (examples/qwen3_1_7b-tilelang/fast/engine.py:69-107): the
        model is the checkpoint directory's ``config.json`` and its safetensors
        weights. ``ref_dir`` (the reference's model-source directory) is accepted
        for the same call shape and not read: the model here is the config's."""
        from .checkpoint import load_qwen3

        cfg, wts = load_qwen3(ckpt, device)
        return cls(cfg, device=device, weights=wts, **kw)

    # ---------------------------------------------------------------- weights
    def _pack(self, wts):
        self.embed, self.gamma_final, self.layers, self.head = pack_weights(self.cfg, wts, self.device)
        self.cos, self.sin = rope_tables(self.cap, self.cfg.head_dim, self.cfg.rope_theta,
                                         self.device)

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
            C.decode_attention(self.qk, None, w["gamma_q"], w["gamma_k"], cfg.eps, self.cos,
                               self.sin, kc, vc, self.pos, self.pos, HQ, HKV, self.split,
                               cfg.scale, self.op, self.mp, self.lp, False, self.err)
            if self.fuse_o:
                C.attn_combine_gemv_residual(self.op, self.mp, self.lp, self.pos, self.split, w["w_o"],
                                             self.hid, self.h1, None)
            else:
                C.attn_combine(self.op, self.mp, self.lp, self.attn, self.pos, self.split)
                C.gemv_residual(self.attn, w["w_o"], self.hid, None, self.h1)
            C.rmsnorm_gemv_swiglu(self.h1, w["gamma_post"], cfg.eps, w["w_gu"], self.act)
            C.gemv_residual(self.act, w["w_down"], self.h1, None, self.hid)
        C.lm_head_argmax(self.hid, self.gamma_final, cfg.eps, self.head, self.logits, self.bv,
                         self.bi)
        C.sample_step(self.bv, self.bi, self.inp, self.plen, self.ids, self.pos, self.sam,
                      self.err)

    def _capture(self):
        side = torch.cuda.Stream(device=self.device)
        side.wait_stream(torch.cuda.current_stream(self.device))
        self._load(*self._capture_inputs())
        with torch.cuda.stream(side):
            self._step()  # one eager step: every kernel has run once before capture
        torch.cuda.current_stream(self.device).wait_stream(side)
        torch.cuda.synchronize(self.device)
        self.graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(self.graph):
            self._step()
        self._reset()

    def _capture_inputs(self):
        return [0], 1

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

    def _walk_or_prefill(self, rows: list[list[int]]):
        """Consume all but the last prompt token of every sequence: one decode
        step per token (the reference's walk), or with ``prompt_prefill`` one
        pass of every layer over all of them (``prefill_caches``), after which
        the position and the next input are set as the walk would leave them."""
        n = len(rows[0]) - 1
        if not self.prompt_prefill or n < 1:
            for _ in range(n):
                self._run_step()
            return
        ids = torch.tensor([r[:n] for r in rows], dtype=torch.int64, device=self.device)
        prefill_caches(self.cfg, self.embed, self.layers, self.kc, self.vc, self.cos, self.sin, ids,
                       self.err)
        self.pos.fill_(n)
        self.ids.copy_(torch.tensor([r[n] for r in rows], dtype=torch.int64, device=self.device))

    # ------------------------------------------------------------ generation
    def generate(self, prompt_ids: list[int], max_new: int) -> Generated:
        """Walk ``prompt_ids`` (or prefill them, with ``prompt_prefill``), then
        continue for ``max_new`` tokens.

        Timing covers exactly the steps that produce the continuation: the step at
        ``pos = len(prompt) - 1`` is the first whose pick is kept
        (examples/qwen3_1_7b-tilelang/fast/engine.py:239-271); ``prefill_seconds``
        is the walk (or the prefill) before it.
        """
        pl = len(prompt_ids)
        if pl < 1:
            raise ValueError("decode needs a prompt of at least one token")
        if pl + max_new > self.nsteps:
            raise ValueError(f"prompt {pl} + {max_new} new exceeds this engine's {self.nsteps} steps")
        self._load(list(prompt_ids), pl)
        torch.cuda.synchronize(self.device)
        t0 = perf_counter()
        self._walk_or_prefill([list(prompt_ids)])
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

        The prompt is walked, or prefilled with ``prompt_prefill``, as in
        ``generate``. Returns the model's pick at each of ``len(teacher) + 1``
        positions (and the f32 logits of each, when asked)."""
        ids = list(prompt_ids) + list(teacher)
        self._load(ids, len(ids))
        pl = len(prompt_ids)
        self._walk_or_prefill([list(prompt_ids)])
        logits = []
        for _ in range(pl - 1, len(ids)):
            self._run_step()
            if record_logits:
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


class BatchEngine:
    """Up to 32 sequences decoded in lockstep, one captured step over all of them.

    Every projection is a skinny bf16-MFMA GEMM over the batch (the weights are
    streamed once per step for all sequences); each sequence has its own KV
    cache, position and prompt. One step is 7 launches per layer plus 3 when
    the sequences x kv heads fill the device (``attention="seq"``):

        rows_norm        embedding gather + input norm (once)
        skinny_gemm      q|k|v projection -> f32 split-K partials
        decode_attention_seq
                         per (sequence, kv head) one block over the whole
                         context: sums the partials, q/k head norm + RoPE,
                         writes the new K and V rows, attends, lands o / l
        skinny_gemm      o_proj -> split-K partials
        rows_norm        residual add + post-attention norm
        skinny_gemm      gate|up + SwiGLU
        skinny_gemm      down_proj -> split-K partials
        rows_norm        residual add + next input norm (final norm after the last layer)
        skinny_gemm      head -> per 16-row group winners per sequence
        batch_sample     greedy step per sequence

    With fewer blocks than that (``attention="split"``) the attention is three
    launches: ``qk_rope_cache`` (the prepared query, once per sequence),
    split-KV ``decode_attention`` and ``attn_combine``. ``"auto"`` picks the
    whole-context form from 256 (sequence, kv head) pairs up.
    """

    MAX_BATCH = 32
    SEQ_GROUPS = (1, 2, 4)   # query heads per kv head the whole-context attention takes
    SEQ_SCORES = 32768       # its per-block score store: group x (cache + 64) at most

    def __init__(self, cfg: Qwen3Config = QWEN3_1_7B, *, batch: int = 32, device="cuda:0",
                 max_new: int = 2048, prompt_room: int = 512, weights: dict | None = None,
                 seed: int = 0, split: int = 128, ks_qkv: int = 2, ks_o: int = 4, ks_down: int = 4,
                 capture: bool = True, prompt_prefill: bool = False, attention: str = "auto",
                 fold_o_norm: bool = False):
        if not 1 <= batch <= self.MAX_BATCH:
            raise ValueError(f"batch {batch} not in [1, {self.MAX_BATCH}]")
        if attention not in ("auto", "seq", "split"):
            raise ValueError(f"attention {attention!r} not in ('auto', 'seq', 'split')")
        self.cfg = cfg
        self.batch = batch
        self.device = torch.device(device)
        self.split = split
        self.prompt_prefill = prompt_prefill
        self.ks = {"qkv": ks_qkv, "o": ks_o, "down": ks_down}
        # fold_o_norm: o_proj unsplit with the residual add and the post-attention
        # norm's sums in its epilogue, the norm itself in the gate|up GEMM's
        # staging -- one launch fewer per layer, but measured slower (15.6-15.7k
        # against 16.26k tok/s at 32 x 2048: the unsplit o_proj has 64 blocks for
        # its 8.4 MB, and the norm lengthens the gate|up staging loop), so off
        self.fold_o_norm = bool(fold_o_norm)
        self.nsteps = max_new + prompt_room
        self.cap = ((self.nsteps + split - 1) // split) * split
        self.ns = self.cap // split
        group = cfg.heads // cfg.kv_heads
        seq_ok = group in self.SEQ_GROUPS and (self.cap + 64) * group <= self.SEQ_SCORES
        if attention == "seq" and not seq_ok:
            raise ValueError(f"attention='seq' needs a group in {self.SEQ_GROUPS} and a cache of at most "
                             f"{self.SEQ_SCORES // max(group, 1) - 64} slots (group {group}, cache {self.cap})")
        if attention == "auto":
            attention = "seq" if seq_ok and batch * cfg.kv_heads >= 256 else "split"
        self.attention = attention
        if weights is None:
            weights = synthetic_weights(cfg, seed, self.device)
        self.embed, self.gamma_final, self.layers, self.head = pack_weights(cfg, weights, self.device)
        del weights
        self.cos, self.sin = rope_tables(self.cap, cfg.head_dim, cfg.rope_theta, self.device)
        self._buffers()
        self.graph = None
        if capture:
            self._capture()

    def _buffers(self):
        cfg, dev, B = self.cfg, self.device, self.batch
        H, HQ, HKV, D, I = cfg.hidden, cfg.heads, cfg.kv_heads, cfg.head_dim, cfg.inter

        def z(*shape, dtype=BF16):
            return torch.zeros(*shape, device=dev, dtype=dtype)

        f32 = torch.float32
        self.h = z(B, H)
        self.h1 = z(B, H)
        self.ssq = z(C.skinny_residual_blocks(H), B, dtype=torch.float32)
        self.xn = z(B, H)
        self.act = z(B, I)
        self.attn = z(B, HQ * D)
        self.q = z(B, HQ * D)
        self.qkv_part = z(self.ks["qkv"], B, cfg.qkv_rows, dtype=f32)
        self.o_part = z(self.ks["o"], B, H, dtype=f32)
        self.d_part = z(self.ks["down"], B, H, dtype=f32)
        self.op = z(B, self.ns, HQ, D, dtype=f32)
        self.mp = z(B, self.ns, HQ, dtype=f32)
        self.lp = z(B, self.ns, HQ, dtype=f32)
        self.kc = z(cfg.layers, B, self.cap, HKV * D)
        self.vc = z(cfg.layers, B, self.cap, HKV * D)
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

    def _step(self, keep_logits: bool = False):
        cfg = self.cfg
        HQ, HKV = cfg.heads, cfg.kv_heads
        L = len(self.layers)
        C.rows_norm(self.embed, self.ids, None, None, self.h, self.layers[0]["gamma_in"], self.xn,
                    cfg.eps, self.err)
        for i, w in enumerate(self.layers):
            C.skinny_gemm(self.xn, w["w_qkv"], self.ks["qkv"], 0, self.qkv_part, None, None, None,
                          None)
            if self.attention == "seq":
                C.decode_attention_seq(self.qkv_part, w["gamma_q"], w["gamma_k"], cfg.eps, self.cos, self.sin,
                                       self.pos, self.pos, self.kc[i], self.vc[i], HQ, HKV, cfg.scale, self.attn,
                                       self.err)
            else:
                # the query prepared once per sequence, not once per split block
                C.qk_rope_cache(self.qkv_part, w["gamma_q"], w["gamma_k"], cfg.eps, self.cos, self.sin,
                                self.pos, self.pos, self.kc[i], self.vc[i], self.q, HQ, HKV, self.err)
                C.decode_attention(self.q, None, None, None, 0.0, None, None, self.kc[i], self.vc[i], None,
                                   self.pos, HQ, HKV, self.split, cfg.scale, self.op, self.mp, self.lp,
                                   False, self.err)
                C.attn_combine(self.op, self.mp, self.lp, self.attn, self.pos, self.split)
            if self.fold_o_norm:
                C.skinny_gemm_residual(self.attn, w["w_o"], self.h, self.h1, self.ssq)
                C.skinny_gemm_norm_swiglu(self.h1, w["w_gu"], self.ssq, w["gamma_post"], cfg.eps, self.act)
            else:
                C.skinny_gemm(self.attn, w["w_o"], self.ks["o"], 0, self.o_part, None, None, None, None)
                C.rows_norm(None, None, self.h, self.o_part, self.h1, w["gamma_post"], self.xn, cfg.eps,
                            self.err)
                C.skinny_gemm(self.xn, w["w_gu"], 1, 1, None, self.act, None, None, None)
            C.skinny_gemm(self.act, w["w_down"], self.ks["down"], 0, self.d_part, None, None, None,
                          None)
            nxt = self.layers[i + 1]["gamma_in"] if i + 1 < L else self.gamma_final
            C.rows_norm(None, None, self.h1, self.d_part, self.h, nxt, self.xn, cfg.eps, self.err)
        C.skinny_gemm(self.xn, self.head, 1, 2, None, None, self.logits if keep_logits else None,
                      self.bv, self.bi)
        C.batch_sample_step(self.bv, self.bi, self.inp, self.plen, self.ids, self.pos, self.sam,
                            self.err)

    _capture = Engine._capture
    _run_step = Engine._run_step
    from_checkpoint = classmethod(Engine.from_checkpoint.__func__)
    _walk_or_prefill = Engine._walk_or_prefill

    def _capture_inputs(self):
        return [[0]] * self.batch, 1
    check_device_errors = Engine.check_device_errors

    def _reset(self):
        self.pos.zero_()
        self.sam.zero_()
        self.err.zero_()

    def _load(self, rows: list[list[int]], plen: int):
        if len(rows) != self.batch:
            raise ValueError(f"{len(rows)} sequences given to an engine of batch {self.batch}")
        if any(len(r) != len(rows[0]) for r in rows):
            raise ValueError("sequences of one batch advance in lockstep: give equal lengths")
        if len(rows[0]) > self.nsteps:
            raise ValueError(f"{len(rows[0])} input ids exceed this engine's {self.nsteps} steps")
        if any(not 0 <= t < self.cfg.vocab for r in rows for t in r):
            raise ValueError(f"token ids out of range [0, {self.cfg.vocab})")
        self._reset()
        self.inp.zero_()
        self.inp[:, : len(rows[0])] = torch.tensor(rows, dtype=torch.int32, device=self.device)
        self.plen.fill_(plen)
        self.ids.copy_(torch.tensor([r[0] for r in rows], dtype=torch.int64, device=self.device))

    def generate(self, prompts: list[list[int]], max_new: int) -> Generated:
        """Walk (or prefill) every prompt, then continue each for ``max_new``
        tokens; timing covers the continuation steps only (all sequences together)."""
        if not prompts or not prompts[0]:
            raise ValueError("decode needs prompts of at least one token")
        pl = len(prompts[0])
        if pl + max_new > self.nsteps:
            raise ValueError(f"prompt {pl} + {max_new} new exceeds this engine's {self.nsteps} steps")
        self._load([list(p) for p in prompts], pl)
        torch.cuda.synchronize(self.device)
        t0 = perf_counter()
        self._walk_or_prefill([list(p) for p in prompts])
        torch.cuda.synchronize(self.device)
        t1 = perf_counter()
        for _ in range(max_new):
            self._run_step()
        torch.cuda.synchronize(self.device)
        t2 = perf_counter()
        self.check_device_errors()
        out = self.sam[:, pl - 1: pl - 1 + max_new].tolist()
        return Generated(out, t2 - t1, t1 - t0, pl)

    def forced(self, prompts: list[list[int]], teachers: list[list[int]], record_logits: bool = False):
        """Teacher-forced picks of every sequence: position ``len(prompt) - 1 + i``
        of sequence b is fed ``teachers[b][i - 1]``; the prompts are walked, or
        prefilled with ``prompt_prefill``. Returns the picks ``[batch]
        [len(teacher) + 1]`` (and, when asked, the f32 logits ``[batch, vocab]`` of
        each of those positions: those steps run eagerly, since the captured step
        writes only the per-group winners)."""
        if len(teachers) != self.batch or any(len(t) != len(teachers[0]) for t in teachers):
            raise ValueError(f"give {self.batch} teacher sequences of equal length")
        rows = [list(p) + list(t) for p, t in zip(prompts, teachers)]
        self._load(rows, len(rows[0]))
        pl = len(prompts[0])
        self._walk_or_prefill([list(p) for p in prompts])
        logits = []
        for _ in range(pl - 1, len(rows[0])):
            if record_logits:
                self._step(keep_logits=True)
                logits.append(self.logits.clone())
            else:
                self._run_step()
        torch.cuda.synchronize(self.device)
        self.check_device_errors()
        picks = self.sam[:, pl - 1: len(rows[0])].tolist()
        return (picks, logits) if record_logits else picks

    def logits_for(self, prompts: list[list[int]]) -> torch.Tensor:
        """f32 logits [batch, vocab] after consuming every token of each prompt
        (eager steps: the captured step writes only the per-group winners)."""
        self._load([list(p) for p in prompts], len(prompts[0]))
        for _ in range(len(prompts[0])):
            self._step(keep_logits=True)
        torch.cuda.synchronize(self.device)
        self.check_device_errors()
        return self.logits.clone()
