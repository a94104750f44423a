"""Published checkpoints as engine weights: a safetensors directory reader and
the Hugging Face config / name mapping for the Qwen3 decode model.

The reference reads a checkpoint directory through ``SafetensorsResource``
(src/tilefoundry/runtime/resource.py:187-300): N shards plus
``model.safetensors.index.json``, or one unsharded ``model.safetensors`` with no
index, each shard opened once and memory-mapped, tensors read onto the
device on demand. Its ``hf_alias`` table
(examples/qwen3_1_7b-tilelang/ref_src/hf_alias.py:25-43) maps the model's canonical
weight names onto the published ``model.layers.{i}.*`` keys, and the engine packs
them (fast/engine.py:110-133).

Here the engines take the published names directly (``qwen3.hf_names``, the
same keys the alias table points at) in the published ``(out, in)`` layout, so
no layout conversion happens on load: every tensor goes from the memory map
to the device once, as bf16, and ``qwen3.pack_weights`` builds the fused
matrices. ``lm_head.weight`` is kept when the checkpoint ships one (an untied
head); without it the embedding doubles as the head, as
``tie_word_embeddings`` says for Qwen3-1.7B.
"""
from __future__ import annotations

import json
from pathlib import Path

import torch

BF16 = torch.bfloat16
INDEX = "model.safetensors.index.json"
SINGLE = "model.safetensors"


class SafetensorsCheckpoint:
    """A safetensors checkpoint directory, sharded (with an index) or not.

    ``keys()`` lists every tensor name; ``read(name)`` returns it on ``device``
    (bf16 unless ``dtype`` says otherwise). Shards are memory-mapped and each
    is opened at most once. Missing directories, shards and keys raise
    ``FileNotFoundError`` / ``KeyError`` naming what is missing (the reference's
    error classes for a missing resource and a missing weight)."""

    def __init__(self, path: str | Path, device="cpu"):
        from safetensors import safe_open  # noqa: F401  (fail early when the package is absent)

        self.dir = Path(path)
        self.device = torch.device(device)
        if not self.dir.is_dir():
            raise FileNotFoundError(f"checkpoint directory {self.dir} does not exist")
        index = self.dir / INDEX
        if index.is_file():
            with open(index, encoding="utf-8") as fh:
                self._shard_of = dict(json.load(fh)["weight_map"])
        elif (self.dir / SINGLE).is_file():
            self._shard_of = dict.fromkeys(self._open(SINGLE).keys(), SINGLE)
        else:
            raise FileNotFoundError(f"{self.dir} holds neither {INDEX} nor {SINGLE}")
        self._handles: dict[str, object] = {}

    def _open(self, shard: str):
        from safetensors import safe_open

        path = self.dir / shard
        if not path.is_file():
            raise FileNotFoundError(f"checkpoint shard {path} (named by {INDEX}) does not exist")
        return safe_open(str(path), framework="pt", device="cpu")

    def keys(self) -> list[str]:
        return sorted(self._shard_of)

    def __contains__(self, name: str) -> bool:
        return name in self._shard_of

    def read(self, name: str, dtype=BF16) -> torch.Tensor:
        shard = self._shard_of.get(name)
        if shard is None:
            raise KeyError(f"weight {name!r} is not in the checkpoint at {self.dir}")
        h = self._handles.get(shard)
        if h is None:
            h = self._handles[shard] = self._open(shard)
        t = h.get_tensor(name)
        return t.to(device=self.device, dtype=dtype).contiguous()


def qwen3_config(path: str | Path):
    """``config.json`` of a Qwen3 checkpoint (the Hugging Face fields of
    examples/qwen3_1_7b-tilelang/ref_src/config.json) -> ``Qwen3Config``.

    Returns ``(cfg, tied)``, ``tied`` being ``tie_word_embeddings``. A config that
    asks for what the decode kernels do not compute (attention bias, rope
    scaling, sliding windows, an activation other than silu) raises ValueError."""
    from .qwen3 import Qwen3Config

    with open(Path(path) / "config.json", encoding="utf-8") as fh:
        c = json.load(fh)
    if c.get("attention_bias"):
        raise ValueError("config.json: attention_bias is not supported by the decode kernels")
    if c.get("rope_scaling"):
        raise ValueError("config.json: rope_scaling is not supported by the decode kernels")
    if c.get("use_sliding_window"):
        raise ValueError("config.json: sliding-window attention is not supported")
    if c.get("hidden_act", "silu") != "silu":
        raise ValueError(f"config.json: hidden_act {c['hidden_act']!r}, only silu is supported")
    heads = int(c["num_attention_heads"])
    cfg = Qwen3Config(
        hidden=int(c["hidden_size"]), heads=heads,
        kv_heads=int(c.get("num_key_value_heads", heads)),
        head_dim=int(c.get("head_dim", int(c["hidden_size"]) // heads)),
        inter=int(c["intermediate_size"]), vocab=int(c["vocab_size"]),
        layers=int(c["num_hidden_layers"]), eps=float(c.get("rms_norm_eps", 1e-6)),
        rope_theta=float(c.get("rope_theta", 1.0e6)),
        max_pos=int(c.get("max_position_embeddings", 40960)))
    return cfg, bool(c.get("tie_word_embeddings", False))


def load_qwen3(path: str | Path, device="cpu", cfg=None) -> tuple:
    """Every tensor the Qwen3 engines use, read from the checkpoint at ``path``
    onto ``device`` as bf16, under the published names.

    Returns ``(cfg, weights)``; ``weights`` holds ``lm_head.weight`` only when the
    checkpoint ships an untied head (``tie_word_embeddings`` false, or -- with an
    explicit ``cfg`` -- whenever the checkpoint has one). Shapes are checked
    against the config, so a checkpoint of another model fails here with the
    name of the first tensor that disagrees rather than inside a kernel."""
    from .qwen3 import hf_names

    ck = SafetensorsCheckpoint(path, device)
    if cfg is None:
        cfg, tied = qwen3_config(path)
    else:
        tied = "lm_head.weight" not in ck
    H, HQ, HKV, D, I = cfg.hidden, cfg.heads, cfg.kv_heads, cfg.head_dim, cfg.inter
    shapes = {
        "gamma_in": (H,), "w_q": (HQ * D, H), "w_k": (HKV * D, H), "w_v": (HKV * D, H),
        "gamma_q": (D,), "gamma_k": (D,), "w_o": (H, HQ * D), "gamma_post": (H,),
        "w_gate": (I, H), "w_up": (I, H), "w_down": (H, I),
    }
    want = {"model.embed_tokens.weight": (cfg.vocab, H), "model.norm.weight": (H,)}
    for i in range(cfg.layers):
        for key, name in hf_names(i).items():
            want[name] = shapes[key]
    if not tied:
        want["lm_head.weight"] = (cfg.vocab, H)
    out = {}
    for name, shape in want.items():
        t = ck.read(name)
        if tuple(t.shape) != shape:
            raise ValueError(f"checkpoint weight {name}: shape {tuple(t.shape)}, the config says {shape}")
        out[name] = t
    return cfg, out


# ------------------------------------------------------------------ MiniCPM3
def minicpm3_config(path: str | Path):
    """``config.json`` of a MiniCPM3 checkpoint (the fields of
    examples/minicpm3_4b-cutedsl/config.json) -> ``minicpm3.MiniCPM3Config``. A
    rope scaling other than longrope, or longrope whose short and long factors
    differ while the cache could pass ``original_max_position_embeddings``, is
    for the engine to refuse; here the fields are only read."""
    from dataclasses import replace

    from .minicpm3 import MINICPM3_4B

    with open(Path(path) / "config.json", encoding="utf-8") as fh:
        c = json.load(fh)
    if c.get("hidden_act", "silu") != "silu":
        raise ValueError(f"config.json: hidden_act {c['hidden_act']!r}, only silu is supported")
    rs = c.get("rope_scaling") or {}
    if rs and rs.get("type", rs.get("rope_type")) != "longrope":
        raise ValueError(f"config.json: rope_scaling type {rs.get('type')!r}, only longrope is supported")
    heads = int(c["num_attention_heads"])
    if int(c.get("num_key_value_heads", heads)) != heads:
        raise ValueError("config.json: MLA needs num_key_value_heads == num_attention_heads")
    short = tuple(float(x) for x in rs.get("short_factor", MINICPM3_4B.short_factor))
    hidden = int(c["hidden_size"])
    return replace(
        MINICPM3_4B, hidden=hidden, heads=heads, q_lora=int(c["q_lora_rank"]), kv_lora=int(c["kv_lora_rank"]),
        nope=int(c["qk_nope_head_dim"]), rope=int(c["qk_rope_head_dim"]),
        v_dim=int(c.get("v_head_dim", c["qk_nope_head_dim"])), layers=int(c["num_hidden_layers"]),
        eps=float(c.get("rms_norm_eps", 1e-5)), rope_theta=float(c.get("rope_theta", 10000.0)),
        scale_depth=float(c.get("scale_depth", 1.4)), short_factor=short, inter=int(c["intermediate_size"]),
        vocab=int(c["vocab_size"]), scale_emb=float(c.get("scale_emb", 1.0)),
        dim_model_base=int(c.get("dim_model_base", hidden)),
        original_max_pos=int(rs.get("original_max_position_embeddings", c.get("max_position_embeddings", 32768))))


class _TorchBinCheckpoint:
    """A single ``pytorch_model.bin`` read with ``torch.load(weights_only=True)``:
    tensors only, nothing in the file is executed."""

    def __init__(self, path: Path, device):
        self.device = torch.device(device)
        self._sd = torch.load(str(path), map_location="cpu", weights_only=True)

    def keys(self) -> list[str]:
        return sorted(self._sd)

    def __contains__(self, name: str) -> bool:
        return name in self._sd

    def read(self, name: str, dtype=BF16) -> torch.Tensor:
        if name not in self._sd:
            raise KeyError(f"weight {name!r} is not in the checkpoint")
        return self._sd[name].to(device=self.device, dtype=dtype).contiguous()


def load_minicpm3(path: str | Path, device="cpu", cfg=None) -> tuple:
    """Every tensor ``minicpm3.MiniCPM3Engine`` uses, from a MiniCPM3 checkpoint at
    ``path`` -- safetensors (sharded or single) or the published single
    ``pytorch_model.bin`` (read without unpickling code) -- onto ``device`` as
    bf16 under the published names, shapes checked against the config.
    Returns ``(cfg, weights)``; an ``lm_head.weight`` is kept only when
    ``tie_word_embeddings`` is false (MiniCPM3 ties it)."""
    from .minicpm3 import hf_layer_names

    p = Path(path)
    if (p / INDEX).is_file() or (p / SINGLE).is_file():
        ck = SafetensorsCheckpoint(p, device)
    elif (p / "pytorch_model.bin").is_file():
        ck = _TorchBinCheckpoint(p / "pytorch_model.bin", device)
    else:
        raise FileNotFoundError(f"{p} holds neither safetensors shards nor pytorch_model.bin")
    tied = True
    if cfg is None:
        cfg = minicpm3_config(p)
        with open(p / "config.json", encoding="utf-8") as fh:
            tied = bool(json.load(fh).get("tie_word_embeddings", True))
    H, NH, QA, KV, R = cfg.hidden, cfg.heads, cfg.q_lora, cfg.kv_lora, cfg.rope
    shapes = {
        "gamma_in": (H,), "w_q_a": (QA, H), "gamma_q_a": (QA,), "w_q_b": (NH * (cfg.nope + R), QA),
        "w_kv_a": (KV + R, H), "gamma_kv_a": (KV,), "w_kv_b": (NH * (cfg.nope + cfg.v_dim), KV),
        "w_o": (H, NH * cfg.v_dim), "gamma_post": (H,), "w_gate": (cfg.inter, H), "w_up": (cfg.inter, H),
        "w_down": (H, cfg.inter),
    }
    want = {"model.embed_tokens.weight": (cfg.vocab, H), "model.norm.weight": (H,)}
    for i in range(cfg.layers):
        for key, name in hf_layer_names(i).items():
            want[name] = shapes[key]
    if not tied:
        want["lm_head.weight"] = (cfg.vocab, H)
    out = {}
    for name, shape in want.items():
        t = ck.read(name)
        if tuple(t.shape) != shape:
            raise ValueError(f"checkpoint weight {name}: shape {tuple(t.shape)}, the config says {shape}")
        out[name] = t
    return cfg, out
