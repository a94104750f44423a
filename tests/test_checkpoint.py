"""The checkpoint path: a safetensors directory written here (single file,
sharded with an index, tied and untied heads) read back through
``checkpoint.load_qwen3`` and run by the engines.

The reader follows the reference's ``SafetensorsResource`` contract
(src/tilefoundry/runtime/resource.py:187-300) and its ``hf_alias`` names
(examples/qwen3_1_7b-tilelang/ref_src/hf_alias.py:25-43). No published checkpoint
is available here, so the files are synthetic weights of the published layout;
tests/golden/qwen3_1_7b_config/config.json is the reference's own
examples/qwen3_1_7b-tilelang/ref_src/config.json, kept as a data fixture.
"""
import json

import pytest
import torch

from tilefoundry_amd.checkpoint import SafetensorsCheckpoint, load_qwen3, qwen3_config
from tilefoundry_amd.qwen3 import Qwen3Config, pack_weights, synthetic_weights

TINY = Qwen3Config(hidden=256, heads=4, kv_heads=2, head_dim=64, inter=512, vocab=1000, layers=2)


def _hf_config(cfg: Qwen3Config, tied=True, **extra) -> dict:
    c = {"architectures": ["Qwen3ForCausalLM"], "attention_bias": False, "head_dim": cfg.head_dim,
         "hidden_act": "silu", "hidden_size": cfg.hidden, "intermediate_size": cfg.inter,
         "max_position_embeddings": cfg.max_pos, "model_type": "qwen3",
         "num_attention_heads": cfg.heads, "num_hidden_layers": cfg.layers,
         "num_key_value_heads": cfg.kv_heads, "rms_norm_eps": cfg.eps, "rope_scaling": None,
         "rope_theta": cfg.rope_theta, "tie_word_embeddings": tied, "torch_dtype": "bfloat16",
         "use_sliding_window": False, "vocab_size": cfg.vocab}
    c.update(extra)
    return c


def write_checkpoint(path, cfg, wts, shards=1, tied=True, **extra):
    """``wts`` under the published names as a checkpoint directory: one
    ``model.safetensors``, or ``shards`` files plus ``model.safetensors.index.json``."""
    from safetensors.torch import save_file

    path.mkdir(parents=True, exist_ok=True)
    (path / "config.json").write_text(json.dumps(_hf_config(cfg, tied, **extra)))
    names = sorted(wts)
    cpu = {k: v.detach().to("cpu").contiguous() for k, v in wts.items()}
    if shards == 1:
        save_file(cpu, str(path / "model.safetensors"))
        return path
    weight_map = {}
    for s in range(shards):
        part = names[s::shards]
        fname = f"model-{s + 1:05d}-of-{shards:05d}.safetensors"
        save_file({k: cpu[k] for k in part}, str(path / fname))
        weight_map.update(dict.fromkeys(part, fname))
    (path / "model.safetensors.index.json").write_text(json.dumps({"metadata": {}, "weight_map": weight_map}))
    return path


def test_config_fields():
    from pathlib import Path

    cfg, tied = qwen3_config(Path(__file__).parent / "golden" / "qwen3_1_7b_config")
    assert tied
    assert (cfg.hidden, cfg.heads, cfg.kv_heads, cfg.head_dim, cfg.inter, cfg.vocab, cfg.layers) == \
        (2048, 16, 8, 128, 6144, 151936, 28)
    assert cfg.eps == 1e-6 and cfg.rope_theta == 1.0e6


@pytest.mark.parametrize("shards", [1, 3])
def test_round_trip(tmp_path, shards):
    wts = synthetic_weights(TINY, seed=4)
    write_checkpoint(tmp_path, TINY, wts, shards=shards)
    cfg, got = load_qwen3(tmp_path)
    assert cfg == TINY
    assert sorted(got) == sorted(wts)
    for k, v in wts.items():
        assert torch.equal(got[k], v), k
    ck = SafetensorsCheckpoint(tmp_path)
    assert ck.keys() == sorted(wts)


def test_untied_head(tmp_path):
    wts = synthetic_weights(TINY, seed=5)
    head = torch.randn(TINY.vocab, TINY.hidden).to(torch.bfloat16)
    write_checkpoint(tmp_path / "untied", TINY, {**wts, "lm_head.weight": head}, tied=False)
    _, got = load_qwen3(tmp_path / "untied")
    assert torch.equal(got["lm_head.weight"], head)
    embed, _, _, packed_head = pack_weights(TINY, got, "cpu")
    assert torch.equal(packed_head, head) and not torch.equal(packed_head, embed)
    # a tied config ignores a stored head copy; the embedding serves
    write_checkpoint(tmp_path / "tied", TINY, {**wts, "lm_head.weight": head}, tied=True)
    _, got = load_qwen3(tmp_path / "tied")
    assert "lm_head.weight" not in got
    embed, _, _, packed_head = pack_weights(TINY, got, "cpu")
    assert packed_head is embed
    # untied by the config but no head stored: the missing weight is named
    write_checkpoint(tmp_path / "nohead", TINY, wts, tied=False)
    with pytest.raises(KeyError, match="lm_head.weight"):
        load_qwen3(tmp_path / "nohead")


def test_errors(tmp_path):
    with pytest.raises(FileNotFoundError):
        SafetensorsCheckpoint(tmp_path / "absent")
    (tmp_path / "empty").mkdir()
    with pytest.raises(FileNotFoundError, match="neither"):
        SafetensorsCheckpoint(tmp_path / "empty")
    wts = synthetic_weights(TINY, seed=6)
    short = {k: v for k, v in wts.items() if "layers.1.mlp.up_proj" not in k}
    write_checkpoint(tmp_path / "short", TINY, short, shards=2)
    with pytest.raises(KeyError, match="layers.1.mlp.up_proj"):
        load_qwen3(tmp_path / "short")
    bad = dict(wts)
    bad["model.layers.0.self_attn.k_proj.weight"] = torch.zeros(3, TINY.hidden, dtype=torch.bfloat16)
    write_checkpoint(tmp_path / "shape", TINY, bad)
    with pytest.raises(ValueError, match="k_proj"):
        load_qwen3(tmp_path / "shape")
    write_checkpoint(tmp_path / "scaled", TINY, wts, rope_scaling={"type": "yarn", "factor": 4.0})
    with pytest.raises(ValueError, match="rope_scaling"):
        load_qwen3(tmp_path / "scaled")
    # an index naming a shard that is not there
    write_checkpoint(tmp_path / "lost", TINY, wts, shards=2)
    next((tmp_path / "lost").glob("model-00002-*")).unlink()
    with pytest.raises(FileNotFoundError, match="shard"):
        load_qwen3(tmp_path / "lost")


# ------------------------------------------------------------------ engines
@pytest.mark.gpu
def test_engine_from_checkpoint_matches_in_memory_weights(dev, tmp_path):
    """A 2-layer Qwen3-1.7B-shaped model written as a sharded checkpoint and
    loaded by ``Engine.from_checkpoint`` decodes the same ids, bit for bit, as
    the engine built from the same weights in memory; the batched engine too."""
    from tilefoundry_amd.qwen3 import BatchEngine, Engine

    cfg = Qwen3Config(layers=2, vocab=8192)
    wts = synthetic_weights(cfg, seed=7)
    write_checkpoint(tmp_path, cfg, wts, shards=2)
    prompt = list(range(100, 120))
    a = Engine(cfg, device=dev, max_new=24, prompt_room=32, weights=wts).generate(prompt, 16).tokens
    eng = Engine.from_checkpoint(tmp_path, None, device=dev, max_new=24, prompt_room=32)
    assert eng.cfg == cfg
    assert eng.generate(prompt, 16).tokens == a
    rows = [prompt, list(range(200, 220))]
    want = BatchEngine(cfg, device=dev, batch=2, max_new=24, prompt_room=32, weights=wts).generate(rows, 16).tokens
    beng = BatchEngine.from_checkpoint(tmp_path, device=dev, batch=2, max_new=24, prompt_room=32)
    assert beng.generate(rows, 16).tokens == want


@pytest.mark.gpu
def test_engine_untied_head_against_oracle(dev, tmp_path):
    """An untied head is the one the engine multiplies by: logits against the
    oracle given the same separate head."""
    from oracle import qwen3 as OQ
    from tests._check import assert_close
    from tests.test_qwen3_engine import oracle_cfg, oracle_model
    from tilefoundry_amd.qwen3 import Engine

    cfg = Qwen3Config(layers=2, vocab=8192)
    wts = synthetic_weights(cfg, seed=8)
    head = (0.02 * torch.randn(cfg.vocab, cfg.hidden, generator=torch.Generator().manual_seed(9))).to(torch.bfloat16)
    write_checkpoint(tmp_path, cfg, {**wts, "lm_head.weight": head}, tied=False)
    eng = Engine.from_checkpoint(tmp_path, device=dev, max_new=8, prompt_room=16)
    prompt = list(range(3, 13))
    got = eng.logits_for(prompt)
    om = oracle_model(wts, cfg)
    om._head32 = head.float()
    oc = oracle_cfg(cfg)
    cos, sin = OQ.rope_tables(len(prompt), cfg.head_dim, cfg.rope_theta)
    caches = OQ.empty_caches(oc, cfg.layers)
    for p, t in enumerate(prompt):
        ref = OQ.step(om, oc, t, p, caches, cos, sin, p_bf16=True)
    assert_close("untied-head logits", got, ref)


# ------------------------------------------------------------------ MiniCPM3
def _minicpm3_hf_config(cfg, tied=True):
    return {"architectures": ["MiniCPM3ForCausalLM"], "hidden_act": "silu", "hidden_size": cfg.hidden,
            "num_hidden_layers": cfg.layers, "intermediate_size": cfg.inter, "num_attention_heads": cfg.heads,
            "num_key_value_heads": cfg.heads, "qk_nope_head_dim": cfg.nope, "qk_rope_head_dim": cfg.rope,
            "q_lora_rank": cfg.q_lora, "kv_lora_rank": cfg.kv_lora, "rms_norm_eps": cfg.eps,
            "rope_scaling": {"type": "longrope", "long_factor": list(cfg.short_factor),
                             "short_factor": list(cfg.short_factor),
                             "original_max_position_embeddings": cfg.original_max_pos},
            "vocab_size": cfg.vocab, "scale_emb": cfg.scale_emb, "dim_model_base": cfg.dim_model_base,
            "scale_depth": cfg.scale_depth, "tie_word_embeddings": tied, "max_position_embeddings": 32768}


def _write_minicpm3(path, cfg, wts, shards=1, bin_file=False):
    from safetensors.torch import save_file

    path.mkdir(parents=True, exist_ok=True)
    (path / "config.json").write_text(json.dumps(_minicpm3_hf_config(cfg)))
    cpu = {k: v.detach().to("cpu").contiguous() for k, v in wts.items()}
    if bin_file:
        torch.save(cpu, str(path / "pytorch_model.bin"))
        return path
    names = sorted(cpu)
    if shards == 1:
        save_file(cpu, str(path / "model.safetensors"))
        return path
    wm = {}
    for s in range(shards):
        part = names[s::shards]
        fname = f"model-{s + 1:05d}-of-{shards:05d}.safetensors"
        save_file({k: cpu[k] for k in part}, str(path / fname))
        wm.update(dict.fromkeys(part, fname))
    (path / "model.safetensors.index.json").write_text(json.dumps({"metadata": {}, "weight_map": wm}))
    return path


def test_minicpm3_published_config():
    from pathlib import Path

    from tilefoundry_amd.checkpoint import minicpm3_config
    from tilefoundry_amd.minicpm3 import MINICPM3_4B

    cfg = minicpm3_config(Path(__file__).parent / "golden" / "minicpm3_4b_config")
    assert cfg == MINICPM3_4B
    assert cfg.logits_scaling == 10.0


@pytest.mark.parametrize("form", ["single", "sharded", "bin"])
def test_minicpm3_round_trip(tmp_path, form):
    from dataclasses import replace

    from tilefoundry_amd.checkpoint import load_minicpm3
    from tilefoundry_amd.minicpm3 import MINICPM3_4B, synthetic_model_weights

    cfg = replace(MINICPM3_4B, hidden=256, heads=4, q_lora=96, kv_lora=64, inter=512, vocab=512, layers=2,
                  dim_model_base=64)
    wts = synthetic_model_weights(cfg, seed=3)
    _write_minicpm3(tmp_path, cfg, wts, shards=3 if form == "sharded" else 1, bin_file=form == "bin")
    got_cfg, got = load_minicpm3(tmp_path)
    assert got_cfg == cfg
    assert sorted(got) == sorted(wts)
    for k, v in wts.items():
        assert torch.equal(got[k], v), k


def test_minicpm3_checkpoint_errors(tmp_path):
    from dataclasses import replace

    from tilefoundry_amd.checkpoint import load_minicpm3
    from tilefoundry_amd.minicpm3 import MINICPM3_4B, synthetic_model_weights

    with pytest.raises(FileNotFoundError):
        (tmp_path / "empty").mkdir()
        load_minicpm3(tmp_path / "empty")
    cfg = replace(MINICPM3_4B, hidden=256, heads=4, q_lora=96, kv_lora=64, inter=512, vocab=512, layers=1,
                  dim_model_base=64)
    wts = synthetic_model_weights(cfg, seed=4)
    p = _write_minicpm3(tmp_path / "yarn", cfg, wts)
    c = json.loads((p / "config.json").read_text())
    c["rope_scaling"]["type"] = "yarn"
    (p / "config.json").write_text(json.dumps(c))
    with pytest.raises(ValueError, match="longrope"):
        load_minicpm3(p)
    short = {k: v for k, v in wts.items() if "kv_b_proj" not in k}
    with pytest.raises(KeyError, match="kv_b_proj"):
        load_minicpm3(_write_minicpm3(tmp_path / "short", cfg, short))


@pytest.mark.gpu
def test_minicpm3_engine_from_checkpoint(dev, tmp_path):
    """A 2-layer MiniCPM3-4B-shaped checkpoint (published layer shapes, vocab 4096)
    decodes the same ids through ``MiniCPM3Engine.from_checkpoint`` as the engine
    built from the same weights in memory."""
    from dataclasses import replace

    from tilefoundry_amd.minicpm3 import MINICPM3_4B, MiniCPM3Engine, synthetic_model_weights

    cfg = replace(MINICPM3_4B, layers=2, vocab=4096)
    wts = synthetic_model_weights(cfg, seed=5)
    _write_minicpm3(tmp_path, cfg, wts, shards=2)
    prompt = [[7, 70, 700, 3000]]
    want = MiniCPM3Engine(cfg, device=dev, max_new=16, prompt_room=8, weights=wts).generate(prompt, 10).tokens
    eng = MiniCPM3Engine.from_checkpoint(tmp_path, device=dev, max_new=16, prompt_room=8)
    assert eng.cfg == cfg
    assert eng.generate(prompt, 10).tokens == want
