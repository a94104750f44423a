"""The captured decode step end to end against the CPU oracle's greedy decode.

Whole-model comparisons use the oracle's kernel-order attention (softmax
weights landed in bf16 before P.V, as the reference kernel and Hugging Face
do): the torch spelling keeps them in f32, and that one rounding alone moves a
2-layer model's logits by ~1% relative L2, which would hide real differences.

Small stacks (Qwen3-1.7B layer shapes, fewer layers, smaller vocabulary) run
the live oracle; the full 28-layer / 151936-vocab model is checked against
golden ids the oracle wrote (tests/golden/make_qwen3_golden.py).
"""
import json
from pathlib import Path

import pytest
import torch

from oracle import qwen3 as OQ
from tests._check import assert_close, assert_l2, max_rel

GOLDEN = Path(__file__).parent / "golden"


def oracle_model(wts: dict, cfg) -> OQ.ModelWeights:
    from tilefoundry_amd.qwen3 import hf_names

    layers = []
    for i in range(cfg.layers):
        n = hf_names(i)
        layers.append(OQ.LayerWeights(**{k: wts[v] for k, v in n.items()}))
    return OQ.ModelWeights(embed=wts["model.embed_tokens.weight"],
                           gamma_final=wts["model.norm.weight"], layers=layers)


def oracle_cfg(cfg) -> OQ.Qwen3Config:
    return OQ.Qwen3Config(hidden=cfg.hidden, heads=cfg.heads, kv_heads=cfg.kv_heads,
                          head_dim=cfg.head_dim, inter=cfg.inter, vocab=cfg.vocab,
                          layers=cfg.layers, eps=cfg.eps, rope_theta=cfg.rope_theta)


def _small(layers=2, vocab=8192):
    from tilefoundry_amd.qwen3 import Qwen3Config, synthetic_weights

    cfg = Qwen3Config(layers=layers, vocab=vocab)
    wts = synthetic_weights(cfg, seed=5)
    return cfg, wts


@pytest.mark.gpu
def test_engine_logits_small(dev):
    from tilefoundry_amd.qwen3 import Engine

    cfg, wts = _small()
    eng = Engine(cfg, device=dev, max_new=64, prompt_room=64, weights=wts)
    prompt = OQ.prompt_ids(cfg.vocab, 12, seed=1)[0]
    got = eng.logits_for(prompt)
    om, oc = oracle_model(wts, cfg), oracle_cfg(cfg)
    cos, sin = OQ.rope_tables(len(prompt), cfg.head_dim, cfg.rope_theta)
    caches = OQ.empty_caches(oc, cfg.layers)
    for p, t in enumerate(prompt):
        ref = OQ.step(om, oc, t, p, caches, cos, sin, p_bf16=True)
    assert_close("logits", got, ref)
    # The cache rows the engine wrote are the oracle's cache, position for
    # position. Layer 0 sees the same inputs as the oracle (the embedding), so it
    # is held to the per-op bar; deeper layers carry a whole layer of independent
    # bf16 landings and are held to relative L2.
    for i in range(cfg.layers):
        kc = eng.kc[i, : len(prompt)].view(len(prompt), cfg.kv_heads, cfg.head_dim)
        vc = eng.vc[i, : len(prompt)].view(len(prompt), cfg.kv_heads, cfg.head_dim)
        check = assert_close if i == 0 else assert_l2
        check(f"k cache layer {i}", kc, caches[i][0])
        check(f"v cache layer {i}", vc, caches[i][1])
        assert float(eng.kc[i, len(prompt):].abs().max()) == 0.0, "rows past the context untouched"


@pytest.mark.gpu
def test_engine_greedy_small(dev):
    """Free-running greedy ids equal the oracle's for every step where the
    oracle's own top-2 margin is resolvable at bf16 precision."""
    from tilefoundry_amd.qwen3 import Engine

    cfg, wts = _small()
    eng = Engine(cfg, device=dev, max_new=64, prompt_room=64, weights=wts)
    prompt = OQ.prompt_ids(cfg.vocab, 16, seed=2)[0]
    gen = eng.generate(prompt, 32)
    rec = []
    want = OQ.decode(oracle_model(wts, cfg), oracle_cfg(cfg), prompt, 32, record=rec, p_bf16=True)
    first_diff = next((i for i, (a, b) in enumerate(zip(gen.tokens, want)) if a != b), None)
    if first_diff is not None:
        logits, pick, gap = rec[first_diff]
        tol = 1e-2 * float(logits.abs().max())
        assert gap < tol, f"step {first_diff}: {gen.tokens[first_diff]} != {want[first_diff]} with a clear margin {gap:.4g}"
    assert gen.tokens == want or first_diff >= 8


@pytest.mark.gpu
def test_engine_teacher_forced_small(dev):
    """Teacher-forced picks and logits agree with the oracle position by position."""
    from tilefoundry_amd.qwen3 import Engine

    cfg, wts = _small()
    eng = Engine(cfg, device=dev, max_new=64, prompt_room=64, weights=wts)
    prompt = OQ.prompt_ids(cfg.vocab, 8, seed=3)[0]
    teacher = OQ.prompt_ids(cfg.vocab, 16, seed=4)[0]
    picks, logits = eng.forced(prompt, teacher, record_logits=True)
    rec = []
    want = OQ.decode(oracle_model(wts, cfg), oracle_cfg(cfg), prompt, len(teacher) + 1,
                     teacher=teacher, record=rec, p_bf16=True)
    for i, ((lg_ref, pick_ref, gap), pick, lg) in enumerate(zip(rec, picks, logits)):
        assert_l2(f"logits at position {i}", lg, lg_ref)
        if pick != pick_ref:
            assert gap < 1e-2 * float(lg_ref.abs().max()), f"position {i}: pick differs at margin {gap:.4g}"


@pytest.mark.gpu
def test_engine_replay_is_deterministic(dev):
    from tilefoundry_amd.qwen3 import Engine

    cfg, wts = _small()
    eng = Engine(cfg, device=dev, max_new=64, prompt_room=64, weights=wts)
    prompt = OQ.prompt_ids(cfg.vocab, 8, seed=6)[0]
    a = eng.generate(prompt, 40).tokens
    b = eng.generate(prompt, 40).tokens
    assert a == b


@pytest.mark.gpu
def test_engine_rejects_bad_requests(dev):
    from tilefoundry_amd.qwen3 import Engine

    cfg, wts = _small()
    eng = Engine(cfg, device=dev, max_new=8, prompt_room=8, weights=wts)
    with pytest.raises(ValueError):
        eng.generate([], 4)
    with pytest.raises(ValueError):
        eng.generate([1] * 10, 10)
    with pytest.raises(ValueError):
        eng.generate([cfg.vocab + 5], 2)


@pytest.mark.gpu
def test_full_model_greedy_golden(dev):
    """28 layers, vocab 151936: the first 256 greedy ids after a 64-token
    prompt against the oracle's (tests/golden/qwen3_greedy_256.json)."""
    from tilefoundry_amd.qwen3 import Engine

    path = GOLDEN / "qwen3_greedy_256.json"
    if not path.exists():
        pytest.skip("golden ids not generated yet (tests/golden/make_qwen3_golden.py)")
    gold = json.loads(path.read_text())
    eng = Engine(device=dev, max_new=256, prompt_room=64, seed=gold["seed"])
    gen = eng.generate(gold["prompt"], len(gold["tokens"]))
    diff = next((i for i, (a, b) in enumerate(zip(gen.tokens, gold["tokens"])) if a != b), None)
    if diff is not None:
        gap, tol = gold["gaps"][diff], gold["tols"][diff]
        assert gap < tol, (f"step {diff}: got {gen.tokens[diff]} want {gold['tokens'][diff]}; "
                           f"oracle margin {gap:.4g} is above the bf16 tolerance {tol:.4g}")
    assert gen.tokens == gold["tokens"] or diff is not None
