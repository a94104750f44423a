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
from tests._check import assert_close, assert_l2, forced_agreement, logit_bounds, max_rel, oracle_candidates

GOLDEN = Path(__file__).parent / "golden"


def check_spread(name, deltas, spread):
    """Median GPU logit error at the deciding candidates against the median
    distance between the oracle's two valid orders at the same positions."""
    import statistics

    got, ref = statistics.median(deltas), statistics.median(spread["deltas"])
    print(f"[spread] {name}: median |delta| {got:.4g} vs the oracle's own order spread {ref:.4g} "
          f"(its picks agree {spread['agree']}/{len(spread['deltas'])})", flush=True)
    assert got <= SPREAD_FACTOR * ref, f"{name}: median logit error {got:.4g} > {SPREAD_FACTOR} x {ref:.4g}"
#: Positions of 256 whose teacher-forced pick must equal the oracle's on the
#: 28-layer random-weight model (the rest may differ only at near ties under the
#: measured logit error). The model's logits are flat -- 132 of the 256
#: positions have a top-2 gap inside twice the logit spread between the oracle's
#: two valid orders -- and those two orders (bf16 or f32 softmax weights into
#: P.V) agree on only 233 of 256 picks along these ids (the golden file's
#: ``order_spread``). The floor is that agreement: the GPU must agree with the
#: oracle at least as often as the oracle's own two orders agree with each other.
FULL_MODEL_FLOOR = 233
#: The GPU's logit error at the deciding candidates, median over positions, may
#: not exceed this multiple of the oracle's own order spread there.
SPREAD_FACTOR = 1.25
#: Absolute bound on the full model's logit error at any position's deciding
#: candidates: twice the largest distance between the oracle's own two orders
#: along the golden ids (0.127 logit units).
FULL_MODEL_MAX_DELTA = 0.25


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
def test_engine_fused_o_proj_is_bit_identical(dev):
    """The step with the split merge folded into o_proj gives the same logits,
    bit for bit, as the step with attn_combine and gemv_residual apart."""
    from tilefoundry_amd.qwen3 import Engine

    cfg, wts = _small()
    prompt = OQ.prompt_ids(cfg.vocab, 70, seed=3)[0]   # 70 positions: two splits of 64
    fused = Engine(cfg, device=dev, max_new=16, prompt_room=80, weights=wts, fuse_o=True)
    apart = Engine(cfg, device=dev, max_new=16, prompt_room=80, weights=wts)
    assert fused.fuse_o and not apart.fuse_o
    assert torch.equal(fused.logits_for(prompt), apart.logits_for(prompt))


@pytest.mark.gpu
def test_engine_greedy_small(dev):
    """Teacher-forced along the oracle's own greedy ids, every pick equals the
    oracle's except at near ties under the measured logit error; the free run
    agrees up to its first divergence, which must be such a near tie."""
    from tilefoundry_amd.qwen3 import Engine

    cfg, wts = _small()
    eng = Engine(cfg, device=dev, max_new=64, prompt_room=64, weights=wts)
    prompt = OQ.prompt_ids(cfg.vocab, 16, seed=2)[0]
    n = 32
    rec = []
    want = OQ.decode(oracle_model(wts, cfg), oracle_cfg(cfg), prompt, n, record=rec, p_bf16=True)
    picks, logits = eng.forced(prompt, want[:-1], record_logits=True)
    ids, vals, gaps = oracle_candidates([r[0] for r in rec])
    _, deltas = forced_agreement("2-layer bs=1, 32 positions", picks, want, logits, ids, vals, gaps,
                                 floor=n - 2, max_delta=logit_bounds([r[0] for r in rec]))
    gen = eng.generate(prompt, n)
    diff = next((i for i, (a, b) in enumerate(zip(gen.tokens, want)) if a != b), None)
    print(f"[free run] first divergence: {diff}", flush=True)
    if diff is not None:
        assert gaps[diff] <= 2 * deltas[diff], f"free run leaves the oracle at a clear margin (step {diff})"


#: Prompt seed of the 256-step exact-id test (a 16-token seeded-uniform prompt).
EXACT_PROMPT_SEED = 120


@pytest.mark.gpu
def test_engine_greedy_256_exact_small(dev):
    """2 layers, vocab 8192, 256 greedy steps, ids held exactly where the
    oracle itself fixes them.

    The oracle is decoded in its two valid orders (bf16 or f32 softmax weights
    into P.V) along the same ids; a position is *clear* when its top-1 / top-2
    gap exceeds twice the largest logit distance between those two orders at
    the deciding candidates. That criterion comes from the oracle alone: at the
    other positions even the oracle's own pick moves with the host CPU's f32
    summation order (two hosts' oracles were seen to part at such a position).
    Teacher-forced along the oracle's ids, the GPU's pick equals the oracle's
    at every clear position -- no allowance taken from the GPU's own error --
    and is one of the oracle's two best candidates elsewhere. The free run is
    identical to the oracle's ids up to the first teacher-forced difference,
    over all 256 steps when there is none (it then sees the teacher's inputs)."""
    from tilefoundry_amd.qwen3 import Engine

    cfg, wts = _small()
    n = 256
    prompt = OQ.prompt_ids(cfg.vocab, 16, seed=EXACT_PROMPT_SEED)[0]
    om, oc = oracle_model(wts, cfg), oracle_cfg(cfg)
    rec, alt = [], []
    want = OQ.decode(om, oc, prompt, n, record=rec, p_bf16=True)
    OQ.decode(om, oc, prompt, n, teacher=want, record=alt, p_bf16=False)
    ids, _, gaps = oracle_candidates([r[0] for r in rec])
    spread = [float((a[0] - r[0])[torch.tensor(c)].abs().max()) for a, r, c in zip(alt, rec, ids)]
    clear = [gaps[i] > 2.0 * spread[i] for i in range(n)]
    eng = Engine(cfg, device=dev, max_new=n, prompt_room=16, weights=wts)
    picks = eng.forced(prompt, want[:-1])
    miss = [i for i in range(n) if picks[i] != want[i]]
    bad = [(i, picks[i], want[i], gaps[i], spread[i]) for i in miss if clear[i] or picks[i] not in ids[i][:2]]
    gen = eng.generate(prompt, n)
    diff = next((i for i, (a, b) in enumerate(zip(gen.tokens, want)) if a != b), None)
    first_miss = miss[0] if miss else None
    print(f"[exact] 2-layer bs=1, 256 steps: {sum(clear)} clear positions, "
          f"{sum(1 for i in range(n) if clear[i] and picks[i] == want[i])} of them equal; "
          f"{n - len(miss)}/{n} teacher-forced picks equal overall; free run identical for "
          f"{n if diff is None else diff}/{n} steps", flush=True)
    assert sum(clear) >= 160, f"only {sum(clear)} clear positions: the test would pin little"
    assert not bad, f"picks differ at clear positions or off the top two (pos, got, want, gap, spread): {bad[:5]}"
    assert diff == first_miss, f"free run leaves the oracle at step {diff}, teacher-forced first miss {first_miss}"


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
    """28 layers, vocab 151936: teacher-forced along the oracle's 256 greedy ids
    after a 64-token prompt (tests/golden/qwen3_greedy_256.json), every pick
    equals the oracle's except at near ties under the measured logit error, and
    the agreement count is printed; the median logit error is held to the
    oracle's own order spread; the free run agrees up to its first divergence,
    which must be such a near tie."""
    from tilefoundry_amd.qwen3 import Engine

    gold = json.loads((GOLDEN / "qwen3_greedy_256.json").read_text())
    n = len(gold["tokens"])
    eng = Engine(device=dev, max_new=n, prompt_room=64, seed=gold["seed"])
    picks, logits = eng.forced(gold["prompt"], gold["tokens"][:-1], record_logits=True)
    _, deltas = forced_agreement("28-layer bs=1, 256 teacher-forced positions", picks, gold["tokens"], logits,
                                 gold["top_ids"], gold["top_vals"], gold["gaps"], floor=FULL_MODEL_FLOOR,
                                 max_delta=FULL_MODEL_MAX_DELTA)
    del logits
    check_spread("28-layer bs=1", deltas, gold["order_spread"])
    gen = eng.generate(gold["prompt"], n)
    diff = next((i for i, (a, b) in enumerate(zip(gen.tokens, gold["tokens"])) if a != b), None)
    print(f"[free run] first divergence from the oracle: {diff}", flush=True)
    if diff is not None:
        assert gold["gaps"][diff] <= 2 * deltas[diff], (
            f"step {diff}: got {gen.tokens[diff]} want {gold['tokens'][diff]} at a clear margin "
            f"{gold['gaps'][diff]:.4g} (measured logit error {deltas[diff]:.4g})")
