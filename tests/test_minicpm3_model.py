"""The whole MiniCPM3 decode model (``minicpm3.MiniCPM3Engine``) against the
oracle's token-by-token decode (oracle/minicpm3.py ``decode_step``, itself
pinned to Hugging Face's MiniCPM3ForCausalLM in test_oracle.py).

Small stacks keep the published layer shapes (hidden 2560, 40 heads, q_lora 768,
kv_lora 256, SwiGLU 6400) with fewer layers and a smaller vocabulary, so the
CPU oracle finishes in seconds; the full 62-layer model is checked against the
oracle's golden ids (tests/golden/minicpm3_greedy_256.json) and as a smoke test
(finite, reproducible).
"""
from dataclasses import replace

import pytest
import torch

from oracle import minicpm3 as OM
from tests._check import assert_close, forced_agreement, logit_bounds, oracle_candidates

BF16 = torch.bfloat16


def _small(layers=2, vocab=4096):
    from tilefoundry_amd.minicpm3 import MINICPM3_4B, synthetic_model_weights

    cfg = replace(MINICPM3_4B, layers=layers, vocab=vocab)
    return cfg, synthetic_model_weights(cfg, seed=11)


def _oracle(cfg, wts):
    from tilefoundry_amd.minicpm3 import hf_layer_names

    ocfg = OM.ModelConfig(hidden=cfg.hidden, heads=cfg.heads, q_lora=cfg.q_lora, kv_lora=cfg.kv_lora,
                          nope=cfg.nope, rope=cfg.rope, v_dim=cfg.v_dim, eps=cfg.eps, lora_eps=cfg.lora_eps,
                          rope_theta=cfg.rope_theta, inter=cfg.inter, vocab=cfg.vocab, layers=cfg.layers,
                          scale_emb=cfg.scale_emb, dim_model_base=cfg.dim_model_base,
                          scale_depth=cfg.scale_depth)
    layers = [OM.LayerWeights(**{k: wts[v].cpu() for k, v in hf_layer_names(i).items()})
              for i in range(cfg.layers)]
    model = OM.ModelWeights(embed=wts["model.embed_tokens.weight"].cpu(),
                            gamma_final=wts["model.norm.weight"].cpu(), layers=layers)
    return ocfg, model


@pytest.mark.gpu
def test_minicpm3_engine_logits_and_caches(dev):
    """After a 9-token prompt the bf16 logits and each layer's compressed cache
    rows agree with the oracle's decode (layer 0's cache at the per-op bar)."""
    from tilefoundry_amd.minicpm3 import MiniCPM3Engine

    cfg, wts = _small()
    eng = MiniCPM3Engine(cfg, device=dev, max_new=16, prompt_room=16, weights=wts)
    prompt = [5, 77, 1023, 4000, 12, 9, 300, 2047, 64]
    eng.generate([prompt], 1)
    ocfg, model = _oracle(cfg, wts)
    cos, sin = OM.rope_tables(len(prompt), ocfg)
    caches = OM.empty_caches(ocfg, cfg.layers)
    for p, t in enumerate(prompt):
        ref = OM.decode_step(model, ocfg, t, p, caches, cos, sin)
    assert_close("logits", eng.logits[0], ref)
    n = len(prompt)
    assert_close("latent cache layer 0", eng.latent[0, 0, :n], caches[0][0])
    assert_close("rope-key cache layer 0", eng.rope_k[0, 0, :n], caches[0][1])
    assert_close("latent cache layer 1", eng.latent[1, 0, :n], caches[1][0], rtol=2e-2)


@pytest.mark.gpu
def test_minicpm3_engine_greedy_against_oracle(dev):
    """Teacher-forced along the oracle's 20 greedy ids, every pick equals the
    oracle's except at near ties under the measured logit error; the free run
    leaves the oracle only at such a tie."""
    from tilefoundry_amd.minicpm3 import MiniCPM3Engine

    cfg, wts = _small()
    eng = MiniCPM3Engine(cfg, device=dev, max_new=32, prompt_room=16, weights=wts)
    prompt = [1, 2200, 17, 3999, 508, 60]
    n = 20
    ocfg, model = _oracle(cfg, wts)
    rec = []
    want = OM.decode(model, ocfg, prompt, n, record=rec)
    picks, logits = eng.forced([prompt], [want[:-1]], record_logits=True)
    ids, vals, gaps = oracle_candidates([r[0] for r in rec])
    _, deltas = forced_agreement("MiniCPM3 2-layer bs=1, 20 positions", picks[0], want, [lg[0] for lg in logits],
                                 ids, vals, gaps, floor=n - 2, max_delta=logit_bounds([r[0] for r in rec]))
    got = eng.generate([prompt], n).tokens[0]
    diff = next((i for i, (a, b) in enumerate(zip(got, want)) if a != b), None)
    if diff is not None:
        assert gaps[diff] <= 2 * deltas[diff], f"step {diff}: {got[diff]} != {want[diff]} at a clear margin"


@pytest.mark.gpu
def test_minicpm3_batched_engine_against_oracle(dev):
    """The batched step (skinny GEMMs, split-K partials, the q_b projection and
    the absorption in one launch, 256-slot attention splits) teacher-forced
    along the oracle's 16 greedy ids of each of three sequences: every pick
    equals the oracle's except at near ties under the measured logit error."""
    from tilefoundry_amd.minicpm3 import MiniCPM3Engine

    cfg, wts = _small()
    prompts = [[3, 4, 5, 6, 7], [4000, 1, 2, 3, 2047], [77, 77, 77, 77, 77]]
    n = 16
    eng = MiniCPM3Engine(cfg, batch=3, device=dev, max_new=32, prompt_room=8, weights=wts)
    ocfg, model = _oracle(cfg, wts)
    wants, recs = [], []
    for p in prompts:
        rec = []
        wants.append(OM.decode(model, ocfg, p, n, record=rec))
        recs.append(rec)
    picks, logits = eng.forced(prompts, [w[:-1] for w in wants], record_logits=True)
    for b in range(3):
        ids, vals, gaps = oracle_candidates([r[0] for r in recs[b]])
        forced_agreement(f"MiniCPM3 2-layer batch 3, sequence {b}, {n} positions", picks[b], wants[b],
                         [lg[b] for lg in logits], ids, vals, gaps, floor=n - 2,
                         max_delta=logit_bounds([r[0] for r in recs[b]]))


@pytest.mark.gpu
def test_minicpm3_engine_batch_rows_are_independent(dev):
    """Three sequences in one batch decode exactly what each decodes in another
    batch (the batched path's rows do not interact); the one-sequence GEMV path
    agrees with the oracle wherever the margin is resolvable."""
    from tilefoundry_amd.minicpm3 import MiniCPM3Engine

    cfg, wts = _small()
    prompts = [[3, 4, 5, 6], [4000, 1, 2, 3], [77, 77, 77, 77]]
    batch = MiniCPM3Engine(cfg, batch=3, device=dev, max_new=16, prompt_room=8, weights=wts)
    got = batch.generate(prompts, 12).tokens
    two = MiniCPM3Engine(cfg, batch=2, device=dev, max_new=16, prompt_room=8, weights=wts)
    for b, p in enumerate(prompts):
        assert two.generate([p, prompts[(b + 1) % 3]], 12).tokens[0] == got[b], f"sequence {b}"
    one = MiniCPM3Engine(cfg, batch=1, device=dev, max_new=16, prompt_room=8, weights=wts)
    ocfg, model = _oracle(cfg, wts)
    for p in prompts[:2]:
        rec = []
        want = OM.decode(model, ocfg, p, 12, record=rec)
        mine = one.generate([p], 12).tokens[0]
        diff = next((i for i, (x, y) in enumerate(zip(mine, want)) if x != y), None)
        if diff is not None:
            logits, pick, gap = rec[diff]
            assert gap < 1e-2 * float(logits.abs().max()), f"step {diff} at margin {gap:.4g}"


@pytest.mark.gpu
def test_minicpm3_sampler(dev):
    """The top-p sampler: reproducible under a seeded generator, and with a
    vanishing top_p it keeps only the most likely token -- the greedy ids."""
    from tilefoundry_amd.minicpm3 import MiniCPM3Engine, sample_top_p

    cfg, wts = _small()
    eng = MiniCPM3Engine(cfg, device=dev, max_new=24, prompt_room=8, weights=wts)
    prompt = [[10, 20, 30, 40]]
    greedy = eng.generate(prompt, 16).tokens
    g = torch.Generator(device=dev)
    g.manual_seed(1)
    a = eng.generate(prompt, 16, sampler=sample_top_p(0.8, 0.8, g)).tokens
    g.manual_seed(1)
    b = eng.generate(prompt, 16, sampler=sample_top_p(0.8, 0.8, g)).tokens
    assert a == b
    assert eng.generate(prompt, 16, sampler=sample_top_p(0.8, 1e-9, g)).tokens == greedy
    assert all(0 <= t < cfg.vocab for t in a[0])
    c = eng.generate(prompt, 16, sampler=sample_top_p(0.8, 0.8, seed=2)).tokens
    assert c != a, "another seed gives another continuation"
    # the greedy step is untouched by the sampling graph beside it
    assert eng.generate(prompt, 16).tokens == greedy


def _draws(dev, logits, temperature, top_p, n, seed=0):
    """``n`` top-p draws per row of ``logits`` [B, V]: the sampling step run n
    times, each at the next position (the generator's counter)."""
    from tilefoundry_amd._lib import C

    B, V = logits.shape
    lg = logits.to(dev).float().contiguous()
    params = torch.tensor([temperature, top_p], dtype=torch.float32, device=dev)
    sd = torch.tensor([seed], dtype=torch.int64, device=dev)
    inp = torch.zeros(B, n + 1, dtype=torch.int32, device=dev)
    plen = torch.zeros(B, dtype=torch.int32, device=dev)
    ids = torch.zeros(B, dtype=torch.int64, device=dev)
    pos = torch.zeros(B, dtype=torch.int32, device=dev)
    sam = torch.full((B, n + 1), -1, dtype=torch.int32, device=dev)
    err = torch.zeros(1, dtype=torch.int32, device=dev)
    for _ in range(n):
        C.top_p_sample_step(lg, params, sd, inp, plen, ids, pos, sam, err)
    torch.cuda.synchronize()
    assert int(err) == 0 and pos.tolist() == [n] * B
    assert torch.equal(ids, sam[:, n - 1].long()), "the draw is fed as the next input"
    return sam[:, :n].cpu()


@pytest.mark.gpu
def test_top_p_step_draws_from_the_kept_set(dev):
    """The device sampling step against the run.py sampler's kept set and
    probabilities (oracle ``top_p_kept``) on bf16-valued logits over the full
    73448-token vocabulary: every draw is a kept token, and the frequencies of
    the likeliest kept tokens match their probabilities within 5 sigma over
    32 x 400 draws."""
    V, B, n = 73448, 32, 400
    g = torch.Generator().manual_seed(31)
    row = (2.5 * torch.randn(V, generator=g)).to(BF16).float()
    ids, probs = OM.top_p_kept(row, 0.8, 0.8)
    draws = _draws(dev, row.expand(B, V), 0.8, 0.8, n).flatten()
    kept = torch.zeros(V, dtype=torch.bool)
    kept[ids] = True
    assert bool(kept[draws.long()].all()), "a draw outside the kept set"
    counts = torch.bincount(draws.long(), minlength=V).double()
    N = draws.numel()
    for i, p in zip(ids[:20].tolist(), probs[:20].tolist()):
        sigma = (N * p * (1 - p)) ** 0.5
        assert abs(counts[i] - N * p) <= 5 * sigma + 1, (i, counts[i], N * p)
    # each sequence (block row) draws its own stream
    per_row = draws.view(B, n)
    assert not torch.equal(per_row[0], per_row[1])


@pytest.mark.gpu
def test_top_p_step_ties_and_limits(dev):
    """Ties at the kept boundary are kept in index order (a stable ranking); a
    uniform row keeps its first ceil(top_p V) tokens; a vanishing top_p gives
    the lowest-index greedy pick; a position past the buffers is flagged."""
    V = 4096
    tie = torch.full((V,), -1.0e4)        # probability zero past the first four tokens
    tie[0], tie[1:4] = 10.0, 5.0          # e^-5 each: the mass before the third tie is past 0.99
    ids, _ = OM.top_p_kept(tie, 1.0, 0.99)
    assert ids.tolist() == [0, 1, 2]
    d = _draws(dev, tie.expand(32, V), 1.0, 0.99, 100)
    assert set(d.flatten().tolist()) <= {0, 1, 2}
    uni = torch.zeros(V)
    d = _draws(dev, uni.expand(32, V), 1.0, 0.25, 50)
    assert int(d.max()) < V // 4 and len(set(d.flatten().tolist())) > 500
    peaks = torch.zeros(V)
    peaks[[7, 900, 3000]] = 3.0           # three equal maxima: greedy takes the lowest index
    d = _draws(dev, peaks.expand(4, V), 0.8, 1e-9, 20)
    assert set(d.flatten().tolist()) == {7}
    from tilefoundry_amd._lib import C

    lg = torch.zeros(1, V, device=dev)
    err = torch.zeros(1, dtype=torch.int32, device=dev)
    pos = torch.tensor([5], dtype=torch.int32, device=dev)
    C.top_p_sample_step(lg, torch.tensor([1.0, 0.5], device=dev), torch.zeros(1, dtype=torch.int64, device=dev),
                        torch.zeros(1, 4, dtype=torch.int32, device=dev), torch.zeros(1, dtype=torch.int32, device=dev),
                        torch.zeros(1, dtype=torch.int64, device=dev), pos,
                        torch.zeros(1, 4, dtype=torch.int32, device=dev), err)
    torch.cuda.synchronize()
    assert int(err) == 2 and int(pos) == 5


@pytest.mark.gpu
def test_minicpm3_full_model_golden(dev):
    """The full MiniCPM3-4B-shaped model (62 layers, vocab 73448, seed-0
    weights) after the decode benchmark's 8-token prompt, against the oracle's
    ids in tests/golden/minicpm3_greedy_256.json (make_minicpm3_golden.py):

    * teacher-forced along 255 seeded random ids, every pick at a clear
      position (top-2 gap above twice the oracle's own two-order spread there)
      equals the oracle's, every other pick is a near tie under the measured
      logit error, and the logit error stays within twice the oracle's largest
      order spread;
    * the free greedy run equals the oracle's 256 ids exactly."""
    import json
    from pathlib import Path

    from tests.test_qwen3_engine import check_spread
    from tilefoundry_amd.minicpm3 import MiniCPM3Engine

    gold = json.loads((Path(__file__).parent / "golden" / "minicpm3_greedy_256.json").read_text())
    f = gold["forced"]
    n = len(f["tokens"])
    spread = f["order_spread"]["deltas"]
    clear = [gap > 2.0 * sp for gap, sp in zip(f["gaps"], spread)]
    eng = MiniCPM3Engine(device=dev, max_new=n, prompt_room=len(gold["prompt"]), seed=gold["seed"])
    picks, logits = eng.forced([gold["prompt"]], [f["teacher"]], record_logits=True)
    picks = picks[0]
    _, deltas = forced_agreement("MiniCPM3 62-layer bs=1, 256 teacher-forced positions", picks, f["tokens"],
                                 [lg[0] for lg in logits], f["top_ids"], f["top_vals"], f["gaps"],
                                 floor=sum(clear), max_delta=2.0 * max(spread))
    del logits
    check_spread("MiniCPM3 62-layer bs=1", deltas, f["order_spread"])
    off = [i for i in range(n) if clear[i] and picks[i] != f["tokens"][i]]
    assert not off, f"picks differ at clear positions: {off[:8]}"
    gen = eng.generate([gold["prompt"]], n).tokens[0]
    diff = next((i for i, (a, b) in enumerate(zip(gen, gold["free"]["tokens"])) if a != b), None)
    print(f"[exact] MiniCPM3 62-layer bs=1: {sum(clear)}/{n} clear teacher-forced positions, all equal; "
          f"free run identical for {n if diff is None else diff}/{n} steps", flush=True)
    assert diff is None, f"free run leaves the oracle at step {diff}"


@pytest.mark.gpu
def test_minicpm3_full_model_smoke(dev):
    """62 layers, vocab 73448, random weights: a greedy continuation is
    reproducible, every id in range, and the bf16 logits finite."""
    from tilefoundry_amd.minicpm3 import MiniCPM3Engine

    eng = MiniCPM3Engine(device=dev, max_new=16, prompt_room=16, seed=1)
    prompt = [[1, 100, 2000, 30000, 73000]]
    a = eng.generate(prompt, 12).tokens
    b = eng.generate(prompt, 12).tokens
    assert a == b and all(0 <= t < 73448 for t in a[0])
    assert bool(torch.isfinite(eng.logits).all())
