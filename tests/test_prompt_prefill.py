"""Prompt prefill for the Qwen3-shaped decode model: every prompt row through
every layer at once instead of one decode step per prompt token.

Each kernel of the prefill is checked on its own against the oracle (or bit for
bit against the decode kernel whose arithmetic it repeats), then the engines
with ``prompt_prefill=True`` against the oracle's token-by-token walk
(examples/qwen3_1_7b-tilelang/fast/engine.py:261-263 is what the prefill
replaces): the K/V cache rows, the logits of the first generated position and
the greedy continuation.
"""
import pytest
import torch

from oracle import qwen3 as OQ
from tests._check import assert_close, assert_l2, assert_ulps, forced_agreement, logit_bounds, oracle_candidates
from tests.test_qwen3_engine import _small, oracle_cfg, oracle_model

BF16 = torch.bfloat16


def _g(seed):
    return torch.Generator().manual_seed(seed)


# ------------------------------------------------------------------ kernels
@pytest.mark.gpu
@pytest.mark.parametrize("m", [1, 37, 300])
def test_gemm_nt_f32(dev, m):
    """f32 product of bf16 operands (no landing) against f64: only the f32
    summation order may differ."""
    from tilefoundry_amd._lib import C

    g = _g(m)
    a = torch.randn(m, 2048, generator=g).to(BF16)
    b = torch.randn(768, 2048, generator=g).to(BF16)
    c = torch.full((m, 768), float("nan"), device=dev)
    C.gemm_nt_f32(a.to(dev), b.to(dev), c)
    ref = a.double() @ b.double().t()
    bound = 2048 * 2.0 ** -23 * (a.double().abs() @ b.double().abs().t())
    err = (c.cpu().double() - ref).abs()
    assert bool((err <= bound + 1e-6).all()), f"max err {float(err.max()):.3g}"


@pytest.mark.gpu
def test_swiglu_pairs(dev):
    """Interleaved gate|up columns -> bf16(bf16(silu(bf16 g)) * bf16 u): the
    oracle's mlp order (oracle/qwen3.py mlp), within one bf16 ulp (the device
    exp may round the last bit of silu differently)."""
    from tilefoundry_amd._lib import C

    rows, inter = 19, 6144
    gu = torch.randn(rows, 2 * inter, generator=_g(3)) * 3
    act = torch.empty(rows, inter, device=dev, dtype=BF16)
    C.swiglu_pairs(gu.to(dev), act)
    g = gu[:, 0::2].to(BF16)
    u = gu[:, 1::2].to(BF16)
    ref = torch.nn.functional.silu(g.float()).to(BF16) * u
    assert_ulps("swiglu", act, ref, max_ulps=1, max_frac=0.01)


@pytest.mark.gpu
@pytest.mark.parametrize("B,n,pos0", [(1, 1, 0), (2, 37, 0), (3, 130, 5)])
def test_prefill_qk_rope_equals_decode_kernel(dev, B, n, pos0):
    """Each prompt row's q, cache k and cache v are bit for bit what the decode
    step's qk_rope_cache writes from the same projection values at that
    position (that kernel is pinned to the oracle in test_kernels_api.py)."""
    from tilefoundry_amd._lib import C

    HQ, HKV, D, cap = 16, 8, 128, 160
    cols = (HQ + 2 * HKV) * D
    g = _g(B * 100 + n)
    qkv = torch.randn(B * n, cols, generator=g)
    gq = (1 + 0.1 * torch.randn(D, generator=g)).to(BF16).to(dev)
    gk = (1 + 0.1 * torch.randn(D, generator=g)).to(BF16).to(dev)
    cos, sin = OQ.rope_tables(cap, D, 1.0e6)
    cos, sin = cos.to(dev), sin.to(dev)
    kc = torch.zeros(B, cap, HKV * D, device=dev, dtype=BF16)
    vc = torch.zeros_like(kc)
    q = torch.empty(B * n, HQ * D, device=dev, dtype=BF16)
    C.prefill_qk_rope(qkv.to(dev), gq, gk, 1e-6, cos, sin, B, n, pos0, kc, vc, q, HQ, HKV)
    # the decode kernel, one "sequence" per prompt row, its position as the slot
    R = B * n
    pos = torch.tensor([pos0 + r for _ in range(B) for r in range(n)], dtype=torch.int32, device=dev)
    kd = torch.zeros(R, cap, HKV * D, device=dev, dtype=BF16)
    vd = torch.zeros_like(kd)
    qd = torch.empty(R, HQ * D, device=dev, dtype=BF16)
    C.qk_rope_cache(qkv.to(dev).view(1, R, cols), gq, gk, 1e-6, cos, sin, pos, pos, kd, vd, qd, HQ, HKV,
                    None)
    torch.cuda.synchronize(dev)
    assert torch.equal(q, qd)
    idx = torch.arange(R, device=dev)
    assert torch.equal(kc[:, pos0: pos0 + n].reshape(R, -1), kd[idx, pos.long()])
    assert torch.equal(vc[:, pos0: pos0 + n].reshape(R, -1), vd[idx, pos.long()])
    # nothing outside the prompt rows was written
    assert float(kc[:, :pos0].abs().sum() + kc[:, pos0 + n:].abs().sum()) == 0.0
    assert float(vc[:, :pos0].abs().sum() + vc[:, pos0 + n:].abs().sum()) == 0.0


def _causal_ref(q, k, v, scale):
    """Row r of every sequence through the oracle's kernel-order attention
    (``OQ.attend`` with bf16 weights): q (B, n, HQ, D), k/v (B, >= n, HKV, D)."""
    B, n, HQ, D = q.shape
    out = torch.empty(B, n, HQ * D, dtype=BF16)
    for b in range(B):
        for r in range(n):
            out[b, r] = OQ.attend(q[b, r], k[b, : r + 1], v[b, : r + 1], scale, p_bf16=True)
    return out


@pytest.mark.gpu
@pytest.mark.parametrize("B,n", [(1, 1), (2, 37), (1, 128), (2, 300)])
def test_causal_attention_from_cache(dev, B, n):
    """Qwen3 shapes (16 query heads over 8, head_dim 128) read in place from a
    decode cache whose rows past the prompt hold NaN: a row n.. read or an
    unmasked key would poison the output."""
    from tilefoundry_amd._lib import C

    HQ, HKV, D, cap = 16, 8, 128, 320
    g = _g(7 * n + B)
    q = torch.randn(B, n, HQ, D, generator=g).to(BF16)
    kc = torch.full((B, cap, HKV, D), float("nan"), dtype=BF16)
    vc = torch.full((B, cap, HKV, D), float("nan"), dtype=BF16)
    kc[:, :n] = torch.randn(B, n, HKV, D, generator=g).to(BF16)
    vc[:, :n] = torch.randn(B, n, HKV, D, generator=g).to(BF16)
    out = torch.empty(B, n, HQ * D, device=dev, dtype=BF16)
    scale = D ** -0.5
    C.causal_attention(q.to(dev), kc.to(dev), vc.to(dev), out, scale)
    got = out.cpu()
    assert bool(torch.isfinite(got.float()).all())
    assert_close("causal attention", got, _causal_ref(q, kc, vc, scale))


@pytest.mark.gpu
def test_causal_attention_256_row_blocks(dev):
    """Two sequences of 2048 rows fill the chip with 256-row blocks (eight
    waves, three stages): sampled rows against the oracle, every row finite."""
    from tilefoundry_amd._lib import C

    B, n, HQ, HKV, D = 2, 2048, 16, 8, 128
    g = _g(13)
    q = torch.randn(B, n, HQ, D, generator=g).to(BF16)
    k = torch.randn(B, n, HKV, D, generator=g).to(BF16)
    v = torch.randn(B, n, HKV, D, generator=g).to(BF16)
    out = torch.empty(B, n, HQ * D, device=dev, dtype=BF16)
    C.causal_attention(q.to(dev), k.to(dev), v.to(dev), out, D ** -0.5)
    got = out.cpu()
    assert bool(torch.isfinite(got.float()).all())
    rows = sorted({0, 1, 31, 32, 255, 256, 257, 1023, 1500, 2046, 2047} | set(range(97, n, 211)))
    for b in range(B):
        ref = torch.stack([OQ.attend(q[b, r], k[b, : r + 1], v[b, : r + 1], D ** -0.5, p_bf16=True)
                           for r in rows])
        assert_close(f"sequence {b} sampled rows", got[b, rows], ref)


@pytest.mark.gpu
def test_causal_attention_head_dim_256_ragged(dev):
    """The ungated head_dim-256 form (the Qwen3.5 layer's kernel without its
    gate) on a ragged length and strided q / k / v views."""
    from tilefoundry_amd._lib import C

    B, n, HQ, HKV, D = 2, 200, 24, 4, 256
    g = _g(11)
    buf = torch.randn(B, n, HQ * D + 2 * HKV * D, generator=g).to(BF16)
    q = buf[:, :, : HQ * D].view(B, n, HQ, D)
    k = buf[:, :, HQ * D: HQ * D + HKV * D].view(B, n, HKV, D)
    v = buf[:, :, HQ * D + HKV * D:].view(B, n, HKV, D)
    bd = buf.to(dev)
    out = torch.empty(B, n, HQ * D, device=dev, dtype=BF16)
    C.causal_attention(bd[:, :, : HQ * D].view(B, n, HQ, D), bd[:, :, HQ * D: HQ * D + HKV * D].view(B, n, HKV, D),
                       bd[:, :, HQ * D + HKV * D:].view(B, n, HKV, D), out, D ** -0.5)
    assert_close("causal attention d256", out.cpu(), _causal_ref(q, k, v, D ** -0.5))


@pytest.mark.gpu
def test_causal_attention_prefix_independence(dev):
    """Row r depends on rows <= r only: the first 100 rows of a 1000-row run
    equal a 100-row run bit for bit (different grids, same per-row work)."""
    from tilefoundry_amd._lib import C

    B, HQ, HKV, D = 1, 16, 8, 128
    g = _g(12)
    q = torch.randn(B, 1000, HQ, D, generator=g).to(BF16).to(dev)
    k = torch.randn(B, 1000, HKV, D, generator=g).to(BF16).to(dev)
    v = torch.randn(B, 1000, HKV, D, generator=g).to(BF16).to(dev)
    long = torch.empty(B, 1000, HQ * D, device=dev, dtype=BF16)
    short = torch.empty(B, 100, HQ * D, device=dev, dtype=BF16)
    C.causal_attention(q, k, v, long, D ** -0.5)
    C.causal_attention(q[:, :100], k, v, short, D ** -0.5)
    assert torch.equal(long[:, :100], short)


# ------------------------------------------------------------------ engines
def _oracle_walk(wts, cfg, prompt):
    om, oc = oracle_model(wts, cfg), oracle_cfg(cfg)
    cos, sin = OQ.rope_tables(len(prompt), cfg.head_dim, cfg.rope_theta)
    caches = OQ.empty_caches(oc, cfg.layers)
    logits = None
    for p, t in enumerate(prompt):
        logits = OQ.step(om, oc, t, p, caches, cos, sin, p_bf16=True)
    return logits, caches


@pytest.mark.gpu
def test_engine_prefill_caches_and_logits(dev):
    """After prefilling 39 of 40 prompt tokens and one decode step, the cache
    rows and the logits agree with the oracle's walk over all 40 (layer 0 at
    the per-op bar, deeper layers at relative L2, as for the walk itself)."""
    from tilefoundry_amd.qwen3 import Engine

    cfg, wts = _small()
    eng = Engine(cfg, device=dev, max_new=16, prompt_room=64, weights=wts, prompt_prefill=True)
    prompt = OQ.prompt_ids(cfg.vocab, 40, seed=21)[0]
    gen = eng.generate(prompt, 1)
    ref_logits, caches = _oracle_walk(wts, cfg, prompt)
    assert_close("logits", eng.logits, ref_logits)
    n = len(prompt)
    for i in range(cfg.layers):
        kc = eng.kc[i, :n].view(n, cfg.kv_heads, cfg.head_dim)
        vc = eng.vc[i, :n].view(n, cfg.kv_heads, cfg.head_dim)
        check = assert_close if i == 0 else assert_l2
        check(f"k cache layer {i}", kc, caches[i][0])
        check(f"v cache layer {i}", vc, caches[i][1])
    assert gen.tokens[0] == OQ.greedy(ref_logits) or _gap(ref_logits) < 1e-2 * float(ref_logits.abs().max())


def _gap(logits):
    top = torch.topk(logits, 2).values
    return float(top[0] - top[1])


@pytest.mark.gpu
def test_engine_prefill_greedy_small(dev):
    """After a prefilled 48-token prompt, teacher-forced along the oracle's 24
    greedy ids: every pick equals the oracle's except at near ties under the
    measured logit error; the free run leaves the oracle only at such a tie."""
    from tilefoundry_amd.qwen3 import Engine

    cfg, wts = _small()
    eng = Engine(cfg, device=dev, max_new=64, prompt_room=64, weights=wts, prompt_prefill=True)
    prompt = OQ.prompt_ids(cfg.vocab, 48, seed=22)[0]
    n = 24
    rec = []
    want = OQ.decode(oracle_model(wts, cfg), oracle_cfg(cfg), prompt, n, record=rec, p_bf16=True)
    picks, logits = eng.forced(prompt, want[:-1], record_logits=True)
    ids, vals, gaps = oracle_candidates([r[0] for r in rec])
    _, deltas = forced_agreement("2-layer bs=1 prefilled, 24 positions", picks, want, logits, ids, vals, gaps,
                                 floor=n - 2, max_delta=logit_bounds([r[0] for r in rec]))
    gen = eng.generate(prompt, n)
    assert gen.prompt_steps == len(prompt)
    diff = next((i for i, (a, b) in enumerate(zip(gen.tokens, want)) if a != b), None)
    if diff is not None:
        assert gaps[diff] <= 2 * deltas[diff], f"free run leaves the oracle at a clear margin (step {diff})"


@pytest.mark.gpu
def test_engine_prefill_then_walk_again(dev):
    """A prefilled generate, a walked one and a prefilled one again on the same
    engine object: the two prefilled runs agree exactly (no state leaks from
    one request into the next), and a one-token prompt takes the walk path."""
    from tilefoundry_amd.qwen3 import Engine

    cfg, wts = _small()
    eng = Engine(cfg, device=dev, max_new=32, prompt_room=64, weights=wts, prompt_prefill=True)
    prompt = OQ.prompt_ids(cfg.vocab, 30, seed=23)[0]
    a = eng.generate(prompt, 20).tokens
    eng.prompt_prefill = False
    eng.generate(OQ.prompt_ids(cfg.vocab, 50, seed=24)[0], 10)
    eng.prompt_prefill = True
    b = eng.generate(prompt, 20).tokens
    assert a == b
    assert len(eng.generate(prompt[:1], 5).tokens) == 5


@pytest.mark.gpu
def test_batch_engine_prefill_small(dev):
    """Three sequences prefilled together, teacher-forced along each one's
    oracle greedy ids: every pick equals the oracle's except at near ties under
    the measured logit error, and each sequence's cache rows agree with its own
    oracle walk."""
    from tilefoundry_amd.qwen3 import BatchEngine

    cfg, wts = _small()
    eng = BatchEngine(cfg, batch=3, device=dev, max_new=32, prompt_room=64, weights=wts,
                      prompt_prefill=True)
    prompts = OQ.prompt_ids(cfg.vocab, 33, seed=25, batch=3)
    om, oc = oracle_model(wts, cfg), oracle_cfg(cfg)
    n = 12
    wants, recs = [], []
    for prompt in prompts:
        rec = []
        wants.append(OQ.decode(om, oc, prompt, n, record=rec, p_bf16=True))
        recs.append(rec)
    picks, logits = eng.forced(prompts, [w[:-1] for w in wants], record_logits=True)
    for b, prompt in enumerate(prompts):
        ids, vals, gaps = oracle_candidates([r[0] for r in recs[b]])
        forced_agreement(f"2-layer batch prefilled, sequence {b}", picks[b], wants[b], [lg[b] for lg in logits],
                         ids, vals, gaps, floor=n - 2, max_delta=logit_bounds([r[0] for r in recs[b]]))
        _, caches = _oracle_walk(wts, cfg, prompt[:-1])
        m = len(prompt) - 1
        assert_close(f"seq {b} k cache layer 0", eng.kc[0, b, :m].view(m, cfg.kv_heads, cfg.head_dim), caches[0][0])
        assert_l2(f"seq {b} v cache layer 1", eng.vc[1, b, :m].view(m, cfg.kv_heads, cfg.head_dim), caches[1][1])


@pytest.mark.gpu
def test_full_model_prefill_greedy_golden(dev):
    """28 layers, vocab 151936, the 64-token prompt prefilled: teacher-forced
    along the oracle's 256 greedy ids (tests/golden/qwen3_greedy_256.json),
    every pick equals the oracle's except at near ties under the measured logit
    error; the agreement count is printed."""
    import json
    from pathlib import Path

    from tests.test_qwen3_engine import FULL_MODEL_FLOOR, FULL_MODEL_MAX_DELTA, check_spread
    from tilefoundry_amd.qwen3 import Engine

    gold = json.loads((Path(__file__).parent / "golden" / "qwen3_greedy_256.json").read_text())
    n = len(gold["tokens"])
    eng = Engine(device=dev, max_new=n, prompt_room=64, seed=gold["seed"], prompt_prefill=True)
    picks, logits = eng.forced(gold["prompt"], gold["tokens"][:-1], record_logits=True)
    _, deltas = forced_agreement("28-layer bs=1 after prompt prefill, 256 teacher-forced positions", picks,
                                 gold["tokens"], logits, gold["top_ids"], gold["top_vals"], gold["gaps"],
                                 floor=FULL_MODEL_FLOOR, max_delta=FULL_MODEL_MAX_DELTA)
    check_spread("28-layer bs=1 after prompt prefill", deltas, gold["order_spread"])
