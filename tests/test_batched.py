"""Batched decode (up to 32 sequences) against the CPU oracle: the skinny MFMA
GEMM and its epilogues, the row norms, attention reading split-K partials, and
the batch engine end to end (each sequence against the oracle's bs=1 decode)."""
import pytest
import torch

from oracle import norms as ON
from oracle import qwen3 as OQ
from tests._check import forced_agreement, logit_bounds, oracle_candidates, assert_close, assert_equal, assert_l2, max_rel

BF = torch.bfloat16
H, HQ, HKV, D, I = 2048, 16, 8, 128, 6144


def gen(seed):
    return torch.Generator().manual_seed(seed)


def randn(*shape, g, std=1.0, mean=0.0):
    return (mean + std * torch.randn(*shape, generator=g)).to(BF)


@pytest.mark.gpu
@pytest.mark.parametrize("M,N,K,ks", [(32, 4096, 2048, 1), (32, 4096, 2048, 2), (5, 2048, 2048, 4),
                                      (1, 96, 256, 1), (32, 2048, 6144, 4), (17, 1000, 1024, 2),
                                      (32, 12288, 2048, 1), (7, 12250, 512, 1)])
def test_skinny_partials(dev, M, N, K, ks):
    from tilefoundry_amd import ops

    g = gen(M * N + K)
    x = randn(M, K, g=g)
    w = randn(N, K, g=g, std=K ** -0.5)
    ref = x.float() @ w.float().t()
    part = ops.skinny_gemm(x.to(dev), w.to(dev), "partial", ks=ks)
    assert part.shape == (ks, M, N)
    assert max_rel(part.sum(0), ref) < 5e-3


@pytest.mark.gpu
def test_skinny_exact_on_integers(dev):
    """Small-integer inputs: every MFMA product and f32 sum is exact."""
    from tilefoundry_amd import ops

    g = gen(3)
    x = torch.randint(-3, 4, (32, 2048), generator=g).to(BF)
    w = torch.randint(-3, 4, (256, 2048), generator=g).to(BF)
    ref = (x.long() @ w.long().t()).float()
    part = ops.skinny_gemm(x.to(dev), w.to(dev), "partial", ks=2)
    assert_equal("integer skinny gemm", part.sum(0).cpu(), ref)


@pytest.mark.gpu
@pytest.mark.parametrize("M", [32, 5])
def test_skinny_residual_then_norm_swiglu(dev, M):
    """The folded post-attention path: o_proj with the residual add and the
    per-32-row sums of squares in its epilogue, then the gate|up GEMM staging
    its tokens as the Qwen3 norm of the residual stream. h1 is the oracle's
    bf16(h + bf16(o)) (within one ulp: the f32 dot's order), the sums of
    squares its f64 sums, and the SwiGLU output the oracle's over the
    normalised h1; against the unfolded launches (split-K partials, rows_norm,
    SwiGLU GEMM) nearly every element is identical."""
    from tilefoundry_amd import ops
    from tilefoundry_amd._lib import C

    g = gen(40 + M)
    attn = randn(M, HQ * D, g=g)
    w_o = randn(H, HQ * D, g=g, std=0.02)
    h = randn(M, H, g=g)
    gamma = randn(H, g=g, std=0.1, mean=1.0)
    wg, wu = randn(I, H, g=g, std=0.02), randn(I, H, g=g, std=0.02)
    w_gu = torch.stack([wg, wu], 1).reshape(2 * I, H)
    d = {k: v.to(dev) for k, v in dict(attn=attn, w_o=w_o, h=h, gamma=gamma, w_gu=w_gu).items()}
    nb = C.skinny_residual_blocks(H)
    h1 = torch.empty(M, H, device=dev, dtype=BF)
    ssq = torch.full((nb, M), float("nan"), device=dev)
    C.skinny_gemm_residual(d["attn"], d["w_o"], d["h"], h1, ssq)
    act = torch.empty(M, I, device=dev, dtype=BF)
    C.skinny_gemm_norm_swiglu(h1, d["w_gu"], ssq, d["gamma"], 1e-6, act)
    torch.cuda.synchronize()
    o_ref = OQ.proj(attn, w_o)
    h1_ref = h + o_ref
    from tests._check import assert_ulps
    # the f32 dot's order may move the landed o by one of its own ulps, which is
    # more than one ulp of h1 where h and o nearly cancel
    spacing = torch.ldexp(torch.ones(()), torch.frexp(o_ref.float())[1] - 8)
    assert bool(((h1.cpu().float() - h1_ref.float()).abs() <= spacing).all()), "h1 beyond one ulp of o"
    assert_ulps("h1", h1, h1_ref, max_ulps=8, max_frac=0.01)
    sq_ref = (h1.cpu().double() ** 2).view(M, nb, 32).sum(-1).t()
    assert float(((ssq.cpu().double() - sq_ref).abs() / sq_ref).max()) < 1e-5
    xn = ON.rms_norm_q(h1.cpu(), gamma, 1e-6)
    act_ref = torch.nn.functional.silu(OQ.proj(xn, wg).float()).to(BF) * OQ.proj(xn, wu)
    assert_close("norm + swiglu", act, act_ref)
    # the unfolded launches over the same h1
    part = ops.skinny_gemm(d["attn"], d["w_o"], "partial", ks=4)
    h1b, xnb = torch.empty_like(h1), torch.empty_like(h1)
    C.rows_norm(None, None, d["h"], part, h1b, d["gamma"], xnb, 1e-6, None)
    actb = ops.skinny_gemm(xnb, d["w_gu"], "swiglu")
    assert bool(((h1.float() - h1b.float()).abs().cpu() <= 2 * spacing).all()), "h1 folded vs unfolded"
    assert_ulps("act folded vs unfolded", act, actb, max_ulps=2, max_frac=0.02)


@pytest.mark.gpu
def test_batch_engine_fold_o_norm_matches(dev):
    """The batch engine with the post-attention norm folded (opt-in) against the
    default launches on a 2-layer model. The two round differently (o_proj as
    one f32 dot instead of four split-K partials, the norm's sum of squares in
    another order), so a near tie may flip: teacher-forced along the default
    engine's free run, every folded pick equals the default one except where
    the default's top-1 / top-2 gap is within twice the measured logit
    difference, which itself stays within 1 % of the largest logit; the folded
    free run leaves the default one only at such a tie; logits agree within
    bf16 relative L2."""
    from tilefoundry_amd.qwen3 import BatchEngine

    cfg, wts = _small()
    B, n = 8, 10
    prompts = OQ.prompt_ids(cfg.vocab, 6, seed=12, batch=B)
    a = BatchEngine(cfg, batch=B, device=dev, max_new=12, prompt_room=8, weights=wts)
    b = BatchEngine(cfg, batch=B, device=dev, max_new=12, prompt_room=8, weights=wts, fold_o_norm=True)
    assert b.fold_o_norm and not a.fold_o_norm
    assert_l2("logits", b.logits_for(prompts), a.logits_for(prompts))
    free_a, free_b = a.generate(prompts, n).tokens, b.generate(prompts, n).tokens
    teachers = [t[:-1] for t in free_a]
    picks_a, logits_a = a.forced(prompts, teachers, record_logits=True)
    picks_b, logits_b = b.forced(prompts, teachers, record_logits=True)
    assert picks_a == free_a, "the default engine's forced picks repeat its free run"
    for s in range(B):
        ref = [lg[s] for lg in logits_a]
        ids, vals, gaps = oracle_candidates(ref)
        _, deltas = forced_agreement(f"2-layer bs=8 folded vs default, sequence {s}", picks_b[s], picks_a[s],
                                     [lg[s] for lg in logits_b], ids, vals, gaps, floor=n - 2,
                                     max_delta=logit_bounds(ref))
        diff = next((i for i, (x, y) in enumerate(zip(free_b[s], free_a[s])) if x != y), None)
        if diff is not None:
            assert gaps[diff] <= 2 * deltas[diff], f"seq {s}: folded free run leaves the default at a clear margin"


@pytest.mark.gpu
def test_skinny_residual_refuses(dev):
    from tilefoundry_amd._lib import C

    x = torch.zeros(33, 256, device=dev, dtype=BF)
    w = torch.zeros(64, 256, device=dev, dtype=BF)
    with pytest.raises(ValueError):
        C.skinny_gemm_residual(x, w, torch.zeros(33 * 64, device=dev, dtype=BF),
                               torch.zeros(33, 64, device=dev, dtype=BF), torch.zeros(2, 33, device=dev))
    h = torch.zeros(4, 256, device=dev, dtype=BF)
    with pytest.raises(ValueError):   # 65 partial rows
        C.skinny_gemm_norm_swiglu(h, w, torch.zeros(65, 4, device=dev), torch.zeros(256, device=dev, dtype=BF),
                                  1e-6, torch.zeros(4, 32, device=dev, dtype=BF))


@pytest.mark.gpu
def test_skinny_swiglu(dev):
    from tilefoundry_amd import ops

    g = gen(5)
    M = 32
    xn = randn(M, H, g=g)
    wg = randn(I, H, g=g, std=0.02)
    wu = randn(I, H, g=g, std=0.02)
    gg, uu = OQ.proj(xn, wg), OQ.proj(xn, wu)
    ref = torch.nn.functional.silu(gg.float()).to(BF) * uu
    w_gu = torch.stack([wg, wu], 1).reshape(2 * I, H)
    got = ops.skinny_gemm(xn.to(dev), w_gu.to(dev), "swiglu")
    assert_close("skinny swiglu", got, ref)


@pytest.mark.gpu
@pytest.mark.parametrize("M,V", [(32, 151936), (17, 65552)])   # the second: odd token count, ragged last block
def test_skinny_argmax(dev, M, V):
    from tilefoundry_amd import ops

    g = gen(7 + M)
    x = randn(M, H, g=g)
    w = randn(V, H, g=g, std=0.02)
    ref = x.float() @ w.float().t()
    logits, bv, bi = ops.skinny_gemm(x.to(dev), w.to(dev), "argmax")
    assert max_rel(logits, ref) < 5e-3
    best = bi.gather(1, bv.argmax(1, keepdim=True)).squeeze(1).cpu()
    assert torch.equal(best, logits.cpu().argmax(1).to(torch.int32))
    # every 16-row group's winner is that group's max of the kernel's own logits
    grp = logits.cpu().view(M, V // 16, 16)
    assert torch.equal(bv.cpu(), grp.max(2).values)
    assert torch.equal(bi.cpu(), (grp.argmax(2) + 16 * torch.arange(V // 16)).to(torch.int32))
    # without the logits store the winners are the same
    none, bv2, bi2 = ops.skinny_gemm(x.to(dev), w.to(dev), "argmax", with_logits=False)
    assert none is None
    assert torch.equal(bv2, bv) and torch.equal(bi2, bi)


@pytest.mark.gpu
def test_skinny_argmax_48_row_blocks(dev):
    """A row count whose 48-row blocks fill 256 CUs in one round (ragged tail)."""
    from tilefoundry_amd import ops

    g = gen(9)
    M, V = 5, 12250
    x = randn(M, H, g=g)
    w = randn(V, H, g=g, std=0.02)
    logits, bv, bi = ops.skinny_gemm(x.to(dev), w.to(dev), "argmax")
    assert max_rel(logits, x.float() @ w.float().t()) < 5e-3
    best = bi.gather(1, bv.argmax(1, keepdim=True)).squeeze(1).cpu()
    assert torch.equal(best, logits.cpu().argmax(1).to(torch.int32))


@pytest.mark.gpu
def test_skinny_argmax_ties(dev):
    from tilefoundry_amd import ops

    M, V, K = 3, 4096, 256
    w = torch.zeros(V, K).to(BF)
    for idx in (3000, 40, 41, 2000):
        w[idx, 0] = 1.0
    x = torch.zeros(M, K).to(BF)
    x[:, 0] = 1.0
    logits, bv, bi = ops.skinny_gemm(x.to(dev), w.to(dev), "argmax")
    best = bi.gather(1, bv.argmax(1, keepdim=True)).squeeze(1).cpu().tolist()
    assert best == [40, 40, 40]


@pytest.mark.gpu
def test_rows_norm_embed_and_residual(dev):
    from tilefoundry_amd import ops

    g = gen(9)
    M = 32
    table = randn(1000, H, g=g, std=0.02)
    ids = torch.randint(0, 1000, (M,), generator=g)
    gamma = randn(H, g=g, std=0.1, mean=1.0)
    h, xn = ops.rows_norm(gamma.to(dev), 1e-6, table=table.to(dev), ids=ids.to(dev))
    assert_equal("gathered rows", h, table[ids])
    assert_close("embed norm", xn, ON.rms_norm_q(table[ids], gamma, 1e-6))
    hin = randn(M, H, g=g)
    part = torch.randn(4, M, H, generator=g)
    h2, xn2 = ops.rows_norm(gamma.to(dev), 1e-6, h_in=hin.to(dev), part=part.to(dev))
    href = hin + part.sum(0).to(BF)
    assert_close("residual", h2, href)
    assert_close("residual norm", xn2, ON.rms_norm_q(href, gamma, 1e-6))


@pytest.mark.gpu
def test_batched_attention_from_partials(dev):
    """Per sequence: q/k/v from summed f32 partials, head norm + RoPE at its own
    position, the new K and V rows written at its own slot, attention over its
    own cache -- each against the oracle."""
    from tilefoundry_amd._lib import C

    g = gen(11)
    B, cap, split, ks = 3, 512, 64, 2
    rows = (HQ + 2 * HKV) * D
    part = torch.randn(ks, B, rows, generator=g) * 0.5
    gq = randn(D, g=g, std=0.1, mean=1.0)
    gk = randn(D, g=g, std=0.1, mean=1.0)
    cos, sin = OQ.rope_tables(cap, D, 1.0e6)
    pos = [0, 100, 511]
    kc = torch.zeros(B, cap, HKV, D).to(BF)
    vc = torch.zeros(B, cap, HKV, D).to(BF)
    for b, p in enumerate(pos):
        kc[b, :p] = randn(p, HKV, D, g=g)
        vc[b, :p] = randn(p, HKV, D, g=g)
    kd, vd = kc.view(B, cap, -1).to(dev), vc.view(B, cap, -1).to(dev)
    ns = cap // split
    op = torch.empty(B, ns, HQ, D, device=dev)
    mp = torch.empty(B, ns, HQ, device=dev)
    lp = torch.empty(B, ns, HQ, device=dev)
    posd = torch.tensor(pos, dtype=torch.int32, device=dev)
    C.decode_attention(None, part.to(dev), gq.to(dev), gk.to(dev), 1e-6, cos.to(dev), sin.to(dev),
                       kd, vd, posd, posd, HQ, HKV, split, D ** -0.5, op, mp, lp, False, None)
    out = torch.empty(B, HQ * D, dtype=BF, device=dev)
    C.attn_combine(op, mp, lp, out, posd, split)
    raw = part.sum(0).to(BF)
    for b, p in enumerate(pos):
        q = OQ.rope(OQ.head_norm(raw[b, : HQ * D].view(HQ, D), gq, 1e-6), cos[p], sin[p])
        k = OQ.rope(OQ.head_norm(raw[b, HQ * D: (HQ + HKV) * D].view(HKV, D), gk, 1e-6), cos[p], sin[p])
        v = raw[b, (HQ + HKV) * D:].view(HKV, D)
        assert_close(f"k row b={b}", kd[b, p].view(HKV, D), k)
        assert_equal(f"v row b={b}", vd[b, p].view(HKV, D), v)
        kk = torch.cat([kc[b, :p], k.unsqueeze(0)])
        vv = torch.cat([vc[b, :p], v.unsqueeze(0)])
        assert_close(f"attention b={b}", out[b], OQ.attend(q, kk, vv, D ** -0.5))


@pytest.mark.gpu
@pytest.mark.parametrize("hq,hkv,pos", [(16, 8, [0, 1, 31, 32, 100, 511, 1000, 2111, 4095]),
                                        (8, 8, [0, 77, 300]), (16, 4, [5, 64, 1023])])
def test_batched_attention_seq(dev, hq, hkv, pos):
    """The whole-context form: one block per (sequence, kv head), the prep fused,
    no split merge. Per sequence: the new K and V rows at its own slot, and its
    output against the oracle's unsplit order (exp against the row max, bf16
    weights, o / l landed once) -- contexts from one position to the full
    4096-slot cache, and around the 32-position step."""
    from tilefoundry_amd._lib import C

    g = gen(12)
    B, cap, ks = len(pos), 4096, 2
    rows = (hq + 2 * hkv) * D
    part = torch.randn(ks, B, rows, generator=g) * 0.5
    gq = randn(D, g=g, std=0.1, mean=1.0)
    gk = randn(D, g=g, std=0.1, mean=1.0)
    cos, sin = OQ.rope_tables(cap, D, 1.0e6)
    kc = torch.zeros(B, cap, hkv, D).to(BF)
    vc = torch.zeros(B, cap, hkv, D).to(BF)
    for b, p in enumerate(pos):
        kc[b, :p] = randn(p, hkv, D, g=g)
        vc[b, :p] = randn(p, hkv, D, g=g)
    # slots past each context hold NaN: they must never be read into the result
    for b, p in enumerate(pos):
        kc[b, p + 1:] = float("nan")
        vc[b, p + 1:] = float("nan")
    kd, vd = kc.view(B, cap, -1).to(dev), vc.view(B, cap, -1).to(dev)
    posd = torch.tensor(pos, dtype=torch.int32, device=dev)
    out = torch.empty(B, hq * D, dtype=BF, device=dev)
    err = torch.zeros(1, dtype=torch.int32, device=dev)
    C.decode_attention_seq(part.to(dev), gq.to(dev), gk.to(dev), 1e-6, cos.to(dev), sin.to(dev), posd, posd,
                           kd, vd, hq, hkv, D ** -0.5, out, err)
    assert int(err) == 0
    raw = part.sum(0).to(BF)
    for b, p in enumerate(pos):
        q = OQ.rope(OQ.head_norm(raw[b, : hq * D].view(hq, D), gq, 1e-6), cos[p], sin[p])
        k = OQ.rope(OQ.head_norm(raw[b, hq * D: (hq + hkv) * D].view(hkv, D), gk, 1e-6), cos[p], sin[p])
        v = raw[b, (hq + hkv) * D:].view(hkv, D)
        assert_close(f"k row b={b}", kd[b, p].view(hkv, D), k)
        assert_equal(f"v row b={b}", vd[b, p].view(hkv, D), v)
        kk = torch.cat([kc[b, :p], k.unsqueeze(0)])
        vv = torch.cat([vc[b, :p], v.unsqueeze(0)])
        assert_close(f"attention b={b} ctx {p + 1}", out[b], OQ.attend(q, kk, vv, D ** -0.5, p_bf16=True))


@pytest.mark.gpu
def test_batched_attention_seq_errors(dev):
    """A newest slot outside the cache is flagged (err 4) and that sequence's
    output is zero; a rope position past the table is flagged (err 5); a cache
    too long for the score store and an unsupported group are refused."""
    from tilefoundry_amd._lib import C

    B, cap, hq, hkv = 2, 256, 16, 8
    rows = (hq + 2 * hkv) * D
    part = torch.ones(1, B, rows, device=dev)
    gam = torch.ones(D, dtype=BF, device=dev)
    cos, sin = (t.to(dev) for t in OQ.rope_tables(cap, D, 1.0e6))
    kc = torch.zeros(B, cap, hkv * D, dtype=BF, device=dev)
    vc = torch.zeros_like(kc)
    out = torch.full((B, hq * D), 7.0, dtype=BF, device=dev)
    err = torch.zeros(1, dtype=torch.int32, device=dev)
    wr = torch.tensor([3, cap], dtype=torch.int32, device=dev)
    C.decode_attention_seq(part, gam, gam, 1e-6, cos, sin, wr.clamp(max=cap - 1), wr, kc, vc, hq, hkv, 0.1, out,
                           err)
    assert int(err) == 4
    assert float(out[1].float().abs().max()) == 0.0
    err.zero_()
    pos = torch.tensor([3, cap + 5], dtype=torch.int32, device=dev)
    C.decode_attention_seq(part, gam, gam, 1e-6, cos, sin, pos, torch.tensor([3, 4], dtype=torch.int32, device=dev),
                           kc, vc, hq, hkv, 0.1, out, err)
    assert int(err) == 5
    big = torch.zeros(B, 16384, hkv * D, dtype=BF, device=dev)
    with pytest.raises(ValueError, match="exceeds"):
        C.decode_attention_seq(part, gam, gam, 1e-6, cos, sin, wr, wr, big, big, hq, hkv, 0.1, out, None)
    part8 = torch.ones(1, B, (16 + 4) * D, device=dev)
    kc2 = torch.zeros(B, cap, 2 * D, dtype=BF, device=dev)
    with pytest.raises(ValueError, match="group"):
        C.decode_attention_seq(part8, gam, gam, 1e-6, cos, sin, wr, wr, kc2, kc2, 16, 2, 0.1, out, None)


def _small(layers=2, vocab=8192, seed=5):
    from tilefoundry_amd.qwen3 import Qwen3Config, synthetic_weights

    cfg = Qwen3Config(layers=layers, vocab=vocab)
    return cfg, synthetic_weights(cfg, seed=seed)


def _oracle(wts, cfg):
    from tests.test_qwen3_engine import oracle_cfg, oracle_model

    return oracle_model(wts, cfg), oracle_cfg(cfg)


@pytest.mark.gpu
@pytest.mark.parametrize("attention", ["split", "seq"])
def test_batch_engine_logits(dev, attention):
    from tilefoundry_amd.qwen3 import BatchEngine

    cfg, wts = _small()
    B = 4
    eng = BatchEngine(cfg, batch=B, device=dev, max_new=32, prompt_room=32, weights=wts, attention=attention)
    assert eng.attention == attention
    prompts = OQ.prompt_ids(cfg.vocab, 9, seed=21, batch=B)
    got = eng.logits_for(prompts)
    om, oc = _oracle(wts, cfg)
    cos, sin = OQ.rope_tables(9, cfg.head_dim, cfg.rope_theta)
    for b in range(B):
        caches = OQ.empty_caches(oc, cfg.layers)
        for p, t in enumerate(prompts[b]):
            ref = OQ.step(om, oc, t, p, caches, cos, sin, p_bf16=True)
        assert_l2(f"logits seq {b}", got[b], ref)
        for i in range(cfg.layers):
            kc = eng.kc[i, b, :9].view(9, cfg.kv_heads, cfg.head_dim)
            check = assert_close if i == 0 else assert_l2
            check(f"k cache seq {b} layer {i}", kc, caches[i][0])


@pytest.mark.gpu
def test_batch_engine_greedy(dev):
    """32 sequences teacher-forced along their oracle greedy ids (three of them
    checked against the oracle's bs=1 decode): every pick equals the oracle's
    except at near ties under the measured logit error; the free run of each
    leaves the oracle only at such a tie."""
    from tilefoundry_amd.qwen3 import BatchEngine

    cfg, wts = _small()
    B, n = 32, 16
    eng = BatchEngine(cfg, batch=B, device=dev, max_new=32, prompt_room=32, weights=wts)
    assert eng.attention == "seq"   # 32 sequences x 8 kv heads fill the device
    prompts = OQ.prompt_ids(cfg.vocab, 8, seed=22, batch=B)
    om, oc = _oracle(wts, cfg)
    checked = (0, 7, 31)
    wants, recs = {}, {}
    for b in checked:
        rec = []
        wants[b] = OQ.decode(om, oc, prompts[b], n, record=rec, p_bf16=True)
        recs[b] = rec
    teachers = [wants[b][:-1] if b in wants else prompts[b][:1] * (n - 1) for b in range(B)]
    picks, logits = eng.forced(prompts, teachers, record_logits=True)
    gen = eng.generate(prompts, n)
    for b in checked:
        ids, vals, gaps = oracle_candidates([r[0] for r in recs[b]])
        _, deltas = forced_agreement(f"2-layer bs=32, sequence {b}", picks[b], wants[b], [lg[b] for lg in logits],
                                     ids, vals, gaps, floor=n - 2,
                                     max_delta=logit_bounds([r[0] for r in recs[b]]))
        diff = next((i for i, (x, y) in enumerate(zip(gen.tokens[b], wants[b])) if x != y), None)
        if diff is not None:
            assert gaps[diff] <= 2 * deltas[diff], f"seq {b}: free run leaves the oracle at a clear margin"


@pytest.mark.gpu
@pytest.mark.parametrize("attention", ["split", "seq"])
def test_batch_engine_matches_single_engine(dev, attention):
    """The batch engine and the bs=1 engine agree on a sequence's logits."""
    from tilefoundry_amd.qwen3 import BatchEngine, Engine

    cfg, wts = _small()
    prompts = OQ.prompt_ids(cfg.vocab, 6, seed=23, batch=2)
    be = BatchEngine(cfg, batch=2, device=dev, max_new=16, prompt_room=16, weights=wts, attention=attention)
    se = Engine(cfg, device=dev, max_new=16, prompt_room=16, weights=wts)
    got = be.logits_for(prompts)
    for b in range(2):
        assert_l2(f"seq {b}", got[b], se.logits_for(prompts[b]))


@pytest.mark.gpu
def test_full_model_batch32_golden(dev):
    """The full Qwen3-1.7B-shaped model (28 layers, vocab 151936) at bs=32:
    teacher-forced along the oracle's 32 greedy ids of 4 of the 32 sequences
    (tests/golden/qwen3_batch_golden.json, the oracle stepping them together),
    every pick equals the oracle's except at near ties under the measured logit
    error; the agreement count is printed per sequence. This model's logits are
    flat: 22-25 of each sequence's 32 positions have a top-2 gap under 0.26, twice
    the largest logit spread between the oracle's own two valid orders."""
    import json
    from pathlib import Path

    from tests.test_qwen3_engine import FULL_MODEL_MAX_DELTA
    from tilefoundry_amd.qwen3 import BatchEngine, QWEN3_1_7B

    gold = json.loads((Path(__file__).parent / "golden" / "qwen3_batch_golden.json").read_text())
    B, keep = gold["batch"], gold["kept"]
    prompts = OQ.prompt_ids(QWEN3_1_7B.vocab, len(gold["prompts"][0]), seed=gold["prompt_seed"], batch=B)
    assert prompts[:keep] == gold["prompts"]
    n = len(gold["tokens"][0])
    eng = BatchEngine(QWEN3_1_7B, batch=B, device=dev, max_new=n, prompt_room=len(prompts[0]), seed=gold["seed"])
    filler = OQ.prompt_ids(QWEN3_1_7B.vocab, n - 1, seed=99, batch=B)
    teachers = [gold["tokens"][b][:-1] if b < keep else filler[b] for b in range(B)]
    picks, logits = eng.forced(prompts, teachers, record_logits=True)
    total = 0
    for b in range(keep):
        agree, _ = forced_agreement(f"28-layer bs=32, sequence {b}, 32 teacher-forced positions", picks[b],
                                    gold["tokens"][b], [lg[b] for lg in logits], gold["top_ids"][b],
                                    gold["top_vals"][b], gold["gaps"][b], floor=n - 8,
                                    max_delta=FULL_MODEL_MAX_DELTA)
        total += agree
    print(f"[agreement] 28-layer bs=32: {total}/{keep * n} over the {keep} checked sequences", flush=True)
    # the bs=1 model's own two valid orders agree on 91 % of picks (233 / 256);
    # over 128 positions hold the batch to 87.5 %
    assert total >= 112, f"{total}/{keep * n}"
