"""Decode kernels (weights [N, K]) on the GPU against the CPU oracle.

Shapes are the Qwen3-1.7B layer's (hidden 2048, 16 q / 8 kv heads, head_dim
128, intermediate 6144, vocab 151936) plus edge shapes. Tolerances: the
reference's GEMV rtol 5e-3 and the bf16 bar (max |d| / max |ref| <= 1e-2)
everywhere else (examples/qwen3_1_7b-tilelang/fast/test_kernels.py:18-29,66,78);
integer and index outputs exactly.
"""
import math

import pytest
import torch

from oracle import norms as ON
from oracle import qwen3 as OQ
from tests._check import assert_close, assert_equal, max_rel

BF = torch.bfloat16
H, HQ, HKV, D, I, V = 2048, 16, 8, 128, 6144, 151936
EPS = 1e-6


def gen(seed):
    return torch.Generator().manual_seed(seed)


def randn(*shape, g, std=1.0, mean=0.0):
    return (mean + std * torch.randn(*shape, generator=g)).to(BF)


@pytest.mark.gpu
@pytest.mark.parametrize("N,K", [(4096, 2048), (2048, 2048), (2048, 6144), (1056, 2560), (3840, 768), (96, 256)])
def test_gemv(dev, N, K):
    from tilefoundry_amd import ops

    g = gen(N + K)
    x = randn(K, g=g)
    w = randn(N, K, g=g, std=K ** -0.5)
    ref = x.float() @ w.float().t()
    got = ops.gemv(x.to(dev), w.to(dev), out_dtype=torch.float32)
    assert max_rel(got, ref) < 5e-3
    gotb = ops.gemv(x.to(dev), w.to(dev))
    assert_close("gemv bf16", gotb, ref.to(BF))


@pytest.mark.gpu
def test_gemv_exact_on_integers(dev):
    """Integer-valued bf16 inputs with small sums: every product and partial sum is
    exact in f32, so the result must equal the integer matmul bit for bit."""
    from tilefoundry_amd import ops

    g = gen(7)
    x = torch.randint(-3, 4, (2048,), generator=g).to(BF)
    w = torch.randint(-3, 4, (512, 2048), generator=g).to(BF)
    ref = (x.to(torch.int64) @ w.to(torch.int64).t()).to(torch.float32)
    got = ops.gemv(x.to(dev), w.to(dev), out_dtype=torch.float32)
    assert_equal("integer gemv", got, ref)


@pytest.mark.gpu
@pytest.mark.parametrize("N,K", [(4096, 2048), (1056, 2560)])
def test_rmsnorm_gemv(dev, N, K):
    from tilefoundry_amd import ops

    g = gen(11)
    h = randn(K, g=g)
    gamma = randn(K, g=g, std=0.1, mean=1.0)
    w = randn(N, K, g=g, std=0.02)
    ref = OQ.proj(ON.rms_norm_q(h, gamma, EPS), w)
    got = ops.rmsnorm_gemv(h.to(dev), gamma.to(dev), EPS, w.to(dev))
    assert_close("rmsnorm_gemv", got, ref)


@pytest.mark.gpu
@pytest.mark.parametrize("N,K,scaled", [(2048, 2048, False), (2048, 6144, False), (2560, 2560, True)])
def test_gemv_residual(dev, N, K, scaled):
    from tilefoundry_amd import ops

    g = gen(13)
    x = randn(K, g=g)
    w = randn(N, K, g=g, std=0.02)
    r = randn(N, g=g)
    alpha = torch.tensor([1.4 / math.sqrt(62)]).to(BF) if scaled else None
    p = OQ.proj(x, w)
    ref = r + (p * alpha if scaled else p)
    got = ops.gemv_residual(x.to(dev), w.to(dev), r.to(dev),
                            alpha.to(dev) if scaled else None)
    assert_close("gemv_residual", got, ref)


@pytest.mark.gpu
def test_rmsnorm_gemv_swiglu(dev):
    from tilefoundry_amd import ops

    g = gen(17)
    h = randn(H, g=g)
    gamma = randn(H, g=g, std=0.1, mean=1.0)
    wg = randn(I, H, g=g, std=0.02)
    wu = randn(I, H, g=g, std=0.02)
    xn = ON.rms_norm_q(h, gamma, EPS)
    gg, uu = OQ.proj(xn, wg), OQ.proj(xn, wu)
    ref = torch.nn.functional.silu(gg.float()).to(BF) * uu
    w_gu = torch.stack([wg, wu], 1).reshape(2 * I, H)
    got = ops.rmsnorm_gemv_swiglu(h.to(dev), gamma.to(dev), EPS, w_gu.to(dev))
    assert_close("swiglu", got, ref)


@pytest.mark.gpu
def test_lm_head_argmax(dev):
    from tilefoundry_amd import ops

    g = gen(19)
    h = randn(H, g=g)
    gamma = randn(H, g=g, std=0.1, mean=1.0)
    w = randn(V, H, g=g, std=0.02)
    ref = OQ.lm_logits(h, gamma, w.float(), EPS)
    logits, best = ops.greedy_pick(h.to(dev), gamma.to(dev), EPS, w.to(dev))
    assert max_rel(logits, ref) < 5e-3
    assert best == int(torch.argmax(logits.cpu())), "argmax of the kernel's own logits"
    top = torch.topk(ref, 2).values
    if float(top[0] - top[1]) > 1e-3 * float(ref.abs().max()):
        assert best == int(torch.argmax(ref))


@pytest.mark.gpu
def test_lm_head_planted_ties(dev):
    """Identical rows give identical logits: the lowest index must win
    (torch.argmax; examples/qwen3_1_7b-tilelang/fast/kernels.py:303-319)."""
    from tilefoundry_amd import ops

    g = gen(23)
    Vs, K = 4096, 256
    w = randn(Vs, K, g=g, std=0.02)
    x = randn(K, g=g)
    winner = torch.tensor([3.0] * 8 + [1.0] * (K - 8)).to(BF)
    for idx in (4000, 17, 2500, 18):   # same max planted at four rows, in two blocks
        w[idx] = winner
    x[:8] = 1.0
    logits, best = ops.greedy_pick(x.to(dev), None, EPS, w.to(dev))
    lg = logits.cpu()
    assert best == int(torch.argmax(lg)) == 17


@pytest.mark.gpu
@pytest.mark.parametrize("pos,expect_prompt", [(2, True), (4, False), (20, False)])
def test_sample_step(dev, pos, expect_prompt):
    """The device-side greedy step: record the pick at pos; feed the next prompt
    id while the prompt lasts, else the pick; advance pos
    (examples/qwen3_1_7b-tilelang/fast/test_kernels.py:171-189)."""
    from tilefoundry_amd import ops

    g = gen(29)
    NB, NSTEPS, PL = 1187, 64, 5
    bv = torch.randn(NB, generator=g)
    bi = torch.randint(0, V, (NB,), generator=g, dtype=torch.int32)
    st = ops.SampleState(NSTEPS, dev)
    st.inp.copy_(torch.arange(NSTEPS, dtype=torch.int32) + 100)
    st.plen.fill_(PL)
    st.pos.fill_(pos)
    ops.sample_step(bv.to(dev), bi.to(dev), st)
    best = int(bi[int(bv.argmax())])
    want_next = pos + 1 + 100 if expect_prompt else best
    assert int(st.sam[pos]) == best
    assert int(st.ids[0]) == want_next
    assert int(st.pos[0]) == pos + 1
    assert int(st.err[0]) == 0


@pytest.mark.gpu
def test_sample_step_ties_lowest_index(dev):
    from tilefoundry_amd import ops

    bv = torch.tensor([1.0, 5.0, 2.0, 5.0, 5.0])
    bi = torch.tensor([10, 900, 20, 300, 301], dtype=torch.int32)
    st = ops.SampleState(8, dev)
    st.plen.fill_(1)
    ops.sample_step(bv.to(dev), bi.to(dev), st)
    assert int(st.sam[0]) == 300


def _qkv_case(g, cap=512):
    h = randn(H, g=g)
    gamma_in = randn(H, g=g, std=0.1, mean=1.0)
    wq = randn(HQ * D, H, g=g, std=0.02)
    wk = randn(HKV * D, H, g=g, std=0.02)
    wv = randn(HKV * D, H, g=g, std=0.02)
    gq = randn(D, g=g, std=0.1, mean=1.0)
    gk = randn(D, g=g, std=0.1, mean=1.0)
    cos, sin = OQ.rope_tables(cap, D, 1.0e6)
    return h, gamma_in, wq, wk, wv, gq, gk, cos, sin


def _qkv_ref(h, gamma_in, wq, wk, wv, gq, gk, cos, sin, pos):
    xn = ON.rms_norm_q(h, gamma_in, EPS)
    q = OQ.rope(OQ.head_norm(OQ.proj(xn, wq).view(HQ, D), gq, EPS), cos[pos], sin[pos])
    k = OQ.rope(OQ.head_norm(OQ.proj(xn, wk).view(HKV, D), gk, EPS), cos[pos], sin[pos])
    v = OQ.proj(xn, wv).view(HKV, D)
    return q, k, v


@pytest.mark.gpu
@pytest.mark.parametrize("wr", [0, 37, 511])
def test_decode_qkv(dev, wr):
    """Raw q|k out, v into exactly one cache row (bit-exact cache indexing)."""
    from tilefoundry_amd import ops

    cap = 512
    h, gamma_in, wq, wk, wv, *_ = _qkv_case(gen(31 + wr), cap)
    xn = ON.rms_norm_q(h, gamma_in, EPS)
    vc = torch.zeros(cap, HKV * D, dtype=BF, device=dev)
    w_qkv = torch.cat([wq, wk, wv], 0).to(dev)
    qk = ops.decode_qkv(h.to(dev), gamma_in.to(dev), EPS, w_qkv, (HQ + HKV) * D, wr, vc)
    assert_close("q raw", qk[: HQ * D], OQ.proj(xn, wq))
    assert_close("k raw", qk[HQ * D:], OQ.proj(xn, wk))
    assert_close("v", vc[wr], OQ.proj(xn, wv))
    written = (vc.cpu().view(torch.int16) != 0).any(1).nonzero().flatten().tolist()
    assert written == [wr]


@pytest.mark.gpu
def test_decode_qkv_embed_mode(dev):
    from tilefoundry_amd import ops

    cap = 64
    g = gen(37)
    table = randn(1000, H, g=g, std=0.02)
    _, gamma_in, wq, wk, wv, *_ = _qkv_case(g, cap)
    tok = 777
    xn = ON.rms_norm_q(table[tok], gamma_in, EPS)
    vc = torch.zeros(cap, HKV * D, dtype=BF, device=dev)
    hcopy = torch.zeros(H, dtype=BF, device=dev)
    w_qkv = torch.cat([wq, wk, wv], 0).to(dev)
    qk = ops.decode_qkv(None, gamma_in.to(dev), EPS, w_qkv, (HQ + HKV) * D, 3, vc,
                        table=table.to(dev), token=tok, h_copy=hcopy)
    assert_equal("gathered row", hcopy, table[tok])
    assert_close("q raw", qk[: HQ * D], OQ.proj(xn, wq))
    assert_close("v", vc[3], OQ.proj(xn, wv))


@pytest.mark.gpu
@pytest.mark.parametrize("pos,wr", [(0, 0), (37, 37), (300, 5), (511, 511)])
def test_fused_attention_prologue(dev, pos, wr):
    """q / k head norm + RoPE at pos inside the attention kernel; the new key lands
    in k_cache[wr] and only there; the output attends slots 0..wr."""
    from tilefoundry_amd import ops

    cap = 512
    args = _qkv_case(gen(53 + pos), cap)
    h, gamma_in, wq, wk, wv, gq, gk, cos, sin = args
    qr, kr, vr = _qkv_ref(*args, pos)
    g = gen(59)
    kc = torch.zeros(cap, HKV, D, dtype=BF)
    vc = torch.zeros(cap, HKV, D, dtype=BF)
    kc[:wr] = randn(wr, HKV, D, g=g)
    vc[:wr] = randn(wr, HKV, D, g=g)
    vc[wr] = vr
    xn = ON.rms_norm_q(h, gamma_in, EPS)
    qk_raw = torch.cat([OQ.proj(xn, wq), OQ.proj(xn, wk)])
    kd, vd = kc.view(cap, -1).to(dev), vc.view(cap, -1).to(dev)
    out = ops.decode_attention(qk_raw.to(dev), kd, vd, wr, HQ, HKV, split=64,
                               rope=(gq.to(dev), gk.to(dev), EPS, cos.to(dev), sin.to(dev), pos))
    assert_close("k written", kd[wr].view(HKV, D), kr)
    before = kc.view(cap, -1).clone()
    before[wr] = kd[wr].cpu()
    assert_equal("no other cache row touched", kd, before)
    kk = torch.cat([kc[:wr], kr.unsqueeze(0)])
    ref = OQ.attend(qr, kk, vc[: wr + 1], D ** -0.5)
    assert_close("attention output", out, ref)


@pytest.mark.gpu
@pytest.mark.parametrize("wr", [512, -1])
def test_fused_attention_bad_write_slot(dev, wr):
    """A write slot outside the cache is flagged (err 4) and no cache row is
    written -- the split path's rule is the whole-context kernel's; a rope
    position past the table is flagged (err 5)."""
    from tilefoundry_amd import ops

    cap = 512
    h, gamma_in, wq, wk, wv, gq, gk, cos, sin = _qkv_case(gen(71), cap)
    xn = ON.rms_norm_q(h, gamma_in, EPS)
    qk_raw = torch.cat([OQ.proj(xn, wq), OQ.proj(xn, wk)]).to(dev)
    kd = randn(cap, HKV * D, g=gen(72)).to(dev)
    vd = randn(cap, HKV * D, g=gen(73)).to(dev)
    k0, v0 = kd.clone(), vd.clone()
    rope = (gq.to(dev), gk.to(dev), EPS, cos.to(dev), sin.to(dev), 7)
    err = torch.zeros(1, dtype=torch.int32, device=dev)
    ops.attn_partial(qk_raw, kd, vd, wr, HQ, HKV, split=64, rope=rope, neutral=True, err=err)
    torch.cuda.synchronize()
    assert int(err) == 4
    assert_equal("k cache untouched", kd, k0)
    assert_equal("v cache untouched", vd, v0)
    err.zero_()
    rope_bad = rope[:5] + (cap + 3,)
    ops.attn_partial(qk_raw, kd, vd, 9, HQ, HKV, split=64, rope=rope_bad, neutral=True, err=err)
    torch.cuda.synchronize()
    assert int(err) == 5


@pytest.mark.gpu
def test_rope_position_zero_is_identity(dev):
    """At position 0 (cos = 1, sin = 0) the key written is exactly the head-normed
    projection: RoPE contributes nothing."""
    from tilefoundry_amd import ops

    cap = 64
    h, gamma_in, wq, wk, wv, gq, gk, cos, sin = _qkv_case(gen(41), cap)
    xn = ON.rms_norm_q(h, gamma_in, EPS)
    k_raw = OQ.proj(xn, wk)
    qk_raw = torch.cat([OQ.proj(xn, wq), k_raw])
    kd = torch.zeros(cap, HKV * D, dtype=BF, device=dev)
    vd = torch.zeros(cap, HKV * D, dtype=BF, device=dev)
    ops.decode_attention(qk_raw.to(dev), kd, vd, 0, HQ, HKV, split=64,
                         rope=(gq.to(dev), gk.to(dev), EPS, cos.to(dev), sin.to(dev), 0))
    assert_equal("k at pos 0", kd[0].view(HKV, D), OQ.head_norm(k_raw.view(HKV, D), gk, EPS))


def _attn_case(g, cap, n):
    q = randn(HQ, D, g=g)
    kc = torch.zeros(cap, HKV, D, dtype=BF)
    vc = torch.zeros(cap, HKV, D, dtype=BF)
    kc[:n] = randn(n, HKV, D, g=g)
    vc[:n] = randn(n, HKV, D, g=g)
    return q, kc, vc


@pytest.mark.gpu
@pytest.mark.parametrize("n", [1, 5, 64, 65, 256, 257, 700, 2048, 4096])
@pytest.mark.parametrize("split", [64, 256])
def test_decode_attention(dev, n, split):
    from tilefoundry_amd import ops

    cap = 4096
    q, kc, vc = _attn_case(gen(n), cap, n)
    ref = OQ.attend(q, kc[:n], vc[:n], D ** -0.5)
    got = ops.decode_attention(q.reshape(-1).to(dev), kc.view(cap, -1).to(dev),
                               vc.view(cap, -1).to(dev), n - 1, HQ, HKV, split=split)
    assert_close(f"attention n={n}", got, ref)


@pytest.mark.gpu
def test_attention_single_key_returns_value(dev):
    from tilefoundry_amd import ops

    cap = 128
    q, kc, vc = _attn_case(gen(43), cap, 1)
    got = ops.decode_attention(q.reshape(-1).to(dev), kc.view(cap, -1).to(dev),
                               vc.view(cap, -1).to(dev), 0, HQ, HKV).cpu()
    want = vc[0].repeat_interleave(HQ // HKV, 0).reshape(-1)
    assert_equal("one key", got, want)


@pytest.mark.gpu
def test_attention_neutral_partials_and_full_combine(dev):
    """Neutral partials past the context merged over every split equal the merge
    over the active splits only."""
    from tilefoundry_amd import ops

    cap, n = 2560, 700
    q, kc, vc = _attn_case(gen(47), cap, n)
    kd, vd, qd = kc.view(cap, -1).to(dev), vc.view(cap, -1).to(dev), q.reshape(-1).to(dev)
    op, mp, lp = ops.attn_partial(qd, kd, vd, n - 1, HQ, HKV, split=256, neutral=True)
    neutral = torch.tensor(-1.0e30, dtype=torch.float32).item()
    assert float(lp[3:].abs().max()) == 0.0 and float(mp[3:].max()) == neutral
    full = ops.attn_combine(op, mp, lp)
    active = ops.attn_combine(op, mp, lp, wr=n - 1, split=256)
    assert_equal("combine over all == over active", full, active)


@pytest.mark.gpu
@pytest.mark.parametrize("hq,n,ns,wr", [(16, 2048, 1, 0), (16, 2048, 17, 1050), (16, 2048, 33, 2100),
                                        (16, 2048, 64, 4095), (16, 2048, 64, 1000), (8, 1000, 40, 2000),
                                        (4, 96, 5, None)])
def test_attn_combine_gemv_residual_bit_equal(dev, hq, n, ns, wr):
    """The split merge folded into o_proj equals attn_combine followed by
    gemv_residual bit for bit: the merged vector and y, with stale splits past
    the write slot (never read into the result), ragged rows and small heads."""
    from tilefoundry_amd._lib import C

    g = gen(51 + ns + hq)
    split = 64
    op = torch.randn(ns, hq, D, generator=g).to(dev)
    mp = (3.0 * torch.randn(ns, hq, generator=g)).to(dev)
    lp = (1.0 + torch.rand(ns, hq, generator=g) * 60).to(dev)
    w_o = randn(n, hq * D, g=g, std=0.02).to(dev)
    res = randn(n, g=g).to(dev)
    wrd = None if wr is None else torch.tensor([wr], dtype=torch.int32, device=dev)
    attn = torch.empty(hq * D, dtype=BF, device=dev)
    C.attn_combine(op, mp, lp, attn, wrd, split)
    want = torch.empty(n, dtype=BF, device=dev)
    C.gemv_residual(attn, w_o, res, None, want)
    got = torch.empty(n, dtype=BF, device=dev)
    a2 = torch.empty(hq * D, dtype=BF, device=dev)
    C.attn_combine_gemv_residual(op, mp, lp, wrd, split, w_o, res, got, a2)
    assert_equal("merged attention", a2, attn)
    assert_equal("o_proj + residual", got, want)


@pytest.mark.gpu
def test_attn_combine_gemv_residual_refuses(dev):
    from tilefoundry_amd._lib import C

    op = torch.zeros(65, 16, D, device=dev)
    mp = torch.zeros(65, 16, device=dev)
    w_o = torch.zeros(2048, 16 * D, dtype=BF, device=dev)
    h = torch.zeros(2048, dtype=BF, device=dev)
    with pytest.raises(ValueError, match="splits"):
        C.attn_combine_gemv_residual(op, mp, mp, None, 64, w_o, h, h.clone(), None)
    w_big = torch.zeros(4096, 16 * D, dtype=BF, device=dev)
    h4 = torch.zeros(4096, dtype=BF, device=dev)
    with pytest.raises(ValueError, match="2560"):
        C.attn_combine_gemv_residual(op[:8], mp[:8], mp[:8], None, 64, w_big, h4, h4.clone(), None)
