"""The per-op factories under the reference's names (tilefoundry_amd.kernels),
each against the oracle's statement of the same operation at Qwen3-1.7B
dimensions -- the cases of examples/qwen3_1_7b-tilelang/fast/test_kernels.py
(t_rms_norm ... t_sample_step), with weights in the (out, in) layout and
inputs drawn on the CPU from seeded generators."""
import pytest
import torch

from oracle import norms as ON
from oracle import qwen3 as OQ
from tests._check import assert_close, assert_equal, assert_ulps

BF = torch.bfloat16
H, HQ, HKV, D, I, V = 2048, 16, 8, 128, 6144, 151936
EPS = 1e-6
MP = 4096


def g(seed):
    return torch.Generator().manual_seed(seed)


@pytest.fixture(scope="module")
def K():
    from tilefoundry_amd import kernels

    return kernels


def randn(*shape, seed, scale=1.0, dtype=BF):
    return (torch.randn(*shape, generator=g(seed)) * scale).to(dtype)


@pytest.mark.gpu
def test_rms_norm(K, dev):
    x, gm = randn(H, seed=1), randn(H, seed=2)
    out = torch.empty(H, device=dev, dtype=BF)
    K.rms_norm(H, EPS)(x.to(dev), gm.to(dev), out)
    assert_ulps("rms_norm", out, ON.rms_norm_q(x, gm, EPS), max_ulps=1, max_frac=0.01)


@pytest.mark.gpu
def test_resid_rms_norm(K, dev):
    SK = 8
    a, gm = randn(H, seed=3), randn(H, seed=4)
    p = randn(SK, H, seed=5, dtype=torch.float32)
    ho = torch.empty(H, device=dev, dtype=BF)
    xn = torch.empty(H, device=dev, dtype=BF)
    K.resid_rms_norm(H, SK, EPS)(a.to(dev), p.to(dev), gm.to(dev), ho, xn)
    h_ref, xn_ref = ON.resid_rms_norm(a, p, gm, EPS)
    assert_ulps("resid_rms_norm.h", ho, h_ref, max_ulps=1, max_frac=0.01)
    assert_ulps("resid_rms_norm.xn", xn, xn_ref, max_ulps=1, max_frac=0.01)


@pytest.mark.gpu
@pytest.mark.parametrize("Kd,N,BN,BK,SK,thr", [
    (H, 4096, 256, 64, 8, 256), (H, H, 128, 128, 8, 128),
    (H, 2 * I, 256, 64, 2, 256), (I, H, 128, 128, 8, 128),
])
def test_gemv(K, dev, Kd, N, BN, BK, SK, thr):
    x = randn(Kd, seed=6)
    w = randn(N, Kd, seed=7, scale=Kd ** -0.5)
    p = torch.empty(SK, N, device=dev, dtype=torch.float32)
    K.gemv(Kd, N, BN, BK, SK, thr)(x.to(dev), w.to(dev), p)
    ref = x.double() @ w.double().t()
    assert_close(f"gemv {Kd}x{N}", p.sum(0), ref, rtol=5e-3)
    # split s is the dot over the s-th contiguous K / SK slice
    ks = Kd // SK
    for s in (0, SK - 1):
        part = x[s * ks:(s + 1) * ks].double() @ w[:, s * ks:(s + 1) * ks].double().t()
        assert_close(f"gemv split {s}", p[s], part, rtol=5e-3)


@pytest.mark.gpu
def test_gemv_rejects_kn_layout(K, dev):
    x = torch.zeros(H, device=dev, dtype=BF)
    w = torch.zeros(H, 4096, device=dev, dtype=BF)
    p = torch.empty(8, 4096, device=dev, dtype=torch.float32)
    with pytest.raises(ValueError, match="layout"):
        K.gemv(H, 4096, 256, 64, 8, 256)(x, w, p)


@pytest.mark.gpu
def test_gemv_attn_combine(K, dev):
    NS, SK = 4, 8
    op = randn(NS, HQ, D, seed=8, dtype=torch.float32)
    mp = randn(NS, HQ, seed=9, dtype=torch.float32)
    lp = (torch.rand(NS, HQ, generator=g(10)) + 0.5)
    # the last split is past the context: the neutral partial
    op[-1], mp[-1], lp[-1] = 0.0, -1.0e30, 0.0
    w = randn(H, HQ * D, seed=11, scale=(HQ * D) ** -0.5)
    p = torch.empty(SK, H, device=dev, dtype=torch.float32)
    K.gemv_attn_combine(HQ, D, H, 128, 128, SK, NS, 128)(op.to(dev), mp.to(dev), lp.to(dev),
                                                        w.to(dev), p)
    m = mp.double().max(0).values
    e = torch.exp(mp.double() - m)
    attn = ((op.double() * e[..., None]).sum(0) / (lp.double() * e).sum(0)[:, None]).to(BF)
    ref = attn.reshape(-1).double() @ w.double().t()
    assert_close("gemv_attn_combine", p.sum(0), ref, rtol=5e-3)
    # a caller-owned workspace gives the same bits; a wrong one is refused
    fn = K.gemv_attn_combine(HQ, D, H, 128, 128, SK, NS, 128)
    p2 = torch.empty_like(p)
    fn(op.to(dev), mp.to(dev), lp.to(dev), w.to(dev), p2, workspace=torch.empty(HQ * D, device=dev, dtype=BF))
    assert torch.equal(p2, p)
    with pytest.raises(ValueError, match="workspace"):
        fn(op.to(dev), mp.to(dev), lp.to(dev), w.to(dev), p2, workspace=torch.empty(HQ * D, device=dev))


@pytest.mark.gpu
def test_gemv_silu(K, dev):
    SK, SKG = 8, 2
    gu = randn(SKG, 2 * I, seed=12, dtype=torch.float32)
    w = randn(H, I, seed=13, scale=I ** -0.5)
    p = torch.empty(SK, H, device=dev, dtype=torch.float32)
    K.gemv_silu(I, H, 128, 128, SK, SKG, 128)(gu.to(dev), w.to(dev), p)
    s = gu.sum(0)
    gb, ub = s[:I].to(BF), s[I:].to(BF)
    act = torch.nn.functional.silu(gb.float()).to(BF) * ub
    assert_close("gemv_silu", p.sum(0), act.double() @ w.double().t(), rtol=5e-3)
    fn = K.gemv_silu(I, H, 128, 128, SK, SKG, 128)
    p2 = torch.empty_like(p)
    fn(gu.to(dev), w.to(dev), p2, workspace=torch.empty(I, device=dev, dtype=BF))
    assert torch.equal(p2, p)
    assert fn.reserve(torch.device(dev)).numel() == I


@pytest.mark.gpu
def test_lm_head(K, dev):
    x = randn(H, seed=14)
    w = randn(V, H, seed=15, scale=H ** -0.5)
    kern, NB = K.lm_head(H, V, 128, 128, 128)
    o = torch.empty(V, device=dev, dtype=torch.float32)
    bv = torch.empty(NB, device=dev, dtype=torch.float32)
    bi = torch.empty(NB, device=dev, dtype=torch.int32)
    kern(x.to(dev), w.to(dev), o, bv, bi)
    ref = x.float() @ w.float().t()
    assert_close("lm_head.logits", o, ref, rtol=5e-3)
    got = int(bi[int(bv.argmax())])
    assert got == int(o.argmax()), "block winners disagree with the logits"
    assert got == int(ref.argmax())


@pytest.mark.gpu
@pytest.mark.parametrize("pos,wr", [(37, 37), (100, 5)])
def test_qk_rope_cache(K, dev, pos, wr):
    """Pos (rotary position) and Wr (cache slot) are separate parameters; the
    authored reference lets them differ."""
    SK, CAP = 8, 512
    p = randn(SK, HQ * D + 2 * HKV * D, seed=16, dtype=torch.float32) / SK
    gq, gk = randn(D, seed=17), randn(D, seed=18)
    cos, sin = OQ.rope_tables(MP, D, 1.0e6)
    kc = torch.zeros(CAP, HKV * D, device=dev, dtype=BF)
    vc = torch.zeros(CAP, HKV * D, device=dev, dtype=BF)
    q = torch.empty(HQ * D, device=dev, dtype=BF)
    pt = torch.tensor([pos], device=dev, dtype=torch.int32)
    wt = torch.tensor([wr], device=dev, dtype=torch.int32)
    K.qk_rope_cache(HQ, HKV, D, MP, CAP, SK, EPS)(p.to(dev), gq.to(dev), gk.to(dev), cos.to(dev),
                                                  sin.to(dev), pt, wt, kc, vc, q)
    flat = p.sum(0).to(BF)
    qr = flat[: HQ * D].view(HQ, D)
    kr = flat[HQ * D: HQ * D + HKV * D].view(HKV, D)
    vr = flat[HQ * D + HKV * D:].view(HKV, D)
    q_ref = OQ.rope(OQ.head_norm(qr, gq, EPS), cos[pos], sin[pos])
    k_ref = OQ.rope(OQ.head_norm(kr, gk, EPS), cos[pos], sin[pos])
    assert_ulps("qk_rope.q", q.view(HQ, D), q_ref, max_ulps=1, max_frac=0.01)
    assert_ulps("qk_rope.k", kc[wr].view(HKV, D), k_ref, max_ulps=1, max_frac=0.01)
    assert_ulps("qk_rope.v", vc[wr].view(HKV, D), vr, max_ulps=1, max_frac=0.001)
    # no other row of either cache is touched
    kc[wr] = 0
    vc[wr] = 0
    assert not bool(kc.any()) and not bool(vc.any())


@pytest.mark.gpu
@pytest.mark.parametrize("cur", [1, 5, 256, 257, 700, 2048])
def test_attn_partial_combine(K, dev, cur):
    CAP, SS = 2560, 256
    pos = cur - 1
    q = randn(HQ, D, seed=19)
    kc = torch.zeros(CAP, HKV, D, dtype=BF)
    vc = torch.zeros(CAP, HKV, D, dtype=BF)
    kc[:cur] = randn(cur, HKV, D, seed=20)
    vc[:cur] = randn(cur, HKV, D, seed=21)
    pt = torch.tensor([pos], device=dev, dtype=torch.int32)
    NS = CAP // SS
    op = torch.empty(NS, HQ, D, device=dev, dtype=torch.float32)
    mp = torch.empty(NS, HQ, device=dev, dtype=torch.float32)
    lp = torch.empty(NS, HQ, device=dev, dtype=torch.float32)
    out = torch.empty(HQ * D, device=dev, dtype=BF)
    K.attn_partial(HQ, HKV, D, CAP, SS, D ** -0.5)(q.reshape(-1).to(dev), kc.view(CAP, -1).to(dev),
                                                    vc.view(CAP, -1).to(dev), pt, op, mp, lp)
    K.attn_combine(HQ, D, CAP, SS)(op, mp, lp, out)
    ref = OQ.attend(q, kc[:cur], vc[:cur], D ** -0.5, p_bf16=True)
    assert_close(f"attn cur={cur}", out, ref, rtol=2e-2, cos_tol=1e-4)
    # splits past the context hold the neutral partial
    live = (cur + SS - 1) // SS
    if live < NS:
        neutral = float(torch.tensor(-1.0e30, dtype=torch.float32))
        assert float(mp[live:].max()) == neutral and float(lp[live:].abs().max()) == 0.0


@pytest.mark.gpu
def test_silu_mul(K, dev):
    SK = 2
    p = randn(SK, 2 * I, seed=22, dtype=torch.float32)
    o = torch.empty(I, device=dev, dtype=BF)
    K.silu_mul(I, SK)(p.to(dev), o)
    s = p.sum(0)
    gb, ub = s[:I].to(BF), s[I:].to(BF)
    ref = torch.nn.functional.silu(gb.float()).to(BF) * ub
    assert_ulps("silu_mul", o, ref, max_ulps=1, max_frac=0.01)


@pytest.mark.gpu
def test_embed(K, dev):
    tbl = randn(1024, H, seed=23)
    ids = torch.tensor([517], device=dev, dtype=torch.int64)
    o = torch.empty(H, device=dev, dtype=BF)
    K.embed(1024, H)(tbl.to(dev), ids, o)
    assert_equal("embed", o, tbl[517])


@pytest.mark.gpu
def test_sample_step(K, dev):
    NB, NSTEPS, PL = 1187, 64, 5
    bv = torch.randn(NB, generator=g(24)).to(dev)
    bi = torch.randint(0, V, (NB,), generator=g(25), dtype=torch.int32).to(dev)
    inp = (torch.arange(NSTEPS, dtype=torch.int32) + 100).to(dev)
    pl = torch.tensor([PL], device=dev, dtype=torch.int32)
    sam = torch.zeros(NSTEPS, device=dev, dtype=torch.int32)
    kern = K.sample_step(NB, NSTEPS)
    for pos, expect_prompt in [(2, True), (PL - 1, False), (20, False)]:
        ids = torch.zeros(1, device=dev, dtype=torch.int64)
        pt = torch.tensor([pos], device=dev, dtype=torch.int32)
        kern(bv, bi, inp, pl, ids, pt, sam)
        best = int(bi[int(bv.argmax())])
        want_next = int(inp[pos + 1]) if expect_prompt else best
        assert int(sam[pos]) == best and int(ids[0]) == want_next and int(pt[0]) == pos + 1
