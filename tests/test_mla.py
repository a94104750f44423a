"""MLA decode (absorbed, MiniCPM3-4B shapes) against the CPU oracle: each kernel
on its own, the attention core at several context lengths and splits, a
closed form at the full batch-8 / 8192-position size, and the whole attention
block against the non-absorbed reference order."""
import pytest
import torch

from oracle import minicpm3 as OM
from oracle.norms import rms_norm_q
from tests._check import assert_close, assert_equal, assert_l2, assert_ulps, bf16_ulps, rel_l2

BF = torch.bfloat16
CFG = OM.MLAConfig()
H, QA, KV, R = CFG.heads, CFG.q_lora, CFG.kv_lora, CFG.rope


def gen(seed):
    return torch.Generator().manual_seed(seed)


def oracle_weights(seed=3, std=0.05):
    return OM.random_weights(CFG, seed=seed, std=std)


@pytest.mark.gpu
def test_mla_prep(dev):
    from tilefoundry_amd._lib import C

    g = gen(1)
    B, ks, cap = 3, 2, 128
    part = torch.randn(ks, B, QA + KV + R, generator=g) * 0.5
    gq = (1 + 0.1 * torch.randn(QA, generator=g)).to(BF)
    gkv = (1 + 0.1 * torch.randn(KV, generator=g)).to(BF)
    cos, sin = OM.rope_tables(cap, CFG)
    pos = [0, 5, 127]
    lat = torch.zeros(B, cap, KV, dtype=BF, device=dev)
    rk = torch.zeros(B, cap, R, dtype=BF, device=dev)
    q_n = torch.empty(B, QA, dtype=BF, device=dev)
    err = torch.zeros(1, dtype=torch.int32, device=dev)
    C.mla_prep(part.to(dev), gq.to(dev), gkv.to(dev), 1e-6, cos.to(dev), sin.to(dev),
               torch.tensor(pos, dtype=torch.int32, device=dev), lat, rk, q_n, err)
    assert int(err.item()) == 0
    red = part.sum(0).to(BF)
    assert_ulps("q_n", q_n, rms_norm_q(red[:, :QA], gq, 1e-6), max_ulps=2)
    for b, p in enumerate(pos):
        assert_ulps(f"latent b={b}", lat[b, p], rms_norm_q(red[b, QA:QA + KV], gkv, 1e-6), max_ulps=2)
        assert_equal(f"rope key b={b}", rk[b, p], OM.rope32(red[b, QA + KV:], cos[p], sin[p]))
    # only the slots at pos were written
    mask = torch.ones(B, cap, dtype=torch.bool)
    for b, p in enumerate(pos):
        mask[b, p] = False
    assert not bool(lat.cpu()[mask].float().abs().sum()) and not bool(rk.cpu()[mask].float().abs().sum())


@pytest.mark.gpu
def test_mla_prep_position_error(dev):
    from tilefoundry_amd._lib import C

    B, cap = 2, 64
    lat = torch.zeros(B, cap, KV, dtype=BF, device=dev)
    rk = torch.zeros(B, cap, R, dtype=BF, device=dev)
    err = torch.zeros(1, dtype=torch.int32, device=dev)
    cos, sin = OM.rope_tables(cap, CFG)
    C.mla_prep(torch.ones(1, B, QA + KV + R, device=dev), torch.ones(QA, dtype=BF, device=dev),
               torch.ones(KV, dtype=BF, device=dev), 1e-6, cos.to(dev), sin.to(dev),
               torch.tensor([3, cap], dtype=torch.int32, device=dev), lat, rk,
               torch.empty(B, QA, dtype=BF, device=dev), err)
    assert int(err.item()) == 6
    assert float(lat[1].float().abs().sum()) == 0.0   # the out-of-range slot wrote nothing


@pytest.mark.gpu
@pytest.mark.parametrize("qa,n,p", [(QA, H * 96, 77), (QA, 999, 0), (1024, 16400, 127), (96, 40, 5)])
def test_mla_prep_q_gemv_equals_prep_then_gemv(dev, qa, n, p):
    """The one-sequence fusion of the prep into the q_b GEMV: q_part, the
    latent and the rope key are bit-equal to mla_prep followed by the f32 GEMV
    over its q_n, and q_part agrees with the oracle's norm and product."""
    from tilefoundry_amd._lib import C

    g = gen(7)
    cap = 128
    part = (torch.randn(qa + KV + R, generator=g) * 0.5).to(dev)
    gq = (1 + 0.1 * torch.randn(qa, generator=g)).to(BF).to(dev)
    gkv = (1 + 0.1 * torch.randn(KV, generator=g)).to(BF).to(dev)
    w = (torch.randn(n, qa, generator=g) * 0.05).to(BF).to(dev)
    cos, sin = (t.to(dev) for t in OM.rope_tables(cap, CFG))
    pos = torch.tensor([p], dtype=torch.int32, device=dev)
    outs = []
    for fused in (False, True):
        lat = torch.zeros(1, cap, KV, dtype=BF, device=dev)
        rk = torch.zeros(1, cap, R, dtype=BF, device=dev)
        q_part = torch.empty(n, dtype=torch.float32, device=dev)
        err = torch.zeros(1, dtype=torch.int32, device=dev)
        if fused:
            C.mla_prep_q_gemv(part, gq, gkv, 1e-6, cos, sin, pos, lat, rk, w, q_part, err)
        else:
            q_n = torch.empty(1, qa, dtype=BF, device=dev)
            C.mla_prep(part.view(1, 1, -1), gq, gkv, 1e-6, cos, sin, pos, lat, rk, q_n, err)
            C.gemv(q_n[0], w, q_part)
        assert int(err.item()) == 0
        outs.append((q_part, lat, rk))
    for name, a, b in zip(("q_part", "latent cache", "rope cache"), *outs):
        assert_equal(name, b, a)
    q_n = rms_norm_q(part[:qa].cpu().to(BF)[None], gq.cpu(), 1e-6)
    assert_close("q_part vs oracle", outs[1][0], q_n.float()[0] @ w.cpu().float().T)


@pytest.mark.gpu
def test_mla_prep_q_gemv_position_error(dev):
    """A position outside the cache sets err = 6 and writes no cache slot; the
    product is still written."""
    from tilefoundry_amd._lib import C

    cap = 64
    lat = torch.zeros(1, cap, KV, dtype=BF, device=dev)
    rk = torch.zeros(1, cap, R, dtype=BF, device=dev)
    err = torch.zeros(1, dtype=torch.int32, device=dev)
    q_part = torch.full((96,), float("nan"), device=dev)
    cos, sin = OM.rope_tables(cap, CFG)
    C.mla_prep_q_gemv(torch.ones(QA + KV + R, device=dev), torch.ones(QA, dtype=BF, device=dev),
                      torch.ones(KV, dtype=BF, device=dev), 1e-6, cos.to(dev), sin.to(dev),
                      torch.tensor([cap], dtype=torch.int32, device=dev), lat, rk,
                      torch.ones(96, QA, dtype=BF, device=dev), q_part, err)
    assert int(err.item()) == 6
    assert float(lat.float().abs().sum()) == 0.0 and float(rk.float().abs().sum()) == 0.0
    assert bool(torch.isfinite(q_part).all())


@pytest.mark.gpu
def test_mla_q_absorb(dev):
    from tilefoundry_amd._lib import C

    g = gen(2)
    B, ks = 4, 3
    w = oracle_weights()
    q_part = torch.randn(ks, B, H * (CFG.nope + R), generator=g) * 0.7
    cos, sin = OM.rope_tables(512, CFG)
    pos = [0, 1, 300, 511]
    q_abs = torch.empty(B, H, KV + R, dtype=BF, device=dev)
    C.mla_q_absorb(q_part.to(dev), w.w_kv_b.to(dev), cos.to(dev), sin.to(dev),
                   torch.tensor(pos, dtype=torch.int32, device=dev), q_abs, None)
    q_up = q_part.sum(0).to(BF).view(B, H, -1)
    for b, p in enumerate(pos):
        ref = OM.absorb_query(q_up[b], w, CFG, p, cos, sin)
        assert_ulps(f"q_lat b={b}", q_abs[b, :, :KV], ref[:, :KV], max_ulps=1, max_frac=0.02)
        assert_equal(f"q_rope b={b}", q_abs[b, :, KV:], ref[:, KV:])


def _qb_absorb(dev, q_n, w, pos, cos, sin, err=None):
    from tilefoundry_amd._lib import C

    heads = w.w_kv_b.shape[0] // (CFG.nope + CFG.v_dim)
    q_abs = torch.full((q_n.shape[0], heads, KV + R), float("nan"), dtype=BF, device=dev)
    C.mla_qb_absorb(q_n.to(dev), w.w_q_b.to(dev), w.w_kv_b.to(dev), cos.to(dev), sin.to(dev),
                    torch.tensor(pos, dtype=torch.int32, device=dev), q_abs, err)
    return q_abs.cpu()


@pytest.mark.gpu
@pytest.mark.parametrize("B", [1, 8, 13, 16, 17, 32])
def test_mla_qb_absorb_vs_oracle(dev, B):
    """The q_b projection and absorption in one launch against the oracle's
    q_up = bf16(q_n . W_q_b^T) and absorb_query, at batch 1 / 8 / 13 (a partial
    16-sequence tile) / 16 and 17 (either side of the one- and two-tile forms) /
    32 (two tiles). The projection's f32 sum runs in another
    order than torch's, so a q_up value whose exact sum lies within the f32
    error (8 u sum|p|, u = 2^-24) of a bf16 rounding boundary may land one ulp
    apart. Those values are found from the f64 sum; each output may differ from
    the oracle's by what they carry (one ulp of each times |W_UK| for q_lat,
    two ulps of a rotated pair for q_rope) plus two ulps of its own landing,
    and a rotated value whose inputs carry nothing must be equal."""
    g = gen(40 + B)
    w = oracle_weights()
    q_n = torch.randn(B, QA, generator=g).to(BF)
    cos, sin = OM.rope_tables(512, CFG)
    pos = [(37 * b + 5 * B) % 512 for b in range(B)]
    pos[-1] = 511
    _check_q_abs(_qb_absorb(dev, q_n, w, pos, cos, sin), q_n, w, pos, cos, sin)


def _check_q_abs(got, q_n, w, pos, cos, sin, cfg=CFG):
    B = q_n.shape[0]
    q_up = OM.proj(q_n, w.w_q_b).view(B, cfg.heads, -1)
    ref = torch.stack([OM.absorb_query(q_up[b], w, cfg, p, cos, sin) for b, p in enumerate(pos)])
    # q_up values whose landing the summation order can change
    exact = (q_n.double() @ w.w_q_b.double().t()).view(B, cfg.heads, -1)
    slack = 8 * 2.0 ** -24 * (q_n.double().abs() @ w.w_q_b.double().abs().t()).view(B, cfg.heads, -1)   # f32: <= 1.3x
    amb = ((exact - slack).to(BF) != (exact + slack).to(BF)).double()
    ulp = lambda x: torch.exp2(torch.floor(torch.log2(x.double().abs().clamp_min(1e-30))) - 7)
    q_ulp = amb * ulp(q_up)
    carry = torch.einsum("bhi,hic->bhc", q_ulp[..., :cfg.nope], w.w_uk(cfg).double().abs())
    # plus the f32 rounding of the 64-term absorbed sum itself, in either order
    accum = 64 * 2.0 ** -24 * torch.einsum("bhi,hic->bhc", q_up[..., :cfg.nope].double().abs(),
                                           w.w_uk(cfg).double().abs())
    err = (got[..., :KV].double() - ref[..., :KV].double()).abs()
    allowed = 2 * ulp(ref[..., :KV]) + 1.01 * carry + accum
    assert bool((err <= allowed).all()), f"q_lat: {int((err > allowed).sum())} elements past the bound"
    assert float((err > 0).double().mean()) <= 0.03
    # the rotation out_d = bf16(bf16(x_d c_d) + bf16(p_d s_d)), p_d = -x_{d+16} or x_{d-16}:
    # equal where neither input's landing is in doubt; elsewhere within what a one-ulp
    # input carries (through |c| or |s| and the product's own landing) plus two ulps
    half = cfg.rope // 2
    xr = q_up[..., cfg.nope:].double()
    pr = torch.cat((-xr[..., half:], xr[..., :half]), -1)
    ux = q_ulp[..., cfg.nope:]
    up = torch.cat((ux[..., half:], ux[..., :half]), -1)
    cs = torch.stack([cos[p].double() for p in pos])[:, None, :]
    sn = torch.stack([sin[p].double() for p in pos])[:, None, :]
    r_amb = (ux > 0) | (up > 0)
    d = bf16_ulps(got[..., KV:], ref[..., KV:])
    assert not bool((d[~r_amb] > 0).any()), "q_rope differs where its inputs land unambiguously"
    rerr = (got[..., KV:].double() - ref[..., KV:].double()).abs()
    rallow = (2 * ulp(ref[..., KV:]) + ux * cs.abs() + (ux > 0) * ulp(xr * cs) + up * sn.abs()
              + (up > 0) * ulp(pr * sn))
    assert bool((rerr <= 1.01 * rallow).all()), f"q_rope: {int((rerr > 1.01 * rallow).sum())} values past the bound"


@pytest.mark.gpu
@pytest.mark.parametrize("heads,B", [(17, 5), (48, 3), (1, 2)])
def test_mla_qb_absorb_other_head_counts(dev, heads, B):
    """The one-launch q_b + absorption for head counts other than MiniCPM3's 40
    (a partial last 16-head attention tile, the 48-head maximum, one head),
    against the oracle with the same rounding-boundary bound."""
    from dataclasses import replace

    cfg = replace(CFG, heads=heads)
    w = OM.random_weights(cfg, seed=heads, std=0.05)
    g = gen(60 + heads)
    q_n = torch.randn(B, QA, generator=g).to(BF)
    cos, sin = OM.rope_tables(256, cfg)
    pos = [(91 * b + heads) % 256 for b in range(B)]
    _check_q_abs(_qb_absorb(dev, q_n, w, pos, cos, sin), q_n, w, pos, cos, sin, cfg)


@pytest.mark.gpu
@pytest.mark.parametrize("B", [8, 20])
def test_mla_qb_absorb_repeatable(dev, B):
    """Thirty calls in a row, each after an MLA attention launch that leaves its
    own data in LDS, give bit-identical queries: every operand the kernel
    reads from LDS (W_UK included) has landed before it is read."""
    from tilefoundry_amd._lib import C

    g = gen(90 + B)
    w = oracle_weights()
    q_n = torch.randn(B, QA, generator=g).to(BF).to(dev)
    cos, sin = (t.to(dev) for t in OM.rope_tables(8192, CFG))
    posd = torch.full((B,), 8191, dtype=torch.int32, device=dev)
    wq, wk = w.w_q_b.to(dev), w.w_kv_b.to(dev)
    lat, rk = (t.to(dev) for t in OM.random_cache(B, 8192, CFG, seed=5))
    ns = 8192 // 256
    op = torch.empty(B, ns, H, KV, dtype=BF, device=dev)
    mp = torch.empty(B, ns, H, device=dev)
    lp = torch.empty(B, ns, H, device=dev)
    outs = []
    for _ in range(30):
        q_abs = torch.empty(B, H, KV + R, dtype=BF, device=dev)
        C.mla_qb_absorb(q_n, wq, wk, cos, sin, posd, q_abs, None)
        C.mla_attention(q_abs, lat, rk, posd, 256, CFG.scale, op, mp, lp, None)
        outs.append(q_abs)
    for i, o in enumerate(outs[1:], 1):
        assert_equal(f"call {i}", o, outs[0])


@pytest.mark.gpu
@pytest.mark.parametrize("p", [0, 77, 511])
def test_mla_prep_qb_absorb(dev, p):
    """One sequence's prep + q_b + absorption in one launch: the cache slots
    bit-equal to mla_prep_q_gemv's (the same norm order), no other slot
    written, and q_abs against the oracle from the oracle's LoRA-normed q_n."""
    from tilefoundry_amd._lib import C

    g = gen(300 + p)
    cap = 512
    w = oracle_weights()
    part = (torch.randn(QA + KV + R, generator=g) * 0.5).to(dev)
    gq = (1 + 0.1 * torch.randn(QA, generator=g)).to(BF).to(dev)
    gkv = (1 + 0.1 * torch.randn(KV, generator=g)).to(BF).to(dev)
    cos, sin = OM.rope_tables(cap, CFG)
    posd = torch.tensor([p], dtype=torch.int32, device=dev)
    caches = []
    for fused in (True, False):
        lat = torch.zeros(1, cap, KV, dtype=BF, device=dev)
        rk = torch.zeros(1, cap, R, dtype=BF, device=dev)
        err = torch.zeros(1, dtype=torch.int32, device=dev)
        if fused:
            q_abs = torch.full((1, H, KV + R), float("nan"), dtype=BF, device=dev)
            C.mla_prep_qb_absorb(part, gq, gkv, 1e-6, cos.to(dev), sin.to(dev), posd, lat, rk,
                                 w.w_q_b.to(dev), w.w_kv_b.to(dev), q_abs, err)
        else:
            C.mla_prep_q_gemv(part, gq, gkv, 1e-6, cos.to(dev), sin.to(dev), posd, lat, rk, w.w_q_b.to(dev),
                              torch.empty(H * 96, device=dev), err)
        assert int(err.item()) == 0
        caches.append((lat, rk))
    assert_equal("latent cache", caches[0][0], caches[1][0])
    assert_equal("rope cache", caches[0][1], caches[1][1])
    mask = torch.ones(cap, dtype=torch.bool)
    mask[p] = False
    assert float(caches[0][0][0].cpu()[mask].float().abs().sum()) == 0.0
    q_n = rms_norm_q(part[:QA].cpu().to(BF)[None], gq.cpu(), 1e-6)
    _check_q_abs(q_abs.cpu(), q_n, w, [p], cos, sin)


@pytest.mark.gpu
def test_mla_prep_qb_absorb_position_error(dev):
    """A position outside the cache sets err = 6 and writes no cache slot; the
    query is still written (finite)."""
    from tilefoundry_amd._lib import C

    cap = 64
    w = oracle_weights()
    lat = torch.zeros(1, cap, KV, dtype=BF, device=dev)
    rk = torch.zeros(1, cap, R, dtype=BF, device=dev)
    err = torch.zeros(1, dtype=torch.int32, device=dev)
    q_abs = torch.full((1, H, KV + R), float("nan"), dtype=BF, device=dev)
    cos, sin = OM.rope_tables(cap, CFG)
    C.mla_prep_qb_absorb(torch.ones(QA + KV + R, device=dev), torch.ones(QA, dtype=BF, device=dev),
                         torch.ones(KV, dtype=BF, device=dev), 1e-6, cos.to(dev), sin.to(dev),
                         torch.tensor([cap], dtype=torch.int32, device=dev), lat, rk, w.w_q_b.to(dev),
                         w.w_kv_b.to(dev), q_abs, err)
    assert int(err.item()) == 6
    assert float(lat.float().abs().sum()) == 0.0 and float(rk.float().abs().sum()) == 0.0
    assert bool(torch.isfinite(q_abs.float()).all())


@pytest.mark.gpu
def test_mla_qb_absorb_exact(dev):
    """Inputs on a grid where every sum is exact in f32 (q_n in {-2..2}, weights
    in {-2..2} / 16): any summation order gives the same f32 values, so the
    projection, its landing, the absorption and the rotation must match the
    oracle bit for bit; and a position past the rope table sets err = 6."""
    g = gen(77)
    B = 11
    w = oracle_weights()
    grid = lambda *s: (torch.randint(-2, 3, s, generator=g).float() / 16).to(BF)
    w.w_q_b, w.w_kv_b = grid(*w.w_q_b.shape), grid(*w.w_kv_b.shape)
    q_n = torch.randint(-2, 3, (B, QA), generator=g).float().to(BF)
    cos, sin = OM.rope_tables(256, CFG)
    pos = list(range(0, 23 * B, 23))
    got = _qb_absorb(dev, q_n, w, pos, cos, sin)
    q_up = OM.proj(q_n, w.w_q_b).view(B, H, -1)
    for b, p in enumerate(pos):
        assert_equal(f"q_abs b={b}", got[b], OM.absorb_query(q_up[b], w, CFG, p, cos, sin))
    err = torch.zeros(1, dtype=torch.int32, device=dev)
    got = _qb_absorb(dev, q_n[:2], w, [3, 256], cos, sin, err)
    assert int(err.item()) == 6
    assert_equal("q_abs, good position", got[0], OM.absorb_query(q_up[0], w, CFG, 3, cos, sin))
    assert bool(torch.isfinite(got[1].float()).all())


def _attend(dev, q_abs, lat, rk, pos, split, w_kv_b, cap):
    from tilefoundry_amd._lib import C

    B = q_abs.shape[0]
    ns = cap // split
    op = torch.empty(B, ns, H, KV, dtype=BF, device=dev)
    mp = torch.empty(B, ns, H, device=dev)
    lp = torch.empty(B, ns, H, device=dev)
    attn = torch.empty(B, H * CFG.v_dim, dtype=BF, device=dev)
    err = torch.zeros(1, dtype=torch.int32, device=dev)
    posd = torch.tensor(pos, dtype=torch.int32, device=dev)
    C.mla_attention(q_abs.to(dev), lat.to(dev), rk.to(dev), posd, split, CFG.scale, op, mp, lp, err)
    C.mla_combine_up(op, mp, lp, posd, split, w_kv_b.to(dev), attn)
    assert int(err.item()) == 0
    return attn.cpu()


@pytest.mark.gpu
@pytest.mark.parametrize("split,pos", [(256, [0, 63, 700]), (128, [128, 1, 1023]), (1024, [500, 1023, 2]),
                                       (32, [0, 31, 700]), (64, [64, 1, 1023]), (96, [95, 96, 500])])
def test_mla_attention_vs_oracle(dev, split, pos):
    g = gen(sum(pos) + split)
    B, cap = 3, 1024 // split * split
    w = oracle_weights()
    lat, rk = OM.random_cache(B, cap, CFG, seed=split)
    q_abs = torch.randn(B, H, KV + R, generator=g).to(BF)
    got = _attend(dev, q_abs, lat, rk, pos, split, w.w_kv_b, cap)
    for b, p in enumerate(pos):
        ref = OM.attend_absorbed(q_abs[b], lat[b, :p + 1], rk[b, :p + 1], w, CFG, p_bf16=True)
        assert_close(f"attn b={b} pos={p}", got[b], ref)
        assert rel_l2(got[b], ref) < 4e-3


@pytest.mark.gpu
@pytest.mark.parametrize("heads,split", [(1, 128), (8, 128), (17, 128), (48, 128), (17, 32), (48, 64)])
def test_mla_attention_split_outputs_other_head_counts(dev, heads, split):
    """The split outputs (op normalised by the split's own sum, natural-log max,
    sum) merged over the live splits equal the oracle's latent sum, for head
    counts that leave whole or partial 16-head tiles empty and contexts that end
    inside a 128-position step."""
    from dataclasses import replace

    from tilefoundry_amd._lib import C

    cfg = replace(CFG, heads=heads)
    B, cap = 2, 512
    pos = [129, 511]
    lat, rk = OM.random_cache(B, cap, cfg, seed=heads)
    g = gen(heads)
    q_abs = torch.randn(B, heads, KV + R, generator=g).to(BF)
    ns = cap // split
    op = torch.empty(B, ns, heads, KV, dtype=BF, device=dev)
    mp = torch.empty(B, ns, heads, device=dev)
    lp = torch.empty(B, ns, heads, device=dev)
    err = torch.zeros(1, dtype=torch.int32, device=dev)
    C.mla_attention(q_abs.to(dev), lat.to(dev), rk.to(dev), torch.tensor(pos, dtype=torch.int32, device=dev),
                    split, cfg.scale, op, mp, lp, err)
    assert int(err.item()) == 0
    w = OM.random_weights(cfg, seed=1)
    for b, p in enumerate(pos):
        live = p // split + 1
        o, m, l = op[b, :live].float().cpu(), mp[b, :live].cpu(), lp[b, :live].cpu()
        wgt = l * torch.exp(m - m.amax(0, keepdim=True))                   # [live, heads]
        got = (o * wgt[..., None]).sum(0) / wgt.sum(0)[:, None]
        _, ref = OM.attend_absorbed(q_abs[b], lat[b, :p + 1], rk[b, :p + 1], w, cfg, p_bf16=True,
                                    return_latent=True)
        assert_close(f"o_lat heads={heads} b={b} pos={p}", got, ref)


@pytest.mark.gpu
def test_mla_attention_stale_slots_ignored(dev):
    """Slots past the context hold NaN: nothing of them reaches the output."""
    g = gen(9)
    B, cap, split = 2, 512, 256
    w = oracle_weights()
    lat, rk = OM.random_cache(B, cap, CFG, seed=9)
    lat[:, 300:] = float("nan")
    rk[:, 300:] = float("nan")
    q_abs = torch.randn(B, H, KV + R, generator=g).to(BF)
    pos = [299, 10]
    got = _attend(dev, q_abs, lat, rk, pos, split, w.w_kv_b, cap)
    assert not bool(torch.isnan(got.float()).any())
    for b, p in enumerate(pos):
        ref = OM.attend_absorbed(q_abs[b], lat[b, :p + 1], rk[b, :p + 1], w, CFG, p_bf16=True)
        assert_close(f"attn b={b}", got[b], ref)


@pytest.mark.gpu
def test_mla_attention_full_size_identical_rows(dev):
    """Batch 8 x 8192 positions, every cached entry equal: each weight is
    exactly 1 / n whatever the query, so head h returns bf16(W_UV_h c)."""
    g = gen(10)
    B, cap, split = 8, 8192, 256
    w = oracle_weights()
    c = torch.randn(KV, generator=g).to(BF)
    r = torch.randn(R, generator=g).to(BF)
    lat = c.view(1, 1, KV).expand(B, cap, KV).contiguous()
    rk = r.view(1, 1, R).expand(B, cap, R).contiguous()
    q_abs = torch.randn(B, H, KV + R, generator=g).to(BF)
    pos = [8191, 4095, 0, 256, 255, 8000, 1, 7777]
    got = _attend(dev, q_abs, lat, rk, pos, split, w.w_kv_b, cap).view(B, H, -1)
    exp = torch.einsum("hvc,c->hv", w.w_uv(CFG).double(), c.double()).to(BF)
    for b in range(B):
        assert_ulps(f"b={b}", got[b], exp, max_ulps=1)


@pytest.mark.gpu
def test_mla_attention_full_size_one_sequence(dev):
    """The config's own size (8 sequences x 8192 positions) with random data;
    two sequences checked against the oracle in full."""
    g = gen(11)
    B, cap, split = 8, 8192, 256
    w = oracle_weights()
    lat, rk = OM.random_cache(B, cap, CFG, seed=11)
    q_abs = torch.randn(B, H, KV + R, generator=g).to(BF)
    pos = [8191] * B
    pos[5] = 5000
    got = _attend(dev, q_abs, lat, rk, pos, split, w.w_kv_b, cap)
    for b in (0, 5):
        ref = OM.attend_absorbed(q_abs[b], lat[b, :pos[b] + 1], rk[b, :pos[b] + 1], w, CFG, p_bf16=True)
        assert_close(f"attn b={b}", got[b], ref)


@pytest.mark.gpu
def test_rows_residual(dev):
    from tilefoundry_amd._lib import C

    g = gen(12)
    part = torch.randn(5, 8, 2560, generator=g)
    res = torch.randn(8, 2560, generator=g).to(BF)
    out = torch.empty(8, 2560, dtype=BF, device=dev)
    alpha = float(torch.tensor(0.1778).to(BF))
    C.rows_residual(part.to(dev), res.to(dev), alpha, out)
    ref = res + part.sum(0).to(BF) * torch.tensor(alpha).to(BF)
    assert_equal("rows_residual", out, ref)


@pytest.mark.gpu
@pytest.mark.parametrize("B,cap,pos,fuse_qb", [
    (2, 512, [100, 511], True),
    (2, 512, [100, 511], False),
    (8, 8192, [8191, 0, 4095, 8191, 17, 6000, 8190, 1234], True),   # the benchmark's shape
])
def test_mla_block_vs_reference(dev, B, cap, pos, fuse_qb):
    """The whole attention block (norm, projections, cache append, absorbed
    attention, o_proj, scaled residual) against the non-absorbed reference
    order, with each sequence at its own position: at batch 2 over 512 slots
    with the q_b projection and the absorption in one launch or as two, and at
    the benchmark's batch 8 over 8192 slots (first, middle and last slots)."""
    from tilefoundry_amd.minicpm3 import MLABlock, MiniCPM3Config, synthetic_weights

    cfg = MiniCPM3Config()
    wts = synthetic_weights(cfg, seed=7)
    blk = MLABlock(cfg, batch=B, cap=cap, device=dev, weights=wts, fuse_qb=fuse_qb)
    ow = OM.MLAWeights(**wts)
    lat, rk = OM.random_cache(B, cap, CFG, seed=13)
    blk.latent.copy_(lat.to(dev))
    blk.rope_k.copy_(rk.to(dev))
    hidden = torch.randn(B, cfg.hidden, generator=gen(14)).to(BF)
    out = blk.step(hidden.to(dev), pos).cpu()
    attn = blk.attn.cpu()
    cos, sin = OM.rope_tables(cap, CFG)
    for b, p in enumerate(pos):
        pr = OM.project(hidden[b], ow, CFG, p, cos, sin)
        assert_ulps(f"latent b={b}", blk.latent[b, p], pr.latent, max_ulps=2)
        assert_ulps(f"rope key b={b}", blk.rope_k[b, p], pr.k_rope, max_ulps=1)
        lat_ctx = torch.cat((lat[b, :p], pr.latent.view(1, -1)))
        rk_ctx = torch.cat((rk[b, :p], pr.k_rope.view(1, -1)))
        ref = OM.attend_reference(pr.q_up, lat_ctx, rk_ctx, ow, CFG, p, cos, sin)
        absd = OM.attend_absorbed(OM.absorb_query(pr.q_up, ow, CFG, p, cos, sin), lat_ctx, rk_ctx, ow, CFG,
                                  p_bf16=True)
        assert_l2(f"attn vs reference b={b}", attn[b], ref)
        assert_close(f"attn vs absorbed oracle b={b}", attn[b], absd)
        o_ref = OM.o_proj_residual(ref, ow.w_o, hidden[b], cfg.residual_scale)
        assert_close(f"block out b={b}", out[b], o_ref)
        # the o_proj branch itself (the residual sum's bf16 landing would hide it)
        branch = blk.part_o.sum(0)[b].cpu()
        assert_l2(f"o_proj b={b}", branch, ref.float() @ ow.w_o.float().t())
