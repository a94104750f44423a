"""Pins for the CPU oracle (no GPU): each check is independent of the formula it
checks -- closed forms, special cases, f64 brute force, exact integer cases and
planted mistakes -- so that a wrong rounding point, sign, index or operand in the
oracle fails one of them."""
import math

import pytest
import torch

from oracle import norms as ON
from oracle import qwen3 as OQ
from tests._check import bf16_ulps

BF = torch.bfloat16


def g(seed):
    return torch.Generator().manual_seed(seed)


# ---------------------------------------------------------------- norms
def test_rms_norm_constant_row_closed_form():
    """A row of one value c normalises to sign(c): y == sign(c) * gamma exactly."""
    H = 2048
    gamma = torch.linspace(-3, 3, H).to(BF)
    for c in (0.5, -3.0, 7.25, -0.125, 100.0):
        x = torch.full((H,), c).to(BF)
        y = ON.rms_norm_q(x, gamma, 1e-6)
        assert torch.equal(y, (math.copysign(1.0, c) * gamma.float()).to(BF))


def test_rms_norm_matches_f64_within_one_rounding():
    x = torch.randn(64, 2048, generator=g(0)).to(BF)
    gamma = (1 + 0.1 * torch.randn(2048, generator=g(1))).to(BF)
    x64 = x.double()
    n64 = x64 * torch.rsqrt(x64.pow(2).mean(-1, keepdim=True) + 1e-6)
    ref = (n64.to(BF).double() * gamma.double()).to(BF)
    assert int(bf16_ulps(ON.rms_norm_q(x, gamma, 1e-6), ref).max()) <= 1


def test_rms_norm_landing_before_gamma_matters():
    """Planted mistake: scaling in f32 before the bf16 landing gives a different
    answer on random rows -- so the oracle's order is actually exercised."""
    x = torch.randn(64, 2048, generator=g(2)).to(BF)
    gamma = (1 + 0.1 * torch.randn(2048, generator=g(3))).to(BF)
    x32 = x.float()
    wrong = (x32 * torch.rsqrt(x32.pow(2).mean(-1, keepdim=True) + 1e-6) * gamma.float()).to(BF)
    assert not torch.equal(ON.rms_norm_q(x, gamma, 1e-6), wrong)


def test_rms_norm_one_plus_gamma():
    """Qwen3.5 form: gamma = 0 is the plain normalisation, in one landing."""
    x = torch.randn(8, 5120, generator=g(4)).to(BF)
    zero = torch.zeros(5120).to(BF)
    x64 = x.double()
    ref = (x64 * torch.rsqrt(x64.pow(2).mean(-1, keepdim=True) + 1e-6)).to(BF)
    assert int(bf16_ulps(ON.rms_norm_1p(x, zero, 1e-6), ref).max()) <= 1


def test_add_rms_norm_residual_is_the_landed_sum():
    x = torch.randn(4, 256, generator=g(5)).to(BF)
    r = torch.randn(4, 256, generator=g(6)).to(BF)
    gamma = torch.ones(256).to(BF)
    y, ro = ON.add_rms_norm(x, r, gamma, 1e-6)
    assert torch.equal(ro, (x.double() + r.double()).to(BF))
    assert torch.equal(y, ON.rms_norm_q(ro, gamma, 1e-6))


def _resid_rms_norm_f64(a, partials, gamma, eps):
    """The residual norm stated in f64: the split-K partials' sum lands once in
    bf16, the residual add lands again, and the Qwen3 norm of the landed sum."""
    h = (a.double() + partials.double().sum(0).to(BF).double()).to(BF)
    h64 = h.double()
    n = (h64 * torch.rsqrt(h64.pow(2).mean(-1, keepdim=True) + eps)).to(BF)
    return h, (n.double() * gamma.double()).to(BF)


def test_resid_rms_norm_matches_f64_within_one_rounding():
    """``resid_rms_norm`` against its f64 statement on random rows and 1-8
    split-K partials: the residual and the normed row within one bf16 ulp."""
    gen = g(60)
    for ks in (1, 4, 8):
        a = torch.randn(16, 2048, generator=gen).to(BF)
        p = torch.randn(ks, 16, 2048, generator=gen)
        gamma = (1 + 0.1 * torch.randn(2048, generator=gen)).to(BF)
        h, xn = ON.resid_rms_norm(a, p, gamma, 1e-6)
        h64, xn64 = _resid_rms_norm_f64(a, p, gamma, 1e-6)
        assert int(bf16_ulps(h, h64).max()) <= 1, ks
        assert int(bf16_ulps(xn, xn64).max()) <= 1, ks


def test_resid_rms_norm_exact_on_integer_partials():
    """Integer partials and residuals small enough that every sum is exact in
    f32 and bf16: the residual is the integer sum, and a row built to sum to
    one constant c normalises to sign(c) * gamma exactly."""
    gen = g(61)
    a = torch.randint(-64, 65, (8, 512), generator=gen).to(BF)
    p = torch.randint(-16, 17, (4, 8, 512), generator=gen).float()
    gamma = (1 + 0.1 * torch.randn(512, generator=gen)).to(BF)
    h, _ = ON.resid_rms_norm(a, p, gamma, 1e-6)
    want = a.to(torch.int64) + p.to(torch.int64).sum(0)
    assert torch.equal(h.to(torch.int64), want)
    for c in (3.0, -20.0, 0.5):
        a_c = (c - p.sum(0)).to(BF)          # exact: |c - sum| <= 84
        h, xn = ON.resid_rms_norm(a_c, p, gamma, 1e-6)
        assert torch.equal(h, torch.full_like(h, c))
        assert torch.equal(xn, (math.copysign(1.0, c) * gamma.float()).to(BF).expand_as(xn))


def _landing_kat(resid):
    """Two hand-worked cases that separate the two bf16 landings of
    ``bf16(a + bf16(sum_s P[s]))`` (bf16 keeps 8 significant bits: the spacing
    at 1.0 is 2^-7, and a tie rounds to even):

    * a = 0, P = [1 + 2^-8, 2^-8]: the f32 sum is 1 + 2^-7 exactly, so h = 1 + 2^-7.
      Landing each partial first gives bf16(1 + 2^-8) + 2^-8 = 1 + 2^-8, a tie -> 1.0.
    * a = 1, P = [2^-8 + 2^-20]: the sum lands as 2^-8; 1 + 2^-8 is a tie -> h = 1.0.
      One landing of a + sum (1 + 2^-8 + 2^-20, above the tie) gives 1 + 2^-7.

    Returns True when ``resid(a, partials)`` gives both expected residuals."""
    H = 64
    one = torch.ones(1, H)
    case1 = resid(torch.zeros(1, H).to(BF), torch.stack([(1 + 2 ** -8) * one, 2 ** -8 * one]))
    case2 = resid(one.to(BF), ((2 ** -8 + 2 ** -20) * one)[None])
    return (torch.equal(case1, torch.full((1, H), 1 + 2 ** -7).to(BF))
            and torch.equal(case2, torch.ones(1, H).to(BF)))


def test_resid_rms_norm_landings_known_answers():
    gamma = torch.ones(64).to(BF)
    assert _landing_kat(lambda a, p: ON.resid_rms_norm(a, p, gamma, 1e-6)[0])


@pytest.mark.parametrize("plant", ["partials_landed_first", "single_landing"])
def test_resid_rms_norm_planted_landing_mistakes_fail(plant):
    """Planted mistakes in the residual's rounding points fail the known answers."""
    if plant == "partials_landed_first":     # bf16(P[s]) summed, instead of bf16(sum P[s])
        wrong = lambda a, p: a + p.to(BF).float().sum(0).to(BF)  # noqa: E731
    else:                                    # bf16(a + sum P[s]) in one landing
        wrong = lambda a, p: (a.float() + p.float().sum(0)).to(BF)  # noqa: E731
    assert not _landing_kat(wrong)


# ---------------------------------------------------------------- rope
def test_rope_position_zero_is_identity():
    cos, sin = OQ.rope_tables(8, 128, 1.0e6)
    x = torch.randn(16, 128, generator=g(7)).to(BF)
    assert torch.equal(OQ.rope(x, cos[0], sin[0]), x)


def test_rope_is_complex_rotation():
    """rotate-half on pairs (x_d, x_{d+64}) is multiplication by e^{i theta_d p}."""
    D, p, theta = 128, 37, 1.0e6
    x = torch.randn(4, D, generator=g(8)).to(BF)
    cos, sin = OQ.rope_tables(p + 1, D, theta)
    got = OQ.rope(x, cos[p], sin[p]).double()
    z = torch.complex(x[:, :64].double(), x[:, 64:].double())
    ang = torch.complex(cos[p, :64].double(), sin[p, :64].double())  # the table's own (landed) angles
    w = z * ang
    ref = torch.cat([w.real, w.imag], -1)
    assert float((got - ref).abs().max()) <= float(ref.abs().max()) * 2 ** -8


def test_rope_tables_against_closed_form():
    cos, sin = OQ.rope_tables(100, 128, 1.0e6)
    d = torch.arange(64, dtype=torch.float64)
    ang = 99 * (1.0e6 ** (-(2 * d) / 128))
    assert int(bf16_ulps(cos[99, :64], torch.cos(ang).to(BF)).max()) <= 1
    assert int(bf16_ulps(sin[99, 64:], torch.sin(ang).to(BF)).max()) <= 1


# ---------------------------------------------------------------- attention
def test_attend_one_key_returns_value():
    q = torch.randn(16, 128, generator=g(9)).to(BF)
    k = torch.randn(1, 8, 128, generator=g(10)).to(BF)
    v = torch.randn(1, 8, 128, generator=g(11)).to(BF)
    for pb in (False, True):
        out = OQ.attend(q, k, v, 128 ** -0.5, p_bf16=pb)
        assert torch.equal(out, v[0].repeat_interleave(2, 0).reshape(-1))


def test_attend_identical_keys_give_mean_value():
    n = 33
    q = torch.randn(16, 128, generator=g(12)).to(BF)
    k = torch.randn(1, 8, 128, generator=g(13)).to(BF).expand(n, 8, 128).contiguous()
    v = torch.randn(n, 8, 128, generator=g(14)).to(BF)
    ref = v.double().mean(0).repeat_interleave(2, 0).reshape(-1).to(BF)
    assert int(bf16_ulps(OQ.attend(q, k, v, 128 ** -0.5), ref).max()) <= 1


def test_attend_matches_f64_brute_force():
    n = 7
    q = torch.randn(4, 128, generator=g(15)).to(BF)
    k = torch.randn(n, 2, 128, generator=g(16)).to(BF)
    v = torch.randn(n, 2, 128, generator=g(17)).to(BF)
    out = OQ.attend(q, k, v, 0.1).double().view(4, 128)
    for h in range(4):
        kv = h // 2
        s = [0.1 * sum(float(q[h, d]) * float(k[j, kv, d]) for d in range(128)) for j in range(n)]
        m = max(s)
        e = [math.exp(x - m) for x in s]
        ref = [sum(e[j] * float(v[j, kv, d]) for j in range(n)) / sum(e) for d in range(128)]
        ref = torch.tensor(ref, dtype=torch.float64)
        assert float((out[h] - ref).abs().max()) <= float(ref.abs().max()) * 2 ** -7


def test_attend_gqa_mapping_planted_mistake():
    """Query head h reads kv head h // G (repeat_interleave), not h % HKV."""
    q = torch.zeros(4, 128).to(BF)
    k = torch.zeros(3, 2, 128).to(BF)
    v = torch.zeros(3, 2, 128).to(BF)
    v[:, 0] = 1.0
    v[:, 1] = 2.0
    out = OQ.attend(q, k, v, 1.0).view(4, 128)
    assert out[:, 0].tolist() == [1.0, 1.0, 2.0, 2.0]


def test_attend_p_bf16_close_to_f32():
    q = torch.randn(16, 128, generator=g(18)).to(BF)
    k = torch.randn(300, 8, 128, generator=g(19)).to(BF)
    v = torch.randn(300, 8, 128, generator=g(20)).to(BF)
    a = OQ.attend(q, k, v, 128 ** -0.5).float()
    b = OQ.attend(q, k, v, 128 ** -0.5, p_bf16=True).float()
    assert float((a - b).abs().max()) <= 1e-2 * float(a.abs().max())


# ---------------------------------------------------------------- projections / argmax
def test_proj_exact_on_integers():
    x = torch.randint(-4, 5, (512,), generator=g(21)).to(BF)
    w = torch.randint(-4, 5, (64, 512), generator=g(22)).to(BF)
    ref = (x.long() @ w.long().t())
    got = OQ.proj(x, w)
    assert torch.equal(got.float(), ref.float().to(BF).float())


def test_greedy_lowest_index_on_ties():
    logits = torch.tensor([0.5, 3.0, -1.0, 3.0, 3.0])
    assert OQ.greedy(logits) == 1


# ---------------------------------------------------------------- the step
def _tiny():
    cfg = OQ.Qwen3Config(hidden=256, heads=4, kv_heads=2, head_dim=128, inter=512, vocab=300, layers=2)
    return cfg, OQ.random_model(cfg, seed=3)


def test_decode_cache_equals_recompute():
    """Decoding with the appended cache equals re-running every prefix from
    scratch (the cache holds exactly the per-position keys and values)."""
    cfg, model = _tiny()
    ids = [5, 17, 250, 3, 99]
    cos, sin = OQ.rope_tables(8, cfg.head_dim, cfg.rope_theta)
    caches = OQ.empty_caches(cfg, cfg.layers)
    for p, t in enumerate(ids):
        inc = OQ.step(model, cfg, t, p, caches, cos, sin)
    fresh = OQ.empty_caches(cfg, cfg.layers)
    for p, t in enumerate(ids):
        again = OQ.step(model, cfg, t, p, fresh, cos, sin)
    assert torch.equal(inc, again)
    assert all(c[0].shape[0] == len(ids) for c in caches)


def test_decode_causal_prefix():
    """A later token does not change an earlier step's logits."""
    cfg, model = _tiny()
    cos, sin = OQ.rope_tables(8, cfg.head_dim, cfg.rope_theta)
    a, b = OQ.empty_caches(cfg, 2), OQ.empty_caches(cfg, 2)
    la = [OQ.step(model, cfg, t, p, a, cos, sin) for p, t in enumerate([7, 8, 9])]
    lb = [OQ.step(model, cfg, t, p, b, cos, sin) for p, t in enumerate([7, 8, 200])]
    assert torch.equal(la[0], lb[0]) and torch.equal(la[1], lb[1])
    assert not torch.equal(la[2], lb[2])


def test_teacher_forcing_reproduces_free_run():
    cfg, model = _tiny()
    free = OQ.decode(model, cfg, [1, 2, 3], 6)
    forced = OQ.decode(model, cfg, [1, 2, 3], 6, teacher=free)
    assert free == forced


def test_step_batch_equals_per_sequence_steps():
    """The batched step (the CPU baseline's bs=32 sample) is the single-sequence
    step row by row: three sequences at different positions, stepped together,
    give each one's own logits and cache rows (the [B, in] matmul may sum in
    another order, so within one bf16 landing)."""
    cfg, model = _tiny()
    cos, sin = OQ.rope_tables(8, cfg.head_dim, cfg.rope_theta)
    seqs = [[5, 17, 250], [3, 99, 1], [42, 7, 8]]
    caches_b = [OQ.empty_caches(cfg, cfg.layers) for _ in seqs]
    singles = [OQ.empty_caches(cfg, cfg.layers) for _ in seqs]
    for p in range(3):
        batch = OQ.step_batch(model, cfg, [s[p] for s in seqs], [p] * 3, caches_b, cos, sin)
        for b, s in enumerate(seqs):
            one = OQ.step(model, cfg, s[p], p, singles[b], cos, sin)
            assert float((batch[b] - one).norm() / one.norm()) < 2e-3
    for b in range(3):
        for li in range(cfg.layers):
            for j in range(2):
                assert int(bf16_ulps(caches_b[b][li][j], singles[b][li][j]).max()) <= 1


# ---------------------------------------------------------------- synthetic weights
def test_synthetic_generator_golden_values():
    """The cross-device generator's first values, pinned (any change to the
    mixing or the transform changes every weight of every test)."""
    from tilefoundry_amd.synthetic import normal

    v = normal((6,), seed=0, stream=3, std=1.0, dtype=torch.float32).tolist()
    want = [0.30610647797584534, -0.6969932913780212, 0.1560002863407135,
            -0.5078309774398804, 0.13809585571289062, -1.1312625408172607]
    assert v == pytest.approx(want, rel=0, abs=1e-7)


def test_synthetic_generator_statistics():
    from tilefoundry_amd.synthetic import normal

    x = normal((1 << 20,), seed=1, stream=0, std=0.02, dtype=torch.float32).double()
    assert abs(float(x.mean())) < 1e-4
    assert abs(float(x.std()) - 0.02) < 1e-4
    assert not torch.equal(normal((64,), 1, 0), normal((64,), 1, 1))
    assert torch.equal(normal((64,), 1, 0), normal((64,), 1, 0))


# ---------------------------------------------------------------- MLA (MiniCPM3)
def _mla_small():
    from oracle import minicpm3 as OM

    cfg = OM.MLAConfig(hidden=64, heads=4, q_lora=32, kv_lora=32, nope=16, rope=8, v_dim=16)
    return OM, cfg, OM.random_weights(cfg, seed=4, std=0.25)


def test_mla_rope_tables_against_closed_form():
    from oracle import minicpm3 as OM

    cfg = OM.MLAConfig()
    cos, sin = OM.rope_tables(5000, cfg)
    i = torch.arange(16, dtype=torch.float64)
    inv = 1.0 / (torch.tensor(OM.SHORT_FACTOR, dtype=torch.float64) * 10000.0 ** (2 * i / 32))
    for p in (0, 1, 77, 4999):
        assert int(bf16_ulps(cos[p, :16], torch.cos(p * inv).to(BF)).max()) <= 1
        assert int(bf16_ulps(sin[p, 16:], torch.sin(p * inv).to(BF)).max()) <= 1


def test_mla_rope_identity_and_rotation():
    from oracle import minicpm3 as OM

    cos, sin = OM.rope_tables(64, OM.MLAConfig())
    x = torch.randn(40, 32, generator=g(30)).to(BF)
    assert torch.equal(OM.rope32(x, cos[0], sin[0]), x)
    p = 41
    got = OM.rope32(x, cos[p], sin[p]).double()
    z = torch.complex(x[:, :16].double(), x[:, 16:].double()) * torch.complex(cos[p, :16].double(), sin[p, :16].double())
    ref = torch.cat([z.real, z.imag], -1)
    assert float((got - ref).abs().max()) <= float(ref.abs().max()) * 2 ** -7


def test_mla_absorbed_equals_reference_attention():
    """The absorption identity: scoring the latent with W_UK^T q_nope and
    up-projecting the weighted latent with W_UV equals attending the assembled
    per-head keys / values (to the bf16 bar; they round at different points)."""
    from tests._check import rel_l2

    OM, cfg, w = _mla_small()
    n, pos = 37, 36
    cos, sin = OM.rope_tables(n, cfg)
    lat, rk = OM.random_cache(1, n, cfg, seed=5)
    q_up = torch.randn(cfg.heads, cfg.qk_dim, generator=g(31)).to(BF)
    ref = OM.attend_reference(q_up, lat[0], rk[0], w, cfg, pos, cos, sin)
    q_abs = OM.absorb_query(q_up, w, cfg, pos, cos, sin)
    for pb in (False, True):
        got = OM.attend_absorbed(q_abs, lat[0], rk[0], w, cfg, p_bf16=pb)
        assert rel_l2(got, ref) < 1e-2
    # planted mistake: absorbing with the value half of W_kv_b breaks the identity
    bad = OM.MLAWeights(**{**w.__dict__, "w_kv_b": w.w_kv_b.view(cfg.heads, 2, 16, cfg.kv_lora).flip(1).reshape(-1, cfg.kv_lora)})
    wrong = OM.attend_absorbed(OM.absorb_query(q_up, bad, cfg, pos, cos, sin), lat[0], rk[0], w, cfg)
    assert rel_l2(wrong, ref) > 0.1


def test_mla_one_position_returns_projected_latent():
    """One position: the softmax weight is 1, so head h's output is W_UV_h c_0."""
    OM, cfg, w = _mla_small()
    cos, sin = OM.rope_tables(4, cfg)
    lat, rk = OM.random_cache(1, 1, cfg, seed=6)
    q_up = torch.randn(cfg.heads, cfg.qk_dim, generator=g(32)).to(BF)
    got = OM.attend_absorbed(OM.absorb_query(q_up, w, cfg, 0, cos, sin), lat[0], rk[0], w, cfg).view(cfg.heads, -1)
    c0 = lat[0, 0].double()
    for h in range(cfg.heads):
        exp = torch.stack([sum(c0[c] * float(w.w_kv_b[h * 32 + 16 + v, c]) for c in range(cfg.kv_lora)) for v in range(16)])
        assert int(bf16_ulps(got[h], exp.to(BF)).max()) <= 1


def test_mla_absorbed_f64_brute_force():
    import math

    OM, cfg, w = _mla_small()
    n = 6
    lat, rk = OM.random_cache(1, n, cfg, seed=7)
    q_abs = torch.randn(cfg.heads, cfg.kv_lora + cfg.rope, generator=g(33)).to(BF)
    got = OM.attend_absorbed(q_abs, lat[0], rk[0], w, cfg).double().view(cfg.heads, -1)
    kc = torch.cat((lat[0], rk[0]), -1)
    for h in range(cfg.heads):
        s = [cfg.scale * sum(float(q_abs[h, d]) * float(kc[j, d]) for d in range(kc.shape[1])) for j in range(n)]
        mx = max(s)
        e = [math.exp(x - mx) for x in s]
        o = [sum(e[j] * float(lat[0, j, c]) for j in range(n)) / sum(e) for c in range(cfg.kv_lora)]
        ref = [sum(o[c] * float(w.w_kv_b[h * 32 + 16 + v, c]) for c in range(cfg.kv_lora)) for v in range(16)]
        ref = torch.tensor(ref, dtype=torch.float64)
        assert float((got[h] - ref).abs().max()) <= float(ref.abs().max()) * 2 ** -7


def _rope_attend_case(n_ctx, seed=40):
    """A small MLA shape, a latent cache of n_ctx + 1 rows expanded to the
    assembled per-head cache; the last row is this token's own."""
    OM, cfg, w = _mla_small()
    pos = n_ctx
    cos, sin = OM.rope_tables(n_ctx + 2, cfg)
    lat, rk_raw = OM.random_cache(1, n_ctx + 1, cfg, seed=seed)
    # rows 0..n_ctx-1 of the rope cache hold rotated keys; the token brings its raw slice
    rk = torch.stack([OM.rope32(rk_raw[0, j], cos[j], sin[j]) for j in range(n_ctx + 1)])
    k_all, v_all = OM.assembled_cache(lat[0], rk, w, cfg)
    q_up = torch.randn(cfg.heads, cfg.qk_dim, generator=g(seed + 1)).to(BF)
    kv_up = torch.cat((k_all[n_ctx, :, : cfg.nope], v_all[n_ctx]), -1).contiguous()
    scale = torch.tensor(cfg.scale).to(BF)
    args = (q_up.reshape(-1), kv_up.reshape(-1), rk_raw[0, n_ctx], cos, sin, pos,
            k_all[:n_ctx], v_all[:n_ctx], n_ctx, scale, cfg.heads, cfg.nope, cfg.rope, cfg.v_dim)
    return OM, cfg, w, args, (q_up, lat[0], rk, cos, sin, pos), k_all[n_ctx], v_all[n_ctx]


def test_rope_attend_empty_context_returns_own_value():
    """ctx = 0: one score, weight 1, the output is the token's value exactly;
    the returned key is [k_nope | rotated k_rope]. Dropping the token's own
    score (planted) leaves nothing to attend and fails."""
    OM, cfg, w, args, _, k_own, v_own = _rope_attend_case(0)
    attn, k_new, v_new = OM.rope_attend(*args)
    assert torch.equal(attn, v_own.reshape(-1))
    assert torch.equal(k_new, k_own.reshape(-1))
    assert torch.equal(v_new, v_own.reshape(-1))
    n_ctx = 5
    OM, cfg, w, args, _, _, _ = _rope_attend_case(n_ctx, seed=41)
    good = OM.rope_attend(*args)[0]
    bad = OM.rope_attend(*args, drop_new=True)[0]
    assert not torch.equal(good, bad)


def test_rope_attend_equals_reference_attention_on_expanded_cache():
    """Two spellings of the same attention: the per-head assembled cache with a
    separate token term (rope_attend) and one softmax over the latent cache
    expanded with the token as its last row (attend_reference)."""
    from tests._check import rel_l2

    for n_ctx in (1, 7, 33):
        OM, cfg, w, args, (q_up, lat, rk, cos, sin, pos), _, _ = _rope_attend_case(n_ctx, seed=50 + n_ctx)
        got = OM.rope_attend(*args)[0]
        ref = OM.attend_reference(q_up, lat, rk, w, cfg, pos, cos, sin)
        assert rel_l2(got, ref) < 2e-3
        assert int(bf16_ulps(got, ref).max()) <= 2


def test_rope_attend_identical_keys_give_mean_value():
    """Every context key equal to the token's own: uniform weights, the output is
    the mean of the context values and the token's value."""
    OM, cfg, w, args, _, k_own, v_own = _rope_attend_case(6, seed=60)
    args = list(args)
    n = 6
    # context keys: [k_nope | rotated k_rope] of the token itself
    k_ctx = k_own.unsqueeze(0).expand(n, -1, -1).contiguous()
    args[6] = k_ctx
    attn = OM.rope_attend(*args)[0].double().view(cfg.heads, cfg.v_dim)
    mean = (args[7].double().sum(0) + v_own.double()) / (n + 1)
    assert float((attn - mean).abs().max()) <= float(mean.abs().max()) * 2 ** -7


def test_rope_attend_f64_brute_force():
    OM, cfg, w, args, _, _, _ = _rope_attend_case(4, seed=70)
    q_up, kv_up, k_rope, cos, sin, pos, kc, vc, n, scale, H, nope, rope, vd = args
    got = OM.rope_attend(*args)[0].double().view(H, vd)
    half = rope // 2
    for h in range(H):
        q = [float(x) for x in q_up.view(H, -1)[h]]
        def rot(x, j):
            c, s = float(cos[pos, j]), float(sin[pos, j])
            r = -x[j + half] if j < half else x[j - half]
            return float(torch.tensor(float(torch.tensor(x[j] * c).to(BF)) + float(torch.tensor(r * s).to(BF))).to(BF))
        qf = q[:nope] + [rot(q[nope:], j) for j in range(rope)]
        sc = float(scale)
        qh = [float(torch.tensor(x * sc).to(BF)) for x in qf]
        kr = [float(x) for x in k_rope]
        kv = [float(x) for x in kv_up.view(H, -1)[h]]
        k_new = kv[:nope] + [rot(kr, j) for j in range(rope)]
        v_new = kv[nope:]
        s = [sum(qh[d] * float(kc[j, h, d]) for d in range(nope + rope)) for j in range(n)]
        s.append(sum(qh[d] * k_new[d] for d in range(nope + rope)))
        mx = max(s)
        e = [math.exp(x - mx) for x in s]
        ref = [(sum(e[j] * float(vc[j, h, v]) for j in range(n)) + e[n] * v_new[v]) / sum(e) for v in range(vd)]
        ref = torch.tensor(ref, dtype=torch.float64)
        assert float((got[h] - ref).abs().max()) <= float(ref.abs().max()) * 2 ** -7


def test_mla_attention_composition_matches_projected_reference():
    """The op-by-op spelling (projections, rope_attend over the assembled cache,
    W_o) equals projecting with ``project`` and attending with
    ``attend_reference`` on the latent cache the assembled one came from."""
    from tests._check import rel_l2

    OM, cfg, w = _mla_small()
    n_ctx = 9
    pos = n_ctx
    cos, sin = OM.rope_tables(n_ctx + 1, cfg)
    hidden = torch.randn(cfg.hidden, generator=g(80)).to(BF)
    lat, rk = OM.random_cache(1, n_ctx, cfg, seed=81)
    k_ctx, v_ctx = OM.assembled_cache(lat[0], rk[0], w, cfg)
    scale = torch.tensor(cfg.scale).to(BF)
    out, k_new, v_new = OM.mla_attention(hidden, w, cfg, pos, cos, sin, k_ctx, v_ctx, n_ctx, scale)
    pr = OM.project(hidden, w, cfg, pos, cos, sin)
    lat_all = torch.cat((lat[0], pr.latent.view(1, -1)), 0)
    rk_all = torch.cat((rk[0], pr.k_rope.view(1, -1)), 0)
    ref = OM.proj(OM.attend_reference(pr.q_up, lat_all, rk_all, w, cfg, pos, cos, sin), w.w_o)
    assert rel_l2(out, ref) < 5e-3
    k_exp, v_exp = OM.assembled_cache(pr.latent.view(1, -1), pr.k_rope.view(1, -1), w, cfg)
    assert torch.equal(k_new, k_exp.reshape(-1)) and torch.equal(v_new, v_exp.reshape(-1))


# ---------------------------------------------------------------- prefill attention layer
def _prefill_small():
    from oracle import prefill as OP

    cfg = OP.PrefillConfig(hidden=64, heads=4, kv_heads=2, head_dim=16, rot=8)
    return OP, cfg, OP.random_layer(cfg, seed=5, std=0.2)


def test_prefill_rope_tables_against_closed_form():
    from oracle import prefill as OP

    cos, sin = OP.rope_tables(9000)
    i = torch.arange(32, dtype=torch.float64)
    inv = 1.0 / (1.0e7 ** (2 * i / 64))
    for p in (0, 3, 4095, 8191):
        assert int(bf16_ulps(cos[p, :32], torch.cos(p * inv).to(BF)).max()) <= 1
        assert int(bf16_ulps(sin[p, 32:], torch.sin(p * inv).to(BF)).max()) <= 1


def test_prefill_causal_prefix_invariance():
    OP, cfg, w = _prefill_small()
    cos, sin = OP.rope_tables(16, cfg)
    hn = torch.randn(12, cfg.hidden, generator=g(40)).to(BF)
    hn2 = hn.clone()
    hn2[7:] = torch.randn(5, cfg.hidden, generator=g(41)).to(BF)
    outs = []
    for x in (hn, hn2):
        q, gate, k, v = OP.qkv(x, w["w_q"], w["w_k"], w["w_v"], w["gamma_q"], w["gamma_k"], cos, sin, cfg)
        outs.append(OP.attention(q, k, v, gate, cfg))
    assert torch.equal(outs[0][:7], outs[1][:7])
    assert not torch.equal(outs[0][7:], outs[1][7:])


def test_prefill_one_row_returns_gated_value():
    OP, cfg, w = _prefill_small()
    q = torch.randn(1, cfg.heads, cfg.head_dim, generator=g(42)).to(BF)
    gate = torch.randn(1, cfg.heads, cfg.head_dim, generator=g(43)).to(BF)
    k = torch.randn(1, cfg.kv_heads, cfg.head_dim, generator=g(44)).to(BF)
    v = torch.randn(1, cfg.kv_heads, cfg.head_dim, generator=g(45)).to(BF)
    out = OP.attention(q, k, v, gate, cfg).view(cfg.heads, -1)
    for h in range(cfg.heads):
        ref = v[0, h // cfg.group].double() / (1.0 + torch.exp(-gate[0, h].double()))
        assert int(bf16_ulps(out[h], ref.to(BF)).max()) <= 1


def test_prefill_identical_keys_give_running_mean():
    OP, cfg, w = _prefill_small()
    N = 9
    q = torch.randn(N, cfg.heads, cfg.head_dim, generator=g(46)).to(BF)
    k = torch.randn(1, cfg.kv_heads, cfg.head_dim, generator=g(47)).to(BF).expand(N, -1, -1).contiguous()
    v = torch.randn(N, cfg.kv_heads, cfg.head_dim, generator=g(48)).to(BF)
    gate = torch.full((N, cfg.heads, cfg.head_dim), 30.0).to(BF)        # sigmoid(30) == 1 in bf16
    out = OP.attention(q, k, v, gate, cfg).view(N, cfg.heads, -1).double()
    for i in range(N):
        for h in range(cfg.heads):
            ref = v[: i + 1, h // cfg.group].double().mean(0)
            assert float((out[i, h] - ref).abs().max()) <= 2 ** -6 * float(ref.abs().max()) + 1e-3


def test_prefill_attention_f64_brute_force_and_causality():
    import math

    OP, cfg, w = _prefill_small()
    N, D = 6, cfg.head_dim
    q = torch.randn(N, cfg.heads, D, generator=g(49)).to(BF)
    k = torch.randn(N, cfg.kv_heads, D, generator=g(50)).to(BF)
    v = torch.randn(N, cfg.kv_heads, D, generator=g(51)).to(BF)
    gate = torch.randn(N, cfg.heads, D, generator=g(52)).to(BF)
    out = OP.attention(q, k, v, gate, cfg).view(N, cfg.heads, D).double()
    for i in range(N):
        for h in range(cfg.heads):
            kv = h // cfg.group
            s = [cfg.scale * sum(float(q[i, h, d]) * float(k[j, kv, d]) for d in range(D)) for j in range(i + 1)]
            mx = max(s)
            e = [math.exp(x - mx) for x in s]
            o = [sum(e[j] * float(v[j, kv, d]) for j in range(i + 1)) / sum(e) for d in range(D)]
            ref = torch.tensor([o[d] / (1 + math.exp(-float(gate[i, h, d]))) for d in range(D)], dtype=torch.float64)
            assert float((out[i, h] - ref).abs().max()) <= 2 ** -6 * float(ref.abs().max())
    # planted mistake: without the causal mask row 0 would see every key
    s = (q[0, 0].float() @ k[:, 0].float().t()) * cfg.scale
    full = (torch.softmax(s, -1).to(BF).float() @ v[:, 0].float()).to(BF) * torch.sigmoid(gate[0, 0])
    assert not torch.equal(full, out[0, 0].to(BF))


# ------------------------------------------------ MiniCPM3 whole-model oracle
def _minicpm3_against_hf(mutate=None):
    """Max relative L2 of the oracle's per-position logits against Hugging Face's
    MiniCPM3ForCausalLM (bf16, eager) built from the same random weights: the
    reference's third-party arithmetic boundary, installed here. ``mutate`` plants
    a mistake in the oracle's config."""
    import dataclasses

    from transformers import MiniCPM3Config
    from transformers.models.minicpm3 import modeling_minicpm3 as HF

    from oracle import minicpm3 as OM

    # scale_depth 0.3 over 2 layers makes the residual scale 0.21, far from 1,
    # so a dropped scale shows
    cfg = OM.ModelConfig(hidden=256, heads=4, q_lora=96, kv_lora=64, inter=512, vocab=512, layers=2,
                         dim_model_base=64, scale_depth=0.3)
    m = OM.random_model(cfg, 3, std=0.05)
    hc = MiniCPM3Config(
        hidden_size=cfg.hidden, num_hidden_layers=cfg.layers, intermediate_size=cfg.inter,
        num_attention_heads=cfg.heads, num_key_value_heads=cfg.heads, qk_nope_head_dim=cfg.nope,
        qk_rope_head_dim=cfg.rope, q_lora_rank=cfg.q_lora, kv_lora_rank=cfg.kv_lora, v_head_dim=cfg.v_dim,
        vocab_size=cfg.vocab, rms_norm_eps=cfg.eps, scale_emb=cfg.scale_emb, dim_model_base=cfg.dim_model_base,
        scale_depth=cfg.scale_depth, max_position_embeddings=4096, tie_word_embeddings=True,
        rope_scaling={"type": "longrope", "factor": 1.0, "long_factor": list(OM.SHORT_FACTOR),
                      "short_factor": list(OM.SHORT_FACTOR), "original_max_position_embeddings": 4096,
                      "rope_theta": cfg.rope_theta})
    hf = HF.MiniCPM3ForCausalLM(hc).eval().to(torch.bfloat16)
    names = {"gamma_in": "input_layernorm", "w_q_a": "self_attn.q_a_proj", "gamma_q_a": "self_attn.q_a_layernorm",
             "w_q_b": "self_attn.q_b_proj", "w_kv_a": "self_attn.kv_a_proj_with_mqa",
             "gamma_kv_a": "self_attn.kv_a_layernorm", "w_kv_b": "self_attn.kv_b_proj", "w_o": "self_attn.o_proj",
             "gamma_post": "post_attention_layernorm", "w_gate": "mlp.gate_proj", "w_up": "mlp.up_proj",
             "w_down": "mlp.down_proj"}
    sd = {"model.embed_tokens.weight": m.embed, "model.norm.weight": m.gamma_final, "lm_head.weight": m.embed}
    for i, lw in enumerate(m.layers):
        for k, n in names.items():
            sd[f"model.layers.{i}.{n}.weight"] = getattr(lw, k)
    missing, unexpected = hf.load_state_dict(sd, strict=False)
    assert not missing and not unexpected, (missing, unexpected)
    prompt = [3, 17, 42, 99, 7, 250]
    with torch.no_grad():
        ref = hf(torch.tensor([prompt])).logits[0].float()
    ocfg = mutate(cfg) if mutate else cfg
    cos, sin = OM.rope_tables(len(prompt), ocfg)
    caches = OM.empty_caches(ocfg, ocfg.layers)
    worst = 0.0
    for p, t in enumerate(prompt):
        lg = OM.decode_step(m, ocfg, t, p, caches, cos, sin)
        worst = max(worst, float((lg - ref[p]).norm() / ref[p].norm()))
    return worst


def test_minicpm3_model_oracle_against_hugging_face():
    assert _minicpm3_against_hf() < 1e-2


def test_minicpm3_model_oracle_planted_mistakes():
    import dataclasses

    from oracle import minicpm3 as OM

    class NoResidualScale(OM.ModelConfig):
        @property
        def residual_scale(self):
            return 1.0

    assert _minicpm3_against_hf(lambda c: NoResidualScale(**dataclasses.asdict(c))) > 0.1
    assert _minicpm3_against_hf(lambda c: dataclasses.replace(c, scale_emb=1.0)) > 0.1
    assert _minicpm3_against_hf(lambda c: dataclasses.replace(c, dim_model_base=c.hidden * c.hidden // c.dim_model_base)) > 0.1


# ------------------------------------------------ Qwen3 oracle against Hugging Face
# The reference builds its decode oracle from the Hugging Face layer
# (tests/core/models/decode_oracle.py:213-233; smoke_qwen3_1_7b.py:78-125):
# Qwen3ForCausalLM, installed here, is the third-party arithmetic boundary. It is
# built from a tiny config and loaded with the oracle's own random weights.
_QWEN3_HF_NAMES = {"gamma_in": "input_layernorm", "w_q": "self_attn.q_proj", "w_k": "self_attn.k_proj",
                   "w_v": "self_attn.v_proj", "gamma_q": "self_attn.q_norm", "gamma_k": "self_attn.k_norm",
                   "w_o": "self_attn.o_proj", "gamma_post": "post_attention_layernorm",
                   "w_gate": "mlp.gate_proj", "w_up": "mlp.up_proj", "w_down": "mlp.down_proj"}
_QWEN3_PROMPT = [3, 17, 42, 99, 7, 250, 31, 400, 5, 77, 128, 9]


def _qwen3_hf(std: float, gspread: float):
    """(oracle config, oracle weights, HF model) from the same tiny random weights.
    ``gspread`` is the spread of the q/k head-norm scales around 1: a wide one makes
    the order of norm and rotation matter (planted-mistake tests)."""
    from transformers import Qwen3Config
    from transformers.models.qwen3 import modeling_qwen3 as HF

    cfg = OQ.Qwen3Config(hidden=256, heads=4, kv_heads=2, head_dim=64, inter=512, vocab=512, layers=2)
    m = OQ.random_model(cfg, seed=11, std=std)
    gen = g(12)
    for lw in m.layers:
        lw.gamma_q = (1 + gspread * torch.randn(cfg.head_dim, generator=gen)).to(BF)
        lw.gamma_k = (1 + gspread * torch.randn(cfg.head_dim, generator=gen)).to(BF)
    hc = Qwen3Config(vocab_size=cfg.vocab, hidden_size=cfg.hidden, intermediate_size=cfg.inter,
                     num_hidden_layers=cfg.layers, num_attention_heads=cfg.heads,
                     num_key_value_heads=cfg.kv_heads, head_dim=cfg.head_dim, rms_norm_eps=cfg.eps,
                     rope_theta=cfg.rope_theta, max_position_embeddings=4096, tie_word_embeddings=True,
                     attention_bias=False)
    hc._attn_implementation = "eager"
    hf = HF.Qwen3ForCausalLM(hc).eval().to(BF)
    # .to(bf16) also lands the rotary inverse frequencies; a bf16 checkpoint load
    # keeps them in f32 (they are recomputed, not stored)
    inv, _ = hf.model.rotary_emb.compute_default_rope_parameters(hc)
    hf.model.rotary_emb.inv_freq = inv.float()
    sd = {"model.embed_tokens.weight": m.embed, "model.norm.weight": m.gamma_final, "lm_head.weight": m.embed}
    for i, lw in enumerate(m.layers):
        for k, n in _QWEN3_HF_NAMES.items():
            sd[f"model.layers.{i}.{n}.weight"] = getattr(lw, k)
    missing, unexpected = hf.load_state_dict(sd, strict=False)
    assert not missing and not unexpected, (missing, unexpected)
    return cfg, m, hf


def _qwen3_vs_hf(cfg, m, hf, prompt=_QWEN3_PROMPT):
    """Worst relative L2 over the prompt's positions of (logits, layer-0 output):
    the oracle's cached step by step against HF's one causal forward."""
    with torch.no_grad():
        out = hf(torch.tensor([prompt]), output_hidden_states=True)
    ref_logits, ref_h0 = out.logits[0].float(), out.hidden_states[1][0].float()
    cos, sin = OQ.rope_tables(len(prompt), cfg.head_dim, cfg.rope_theta)
    caches = OQ.empty_caches(cfg, cfg.layers)
    worst_l, worst_h = 0.0, 0.0
    for p, t in enumerate(prompt):
        h = m.embed[t].clone()
        for li, (lw, cache) in enumerate(zip(m.layers, caches)):
            h, k, v = OQ.decoder_layer(h, lw, cfg, cos[p], sin[p], cache[0], cache[1], p_bf16=True)
            cache[0] = torch.cat([cache[0], k.unsqueeze(0)], 0)
            cache[1] = torch.cat([cache[1], v.unsqueeze(0)], 0)
            if li == 0:
                worst_h = max(worst_h, float((h.float() - ref_h0[p]).norm() / ref_h0[p].norm()))
        lg = OQ.lm_logits(h, m.gamma_final, m.head32(), cfg.eps)
        worst_l = max(worst_l, float((lg - ref_logits[p]).norm() / ref_logits[p].norm()))
    return worst_l, worst_h


def test_qwen3_oracle_against_hugging_face():
    """Per-position logits and the first decoder layer's output agree with HF's
    Qwen3ForCausalLM within the bf16 bar. HF lands the RoPE products, the scores
    and the logits in bf16 where the oracle keeps f32 (the reference kernel's
    order), which is what remains."""
    lg, h0 = _qwen3_vs_hf(*_qwen3_hf(std=0.02, gspread=0.1))
    assert lg < 1e-2 and h0 < 1e-2, (lg, h0)
    # sharp attention (larger weights, widely spread head-norm scales)
    lg, h0 = _qwen3_vs_hf(*_qwen3_hf(std=0.05, gspread=0.5))
    assert lg < 2e-2 and h0 < 1.5e-2, (lg, h0)


def _sa_planted(kind):
    """``self_attention`` with one planted mistake."""
    def sa(h, lw, c, cos_row, sin_row, k_cache, v_cache, p_bf16=False):
        HQ, HKV, D = c.heads, c.kv_heads, c.head_dim
        xn = ON.rms_norm_q(h, lw.gamma_in, c.eps)
        q = OQ._proj(xn, lw, "w_q").view(HQ, D)
        k = OQ._proj(xn, lw, "w_k").view(HKV, D)
        v = OQ._proj(xn, lw, "w_v").view(HKV, D)
        if kind == "rope_before_norm":
            q = OQ.head_norm(OQ.rope(q, cos_row, sin_row), lw.gamma_q, c.eps)
            k = OQ.head_norm(OQ.rope(k, cos_row, sin_row), lw.gamma_k, c.eps)
        elif kind == "no_head_norm":
            q, k = OQ.rope(q, cos_row, sin_row), OQ.rope(k, cos_row, sin_row)
        elif kind == "k_gamma_for_q":
            q = OQ.rope(OQ.head_norm(q, lw.gamma_k, c.eps), cos_row, sin_row)
            k = OQ.rope(OQ.head_norm(k, lw.gamma_k, c.eps), cos_row, sin_row)
        kk = torch.cat([k_cache, k.unsqueeze(0)], 0)
        vv = torch.cat([v_cache, v.unsqueeze(0)], 0)
        return OQ._proj(OQ.attend(q, kk, vv, c.scale, p_bf16), lw, "w_o"), k, v
    return sa


def _mlp_swapped(h1, lw, c):
    xn = ON.rms_norm_q(h1, lw.gamma_post, c.eps)
    act = torch.nn.functional.silu(OQ._proj(xn, lw, "w_up").float()).to(BF) * OQ._proj(xn, lw, "w_gate")
    return OQ._proj(act, lw, "w_down")


@pytest.mark.parametrize("plant", ["gate_up_swapped", "rope_before_norm", "no_head_norm", "k_gamma_for_q",
                                   "no_residual"])
def test_qwen3_oracle_planted_mistakes_fail_the_hf_pin(plant, monkeypatch):
    """Each planted mistake moves the logits far past the tolerance of the pin above."""
    built = _qwen3_hf(std=0.05, gspread=0.5)
    if plant == "gate_up_swapped":
        monkeypatch.setattr(OQ, "mlp", _mlp_swapped)
    elif plant == "no_residual":
        orig = OQ.self_attention
        monkeypatch.setattr(OQ, "decoder_layer", lambda h, lw, c, cr, sr, kc, vc, p_bf16=False: (
            lambda a: (a[0] + OQ.mlp(a[0], lw, c), a[1], a[2]))(orig(h, lw, c, cr, sr, kc, vc, p_bf16)))
    else:
        monkeypatch.setattr(OQ, "self_attention", _sa_planted(plant))
    lg, _ = _qwen3_vs_hf(*built)
    assert lg > 0.1, (plant, lg)


# ------------------------------------ Qwen3.5 attention-layer oracle against Hugging Face
def _qwen35_vs_hf(std=0.05, gspread=0.5, n=24):
    """Relative L2 of the prefill oracle's attention block (``qkv`` -> ``attention``
    -> ``o_proj``) against Hugging Face's Qwen3_5Attention (eager, bf16) with the
    same weights, plus the rope tables' largest difference from HF's rotary
    module. The residual is left out of the comparison (``o_proj`` over a zero
    hidden state) so that a small block output is not hidden under it."""
    from transformers.models.qwen3_5 import modeling_qwen3_5 as HF
    from transformers.models.qwen3_5.configuration_qwen3_5 import Qwen3_5TextConfig

    from oracle import prefill as OP

    pc = OP.PrefillConfig(hidden=256, heads=6, kv_heads=2, head_dim=64, rot=16)
    lw = OP.random_layer(pc, seed=5, std=std)
    gen = g(6)
    lw["gamma_q"] = (gspread * torch.randn(pc.head_dim, generator=gen)).to(BF)
    lw["gamma_k"] = (gspread * torch.randn(pc.head_dim, generator=gen)).to(BF)
    hc = Qwen3_5TextConfig(hidden_size=pc.hidden, num_attention_heads=pc.heads, num_key_value_heads=pc.kv_heads,
                           head_dim=pc.head_dim, rms_norm_eps=pc.eps, num_hidden_layers=1,
                           layer_types=["full_attention"], vocab_size=64, intermediate_size=128,
                           rope_parameters={"rope_type": "default", "rope_theta": pc.rope_theta,
                                            "partial_rotary_factor": pc.rot / pc.head_dim},
                           max_position_embeddings=4096, attention_bias=False)
    hc._attn_implementation = "eager"
    att = HF.Qwen3_5Attention(hc, 0).eval().to(BF)
    att.load_state_dict({"q_proj.weight": lw["w_q"], "k_proj.weight": lw["w_k"], "v_proj.weight": lw["w_v"],
                         "o_proj.weight": lw["w_o"], "q_norm.weight": lw["gamma_q"],
                         "k_norm.weight": lw["gamma_k"]})
    rot = HF.Qwen3_5TextRotaryEmbedding(hc)
    hn = torch.randn(1, n, pc.hidden, generator=gen).to(BF)
    with torch.no_grad():
        cos_h, sin_h = rot(hn, torch.arange(n)[None])
        mask = torch.full((n, n), float("-inf")).triu(1)[None, None].to(BF)
        ref = att(hn, (cos_h, sin_h), mask)[0][0].float()
    cos, sin = OP.rope_tables(n, pc)
    table_diff = max(float((cos.float() - cos_h[0].float()).abs().max()),
                     float((sin.float() - sin_h[0].float()).abs().max()))
    q, gate, k, v = OP.qkv(hn[0], lw["w_q"], lw["w_k"], lw["w_v"], lw["gamma_q"], lw["gamma_k"], cos, sin, pc)
    out = OP.o_proj(OP.attention(q, k, v, gate, pc), torch.zeros(n, pc.hidden), lw["w_o"]).float()
    return float((out - ref).norm() / ref.norm()), table_diff


def test_prefill_oracle_against_hugging_face():
    """``qkv`` (per-head [q | gate] split, (1+gamma) head norms, 16 of 64 dims
    rotated), ``attention`` (causal, sigmoid output gate) and ``o_proj`` agree
    with HF's Qwen3_5Attention; the rope tables are HF's exactly."""
    err, table_diff = _qwen35_vs_hf()
    assert err < 1e-2 and table_diff == 0.0, (err, table_diff)
    err, _ = _qwen35_vs_hf(std=0.02, gspread=0.1)
    assert err < 1e-2, err


@pytest.mark.parametrize("plant", ["plain_gamma", "gate_dropped", "no_rope", "full_rotation"])
def test_prefill_oracle_planted_mistakes_fail_the_hf_pin(plant, monkeypatch):
    from oracle import prefill as OP

    if plant == "plain_gamma":        # gamma instead of (1 + gamma)
        monkeypatch.setattr(OP, "rms_norm_1p", lambda x, gm, eps: (
            x.float() * torch.rsqrt(x.float().pow(2).mean(-1, keepdim=True) + eps) * gm.float()).to(BF))
    elif plant == "gate_dropped":     # sigmoid(gate) -> 1
        orig = OP.attention
        monkeypatch.setattr(OP, "attention", lambda q, k, v, gate, cfg=None, heads=None: orig(
            q, k, v, torch.full_like(gate, 30.0), cfg))
    elif plant == "no_rope":
        orig_r = OP.rope_partial
        monkeypatch.setattr(OP, "rope_partial", lambda x, c, s, rot: orig_r(x, torch.ones_like(c),
                                                                            torch.zeros_like(s), rot))
    elif plant == "full_rotation":    # rotate all 64 dims with the 16-dim tables tiled
        orig_r = OP.rope_partial
        monkeypatch.setattr(OP, "rope_partial", lambda x, c, s, rot: orig_r(
            x, c.repeat(*([1] * (c.dim() - 1)), x.shape[-1] // rot), s.repeat(*([1] * (s.dim() - 1)),
                                                                             x.shape[-1] // rot), x.shape[-1]))
    err, _ = _qwen35_vs_hf()
    assert err > 5e-2, (plant, err)


def test_prefill_attention_rows_equals_full_attention():
    """The sampled-rows form (used at 4096-8192 tokens) is the full causal
    attention at those rows: within one bf16 landing (a shorter softmax row
    may sum in another order)."""
    from oracle import prefill as OP

    cfg = OP.PrefillConfig(hidden=256, heads=6, kv_heads=2, head_dim=64, rot=16)
    gen = g(41)
    n = 96
    q, gate = (torch.randn(n, 6, 64, generator=gen).to(BF) for _ in range(2))
    k, v = (torch.randn(n, 2, 64, generator=gen).to(BF) for _ in range(2))
    rows, heads = [0, 1, 47, 95], [0, 3, 5]
    full = OP.attention(q, k, v, gate, cfg).view(n, 6, 64)
    got = OP.attention_rows(q, k, v, gate, rows, heads, cfg)
    assert int(bf16_ulps(got, full[rows][:, heads]).max()) <= 1
    # row 0 sees only key 0: its output is v0 * sigmoid(gate)
    assert torch.equal(got[0, 0], v[0, 0] * torch.sigmoid(gate[0, 0]))


def test_prefill_o_proj_double_landing_f64_and_known_answer():
    """``o_proj`` is ``bf16(hidden + bf16(gated . W_o^T))`` with a non-zero
    hidden state: within one bf16 ulp of its f64 statement on random rows, and
    on a hand-worked row the product's own landing decides the answer -- the
    product 2^-8 + 2^-20 lands as 2^-8, and 1 + 2^-8 is a tie that rounds to
    1.0 (even); one landing of hidden + product gives 1 + 2^-7."""
    from oracle import prefill as OP

    gen = g(62)
    gated = torch.randn(32, 384, generator=gen).to(BF)
    w_o = (0.05 * torch.randn(256, 384, generator=gen)).to(BF)
    hidden = torch.randn(32, 256, generator=gen).to(BF)
    got = OP.o_proj(gated, hidden, w_o)
    prod = (gated.double() @ w_o.double().t()).to(BF)
    want = (hidden.double() + prod.double()).to(BF)
    assert int(bf16_ulps(got, want).max()) <= 1
    single = (hidden.float() + gated.float() @ w_o.float().t()).to(BF)
    assert not torch.equal(got, single), "the double landing is exercised on random rows"
    # known answer
    g2 = torch.tensor([[2 ** -8, 2 ** -20]]).to(BF)
    w2 = torch.ones(4, 2).to(BF)
    h2 = torch.ones(1, 4).to(BF)
    assert torch.equal(OP.o_proj(g2, h2, w2), torch.ones(1, 4).to(BF))
    assert torch.equal((h2.float() + g2.float() @ w2.float().t()).to(BF), torch.full((1, 4), 1 + 2 ** -7).to(BF))


def test_top_p_kept_closed_forms():
    """The sampler's kept set: one dominant logit keeps it alone; a uniform row
    keeps the first ceil(top_p V) tokens in index order with equal
    probabilities; top_p >= 1 keeps every token of nonzero probability; a
    planted mistake (keeping while the mass *including* the token is below
    top_p) drops the boundary token of the uniform row."""
    from oracle import minicpm3 as OM

    lg = torch.zeros(1000)
    lg[417] = 100.0
    ids, p = OM.top_p_kept(lg, 0.8, 0.8)
    assert ids.tolist() == [417] and float(p[0]) == 1.0
    uni = torch.zeros(1000)
    for top_p in (0.25, 0.5, 0.8, 0.999):
        ids, p = OM.top_p_kept(uni, 1.0, top_p)
        n = math.ceil(top_p * 1000 - 1e-9)
        assert ids.tolist() == list(range(n)), (top_p, len(ids))
        assert float((p - 1.0 / n).abs().max()) < 1e-12
    ids, _ = OM.top_p_kept(torch.randn(500, generator=g(70)), 0.8, 1.0)
    assert sorted(ids.tolist()) == list(range(500))
    probs = torch.softmax(uni / 1.0, -1)
    wrong = (torch.cumsum(probs, -1) < 0.25).sum()   # mass including the token
    assert int(wrong) != len(OM.top_p_kept(uni, 1.0, 0.25)[0])
