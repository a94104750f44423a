"""The reference-signature APIs -- the Qwen3 layer / root twins, the MiniCPM3
``reference_ops`` and layer twin, the prefill ``Attention`` -- against the
oracle on the same seeded inputs. The GPU cases call the HIP kernels through
the twins; the CPU cases check the host-side contract (argument checks,
cache containers) without a GPU."""
import pytest
import torch

from oracle import minicpm3 as OM
from oracle import norms as ON
from oracle import prefill as OP
from oracle import qwen3 as OQ
from tests._check import assert_close, assert_equal, assert_l2, assert_ulps

BF = torch.bfloat16


def g(seed):
    return torch.Generator().manual_seed(seed)


def randn(*shape, seed, scale=1.0, dtype=BF):
    return (torch.randn(*shape, generator=g(seed)) * scale).to(dtype)


def authored(w: torch.Tensor) -> torch.Tensor:
    """An (out, in) matrix in the authored ConstTensor shape [1, in, out] (a view)."""
    return w.t().unsqueeze(0)


# ------------------------------------------------------------------ Qwen3 layer
def _qwen3_layer(dev, ctx, seed=0):
    cfg = OQ.Qwen3Config()
    lw = OQ.random_model(cfg, seed=seed, n_layers=1).layers[0]
    cos, sin = OQ.rope_tables(ctx + 1, cfg.head_dim, cfg.rope_theta)
    h = randn(cfg.hidden, seed=seed + 1)
    kc = randn(ctx, cfg.kv_heads, cfg.head_dim, seed=seed + 2)
    vc = randn(ctx, cfg.kv_heads, cfg.head_dim, seed=seed + 3)
    return cfg, lw, cos, sin, h, kc, vc


@pytest.mark.gpu
@pytest.mark.parametrize("ctx", [0, 300])
def test_layer_twin_self_attention_and_decoder_layer(dev, ctx):
    from tilefoundry_amd.twin import LayerTwin

    cfg, lw, cos, sin, h, kc, vc = _qwen3_layer(dev, ctx, seed=10)
    pos = ctx
    t = LayerTwin()
    d = lambda x: x.to(dev)  # noqa: E731
    W = {k: d(getattr(lw, k)) for k in ("gamma_in", "w_q", "w_k", "w_v", "gamma_q", "gamma_k",
                                        "w_o", "gamma_post", "w_gate", "w_up", "w_down")}
    A = {k: (authored(v) if v.dim() == 2 else v) for k, v in W.items()}
    scale = torch.full((1, 1, 1, 1), cfg.scale, device=dev, dtype=BF)
    pos_ids = torch.tensor([pos], device=dev, dtype=torch.int32)
    k4, v4 = d(kc).unsqueeze(0), d(vc).unsqueeze(0)
    cos_d, sin_d = d(cos), d(sin)

    # input_rms_norm
    got = t.input_rms_norm(d(h).view(1, 1, -1), A["gamma_in"])
    assert_ulps("input_rms_norm", got.view(-1), ON.rms_norm_q(h, lw.gamma_in, cfg.eps), 1, 0.01)

    # self_attention: (out, k_new, v_new)
    out, k_new, v_new = t.self_attention(d(h).view(1, 1, -1), A["gamma_in"], A["w_q"], A["w_k"],
                                         A["w_v"], A["gamma_q"], A["gamma_k"], cos_d, sin_d,
                                         pos_ids, k4, v4, scale, A["w_o"])
    o_ref, k_ref, v_ref = OQ.self_attention(h, lw, cfg, cos[pos], sin[pos], kc, vc, p_bf16=True)
    assert out.shape == (1, 1, cfg.hidden) and k_new.shape == (1, 1, cfg.kv_heads, cfg.head_dim)
    assert_close("self_attention.out", out.view(-1), o_ref)
    assert_ulps("self_attention.k_new", k_new.view(cfg.kv_heads, -1), k_ref, 2, 0.02)
    assert_ulps("self_attention.v_new", v_new.view(cfg.kv_heads, -1), v_ref, 1, 0.01)

    # mlp
    m = t.mlp(d(h).view(1, 1, -1), A["gamma_post"], A["w_gate"], A["w_up"], A["w_down"])
    assert_close("mlp", m.view(-1), OQ.mlp(h, lw, cfg))

    # decoder_layer = attention + residual, mlp + residual
    hl, k2, v2 = t.decoder_layer(d(h).view(1, 1, -1), A["gamma_in"], A["w_q"], A["w_k"], A["w_v"],
                                 A["gamma_q"], A["gamma_k"], cos_d, sin_d, pos_ids, k4, v4, scale,
                                 A["w_o"], A["gamma_post"], A["w_gate"], A["w_up"], A["w_down"])
    h_ref, _, _ = OQ.decoder_layer(h, lw, cfg, cos[pos], sin[pos], kc, vc, p_bf16=True)
    assert_close("decoder_layer", hl.view(-1), h_ref)
    assert_equal("decoder_layer.k_new", k2, k_new)
    # (out, in) weights are read as they are, with the same result
    hl2, _, _ = t.decoder_layer(d(h).view(1, 1, -1), W["gamma_in"], W["w_q"], W["w_k"], W["w_v"],
                                W["gamma_q"], W["gamma_k"], cos_d, sin_d, pos_ids, k4, v4, scale,
                                W["w_o"], W["gamma_post"], W["w_gate"], W["w_up"], W["w_down"])
    assert_equal("decoder_layer (out, in)", hl2, hl)


@pytest.mark.gpu
def test_root_twin_greedy_loop(dev):
    """The root's step loop (prepare_inputs_for_generation -> forward ->
    append_cache) on a two-layer model, teacher-forced with the oracle's own
    greedy tokens: the logits agree at every step and so do the picks wherever
    the oracle's top two are more than a bf16 step apart."""
    from tilefoundry_amd.qwen3 import Qwen3Config, synthetic_weights, hf_names
    from tilefoundry_amd.twin import RootTwin

    cfg = Qwen3Config(hidden=512, heads=4, kv_heads=2, head_dim=128, inter=1024, vocab=4096,
                      layers=2, max_pos=64)
    wts = synthetic_weights(cfg, seed=3)
    model = OQ.ModelWeights(
        embed=wts["model.embed_tokens.weight"], gamma_final=wts["model.norm.weight"],
        layers=[OQ.LayerWeights(**{k: wts[n] for k, n in hf_names(i).items()})
                for i in range(cfg.layers)])
    ocfg = OQ.Qwen3Config(hidden=512, heads=4, kv_heads=2, head_dim=128, inter=1024, vocab=4096,
                          layers=2)
    prompt = [5, 17, 99, 2048, 7]
    max_new = 6
    record = []
    want = OQ.decode(model, ocfg, prompt, max_new, record=record, p_bf16=True)

    root = RootTwin(cfg, {k: v.to(dev) for k, v in wts.items()}, device=dev)
    feed = torch.tensor(prompt + want, dtype=torch.int64)
    caches = root.init_caches(dev)
    assert len(caches) == cfg.layers and caches[0][0].shape == (1, 0, cfg.kv_heads, cfg.head_dim)
    for step in range(len(prompt) + max_new - 1):
        inputs = root.prepare_inputs_for_generation(feed, step, caches, dev)
        logits, entries = root.forward(*inputs)
        caches = root.append_cache(caches, entries)
        assert caches[0][0].shape[1] == step + 1
        i = step - (len(prompt) - 1)
        if i >= 0:
            ref_logits, pick, gap = record[i]
            assert_close(f"logits step {step}", logits.view(-1).float(), ref_logits, rtol=2e-2)
            if gap > 2 * 2 ** -7 * float(ref_logits.abs().max()):
                assert int(logits.view(-1).float().argmax()) == pick


def test_root_twin_contract_on_cpu():
    from tilefoundry_amd.qwen3 import Qwen3Config
    from tilefoundry_amd.twin import LayerTwin, RootTwin

    cfg = Qwen3Config(layers=3)
    root = RootTwin(cfg)
    caches = root.init_caches("cpu")
    assert len(caches) == 3 and caches[2][1].shape == (1, 0, cfg.kv_heads, cfg.head_dim)
    with pytest.raises(ValueError, match="3 layers but was given 2"):
        root.decode_hidden(None, None, None, None, None, caches[:2])
    fresh = tuple((torch.ones(1, 1, cfg.kv_heads, cfg.head_dim, dtype=BF),) * 2 for _ in range(3))
    grown = root.append_cache(caches, fresh)
    assert grown[1][0].shape == (1, 1, cfg.kv_heads, cfg.head_dim)
    with pytest.raises(TypeError, match="no bound weights"):
        LayerTwin(cfg)(None, None, None, None, None, None, None)
    with pytest.raises(KeyError, match="missing"):
        RootTwin(cfg, {"model.embed_tokens.weight": torch.zeros(1)})


# ----------------------------------------------------------- MiniCPM3 reference_ops
MCFG = OM.MLAConfig()


@pytest.mark.gpu
def test_reference_ops_projections(dev):
    from tilefoundry_amd import reference_ops as R

    Hd, N, I = MCFG.hidden, 1056, 6400
    x, gm = randn(Hd, seed=30), (1 + 0.1 * torch.randn(Hd, generator=g(31))).to(BF)
    w = randn(N, Hd, seed=32, scale=0.02)
    d = lambda t: t.to(dev)  # noqa: E731
    assert_ulps("rmsnorm", R.rmsnorm(d(x), d(gm), MCFG.eps), ON.rms_norm_q(x, gm, MCFG.eps), 1, 0.01)
    xn = ON.rms_norm_q(x, gm, MCFG.eps)
    assert_close("rmsnorm_gemv", R.rmsnorm_gemv(d(x), d(gm), d(w), MCFG.eps), OM.proj(xn, w))
    out1 = torch.empty(N, device=dev, dtype=BF)
    w2 = randn(640, Hd, seed=33, scale=0.02)
    o1, o2 = R.rmsnorm_gemv_pair(d(x), d(gm), d(w), d(x), d(gm), d(w2), MCFG.eps, out1=out1)
    assert o1 is out1
    assert_close("pair.1", o1, OM.proj(xn, w))
    assert_close("pair.2", o2, OM.proj(xn, w2))
    assert_close("gemv", R.gemv(d(x), d(w)), OM.proj(x, w))
    res = randn(N, seed=34)
    alpha = torch.tensor(1.4 / 62 ** 0.5).to(BF)
    got = R.gemv_residual(d(x), d(w), d(res), d(alpha.reshape(1)))
    assert_close("gemv_residual", got, OM.o_proj_residual(x, w, res, float(alpha)))
    wg, wu = randn(I, Hd, seed=35, scale=0.02), randn(I, Hd, seed=36, scale=0.02)
    got = R.rmsnorm_gemv_swiglu(d(x), d(gm), d(wg), d(wu), MCFG.eps)
    ref = torch.nn.functional.silu(OM.proj(xn, wg).float()).to(BF) * OM.proj(xn, wu)
    assert_close("rmsnorm_gemv_swiglu", got, ref)
    table = randn(1000, Hd, seed=37)
    tok = torch.tensor([613], device=dev)
    assert_equal("embed_scaled", R.embed_scaled(d(table), tok, 12.0), (table[613].float() * 12.0).to(BF))
    wh = randn(4096, Hd, seed=38, scale=0.02)
    ref = ((x.float() / 10.0).to(BF).float() @ wh.float().t()).to(BF)
    assert_close("lm_head_gemv", R.lm_head_gemv(d(x), d(wh), 10.0), ref)


@pytest.mark.gpu
@pytest.mark.parametrize("ctx", [0, 5, 300, 700])
def test_reference_ops_rope_attend(dev, ctx):
    from tilefoundry_amd import reference_ops as R

    NH, NOPE, ROPE, VD, CAP = MCFG.heads, MCFG.nope, MCFG.rope, MCFG.v_dim, 1024
    QK = NOPE + ROPE
    cos, sin = OM.rope_tables(CAP + 1, MCFG)
    q_up, kv_up = randn(NH * QK, seed=40), randn(NH * (NOPE + VD), seed=41)
    k_rope = randn(ROPE, seed=42)
    kc, vc = randn(CAP, NH, QK, seed=43), randn(CAP, NH, VD, seed=44)
    scale = torch.tensor(MCFG.scale).to(BF)
    pos = ctx
    d = lambda t: t.to(dev)  # noqa: E731
    attn, k_new, v_new = R.rope_attend(
        d(q_up), d(kv_up), d(k_rope), d(cos), d(sin), torch.tensor([pos], device=dev, dtype=torch.int32),
        d(kc), d(vc), torch.tensor([ctx], device=dev, dtype=torch.int32), d(scale.reshape(1)),
        NH, NOPE, ROPE, VD)
    a_ref, k_ref, v_ref = OM.rope_attend(q_up, kv_up, k_rope, cos, sin, pos, kc, vc, ctx, scale,
                                         NH, NOPE, ROPE, VD)
    assert_close("rope_attend.attn", attn, a_ref)
    assert_equal("rope_attend.k_new", k_new, k_ref)
    assert_equal("rope_attend.v_new", v_new, v_ref)


@pytest.mark.gpu
def test_minicpm3_layer_twin(dev):
    """mla_attention, mlp and decoder_layer (with the scale_depth residual) in
    the authored signatures, against the oracle's op-by-op spelling."""
    from tilefoundry_amd.twin import MiniCPM3LayerTwin

    cfg = MCFG
    I = 6400
    w = OM.random_weights(cfg, seed=50)
    ctx = 40
    pos = ctx
    cos, sin = OM.rope_tables(ctx + 1, cfg)
    lat, rk = OM.random_cache(1, ctx, cfg, seed=51)
    k_ctx, v_ctx = OM.assembled_cache(lat[0], rk[0], w, cfg)
    h = randn(cfg.hidden, seed=52)
    scale = torch.tensor(cfg.scale).to(BF)
    gp = (1 + 0.1 * torch.randn(cfg.hidden, generator=g(53))).to(BF)
    wg, wu = randn(I, cfg.hidden, seed=54, scale=0.02), randn(I, cfg.hidden, seed=55, scale=0.02)
    wd = randn(cfg.hidden, I, seed=56, scale=0.02)
    alpha = torch.tensor(1.4 / 62 ** 0.5).to(BF)

    d = lambda t: t.to(dev)  # noqa: E731
    t = MiniCPM3LayerTwin(cfg, inter=I)
    args = (d(h).view(1, 1, -1), d(w.gamma_in), d(authored(w.w_q_a)), d(w.gamma_q_a),
            d(authored(w.w_q_b)), d(authored(w.w_kv_a)), d(w.gamma_kv_a), d(authored(w.w_kv_b)),
            d(cos), d(sin), torch.tensor([pos], device=dev, dtype=torch.int32),
            d(k_ctx).unsqueeze(0), d(v_ctx).unsqueeze(0), d(scale).view(1, 1, 1, 1),
            d(authored(w.w_o)))
    out, k_new, v_new = t.mla_attention(*args)
    o_ref, k_ref, v_ref = OM.mla_attention(h, w, cfg, pos, cos, sin, k_ctx, v_ctx, ctx, scale)
    assert out.shape == (1, 1, cfg.hidden) and k_new.shape == (1, 1, cfg.heads, cfg.qk_dim)
    assert_close("mla_attention.out", out.view(-1), o_ref)
    assert_ulps("mla_attention.k_new", k_new.view(-1), k_ref, 1, 0.01)
    assert_ulps("mla_attention.v_new", v_new.view(-1), v_ref, 1, 0.01)

    def mlp_ref(x):
        n = ON.rms_norm_q(x, gp, cfg.eps)
        return OM.proj(torch.nn.functional.silu(OM.proj(n, wg).float()).to(BF) * OM.proj(n, wu), wd)

    m = t.mlp(d(h).view(1, 1, -1), d(gp), d(authored(wg)), d(authored(wu)), d(authored(wd)))
    assert_close("mlp", m.view(-1), mlp_ref(h))
    hl, _, _ = t.decoder_layer(*args, d(gp), d(authored(wg)), d(authored(wu)), d(authored(wd)),
                               d(alpha).view(1, 1, 1))
    h1 = h + (o_ref * alpha)
    assert_close("decoder_layer", hl.view(-1), h1 + mlp_ref(h1) * alpha)


# ------------------------------------------------------------------ prefill layer
@pytest.mark.gpu
def test_prefill_attention_twin(dev):
    from tilefoundry_amd.prefill import Attention, PrefillConfig, rope_tables

    cfg = OP.PrefillConfig()
    N = 256
    lay = OP.random_layer(cfg, seed=60)
    hn = randn(N, cfg.hidden, seed=61)
    hidden = randn(N, cfg.hidden, seed=62)
    cos, sin = OP.rope_tables(N, cfg)
    c2, s2 = rope_tables(N, PrefillConfig())
    assert_equal("rope cos", c2, cos)
    assert_equal("rope sin", s2, sin)
    d = lambda t: t.to(dev)  # noqa: E731
    at = Attention()
    q, gate, k, v = at.qkv(d(hn).unsqueeze(0), d(cos), d(sin), d(lay["w_q"]), d(lay["w_k"]),
                           d(lay["w_v"]), d(lay["gamma_q"]), d(lay["gamma_k"]))
    rq, rg, rk, rv = OP.qkv(hn, lay["w_q"], lay["w_k"], lay["w_v"], lay["gamma_q"], lay["gamma_k"],
                            cos, sin, cfg)
    assert q.shape == (1, N, cfg.heads, cfg.head_dim) and k.shape == (1, N, cfg.kv_heads, cfg.head_dim)
    assert_close("qkv.q", q[0], rq)
    assert_close("qkv.gate", gate[0], rg)
    assert_close("qkv.k", k[0], rk)
    assert_close("qkv.v", v[0], rv)
    att = at.attention(q, k, v, gate)
    qc, kc_, vc_, gc = (t[0].cpu() for t in (q, k, v, gate))
    ref = OP.attention(qc, kc_, vc_, gc, cfg)
    assert_close("attention", att[0], ref)
    out = at.o_proj(att, d(hidden).unsqueeze(0), d(lay["w_o"]))
    assert_close("o_proj", out[0], OP.o_proj(att[0].cpu(), hidden, lay["w_o"]))
