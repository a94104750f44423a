"""Parity at the workloads' full sizes, where the oracle cannot run the whole
output in seconds: sampled rows / heads against the oracle, plus the
size-independent properties (causal-prefix invariance, untouched cache rows).

* causal prefill attention at 8192 tokens (24 / 4 heads, head_dim 256);
* the qkv projection with the per-head (1+gamma) norm and partial RoPE at
  1024 / 4096 / 8192 tokens;
* o_proj + residual at 4096 / 8192 tokens;
* one Qwen3-1.7B-shaped decode layer in the engine's fused form, writing slot
  4095 of a 4096-slot cache and attending all 4096 positions.
"""
import pytest
import torch

from oracle import norms as ON
from oracle import prefill as OP
from oracle import qwen3 as OQ
from tests._check import assert_close, assert_equal, rel_l2

BF = torch.bfloat16
CFG = OP.PrefillConfig()
HQ, HKV, D = CFG.heads, CFG.kv_heads, CFG.head_dim


def _rows(n, seed, extra=12):
    """First, last, both sides of the midpoint and of every 1024 boundary, plus random rows."""
    g = torch.Generator().manual_seed(seed)
    fixed = {0, 1, 2, n // 2 - 1, n // 2, n - 2, n - 1}
    fixed |= {b + d for b in range(1024, n, 1024) for d in (-1, 0)}
    fixed |= set(torch.randint(0, n, (extra,), generator=g).tolist())
    return sorted(fixed)


@pytest.mark.gpu
def test_prefill_attention_8192(dev):
    """8192 tokens: sampled rows of three heads (one per kv-group edge) against
    the oracle, and rows before 4096 bit-identical when every later row changes."""
    from tilefoundry_amd._lib import C

    n = 8192
    g = torch.Generator().manual_seed(81)
    q, gate = (torch.randn(n, HQ, D, generator=g).to(BF) for _ in range(2))
    k, v = (torch.randn(n, HKV, D, generator=g).to(BF) for _ in range(2))
    qd, kd, vd, gd = (t.to(dev) for t in (q, k, v, gate))
    out = torch.empty(n, HQ * D, dtype=BF, device=dev)
    C.prefill_attention(qd, kd, vd, gd, out, CFG.scale)
    got = out.cpu().view(n, HQ, D)
    rows, heads = _rows(n, 82), [0, 11, 23]
    ref = OP.attention_rows(q, k, v, gate, rows, heads, CFG)
    assert_close("sampled rows", got[rows][:, heads], ref)
    assert rel_l2(got[rows][:, heads], ref) < 5e-3
    # causal prefix: change rows 4096.. of q, k, v and the gate
    for t in (qd, kd, vd, gd):
        t[4096:] = torch.randn(t[4096:].shape, device=dev, generator=torch.Generator(device=dev).manual_seed(83)).to(BF)
    out2 = torch.empty_like(out)
    C.prefill_attention(qd, kd, vd, gd, out2, CFG.scale)
    assert_equal("rows before 4096", out2[:4096], out[:4096])
    assert not torch.equal(out2[4096:], out[4096:])


def _pack_qkv(w):
    wq = w["w_q"].view(HQ, 2 * D, CFG.hidden)
    return torch.cat([wq.reshape(-1, CFG.hidden), w["w_k"], w["w_v"]], 0).contiguous()


@pytest.mark.gpu
@pytest.mark.parametrize("n", [1024, 4096, 8192])
def test_qkv_norm_rope_full_lengths(dev, n):
    """The packed [q | gate] x 24, k x 4, v x 4 projection with the head norms and
    the 64-dim RoPE, at every prompt length: sampled rows (each at its own
    position) against the oracle."""
    from tilefoundry_amd._lib import C

    w = OP.random_layer(CFG, seed=n)
    g = torch.Generator().manual_seed(n + 1)
    hn = torch.randn(n, CFG.hidden, generator=g).to(BF)
    cos, sin = OP.rope_tables(n, CFG)
    W = (2 * HQ + 2 * HKV) * D
    out = torch.empty(n, W, dtype=BF, device=dev)
    C.qkv_norm_rope(hn.to(dev), _pack_qkv(w).to(dev), out, HQ, HKV, w["gamma_q"].to(dev), w["gamma_k"].to(dev),
                    CFG.eps, cos.to(dev), sin.to(dev))
    rows = _rows(n, n + 2)
    q, gate, k, v = OP.qkv(hn[rows], w["w_q"], w["w_k"], w["w_v"], w["gamma_q"], w["gamma_k"], cos[rows],
                           sin[rows], CFG)
    o = out[rows].cpu()
    m = len(rows)
    qg = o[:, : HQ * 2 * D].view(m, HQ, 2 * D)
    assert_close("q", qg[..., :D], q)
    assert_close("gate", qg[..., D:], gate)
    assert_close("k", o[:, HQ * 2 * D: HQ * 2 * D + HKV * D].view(m, HKV, D), k)
    assert_close("v", o[:, HQ * 2 * D + HKV * D:].view(m, HKV, D), v)
    frac = float((qg[..., :D] != q).float().mean())
    assert frac < 0.05, f"{frac:.3%} of q differs from the oracle"


@pytest.mark.gpu
@pytest.mark.parametrize("n", [4096, 8192])
def test_o_proj_residual_full_lengths(dev, n):
    """``bf16(hidden + bf16(gated @ W_o^T))`` over [n, 6144] x [5120, 6144]: sampled
    rows against the oracle, and the share of outputs that differ at all."""
    from tilefoundry_amd._lib import C

    g = torch.Generator().manual_seed(n + 3)
    gated = torch.randn(n, HQ * D, generator=g).to(BF)
    hidden = torch.randn(n, CFG.hidden, generator=g).to(BF)
    w_o = (0.02 * torch.randn(CFG.hidden, HQ * D, generator=g)).to(BF)
    out = torch.empty(n, CFG.hidden, dtype=BF, device=dev)
    C.gemm_nt(gated.to(dev), w_o.to(dev), out, hidden.to(dev))
    rows = _rows(n, n + 4, extra=48)
    ref = OP.o_proj(gated[rows], hidden[rows], w_o)
    got = out[rows].cpu()
    assert_close("o_proj + residual", got, ref)
    frac = float((got != ref).float().mean())
    assert frac < 0.02, f"{frac:.3%} of outputs differ from the oracle"
    branch = got.float() - hidden[rows].float()
    assert rel_l2(branch, ref.float() - hidden[rows].float()) < 0.1


@pytest.mark.gpu
def test_decode_layer_fused_at_slot_4095(dev):
    """The engine's six launches for one layer (input norm + q|k|v with v into the
    cache; head norms + RoPE + K write + split attention; merge; o_proj +
    residual; post norm + gate|up + SwiGLU; down + residual) at position 4095
    of a 4096-slot cache holding 4095 random rows, against the oracle's
    ``decoder_layer``: the layer output, the K and V rows written at 4095, and
    every other cache row untouched."""
    from tilefoundry_amd._lib import C
    from tilefoundry_amd.qwen3 import Qwen3Config, hf_names, pack_weights, rope_tables, synthetic_weights

    cfg = Qwen3Config(layers=1)
    wts = synthetic_weights(cfg, seed=44)
    _, _, layers, _ = pack_weights(cfg, {**wts, "model.embed_tokens.weight": torch.zeros(1, cfg.hidden),
                                         "model.norm.weight": torch.ones(cfg.hidden)}, dev)
    w = layers[0]
    H, HQ_, HKV_, D_ = cfg.hidden, cfg.heads, cfg.kv_heads, cfg.head_dim
    cap, wr, split = 4096, 4095, 64
    g = torch.Generator().manual_seed(45)
    kc = torch.zeros(cap, HKV_ * D_, dtype=BF)
    vc = torch.zeros(cap, HKV_ * D_, dtype=BF)
    kc[:wr] = torch.randn(wr, HKV_ * D_, generator=g).to(BF)
    vc[:wr] = torch.randn(wr, HKV_ * D_, generator=g).to(BF)
    h = torch.randn(H, generator=g).to(BF)
    cos, sin = rope_tables(cap, D_, cfg.rope_theta, dev)
    kd, vd, hd = kc.to(dev), vc.to(dev), h.to(dev)
    pos = torch.tensor([wr], dtype=torch.int32, device=dev)
    ns = cap // split
    op = torch.empty(ns, HQ_, D_, device=dev)
    mp = torch.empty(ns, HQ_, device=dev)
    lp = torch.empty(ns, HQ_, device=dev)
    nqk = (HQ_ + HKV_) * D_
    qk = torch.empty(nqk, dtype=BF, device=dev)
    attn = torch.empty(HQ_ * D_, dtype=BF, device=dev)
    h1 = torch.empty(H, dtype=BF, device=dev)
    act = torch.empty(cfg.inter, dtype=BF, device=dev)
    err = torch.zeros(1, dtype=torch.int32, device=dev)
    C.decode_qkv(hd, None, None, None, w["gamma_in"], cfg.eps, w["w_qkv"], nqk, qk, pos, vd, err)
    C.decode_attention(qk, None, w["gamma_q"], w["gamma_k"], cfg.eps, cos, sin, kd, vd, pos, pos, HQ_, HKV_,
                       split, cfg.scale, op, mp, lp, False, err)
    C.attn_combine(op, mp, lp, attn, pos, split)
    C.gemv_residual(attn, w["w_o"], hd, None, h1)
    C.rmsnorm_gemv_swiglu(h1, w["gamma_post"], cfg.eps, w["w_gu"], act)
    C.gemv_residual(act, w["w_down"], h1, None, hd)
    torch.cuda.synchronize()
    assert int(err.item()) == 0

    lw = OQ.LayerWeights(**{k: wts[v] for k, v in hf_names(0).items()})
    ocfg = OQ.Qwen3Config(layers=1)
    ocos, osin = OQ.rope_tables(cap, ocfg.head_dim, ocfg.rope_theta)
    ref, k_new, v_new = OQ.decoder_layer(h, lw, ocfg, ocos[wr], osin[wr], kc[:wr].view(wr, HKV_, D_),
                                         vc[:wr].view(wr, HKV_, D_), p_bf16=True)
    assert_close("layer output", hd, ref)
    assert_close("k written at 4095", kd[wr].view(HKV_, D_), k_new)
    assert_close("v written at 4095", vd[wr].view(HKV_, D_), v_new)
    assert_equal("k rows 0..4094 untouched", kd[:wr], kc[:wr])
    assert_equal("v rows 0..4094 untouched", vd[:wr], vc[:wr])
    # the attention itself, isolated: the merged output against the oracle's
    xn = ON.rms_norm_q(h, lw.gamma_in, ocfg.eps)
    qr = OQ.rope(OQ.head_norm(OQ.proj(xn, lw.w_q).view(HQ_, D_), lw.gamma_q, ocfg.eps), ocos[wr], osin[wr])
    kk = torch.cat([kc[:wr].view(wr, HKV_, D_), k_new.unsqueeze(0)])
    vv = torch.cat([vc[:wr].view(wr, HKV_, D_), v_new.unsqueeze(0)])
    assert_close("attention over 4096 positions", attn, OQ.attend(qr, kk, vv, ocfg.scale, p_bf16=True))
