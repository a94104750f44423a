"""Causal GQA prefill attention (Qwen3.5 layer, head_dim 256, 24 / 4 heads) against
the CPU oracle: small prompts in full, a 1024-token prompt on a subset of heads,
strided views into the packed qkv projection output, and causal-prefix
invariance at the 4096-token size."""
import pytest
import torch

from oracle import prefill as OP
from tests._check import assert_close, assert_equal, rel_l2

BF = torch.bfloat16
CFG = OP.PrefillConfig()
HQ, HKV, D = CFG.heads, CFG.kv_heads, CFG.head_dim


def inputs(n, seed):
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(n, HQ, D, generator=g).to(BF)
    k = torch.randn(n, HKV, D, generator=g).to(BF)
    v = torch.randn(n, HKV, D, generator=g).to(BF)
    gate = torch.randn(n, HQ, D, generator=g).to(BF)
    return q, k, v, gate


def run(dev, q, k, v, gate):
    from tilefoundry_amd._lib import C

    out = torch.empty(q.shape[0], HQ * D, dtype=BF, device=dev)
    C.prefill_attention(q.to(dev), k.to(dev), v.to(dev), gate.to(dev), out, CFG.scale)
    return out


@pytest.mark.gpu
@pytest.mark.parametrize("n", [128, 256])
def test_prefill_attention_small(dev, n):
    q, k, v, gate = inputs(n, n)
    got = run(dev, q, k, v, gate).cpu()
    ref = OP.attention(q, k, v, gate, CFG)
    assert_close("prefill attention", got, ref)
    assert rel_l2(got, ref) < 5e-3


@pytest.mark.gpu
def test_prefill_attention_1024_subset(dev):
    n = 1024
    q, k, v, gate = inputs(n, 7)
    got = run(dev, q, k, v, gate).cpu().view(n, HQ, D)
    heads = [0, 5, 6, 17, 23]
    ref = OP.attention(q, k, v, gate, CFG, heads=heads).view(n, len(heads), D)
    for i, h in enumerate(heads):
        assert_close(f"head {h}", got[:, h], ref[:, i])


@pytest.mark.gpu
def test_prefill_attention_2048_sampled_rows(dev):
    """2048 tokens, 24 / 4 heads: still the 128-row blocks with two key groups
    (their shared query rows staged once through LDS), 16 query tiles per
    head. Sampled rows -- both ends of every fourth tile and rows at the tile
    and 32-row wave boundaries -- of four heads (both edges of two kv groups)
    against the oracle."""
    n = 2048
    q, k, v, gate = inputs(n, 29)
    got = run(dev, q, k, v, gate).cpu().view(n, HQ, D)
    rows = sorted({r for t in range(0, n // 128, 4) for r in (128 * t, 128 * t + 127)}
                  | {31, 32, 63, 64, 95, 96, 1023, 1024, 1055, 2047})
    heads = [0, 5, 6, 23]
    ref = OP.attention_rows(q, k, v, gate, rows, heads, CFG)
    assert_close("sampled rows", got[rows][:, heads], ref)
    assert rel_l2(got[rows][:, heads], ref) < 5e-3


@pytest.mark.gpu
def test_prefill_attention_reads_packed_qkv(dev):
    """q, gate, k, v as strided views of one [n, 24*512 + 2*4*256] projection
    output (per head [q | gate], then k heads, then v heads)."""
    from tilefoundry_amd._lib import C

    n = 256
    q, k, v, gate = inputs(n, 11)
    packed = torch.cat([torch.stack([q, gate], 2).reshape(n, -1), k.reshape(n, -1), v.reshape(n, -1)], 1)
    pd = packed.to(dev)
    qv = pd[:, : HQ * 2 * D].view(n, HQ, 2 * D)
    kv0 = HQ * 2 * D
    out = torch.empty(n, HQ * D, dtype=BF, device=dev)
    C.prefill_attention(qv[:, :, :D], pd[:, kv0: kv0 + HKV * D].view(n, HKV, D),
                        pd[:, kv0 + HKV * D:].view(n, HKV, D), qv[:, :, D:], out, CFG.scale)
    assert_equal("packed == separate", out, run(dev, q, k, v, gate))


@pytest.mark.gpu
def test_prefill_attention_causal_prefix_4096(dev):
    """Rows before 2048 are bit-identical when every later row changes."""
    n = 4096
    q, k, v, gate = inputs(n, 13)
    q2, k2, v2, gate2 = q.clone(), k.clone(), v.clone(), gate.clone()
    g = torch.Generator().manual_seed(14)
    for t in (q2, k2, v2, gate2):
        t[2048:] = torch.randn(t[2048:].shape, generator=g).to(BF)
    a = run(dev, q, k, v, gate)
    b = run(dev, q2, k2, v2, gate2)
    assert_equal("prefix rows", a[:2048], b[:2048])
    assert not torch.equal(a[2048:].cpu(), b[2048:].cpu())
    # and the last rows of one head against the oracle (rows 4088..4095 attend everything)
    ref = OP.attention(q[:, :1].contiguous(), k[:, :1].contiguous(), v[:, :1].contiguous(), gate[:, :1].contiguous(),
                       OP.PrefillConfig(heads=1, kv_heads=1))
    assert_close("head 0, whole prompt", a.cpu().view(n, HQ, D)[:, 0], ref.view(n, D))


# ------------------------------------------------------------------ projections
@pytest.mark.gpu
@pytest.mark.parametrize("M,N,K", [(256, 256, 64), (512, 768, 320), (1024, 5120, 6144)])
def test_gemm_nt(dev, M, N, K):
    """bf16 store against the f32 product (the 128 x 128 tile: small grids)."""
    from tilefoundry_amd._lib import C

    g = torch.Generator().manual_seed(M + N + K)
    a = torch.randn(M, K, generator=g).to(BF)
    b = (0.05 * torch.randn(N, K, generator=g)).to(BF)
    c = torch.empty(M, N, dtype=BF, device=dev)
    C.gemm_nt(a.to(dev), b.to(dev), c, None)
    ref = a.float() @ b.float().t()
    assert_close("gemm", c, ref.to(BF))
    assert rel_l2(c, ref) < 4e-3


@pytest.mark.gpu
def test_gemm_exact_on_integers(dev):
    from tilefoundry_amd._lib import C

    g = torch.Generator().manual_seed(3)
    a = torch.randint(-3, 4, (256, 512), generator=g).to(BF)
    b = torch.randint(-3, 4, (512, 512), generator=g).to(BF)
    c = torch.empty(256, 512, dtype=BF, device=dev)
    C.gemm_nt(a.to(dev), b.to(dev), c, None)
    assert_equal("integer gemm", c, (a.long() @ b.long().t()).float().to(BF))


@pytest.mark.gpu
def test_o_proj_residual(dev):
    from tilefoundry_amd._lib import C

    cfg = OP.PrefillConfig()
    n = 256
    g = torch.Generator().manual_seed(21)
    gated = torch.randn(n, cfg.heads * D, generator=g).to(BF)
    hidden = torch.randn(n, cfg.hidden, generator=g).to(BF)
    w_o = (0.02 * torch.randn(cfg.hidden, cfg.heads * D, generator=g)).to(BF)
    out = torch.empty(n, cfg.hidden, dtype=BF, device=dev)
    C.gemm_nt(gated.to(dev), w_o.to(dev), out, hidden.to(dev))
    ref = OP.o_proj(gated, hidden, w_o)
    assert_close("o_proj + residual", out, ref)
    frac = float((out.cpu() != ref).float().mean())
    assert frac < 0.02, f"{frac:.3%} of outputs differ from the oracle"


@pytest.mark.gpu
@pytest.mark.parametrize("M,N,K", [(512, 768, 320), (37, 2048, 2048), (1024, 12288, 2048), (4096, 4096, 2048)])
def test_gemm_tiles_f32_and_ragged(dev, M, N, K):
    """Each tile shape the launch picks (128 x 128 for small grids, 256 x 256 for
    full rounds) with the f32 store -- including a 37-row ragged edge and a
    gate|up-sized product at 1024 rows -- within an f64 error bound, and the bf16
    store of the same product equal to the f32 sums landed in bf16."""
    from tilefoundry_amd._lib import C

    g = torch.Generator().manual_seed(M + N + K)
    a = torch.randn(M, K, generator=g).to(BF)
    b = (0.05 * torch.randn(N, K, generator=g)).to(BF)
    ad, bd = a.to(dev), b.to(dev)
    f32 = torch.full((M, N), float("nan"), device=dev)
    C.gemm_nt_f32(ad, bd, f32)
    plain = torch.empty(M, N, dtype=BF, device=dev)
    C.gemm_nt(ad, bd, plain, None)
    ref64 = a.double() @ b.double().t()
    bound = K * 2.0 ** -23 * (a.double().abs() @ b.double().abs().t()) + 1e-6
    assert bool(((f32.cpu().double() - ref64).abs() <= bound).all()), "f32 store outside the f64 bound"
    assert_equal("bf16 store == landed f32 sums", plain, f32.to(BF))


def _layer_weights(seed=5):
    return OP.random_layer(CFG, seed=seed)


def _pack_qkv(w):
    wq = w["w_q"].view(HQ, 2 * D, CFG.hidden)
    return torch.cat([wq.reshape(-1, CFG.hidden), w["w_k"], w["w_v"]], 0).contiguous()


@pytest.mark.gpu
def test_qkv_norm_rope(dev):
    from tilefoundry_amd._lib import C

    n = 256
    w = _layer_weights()
    g = torch.Generator().manual_seed(22)
    hn = torch.randn(n, CFG.hidden, generator=g).to(BF)
    cos, sin = OP.rope_tables(n, CFG)
    W = (2 * HQ + 2 * HKV) * D
    out = torch.empty(n, W, dtype=BF, device=dev)
    C.qkv_norm_rope(hn.to(dev), _pack_qkv(w).to(dev), out, HQ, HKV, w["gamma_q"].to(dev), w["gamma_k"].to(dev),
                    CFG.eps, cos.to(dev), sin.to(dev))
    q, gate, k, v = OP.qkv(hn, w["w_q"], w["w_k"], w["w_v"], w["gamma_q"], w["gamma_k"], cos, sin, CFG)
    o = out.cpu()
    qg = o[:, : HQ * 2 * D].view(n, HQ, 2 * D)
    assert_close("q", qg[..., :D], q)
    assert_close("gate", qg[..., D:], gate)
    assert_close("k", o[:, HQ * 2 * D: HQ * 2 * D + HKV * D].view(n, HKV, D), k)
    assert_close("v", o[:, HQ * 2 * D + HKV * D:].view(n, HKV, D), v)
    frac = float((qg[..., :D] != q).float().mean())
    assert frac < 0.05, f"{frac:.3%} of q differs from the oracle"


@pytest.mark.gpu
def test_attention_layer_end_to_end(dev):
    """qkv projection (+ norm / RoPE) -> causal gated attention read in place ->
    o_proj + residual, against the oracle's layer at 256 tokens."""
    from tilefoundry_amd._lib import C

    n = 256
    w = _layer_weights(seed=6)
    g = torch.Generator().manual_seed(23)
    hn = torch.randn(n, CFG.hidden, generator=g).to(BF)
    hidden = torch.randn(n, CFG.hidden, generator=g).to(BF)
    cos, sin = OP.rope_tables(n, CFG)
    W = (2 * HQ + 2 * HKV) * D
    qkv = torch.empty(n, W, dtype=BF, device=dev)
    C.qkv_norm_rope(hn.to(dev), _pack_qkv(w).to(dev), qkv, HQ, HKV, w["gamma_q"].to(dev), w["gamma_k"].to(dev),
                    CFG.eps, cos.to(dev), sin.to(dev))
    qv = qkv[:, : HQ * 2 * D].view(n, HQ, 2 * D)
    k0 = HQ * 2 * D
    attn = torch.empty(n, HQ * D, dtype=BF, device=dev)
    C.prefill_attention(qv[:, :, :D], qkv[:, k0: k0 + HKV * D].view(n, HKV, D),
                        qkv[:, k0 + HKV * D:].view(n, HKV, D), qv[:, :, D:], attn, CFG.scale)
    out = torch.empty(n, CFG.hidden, dtype=BF, device=dev)
    C.gemm_nt(attn, w["w_o"].to(dev), out, hidden.to(dev))
    q, gate, k, v = OP.qkv(hn, w["w_q"], w["w_k"], w["w_v"], w["gamma_q"], w["gamma_k"], cos, sin, CFG)
    ref_attn = OP.attention(q, k, v, gate, CFG)
    assert_close("attention", attn, ref_attn)
    ref = OP.o_proj(ref_attn, hidden, w["w_o"])
    assert_close("layer output", out, ref)
    branch = out.cpu().float() - hidden.float()
    assert rel_l2(branch, ref.float() - hidden.float()) < 0.1


@pytest.mark.gpu
@pytest.mark.parametrize("M,N,K,ks", [(63, 4096, 2048, 8), (63, 2048, 6144, 8), (511, 12288, 2048, 2), (37, 768, 320, 5)])
def test_gemm_f32_split_partials(dev, M, N, K, ks):
    """K split into ks ranges: the partial slices sum (in split order) to the
    product within the f64 bound, each slice is the product over its own K
    range, and the library's own split choice for few rows is > 1 where the
    k-tiles divide."""
    from tilefoundry_amd._lib import C

    g = torch.Generator().manual_seed(M * ks + N)
    a = torch.randn(M, K, generator=g).to(BF)
    b = (0.05 * torch.randn(N, K, generator=g)).to(BF)
    part = torch.full((ks, M, N), float("nan"), device=dev)
    C.gemm_nt_f32(a.to(dev), b.to(dev), part)
    got = part.cpu().double()
    kr = K // ks
    for z in range(ks):
        ref = a[:, z * kr:(z + 1) * kr].double() @ b[:, z * kr:(z + 1) * kr].double().t()
        bound = kr * 2.0 ** -23 * (a[:, z * kr:(z + 1) * kr].double().abs() @ b[:, z * kr:(z + 1) * kr].double().abs().t())
        assert bool(((got[z] - ref).abs() <= bound + 1e-6).all()), f"slice {z}"
    if M < 128 and (K // 64) % 8 == 0:   # few rows, and the k-tiles allow splits
        assert C.gemm_f32_splits(M, N, K) > 1
