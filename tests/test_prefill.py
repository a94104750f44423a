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
