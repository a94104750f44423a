"""RMSNorm family on the GPU against the CPU oracle (config: fused add+RMSNorm,
x / residual bf16 [4096, 2048] ~N(0,1), gamma ~N(1, 0.1), eps 1e-6)."""
import pytest
import torch

from oracle import norms as O
from tests._check import assert_close, assert_equal, assert_ulps

BF = torch.bfloat16


def _draw(rows, hidden, seed=0):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(rows, hidden, generator=g).to(BF)
    r = torch.randn(rows, hidden, generator=g).to(BF)
    gamma = (1.0 + 0.1 * torch.randn(hidden, generator=g)).to(BF)
    return x, r, gamma


@pytest.mark.gpu
@pytest.mark.parametrize("rows,hidden,mode", [
    (4096, 2048, 0),   # the fused add+RMSNorm workload
    (1, 2048, 0), (3, 2560, 0), (7, 128, 0), (5, 5120, 1), (2, 8, 0), (33, 8192, 1),
])
def test_add_rms_norm(dev, rows, hidden, mode):
    from tilefoundry_amd import ops

    x, r, gamma = _draw(rows, hidden)
    y_ref, r_ref = O.add_rms_norm(x, r, gamma, 1e-6, mode)
    y, r_out = ops.add_rms_norm(x.to(dev), r.to(dev), gamma.to(dev), 1e-6, mode=mode)
    assert_equal("residual_out", r_out, r_ref)
    # The landed sum is bit exact. The norm differs from the CPU only where the
    # f32 sum of squares rounds differently: that moves bf16(x*r) by one step,
    # which the multiply by gamma can widen to two.
    assert_ulps("normed", y, y_ref, max_ulps=2, max_frac=1e-3)
    assert_close("normed", y, y_ref)


@pytest.mark.gpu
def test_add_rms_norm_in_place(dev):
    from tilefoundry_amd import ops

    x, r, gamma = _draw(64, 2048, seed=3)
    y_ref, r_ref = O.add_rms_norm(x, r, gamma, 1e-6)
    xd, rd = x.to(dev), r.to(dev)
    ops.add_rms_norm(xd, rd, gamma.to(dev), 1e-6, out=xd, residual_out=rd)
    assert_equal("residual in place", rd, r_ref)
    assert_ulps("normed in place", xd, y_ref, max_ulps=2, max_frac=1e-3)


@pytest.mark.gpu
@pytest.mark.parametrize("rows,hidden,mode", [(1, 2048, 0), (16, 2560, 0), (9, 5120, 1), (0, 2048, 0)])
def test_rms_norm(dev, rows, hidden, mode):
    from tilefoundry_amd import ops

    x, _, gamma = _draw(rows, hidden, seed=1)
    ref = O.rms_norm(x, gamma, 1e-6, mode)
    got = ops.rms_norm(x.to(dev), gamma.to(dev), 1e-6, mode=mode)
    assert_ulps("rms_norm", got, ref, max_ulps=2, max_frac=1e-3)


@pytest.mark.gpu
def test_rms_norm_constant_rows(dev):
    """A constant row normalises to its sign exactly: y == sign(c) * gamma."""
    from tilefoundry_amd import ops

    H = 2048
    c = torch.tensor([0.5, -3.0, 7.25, -0.125]).to(BF)
    x = c[:, None].expand(4, H).contiguous()
    gamma = torch.linspace(-2, 2, H).to(BF)
    got = ops.rms_norm(x.to(dev), gamma.to(dev), 1e-6).cpu()
    assert_equal("constant rows", got, (torch.sign(c.float())[:, None] * gamma.float()).to(BF))


@pytest.mark.gpu
def test_resid_rms_norm_partials(dev):
    from tilefoundry_amd import ops

    H, SK = 2048, 8
    g = torch.Generator().manual_seed(0)
    a = torch.randn(H, generator=g).to(BF)
    p = torch.randn(SK, H, generator=g)
    gamma = torch.randn(H, generator=g).to(BF)
    h_ref, xn_ref = O.resid_rms_norm(a, p, gamma, 1e-6)
    h, xn = ops.resid_rms_norm(a.to(dev), p.to(dev), gamma.to(dev), 1e-6)
    # The 8-way f32 sum may round differently from torch's, by one bf16 step.
    assert_ulps("Hout", h, h_ref, max_ulps=1, max_frac=1e-2)
    assert_close("Xn", xn, xn_ref)
