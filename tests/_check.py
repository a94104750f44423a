"""Comparison helpers: the reference's own tolerance measures, plus exact and
ulp-level checks for the outputs that must agree bit for bit.

``max_rel`` and ``cosine`` follow examples/qwen3_1_7b-tilelang/fast/test_kernels.py:18-29
(``report``): ``max|got - ref| / max|ref|`` and the cosine similarity of the
flattened tensors.
"""
from __future__ import annotations

import torch

#: bf16 tolerance every floating-point kernel is held to (max |d| / max |ref|).
BF16_RTOL = 1e-2


def max_rel(got: torch.Tensor, ref: torch.Tensor) -> float:
    g, r = got.detach().float().cpu(), ref.detach().float().cpu()
    scale = r.abs().max().clamp(min=1e-6)
    return float((g - r).abs().max() / scale)


def cosine(got: torch.Tensor, ref: torch.Tensor) -> float:
    g, r = got.detach().float().cpu().flatten(), ref.detach().float().cpu().flatten()
    if g.numel() == 0:
        return 1.0
    return float(torch.nn.functional.cosine_similarity(g, r, dim=0))


def rel_l2(got: torch.Tensor, ref: torch.Tensor) -> float:
    g, r = got.detach().double().cpu(), ref.detach().double().cpu()
    return float((g - r).norm() / r.norm().clamp(min=1e-30))


def assert_l2(name: str, got, ref, tol: float = 1e-2, cos_tol: float = 1e-4):
    """Whole-tensor agreement for states that passed through many landings."""
    assert got.shape == ref.shape, f"{name}: shape {tuple(got.shape)} != {tuple(ref.shape)}"
    e, c = rel_l2(got, ref), cosine(got, ref)
    assert e <= tol and c >= 1 - cos_tol, f"{name}: rel_l2={e:.3g} cosine={c:.6f}"


def assert_close(name: str, got, ref, rtol: float = BF16_RTOL, cos_tol: float = 1e-3):
    assert got.shape == ref.shape, f"{name}: shape {tuple(got.shape)} != {tuple(ref.shape)}"
    if got.numel() == 0:
        return
    rel = max_rel(got, ref)
    cos = cosine(got, ref)
    assert rel <= rtol and cos >= 1 - cos_tol, f"{name}: max_rel={rel:.3g} cosine={cos:.6f}"


def bf16_ulps(got: torch.Tensor, ref: torch.Tensor) -> torch.Tensor:
    """Distance in bf16 units-in-the-last-place between two bf16 tensors."""
    def key(t):
        i = t.detach().cpu().to(torch.bfloat16).view(torch.int16).to(torch.int32)
        # map sign-magnitude to a monotone integer line
        return torch.where(i < 0, -(i & 0x7FFF), i)
    return (key(got) - key(ref)).abs()


def assert_ulps(name: str, got, ref, max_ulps: int = 1, max_frac: float = 1.0):
    """Every element within `max_ulps` bf16 ulps; at most `max_frac` of them nonzero."""
    d = bf16_ulps(got, ref)
    worst = int(d.max()) if d.numel() else 0
    frac = float((d > 0).float().mean()) if d.numel() else 0.0
    assert worst <= max_ulps and frac <= max_frac, (
        f"{name}: worst {worst} ulps, {frac:.4%} of elements differ")


def assert_equal(name: str, got, ref):
    g, r = got.detach().cpu(), ref.detach().cpu()
    assert g.shape == r.shape, f"{name}: shape {tuple(g.shape)} != {tuple(r.shape)}"
    if g.dtype == torch.bfloat16:
        g, r = g.view(torch.int16), r.view(torch.int16)
    bad = (g != r)
    assert not bool(bad.any()), f"{name}: {int(bad.sum())} of {g.numel()} elements differ"


def forced_agreement(name: str, picks, gold, gpu_logits, top_ids, top_vals, gaps, floor: int,
                     max_delta=None):
    """Teacher-forced greedy agreement with the oracle, position by position.

    ``picks[i]`` is the GPU's pick at position i when fed the oracle's ids;
    ``gold[i]`` the oracle's; ``gpu_logits[i]`` the GPU's logits there;
    ``top_ids[i]`` / ``top_vals[i]`` the oracle's largest logits and
    ``gaps[i]`` its top-1 / top-2 gap. At each position ``delta`` is the
    largest |GPU - oracle| over those candidates: a pick can only flip where
    the gap is at most ``2 * delta``. Every differing pick must be such a near
    tie and one of the oracle's candidates; the count of equal picks is printed
    and must reach ``floor``. ``max_delta`` (a number, or one per position) is
    an absolute bound every ``delta`` must stay within, so that a regression
    raising the logit error fails instead of widening the set of allowed
    near ties. Returns ``(agree, deltas)``."""
    n = len(gold)
    agree, ties, bad, deltas = 0, 0, [], []
    caps = [max_delta] * n if max_delta is None or isinstance(max_delta, (int, float)) else list(max_delta)
    over = []
    for i in range(n):
        ids = torch.as_tensor(top_ids[i], dtype=torch.int64)
        got = gpu_logits[i].reshape(-1)[ids.to(gpu_logits[i].device)].double().cpu()
        delta = float((got - torch.as_tensor(top_vals[i], dtype=torch.float64)).abs().max())
        deltas.append(delta)
        if caps[i] is not None and delta > caps[i]:
            over.append((i, delta, caps[i]))
        tie = gaps[i] <= 2.0 * delta
        ties += int(tie)
        if picks[i] == gold[i]:
            agree += 1
        elif not tie or picks[i] not in top_ids[i]:
            bad.append((i, picks[i], gold[i], gaps[i], delta))
    print(f"\n[agreement] {name}: {agree}/{n} picks equal the oracle's; {ties} positions are near ties "
          f"under the measured logit error (max |delta| {max(deltas):.4g}, median "
          f"{sorted(deltas)[n // 2]:.4g})", flush=True)
    assert not over, f"{name}: logit error above its absolute bound (pos, delta, bound): {over[:5]}"
    assert not bad, f"{name}: picks differ at clear margins (pos, got, want, gap, delta): {bad[:5]}"
    assert agree >= floor, f"{name}: {agree}/{n} picks agree, below the floor {floor}"
    return agree, deltas


def logit_bounds(logits_list, frac: float = 1e-2):
    """Per-position absolute logit-error bounds: ``frac`` of the oracle's
    largest |logit| at each position (the reference's bf16 bar on logits)."""
    return [frac * float(lg.float().abs().max()) for lg in logits_list]


def oracle_candidates(logits_list, k: int = 16):
    """(top_ids, top_vals, gaps) of a list of oracle logits."""
    ids, vals, gaps = [], [], []
    for lg in logits_list:
        t = torch.topk(lg.float(), k)
        ids.append(t.indices.tolist())
        vals.append([float(v) for v in t.values])
        gaps.append(float(t.values[0] - t.values[1]))
    return ids, vals, gaps
