"""The Qwen3 decode kernels as per-op factories, under the reference's names.

Mirrors examples/qwen3_1_7b-tilelang/fast/kernels.py: each factory takes the
same static dimensions and tile arguments as the reference's and returns a
cached callable ``(inputs..., outputs...)`` that writes caller-owned outputs on
torch's current stream. The step position and the cache write slot are
one-element device ``int32`` tensors (``Pos``, ``Wr``), so a sequence of calls
can be captured once as a HIP graph and replayed for every step.

Departures, each forced by the hardware or stated for the caller:

* **Weight layout.** Matrices are read in the checkpoint's ``(out, in)`` =
  ``[N, K]`` layout, the one a row-per-wave GEMV on gfx950 streams; the
  reference's TileLang engine stores ``[K, N]`` (its ``hf_alias`` transposes).
  A ``[K, N]`` matrix is refused with ``ValueError`` rather than silently
  transposed (``K != N``; a square matrix cannot be told apart -- pass
  ``(out, in)``).
* **Tile arguments** (``BN``, ``BK``, ``threads``, ``stages``) size the
  reference's TileLang kernels. The gfx950 kernels pick their own tiling, so
  these are checked to be positive and otherwise not used. ``SK`` keeps its
  meaning: a partial buffer ``P[SK, N]`` holds split ``s``'s dot over the
  ``s``-th contiguous ``K / SK`` slice, and consumers sum the splits in order.
* **Workspaces.** ``gemv_attn_combine`` and ``gemv_silu`` are two launches here
  (merge / activation, then the GEMV) through an intermediate bf16 vector
  (``HQ * D`` or ``I`` elements). The caller may own it -- ``workspace=`` on the
  call, then nothing allocates -- or leave it to the callable, which allocates
  one buffer per device on that device's first call and keeps it (so the first
  call must not be the one under graph capture; ``callable.reserve(device)``
  allocates it ahead).
* **Block winners.** ``lm_head`` returns ``(kernel, NB)`` like the reference,
  with ``NB`` the gfx950 head's own count of 16-row blocks.

Errors: ``ValueError`` for a shape, dtype, layout or argument the kernel cannot
take (the reference's checks happen inside TileLang), ``RuntimeError`` for a
refused launch. No call synchronises.
"""
from __future__ import annotations

from functools import lru_cache

import torch

from ._lib import C

__all__ = [
    "rms_norm", "resid_rms_norm", "gemv", "gemv_attn_combine", "gemv_silu", "lm_head",
    "qk_rope_cache", "attn_partial", "attn_combine", "silu_mul", "embed", "sample_step",
]


def _positive(**kw):
    for k, v in kw.items():
        if int(v) <= 0:
            raise ValueError(f"{k}={v} must be positive")


def _weight(w: torch.Tensor, n: int, k: int, name: str = "W") -> torch.Tensor:
    """``w`` as the ``[n, k]`` (out, in) matrix the kernels read."""
    if w.dim() == 2 and tuple(w.shape) == (n, k):
        return w
    if w.dim() == 2 and tuple(w.shape) == (k, n):
        raise ValueError(
            f"{name}: got the [K, N] = [{k}, {n}] layout; these kernels read the checkpoint's "
            f"(out, in) = [{n}, {k}] layout (transpose once, e.g. w.t().contiguous())")
    raise ValueError(f"{name}: expected shape ({n}, {k}), got {tuple(w.shape)}")


def _partials(P: torch.Tensor, sk: int, n: int, name: str = "P") -> None:
    if P.dtype != torch.float32 or P.numel() != sk * n:
        raise ValueError(f"{name}: expected float32 ({sk}, {n}), got {P.dtype} {tuple(P.shape)}")


class _Workspace:
    """One buffer per device, allocated on first use and kept -- or the
    caller's own (``given``), checked and used as is."""

    def __init__(self, n: int, dtype: torch.dtype):
        self.n, self.dtype, self.bufs = n, dtype, {}

    def get(self, device: torch.device, given: torch.Tensor | None = None) -> torch.Tensor:
        if given is not None:
            if given.dtype != self.dtype or given.numel() != self.n or not given.is_contiguous() \
                    or given.device != torch.device(device):
                raise ValueError(f"workspace: expected a contiguous {self.dtype} tensor of {self.n} elements "
                                 f"on {device}, got {given.dtype} {tuple(given.shape)} on {given.device}")
            return given
        buf = self.bufs.get(device)
        if buf is None:
            buf = torch.empty(self.n, device=device, dtype=self.dtype)
            self.bufs[device] = buf
        return buf


def _split_gemv(x: torch.Tensor, w: torch.Tensor, P: torch.Tensor, sk: int) -> None:
    """``P[s] = x[slice s] . W[:, slice s]^T`` on the skinny MFMA kernel (one token row)."""
    n, k = w.shape
    if k % (256 * sk):
        raise ValueError(f"K={k} must be a multiple of 256 * SK = {256 * sk}")
    C.skinny_gemm(x.view(1, k), w, sk, 0, P.view(sk, 1, n), None, None, None, None)


# ---------------------------------------------------------------------- norms
@lru_cache(maxsize=None)
def rms_norm(H: int, eps: float, threads: int = 256):
    """``Xn = bf16(bf16(x * rsqrt(mean(x^2) + eps)) * gamma)`` (kernels.py:58-79)."""
    _positive(H=H, threads=threads)

    def main(X, G, Xn):
        C.rms_norm(X, G, Xn, float(eps), 0)

    return main


@lru_cache(maxsize=None)
def resid_rms_norm(H: int, SK: int, eps: float, threads: int = 256):
    """``Hout = bf16(A + bf16(sum_s P[s]))``; ``Xn = norm(Hout) * gamma`` (kernels.py:82-116)."""
    _positive(H=H, SK=SK, threads=threads)

    def main(A, P, G, Hout, Xn):
        _partials(P, SK, H)
        C.resid_rms_norm_partials(A, P, G, Hout, Xn, float(eps))

    return main


# ----------------------------------------------------------------------- GEMV
@lru_cache(maxsize=None)
def gemv(K: int, N: int, BN: int, BK: int, SK: int, threads: int, stages: int = 3):
    """``P[s, n] = sum_k X[k] W[n, k]`` over split ``s``'s share of ``K`` (kernels.py:123-145)."""
    _positive(K=K, N=N, BN=BN, BK=BK, SK=SK, threads=threads, stages=stages)

    def main(X, W, P):
        _partials(P, SK, N)
        _split_gemv(X, _weight(W, N, K), P, SK)

    return main


@lru_cache(maxsize=None)
def gemv_attn_combine(HQ: int, D: int, N: int, BN: int, BK: int, SK: int, NS: int,
                      threads: int, stages: int = 3):
    """``o_proj`` of the merged attention splits (kernels.py:154-207): the
    ``NS`` partials ``(Op, Mp, Lp)`` merged against their joint max into a bf16
    head-major vector, then split-K partials ``P[SK, N]`` of its product with
    ``W [N, HQ * D]``."""
    _positive(HQ=HQ, D=D, N=N, BN=BN, BK=BK, SK=SK, NS=NS, threads=threads, stages=stages)
    K = HQ * D
    ws = _Workspace(K, torch.bfloat16)

    def main(Op, Mp, Lp, W, P, workspace=None):
        if Op.numel() != NS * HQ * D or Mp.numel() != NS * HQ or Lp.numel() != NS * HQ:
            raise ValueError(f"Op / Mp / Lp: expected ({NS}, {HQ}, {D}) / ({NS}, {HQ})")
        _partials(P, SK, N)
        w = _weight(W, N, K)
        attn = ws.get(Op.device, workspace)
        C.attn_combine(Op.view(NS, HQ, D), Mp.view(NS, HQ), Lp.view(NS, HQ), attn, None, 0)
        _split_gemv(attn, w, P, SK)

    main.reserve = ws.get
    return main


@lru_cache(maxsize=None)
def gemv_silu(I: int, N: int, BN: int, BK: int, SK: int, SKG: int, threads: int,
              stages: int = 3):
    """``down_proj`` of ``silu(gate) * up`` (kernels.py:210-257): ``GU[SKG, 2I]``
    holds the gate|up projection's partials (gate in ``[0, I)``, up in
    ``[I, 2I)``); the activation ``bf16(bf16(silu(bf16 g)) * bf16 u)`` is formed
    once, then ``P[SK, N]`` are the partials of its product with ``W [N, I]``."""
    _positive(I=I, N=N, BN=BN, BK=BK, SK=SK, SKG=SKG, threads=threads, stages=stages)
    ws = _Workspace(I, torch.bfloat16)

    def main(GU, W, P, workspace=None):
        _partials(GU, SKG, 2 * I, "GU")
        _partials(P, SK, N)
        w = _weight(W, N, I)
        act = ws.get(GU.device, workspace)
        C.silu_mul(GU.view(SKG, 2 * I), act)
        _split_gemv(act, w, P, SK)

    main.reserve = ws.get
    return main


@lru_cache(maxsize=None)
def lm_head(K: int, N: int, BN: int, BK: int, threads: int, stages: int = 3):
    """f32 logits ``O = X . W^T`` and each block's best ``(value, lowest index)``
    into ``Bv`` / ``Bi`` (kernels.py:260-321). Returns ``(kernel, NB)``."""
    _positive(K=K, N=N, BN=BN, BK=BK, threads=threads, stages=stages)
    nb = int(C.lm_head_blocks(N))

    def main(X, W, O, Bv, Bi):
        C.lm_head_argmax(X, None, 0.0, _weight(W, N, K), O, Bv, Bi)

    return main, nb


# ------------------------------------------------------------------ attention
@lru_cache(maxsize=None)
def qk_rope_cache(HQ: int, HKV: int, D: int, MP: int, CAP: int, SK: int, eps: float):
    """Reduce the fused ``[q | k | v]`` partials ``P[SK, (HQ + 2 HKV) D]``; per
    head Qwen3RMSNorm + rotate-half RoPE at ``Pos``; the query to ``Q``, the key
    and value into cache row ``Wr`` (kernels.py:328-411). ``1/sqrt(D)`` is not
    applied here (``attn_partial`` scales the f32 dot)."""
    _positive(HQ=HQ, HKV=HKV, D=D, MP=MP, CAP=CAP, SK=SK)
    if D != 128:
        raise ValueError(f"D={D}: the gfx950 decode kernels take head_dim 128")
    rows = (HQ + 2 * HKV) * D

    def main(P, Gq, Gk, Cos, Sin, Pos, Wr, Kc, Vc, Q):
        _partials(P, SK, rows)
        if Cos.shape != (MP, D) or Kc.numel() != CAP * HKV * D:
            raise ValueError(f"Cos / Kc: expected ({MP}, {D}) / ({CAP}, {HKV * D})")
        C.qk_rope_cache(P, Gq, Gk, float(eps), Cos, Sin, Pos, Wr, Kc, Vc, Q, HQ, HKV, None)

    return main


@lru_cache(maxsize=None)
def attn_partial(HQ: int, HKV: int, D: int, CAP: int, SS: int, scale: float, threads: int = 128):
    """One split's ``(max, sum, weighted values)`` over its ``SS`` slots of the
    context ``0..Pos`` (kernels.py:418-501): f32 scores scaled after the dot,
    f32 softmax against the split's max, bf16 weights into ``P.V``; splits past
    the context write the neutral partial ``(0, -1e30, 0)``. ``SS`` is 32, 64, 128 or
    256 and divides ``CAP``."""
    _positive(HQ=HQ, HKV=HKV, D=D, CAP=CAP, SS=SS, threads=threads)
    if SS not in (32, 64, 128, 256) or CAP % SS:
        raise ValueError(f"SS={SS} must be 32, 64, 128 or 256 and divide CAP={CAP}")
    if D != 128:
        raise ValueError(f"D={D}: the gfx950 decode kernels take head_dim 128")

    def main(Q, Kc, Vc, Pos, Op, Mp, Lp):
        if Kc.numel() != CAP * HKV * D:
            raise ValueError(f"Kc: expected ({CAP}, {HKV * D})")
        C.decode_attention(Q, None, None, None, 0.0, None, None, Kc, Vc, None, Pos, HQ, HKV, SS,
                           float(scale), Op, Mp, Lp, True, None)

    return main


@lru_cache(maxsize=None)
def attn_combine(HQ: int, D: int, CAP: int, SS: int):
    """Merge the ``CAP / SS`` splits against their joint max into bf16
    head-major ``O[HQ * D]`` (kernels.py:504-540)."""
    _positive(HQ=HQ, D=D, CAP=CAP, SS=SS)
    ns = (CAP + SS - 1) // SS

    def main(Op, Mp, Lp, O):
        if Mp.numel() != ns * HQ:
            raise ValueError(f"Mp: expected ({ns}, {HQ})")
        C.attn_combine(Op.view(ns, HQ, D), Mp.view(ns, HQ), Lp.view(ns, HQ), O, None, 0)

    return main


# -------------------------------------------------------- activation, sampling
@lru_cache(maxsize=None)
def silu_mul(I: int, SK: int, BN: int = 256, threads: int = 256):
    """``O = bf16(bf16(silu(bf16 g)) * bf16 u)`` from the gate|up partials
    ``P[SK, 2I]`` (kernels.py:547-572)."""
    _positive(I=I, SK=SK, BN=BN, threads=threads)

    def main(P, O):
        _partials(P, SK, 2 * I)
        C.silu_mul(P.view(SK, 2 * I), O)

    return main


@lru_cache(maxsize=None)
def embed(V: int, H: int, threads: int = 256):
    """``O = Tbl[Ids[0]]`` (kernels.py:579-588)."""
    _positive(V=V, H=H, threads=threads)

    def main(Tbl, Ids, O):
        if tuple(Tbl.shape) != (V, H):
            raise ValueError(f"Tbl: expected ({V}, {H}), got {tuple(Tbl.shape)}")
        C.embed(Tbl, Ids, O, None, None)

    return main


@lru_cache(maxsize=None)
def sample_step(NB: int, NSTEPS: int, threads: int = 256):
    """Greedy pick over the ``NB`` block winners (lowest index on ties), recorded
    at ``Sam[Pos]``; ``Ids`` gets the next prompt token while the prompt lasts,
    else the pick; ``Pos += 1`` (kernels.py:591-637)."""
    _positive(NB=NB, NSTEPS=NSTEPS, threads=threads)

    def main(Bv, Bi, Inp, PromptLen, Ids, Pos, Sam):
        if Bv.numel() != NB or Inp.numel() != NSTEPS:
            raise ValueError(f"Bv / Inp: expected {NB} / {NSTEPS} entries")
        C.sample_step(Bv, Bi, Inp, PromptLen, Ids, Pos, Sam, None)

    return main
