"""Per-op functions over the HIP kernels, torch tensors in and out.

Every function writes into caller-owned buffers when ``out=`` (and friends)
are given and allocates them otherwise -- the convention of the reference's
``CompiledModule`` (src/tilefoundry/runtime/module.py:75-142) and of
``examples/minicpm3_4b-cutedsl/kernels/reference_ops.py:24-28`` (``_into``).
A call that passes every output allocates nothing and may be captured in a
HIP graph.
"""
from __future__ import annotations

import torch

from ._lib import C

BF16 = torch.bfloat16


def _out(out, like, shape=None, dtype=None):
    if out is not None:
        return out
    return torch.empty(like.shape if shape is None else shape, device=like.device,
                       dtype=like.dtype if dtype is None else dtype)


def rms_norm(x, gamma, eps: float, out=None, mode: int = 0):
    """RMSNorm over the last axis. mode 0: ``bf16(bf16(x*r)*gamma)`` (Qwen3,
    MiniCPM3); mode 1: ``bf16(x*r*(1+gamma))`` (Qwen3.5)."""
    out = _out(out, x)
    C.rms_norm(x, gamma, out, float(eps), int(mode))
    return out


def add_rms_norm(x, residual, gamma, eps: float, out=None, residual_out=None, mode: int = 0):
    """Fused residual add + RMSNorm; returns ``(normed, bf16(x + residual))``.

    ``residual_out`` may be ``residual`` itself (in-place update)."""
    out = _out(out, x)
    residual_out = _out(residual_out, x)
    C.add_rms_norm(x, residual, gamma, out, residual_out, float(eps), int(mode))
    return out, residual_out


def resid_rms_norm(a, partials, gamma, eps: float, h_out=None, xn=None):
    """``Hout = A + bf16(sum_s P[s])``; ``Xn = rms_norm(Hout)`` for one row."""
    h_out = _out(h_out, a)
    xn = _out(xn, a)
    C.resid_rms_norm_partials(a, partials, gamma, h_out, xn, float(eps))
    return h_out, xn


# --------------------------------------------------------------- decode GEMVs
# Weights are (out, in) = [N, K] row-major (the checkpoint's layout).

def _dev_i32(v, device):
    if isinstance(v, torch.Tensor):
        return v
    return torch.tensor([int(v)], dtype=torch.int32, device=device)


def gemv(x, w, out=None, out_dtype=None):
    """``x @ w.T`` for one row; f32 or bf16 out
    (examples/minicpm3_4b-cutedsl/kernels/reference_ops.py:57-58)."""
    dt = out_dtype or (out.dtype if out is not None else BF16)
    out = _out(out, x, (w.shape[0],), dt)
    C.gemv(x, w, out)
    return out


def rmsnorm_gemv(h, gamma, eps: float, w, out=None):
    """``bf16(rms_norm(h, gamma) @ w.T)``
    (examples/minicpm3_4b-cutedsl/kernels/reference_ops.py:46-48)."""
    out = _out(out, h, (w.shape[0],))
    C.rmsnorm_gemv(h, gamma, float(eps), w, out)
    return out


def gemv_residual(x, w, residual, alpha=None, out=None):
    """``residual + bf16(x @ w.T)`` (``* alpha`` first when given)
    (examples/minicpm3_4b-cutedsl/kernels/reference_ops.py:61-63)."""
    out = _out(out, residual)
    C.gemv_residual(x, w, residual, alpha, out)
    return out


def rmsnorm_gemv_swiglu(h, gamma, eps: float, w_gu, out=None):
    """``bf16(silu(g)) * u`` for ``(g, u)`` the interleaved row pairs of
    ``rms_norm(h) @ w_gu.T`` (examples/minicpm3_4b-cutedsl/kernels/reference_ops.py:66-69)."""
    out = _out(out, h, (w_gu.shape[0] // 2,))
    C.rmsnorm_gemv_swiglu(h, gamma, float(eps), w_gu, out)
    return out


class SampleState:
    """Device-side greedy-loop state: prompt ids, length, next id, position, picks."""

    def __init__(self, nsteps: int, device):
        z = lambda n, dt=torch.int32: torch.zeros(n, dtype=dt, device=device)  # noqa: E731
        self.inp = z(nsteps)
        self.sam = z(nsteps)
        self.plen = z(1)
        self.ids = z(1, torch.int64)
        self.pos = z(1)
        self.err = z(1)


def lm_head_argmax(h, gamma, eps: float, w, logits=None, block_val=None, block_idx=None):
    """f32 logits of ``rms_norm(h) @ w.T`` (``h`` as is when ``gamma`` is None) and
    the per-block winners. Returns ``(logits, block_val, block_idx)``
    (examples/qwen3_1_7b-tilelang/fast/kernels.py:260-321)."""
    V = w.shape[0]
    nb = C.lm_head_blocks(V)
    logits = _out(logits, h, (V,), torch.float32)
    block_val = _out(block_val, h, (nb,), torch.float32)
    block_idx = _out(block_idx, h, (nb,), torch.int32)
    C.lm_head_argmax(h, gamma, float(eps), w, logits, block_val, block_idx)
    return logits, block_val, block_idx


def sample_step(block_val, block_idx, state: SampleState):
    """The greedy step on the device (examples/qwen3_1_7b-tilelang/fast/kernels.py:591-637)."""
    C.sample_step(block_val, block_idx, state.inp, state.plen, state.ids, state.pos, state.sam,
                  state.err)


def greedy_pick(h, gamma, eps: float, w):
    """Logits and their argmax (lowest index on ties), read back to the host."""
    logits, bv, bi = lm_head_argmax(h, gamma, eps, w)
    return logits, int(bi[int(torch.argmax(bv))])


def decode_qkv(h, gamma_in, eps: float, w_qkv, n_qk: int, wr, v_cache, *, table=None,
               token=None, h_copy=None, qk_out=None, err=None):
    """Input norm + fused q|k|v GEMV: raw q|k (bf16 [n_qk]) returned, v written
    into ``v_cache`` row ``wr``. With ``table`` the input row is ``table[token]``
    (copied into ``h_copy``)."""
    dev = gamma_in.device
    qk_out = _out(qk_out, gamma_in, (n_qk,))
    ids = None
    if table is not None:
        ids = token if isinstance(token, torch.Tensor) else torch.tensor([int(token)], dtype=torch.int64, device=dev)
    C.decode_qkv(h, table, ids, h_copy, gamma_in, float(eps), w_qkv, n_qk, qk_out,
                 _dev_i32(wr, dev), v_cache, err)
    return qk_out


def _attn_bufs(q, k_cache, hq, hkv, split):
    cap = k_cache.numel() // (hkv * 128)
    ns = cap // split
    op = torch.empty(ns, hq, 128, dtype=torch.float32, device=q.device)
    mp = torch.empty(ns, hq, dtype=torch.float32, device=q.device)
    lp = torch.empty(ns, hq, dtype=torch.float32, device=q.device)
    return op, mp, lp


def attn_partial(q, k_cache, v_cache, wr, hq: int, hkv: int, split: int = 256,
                 scale: float | None = None, partials=None, rope=None, neutral: bool = True,
                 err=None):
    """Split partials ``(Op [NS,HQ,128], Mp [NS,HQ], Lp [NS,HQ])`` of decode
    attention over cache slots 0..wr (examples/qwen3_1_7b-tilelang/fast/kernels.py:418-501).

    ``rope=None``: ``q`` is the final query and the cache already holds slot wr.
    ``rope=(gamma_q, gamma_k, eps, cos, sin, pos)``: ``q`` is the raw q|k
    projection; the head norm + RoPE happen here and the new key is written to
    ``k_cache[wr]``."""
    dev = q.device
    scale = 128 ** -0.5 if scale is None else scale
    op, mp, lp = partials if partials is not None else _attn_bufs(q, k_cache, hq, hkv, split)
    if rope is None:
        C.decode_attention(q, None, None, None, 0.0, None, None, k_cache, v_cache, None,
                           _dev_i32(wr, dev), hq, hkv, split, float(scale), op, mp, lp,
                           bool(neutral), err)
    else:
        gq, gk, eps, cos, sin, pos = rope
        C.decode_attention(q, None, gq, gk, float(eps), cos, sin, k_cache, v_cache,
                           _dev_i32(pos, dev), _dev_i32(wr, dev), hq, hkv, split, float(scale),
                           op, mp, lp, bool(neutral), err)
    return op, mp, lp


def attn_combine(op, mp, lp, out=None, wr=None, split: int = 0):
    """LSE merge of split partials into bf16 ``[HQ*D]``
    (examples/qwen3_1_7b-tilelang/fast/kernels.py:504-540); with ``wr`` only the
    splits holding slots 0..wr are read."""
    ns, hq = mp.shape
    out = _out(out, op, (op.numel() // ns,), BF16)
    C.attn_combine(op, mp, lp, out, None if wr is None else _dev_i32(wr, op.device), int(split))
    return out


def decode_attention(q, k_cache, v_cache, wr, hq: int, hkv: int, split: int = 64,
                     scale: float | None = None, rope=None, out=None, partials=None, err=None):
    """Decode attention merged to bf16 ``[hq*128]`` (partials + combine)."""
    op, mp, lp = attn_partial(q, k_cache, v_cache, wr, hq, hkv, split, scale, partials, rope,
                              neutral=False, err=err)
    return attn_combine(op, mp, lp, out, wr=wr, split=split)


# ------------------------------------------------------- batched (<= 32 rows)

def skinny_gemm(x, w, epilogue: str = "partial", ks: int = 1, part=None, act=None, logits=None,
                block_val=None, block_idx=None, with_logits: bool = True):
    """``X[m, k] @ W[n, k]^T`` for m <= 32 on bf16 MFMA. ``epilogue``:
    ``"partial"`` -> f32 ``[ks, m, n]`` (sum over ks is the product);
    ``"swiglu"`` -> bf16 ``[m, n/2]`` over interleaved gate/up rows;
    ``"argmax"`` -> ``(logits [m, n] f32 or None, block_val, block_idx)``, the
    per-token best (value, lowest index) of every 16-row group; the logits are
    written only ``with_logits``."""
    m, n = x.shape[0], w.shape[0]
    if epilogue == "partial":
        part = _out(part, x, (ks, m, n), torch.float32)
        C.skinny_gemm(x, w, ks, 0, part, None, None, None, None)
        return part
    if epilogue == "swiglu":
        act = _out(act, x, (m, n // 2), BF16)
        C.skinny_gemm(x, w, 1, 1, None, act, None, None, None)
        return act
    nb = C.skinny_blocks(n)
    if with_logits:
        logits = _out(logits, x, (m, n), torch.float32)
    block_val = _out(block_val, x, (m, nb), torch.float32)
    block_idx = _out(block_idx, x, (m, nb), torch.int32)
    C.skinny_gemm(x, w, 1, 2, None, None, logits, block_val, block_idx)
    return logits, block_val, block_idx


def rows_norm(gamma, eps: float, *, table=None, ids=None, h_in=None, part=None, h_out=None,
              xn=None, err=None):
    """Embed-and-norm (``table``, ``ids``) or reduce-partials + residual + norm
    (``h_in``, ``part [ks, m, H]``) for every token row; returns ``(h, xn)``."""
    like = h_in if h_in is not None else gamma
    m = ids.numel() if table is not None else h_in.shape[0]
    H = gamma.numel()
    h_out = _out(h_out, like, (m, H), BF16)
    xn = _out(xn, like, (m, H), BF16)
    C.rows_norm(table, ids, h_in, part, h_out, gamma, xn, float(eps), err)
    return h_out, xn


# ------------------------------------------------- MLA decode (absorbed)

def mla_attention(q_abs, latent, rope_keys, wr, w_kv_b, split: int = 256, scale: float | None = None,
                  attn=None, err=None):
    """Absorbed MLA attention of ``q_abs`` [B, H, 288] over slots ``0..wr[b]`` of
    the compressed cache (``latent`` [B, cap, 256], ``rope_keys`` [B, cap, 32])
    followed by the value up-projection: bf16 ``[B, H*64]``."""
    B, Hh = q_abs.shape[0], q_abs.shape[1]
    cap = latent.shape[1]
    ns = cap // split
    dev = q_abs.device
    op = torch.empty(B, ns, Hh, 256, dtype=BF16, device=dev)
    mp = torch.empty(B, ns, Hh, dtype=torch.float32, device=dev)
    lp = torch.empty_like(mp)
    wr = _dev_i32(wr, dev)
    if scale is None:
        scale = float(torch.tensor(96 ** -0.5).to(BF16))
    C.mla_attention(q_abs, latent, rope_keys, wr, split, scale, op, mp, lp, err)
    attn = _out(attn, q_abs, (B, Hh * 64), BF16)
    C.mla_combine_up(op, mp, lp, wr, split, w_kv_b, attn)
    return attn


def rows_residual(part, residual, alpha: float, out=None):
    """``bf16(residual + bf16(bf16(sum_s part[s]) * alpha))``."""
    out = _out(out, residual)
    C.rows_residual(part, residual, float(alpha), out)
    return out
