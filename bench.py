"""Headline benchmark: Qwen3-1.7B-shaped greedy decode on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W]

A step is one greedy decode step of the whole model (28 layers, vocab 151936,
tied head) for every sequence of the batch, replayed from one captured HIP
graph; the workload is a 64-token seeded-uniform prompt followed by K new
tokens per sequence (random-init bf16 weights ~N(0, 0.02), synthetic data).
W untimed warmup steps run first (a full generate() of W tokens). The timed
region is bracketed by torch.cuda.synchronize() on both sides.

The JSON line also carries:
  roofline      the dominant kernel (post-attention norm + gate|up GEMV +
                SwiGLU): algorithmic bytes per launch / average launch time,
                measured here with HIP events on the stream it runs on, over
                all 28 layers' real weights; `traffic` comes from the
                rocprofv3 FETCH_SIZE / WRITE_SIZE runs recorded under profiles/
  cpu_baseline  the CPU oracle (the torch restatement the tests check against)
                timed on this host on a bounded sample of the same workload
  kernels       the fused add+RMSNorm workload ([4096, 2048] bf16) and the
                decode-layer GEMVs, each with achieved GB/s and HBM fraction
  decode_layer_bs1_ctx4096   one decode layer over a 4096-position cache
  bs32          the same greedy decode for 32 sequences (tok/s, all sequences)
  mla_decode_b8_ctx8192      MiniCPM3-shaped absorbed MLA block, batch 8
  minicpm3_decode_bs1        the whole MiniCPM3-4B-shaped model, greedy, bs=1
  prefill_attention_layer    Qwen3.5 attention layer at 1024 / 4096 / 8192 tokens
  prompt_prefill_bs1         time to consume a 64- and a 512-token prompt, walked
                             (one decode step per token) and prefilled (every layer
                             over all prompt rows at once); bs32.prompt likewise
"""
from __future__ import annotations

import argparse
import json
import os
import platform
import statistics
import sys
import time
from pathlib import Path

import torch

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

HBM_PEAK_GBS = 8000.0           # MI355X HBM3E, published
REFERENCE_TOKS = 612.5          # reference's published bs=1 decode tok/s (one H200)
PROMPT = 64


def _events_time(fn, reps: int) -> float:
    """Average milliseconds of fn() over reps, HIP events on torch's current
    stream (the stream every kernel of this library is launched on)."""
    fn()
    torch.cuda.synchronize()
    e0 = torch.cuda.Event(enable_timing=True)
    e1 = torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(reps):
        fn()
    e1.record()
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) / reps


def _graph_time(fn, reps: int, calls: int = 1, copies: int = 16) -> float:
    """Average milliseconds per launch of fn() -- which makes `calls` launches --
    replayed from a HIP graph, the way the decode step runs them: fn is warmed up
    eagerly once on a side stream, captured `copies` times back to back into one
    graph (so the host's cost of launching a graph is spread over many kernels),
    and the graph replayed `reps` times between two HIP events on torch's
    current stream."""
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        fn()
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        for _ in range(copies):
            fn()
    graph.replay()
    torch.cuda.synchronize()
    e0 = torch.cuda.Event(enable_timing=True)
    e1 = torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(reps):
        graph.replay()
    e1.record()
    torch.cuda.synchronize()
    del graph
    return e0.elapsed_time(e1) / (reps * calls * copies)


def dominant_kernel(eng) -> dict:
    """Post-attention norm + gate|up GEMV + SwiGLU, timed launch by launch
    across the 28 layers' weights (1.4 GB, so the 256 MB last-level cache holds
    none of it between launches)."""
    from tilefoundry_amd._lib import C

    cfg = eng.cfg
    layers = eng.layers

    def one_pass():
        for w in layers:
            C.rmsnorm_gemv_swiglu(eng.h1, w["gamma_post"], cfg.eps, w["w_gu"], eng.act)

    ms = _graph_time(one_pass, 10, len(layers), copies=4)
    H, I = cfg.hidden, cfg.inter
    algo = 2 * I * H * 2 + 2 * H * 2 + I * 2   # W_gu + h + gamma in, act out
    achieved = algo / (ms * 1e-3) / 1e9
    roof = {"kernel": "rmsnorm_gemv_swiglu (gate|up 12288x2048)", "bound": "hbm",
            "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": None,
            "avg_launch_us": round(ms * 1e3, 3), "algorithmic_bytes": algo}
    prof = ROOT / "profiles" / "roofline_traffic.json"
    if prof.exists():
        rec = json.loads(prof.read_text())
        roof["traffic"] = rec.get("traffic_bytes_per_launch")
    return roof


def kernel_lines(eng) -> dict:
    """Per-kernel throughput for the other workloads (each a parity-tested config)."""
    from tilefoundry_amd._lib import C

    out = {}
    dev = eng.device
    bf = torch.bfloat16
    # fused residual add + RMSNorm, x / residual bf16 [4096, 2048]; 8 rotating sets
    R, H = 4096, 2048
    g = torch.Generator(device=dev).manual_seed(0)
    sets = [(torch.randn(R, H, device=dev, generator=g).to(bf),
             torch.randn(R, H, device=dev, generator=g).to(bf)) for _ in range(8)]
    gamma = (1 + 0.1 * torch.randn(H, device=dev, generator=g)).to(bf)
    y = torch.empty(R, H, device=dev, dtype=bf)
    ro = torch.empty(R, H, device=dev, dtype=bf)
    def add_norm():
        for x, r in sets:
            C.add_rms_norm(x, r, gamma, y, ro, 1e-6, 0)

    ms = _graph_time(add_norm, 10, len(sets), copies=4)
    algo = 4 * R * H * 2 + H * 2
    gbs = algo / (ms * 1e-3) / 1e9
    out["add_rms_norm_4096x2048"] = {"us": round(ms * 1e3, 2), "GB/s": round(gbs, 1),
                                     "frac": round(gbs / HBM_PEAK_GBS, 4), "bytes": algo}
    del sets, y, ro
    # decode-layer GEMVs over the 28 layers' weights
    cfg = eng.cfg
    L = eng.layers
    H, I, HQ, HKV, D = cfg.hidden, cfg.inter, cfg.heads, cfg.kv_heads, cfg.head_dim
    nqk = (HQ + HKV) * D

    def per_layer(fn):
        return _graph_time(lambda: [fn(w) for w in L], 10, len(L), copies=4)

    rows = {
        "qkv_2048x4096": (lambda w: C.decode_qkv(eng.hid, None, None, None, w["gamma_in"], cfg.eps,
                                                 w["w_qkv"], nqk, eng.qk, eng.pos, eng.vc[0], None),
                          cfg.qkv_rows * H * 2),
        "o_proj_2048x2048": (lambda w: C.gemv_residual(eng.attn, w["w_o"], eng.hid, None, eng.h1),
                             H * HQ * D * 2),
        "down_6144x2048": (lambda w: C.gemv_residual(eng.act, w["w_down"], eng.h1, None, eng.hid),
                           H * I * 2),
    }
    for name, (fn, nbytes) in rows.items():
        ms = per_layer(fn)
        gbs = nbytes / (ms * 1e-3) / 1e9
        out[name] = {"us": round(ms * 1e3, 2), "GB/s": round(gbs, 1),
                     "frac": round(gbs / HBM_PEAK_GBS, 4), "bytes": nbytes}
    ms = _graph_time(lambda: C.lm_head_argmax(eng.hid, eng.gamma_final, cfg.eps, eng.embed,
                                              eng.logits, eng.bv, eng.bi), 20)
    nbytes = cfg.vocab * H * 2
    gbs = nbytes / (ms * 1e-3) / 1e9
    out["lm_head_151936x2048"] = {"us": round(ms * 1e3, 2), "GB/s": round(gbs, 1),
                                  "frac": round(gbs / HBM_PEAK_GBS, 4), "bytes": nbytes}
    return out


def decode_layer_ctx4096(eng) -> dict:
    """One Qwen3 decode layer at bs=1 over a 4096-position cache (the single-layer
    workload): the layer's six launches, timed over the 28 layers' weights; its
    algorithmic bytes are the layer's weights plus the K and V it reads."""
    from tilefoundry_amd._lib import C

    cfg = eng.cfg
    H, HQ, HKV, D = cfg.hidden, cfg.heads, cfg.kv_heads, cfg.head_dim
    dev = eng.device
    ctx = 4096
    split = 64
    bf = torch.bfloat16
    g = torch.Generator(device=dev).manual_seed(1)
    kc = torch.randn(ctx, HKV * D, device=dev, generator=g).to(bf)
    vc = torch.randn(ctx, HKV * D, device=dev, generator=g).to(bf)
    ns = ctx // split
    op = torch.empty(ns, HQ, D, device=dev)
    mp = torch.empty(ns, HQ, device=dev)
    lp = torch.empty(ns, HQ, device=dev)
    wr = torch.tensor([ctx - 1], dtype=torch.int32, device=dev)
    from tilefoundry_amd.qwen3 import rope_tables
    cos, sin = rope_tables(ctx, D, cfg.rope_theta, dev)
    nqk = (HQ + HKV) * D
    qk = torch.empty(nqk, device=dev, dtype=bf)
    attn = torch.empty(HQ * D, device=dev, dtype=bf)
    h = torch.randn(H, device=dev, generator=g).to(bf)
    h1 = torch.empty_like(h)
    act = torch.empty(cfg.inter, device=dev, dtype=bf)
    err = torch.zeros(1, dtype=torch.int32, device=dev)

    def layer(w):
        C.decode_qkv(h, None, None, None, w["gamma_in"], cfg.eps, w["w_qkv"], nqk, qk, wr, vc, err)
        C.decode_attention(qk, None, w["gamma_q"], w["gamma_k"], cfg.eps, cos, sin, kc, vc, wr, wr, HQ, HKV,
                           split, cfg.scale, op, mp, lp, False, err)
        C.attn_combine(op, mp, lp, attn, wr, split)
        C.gemv_residual(attn, w["w_o"], h, None, h1)
        C.rmsnorm_gemv_swiglu(h1, w["gamma_post"], cfg.eps, w["w_gu"], act)
        C.gemv_residual(act, w["w_down"], h1, None, h)

    ms = _graph_time(lambda: [layer(w) for w in eng.layers], 10, len(eng.layers), copies=2)
    wbytes = sum(t.numel() * 2 for t in eng.layers[0].values())
    kv = 2 * ctx * HKV * D * 2
    nbytes = wbytes + kv
    gbs = nbytes / (ms * 1e-3) / 1e9
    ms_attn = _graph_time(lambda: (
        C.decode_attention(qk, None, eng.layers[0]["gamma_q"], eng.layers[0]["gamma_k"], cfg.eps, cos, sin, kc,
                           vc, wr, wr, HQ, HKV, split, cfg.scale, op, mp, lp, False, err),
        C.attn_combine(op, mp, lp, attn, wr, split)), 50)
    return {"workload": "one Qwen3-1.7B-shaped decode layer, bs=1, 4096 cached positions attended",
            "us": round(ms * 1e3, 2), "bytes": int(nbytes), "GB/s": round(gbs, 1),
            "frac": round(gbs / HBM_PEAK_GBS, 4),
            "attention_us": round(ms_attn * 1e3, 2),
            "attention_GB/s": round(kv / (ms_attn * 1e-3) / 1e9, 1)}


def batch32(seed: int, steps: int) -> dict:
    """bs=32 greedy decode: 32 seeded 64-token prompts, `steps` new tokens each,
    one captured step for all sequences."""
    from tilefoundry_amd.qwen3 import BatchEngine, QWEN3_1_7B

    cfg = QWEN3_1_7B
    eng = BatchEngine(cfg, batch=32, device="cuda:0", max_new=steps, prompt_room=PROMPT, seed=seed)
    g = torch.Generator().manual_seed(seed + 1)
    prompts = torch.randint(0, cfg.vocab, (32, PROMPT), generator=g).tolist()
    eng.generate(prompts, min(16, steps))     # warm
    gen = eng.generate(prompts, steps)
    walk = _first_token_ms(eng, prompts, False, reps=3)
    pre = _first_token_ms(eng, prompts, True, reps=3)
    weight_bytes = sum(t.numel() * 2 for w in eng.layers for t in w.values()) + eng.embed.numel() * 2
    mean_ctx = PROMPT + steps / 2.0
    kv_bytes = 32 * cfg.layers * mean_ctx * 2 * cfg.kv_heads * cfg.head_dim * 2
    ms = gen.seconds * 1e3 / steps
    out = {"value": round(gen.tokens_per_second, 1), "unit": "tok/s", "batch": 32, "new_tokens": steps,
           "prompt_tokens": PROMPT, "ms_per_step": round(ms, 4),
           "step_hbm": {"bytes_per_step": int(weight_bytes + kv_bytes),
                        "GB/s": round((weight_bytes + kv_bytes) / (ms * 1e-3) / 1e9, 1)},
           "prompt": {"walk": walk, "prefill": pre,
                      "speedup": round(walk["prompt_ms"] / pre["prompt_ms"], 1)}}
    del eng
    torch.cuda.empty_cache()
    return out


def _first_token_ms(eng, prompts, prefill: bool, reps: int = 5) -> dict:
    """Median over `reps` of the time spent consuming the prompt before the first
    kept pick (`prefill_seconds`) and of that plus the first decode step."""
    eng.prompt_prefill = prefill
    pre, ttft = [], []
    for _ in range(reps + 1):
        gen = eng.generate(prompts, 1)
        pre.append(gen.prefill_seconds * 1e3)
        ttft.append((gen.prefill_seconds + gen.seconds) * 1e3)
    eng.prompt_prefill = False
    return {"prompt_ms": round(statistics.median(pre[1:]), 3),
            "first_token_ms": round(statistics.median(ttft[1:]), 3), "first_pick": gen.tokens[0]}


def prompt_prefill(eng, seed: int, lengths=(64, 512)) -> dict:
    """bs=1 prompt consumption on the decode model: the reference's walk (one
    captured decode step per prompt token) against the prompt prefill (every
    layer over all prompt rows at once: f32 GEMMs, row norms, one causal
    attention launch per layer), same engine, same prompt."""
    cfg = eng.cfg
    out = {}
    for n in lengths:
        g = torch.Generator().manual_seed(seed + n)
        prompt = torch.randint(0, cfg.vocab, (n,), generator=g).tolist()
        walk = _first_token_ms(eng, prompt, False)
        pre = _first_token_ms(eng, prompt, True)
        out[str(n)] = {"walk": walk, "prefill": pre,
                       "speedup": round(walk["prompt_ms"] / pre["prompt_ms"], 1),
                       "same_first_pick": walk["first_pick"] == pre["first_pick"]}
    return out


def prompt_only(seed: int) -> dict:
    from tilefoundry_amd.qwen3 import Engine, QWEN3_1_7B

    eng = Engine(QWEN3_1_7B, device="cuda:0", max_new=16, prompt_room=512, seed=seed)
    return prompt_prefill(eng, seed)


def minicpm3_decode(seed: int, lengths=(32, 128, 512)) -> dict:
    """MiniCPM3-4B-shaped greedy decode at bs=1 (62 layers, vocab 73448 tied,
    random-init weights): an 8-token seeded prompt, then 32 / 128 / 512 new
    tokens, one captured step per token; tok/s beside the reference's H200
    figures for the same lengths."""
    from tilefoundry_amd.minicpm3 import MINICPM3_4B, MiniCPM3Engine

    ref = {32: 281.5, 128: 281.3, 512: 223.7}
    eng = MiniCPM3Engine(MINICPM3_4B, device="cuda:0", max_new=max(lengths), prompt_room=16, seed=seed)
    g = torch.Generator().manual_seed(seed + 3)
    prompt = torch.randint(0, MINICPM3_4B.vocab, (8,), generator=g).tolist()
    eng.generate([prompt], 8)   # warm
    out = {"workload": "MiniCPM3-4B-shaped greedy decode, bs=1, 8-token prompt", "by_new_tokens": {}}
    for n in lengths:
        gen = eng.generate([prompt], n)
        tps = gen.tokens_per_second
        out["by_new_tokens"][str(n)] = {"tok/s": round(tps, 1), "ms_per_step": round(gen.seconds * 1e3 / n, 4),
                                        "vs_reference_h200": round(tps / ref[n], 3)}
    out["first_tokens"] = gen.tokens[0][:8]
    del eng
    torch.cuda.empty_cache()
    return out


def mla_decode() -> dict:
    """MiniCPM3-4B-shaped MLA attention block, batch 8 x 8192 positions, absorbed:
    the whole block (one captured step) and its attention core (split attention
    over the compressed cache + merge / W_UV)."""
    from tilefoundry_amd._lib import C
    from tilefoundry_amd.minicpm3 import MLABlock, MiniCPM3Config

    cfg = MiniCPM3Config()
    B, cap = 8, 8192
    blk = MLABlock(cfg, batch=B, cap=cap, device="cuda:0")
    g = torch.Generator(device="cuda:0").manual_seed(2)
    blk.latent.normal_(generator=g)
    blk.rope_k.normal_(generator=g)
    blk.hidden.normal_(generator=g)
    blk.pos.fill_(cap - 1)
    blk.capture()
    ms_blk = _events_time(blk.run, 100)

    def core():
        C.mla_attention(blk.q_abs, blk.latent, blk.rope_k, blk.pos, blk.split, cfg.scale, blk.op, blk.mp,
                        blk.lp, blk.err)
        C.mla_combine_up(blk.op, blk.mp, blk.lp, blk.pos, blk.split, blk.w["w_kv_b"], blk.attn)

    ms_core = _graph_time(core, 20)
    cache = B * cap * (cfg.kv_lora + cfg.rope) * 2
    weights = sum(t.numel() * 2 for k, t in blk.w.items() if k.startswith("w_"))
    out = {"workload": "MiniCPM3-4B-shaped MLA decode attention block, batch 8, 8192 positions, absorbed",
           "block_us": round(ms_blk * 1e3, 2),
           "block_bytes": int(cache + weights),
           "block_GB/s": round((cache + weights) / (ms_blk * 1e-3) / 1e9, 1),
           "attention_core_us": round(ms_core * 1e3, 2),
           "attention_core_bytes": int(cache),
           "attention_core_GB/s": round(cache / (ms_core * 1e-3) / 1e9, 1),
           "attention_core_frac": round(cache / (ms_core * 1e-3) / 1e9 / HBM_PEAK_GBS, 4)}
    del blk
    torch.cuda.empty_cache()
    return out


def prefill_layer(ns=(1024, 4096, 8192)) -> dict:
    """Qwen3.5 full-attention layer (hidden 5120, 24/4 heads, head_dim 256):
    qkv projection with the q/k head norm + RoPE, causal gated attention read in
    place, o_proj + residual; TFLOP/s by the reference's convention (attention
    2*N^2*heads*head_dim)."""
    from tilefoundry_amd._lib import C

    dev = "cuda:0"
    bf = torch.bfloat16
    HID, HQ, HKV, D = 5120, 24, 4, 256
    W = (2 * HQ + 2 * HKV) * D
    g = torch.Generator(device=dev).manual_seed(3)
    w_qkv = (0.02 * torch.randn(W, HID, device=dev, generator=g)).to(bf)
    w_o = (0.02 * torch.randn(HID, HQ * D, device=dev, generator=g)).to(bf)
    gq = (0.1 * torch.randn(D, device=dev, generator=g)).to(bf)
    gk = (0.1 * torch.randn(D, device=dev, generator=g)).to(bf)
    out = {}
    for n in ns:
        hn = torch.randn(n, HID, device=dev, generator=g).to(bf)
        hidden = torch.randn(n, HID, device=dev, generator=g).to(bf)
        inv = 1.0 / (1.0e7 ** (torch.arange(0, 64, 2, device=dev).float() / 64))
        ph = torch.arange(n, device=dev).float()[:, None] * inv[None]
        ph = torch.cat((ph, ph), -1)
        cos, sin = ph.cos().to(bf), ph.sin().to(bf)
        qkv = torch.empty(n, W, device=dev, dtype=bf)
        attn = torch.empty(n, HQ * D, device=dev, dtype=bf)
        res = torch.empty(n, HID, device=dev, dtype=bf)
        qv = qkv[:, : HQ * 2 * D].view(n, HQ, 2 * D)
        k0 = HQ * 2 * D
        kv = qkv[:, k0: k0 + HKV * D].view(n, HKV, D)
        vv = qkv[:, k0 + HKV * D:].view(n, HKV, D)
        f_qkv = lambda: C.qkv_norm_rope(hn, w_qkv, qkv, HQ, HKV, gq, gk, 1e-6, cos, sin)
        f_att = lambda: C.prefill_attention(qv[:, :, :D], kv, vv, qv[:, :, D:], attn, D ** -0.5)
        f_o = lambda: C.gemm_nt(attn, w_o, res, hidden)
        f_qkv()
        reps = 20 if n <= 4096 else 8
        t_qkv = _events_time(f_qkv, reps)
        t_att = _events_time(f_att, reps)
        t_o = _events_time(f_o, reps)
        t_layer = _events_time(lambda: (f_qkv(), f_att(), f_o()), max(4, reps // 2))
        fl_att = 12288.0 * n * n
        fl_qkv = 2.0 * n * W * HID
        fl_o = 2.0 * n * HID * HQ * D
        tf = lambda fl, ms: round(fl / (ms * 1e-3) / 1e12, 1)
        out[str(n)] = {"attention_us": round(t_att * 1e3, 1), "attention_TFLOP/s": tf(fl_att, t_att),
                       "attention_frac": round(fl_att / (t_att * 1e-3) / 2.5e15, 4),
                       "qkv_us": round(t_qkv * 1e3, 1), "qkv_TFLOP/s": tf(fl_qkv, t_qkv),
                       "o_proj_us": round(t_o * 1e3, 1), "o_proj_TFLOP/s": tf(fl_o, t_o),
                       "layer_us": round(t_layer * 1e3, 1),
                       "layer_TFLOP/s": tf(fl_att + fl_qkv + fl_o, t_layer)}
        del hn, hidden, qkv, attn, res
    torch.cuda.empty_cache()
    return {"workload": "Qwen3.5 full-attention layer (Qwen3.8-27B shapes), causal GQA 24/4 x 256, "
                        "qkv (+head norm, RoPE 64 dims) + attention (+gate) + o_proj (+residual)",
            "peak_TFLOP/s": 2500.0, "by_tokens": out}


def copy_bandwidth(dev) -> dict:
    """Sustained HBM bandwidth of this device for the decode kernels' access
    pattern: a 2 GiB read + 2 GiB write copy with 16-byte streaming loads."""
    from tilefoundry_amd._lib import C

    src = torch.empty(2 << 30, dtype=torch.uint8, device=dev)
    dst = torch.empty_like(src)
    ms = _events_time(lambda: C.copy_stream(src, dst), 5)
    gbs = 2 * src.numel() / (ms * 1e-3) / 1e9
    del src, dst
    return {"GB/s": round(gbs, 1), "frac_of_nominal": round(gbs / HBM_PEAK_GBS, 4)}


def cpu_baseline(seed: int, prompt: list[int], n_steps: int = 48) -> dict:
    """The CPU oracle on this host's cores: the same model (28 layers, vocab
    151936, same synthetic weights), a 4-token prompt walk then n_steps timed
    greedy steps. Weights are drawn on the GPU (identical values, see
    tilefoundry_amd.synthetic) and copied to host memory."""
    from oracle import qwen3 as OQ
    from tilefoundry_amd.qwen3 import QWEN3_1_7B, hf_names, synthetic_weights

    cfg = QWEN3_1_7B
    torch.set_num_threads(os.cpu_count() or 1)
    wts = {k: v.cpu() for k, v in synthetic_weights(cfg, seed, "cuda:0").items()}
    layers = [OQ.LayerWeights(**{k: wts[v] for k, v in hf_names(i).items()})
              for i in range(cfg.layers)]
    model = OQ.ModelWeights(embed=wts["model.embed_tokens.weight"],
                            gamma_final=wts["model.norm.weight"], layers=layers)
    ocfg = OQ.Qwen3Config()
    p = prompt[:4]
    cos, sin = OQ.rope_tables(len(p) + n_steps + 1, ocfg.head_dim, ocfg.rope_theta)
    caches = OQ.empty_caches(ocfg, ocfg.layers)
    for i, t in enumerate(p):                       # untimed: also converts weights to f32
        logits = OQ.step(model, ocfg, t, i, caches, cos, sin, p_bf16=True)
    t0 = time.perf_counter()
    tok = OQ.greedy(logits)
    for s in range(n_steps):
        logits = OQ.step(model, ocfg, tok, len(p) + s, caches, cos, sin, p_bf16=True)
        tok = OQ.greedy(logits)
    dt = time.perf_counter() - t0
    cpu = platform.processor() or platform.machine()
    try:
        for line in Path("/proc/cpuinfo").read_text().splitlines():
            if line.startswith("model name"):
                cpu = line.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    return {"value": round(n_steps / dt, 3), "unit": "tok/s", "cores": torch.get_num_threads(),
            "kind": "port",
            "sample": (f"oracle (torch CPU, f32 matmuls) of the same 28-layer model: {n_steps} greedy "
                       f"decode steps at bs=1 after a 4-token prompt walk; {dt:.1f} s; "
                       f"os.cpu_count()={os.cpu_count()}; cpu='{cpu}'")}


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=2048, help="timed decode steps (new tokens)")
    ap.add_argument("--warmup", type=int, default=64, help="untimed decode steps first")
    ap.add_argument("--seed", type=int, default=0)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-kernels", action="store_true", help="skip the per-kernel lines")
    ap.add_argument("--no-configs", action="store_true",
                    help="skip the bs=32, MLA and prefill measurements")
    ap.add_argument("--kernel-only", action="store_true",
                    help="only launch the dominant kernel loop (for rocprofv3 counter runs)")
    ap.add_argument("--only", choices=("bs32", "mla", "prefill", "prompt", "minicpm3"),
                    help="run one of the secondary configurations alone and print its line "
                         "(for rocprofv3 kernel traces of that workload)")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU: the decode path runs on a single MI355X; "
              "run with --gpus 1 (multi-GPU sharding is described, not run).", file=sys.stderr)
        return 2
    if not torch.cuda.is_available():
        print("bench.py needs a GPU", file=sys.stderr)
        return 2

    if args.only:
        run = {"bs32": lambda: batch32(args.seed, args.steps), "mla": mla_decode,
               "prefill": prefill_layer, "prompt": lambda: prompt_only(args.seed),
               "minicpm3": lambda: minicpm3_decode(args.seed)}[args.only]
        print(json.dumps({args.only: run()}))
        return 0

    from tilefoundry_amd.qwen3 import Engine, QWEN3_1_7B

    cfg = QWEN3_1_7B
    dev = torch.device("cuda:0")
    eng = Engine(cfg, device=dev, max_new=max(args.steps, args.warmup), prompt_room=PROMPT,
                 seed=args.seed)
    g = torch.Generator().manual_seed(args.seed)
    prompt = torch.randint(0, cfg.vocab, (PROMPT,), generator=g).tolist()

    if args.kernel_only:
        # the dominant kernel's launch loop, then a plain copy of known size (the
        # calibration dispatch for FETCH_SIZE / WRITE_SIZE counter runs)
        from tilefoundry_amd._lib import C

        roof = dominant_kernel(eng)
        src = torch.empty(64 << 20, dtype=torch.uint8, device=dev)
        dst = torch.empty_like(src)
        for _ in range(4):
            C.copy_stream(src, dst)
        torch.cuda.synchronize()
        print(json.dumps({"kernel_only": roof, "copy_bytes": src.numel()}))
        return 0

    if args.warmup > 0:
        eng.generate(prompt, args.warmup)
    torch.cuda.synchronize()
    gen = eng.generate(prompt, args.steps)      # synchronize() on both sides inside
    toks = gen.tokens_per_second
    ms_per_step = gen.seconds * 1e3 / args.steps

    roof = dominant_kernel(eng)
    kernels = {} if args.no_kernels else kernel_lines(eng)
    layer = None if args.no_kernels else decode_layer_ctx4096(eng)
    copy_bw = copy_bandwidth(dev)
    weight_bytes = sum(t.numel() * 2 for w in eng.layers for t in w.values()) + eng.embed.numel() * 2
    mean_ctx = PROMPT + args.steps / 2.0
    kv_bytes = cfg.layers * mean_ctx * 2 * cfg.kv_heads * cfg.head_dim * 2
    step_bytes = weight_bytes + kv_bytes
    line = {
        "metric": "decode tok/s Qwen3-1.7B-shape bs=1/32; kernel HBM GB/s as % of MI355X peak",
        "value": round(toks, 2),
        "unit": "tok/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": round(toks / REFERENCE_TOKS, 4),
        "dtype": "bf16",
        "data": "synthetic (seeded-uniform prompt ids, random-init weights ~N(0,0.02))",
        "config": {"workload": "Qwen3-1.7B-shaped greedy decode: 28 layers, hidden 2048, 16/8 heads, "
                               "head_dim 128, SwiGLU 6144, vocab 151936 tied; 64-token prompt",
                   "batch": 1, "prompt_tokens": PROMPT, "new_tokens": args.steps,
                   "parallelism": "single GPU"},
        "step_hbm": {"bytes_per_step": int(step_bytes),
                     "GB/s": round(step_bytes / (ms_per_step * 1e-3) / 1e9, 1),
                     "frac": round(step_bytes / (ms_per_step * 1e-3) / 1e9 / HBM_PEAK_GBS, 4)},
        "roofline": roof,
        "hbm_copy_measured": copy_bw,
        "kernels": kernels,
        "decode_layer_bs1_ctx4096": layer,
        "first_tokens": gen.tokens[:8],
        "prompt_prefill_bs1": None if args.no_kernels else prompt_prefill(eng, args.seed),
    }
    del eng
    torch.cuda.empty_cache()
    if not args.no_configs:
        line["bs32"] = batch32(args.seed, args.steps)
        line["mla_decode_b8_ctx8192"] = mla_decode()
        line["minicpm3_decode_bs1"] = minicpm3_decode(args.seed)
        line["prefill_attention_layer"] = prefill_layer()
    if not args.no_cpu_baseline:
        line["cpu_baseline"] = cpu_baseline(args.seed, prompt)
    else:
        line["cpu_baseline"] = None
    print(json.dumps(line))
    return 0


if __name__ == "__main__":
    sys.exit(main())
