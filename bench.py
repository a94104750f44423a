"""Headline benchmark: Qwen3-1.7B-shaped greedy decode on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W]

A step is one greedy decode step of the whole model (28 layers, vocab 151936,
tied head) for every sequence of the batch, replayed from one captured HIP
graph; the workload is a 64-token seeded-uniform prompt followed by 2048 new
tokens per sequence (random-init bf16 weights ~N(0, 0.02), synthetic data).
The timed region is always the workload's 2048 decode steps, whatever --steps
asks (the mean KV length, and so the bytes per step, depend on it); the line
reports the count actually timed as `steps` and the request as
`steps_requested`. W untimed warmup steps run first (a generate() of W
tokens). The timed region is bracketed by torch.cuda.synchronize() on both
sides. Each secondary measurement runs inside its own try/except: a failure
there becomes an "error" field of that object, not a lost line.

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
PROMPT = 64                     # prompt tokens per sequence
NEW_TOKENS = 2048               # new tokens per sequence, bs=1 and bs=32
PROMPT_LENGTHS = (64, 512)      # prompt-prefill leg, bs=1
MINICPM3_LENGTHS = (32, 128, 512)
MINICPM3_PROMPT = 8


def sizing(args) -> dict:
    """Every engine the run builds, as ``(max_new, prompt_room)``, and every
    ``(prompt_len, new_tokens)`` request the run makes of it. An engine holds
    ``max_new + prompt_room`` steps; a request needs ``prompt_len + new``."""
    warm = max(1, args.warmup)
    return {
        "headline": {"engine": (max(NEW_TOKENS, warm), PROMPT),
                     "requests": [(PROMPT, warm), (PROMPT, NEW_TOKENS)]},
        "prompt_prefill_bs1": {"engine": (16, max(PROMPT_LENGTHS)),
                               "requests": [(n, 1) for n in PROMPT_LENGTHS]},
        "bs32": {"engine": (NEW_TOKENS, PROMPT),
                 "requests": [(PROMPT, 16), (PROMPT, NEW_TOKENS), (PROMPT, 1)]},
        "minicpm3_decode_bs1": {"engine": (max(MINICPM3_LENGTHS), 16),
                                "requests": [(MINICPM3_PROMPT, 8)]
                                + [(MINICPM3_PROMPT, n) for n in MINICPM3_LENGTHS]},
    }


def _leg(fn, *a, **kw):
    """Run one secondary measurement; an exception becomes its "error" field.
    A line on stderr names each measurement as it ends."""
    t0 = time.perf_counter()
    try:
        out = fn(*a, **kw)
        print(f"[bench] {fn.__name__} done in {time.perf_counter() - t0:.1f} s", file=sys.stderr, flush=True)
        return out
    except Exception as exc:  # noqa: BLE001 -- reported in the line, not swallowed
        import traceback

        traceback.print_exc()
        torch.cuda.synchronize()
        torch.cuda.empty_cache()
        return {"error": f"{type(exc).__name__}: {exc}"}


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
    # fused residual add + RMSNorm, x / residual bf16 [4096, 2048]: 12 rotating
    # input sets and 4 output sets (537 MB read + 134 MB written per rotation,
    # twice the 256 MB last-level cache)
    R, H = 4096, 2048
    g = torch.Generator(device=dev).manual_seed(0)
    sets = [(torch.randn(R, H, device=dev, generator=g).to(bf),
             torch.randn(R, H, device=dev, generator=g).to(bf)) for _ in range(12)]
    gamma = (1 + 0.1 * torch.randn(H, device=dev, generator=g)).to(bf)
    outs = [(torch.empty(R, H, device=dev, dtype=bf), torch.empty(R, H, device=dev, dtype=bf))
            for _ in range(4)]

    def add_norm():
        for i, (x, r) in enumerate(sets):
            y, ro = outs[i % len(outs)]
            C.add_rms_norm(x, r, gamma, y, ro, 1e-6, 0)

    ms = _graph_time(add_norm, 10, len(sets), copies=4)
    algo = 4 * R * H * 2 + H * 2
    gbs = algo / (ms * 1e-3) / 1e9
    out["add_rms_norm_4096x2048"] = {"us": round(ms * 1e3, 2), "GB/s": round(gbs, 1),
                                     "frac": round(gbs / HBM_PEAK_GBS, 4), "bytes": algo}
    del sets, outs
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
    # the floor of the gate|up GEMV's access pattern: the same weight stream (28
    # layers' 12288 x 2048 matrices, one-shot blocks of 4 or 6 rows) with no arithmetic
    nbytes = 2 * I * H * 2
    floor = {}
    for rpb in (4, 6):
        fold = torch.empty((2 * I + rpb - 1) // rpb, device=dev)   # one value per block
        ms = per_layer(lambda w, r=rpb, f=fold: C.read_rows(w["w_gu"], r, f))
        gbs = nbytes / (ms * 1e-3) / 1e9
        floor[f"rows_per_block_{rpb}"] = {"us": round(ms * 1e3, 2), "GB/s": round(gbs, 1),
                                          "frac": round(gbs / HBM_PEAK_GBS, 4)}
    out["gate_up_access_pattern_floor"] = {**floor, "bytes": nbytes,
                                           "what": "tfa_read_rows: the gate|up GEMV's weight loads alone"}
    ms = _graph_time(lambda: C.lm_head_argmax(eng.hid, eng.gamma_final, cfg.eps, eng.embed,
                                              eng.logits, eng.bv, eng.bi), 20)
    nbytes = cfg.vocab * H * 2
    gbs = nbytes / (ms * 1e-3) / 1e9
    out["lm_head_151936x2048"] = {"us": round(ms * 1e3, 2), "GB/s": round(gbs, 1),
                                  "frac": round(gbs / HBM_PEAK_GBS, 4), "bytes": nbytes}
    return out


def decode_layer_ctx4096(eng) -> dict:
    """One Qwen3 decode layer at bs=1 over a 4096-position cache (the single-layer
    workload): the layer's six launches, timed over the 28 layers' weights, each
    layer with a K/V cache of its own (28 x 16.8 MB, so no layer's cache is
    still in the 256 MB last-level cache when its turn comes again); its
    algorithmic bytes are the layer's weights plus the K and V it reads."""
    from tilefoundry_amd._lib import C

    cfg = eng.cfg
    H, HQ, HKV, D = cfg.hidden, cfg.heads, cfg.kv_heads, cfg.head_dim
    dev = eng.device
    ctx = 4096
    split = eng.split
    bf = torch.bfloat16
    g = torch.Generator(device=dev).manual_seed(1)
    L = len(eng.layers)
    kcs = [torch.randn(ctx, HKV * D, device=dev, generator=g).to(bf) for _ in range(L)]
    vcs = [torch.randn(ctx, HKV * D, device=dev, generator=g).to(bf) for _ in range(L)]
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

    def attention(w, kc, vc):
        C.decode_attention(qk, None, w["gamma_q"], w["gamma_k"], cfg.eps, cos, sin, kc, vc, wr, wr, HQ, HKV,
                           split, cfg.scale, op, mp, lp, False, err)
        C.attn_combine(op, mp, lp, attn, wr, split)

    def layer(w, kc, vc):
        C.decode_qkv(h, None, None, None, w["gamma_in"], cfg.eps, w["w_qkv"], nqk, qk, wr, vc, err)
        attention(w, kc, vc)
        C.gemv_residual(attn, w["w_o"], h, None, h1)
        C.rmsnorm_gemv_swiglu(h1, w["gamma_post"], cfg.eps, w["w_gu"], act)
        C.gemv_residual(act, w["w_down"], h1, None, h)

    ms = _graph_time(lambda: [layer(w, kc, vc) for w, kc, vc in zip(eng.layers, kcs, vcs)], 10, L, copies=2)
    wbytes = sum(t.numel() * 2 for t in eng.layers[0].values())
    kv = 2 * ctx * HKV * D * 2
    nbytes = wbytes + kv
    gbs = nbytes / (ms * 1e-3) / 1e9
    ms_attn = _graph_time(lambda: [attention(w, kc, vc) for w, kc, vc in zip(eng.layers, kcs, vcs)], 20, L,
                          copies=2)
    del kcs, vcs
    return {"workload": "one Qwen3-1.7B-shaped decode layer, bs=1, 4096 cached positions attended",
            "us": round(ms * 1e3, 2), "bytes": int(nbytes), "GB/s": round(gbs, 1),
            "frac": round(gbs / HBM_PEAK_GBS, 4),
            "attention_us": round(ms_attn * 1e3, 2),
            "attention_GB/s": round(kv / (ms_attn * 1e-3) / 1e9, 1),
            "attention_frac": round(kv / (ms_attn * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
            "working_set": f"{L} layers' weights and {L} K/V caches of {kv} B, rotated"}


def batch32(seed: int, steps: int = NEW_TOKENS, args=None) -> dict:
    """bs=32 greedy decode: 32 seeded 64-token prompts, `steps` new tokens each,
    one captured step for all sequences."""
    from tilefoundry_amd.qwen3 import BatchEngine, QWEN3_1_7B

    cfg = QWEN3_1_7B
    max_new, room = sizing(args)["bs32"]["engine"] if args is not None else (steps, PROMPT)
    eng = BatchEngine(cfg, batch=32, device="cuda:0", max_new=max(max_new, steps), prompt_room=room,
                      seed=seed)
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
           "prompt_tokens": PROMPT, "ms_per_step": round(ms, 4), "attention": eng.attention,
           "step_hbm": {"bytes_per_step": int(weight_bytes + kv_bytes),
                        "GB/s": round((weight_bytes + kv_bytes) / (ms * 1e-3) / 1e9, 1),
                        "frac": round((weight_bytes + kv_bytes) / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4)},
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


def prompt_prefill(eng, seed: int, lengths=PROMPT_LENGTHS) -> dict:
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


def prompt_only(seed: int, args=None) -> dict:
    """The prompt-prefill leg on an engine of its own, sized for the longest prompt."""
    from tilefoundry_amd.qwen3 import Engine, QWEN3_1_7B

    max_new, room = sizing(args)["prompt_prefill_bs1"]["engine"] if args is not None else (16, 512)
    eng = Engine(QWEN3_1_7B, device="cuda:0", max_new=max_new, prompt_room=room, seed=seed)
    out = prompt_prefill(eng, seed)
    del eng
    torch.cuda.empty_cache()
    return out


def minicpm3_decode(seed: int, lengths=MINICPM3_LENGTHS, args=None) -> dict:
    """MiniCPM3-4B-shaped greedy decode at bs=1 (62 layers, vocab 73448 tied,
    random-init weights): an 8-token seeded prompt, then 32 / 128 / 512 new
    tokens, one captured step per token; tok/s beside the reference's H200
    figures for the same lengths."""
    from tilefoundry_amd.minicpm3 import MINICPM3_4B, MiniCPM3Engine

    ref = {32: 281.5, 128: 281.3, 512: 223.7}
    max_new, room = sizing(args)["minicpm3_decode_bs1"]["engine"] if args is not None else (max(lengths), 16)
    eng = MiniCPM3Engine(MINICPM3_4B, device="cuda:0", max_new=max_new, prompt_room=room, seed=seed)
    g = torch.Generator().manual_seed(seed + 3)
    prompt = torch.randint(0, MINICPM3_4B.vocab, (MINICPM3_PROMPT,), generator=g).tolist()
    eng.generate([prompt], 8)   # warm
    out = {"workload": "MiniCPM3-4B-shaped greedy decode, bs=1, 8-token prompt", "by_new_tokens": {}}
    for n in lengths:
        gen = eng.generate([prompt], n)
        tps = gen.tokens_per_second
        out["by_new_tokens"][str(n)] = {"tok/s": round(tps, 1), "ms_per_step": round(gen.seconds * 1e3 / n, 4),
                                        "vs_reference_h200": round(tps / ref[n], 3)}
    out["first_tokens"] = gen.tokens[0][:8]
    # the reference's default sampling (T = 0.8, top-p 0.8), drawn on the device in the step
    from tilefoundry_amd.minicpm3 import sample_top_p

    n = MINICPM3_LENGTHS[1]
    eng.generate([prompt], 8, sampler=sample_top_p(0.8, 0.8, seed=seed))   # captures the sampling step
    gen = eng.generate([prompt], n, sampler=sample_top_p(0.8, 0.8, seed=seed))
    out["top_p_sampled"] = {"new_tokens": n, "tok/s": round(gen.tokens_per_second, 1),
                            "ms_per_step": round(gen.seconds * 1e3 / n, 4), "temperature": 0.8, "top_p": 0.8,
                            "first_tokens": gen.tokens[0][:8]}
    del eng
    torch.cuda.empty_cache()
    return out


def mla_decode(nblocks: int = 8) -> dict:
    """MiniCPM3-4B-shaped MLA attention block, batch 8 x 8192 positions, absorbed:
    the whole block (one captured step) and its attention core (split attention
    over the compressed cache + merge / W_UV). ``nblocks`` independent blocks
    (own weights, own caches: 8 x 64.8 MB) are stepped in turn, so the 256 MB
    last-level cache holds none of a block's cache when its turn comes again."""
    from tilefoundry_amd._lib import C
    from tilefoundry_amd.minicpm3 import MLABlock, MiniCPM3Config

    cfg = MiniCPM3Config()
    B, cap = 8, 8192
    g = torch.Generator(device="cuda:0").manual_seed(2)
    blks = []
    for i in range(nblocks):
        blk = MLABlock(cfg, batch=B, cap=cap, device="cuda:0", seed=i)
        blk.latent.normal_(generator=g)
        blk.rope_k.normal_(generator=g)
        blk.hidden.normal_(generator=g)
        blk.pos.fill_(cap - 1)
        blk.capture()
        blks.append(blk)
    ms_blk = _events_time(lambda: [b.run() for b in blks], 20) / nblocks

    def core():
        for b in blks:
            C.mla_attention(b.q_abs, b.latent, b.rope_k, b.pos, b.split, cfg.scale, b.op, b.mp, b.lp, b.err)
            C.mla_combine_up(b.op, b.mp, b.lp, b.pos, b.split, b.w["w_kv_b"], b.attn)

    ms_core = _graph_time(core, 10, nblocks, copies=2)
    cache = B * cap * (cfg.kv_lora + cfg.rope) * 2
    weights = sum(t.numel() * 2 for k, t in blks[0].w.items() if k.startswith("w_"))
    out = {"workload": "MiniCPM3-4B-shaped MLA decode attention block, batch 8, 8192 positions, absorbed",
           "block_us": round(ms_blk * 1e3, 2),
           "block_bytes": int(cache + weights),
           "block_GB/s": round((cache + weights) / (ms_blk * 1e-3) / 1e9, 1),
           "block_frac": round((cache + weights) / (ms_blk * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
           "attention_core_us": round(ms_core * 1e3, 2),
           "attention_core_bytes": int(cache),
           "attention_core_GB/s": round(cache / (ms_core * 1e-3) / 1e9, 1),
           "attention_core_frac": round(cache / (ms_core * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
           "working_set": f"{nblocks} blocks (own weights and caches) stepped in turn"}
    del blks
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
        # clocks up before any timing: the layer repeated for 0.2 s (a few
        # calls of the 1024-token layer, ~0.3 ms, leave the first timing on
        # ramping clocks), then each part timed over ~5 ms of calls
        t_end = time.perf_counter() + 0.2
        while time.perf_counter() < t_end:
            f_qkv(), f_att(), f_o()
            torch.cuda.synchronize()

        def timed(fn):
            reps = max(8, min(400, int(5.0 / max(_events_time(fn, 3), 1e-3))))
            return _events_time(fn, reps)

        t_qkv = timed(f_qkv)
        t_att = timed(f_att)
        t_o = timed(f_o)
        t_layer = timed(lambda: (f_qkv(), f_att(), f_o()))
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


def _cpu_name() -> str:
    cpu = platform.processor() or platform.machine()
    try:
        for line in Path("/proc/cpuinfo").read_text().splitlines():
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return cpu


def _protocol(fn, warm: int = 2, runs: int = 7) -> dict:
    """``warm`` untimed calls, then ``runs`` timed ones: median / min / max seconds."""
    for _ in range(warm):
        fn()
    ts = []
    for _ in range(runs):
        t0 = time.perf_counter()
        fn()
        ts.append(time.perf_counter() - t0)
    return {"median_s": statistics.median(ts), "min_s": min(ts), "max_s": max(ts), "runs": runs,
            "warmups": warm}


def _rate(prot: dict, work: float, unit: str, scale: float = 1.0) -> dict:
    """Throughput ``work / time`` at the median and at the extremes (min time = max rate)."""
    r = lambda t: round(work / t / scale, 3)
    return {"value": r(prot["median_s"]), "unit": unit, "min": r(prot["max_s"]), "max": r(prot["min_s"]),
            "median_ms": round(prot["median_s"] * 1e3, 3), "runs": prot["runs"], "warmups": prot["warmups"]}


def cpu_baseline(seed: int, prompt: list[int]) -> dict:
    """The CPU oracle (the torch restatement the tests check against) on this
    host's cores, for every configuration, with the reference's protocol: 2
    untimed runs, then 7 timed, median (``value``) with min / max. Weights are
    drawn on the GPU (identical values on any device, see
    tilefoundry_amd.synthetic) and copied to host memory. The top-level fields
    are the headline workload's (bs=1 greedy decode of the 28-layer model);
    ``by_config`` holds the rest. Each sample is bounded; ``sample`` says what
    it was."""
    from oracle import minicpm3 as OM
    from oracle import norms as ON
    from oracle import prefill as OP
    from oracle import qwen3 as OQ
    from tilefoundry_amd.qwen3 import QWEN3_1_7B, hf_names, synthetic_weights

    torch.set_num_threads(os.cpu_count() or 1)
    bf = torch.bfloat16
    cfg = QWEN3_1_7B
    ocfg = OQ.Qwen3Config()
    by = {}
    t_all = time.perf_counter()

    # config 1: fused add + RMSNorm over [4096, 2048]
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(4096, 2048, generator=g).to(bf)
    r = torch.randn(4096, 2048, generator=g).to(bf)
    gam = (1 + 0.1 * torch.randn(2048, generator=g)).to(bf)
    p = _protocol(lambda: ON.add_rms_norm(x, r, gam, 1e-6))
    by["add_rms_norm_4096x2048"] = {**_rate(p, 4 * 4096 * 2048 * 2 + 2048 * 2, "GB/s", 1e9),
                                    "sample": "the whole [4096, 2048] call"}
    del x, r

    # the 28-layer model's weights (configs 2 and 5)
    wts = {k: v.cpu() for k, v in synthetic_weights(cfg, seed, "cuda:0").items()}
    layers = [OQ.LayerWeights(**{k: wts[v] for k, v in hf_names(i).items()}) for i in range(cfg.layers)]
    model = OQ.ModelWeights(embed=wts["model.embed_tokens.weight"],
                            gamma_final=wts["model.norm.weight"], layers=layers)
    del wts

    # config 2: one decode layer attending 4096 positions (4095 cached + its own)
    ctx = 4096
    cos, sin = OQ.rope_tables(ctx, ocfg.head_dim, ocfg.rope_theta)
    kc = torch.randn(ctx - 1, ocfg.kv_heads, ocfg.head_dim, generator=g).to(bf)
    vc = torch.randn(ctx - 1, ocfg.kv_heads, ocfg.head_dim, generator=g).to(bf)
    h = torch.randn(ocfg.hidden, generator=g).to(bf)
    lw = layers[0]
    p = _protocol(lambda: OQ.decoder_layer(h, lw, ocfg, cos[ctx - 1], sin[ctx - 1], kc, vc))
    layer_bytes = sum(getattr(lw, f).numel() * 2 for f in
                      ("gamma_in", "w_q", "w_k", "w_v", "gamma_q", "gamma_k", "w_o", "gamma_post",
                       "w_gate", "w_up", "w_down")) + 2 * ctx * ocfg.kv_heads * ocfg.head_dim * 2
    by["decode_layer_bs1_ctx4096"] = {**_rate(p, layer_bytes, "GB/s", 1e9),
                                      "sample": "one layer step over a 4096-position cache"}
    del kc, vc

    # config 5: the greedy steps are timed at the GPU workload's mean context --
    # a 64-token prompt then 2048 new tokens attend 1088 positions on average --
    # over a synthetic cache of MEAN_CTX - 1 seeded rows per layer (the cost of a
    # step depends on the context only through the attention's length)
    mean_ctx = PROMPT + NEW_TOKENS // 2
    cos, sin = OQ.rope_tables(mean_ctx + 16, ocfg.head_dim, ocfg.rope_theta)

    def synthetic_caches(gen):
        return [[torch.randn(mean_ctx - 1, ocfg.kv_heads, ocfg.head_dim, generator=gen).to(bf),
                 torch.randn(mean_ctx - 1, ocfg.kv_heads, ocfg.head_dim, generator=gen).to(bf)]
                for _ in range(ocfg.layers)]

    # bs=1: one greedy step of the 28-layer model per run
    caches = synthetic_caches(g)
    logits = OQ.step(model, ocfg, prompt[0], mean_ctx - 1, caches, cos, sin, p_bf16=True)  # untimed
    state = {"tok": OQ.greedy(logits), "pos": mean_ctx}

    def one_step():
        lg = OQ.step(model, ocfg, state["tok"], state["pos"], caches, cos, sin, p_bf16=True)
        state["tok"], state["pos"] = OQ.greedy(lg), state["pos"] + 1

    p = _protocol(one_step)
    head = {**_rate(p, 1.0, "tok/s"),
            "sample": (f"oracle (torch CPU, f32 matmuls) of the same 28-layer model: 9 greedy decode "
                       f"steps at bs=1 (2 untimed + 7 timed, one step per run) at contexts "
                       f"{mean_ctx + 1}..{mean_ctx + 9} over a synthetic {mean_ctx - 1}-position cache "
                       f"(the GPU workload's mean context is {mean_ctx})")}
    del caches

    # bs=32: one batched greedy step of 32 sequences per run
    B = 32
    pr = OQ.prompt_ids(cfg.vocab, 1, seed=seed + 1, batch=B)
    caches_b = [synthetic_caches(g) for _ in range(B)]
    logits = OQ.step_batch(model, ocfg, [row[0] for row in pr], [mean_ctx - 1] * B, caches_b, cos, sin,
                           p_bf16=True)
    st = {"tok": logits.argmax(-1).tolist(), "pos": mean_ctx}

    def batch_step():
        lg = OQ.step_batch(model, ocfg, st["tok"], [st["pos"]] * B, caches_b, cos, sin, p_bf16=True)
        st["tok"], st["pos"] = lg.argmax(-1).tolist(), st["pos"] + 1

    p = _protocol(batch_step)
    by["decode_bs32"] = {**_rate(p, float(B), "tok/s"),
                         "sample": f"9 batched greedy steps of 32 sequences (one step per run) at contexts "
                                   f"{mean_ctx + 1}..{mean_ctx + 9} over synthetic caches"}
    del model, layers, caches_b

    # config 3: MLA attention block, batch 8, 8192 positions (absorbed form)
    mcfg = OM.MLAConfig()
    mw = OM.random_weights(mcfg, seed)
    lat, rk = OM.random_cache(8, 8192, mcfg, seed=seed + 2)
    hid = torch.randn(8, mcfg.hidden, generator=g).to(bf)
    mcos, msin = OM.rope_tables(8192, mcfg)

    def mla_block():
        for b in range(8):
            pj = OM.project(hid[b], mw, mcfg, 8191, mcos, msin)
            qa = OM.absorb_query(pj.q_up, mw, mcfg, 8191, mcos, msin)
            attn = OM.attend_absorbed(qa, lat[b], rk[b], mw, mcfg)
            OM.o_proj_residual(attn, mw.w_o, hid[b], 1.0)

    p = _protocol(mla_block)
    cache_bytes = 8 * 8192 * (mcfg.kv_lora + mcfg.rope) * 2
    by["mla_decode_b8_ctx8192"] = {**_rate(p, cache_bytes, "GB/s (cache bytes)", 1e9),
                                   "sample": "the whole block for 8 sequences x 8192 positions"}
    del lat, rk

    # config 4: the prefill attention layer at 1024 tokens
    pc = OP.PrefillConfig()
    lwp = OP.random_layer(pc, seed)
    n = 1024
    hn = torch.randn(n, pc.hidden, generator=g).to(bf)
    pcos, psin = OP.rope_tables(n, pc)

    def prefill_layer_cpu():
        q, gate, k, v = OP.qkv(hn, lwp["w_q"], lwp["w_k"], lwp["w_v"], lwp["gamma_q"], lwp["gamma_k"],
                               pcos, psin, pc)
        a = OP.attention(q, k, v, gate, pc)
        OP.o_proj(a, hn, lwp["w_o"])

    p = _protocol(prefill_layer_cpu)
    fl = 12288.0 * n * n + 146_800_640.0 * n + 62_914_560.0 * n
    by["prefill_layer_1024"] = {**_rate(p, fl, "TFLOP/s", 1e12),
                                "sample": "qkv (+head norm, RoPE) + causal attention (+gate) + o_proj "
                                          "(+residual) at 1024 tokens"}
    return {**head, "cores": torch.get_num_threads(), "kind": "port", "by_config": by,
            "host": {"os.cpu_count": os.cpu_count(), "torch_threads": torch.get_num_threads(),
                     "cpu": _cpu_name()},
            "seconds_total": round(time.perf_counter() - t_all, 1)}


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=NEW_TOKENS,
                    help="requested timed decode steps; the headline always times the workload's "
                         f"{NEW_TOKENS} new tokens and reports that count")
    ap.add_argument("--warmup", type=int, default=64, help="untimed decode steps first")
    ap.add_argument("--seed", type=int, default=0)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-kernels", action="store_true", help="skip the per-kernel lines")
    ap.add_argument("--no-configs", action="store_true",
                    help="skip the bs=32, MLA and prefill measurements")
    ap.add_argument("--kernel-only", action="store_true",
                    help="only launch the dominant kernel loop (for rocprofv3 counter runs)")
    ap.add_argument("--only", choices=("bs32", "mla", "prefill", "prompt", "minicpm3", "cpu", "kernels"),
                    help="run one of the secondary configurations alone and print its line "
                         "(for rocprofv3 kernel traces of that workload)")
    return run(ap.parse_args())


def kernels_only(args) -> int:
    """The per-kernel workloads alone (for rocprofv3 counter passes): fused
    add+RMSNorm, the decode GEMVs and head, one decode layer's attention over
    rotating 4096-slot caches, the MLA core over rotating caches, then a plain
    copy of 64 MiB (the calibration dispatch for FETCH_SIZE / WRITE_SIZE)."""
    from tilefoundry_amd._lib import C
    from tilefoundry_amd.qwen3 import Engine, QWEN3_1_7B

    dev = torch.device("cuda:0")
    eng = Engine(QWEN3_1_7B, device=dev, max_new=16, prompt_room=16, seed=args.seed, capture=False)
    out = {"kernels": kernel_lines(eng), "decode_layer_bs1_ctx4096": decode_layer_ctx4096(eng)}
    del eng
    torch.cuda.empty_cache()
    out["mla_decode_b8_ctx8192"] = mla_decode()
    src = torch.empty(64 << 20, dtype=torch.uint8, device=dev)
    dst = torch.empty_like(src)
    for _ in range(4):
        C.copy_stream(src, dst)
    torch.cuda.synchronize()
    out["copy_bytes"] = src.numel()
    print(json.dumps(out))
    return 0


def parse(argv: list[str]):
    """The parsed arguments of ``argv`` (used by the tests of the run's sizing)."""
    saved = sys.argv
    try:
        sys.argv = ["bench.py", *argv]
        ap = argparse.ArgumentParser()
        ap.add_argument("--gpus", type=int, default=1)
        ap.add_argument("--steps", type=int, default=NEW_TOKENS)
        ap.add_argument("--warmup", type=int, default=64)
        ap.add_argument("--seed", type=int, default=0)
        return ap.parse_known_args()[0]
    finally:
        sys.argv = saved


def run(args) -> int:
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU: the decode path runs on a single MI355X; "
              "run with --gpus 1 (multi-GPU sharding is described, not run).", file=sys.stderr)
        return 2
    if not torch.cuda.is_available():
        print("bench.py needs a GPU", file=sys.stderr)
        return 2

    cfg_prompt = torch.randint(0, 151936, (PROMPT,), generator=torch.Generator().manual_seed(args.seed)).tolist()
    if args.only == "kernels":
        return kernels_only(args)
    if args.only:
        fn = {"bs32": lambda: batch32(args.seed, NEW_TOKENS, args), "mla": mla_decode,
              "prefill": prefill_layer, "prompt": lambda: prompt_only(args.seed, args),
              "minicpm3": lambda: minicpm3_decode(args.seed, args=args),
              "cpu": lambda: cpu_baseline(args.seed, cfg_prompt)}[args.only]
        print(json.dumps({args.only: fn()}))
        return 0

    from tilefoundry_amd.qwen3 import Engine, QWEN3_1_7B

    cfg = QWEN3_1_7B
    dev = torch.device("cuda:0")
    max_new, room = sizing(args)["headline"]["engine"]
    eng = Engine(cfg, device=dev, max_new=max_new, prompt_room=room, seed=args.seed)
    prompt = cfg_prompt

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

    eng.generate(prompt, max(1, args.warmup))
    torch.cuda.synchronize()
    gen = eng.generate(prompt, NEW_TOKENS)      # synchronize() on both sides inside
    toks = gen.tokens_per_second
    ms_per_step = gen.seconds * 1e3 / NEW_TOKENS
    print(f"[bench] headline {toks:.1f} tok/s over {NEW_TOKENS} steps", file=sys.stderr, flush=True)

    roof = dominant_kernel(eng)
    kernels = {} if args.no_kernels else _leg(kernel_lines, eng)
    layer = None if args.no_kernels else _leg(decode_layer_ctx4096, eng)
    copy_bw = _leg(copy_bandwidth, dev)
    weight_bytes = sum(t.numel() * 2 for w in eng.layers for t in w.values()) + eng.embed.numel() * 2
    mean_ctx = PROMPT + NEW_TOKENS / 2.0
    kv_bytes = cfg.layers * mean_ctx * 2 * cfg.kv_heads * cfg.head_dim * 2
    step_bytes = weight_bytes + kv_bytes
    line = {
        "metric": "decode tok/s Qwen3-1.7B-shape bs=1/32; kernel HBM GB/s as % of MI355X peak",
        "value": round(toks, 2),
        "unit": "tok/s",
        "n_gpus": 1,
        "steps": NEW_TOKENS,
        "steps_requested": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": round(toks / REFERENCE_TOKS, 4),
        "dtype": "bf16",
        "data": "synthetic (seeded-uniform prompt ids, random-init weights ~N(0,0.02))",
        "config": {"workload": "Qwen3-1.7B-shaped greedy decode: 28 layers, hidden 2048, 16/8 heads, "
                               "head_dim 128, SwiGLU 6144, vocab 151936 tied; 64-token prompt, "
                               f"{NEW_TOKENS} new tokens",
                   "batch": 1, "prompt_tokens": PROMPT, "new_tokens": NEW_TOKENS,
                   "parallelism": "single GPU"},
        "step_hbm": {"bytes_per_step": int(step_bytes),
                     "GB/s": round(step_bytes / (ms_per_step * 1e-3) / 1e9, 1),
                     "frac": round(step_bytes / (ms_per_step * 1e-3) / 1e9 / HBM_PEAK_GBS, 4)},
        "roofline": roof,
        "hbm_copy_measured": copy_bw,
        "kernels": kernels,
        "decode_layer_bs1_ctx4096": layer,
        "first_tokens": gen.tokens[:8],
    }
    del eng
    torch.cuda.empty_cache()
    if not args.no_kernels:
        line["prompt_prefill_bs1"] = _leg(prompt_only, args.seed, args)
    if not args.no_configs:
        line["bs32"] = _leg(batch32, args.seed, NEW_TOKENS, args)
        line["mla_decode_b8_ctx8192"] = _leg(mla_decode)
        line["minicpm3_decode_bs1"] = _leg(minicpm3_decode, args.seed, args=args)
        line["prefill_attention_layer"] = _leg(prefill_layer)
    if not args.no_cpu_baseline:
        line["cpu_baseline"] = _leg(cpu_baseline, args.seed, prompt)
    else:
        line["cpu_baseline"] = None
    print(json.dumps(line))
    return 0


if __name__ == "__main__":
    sys.exit(main())
