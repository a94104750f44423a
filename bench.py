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
"""
from __future__ import annotations

import argparse
import json
import os
import platform
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

    ms = _events_time(one_pass, 20) / len(layers)
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
    it = [0]

    def add_norm():
        x, r = sets[it[0] % 8]
        it[0] += 1
        C.add_rms_norm(x, r, gamma, y, ro, 1e-6, 0)

    ms = _events_time(add_norm, 80)
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
        return _events_time(lambda: [fn(w) for w in L], 10) / len(L)

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
    ms = _events_time(lambda: C.lm_head_argmax(eng.hid, eng.gamma_final, cfg.eps, eng.embed,
                                               eng.logits, eng.bv, eng.bi), 20)
    nbytes = cfg.vocab * H * 2
    gbs = nbytes / (ms * 1e-3) / 1e9
    out["lm_head_151936x2048"] = {"us": round(ms * 1e3, 2), "GB/s": round(gbs, 1),
                                  "frac": round(gbs / HBM_PEAK_GBS, 4), "bytes": nbytes}
    return out


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
    ap.add_argument("--kernel-only", action="store_true",
                    help="only launch the dominant kernel loop (for rocprofv3 counter runs)")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU: the decode path runs on a single MI355X; "
              "run with --gpus 1 (multi-GPU sharding is described, not run).", file=sys.stderr)
        return 2
    if not torch.cuda.is_available():
        print("bench.py needs a GPU", file=sys.stderr)
        return 2

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
        "first_tokens": gen.tokens[:8],
    }
    if not args.no_cpu_baseline:
        del eng
        torch.cuda.empty_cache()
        line["cpu_baseline"] = cpu_baseline(args.seed, prompt)
    else:
        line["cpu_baseline"] = None
    print(json.dumps(line))
    return 0


if __name__ == "__main__":
    sys.exit(main())
