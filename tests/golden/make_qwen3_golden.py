"""Write the CPU oracle's greedy decodes of the full Qwen3-1.7B-shaped model
(28 layers, vocab 151936, tied head, seed-0 synthetic weights) that the
full-model GPU tests compare against:

* ``qwen3_greedy_256.json`` -- one sequence: a 64-token seeded-uniform prompt,
  then 256 greedy ids; with them, how far the oracle's other valid order (f32
  softmax weights into P.V instead of bf16) lies from these logits along the
  same ids (``order_spread``): the model's own sensitivity to rounding order;
* ``qwen3_batch_golden.json`` -- the first 4 of 32 seeded 64-token prompts
  (``oracle.qwen3.prompt_ids(vocab, 64, seed=7, batch=32)``), 32 greedy ids
  each, stepped together (``oracle.qwen3.step_batch``).

Stored per generated step: the id, the oracle's top-1 / top-2 logit gap, the
old fixed near-tie tolerance (1e-2 of the step's largest |logit|), and the
oracle's 16 largest logits with their ids, so that a test can measure the GPU
logits' error at the candidates that decide the pick. The whole run is the
oracle alone -- nothing from the reference is imported or run.

    python tests/golden/make_qwen3_golden.py [--steps 256] [--batch-only]
"""
from __future__ import annotations

import argparse
import json
import sys
import time
from pathlib import Path

import torch

ROOT = Path(__file__).resolve().parents[2]
sys.path.insert(0, str(ROOT))

from oracle import qwen3 as OQ  # noqa: E402
from tilefoundry_amd.qwen3 import QWEN3_1_7B, hf_names, synthetic_weights  # noqa: E402

TOPK = 16


def _model(seed):
    cfg = QWEN3_1_7B
    wts = synthetic_weights(cfg, seed, "cpu")
    layers = [OQ.LayerWeights(**{k: wts[v] for k, v in hf_names(i).items()}) for i in range(cfg.layers)]
    return OQ.ModelWeights(embed=wts["model.embed_tokens.weight"], gamma_final=wts["model.norm.weight"],
                           layers=layers)


def _step_record(logits):
    top = torch.topk(logits, TOPK)
    return {"gap": float(top.values[0] - top.values[1]), "tol": 1e-2 * float(logits.abs().max()),
            "top_ids": top.indices.tolist(), "top_vals": [float(v) for v in top.values]}


def single(model, seed, steps, out):
    t0 = time.time()
    cfg = QWEN3_1_7B
    g = torch.Generator().manual_seed(seed)
    prompt = torch.randint(0, cfg.vocab, (64,), generator=g).tolist()
    rec = []
    ids = OQ.decode(model, OQ.Qwen3Config(), prompt, steps, record=rec, p_bf16=True)
    steps_rec = [_step_record(r[0]) for r in rec]
    # the oracle's other valid order (f32 softmax weights into P.V), teacher-forced
    # along the same ids: how far two correct orders of this model lie apart
    alt = []
    OQ.decode(model, OQ.Qwen3Config(), prompt, steps, teacher=ids, record=alt, p_bf16=False)
    spread = []
    for s, (lg, _, _) in zip(steps_rec, alt):
        top = torch.tensor(s["top_ids"])
        spread.append(float((lg[top].double() - torch.tensor(s["top_vals"], dtype=torch.float64)).abs().max()))
    alt_agree = sum(int(r[1] == t) for r, t in zip(alt, ids))
    data = {"seed": seed, "prompt": prompt, "tokens": ids,
            "order_spread": {"what": "oracle p_bf16=False teacher-forced along these ids: per-position max "
                                     "|logit - golden logit| over the 16 candidates, and its picks' agreement",
                             "deltas": spread, "agree": alt_agree},
            "gaps": [s["gap"] for s in steps_rec], "tols": [s["tol"] for s in steps_rec],
            "top_ids": [s["top_ids"] for s in steps_rec], "top_vals": [s["top_vals"] for s in steps_rec],
            "oracle": "oracle.qwen3.decode(p_bf16=True)", "weights": "tilefoundry_amd.qwen3.synthetic_weights",
            "first_logits_sum": float(rec[0][0].double().sum()),
            "first_logits_head": [round(float(v), 5) for v in rec[0][0][:8]]}
    Path(out).write_text(json.dumps(data) + "\n")
    print(f"wrote {out}: {len(ids)} ids, min gap {min(data['gaps']):.4g}, {time.time() - t0:.0f}s", flush=True)


def batch(model, seed, steps, out, keep=4, prompt_len=64):
    t0 = time.time()
    cfg = QWEN3_1_7B
    ocfg = OQ.Qwen3Config()
    prompts = OQ.prompt_ids(cfg.vocab, prompt_len, seed=7, batch=32)[:keep]
    cos, sin = OQ.rope_tables(prompt_len + steps, ocfg.head_dim, ocfg.rope_theta)
    caches = [OQ.empty_caches(ocfg, ocfg.layers) for _ in range(keep)]
    for p in range(prompt_len):
        logits = OQ.step_batch(model, ocfg, [r[p] for r in prompts], [p] * keep, caches, cos, sin, p_bf16=True)
    toks = [[] for _ in range(keep)]
    recs = [[] for _ in range(keep)]
    for i in range(steps):
        picks = [int(torch.argmax(logits[b])) for b in range(keep)]
        for b in range(keep):
            toks[b].append(picks[b])
            recs[b].append(_step_record(logits[b]))
        if i + 1 < steps:
            logits = OQ.step_batch(model, ocfg, picks, [prompt_len + i] * keep, caches, cos, sin, p_bf16=True)
    data = {"seed": seed, "prompt_seed": 7, "batch": 32, "kept": keep, "prompts": prompts, "tokens": toks,
            "gaps": [[s["gap"] for s in r] for r in recs], "top_ids": [[s["top_ids"] for s in r] for r in recs],
            "top_vals": [[s["top_vals"] for s in r] for r in recs],
            "oracle": "oracle.qwen3.step_batch(p_bf16=True)", "weights": "tilefoundry_amd.qwen3.synthetic_weights"}
    Path(out).write_text(json.dumps(data) + "\n")
    print(f"wrote {out}: {keep} x {steps} ids, {time.time() - t0:.0f}s", flush=True)


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--steps", type=int, default=256)
    ap.add_argument("--batch-steps", type=int, default=32)
    ap.add_argument("--seed", type=int, default=0)
    ap.add_argument("--batch-only", action="store_true")
    ap.add_argument("--single-only", action="store_true")
    args = ap.parse_args()
    here = Path(__file__).parent
    model = _model(args.seed)
    if not args.batch_only:
        single(model, args.seed, args.steps, here / "qwen3_greedy_256.json")
    if not args.single_only:
        batch(model, args.seed, args.batch_steps, here / "qwen3_batch_golden.json")


if __name__ == "__main__":
    main()
