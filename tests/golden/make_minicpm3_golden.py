"""Write the CPU oracle's greedy decode of the full MiniCPM3-4B-shaped model
(62 layers, vocab 73448, tied head, seed-0 synthetic weights) that the
full-model GPU test compares against: ``minicpm3_greedy_256.json``.

The prompt is the MiniCPM3 decode benchmark's: 8 ids drawn by
``torch.randint(0, 73448, (8,), generator=torch.Generator().manual_seed(seed + 3))``.

* ``free``: the oracle's free greedy run of 256 ids over the bf16 logits the
  model returns. With random weights this model settles on one id at once
  (the same id at every step), so it is kept as a check of the free run only;
* ``forced``: 256 positions teacher-forced along seeded uniform-random ids
  (``torch.randint(0, 73448, (255,), generator=torch.Generator().manual_seed(seed + 11))``),
  so that the pick differs from position to position: per position the
  oracle's pick, its top-1 / top-2 gap and its 16 largest logits with their
  ids, and how far the oracle's other valid order (f32 softmax weights into
  the latent sum instead of bf16) lies from these logits along the same ids
  (``order_spread``).

A test can then measure the GPU logits' error at the candidates that decide
each pick. The whole run is the oracle alone -- nothing from the reference is
imported or run. About 45 minutes on 8 cores.

    python tests/golden/make_minicpm3_golden.py [--steps 256] [--seed 0]
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

from oracle import minicpm3 as OM  # noqa: E402
from tilefoundry_amd.minicpm3 import MINICPM3_4B, hf_layer_names, synthetic_model_weights  # noqa: E402

TOPK = 16
PROMPT = 8


def oracle_config(cfg) -> OM.ModelConfig:
    return OM.ModelConfig(hidden=cfg.hidden, heads=cfg.heads, q_lora=cfg.q_lora, kv_lora=cfg.kv_lora,
                          nope=cfg.nope, rope=cfg.rope, v_dim=cfg.v_dim, eps=cfg.eps, lora_eps=cfg.lora_eps,
                          rope_theta=cfg.rope_theta, inter=cfg.inter, vocab=cfg.vocab, layers=cfg.layers,
                          scale_emb=cfg.scale_emb, dim_model_base=cfg.dim_model_base,
                          scale_depth=cfg.scale_depth)


def _model(cfg, seed):
    wts = synthetic_model_weights(cfg, seed)
    layers = [OM.LayerWeights(**{k: wts[v] for k, v in hf_layer_names(i).items()}) for i in range(cfg.layers)]
    return OM.ModelWeights(embed=wts["model.embed_tokens.weight"], gamma_final=wts["model.norm.weight"],
                           layers=layers)


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--steps", type=int, default=256)
    ap.add_argument("--seed", type=int, default=0)
    args = ap.parse_args()
    t0 = time.time()
    cfg = MINICPM3_4B
    ocfg = oracle_config(cfg)
    model = _model(cfg, args.seed)
    print(f"weights {time.time() - t0:.0f}s", flush=True)
    prompt = torch.randint(0, cfg.vocab, (PROMPT,), generator=torch.Generator().manual_seed(args.seed + 3)).tolist()
    free = OM.decode(model, ocfg, prompt, args.steps, p_bf16=True)
    print(f"free run {time.time() - t0:.0f}s", flush=True)
    teacher = torch.randint(0, cfg.vocab, (args.steps - 1,),
                            generator=torch.Generator().manual_seed(args.seed + 11)).tolist()
    rec = []
    picks = OM.decode(model, ocfg, prompt, args.steps, record=rec, p_bf16=True, teacher=teacher)
    print(f"forced {time.time() - t0:.0f}s", flush=True)
    alt = []
    OM.decode(model, ocfg, prompt, args.steps, record=alt, p_bf16=False, teacher=teacher)
    print(f"other order {time.time() - t0:.0f}s", flush=True)
    top_ids, top_vals, gaps, spread = [], [], [], []
    for (lg, _, _), (la, _, _) in zip(rec, alt):
        top = torch.topk(lg, TOPK)
        top_ids.append(top.indices.tolist())
        top_vals.append([float(v) for v in top.values])
        gaps.append(float(top.values[0] - top.values[1]))
        spread.append(float((la[top.indices].double() - top.values.double()).abs().max()))
    alt_agree = sum(int(r[1] == t) for r, t in zip(alt, picks))
    data = {"seed": args.seed, "prompt": prompt,
            "free": {"tokens": free, "oracle": "oracle.minicpm3.decode(p_bf16=True)"},
            "forced": {"teacher_seed": args.seed + 11, "teacher": teacher, "tokens": picks,
                       "order_spread": {"what": "oracle p_bf16=False along the same teacher: per-position max "
                                                "|logit - golden logit| over the 16 candidates, and its picks' "
                                                "agreement", "deltas": spread, "agree": alt_agree},
                       "gaps": gaps, "top_ids": top_ids, "top_vals": top_vals,
                       "oracle": "oracle.minicpm3.decode(p_bf16=True, teacher=teacher)"},
            "weights": "tilefoundry_amd.minicpm3.synthetic_model_weights",
            "first_logits_head": [round(float(v), 5) for v in rec[0][0][:8]]}
    out = Path(__file__).parent / "minicpm3_greedy_256.json"
    out.write_text(json.dumps(data) + "\n")
    print(f"wrote {out}: free run {len(set(free))} distinct ids; forced {len(set(picks))} distinct picks, "
          f"orders agree {alt_agree}/{len(picks)}, min gap {min(gaps):.4g}, {time.time() - t0:.0f}s", flush=True)


if __name__ == "__main__":
    main()
