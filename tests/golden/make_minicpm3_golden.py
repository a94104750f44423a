"""Write the CPU oracle's greedy decode of the full MiniCPM3-4B-shaped model
(62 layers, vocab 73448, tied head, seed-0 synthetic weights) that the
full-model GPU test compares against: ``minicpm3_greedy_256.json``.

The prompt is the MiniCPM3 decode benchmark's: 8 ids drawn by
``torch.randint(0, 73448, (8,), generator=torch.Generator().manual_seed(seed + 3))``.
Then 256 greedy ids over the bf16 logits the model returns, and with them how
far the oracle's other valid order (f32 softmax weights into the latent sum
instead of bf16) lies from these logits along the same ids (``order_spread``).
Stored per generated step: the id, the oracle's top-1 / top-2 gap and its 16
largest logits with their ids, so that a test can measure the GPU logits' error
at the candidates that decide the pick. The whole run is the oracle alone --
nothing from the reference is imported or run. About 25 minutes on 8 cores.

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
    rec = []
    ids = OM.decode(model, ocfg, prompt, args.steps, record=rec, p_bf16=True)
    print(f"decode {time.time() - t0:.0f}s", flush=True)
    alt = []
    OM.decode(model, ocfg, prompt, args.steps, record=alt, p_bf16=False, teacher=ids)
    print(f"other order {time.time() - t0:.0f}s", flush=True)
    top_ids, top_vals, gaps, spread = [], [], [], []
    for (lg, _, _), (la, _, _) in zip(rec, alt):
        top = torch.topk(lg, TOPK)
        top_ids.append(top.indices.tolist())
        top_vals.append([float(v) for v in top.values])
        gaps.append(float(top.values[0] - top.values[1]))
        spread.append(float((la[top.indices].double() - top.values.double()).abs().max()))
    alt_agree = sum(int(r[1] == t) for r, t in zip(alt, ids))
    data = {"seed": args.seed, "prompt": prompt, "tokens": ids,
            "order_spread": {"what": "oracle p_bf16=False teacher-forced along these ids: per-position max "
                                     "|logit - golden logit| over the 16 candidates, and its picks' agreement",
                             "deltas": spread, "agree": alt_agree},
            "gaps": gaps, "top_ids": top_ids, "top_vals": top_vals,
            "oracle": "oracle.minicpm3.decode(p_bf16=True)",
            "weights": "tilefoundry_amd.minicpm3.synthetic_model_weights",
            "first_logits_head": [round(float(v), 5) for v in rec[0][0][:8]]}
    out = Path(__file__).parent / "minicpm3_greedy_256.json"
    out.write_text(json.dumps(data) + "\n")
    print(f"wrote {out}: {len(ids)} ids, orders agree {alt_agree}/{len(ids)}, min gap {min(gaps):.4g}, "
          f"{time.time() - t0:.0f}s", flush=True)


if __name__ == "__main__":
    main()
