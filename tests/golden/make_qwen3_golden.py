"""Write tests/golden/qwen3_greedy_256.json: the CPU oracle's greedy decode of
the full Qwen3-1.7B-shaped model (28 layers, vocab 151936, tied head) with the
seed-0 synthetic weights, after a 64-token seeded-uniform prompt.

Stored per generated step: the id, the oracle's top-1 / top-2 logit gap, and
the tolerance a kernel-vs-oracle disagreement must fall under to count as a
near-tie (1e-2 of the step's largest |logit|, the bf16 bar). The whole run is
the oracle alone -- nothing from the reference is imported or run.

    python tests/golden/make_qwen3_golden.py [--steps 256]
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


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--steps", type=int, default=256)
    ap.add_argument("--seed", type=int, default=0)
    ap.add_argument("--out", default=str(Path(__file__).parent / "qwen3_greedy_256.json"))
    args = ap.parse_args()
    t0 = time.time()
    cfg = QWEN3_1_7B
    wts = synthetic_weights(cfg, args.seed, "cpu")
    layers = [OQ.LayerWeights(**{k: wts[v] for k, v in hf_names(i).items()}) for i in range(cfg.layers)]
    model = OQ.ModelWeights(embed=wts["model.embed_tokens.weight"],
                            gamma_final=wts["model.norm.weight"], layers=layers)
    g = torch.Generator().manual_seed(args.seed)
    prompt = torch.randint(0, cfg.vocab, (64,), generator=g).tolist()
    print(f"weights {time.time() - t0:.0f}s", flush=True)
    rec = []
    ids = OQ.decode(model, OQ.Qwen3Config(), prompt, args.steps, record=rec, p_bf16=True)
    gaps = [r[2] for r in rec]
    tols = [1e-2 * float(r[0].abs().max()) for r in rec]
    out = {"seed": args.seed, "prompt": prompt, "tokens": ids, "gaps": gaps, "tols": tols,
           "oracle": "oracle.qwen3.decode(p_bf16=True)", "weights": "tilefoundry_amd.qwen3.synthetic_weights",
           "first_logits_sum": float(rec[0][0].double().sum()),
           "first_logits_head": [round(float(v), 5) for v in rec[0][0][:8]]}
    Path(args.out).write_text(json.dumps(out) + "\n")
    print(f"wrote {args.out}: {len(ids)} ids, min gap {min(gaps):.4g}, "
          f"{sum(g < t for g, t in zip(gaps, tols))} near-ties, {time.time() - t0:.0f}s")


if __name__ == "__main__":
    main()
