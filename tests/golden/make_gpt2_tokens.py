"""Writes tests/golden/gpt2_c1_greedy.json: the greedy token sequence of
BASELINE config 1 (GPT-2 small, random fp32 weights N(0, 0.02) from
numpy default_rng(0), a 64-token prompt uniform over the vocabulary,
32 greedy tokens) computed by the CPU oracle's op chain (oracle/gpt2.py), with
each step's top-1 minus top-2 logit margin.  Takes a minute or two on one
core.  Run from the repository root: python tests/golden/make_gpt2_tokens.py"""
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path.insert(0, ROOT)

from oracle import oracle as O  # noqa: E402
from oracle.gpt2 import GPT2Oracle  # noqa: E402
from sandyrt_amd.gpt2 import GPT2Config, prompt_ids, random_weights  # noqa: E402


def main():
    cfg = GPT2Config()
    if not os.path.exists(O.LIB_PATH):
        O.build()
    w = random_weights(cfg, seed=0)
    prompt = prompt_ids(cfg, 64, seed=0)
    t0 = time.perf_counter()
    tokens, margins = GPT2Oracle(O.Oracle(), cfg, w).greedy(prompt, 32)
    secs = time.perf_counter() - t0
    out = {"config": "GPT-2 small (12 layers, d 768, 12 heads, FFN 3072, vocab 50257), fp32 weights N(0, 0.02) "
                     "numpy default_rng(0), LayerNorm gain 1 / shift 0; prompt default_rng([0, 1]) 64 ids",
           "prompt": prompt, "tokens": tokens, "margins": margins, "oracle_seconds": round(secs, 1)}
    path = os.path.join(ROOT, "tests", "golden", "gpt2_c1_greedy.json")
    with open(path, "w") as f:
        json.dump(out, f, indent=1)
    print(f"wrote {path}: {tokens} in {secs:.1f} s; min margin {min(margins):.3g}")


if __name__ == "__main__":
    main()
