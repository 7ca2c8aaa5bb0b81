"""Writes the greedy-decoding fixtures of the seeded synthetic Qwen3 models (weights
~N(0, 0.02) from seed 0 stored as F16, RMSNorm weights 1.0, tied head, RoPE theta 1e6) on the
CPU oracle (the reference CPU worker's arithmetic, F32 execution from the F16 checkpoint):

* tests/golden/qwen3_0_6b_greedy.json: Qwen3-0.6B (28 layers, hidden 1024, 16/8 heads,
  head_dim 128, SwiGLU 3072, vocabulary 151936): 8 prompts with lengths uniform in
  [32, 512] and uniform token IDs (numpy default_rng(1)), each prefilled whole and then
  decoded for 128 greedy steps;
* tests/golden/qwen3_4b_greedy.json: Qwen3-4B at full depth (36 layers, hidden 2560, 32/8
  heads, head_dim 128, SwiGLU 9728, vocabulary 151936): two ragged prompts of 32 and 96
  uniform token IDs (numpy default_rng(2)), each prefilled whole and then decoded for 64
  greedy steps.

Per prompt and step it keeps the oracle's token, its eight largest logits (IDs and values,
descending) and the top-two margin; the GPU greedy test compares its own tokens and logits
with these. Run from the repository root:
python tests/golden/make_greedy_fixture.py [qwen3-0.6b | qwen3-4b]
(about ten minutes each on eight cores; the Qwen3-4B oracle holds 16 GB of F32 weights)."""
from __future__ import annotations

import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path.insert(0, ROOT)

import oracle  # noqa: E402
from hllm_amd import synthetic  # noqa: E402
from tests import models  # noqa: E402

HERE = os.path.dirname(os.path.abspath(__file__))
TOP = 8
# model -> (output file, prompt lengths (None: 8 uniform in [32, 512]), prompt seed, steps)
PLANS = {"qwen3-0.6b": ("qwen3_0_6b_greedy.json", None, 1, 128),
         "qwen3-4b": ("qwen3_4b_greedy.json", [32, 96], 2, 64)}


def prompts(shape, lengths=None, seed=1):
    rng = np.random.default_rng(seed)
    if lengths is None:
        lengths = rng.integers(32, 513, 8)
    return [rng.integers(0, shape.vocab, int(n)).tolist() for n in lengths]


def top_entries(logits, k=TOP):
    lg = np.asarray(logits, np.float32).reshape(-1)
    # descending value, lower ID first among equals (the first-maximum rule)
    order = np.lexsort((np.arange(lg.size), -lg.astype(np.float64)))[:k]
    return [int(i) for i in order], [float(lg[i]) for i in order]


def run(shape, prompt_list, steps, log=print):
    ost = oracle.OracleStage(models.synthetic_stage(shape, seed=0, norm_sigma=0.0))
    cases = []
    for i, p in enumerate(prompt_list):
        t0 = time.time()
        tokens, logits = ost.generate(p, steps)
        case = {"prompt": p, "tokens": [int(t) for t in tokens], "top_ids": [], "top_logits": [],
                "margin": []}
        for lg in logits:
            ids, vals = top_entries(lg)
            case["top_ids"].append(ids)
            case["top_logits"].append(vals)
            case["margin"].append(vals[0] - vals[1])
        cases.append(case)
        log(f"prompt {i}: {len(p)} tokens, {steps} steps in {time.time() - t0:.0f}s; "
            f"smallest margin {min(case['margin']):.2e}")
    return cases


def main(name="qwen3-0.6b"):
    out_name, lengths, prompt_seed, steps = PLANS[name]
    shape = synthetic.SHAPES[name]
    cases = run(shape, prompts(shape, lengths, prompt_seed), steps)
    out = os.path.join(HERE, out_name)
    with open(out, "w") as f:
        json.dump({"model": shape.name, "seed": 0, "norm_weights": 1.0, "steps": steps,
                   "top": TOP, "cases": cases}, f, separators=(",", ":"))
    print("wrote", out)


if __name__ == "__main__":
    main(*sys.argv[1:2])
