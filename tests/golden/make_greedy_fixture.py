"""Writes tests/golden/qwen3_0_6b_greedy.json: greedy decoding of the seeded synthetic
Qwen3-0.6B (28 layers, hidden 1024, 16/8 heads, head_dim 128, SwiGLU 3072, vocabulary
151936, tied head, RoPE theta 1e6; weights ~N(0, 0.02) from seed 0 stored as F16, RMSNorm
weights 1.0) on the CPU oracle (the reference CPU worker's arithmetic, F32 execution from
the F16 checkpoint): 8 prompts with lengths uniform in [32, 512] and uniform token IDs
(numpy default_rng(1)), each prefilled whole and then decoded for 128 greedy steps.

Per prompt and step it keeps the oracle's token, its eight largest logits (IDs and values,
descending) and the top-two margin; the GPU greedy test compares its own tokens and logits
with these. Run from the repository root: python tests/golden/make_greedy_fixture.py
(about ten minutes on eight cores)."""
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

OUT = os.path.join(os.path.dirname(os.path.abspath(__file__)), "qwen3_0_6b_greedy.json")
PROMPTS, STEPS, TOP = 8, 128, 8


def prompts(shape, count=PROMPTS):
    rng = np.random.default_rng(1)
    lengths = rng.integers(32, 513, count)
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


def main():
    shape = synthetic.QWEN3_0_6B
    cases = run(shape, prompts(shape), STEPS)
    with open(OUT, "w") as f:
        json.dump({"model": shape.name, "seed": 0, "norm_weights": 1.0, "steps": STEPS,
                   "top": TOP, "cases": cases}, f, separators=(",", ":"))
    print("wrote", OUT)


if __name__ == "__main__":
    main()
