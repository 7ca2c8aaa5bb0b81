"""Writes tests/golden/sampling_vectors.json: sampled tokens and log-probabilities for
fixed logits under a spread of sampling options, computed by the oracle's sampler (which
tests/test_oracle.py pins bit for bit to the reference's cpp/src/sampling.cpp). Used by
the host sampler test in tests/host/host_tests.cpp.

    python tests/golden/make_sampling_vectors.py
"""
import itertools
import json
import os
import sys

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path.insert(0, ROOT)
import oracle  # noqa: E402


def main():
    rng = np.random.default_rng(7)
    sets = [
        np.array([1.0, 3.0, 3.0, 2.0, -1.0], np.float32),           # a tie at the maximum
        np.array([0.5] * 6 + [0.25] * 2, np.float32),                # many equal probabilities
        (rng.standard_normal(1000) * 3.0).astype(np.float32),       # a vocabulary-like spread
        (rng.standard_normal(257) * 0.2).astype(np.float32),        # nearly flat
    ]
    cases = []
    grid = itertools.product(range(len(sets)), (0.0, 0.5, 0.8, 1.3), (1.0, 0.9, 0.5), (0, 1, 8, 50))
    for n, (li, t, p, k) in enumerate(grid):
        if n % 3:  # a third of the grid keeps the file small while covering every option
            continue
        seed, index = 11 + 13 * n, (0, 5, 77)[n % 3]
        logprobs = n % 2 == 0
        top = (0, 3, 5)[n % 3] if logprobs else 0
        s = oracle.Sampling(temperature=t, top_p=p, top_k=k, seed=seed, return_logprobs=logprobs,
                            top_logprobs=top)
        tok, lp, tops = oracle.sample_token(sets[li], s, index)
        case = {"logits_index": li, "temperature": t, "top_p": p, "top_k": k, "seed": seed,
                "generated_index": index, "return_logprobs": logprobs, "top_logprobs": top, "token": tok}
        if logprobs:
            case.update(logprob=lp, top_ids=[i for i, _ in tops], top_values=[v for _, v in tops])
        cases.append(case)
    doc = {"source": "oracle.sample_token (pinned to cpp/src/sampling.cpp)",
           "logits": [[float(x) for x in s] for s in sets], "cases": cases}
    path = os.path.join(ROOT, "tests", "golden", "sampling_vectors.json")
    with open(path, "w") as f:
        json.dump(doc, f, separators=(",", ":"))
    print(f"wrote {len(cases)} cases to {path}")


if __name__ == "__main__":
    main()
