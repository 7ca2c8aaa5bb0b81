"""The committed greedy fixture (tests/golden/qwen3_0_6b_greedy.json) is the oracle's output:
its shortest prompt's first steps recomputed on the CPU give the same tokens and the same
top-8 logits bit for bit."""
import json
import os

import numpy as np

import oracle
from hllm_amd import synthetic
from tests import models

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden",
                      "qwen3_0_6b_greedy.json")


def test_greedy_fixture_is_the_oracle():
    with open(GOLDEN) as f:
        fx = json.load(f)
    assert fx["steps"] >= 64 and len(fx["cases"]) == 8
    shape = synthetic.QWEN3_0_6B
    for c in fx["cases"]:
        assert 32 <= len(c["prompt"]) <= 512 and len(c["tokens"]) == fx["steps"] + 1
    case = min(fx["cases"], key=lambda c: len(c["prompt"]))
    ost = oracle.OracleStage(models.synthetic_stage(shape, seed=0, norm_sigma=0.0))
    tokens, logits = ost.generate(case["prompt"], 3)
    assert tokens == case["tokens"][:4]
    for step, lg in enumerate(logits):
        assert np.array_equal(lg[case["top_ids"][step]], np.float32(case["top_logits"][step]))
        assert int(np.argmax(lg)) == case["top_ids"][step][0]
