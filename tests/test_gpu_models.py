"""Whole-model greedy decoding on the GPU against the CPU oracle, through the C ABI, on
the seeded synthetic Qwen3-0.6B (28 layers, full vocabulary, RMSNorm weights jittered): two
sequences prefilled in small chunks inside shared ragged passes, then decoded together with
device-fed tokens. (Qwen3-4B at full depth is checked over 65 greedy steps per sequence by
tests/test_gpu_greedy_identity.py against a committed oracle fixture.)

F32 execution must produce the oracle's greedy tokens exactly. F16 execution must produce
the first LEADING tokens exactly, and may only depart after them at a step where the
oracle's top-two logit margin is within the F16 tolerance (2e-2 per logit), after which the
sequences legitimately diverge."""
import numpy as np
import pytest

import oracle
from hllm_amd import capi, model, synthetic
from tests import models

pytestmark = [pytest.mark.gpu, pytest.mark.slow]

# F16 tokens that must equal the oracle's before any departure at a near tie (this seeded
# run measured every token equal: 11 of 11).
LEADING = 4
# model -> (prompt lengths, prefill chunk, decode steps)
PLANS = {"qwen3-0.6b": ({"a": 24, "b": 17}, 8, 10)}
SHAPES = {"qwen3-0.6b": synthetic.QWEN3_0_6B}


@pytest.fixture(scope="module", params=list(PLANS))
def oracle_run(request):
    name = request.param
    shape = SHAPES[name]
    lengths, chunk, decodes = PLANS[name]
    print(f"[gpu-case] building the {name} oracle", flush=True)
    ost = oracle.OracleStage(models.synthetic_stage(shape, seed=5, norm_sigma=0.1))
    rng = np.random.default_rng(11)
    prompts = {k: rng.integers(0, shape.vocab, n).tolist() for k, n in lengths.items()}
    ref = {k: ost.generate(p, decodes + 2, chunk=chunk) for k, p in prompts.items()}
    del ost
    return shape, prompts, chunk, decodes, ref


def _gpu_tokens(shape, prompts, chunk, decodes, execution):
    cfg = model.stage_config(shape, execution=execution, kv_cache_bytes=256 << 20, max_sequences=4,
                             max_pass_rows=64, max_seq=256)
    st = capi.Stage(cfg)
    model.synthesize(st, shape, seed=5, norm_sigma=0.1)
    seqs = {k: st.allocate(len(p) + decodes + 4) for k, p in prompts.items()}
    pos = {k: 0 for k in prompts}
    got = {k: [] for k in prompts}
    while min(len(v) for v in got.values()) < decodes + 1:
        items, ids, order = [], [], []
        for k, p in prompts.items():
            if pos[k] < len(p):
                take = min(chunk, len(p) - pos[k])
                done = pos[k] + take == len(p)
                items.append(capi.item(seqs[k], take, pos[k], sample=done))
                ids += p[pos[k]:pos[k] + take]
                pos[k] += take
                order.append((k, done))
            elif len(got[k]) < decodes + 2:
                items.append(capi.item(seqs[k], 1, pos[k], from_device=True))
                ids.append(0)
                pos[k] += 1
                order.append((k, True))
        out = st.execute(items, token_ids=ids)
        for i, (k, sampled) in enumerate(order):
            if sampled:
                got[k].append(int(out["tokens"][i]))
    st.close()
    return got


def test_f32_greedy_tokens_equal_the_oracle(oracle_run):
    shape, prompts, chunk, decodes, ref = oracle_run
    got = _gpu_tokens(shape, prompts, chunk, decodes, "f32")
    for k in prompts:
        n = min(len(got[k]), len(ref[k][0]))
        assert n >= decodes + 1
        assert got[k][:n] == ref[k][0][:n], k


def test_f16_greedy_departs_only_at_near_ties(oracle_run):
    shape, prompts, chunk, decodes, ref = oracle_run
    got = _gpu_tokens(shape, prompts, chunk, decodes, "f16")
    for k in prompts:
        tokens, logits = ref[k]
        same = 0
        for g, r in zip(got[k], tokens):
            if g != r:
                break
            same += 1
        n = min(len(got[k]), len(tokens))
        print(f"[gpu-case] {k}: {same} of {n} leading tokens equal", flush=True)
        # At least the first LEADING tokens (prefill's and the first decode steps') agree.
        assert same >= min(n, LEADING), (k, same)
        for step, (g, r) in enumerate(zip(got[k], tokens)):
            if g == r:
                continue
            top2 = np.sort(np.asarray(logits[step]).reshape(-1))[-2:]
            margin = float(top2[1] - top2[0])
            assert margin <= 4e-2, (k, step, margin)
            break  # the sequences differ from here on
