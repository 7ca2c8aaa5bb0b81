"""Sampled decode at the Falcon3-3B shape (hidden 3072, 12/4 heads, head_dim 256, SwiGLU 9216,
vocabulary 131072, untied head, no QK-norm), on a two-layer slice with the full vocabulary:
32 sequences with prompts uniform in [128, 1024] decode 8 steps together with temperature
0.8, top-p 0.9 and a per-request seed (the request index), inputs fed from the device after
the first step.

* Every pass's tokens equal the oracle's runtime::sample_token on the pass's own logits, bit
  for bit (hLLM cpp/src/sampling.cpp:19-63).
* The batched passes give the same tokens as running every sequence alone
  (tests/cpp/decode_batch_contract.hpp:8-47 at T = 0.8), and logits within 2e-2.
* The first decode pass's last-layer hidden states and logits are within max-abs 2e-2 and
  cosine 0.9999 of the F32 CPU oracle run from the same cache state."""
import numpy as np
import pytest

import oracle
from hllm_amd import capi, model, synthetic
from tests import helpers_parity as hp
from tests import models

pytestmark = pytest.mark.gpu
SHAPE = synthetic.with_layers(synthetic.FALCON3_3B, 2)
ITEMS, STEPS, MAX_ROWS, CAPACITY = 32, 8, 2048, 1100
TEMPERATURE, TOP_P = 0.8, 0.9


def _item(seq, position, index, step, from_device):
    return capi.item(seq, 1, position, from_device=from_device, temperature=TEMPERATURE,
                     top_p=TOP_P, seed=index, generated_index=step)


def test_seeded_top_p_decode_at_head_dim_256():
    hp.say("falcon3 slice: oracle weights")
    ost = oracle.OracleStage(models.synthetic_stage(SHAPE, seed=11, norm_sigma=0.1))
    cfg = model.stage_config(SHAPE, execution="f16", kv_cache_bytes=1 << 30, max_sequences=2 * ITEMS + 4,
                             max_pass_rows=MAX_ROWS, max_seq=2048)
    st = capi.Stage(cfg)
    model.synthesize(st, SHAPE, seed=11, norm_sigma=0.1)
    rng = np.random.default_rng(41)
    lengths = [int(n) for n in rng.integers(128, 1025, ITEMS)]
    prompts = [rng.integers(0, SHAPE.vocab, n) for n in lengths]
    first_ids = rng.integers(0, SHAPE.vocab, ITEMS)
    batched = [st.allocate(CAPACITY) for _ in range(ITEMS)]
    serial = [st.allocate(CAPACITY) for _ in range(ITEMS)]
    hp.say("falcon3 slice: GPU prefill of", 2 * sum(lengths), "tokens")
    hp.prefill(st, batched, lengths, MAX_ROWS, token_ids=prompts)
    hp.prefill(st, serial, lengths, MAX_ROWS, token_ids=prompts)
    oseqs = hp.oracle_sequences(ost, st, batched, CAPACITY)
    sampling = [oracle.Sampling(temperature=TEMPERATURE, top_p=TOP_P, seed=i) for i in range(ITEMS)]
    for step in range(STEPS):
        pos = [n + step for n in lengths]
        fed = step > 0
        items = [_item(s, p, i, step, fed) for i, (s, p) in enumerate(zip(batched, pos))]
        out = st.execute(items, token_ids=[0] * ITEMS if fed else first_ids, want_logits=True,
                         trace=step == 0)
        for i in range(ITEMS):
            expect = oracle.sample_token(out["logits"][i], sampling[i], step)[0]
            assert int(out["tokens"][i]) == expect, (step, i)
        if step == 0:
            hidden, logits = hp.oracle_decode(ost, oseqs, first_ids, lengths)
            hp.check_rows(out["trace"][-1], hidden, "falcon3 hidden")
            hp.check_rows(out["logits"], logits, "falcon3 logits")
        for i, (s, p) in enumerate(zip(serial, pos)):
            one = st.execute([_item(s, p, i, step, fed)], token_ids=[0] if fed else [first_ids[i]],
                             want_logits=True)
            assert int(one["tokens"][0]) == int(out["tokens"][i]), ("batched != serial", step, i)
            assert np.abs(one["logits"][0] - out["logits"][i]).max() <= hp.MAX_ABS
        hp.say(f"falcon3 step {step}: 32 sampled tokens equal the oracle's sampler and serial runs")
    for s in batched + serial:
        assert st.length(s) in {n + STEPS for n in lengths}
    st.close()
