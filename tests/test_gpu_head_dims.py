"""The MFMA attention at head dims 64 and 256 against the oracle, from a ragged prefill
through decode rows whose key ranges split.

The attention kernel is compiled for head dims 64, 128 and 256; the Qwen3 slices cover 128.
Two slices at the other dims, F16 execution, seeded synthetic weights (RMSNorm weights
jittered):
* head_dim 64: a Llama-3.2-1B-shaped slice (hidden 2048, 32 / 8 heads, SwiGLU 8192, no
  QK-norm, untied head, rope theta 5e5), two layers, a vocabulary of 4096;
* head_dim 256: a Falcon3-3B-shaped slice (hidden 3072, 12 / 4 heads, SwiGLU 9216), one
  layer, a vocabulary of 8192.
Three sequences of 1200, 700 and 40 tokens are prefilled together in ragged passes of at
most 512 rows (prefill blocks over up to 1200 keys, split in two past 1024), then three decode
passes run the three rows together (the 1200- and 700-token rows' key ranges split in three
and two and are merged inside the attention kernel). The oracle (the reference CPU worker's
arithmetic in F32) runs the same tokens from scratch, one sequence at a time. Compared: every
layer's keys and values after the prefill and each decode pass's logits, per row within
max-abs 2e-2 and cosine 0.9999; the decode passes' greedy tokens equal the oracle's except
at near ties (tests/helpers_parity.py)."""
from dataclasses import replace

import numpy as np
import pytest

import oracle
from hllm_amd import capi, model, synthetic
from tests import helpers_parity as hp
from tests import models

pytestmark = pytest.mark.gpu

SHAPES = {
    "d64-llama": synthetic.ModelShape("d64-llama", 2, 2048, 8192, 32, 8, 64, 4096, eps=1e-5,
                                      theta=5e5, qk_norm=False, tied=False),
    "d256-falcon3": replace(synthetic.FALCON3_3B, layers=1, vocab=8192),
}
LENGTHS, SEED, STEPS = (1200, 700, 40), 6, 3


@pytest.mark.parametrize("name", list(SHAPES))
def test_ragged_prefill_and_split_decode_match_the_oracle(name):
    shape = SHAPES[name]
    rng = np.random.default_rng(17)
    prompts = [rng.integers(0, shape.vocab, n).astype(np.uint64) for n in LENGTHS]
    decode_ids = rng.integers(0, shape.vocab, (STEPS, len(LENGTHS))).astype(np.uint64)

    hp.say(name, "oracle prefill of", sum(LENGTHS), "tokens")
    ost = oracle.OracleStage(models.synthetic_stage(shape, seed=SEED, norm_sigma=0.1))
    oseqs = [ost.allocate_sequence(n + STEPS + 1) for n in LENGTHS]
    for o, p in zip(oseqs, prompts):
        o.prefill_only = True
        ost.execute(p, 0, o)
        o.prefill_only = False

    cfg = model.stage_config(shape, execution="f16", kv_cache_bytes=256 << 20, max_sequences=4,
                             max_pass_rows=512, max_seq=2048)
    st = capi.Stage(cfg)
    model.synthesize(st, shape, seed=SEED, norm_sigma=0.1)
    seqs = [st.allocate(n + STEPS + 1) for n in LENGTHS]
    hp.prefill(st, seqs, LENGTHS, 512, token_ids=prompts)
    for layer in range(shape.layers):
        for s, o, n in zip(seqs, oseqs, LENGTHS):
            k, v = st.read_kv(s, layer)
            rk, rv = o.cache_arrays(layer)
            hp.check_rows(k.reshape(n, -1), rk.reshape(n, -1), f"{name} layer {layer} keys ({n} tokens)")
            hp.check_rows(v.reshape(n, -1), rv.reshape(n, -1), f"{name} layer {layer} values ({n} tokens)")

    for step in range(STEPS):
        positions = [n + step for n in LENGTHS]
        items = [capi.item(s, 1, pos) for s, pos in zip(seqs, positions)]
        out = st.execute(items, token_ids=decode_ids[step], want_logits=True)
        expect = []
        for o, pos, tok in zip(oseqs, positions, decode_ids[step]):
            tr = []
            ost.execute(np.array([tok], np.uint64), pos, o, tr)
            expect.append(tr[-1])
        expect = np.stack(expect)
        hp.check_rows(out["logits"], expect, f"{name} decode pass {step} logits")
        hp.greedy_agrees(out["tokens"], expect, out["logits"], f"{name} decode pass {step}")
    st.close()
