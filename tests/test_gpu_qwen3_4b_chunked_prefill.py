"""Chunked prefill at the Qwen3-4B shape against the oracle run from scratch.

A two-layer slice at the real Qwen3-4B widths (hidden 2560, 32/8 heads, head_dim 128, SwiGLU
9728, vocabulary 151936, QK-norm, tied head; F16 weights from seed 3, RMSNorm weights
jittered) prefills one 2048-token sequence on the GPU in four 512-token chunks: positions 0,
512, 1024 and 1536, the continuous-batching workload's chunk size, the last one at the past
of the benchmark's second prefill point. The oracle (the reference CPU worker's arithmetic in
F32) prefills the same 2048 tokens in one pass: chunking must not change what the stage
computes (the reference's rule, tests/integration/test_chunked_prefill.py:18-76), so nothing
on the oracle's side comes from the GPU.

Compared, each within max-abs 2e-2 and cosine 0.9999 per row (F16 execution against F32):
* every layer's cached keys and values at all 2048 positions;
* the last chunk's hidden state after each layer (512 rows);
* the last row's logits over the whole vocabulary, and its greedy token unless the oracle's
  top two logits lie within 4e-2 of each other."""
import numpy as np
import pytest

import oracle
from hllm_amd import capi, model, synthetic
from tests import helpers_parity as hp
from tests import models

pytestmark = pytest.mark.gpu
SHAPE = synthetic.with_layers(synthetic.QWEN3_4B, 2)
TOKENS, CHUNK, SEED = 2048, 512, 3


@pytest.fixture(scope="module")
def reference():
    hp.say("qwen3-4b chunked prefill: oracle weights and one-pass prefill of", TOKENS, "tokens")
    ost = oracle.OracleStage(models.synthetic_stage(SHAPE, seed=SEED, norm_sigma=0.1))
    ids = np.random.default_rng(31).integers(0, SHAPE.vocab, TOKENS).astype(np.uint64)
    seq = ost.allocate_sequence(TOKENS + 1)
    trace = []
    out = ost.execute(ids, 0, seq, trace)
    kv = [seq.cache_arrays(layer) for layer in range(SHAPE.layers)]
    hidden = [t[TOKENS - CHUNK:] for t in trace[:SHAPE.layers]]
    return {"ids": ids, "kv": kv, "hidden": hidden, "logits": trace[-1], "token": out[1]}


def test_four_512_token_chunks_match_the_oracle_run_from_scratch(reference):
    cfg = model.stage_config(SHAPE, execution="f16", kv_cache_bytes=1 << 30, max_sequences=4,
                             max_pass_rows=CHUNK, max_seq=4096)
    st = capi.Stage(cfg)
    model.synthesize(st, SHAPE, seed=SEED, norm_sigma=0.1)
    s = st.allocate(TOKENS + 1)
    ids = reference["ids"]
    for pos in range(0, TOKENS, CHUNK):
        last = pos + CHUNK == TOKENS
        hp.say("qwen3-4b chunked prefill: chunk at", pos)
        out = st.execute([capi.item(s, CHUNK, pos, sample=last)], token_ids=ids[pos:pos + CHUNK],
                         want_logits=last, trace=last)
    assert st.length(s) == TOKENS
    for layer in range(SHAPE.layers):
        k, v = st.read_kv(s, layer)
        rk, rv = reference["kv"][layer]
        hp.check_rows(k.reshape(TOKENS, -1), rk.reshape(TOKENS, -1), f"layer {layer} keys")
        hp.check_rows(v.reshape(TOKENS, -1), rv.reshape(TOKENS, -1), f"layer {layer} values")
        hp.check_rows(out["trace"][layer], reference["hidden"][layer], f"layer {layer} last-chunk hidden")
    hp.check_rows(out["logits"], reference["logits"].reshape(1, -1), "last-row logits")
    lg = np.asarray(reference["logits"], np.float64)
    top2 = np.sort(lg)[-2:]
    if top2[1] - top2[0] > 4e-2:
        assert int(out["tokens"][0]) == reference["token"]
    hp.say("qwen3-4b chunked prefill: token", int(out["tokens"][0]), "oracle", reference["token"],
           "oracle top-2 margin", float(top2[1] - top2[0]))
    st.close()
