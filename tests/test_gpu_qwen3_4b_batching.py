"""The continuous-batching workload's passes at the Qwen3-4B shape (hidden 2560, 32/8 heads,
head_dim 128, SwiGLU 9728, vocabulary 151936, QK-norm, tied head), on a two-layer slice
with the full vocabulary, against the F32 CPU oracle:

* one pass of 64 decode rows at lognormal contexts (median 256, sigma 1, clipped to
  [16, 2048]) with the projection GEMMs chosen by shape, and with each of the decode
  configurations forced (0, 1, 2: register-streaming tiles of 16/32/64 rows; 12:
  activation-staged 64 x 256 tiles; 17: the decode kernel, one weight stream per wave with
  gate/up pairs and a SwiGLU register epilogue), and the decode kernel once more with its
  deferred projections staging their activations chunk by chunk instead of whole
  (HLLM_ROCM_DECODE_WHOLE=0: the path for K ranges that do not fit in LDS);
* the same pass's greedy tokens from the LM head's argmax epilogue (no logits written) and
  from the argmax kernels over the logits: identical;
* one pass mixing a 512-token prefill chunk of a new sequence with the same 64 decode rows.

Per row: last-layer hidden state and logits within max-abs 2e-2 and cosine 0.9999."""
import os

import numpy as np
import pytest

import oracle
from hllm_amd import capi, model, synthetic
from tests import helpers_parity as hp
from tests import models

pytestmark = pytest.mark.gpu
SHAPE = synthetic.with_layers(synthetic.QWEN3_4B, 2)
ROWS, CHUNK, MAX_ROWS, CAPACITY = 64, 512, 2048, 2100


@pytest.fixture(scope="module")
def world():
    hp.say("qwen3-4b slice: oracle weights")
    ost = oracle.OracleStage(models.synthetic_stage(SHAPE, seed=7, norm_sigma=0.1))
    cfg = model.stage_config(SHAPE, execution="f16", kv_cache_bytes=1 << 30, max_sequences=2 * ROWS + 4,
                             max_pass_rows=MAX_ROWS, max_seq=4096)
    st = capi.Stage(cfg)
    model.synthesize(st, SHAPE, seed=7, norm_sigma=0.1)
    rng = np.random.default_rng(21)
    lengths = hp.lognormal_contexts(rng, ROWS)
    prompts = [rng.integers(0, SHAPE.vocab, n) for n in lengths]
    decode_ids = rng.integers(0, SHAPE.vocab, ROWS)
    chunk_ids = rng.integers(0, SHAPE.vocab, CHUNK)
    hp.say("qwen3-4b slice: GPU prefill of", sum(lengths), "tokens; cache state into the oracle")
    seqs = [st.allocate(n + 4) for n in lengths]
    hp.prefill(st, seqs, lengths, MAX_ROWS, token_ids=prompts)
    reference_kv = st.read_kv(seqs[0], 1)
    oseqs = hp.oracle_sequences(ost, st, seqs, CAPACITY)
    for s in seqs:
        st.release(s)
    hp.say("qwen3-4b slice: oracle decode rows and 512-token chunk")
    hidden, logits = hp.oracle_decode(ost, oseqs, decode_ids, lengths)
    del oseqs
    chunk_seq = ost.allocate_sequence(CAPACITY)
    tr = []
    ost.execute(np.asarray(chunk_ids, np.uint64), 0, chunk_seq, tr)
    w = {"ost": ost, "stage": st, "lengths": lengths, "prompts": prompts, "decode_ids": decode_ids,
         "hidden": hidden, "logits": logits, "chunk_ids": chunk_ids, "chunk_hidden": tr[-2],
         "chunk_logits": tr[-1], "reference_kv": reference_kv}
    yield w
    st.close()


def _fresh_sequences(w):
    """The 64 sequences prefilled again with the default GEMM choice: the same cache bits
    (the passes are deterministic; checked on one sequence)."""
    st = w["stage"]
    previous = capi.set_gemm_config(-1)
    try:
        seqs = [st.allocate(n + 4) for n in w["lengths"]]
        hp.prefill(st, seqs, w["lengths"], MAX_ROWS, token_ids=w["prompts"])
    finally:
        capi.set_gemm_config(previous)
    k, v = st.read_kv(seqs[0], 1)
    assert np.array_equal(k, w["reference_kv"][0]) and np.array_equal(v, w["reference_kv"][1])
    return seqs


def _decode_items(seqs, lengths):
    return [capi.item(s, 1, n) for s, n in zip(seqs, lengths)]


@pytest.mark.parametrize("config", [-1, 0, 1, 2, 12, 17])
def test_64_decode_rows_match_the_oracle(world, config):
    w, st = world, world["stage"]
    hp.say("qwen3-4b 64 decode rows, gemm configuration", config)
    seqs = _fresh_sequences(w)
    previous = capi.set_gemm_config(config)
    try:
        out = st.execute(_decode_items(seqs, w["lengths"]), token_ids=w["decode_ids"], want_logits=True,
                         trace=True)
    finally:
        capi.set_gemm_config(previous)
    hp.check_rows(out["trace"][-1], w["hidden"], f"config {config} hidden")
    hp.check_rows(out["logits"], w["logits"], f"config {config} logits")
    hp.greedy_agrees(out["tokens"], w["logits"], out["logits"], f"config {config}")
    for s in seqs:
        st.release(s)


def test_64_decode_rows_with_chunked_activation_staging_match_the_oracle(world):
    w, st = world, world["stage"]
    hp.say("qwen3-4b 64 decode rows, decode kernel with chunked activation staging")
    seqs = _fresh_sequences(w)
    previous = capi.set_gemm_config(17)
    before = os.environ.get("HLLM_ROCM_DECODE_WHOLE")
    os.environ["HLLM_ROCM_DECODE_WHOLE"] = "0"  # read by the launcher at every launch
    try:
        out = st.execute(_decode_items(seqs, w["lengths"]), token_ids=w["decode_ids"], want_logits=True,
                         trace=True)
    finally:
        capi.set_gemm_config(previous)
        if before is None:
            del os.environ["HLLM_ROCM_DECODE_WHOLE"]
        else:
            os.environ["HLLM_ROCM_DECODE_WHOLE"] = before
    hp.check_rows(out["trace"][-1], w["hidden"], "chunked staging hidden")
    hp.check_rows(out["logits"], w["logits"], "chunked staging logits")
    hp.greedy_agrees(out["tokens"], w["logits"], out["logits"], "chunked staging")
    for s in seqs:
        st.release(s)


def test_lm_head_argmax_epilogue_matches_the_argmax_kernels(world):
    """Greedy passes that return no logits take each row's first maximum from the LM head's
    epilogue (per-workgroup candidates, the logits never written): the same tokens as the
    argmax kernels over the logits, with HLLM_ROCM_FUSED_ARGMAX=0 (read at every pass) and
    in a pass that returns its logits, and the oracle's tokens up to near ties."""
    w, st = world, world["stage"]
    outs = {}
    for name, want, flag in (("epilogue", False, "1"), ("kernels", False, "0"), ("with logits", True, "1")):
        hp.say("qwen3-4b 64 decode rows, greedy argmax:", name)
        seqs = _fresh_sequences(w)
        before = os.environ.get("HLLM_ROCM_FUSED_ARGMAX")
        os.environ["HLLM_ROCM_FUSED_ARGMAX"] = flag
        try:
            outs[name] = st.execute(_decode_items(seqs, w["lengths"]), token_ids=w["decode_ids"], want_logits=want)
        finally:
            if before is None:
                del os.environ["HLLM_ROCM_FUSED_ARGMAX"]
            else:
                os.environ["HLLM_ROCM_FUSED_ARGMAX"] = before
        for s in seqs:
            st.release(s)
    assert np.array_equal(outs["epilogue"]["tokens"], outs["kernels"]["tokens"])
    assert np.array_equal(outs["epilogue"]["tokens"], outs["with logits"]["tokens"])
    hp.greedy_agrees(outs["epilogue"]["tokens"], w["logits"], outs["with logits"]["logits"], "argmax epilogue")


def test_512_chunk_mixed_with_64_decode_rows_matches_the_oracle(world):
    w, st = world, world["stage"]
    hp.say("qwen3-4b 512-token chunk + 64 decode rows")
    seqs = _fresh_sequences(w)
    new = st.allocate(CHUNK + 4)
    items = [capi.item(new, CHUNK, 0)] + _decode_items(seqs, w["lengths"])
    ids = np.concatenate([w["chunk_ids"], w["decode_ids"]])
    out = st.execute(items, token_ids=ids, want_logits=True, trace=True)
    last = out["trace"][-1]
    hp.check_rows(last[:CHUNK], w["chunk_hidden"], "chunk hidden")
    hp.check_rows(last[CHUNK:], w["hidden"], "decode hidden (mixed pass)")
    hp.check_rows(out["logits"][:1], w["chunk_logits"][None], "chunk logits")
    hp.check_rows(out["logits"][1:], w["logits"], "decode logits (mixed pass)")
    for s in seqs + [new]:
        st.release(s)
