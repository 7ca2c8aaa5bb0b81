"""Every projection GEMM forced onto one configuration of the kernel table (through
hllm_rocm_set_gemm_config): a ragged pass with a 512-token prefill chunk and decode rows, then
a decode pass, of a Qwen3-0.6B-shaped two-layer slice in F16 execution, against the F32 CPU
oracle run per sequence. Covers the configurations that copy both operands into LDS (128-,
192- and 256-row tiles, four and eight waves), the activation-staged kernel (64- and 128-row
tiles: 12, 9), the register-streaming kernel (16-, 32- and 64-row tiles: 0, 1, 2; the
choice for plain and F32-execution projections of at most 64 rows), the decode kernel
(17: the projections it takes in passes of at most 64 rows) and the choice by shape (-1) on
every epilogue: deferred K-split partials (q/k/v), residual accumulation (o, down), SwiGLU
(gate+up) and plain stores (LM head), for row counts from 2 to 554. Bounds: max-abs <= 2e-2
and cosine >= 0.9999, as for the other F16 slices."""
import numpy as np
import pytest

import oracle
from hllm_amd import capi, model, synthetic
from tests import models
from tests.test_gpu_stage import cosine, within

pytestmark = pytest.mark.gpu
SHAPE = synthetic.with_layers(synthetic.QWEN3_0_6B, 2)
LENGTHS = (37, 5, 602)


def _say(*what):
    print("[gpu-case]", *what, flush=True)


@pytest.fixture(scope="module")
def expected():
    """Oracle traces: pass 1 (sequences 0 and 1 whole, the first 512 tokens of sequence 2),
    pass 2 (one decode token each for 0 and 1, the remaining 90 tokens of 2)."""
    ost = oracle.OracleStage(models.synthetic_stage(SHAPE, seed=4, norm_sigma=0.1))
    rng = np.random.default_rng(6)
    prompts = [rng.integers(0, SHAPE.vocab, n).tolist() for n in LENGTHS]
    seqs = [ost.allocate_sequence(640) for _ in LENGTHS]
    first, logits, tokens = [], [], []
    for s, p in zip(seqs[:2], prompts[:2]):
        tr = []
        ref = ost.execute(np.array(p, np.uint64), 0, s, tr)
        first.append(tr[1])
        logits.append(tr[2])
        tokens.append(ref[1])
    seqs[2].prefill_only = True
    tr = []
    ost.execute(np.array(prompts[2][:512], np.uint64), 0, seqs[2], tr)
    first.append(tr[1])
    seqs[2].prefill_only = False
    second = []
    for s, t, n in zip(seqs[:2], tokens, LENGTHS[:2]):
        tr = []
        ost.execute(np.array([t], np.uint64), n, s, tr)
        second.append(tr[2])
    tr = []
    ost.execute(np.array(prompts[2][512:], np.uint64), 512, seqs[2], tr)
    second.append(tr[2])
    return prompts, first, logits, tokens, second


@pytest.fixture(scope="module")
def stage():
    cfg = model.stage_config(SHAPE, execution="f16", kv_cache_bytes=128 << 20, max_sequences=12,
                             max_pass_rows=640, max_seq=1024)
    st = capi.Stage(cfg)
    model.synthesize(st, SHAPE, seed=4, norm_sigma=0.1)
    yield st
    st.close()


@pytest.mark.parametrize("config", [-1, 0, 1, 2, 9, 12, 14, 15, 16, 17, 18])
def test_forced_configuration_matches_the_oracle(stage, expected, config):
    prompts, first, logits, tokens, second = expected
    _say("gemm configuration", config)
    previous = capi.set_gemm_config(config)
    try:
        seqs = [stage.allocate(640) for _ in LENGTHS]
        items = [capi.item(seqs[0], 37, 0), capi.item(seqs[1], 5, 0),
                 capi.item(seqs[2], 512, 0, sample=False)]
        out = stage.execute(items, token_ids=prompts[0] + prompts[1] + prompts[2][:512],
                            want_logits=True, trace=True)
        got = out["trace"][-1]
        for (a, b), expect in zip(((0, 37), (37, 42), (42, 554)), first):
            assert within(got[a:b], expect, "f16") and cosine(got[a:b], expect) >= 0.9999, (config, a)
        for r in range(2):
            assert within(out["logits"][r], logits[r], "f16"), (config, r)
            assert cosine(out["logits"][r], logits[r]) >= 0.9999
        # decode rows fed the oracle's tokens, plus the last 90-token chunk of sequence 2
        items = [capi.item(seqs[0], 1, 37), capi.item(seqs[1], 1, 5), capi.item(seqs[2], 90, 512)]
        out2 = stage.execute(items, token_ids=[tokens[0], tokens[1]] + prompts[2][512:],
                             want_logits=True)
        for r in range(3):
            assert within(out2["logits"][r], second[r], "f16"), (config, r)
            assert cosine(out2["logits"][r], second[r]) >= 0.9999
        for s in seqs:
            stage.release(s)
    finally:
        capi.set_gemm_config(previous)


def test_read_probe_measures_a_plausible_ceiling():
    """The read ceiling the benchmark compares decode rates with: between 1 and 8.5 TB/s."""
    gb_s = capi.measure_read_bandwidth(256 << 20)
    assert 1000.0 < gb_s < 8500.0, gb_s
