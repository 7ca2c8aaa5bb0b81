"""One pipeline stage's share at its real shape: a Qwen3-4B stage that owns layers 18-19, the
final norm and the (tied) LM head, and is fed F16 boundary activations ~N(0, 1) through the
stage contract (first_stage = 0; hLLM cpp/src/cpu/stage.cpp:143-159,
cpp/src/cuda/stage.cpp:363-391). 128 sequences hold paged KV of lengths log-uniform in
[1, 8192], prefilled from boundary rows; one pass of 128 decode rows is compared with the
F32 CPU oracle fed the same boundary bits from the same cache state: last-layer hidden state
and logits per row within max-abs 2e-2 and cosine 0.9999, greedy tokens equal except at
near ties."""
import numpy as np
import pytest

import oracle
from hllm_amd import capi, model, synthetic
from tests import helpers_parity as hp
from tests import models

pytestmark = pytest.mark.gpu
SHAPE = synthetic.QWEN3_4B
START, END = 18, 20
ROWS, MAX_ROWS, LONGEST = 128, 2048, 8192


def test_boundary_stage_128_decode_rows_to_8192_context():
    hp.say("qwen3-4b stage 18-19 + head: oracle weights")
    ost = oracle.OracleStage(models.synthetic_stage(SHAPE, START, END, first=False, final=True,
                                                    seed=9, norm_sigma=0.1))
    cfg = model.stage_config(SHAPE, START, END, first=False, final=True, execution="f16",
                             kv_cache_bytes=2 << 30, max_sequences=ROWS + 4, max_pass_rows=MAX_ROWS,
                             max_seq=LONGEST + 8)
    st = capi.Stage(cfg)
    model.synthesize(st, SHAPE, seed=9, norm_sigma=0.1)
    rng = np.random.default_rng(31)
    lengths = [int(min(LONGEST, max(1, np.floor(np.exp(rng.uniform(0.0, np.log(LONGEST + 1)))))))
               for _ in range(ROWS)]
    lengths[0] = LONGEST  # the longest context is always present
    boundary = [models.f16_normal(rng, (n, SHAPE.hidden)) for n in lengths]
    hp.say("stage share: GPU prefill of", sum(lengths), "boundary rows, longest", max(lengths))
    seqs = [st.allocate(n + 4) for n in lengths]
    hp.prefill(st, seqs, lengths, MAX_ROWS, boundary=boundary)
    del boundary
    hp.say("stage share: cache state into the oracle")
    oseqs = hp.oracle_sequences(ost, st, seqs, LONGEST + 8)
    rows_in = models.f16_normal(rng, (ROWS, SHAPE.hidden))
    hp.say("stage share: 128-row decode pass")
    out = st.execute([capi.item(s, 1, n) for s, n in zip(seqs, lengths)], boundary=rows_in,
                     want_logits=True, trace=True)
    hp.say("stage share: oracle decode rows")
    hidden, logits = hp.oracle_decode(ost, oseqs, list(rows_in), lengths)
    hp.check_rows(out["trace"][-1], hidden, "stage share hidden")
    hp.check_rows(out["logits"], logits, "stage share logits")
    hp.greedy_agrees(out["tokens"], logits, out["logits"], "stage share")
    for s, n in zip(seqs, lengths):
        assert st.length(s) == n + 1
    st.close()
