"""Device sampling against the oracle's sampler (which tests/test_oracle.py pins bit for bit
to the reference's cpp/src/sampling.cpp), through the C ABI: hllm_rocm_sample_logits on
chosen logits, and sampled stage passes.

Tokens must be identical. The device sums probabilities exactly (integers in units of
2^-80) where the reference sums them in sorted order in double, so a draw falling within
~1e-13 (relative) of a candidate boundary could go either way; no case here comes near.
Log-probabilities: |d| <= 1e-12, since the log-sum-exp is summed in another order.
"""
import json
import os

import numpy as np
import pytest

import oracle
from hllm_amd import capi
from tests.test_gpu_stage import tiny_stage

pytestmark = pytest.mark.gpu
GOLDEN = os.path.join(os.path.dirname(__file__), "golden", "sampling_vectors.json")
NONE = np.iinfo(np.uint64).max


def _say(*what):
    print("[gpu-case]", *what, flush=True)


def option(t=0.0, p=1.0, k=0, seed=0, index=0, logprobs=False, top=0):
    return capi.item(0, 1, 0, temperature=t, top_p=p, top_k=k, seed=seed, generated_index=index,
                     logprobs=logprobs, top_logprobs=top)


def expected(logits, o):
    s = oracle.Sampling(o.temperature, o.top_p, o.top_k, o.seed,
                        bool(o.flags & capi.ITEM_LOGPROBS), o.top_logprobs)
    return oracle.sample_token(np.asarray(logits, np.float32), s, o.generated_index)


def check(logits, options, tokens, logprobs, top_ids, top_values, where=""):
    logits = np.asarray(logits, np.float32)
    for r, o in enumerate(options):
        tok, lp, top = expected(logits[r], o)
        assert int(tokens[r]) == tok, f"{where} row {r}: token {int(tokens[r])} != {tok}"
        if not o.flags & capi.ITEM_LOGPROBS:
            continue
        assert abs(logprobs[r] - lp) <= 1e-12, (where, r, logprobs[r], lp)
        n = min(o.top_logprobs, logits.shape[1])
        assert [int(i) for i in top_ids[r][:n]] == [i for i, _ in top[:n]], (where, r)
        np.testing.assert_allclose(top_values[r][:n], [v for _, v in top[:n]], rtol=0, atol=1e-12)
        assert all(int(i) == NONE for i in top_ids[r][n:])


def run(logits, options, where=""):
    out = capi.sample_logits(logits, options)
    check(logits, options, *out, where=where)
    return out


def test_golden_vectors():
    _say("sampling golden vectors")
    doc = json.load(open(GOLDEN))
    sets = [np.asarray(s, np.float32) for s in doc["logits"]]
    for li, lg in enumerate(sets):
        cases = [c for c in doc["cases"] if c["logits_index"] == li]
        opts = [option(c["temperature"], c["top_p"], c["top_k"], c["seed"], c["generated_index"],
                       c["return_logprobs"], c["top_logprobs"]) for c in cases]
        tokens, lps, ids, vals = capi.sample_logits(np.tile(lg, (len(cases), 1)), opts)
        for r, c in enumerate(cases):
            assert int(tokens[r]) == c["token"], (li, r, c)
            if c["return_logprobs"]:
                assert abs(lps[r] - c["logprob"]) <= 1e-12
                n = c["top_logprobs"]
                assert [int(i) for i in ids[r][:n]] == c["top_ids"]
                np.testing.assert_allclose(vals[r][:n], c["top_values"], rtol=0, atol=1e-12)


def _logit_sets(rng, vocab):
    normal = (rng.standard_normal(vocab) * 3.0).astype(np.float32)
    return {
        "normal": normal,
        "quantized ties": (np.round(normal * 2.0) / 2.0).astype(np.float32),
        "flat": np.zeros(vocab, np.float32),
        "signed zeros": np.where(rng.random(vocab) < 0.5, np.float32(0.0), np.float32(-0.0)),
        "wide (underflowing probabilities)": (rng.standard_normal(vocab) * 400.0).astype(np.float32),
        "peaked": np.where(np.arange(vocab) == vocab // 3, np.float32(30.0), normal * 0.1).astype(
            np.float32),
    }


@pytest.mark.parametrize("vocab", [1, 2, 7, 1000, 32000])
def test_random_options_match_the_oracle(vocab):
    rng = np.random.default_rng(vocab)
    for name, lg in _logit_sets(rng, vocab).items():
        opts = []
        for t in (0.0, 0.25, 0.8, 1.0, 2.5, 100.0):
            for p in (1.0, 0.95, 0.5, 1e-9):
                k = int(rng.choice([0, 1, 3, 40, max(1, vocab - 1), vocab, vocab + 5]))
                lp = bool(rng.random() < 0.5)
                opts.append(option(t, p, k, int(rng.integers(0, 2**63)), int(rng.integers(0, 1000)),
                                   lp, int(rng.integers(0, 6)) if lp else 0))
        _say("random options", vocab, name, len(opts))
        run(np.tile(lg, (len(opts), 1)), opts, where=f"{vocab} {name}")


def test_qwen_vocabulary_rows():
    """151936-entry rows (Qwen3's vocabulary), one option set per row, many draws."""
    rng = np.random.default_rng(3)
    vocab, rows = 151936, 48
    lg = (rng.standard_normal((rows, vocab)) * 2.5).astype(np.float32)
    lg[:, 17] += 6.0
    opts = [option(float(rng.choice([0.6, 0.8, 1.0, 1.3])), float(rng.choice([1.0, 0.95, 0.8])),
                   int(rng.choice([0, 20, 1000])), int(rng.integers(0, 2**63)), r, r % 2 == 0,
                   (r // 2) % 6 if r % 2 == 0 else 0) for r in range(rows)]
    _say("qwen vocabulary rows", rows)
    run(lg, opts, where="qwen")


def test_deterministic_and_validated():
    rng = np.random.default_rng(5)
    lg = (rng.standard_normal((8, 5000)) * 2.0).astype(np.float32)
    opts = [option(0.9, 0.9, 0, 1234, i, True, 5) for i in range(8)]
    _say("determinism")
    a = capi.sample_logits(lg, opts)
    b = capi.sample_logits(lg, opts)
    for x, y in zip(a, b):
        np.testing.assert_array_equal(x, y)
    for bad in (option(-1.0), option(101.0), option(1.0, 0.0), option(1.0, 1.5),
                option(1.0, 1.0, 0, 0, 0, False, 2), option(1.0, 1.0, 0, 0, 0, True, 6)):
        with pytest.raises(capi.StageError) as e:
            capi.sample_logits(lg[:1], [bad])
        assert e.value.status == capi.INVALID_REQUEST
    nan = lg[:1].copy()
    nan[0, 7] = np.nan
    with pytest.raises(capi.StageError) as e:
        capi.sample_logits(nan, [option(1.0)])
    assert e.value.status == capi.INTERNAL


def test_stage_passes_sample_on_the_device():
    """A decode pass whose items carry different sampling options: every item's token and
    log-probabilities equal the oracle's on the logits the pass produced."""
    _say("stage sampling")
    st = tiny_stage("f32")
    seqs = [st.allocate(16) for _ in range(6)]
    for i, s in enumerate(seqs):
        st.execute([capi.item(s, 3, 0, sample=False)], token_ids=[1 + i, 2, 3])
    opts = [dict(temperature=0.0), dict(temperature=0.0, logprobs=True, top_logprobs=5),
            dict(temperature=0.7, top_p=0.9, seed=9, generated_index=3),
            dict(temperature=1.3, top_k=4, seed=10, generated_index=0, logprobs=True, top_logprobs=2),
            dict(temperature=2.0, top_p=0.5, top_k=0, seed=2**63 + 5, generated_index=77),
            dict(temperature=100.0, seed=1, generated_index=1, logprobs=True)]
    for step in range(3):
        items = [capi.item(s, 1, 3 + step, **o) for s, o in zip(seqs, opts)]
        out = st.execute(items, token_ids=[4 + step] * len(seqs), want_logits=True)
        check(out["logits"], items, out["tokens"], out.get("logprobs"), out.get("top_ids"),
              out.get("top_logprobs"), where=f"step {step}")
        for o in opts:
            o["generated_index"] = o.get("generated_index", 0) + 1
    st.close()
