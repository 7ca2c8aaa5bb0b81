"""hllm_rocm_sample_logits_noalloc (the sampler entry point that allocates nothing) against
hllm_rocm_sample_logits on the same host logits: identical tokens, log-probabilities and top
tokens, on two calls in a row (the second with a smaller input), plus its limits and its
recovery after a failed call."""
import numpy as np
import pytest

import oracle
from hllm_amd import capi

pytestmark = pytest.mark.gpu


def _say(*what):
    print("[gpu-case]", *what, flush=True)


def _options(rows, rng):
    """Greedy, temperature/top-p/top-k and log-probability rows, mixed."""
    out = []
    for r in range(rows):
        kind = r % 4
        if kind == 0:
            out.append(capi.item(0, 1, 0))
        elif kind == 1:
            out.append(capi.item(0, 1, 0, temperature=0.8, top_p=0.9, seed=r, generated_index=3 * r))
        elif kind == 2:
            out.append(capi.item(0, 1, 0, temperature=1.3, top_p=0.5, top_k=40, seed=100 + r,
                                 logprobs=True, top_logprobs=5))
        else:
            out.append(capi.item(0, 1, 0, logprobs=True, top_logprobs=2))
    return out


def _same(a, b):
    for x, y in zip(a, b):
        assert np.array_equal(np.asarray(x), np.asarray(y), equal_nan=True)


@pytest.mark.parametrize("rows,vocab", [(9, 151936), (3, 1000)])
def test_noalloc_sampler_equals_the_allocating_one(rows, vocab):
    """Run in this order: a large call, then a smaller one that reuses the same device area."""
    _say("noalloc sampler", rows, vocab)
    rng = np.random.default_rng(rows * 7 + vocab)
    logits = (rng.standard_normal((rows, vocab)) * 2.0).astype(np.float32)
    opts = _options(rows, rng)
    expect = capi.sample_logits(logits, opts)
    got = capi.sample_logits_noalloc(logits, opts)
    _same(got, expect)
    for r, it in enumerate(opts):
        s = oracle.Sampling(it.temperature, it.top_p, it.top_k, it.seed,
                            bool(it.flags & capi.ITEM_LOGPROBS), it.top_logprobs)
        assert int(got[0][r]) == oracle.sample_token(logits[r], s, it.generated_index)[0]


def test_noalloc_sampler_limits_and_recovery():
    _say("noalloc sampler limits")
    rng = np.random.default_rng(2)
    too_wide = np.zeros((1, capi.NOALLOC_MAX_VOCABULARY + 1), np.float32)
    with pytest.raises(capi.StageError) as e:
        capi.sample_logits_noalloc(too_wide, [capi.item(0, 1, 0)])
    assert e.value.status == capi.RESOURCE_EXHAUSTED
    bad = rng.standard_normal((2, 500)).astype(np.float32)
    bad[1, 7] = np.nan
    with pytest.raises(capi.StageError) as e:
        capi.sample_logits_noalloc(bad, [capi.item(0, 1, 0), capi.item(0, 1, 0)])
    assert e.value.status == capi.INTERNAL
    with pytest.raises(capi.StageError) as e:
        capi.sample_logits_noalloc(bad[:1], [capi.item(0, 1, 0, top_p=0.0)])
    assert e.value.status == capi.INVALID_REQUEST
    good = rng.standard_normal((5, capi.NOALLOC_MAX_VOCABULARY)).astype(np.float32)
    opts = _options(5, rng)
    _same(capi.sample_logits_noalloc(good, opts), capi.sample_logits(good, opts))
