"""The stage contract on the GPU, through the C ABI: admission figures against their closed
form, KV pool exhaustion, sequence release while a pass is in flight, device-fed input
validation, cancellation, and the profiled pass (hLLM cpp/include/hllm/runtime/
stage_backend.hpp:69-107)."""
import math

import numpy as np
import pytest

from hllm_amd import capi, model, synthetic
from tests import models

pytestmark = pytest.mark.gpu
SHAPE = synthetic.ModelShape("contract", 3, 128, 256, 4, 2, 64, 512, qk_norm=True)


def _say(*what):
    print("[gpu-case]", *what, flush=True)


def _stage(execution="f16", kv_bytes=8 << 20, block=32, first=True, final=True, layer_start=0,
           layer_end=None, max_sequences=8):
    cfg = model.stage_config(SHAPE, layer_start, layer_end, first, final, execution=execution,
                             kv_cache_bytes=kv_bytes, kv_block_tokens=block,
                             max_sequences=max_sequences, max_pass_rows=256, max_seq=1024)
    st = capi.Stage(cfg)
    model.synthesize(st, SHAPE, seed=1, norm_sigma=0.1)
    return st


def _kv_block_bytes(layers, block, element):
    return block * layers * 2 * SHAPE.kv_heads * SHAPE.head_dim * element


@pytest.mark.parametrize("execution,element", [("f16", 2), ("f32", 4)])
def test_sequence_memory_closed_form(execution, element):
    """cache = {tokens * 24 + rows * H * 6, ceil(tokens / bt) * bt * L * 2 * K * D * el};
    workspace = {rows * H * 6 + 65536, 0}; rows = query_rows(tokens, max_query)
    (stage_backend.hpp:36-40,62-67)."""
    _say("sequence_memory", execution)
    st = _stage(execution)
    for tokens, max_query in ((1, 0), (31, 0), (32, 8), (33, 64), (700, 512), (1024, 1024),
                              (100, 101)):
        cache, ws = st.sequence_memory(tokens, max_query)
        rows = tokens if max_query == 0 or max_query > tokens else max_query
        blocks = math.ceil(tokens / 32)
        assert cache.device_bytes == blocks * _kv_block_bytes(SHAPE.layers, 1, element) * 32
        assert cache.host_bytes == tokens * 24 + rows * SHAPE.hidden * 6
        assert ws.host_bytes == rows * SHAPE.hidden * 6 + 65536 and ws.device_bytes == 0
        assert cache.pinned_host_bytes == 0 and ws.pinned_host_bytes == 0
    for bad in (0, 1025):
        with pytest.raises(capi.StageError) as e:
            st.sequence_memory(bad, 0)
        assert e.value.status == capi.INVALID_REQUEST
    st.close()


def test_kv_pool_exhaustion_and_reuse():
    """A pool of exactly 10 blocks: allocations fail with RESOURCE_EXHAUSTED once the blocks
    run out, and released blocks are handed out again."""
    _say("kv pool exhaustion")
    st = _stage(kv_bytes=10 * _kv_block_bytes(SHAPE.layers, 32, 2))
    a = st.allocate(32 * 6)
    b = st.allocate(32 * 4)
    with pytest.raises(capi.StageError) as e:
        st.allocate(1)
    assert e.value.status == capi.RESOURCE_EXHAUSTED and "KV cache is full" in str(e.value)
    blocks_a = set(st.blocks(a)[0].tolist())
    st.release(a)
    c = st.allocate(32 * 5)
    assert set(st.blocks(c)[0].tolist()) <= blocks_a
    with pytest.raises(capi.StageError) as e:
        st.allocate(33)  # two blocks, one left
    assert e.value.status == capi.RESOURCE_EXHAUSTED
    d = st.allocate(32)
    st.execute([capi.item(d, 5, 0)], token_ids=[1, 2, 3, 4, 5])
    assert st.length(d) == 5
    for s in (b, c, d):
        st.release(s)
    st.close()


def test_sequence_slots_run_out():
    _say("sequence slots")
    st = _stage(max_sequences=3)
    seqs = [st.allocate(8) for _ in range(3)]
    with pytest.raises(capi.StageError) as e:
        st.allocate(8)
    assert e.value.status == capi.RESOURCE_EXHAUSTED
    st.release(seqs[1])
    assert st.allocate(8) == seqs[1]
    st.close()


def test_release_while_a_pass_is_in_flight():
    """Releasing a sequence whose pass is in flight invalidates the handle at once, but its
    slot and blocks stay out of the pools until the pass completes: a sequence allocated in
    between gets fresh blocks and starts at length 0, and the pass's results still arrive."""
    _say("release in flight")
    st = _stage()
    a = st.allocate(128)
    blocks_a = set(st.blocks(a)[0].tolist())
    h = st.submit([capi.item(a, 40, 0)], token_ids=list(range(1, 41)))
    st.release(a)
    with pytest.raises(capi.StageError):
        st.length(a)
    b = st.allocate(128)
    assert b != a
    assert not (set(st.blocks(b)[0].tolist()) & blocks_a)
    out = st.wait(h)
    assert int(out["tokens"][0]) < SHAPE.vocab
    assert st.length(b) == 0
    out_b = st.execute([capi.item(b, 3, 0)], token_ids=[5, 6, 7])
    assert st.length(b) == 3 and int(out_b["tokens"][0]) < SHAPE.vocab
    c = st.allocate(128)  # the completed pass returned a's slot
    assert c == a
    assert st.length(c) == 0
    st.close()


def test_release_in_flight_keeps_other_results_equal():
    """The same two-sequence pass with and without a concurrent release of one member gives
    the other member the same token."""
    _say("release in flight, results")
    tokens = []
    for release in (False, True):
        st = _stage()
        a, b = st.allocate(64), st.allocate(64)
        h = st.submit([capi.item(a, 9, 0), capi.item(b, 7, 0)], token_ids=list(range(3, 19)))
        if release:
            st.release(a)
        tokens.append(int(st.wait(h)["tokens"][1]))
        st.close()
    assert tokens[0] == tokens[1]


def test_device_fed_input_validation():
    """HLLM_ITEM_TOKEN_FROM_DEVICE needs a stage that embeds and samples, and a sequence whose
    previous pass sampled."""
    _say("device-fed validation")
    st = _stage()
    s = st.allocate(64)
    with pytest.raises(capi.StageError) as e:  # a new sequence has no sampled token
        st.execute([capi.item(s, 1, 0, from_device=True)], token_ids=[0])
    assert e.value.status == capi.INVALID_REQUEST
    st.execute([capi.item(s, 4, 0, sample=False)], token_ids=[1, 2, 3, 4])
    with pytest.raises(capi.StageError) as e:  # the previous pass did not sample
        st.execute([capi.item(s, 1, 4, from_device=True)], token_ids=[0])
    assert e.value.status == capi.INVALID_REQUEST
    out = st.execute([capi.item(s, 1, 4)], token_ids=[5])
    fed = st.execute([capi.item(s, 1, 5, from_device=True)], token_ids=[0])
    # the same step fed from the host gives the same token
    t = st.allocate(64)
    st.execute([capi.item(t, 4, 0, sample=False)], token_ids=[1, 2, 3, 4])
    st.execute([capi.item(t, 1, 4)], token_ids=[5])
    host = st.execute([capi.item(t, 1, 5)], token_ids=[int(out["tokens"][0])])
    assert int(fed["tokens"][0]) == int(host["tokens"][0])
    with pytest.raises(capi.StageError) as e:  # two tokens cannot come from the device
        st.execute([capi.item(s, 2, 6, from_device=True)], token_ids=[0, 0])
    assert e.value.status == capi.INVALID_REQUEST
    st.close()
    first = _stage(final=False, layer_end=2)
    s = first.allocate(16)
    first.execute([capi.item(s, 2, 0)], token_ids=[1, 2])
    with pytest.raises(capi.StageError) as e:  # no sampled token on a non-final stage
        first.execute([capi.item(s, 1, 2, from_device=True)], token_ids=[0])
    assert e.value.status == capi.INVALID_REQUEST
    first.close()


def test_cancellation_before_and_during_a_pass():
    """Cancelled before the pass: CANCELLED, nothing changes and the sequence goes on.
    Cancelled while the pass runs (set between submit and wait): the results are discarded,
    CANCELLED, and the sequence is failed for good (cpp/src/cuda/stage.cpp:456,463-468)."""
    _say("cancellation")
    st = _stage()
    s = st.allocate(64)
    flag = np.ones(1, np.int32)
    with pytest.raises(capi.StageError) as e:
        st.execute([capi.item(s, 3, 0)], token_ids=[1, 2, 3], cancelled=flag)
    assert e.value.status == capi.CANCELLED
    assert st.length(s) == 0
    flag[0] = 0
    st.execute([capi.item(s, 3, 0)], token_ids=[1, 2, 3], cancelled=flag)
    assert st.length(s) == 3
    h = st.submit([capi.item(s, 2, 3)], token_ids=[4, 5], cancelled=flag)
    flag[0] = 1
    with pytest.raises(capi.StageError) as e:
        st.wait(h)
    assert e.value.status == capi.CANCELLED
    assert st.length(s) == 3
    flag[0] = 0
    with pytest.raises(capi.StageError) as e:
        st.execute([capi.item(s, 2, 3)], token_ids=[4, 5])
    assert e.value.status == capi.INVALID_REQUEST
    other = st.allocate(16)  # the stage itself keeps working
    st.execute([capi.item(other, 2, 0)], token_ids=[4, 5])
    st.close()


def test_cancel_poll_at_every_checkpoint():
    """The cancel_poll callback is read where the flag is: once before the pass is enqueued,
    before each of the stage's layers is enqueued, and once when the pass completes (1 + L + 1
    polls). Cancelled at the first poll nothing ran and the sequence goes on; cancelled at
    any later one the pass is discarded and its sequences are failed for good
    (cpp/src/cpu/stage.cpp:109-111; cpp/src/cuda/stage.cpp:357,396,456,463-468)."""
    _say("cancel poll checkpoints")
    st = _stage()
    layers = SHAPE.layers
    calls = []
    st.execute([capi.item(st.allocate(8), 3, 0)], token_ids=[1, 2, 3],
               cancelled=lambda: calls.append(1) and False)
    assert len(calls) == 1 + layers + 1
    for at in range(1, layers + 3):
        s = st.allocate(16)
        seen = []

        def poll():
            seen.append(1)
            return len(seen) == at

        with pytest.raises(capi.StageError) as e:
            st.execute([capi.item(s, 3, 0)], token_ids=[1, 2, 3], cancelled=poll)
        assert e.value.status == capi.CANCELLED and len(seen) == at
        assert st.length(s) == 0
        if at == 1:
            st.execute([capi.item(s, 3, 0)], token_ids=[1, 2, 3])  # never started: goes on
            assert st.length(s) == 3
        else:
            with pytest.raises(capi.StageError) as e:
                st.execute([capi.item(s, 3, 0)], token_ids=[1, 2, 3])
            assert e.value.status == capi.INVALID_REQUEST
        st.release(s)
    st.close()


def test_allocator_metrics_and_device_info():
    """The factory diagnostics behind BackendFactory::allocator_metrics / profiling_reset_peak
    / profiling_device_info (cpp/include/hllm/runtime/backend_factory.hpp:31-39): the bytes
    held follow stage creation and destruction, no caching (cached 0), the peak resets to the
    bytes held, and the device reports its identity and memory."""
    _say("allocator metrics")
    before = capi.allocator_metrics(0)
    assert before["cached_bytes"] == 0 and before["peak_bytes"] >= before["active_bytes"]
    st = _stage(kv_bytes=32 << 20)
    held = capi.allocator_metrics(0)
    assert held["active_bytes"] - before["active_bytes"] >= 16 << 20
    st.close()
    after = capi.allocator_metrics(0)
    assert after["active_bytes"] == before["active_bytes"] and after["peak_bytes"] >= held["active_bytes"]
    capi.reset_peak(0)
    assert capi.allocator_metrics(0)["peak_bytes"] == after["active_bytes"]
    info = capi.device_info(0)
    _say("device", info)
    assert len(info["identity"]) in (16, 32) and info["name"] and info["architecture"].startswith("gfx950")
    assert 0 < info["available_bytes"] <= info["total_bytes"] and info["compute_units"] > 0
    with pytest.raises(capi.StageError) as e:
        capi.device_info(1 << 20)
    assert e.value.status == capi.INVALID_REQUEST


@pytest.mark.parametrize("first,final", [(True, True), (True, False), (False, True)])
def test_profiled_pass_equals_execute(first, final):
    """execute_profiled returns execute's outputs bit for bit, with one timed phase per
    component in pass order (cpp/src/profiling/compute_probe.hpp:28-113)."""
    _say("profiled pass", first, final)
    layer_start, layer_end = (0, 2) if first else (1, 3)
    st = _stage(first=first, final=final, layer_start=layer_start, layer_end=layer_end)
    rng = np.random.default_rng(8)
    a, b = st.allocate(64), st.allocate(64)
    if first:
        kw = {"token_ids": rng.integers(0, SHAPE.vocab, 11).tolist()}
    else:
        kw = {"boundary": models.f16_normal(rng, (11, SHAPE.hidden))}
    plain = st.execute([capi.item(a, 11, 0)], **kw)
    prof = st.execute_profiled([capi.item(b, 11, 0)], **kw)
    for key in ("tokens", "boundary"):
        if key in plain:
            assert np.array_equal(plain[key], prof[key]), key
    names = [(c, layer) for c, layer, _ in prof["phases"]]
    expect = [("embedding" if first else "from-wire", None)]
    expect += [("layer", i) for i in range(layer_start, layer_end)]
    expect += [("final_norm", None), ("lm_head", None), ("sampling", None)] if final else \
        [("to-wire", None)]
    assert names == expect
    assert all(ms >= 0.0 for _, _, ms in prof["phases"])
    assert st.length(a) == st.length(b) == 11
    st.close()
