"""GPU parity of the stage worker against the oracle and the reference's golden vectors,
through the C ABI.

Tolerances: F32 execution 3e-5 and F16 execution 5e-3 on the tiny Transformers fixture
(the reference's own CUDA-backend bars, hLLM tests/cpp/cuda_stage_test.cpp:102); synthetic
Qwen3-shaped slices in F16 execution: max-abs <= 2e-2 and cosine >= 0.9999 against the F32
CPU oracle; F32 execution (split-precision GEMMs, F32 KV): |d| <= 2e-4 + 1e-4 |expected|.
"""
from dataclasses import replace

import numpy as np
import pytest

import oracle
from hllm_amd import capi, model, synthetic
from tests import models

pytestmark = pytest.mark.gpu
KV_BYTES = 256 << 20


def _say(*what):
    print("[gpu-case]", *what, flush=True)


def within(got, expect, execution):
    """F16 execution: max-abs <= 2e-2. F32 execution:
    |d| <= 2e-4 + 1e-4 |expect|: products are emulated with 22-bit activation splits and
    summed in a different order than the CPU worker, which over 512-token prefills of a
    two-layer slice moves single elements by up to ~1.2e-4."""
    got, expect = np.asarray(got), np.asarray(expect)
    if execution == "f16":
        return np.abs(got - expect).max() <= 2e-2
    return bool(np.all(np.abs(got - expect) <= 2e-4 + 1e-4 * np.abs(expect)))


def cosine(a, b):
    a, b = np.asarray(a, np.float64).ravel(), np.asarray(b, np.float64).ravel()
    return float(a @ b / (np.linalg.norm(a) * np.linalg.norm(b)))


def tiny_stage(execution, layer_start=0, layer_end=2, first=True, final=True):
    shape = models.tiny_reference_shape()
    cfg = model.stage_config(shape, layer_start, layer_end, first, final, execution=execution,
                             weights="f32" if execution == "f32" else "f16",
                             kv_cache_bytes=4 << 20, max_sequences=8, max_pass_rows=64)
    st = capi.Stage(cfg)
    w = models.tiny_reference_stage(layer_start, layer_end, first, final)
    model.load(st, w.tensors)
    return st


@pytest.mark.parametrize("execution,tol", [("f32", 3e-5), ("f16", 5e-3)])
def test_tiny_reference_prefill_layers_kv_logits(execution, tol):
    _say("tiny-reference prefill", execution)
    fx = models.tiny_reference()
    st = tiny_stage(execution)
    seq = st.allocate(32)
    out = st.execute([capi.item(seq, 5, 0)], token_ids=[1, 4, 2, 8, 3], want_logits=True,
                     trace=True)
    for layer in range(2):
        np.testing.assert_allclose(out["trace"][layer],
                                   models.tiny_rows(fx["layer_outputs"][layer], 0, 5), atol=tol,
                                   rtol=0)
        k, v = st.read_kv(seq, layer)
        ek = np.asarray(fx["keys"][layer]["values"], np.float32).reshape(2, 5, 4).transpose(1, 0, 2)
        ev = np.asarray(fx["values"][layer]["values"], np.float32).reshape(2, 5, 4).transpose(
            1, 0, 2)
        np.testing.assert_allclose(k, ek, atol=tol, rtol=0)
        np.testing.assert_allclose(v, ev, atol=tol, rtol=0)
    np.testing.assert_allclose(out["logits"][0], models.tiny_rows(fx["logits"], 4, 1)[0],
                               atol=tol, rtol=0)
    assert out["tokens"][0] == int(np.argmax(models.tiny_rows(fx["logits"], 4, 1)))
    assert st.length(seq) == 5
    st.close()


def test_tiny_reference_prefill_then_two_decodes():
    _say("tiny-reference prefill + decodes")
    fx = models.tiny_reference()
    st = tiny_stage("f32")
    seq = st.allocate(32)
    ids = [1, 4, 2, 8, 3]
    for position, count in ((0, 3), (3, 1), (4, 1)):
        out = st.execute([capi.item(seq, count, position)], token_ids=ids[position:position + count],
                         want_logits=True, trace=True)
        for layer in range(2):
            np.testing.assert_allclose(out["trace"][layer],
                                       models.tiny_rows(fx["layer_outputs"][layer], position, count),
                                       atol=3e-5, rtol=0)
        np.testing.assert_allclose(out["logits"][0],
                                   models.tiny_rows(fx["logits"], position + count - 1, 1)[0],
                                   atol=3e-5, rtol=0)
    st.close()


def test_tiny_reference_split_stages_over_f16_boundary():
    _say("tiny-reference split stages")
    fx = models.tiny_reference()
    first = tiny_stage("f32", 0, 1, True, False)
    last = tiny_stage("f32", 1, 2, False, True)
    s0, s1 = first.allocate(32), last.allocate(32)
    out0 = first.execute([capi.item(s0, 5, 0)], token_ids=[1, 4, 2, 8, 3])
    expect_wire = oracle.f16_encode(models.tiny_rows(fx["layer_outputs"][0], 0, 5))
    assert np.abs(oracle.f16_decode(out0["boundary"]) - oracle.f16_decode(expect_wire)).max() < 1e-3
    out1 = last.execute([capi.item(s1, 5, 0)], boundary=out0["boundary"], trace=True)
    np.testing.assert_allclose(out1["trace"][0], models.tiny_rows(fx["layer_outputs"][1], 0, 5),
                               atol=1e-3, rtol=0)
    assert out1["tokens"][0] == int(np.argmax(models.tiny_rows(fx["logits"], 4, 1)))
    first.close()
    last.close()


def test_boundary_encode_is_the_reference_codec():
    """Non-final stage output bits equal the oracle's F16 RNE of the stage's F32 hidden."""
    _say("boundary codec")
    first = tiny_stage("f32", 0, 1, True, False)
    s0 = first.allocate(32)
    out = first.execute([capi.item(s0, 5, 0)], token_ids=[1, 4, 2, 8, 3], trace=True)
    assert np.array_equal(out["boundary"], oracle.f16_encode(out["trace"][0]))
    first.close()


def _oracle_generate(shape, prompt, steps, seed=0, norm_sigma=0.1):
    st = oracle.OracleStage(models.synthetic_stage(shape, seed=seed, norm_sigma=norm_sigma))
    return st.generate(prompt, steps)


@pytest.mark.parametrize("execution", ["f32", "f16"])
def test_tiny_llama_greedy_matches_oracle(execution):
    _say("tiny-llama greedy", execution)
    shape = synthetic.TINY_LLAMA
    rng = np.random.default_rng(0)
    prompt = rng.integers(0, shape.vocab, 8).tolist()
    expect, expect_logits = _oracle_generate(shape, prompt, 16)
    cfg = model.stage_config(shape, execution=execution, kv_cache_bytes=8 << 20, max_sequences=4,
                             max_pass_rows=64)
    st = capi.Stage(cfg)
    model.synthesize(st, shape, seed=0, norm_sigma=0.1)
    seq = st.allocate(64)
    out = st.execute([capi.item(seq, 8, 0)], token_ids=prompt, want_logits=True)
    tokens, logits = [int(out["tokens"][0])], [out["logits"][0]]
    for step in range(16):
        out = st.execute([capi.item(seq, 1, 8 + step)], token_ids=[tokens[-1]], want_logits=True)
        tokens.append(int(out["tokens"][0]))
        logits.append(out["logits"][0])
    for a, b in zip(logits, expect_logits):
        assert within(a, b, execution)
    assert tokens == expect
    st.close()


@pytest.mark.parametrize("dtype,execution", [("f16", "f16"), ("f16", "f32"), ("f32", "f32")])
def test_synthesized_and_uploaded_tensors_equal_the_oracle_bitwise(dtype, execution):
    """Device generator == host generator, and the F-layout relayout round-trips every
    element (including gate/up interleave and fused q/k/v rows). F16-resident weights are
    bit-exact; F32-resident weights are held as hi + lo/2048 F16 parts, which keeps about
    22 significand bits: error <= 2^-20 relative, with an absolute floor of 2^-35 where the
    parts fall below F16's normal range (|w| < 6.1e-5)."""
    _say("tensor readback", dtype, execution)
    from dataclasses import replace
    shape = replace(synthetic.ModelShape("s", 1, 96, 80, 3, 1, 32, 300), dtype=dtype)
    names = synthetic.stage_tensor_names(shape, 0, 1, True, True)
    for how in ("synth", "upload"):
        st = capi.Stage(model.stage_config(shape, execution=execution, kv_cache_bytes=4 << 20,
                                           max_sequences=2, max_pass_rows=32))
        if how == "synth":
            model.synthesize(st, shape, seed=7, norm_sigma=0.1)
        else:
            model.load(st, {n: models.synthetic_tensor(shape, n, 7, 0.1)[1] for n in names})
        for n in names:
            expect = models.synthetic_tensor(shape, n, 7, 0.1)[0]
            got = st.read_tensor(n, expect.shape)
            if execution == "f32" and dtype == "f32":
                bound = np.maximum(np.abs(expect) * 2.0 ** -20, 2.0 ** -35)
                assert np.all(np.abs(got - expect) <= bound), (how, n)
            else:
                assert np.array_equal(got.view(np.uint32), expect.view(np.uint32)), (how, n)
        st.close()


def test_synthesized_weights_equal_uploaded_weights():
    _say("synthesize == upload")
    shape = synthetic.ModelShape("s", 1, 256, 512, 4, 2, 64, 1000)
    outs = []
    for how in ("synth", "upload"):
        st = capi.Stage(model.stage_config(shape, kv_cache_bytes=8 << 20, max_sequences=4,
                                           max_pass_rows=64))
        if how == "synth":
            model.synthesize(st, shape, seed=3, norm_sigma=0.1)
        else:
            tensors = {n: models.synthetic_tensor(shape, n, 3, 0.1)[1]
                       for n in synthetic.stage_tensor_names(shape, 0, 1, True, True)}
            model.load(st, tensors)
        seq = st.allocate(64)
        outs.append(st.execute([capi.item(seq, 7, 0)], token_ids=[1, 2, 3, 4, 5, 6, 7],
                               want_logits=True, trace=True))
        st.close()
    assert np.array_equal(outs[0]["trace"], outs[1]["trace"])
    assert np.array_equal(outs[0]["logits"], outs[1]["logits"])


def _slice_shape(shape, layers):
    return synthetic.with_layers(shape, layers)


@pytest.mark.parametrize("execution", ["f16", "f32"])
def test_qwen3_slice_ragged_batch_matches_oracle(execution):
    """Qwen3-0.6B-shaped 2-layer slice, full vocabulary: a ragged pass mixing a prefill
    chunk with decode rows of other sequences, against the oracle run per sequence."""
    _say("qwen3-0.6b slice ragged", execution)
    shape = _slice_shape(synthetic.QWEN3_0_6B, 2)
    cfg = model.stage_config(shape, execution=execution, kv_cache_bytes=64 << 20,
                             max_sequences=8, max_pass_rows=256, max_seq=4096)
    st = capi.Stage(cfg)
    model.synthesize(st, shape, seed=0, norm_sigma=0.1)
    ost = oracle.OracleStage(models.synthetic_stage(shape, seed=0, norm_sigma=0.1))
    rng = np.random.default_rng(1)
    lengths = [37, 5, 70]
    prompts = [rng.integers(0, shape.vocab, n).tolist() for n in lengths]
    seqs = [st.allocate(128) for _ in lengths]
    oseqs = [ost.allocate_sequence(128) for _ in lengths]
    # pass 1: prefill sequences 0 and 1 whole; sequence 2 only its first 64-token chunk
    items = [capi.item(seqs[0], 37, 0), capi.item(seqs[1], 5, 0),
             capi.item(seqs[2], 64, 0, sample=False)]
    ids = prompts[0] + prompts[1] + prompts[2][:64]
    out = st.execute(items, token_ids=ids, want_logits=True, trace=True)
    tr = []
    ref0 = ost.execute(np.array(prompts[0], np.uint64), 0, oseqs[0], tr)
    tr1 = []
    ref1 = ost.execute(np.array(prompts[1], np.uint64), 0, oseqs[1], tr1)
    oseqs[2].prefill_only = True
    tr2 = []
    ost.execute(np.array(prompts[2][:64], np.uint64), 0, oseqs[2], tr2)
    oseqs[2].prefill_only = False
    got = out["trace"][-1]
    for (a, b), expect in zip(((0, 37), (37, 42), (42, 106)), (tr[1], tr1[1], tr2[1])):
        d = got[a:b]
        assert within(d, expect, execution) and cosine(d, expect) >= 0.9999
    assert within(out["logits"][0], tr[2], execution)
    assert within(out["logits"][1], tr1[2], execution)
    assert cosine(out["logits"][0], tr[2]) >= 0.9999
    if execution == "f32":
        assert int(out["tokens"][0]) == ref0[1] and int(out["tokens"][1]) == ref1[1]
    assert int(out["tokens"][2]) == np.iinfo(np.uint64).max
    # pass 2: decode rows for sequences 0 and 1 (device-fed tokens) + the last chunk of 2
    items = [capi.item(seqs[0], 1, 37, from_device=True), capi.item(seqs[1], 1, 5, from_device=True),
             capi.item(seqs[2], 6, 64)]
    out2 = st.execute(items, token_ids=[0, 0] + prompts[2][64:], want_logits=True)
    tr, tr_b, tr_c = [], [], []
    e0 = ost.execute(np.array([int(out["tokens"][0])], np.uint64), 37, oseqs[0], tr)
    e1 = ost.execute(np.array([int(out["tokens"][1])], np.uint64), 5, oseqs[1], tr_b)
    e2 = ost.execute(np.array(prompts[2][64:], np.uint64), 64, oseqs[2], tr_c)
    for got_l, exp_l in zip(out2["logits"], (tr[2], tr_b[2], tr_c[2])):
        assert within(got_l, exp_l, execution)
    if execution == "f32":
        assert [int(t) for t in out2["tokens"]] == [e0[1], e1[1], e2[1]]
    st.close()


def test_packing_offsets_and_kv_slots_bit_exact():
    _say("packing layout")
    shape = synthetic.ModelShape("p", 1, 64, 128, 4, 2, 16, 256, qk_norm=False)
    cfg = model.stage_config(shape, kv_cache_bytes=8 << 20, max_sequences=8, max_pass_rows=512,
                             kv_block_tokens=32, max_seq=1024)
    st = capi.Stage(cfg)
    model.synthesize(st, shape, seed=0)
    seqs = [st.allocate(n) for n in (300, 20, 150, 9)]
    rng = np.random.default_rng(5)
    lengths = [0, 0, 0, 0]
    for plan in ([(0, 100), (1, 7), (2, 33), (3, 9)], [(1, 1), (0, 120), (2, 1)],
                 [(2, 1), (1, 1), (0, 1)]):
        items = [capi.item(seqs[i], n, lengths[i], sample=False) for i, n in plan]
        ids = rng.integers(0, 256, sum(n for _, n in plan)).tolist()
        st.execute(items, token_ids=ids)
        cu, pos, slots = st.last_layout(len(plan), sum(n for _, n in plan))
        width = 64
        table = np.full((8, width), -1, np.int32)
        for s in seqs:
            b, bt = st.blocks(s)
            table[s, :len(b)] = b
        ecu, _, epos, eslots = oracle.pack([seqs[i] for i, _ in plan],
                                           [lengths[i] for i, _ in plan], [n for _, n in plan],
                                           table, 32)
        assert np.array_equal(cu, ecu.astype(np.int32))
        assert np.array_equal(pos, epos.astype(np.int32))
        assert np.array_equal(slots, eslots.astype(np.int32))
        for i, n in plan:
            lengths[i] += n
    st.close()


def test_decode_batch_equals_serial_execution():
    """hLLM tests/cpp/decode_batch_contract.hpp:8-47 at T=0: ragged lengths {7,2,4,1}."""
    _say("decode batch contract")
    fx = models.tiny_reference()
    del fx
    st = tiny_stage("f32")
    lengths = [7, 2, 4, 1]
    reference, batched, expected = [], [], []
    for n in lengths:
        a, b = st.allocate(n + 1), st.allocate(n + 1)
        for s in (a, b):
            st.execute([capi.item(s, n, 0)], token_ids=[1] * n)
        expected.append(int(st.execute([capi.item(a, 1, n)], token_ids=[4])["tokens"][0]))
        reference.append(a)
        batched.append(b)
    out = st.execute([capi.item(b, 1, n) for b, n in zip(batched, lengths)], token_ids=[4] * 4)
    assert [int(t) for t in out["tokens"]] == expected
    for b, n in zip(batched, lengths):
        assert st.length(b) == n + 1
    st.close()


def test_request_validation_errors():
    _say("validation errors")
    st = tiny_stage("f32")
    seq = st.allocate(4)
    with pytest.raises(capi.StageError) as e:
        st.execute([capi.item(seq, 1, 0)], token_ids=[11])
    assert e.value.status == capi.INVALID_REQUEST
    with pytest.raises(capi.StageError) as e:
        st.execute([capi.item(seq, 1, 3)], token_ids=[1])
    assert e.value.status == capi.INVALID_REQUEST
    with pytest.raises(capi.StageError) as e:
        st.execute([capi.item(seq, 5, 0)], token_ids=[1] * 5)
    assert e.value.status == capi.INVALID_REQUEST
    with pytest.raises(capi.StageError) as e:
        st.execute([capi.item(seq, 1, 0), capi.item(seq, 1, 0)], token_ids=[1, 1])
    assert e.value.status == capi.INVALID_REQUEST
    with pytest.raises(capi.StageError) as e:
        st.allocate(33)
    assert e.value.status == capi.INVALID_REQUEST
    st.execute([capi.item(seq, 1, 0)], token_ids=[1])
    assert st.length(seq) == 1
    st.close()
    last = tiny_stage("f32", 1, 2, False, True)
    s1 = last.allocate(8)
    bad = np.zeros((1, 6), np.uint16)
    bad[0, 3] = 0x7C00
    with pytest.raises(capi.StageError) as e:
        last.execute([capi.item(s1, 1, 0)], boundary=bad)
    assert e.value.status == capi.INVALID_REQUEST
    last.close()


def test_pass_size_limits():
    """The pass's size limits on the tiny reference stage (8 sequence slots, 64 rows per pass,
    a 32-position context): an empty pass is INVALID_REQUEST and a pass of 65 rows
    RESOURCE_EXHAUSTED, with nothing changed; a pass of exactly 64 rows over all 8 slots runs
    and every item's logits equal the oracle's run of that sequence alone (F32 bounds); a
    sequence takes its 32nd and last position in a decode pass, and a 33rd is refused."""
    _say("pass size limits")
    shape = models.tiny_reference_shape()
    st = tiny_stage("f32")
    ost = oracle.OracleStage(models.tiny_reference_stage())
    rng = np.random.default_rng(5)
    with pytest.raises(capi.StageError) as e:
        st.execute([], token_ids=[])
    assert e.value.status == capi.INVALID_REQUEST
    seqs = [st.allocate(32) for _ in range(8)]
    ids = [rng.integers(0, shape.vocab, 9 if i == 0 else 8).tolist() for i in range(8)]
    with pytest.raises(capi.StageError) as e:
        st.execute([capi.item(s, len(t), 0) for s, t in zip(seqs, ids)], token_ids=sum(ids, []))
    assert e.value.status == capi.RESOURCE_EXHAUSTED
    assert all(st.length(s) == 0 for s in seqs)
    ids[0] = ids[0][:8]
    out = st.execute([capi.item(s, 8, 0) for s in seqs], token_ids=sum(ids, []), want_logits=True)
    for i, t in enumerate(ids):
        o = ost.allocate_sequence(32)
        tr = []
        ost.execute(np.array(t, np.uint64), 0, o, tr)
        assert within(out["logits"][i], tr[-1], "f32"), i
    # Fill the first sequence to 31 positions, then decode its last position.
    rest = rng.integers(0, shape.vocab, 23).tolist()
    st.execute([capi.item(seqs[0], 23, 8, sample=False)], token_ids=rest)
    out = st.execute([capi.item(seqs[0], 1, 31)], token_ids=[1])
    assert st.length(seqs[0]) == 32 and int(out["tokens"][0]) < shape.vocab
    with pytest.raises(capi.StageError) as e:
        st.execute([capi.item(seqs[0], 1, 32)], token_ids=[1])
    assert e.value.status == capi.INVALID_REQUEST
    st.close()


def test_weight_validation_errors():
    _say("weight validation")
    shape = models.tiny_reference_shape()
    w = models.tiny_reference_stage()
    cfg = model.stage_config(shape, execution="f16", weights="f16", kv_cache_bytes=4 << 20,
                             max_sequences=4, max_pass_rows=16)
    st = capi.Stage(cfg)
    with pytest.raises(capi.StageError) as e:
        st.load_tensor("model.layers.7.mlp.up_proj.weight", w.tensors["model.layers.0.mlp.up_proj.weight"])
    assert e.value.status == capi.INCOMPATIBLE_WORKER
    with pytest.raises(capi.StageError) as e:
        st.load_tensor("model.layers.0.mlp.up_proj.weight", np.zeros((3, 3), np.float32))
    assert e.value.status == capi.INCOMPATIBLE_WORKER
    big = w.tensors["model.layers.0.mlp.up_proj.weight"].copy()
    big[0, 0] = 1e6  # not representable as finite F16
    with pytest.raises(capi.StageError) as e:
        st.load_tensor("model.layers.0.mlp.up_proj.weight", big)
    assert e.value.status == capi.INCOMPATIBLE_WORKER
    nan = w.tensors["model.layers.0.mlp.up_proj.weight"].copy()
    nan[1, 1] = np.nan
    with pytest.raises(capi.StageError) as e:
        st.load_tensor("model.layers.0.mlp.up_proj.weight", nan)
    assert e.value.status == capi.INCOMPATIBLE_WORKER
    with pytest.raises(capi.StageError) as e:
        st.finalize()
    assert e.value.status == capi.INCOMPATIBLE_WORKER
    st.close()


@pytest.mark.parametrize("execution", ["f16", "f32"])
def test_long_context_split_attention_matches_oracle(execution):
    """Qwen3-0.6B-shaped 2-layer slice: a 1500-token prompt in 512-token chunks (prefill
    blocks over up to 1500 keys) then decode rows whose key range splits in two."""
    _say("long context", execution)
    shape = _slice_shape(synthetic.QWEN3_0_6B, 2)
    cfg = model.stage_config(shape, execution=execution, kv_cache_bytes=128 << 20,
                             max_sequences=4, max_pass_rows=512, max_seq=4096)
    st = capi.Stage(cfg)
    model.synthesize(st, shape, seed=2, norm_sigma=0.1)
    ost = oracle.OracleStage(models.synthetic_stage(shape, seed=2, norm_sigma=0.1))
    rng = np.random.default_rng(3)
    prompt = rng.integers(0, shape.vocab, 1500).tolist()
    seq, oseq = st.allocate(1600), ost.allocate_sequence(1600)
    pos = 0
    while pos < len(prompt):
        take = min(512, len(prompt) - pos)
        last = pos + take == len(prompt)
        out = st.execute([capi.item(seq, take, pos, sample=last)], token_ids=prompt[pos:pos + take],
                         want_logits=last, trace=True)
        oseq.prefill_only = not last
        tr = []
        ref = ost.execute(np.array(prompt[pos:pos + take], np.uint64), pos, oseq, tr)
        got = out["trace"][-1]
        assert within(got, tr[1], execution) and cosine(got, tr[1]) >= 0.9999, pos
        pos += take
    oseq.prefill_only = False
    assert within(out["logits"][0], tr[2], execution)
    token = int(out["tokens"][0])
    for step in range(3):
        out = st.execute([capi.item(seq, 1, pos, from_device=True)], token_ids=[0], want_logits=True)
        tr = []
        ref = ost.execute(np.array([token], np.uint64), pos, oseq, tr)
        assert within(out["logits"][0], tr[2], execution)
        if execution == "f32":
            assert int(out["tokens"][0]) == ref[1]
        token = int(out["tokens"][0]) if execution == "f16" else ref[1]
        pos += 1
    st.close()


SPLIT_MERGE_SHAPES = {
    "d128-qwen3": (synthetic.with_layers(synthetic.QWEN3_0_6B, 2), 2),
    "d64-llama": (synthetic.ModelShape("d64-llama", 2, 2048, 8192, 32, 8, 64, 4096, qk_norm=False,
                                       tied=False), 1),
    "d256-falcon3": (replace(synthetic.FALCON3_3B, layers=1, vocab=8192), 1),
}


@pytest.mark.parametrize("name", list(SPLIT_MERGE_SHAPES))
def test_in_kernel_split_merge_is_bit_identical_to_the_combine_kernel(monkeypatch, name):
    """Decode rows whose key ranges split (up to 3001 keys: seven splits of 512 at most, and
    several blocks of one pass arriving in any order) merge their splits in the attention
    kernel: the split's workgroup that arrives last merges them with the combine kernel's
    arithmetic. With the combine kernel instead (HLLM_ROCM_ATTN_FOLD=0) every pass must give
    bit-identical logits, tokens and caches, over eight decode passes and every layer (the
    arrival counts reset themselves between launches), eager and replayed from HIP graphs,
    then a mixed pass of short chunks at long positions, at head dims 128, 64 and 256."""
    shape, copies = SPLIT_MERGE_SHAPES[name]
    lengths = [1, 31, 480, 511, 512, 513, 1024, 1500, 2047, 2048, 3000, 700] * copies
    rng = np.random.default_rng(9)
    prompts = [rng.integers(0, shape.vocab, n).tolist() for n in lengths]
    results = {}
    for fold in ("1", "0"):
        _say("split merge, fold", fold)
        monkeypatch.setenv("HLLM_ROCM_ATTN_FOLD", fold)
        cfg = model.stage_config(shape, execution="f16", kv_cache_bytes=512 << 20, max_sequences=32,
                                 max_pass_rows=512, max_seq=4096)
        st = capi.Stage(cfg)
        model.synthesize(st, shape, seed=5, norm_sigma=0.1)
        seqs = [st.allocate(n + 16) for n in lengths]
        for s, p in zip(seqs, prompts):
            for pos in range(0, len(p), 512):
                take = min(512, len(p) - pos)
                st.execute([capi.item(s, take, pos, sample=pos + take == len(p))], token_ids=p[pos:pos + take])
        got = []
        for step in range(8):
            st.set_graphs(step >= 4)  # passes 4..7 captured and replayed (same shapes as 0..3)
            items = [capi.item(s, 1, n + step, from_device=True) for s, n in zip(seqs, lengths)]
            out = st.execute(items, token_ids=[0] * len(seqs), want_logits=step < 4)
            got.append((np.array(out["tokens"]), out.get("logits")))
        # One mixed pass: short chunks of 2-8 rows at long positions (blocks of at most 16
        # query vectors merge in the kernel, larger ones in the combine kernel, in one launch)
        # beside single-token rows.
        st.set_graphs(False)
        tails = [(2, 3, 4, 5, 8)[i % 5] if n >= 513 else 1 for i, n in enumerate(lengths)]
        items = [capi.item(s, q, n + 8) for s, n, q in zip(seqs, lengths, tails)]
        ids = np.random.default_rng(10).integers(0, shape.vocab, sum(tails)).tolist()
        out = st.execute(items, token_ids=ids, want_logits=True)
        got.append((np.array(out["tokens"]), out.get("logits")))
        kv = [st.read_kv(s, layer) for s in seqs[:12] for layer in range(shape.layers)]
        results[fold] = (got, kv)
        st.close()
    (a_out, a_kv), (b_out, b_kv) = results["1"], results["0"]
    for step, ((ta, la), (tb, lb)) in enumerate(zip(a_out, b_out)):
        assert np.array_equal(ta, tb), step
        if la is not None:
            assert np.array_equal(la.view(np.uint32), lb.view(np.uint32)), step
    for (ka, va), (kb, vb) in zip(a_kv, b_kv):
        assert np.array_equal(ka.view(np.uint32), kb.view(np.uint32))
        assert np.array_equal(va.view(np.uint32), vb.view(np.uint32))


def test_falcon3_slice_head_dim_256_matches_oracle():
    """Falcon3-3B-shaped 1-layer slice (head_dim 256, 12/4 heads, untied head, no QK-norm)."""
    _say("falcon3 slice")
    shape = _slice_shape(synthetic.FALCON3_3B, 1)
    cfg = model.stage_config(shape, execution="f16", kv_cache_bytes=64 << 20, max_sequences=4,
                             max_pass_rows=256, max_seq=2048)
    st = capi.Stage(cfg)
    model.synthesize(st, shape, seed=4, norm_sigma=0.1)
    ost = oracle.OracleStage(models.synthetic_stage(shape, seed=4, norm_sigma=0.1))
    rng = np.random.default_rng(4)
    prompts = [rng.integers(0, shape.vocab, n).tolist() for n in (90, 3)]
    seqs = [st.allocate(128) for _ in prompts]
    oseqs = [ost.allocate_sequence(128) for _ in prompts]
    out = st.execute([capi.item(s, len(p), 0) for s, p in zip(seqs, prompts)],
                     token_ids=prompts[0] + prompts[1], want_logits=True, trace=True)
    rows = 0
    for i, p in enumerate(prompts):
        tr = []
        ost.execute(np.array(p, np.uint64), 0, oseqs[i], tr)
        got = out["trace"][0][rows:rows + len(p)]
        assert np.abs(got - tr[0]).max() <= 2e-2 and cosine(got, tr[0]) >= 0.9999
        assert np.abs(out["logits"][i] - tr[1]).max() <= 2e-2
        rows += len(p)
    st.close()
