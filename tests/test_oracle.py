"""Pins the CPU oracle before anything is checked against it.

* golden vectors: the reference's Transformers fixture (tests/golden/qwen3_tiny_reference.json,
  used by hLLM tests/cpp/qwen3_test.cpp:103-135 at 2e-5);
* known answers from the reference's tests (half_test.cpp, sampling_test.cpp,
  llama_test.cpp);
* the reference's own arithmetic compiled into oracle/_ref: bit-exact agreement;
* closed forms and invariants (incremental decode == one-shot causal, RoPE identities,
  packing by brute force, generator statistics).
A planted mistake in the oracle (dropped term, wrong sign, swapped operand) fails at least
one of these: see test_planted_mistakes_are_caught.
"""
import ctypes as C
import math

import numpy as np
import pytest

import oracle
from hllm_amd import synthetic
from tests import models

REF = oracle.ref()
needs_ref = pytest.mark.skipif(REF is None, reason="oracle/_ref not built (reference absent)")


# ----------------------------------------------------------------------- half codec

def test_f16_known_values():  # hLLM tests/cpp/half_test.cpp:13-33
    L = oracle.lib()
    assert L.orc_f32_from_f16(0x0000) == 0.0
    assert L.orc_f32_from_f16(0x3C00) == 1.0
    assert L.orc_f32_from_f16(0xC000) == -2.0
    assert L.orc_f16_from_f32(1.0) == 0x3C00
    assert L.orc_f16_from_f32(-2.0) == 0xC000
    assert math.isinf(L.orc_f32_from_f16(0x7C00))
    assert math.isnan(L.orc_f32_from_f16(0x7E00))
    assert L.orc_f16_from_f32(float("inf")) == 0x7C00
    assert L.orc_f16_from_f32(float("-inf")) == 0xFC00
    assert L.orc_f16_from_f32(float("nan")) & 0x7C00 == 0x7C00
    assert L.orc_f16_from_f32(1.00048828125) == 0x3C00  # ties to even
    assert L.orc_f16_from_f32(1.00146484375) == 0x3C02


def test_f16_decode_matches_numpy_for_all_finite_codes():
    bits = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    ours = oracle.f16_decode(bits)
    npv = bits.view(np.float16).astype(np.float32)
    finite = np.isfinite(npv)
    assert np.array_equal(ours[finite].view(np.uint32), npv[finite].view(np.uint32))
    assert np.array_equal(np.isnan(ours), np.isnan(npv))


def test_f16_encode_matches_numpy_rne():
    rng = np.random.default_rng(0)
    vals = np.concatenate([
        rng.standard_normal(200000).astype(np.float32) * 10.0 ** rng.integers(-9, 6, 200000),
        np.arange(65536, dtype=np.uint32).astype(np.uint16).view(np.float16).astype(np.float32),
        np.array([65504.0, 65519.99, 65520.0, 6.1e-5, 5.96e-8, 2.98e-8, 2.99e-8, -0.0],
                 np.float32)]).astype(np.float32)
    vals = vals[np.isfinite(vals)]
    assert np.array_equal(oracle.f16_encode(vals), vals.astype(np.float16).view(np.uint16))


@needs_ref
def test_half_codecs_equal_reference_bitwise():
    L = oracle.lib()
    for b in range(0, 65536, 7):
        assert np.float32(L.orc_f32_from_f16(b)).tobytes() == \
            np.float32(REF.ref_f32_from_f16(b)).tobytes() or math.isnan(REF.ref_f32_from_f16(b))
        assert np.float32(L.orc_f32_from_bf16(b)).tobytes() == \
            np.float32(REF.ref_f32_from_bf16(b)).tobytes() or math.isnan(REF.ref_f32_from_bf16(b))
    rng = np.random.default_rng(1)
    samples = rng.integers(0, 2**32, 20000, dtype=np.uint64).astype(np.uint32).view(np.float32)
    for v in samples:
        assert L.orc_f16_from_f32(float(v)) == REF.ref_f16_from_f32(float(v))
        assert L.orc_bf16_from_f32(float(v)) == REF.ref_bf16_from_f32(float(v))


def test_bf16_known_values():  # hLLM tests/cpp/half_test.cpp:35-50
    L = oracle.lib()
    for bits in (0x7F800001, 0x7FFFFFFF, 0xFF800001, 0xFFFFFFFF):
        f = np.uint32(bits).view(np.float32)
        out = L.orc_bf16_from_f32(float(f))
        assert math.isnan(L.orc_f32_from_bf16(out))
        assert out & 0x8000 == (bits >> 16) & 0x8000
    assert L.orc_bf16_from_f32(float("inf")) == 0x7F80
    assert L.orc_bf16_from_f32(float("-inf")) == 0xFF80
    assert L.orc_bf16_from_f32(-0.0) == 0x8000
    assert L.orc_f32_from_bf16(0x3F80) == 1.0
    assert L.orc_bf16_from_f32(L.orc_f32_from_bf16(0x3F81)) == 0x3F81


# ------------------------------------------------------------------------- sampling

def test_sampling_known_answers():  # hLLM tests/cpp/sampling_test.cpp:11-23
    lg = np.array([0.0, 2.0, 2.0], np.float32)
    assert oracle.sample_token(lg, oracle.Sampling(), 0)[0] == 1
    for seed in range(100):
        assert oracle.sample_token(lg, oracle.Sampling(1.0, 1.0, 1, seed), 0)[0] == 1
        assert oracle.sample_token(lg, oracle.Sampling(1.0, 0.1, 0, seed), 0)[0] == 1
    with pytest.raises(oracle.OracleError):
        oracle.sample_token(lg, oracle.Sampling(-1.0, 1.0), 0)
    with pytest.raises(oracle.OracleError):
        oracle.sample_token(lg, oracle.Sampling(1.0, 0.0), 0)
    with pytest.raises(oracle.OracleError):
        oracle.sample_token(np.array([np.nan], np.float32), oracle.Sampling(), 0)


def test_sampling_seeded_distribution():  # hLLM tests/cpp/sampling_test.cpp:25-39
    lg = np.zeros(3, np.float32)
    counts = [0, 0, 0]
    for step in range(6000):
        a = oracle.sample_token(lg, oracle.Sampling(1.0, 1.0, 0, 42), step)[0]
        assert a == oracle.sample_token(lg, oracle.Sampling(1.0, 1.0, 0, 42), step)[0]
        counts[a] += 1
    assert all(1800 < c < 2200 for c in counts)


def test_sampling_logprobs():  # hLLM tests/cpp/sampling_test.cpp:41-56
    lg = np.zeros(3, np.float32)
    s = oracle.Sampling(0.0, 1.0, 0, 42, True, 2)
    tok, lp, top = oracle.sample_token(lg, s, 0)
    assert tok == 0 and abs(lp + math.log(3.0)) < 1e-12
    assert [t for t, _ in top] == [0, 1]
    s.temperature = 0.8
    assert oracle.sample_token(lg, s, 8)[0] == oracle.sample_token(
        lg, oracle.Sampling(0.8, 1.0, 0, 42), 8)[0]
    s.top_logprobs = 6
    with pytest.raises(oracle.OracleError):
        oracle.sample_token(lg, s, 0)


def _ref_sample(lg, s, gi):
    tok, lp = C.c_uint64(), C.c_double()
    ids, vals = np.zeros(8, np.uint64), np.zeros(8, np.float64)
    st = REF.ref_sample_token(lg, lg.size, s.temperature, s.top_p, s.top_k, s.seed, gi,
                              int(s.return_logprobs), s.top_logprobs, C.byref(tok), C.byref(lp),
                              ids, vals)
    return st, tok.value, lp.value, list(ids[:s.top_logprobs]), list(vals[:s.top_logprobs])


@needs_ref
def test_sampling_equals_reference_bitwise():
    rng = np.random.default_rng(3)
    for trial in range(60):
        n = int(rng.choice([3, 11, 256, 4096, 151936]))
        lg = (rng.standard_normal(n) * rng.choice([0.5, 1.0, 4.0])).astype(np.float32)
        if trial % 5 == 0:
            lg[rng.integers(0, n, 4)] = lg.max()  # ties at the maximum
        s = oracle.Sampling(float(rng.choice([0.0, 0.3, 0.8, 1.0, 2.5])),
                            float(rng.choice([1.0, 0.95, 0.9, 0.5, 0.01])),
                            int(rng.choice([0, 0, 1, 8, 50])), int(rng.integers(0, 2**63)),
                            True, int(rng.integers(0, 6)))
        gi = int(rng.integers(0, 1000))
        tok, lp, top = oracle.sample_token(lg, s, gi)
        st, rtok, rlp, rids, rvals = _ref_sample(lg, s, gi)
        assert st == 0 and tok == rtok and lp == rlp
        assert [t for t, _ in top] == rids and [v for _, v in top] == rvals


# ------------------------------------------------------------- layer closed forms

def test_rms_norm_hand_calculation():  # hLLM tests/cpp/llama_test.cpp:70-76
    out = oracle.rms_norm(np.array([[3.0, 4.0]]), np.array([1.0, 2.0]), 1e-6)
    inv = 1.0 / math.sqrt(12.5 + 1e-6)
    assert abs(out[0, 0] - 3.0 * inv) < 1e-6 and abs(out[0, 1] - 8.0 * inv) < 1e-6


def test_rope_half_rotation_layout():  # hLLM tests/cpp/llama_test.cpp:78-85
    v = oracle.apply_rope(np.array([[1.0, 2.0, 3.0, 4.0]]), 1, 4, 1, 1e4)
    assert abs(v[0, 0] - (math.cos(1.0) - 3.0 * math.sin(1.0))) < 1e-6
    assert abs(v[0, 2] - (3.0 * math.cos(1.0) + math.sin(1.0))) < 1e-6
    assert abs(v[0, 1] - (2.0 * math.cos(0.01) - 4.0 * math.sin(0.01))) < 1e-6


def test_rope_preserves_pair_norms_and_is_identity_at_zero():
    rng = np.random.default_rng(2)
    x = rng.standard_normal((5, 3 * 8)).astype(np.float32)
    assert np.array_equal(oracle.apply_rope(x[:1], 3, 8, 0, 1e6), x[:1])
    y = oracle.apply_rope(x, 3, 8, 17, 1e6).reshape(5, 3, 2, 4)
    xx = x.reshape(5, 3, 2, 4)
    assert np.allclose((y ** 2).sum(2), (xx ** 2).sum(2), rtol=1e-5)


def test_linear_matches_float64_and_reference_order():
    rng = np.random.default_rng(4)
    x = rng.standard_normal((3, 70)).astype(np.float32)
    w = rng.standard_normal((9, 70)).astype(np.float32)
    y = oracle.linear(x, w)
    assert np.allclose(y, x.astype(np.float64) @ w.T.astype(np.float64), atol=1e-4)
    seq = np.zeros((3, 9), np.float32)  # the reference's sequential F32 sum, in numpy
    for k in range(70):
        seq = (seq + x[:, k:k + 1] * w[:, k][None, :]).astype(np.float32)
    assert np.array_equal(y, seq)


def test_greedy_first_maximum_and_nonfinite():  # hLLM tests/cpp/llama_test.cpp:118-136
    assert oracle.greedy_last(np.array([[9, 1, 2, 3], [-1, 4, 4, 0]], np.float32)) == 1
    nan, inf = float("nan"), float("inf")
    for row in ([nan, 1, 2], [1, nan, 2], [1, 2, inf], [-inf, 0, 1]):
        with pytest.raises(oracle.OracleError):
            oracle.greedy_last(np.array([[0, 0, 0], row], np.float32))
    assert oracle.greedy_last(np.array([[nan, nan, nan], [0, 5, 1]], np.float32)) == 1


def _layer_cfg():  # hLLM tests/cpp/llama_test.cpp:50-66
    return oracle.Config(4, 6, 2, 1, 2, 16, 1e-5, 1e4, 0)


def _det_layer(cfg, phase):
    def m(r, c, p):
        i = np.arange(r * c, dtype=np.float32)
        return (0.12 * np.sin((i + 1) * np.float32(0.37) + np.float32(p))).astype(
            np.float32).reshape(r, c)
    H, I, kw = cfg.hidden_size, cfg.intermediate_size, cfg.key_value_heads * cfg.head_dimension
    return [0.9 + np.arange(H, dtype=np.float32) * 0.03, m(H, H, phase), m(kw, H, phase + .1),
            m(kw, H, phase + .2), m(H, H, phase + .3), 1.1 - np.arange(H, dtype=np.float32) * 0.02,
            m(I, H, phase + .4), m(I, H, phase + .5), m(H, I, phase + .6)]


def _run_layer(cfg, arrays, x, first, kv):
    arrays = [np.ascontiguousarray(a, np.float32) for a in arrays]
    ptrs = [a.ctypes.data for a in arrays] + [None] * (11 - len(arrays))
    layer = oracle._Layer(*ptrs)
    out = np.empty_like(x)
    st = oracle.lib().orc_transformer_layer(x, x.shape[0], C.byref(layer), C.byref(cfg), first,
                                            C.byref(kv), out)
    assert st == 0
    return out


def test_incremental_decode_equals_one_shot():  # hLLM tests/cpp/llama_test.cpp:87-109
    cfg = _layer_cfg()
    w = _det_layer(cfg, 0.2)
    prompt = np.array([[0.2, -0.1, 0.5, 0.7], [-0.4, 0.3, 0.1, 0.6]], np.float32)
    dec = np.array([[0.8, -0.2, 0.4, -0.5]], np.float32)
    kv1, kv2 = oracle._Kv(), oracle._Kv()
    oracle.lib().orc_kv_init(C.byref(kv1), 16, 1, 2)
    oracle.lib().orc_kv_init(C.byref(kv2), 16, 1, 2)
    one = _run_layer(cfg, w, np.concatenate([prompt, dec]), 0, kv1)
    _run_layer(cfg, w, prompt, 0, kv2)
    inc = _run_layer(cfg, w, dec, 2, kv2)
    assert np.allclose(inc[0], one[2], atol=1e-6) and kv2.length == 3


# ------------------------------------------------------- Transformers golden vectors

def test_tiny_reference_full_prefill():  # hLLM tests/cpp/qwen3_test.cpp:103-116
    fx = models.tiny_reference()
    stage = oracle.OracleStage(models.tiny_reference_stage())
    seq = stage.allocate_sequence(32)
    trace = []
    h = stage.forward(models.tiny_rows(fx["embeddings"], 0, 5), 0, seq, trace)
    for layer in range(2):
        np.testing.assert_allclose(trace[layer], models.tiny_rows(fx["layer_outputs"][layer], 0, 5),
                                   atol=2e-5, rtol=0)
        k, v = seq.cache_arrays(layer)
        ek = np.asarray(fx["keys"][layer]["values"], np.float32).reshape(2, 5, 4).transpose(1, 0, 2)
        ev = np.asarray(fx["values"][layer]["values"], np.float32).reshape(2, 5, 4).transpose(
            1, 0, 2)
        np.testing.assert_allclose(k, ek, atol=2e-5, rtol=0)
        np.testing.assert_allclose(v, ev, atol=2e-5, rtol=0)
    w = stage.w
    logits = np.empty((5, 11), np.float32)
    oracle.lib().orc_final_logits(h, 5, 6, w.tensors["model.norm.weight"], w.head, 11, 1e-6,
                                  logits)
    np.testing.assert_allclose(logits, models.tiny_rows(fx["logits"], 0, 5), atol=2e-5, rtol=0)


def test_tiny_reference_prefill_then_two_decodes():  # hLLM tests/cpp/qwen3_test.cpp:118-135
    fx = models.tiny_reference()
    stage = oracle.OracleStage(models.tiny_reference_stage())
    seq = stage.allocate_sequence(32)
    for position, count in ((0, 3), (3, 1), (4, 1)):
        trace = []
        out = stage.execute(np.array([1, 4, 2, 8, 3][position:position + count], np.uint64),
                            position, seq, trace)
        for layer in range(2):
            np.testing.assert_allclose(
                trace[layer], models.tiny_rows(fx["layer_outputs"][layer], position, count),
                atol=2e-5, rtol=0)
        np.testing.assert_allclose(trace[2], models.tiny_rows(fx["logits"], position + count - 1,
                                                              1)[0], atol=2e-5, rtol=0)
        assert out[1] == int(np.argmax(models.tiny_rows(fx["logits"], position + count - 1, 1)))


def test_tiny_reference_split_stages_match_whole():  # hLLM tests/cpp/stage_test.cpp:26-55
    fx = models.tiny_reference()
    first = oracle.OracleStage(models.tiny_reference_stage(0, 1, True, False))
    last = oracle.OracleStage(models.tiny_reference_stage(1, 2, False, True))
    s0, s1 = first.allocate_sequence(32), last.allocate_sequence(32)
    out = first.execute(np.array([1, 4, 2, 8, 3], np.uint64), 0, s0)
    assert out[0] == "boundary"
    wire = oracle.f16_decode(out[1])
    np.testing.assert_allclose(wire, models.tiny_rows(fx["layer_outputs"][0], 0, 5), atol=1e-3)
    trace = []
    tok = last.execute(out[1], 0, s1, trace)
    np.testing.assert_allclose(trace[0], models.tiny_rows(fx["layer_outputs"][1], 0, 5),
                               atol=1e-3)
    assert tok[1] == int(np.argmax(models.tiny_rows(fx["logits"], 4, 1)))


# ------------------------------------------------ bit-exact against the reference code

def _ref_layer(cfg, arrays):
    arrays = [np.ascontiguousarray(a, np.float32) for a in arrays]
    ptrs = [a.ctypes.data for a in arrays] + [None] * (11 - len(arrays))
    return REF.ref_layer_create(C.byref(cfg), *ptrs), arrays


@needs_ref
@pytest.mark.parametrize("qk_norm,rows_plan", [(1, [(0, 7), (7, 1), (8, 3)]),
                                               (0, [(0, 1), (1, 5), (6, 1)]),
                                               # large enough for the threaded attention
                                               (1, [(0, 260), (260, 1), (261, 120)])])
def test_transformer_layer_equals_reference_bitwise(qk_norm, rows_plan):
    shape = synthetic.ModelShape("t", 1, 48, 80, 6, 2, 16, 97, theta=1e4, qk_norm=bool(qk_norm),
                                 tied=True, dtype="f32", max_seq=512)
    w = models.synthetic_stage(shape, seed=5, norm_sigma=0.2)
    cfg = models.oracle_config(shape)
    arrays = w.layer(0)
    handle, keep = _ref_layer(cfg, arrays)
    cache = REF.ref_cache_create(512, 2, 16)
    kv = oracle._Kv()
    oracle.lib().orc_kv_init(C.byref(kv), 512, 2, 16)
    rng = np.random.default_rng(qk_norm)
    for first, rows in rows_plan:
        x = rng.standard_normal((rows, 48)).astype(np.float32)
        ours = _run_layer(cfg, arrays, x, first, kv)
        theirs = np.empty_like(x)
        assert REF.ref_transformer_layer(C.byref(cfg), handle, x, rows, first, cache, theirs) == 0
        assert np.array_equal(ours.view(np.uint32), theirs.view(np.uint32))
    n = kv.length * 2 * 16
    rk, rv = np.empty(n, np.float32), np.empty(n, np.float32)
    REF.ref_cache_read(cache, rk, rv)
    assert np.array_equal(np.ctypeslib.as_array(kv.keys, (n,)), rk)
    assert np.array_equal(np.ctypeslib.as_array(kv.values, (n,)), rv)
    REF.ref_layer_destroy(handle)
    REF.ref_cache_destroy(cache)


@needs_ref
def test_final_logits_and_greedy_equal_reference_bitwise():
    rng = np.random.default_rng(9)
    h = rng.standard_normal((3, 40)).astype(np.float32)
    norm = (1 + 0.1 * rng.standard_normal(40)).astype(np.float32)
    head = (0.02 * rng.standard_normal((333, 40))).astype(np.float32)
    ours, theirs = np.empty((3, 333), np.float32), np.empty((3, 333), np.float32)
    oracle.lib().orc_final_logits(h, 3, 40, norm, head, 333, 1e-6, ours)
    assert REF.ref_final_logits(h, 3, 40, norm, head, 333, 1e-6, theirs) == 0
    assert np.array_equal(ours, theirs)
    tok = C.c_uint64()
    assert REF.ref_greedy_last(theirs, 3, 333, C.byref(tok)) == 0
    assert oracle.greedy_last(ours) == tok.value


# ------------------------------------------------------------------------ packing

def test_pack_matches_brute_force():
    rng = np.random.default_rng(11)
    block, width = 16, 12
    table = np.full((5, width), -1, np.int32)
    perm = rng.permutation(5 * width).astype(np.int32)
    table[:] = perm.reshape(5, width)
    slots = np.array([3, 0, 4, 1], np.uint32)
    firsts = np.array([0, 37, 100, 5], np.uint64)
    lens = np.array([20, 1, 9, 1], np.uint32)
    cu, items, pos, sl = oracle.pack(slots, firsts, lens, table, block)
    assert list(cu) == [0, 20, 21, 30, 31]
    r = 0
    for i in range(4):
        for j in range(lens[i]):
            p = int(firsts[i]) + j
            assert items[r] == i and pos[r] == p
            assert sl[r] == table[slots[i], p // block] * block + p % block
            r += 1


# ---------------------------------------------------------------- weight generator

def test_synthetic_weights_are_seeded_normal_and_f16_consistent():
    a = oracle.synth_f32(0, 17, 200000)
    assert np.array_equal(a, oracle.synth_f32(0, 17, 200000))
    assert not np.array_equal(a, oracle.synth_f32(1, 17, 200000))
    assert not np.array_equal(a, oracle.synth_f32(0, 18, 200000))
    assert abs(a.mean()) < 2e-4 and abs(a.std() - 0.02) < 2e-4
    assert np.abs(a).max() <= 6 * 0.02 + 1e-6
    # Irwin-Hall(12) kurtosis is 3 - 1.2/12 = 2.9
    assert abs(((a / a.std()) ** 4).mean() - 2.9) < 0.05
    part = oracle.synth_f32(0, 17, 1000, first=5000)
    assert np.array_equal(part, a[5000:6000])
    assert np.array_equal(oracle.synth_f16(0, 17, 1000), oracle.f16_encode(a[:1000]))
    ones = oracle.synth_f32(3, 2, 64, mean=1.0, sigma=0.0)
    assert np.all(ones == 1.0)
    # the first draw, worked by hand from the definition
    sm = oracle.lib().orc_splitmix64
    total = sum(((sm(0 + 0x9E3779B97F4A7C15 * ((17 << 40) + j) & (2**64 - 1)) >> (16 * q))
                 & 0xFFFF) for j in range(3) for q in range(4))
    assert a[0] == np.float32(np.float32((total + 6 - 6 * 65536) / 65536.0) * np.float32(0.02))


def test_splitmix64_published_vector():
    # SplitMix64 seeded with 0: first output 0xE220A8397B1DCDAF (Vigna's reference code).
    assert oracle.lib().orc_splitmix64(0) == 0xE220A8397B1DCDAF


# ------------------------------------------------------------ planted mistakes

def test_planted_mistakes_are_caught():
    """Perturbations of the oracle's formulas fail the golden comparison."""
    fx = models.tiny_reference()
    base = models.tiny_reference_stage()
    x = models.tiny_rows(fx["embeddings"], 0, 5)
    expect = models.tiny_rows(fx["layer_outputs"][1], 0, 5)

    def run(mutate):
        w = models.tiny_reference_stage()
        mutate(w.tensors)
        st = oracle.OracleStage(w)
        seq = st.allocate_sequence(32)
        return st.forward(x, 0, seq)

    good = run(lambda t: None)
    assert np.abs(good - expect).max() < 2e-5
    mistakes = [
        lambda t: t.__setitem__("model.layers.0.self_attn.q_norm.weight",
                                t["model.layers.0.self_attn.k_norm.weight"]),
        lambda t: t.__setitem__("model.layers.1.mlp.up_proj.weight",
                                t["model.layers.1.mlp.gate_proj.weight"]),
        lambda t: t.__setitem__("model.layers.0.input_layernorm.weight",
                                t["model.layers.0.post_attention_layernorm.weight"]),
        lambda t: t.__setitem__("model.layers.1.self_attn.v_proj.weight",
                                -t["model.layers.1.self_attn.v_proj.weight"]),
    ]
    for mutate in mistakes:
        assert np.abs(run(mutate) - expect).max() > 1e-3
    assert base is not None


@pytest.mark.parametrize("mistake", [1, 2, 3, 4, 5])
def test_planted_formula_mistakes_fail_the_golden_vectors(mistake):
    """Each formula mistake planted in the oracle (dropped residual, RoPE sign, causal
    off-by-one, swapped SwiGLU halves, wrong RMS mean) fails the reference fixture."""
    fx = models.tiny_reference()
    x = models.tiny_rows(fx["embeddings"], 0, 5)
    expect = models.tiny_rows(fx["layer_outputs"][1], 0, 5)
    flag = C.c_int.in_dll(oracle.lib(), "orc_planted_mistake")
    try:
        flag.value = mistake
        st = oracle.OracleStage(models.tiny_reference_stage())
        got = st.forward(x, 0, st.allocate_sequence(32))
    finally:
        flag.value = 0
    assert np.abs(got - expect).max() > 1e-3
    st = oracle.OracleStage(models.tiny_reference_stage())
    assert np.abs(st.forward(x, 0, st.allocate_sequence(32)) - expect).max() < 2e-5
