"""Passes replayed from captured HIP graphs equal eager passes bit for bit: sampled tokens,
boundary activations and the paged KV caches, over repeated decode steps with eager passes
of other shapes (prefill chunks of another sequence) between the replays, on a single
stage and on a two-stage split."""
import numpy as np
import pytest

from hllm_amd import capi, model, synthetic

pytestmark = pytest.mark.gpu


def _say(*what):
    print("[gpu-case]", *what, flush=True)


SHAPE = synthetic.with_layers(synthetic.QWEN3_0_6B, 2)


def _stage(first=True, final=True, layer_start=0, layer_end=2):
    cfg = model.stage_config(SHAPE, layer_start, layer_end, first, final, execution="f16",
                             kv_cache_bytes=64 << 20, max_sequences=16, max_pass_rows=256,
                             max_seq=1024)
    st = capi.Stage(cfg)
    model.synthesize(st, SHAPE, seed=3, norm_sigma=0.1)
    return st


def _run(st, graphs, steps=7):
    """Prefill four sequences, then decode them together for `steps` passes; every other
    step an eager pass of another shape (a prefill chunk of a side sequence) runs between."""
    st.set_graphs(graphs)
    rng = np.random.default_rng(11)
    lengths = [9, 30, 17, 64]
    seqs = [st.allocate(n + steps + 4) for n in lengths]
    side = st.allocate(256)
    for s, n in zip(seqs, lengths):
        st.execute([capi.item(s, n, 0)], token_ids=rng.integers(0, SHAPE.vocab, n).tolist())
    tokens, side_pos = [], 0
    for step in range(steps):
        items = [capi.item(s, 1, n + step, from_device=True) for s, n in zip(seqs, lengths)]
        out = st.execute(items, token_ids=[0] * len(seqs))
        tokens.append(out["tokens"].copy())
        if step % 2:
            st.execute([capi.item(side, 5 + step, side_pos, sample=False)],
                       token_ids=rng.integers(0, SHAPE.vocab, 5 + step).tolist())
            side_pos += 5 + step
    kv = [st.read_kv(s, layer) for s in seqs for layer in range(2)]
    for s in seqs + [side]:
        st.release(s)
    return np.array(tokens), kv


def test_graph_replay_equals_eager_single_stage():
    _say("graph replay, single stage")
    st = _stage()
    t_eager, kv_eager = _run(st, False)
    cap0, rep0 = st.graph_stats()
    t_graph, kv_graph = _run(st, True)
    cap, rep = st.graph_stats()
    assert cap - cap0 >= 1 and rep - rep0 >= 5  # decode shape captured at its second pass
    np.testing.assert_array_equal(t_eager, t_graph)
    for (ke, ve), (kg, vg) in zip(kv_eager, kv_graph):
        np.testing.assert_array_equal(ke, kg)
        np.testing.assert_array_equal(ve, vg)
    st.close()


def test_graph_replay_equals_eager_two_stages():
    """Stage 0 (layer 0) hands F16 boundary activations to stage 1 (layer 1, final):
    identical boundaries and tokens with and without graphs."""
    _say("graph replay, two stages")
    s0, s1 = _stage(True, False, 0, 1), _stage(False, True, 1, 2)
    runs = []
    for graphs in (False, True):
        s0.set_graphs(graphs)
        s1.set_graphs(graphs)
        rng = np.random.default_rng(5)
        lengths = [12, 40, 7]
        a = [s0.allocate(n + 12) for n in lengths]
        b = [s1.allocate(n + 12) for n in lengths]
        bounds, toks = [], []
        for x, y, n in zip(a, b, lengths):
            o = s0.execute([capi.item(x, n, 0)], token_ids=rng.integers(0, SHAPE.vocab, n).tolist())
            t = s1.execute([capi.item(y, n, 0)], boundary=o["boundary"])
            toks.append(int(t["tokens"][0]))
        last = list(toks)
        for step in range(6):
            o = s0.execute([capi.item(x, 1, n + step) for x, n in zip(a, lengths)],
                           token_ids=last)
            bounds.append(o["boundary"].copy())
            t = s1.execute([capi.item(y, 1, n + step) for y, n in zip(b, lengths)],
                           boundary=o["boundary"])
            last = [int(v) for v in t["tokens"]]
            toks.extend(last)
        runs.append((np.array(bounds), toks))
        for x, y in zip(a, b):
            s0.release(x)
            s1.release(y)
    assert s0.graph_stats()[1] >= 3 and s1.graph_stats()[1] >= 3
    np.testing.assert_array_equal(runs[0][0], runs[1][0])
    assert runs[0][1] == runs[1][1]
    s0.close()
    s1.close()
