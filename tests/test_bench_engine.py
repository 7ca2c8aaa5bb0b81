"""The benchmark's continuous-batching engine against a stand-in stage (no GPU): with the next
pass planned while the current one runs, every pass still starts each sequence at its current
length, at most one pass is in flight, no sequence is released or reused while a pass that
reads it is in flight, a device-fed row only follows a pass that sampled its sequence, and a
drained timed region holds exactly the passes it counts. The pre-start brings the engine to
its stated concurrency before the first timed step."""
import numpy as np

import bench
from hllm_amd import capi


class _Lib:
    def __init__(self, stage):
        self.stage = stage

    def hllm_rocm_stage_submit(self, handle, pass_ref):
        st = self.stage
        assert st.in_flight is None, "a pass is already in flight"
        p = pass_ref._obj
        used = set()
        for i in range(p.items):
            it = p.item[i]
            assert st.live.get(it.sequence), "pass over a released sequence"
            assert it.first_position == st.length[it.sequence]
            assert it.query_tokens >= 1 and it.sequence not in used
            if it.flags & capi.ITEM_TOKEN_FROM_DEVICE:
                assert it.query_tokens == 1 and st.sampled.get(it.sequence), "no device token"
            st.length[it.sequence] += it.query_tokens
            st.sampled[it.sequence] = bool(it.flags & capi.ITEM_SAMPLE)
            used.add(it.sequence)
        st.in_flight = used
        st.passes += 1
        return 0

    def hllm_rocm_stage_wait(self, handle):
        assert self.stage.in_flight is not None, "no pass in flight"
        self.stage.in_flight = None
        return 0


class _Ref:
    def __init__(self, obj):
        self._obj = obj


class _Stage:
    handle = None

    def __init__(self):
        self.count, self.length, self.live, self.in_flight, self.passes = 0, {}, {}, None, 0
        self.sampled = {}
        self.lib = _Lib(self)

    def execute(self, items, token_ids=None):
        p = capi.Pass()
        arr = (capi.Item * len(items))(*items)
        p.items, p.item = len(items), arr
        assert sum(it.query_tokens for it in items) == len(token_ids)
        self.lib.hllm_rocm_stage_submit(None, _Ref(p))
        self.lib.hllm_rocm_stage_wait(None)
        return {}

    def allocate(self, tokens):
        self.count += 1
        self.length[self.count], self.live[self.count] = 0, True
        return self.count

    def release(self, seq):
        assert self.in_flight is None or seq not in self.in_flight, "released while in flight"
        assert self.live[seq]
        self.live[seq] = False


def test_pipelined_engine_keeps_sequence_state(monkeypatch):
    monkeypatch.setattr(capi, "check", lambda status: None)
    stage = _Stage()
    engine = bench.Engine(stage, 16, 64, bench.request_stream(np.random.default_rng(3), 1000, 1.0))
    for _ in range(150):
        engine.step()
    engine.drain()
    assert stage.in_flight is None
    before = stage.passes
    tokens = 0
    for i in range(200):
        tokens += engine.step(last=i == 199)[0]
    assert stage.in_flight is None and stage.passes - before == 200
    assert tokens > 0
    engine.release_all()
    assert not any(stage.live.values())


def test_prestart_reaches_the_stated_concurrency(monkeypatch):
    """With no warmup at all, every timed pass holds (nearly) the stated number of requests."""
    monkeypatch.setattr(capi, "check", lambda status: None)
    stage = _Stage()
    engine = bench.Engine(stage, 16, 64, bench.request_stream(np.random.default_rng(4), 1000, 1.0))
    engine.prestart(np.random.default_rng(5), 1000, 128)
    assert len(engine.active) == 16 and stage.in_flight is None
    assert all(stage.sampled[r.seq] for r in engine.active)
    active = [engine.step(last=i == 99)[3] for i in range(100)]
    assert min(active) >= 15 and np.mean(active) >= 0.95 * 16
    engine.release_all()
    assert not any(stage.live.values())


def test_step_work_closed_form():
    """The workload step roofline's algorithmic work of one pass holding a decode row at
    context 100 and a 512-token prefill chunk that completes its prompt: every layer weight
    and the LM head read once, 100 cached positions read and 513 written, FLOPs 2 per weight
    and row (the head for the two sampled rows) plus attention's 4 * heads * head_dim per
    (query, key) pair per layer."""
    from hllm_amd import synthetic
    shape = synthetic.QWEN3_4B

    class Req:
        def __init__(self, length, fed, prompt):
            self.length, self.fed, self.prompt = length, fed, [0] * prompt

    w = bench.StepWork(shape)
    w.add([Req(100, 10, 10)], [(Req(0, 0, 512), 512)])
    params = 36 * (4096 * 2560 + 2 * 1024 * 2560 + 2560 * 4096 + 3 * 9728 * 2560 + 2 * 2560 + 2 * 128)
    head = 151936 * 2560
    kv_tok = 36 * 8 * 128 * 2 * 2
    assert w.bytes == 2 * (params + head) + (100 + 513) * kv_tok
    pairs = 101 + 512 * 513 // 2
    assert w.flops == 2.0 * 513 * params + 2.0 * 2 * head + 4.0 * 32 * 128 * 36 * pairs
    t = max(w.bytes / 8e12, w.flops / 2.5e15)
    assert abs(w.roof_s - t) < 1e-15 and w.hbm_passes == 0
    s = w.summary(2 * t)
    assert abs(s["frac"] - 0.5) < 1e-12 and s["steps"] == 1
