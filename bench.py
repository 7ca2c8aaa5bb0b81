"""Benchmark of the MI355X decoder stage worker on its headline workload.

Workload (one GPU): a Qwen3-4B-shaped dense decoder (36 layers, hidden 2560, 32/8 heads,
head_dim 128, SwiGLU 9728, vocabulary 151936, QK-norm, tied head) with seeded
random-init F16 weights, serving 64 concurrent requests by continuous batching: Poisson
arrivals, prompt lengths lognormal (median 256, sigma 1, clipped to [16, 2048]), output
lengths uniform in [64, 256], prefill in chunks of at most 512 tokens per pass mixed with
the decode rows of every running request. One step = one pass of the stage over one such
ragged batch; the value is output (sampled) tokens per second over the timed steps.

Also measured: pure decode passes of 64 rows (HBM bytes / step time against 8 TB/s and
against a measured streaming-read ceiling),
512-token prefill passes (FLOPs / time against 2.5 PFLOP/s dense F16), p50/p99 step
latency, per-kernel HIP-event roofline of the dominant kernel, and the reference CPU
worker's arithmetic (oracle/_ref, one thread) timed on this host.

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W]
"""
from __future__ import annotations

import argparse
import collections
import ctypes as C
import json
import math
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

from hllm_amd import capi, model, synthetic  # noqa: E402

METRIC = "Qwen3-4B F16 output tok/s @64 concurrent; decode HBM GB/s as % of peak"
HBM_PEAK_GBS = 8000.0
MFMA_F16_PEAK_TFLOPS = 2500.0


def log(*what):
    print("[bench]", *what, file=sys.stderr, flush=True)


# ------------------------------------------------------------------ workload

class Request:
    __slots__ = ("prompt", "out_len", "seq", "fed", "generated", "length", "arrival")

    def __init__(self, prompt, out_len, arrival):
        self.prompt, self.out_len, self.arrival = prompt, out_len, arrival
        self.seq, self.fed, self.generated, self.length = -1, 0, 0, 0


def request_stream(rng, vocab, rate_per_step):
    step = 0.0
    while True:
        step += rng.exponential(1.0 / rate_per_step)
        n = int(np.clip(round(math.exp(math.log(256.0) + rng.standard_normal())), 16, 2048))
        prompt = rng.integers(0, vocab, n, dtype=np.uint64)
        yield Request(prompt, int(rng.integers(64, 257)), step)


ITEM_DTYPE = np.dtype({"names": [f for f, _ in capi.Item._fields_],
                       "formats": [np.dtype(t) for _, t in capi.Item._fields_],
                       "offsets": [getattr(capi.Item, f).offset for f, _ in capi.Item._fields_],
                       "itemsize": C.sizeof(capi.Item)})


class Engine:
    """Continuous batching over one stage: every running request contributes one decode row
    (its input token fed from the device), and prefilling requests share a chunk budget.

    Steps are pipelined on the host: a step's effect on the requests (positions, finished
    outputs) does not depend on the sampled token values, so the next pass is planned and its
    inputs built while the current one runs, and submitted as soon as it completes
    (hllm_rocm_stage_submit / hllm_rocm_stage_wait). Sequences of finished requests are
    released only after their last pass has completed."""

    def __init__(self, stage, concurrency, chunk, stream):
        self.stage, self.concurrency, self.chunk, self.stream = stage, concurrency, chunk, stream
        self.waiting = collections.deque()
        self.active = []
        self.clock = 0
        self.offset = 0.0  # arrival times are counted from this step of the stream
        self.next_req = next(stream)
        self.buffers = []
        for _ in range(2):  # the pass in flight keeps its output buffer until it completes
            items = np.zeros(concurrency + chunk, ITEM_DTYPE)
            items["top_p"] = 1.0
            self.buffers.append((items, np.zeros(concurrency + chunk + 8, np.uint64),
                                 np.zeros(concurrency + chunk, np.uint64), capi.Pass()))
        self.flip = 0
        self.current = None  # the submitted pass: (sampled, rows, decode rows, finished)
        self.work = None     # StepWork accumulating the submitted passes' algorithmic work

    def _plan(self):
        """Admits arrivals and builds the next pass; None for an idle step."""
        while self.next_req.arrival - self.offset <= self.clock:
            self.waiting.append(self.next_req)
            self.next_req = next(self.stream)
        while len(self.active) < self.concurrency and self.waiting:
            r = self.waiting.popleft()
            r.seq = self.stage.allocate(len(r.prompt) + r.out_len)
            self.active.append(r)
        items, ids, tokens_out, p = self.buffers[self.flip]
        self.flip ^= 1
        n = rows = 0
        decode, prefill = [], []
        for r in self.active:
            if r.fed == len(r.prompt):
                it = items[n]
                it["sequence"], it["query_tokens"], it["first_position"] = r.seq, 1, r.length
                it["flags"] = capi.ITEM_SAMPLE | capi.ITEM_TOKEN_FROM_DEVICE
                ids[rows] = 0
                n, rows = n + 1, rows + 1
                decode.append(r)
        budget = self.chunk
        for r in self.active:
            if budget == 0:
                break
            if r.fed < len(r.prompt):
                take = min(budget, len(r.prompt) - r.fed)
                it = items[n]
                it["sequence"], it["query_tokens"], it["first_position"] = r.seq, take, r.length
                it["flags"] = capi.ITEM_SAMPLE if r.fed + take == len(r.prompt) else 0
                ids[rows:rows + take] = r.prompt[r.fed:r.fed + take]
                n, rows, budget = n + 1, rows + take, budget - take
                prefill.append((r, take))
        if n == 0:
            return None
        self.planned_active = len(self.active)
        p.items = n
        p.item = items.ctypes.data_as(C.POINTER(capi.Item))
        p.token_ids = ids.ctypes.data_as(C.POINTER(C.c_uint64))
        p.tokens = tokens_out.ctypes.data_as(C.POINTER(C.c_uint64))
        return p, rows, decode, prefill

    def _launch(self, plan):
        """Submits a planned pass (nothing for an idle step) and applies its effect on the
        requests; finished requests leave the running set now."""
        self.clock += 1
        if plan is None:  # nothing has arrived yet: an idle step launches nothing
            return (0, 0, 0, [], False, 0)
        p, rows, decode, prefill = plan
        if self.work is not None:
            self.work.add(decode, prefill)
        capi.check(self.stage.lib.hllm_rocm_stage_submit(self.stage.handle, C.byref(p)))
        sampled = len(decode)
        finished = []
        for r in decode:
            r.length += 1
            r.generated += 1
            if r.generated >= r.out_len:
                finished.append(r)
        for r, take in prefill:
            r.fed += take
            r.length += take
            if r.fed == len(r.prompt):
                r.generated = 1
                sampled += 1
        active = self.planned_active
        for r in finished:
            self.active.remove(r)
        return (sampled, rows, len(decode), finished, True, active)

    def step(self, last=False):
        """Completes one step; unless `last`, the next one is planned while it runs and
        submitted when it completes. Returns (sampled tokens, rows, decode rows, requests in
        the pass)."""
        if self.current is None:
            self.current = self._launch(self._plan())
        sampled, rows, decode, finished, submitted, active = self.current
        plan = None if last else self._plan()
        if submitted:
            capi.check(self.stage.lib.hllm_rocm_stage_wait(self.stage.handle))
        for r in finished:
            self.stage.release(r.seq)
        self.current = None if last else self._launch(plan)
        return sampled, rows, decode, active

    def prestart(self, rng, vocab, max_rows):
        """Brings the engine to its steady state before any timed step: `concurrency`
        requests of the stream are admitted at once, each with an output length drawn in
        proportion to its length from the stream's U[64, 256] and already `g ~ U[0,
        out_len)` tokens into it. A request running at a random moment is length-biased
        (long ones run more of the time) and uniformly aged, so the pre-started batch
        completes requests at the steady rate from its first step (with unbiased lengths
        it completes them almost twice as fast at first: a burst of prefill passes, then a
        lull, for a few hundred steps). Each request comes with its prompt and those tokens
        prefilled by untimed passes of up to `max_rows` rows (random IDs stand in for the
        generated tokens: only the cache contents and lengths matter to later steps). Each request's last prefill row samples, so its next
        input comes from the device like every decode row's."""
        pieces = []  # (sequence, first position, token IDs, samples)
        while len(self.active) < self.concurrency:
            r = self.next_req
            self.next_req = next(self.stream)
            while True:  # length-biased output length: accept L with probability L / 256
                r.out_len = int(rng.integers(64, 257))
                if rng.random() * 256 < r.out_len:
                    break
            g = int(rng.integers(0, r.out_len))
            r.seq = self.stage.allocate(len(r.prompt) + r.out_len)
            history = np.concatenate([r.prompt, rng.integers(0, vocab, g, dtype=np.uint64)])
            r.fed, r.length, r.generated = len(r.prompt), len(history), g + 1
            self.active.append(r)
            for pos in range(0, len(history), max_rows):
                part = history[pos:pos + max_rows]
                pieces.append((r.seq, pos, part, pos + len(part) == len(history)))
        batch, ids, rows = [], [], 0
        for seq, pos, part, last in pieces:
            if rows + len(part) > max_rows:
                self.stage.execute(batch, token_ids=np.concatenate(ids))
                batch, ids, rows = [], [], 0
            batch.append(capi.item(seq, len(part), pos, sample=last))
            ids.append(part)
            rows += len(part)
        if batch:
            self.stage.execute(batch, token_ids=np.concatenate(ids))
        # later arrivals keep their spacing, counted from the engine's next step
        self.offset = self.next_req.arrival - self.clock

    def drain(self):
        """Completes the pass in flight without starting another."""
        if self.current is not None:
            self.step(last=True)

    def release_all(self):
        self.drain()
        for r in self.active:
            self.stage.release(r.seq)
        self.active = []


# ------------------------------------------------------------------ measurements

class StepWork:
    """Algorithmic HBM bytes and FLOPs of submitted workload passes, and the time each pass
    needs at the roofline (the longer of its bytes at 8 TB/s and its FLOPs at 2.5 PFLOP/s).
    A pass reads every layer weight once (and the LM head when it samples), reads each
    item's cached keys and values once and writes its new ones; FLOPs are 2 per weight and
    row (the head only for sampled rows) plus attention's 4 * heads * head_dim per (query,
    attended key) pair per layer."""

    def __init__(self, shape):
        self.shape = shape
        self.layer_params = shape.layers * (shape.layer_weight_bytes() // 2)
        self.head_params = shape.vocab * shape.hidden
        self.kv_tok = shape.kv_bytes_per_token()
        self.passes, self.bytes, self.flops, self.roof_s, self.hbm_passes = 0, 0.0, 0.0, 0.0, 0

    def add(self, decode, prefill):
        s = self.shape
        rows = len(decode) + sum(t for _, t in prefill)
        sampled = len(decode) + sum(1 for r, t in prefill if r.fed + t == len(r.prompt))
        kv_read = sum(r.length for r in decode) + sum(r.length for r, _ in prefill)
        pairs = sum(r.length + 1 for r in decode) + sum(t * r.length + t * (t + 1) // 2 for r, t in prefill)
        nbytes = 2 * (self.layer_params + (self.head_params if sampled else 0)) + (kv_read + rows) * self.kv_tok
        flops = 2.0 * rows * self.layer_params + 2.0 * sampled * self.head_params + \
            4.0 * s.heads * s.head_dim * s.layers * pairs
        t_hbm, t_mfma = nbytes / (HBM_PEAK_GBS * 1e9), flops / (MFMA_F16_PEAK_TFLOPS * 1e12)
        self.passes += 1
        self.bytes += nbytes
        self.flops += flops
        self.roof_s += max(t_hbm, t_mfma)
        self.hbm_passes += t_hbm >= t_mfma

    def summary(self, elapsed):
        return {"frac": self.roof_s / elapsed, "roofline_ms_per_step": 1e3 * self.roof_s / self.passes,
                "bytes_per_step": self.bytes / self.passes, "flops_per_step": self.flops / self.passes,
                "hbm_bound_steps": self.hbm_passes, "steps": self.passes,
                "hbm_gb_s": self.bytes / elapsed / 1e9, "tflops": self.flops / elapsed / 1e12}


def decode_bench(stage, shape, rng, rows, steps):
    """Pure decode passes: `rows` sequences prefilled to workload-distributed lengths."""
    lengths = [int(np.clip(round(math.exp(math.log(256.0) + rng.standard_normal())), 16, 2048))
               for _ in range(rows)]
    seqs = [stage.allocate(n + steps + 8) for n in lengths]
    for s, n in zip(seqs, lengths):  # untimed prefill, 512-token chunks
        pos = 0
        while pos < n:
            take = min(512, n - pos)
            stage.execute([capi.item(s, take, pos, sample=pos + take == n)],
                          token_ids=rng.integers(0, shape.vocab, take).tolist())
            pos += take
    items = np.zeros(rows, ITEM_DTYPE)
    items["top_p"] = 1.0
    items["sequence"] = seqs
    items["query_tokens"] = 1
    items["flags"] = capi.ITEM_SAMPLE | capi.ITEM_TOKEN_FROM_DEVICE
    ids = np.zeros(rows, np.uint64)
    out = np.zeros(rows, np.uint64)
    p = capi.Pass()
    p.items = rows
    p.item = items.ctypes.data_as(C.POINTER(capi.Item))
    p.token_ids = ids.ctypes.data_as(C.POINTER(C.c_uint64))
    p.tokens = out.ctypes.data_as(C.POINTER(C.c_uint64))
    ctx = np.array(lengths, np.int64)
    times, kv_read = [], 0
    for i in range(steps + 4):
        if i == steps:  # per-kernel HIP-event timing in 4 extra, untimed passes
            stage.profile("gemm_;attention")
        items["first_position"] = ctx
        t0 = time.perf_counter()
        capi.check(stage.lib.hllm_rocm_stage_execute(stage.handle, C.byref(p)))
        if i < steps:
            times.append(time.perf_counter() - t0)
            kv_read += int((ctx + 1).sum())
        ctx += 1
    fam = {f: stage.profile_read(f)[:3] for f in ("gemm_qkv", "gemm_o", "gemm_gate_up", "gemm_down",
                                                  "gemm_lm_head", "attention")}
    stage.profile(None)
    for s in seqs:
        stage.release(s)
    kv_tok = shape.kv_bytes_per_token()
    weights = shape.layers * shape.layer_weight_bytes() + shape.vocab * shape.hidden * 2
    total_bytes = steps * (weights + rows * kv_tok) + kv_read * kv_tok
    elapsed = sum(times)
    gbs = total_bytes / elapsed / 1e9
    return {"rows": rows, "steps": steps, "mean_context": float(np.mean(lengths) + steps / 2),
            "ms_per_step": 1e3 * elapsed / steps, "tok_s": rows * steps / elapsed,
            "bytes_per_step": total_bytes / steps, "hbm_gb_s": gbs, "hbm_frac": gbs / HBM_PEAK_GBS,
            "kernels": {f: {"ms_per_launch": v[0] / max(v[1], 1), "launches": v[1],
                            "gb_s": (v[2] / v[1]) / (v[0] / v[1] * 1e-3) / 1e9 if v[1] else 0.0}
                        for f, v in fam.items()}}


def prefill_bench(stage, shape, rng, past, reps):
    """512-token prefill chunks (no sampling) at context offset `past`: MFMA utilisation."""
    flops_linear = 2 * 512 * shape.layers * (shape.layer_weight_bytes() // 2)
    pairs = sum(past + i + 1 for i in range(512))
    flops_attn = 4 * shape.heads * shape.head_dim * shape.layers * pairs
    times = []
    for _ in range(reps):
        s = stage.allocate(past + 512)
        pos = 0
        while pos < past:
            take = min(512, past - pos)
            stage.execute([capi.item(s, take, pos, sample=False)],
                          token_ids=rng.integers(0, shape.vocab, take).tolist())
            pos += take
        ids = rng.integers(0, shape.vocab, 512).tolist()
        t0 = time.perf_counter()
        stage.execute([capi.item(s, 512, past, sample=False)], token_ids=ids)
        times.append(time.perf_counter() - t0)
        stage.release(s)
    t = float(np.median(times))
    tflops = (flops_linear + flops_attn) / t / 1e12
    return {"past": past, "ms": 1e3 * t, "tflop": (flops_linear + flops_attn) / 1e12,
            "tflops": tflops, "mfma_frac": tflops / MFMA_F16_PEAK_TFLOPS}


def stage_share_bench(rng, steps, rows=128, first_layer=18):
    """One pipeline stage's share at its real shape: Qwen3-4B layers 18-35 plus the final
    norm and LM head behind an F16 boundary, 128 decode rows whose KV caches hold
    log-uniform lengths in [1, 8192] (prefilled by untimed passes of N(0, 1) boundary rows),
    greedy. Each timed step feeds 128 fresh N(0, 1) boundary rows from host memory (the
    boundary crosses PCIe, as it does between pipeline stages) and returns the tokens."""
    full = synthetic.QWEN3_4B
    layers = full.layers - first_layer
    lengths = np.exp(rng.uniform(0.0, math.log(8192.0), rows)).astype(np.int64)
    lengths = np.clip(lengths, 1, 8192)
    cfg = model.stage_config(full, first_layer, full.layers, False, True, execution="f16",
                             kv_cache_bytes=int((lengths.sum() + rows * (steps + 40)) * 73728 * 1.1) + (1 << 30),
                             max_sequences=rows + 8, max_pass_rows=2048, max_seq=8192 + steps + 64)
    stage = capi.Stage(cfg)
    model.synthesize(stage, full, seed=0, norm_sigma=0.0)
    seqs = [stage.allocate(int(n) + steps + 8) for n in lengths]
    pieces = []
    for s_, n in zip(seqs, lengths):
        for pos in range(0, int(n), 2048):
            pieces.append((s_, pos, min(2048, int(n) - pos)))
    batch, rows_in = [], 0
    for piece in pieces + [None]:
        if piece is None or rows_in + piece[2] > 2048:
            if batch:
                b = np.asarray(rng.standard_normal((rows_in, full.hidden)), np.float16).view(np.uint16)
                stage.execute([capi.item(q, t, pos, sample=False) for q, pos, t in batch], boundary=b)
            batch, rows_in = [], 0
        if piece is not None:
            batch.append(piece)
            rows_in += piece[2]
    ctx = lengths.copy()
    times = []
    for i in range(steps + 2):
        items = [capi.item(q, 1, int(c)) for q, c in zip(seqs, ctx)]
        b = np.asarray(rng.standard_normal((rows, full.hidden)), np.float16).view(np.uint16)
        t0 = time.perf_counter()
        stage.execute(items, boundary=b)
        if i >= 2:  # two untimed passes first
            times.append(time.perf_counter() - t0)
        ctx += 1
    for q in seqs:
        stage.release(q)
    stage.close()
    kv_tok = full.kv_bytes_per_token(layers)
    weights = layers * full.layer_weight_bytes() + full.vocab * full.hidden * 2
    mean_ctx = float(lengths.mean()) + 2 + (steps - 1) / 2
    bytes_per_step = weights + rows * (mean_ctx + 1) * kv_tok
    t = float(np.mean(times))
    return {"workload": f"Qwen3-4B layers {first_layer}-{full.layers - 1} + final norm and LM head, F16 "
                        f"boundary input, {rows} decode rows, KV lengths log-uniform in [1, 8192]",
            "rows": rows, "steps": steps, "mean_context": mean_ctx, "ms_per_step": 1e3 * t,
            "tok_s": rows / t, "bytes_per_step": bytes_per_step, "hbm_gb_s": bytes_per_step / t / 1e9,
            "hbm_frac": bytes_per_step / t / 1e9 / HBM_PEAK_GBS,
            "roofline_ms_per_step": 1e3 * bytes_per_step / (HBM_PEAK_GBS * 1e9)}


def cpu_baseline(shape, mean_context):
    """The reference CPU worker's own arithmetic (oracle/_ref, compiled from its sources),
    one thread: one decode step of one Qwen3-4B layer at the workload's mean context, and
    the final norm + LM head over one eighth of the vocabulary; the per-token time is
    36 layer steps + 8 head slices (an extrapolation from the measured sample)."""
    import oracle  # the CPU-baseline leg runs the reference's arithmetic as the baseline
    R = oracle.ref()
    kind = "reference"
    if R is None:
        return None
    cfg = oracle.Config(shape.hidden, shape.intermediate, shape.heads, shape.kv_heads,
                        shape.head_dim, shape.max_seq, shape.eps, shape.theta, int(shape.qk_norm))
    names = synthetic.LAYER_TENSORS
    arrays = []
    for n in names:
        tid, dims, mean, sigma = synthetic.tensor_spec(shape, f"model.layers.0.{n}")
        bits = oracle.synth_f16(0, tid, int(np.prod(dims)), mean, sigma)
        arrays.append(oracle.f16_decode(bits))
    layer = R.ref_layer_create(C.byref(cfg), *[a.ctypes.data for a in arrays])
    width = shape.kv_heads * shape.head_dim
    ctx = int(mean_context)
    cache = R.ref_cache_create(ctx + 4, shape.kv_heads, shape.head_dim)
    rng = np.random.default_rng(0)
    kv = rng.standard_normal((2, ctx, width)).astype(np.float32)
    assert R.ref_cache_append(cache, 0, np.ascontiguousarray(kv[0]), np.ascontiguousarray(kv[1]),
                              ctx, width) == 0
    x = rng.standard_normal((1, shape.hidden)).astype(np.float32)
    out = np.empty_like(x)
    layer_times = []
    for i in range(2):
        t0 = time.perf_counter()
        assert R.ref_transformer_layer(C.byref(cfg), layer, x, 1, ctx + i, cache, out) == 0
        layer_times.append(time.perf_counter() - t0)
    R.ref_layer_destroy(layer)
    R.ref_cache_destroy(cache)
    del arrays
    slice_rows = shape.vocab // 8
    tid, _, mean, sigma = synthetic.tensor_spec(shape, "model.embed_tokens.weight")
    head = oracle.f16_decode(oracle.synth_f16(0, tid, slice_rows * shape.hidden, mean, sigma))
    norm = np.ones(shape.hidden, np.float32)
    logits = np.empty((1, slice_rows), np.float32)
    t0 = time.perf_counter()
    assert R.ref_final_logits(x, 1, shape.hidden, norm, head, slice_rows, shape.eps, logits) == 0
    t_head = (time.perf_counter() - t0) * 8
    t_layer = min(layer_times)
    per_token = shape.layers * t_layer + t_head
    return {"value": 1.0 / per_token, "unit": "tok/s", "cores": 1, "kind": kind,
            "sample": f"reference CPU worker arithmetic (cpp/src/cpu/llama.cpp via oracle/_ref), "
                      f"1 thread: one Qwen3-4B layer decode step at context {ctx} "
                      f"({1e3 * t_layer:.0f} ms, x36) + final norm/LM head over 1/8 of the "
                      f"vocabulary ({1e3 * t_head / 8:.0f} ms, x8); extrapolated per-token time "
                      f"{per_token:.2f} s at batch 1; host nproc {os.cpu_count()}",
            "ms_per_token": 1e3 * per_token}


# ------------------------------------------------------------------ main

def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=int(os.environ.get("WORLD_SIZE", "1")))
    ap.add_argument("--steps", type=int, default=400)
    ap.add_argument("--warmup", type=int, default=120)
    ap.add_argument("--concurrency", type=int, default=64)
    ap.add_argument("--chunk", type=int, default=512)
    ap.add_argument("--rate", type=float, default=1.0, help="Poisson arrivals per step")
    ap.add_argument("--seed", type=int, default=0)
    ap.add_argument("--layers", type=int, default=0, help="truncate the model (debug only)")
    ap.add_argument("--decode-steps", type=int, default=32)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--kv-gb", type=float, default=48.0, help="paged KV pool size (GiB)")
    ap.add_argument("--kv-block", type=int, default=0, help="tokens per KV block (0 = default)")
    ap.add_argument("--decode-only", action="store_true", help="only the pure-decode measurement")
    ap.add_argument("--skip-extras", action="store_true")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="end with three plain 1 GiB device copies (the reference kernel for "
                         "scaling rocprofv3 FETCH_SIZE / WRITE_SIZE counters to bytes)")
    ap.add_argument("--region-markers", action="store_true",
                    help="a 1 MiB device copy right before and right after the timed region, so "
                         "that counter runs can select the region's dispatches")
    ap.add_argument("--timed-only", action="store_true",
                    help="stop after the timed region (counter runs)")
    ap.add_argument("--traffic-summary", nargs=2, metavar=("FETCH_CSV", "WRITE_CSV"),
                    help="summarize two rocprofv3 counter runs (FETCH_SIZE, WRITE_SIZE) of "
                         "--timed-only --region-markers --copy-calibration into profiles/traffic.json")
    args = ap.parse_args()
    if args.traffic_summary:
        traffic_summary(*args.traffic_summary)
        return
    if args.gpus != 1:
        sys.exit("bench.py measures one GPU: the stage worker runs the whole model (or one "
                 "pipeline stage's share) on a single MI355X; multi-GPU runs are not part of "
                 "this build")

    shape = synthetic.QWEN3_4B
    if args.layers:
        shape = synthetic.with_layers(shape, args.layers)
    rows_max = args.chunk + args.concurrency
    cfg = model.stage_config(shape, execution="f16", kv_cache_bytes=int(args.kv_gb * (1 << 30)),
                             kv_block_tokens=args.kv_block,
                             max_sequences=4 * args.concurrency,
                             max_pass_rows=((rows_max + 127) // 128) * 128, max_seq=4096)
    t0 = time.perf_counter()
    stage = capi.Stage(cfg)
    model.synthesize(stage, shape, seed=args.seed, norm_sigma=0.0)
    log(f"stage ready in {time.perf_counter() - t0:.1f}s; weights "
        f"{stage.weight_memory().device_bytes / 1e9:.2f} GB")

    rng = np.random.default_rng(args.seed)
    if args.decode_only:
        d = decode_bench(stage, shape, rng, args.concurrency, args.decode_steps)
        print(json.dumps({"decode": d}), flush=True)
        stage.close()
        return
    engine = Engine(stage, args.concurrency, args.chunk,
                    request_stream(np.random.default_rng(args.seed + 1), shape.vocab, args.rate))
    t0 = time.perf_counter()
    engine.prestart(np.random.default_rng(args.seed + 2), shape.vocab, cfg.max_pass_rows)
    log(f"{len(engine.active)} requests pre-started at staggered progress in "
        f"{time.perf_counter() - t0:.1f}s")
    for i in range(args.warmup):
        engine.step()
    engine.drain()

    # The timed region starts with no pass in flight and ends when its K-th pass completes.
    if args.region_markers:
        region_marker()
    engine.work = StepWork(shape)
    step_ms, tokens, rows_total, decode_rows, active_total = [], 0, 0, 0, 0
    t_start = time.perf_counter()
    for i in range(args.steps):
        t0 = time.perf_counter()
        s, r, d, a = engine.step(last=i == args.steps - 1)
        step_ms.append(1e3 * (time.perf_counter() - t0))
        tokens += s
        rows_total += r
        decode_rows += d
        active_total += a
    elapsed = time.perf_counter() - t_start
    step_roofline = engine.work.summary(elapsed)
    engine.work = None
    if args.region_markers:
        region_marker()
    mean_active = active_total / args.steps
    log(f"timed {args.steps} steps in {elapsed:.3f}s: {tokens} tokens, {rows_total} rows "
        f"({decode_rows} decode rows), {mean_active:.1f} requests per pass on average")
    log("workload step roofline:", json.dumps(step_roofline))
    if args.timed_only:
        engine.release_all()
        stage.close()
        print(json.dumps({"metric": METRIC, "value": tokens / elapsed, "unit": "tok/s",
                          "steps": args.steps, "warmup": args.warmup,
                          "ms_per_step": 1e3 * elapsed / args.steps, "step_roofline": step_roofline}),
              flush=True)
        if args.copy_calibration:
            copy_calibration()
        return
    # The dominant kernel: most HIP-event time over steps that continue the same steady
    # workload (events perturb the host's launch rate, so the throughput region above runs
    # without them).
    stage.profile("*")
    for i in range(min(args.steps, 20)):
        engine.step(last=i == min(args.steps, 20) - 1)
    records = stage.profile_records()
    fam = {r: stage.profile_read(r) for r in records if "/" not in r and not r.startswith("k:")}
    kern = {r[2:]: stage.profile_read(r) for r in records if r.startswith("k:")}
    dominant = max(kern, key=lambda k: kern[k][0])
    owners = sorted({r.split("/", 1)[0] for r in records if r.endswith("/" + dominant)})
    log("kernel time (ms) by family:",
        {f: round(v[0], 2) for f, v in sorted(fam.items(), key=lambda kv: -kv[1][0])})
    log("kernel time (ms) by kernel:",
        {k: round(v[0], 2) for k, v in sorted(kern.items(), key=lambda kv: -kv[1][0])[:8]})
    log(f"active {len(engine.active)} waiting {len(engine.waiting)}; dominant kernel {dominant} "
        f"(launched by {owners})")
    # Per-kernel roofline: HIP events around the dominant kernel's launches only, over a
    # further region of the same length.
    stage.profile("k:" + dominant)
    t_prof = time.perf_counter()
    for i in range(args.steps):
        engine.step(last=i == args.steps - 1)
    prof_elapsed = time.perf_counter() - t_prof
    dom_ms, dom_n, dom_bytes, dom_flops = stage.profile_read("k:" + dominant)
    stage.profile(None)
    engine.release_all()

    avg_launch_s = dom_ms / max(dom_n, 1) * 1e-3
    # Bound: whichever peak the kernel's algorithmic work needs longer on.
    t_hbm = dom_bytes / (HBM_PEAK_GBS * 1e9)
    t_mfma = dom_flops / (MFMA_F16_PEAK_TFLOPS * 1e12)
    if t_mfma > t_hbm:
        achieved = dom_flops / max(dom_n, 1) / avg_launch_s / 1e12 if dom_n else 0.0
        roof = {"bound": "mfma", "achieved": achieved, "peak": MFMA_F16_PEAK_TFLOPS, "unit": "TFLOP/s",
                "frac": achieved / MFMA_F16_PEAK_TFLOPS}
    else:
        achieved = dom_bytes / max(dom_n, 1) / avg_launch_s / 1e9 if dom_n else 0.0
        roof = {"bound": "hbm", "achieved": achieved, "peak": HBM_PEAK_GBS, "unit": "GB/s",
                "frac": achieved / HBM_PEAK_GBS}
    roof.update({"traffic": measured_traffic(dominant), "kernel": dominant, "families": owners, "launches": dom_n,
                 "region": f"{args.steps} further workload steps with HIP events on this kernel "
                           f"({1e3 * prof_elapsed / args.steps:.2f} ms/step)",
                 "avg_launch_us": avg_launch_s * 1e6,
                 "algorithmic_bytes_per_launch": dom_bytes / max(dom_n, 1),
                 "algorithmic_flops_per_launch": dom_flops / max(dom_n, 1)})
    # The line stands for the stated concurrency only if the timed passes held it.
    at_target = mean_active >= 0.95 * args.concurrency
    result = {
        "metric": METRIC,
        "value": tokens / elapsed if at_target else None,
        "unit": "tok/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": 1e3 * elapsed / args.steps,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f16",
        "data": "synthetic (seeded random-init weights, random prompt token IDs)",
        "config": {"workload": f"{shape.name} continuous batching: {args.concurrency} concurrent, "
                               f"Poisson arrivals {args.rate}/step, prompts lognormal(median 256, "
                               f"sigma 1) in [16,2048], outputs U[64,256], chunked prefill "
                               f"{args.chunk} mixed with decode rows",
                   "concurrency": args.concurrency, "chunk": args.chunk,
                   "mean_active_requests": mean_active,
                   "rows_per_step": rows_total / args.steps,
                   "decode_rows_per_step": decode_rows / args.steps},
        "latency_ms": {"p50": float(np.percentile(step_ms, 50)),
                       "p99": float(np.percentile(step_ms, 99))},
        "roofline": roof,
        "step_roofline": step_roofline,
    }
    if not at_target:
        result["error"] = (f"the timed passes held {mean_active:.1f} requests on average, below the "
                           f"stated concurrency {args.concurrency}: no value is reported")
    if not args.skip_extras:
        result["decode"] = decode_bench(stage, shape, rng, args.concurrency, args.decode_steps)
        peak = capi.measure_read_bandwidth(4 << 30)
        result["decode"]["hbm_read_ceiling_gb_s"] = peak
        result["decode"]["hbm_frac_of_read_ceiling"] = result["decode"]["hbm_gb_s"] / peak
        log("decode:", json.dumps({k: v for k, v in result["decode"].items() if k != "kernels"}))
        result["prefill"] = [prefill_bench(stage, shape, rng, past, 3) for past in (0, 1536)]
        ceiling = {str(k): capi.measure_mfma_rate(k) for k in (16, 32)}
        best = max(ceiling.values())
        for entry in result["prefill"]:
            entry["mfma_ceiling_tflops"] = best
            entry["mfma_frac_of_ceiling"] = entry["tflops"] / best
        result["mfma_ceiling_tflops"] = {"v_mfma_f32_16x16x32_f16": ceiling["16"],
                                         "v_mfma_f32_32x32x16_f16": ceiling["32"],
                                         "spec_dense_f16": MFMA_F16_PEAK_TFLOPS}
        log("prefill:", json.dumps(result["prefill"]))
        log("MFMA ceiling:", json.dumps(result["mfma_ceiling_tflops"]))
    stage.close()
    if not args.skip_extras:
        result["stage_share"] = stage_share_bench(np.random.default_rng(args.seed + 3), args.decode_steps)
        log("stage share:", json.dumps(result["stage_share"]))
    if not args.no_cpu_baseline:
        mean_ctx = result.get("decode", {}).get("mean_context", 483.0)
        result["cpu_baseline"] = cpu_baseline(synthetic.QWEN3_4B, mean_ctx)
    print(json.dumps(result), flush=True)
    if args.copy_calibration:
        copy_calibration()


def region_marker():
    """A 1 MiB device-to-device copy (the runtime's blit kernel) that counter runs find
    before and after the timed region."""
    hip = C.CDLL("libamdhip64.so")
    n = 1 << 20
    src, dst = C.c_void_p(), C.c_void_p()
    for ptr in (src, dst):
        if hip.hipMalloc(C.byref(ptr), C.c_size_t(n)) != 0:
            raise RuntimeError("hipMalloc failed")
    try:
        if hip.hipMemcpy(dst, src, C.c_size_t(n), 3) != 0 or hip.hipDeviceSynchronize() != 0:
            raise RuntimeError("hipMemcpy failed")
    finally:
        hip.hipFree(src)
        hip.hipFree(dst)


def kernel_key(profiler_name):
    """A kernel as the stage's profiling records name it ("gemm_decode_kernel<4, 8, 1, 4, 4, 0>")
    from its name in a rocprofv3 CSV ("void hllm_rocm::(anonymous namespace)::gemm_decode_kernel<4,
    8, 1, 4, 4, false>(hllm_rocm::GemmArgs, int, int)")."""
    name = profiler_name.replace("void ", "", 1).replace("hllm_rocm::(anonymous namespace)::", "")
    name = name.replace("hllm_rocm::", "")
    depth, cut = 0, len(name)
    for j, ch in enumerate(name):
        depth += ch == "<"
        depth -= ch == ">"
        if ch == "(" and depth == 0:
            cut = j
            break
    return name[:cut].replace("true", "1").replace("false", "0").strip()


def traffic_summary(fetch_csv, write_csv):
    """Per-kernel HBM bytes per launch over the timed region only: the dispatches between the
    two 1 MiB marker copies of a --timed-only --region-markers --copy-calibration run, FETCH_SIZE
    and WRITE_SIZE (KiB per dispatch) each scaled by what the counter reads for the 1 GiB
    copies after the region. Kernels launched with several grid sizes (the decode GEMM runs
    the projections and the LM head) are also kept per grid size."""
    import csv

    def load(path, counter):
        rows = [r for r in csv.DictReader(open(path)) if r["Counter_Name"].startswith(counter)]
        per = collections.OrderedDict()
        for r in rows:
            d = per.setdefault(int(r["Dispatch_Id"]), {"name": r["Kernel_Name"], "grid": int(r["Grid_Size"]),
                                                       "value": 0.0})
            d["value"] += float(r["Counter_Value"])
        return per

    out = {}
    for counter, path in (("FETCH_SIZE", fetch_csv), ("WRITE_SIZE", write_csv)):
        per = load(path, counter)
        ids = sorted(per)
        # The runtime's copy kernel also runs the stage's small copies: the 1 GiB calibration
        # copies are the largest grids, the two 1 MiB markers the next largest.
        copies = [i for i in ids if "copyBuffer" in per[i]["name"]]
        grids = sorted({per[i]["grid"] for i in copies}, reverse=True)
        big = [i for i in copies if per[i]["grid"] == grids[0]] if grids else []
        markers = [i for i in copies if len(grids) > 1 and per[i]["grid"] == grids[1]]
        if len(markers) != 2 or len(big) < 1:
            raise SystemExit(f"{path}: expected two marker copies and the 1 GiB calibration copies")
        lo, hi = markers[0], markers[-1]
        scale_key = "fetch" if counter == "FETCH_SIZE" else "write"
        cal = sum(per[i]["value"] for i in big) / len(big)
        scale = (1 << 20) / cal  # KiB per GiB copied -> bytes factor: a GiB copy reads and writes 1 GiB
        out[scale_key] = {"kib_per_gib_copy": cal, "scale": scale, "kernels": collections.defaultdict(list)}
        for i in ids:
            if lo < i < hi and "copyBuffer" not in per[i]["name"]:
                out[scale_key]["kernels"][kernel_key(per[i]["name"])].append((per[i]["grid"], per[i]["value"]))
    kernels = {}
    for name, f in out["fetch"]["kernels"].items():
        w = out["write"]["kernels"].get(name, [])
        if len(w) != len(f):
            continue
        entry = {"dispatches": len(f), "fetch_kib_per_dispatch": sum(v for _, v in f) / len(f),
                 "write_kib_per_dispatch": sum(v for _, v in w) / len(w)}
        entry["bytes_per_launch"] = 1024 * (entry["fetch_kib_per_dispatch"] * out["fetch"]["scale"] +
                                            entry["write_kib_per_dispatch"] * out["write"]["scale"])
        grids = sorted({g for g, _ in f})
        if len(grids) > 1:
            entry["by_grid"] = {}
            for g in grids:
                fv = [v for gg, v in f if gg == g]
                wv = [v for gg, v in w if gg == g]
                entry["by_grid"][str(g)] = {"dispatches": len(fv), "bytes_per_launch": 1024 * (
                    sum(fv) / len(fv) * out["fetch"]["scale"] + sum(wv) / len(wv) * out["write"]["scale"])}
        kernels[name] = entry
    doc = {"region": "the timed region's dispatches only (between the marker copies)",
           "copy_calibration": {"fetch_kib_per_gib_copy": out["fetch"]["kib_per_gib_copy"],
                                "write_kib_per_gib_copy": out["write"]["kib_per_gib_copy"],
                                "fetch_scale": out["fetch"]["scale"], "write_scale": out["write"]["scale"]},
           "kernels": kernels}
    path = os.path.join(ROOT, "profiles", "traffic.json")
    with open(path, "w") as f:
        json.dump(doc, f, indent=1)
    print(json.dumps(doc, indent=1))


def measured_traffic(kernel):
    """HBM bytes per launch of `kernel` from the committed rocprofv3 counter runs of this
    workload (FETCH_SIZE and WRITE_SIZE per dispatch, each scaled by what the counter reads
    for a 1 GiB device copy), or None when the kernel has not been measured."""
    path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "profiles", "traffic.json")
    try:
        with open(path) as f:
            entry = json.load(f).get("kernels", {}).get(kernel)
    except (OSError, ValueError):
        return None
    return entry["bytes_per_launch"] if entry else None


def copy_calibration():
    """Three device-to-device copies of 1 GiB through the HIP runtime (its blit copy kernel):
    a kernel whose HBM traffic is known (1 GiB read, 1 GiB written), profiled beside the
    stage's kernels."""
    hip = C.CDLL("libamdhip64.so")
    n = 1 << 30
    src, dst = C.c_void_p(), C.c_void_p()
    for ptr in (src, dst):
        if hip.hipMalloc(C.byref(ptr), C.c_size_t(n)) != 0:
            raise RuntimeError("hipMalloc failed")
    try:
        if hip.hipMemset(src, 1, C.c_size_t(n)) != 0:
            raise RuntimeError("hipMemset failed")
        for _ in range(3):
            if hip.hipMemcpy(dst, src, C.c_size_t(n), 3) != 0:  # hipMemcpyDeviceToDevice
                raise RuntimeError("hipMemcpy failed")
        if hip.hipDeviceSynchronize() != 0:
            raise RuntimeError("hipDeviceSynchronize failed")
    finally:
        hip.hipFree(src)
        hip.hipFree(dst)
    log("copy calibration: 3 x 1 GiB device-to-device copies")


if __name__ == "__main__":
    main()
