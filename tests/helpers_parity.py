"""Shared pieces of the workload-shaped parity tests: GPU prefill of many sequences in ragged
passes, the cache state read back into the oracle, and the per-row comparison bounds.

The oracle cannot prefill thousands of tokens through Qwen3-4B-sized layers in test time,
so a decode pass is checked against the oracle from the same cache state: the GPU prefills,
its F16 KV cache is read back (exact in F32) into the oracle's sequences, and both then run
the same decode rows. Prefill itself is checked against the oracle by the chunk tests."""
from __future__ import annotations

import numpy as np

import oracle
from hllm_amd import capi

MAX_ABS, MIN_COSINE = 2e-2, 0.9999  # F16 execution against the F32 oracle, per row


def say(*what):
    print("[gpu-case]", *what, flush=True)


def cosine(a, b):
    a, b = np.asarray(a, np.float64).ravel(), np.asarray(b, np.float64).ravel()
    return float(a @ b / (np.linalg.norm(a) * np.linalg.norm(b)))


def check_rows(got, expect, what):
    """Every row within max-abs 2e-2 and cosine 0.9999 of the oracle's."""
    got, expect = np.asarray(got), np.asarray(expect)
    assert got.shape == expect.shape, (what, got.shape, expect.shape)
    worst_abs, worst_cos = 0.0, 1.0
    for r in range(got.shape[0]):
        d = float(np.abs(got[r] - expect[r]).max())
        c = cosine(got[r], expect[r])
        worst_abs, worst_cos = max(worst_abs, d), min(worst_cos, c)
        assert d <= MAX_ABS and c >= MIN_COSINE, (what, r, d, c)
    say(what, f"max-abs {worst_abs:.2e} min-cosine {worst_cos:.6f}")
    return worst_abs


def prefill(stage, seqs, lengths, max_rows, token_ids=None, boundary=None):
    """Prefills every sequence to its length in ragged passes of at most `max_rows` rows,
    without sampling. token_ids / boundary: per-sequence inputs (lists of arrays)."""
    pieces = []
    for i, (s, n) in enumerate(zip(seqs, lengths)):
        for pos in range(0, n, max_rows):
            pieces.append((i, s, pos, min(max_rows, n - pos)))
    batch, rows = [], 0

    def flush():
        items = [capi.item(s, take, pos, sample=False) for _, s, pos, take in batch]
        if token_ids is not None:
            ids = np.concatenate([token_ids[i][pos:pos + take] for i, _, pos, take in batch])
            stage.execute(items, token_ids=ids)
        else:
            b = np.concatenate([boundary[i][pos:pos + take] for i, _, pos, take in batch])
            stage.execute(items, boundary=b)

    for piece in pieces:
        if rows + piece[3] > max_rows:
            flush()
            batch, rows = [], 0
        batch.append(piece)
        rows += piece[3]
    if batch:
        flush()


def oracle_sequences(ost, stage, seqs, capacity):
    """Oracle sequences holding the GPU's cache state of `seqs` (every owned layer)."""
    out = []
    layers = stage.config.layer_end - stage.config.layer_start
    for s in seqs:
        o = ost.allocate_sequence(capacity)
        for layer in range(layers):
            k, v = stage.read_kv(s, layer)
            o.load_cache(layer, k, v)
        out.append(o)
    return out


def oracle_decode(ost, oseqs, inputs, positions):
    """One decode row per sequence through the oracle's layers: (last-layer hidden [rows, H],
    logits [rows, V] when the stage is final). inputs: token IDs, or F16 rows [rows, H]."""
    hidden = []
    for i, (o, pos) in enumerate(zip(oseqs, positions)):
        o.prefill_only = True  # layers only; the head runs once for all rows below
        tr = []
        x = np.array([inputs[i]], np.uint64) if np.ndim(inputs[i]) == 0 else \
            np.ascontiguousarray(inputs[i], np.uint16).reshape(1, -1)
        ost.execute(x, pos, o, tr)
        o.prefill_only = False
        hidden.append(tr[-1][0])
    hidden = np.stack(hidden)
    return hidden, (ost.logits_rows(hidden) if ost.w.final else None)


def lognormal_contexts(rng, count, median=256.0, sigma=1.0, low=16, high=2048):
    return [int(np.clip(round(np.exp(np.log(median) + sigma * rng.standard_normal())), low, high))
            for _ in range(count)]


def greedy_agrees(gpu_tokens, oracle_logits, gpu_logits, what):
    """Greedy tokens equal the oracle's first maximum, except at a near tie: where they
    differ, the GPU's token is within the F16 logit bound of the oracle's best, and the GPU's
    logits of both tokens are within 2e-2 of the oracle's."""
    departures = []
    for r, tok in enumerate(gpu_tokens):
        best = int(np.argmax(oracle_logits[r]))
        if int(tok) == best:
            continue
        gap = float(oracle_logits[r][best] - oracle_logits[r][int(tok)])
        err = max(abs(float(gpu_logits[r][best] - oracle_logits[r][best])),
                  abs(float(gpu_logits[r][int(tok)] - oracle_logits[r][int(tok)])))
        assert gap <= 2 * MAX_ABS and err <= MAX_ABS, (what, r, gap, err)
        departures.append((r, gap))
    say(what, f"greedy tokens: {len(gpu_tokens) - len(departures)}/{len(gpu_tokens)} equal the oracle's",
        f"near-tie departures (row, oracle margin): {departures}" if departures else "")
    return departures
