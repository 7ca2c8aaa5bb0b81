"""Test-side model construction: oracle weights for synthetic shapes and the reference's
tiny Transformers fixture."""
from __future__ import annotations

import json
import os

import numpy as np

import oracle
from hllm_amd import synthetic

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def oracle_config(shape: synthetic.ModelShape) -> oracle.Config:
    return oracle.Config(shape.hidden, shape.intermediate, shape.heads, shape.kv_heads,
                         shape.head_dim, shape.max_seq, shape.eps, shape.theta,
                         int(shape.qk_norm))


def synthetic_tensor(shape, name, seed=0, norm_sigma=0.0):
    """(F32 values as the CPU worker sees them, checkpoint payload array)."""
    tid, dims, mean, sigma = synthetic.tensor_spec(shape, name, norm_sigma)
    n = int(np.prod(dims))
    if shape.dtype == "f16":
        bits = oracle.synth_f16(seed, tid, n, mean, sigma).reshape(dims)
        return oracle.f16_decode(bits), bits
    values = oracle.synth_f32(seed, tid, n, mean, sigma).reshape(dims)
    return values, values


def synthetic_stage(shape, layer_start=0, layer_end=None, first=True, final=True, seed=0,
                    norm_sigma=0.0) -> oracle.StageWeights:
    layer_end = shape.layers if layer_end is None else layer_end
    w = oracle.StageWeights(oracle_config(shape), shape.vocab, layer_start, layer_end, first,
                            final, shape.tied)
    for name in synthetic.stage_tensor_names(shape, layer_start, layer_end, first, final):
        w.tensors[name] = synthetic_tensor(shape, name, seed, norm_sigma)[0]
    return w


def tiny_reference():
    with open(os.path.join(GOLDEN, "qwen3_tiny_reference.json")) as f:
        return json.load(f)


def tiny_reference_shape():
    c = tiny_reference()["config"]
    return synthetic.ModelShape("qwen3-tiny-reference", c["num_hidden_layers"], c["hidden_size"],
                                c["intermediate_size"], c["num_attention_heads"],
                                c["num_key_value_heads"], c["head_dim"], c["vocab_size"],
                                eps=c["rms_norm_eps"], theta=c["rope_theta"], qk_norm=True,
                                tied=True, dtype="f32", max_seq=c["max_position_embeddings"])


def tiny_reference_stage(layer_start=0, layer_end=2, first=True, final=True):
    fx = tiny_reference()
    shape = tiny_reference_shape()
    w = oracle.StageWeights(oracle_config(shape), shape.vocab, layer_start, layer_end, first,
                            final, True)
    for name in synthetic.stage_tensor_names(shape, layer_start, layer_end, first, final):
        t = fx["weights"][name]
        w.tensors[name] = np.asarray(t["values"], np.float32).reshape(t["shape"])
    return w


def tiny_rows(tensor, start, count):
    """Rows [start, start+count) of a [1, seq, width] fixture tensor."""
    a = np.asarray(tensor["values"], np.float32).reshape(tensor["shape"])
    return a[0, start:start + count]


def f16_normal(rng, shape):
    """F16 bits of N(0, 1) draws (boundary activations fed to a non-first stage)."""
    return oracle.f16_encode(rng.standard_normal(shape).astype(np.float32))
