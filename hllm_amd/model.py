"""Stage construction helpers over the C ABI: configuration from a model shape, and
weights from host arrays (checkpoint tensors) or from the on-device seeded generator."""
from __future__ import annotations

import numpy as np

from . import capi, synthetic


def stage_config(shape: synthetic.ModelShape, layer_start: int = 0, layer_end: int | None = None,
                 first: bool = True, final: bool = True, execution: str = "f16",
                 weights: str | None = None, kv_cache_bytes: int = 0, kv_block_tokens: int = 0,
                 max_sequences: int = 0, max_pass_rows: int = 0, device: int = 0,
                 max_seq: int | None = None) -> capi.StageConfig:
    layer_end = shape.layers if layer_end is None else layer_end
    execution_dtype = capi.F16 if execution == "f16" else capi.F32
    if weights is None:  # the plan's default: weights resident at the execution dtype, except
        # that F32 execution keeps an F16 checkpoint resident as F16 (mixed contract).
        weights = "f32" if (execution == "f32" and shape.dtype == "f32") else "f16"
    weight_dtype = capi.F16 if weights == "f16" else capi.F32
    return capi.StageConfig(
        capi.ABI_VERSION, shape.hidden, shape.intermediate, shape.heads, shape.kv_heads,
        shape.head_dim, max_seq or shape.max_seq, shape.vocab, shape.eps, shape.theta,
        int(shape.qk_norm), layer_start, layer_end, int(first), int(final), int(shape.tied),
        execution_dtype, weight_dtype, device, kv_cache_bytes, kv_block_tokens, max_sequences,
        max_pass_rows)


def synthesize(stage: capi.Stage, shape: synthetic.ModelShape, seed: int = 0,
               norm_sigma: float = 0.0) -> None:
    """Fill every owned tensor with the seeded synthetic checkpoint, on the device."""
    c = stage.config
    source = capi.F16 if shape.dtype == "f16" else capi.F32
    for name in synthetic.stage_tensor_names(shape, c.layer_start, c.layer_end,
                                             bool(c.first_stage), bool(c.final_stage)):
        tid, _, mean, sigma = synthetic.tensor_spec(shape, name, norm_sigma)
        stage.synthesize_tensor(name, seed, tid, mean, sigma, source)
    stage.finalize()


def load(stage: capi.Stage, tensors: dict) -> None:
    """Upload checkpoint tensors (name -> numpy array: float32, or uint16 F16 bits)."""
    for name, array in tensors.items():
        stage.load_tensor(name, np.asarray(array))
    stage.finalize()
