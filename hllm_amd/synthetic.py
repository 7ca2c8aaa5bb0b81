"""Seeded synthetic models for the decoder stage worker's workloads.

Weights are defined element by element, so any tensor (or any slice of one) can be
regenerated independently on the host or on the device with identical bits:

* tensor IDs: token embedding 1, final norm 2, LM head 3; layer ``l`` tensor ``k`` is
  ``(l + 1) * 16 + k`` with ``k`` the index in ``LAYER_TENSORS``;
* element ``i`` of tensor ``t`` with seed ``s``: three SplitMix64 outputs at counters
  ``(t << 40) + 3 i + j`` (j = 0, 1, 2; output(c) = mix(s + 0x9e3779b97f4a7c15 * (c + 1)))
  give twelve 16-bit uniforms; their Irwin-Hall sum ``n = (sum + 6 - 6 * 65536) / 65536``
  (exact in F32) approximates N(0, 1); the value is ``mean + n * sigma`` in F32 with one
  rounding per operation, then F16 round-to-nearest-even for F16 checkpoints;
* projections and embeddings: mean 0, sigma 0.02; RMSNorm weights: mean 1 with sigma
  ``norm_sigma`` (0 = the Hugging Face initialisation of ones, used by the benchmarks;
  tests use a jitter so that a misapplied norm weight cannot go unnoticed).
"""
from __future__ import annotations

from dataclasses import dataclass, replace

LAYER_TENSORS = ("input_layernorm.weight", "self_attn.q_proj.weight", "self_attn.k_proj.weight",
                 "self_attn.v_proj.weight", "self_attn.o_proj.weight",
                 "post_attention_layernorm.weight", "mlp.gate_proj.weight", "mlp.up_proj.weight",
                 "mlp.down_proj.weight", "self_attn.q_norm.weight", "self_attn.k_norm.weight")
EMBEDDING, FINAL_NORM, LM_HEAD = 1, 2, 3
WEIGHT_SIGMA = 0.02


@dataclass(frozen=True)
class ModelShape:
    name: str
    layers: int
    hidden: int
    intermediate: int
    heads: int
    kv_heads: int
    head_dim: int
    vocab: int
    eps: float = 1e-6
    theta: float = 1e6
    qk_norm: bool = True
    tied: bool = True
    dtype: str = "f16"          # checkpoint storage dtype: "f16" or "f32"
    max_seq: int = 32768

    @property
    def architecture(self) -> str:
        return "qwen3.v1" if self.qk_norm else "llama.v1"

    def layer_shapes(self) -> dict:
        H, I, D = self.hidden, self.intermediate, self.head_dim
        q, kv = self.heads * D, self.kv_heads * D
        shapes = {
            "input_layernorm.weight": (H,), "self_attn.q_proj.weight": (q, H),
            "self_attn.k_proj.weight": (kv, H), "self_attn.v_proj.weight": (kv, H),
            "self_attn.o_proj.weight": (H, q), "post_attention_layernorm.weight": (H,),
            "mlp.gate_proj.weight": (I, H), "mlp.up_proj.weight": (I, H),
            "mlp.down_proj.weight": (H, I)}
        if self.qk_norm:
            shapes["self_attn.q_norm.weight"] = (D,)
            shapes["self_attn.k_norm.weight"] = (D,)
        return shapes

    def layer_weight_bytes(self, element_bytes: int = 2) -> int:
        total = 0
        for shape in self.layer_shapes().values():
            n = 1
            for d in shape:
                n *= d
            total += n
        return total * element_bytes

    def kv_bytes_per_token(self, layers: int | None = None, element_bytes: int = 2) -> int:
        return (self.layers if layers is None else layers) * self.kv_heads * self.head_dim * 2 \
            * element_bytes


def tensor_spec(shape: ModelShape, name: str, norm_sigma: float = 0.0):
    """(tensor_id, shape, mean, sigma) for a checkpoint tensor name."""
    if name == "model.embed_tokens.weight":
        return EMBEDDING, (shape.vocab, shape.hidden), 0.0, WEIGHT_SIGMA
    if name == "model.norm.weight":
        return FINAL_NORM, (shape.hidden,), 1.0, norm_sigma
    if name == "lm_head.weight":
        return LM_HEAD, (shape.vocab, shape.hidden), 0.0, WEIGHT_SIGMA
    prefix, _, rest = name.partition(".layers.")
    layer_text, _, suffix = rest.partition(".")
    layer = int(layer_text)
    kind = LAYER_TENSORS.index(suffix)
    dims = shape.layer_shapes()[suffix]
    is_norm = suffix.endswith("norm.weight")
    return (layer + 1) * 16 + kind, dims, (1.0 if is_norm else 0.0), \
        (norm_sigma if is_norm else WEIGHT_SIGMA)


def stage_tensor_names(shape: ModelShape, layer_start: int, layer_end: int, first: bool,
                       final: bool) -> list:
    """Tensors a stage owns (hLLM cpp/src/model/dense_loader.cpp:107-140)."""
    names = []
    if first or (final and shape.tied):
        names.append("model.embed_tokens.weight")
    if final:
        names.append("model.norm.weight")
        if not shape.tied:
            names.append("lm_head.weight")
    for layer in range(layer_start, layer_end):
        names += [f"model.layers.{layer}.{n}" for n in shape.layer_shapes()]
    return names


# The workloads' model shapes. c4's RoPE theta (1000042) follows the public Falcon3
# configuration; the workload description gives none.
TINY_LLAMA = ModelShape("tiny-llama", 2, 64, 128, 4, 2, 16, 256, eps=1e-6, theta=1e4,
                        qk_norm=False, tied=False, dtype="f32", max_seq=512)
QWEN3_0_6B = ModelShape("qwen3-0.6b", 28, 1024, 3072, 16, 8, 128, 151936)
QWEN3_4B = ModelShape("qwen3-4b", 36, 2560, 9728, 32, 8, 128, 151936)
FALCON3_3B = ModelShape("falcon3-3b", 22, 3072, 9216, 12, 4, 256, 131072, theta=1000042.0,
                        qk_norm=False, tied=False)
SHAPES = {s.name: s for s in (TINY_LLAMA, QWEN3_0_6B, QWEN3_4B, FALCON3_3B)}


def with_layers(shape: ModelShape, layers: int) -> ModelShape:
    """The same shape truncated to its first `layers` layers (parity slices)."""
    return replace(shape, name=f"{shape.name}-{layers}l", layers=layers)
