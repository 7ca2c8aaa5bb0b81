"""CPU oracle for the decoder stage worker.

TEST INFRASTRUCTURE ONLY: tests/, ``__graft_entry__.smoke()`` and bench.py's CPU-baseline
leg may import this package, and only as the checker. The product package
(``hllm_amd``) never imports it.

Two libraries back it:

* ``liboracle.so`` — the plain-C restatement in ``hllm_oracle.c`` (each function cites the
  reference file:line it follows);
* ``_ref/libhllm_ref.so`` — the reference CPU worker's own arithmetic sources compiled in
  place (``make -C oracle ref``), used to pin the restatement bit for bit and as the
  reported CPU baseline. Present wherever it was built (it travels with the tree).

``OracleStage`` mirrors ``DenseStage::run`` (hLLM ``cpp/src/cpu/stage.cpp:118-191``):
embedding or boundary decode, the owned layers, then final norm + LM head + sampling on
the last row, or the F16 boundary encode.
"""
from __future__ import annotations

import ctypes as C
import os
import subprocess
from dataclasses import dataclass, field

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
_LIB = None
_REF = None

OK, INVALID_REQUEST, INCOMPATIBLE_WORKER, RESOURCE_EXHAUSTED, INTERNAL = 0, 1, 2, 3, 6

_f32p = np.ctypeslib.ndpointer(np.float32, flags="C_CONTIGUOUS")
_u16p = np.ctypeslib.ndpointer(np.uint16, flags="C_CONTIGUOUS")
_u32p = np.ctypeslib.ndpointer(np.uint32, flags="C_CONTIGUOUS")
_i32p = np.ctypeslib.ndpointer(np.int32, flags="C_CONTIGUOUS")
_u64p = np.ctypeslib.ndpointer(np.uint64, flags="C_CONTIGUOUS")
_i64p = np.ctypeslib.ndpointer(np.int64, flags="C_CONTIGUOUS")
_f64p = np.ctypeslib.ndpointer(np.float64, flags="C_CONTIGUOUS")
_sz = C.c_size_t


class OracleError(RuntimeError):
    def __init__(self, status: int, what: str):
        super().__init__(f"{what}: status {status}")
        self.status = status


class Config(C.Structure):
    _fields_ = [("hidden_size", _sz), ("intermediate_size", _sz), ("attention_heads", _sz),
                ("key_value_heads", _sz), ("head_dimension", _sz),
                ("maximum_sequence_length", _sz), ("rms_norm_epsilon", C.c_float),
                ("rope_theta", C.c_float), ("query_key_norm", C.c_int)]


class _Layer(C.Structure):
    _fields_ = [(n, C.c_void_p) for n in (
        "input_norm", "query", "key", "value", "attention_output", "post_attention_norm",
        "gate", "up", "down", "query_norm", "key_norm")]


class _Kv(C.Structure):
    _fields_ = [("capacity", _sz), ("heads", _sz), ("head_dimension", _sz), ("length", _sz),
                ("keys", C.POINTER(C.c_float)), ("values", C.POINTER(C.c_float))]


def build(reference: bool | None = None) -> None:
    """Compile liboracle.so (and oracle/_ref when the reference sources are present)."""
    targets = ["all"]
    if reference or (reference is None and os.path.isdir("/root/reference/cpp")):
        targets.append("ref")
    subprocess.run(["make", "-s", "-C", HERE, *targets], check=True)


def lib() -> C.CDLL:
    global _LIB
    if _LIB is None:
        path = os.path.join(HERE, "liboracle.so")
        if not os.path.exists(path):
            build(reference=False)
        L = C.CDLL(path)
        L.orc_f32_from_f16.restype = C.c_float
        L.orc_f32_from_f16.argtypes = [C.c_uint16]
        L.orc_f16_from_f32.restype = C.c_uint16
        L.orc_f16_from_f32.argtypes = [C.c_float]
        L.orc_f32_from_bf16.restype = C.c_float
        L.orc_f32_from_bf16.argtypes = [C.c_uint16]
        L.orc_bf16_from_f32.restype = C.c_uint16
        L.orc_bf16_from_f32.argtypes = [C.c_float]
        L.orc_f16_encode.argtypes = [_f32p, _sz, _u16p]
        L.orc_f16_decode.argtypes = [_u16p, _sz, _f32p]
        L.orc_set_threads.argtypes = [C.c_int]
        L.orc_rms_norm.argtypes = [_f32p, _sz, _sz, _f32p, C.c_float, _f32p]
        L.orc_linear.argtypes = [_f32p, _sz, _sz, _f32p, _sz, _f32p]
        L.orc_normalize_heads.argtypes = [_f32p, _sz, _f32p, _sz, C.c_float]
        L.orc_apply_rope.argtypes = [_f32p, _sz, _sz, _sz, _sz, C.c_float]
        L.orc_kv_init.argtypes = [C.POINTER(_Kv), _sz, _sz, _sz]
        L.orc_kv_free.argtypes = [C.POINTER(_Kv)]
        L.orc_kv_append.argtypes = [C.POINTER(_Kv), _sz, _f32p, _f32p, _sz]
        L.orc_attention.argtypes = [_f32p, _sz, C.POINTER(Config), _sz, C.POINTER(_Kv), _f32p]
        L.orc_transformer_layer.argtypes = [_f32p, _sz, C.POINTER(_Layer), C.POINTER(Config),
                                            _sz, C.POINTER(_Kv), _f32p]
        L.orc_final_logits.argtypes = [_f32p, _sz, _sz, _f32p, _f32p, _sz, C.c_float, _f32p]
        L.orc_greedy_last.argtypes = [_f32p, _sz, _sz, C.POINTER(C.c_uint64)]
        L.orc_sample_logits.argtypes = [_f32p, _sz, C.c_double, C.c_double, C.c_uint64,
                                        C.c_uint64, C.c_uint64, C.POINTER(C.c_uint64)]
        L.orc_sample_token.argtypes = [_f32p, _sz, C.c_double, C.c_double, C.c_uint64,
                                       C.c_uint64, C.c_uint64, C.c_int, C.c_uint32,
                                       C.POINTER(C.c_uint64), C.POINTER(C.c_double), _u64p, _f64p]
        L.orc_pack.argtypes = [_sz, _u32p, _u64p, _u32p, _i32p, _sz, _sz, _u32p, _u32p, _u64p,
                               _i64p]
        L.orc_synth_f32.argtypes = [C.c_uint64, C.c_uint64, C.c_uint64, _sz, C.c_float,
                                    C.c_float, _f32p]
        L.orc_synth_f16.argtypes = [C.c_uint64, C.c_uint64, C.c_uint64, _sz, C.c_float,
                                    C.c_float, _u16p]
        L.orc_splitmix64.restype = C.c_uint64
        L.orc_splitmix64.argtypes = [C.c_uint64]
        _LIB = L
    return _LIB


def ref() -> C.CDLL | None:
    """The reference's own arithmetic (oracle/_ref), or None where it was not built."""
    global _REF
    if _REF is None:
        path = os.path.join(HERE, "_ref", "libhllm_ref.so")
        if not os.path.exists(path):
            if not os.path.isdir("/root/reference/cpp"):
                return None
            build(reference=True)
        R = C.CDLL(path)
        R.ref_f32_from_f16.restype = C.c_float
        R.ref_f32_from_f16.argtypes = [C.c_uint16]
        R.ref_f16_from_f32.restype = C.c_uint16
        R.ref_f16_from_f32.argtypes = [C.c_float]
        R.ref_f32_from_bf16.restype = C.c_float
        R.ref_f32_from_bf16.argtypes = [C.c_uint16]
        R.ref_bf16_from_f32.restype = C.c_uint16
        R.ref_bf16_from_f32.argtypes = [C.c_float]
        R.ref_layer_create.restype = C.c_void_p
        R.ref_layer_create.argtypes = [C.POINTER(Config)] + [C.c_void_p] * 11
        R.ref_layer_destroy.argtypes = [C.c_void_p]
        R.ref_cache_create.restype = C.c_void_p
        R.ref_cache_create.argtypes = [_sz, _sz, _sz]
        R.ref_cache_destroy.argtypes = [C.c_void_p]
        R.ref_cache_length.restype = _sz
        R.ref_cache_length.argtypes = [C.c_void_p]
        R.ref_cache_read.argtypes = [C.c_void_p, _f32p, _f32p]
        R.ref_cache_append.argtypes = [C.c_void_p, _sz, _f32p, _f32p, _sz, _sz]
        R.ref_transformer_layer.argtypes = [C.POINTER(Config), C.c_void_p, _f32p, _sz, _sz,
                                            C.c_void_p, _f32p]
        R.ref_rms_norm.argtypes = [_f32p, _sz, _sz, _f32p, C.c_float, _f32p]
        R.ref_apply_rope.argtypes = [_f32p, _sz, _sz, _sz, _sz, C.c_float]
        R.ref_linear.argtypes = [_f32p, _sz, _sz, _f32p, _sz, _f32p]
        R.ref_final_logits.argtypes = [_f32p, _sz, _sz, _f32p, _f32p, _sz, C.c_float, _f32p]
        R.ref_greedy_last.argtypes = [_f32p, _sz, _sz, C.POINTER(C.c_uint64)]
        R.ref_sample_token.argtypes = [_f32p, _sz, C.c_double, C.c_double, C.c_uint64,
                                       C.c_uint64, C.c_uint64, C.c_int, C.c_uint32,
                                       C.POINTER(C.c_uint64), C.POINTER(C.c_double), _u64p,
                                       _f64p]
        R.ref_combine_decode_tokens.argtypes = [_sz, _u64p, C.POINTER(_sz), C.POINTER(C.c_int),
                                                C.POINTER(C.c_int), _u64p]
        _REF = R
    return _REF


def _f32(a) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=np.float32)


def _check(status: int, what: str) -> None:
    if status != OK:
        raise OracleError(status, what)


# ---------------------------------------------------------------- thin wrappers

def f16_encode(values) -> np.ndarray:
    v = _f32(values)
    out = np.empty(v.shape, np.uint16)
    lib().orc_f16_encode(v.reshape(-1), v.size, out.reshape(-1))
    return out


def f16_decode(bits) -> np.ndarray:
    b = np.ascontiguousarray(bits, dtype=np.uint16)
    out = np.empty(b.shape, np.float32)
    lib().orc_f16_decode(b.reshape(-1), b.size, out.reshape(-1))
    return out


def rms_norm(x, w, eps) -> np.ndarray:
    x = _f32(x)
    out = np.empty_like(x)
    lib().orc_rms_norm(x, x.shape[0], x.shape[1], _f32(w), eps, out)
    return out


def linear(x, w) -> np.ndarray:
    x, w = _f32(x), _f32(w)
    out = np.empty((x.shape[0], w.shape[0]), np.float32)
    lib().orc_linear(x, x.shape[0], x.shape[1], w, w.shape[0], out)
    return out


def apply_rope(x, heads, head_dim, first_position, theta) -> np.ndarray:
    v = _f32(x).copy()
    _check(lib().orc_apply_rope(v, v.shape[0], heads, head_dim, first_position, theta), "rope")
    return v


def greedy_last(logits) -> int:
    lg = _f32(logits)
    if lg.ndim == 1:
        lg = lg[None]
    tok = C.c_uint64()
    _check(lib().orc_greedy_last(lg, lg.shape[0], lg.shape[1], C.byref(tok)), "greedy")
    return tok.value


@dataclass
class Sampling:
    """runtime::SamplingOptions (hLLM cpp/include/hllm/runtime/sampling.hpp:10-17)."""
    temperature: float = 0.0
    top_p: float = 1.0
    top_k: int = 0
    seed: int = 0
    return_logprobs: bool = False
    top_logprobs: int = 0


def sample_token(logits, s: Sampling, generated_index: int):
    """runtime::sample_token: (token, logprob or None, [(id, logprob)...])."""
    lg = _f32(logits).reshape(-1)
    tok, lp = C.c_uint64(), C.c_double()
    ids, vals = np.zeros(8, np.uint64), np.zeros(8, np.float64)
    _check(lib().orc_sample_token(lg, lg.size, s.temperature, s.top_p, s.top_k, s.seed,
                                  generated_index, int(s.return_logprobs), s.top_logprobs,
                                  C.byref(tok), C.byref(lp), ids, vals), "sample_token")
    if not s.return_logprobs:
        return tok.value, None, []
    return tok.value, lp.value, [(int(ids[i]), float(vals[i])) for i in range(s.top_logprobs)]


def pack(sequence_slots, first_positions, query_lengths, block_table, block_size):
    """Closed-form ragged packing: (cu_seqlens, row_items, row_positions, row_slots)."""
    slots = np.ascontiguousarray(sequence_slots, np.uint32)
    firsts = np.ascontiguousarray(first_positions, np.uint64)
    lens = np.ascontiguousarray(query_lengths, np.uint32)
    table = np.ascontiguousarray(block_table, np.int32)
    n, rows = len(slots), int(lens.sum())
    cu = np.zeros(n + 1, np.uint32)
    items, pos, sl = np.zeros(rows, np.uint32), np.zeros(rows, np.uint64), np.zeros(rows, np.int64)
    _check(lib().orc_pack(n, slots, firsts, lens, table, table.shape[1], block_size, cu, items,
                          pos, sl), "pack")
    return cu, items, pos, sl


def synth_f32(seed, tensor_id, count, mean=0.0, sigma=0.02, first=0) -> np.ndarray:
    out = np.empty(count, np.float32)
    lib().orc_synth_f32(seed, tensor_id, first, count, mean, sigma, out)
    return out


def synth_f16(seed, tensor_id, count, mean=0.0, sigma=0.02, first=0) -> np.ndarray:
    out = np.empty(count, np.uint16)
    lib().orc_synth_f16(seed, tensor_id, first, count, mean, sigma, out)
    return out


# ---------------------------------------------------------------- stage model

LAYER_TENSORS = ("input_layernorm.weight", "self_attn.q_proj.weight", "self_attn.k_proj.weight",
                 "self_attn.v_proj.weight", "self_attn.o_proj.weight",
                 "post_attention_layernorm.weight", "mlp.gate_proj.weight", "mlp.up_proj.weight",
                 "mlp.down_proj.weight", "self_attn.q_norm.weight", "self_attn.k_norm.weight")


@dataclass
class StageWeights:
    """F32 weights of one stage, keyed by Safetensors tensor name."""
    config: Config
    vocabulary_size: int
    layer_start: int
    layer_end: int
    first: bool
    final: bool
    tied: bool
    tensors: dict = field(default_factory=dict)

    def layer(self, i: int) -> list:
        p = f"model.layers.{i}."
        names = LAYER_TENSORS if self.config.query_key_norm else LAYER_TENSORS[:9]
        return [_f32(self.tensors[p + n]) for n in names]

    @property
    def head(self) -> np.ndarray:
        return _f32(self.tensors["model.embed_tokens.weight" if self.tied else "lm_head.weight"])


class OracleSequence:
    """Per-sequence state: one contiguous KV cache per owned layer (CpuSequence)."""

    def __init__(self, stage: "OracleStage", tokens: int, sampling: Sampling | None = None):
        c = stage.w.config
        self.caches = []
        for _ in range(stage.w.layer_start, stage.w.layer_end):
            kv = _Kv()
            _check(lib().orc_kv_init(C.byref(kv), tokens, c.key_value_heads, c.head_dimension),
                   "kv_init")
            self.caches.append(kv)
        self.sampling = sampling or Sampling()
        self.prefill_only = False
        self.generated_index = 0

    @property
    def length(self) -> int:
        return self.caches[0].length

    def load_cache(self, layer: int, keys, values) -> None:
        """Appends positions [length, length + n) of one layer's cache from [n, kv_heads,
        head_dim] arrays (a cache state produced elsewhere, e.g. read back from the GPU)."""
        kv = self.caches[layer]
        k = _f32(keys).reshape(len(keys), -1)
        v = _f32(values).reshape(len(values), -1)
        _check(lib().orc_kv_append(C.byref(kv), kv.length, k, v, k.shape[0]), "kv_append")

    def cache_arrays(self, layer: int):
        kv = self.caches[layer]
        c_n = kv.length * kv.heads * kv.head_dimension
        k = np.ctypeslib.as_array(kv.keys, (c_n,)).reshape(kv.length, kv.heads, kv.head_dimension)
        v = np.ctypeslib.as_array(kv.values, (c_n,)).reshape(kv.length, kv.heads,
                                                             kv.head_dimension)
        return k.copy(), v.copy()

    def __del__(self):
        for kv in getattr(self, "caches", []):
            lib().orc_kv_free(C.byref(kv))


class OracleStage:
    """DenseStage::run (hLLM cpp/src/cpu/stage.cpp:118-191) over the plain-C oracle."""

    def __init__(self, weights: StageWeights):
        self.w = weights
        self._layers = []
        for i in range(weights.layer_start, weights.layer_end):
            arrays = weights.layer(i)
            ptrs = [a.ctypes.data for a in arrays] + [None] * (11 - len(arrays))
            self._layers.append((arrays, _Layer(*ptrs)))

    def allocate_sequence(self, tokens: int, sampling: Sampling | None = None) -> OracleSequence:
        if tokens == 0 or tokens > self.w.config.maximum_sequence_length:
            raise OracleError(INVALID_REQUEST, "request exceeds model context capacity")
        return OracleSequence(self, tokens, sampling)

    def embed(self, ids) -> np.ndarray:
        emb = self.w.tensors["model.embed_tokens.weight"]
        ids = np.asarray(ids, np.uint64)
        if len(ids) == 0 or np.any(ids >= self.w.vocabulary_size):
            raise OracleError(INVALID_REQUEST, "token ID exceeds vocabulary")
        return _f32(emb[ids.astype(np.int64)])

    def forward(self, hidden, position: int, seq: OracleSequence, trace: list | None = None):
        h = _f32(hidden)
        for (arrays, layer), kv in zip(self._layers, seq.caches):
            out = np.empty_like(h)
            _check(lib().orc_transformer_layer(h, h.shape[0], C.byref(layer),
                                               C.byref(self.w.config), position, C.byref(kv),
                                               out), "transformer_layer")
            h = out
            if trace is not None:
                trace.append(h.copy())
        return h

    def logits(self, hidden_last) -> np.ndarray:
        c = self.w.config
        h = _f32(hidden_last).reshape(1, -1)
        out = np.empty((1, self.w.vocabulary_size), np.float32)
        lib().orc_final_logits(h, 1, c.hidden_size, _f32(self.w.tensors["model.norm.weight"]),
                               self.w.head, self.w.vocabulary_size, c.rms_norm_epsilon, out)
        return out[0]

    def logits_rows(self, hidden) -> np.ndarray:
        """final_logits for every row of [rows, hidden] (the per-row final norm + LM head of
        a decode batch, cpp/src/cuda/stage.cpp:415-436)."""
        c = self.w.config
        h = _f32(hidden).reshape(-1, c.hidden_size)
        out = np.empty((h.shape[0], self.w.vocabulary_size), np.float32)
        lib().orc_final_logits(h, h.shape[0], c.hidden_size, _f32(self.w.tensors["model.norm.weight"]),
                               self.w.head, self.w.vocabulary_size, c.rms_norm_epsilon, out)
        return out

    def execute(self, stage_input, position: int, seq: OracleSequence, trace: list | None = None):
        """Returns ('token', id, logprob, top) | ('boundary', f16 bits [T,H]) | ('progress',)."""
        if isinstance(stage_input, np.ndarray) and stage_input.dtype == np.uint16:
            if self.w.first:
                raise OracleError(INVALID_REQUEST, "stage zero requires tokens")
            hidden = f16_decode(stage_input)
            if not np.all(np.isfinite(hidden)):
                raise OracleError(INVALID_REQUEST, "non-finite activation")
        else:
            if not self.w.first:
                raise OracleError(INVALID_REQUEST, "only stage zero accepts tokens")
            hidden = self.embed(stage_input)
        hidden = self.forward(hidden, position, seq, trace)
        if self.w.final:
            if seq.prefill_only:
                return ("progress",)
            logits = self.logits(hidden[-1])
            if trace is not None:
                trace.append(logits)
            s = seq.sampling
            if s.temperature == 0.0 and not s.return_logprobs:
                return ("token", greedy_last(logits), None, [])
            tok, lp, top = sample_token(logits, s, seq.generated_index)
            seq.generated_index += 1
            return ("token", tok, lp, top)
        bits = f16_encode(hidden)
        if np.any((bits & 0x7C00) == 0x7C00):
            raise OracleError(INTERNAL, "activation is not representable as finite FP16")
        return ("boundary", bits)

    def generate(self, prompt, steps: int, sampling: Sampling | None = None, chunk: int = 0,
                 capacity: int | None = None):
        """Greedy (or seeded) generation: prefill (optionally chunked) then `steps` decodes.

        Returns the sampled token IDs (prefill's token first) and per-pass logits of the
        final row when the stage is final."""
        prompt = list(prompt)
        seq = self.allocate_sequence(capacity or len(prompt) + steps + 1, sampling)
        tokens, logits = [], []
        pos, chunk = 0, chunk or len(prompt)
        while pos < len(prompt):
            part = prompt[pos:pos + chunk]
            seq.prefill_only = pos + len(part) < len(prompt)
            trace = []
            out = self.execute(np.asarray(part, np.uint64), pos, seq, trace)
            pos += len(part)
        tokens.append(out[1])
        logits.append(trace[-1])
        for _ in range(steps):
            trace = []
            out = self.execute(np.asarray([tokens[-1]], np.uint64), pos, seq, trace)
            pos += 1
            tokens.append(out[1])
            logits.append(trace[-1])
        return tokens, logits
