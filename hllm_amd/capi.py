"""ctypes binding of the C ABI in include/hllm_rocm.h (libhllm_rocm.so, built in-tree).

There is no fallback: if the library is missing or fails to load, every entry point
raises. ``Stage`` is a thin owner of one ``hllm_rocm_stage``.
"""
from __future__ import annotations

import ctypes as C
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIBRARY = os.path.join(HERE, "libhllm_rocm.so")
ABI_VERSION = 2

OK, INVALID_REQUEST, INCOMPATIBLE_WORKER, RESOURCE_EXHAUSTED = 0, 1, 2, 3
DEADLINE_EXCEEDED, CANCELLED, INTERNAL = 4, 5, 6
F32, F16, BF16 = 0, 1, 2
ITEM_SAMPLE, ITEM_TOKEN_FROM_DEVICE, ITEM_LOGPROBS = 1, 2, 4
STATUS_NAMES = {0: "OK", 1: "INVALID_REQUEST", 2: "INCOMPATIBLE_WORKER", 3: "RESOURCE_EXHAUSTED",
                4: "DEADLINE_EXCEEDED", 5: "CANCELLED", 6: "INTERNAL"}
EXPORTS = ("hllm_rocm_last_error", "hllm_rocm_abi_version", "hllm_rocm_stage_create",
           "hllm_rocm_stage_destroy", "hllm_rocm_stage_load_tensor",
           "hllm_rocm_stage_synthesize_tensor", "hllm_rocm_stage_finalize",
           "hllm_rocm_stage_weight_memory", "hllm_rocm_stage_sequence_memory",
           "hllm_rocm_sequence_allocate", "hllm_rocm_sequence_release",
           "hllm_rocm_sequence_length", "hllm_rocm_stage_execute", "hllm_rocm_stage_submit",
           "hllm_rocm_stage_wait", "hllm_rocm_stage_last_layout", "hllm_rocm_sequence_blocks",
           "hllm_rocm_sequence_read_kv", "hllm_rocm_stage_read_tensor", "hllm_rocm_stage_profile", "hllm_rocm_stage_profile_read",
           "hllm_rocm_stage_profile_records", "hllm_rocm_sample_logits",
           "hllm_rocm_stage_set_graphs", "hllm_rocm_stage_graph_stats", "hllm_rocm_set_gemm_config",
           "hllm_rocm_measure_read_bandwidth", "hllm_rocm_stage_execute_profiled",
           "hllm_rocm_sample_logits_noalloc", "hllm_rocm_device_allocator_metrics",
           "hllm_rocm_device_reset_peak", "hllm_rocm_device_query", "hllm_rocm_measure_mfma_rate")
NOALLOC_MAX_VOCABULARY = 262144


class StageError(RuntimeError):
    def __init__(self, status: int, message: str):
        super().__init__(f"{STATUS_NAMES.get(status, status)}: {message}")
        self.status = status


class StageConfig(C.Structure):
    _fields_ = [("abi_version", C.c_uint32), ("hidden_size", C.c_uint64),
                ("intermediate_size", C.c_uint64), ("attention_heads", C.c_uint64),
                ("key_value_heads", C.c_uint64), ("head_dimension", C.c_uint64),
                ("maximum_sequence_length", C.c_uint64), ("vocabulary_size", C.c_uint64),
                ("rms_norm_epsilon", C.c_float), ("rope_theta", C.c_float),
                ("query_key_norm", C.c_uint32), ("layer_start", C.c_uint32),
                ("layer_end", C.c_uint32), ("first_stage", C.c_uint32),
                ("final_stage", C.c_uint32), ("tied_head", C.c_uint32),
                ("execution_dtype", C.c_uint32), ("weight_dtype", C.c_uint32),
                ("device", C.c_int32), ("kv_cache_bytes", C.c_uint64),
                ("kv_block_tokens", C.c_uint32), ("max_sequences", C.c_uint32),
                ("max_pass_rows", C.c_uint32)]


class Item(C.Structure):
    _fields_ = [("sequence", C.c_uint32), ("query_tokens", C.c_uint32),
                ("first_position", C.c_uint64), ("flags", C.c_uint32),
                ("top_logprobs", C.c_uint32), ("temperature", C.c_double),
                ("top_p", C.c_double), ("top_k", C.c_uint64), ("seed", C.c_uint64),
                ("generated_index", C.c_uint64)]


CancelPoll = C.CFUNCTYPE(C.c_int32, C.c_void_p)


class Pass(C.Structure):
    _fields_ = [("items", C.c_uint32), ("item", C.POINTER(Item)),
                ("token_ids", C.POINTER(C.c_uint64)), ("boundary_in", C.POINTER(C.c_uint16)),
                ("cancelled", C.POINTER(C.c_int32)), ("tokens", C.POINTER(C.c_uint64)),
                ("logprobs", C.POINTER(C.c_double)), ("top_ids", C.POINTER(C.c_uint64)),
                ("top_logprobs", C.POINTER(C.c_double)),
                ("boundary_out", C.POINTER(C.c_uint16)), ("logits", C.POINTER(C.c_float)),
                ("trace_hidden", C.POINTER(C.c_float)), ("cancel_poll", CancelPoll),
                ("cancel_context", C.c_void_p)]


class AllocatorMetrics(C.Structure):
    _fields_ = [("active_bytes", C.c_uint64), ("cached_bytes", C.c_uint64), ("peak_bytes", C.c_uint64)]


class DeviceInfo(C.Structure):
    _fields_ = [("identity", C.c_char * 40), ("name", C.c_char * 64), ("architecture", C.c_char * 64),
                ("runtime_version", C.c_int32), ("driver_version", C.c_int32),
                ("compute_units", C.c_uint32), ("available_bytes", C.c_uint64), ("total_bytes", C.c_uint64)]


class PhaseTime(C.Structure):
    _fields_ = [("component", C.c_char * 16), ("layer", C.c_int32), ("milliseconds", C.c_double)]


class Memory(C.Structure):
    _fields_ = [("host_bytes", C.c_uint64), ("device_bytes", C.c_uint64),
                ("pinned_host_bytes", C.c_uint64), ("unified_bytes", C.c_uint64)]


_LIB = None


def library() -> C.CDLL:
    """Load libhllm_rocm.so; raises if it was not built (run hllm_amd/build.py)."""
    global _LIB
    if _LIB is not None:
        return _LIB
    if not os.path.exists(LIBRARY):
        raise RuntimeError(f"{LIBRARY} is missing: build it with `python hllm_amd/build.py`")
    L = C.CDLL(LIBRARY)
    st, vp, u32, u64 = C.c_int, C.c_void_p, C.c_uint32, C.c_uint64
    L.hllm_rocm_last_error.restype = C.c_char_p
    L.hllm_rocm_abi_version.restype = u32
    L.hllm_rocm_stage_create.argtypes = [C.POINTER(StageConfig), C.POINTER(vp)]
    L.hllm_rocm_stage_destroy.argtypes = [vp]
    L.hllm_rocm_stage_destroy.restype = None
    L.hllm_rocm_stage_load_tensor.argtypes = [vp, C.c_char_p, u32, C.POINTER(u64), u32, vp, u64]
    L.hllm_rocm_stage_synthesize_tensor.argtypes = [vp, C.c_char_p, u64, u64, C.c_float,
                                                    C.c_float, u32]
    L.hllm_rocm_stage_finalize.argtypes = [vp]
    L.hllm_rocm_stage_weight_memory.argtypes = [vp, C.POINTER(Memory)]
    L.hllm_rocm_stage_sequence_memory.argtypes = [vp, u64, u64, C.POINTER(Memory),
                                                  C.POINTER(Memory)]
    L.hllm_rocm_sequence_allocate.argtypes = [vp, u64, C.POINTER(u32)]
    L.hllm_rocm_sequence_release.argtypes = [vp, u32]
    L.hllm_rocm_sequence_length.argtypes = [vp, u32, C.POINTER(u64)]
    L.hllm_rocm_stage_execute.argtypes = [vp, C.POINTER(Pass)]
    L.hllm_rocm_stage_submit.argtypes = [vp, C.POINTER(Pass)]
    L.hllm_rocm_stage_wait.argtypes = [vp]
    L.hllm_rocm_stage_execute_profiled.argtypes = [vp, C.POINTER(Pass), C.POINTER(PhaseTime), u32,
                                                   C.POINTER(u32)]
    L.hllm_rocm_stage_last_layout.argtypes = [vp, u32, u32, C.POINTER(C.c_int32),
                                              C.POINTER(C.c_int32), C.POINTER(C.c_int32)]
    L.hllm_rocm_sequence_blocks.argtypes = [vp, u32, C.POINTER(C.c_int32), u32, C.POINTER(u32),
                                            C.POINTER(u32)]
    L.hllm_rocm_sequence_read_kv.argtypes = [vp, u32, u32, C.POINTER(C.c_float),
                                             C.POINTER(C.c_float)]
    L.hllm_rocm_stage_read_tensor.argtypes = [vp, C.c_char_p, C.POINTER(C.c_float), u64]
    L.hllm_rocm_stage_profile.argtypes = [vp, C.c_char_p]
    L.hllm_rocm_stage_profile_read.argtypes = [vp, C.c_char_p, C.POINTER(C.c_double),
                                               C.POINTER(C.c_uint64), C.POINTER(C.c_uint64),
                                               C.POINTER(C.c_double)]
    L.hllm_rocm_stage_profile_records.argtypes = [vp, C.c_char_p, C.c_uint64, C.POINTER(C.c_uint64)]
    L.hllm_rocm_stage_set_graphs.argtypes = [vp, u32]
    L.hllm_rocm_stage_graph_stats.argtypes = [vp, C.POINTER(u64), C.POINTER(u64)]
    L.hllm_rocm_set_gemm_config.argtypes = [C.c_int32, C.POINTER(C.c_int32)]
    L.hllm_rocm_measure_read_bandwidth.argtypes = [C.c_int32, u64, C.POINTER(C.c_double)]
    L.hllm_rocm_measure_mfma_rate.argtypes = [C.c_int32, u32, C.POINTER(C.c_double)]
    L.hllm_rocm_sample_logits.argtypes = [C.c_int32, C.POINTER(C.c_float), u64, u64, C.POINTER(Item),
                                          C.POINTER(u64), C.POINTER(C.c_double), C.POINTER(u64),
                                          C.POINTER(C.c_double)]
    L.hllm_rocm_sample_logits_noalloc.argtypes = L.hllm_rocm_sample_logits.argtypes
    L.hllm_rocm_device_allocator_metrics.argtypes = [C.c_int32, C.POINTER(AllocatorMetrics)]
    L.hllm_rocm_device_reset_peak.argtypes = [C.c_int32]
    L.hllm_rocm_device_query.argtypes = [C.c_int32, C.POINTER(DeviceInfo)]
    for name in EXPORTS:
        fn = getattr(L, name)
        if fn.restype is C.c_int or (fn.restype is None and name != "hllm_rocm_stage_destroy"):
            fn.restype = st
    if L.hllm_rocm_abi_version() != ABI_VERSION:
        raise RuntimeError("libhllm_rocm.so ABI version mismatch")
    _LIB = L
    return L


def check(status: int) -> None:
    if status != OK:
        raise StageError(status, library().hllm_rocm_last_error().decode())


def _ptr(a, ctype):
    return None if a is None else a.ctypes.data_as(C.POINTER(ctype))


def allocator_metrics(device: int = 0) -> dict:
    """Device memory the library holds on `device` (hllm_rocm_device_allocator_metrics)."""
    m = AllocatorMetrics()
    check(library().hllm_rocm_device_allocator_metrics(device, C.byref(m)))
    return {"active_bytes": m.active_bytes, "cached_bytes": m.cached_bytes, "peak_bytes": m.peak_bytes}


def reset_peak(device: int = 0) -> None:
    check(library().hllm_rocm_device_reset_peak(device))


def device_info(device: int = 0) -> dict:
    d = DeviceInfo()
    check(library().hllm_rocm_device_query(device, C.byref(d)))
    return {f: (getattr(d, f).decode() if isinstance(getattr(d, f), bytes) else getattr(d, f))
            for f, _ in DeviceInfo._fields_}


class Stage:
    """One stage on one GPU (owner of an ``hllm_rocm_stage``)."""

    def __init__(self, config: StageConfig):
        self.lib = library()
        self.config = config
        handle = C.c_void_p()
        check(self.lib.hllm_rocm_stage_create(C.byref(config), C.byref(handle)))
        self.handle = handle

    def close(self) -> None:
        if getattr(self, "handle", None):
            self.lib.hllm_rocm_stage_destroy(self.handle)
            self.handle = None

    def __del__(self):
        self.close()

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    # --------------------------------------------------------------- weights
    def load_tensor(self, name: str, array: np.ndarray, dtype: int | None = None) -> None:
        a = np.ascontiguousarray(array)
        if dtype is None:
            dtype = {np.dtype(np.float32): F32, np.dtype(np.float16): F16,
                     np.dtype(np.uint16): F16}[a.dtype]
        shape = (C.c_uint64 * a.ndim)(*a.shape)
        check(self.lib.hllm_rocm_stage_load_tensor(self.handle, name.encode(), dtype, shape, a.ndim,
                                                   a.ctypes.data, a.nbytes))

    def synthesize_tensor(self, name: str, seed: int, tensor_id: int, mean: float, sigma: float,
                          source_dtype: int) -> None:
        check(self.lib.hllm_rocm_stage_synthesize_tensor(self.handle, name.encode(), seed,
                                                         tensor_id, mean, sigma, source_dtype))

    def finalize(self) -> None:
        check(self.lib.hllm_rocm_stage_finalize(self.handle))

    def weight_memory(self) -> Memory:
        m = Memory()
        check(self.lib.hllm_rocm_stage_weight_memory(self.handle, C.byref(m)))
        return m

    def sequence_memory(self, tokens: int, max_query: int = 0):
        cache, ws = Memory(), Memory()
        check(self.lib.hllm_rocm_stage_sequence_memory(self.handle, tokens, max_query,
                                                       C.byref(cache), C.byref(ws)))
        return cache, ws

    # --------------------------------------------------------------- sequences
    def allocate(self, tokens: int) -> int:
        h = C.c_uint32()
        check(self.lib.hllm_rocm_sequence_allocate(self.handle, tokens, C.byref(h)))
        return h.value

    def release(self, sequence: int) -> None:
        check(self.lib.hllm_rocm_sequence_release(self.handle, sequence))

    def length(self, sequence: int) -> int:
        n = C.c_uint64()
        check(self.lib.hllm_rocm_sequence_length(self.handle, sequence, C.byref(n)))
        return n.value

    def blocks(self, sequence: int):
        count, bt = C.c_uint32(), C.c_uint32()
        check(self.lib.hllm_rocm_sequence_blocks(self.handle, sequence, None, 0, C.byref(count),
                                                 C.byref(bt)))
        out = np.zeros(count.value, np.int32)
        check(self.lib.hllm_rocm_sequence_blocks(self.handle, sequence, _ptr(out, C.c_int32),
                                                 count.value, C.byref(count), C.byref(bt)))
        return out, bt.value

    def read_kv(self, sequence: int, layer: int):
        n = self.length(sequence)
        c = self.config
        k = np.zeros((n, c.key_value_heads, c.head_dimension), np.float32)
        v = np.zeros_like(k)
        check(self.lib.hllm_rocm_sequence_read_kv(self.handle, sequence, layer,
                                                  _ptr(k, C.c_float), _ptr(v, C.c_float)))
        return k, v

    def read_tensor(self, name: str, shape) -> np.ndarray:
        out = np.zeros(shape, np.float32)
        check(self.lib.hllm_rocm_stage_read_tensor(self.handle, name.encode(), _ptr(out, C.c_float),
                                                   out.size))
        return out

    def last_layout(self, items: int, rows: int):
        cu = np.zeros(items + 1, np.int32)
        pos, slots = np.zeros(rows, np.int32), np.zeros(rows, np.int32)
        check(self.lib.hllm_rocm_stage_last_layout(self.handle, items, rows, _ptr(cu, C.c_int32),
                                                   _ptr(pos, C.c_int32), _ptr(slots, C.c_int32)))
        return cu, pos, slots

    # --------------------------------------------------------------- passes
    def make_pass(self, items, token_ids=None, boundary=None, want_logits=False,
                  trace=False, cancelled=None):
        """Build a Pass (and the output arrays it points at) from a list of Item.
        `cancelled`: an int32 array (the flag), or a Python callable polled through
        cancel_poll (returns true when the pass is cancelled)."""
        n = len(items)
        arr = (Item * n)(*items)
        rows = sum(int(it.query_tokens) for it in items)
        c = self.config
        p = Pass()
        p.items = n
        p.item = arr
        keep = {"items": arr}
        if token_ids is not None:
            ids = np.ascontiguousarray(token_ids, np.uint64)
            keep["ids"] = ids
            p.token_ids = _ptr(ids, C.c_uint64)
        if boundary is not None:
            b = np.ascontiguousarray(boundary, np.uint16)
            keep["boundary"] = b
            p.boundary_in = _ptr(b, C.c_uint16)
        if callable(cancelled):
            poll = CancelPoll(lambda _context: 1 if cancelled() else 0)
            keep["cancel_poll"] = poll
            p.cancel_poll = poll
        elif cancelled is not None:
            keep["cancelled"] = cancelled
            p.cancelled = _ptr(cancelled, C.c_int32)
        out = {"tokens": np.zeros(n, np.uint64)}
        p.tokens = _ptr(out["tokens"], C.c_uint64)
        if c.final_stage and any(it.flags & ITEM_LOGPROBS for it in items):
            out["logprobs"] = np.full(n, np.nan)
            out["top_ids"] = np.full((n, 5), np.iinfo(np.uint64).max, np.uint64)
            out["top_logprobs"] = np.full((n, 5), np.nan)
            p.logprobs = _ptr(out["logprobs"], C.c_double)
            p.top_ids = _ptr(out["top_ids"], C.c_uint64)
            p.top_logprobs = _ptr(out["top_logprobs"], C.c_double)
        if not c.final_stage:
            out["boundary"] = np.zeros((rows, c.hidden_size), np.uint16)
            p.boundary_out = _ptr(out["boundary"], C.c_uint16)
        if want_logits and c.final_stage:
            sampled = sum(1 for it in items if it.flags & ITEM_SAMPLE)
            out["logits"] = np.zeros((sampled, c.vocabulary_size), np.float32)
            p.logits = _ptr(out["logits"], C.c_float)
        if trace:
            out["trace"] = np.zeros((c.layer_end - c.layer_start, rows, c.hidden_size), np.float32)
            p.trace_hidden = _ptr(out["trace"], C.c_float)
        return p, out, keep

    def execute(self, items, token_ids=None, boundary=None, want_logits=False, trace=False,
                cancelled=None):
        p, out, keep = self.make_pass(items, token_ids, boundary, want_logits, trace, cancelled)
        check(self.lib.hllm_rocm_stage_execute(self.handle, C.byref(p)))
        del keep
        return out

    def execute_profiled(self, items, token_ids=None, boundary=None, want_logits=False,
                         cancelled=None):
        """execute() plus per-phase device times: out["phases"] = [(component, layer or None,
        milliseconds)] (runtime::ExecutionTiming)."""
        p, out, keep = self.make_pass(items, token_ids, boundary, want_logits, False, cancelled)
        c = self.config
        capacity = (c.layer_end - c.layer_start) + 8
        phases = (PhaseTime * capacity)()
        count = C.c_uint32(0)
        check(self.lib.hllm_rocm_stage_execute_profiled(self.handle, C.byref(p), phases, capacity,
                                                        C.byref(count)))
        del keep
        out["phases"] = [(phases[i].component.decode(), None if phases[i].layer < 0 else phases[i].layer,
                          phases[i].milliseconds) for i in range(min(count.value, capacity))]
        return out

    def submit(self, items, token_ids=None, boundary=None, want_logits=False, cancelled=None):
        """Enqueue a pass without waiting: returns a handle for wait()."""
        p, out, keep = self.make_pass(items, token_ids, boundary, want_logits, False, cancelled)
        check(self.lib.hllm_rocm_stage_submit(self.handle, C.byref(p)))
        return (p, out, keep)

    def wait(self, handle):
        """Completes the submitted pass; returns its outputs."""
        check(self.lib.hllm_rocm_stage_wait(self.handle))
        return handle[1]

    # --------------------------------------------------------------- graphs
    def set_graphs(self, enabled: bool) -> None:
        """Replay repeated pass shapes from captured HIP graphs (default off)."""
        check(self.lib.hllm_rocm_stage_set_graphs(self.handle, 1 if enabled else 0))

    def graph_stats(self):
        """(pass shapes captured, passes replayed from a graph)."""
        cap, rep = C.c_uint64(), C.c_uint64()
        check(self.lib.hllm_rocm_stage_graph_stats(self.handle, C.byref(cap), C.byref(rep)))
        return cap.value, rep.value

    # --------------------------------------------------------------- profiling
    def profile(self, families: str | None) -> None:
        """Time the named families (';'-separated prefixes, "*" = all, "k:<kernel>" = one
        kernel, None = off)."""
        check(self.lib.hllm_rocm_stage_profile(self.handle, families.encode() if families else None))

    def profile_read(self, record: str):
        """(milliseconds, launches, algorithmic bytes, algorithmic FLOPs) of a family record
        or a "k:<kernel>" record ('*' suffix = prefix match)."""
        ms, n, b, f = C.c_double(), C.c_uint64(), C.c_uint64(), C.c_double()
        check(self.lib.hllm_rocm_stage_profile_read(self.handle, record.encode(), C.byref(ms),
                                                    C.byref(n), C.byref(b), C.byref(f)))
        return ms.value, n.value, b.value, f.value

    def profile_records(self) -> list[str]:
        need = C.c_uint64()
        check(self.lib.hllm_rocm_stage_profile_records(self.handle, None, 0, C.byref(need)))
        buf = C.create_string_buffer(need.value)
        check(self.lib.hllm_rocm_stage_profile_records(self.handle, buf, need.value, C.byref(need)))
        return [r for r in buf.value.decode().split("\n") if r]


def sample_logits(logits, options, device: int = 0):
    """runtime::sample_token on the device for each row of `logits` ([rows, vocabulary]
    F32) with the sampling fields of the matching Item of `options`: (tokens, logprobs,
    top_ids [rows, 5], top_logprobs [rows, 5])."""
    lg = np.ascontiguousarray(logits, np.float32)
    if lg.ndim != 2 or len(options) != lg.shape[0]:
        raise ValueError("one option per row of [rows, vocabulary] logits")
    rows, vocab = lg.shape
    opts = (Item * rows)(*options)
    tokens = np.zeros(rows, np.uint64)
    logprobs = np.full(rows, np.nan)
    top_ids = np.full((rows, 5), np.iinfo(np.uint64).max, np.uint64)
    top_lp = np.full((rows, 5), np.nan)
    check(library().hllm_rocm_sample_logits(device, _ptr(lg, C.c_float), rows, vocab, opts,
                                             _ptr(tokens, C.c_uint64), _ptr(logprobs, C.c_double),
                                             _ptr(top_ids, C.c_uint64), _ptr(top_lp, C.c_double)))
    return tokens, logprobs, top_ids, top_lp


def sample_logits_noalloc(logits, options, device: int = 0):
    """sample_logits through the entry point that allocates nothing (a fixed device area in
    the library; vocabularies up to NOALLOC_MAX_VOCABULARY)."""
    lg = np.ascontiguousarray(logits, np.float32)
    if lg.ndim != 2 or len(options) != lg.shape[0]:
        raise ValueError("one option per row of [rows, vocabulary] logits")
    rows, vocab = lg.shape
    opts = (Item * rows)(*options)
    tokens = np.zeros(rows, np.uint64)
    logprobs = np.full(rows, np.nan)
    top_ids = np.full((rows, 5), np.iinfo(np.uint64).max, np.uint64)
    top_lp = np.full((rows, 5), np.nan)
    check(library().hllm_rocm_sample_logits_noalloc(device, _ptr(lg, C.c_float), rows, vocab, opts,
                                                     _ptr(tokens, C.c_uint64),
                                                     _ptr(logprobs, C.c_double),
                                                     _ptr(top_ids, C.c_uint64),
                                                     _ptr(top_lp, C.c_double)))
    return tokens, logprobs, top_ids, top_lp


def measure_read_bandwidth(nbytes: int = 4 << 30, device: int = 0) -> float:
    """Measured HBM read ceiling of the device in GB/s (best of five streaming reads)."""
    out = C.c_double(0.0)
    check(library().hllm_rocm_measure_read_bandwidth(device, nbytes, C.byref(out)))
    return out.value


def measure_mfma_rate(shape: int = 16, device: int = 0) -> float:
    """Measured F16 MFMA rate of the device in TFLOP/s, no memory traffic (shape 16:
    v_mfma_f32_16x16x32_f16, 32: v_mfma_f32_32x32x16_f16)."""
    out = C.c_double(0.0)
    check(library().hllm_rocm_measure_mfma_rate(device, shape, C.byref(out)))
    return out.value


def set_gemm_config(config: int) -> int:
    """Process-wide projection GEMM configuration override (-1: the choice by shape);
    returns the previous value."""
    prev = C.c_int32(0)
    check(library().hllm_rocm_set_gemm_config(config, C.byref(prev)))
    return prev.value


def item(sequence: int, query_tokens: int, first_position: int, sample: bool = True,
         from_device: bool = False, temperature: float = 0.0, top_p: float = 1.0, top_k: int = 0,
         seed: int = 0, generated_index: int = 0, logprobs: bool = False,
         top_logprobs: int = 0) -> Item:
    flags = (ITEM_SAMPLE if sample else 0) | (ITEM_TOKEN_FROM_DEVICE if from_device else 0) | \
        (ITEM_LOGPROBS if logprobs else 0)
    return Item(sequence, query_tokens, first_position, flags, top_logprobs, temperature, top_p,
                top_k, seed, generated_index)
