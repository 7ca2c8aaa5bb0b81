/*
 * hllm_rocm: MI355X (gfx950) decoder stage worker, C ABI.
 *
 * One `hllm_rocm_stage` is one loaded stage (a contiguous layer range, plus the token
 * embedding on the first stage and final norm + LM head + sampling on the last) on one
 * GPU. It is the device side of an hLLM `runtime::StageBackend`
 * (cpp/include/hllm/runtime/stage_backend.hpp:69-107) created by a `BackendFactory`
 * (cpp/include/hllm/runtime/backend_factory.hpp:28-47). Plain pointers and sizes only;
 * no exceptions cross this boundary. Every call returns an `hllm_status`; on failure,
 * `hllm_rocm_last_error()` holds a message for the calling thread.
 *
 * Threading mirrors the reference contract: passes on one stage are serialized by the
 * caller's scheduler (cpp/src/worker/scheduler.cpp:60-112); sequence allocation and
 * release may run concurrently with a pass and take the stage's own lock
 * (cpp/src/cuda/stage.cpp:185-202,345).
 */
#ifndef HLLM_ROCM_H
#define HLLM_ROCM_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define HLLM_ROCM_ABI_VERSION 2u

/* runtime::ErrorCode (cpp/include/hllm/runtime/error.hpp:10-17), numbered from 1. */
typedef enum {
  HLLM_OK = 0,
  HLLM_INVALID_REQUEST = 1,
  HLLM_INCOMPATIBLE_WORKER = 2,
  HLLM_RESOURCE_EXHAUSTED = 3,
  HLLM_DEADLINE_EXCEEDED = 4,
  HLLM_CANCELLED = 5,
  HLLM_INTERNAL = 6,
} hllm_status;

/* runtime::DataType subset used by dense checkpoints (cpp/include/hllm/runtime/safetensors.hpp:15-29). */
typedef enum { HLLM_DTYPE_F32 = 0, HLLM_DTYPE_F16 = 1, HLLM_DTYPE_BF16 = 2 } hllm_dtype;

typedef struct hllm_rocm_stage hllm_rocm_stage;

/* model::DenseConfig + model::DenseSource ownership (cpp/include/hllm/model/dense_source.hpp:15-44)
 * + the device resources of this worker. */
typedef struct {
  uint32_t abi_version;             /* HLLM_ROCM_ABI_VERSION */
  uint64_t hidden_size;
  uint64_t intermediate_size;
  uint64_t attention_heads;
  uint64_t key_value_heads;
  uint64_t head_dimension;
  uint64_t maximum_sequence_length;
  uint64_t vocabulary_size;
  float rms_norm_epsilon;
  float rope_theta;
  uint32_t query_key_norm;          /* Qwen3 per-head q/k RMSNorm */
  uint32_t layer_start, layer_end;  /* owned layers [start, end) */
  uint32_t first_stage;             /* owns the token embedding */
  uint32_t final_stage;             /* owns final norm, LM head, sampling */
  uint32_t tied_head;               /* LM head is the token embedding */
  uint32_t execution_dtype;         /* HLLM_DTYPE_F16 or HLLM_DTYPE_F32 (plan execution dtype) */
  uint32_t weight_dtype;            /* resident weights: F16, or F32 with F32 execution */
  int32_t device;                   /* HIP device ordinal */
  uint64_t kv_cache_bytes;          /* paged KV pool size; 0 = 90% of free HBM after weights */
  uint32_t kv_block_tokens;         /* tokens per KV block (power of two); 0 = 64 */
  uint32_t max_sequences;           /* live sequence slots; 0 = 512 */
  uint32_t max_pass_rows;           /* rows per pass (prefill chunks + decode rows); 0 = 2048 */
} hllm_rocm_stage_config;

/* One request's share of a pass. */
typedef struct {
  uint32_t sequence;        /* handle from hllm_rocm_sequence_allocate */
  uint32_t query_tokens;    /* rows this item contributes (prefill chunk length, or 1) */
  uint64_t first_position;  /* must equal the sequence's current length */
  uint32_t flags;           /* HLLM_ITEM_* */
  uint32_t top_logprobs;    /* 0..5, with return_logprobs */
  double temperature;       /* runtime::SamplingOptions (cpp/include/hllm/runtime/sampling.hpp:10-17) */
  double top_p;
  uint64_t top_k;
  uint64_t seed;
  uint64_t generated_index; /* counter of the sequence's sampling RNG */
} hllm_rocm_item;

/* The final stage projects the item's last row and samples a token (otherwise the item
 * only extends the KV cache: PrefillProgress, cpp/src/cpu/stage.cpp:164). */
#define HLLM_ITEM_SAMPLE 1u
/* The item's single input token is the token its sequence sampled in its previous pass,
 * read on the device (no host round trip). Only on a stage that is both first and final,
 * and only when the sequence's previous pass sampled (HLLM_INVALID_REQUEST otherwise). */
#define HLLM_ITEM_TOKEN_FROM_DEVICE 2u
/* Return log-probabilities (runtime::SampledToken, cpp/src/sampling.cpp:65-89). */
#define HLLM_ITEM_LOGPROBS 4u

/* A ragged pass: any mix of prefill chunks and decode rows, rows packed in item order. */
typedef struct {
  uint32_t items;
  const hllm_rocm_item* item;
  const uint64_t* token_ids;     /* first stage: sum(query_tokens) IDs in item order */
  const uint16_t* boundary_in;   /* other stages: [sum(query_tokens), hidden] F16 LE */
  /* Optional. Checked before the pass is enqueued, before each layer is enqueued, and once
   * more when the pass completes (cpp/src/cuda/stage.cpp:357,396,456). Set before the
   * device runs the pass, nothing changes; set while it runs, the pass's results are
   * discarded, its sequences are failed (never resumed, cpp/src/cuda/stage.cpp:463-468)
   * and the call returns HLLM_CANCELLED. */
  const volatile int32_t* cancelled;
  /* outputs (host pointers; NULL = not wanted) */
  uint64_t* tokens;              /* final stage: [items]; items without SAMPLE get UINT64_MAX */
  /* For sampled items with HLLM_ITEM_LOGPROBS (runtime::SampledToken): the token's
   * log-probability, and the top_logprobs best tokens and theirs in entries item * 5 + r,
   * r < top_logprobs (later entries UINT64_MAX / NaN). Other items' entries are untouched. */
  double* logprobs;              /* [items] */
  uint64_t* top_ids;             /* [items * 5] */
  double* top_logprobs;          /* [items * 5] */
  uint16_t* boundary_out;        /* non-final: [sum(query_tokens), hidden] F16 LE */
  float* logits;                 /* final: [sampled items, vocabulary] F32, for tests */
  float* trace_hidden;           /* [owned layers, sum(query_tokens), hidden] F32, for tests */
  /* Optional, read at the same points as `cancelled`: cancel_poll(cancel_context) != 0 means
   * the pass is cancelled. For callers whose flag is not an int32_t (the reference's
   * `const std::atomic_bool& cancelled` of StageBackend::execute, stage_backend.hpp:86-89).
   * The context must stay valid until the pass's execute or wait call returns. */
  int32_t (*cancel_poll)(void* cancel_context);
  void* cancel_context;
} hllm_rocm_pass;

typedef struct {
  uint64_t host_bytes;
  uint64_t device_bytes;
  uint64_t pinned_host_bytes;
  uint64_t unified_bytes;
} hllm_rocm_memory;  /* runtime::MemoryAmounts (cpp/include/hllm/runtime/memory.hpp:11-17) */

/* BackendFactory::allocator_metrics (cpp/include/hllm/runtime/backend_factory.hpp:24-33):
 * device memory this library holds on `device`. Stages reserve every buffer when they are
 * created, straight from hipMalloc with no caching layer, so cached_bytes is always 0;
 * peak_bytes is the most held at once since the process started or the last reset. */
typedef struct {
  uint64_t active_bytes;
  uint64_t cached_bytes;
  uint64_t peak_bytes;
} hllm_rocm_allocator_metrics;

/* BackendFactory::profiling_device_info (cpp/include/hllm/runtime/profiling.hpp:8-15; the CUDA
 * worker's cpp/src/cuda/device.cpp:93-108): the device's identity (its UUID as hex digits:
 * 16 as ROCm reports them, or 32 for binary UUIDs), product name (the ISA name when the driver
 * reports none), ISA, HIP runtime and driver versions, compute units and free / total HBM. */
typedef struct {
  char identity[40];
  char name[64];
  char architecture[64];
  int32_t runtime_version;
  int32_t driver_version;
  uint32_t compute_units;
  uint64_t available_bytes;
  uint64_t total_bytes;
} hllm_rocm_device_info;

/* Thread-local message of the last failed call on this thread. */
const char* hllm_rocm_last_error(void);
uint32_t hllm_rocm_abi_version(void);

/* Stage construction, replacing the CUDA worker's CudaStage constructor
 * (cpp/src/cuda/stage.cpp:87-144) and the CPU loader (cpp/src/cpu/stage.cpp:207-255):
 * validate the configuration and reserve every device buffer up front. */
hllm_status hllm_rocm_stage_create(const hllm_rocm_stage_config* config, hllm_rocm_stage** out);
void hllm_rocm_stage_destroy(hllm_rocm_stage* stage);

/* Upload one checkpoint tensor (Safetensors name and row-major LE payload), replacing the
 * per-tensor read + upload of cpp/src/cuda/stage.cpp:123-143. Rejects unknown names,
 * wrong shapes, non-finite values (cpp/src/model/dense_source.cpp:151-153) and values
 * not representable as finite F16 for F16 residency (cpp/src/cuda/stage.cpp:126-133). */
hllm_status hllm_rocm_stage_load_tensor(hllm_rocm_stage* stage, const char* name, uint32_t dtype,
                                        const uint64_t* shape, uint32_t rank, const void* data,
                                        uint64_t bytes);
/* Fill one tensor with the seeded synthetic values (hllm_amd/synthetic.py) on the device. */
hllm_status hllm_rocm_stage_synthesize_tensor(hllm_rocm_stage* stage, const char* name,
                                              uint64_t seed, uint64_t tensor_id, float mean,
                                              float sigma, uint32_t source_dtype);
/* Verify that every owned tensor arrived; the stage accepts passes afterwards. */
hllm_status hllm_rocm_stage_finalize(hllm_rocm_stage* stage);

/* StageBackend::weight_memory / sequence_memory (stage_backend.hpp:72-83). With
 * rows = query_rows(tokens, maximum_query_tokens) (stage_backend.hpp:62-67) and bt the KV
 * block size: cache = {host: tokens * 24 + rows * hidden * 6 (request_transport_bytes,
 * stage_backend.hpp:36-40), device: ceil(tokens / bt) * bt * layers * 2 * kv_heads *
 * head_dim * (2 for F16 KV, 4 for F32 KV)}; workspace = {host: rows * hidden * 6 + 65536,
 * device: 0} (pass workspaces are reserved when the stage is created). tokens = 0 or above
 * maximum_sequence_length is HLLM_INVALID_REQUEST. */
hllm_status hllm_rocm_stage_weight_memory(const hllm_rocm_stage* stage, hllm_rocm_memory* out);
hllm_status hllm_rocm_stage_sequence_memory(const hllm_rocm_stage* stage, uint64_t tokens,
                                            uint64_t maximum_query_tokens,
                                            hllm_rocm_memory* cache, hllm_rocm_memory* workspace);

/* StageBackend::allocate_sequence (stage_backend.hpp:84-85): reserve paged KV for `tokens`
 * positions (HLLM_RESOURCE_EXHAUSTED when the block pool or the sequence slots run out).
 * Release is SequenceState destruction: the handle is invalid at once; when a submitted pass
 * still uses the sequence, its slot and blocks return to the pools when that pass completes. */
hllm_status hllm_rocm_sequence_allocate(hllm_rocm_stage* stage, uint64_t tokens, uint32_t* sequence);
hllm_status hllm_rocm_sequence_release(hllm_rocm_stage* stage, uint32_t sequence);
hllm_status hllm_rocm_sequence_length(const hllm_rocm_stage* stage, uint32_t sequence,
                                      uint64_t* length);

/* StageBackend::execute / execute_decode_batch (stage_backend.hpp:90-101), generalised to
 * ragged passes that mix prefill chunks with decode rows. Synchronous: outputs are on the
 * host when it returns. A pass that fails after touching the KV cache poisons its
 * sequences (cpp/src/cuda/stage.cpp:463-468). */
hllm_status hllm_rocm_stage_execute(hllm_rocm_stage* stage, const hllm_rocm_pass* pass);

/* The same pass, enqueued on the stage's stream without waiting; outputs are valid after
 * hllm_rocm_stage_wait. At most one pass is in flight per stage. */
hllm_status hllm_rocm_stage_submit(hllm_rocm_stage* stage, const hllm_rocm_pass* pass);
hllm_status hllm_rocm_stage_wait(hllm_rocm_stage* stage);

/* One timed phase of a profiled pass: runtime::ComponentTiming
 * (cpp/include/hllm/runtime/timing.hpp:11-15). Components, in pass order: "embedding" or
 * "from-wire", "layer" (layer = its model layer index) per owned layer, then "final_norm",
 * "lm_head" and "sampling" (final stage, when the pass samples) or "to-wire" (other
 * stages); layer is -1 except for "layer". */
typedef struct {
  char component[16];
  int32_t layer;
  double milliseconds;
} hllm_rocm_phase_time;

/* StageBackend::execute_profiled (stage_backend.hpp:103-106): hllm_rocm_stage_execute with
 * HIP events between phases on the stage's stream (no synchronisation inside the pass, so
 * the outputs equal hllm_rocm_stage_execute's bit for bit). Writes up to `capacity` phases
 * and their number to *count. */
hllm_status hllm_rocm_stage_execute_profiled(hllm_rocm_stage* stage, const hllm_rocm_pass* pass,
                                             hllm_rocm_phase_time* phases, uint32_t capacity,
                                             uint32_t* count);

/* runtime::sample_token (cpp/src/sampling.cpp:65-89) on the device for `rows` rows of
 * `vocabulary` F32 logits (host memory), each with the sampling fields of options[r]
 * (temperature, top_p, top_k, seed, generated_index; flags HLLM_ITEM_LOGPROBS and
 * top_logprobs). The stage's sampler, for callers that hold logits of their own. Errors as
 * the reference: invalid options are HLLM_INVALID_REQUEST, non-finite logits HLLM_INTERNAL.
 * Outputs (host) as hllm_rocm_pass's; logprobs / top_ids / top_logprobs may be NULL. */
hllm_status hllm_rocm_sample_logits(int32_t device, const float* logits, uint64_t rows,
                                    uint64_t vocabulary, const hllm_rocm_item* options,
                                    uint64_t* tokens, double* logprobs, uint64_t* top_ids,
                                    double* top_logprobs);

/* No counterpart in the reference: hllm_rocm_sample_logits for callers that cannot allocate
 * device memory (serving loops and harnesses that must not call hipMalloc). Same arguments,
 * results and errors; it allocates nothing (no device or host heap memory, no streams or
 * events): the rows are staged and sampled two at a time through one fixed area of device
 * memory in the library, HLLM_ROCM_NOALLOC_SCRATCH_BYTES per GPU, held from the first call
 * on that GPU until the process ends. Vocabularies above HLLM_ROCM_NOALLOC_MAX_VOCABULARY
 * are HLLM_RESOURCE_EXHAUSTED. Work runs on the device's null stream and the call returns
 * when it is done. Calls on one GPU share the area: the library runs one call at a time per
 * process (a lock), and each call clears what must start at zero; a caller that drives the
 * area's device from elsewhere while a call runs (another process aside) races with it. */
#define HLLM_ROCM_NOALLOC_MAX_VOCABULARY 262144u
#define HLLM_ROCM_NOALLOC_SCRATCH_BYTES 17320704u
hllm_status hllm_rocm_sample_logits_noalloc(int32_t device, const float* logits, uint64_t rows,
                                            uint64_t vocabulary, const hllm_rocm_item* options,
                                            uint64_t* tokens, double* logprobs, uint64_t* top_ids,
                                            double* top_logprobs);

/* Replay of repeated pass shapes (items, rows, sampled rows, sampler use, attention work
 * items) from captured HIP graphs, off by default: a shape's second pass is captured and
 * later ones replay it, with the same kernels and results as eager launches and less host
 * launch work. Passes that request logits, traces or profiling run eagerly. No counterpart
 * in the reference (its CUDA stage launches eagerly). Counters: shapes captured, passes
 * replayed from a graph. */
hllm_status hllm_rocm_stage_set_graphs(hllm_rocm_stage* stage, uint32_t enabled);
hllm_status hllm_rocm_stage_graph_stats(hllm_rocm_stage* stage, uint64_t* captured,
                                        uint64_t* replayed);

/* BackendFactory::allocator_metrics / profiling_reset_peak / profiling_device_info
 * (cpp/include/hllm/runtime/backend_factory.hpp:31-39; cpp/src/cuda/device.cpp:41-54,84-108).
 * reset_peak waits for the device's work to complete, then sets the peak to the bytes held. */
hllm_status hllm_rocm_device_allocator_metrics(int32_t device, hllm_rocm_allocator_metrics* out);
hllm_status hllm_rocm_device_reset_peak(int32_t device);
hllm_status hllm_rocm_device_query(int32_t device, hllm_rocm_device_info* out);

/* Diagnostics: the HBM read ceiling of `device`, measured as the best of five streaming
 * reads of `bytes` (at least 1 MiB, a multiple of 16) with a plain read kernel, in GB/s.
 * For comparing the stage's memory-bound rates with what the device delivers; no
 * counterpart in the reference. */
hllm_status hllm_rocm_measure_read_bandwidth(int32_t device, uint64_t bytes, double* gb_s);

/* Diagnostics: the F16 matrix-core rate of `device` in TFLOP/s with no memory traffic, for
 * v_mfma_f32_16x16x32_f16 (shape 16) or v_mfma_f32_32x32x16_f16 (shape 32): best of five
 * launches of eight workgroups of four waves per CU, each wave running eight independent
 * accumulation chains from registers. The measured ceiling the prefill GEMMs' MFMA fractions
 * are read against beside the 2.5 PFLOP/s dense F16 specification; no counterpart in the
 * reference. */
hllm_status hllm_rocm_measure_mfma_rate(int32_t device, uint32_t shape, double* tflops);

/* Tuning and test hook, process-wide: every later projection GEMM uses configuration
 * `config` of the kernel table (0 .. 18; 17: the decode kernel for every F16 projection of at
 * most 64 rows whose K splits are summed by the consumer or that applies SwiGLU) instead of the
 * choice by shape; -1 restores the
 * choice by shape. *previous (may be NULL) receives the value replaced. Results stay within
 * the execution mode's tolerance for every configuration; no counterpart in the reference.
 * HLLM_ROCM_GEMM_CONFIG gives the initial value. */
hllm_status hllm_rocm_set_gemm_config(int32_t config, int32_t* previous);

/* Diagnostics for parity tests, like the reference's traced execution
 * (cpp/include/hllm/cuda/stage.hpp:8-21): the last pass's device-built packing
 * (cu_seqlens [items + 1], per-row positions and KV slots [rows]), a sequence's physical
 * KV blocks (in logical order), and one layer's cached K and V as F32 [length, kv_heads,
 * head_dim] (the CPU cache order, cpp/src/cpu/llama.cpp:152-158). */
hllm_status hllm_rocm_stage_last_layout(hllm_rocm_stage* stage, uint32_t items, uint32_t rows,
                                        int32_t* cu_seqlens, int32_t* row_positions,
                                        int32_t* row_slots);
hllm_status hllm_rocm_sequence_blocks(hllm_rocm_stage* stage, uint32_t sequence, int32_t* blocks,
                                      uint32_t capacity, uint32_t* count, uint32_t* block_tokens);
/* One loaded tensor back as row-major F32 (hi + lo parts recombined), for loader tests. */
hllm_status hllm_rocm_stage_read_tensor(hllm_rocm_stage* stage, const char* name, float* out,
                                        uint64_t elements);
hllm_status hllm_rocm_sequence_read_kv(hllm_rocm_stage* stage, uint32_t sequence, uint32_t layer,
                                       float* keys, float* values);

/* Profiling hooks for benchmarks: HIP events on the stage's stream around every kernel
 * launched for the operation families named in `families` (';'-separated prefixes such
 * as "gemm_gate_up;attention"; "*" = all; "k:<kernel>" = that kernel only, whichever family
 * launches it; NULL or "" = off). Each family launch carries its
 * algorithmic HBM bytes and FLOPs. Records are kept per family (all kernels of the
 * family's launches), per kernel under "k:<kernel>" (the kernel as rocprofv3 names it,
 * with the bytes and FLOPs of the family launch attributed to its first kernel) and per
 * (family, kernel) pair under "<family>/<kernel>". Read back
 * as sums per record (a trailing '*' matches a prefix); `launches` counts family launches,
 * or kernel launches for "k:" records. */
hllm_status hllm_rocm_stage_profile(hllm_rocm_stage* stage, const char* families);
hllm_status hllm_rocm_stage_profile_read(hllm_rocm_stage* stage, const char* record,
                                         double* milliseconds, uint64_t* launches,
                                         uint64_t* bytes, double* flops);
/* Names of the records collected so far, newline-separated, NUL-terminated in `buffer`
 * (truncated to `capacity` bytes); `needed` receives the full length including the NUL. */
hllm_status hllm_rocm_stage_profile_records(hllm_rocm_stage* stage, char* buffer,
                                            uint64_t capacity, uint64_t* needed);

#ifdef __cplusplus
}
#endif
#endif
