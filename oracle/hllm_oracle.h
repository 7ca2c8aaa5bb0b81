/*
 * CPU oracle for the decoder stage worker: a plain-C restatement of the reference
 * CPU worker's F32 arithmetic (hLLM cpp/src/cpu/, cpp/src/half.cpp,
 * cpp/src/sampling.cpp, cpp/src/decode_batch.cpp).
 *
 * TEST INFRASTRUCTURE ONLY. Only tests/, __graft_entry__.smoke() and bench.py's
 * CPU-baseline leg may load this library, and only as the checker. The product
 * (hllm_amd/) never links, loads or calls it.
 *
 * Every function keeps the reference's operation order and association (sequential
 * F32 sums, no FMA contraction: build with -ffp-contract=off), so that on the same
 * inputs it reproduces the reference bit for bit. Pinning (tests/test_oracle_*.py):
 *   - the Transformers golden vectors (tests/golden/qwen3_tiny_reference.json) at 2e-5,
 *   - the reference's own sources compiled into oracle/_ref (bit-exact comparisons),
 *   - the reference's known-answer tests (half, sampling, llama closed forms),
 *   - closed forms and invariants (incremental == one-shot causal, RoPE identities).
 * Functions without any of these say "parity unpinned" below; there are none.
 */
#ifndef HLLM_ORACLE_H
#define HLLM_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Status codes, numbered like the product's C ABI (runtime::ErrorCode order). */
enum {
  ORC_OK = 0,
  ORC_INVALID_REQUEST = 1,
  ORC_INCOMPATIBLE_WORKER = 2,
  ORC_RESOURCE_EXHAUSTED = 3,
  ORC_INTERNAL = 6,
};

/* ---- F16 / BF16 codec: cpp/src/half.cpp:8-103 -------------------------------- */
float orc_f32_from_f16(uint16_t bits);
uint16_t orc_f16_from_f32(float value);
float orc_f32_from_bf16(uint16_t bits);
uint16_t orc_bf16_from_f32(float value);
void orc_f16_encode(const float* values, size_t count, uint16_t* out);
void orc_f16_decode(const uint16_t* bits, size_t count, float* out);

/* ---- Dense layer arithmetic: cpp/src/cpu/llama.cpp, cpp/src/cpu/tensor.cpp ----- */
typedef struct {
  size_t hidden_size;
  size_t intermediate_size;
  size_t attention_heads;
  size_t key_value_heads;
  size_t head_dimension;
  size_t maximum_sequence_length;
  float rms_norm_epsilon;
  float rope_theta;
  int query_key_norm; /* Qwen3 per-head RMSNorm on q and k */
} orc_config;

typedef struct {
  const float* input_norm;          /* [H] */
  const float* query;               /* [Q*D, H] */
  const float* key;                 /* [K*D, H] */
  const float* value;               /* [K*D, H] */
  const float* attention_output;    /* [H, Q*D] */
  const float* post_attention_norm; /* [H] */
  const float* gate;                /* [I, H] */
  const float* up;                  /* [I, H] */
  const float* down;                /* [H, I] */
  const float* query_norm;          /* [D] or NULL */
  const float* key_norm;            /* [D] or NULL */
} orc_layer;

/* Contiguous per-sequence cache, element (pos, head, dim) at (pos*K + head)*D + dim
 * (cpp/src/cpu/llama.cpp:152-158). */
typedef struct {
  size_t capacity;
  size_t heads;
  size_t head_dimension;
  size_t length;
  float* keys;
  float* values;
} orc_kv_cache;

/* Worker threads for orc_linear (0 = one per core). Threads split output elements;
 * each element's sum keeps the reference order, so results do not depend on it. */
void orc_set_threads(int threads);

void orc_rms_norm(const float* input, size_t rows, size_t columns, const float* weights,
                  float epsilon, float* output);
void orc_linear(const float* input, size_t rows, size_t inner, const float* weights,
                size_t outputs, float* output);
void orc_normalize_heads(float* values, size_t count, const float* weights, size_t width,
                         float epsilon);
int orc_apply_rope(float* values, size_t rows, size_t heads, size_t head_dimension,
                   size_t first_position, float theta);
int orc_kv_init(orc_kv_cache* cache, size_t capacity, size_t heads, size_t head_dimension);
void orc_kv_free(orc_kv_cache* cache);
int orc_kv_append(orc_kv_cache* cache, size_t first_position, const float* keys,
                  const float* values, size_t rows);
void orc_attention(const float* queries, size_t rows, const orc_config* config,
                   size_t first_position, const orc_kv_cache* cache, float* output);
int orc_transformer_layer(const float* input, size_t rows, const orc_layer* layer,
                          const orc_config* config, size_t first_position,
                          orc_kv_cache* cache, float* output);
void orc_final_logits(const float* hidden, size_t rows, size_t hidden_size,
                      const float* final_norm, const float* head, size_t vocabulary,
                      float epsilon, float* logits);
/* First maximum of the last row; ORC_INTERNAL on a non-finite value in that row. */
int orc_greedy_last(const float* logits, size_t rows, size_t columns, uint64_t* token);

/* ---- Sampling: cpp/src/sampling.cpp:10-89 ------------------------------------- */
int orc_validate_sampling(double temperature, double top_p, uint32_t top_logprobs,
                          int return_logprobs);
int orc_sample_logits(const float* logits, size_t count, double temperature, double top_p,
                      uint64_t top_k, uint64_t seed, uint64_t generated_index,
                      uint64_t* token);
/* top_ids / top_logprobs hold `top_logprobs` entries when return_logprobs is set. */
int orc_sample_token(const float* logits, size_t count, double temperature, double top_p,
                     uint64_t top_k, uint64_t seed, uint64_t generated_index,
                     int return_logprobs, uint32_t top_logprobs, uint64_t* token,
                     double* logprob, uint64_t* top_ids, double* top_values);

/* ---- Ragged packing and paged KV slots (closed forms of this worker) ------------
 * cu_seqlens[i] = exclusive prefix sum of query_lengths in item order (the scheduler's
 * claim order, cpp/src/worker/scheduler.cpp:69-89; cpp/src/decode_batch.cpp:10-31);
 * for each packed row r of item i: position = first_positions[i] + (r - cu_seqlens[i]),
 * slot = block_table[seq][position / block_size] * block_size + position % block_size,
 * with block_table row `seq = sequence_slots[i]` of width `table_width`. */
int orc_pack(size_t items, const uint32_t* sequence_slots, const uint64_t* first_positions,
             const uint32_t* query_lengths, const int32_t* block_table, size_t table_width,
             size_t block_size, uint32_t* cu_seqlens, uint32_t* row_items,
             uint64_t* row_positions, int64_t* row_slots);

/* ---- Seeded synthetic weights -------------------------------------------------
 * Element i of tensor `tensor_id`: three SplitMix64 outputs at counters
 * (tensor_id << 40) + 3i + j give twelve 16-bit uniforms u; the Irwin-Hall(12) sum
 * n = (sum(u) + 6 - 6*65536) / 65536 (exact in F32) approximates N(0,1);
 * value = mean + n * sigma in F32 (one rounding each). Bit-identical on CPU and GPU. */
void orc_synth_f32(uint64_t seed, uint64_t tensor_id, uint64_t first, size_t count,
                   float mean, float sigma, float* out);
void orc_synth_f16(uint64_t seed, uint64_t tensor_id, uint64_t first, size_t count,
                   float mean, float sigma, uint16_t* out);
uint64_t orc_splitmix64(uint64_t state);

/* Test switch: a nonzero value plants one of the numbered formula mistakes described in
 * hllm_oracle.c, so tests can show the golden checks catch them. */
extern int orc_planted_mistake;

#ifdef __cplusplus
}
#endif
#endif
