/*
 * CPU oracle: plain-C restatement of the reference CPU worker's arithmetic.
 * TEST INFRASTRUCTURE ONLY (see hllm_oracle.h). Build: oracle/Makefile
 * (-O2 -ffp-contract=off, default x86-64 target: no FMA, like the reference build).
 */
#include "hllm_oracle.h"

#include <math.h>
#include <pthread.h>
#include <stdlib.h>
#include <string.h>
#include <unistd.h>

/* Planted mistakes, for the tests that show the oracle's checks catch them: 0 = none,
 * 1 = residual after attention dropped, 2 = RoPE rotation sign flipped, 3 = causal mask
 * excludes the query's own position (off by one), 4 = SwiGLU gates the wrong half,
 * 5 = RMSNorm without epsilon inside the root but over n - 1 (a wrong mean). */
int orc_planted_mistake = 0;

/* ---------------------------------------------------------------- F16 / BF16 */

/* cpp/src/half.cpp:8-34 */
float orc_f32_from_f16(uint16_t bits) {
  uint32_t sign = (uint32_t)(bits & 0x8000u) << 16;
  uint32_t exponent = (bits >> 10) & 0x1fu;
  uint32_t mantissa = bits & 0x3ffu;
  uint32_t out;
  if (exponent == 0u) {
    if (mantissa == 0u) {
      out = sign;
    } else {
      /* Subnormal: shift the leading one into the implicit position. */
      uint32_t shifts = 0u;
      while ((mantissa & 0x400u) == 0u) {
        mantissa <<= 1u;
        ++shifts;
      }
      out = sign | ((113u - shifts) << 23) | ((mantissa & 0x3ffu) << 13);
    }
  } else if (exponent == 0x1fu) {
    out = sign | 0x7f800000u | (mantissa << 13);
  } else {
    out = sign | ((exponent + 112u) << 23) | (mantissa << 13);
  }
  float value;
  memcpy(&value, &out, sizeof value);
  return value;
}

/* cpp/src/half.cpp:36-88: round to nearest, ties to even. */
uint16_t orc_f16_from_f32(float value) {
  uint32_t bits;
  memcpy(&bits, &value, sizeof bits);
  uint16_t sign = (uint16_t)((bits >> 16) & 0x8000u);
  uint32_t exponent = (bits >> 23) & 0xffu;
  uint32_t mantissa = bits & 0x7fffffu;
  if (exponent == 0xffu) {
    if (mantissa == 0u) return (uint16_t)(sign | 0x7c00u);
    return (uint16_t)(sign | 0x7c00u | (mantissa >> 13) | 1u);
  }
  int half_exponent = (int)exponent - 112;
  if (half_exponent >= 31) return (uint16_t)(sign | 0x7c00u);
  if (half_exponent <= 0) {
    if (half_exponent < -10) return sign;
    uint32_t significand = mantissa | 0x800000u;
    uint32_t shift = (uint32_t)(14 - half_exponent);
    uint32_t kept = significand >> shift;
    uint32_t dropped = significand & ((1u << shift) - 1u);
    uint32_t halfway = 1u << (shift - 1u);
    if (dropped > halfway || (dropped == halfway && (kept & 1u))) ++kept;
    return (uint16_t)(sign | kept);
  }
  uint32_t kept = mantissa >> 13;
  uint32_t dropped = mantissa & 0x1fffu;
  if (dropped > 0x1000u || (dropped == 0x1000u && (kept & 1u))) {
    ++kept;
    if (kept == 0x400u) {
      kept = 0u;
      ++half_exponent;
      if (half_exponent >= 31) return (uint16_t)(sign | 0x7c00u);
    }
  }
  return (uint16_t)(sign | ((uint32_t)half_exponent << 10) | kept);
}

/* cpp/src/half.cpp:90-92 */
float orc_f32_from_bf16(uint16_t bits) {
  uint32_t wide = (uint32_t)bits << 16;
  float value;
  memcpy(&value, &wide, sizeof value);
  return value;
}

/* cpp/src/half.cpp:94-103 */
uint16_t orc_bf16_from_f32(float value) {
  uint32_t bits;
  memcpy(&bits, &value, sizeof bits);
  if ((bits & 0x7f800000u) == 0x7f800000u && (bits & 0x7fffffu) != 0u) {
    return (uint16_t)((bits >> 16) | 0x40u);
  }
  return (uint16_t)((bits + 0x7fffu + ((bits >> 16) & 1u)) >> 16);
}

void orc_f16_encode(const float* values, size_t count, uint16_t* out) {
  for (size_t i = 0; i < count; ++i) out[i] = orc_f16_from_f32(values[i]);
}

static void parallel_elements(size_t count, void (*body)(void*, size_t, size_t), void* context);

static void f16_decode_range(void* context, size_t begin, size_t end) {
  const void* const* io = (const void* const*)context;
  const uint16_t* bits = (const uint16_t*)io[0];
  float* out = (float*)io[1];
  for (size_t i = begin; i < end; ++i) out[i] = orc_f32_from_f16(bits[i]);
}

void orc_f16_decode(const uint16_t* bits, size_t count, float* out) {
  const void* io[2] = {bits, out};
  parallel_elements(count, f16_decode_range, (void*)io);
}

/* ------------------------------------------------------------ layer arithmetic */

static int g_threads = 0;

void orc_set_threads(int threads) { g_threads = threads; }

static int thread_count(void) {
  if (g_threads > 0) return g_threads;
  long cores = sysconf(_SC_NPROCESSORS_ONLN);
  return cores > 0 ? (int)(cores > 16 ? 16 : cores) : 1;
}

typedef struct {
  void (*body)(void*, size_t, size_t);
  void* context;
  size_t begin, end;
} element_job;

static void* element_worker(void* arg) {
  element_job* j = (element_job*)arg;
  j->body(j->context, j->begin, j->end);
  return NULL;
}

/* body(context, begin, end) over [0, count) in contiguous ranges, one per thread; element
 * results do not depend on the split. */
static void parallel_elements(size_t count, void (*body)(void*, size_t, size_t), void* context) {
  int threads = thread_count();
  if (count < (1u << 16)) threads = 1;
  if (threads > 64) threads = 64;
  if (threads <= 1) {
    body(context, 0, count);
    return;
  }
  element_job jobs[64];
  pthread_t ids[64];
  const size_t per = (count + (size_t)threads - 1) / (size_t)threads;
  for (int t = 0; t < threads; ++t) {
    const size_t b = (size_t)t * per;
    jobs[t] = (element_job){body, context, b < count ? b : count, b + per < count ? b + per : count};
  }
  for (int t = 1; t < threads; ++t) pthread_create(&ids[t], NULL, element_worker, &jobs[t]);
  element_worker(&jobs[0]);
  for (int t = 1; t < threads; ++t) pthread_join(ids[t], NULL);
}

/* body(context, begin, end) over [0, count) units in contiguous ranges, one per thread
 * (for units that each carry much work). */
static void parallel_units(size_t count, void (*body)(void*, size_t, size_t), void* context) {
  int threads = thread_count();
  if ((size_t)threads > count) threads = (int)count;
  if (threads > 64) threads = 64;
  if (threads <= 1) {
    body(context, 0, count);
    return;
  }
  element_job jobs[64];
  pthread_t ids[64];
  const size_t per = (count + (size_t)threads - 1) / (size_t)threads;
  for (int t = 0; t < threads; ++t) {
    const size_t b = (size_t)t * per;
    jobs[t] = (element_job){body, context, b < count ? b : count, b + per < count ? b + per : count};
  }
  for (int t = 1; t < threads; ++t) pthread_create(&ids[t], NULL, element_worker, &jobs[t]);
  element_worker(&jobs[0]);
  for (int t = 1; t < threads; ++t) pthread_join(ids[t], NULL);
}

/* cpp/src/cpu/llama.cpp:193-212: y = (x * inv_rms) * w, sequential F32 square sum. */
void orc_rms_norm(const float* input, size_t rows, size_t columns, const float* weights,
                  float epsilon, float* output) {
  for (size_t r = 0; r < rows; ++r) {
    const float* x = input + r * columns;
    float squares = 0.0f;
    for (size_t c = 0; c < columns; ++c) squares += x[c] * x[c];
    const float n = orc_planted_mistake == 5 ? (float)(columns - 1) : (float)columns;
    const float inverse = 1.0f / sqrtf(squares / n + epsilon);
    for (size_t c = 0; c < columns; ++c) output[r * columns + c] = x[c] * inverse * weights[c];
  }
}

typedef struct {
  const float* input;
  const float* weights;
  float* output;
  size_t rows, inner, outputs;
  size_t first_output, last_output;
} linear_job;

typedef float v4sf __attribute__((vector_size(16)));

/* Eight output columns and two rows at a time: the eight weight rows are interleaved into
 * [k][8] once per block, and each lane of the four-wide vectors carries one (row, column)
 * sum. Every sum is still the reference's sequential `sum += x * w` over the inner index
 * (one multiplication, then one addition, per lane and step; no fused multiply-add). */
static void* linear_worker(void* opaque) {
  const linear_job* job = (const linear_job*)opaque;
  const size_t n = job->inner;
  size_t o = job->first_output;
  v4sf* block = (v4sf*)aligned_alloc(16, n * 2 * sizeof(v4sf) + 16);
  for (; o + 8 <= job->last_output; o += 8) {
    for (size_t k = 0; k < n; ++k) {
      for (int c = 0; c < 4; ++c) {
        block[2 * k][c] = job->weights[(o + (size_t)c) * n + k];
        block[2 * k + 1][c] = job->weights[(o + 4 + (size_t)c) * n + k];
      }
    }
    size_t r = 0;
    for (; r + 2 <= job->rows; r += 2) {
      const float* x0 = job->input + r * n;
      const float* x1 = x0 + n;
      v4sf a0 = {0, 0, 0, 0}, a1 = {0, 0, 0, 0}, b0 = {0, 0, 0, 0}, b1 = {0, 0, 0, 0};
      for (size_t k = 0; k < n; ++k) {
        const v4sf w0 = block[2 * k], w1 = block[2 * k + 1];
        const v4sf u = {x0[k], x0[k], x0[k], x0[k]};
        const v4sf v = {x1[k], x1[k], x1[k], x1[k]};
        a0 += u * w0;
        a1 += u * w1;
        b0 += v * w0;
        b1 += v * w1;
      }
      float* y0 = job->output + r * job->outputs + o;
      float* y1 = y0 + job->outputs;
      for (int c = 0; c < 4; ++c) {
        y0[c] = a0[c];
        y0[4 + c] = a1[c];
        y1[c] = b0[c];
        y1[4 + c] = b1[c];
      }
    }
    for (; r < job->rows; ++r) {
      const float* x = job->input + r * n;
      v4sf a0 = {0, 0, 0, 0}, a1 = {0, 0, 0, 0};
      for (size_t k = 0; k < n; ++k) {
        const v4sf u = {x[k], x[k], x[k], x[k]};
        a0 += u * block[2 * k];
        a1 += u * block[2 * k + 1];
      }
      float* y = job->output + r * job->outputs + o;
      for (int c = 0; c < 4; ++c) {
        y[c] = a0[c];
        y[4 + c] = a1[c];
      }
    }
  }
  free(block);
  for (; o < job->last_output; ++o) {
    const float* w = job->weights + o * n;
    for (size_t r = 0; r < job->rows; ++r) {
      const float* x = job->input + r * n;
      float s = 0.0f;
      for (size_t k = 0; k < n; ++k) s += x[k] * w[k];
      job->output[r * job->outputs + o] = s;
    }
  }
  return NULL;
}

/* cpp/src/cpu/tensor.cpp:47-62: y[r][o] = sum_k x[r][k] * W[o][k], W is [out, in]. */
void orc_linear(const float* input, size_t rows, size_t inner, const float* weights,
                size_t outputs, float* output) {
  int threads = thread_count();
  const double work = (double)rows * (double)inner * (double)outputs;
  if (work < 4.0e6 || outputs < 64) threads = 1;
  if ((size_t)threads > outputs / 8) threads = (int)(outputs / 8 > 0 ? outputs / 8 : 1);
  linear_job jobs[64];
  pthread_t ids[64];
  if (threads > 64) threads = 64;
  const size_t per = ((outputs + (size_t)threads - 1) / (size_t)threads + 7) / 8 * 8;
  int launched = 0;
  for (int t = 0; t < threads; ++t) {
    size_t first = (size_t)t * per;
    if (first >= outputs) break;
    size_t last = first + per > outputs ? outputs : first + per;
    jobs[t] = (linear_job){input, weights, output, rows, inner, outputs, first, last};
    ++launched;
  }
  for (int t = 1; t < launched; ++t) pthread_create(&ids[t], NULL, linear_worker, &jobs[t]);
  if (launched > 0) linear_worker(&jobs[0]);
  for (int t = 1; t < launched; ++t) pthread_join(ids[t], NULL);
}

/* cpp/src/cpu/llama.cpp:114-130: per head, v *= (inv_rms * w); one weight vector for
 * all heads. */
void orc_normalize_heads(float* values, size_t count, const float* weights, size_t width,
                         float epsilon) {
  for (size_t offset = 0; offset < count; offset += width) {
    float squares = 0.0f;
    for (size_t d = 0; d < width; ++d) squares += values[offset + d] * values[offset + d];
    const float inverse = 1.0f / sqrtf(squares / (float)width + epsilon);
    for (size_t d = 0; d < width; ++d) values[offset + d] *= inverse * weights[d];
  }
}

/* cpp/src/cpu/llama.cpp:214-240: rotate-half RoPE, angle = pos / theta^(2i/D) in F32. */
int orc_apply_rope(float* values, size_t rows, size_t heads, size_t head_dimension,
                   size_t first_position, float theta) {
  if (heads == 0 || head_dimension == 0 || head_dimension % 2 != 0 || theta <= 0.0f) {
    return ORC_INVALID_REQUEST;
  }
  const size_t half = head_dimension / 2;
  const size_t width = heads * head_dimension;
  for (size_t t = 0; t < rows; ++t) {
    const float position = (float)(first_position + t);
    for (size_t h = 0; h < heads; ++h) {
      float* v = values + t * width + h * head_dimension;
      for (size_t i = 0; i < half; ++i) {
        const float exponent = (float)(2 * i) / (float)head_dimension;
        const float angle = position / powf(theta, exponent);
        const float c = cosf(angle);
        const float s = sinf(angle);
        const float a = v[i];
        const float b = v[half + i];
        if (orc_planted_mistake == 2) {
          v[i] = a * c + b * s;
          v[half + i] = b * c - a * s;
        } else {
          v[i] = a * c - b * s;
          v[half + i] = b * c + a * s;
        }
      }
    }
  }
  return ORC_OK;
}

int orc_kv_init(orc_kv_cache* cache, size_t capacity, size_t heads, size_t head_dimension) {
  memset(cache, 0, sizeof *cache);
  if (capacity == 0 || heads == 0 || head_dimension == 0) return ORC_INVALID_REQUEST;
  const size_t elements = capacity * heads * head_dimension;
  cache->keys = (float*)calloc(elements, sizeof(float));
  cache->values = (float*)calloc(elements, sizeof(float));
  if (!cache->keys || !cache->values) {
    orc_kv_free(cache);
    return ORC_RESOURCE_EXHAUSTED;
  }
  cache->capacity = capacity;
  cache->heads = heads;
  cache->head_dimension = head_dimension;
  return ORC_OK;
}

void orc_kv_free(orc_kv_cache* cache) {
  free(cache->keys);
  free(cache->values);
  cache->keys = cache->values = NULL;
  cache->length = cache->capacity = 0;
}

/* cpp/src/cpu/llama.cpp:170-191: appends must start at the current length. */
int orc_kv_append(orc_kv_cache* cache, size_t first_position, const float* keys,
                  const float* values, size_t rows) {
  if (first_position != cache->length) return ORC_INVALID_REQUEST;
  if (rows > cache->capacity - cache->length) return ORC_RESOURCE_EXHAUSTED;
  const size_t width = cache->heads * cache->head_dimension;
  memcpy(cache->keys + cache->length * width, keys, rows * width * sizeof(float));
  memcpy(cache->values + cache->length * width, values, rows * width * sizeof(float));
  cache->length += rows;
  return ORC_OK;
}

typedef struct {
  const float* queries;
  size_t rows;
  const orc_config* config;
  size_t first_position;
  const orc_kv_cache* cache;
  float* output;
} attention_job;

/* Attention of (row, query head) units [begin, end). Each unit's arithmetic is the
 * reference's: scores in key order, the running maximum, exp and the denominator in key
 * order, then every output dimension's sum over keys in key order with the probability
 * divided by the denominator inside the sum. The value loop visits keys in the outer loop
 * (every dimension's partial sum advances one key at a time), which keeps each dimension's
 * additions in the same order. */
static void attention_units(void* context, size_t begin, size_t end) {
  const attention_job* job = (const attention_job*)context;
  const orc_config* config = job->config;
  const size_t D = config->head_dimension;
  const size_t K = config->key_value_heads;
  const size_t Q = config->attention_heads;
  const size_t group = Q / K;
  const size_t width = Q * D;
  const float scale = 1.0f / sqrtf((float)D);
  float* scores = (float*)malloc((job->first_position + job->rows) * sizeof(float));
  float* sums = (float*)malloc(D * sizeof(float));
  for (size_t unit = begin; unit < end; ++unit) {
    const size_t t = unit / Q, qh = unit % Q;
    const size_t last = job->first_position + t - (orc_planted_mistake == 3 && job->first_position + t > 0);
    const size_t kvh = qh / group;
    const float* q = job->queries + t * width + qh * D;
    float maximum = -INFINITY;
    for (size_t p = 0; p <= last; ++p) {
      const float* k = job->cache->keys + (p * K + kvh) * D;
      float score = 0.0f;
      for (size_t d = 0; d < D; ++d) score += q[d] * k[d];
      score *= scale;
      scores[p] = score;
      if (maximum < score) maximum = score;
    }
    float denominator = 0.0f;
    for (size_t p = 0; p <= last; ++p) {
      scores[p] = expf(scores[p] - maximum);
      denominator += scores[p];
    }
    for (size_t d = 0; d < D; ++d) sums[d] = 0.0f;
    for (size_t p = 0; p <= last; ++p) {
      const float weight = scores[p] / denominator;
      const float* v = job->cache->values + (p * K + kvh) * D;
      for (size_t d = 0; d < D; ++d) sums[d] += weight * v[d];
    }
    float* out = job->output + t * width + qh * D;
    for (size_t d = 0; d < D; ++d) out[d] = sums[d];
  }
  free(sums);
  free(scores);
}

/* cpp/src/cpu/llama.cpp:67-112: causal GQA attention over the whole cache prefix;
 * probabilities are divided by the denominator inside the value sum. Units of (row, query
 * head) are independent, so they are spread over threads without changing any result. */
void orc_attention(const float* queries, size_t rows, const orc_config* config,
                   size_t first_position, const orc_kv_cache* cache, float* output) {
  attention_job job = {queries, rows, config, first_position, cache, output};
  const size_t units = rows * config->attention_heads;
  const double work = (double)units * (double)(first_position + rows) * (double)config->head_dimension;
  if (work < 4.0e6) {
    attention_units(&job, 0, units);
    return;
  }
  parallel_units(units, attention_units, &job);
}

/* cpp/src/cpu/llama.cpp:242-282: norm -> q,k,v -> QK-norm -> RoPE -> append ->
 * attention -> o -> +residual -> norm -> gate, up -> SiLU(g)*u -> down -> +residual. */
int orc_transformer_layer(const float* input, size_t rows, const orc_layer* layer,
                          const orc_config* config, size_t first_position,
                          orc_kv_cache* cache, float* output) {
  const size_t H = config->hidden_size;
  const size_t I = config->intermediate_size;
  const size_t D = config->head_dimension;
  const size_t qw = config->attention_heads * D;
  const size_t kw = config->key_value_heads * D;
  if (rows == 0 || first_position != cache->length || cache->heads != config->key_value_heads ||
      cache->head_dimension != D || first_position > config->maximum_sequence_length ||
      rows > config->maximum_sequence_length - first_position ||
      (config->query_key_norm != 0) != (layer->query_norm != NULL && layer->key_norm != NULL)) {
    return ORC_INVALID_REQUEST;
  }
  float* normalized = (float*)malloc(rows * H * sizeof(float));
  float* q = (float*)malloc(rows * qw * sizeof(float));
  float* k = (float*)malloc(rows * kw * sizeof(float));
  float* v = (float*)malloc(rows * kw * sizeof(float));
  float* attended = (float*)malloc(rows * qw * sizeof(float));
  float* gated = (float*)malloc(rows * I * sizeof(float));
  float* up = (float*)malloc(rows * I * sizeof(float));
  float* down = (float*)malloc(rows * H * sizeof(float));
  int status = ORC_OK;
  orc_rms_norm(input, rows, H, layer->input_norm, config->rms_norm_epsilon, normalized);
  orc_linear(normalized, rows, H, layer->query, qw, q);
  orc_linear(normalized, rows, H, layer->key, kw, k);
  orc_linear(normalized, rows, H, layer->value, kw, v);
  if (config->query_key_norm) {
    orc_normalize_heads(q, rows * qw, layer->query_norm, D, config->rms_norm_epsilon);
    orc_normalize_heads(k, rows * kw, layer->key_norm, D, config->rms_norm_epsilon);
  }
  orc_apply_rope(q, rows, config->attention_heads, D, first_position, config->rope_theta);
  orc_apply_rope(k, rows, config->key_value_heads, D, first_position, config->rope_theta);
  status = orc_kv_append(cache, first_position, k, v, rows);
  if (status == ORC_OK) {
    orc_attention(q, rows, config, first_position, cache, attended);
    orc_linear(attended, rows, qw, layer->attention_output, H, output);
    if (orc_planted_mistake != 1)
      for (size_t i = 0; i < rows * H; ++i) output[i] += input[i];
    orc_rms_norm(output, rows, H, layer->post_attention_norm, config->rms_norm_epsilon,
                 normalized);
    orc_linear(normalized, rows, H, layer->gate, I, gated);
    orc_linear(normalized, rows, H, layer->up, I, up);
    for (size_t i = 0; i < rows * I; ++i) {
      const float g = orc_planted_mistake == 4 ? up[i] : gated[i];
      gated[i] = (g / (1.0f + expf(-g))) * (orc_planted_mistake == 4 ? gated[i] : up[i]);
    }
    orc_linear(gated, rows, I, layer->down, H, down);
    for (size_t i = 0; i < rows * H; ++i) output[i] += down[i];
  }
  free(normalized);
  free(q);
  free(k);
  free(v);
  free(attended);
  free(gated);
  free(up);
  free(down);
  return status;
}

/* cpp/src/cpu/llama.cpp:284-288 */
void orc_final_logits(const float* hidden, size_t rows, size_t hidden_size,
                      const float* final_norm, const float* head, size_t vocabulary,
                      float epsilon, float* logits) {
  float* normalized = (float*)malloc(rows * hidden_size * sizeof(float));
  orc_rms_norm(hidden, rows, hidden_size, final_norm, epsilon, normalized);
  orc_linear(normalized, rows, hidden_size, head, vocabulary, logits);
  free(normalized);
}

/* cpp/src/cpu/llama.cpp:290-308 */
int orc_greedy_last(const float* logits, size_t rows, size_t columns, uint64_t* token) {
  if (rows == 0 || columns == 0) return ORC_INVALID_REQUEST;
  const float* row = logits + (rows - 1) * columns;
  for (size_t i = 0; i < columns; ++i) {
    if (!isfinite(row[i])) return ORC_INTERNAL;
  }
  size_t best = 0;
  for (size_t i = 1; i < columns; ++i) {
    if (row[i] > row[best]) best = i;
  }
  *token = best;
  return ORC_OK;
}

/* ------------------------------------------------------------------- sampling */

/* cpp/src/sampling.cpp:10-17 */
int orc_validate_sampling(double temperature, double top_p, uint32_t top_logprobs,
                          int return_logprobs) {
  if (!isfinite(temperature) || temperature < 0.0 || temperature > 100.0 || !isfinite(top_p) ||
      top_p <= 0.0 || top_p > 1.0 || top_logprobs > 5u ||
      (!return_logprobs && top_logprobs != 0u)) {
    return ORC_INVALID_REQUEST;
  }
  return ORC_OK;
}

typedef struct {
  double probability;
  uint64_t token;
} candidate;

/* Descending probability; equal probabilities by ascending token ID. */
static int by_probability(const void* left, const void* right) {
  const candidate* a = (const candidate*)left;
  const candidate* b = (const candidate*)right;
  if (a->probability == b->probability) return a->token < b->token ? -1 : (a->token > b->token);
  return a->probability > b->probability ? -1 : 1;
}

static size_t first_maximum(const float* logits, size_t count) {
  size_t best = 0;
  for (size_t i = 1; i < count; ++i) {
    if (logits[best] < logits[i]) best = i;
  }
  return best;
}

/* cpp/src/sampling.cpp:19-63 */
int orc_sample_logits(const float* logits, size_t count, double temperature, double top_p,
                      uint64_t top_k, uint64_t seed, uint64_t generated_index,
                      uint64_t* token) {
  if (orc_validate_sampling(temperature, top_p, 0u, 0) != ORC_OK) return ORC_INVALID_REQUEST;
  if (count == 0) return ORC_INTERNAL;
  for (size_t i = 0; i < count; ++i) {
    if (!isfinite(logits[i])) return ORC_INTERNAL;
  }
  const size_t best = first_maximum(logits, count);
  if (temperature == 0.0) {
    *token = best;
    return ORC_OK;
  }
  candidate* pool = (candidate*)malloc(count * sizeof(candidate));
  if (!pool) return ORC_RESOURCE_EXHAUSTED;
  const double maximum = (double)logits[best];
  for (size_t i = 0; i < count; ++i) {
    pool[i].probability = exp(((double)logits[i] - maximum) / temperature);
    pool[i].token = i;
  }
  qsort(pool, count, sizeof(candidate), by_probability);
  size_t kept = count;
  if (top_k != 0 && top_k < kept) kept = (size_t)top_k;
  double total = 0.0;
  for (size_t i = 0; i < kept; ++i) total += pool[i].probability;
  const double threshold = total * top_p;
  double retained = 0.0;
  size_t taken = 0;
  do {
    retained += pool[taken++].probability;
  } while (retained < threshold && taken < kept);
  const uint64_t bits = orc_splitmix64(seed + 0x9e3779b97f4a7c15ull * generated_index);
  double target = (double)(bits >> 11) * 0x1.0p-53 * retained;
  uint64_t chosen = pool[taken - 1].token;
  for (size_t i = 0; i + 1 < taken; ++i) {
    target -= pool[i].probability;
    if (target < 0.0) {
      chosen = pool[i].token;
      break;
    }
  }
  free(pool);
  *token = chosen;
  return ORC_OK;
}

typedef struct {
  uint64_t token;
  double logprob;
} ranked;

static int by_logprob(const void* left, const void* right) {
  const ranked* a = (const ranked*)left;
  const ranked* b = (const ranked*)right;
  if (a->logprob == b->logprob) return a->token < b->token ? -1 : (a->token > b->token);
  return a->logprob > b->logprob ? -1 : 1;
}

/* cpp/src/sampling.cpp:65-89 */
int orc_sample_token(const float* logits, size_t count, double temperature, double top_p,
                     uint64_t top_k, uint64_t seed, uint64_t generated_index,
                     int return_logprobs, uint32_t top_logprobs, uint64_t* token,
                     double* logprob, uint64_t* top_ids, double* top_values) {
  if (orc_validate_sampling(temperature, top_p, top_logprobs, return_logprobs) != ORC_OK) {
    return ORC_INVALID_REQUEST;
  }
  int status = orc_sample_logits(logits, count, temperature, top_p, top_k, seed,
                                 generated_index, token);
  if (status != ORC_OK || !return_logprobs) return status;
  const double maximum = (double)logits[first_maximum(logits, count)];
  double sum = 0.0;
  for (size_t i = 0; i < count; ++i) sum += exp((double)logits[i] - maximum);
  const double log_sum = log(sum);
  *logprob = (double)logits[*token] - maximum - log_sum;
  if (top_logprobs) {
    ranked* all = (ranked*)malloc(count * sizeof(ranked));
    if (!all) return ORC_RESOURCE_EXHAUSTED;
    for (size_t i = 0; i < count; ++i) {
      all[i].token = i;
      all[i].logprob = (double)logits[i] - maximum - log_sum;
    }
    qsort(all, count, sizeof(ranked), by_logprob);
    const size_t n = top_logprobs < count ? top_logprobs : count;
    for (size_t i = 0; i < n; ++i) {
      top_ids[i] = all[i].token;
      top_values[i] = all[i].logprob;
    }
    free(all);
  }
  return ORC_OK;
}

/* ------------------------------------------------------------------- packing */

int orc_pack(size_t items, const uint32_t* sequence_slots, const uint64_t* first_positions,
             const uint32_t* query_lengths, const int32_t* block_table, size_t table_width,
             size_t block_size, uint32_t* cu_seqlens, uint32_t* row_items,
             uint64_t* row_positions, int64_t* row_slots) {
  if (block_size == 0) return ORC_INVALID_REQUEST;
  uint32_t offset = 0;
  for (size_t i = 0; i < items; ++i) {
    cu_seqlens[i] = offset;
    for (uint32_t j = 0; j < query_lengths[i]; ++j) {
      const uint64_t position = first_positions[i] + j;
      const size_t logical = (size_t)(position / block_size);
      if (logical >= table_width) return ORC_INVALID_REQUEST;
      const int32_t physical = block_table[sequence_slots[i] * table_width + logical];
      if (physical < 0) return ORC_INVALID_REQUEST;
      row_items[offset + j] = (uint32_t)i;
      row_positions[offset + j] = position;
      row_slots[offset + j] = (int64_t)physical * (int64_t)block_size +
                              (int64_t)(position % block_size);
    }
    offset += query_lengths[i];
  }
  cu_seqlens[items] = offset;
  return ORC_OK;
}

/* ------------------------------------------------------------ synthetic weights */

uint64_t orc_splitmix64(uint64_t state) {
  uint64_t z = state + 0x9e3779b97f4a7c15ull;
  z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ull;
  z = (z ^ (z >> 27)) * 0x94d049bb133111ebull;
  return z ^ (z >> 31);
}

static float irwin_hall_normal(uint64_t seed, uint64_t tensor_id, uint64_t index) {
  const uint64_t base = (tensor_id << 40) + 3u * index;
  int32_t sum = 0;
  for (uint64_t j = 0; j < 3; ++j) {
    const uint64_t bits = orc_splitmix64(seed + 0x9e3779b97f4a7c15ull * (base + j));
    sum += (int32_t)(bits & 0xffffu) + (int32_t)((bits >> 16) & 0xffffu) +
           (int32_t)((bits >> 32) & 0xffffu) + (int32_t)(bits >> 48);
  }
  return (float)(sum + 6 - 6 * 65536) / 65536.0f;
}

/* Each element depends only on (seed, tensor, index): ranges are generated in parallel. */
typedef struct {
  uint64_t seed, tensor_id, first;
  float mean, sigma;
  void* out;
} synth_job;

static void synth_f32_range(void* context, size_t begin, size_t end) {
  const synth_job* j = (const synth_job*)context;
  float* out = (float*)j->out;
  for (size_t i = begin; i < end; ++i) {
    const float scaled = irwin_hall_normal(j->seed, j->tensor_id, j->first + i) * j->sigma;
    out[i] = j->mean + scaled;
  }
}

static void synth_f16_range(void* context, size_t begin, size_t end) {
  const synth_job* j = (const synth_job*)context;
  uint16_t* out = (uint16_t*)j->out;
  for (size_t i = begin; i < end; ++i) {
    const float scaled = irwin_hall_normal(j->seed, j->tensor_id, j->first + i) * j->sigma;
    out[i] = orc_f16_from_f32(j->mean + scaled);
  }
}

void orc_synth_f32(uint64_t seed, uint64_t tensor_id, uint64_t first, size_t count,
                   float mean, float sigma, float* out) {
  synth_job j = {seed, tensor_id, first, mean, sigma, out};
  parallel_elements(count, synth_f32_range, &j);
}

void orc_synth_f16(uint64_t seed, uint64_t tensor_id, uint64_t first, size_t count,
                   float mean, float sigma, uint16_t* out) {
  synth_job j = {seed, tensor_id, first, mean, sigma, out};
  parallel_elements(count, synth_f16_range, &j);
}
