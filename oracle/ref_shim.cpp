// C entry points over the reference CPU worker's own arithmetic, compiled from the
// reference sources in place (oracle/Makefile, target `ref`): cpp/src/cpu/llama.cpp,
// cpp/src/cpu/tensor.cpp, cpp/src/half.cpp, cpp/src/sampling.cpp,
// cpp/src/decode_batch.cpp. TEST INFRASTRUCTURE ONLY: used to pin the plain-C oracle
// bit for bit and as the reported CPU baseline. Never linked into the product.
#include <atomic>
#include <cstdint>
#include <cstring>
#include <exception>
#include <memory>
#include <vector>

#include "hllm/cpu/llama.hpp"
#include "hllm/runtime/error.hpp"
#include "hllm/runtime/half.hpp"
#include "hllm/runtime/sampling.hpp"
#include "hllm/runtime/stage_backend.hpp"

namespace {
using hllm::cpu::LayerKvCache;
using hllm::cpu::LayerWeights;
using hllm::cpu::LlamaConfig;
using hllm::cpu::Matrix;

struct RefConfig {
  std::size_t hidden_size, intermediate_size, attention_heads, key_value_heads, head_dimension,
      maximum_sequence_length;
  float rms_norm_epsilon, rope_theta;
  int query_key_norm;
};

LlamaConfig to_config(const RefConfig* c) {
  return {c->hidden_size,     c->intermediate_size,       c->attention_heads,
          c->key_value_heads, c->head_dimension,          c->maximum_sequence_length,
          c->rms_norm_epsilon, c->rope_theta,             c->query_key_norm != 0};
}

Matrix matrix(const float* data, std::size_t rows, std::size_t columns) {
  return Matrix(rows, columns, std::vector<float>(data, data + rows * columns));
}

std::vector<float> vec(const float* data, std::size_t n) {
  return data ? std::vector<float>(data, data + n) : std::vector<float>{};
}

int status_of(const std::exception& error) {
  if (const auto* e = dynamic_cast<const hllm::runtime::Error*>(&error)) {
    return static_cast<int>(e->code()) + 1;
  }
  return 7;  // any other std::exception (std::invalid_argument, std::length_error, ...)
}

// One layer's weights copied into the reference's types once.
struct RefLayer {
  LayerWeights weights;
};
}  // namespace

extern "C" {

float ref_f32_from_f16(std::uint16_t bits) { return hllm::runtime::float16_to_float(bits); }
std::uint16_t ref_f16_from_f32(float v) { return hllm::runtime::float_to_float16(v); }
float ref_f32_from_bf16(std::uint16_t bits) { return hllm::runtime::bfloat16_to_float(bits); }
std::uint16_t ref_bf16_from_f32(float v) { return hllm::runtime::float_to_bfloat16(v); }

void* ref_layer_create(const RefConfig* c, const float* input_norm, const float* query,
                       const float* key, const float* value, const float* attention_output,
                       const float* post_attention_norm, const float* gate, const float* up,
                       const float* down, const float* query_norm, const float* key_norm) {
  const auto H = c->hidden_size, I = c->intermediate_size, D = c->head_dimension;
  const auto qw = c->attention_heads * D, kw = c->key_value_heads * D;
  auto* layer = new RefLayer{LayerWeights{vec(input_norm, H),
                                          matrix(query, qw, H),
                                          matrix(key, kw, H),
                                          matrix(value, kw, H),
                                          matrix(attention_output, H, qw),
                                          vec(post_attention_norm, H),
                                          matrix(gate, I, H),
                                          matrix(up, I, H),
                                          matrix(down, H, I),
                                          vec(query_norm, D),
                                          vec(key_norm, D)}};
  return layer;
}

void ref_layer_destroy(void* layer) { delete static_cast<RefLayer*>(layer); }

void* ref_cache_create(std::size_t capacity, std::size_t heads, std::size_t head_dimension) {
  try {
    return new LayerKvCache(capacity, heads, head_dimension);
  } catch (...) {
    return nullptr;
  }
}
void ref_cache_destroy(void* cache) { delete static_cast<LayerKvCache*>(cache); }
std::size_t ref_cache_length(const void* cache) {
  return static_cast<const LayerKvCache*>(cache)->length();
}
// Copies the cache prefix in (pos, head, dim) order.
void ref_cache_read(const void* opaque, float* keys, float* values) {
  const auto* cache = static_cast<const LayerKvCache*>(opaque);
  std::size_t i = 0;
  for (std::size_t p = 0; p < cache->length(); ++p)
    for (std::size_t h = 0; h < cache->heads(); ++h)
      for (std::size_t d = 0; d < cache->head_dimension(); ++d, ++i) {
        keys[i] = cache->key(p, h, d);
        values[i] = cache->value(p, h, d);
      }
}

// LayerKvCache::append with given K/V rows (positions first_position..+rows).
int ref_cache_append(void* cache, std::size_t first_position, const float* keys,
                     const float* values, std::size_t rows, std::size_t width) {
  try {
    static_cast<LayerKvCache*>(cache)->append(first_position, matrix(keys, rows, width),
                                              matrix(values, rows, width));
    return 0;
  } catch (const std::exception& e) {
    return status_of(e);
  }
}

int ref_transformer_layer(const RefConfig* c, const void* layer, const float* input,
                          std::size_t rows, std::size_t first_position, void* cache,
                          float* output) {
  try {
    const auto out = hllm::cpu::transformer_layer(
        matrix(input, rows, c->hidden_size), static_cast<const RefLayer*>(layer)->weights,
        to_config(c), first_position, *static_cast<LayerKvCache*>(cache));
    std::memcpy(output, out.values().data(), out.size() * sizeof(float));
    return 0;
  } catch (const std::exception& e) {
    return status_of(e);
  }
}

int ref_rms_norm(const float* input, std::size_t rows, std::size_t columns,
                 const float* weights, float epsilon, float* output) {
  try {
    const auto out = hllm::cpu::rms_norm(matrix(input, rows, columns),
                                         std::vector<float>(weights, weights + columns), epsilon);
    std::memcpy(output, out.values().data(), out.size() * sizeof(float));
    return 0;
  } catch (const std::exception& e) {
    return status_of(e);
  }
}

int ref_apply_rope(float* values, std::size_t rows, std::size_t heads, std::size_t head_dimension,
                   std::size_t first_position, float theta) {
  try {
    auto m = matrix(values, rows, heads * head_dimension);
    hllm::cpu::apply_rope(m, heads, head_dimension, first_position, theta);
    std::memcpy(values, m.values().data(), m.size() * sizeof(float));
    return 0;
  } catch (const std::exception& e) {
    return status_of(e);
  }
}

int ref_linear(const float* input, std::size_t rows, std::size_t inner, const float* weights,
               std::size_t outputs, float* output) {
  try {
    const auto out = hllm::cpu::linear(matrix(input, rows, inner), matrix(weights, outputs, inner));
    std::memcpy(output, out.values().data(), out.size() * sizeof(float));
    return 0;
  } catch (const std::exception& e) {
    return status_of(e);
  }
}

int ref_final_logits(const float* hidden, std::size_t rows, std::size_t hidden_size,
                     const float* final_norm, const float* head, std::size_t vocabulary,
                     float epsilon, float* logits) {
  try {
    const auto out = hllm::cpu::final_logits(
        matrix(hidden, rows, hidden_size),
        std::vector<float>(final_norm, final_norm + hidden_size),
        matrix(head, vocabulary, hidden_size), epsilon);
    std::memcpy(logits, out.values().data(), out.size() * sizeof(float));
    return 0;
  } catch (const std::exception& e) {
    return status_of(e);
  }
}

int ref_greedy_last(const float* logits, std::size_t rows, std::size_t columns,
                    std::uint64_t* token) {
  try {
    *token = hllm::cpu::greedy_sample_last(matrix(logits, rows, columns));
    return 0;
  } catch (const std::exception& e) {
    return status_of(e);
  }
}

int ref_sample_token(const float* logits, std::size_t count, double temperature, double top_p,
                     std::uint64_t top_k, std::uint64_t seed, std::uint64_t generated_index,
                     int return_logprobs, std::uint32_t top_logprobs, std::uint64_t* token,
                     double* logprob, std::uint64_t* top_ids, double* top_values) {
  try {
    hllm::runtime::SamplingOptions options{temperature, top_p, top_k, seed,
                                           return_logprobs != 0, top_logprobs};
    const auto result = hllm::runtime::sample_token(std::span<const float>(logits, count),
                                                    options, generated_index);
    *token = result.id;
    if (result.logprob) *logprob = *result.logprob;
    for (std::size_t i = 0; i < result.top_logprobs.size(); ++i) {
      top_ids[i] = result.top_logprobs[i].token_id;
      top_values[i] = result.top_logprobs[i].logprob;
    }
    return 0;
  } catch (const std::exception& e) {
    return status_of(e);
  }
}

// cpp/src/decode_batch.cpp: combine one-token inputs of `items` sequences; returns the
// packed IDs in item order, or an error status.
int ref_combine_decode_tokens(std::size_t items, const std::uint64_t* ids,
                              const std::size_t* positions, const int* prefilling,
                              const int* duplicate_of, std::uint64_t* packed) {
  try {
    std::vector<std::unique_ptr<hllm::runtime::SequenceState>> states;
    std::atomic_bool cancelled{false};
    std::vector<hllm::runtime::DecodeBatchItem> batch;
    for (std::size_t i = 0; i < items; ++i) {
      states.push_back(std::make_unique<hllm::runtime::SequenceState>());
      states.back()->prefilling = prefilling[i] != 0;
    }
    for (std::size_t i = 0; i < items; ++i) {
      auto* state = duplicate_of[i] >= 0 ? states[static_cast<std::size_t>(duplicate_of[i])].get()
                                         : states[i].get();
      batch.push_back({hllm::runtime::TokenInput{{ids[i]}}, positions[i], state, &cancelled});
    }
    const auto combined = hllm::runtime::combine_decode_inputs(batch);
    const auto& tokens = std::get<hllm::runtime::TokenInput>(combined);
    for (std::size_t i = 0; i < tokens.ids.size(); ++i) packed[i] = tokens.ids[i];
    return 0;
  } catch (const std::exception& e) {
    return status_of(e);
  }
}
}
