// Stage admission for dense checkpoints (cpp/src/model/dense_loader.cpp:23-245,
// cpp/include/hllm/model/dense_source.hpp): the load request's plan and manifest are
// checked against the supported architectures and configuration, the stage's tensor
// ownership, every expected tensor's role / shape / file, and the Safetensors metadata of
// each file, before any weight is read. The request types restate the control-plane
// messages (proto/control.proto LoadStageRequest, proto/model.proto ModelManifest,
// proto/placement.proto DeploymentPlan) as plain structs.
#pragma once

#include <cstdint>
#include <filesystem>
#include <map>
#include <optional>
#include <string>
#include <vector>

#include "safetensors.hpp"

namespace hllm_rocm::model {

enum class WireDType { kUnspecified, kF32, kF16, kBF16 };
enum class TensorRole { kUnspecified, kTokenEmbedding, kTransformerLayer, kFinalNorm, kLmHead };

struct TensorRecord {
  std::string name, file;
  WireDType dtype{WireDType::kUnspecified};
  std::vector<std::size_t> shape;
  std::size_t data_offset{0}, byte_length{0};
  TensorRole role{TensorRole::kUnspecified};
  std::optional<std::uint32_t> layer_index;
};
struct ArchitectureDescriptor {
  std::string architecture_id, architecture_revision;
  std::vector<std::string> feature_flags;
};
struct ModelConfig {
  std::size_t hidden_size{0}, intermediate_size{0};
  std::uint32_t num_layers{0}, num_attention_heads{0}, num_kv_heads{0}, head_dim{0};
  std::size_t vocabulary_size{0}, maximum_sequence_length{0};
  bool tied_embeddings{false};
  double rms_norm_eps{0.0}, rope_theta{0.0};
  bool has_rope_scaling{false};
  std::string hidden_activation;
  bool attention_bias{false}, mlp_bias{false};
};
struct ModelManifest {
  ArchitectureDescriptor architecture;
  ModelConfig config;
  std::vector<TensorRecord> tensors;
};
struct StageAssignment {
  std::uint32_t layer_start{0}, layer_end{0};
  bool owns_token_embedding{false}, owns_final_norm{false}, owns_lm_head{false}, owns_sampling{false};
};
struct DeploymentPlan {
  std::uint32_t schema_major{1}, schema_minor{1};
  WireDType execution_dtype{WireDType::kF16};
  std::optional<WireDType> weight_dtype;  // mixed residency (schema 1.2): F16 weights, F32 execution
  std::vector<StageAssignment> stages;
};
struct LoadStageRequest {
  DeploymentPlan plan;
  std::uint32_t stage_index{0};
  ModelManifest manifest;
};

struct DenseConfig {
  std::size_t hidden_size, intermediate_size, attention_heads, key_value_heads, head_dimension,
      maximum_sequence_length;
  float rms_norm_epsilon, rope_theta;
  bool query_key_norm;
};
struct TensorSource {
  std::string file;
  std::vector<std::size_t> shape;
  runtime::DataType dtype;
};
struct DenseSource {
  DenseConfig config{};
  std::size_t vocabulary_size{0};
  bool first{false}, final{false}, tied_head{false};
  std::uint32_t layer_start{0}, layer_end{0};
  runtime::DataType execution_dtype{runtime::DataType::kF16}, weight_dtype{runtime::DataType::kF16};
  std::map<std::string, TensorSource> tensors;
  std::map<std::string, runtime::SafetensorsFile> files;
  std::size_t resident_bytes{0};       // weights as the stage holds them
  std::size_t largest_payload_bytes{0};
};

// Validates the request against `root` (files must lie directly in it) and opens every
// Safetensors file it needs; throws runtime::Error (INCOMPATIBLE_WORKER) on any mismatch.
DenseSource inspect_dense_stage(const LoadStageRequest& request, const std::filesystem::path& root);

// A manifest for a Hugging Face style checkpoint directory: config.json (Llama / Qwen3)
// plus the *.safetensors files in it, with roles and layer indices from the tensor names.
ModelManifest manifest_from_checkpoint(const std::filesystem::path& root);

}  // namespace hllm_rocm::model
