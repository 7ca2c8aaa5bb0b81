#include "dense_loader.hpp"

#include <algorithm>
#include <cmath>
#include <fstream>
#include <set>
#include <sstream>

#include "json.hpp"

namespace hllm_rocm::model {

using runtime::Error;

namespace {

struct Expected {
  std::vector<std::size_t> shape;
  TensorRole role;
  int layer;  // -1 for non-layer tensors
};

std::size_t mul(std::size_t a, std::size_t b) {
  if (b != 0 && a > SIZE_MAX / b) throw Error::resource_exhausted("size overflow");
  return a * b;
}

runtime::DataType storage_type(WireDType d) {
  return d == WireDType::kF16 ? runtime::DataType::kF16
                              : d == WireDType::kBF16 ? runtime::DataType::kBF16 : runtime::DataType::kF32;
}

WireDType wire_type(runtime::DataType d) {
  switch (d) {
    case runtime::DataType::kF32: return WireDType::kF32;
    case runtime::DataType::kF16: return WireDType::kF16;
    case runtime::DataType::kBF16: return WireDType::kBF16;
    default: return WireDType::kUnspecified;
  }
}

// A file name with no directory part, resolving to a file directly inside `root`.
bool confined(const std::filesystem::path& root, const std::string& file) {
  const std::filesystem::path rel(file);
  if (rel.empty() || rel.is_absolute() || rel.has_parent_path() || rel == "." || rel == "..") return false;
  std::error_code ec;
  const auto target = std::filesystem::canonical(root / rel, ec);
  if (ec) return false;
  const auto base = std::filesystem::canonical(root, ec);
  return !ec && target.parent_path() == base;
}

}  // namespace

DenseSource inspect_dense_stage(const LoadStageRequest& request, const std::filesystem::path& root) {
  const DeploymentPlan& plan = request.plan;
  if (request.stage_index >= plan.stages.size() ||
      (plan.execution_dtype != WireDType::kF32 && plan.execution_dtype != WireDType::kF16))
    throw Error::incompatible_worker("invalid stage index or unsupported execution dtype");
  const bool mixed = plan.weight_dtype.has_value();
  if (mixed != (plan.schema_major == 1 && plan.schema_minor == 2) ||
      (mixed && (*plan.weight_dtype != WireDType::kF16 || plan.execution_dtype != WireDType::kF32)))
    throw Error::incompatible_worker("unsupported resident/execution precision contract");

  const ModelManifest& manifest = request.manifest;
  const ArchitectureDescriptor& arch = manifest.architecture;
  const bool known = arch.architecture_id == "llama.v1" || arch.architecture_id == "qwen3.v1";
  if (!known || arch.architecture_revision != "1")
    throw Error::incompatible_worker("unsupported architecture ID or revision");
  const bool qwen = arch.architecture_id == "qwen3.v1";
  static const std::set<std::string> kFeatures{"gqa", "mha", "tied_embeddings", "untied_embeddings",
                                               "explicit_head_dim"};
  bool qk_norm = false;
  for (const std::string& f : arch.feature_flags) {
    if (qwen && f == "qk_norm")
      qk_norm = true;
    else if (!kFeatures.count(f))
      throw Error::incompatible_worker("unsupported architecture feature: " + f);
  }
  if (qwen && !qk_norm) throw Error::incompatible_worker("Qwen3 requires qk_norm feature");

  const ModelConfig& c = manifest.config;
  const bool shape_ok = c.hidden_size && c.intermediate_size && c.num_layers && c.num_attention_heads &&
                        c.num_kv_heads && c.head_dim && c.head_dim % 2 == 0 &&
                        c.num_attention_heads % c.num_kv_heads == 0 && c.maximum_sequence_length &&
                        c.vocabulary_size;
  const bool math_ok = c.hidden_activation == "silu" && !c.attention_bias && !c.mlp_bias && !c.has_rope_scaling &&
                       std::isfinite(c.rms_norm_eps) && c.rms_norm_eps > 0 && std::isfinite(c.rope_theta) &&
                       c.rope_theta > 0 && std::isfinite(static_cast<float>(c.rope_theta)) &&
                       std::isfinite(static_cast<float>(c.rms_norm_eps)) && static_cast<float>(c.rms_norm_eps) > 0;
  if (!shape_ok || !math_ok) throw Error::incompatible_worker("unsupported dense model configuration");

  const StageAssignment& stage = plan.stages[request.stage_index];
  const std::size_t per_layer = qwen ? 11 : 9;
  if (stage.layer_start >= stage.layer_end || stage.layer_end > c.num_layers ||
      stage.layer_end - stage.layer_start > manifest.tensors.size() / per_layer)
    throw Error::incompatible_worker("layer range exceeds available tensor records");
  const bool first = request.stage_index == 0;
  const bool final = request.stage_index + 1 == plan.stages.size();
  if (stage.owns_token_embedding != first || stage.owns_sampling != final || stage.owns_final_norm != final ||
      stage.owns_lm_head != final)
    throw Error::incompatible_worker("inconsistent stage tensor ownership");

  DenseSource src;
  src.config = {c.hidden_size,
                c.intermediate_size,
                c.num_attention_heads,
                c.num_kv_heads,
                c.head_dim,
                c.maximum_sequence_length,
                static_cast<float>(c.rms_norm_eps),
                static_cast<float>(c.rope_theta),
                qwen};
  src.vocabulary_size = c.vocabulary_size;
  src.first = first;
  src.final = final;
  src.layer_start = stage.layer_start;
  src.layer_end = stage.layer_end;
  src.tied_head = stage.owns_lm_head && c.tied_embeddings;
  src.execution_dtype = storage_type(plan.execution_dtype);
  src.weight_dtype = mixed ? runtime::DataType::kF16 : src.execution_dtype;

  const std::size_t H = c.hidden_size, I = c.intermediate_size;
  const std::size_t QD = mul(c.num_attention_heads, c.head_dim), KD = mul(c.num_kv_heads, c.head_dim);
  std::map<std::string, Expected> expected;
  if (stage.owns_token_embedding || src.tied_head)
    expected["model.embed_tokens.weight"] = {{c.vocabulary_size, H}, TensorRole::kTokenEmbedding, -1};
  if (stage.owns_final_norm) expected["model.norm.weight"] = {{H}, TensorRole::kFinalNorm, -1};
  if (stage.owns_lm_head && !c.tied_embeddings)
    expected["lm_head.weight"] = {{c.vocabulary_size, H}, TensorRole::kLmHead, -1};
  for (std::uint32_t l = stage.layer_start; l < stage.layer_end; ++l) {
    const std::string p = "model.layers." + std::to_string(l) + ".";
    const int li = static_cast<int>(l);
    const std::pair<const char*, std::vector<std::size_t>> shapes[] = {
        {"input_layernorm.weight", {H}},      {"post_attention_layernorm.weight", {H}},
        {"self_attn.q_proj.weight", {QD, H}}, {"self_attn.k_proj.weight", {KD, H}},
        {"self_attn.v_proj.weight", {KD, H}}, {"self_attn.o_proj.weight", {H, QD}},
        {"mlp.gate_proj.weight", {I, H}},     {"mlp.up_proj.weight", {I, H}},
        {"mlp.down_proj.weight", {H, I}}};
    for (const auto& [n, s] : shapes) expected[p + n] = {s, TensorRole::kTransformerLayer, li};
    if (qwen) {
      expected[p + "self_attn.q_norm.weight"] = {{c.head_dim}, TensorRole::kTransformerLayer, li};
      expected[p + "self_attn.k_norm.weight"] = {{c.head_dim}, TensorRole::kTransformerLayer, li};
    }
  }

  std::map<std::string, const TensorRecord*> records;
  for (const TensorRecord& r : manifest.tensors)
    if (!records.emplace(r.name, &r).second) throw Error::incompatible_worker("duplicate tensor in manifest");
  // A serialized head beside tied embeddings is checked against the embedding, never held.
  const bool redundant_head = src.tied_head && records.count("lm_head.weight");
  if (redundant_head) expected["lm_head.weight"] = {{c.vocabulary_size, H}, TensorRole::kLmHead, -1};
  for (const auto& [name, r] : records) {
    const bool owned =
        (r->role == TensorRole::kTransformerLayer && r->layer_index && *r->layer_index >= stage.layer_start &&
         *r->layer_index < stage.layer_end) ||
        (r->role == TensorRole::kTokenEmbedding && stage.owns_token_embedding) ||
        (r->role == TensorRole::kFinalNorm && stage.owns_final_norm) ||
        (r->role == TensorRole::kLmHead && stage.owns_lm_head && !c.tied_embeddings);
    if (owned && !expected.count(name)) throw Error::incompatible_worker("unsupported selected tensor: " + name);
  }

  const std::size_t resident_element = src.weight_dtype == runtime::DataType::kF32 ? 4 : 2;
  for (const auto& [name, want] : expected) {
    const auto hit = records.find(name);
    if (hit == records.end()) throw Error::incompatible_worker("missing required tensor: " + name);
    const TensorRecord& r = *hit->second;
    const bool layer_ok = want.layer >= 0 ? (r.layer_index && *r.layer_index == static_cast<std::uint32_t>(want.layer))
                                          : !r.layer_index.has_value();
    if (r.role != want.role || !layer_ok || r.shape != want.shape)
      throw Error::incompatible_worker("incorrect tensor shape or ownership: " + name);
    if (!confined(root, r.file)) throw Error::incompatible_worker("tensor path escapes model root");
    auto file = src.files.find(r.file);
    if (file == src.files.end()) file = src.files.emplace(r.file, runtime::SafetensorsFile(root / r.file)).first;
    const runtime::TensorMetadata& meta = file->second.tensor(name);
    const WireDType stored = wire_type(meta.dtype);
    if (stored == WireDType::kUnspecified || r.dtype != stored || meta.shape != want.shape ||
        meta.data_offset != r.data_offset || meta.byte_length != r.byte_length)
      throw Error::incompatible_worker("Safetensors metadata mismatch or unsupported dtype: " + name);
    if (redundant_head && name == "lm_head.weight") continue;
    std::size_t elements = 1;
    for (std::size_t d : want.shape) elements = mul(elements, d);
    src.resident_bytes += mul(elements, want.shape.size() == 1 ? 4 : resident_element);
    src.largest_payload_bytes = std::max(src.largest_payload_bytes, meta.byte_length);
    src.tensors.emplace(name, TensorSource{r.file, want.shape, meta.dtype});
  }
  if (redundant_head) {
    const auto& emb = src.files.at(records.at("model.embed_tokens.weight")->file).tensor("model.embed_tokens.weight");
    const auto& head = src.files.at(records.at("lm_head.weight")->file).tensor("lm_head.weight");
    if (emb.dtype != head.dtype || emb.shape != head.shape || emb.byte_length != head.byte_length)
      throw Error::incompatible_worker("redundant tied head must match embedding storage metadata");
  }
  return src;
}

namespace {

std::uint64_t get_uint(const json::Value& cfg, const char* key, bool required = true, std::uint64_t fallback = 0) {
  const json::Value* v = cfg.find(key);
  if (!v || v->is_null()) {
    if (required) throw Error::incompatible_worker(std::string("config.json lacks ") + key);
    return fallback;
  }
  if (!v->is_number() || !v->is_unsigned) throw Error::incompatible_worker(std::string("config.json has invalid ") + key);
  return v->unsigned_value;
}

double get_number(const json::Value& cfg, const char* key, double fallback) {
  const json::Value* v = cfg.find(key);
  if (!v || v->is_null()) return fallback;
  if (!v->is_number()) throw Error::incompatible_worker(std::string("config.json has invalid ") + key);
  return v->number;
}

bool get_bool(const json::Value& cfg, const char* key, bool fallback) {
  const json::Value* v = cfg.find(key);
  if (!v || v->is_null()) return fallback;
  if (!v->is_bool()) throw Error::incompatible_worker(std::string("config.json has invalid ") + key);
  return v->boolean;
}

}  // namespace

ModelManifest manifest_from_checkpoint(const std::filesystem::path& root) {
  std::ifstream in(root / "config.json");
  if (!in) throw Error::incompatible_worker("checkpoint has no config.json");
  std::stringstream text;
  text << in.rdbuf();
  json::Value cfg;
  try {
    cfg = json::parse(text.str());
  } catch (const json::ParseError& e) {
    throw Error::incompatible_worker(std::string("config.json: ") + e.what());
  }
  const json::Value* type = cfg.find("model_type");
  if (!cfg.is_object() || !type || !type->is_string()) throw Error::incompatible_worker("config.json lacks model_type");
  ModelManifest m;
  const bool qwen = type->string == "qwen3";
  if (!qwen && type->string != "llama") throw Error::incompatible_worker("unsupported model_type " + type->string);
  m.architecture.architecture_id = qwen ? "qwen3.v1" : "llama.v1";
  m.architecture.architecture_revision = "1";
  ModelConfig& c = m.config;
  c.hidden_size = get_uint(cfg, "hidden_size");
  c.intermediate_size = get_uint(cfg, "intermediate_size");
  c.num_layers = static_cast<std::uint32_t>(get_uint(cfg, "num_hidden_layers"));
  c.num_attention_heads = static_cast<std::uint32_t>(get_uint(cfg, "num_attention_heads"));
  c.num_kv_heads = static_cast<std::uint32_t>(get_uint(cfg, "num_key_value_heads", false, c.num_attention_heads));
  const bool explicit_head = cfg.find("head_dim") && !cfg.find("head_dim")->is_null();
  c.head_dim = static_cast<std::uint32_t>(
      get_uint(cfg, "head_dim", false, c.num_attention_heads ? c.hidden_size / c.num_attention_heads : 0));
  c.vocabulary_size = get_uint(cfg, "vocab_size");
  c.maximum_sequence_length = get_uint(cfg, "max_position_embeddings");
  c.tied_embeddings = get_bool(cfg, "tie_word_embeddings", false);
  c.rms_norm_eps = get_number(cfg, "rms_norm_eps", 1e-6);
  c.rope_theta = get_number(cfg, "rope_theta", 10000.0);
  const json::Value* scaling = cfg.find("rope_scaling");
  c.has_rope_scaling = scaling && !scaling->is_null();
  const json::Value* act = cfg.find("hidden_act");
  c.hidden_activation = act && act->is_string() ? act->string : "silu";
  c.attention_bias = get_bool(cfg, "attention_bias", false);
  c.mlp_bias = get_bool(cfg, "mlp_bias", false);
  auto& f = m.architecture.feature_flags;
  f.push_back(c.num_kv_heads == c.num_attention_heads ? "mha" : "gqa");
  f.push_back(c.tied_embeddings ? "tied_embeddings" : "untied_embeddings");
  if (explicit_head) f.push_back("explicit_head_dim");
  if (qwen) f.push_back("qk_norm");

  std::vector<std::filesystem::path> files;
  for (const auto& entry : std::filesystem::directory_iterator(root))
    if (entry.is_regular_file() && entry.path().extension() == ".safetensors") files.push_back(entry.path());
  std::sort(files.begin(), files.end());
  if (files.empty()) throw Error::incompatible_worker("checkpoint has no .safetensors files");
  for (const auto& path : files) {
    const runtime::SafetensorsFile st(path);
    for (const runtime::TensorMetadata& t : st.tensors()) {
      TensorRecord r;
      r.name = t.name;
      r.file = path.filename().string();
      r.dtype = wire_type(t.dtype);
      r.shape = t.shape;
      r.data_offset = t.data_offset;
      r.byte_length = t.byte_length;
      if (t.name == "model.embed_tokens.weight") {
        r.role = TensorRole::kTokenEmbedding;
      } else if (t.name == "model.norm.weight") {
        r.role = TensorRole::kFinalNorm;
      } else if (t.name == "lm_head.weight") {
        r.role = TensorRole::kLmHead;
      } else if (t.name.rfind("model.layers.", 0) == 0) {
        r.role = TensorRole::kTransformerLayer;
        r.layer_index = static_cast<std::uint32_t>(std::stoul(t.name.substr(13)));
      }
      m.tensors.push_back(std::move(r));
    }
  }
  return m;
}

}  // namespace hllm_rocm::model
