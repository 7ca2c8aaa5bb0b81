#include "dense_loader.hpp"

#include <algorithm>
#include <cmath>
#include <fstream>
#include <set>
#include <sstream>
#include <string_view>

#include "json.hpp"

namespace hllm_rocm::model {

using runtime::Error;

namespace {

// The model families a dense stage runs, by manifest architecture id; revision "1" only.
struct Family {
  std::string_view id;
  bool query_key_norm;  // carries per-head q/k norms and must declare "qk_norm"
};
constexpr Family kFamilies[] = {{"llama.v1", false}, {"qwen3.v1", true}};
// Feature flags any family may declare; they change nothing the stage computes.
constexpr std::string_view kNeutralFeatures[] = {"gqa", "mha", "tied_embeddings", "untied_embeddings",
                                                 "explicit_head_dim"};

// Dimensions a tensor's shape is written in.
enum class Dim { kNone, kHidden, kIntermediate, kQueryWidth, kKeyValueWidth, kHeadDim, kVocabulary };

// The tensors of one transformer layer, as "model.layers.<i>." + suffix; a vector has one
// dimension (cols kNone).
struct LayerTensor {
  std::string_view suffix;
  Dim rows, cols;
  bool query_key_norm_only;
};
constexpr LayerTensor kLayerTensors[] = {
    {"input_layernorm.weight", Dim::kHidden, Dim::kNone, false},
    {"self_attn.q_proj.weight", Dim::kQueryWidth, Dim::kHidden, false},
    {"self_attn.k_proj.weight", Dim::kKeyValueWidth, Dim::kHidden, false},
    {"self_attn.v_proj.weight", Dim::kKeyValueWidth, Dim::kHidden, false},
    {"self_attn.q_norm.weight", Dim::kHeadDim, Dim::kNone, true},
    {"self_attn.k_norm.weight", Dim::kHeadDim, Dim::kNone, true},
    {"self_attn.o_proj.weight", Dim::kHidden, Dim::kQueryWidth, false},
    {"post_attention_layernorm.weight", Dim::kHidden, Dim::kNone, false},
    {"mlp.gate_proj.weight", Dim::kIntermediate, Dim::kHidden, false},
    {"mlp.up_proj.weight", Dim::kIntermediate, Dim::kHidden, false},
    {"mlp.down_proj.weight", Dim::kHidden, Dim::kIntermediate, false},
};

[[noreturn]] void refuse(const std::string& why) { throw Error::incompatible_worker("stage not admitted: " + why); }

std::size_t mul(std::size_t a, std::size_t b) {
  if (b != 0 && a > SIZE_MAX / b) refuse("a tensor size overflows");
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

// A bare file name naming a file that resolves (links included) directly inside `root`.
bool inside(const std::filesystem::path& root, const std::string& file) {
  const std::filesystem::path name(file);
  if (name.empty() || name.is_absolute() || name.has_parent_path() || name == "." || name == "..") return false;
  std::error_code ec;
  const auto target = std::filesystem::canonical(root / name, ec);
  if (ec) return false;
  const auto base = std::filesystem::canonical(root, ec);
  return !ec && target.parent_path() == base;
}

// One tensor the stage needs, with the record role and layer index it must carry.
struct Slot {
  std::string name;
  TensorRole role;
  std::optional<std::uint32_t> layer;
  std::vector<std::size_t> shape;
  bool uploaded{true};  // false: a serialized head beside tied embeddings, checked, never held
};

// Admission of one LoadStageRequest, rule group by rule group; every failure is
// INCOMPATIBLE_WORKER.
class Admission {
 public:
  Admission(const LoadStageRequest& request, const std::filesystem::path& root)
      : request_(request), plan_(request.plan), manifest_(request.manifest), config_(request.manifest.config),
        root_(root) {}

  DenseSource run() {
    precision();
    const Family& family = architecture();
    configuration();
    const StageAssignment& stage = assignment();
    fill_source(family, stage);
    index_records();
    const std::vector<Slot> slots = slots_for(family, stage);
    no_unexpected_selection(slots, stage);
    for (const Slot& slot : slots) bind(slot);
    if (src_.tied_head && records_.count("lm_head.weight")) redundant_head();
    return std::move(src_);
  }

 private:
  // Execution F32 or F16; F16 weights under F32 execution exactly when the plan is schema 1.2.
  void precision() {
    const WireDType exec = plan_.execution_dtype;
    if (exec != WireDType::kF32 && exec != WireDType::kF16) refuse("execution precision must be F32 or F16");
    const bool schema_1_2 = plan_.schema_major == 1 && plan_.schema_minor == 2;
    if (plan_.weight_dtype.has_value() != schema_1_2)
      refuse("a resident weight precision is given exactly by schema 1.2 plans");
    if (plan_.weight_dtype && (*plan_.weight_dtype != WireDType::kF16 || exec != WireDType::kF32))
      refuse("mixed residency holds F16 weights under F32 execution only");
    mixed_ = plan_.weight_dtype.has_value();
  }

  const Family& architecture() {
    const ArchitectureDescriptor& a = manifest_.architecture;
    const Family* family = nullptr;
    for (const Family& f : kFamilies)
      if (a.architecture_id == f.id) family = &f;
    if (!family || a.architecture_revision != "1")
      refuse("architecture " + a.architecture_id + " revision " + a.architecture_revision + " is not served");
    bool declares_qk_norm = false;
    for (const std::string& flag : a.feature_flags) {
      if (family->query_key_norm && flag == "qk_norm") {
        declares_qk_norm = true;
        continue;
      }
      if (std::find(std::begin(kNeutralFeatures), std::end(kNeutralFeatures), flag) == std::end(kNeutralFeatures))
        refuse("feature " + flag + " is not served");
    }
    if (family->query_key_norm && !declares_qk_norm) refuse(a.architecture_id + " must declare qk_norm");
    return *family;
  }

  void configuration() {
    const ModelConfig& c = config_;
    const bool dims = c.hidden_size > 0 && c.intermediate_size > 0 && c.num_layers > 0 && c.num_attention_heads > 0 &&
                      c.num_kv_heads > 0 && c.head_dim > 0 && c.maximum_sequence_length > 0 &&
                      c.vocabulary_size > 0;
    if (!dims) refuse("a model dimension is zero");
    if (c.head_dim % 2 != 0) refuse("rotary embedding needs an even head dimension");
    if (c.num_attention_heads % c.num_kv_heads != 0) refuse("query heads must group evenly over key/value heads");
    if (c.hidden_activation != "silu" || c.attention_bias || c.mlp_bias || c.has_rope_scaling)
      refuse("only SiLU MLPs without biases and unscaled rotary embedding are served");
    // Both constants are used as F32 on the device: positive and finite there, and the
    // epsilon must not round to zero.
    auto finite_positive = [](double v) { return std::isfinite(v) && v > 0 && std::isfinite(static_cast<float>(v)); };
    if (!finite_positive(c.rms_norm_eps) || static_cast<float>(c.rms_norm_eps) <= 0 || !finite_positive(c.rope_theta))
      refuse("norm epsilon and rope theta must be positive and finite as F32");
  }

  // The stage's layers lie in the model; the first stage alone owns the embedding, the
  // last alone the final norm, the head and sampling.
  const StageAssignment& assignment() {
    if (request_.stage_index >= plan_.stages.size()) refuse("stage index outside the plan");
    const StageAssignment& s = plan_.stages[request_.stage_index];
    if (s.layer_start >= s.layer_end || s.layer_end > config_.num_layers) refuse("empty or out-of-model layer range");
    const bool first = request_.stage_index == 0, last = request_.stage_index + 1 == plan_.stages.size();
    if (s.owns_token_embedding != first || s.owns_final_norm != last || s.owns_lm_head != last ||
        s.owns_sampling != last)
      refuse("tensor ownership does not follow the stage's place in the plan");
    return s;
  }

  void fill_source(const Family& family, const StageAssignment& s) {
    const ModelConfig& c = config_;
    src_.config = {c.hidden_size,        c.intermediate_size,
                   c.num_attention_heads, c.num_kv_heads,
                   c.head_dim,            c.maximum_sequence_length,
                   static_cast<float>(c.rms_norm_eps), static_cast<float>(c.rope_theta),
                   family.query_key_norm};
    src_.vocabulary_size = c.vocabulary_size;
    src_.first = s.owns_token_embedding;
    src_.final = s.owns_sampling;
    src_.layer_start = s.layer_start;
    src_.layer_end = s.layer_end;
    src_.tied_head = s.owns_lm_head && c.tied_embeddings;
    src_.execution_dtype = storage_type(plan_.execution_dtype);
    src_.weight_dtype = mixed_ ? runtime::DataType::kF16 : src_.execution_dtype;
  }

  void index_records() {
    for (const TensorRecord& r : manifest_.tensors)
      if (!records_.emplace(r.name, &r).second) refuse("the manifest lists " + r.name + " twice");
  }

  std::size_t extent(Dim d) const {
    const ModelConfig& c = config_;
    switch (d) {
      case Dim::kHidden: return c.hidden_size;
      case Dim::kIntermediate: return c.intermediate_size;
      case Dim::kQueryWidth: return mul(c.num_attention_heads, c.head_dim);
      case Dim::kKeyValueWidth: return mul(c.num_kv_heads, c.head_dim);
      case Dim::kHeadDim: return c.head_dim;
      case Dim::kVocabulary: return c.vocabulary_size;
      case Dim::kNone: break;
    }
    return 0;
  }

  std::vector<Slot> slots_for(const Family& family, const StageAssignment& s) const {
    std::vector<Slot> slots;
    const std::vector<std::size_t> table{extent(Dim::kVocabulary), extent(Dim::kHidden)};
    // The embedding serves the first stage's lookup and, tied, the last stage's head.
    if (s.owns_token_embedding || src_.tied_head)
      slots.push_back({"model.embed_tokens.weight", TensorRole::kTokenEmbedding, std::nullopt, table});
    for (std::uint32_t l = s.layer_start; l < s.layer_end; ++l)
      for (const LayerTensor& t : kLayerTensors) {
        if (t.query_key_norm_only && !family.query_key_norm) continue;
        std::vector<std::size_t> shape{extent(t.rows)};
        if (t.cols != Dim::kNone) shape.push_back(extent(t.cols));
        slots.push_back({"model.layers." + std::to_string(l) + "." + std::string(t.suffix),
                         TensorRole::kTransformerLayer, l, std::move(shape)});
      }
    if (s.owns_final_norm) slots.push_back({"model.norm.weight", TensorRole::kFinalNorm, std::nullopt, {table[1]}});
    if (s.owns_lm_head && (!config_.tied_embeddings || records_.count("lm_head.weight")))
      slots.push_back({"lm_head.weight", TensorRole::kLmHead, std::nullopt, table, !config_.tied_embeddings});
    return slots;
  }

  // Every record the stage's ownership selects (its layers, and the embedding, final norm
  // or untied head it owns) must be one of its slots.
  void no_unexpected_selection(const std::vector<Slot>& slots, const StageAssignment& s) const {
    std::set<std::string_view> wanted;
    for (const Slot& slot : slots) wanted.insert(slot.name);
    for (const auto& [name, r] : records_) {
      bool selected = false;
      switch (r->role) {
        case TensorRole::kTransformerLayer:
          selected = r->layer_index && *r->layer_index >= s.layer_start && *r->layer_index < s.layer_end;
          break;
        case TensorRole::kTokenEmbedding: selected = s.owns_token_embedding; break;
        case TensorRole::kFinalNorm: selected = s.owns_final_norm; break;
        case TensorRole::kLmHead: selected = s.owns_lm_head && !config_.tied_embeddings; break;
        default: break;
      }
      if (selected && !wanted.count(name)) refuse(name + " is not a tensor this stage runs");
    }
  }

  // The slot's record (role, layer, shape) and its Safetensors entry (element type, shape,
  // offset, length) must agree; the file must lie in the model root.
  void bind(const Slot& slot) {
    const auto found = records_.find(slot.name);
    if (found == records_.end()) refuse("the manifest lacks " + slot.name);
    const TensorRecord& r = *found->second;
    if (r.role != slot.role || r.layer_index != slot.layer || r.shape != slot.shape)
      refuse(slot.name + " has the wrong role, layer or shape");
    if (!inside(root_, r.file)) refuse(slot.name + " names a file outside the model root");
    auto file = src_.files.find(r.file);
    if (file == src_.files.end()) file = src_.files.emplace(r.file, runtime::SafetensorsFile(root_ / r.file)).first;
    const runtime::TensorMetadata& stored = file->second.tensor(slot.name);
    const WireDType stored_type = wire_type(stored.dtype);
    if (stored_type == WireDType::kUnspecified) refuse(slot.name + " is stored in an unsupported element type");
    if (stored_type != r.dtype || stored.shape != slot.shape || stored.data_offset != r.data_offset ||
        stored.byte_length != r.byte_length)
      refuse(slot.name + ": the manifest record and the Safetensors header disagree");
    if (!slot.uploaded) return;
    std::size_t elements = 1;
    for (std::size_t d : slot.shape) elements = mul(elements, d);
    // Norm vectors stay F32; matrices are held in the resident weight precision.
    const std::size_t held = slot.shape.size() == 1 || src_.weight_dtype == runtime::DataType::kF32 ? 4 : 2;
    src_.resident_bytes += mul(elements, held);
    src_.largest_payload_bytes = std::max(src_.largest_payload_bytes, stored.byte_length);
    src_.tensors.emplace(slot.name, TensorSource{r.file, slot.shape, stored.dtype});
  }

  // A serialized head beside tied embeddings is never used; it must be stored like the
  // embedding it duplicates.
  void redundant_head() const {
    auto stored = [&](const std::string& name) -> const runtime::TensorMetadata& {
      return src_.files.at(records_.at(name)->file).tensor(name);
    };
    const runtime::TensorMetadata& emb = stored("model.embed_tokens.weight");
    const runtime::TensorMetadata& head = stored("lm_head.weight");
    if (emb.dtype != head.dtype || emb.shape != head.shape || emb.byte_length != head.byte_length)
      refuse("a serialized head beside tied embeddings must be stored like the embedding");
  }

  const LoadStageRequest& request_;
  const DeploymentPlan& plan_;
  const ModelManifest& manifest_;
  const ModelConfig& config_;
  const std::filesystem::path& root_;
  bool mixed_{false};
  std::map<std::string, const TensorRecord*> records_;
  DenseSource src_;
};

}  // namespace

DenseSource inspect_dense_stage(const LoadStageRequest& request, const std::filesystem::path& root) {
  return Admission(request, root).run();
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
