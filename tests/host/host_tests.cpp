// Tests of the host-side stage contract (hllm_amd/host): JSON and Safetensors readers,
// stage admission, decode-batch rules, host sampling, the mixed-pass scheduler, and (on a
// GPU) the RocmStage adapter over the C ABI. Run one case per process:
//   host_tests --list | host_tests <case> [args...]
// The GPU decode-batch case follows tests/cpp/decode_batch_contract.hpp.
#include <chrono>
#include <cmath>
#include <deque>
#include <cstdio>
#include <cstring>
#include <fstream>
#include <functional>
#include <future>
#include <map>
#include <memory>
#include <optional>
#include <sstream>
#include <thread>

#include "dense_loader.hpp"
#include "host_sampling.hpp"
#include "json.hpp"
#include "rocm_stage.hpp"
#include "runtime.hpp"
#include "safetensors.hpp"
#include "scheduler.hpp"

using namespace hllm_rocm;
using namespace std::chrono_literals;
namespace fs = std::filesystem;

namespace {

struct Failure : std::runtime_error {
  using std::runtime_error::runtime_error;
};
#define CHECK(cond)                                                                               \
  do {                                                                                            \
    if (!(cond)) throw Failure(std::string(__FILE__) + ":" + std::to_string(__LINE__) + ": " #cond); \
  } while (0)

template <class F>
void expect_error(F&& f, runtime::ErrorCode code, const char* where) {
  try {
    f();
  } catch (const runtime::Error& e) {
    if (e.code() != code) throw Failure(std::string(where) + ": wrong error category: " + e.what());
    return;
  }
  throw Failure(std::string(where) + ": no error raised");
}
#define EXPECT_ERROR(expr, code) expect_error([&] { (void)(expr); }, runtime::ErrorCode::code, #expr)

template <class Predicate>
bool wait_for(Predicate p) {
  const auto until = std::chrono::steady_clock::now() + 2s;
  while (!p() && std::chrono::steady_clock::now() < until) std::this_thread::sleep_for(1ms);
  return p();
}

fs::path scratch_dir(const char* name) {
  const fs::path p = fs::temp_directory_path() / (std::string("hllm_host_") + name + "_" + std::to_string(::getpid()));
  fs::remove_all(p);
  fs::create_directories(p);
  return p;
}

// Writes a Safetensors file: `header` is the JSON text, `data` the data section.
void write_raw(const fs::path& path, const std::string& header, const std::string& data) {
  std::ofstream out(path, std::ios::binary);
  std::uint64_t n = header.size();
  for (int b = 0; b < 8; ++b) out.put(static_cast<char>((n >> (8 * b)) & 0xff));
  out << header << data;
}

struct Tensor {
  std::string name, dtype;
  std::vector<std::size_t> shape;
  std::string bytes;
};
void write_safetensors(const fs::path& path, const std::vector<Tensor>& tensors) {
  std::ostringstream h;
  std::string data;
  h << "{\"__metadata__\":{\"format\":\"pt\"}";
  for (const Tensor& t : tensors) {
    h << ",\"" << t.name << "\":{\"dtype\":\"" << t.dtype << "\",\"shape\":[";
    for (std::size_t i = 0; i < t.shape.size(); ++i) h << (i ? "," : "") << t.shape[i];
    h << "],\"data_offsets\":[" << data.size() << "," << data.size() + t.bytes.size() << "]}";
    data += t.bytes;
  }
  h << "}";
  write_raw(path, h.str(), data);
}
std::string f32_bytes(std::size_t n, float v) {
  std::string s(n * 4, '\0');
  for (std::size_t i = 0; i < n; ++i) std::memcpy(&s[i * 4], &v, 4);
  return s;
}

// ------------------------------------------------------------------ JSON

void json_reader() {
  const json::Value v = json::parse(R"( {"a": [1, -2, 3.5e1, true, null], "s": "x\"\u00e9\ud83d\ude00", "big": 18446744073709551615} )");
  CHECK(v.is_object());
  const json::Value* a = v.find("a");
  CHECK(a && a->array.size() == 5);
  CHECK(a->array[0].is_unsigned && a->array[0].unsigned_value == 1);
  CHECK(!a->array[1].is_unsigned && a->array[1].is_integer && a->array[1].signed_value == -2);
  CHECK(!a->array[2].is_integer && a->array[2].number == 35.0);
  CHECK(a->array[3].is_bool() && a->array[3].boolean && a->array[4].is_null());
  CHECK(v.find("s")->string == "x\"\xc3\xa9\xf0\x9f\x98\x80");
  CHECK(v.find("big")->unsigned_value == 18446744073709551615ull);
  for (const char* bad : {"", "{", "[1,]", "{\"a\" 1}", "01", "1.", "\"\\x\"", "tru", "[1] 2", "\"\\ud800\""}) {
    bool threw = false;
    try {
      json::parse(bad);
    } catch (const json::ParseError&) {
      threw = true;
    }
    CHECK(threw);
  }
}

// ------------------------------------------------------------------ Safetensors

void safetensors_reader() {
  const fs::path dir = scratch_dir("st");
  write_safetensors(dir / "ok.safetensors", {{"b", "F32", {2, 2}, f32_bytes(4, 1.5f)}, {"a", "F16", {3}, std::string(6, '\1')}});
  runtime::SafetensorsFile f(dir / "ok.safetensors");
  CHECK(f.tensors().size() == 2 && f.tensors()[0].name == "a");
  const auto& b = f.tensor("b");
  CHECK(b.dtype == runtime::DataType::kF32 && b.shape == (std::vector<std::size_t>{2, 2}) && b.byte_length == 16);
  const std::span<const std::byte> bytes = f.payload(b);
  float vals[4];
  CHECK(bytes.size() == 16 && f.payload(f.tensor("a")).size() == 6);
  std::memcpy(vals, bytes.data(), 16);
  CHECK(vals[0] == 1.5f && vals[3] == 1.5f);
  CHECK(std::to_integer<int>(f.payload(f.tensor("a"))[5]) == 1);
  EXPECT_ERROR(f.tensor("missing"), kIncompatibleWorker);
  // The mapping moves with the file object.
  runtime::SafetensorsFile moved(std::move(f));
  CHECK(moved.tensors().size() == 2 && moved.payload(moved.tensor("b")).data() == bytes.data());
  const std::pair<std::string, std::string> bad[] = {
      {R"({"x":{"dtype":"F32","shape":[2],"data_offsets":[0,4]}})", std::string(8, '\0')},     // length mismatch
      {R"({"x":{"dtype":"Q4","shape":[2],"data_offsets":[0,8]}})", std::string(8, '\0')},      // dtype
      {R"({"x":{"dtype":"F32","shape":[2],"data_offsets":[0,8]},"y":{"dtype":"F32","shape":[1],"data_offsets":[4,8]}})",
       std::string(8, '\0')},                                                                  // overlap
      {R"({"x":{"dtype":"F32","shape":[4],"data_offsets":[0,16]}})", std::string(8, '\0')},    // past the end
      {R"({"x":{"dtype":"F32","shape":[-1],"data_offsets":[0,4]}})", std::string(4, '\0')},    // negative dim
      {R"({"x":{"dtype":"F32","shape":[1],"data_offsets":[4,0]}})", std::string(4, '\0')},     // reversed
      {R"({"__metadata__":{}})", ""},                                                          // no tensors
      {R"([1,2])", ""},                                                                        // not an object
      {R"({"x":)", ""},                                                                        // invalid JSON
      {R"({"x":{"dtype":"F32","shape":[2.5],"data_offsets":[0,8]}})", std::string(8, '\0')},  // fractional dim
      {R"({"x":{"dtype":"F32","shape":[2],"data_offsets":[0]}})", std::string(8, '\0')},      // one offset
      {R"({"x":{"shape":[2],"data_offsets":[0,8]}})", std::string(8, '\0')},                  // no dtype
      {R"({"x":7})", std::string(8, '\0')},                                                   // record not an object
  };
  int i = 0;
  for (const auto& [header, data] : bad) {
    const fs::path p = dir / ("bad" + std::to_string(i++) + ".safetensors");
    write_raw(p, header, data);
    EXPECT_ERROR(runtime::SafetensorsFile(p), kIncompatibleWorker);
  }
  {
    std::ofstream(dir / "short.safetensors") << "abc";
    EXPECT_ERROR(runtime::SafetensorsFile(dir / "short.safetensors"), kIncompatibleWorker);
    std::ofstream out(dir / "huge.safetensors", std::ios::binary);
    const unsigned char prefix[8] = {0xff, 0xff, 0xff, 0xff, 0, 0, 0, 0};
    out.write(reinterpret_cast<const char*>(prefix), 8);
    out << "{}";
  }
  EXPECT_ERROR(runtime::SafetensorsFile(dir / "huge.safetensors"), kIncompatibleWorker);
  fs::remove_all(dir);
}

// ------------------------------------------------------------------ stage admission

// A two-layer Qwen3 checkpoint with zero-filled F32 weights (shapes only matter here).
fs::path tiny_checkpoint(const char* name, bool tied) {
  const fs::path dir = scratch_dir(name);
  const std::size_t H = 8, I = 16, Q = 2, K = 1, D = 4, V = 32;
  std::vector<Tensor> t;
  auto add = [&](std::string n, std::vector<std::size_t> shape) {
    std::size_t e = 1;
    for (auto d : shape) e *= d;
    t.push_back({std::move(n), "F32", shape, f32_bytes(e, 0.01f)});
  };
  add("model.embed_tokens.weight", {V, H});
  add("model.norm.weight", {H});
  if (!tied) add("lm_head.weight", {V, H});
  for (int l = 0; l < 2; ++l) {
    const std::string p = "model.layers." + std::to_string(l) + ".";
    add(p + "input_layernorm.weight", {H});
    add(p + "post_attention_layernorm.weight", {H});
    add(p + "self_attn.q_proj.weight", {Q * D, H});
    add(p + "self_attn.k_proj.weight", {K * D, H});
    add(p + "self_attn.v_proj.weight", {K * D, H});
    add(p + "self_attn.o_proj.weight", {H, Q * D});
    add(p + "mlp.gate_proj.weight", {I, H});
    add(p + "mlp.up_proj.weight", {I, H});
    add(p + "mlp.down_proj.weight", {H, I});
    add(p + "self_attn.q_norm.weight", {D});
    add(p + "self_attn.k_norm.weight", {D});
  }
  write_safetensors(dir / "model.safetensors", t);
  std::ofstream(dir / "config.json") << R"({"model_type":"qwen3","hidden_size":8,"intermediate_size":16,)"
                                     << R"("num_hidden_layers":2,"num_attention_heads":2,"num_key_value_heads":1,)"
                                     << R"("head_dim":4,"vocab_size":32,"max_position_embeddings":64,)"
                                     << R"("rms_norm_eps":1e-6,"rope_theta":1000000.0,"hidden_act":"silu",)"
                                     << R"("tie_word_embeddings":)" << (tied ? "true" : "false") << "}";
  return dir;
}

model::LoadStageRequest request_for(const model::ModelManifest& m, std::uint32_t stage, std::uint32_t stages) {
  model::LoadStageRequest r;
  r.manifest = m;
  r.stage_index = stage;
  r.plan.execution_dtype = model::WireDType::kF16;
  for (std::uint32_t s = 0; s < stages; ++s) {
    model::StageAssignment a;
    a.layer_start = s * m.config.num_layers / stages;
    a.layer_end = (s + 1) * m.config.num_layers / stages;
    a.owns_token_embedding = s == 0;
    a.owns_final_norm = a.owns_lm_head = a.owns_sampling = s + 1 == stages;
    r.plan.stages.push_back(a);
  }
  return r;
}

void dense_admission() {
  const fs::path dir = tiny_checkpoint("adm", false);
  const model::ModelManifest m = model::manifest_from_checkpoint(dir);
  CHECK(m.architecture.architecture_id == "qwen3.v1" && m.tensors.size() == 3 + 22);
  const model::DenseSource whole = model::inspect_dense_stage(request_for(m, 0, 1), dir);
  CHECK(whole.first && whole.final && !whole.tied_head && whole.tensors.size() == 25);
  CHECK(whole.config.query_key_norm && whole.config.head_dimension == 4);
  const model::DenseSource second = model::inspect_dense_stage(request_for(m, 1, 2), dir);
  CHECK(!second.first && second.final && second.layer_start == 1 && second.tensors.size() == 11 + 2);
  const model::DenseSource first = model::inspect_dense_stage(request_for(m, 0, 2), dir);
  CHECK(first.first && !first.final && first.tensors.size() == 11 + 1);

  auto mutated = [&](std::function<void(model::LoadStageRequest&)> change) {
    model::LoadStageRequest r = request_for(m, 0, 1);
    change(r);
    return r;
  };
  const std::vector<std::function<void(model::LoadStageRequest&)>> incompatible = {
      [](auto& r) { r.stage_index = 3; },
      [](auto& r) { r.plan.execution_dtype = model::WireDType::kBF16; },
      [](auto& r) { r.plan.weight_dtype = model::WireDType::kF16; },  // mixed needs schema 1.2 and F32 execution
      [](auto& r) { r.manifest.architecture.architecture_id = "mistral.v1"; },
      [](auto& r) { r.manifest.architecture.architecture_revision = "2"; },
      [](auto& r) { r.manifest.architecture.feature_flags.push_back("sliding_window"); },
      [](auto& r) { std::erase(r.manifest.architecture.feature_flags, std::string("qk_norm")); },
      [](auto& r) { r.manifest.config.hidden_activation = "gelu"; },
      [](auto& r) { r.manifest.config.has_rope_scaling = true; },
      [](auto& r) { r.manifest.config.attention_bias = true; },
      [](auto& r) { r.manifest.config.head_dim = 3; },
      [](auto& r) { r.manifest.config.rms_norm_eps = 0.0; },
      [](auto& r) { r.manifest.config.rope_theta = 1e300; },  // not finite as F32
      [](auto& r) { r.plan.stages[0].layer_end = 5; },
      [](auto& r) { r.plan.stages[0].owns_sampling = false; },
      [](auto& r) { r.manifest.tensors.push_back(r.manifest.tensors[0]); },  // duplicate
      [](auto& r) { r.manifest.tensors.erase(r.manifest.tensors.begin()); },  // missing
      [](auto& r) { r.manifest.tensors[0].shape[0] += 1; },
      [](auto& r) { r.manifest.tensors[0].data_offset += 4; },
      [](auto& r) { r.manifest.tensors[0].dtype = model::WireDType::kF16; },
      [](auto& r) { r.manifest.tensors[0].file = "../model.safetensors"; },
      [](auto& r) { r.manifest.tensors[0].file = "/tmp/model.safetensors"; },
      [](auto& r) {
        for (auto& t : r.manifest.tensors)
          if (t.role == model::TensorRole::kTransformerLayer) t.layer_index = 7;
      },
      [](auto& r) {
        auto extra = r.manifest.tensors.back();
        extra.name = "model.layers.0.self_attn.rotary.weight";
        extra.layer_index = 0;
        r.manifest.tensors.push_back(extra);
      },
  };
  for (const auto& change : incompatible) EXPECT_ERROR(model::inspect_dense_stage(mutated(change), dir), kIncompatibleWorker);

  const fs::path tied = tiny_checkpoint("adm_tied", true);
  const model::ModelManifest mt = model::manifest_from_checkpoint(tied);
  const model::DenseSource s2 = model::inspect_dense_stage(request_for(mt, 1, 2), tied);
  CHECK(s2.tied_head && s2.tensors.count("model.embed_tokens.weight") && !s2.tensors.count("lm_head.weight"));
  fs::remove_all(dir);
  fs::remove_all(tied);
}

// ------------------------------------------------------------------ decode batches

// The adapter's decode-batch rules (tests/cpp/decode_batch_contract.hpp runs the batch;
// these are its admission rules).
void decode_batch_rules() {
  std::atomic_bool stop{false};
  runtime::SequenceState a, b, busy;
  busy.prefilling = true;
  using Items = std::vector<runtime::DecodeBatchItem>;
  auto tok = [](std::uint64_t id) { return runtime::StageInput{runtime::TokenInput{{id}}}; };
  auto row = [](std::size_t width) {
    return runtime::StageInput{runtime::BoundaryActivation{1, width, std::vector<std::byte>(width * 2)}};
  };
  backend::require_decode_batch(Items{{tok(5), 3, &a, &stop}, {tok(9), 1, &b, &stop}}, 6);
  backend::require_decode_batch(Items{{row(6), 3, &a, &stop}, {row(6), 1, &b, &stop}}, 6);
  EXPECT_ERROR(backend::require_decode_batch(Items{}, 6), kInvalidRequest);
  EXPECT_ERROR(backend::require_decode_batch(Items{{tok(1), 0, &a, &stop}}, 6), kInvalidRequest);  // not started
  EXPECT_ERROR(backend::require_decode_batch(Items{{tok(1), 2, &busy, &stop}}, 6), kInvalidRequest);
  runtime::SequenceState only;
  only.prefill_only = true;
  EXPECT_ERROR(backend::require_decode_batch(Items{{tok(5), 3, &a, &stop}, {tok(1), 2, &only, &stop}}, 6),
               kInvalidRequest);
  EXPECT_ERROR(backend::require_decode_batch(Items{{tok(1), 2, &a, &stop}, {tok(2), 2, &a, &stop}}, 6),
               kInvalidRequest);
  EXPECT_ERROR(backend::require_decode_batch(Items{{tok(1), 2, &a, &stop}, {row(6), 2, &b, &stop}}, 6),
               kInvalidRequest);
  EXPECT_ERROR(backend::require_decode_batch(Items{{runtime::TokenInput{{1, 2}}, 2, &a, &stop}}, 6),
               kInvalidRequest);
  EXPECT_ERROR(backend::require_decode_batch(Items{{row(5), 2, &a, &stop}}, 6), kInvalidRequest);
  EXPECT_ERROR(backend::require_decode_batch(Items{{tok(1), 2, nullptr, &stop}}, 6), kInvalidRequest);
  std::vector<runtime::SequenceState> many(65);
  Items big;
  for (auto& s : many) big.push_back({tok(1), 1, &s, &stop});
  EXPECT_ERROR(backend::require_decode_batch(big, 6), kInvalidRequest);
  big.pop_back();
  backend::require_decode_batch(big, 6);
}

// ------------------------------------------------------------------ host sampling

// Fixture written by tests/golden/make_sampling_vectors.py from the oracle (itself pinned
// bitwise to the reference's sampling.cpp): logits, options, expected token / logprobs.
void host_sampling(const std::vector<std::string>& args) {
  CHECK(args.size() == 1);
  std::ifstream in(args[0]);
  std::stringstream text;
  text << in.rdbuf();
  const json::Value doc = json::parse(text.str());
  int cases = 0;
  std::vector<std::vector<float>> sets;
  for (const json::Value& set : doc.find("logits")->array) {
    sets.emplace_back();
    for (const json::Value& v : set.array) sets.back().push_back(static_cast<float>(v.number));
  }
  for (const json::Value& c : doc.find("cases")->array) {
    const std::vector<float>& logits = sets.at(c.find("logits_index")->unsigned_value);
    runtime::SamplingOptions o;
    o.temperature = c.find("temperature")->number;
    o.top_p = c.find("top_p")->number;
    o.top_k = c.find("top_k")->unsigned_value;
    o.seed = c.find("seed")->unsigned_value;
    o.return_logprobs = c.find("return_logprobs")->boolean;
    o.top_logprobs = static_cast<std::uint32_t>(c.find("top_logprobs")->unsigned_value);
    const auto got = runtime::sample_token(logits.data(), logits.size(), o, c.find("generated_index")->unsigned_value);
    CHECK(got.id == c.find("token")->unsigned_value);
    if (o.return_logprobs) {
      CHECK(got.logprob && *got.logprob == c.find("logprob")->number);
      const auto& tops = c.find("top_ids")->array;
      CHECK(got.top_logprobs.size() == tops.size());
      for (std::size_t i = 0; i < tops.size(); ++i) {
        CHECK(got.top_logprobs[i].token_id == tops[i].unsigned_value);
        CHECK(got.top_logprobs[i].logprob == c.find("top_values")->array[i].number);
      }
    }
    ++cases;
  }
  CHECK(cases > 0);
  const float bad[2] = {1.0f, NAN};
  runtime::SamplingOptions o;
  EXPECT_ERROR(runtime::sample_logits(bad, 2, o, 0), kInternal);
  o.top_p = 0.0;
  EXPECT_ERROR(runtime::sample_logits(bad, 1, o, 0), kInvalidRequest);
  o = {};
  o.top_logprobs = 2;  // without return_logprobs
  EXPECT_ERROR(runtime::sample_logits(bad, 1, o, 0), kInvalidRequest);
}

// ------------------------------------------------------------------ scheduler

// A stand-in stage: records every pass as the first token ID of each member; a member with
// token 999 waits for `gate` (to hold the dispatcher inside a pass). With `mixed`, it runs
// mixed passes; otherwise prefills alone and decode batches.
class RecordingStage : public runtime::StageBackend {
 public:
  mutable std::mutex mutex;
  mutable std::vector<std::vector<std::uint64_t>> passes;
  std::promise<void> open;
  std::shared_future<void> gate = open.get_future().share();
  bool batches{true};
  mutable std::atomic<bool> fail{false};
  bool supports_decode_batch() const override { return batches; }
  runtime::MemoryAmounts weight_memory() const override { return {}; }
  std::size_t hidden_size() const override { return 1; }
  std::size_t vocabulary_size() const override { return 1000; }
  std::size_t maximum_tokens() const override { return 1024; }
  runtime::SequenceMemory sequence_memory(std::size_t, std::size_t) const override { return {}; }
  std::unique_ptr<runtime::SequenceState> allocate_sequence(std::size_t) const override {
    return std::make_unique<runtime::SequenceState>();
  }
  runtime::StageOutput execute(runtime::StageInput input, std::size_t, runtime::SequenceState& s,
                               const std::atomic_bool&) const override {
    std::vector<runtime::DecodeBatchItem> one;
    one.push_back({std::move(input), 0, &s, nullptr});
    return record(one).front();
  }
  std::vector<runtime::StageOutput> execute_decode_batch(std::vector<runtime::DecodeBatchItem> items) const override {
    return record(items);
  }

 protected:
  std::vector<runtime::StageOutput> record(const std::vector<runtime::DecodeBatchItem>& items) const {
    std::vector<std::uint64_t> ids;
    for (const auto& it : items) ids.push_back(std::get<runtime::TokenInput>(it.input).ids.at(0));
    if (ids.front() == 999 && gate.wait_for(5s) != std::future_status::ready)
      throw std::runtime_error("test gate timed out");
    {
      std::scoped_lock lock(mutex);
      passes.push_back(ids);
    }
    if (fail.load()) throw std::runtime_error("injected pass failure");
    std::vector<runtime::StageOutput> out;
    for (const auto& it : items) {
      it.sequence->generated_index += 1;
      out.push_back(runtime::SampledToken{std::get<runtime::TokenInput>(it.input).ids.at(0)});
    }
    return out;
  }
};

class MixedRecordingStage final : public RecordingStage, public worker::MixedPassBackend {
 public:
  std::vector<runtime::StageOutput> execute_mixed(std::vector<runtime::DecodeBatchItem> items) const override {
    return record(items);
  }
};

// Callers, each with its own sequence and cancellation flag, submitting through one scheduler.
struct Callers {
  worker::StageScheduler& scheduler;
  const runtime::StageBackend& backend;
  std::deque<runtime::SequenceState> sequences;
  std::deque<std::atomic_bool> flags;
  std::vector<std::future<runtime::StageOutput>> results;
  // Queues one request (ids: its token IDs, first = its name) and waits until it is queued.
  // `position` defaults to 0 for prompts and 1 for single tokens.
  std::size_t submit(std::vector<std::uint64_t> ids, bool prefill,
                      std::chrono::milliseconds deadline = std::chrono::milliseconds(5000),
                      std::optional<std::size_t> position = std::nullopt, bool prefill_only = false) {
    sequences.emplace_back();
    sequences.back().prefilling = prefill;
    sequences.back().prefill_only = prefill_only;
    const std::size_t at = position ? *position : prefill_position(ids);
    flags.emplace_back(false);
    runtime::SequenceState& s = sequences.back();
    std::atomic_bool& stop = flags.back();
    // Queued, running or already done: a request may complete before it is seen queued.
    auto seen = [this] {
      const auto m = scheduler.metrics();
      return m.queued_prefills + m.queued_decodes + m.executing + m.completed_steps;
    };
    const std::size_t queued = seen();
    results.push_back(std::async(std::launch::async, [this, ids, &s, &stop, deadline, at] {
      return scheduler.execute(backend, runtime::TokenInput{ids}, at, s, stop,
                               std::chrono::system_clock::now() + deadline);
    }));
    CHECK(wait_for([&] { return seen() > queued; }));
    return results.size() - 1;
  }
  static std::size_t prefill_position(const std::vector<std::uint64_t>& ids) { return ids.size() == 1 ? 1 : 0; }
  std::uint64_t token(std::size_t i) { return std::get<runtime::SampledToken>(results[i].get()).id; }
};

std::vector<std::uint64_t> prefill_ids(std::uint64_t name, std::size_t rows) {
  std::vector<std::uint64_t> ids(rows, 1);
  ids[0] = name;
  return ids;
}

// Mixed passes: all waiting decodes (up to the limit) plus prefills in arrival order within
// the row budget, decodes first.
void scheduler_mixed_passes() {
  worker::StageScheduler scheduler;
  scheduler.configure(worker::PassPolicy{4, 10});
  MixedRecordingStage stage;
  stage.open.set_value();
  Callers c{scheduler, stage, {}, {}, {}};
  scheduler.hold();
  for (std::uint64_t d = 0; d < 6; ++d) c.submit({d}, false);
  c.submit(prefill_ids(100, 6), true);
  c.submit(prefill_ids(101, 3), true);
  c.submit(prefill_ids(102, 5), true);
  CHECK(scheduler.metrics().queued_decodes == 6 && scheduler.metrics().queued_prefills == 3);
  scheduler.resume();
  for (std::size_t i = 0; i < 6; ++i) CHECK(c.token(i) == i);
  CHECK(c.token(6) == 100 && c.token(7) == 101 && c.token(8) == 102);
  using P = std::vector<std::vector<std::uint64_t>>;
  CHECK(stage.passes == (P{{0, 1, 2, 3, 100, 101}, {4, 5, 102}}));
  const auto m = scheduler.metrics();
  CHECK(m.passes == 2 && m.mixed_passes == 2 && m.completed_steps == 9 && m.largest_decode_batch == 4);
  CHECK(m.largest_pass_rows == 4 + 6 + 3 && m.executing == 0 && m.queued_decodes + m.queued_prefills == 0);
}

// A prefill larger than the budget still runs (alone with the decodes), and requests keep
// arriving while a pass runs.
void scheduler_large_prefill() {
  worker::StageScheduler scheduler;
  scheduler.configure(worker::PassPolicy{8, 4});
  MixedRecordingStage stage;
  Callers c{scheduler, stage, {}, {}, {}};
  c.submit({999}, false);  // holds the first pass until the gate opens
  CHECK(wait_for([&] { return scheduler.metrics().executing == 1; }));
  c.submit(prefill_ids(200, 9), true);
  c.submit({1}, false);
  c.submit(prefill_ids(201, 2), true);
  stage.open.set_value();
  CHECK(c.token(0) == 999 && c.token(1) == 200 && c.token(2) == 1 && c.token(3) == 201);
  using P = std::vector<std::vector<std::uint64_t>>;
  CHECK(stage.passes == (P{{999}, {1, 200}, {201}}));
}

// Cancelled or expired requests leave the queue without reaching the backend; the others run.
void scheduler_retires_unready_requests() {
  worker::StageScheduler scheduler;
  MixedRecordingStage stage;
  stage.open.set_value();
  Callers c{scheduler, stage, {}, {}, {}};
  scheduler.hold();
  const std::size_t cancelled = c.submit({7}, false);
  const std::size_t expiring = c.submit({8}, false, std::chrono::milliseconds(30));
  const std::size_t kept = c.submit(prefill_ids(300, 2), true);
  c.flags[cancelled] = true;
  EXPECT_ERROR(c.results[cancelled].get(), kCancelled);
  EXPECT_ERROR(c.results[expiring].get(), kDeadlineExceeded);
  CHECK(scheduler.metrics().queued_decodes == 0 && scheduler.metrics().queued_prefills == 1);
  scheduler.resume();
  CHECK(c.token(kept) == 300);
  using P = std::vector<std::vector<std::uint64_t>>;
  CHECK(stage.passes == (P{{300}}));
}

// A member cancelled while its pass runs gets the pass's result (or its failure); the
// scheduler takes new work afterwards.
void scheduler_in_flight(bool fail) {
  worker::StageScheduler scheduler;
  MixedRecordingStage stage;
  Callers c{scheduler, stage, {}, {}, {}};
  const std::size_t gate = c.submit({999}, false);
  CHECK(wait_for([&] { return scheduler.metrics().executing == 1; }));
  c.flags[gate] = true;  // cancelled inside its pass
  const std::size_t a = c.submit({1}, false);
  stage.fail = fail;
  stage.open.set_value();
  if (fail) {
    bool threw = false;
    try {
      static_cast<void>(c.results[gate].get());
    } catch (const std::runtime_error&) {
      threw = true;
    }
    CHECK(threw);
    try {
      static_cast<void>(c.results[a].get());
      threw = false;
    } catch (const std::runtime_error&) {
      threw = true;
    }
    CHECK(threw);
  } else {
    CHECK(c.token(gate) == 999 && c.token(a) == 1);
    CHECK(c.sequences[gate].generated_index == 1);
  }
  stage.fail = false;
  const std::size_t after = c.submit({5}, false);
  CHECK(c.token(after) == 5 && scheduler.metrics().executing == 0);
}

// Backends without mixed passes: a prefill alone or a decode batch, alternating while both
// queues wait, the first pass serving the older request; single decodes when the backend
// has no decode batches.
void scheduler_without_mixed_passes(bool batches) {
  worker::StageScheduler scheduler;
  scheduler.configure(worker::PassPolicy{2, 512});
  RecordingStage stage;
  stage.batches = batches;
  stage.open.set_value();
  Callers c{scheduler, stage, {}, {}, {}};
  scheduler.hold();
  for (std::uint64_t d = 0; d < 3; ++d) c.submit({d}, false);
  c.submit(prefill_ids(100, 4), true);
  c.submit(prefill_ids(101, 4), true);
  scheduler.resume();
  for (std::size_t i = 0; i < 5; ++i) static_cast<void>(c.results[i].get());
  using P = std::vector<std::vector<std::uint64_t>>;
  if (batches)
    CHECK(stage.passes == (P{{0, 1}, {100}, {2}, {101}}));
  else
    CHECK(stage.passes == (P{{0}, {100}, {1}, {101}, {2}}));
  CHECK(scheduler.metrics().mixed_passes == 0);
}

// A one-token request at position 0 starts its sequence and a prefill-only sequence never
// decodes: both are prefills (cpp/src/worker/scheduler.cpp:48; cpp/src/decode_batch.cpp:16-17),
// so neither joins a decode batch and fails its healthy members.
void scheduler_classifies_first_tokens_as_prefills() {
  worker::StageScheduler scheduler;
  scheduler.configure(worker::PassPolicy{8, 512});
  RecordingStage stage;
  stage.open.set_value();
  Callers c{scheduler, stage, {}, {}, {}};
  scheduler.hold();
  c.submit({1}, false);
  c.submit({50}, false, std::chrono::milliseconds(5000), 0);         // position 0
  c.submit({2}, false);
  c.submit({60}, false, std::chrono::milliseconds(5000), 7, true);   // prefill-only
  CHECK(scheduler.metrics().queued_decodes == 2 && scheduler.metrics().queued_prefills == 2);
  scheduler.resume();
  for (std::size_t i = 0; i < 4; ++i) static_cast<void>(c.results[i].get());
  using P = std::vector<std::vector<std::uint64_t>>;
  CHECK(stage.passes == (P{{1, 2}, {50}, {60}}));
}

// Destroying the scheduler: the running pass delivers its result, queued requests fail
// CANCELLED, and the destructor returns only once every caller has left execute().
void scheduler_shutdown(bool running) {
  MixedRecordingStage stage;
  auto scheduler = std::make_unique<worker::StageScheduler>();
  Callers c{*scheduler, stage, {}, {}, {}};
  std::size_t gate = 0;
  if (running) {
    gate = c.submit({999}, false);  // holds the dispatcher inside its pass
    CHECK(wait_for([&] { return scheduler->metrics().executing == 1; }));
  } else {
    scheduler->hold();
  }
  const std::size_t decode = c.submit({1}, false);
  const std::size_t prefill = c.submit(prefill_ids(100, 3), true);
  std::thread opener([&] {
    std::this_thread::sleep_for(50ms);
    stage.open.set_value();
  });
  scheduler.reset();
  opener.join();
  if (running) CHECK(c.token(gate) == 999);
  EXPECT_ERROR(c.results[decode].get(), kCancelled);
  EXPECT_ERROR(c.results[prefill].get(), kCancelled);
  using P = std::vector<std::vector<std::uint64_t>>;
  CHECK(stage.passes == (running ? P{{999}} : P{}));
}

void scheduler_configuration() {
  worker::StageScheduler s;
  EXPECT_ERROR(s.configure(worker::PassPolicy{0, 512}), kInvalidRequest);
  EXPECT_ERROR(s.configure(worker::PassPolicy{65, 512}), kInvalidRequest);
  EXPECT_ERROR(s.configure(worker::PassPolicy{8, 0}), kInvalidRequest);
  s.configure(worker::PassPolicy{64, 2048});
  CHECK(s.policy().maximum_decode_rows == 64 && s.policy().prefill_row_budget == 2048);
  s.configure(1);
  CHECK(s.policy().maximum_decode_rows == 1 && s.policy().prefill_row_budget == 2048);
}

// ------------------------------------------------------------------ GPU: the adapter

// Loads a checkpoint directory through the factory and runs a greedy prefill then
// `decodes` decode steps; prints the sampled tokens as a JSON list. With a fifth argument
// "logprobs", every step also returns the five best log-probabilities, printed per step as
// "TOP [[id, logprob], ...]".
void gpu_checkpoint_greedy(const std::vector<std::string>& args) {
  CHECK(args.size() == 4 || (args.size() == 5 && args[4] == "logprobs"));
  const bool logprobs = args.size() == 5;
  const fs::path dir = args[0];
  const std::string dtype = args[1];
  std::vector<std::uint64_t> prompt;
  {
    std::stringstream s(args[2]);
    std::string tok;
    while (std::getline(s, tok, ',')) prompt.push_back(std::stoull(tok));
  }
  const int decodes = std::stoi(args[3]);
  const model::ModelManifest m = model::manifest_from_checkpoint(dir);
  model::LoadStageRequest r = request_for(m, 0, 1);
  r.plan.execution_dtype = dtype == "f32" ? model::WireDType::kF32 : model::WireDType::kF16;
  backend::StageOptions options;
  options.kv_cache_bytes = 64u << 20;
  options.kv_block_tokens = 32;
  options.max_sequences = 8;
  options.max_pass_rows = 256;
  backend::RocmBackendFactory factory(options);
  runtime::MemoryAmounts capacity{1ull << 40, 1ull << 40, 0, 0};
  auto stage = factory.load(r, dir, capacity);
  std::atomic_bool stop{false};
  auto seq = stage->allocate_sequence(prompt.size() + decodes + 1);
  if (logprobs) seq->sampling = {0.0, 1.0, 0, 0, true, 5};
  std::vector<std::uint64_t> out;
  auto step = [&](runtime::StageInput input, std::size_t position) {
    const auto token = std::get<runtime::SampledToken>(stage->execute(std::move(input), position, *seq, stop));
    if (logprobs) {
      std::printf("TOP [");
      for (std::size_t i = 0; i < token.top_logprobs.size(); ++i)
        std::printf("%s[%llu,%.9g]", i ? "," : "", static_cast<unsigned long long>(token.top_logprobs[i].token_id),
                    token.top_logprobs[i].logprob);
      std::printf("]\n");
    }
    out.push_back(token.id);
    return token.id;
  };
  auto t = step(runtime::TokenInput{prompt}, 0);
  for (int i = 0; i < decodes; ++i) t = step(runtime::TokenInput{{t}}, prompt.size() + i);
  std::printf("TOKENS [");
  for (std::size_t i = 0; i < out.size(); ++i) std::printf("%s%llu", i ? "," : "", static_cast<unsigned long long>(out[i]));
  std::printf("]\n");
  // State rules of the contract.
  EXPECT_ERROR(stage->execute(runtime::TokenInput{{1}}, 0, *seq, stop), kInvalidRequest);  // wrong position
  EXPECT_ERROR(stage->execute(runtime::TokenInput{{m.config.vocabulary_size}}, prompt.size() + decodes, *seq, stop),
               kInvalidRequest);  // token ID outside the vocabulary
  std::atomic_bool cancelled{true};
  auto other = stage->allocate_sequence(4);
  bool threw = false;
  try {
    static_cast<void>(stage->execute(runtime::TokenInput{{1}}, 0, *other, cancelled));
  } catch (const std::runtime_error&) {
    threw = true;
  }
  CHECK(threw);
}

// tests/cpp/decode_batch_contract.hpp: a decode batch returns what serial execution
// returns, in item order, advancing each member's generated index, for greedy and
// temperature sampling with log-probabilities.
void gpu_decode_batch_contract(const std::vector<std::string>& args) {
  CHECK(args.size() == 1);
  const fs::path dir = args[0];
  const model::ModelManifest m = model::manifest_from_checkpoint(dir);
  model::LoadStageRequest r = request_for(m, 0, 1);
  r.plan.execution_dtype = model::WireDType::kF32;
  backend::StageOptions options;
  options.kv_cache_bytes = 64u << 20;
  options.kv_block_tokens = 32;
  options.max_sequences = 32;
  options.max_pass_rows = 256;
  backend::RocmBackendFactory factory(options);
  auto stage = factory.load(r, dir, {1ull << 40, 1ull << 40, 0, 0});
  CHECK(stage->supports_decode_batch());
  for (double temperature : {0.0, 0.8}) {
    std::atomic_bool cancelled{false};
    std::vector<std::unique_ptr<runtime::SequenceState>> reference, batched;
    const std::vector<std::size_t> lengths{7, 2, 4, 1};
    std::vector<runtime::SampledToken> expected;
    for (std::size_t i = 0; i < lengths.size(); ++i) {
      reference.push_back(stage->allocate_sequence(lengths[i] + 1));
      batched.push_back(stage->allocate_sequence(lengths[i] + 1));
      for (auto* state : {reference.back().get(), batched.back().get()}) {
        state->sampling = {temperature, 0.95, 8, i + 42, true, 3};
        static_cast<void>(stage->execute(runtime::TokenInput{std::vector<std::uint64_t>(lengths[i], 1)}, 0, *state, cancelled));
      }
      expected.push_back(std::get<runtime::SampledToken>(
          stage->execute(runtime::TokenInput{{4}}, lengths[i], *reference.back(), cancelled)));
    }
    std::vector<runtime::DecodeBatchItem> items;
    for (std::size_t i = 0; i < lengths.size(); ++i)
      items.push_back({runtime::TokenInput{{4}}, lengths[i], batched[i].get(), &cancelled});
    const auto actual = stage->execute_decode_batch(std::move(items));
    CHECK(actual.size() == expected.size());
    for (std::size_t i = 0; i < expected.size(); ++i) {
      const auto& token = std::get<runtime::SampledToken>(actual[i]);
      CHECK(token.id == expected[i].id);
      CHECK(token.logprob && expected[i].logprob && std::fabs(*token.logprob - *expected[i].logprob) < 0.02);
      CHECK(token.top_logprobs.size() == 3);
      CHECK(batched[i]->generated_index == reference[i]->generated_index);
    }
  }
}

// The scheduler over the ROCm stage: a decode of one sequence and a prefill of another,
// queued together, run as one mixed pass and give the tokens serial execution gives.
void gpu_scheduler_mixed_pass(const std::vector<std::string>& args) {
  CHECK(args.size() == 1);
  const fs::path dir = args[0];
  const model::ModelManifest m = model::manifest_from_checkpoint(dir);
  model::LoadStageRequest r = request_for(m, 0, 1);
  r.plan.execution_dtype = model::WireDType::kF32;
  backend::StageOptions options;
  options.kv_cache_bytes = 64u << 20;
  options.kv_block_tokens = 32;
  options.max_sequences = 16;
  options.max_pass_rows = 256;
  backend::RocmBackendFactory factory(options);
  auto stage = factory.load(r, dir, {1ull << 40, 1ull << 40, 0, 0});
  std::atomic_bool go{false};
  const std::vector<std::uint64_t> prompt_a{1, 4, 2, 8, 3}, prompt_b{2, 7, 1};
  auto token = [](const runtime::StageOutput& o) { return std::get<runtime::SampledToken>(o).id; };
  auto ra = stage->allocate_sequence(16), rb = stage->allocate_sequence(16);
  static_cast<void>(stage->execute(runtime::TokenInput{prompt_a}, 0, *ra, go));
  const std::uint64_t ta = token(stage->execute(runtime::TokenInput{{4}}, 5, *ra, go));
  const std::uint64_t tb = token(stage->execute(runtime::TokenInput{prompt_b}, 0, *rb, go));
  auto sa = stage->allocate_sequence(16), sb = stage->allocate_sequence(16);
  static_cast<void>(stage->execute(runtime::TokenInput{prompt_a}, 0, *sa, go));
  sb->prefilling = true;
  worker::StageScheduler scheduler;
  scheduler.hold();
  auto fa = std::async(std::launch::async, [&] {
    return scheduler.execute(*stage, runtime::TokenInput{{4}}, 5, *sa, go, std::chrono::system_clock::now() + 5s);
  });
  CHECK(wait_for([&] { return scheduler.metrics().queued_decodes == 1; }));
  auto fb = std::async(std::launch::async, [&] {
    return scheduler.execute(*stage, runtime::TokenInput{prompt_b}, 0, *sb, go, std::chrono::system_clock::now() + 5s);
  });
  CHECK(wait_for([&] { return scheduler.metrics().queued_prefills == 1; }));
  scheduler.resume();
  CHECK(token(fa.get()) == ta);
  CHECK(token(fb.get()) == tb);
  const auto metrics = scheduler.metrics();
  CHECK(metrics.passes == 1 && metrics.mixed_passes == 1 && metrics.largest_pass_rows == 4);
}

// StageBackend::execute_profiled through the adapter (cpp/src/cuda/stage.cpp:234-239): the
// same outputs as execute() bit for bit, with "embedding", one "layer" per owned layer, then
// "to-wire" (a first stage of two) or "final_norm", "lm_head", "sampling" (a whole-model
// stage). And the factory's diagnostics (backend_factory.hpp:31-39): the bytes the library
// holds on the device follow stage creation and destruction, the peak resets to them, and
// the device reports its identity and free memory.
void gpu_adapter_profiled_and_diagnostics(const std::vector<std::string>& args) {
  CHECK(args.size() == 1);
  const fs::path dir = args[0];
  const model::ModelManifest m = model::manifest_from_checkpoint(dir);
  backend::StageOptions options;
  options.kv_cache_bytes = 16u << 20;
  options.kv_block_tokens = 32;
  options.max_sequences = 8;
  options.max_pass_rows = 64;
  backend::RocmBackendFactory factory(options);
  const runtime::MemoryAmounts capacity{1ull << 40, 1ull << 40, 0, 0};
  const auto before = factory.allocator_metrics();
  CHECK(before && before->cached_bytes == 0);
  std::atomic_bool go{false};
  const std::vector<std::uint64_t> prompt{1, 4, 2, 8, 3};
  {
    auto first = factory.load(request_for(m, 0, 2), dir, capacity);
    const auto held = factory.allocator_metrics();
    CHECK(held->active_bytes >= before->active_bytes + first->weight_memory().device_bytes);
    CHECK(held->peak_bytes >= held->active_bytes);
    auto a = first->allocate_sequence(8), b = first->allocate_sequence(8);
    const auto plain = std::get<runtime::BoundaryActivation>(first->execute(runtime::TokenInput{prompt}, 0, *a, go));
    runtime::ExecutionTiming timing;
    const auto timed = std::get<runtime::BoundaryActivation>(
        first->execute_profiled(runtime::TokenInput{prompt}, 0, *b, go, timing));
    CHECK(plain.tokens == timed.tokens && plain.payload == timed.payload);
    CHECK(timing.components.size() == 3);
    CHECK(timing.components[0].component == "embedding" && !timing.components[0].layer_index);
    CHECK(timing.components[1].component == "layer" && timing.components[1].layer_index == 0);
    CHECK(timing.components[2].component == "to-wire");
    for (const auto& c : timing.components) CHECK(c.milliseconds >= 0.0);
    {
      auto whole = factory.load(request_for(m, 0, 1), dir, capacity);
      CHECK(factory.allocator_metrics()->active_bytes > held->active_bytes);
      auto c = whole->allocate_sequence(8), d = whole->allocate_sequence(8);
      const auto t1 = std::get<runtime::SampledToken>(whole->execute(runtime::TokenInput{prompt}, 0, *c, go));
      runtime::ExecutionTiming t;
      const auto t2 = std::get<runtime::SampledToken>(whole->execute_profiled(runtime::TokenInput{prompt}, 0, *d, go, t));
      CHECK(t1.id == t2.id);
      std::vector<std::string> names;
      for (const auto& x : t.components) names.push_back(x.component);
      CHECK((names == std::vector<std::string>{"embedding", "layer", "layer", "final_norm", "lm_head", "sampling"}));
      CHECK(t.components[1].layer_index == 0 && t.components[2].layer_index == 1);
      // The sequences continue after a profiled pass.
      static_cast<void>(whole->execute_profiled(runtime::TokenInput{{t2.id}}, prompt.size(), *d, go, t));
      CHECK(t.components.size() == 6);
    }
    const auto after_whole = factory.allocator_metrics();
    CHECK(after_whole->active_bytes == held->active_bytes && after_whole->peak_bytes > held->active_bytes);
    CHECK(factory.profiling_reset_peak());
    CHECK(factory.allocator_metrics()->peak_bytes == held->active_bytes);
  }
  CHECK(factory.allocator_metrics()->active_bytes == before->active_bytes);
  const runtime::ProfilingDeviceInfo info = factory.profiling_device_info();
  CHECK((info.identity.size() == 16 || info.identity.size() == 32) && !info.name.empty() && info.available_bytes &&
        *info.available_bytes > 0);
  CHECK(factory.boundary_transport_mode() == "pinned");
  std::printf("DEVICE %s | %s | %s | driver %s\n", info.identity.c_str(), info.name.c_str(),
              info.backend_version.c_str(), info.driver_version.c_str());
}

// In-pass cancellation through the adapter: another thread sets the request's flag while
// the caller is inside execute(). A flag seen before the call throws without running
// anything, and the sequence continues; a flag seen inside the pass (between layers or when
// it completes) fails it with CANCELLED and the sequence is never resumed
// (cpp/src/cpu/stage.cpp:109-111; cpp/src/cuda/stage.cpp:357,396,456,463-468); a pass that
// completed first keeps its result. When the flag lands is up to timing: the attempts spread
// it over the pass, and at least one must land inside.
void gpu_adapter_cancellation(const std::vector<std::string>& args) {
  CHECK(args.size() == 1);
  const fs::path dir = args[0];
  const model::ModelManifest m = model::manifest_from_checkpoint(dir);
  backend::StageOptions options;
  options.kv_cache_bytes = 64u << 20;
  options.kv_block_tokens = 32;
  options.max_sequences = 8;
  options.max_pass_rows = 512;
  backend::RocmBackendFactory factory(options);
  auto stage = factory.load(request_for(m, 0, 1), dir, {1ull << 40, 1ull << 40, 0, 0});
  const std::vector<std::uint64_t> prompt(400, 3);
  std::atomic_bool no{false};
  int inside = 0, before = 0, completed = 0;
  for (int attempt = 0; attempt < 300 && inside < 3; ++attempt) {
    auto seq = stage->allocate_sequence(prompt.size() + 2);
    std::atomic_bool cancelled{false}, entered{false};
    const long spin = (attempt * 7919L) % 400000L;
    std::thread setter([&] {
      while (!entered.load()) std::this_thread::yield();
      for (volatile long i = 0; i < spin; i = i + 1) {
      }
      cancelled.store(true);
    });
    entered.store(true);
    try {
      static_cast<void>(stage->execute(runtime::TokenInput{prompt}, 0, *seq, cancelled));
      setter.join();
      ++completed;
    } catch (const runtime::Error& e) {
      setter.join();
      CHECK(e.code() == runtime::ErrorCode::kCancelled);
      ++inside;
      EXPECT_ERROR(stage->execute(runtime::TokenInput{{1}}, prompt.size(), *seq, no), kInvalidRequest);
      EXPECT_ERROR(stage->execute(runtime::TokenInput{prompt}, 0, *seq, no), kInvalidRequest);
    } catch (const std::runtime_error&) {
      setter.join();
      ++before;
      static_cast<void>(stage->execute(runtime::TokenInput{prompt}, 0, *seq, no));  // never started
    }
  }
  std::printf("CANCELLATION inside %d, before %d, completed %d\n", inside, before, completed);
  CHECK(inside >= 1);
  // The stage still serves other sequences.
  auto fresh = stage->allocate_sequence(8);
  static_cast<void>(stage->execute(runtime::TokenInput{{1, 4, 2}}, 0, *fresh, no));
}

struct Case {
  const char* name;
  std::function<void(const std::vector<std::string>&)> run;
  bool gpu;
};
const std::vector<Case>& cases() {
  static const std::vector<Case> all = {
      {"json_reader", [](auto&) { json_reader(); }, false},
      {"safetensors_reader", [](auto&) { safetensors_reader(); }, false},
      {"dense_admission", [](auto&) { dense_admission(); }, false},
      {"decode_batch_rules", [](auto&) { decode_batch_rules(); }, false},
      {"host_sampling", host_sampling, false},
      {"scheduler_mixed_passes", [](auto&) { scheduler_mixed_passes(); }, false},
      {"scheduler_large_prefill", [](auto&) { scheduler_large_prefill(); }, false},
      {"scheduler_retires_unready_requests", [](auto&) { scheduler_retires_unready_requests(); }, false},
      {"scheduler_in_flight_ok", [](auto&) { scheduler_in_flight(false); }, false},
      {"scheduler_in_flight_failure", [](auto&) { scheduler_in_flight(true); }, false},
      {"scheduler_without_mixed_passes", [](auto&) { scheduler_without_mixed_passes(true); }, false},
      {"scheduler_without_decode_batches", [](auto&) { scheduler_without_mixed_passes(false); }, false},
      {"scheduler_configuration", [](auto&) { scheduler_configuration(); }, false},
      {"scheduler_classifies_first_tokens_as_prefills", [](auto&) { scheduler_classifies_first_tokens_as_prefills(); }, false},
      {"scheduler_shutdown_with_queued_requests", [](auto&) { scheduler_shutdown(false); }, false},
      {"scheduler_shutdown_during_a_pass", [](auto&) { scheduler_shutdown(true); }, false},
      {"gpu_checkpoint_greedy", gpu_checkpoint_greedy, true},
      {"gpu_decode_batch_contract", gpu_decode_batch_contract, true},
      {"gpu_scheduler_mixed_pass", gpu_scheduler_mixed_pass, true},
      {"gpu_adapter_profiled_and_diagnostics", gpu_adapter_profiled_and_diagnostics, true},
      {"gpu_adapter_cancellation", gpu_adapter_cancellation, true},
  };
  return all;
}

}  // namespace

int main(int argc, char** argv) {
  if (argc < 2) {
    std::fprintf(stderr, "usage: host_tests --list | <case> [args]\n");
    return 2;
  }
  const std::string name = argv[1];
  if (name == "--list") {
    for (const Case& c : cases()) std::printf("%s %s\n", c.name, c.gpu ? "gpu" : "cpu");
    return 0;
  }
  for (const Case& c : cases()) {
    if (name != c.name) continue;
    try {
      c.run(std::vector<std::string>(argv + 2, argv + argc));
    } catch (const std::exception& e) {
      std::printf("FAIL %s: %s\n", c.name, e.what());
      return 1;
    }
    std::printf("PASS %s\n", c.name);
    return 0;
  }
  std::fprintf(stderr, "unknown case %s\n", name.c_str());
  return 2;
}
