#include "rocm_stage.hpp"

#include <cmath>
#include <cstring>
#include <limits>
#include <span>
#include <unordered_set>

namespace hllm_rocm::runtime {

void validate_sampling(const SamplingOptions& o) {
  const bool ok = std::isfinite(o.temperature) && o.temperature >= 0.0 && o.temperature <= 100.0 &&
                  std::isfinite(o.top_p) && o.top_p > 0.0 && o.top_p <= 1.0 && o.top_logprobs <= 5 &&
                  (o.return_logprobs || o.top_logprobs == 0);
  if (!ok) throw Error::invalid_request("invalid sampling parameters");
}

}  // namespace hllm_rocm::runtime

namespace hllm_rocm::backend {

using runtime::Error;

void check(hllm_status status) {
  if (status == HLLM_OK) return;
  const std::string message = hllm_rocm_last_error();
  switch (status) {
    case HLLM_INVALID_REQUEST: throw Error::invalid_request(message);
    case HLLM_INCOMPATIBLE_WORKER: throw Error::incompatible_worker(message);
    case HLLM_RESOURCE_EXHAUSTED: throw Error::resource_exhausted(message);
    case HLLM_DEADLINE_EXCEEDED: throw Error::deadline_exceeded(message);
    case HLLM_CANCELLED: throw Error::cancelled(message);
    default: throw Error::internal(message);
  }
}

void require_decode_batch(const std::vector<runtime::DecodeBatchItem>& items, std::size_t hidden) {
  if (items.empty() || items.size() > worker::StageScheduler::kMaximumDecodeRows)
    throw Error::invalid_request("a decode batch holds 1 to 64 members");
  const bool tokens = std::holds_alternative<runtime::TokenInput>(items.front().input);
  std::unordered_set<const runtime::SequenceState*> members;
  for (const runtime::DecodeBatchItem& it : items) {
    if (!it.sequence || !it.cancelled) throw Error::invalid_request("decode batch member without a sequence");
    if (!members.insert(it.sequence).second) throw Error::invalid_request("a sequence is in a decode batch twice");
    if (it.sequence->prefilling || it.sequence->prefill_only || it.position == 0)
      throw Error::invalid_request("decode batch members must be decoding started sequences");
    if (std::holds_alternative<runtime::TokenInput>(it.input) != tokens)
      throw Error::invalid_request("a decode batch mixes token and boundary inputs");
    if (const auto* t = std::get_if<runtime::TokenInput>(&it.input)) {
      if (t->ids.size() != 1) throw Error::invalid_request("a decode batch member carries one token");
    } else {
      const auto& b = std::get<runtime::BoundaryActivation>(it.input);
      if (b.tokens != 1 || b.width != hidden || b.payload.size() != hidden * 2)
        throw Error::invalid_request("a decode batch member carries one boundary row");
    }
  }
}

namespace {

// A sequence's paged KV blocks on the device; destroying the state returns them.
struct RocmSequence final : runtime::SequenceState {
  const RocmStage* owner{nullptr};
  std::uint32_t handle{0};
  std::size_t capacity{0};
  std::size_t length{0};
  bool failed{false};
  ~RocmSequence() override {
    if (owner) static_cast<void>(hllm_rocm_sequence_release(owner->handle(), handle));
  }
};

std::uint32_t abi_dtype(runtime::DataType d) {
  switch (d) {
    case runtime::DataType::kF32: return HLLM_DTYPE_F32;
    case runtime::DataType::kF16: return HLLM_DTYPE_F16;
    case runtime::DataType::kBF16: return HLLM_DTYPE_BF16;
    default: throw Error::incompatible_worker("unsupported tensor dtype");
  }
}

hllm_rocm_stage_config config_of(const model::DenseSource& s, const StageOptions& o) {
  hllm_rocm_stage_config c{};
  c.abi_version = HLLM_ROCM_ABI_VERSION;
  c.hidden_size = s.config.hidden_size;
  c.intermediate_size = s.config.intermediate_size;
  c.attention_heads = s.config.attention_heads;
  c.key_value_heads = s.config.key_value_heads;
  c.head_dimension = s.config.head_dimension;
  c.maximum_sequence_length = s.config.maximum_sequence_length;
  c.vocabulary_size = s.vocabulary_size;
  c.rms_norm_epsilon = s.config.rms_norm_epsilon;
  c.rope_theta = s.config.rope_theta;
  c.query_key_norm = s.config.query_key_norm;
  c.layer_start = s.layer_start;
  c.layer_end = s.layer_end;
  c.first_stage = s.first;
  c.final_stage = s.final;
  c.tied_head = s.tied_head;
  c.execution_dtype = abi_dtype(s.execution_dtype);
  c.weight_dtype = abi_dtype(s.weight_dtype);
  c.device = o.device;
  c.kv_cache_bytes = o.kv_cache_bytes;
  c.kv_block_tokens = o.kv_block_tokens;
  c.max_sequences = o.max_sequences;
  c.max_pass_rows = o.max_pass_rows;
  return c;
}

runtime::MemoryAmounts amounts(const hllm_rocm_memory& m) {
  return {m.host_bytes, m.device_bytes, m.pinned_host_bytes, m.unified_bytes};
}

}  // namespace

RocmStage::RocmStage(const model::DenseSource& source, const std::filesystem::path& root, const StageOptions& options)
    : config_(config_of(source, options)) {
  (void)root;
  check(hllm_rocm_stage_create(&config_, &stage_));
  try {
    // Payloads go to the device straight from the files' read-only mappings.
    for (const auto& [name, t] : source.tensors) {
      const runtime::SafetensorsFile& file = source.files.at(t.file);
      const std::span<const std::byte> payload = file.payload(file.tensor(name));
      std::vector<std::uint64_t> shape(t.shape.begin(), t.shape.end());
      check(hllm_rocm_stage_load_tensor(stage_, name.c_str(), abi_dtype(t.dtype), shape.data(),
                                        static_cast<std::uint32_t>(shape.size()), payload.data(), payload.size()));
    }
    check(hllm_rocm_stage_finalize(stage_));
  } catch (...) {
    hllm_rocm_stage_destroy(stage_);
    stage_ = nullptr;
    throw;
  }
}

RocmStage::RocmStage(hllm_rocm_stage* stage, const hllm_rocm_stage_config& config) : stage_(stage), config_(config) {
  if (!stage_) throw Error::internal("null stage");
}

RocmStage::~RocmStage() {
  if (stage_) hllm_rocm_stage_destroy(stage_);
}

runtime::MemoryAmounts RocmStage::weight_memory() const {
  hllm_rocm_memory m{};
  check(hllm_rocm_stage_weight_memory(stage_, &m));
  return amounts(m);
}

runtime::SequenceMemory RocmStage::sequence_memory(std::size_t tokens, std::size_t maximum_query_tokens) const {
  if (tokens == 0 || tokens > maximum_tokens()) throw Error::invalid_request("request exceeds model context capacity");
  hllm_rocm_memory cache{}, workspace{};
  check(hllm_rocm_stage_sequence_memory(stage_, tokens, runtime::query_rows(tokens, maximum_query_tokens), &cache,
                                        &workspace));
  return {amounts(cache), amounts(workspace)};
}

std::unique_ptr<runtime::SequenceState> RocmStage::allocate_sequence(std::size_t tokens) const {
  static_cast<void>(sequence_memory(tokens, tokens));
  auto state = std::make_unique<RocmSequence>();
  std::uint32_t handle = 0;
  check(hllm_rocm_sequence_allocate(stage_, tokens, &handle));
  state->owner = this;
  state->handle = handle;
  state->capacity = tokens;
  return state;
}

namespace {
int32_t poll_cancelled(void* flag) { return static_cast<const std::atomic_bool*>(flag)->load() ? 1 : 0; }
}  // namespace

std::vector<runtime::StageOutput> RocmStage::run(std::vector<Member>& members, bool batch_outputs,
                                                 const std::atomic_bool* cancelled,
                                                 runtime::ExecutionTiming* timing) const {
  std::scoped_lock lock(mutex_);
  const std::size_t n = members.size();
  const std::size_t hidden = config_.hidden_size;
  std::vector<hllm_rocm_item> items(n);
  std::vector<RocmSequence*> states(n);
  std::vector<std::uint64_t> ids;
  std::vector<std::uint16_t> rows;
  std::size_t total_rows = 0;
  bool logprobs = false;
  for (std::size_t i = 0; i < n; ++i) {
    auto* s = dynamic_cast<RocmSequence*>(members[i].state);
    if (!s || s->owner != this || s->failed || members[i].position != s->length)
      throw Error::invalid_request("ROCm sequence state or position is invalid");
    for (std::size_t j = 0; j < i; ++j)
      if (states[j] == s) throw Error::invalid_request("a pass holds each sequence once");
    states[i] = s;
    const auto* tokens = std::get_if<runtime::TokenInput>(members[i].input);
    const auto* boundary = std::get_if<runtime::BoundaryActivation>(members[i].input);
    const std::size_t count = tokens ? tokens->ids.size() : boundary->tokens;
    if ((tokens != nullptr) != (config_.first_stage != 0) || count == 0 || members[i].position > s->capacity ||
        count > s->capacity - members[i].position)
      throw Error::invalid_request("invalid ROCm stage input or context capacity");
    if (tokens) {
      ids.insert(ids.end(), tokens->ids.begin(), tokens->ids.end());
    } else {
      if (boundary->width != hidden || boundary->payload.size() != count * hidden * 2)
        throw Error::invalid_request("invalid ROCm boundary shape");
      const std::size_t at = rows.size();
      rows.resize(at + count * hidden);
      std::memcpy(rows.data() + at, boundary->payload.data(), boundary->payload.size());
    }
    hllm_rocm_item& it = items[i];
    it.sequence = s->handle;
    it.query_tokens = static_cast<std::uint32_t>(count);
    it.first_position = members[i].position;
    it.top_p = 1.0;
    if (config_.final_stage && !s->prefill_only) {
      // The device samples (cpp/src/cpu/stage.cpp:170-176 samples on the host).
      const runtime::SamplingOptions& o = s->sampling;
      runtime::validate_sampling(o);
      it.flags = HLLM_ITEM_SAMPLE | (o.return_logprobs ? HLLM_ITEM_LOGPROBS : 0u);
      it.top_logprobs = o.top_logprobs;
      it.temperature = o.temperature;
      it.top_p = o.top_p;
      it.top_k = o.top_k;
      it.seed = o.seed;
      it.generated_index = s->generated_index;
      logprobs |= o.return_logprobs;
    }
    total_rows += count;
  }
  if (total_rows > std::numeric_limits<std::uint32_t>::max()) throw Error::invalid_request("pass too large");

  hllm_rocm_pass pass{};
  pass.items = static_cast<std::uint32_t>(n);
  pass.item = items.data();
  pass.token_ids = config_.first_stage ? ids.data() : nullptr;
  pass.boundary_in = config_.first_stage ? nullptr : rows.data();
  std::vector<std::uint64_t> tokens_out(n, 0);
  std::vector<double> logprob_out, top_out;
  std::vector<std::uint64_t> top_ids_out;
  std::vector<std::uint16_t> boundary_out;
  if (config_.final_stage) {
    pass.tokens = tokens_out.data();
    if (logprobs) {
      logprob_out.resize(n);
      top_ids_out.resize(n * 5);
      top_out.resize(n * 5);
      pass.logprobs = logprob_out.data();
      pass.top_ids = top_ids_out.data();
      pass.top_logprobs = top_out.data();
    }
  } else {
    boundary_out.resize(total_rows * hidden);
    pass.boundary_out = boundary_out.data();
  }
  if (cancelled) {
    pass.cancel_poll = poll_cancelled;
    pass.cancel_context = const_cast<std::atomic_bool*>(cancelled);
  }
  hllm_status status = HLLM_OK;
  if (timing) {
    std::vector<hllm_rocm_phase_time> phases(config_.layer_end - config_.layer_start + 8);
    std::uint32_t count = 0;
    status = hllm_rocm_stage_execute_profiled(stage_, &pass, phases.data(), static_cast<std::uint32_t>(phases.size()),
                                              &count);
    if (status == HLLM_OK) {
      timing->components.clear();
      for (std::uint32_t i = 0; i < std::min<std::size_t>(count, phases.size()); ++i) {
        const hllm_rocm_phase_time& p = phases[i];
        timing->components.push_back({p.component, p.layer >= 0 ? std::optional<std::size_t>(p.layer) : std::nullopt,
                                      p.milliseconds});
      }
    }
  } else {
    status = hllm_rocm_stage_execute(stage_, &pass);
  }
  // A pass that failed inside (non-finite values) or was cancelled after it started may
  // have written part of the caches: its sequences are never resumed
  // (cpp/src/cuda/stage.cpp:463-468). Cancellation seen before the call throws earlier.
  if (status == HLLM_INTERNAL || status == HLLM_CANCELLED)
    for (RocmSequence* s : states) s->failed = true;
  check(status);

  std::vector<runtime::StageOutput> out;
  out.reserve(n);
  if (config_.final_stage) {
    for (std::size_t i = 0; i < n; ++i) {
      RocmSequence* s = states[i];
      if (!(items[i].flags & HLLM_ITEM_SAMPLE)) {
        out.emplace_back(runtime::PrefillProgress{});
        continue;
      }
      runtime::SampledToken token{tokens_out[i]};
      if (items[i].flags & HLLM_ITEM_LOGPROBS) {
        token.logprob = logprob_out[i];
        for (std::uint32_t r = 0; r < items[i].top_logprobs && top_ids_out[i * 5 + r] != UINT64_MAX; ++r)
          token.top_logprobs.push_back({top_ids_out[i * 5 + r], top_out[i * 5 + r]});
      }
      ++s->generated_index;  // every sampled token advances the counter (cpp/src/cpu/stage.cpp:175)
      out.emplace_back(std::move(token));
    }
  } else {
    std::size_t row = 0;
    if (!batch_outputs) {
      runtime::BoundaryActivation b{total_rows, hidden, std::vector<std::byte>(total_rows * hidden * 2)};
      std::memcpy(b.payload.data(), boundary_out.data(), b.payload.size());
      out.emplace_back(std::move(b));
    } else {
      for (std::size_t i = 0; i < n; ++i) {
        const std::size_t count = items[i].query_tokens;
        runtime::BoundaryActivation b{count, hidden, std::vector<std::byte>(count * hidden * 2)};
        std::memcpy(b.payload.data(), boundary_out.data() + row * hidden, b.payload.size());
        row += count;
        out.emplace_back(std::move(b));
      }
    }
  }
  for (std::size_t i = 0; i < n; ++i) states[i]->length += items[i].query_tokens;
  return out;
}

runtime::StageOutput RocmStage::execute(runtime::StageInput input, std::size_t first_position,
                                        runtime::SequenceState& state, const std::atomic_bool& cancelled) const {
  if (cancelled.load()) throw std::runtime_error("request cancelled");
  std::vector<Member> members{{&input, first_position, &state}};
  auto out = run(members, false, &cancelled);
  return std::move(out.front());
}

runtime::StageOutput RocmStage::execute_profiled(runtime::StageInput input, std::size_t first_position,
                                                 runtime::SequenceState& state, const std::atomic_bool& cancelled,
                                                 runtime::ExecutionTiming& timing) const {
  timing = {};
  if (cancelled.load()) throw std::runtime_error("request cancelled");
  std::vector<Member> members{{&input, first_position, &state}};
  auto out = run(members, false, &cancelled, &timing);
  return std::move(out.front());
}

std::vector<runtime::StageOutput> RocmStage::execute_decode_batch(std::vector<runtime::DecodeBatchItem> items) const {
  require_decode_batch(items, config_.hidden_size);
  // An in-flight batch is not preempted: a member's cancellation is its caller's to observe.
  std::vector<Member> members;
  members.reserve(items.size());
  for (auto& item : items) members.push_back({&item.input, item.position, item.sequence});
  return run(members, true);
}

std::vector<runtime::StageOutput> RocmStage::execute_mixed(std::vector<runtime::DecodeBatchItem> items) const {
  if (items.empty()) throw Error::invalid_request("empty pass");
  std::vector<Member> members;
  members.reserve(items.size());
  for (auto& item : items) {
    if (!item.sequence) throw Error::invalid_request("pass member without a sequence");
    members.push_back({&item.input, item.position, item.sequence});
  }
  return run(members, true);
}

BackendCapabilities RocmBackendFactory::capabilities() const {
  BackendCapabilities c;
  c.kind = "ROCM";
  c.primary_memory_domain = "DEVICE";
  c.architectures = {"llama.v1", "qwen3.v1"};
  c.execution_dtypes = {"F16", "F32"};
  c.detail = "hllm-rocm stage worker (gfx950, ABI " + std::to_string(hllm_rocm_abi_version()) + ")";
  c.supports_mixed_precision = true;
  return c;
}

std::optional<runtime::AllocatorMetrics> RocmBackendFactory::allocator_metrics() const {
  hllm_rocm_allocator_metrics m{};
  check(hllm_rocm_device_allocator_metrics(options_.device, &m));
  return runtime::AllocatorMetrics{m.active_bytes, m.cached_bytes, m.peak_bytes};
}

bool RocmBackendFactory::profiling_reset_peak() const {
  check(hllm_rocm_device_reset_peak(options_.device));
  return true;
}

runtime::ProfilingDeviceInfo RocmBackendFactory::profiling_device_info() const {
  hllm_rocm_device_info d{};
  check(hllm_rocm_device_query(options_.device, &d));
  auto text = [](const char* s, std::size_t n) { return std::string(s, strnlen(s, n)); };
  return {text(d.identity, sizeof(d.identity)),
          text(d.name, sizeof(d.name)) + " (" + text(d.architecture, sizeof(d.architecture)) + ")",
          "HIP " + std::to_string(d.runtime_version) + ", hllm-rocm ABI " + std::to_string(hllm_rocm_abi_version()),
          std::to_string(d.driver_version),
          "hllm-rocm (reserved at stage creation)",
          static_cast<std::size_t>(d.available_bytes)};
}

std::unique_ptr<runtime::StageBackend> RocmBackendFactory::load(const model::LoadStageRequest& request,
                                                                const std::filesystem::path& root,
                                                                const runtime::MemoryAmounts& capacity) const {
  model::DenseSource source = model::inspect_dense_stage(request, root);
  if (source.resident_bytes > capacity.device_bytes)
    throw Error::resource_exhausted("stage weights exceed the device memory budget");
  if (source.largest_payload_bytes > capacity.host_bytes)
    throw Error::resource_exhausted("largest tensor exceeds the host memory budget for loading");
  return std::make_unique<RocmStage>(source, root, options_);
}

}  // namespace hllm_rocm::backend
