// The stage-backend contract the ROCm worker is a drop-in for, restated in this
// repository's own namespace: the same type names, fields and error categories as the
// reference runtime (cpp/include/hllm/runtime/stage_backend.hpp,
// cpp/include/hllm/runtime/error.hpp, cpp/include/hllm/runtime/memory.hpp,
// cpp/include/hllm/runtime/sampling.hpp), so an adapter in the reference tree is a field
// copy between the two.
#pragma once

#include <atomic>
#include <cstddef>
#include <cstdint>
#include <memory>
#include <optional>
#include <stdexcept>
#include <string>
#include <variant>
#include <vector>

namespace hllm_rocm::runtime {

// error.hpp:10-17
enum class ErrorCode {
  kInvalidRequest,
  kIncompatibleWorker,
  kResourceExhausted,
  kDeadlineExceeded,
  kCancelled,
  kInternal,
};

// error.hpp:19-40: a category the worker services translate to wire codes.
class Error : public std::runtime_error {
 public:
  Error(ErrorCode code, const std::string& message) : std::runtime_error(message), code_(code) {}
  [[nodiscard]] ErrorCode code() const noexcept { return code_; }
  static Error invalid_request(const std::string& m) { return {ErrorCode::kInvalidRequest, m}; }
  static Error incompatible_worker(const std::string& m) { return {ErrorCode::kIncompatibleWorker, m}; }
  static Error resource_exhausted(const std::string& m) { return {ErrorCode::kResourceExhausted, m}; }
  static Error deadline_exceeded(const std::string& m) { return {ErrorCode::kDeadlineExceeded, m}; }
  static Error cancelled(const std::string& m) { return {ErrorCode::kCancelled, m}; }
  static Error internal(const std::string& m) { return {ErrorCode::kInternal, m}; }

 private:
  ErrorCode code_;
};

// memory.hpp:11-17, 46-49
struct MemoryAmounts {
  std::size_t host_bytes{0};
  std::size_t device_bytes{0};
  std::size_t pinned_host_bytes{0};
  std::size_t unified_bytes{0};
};
struct SequenceMemory {
  MemoryAmounts cache;
  MemoryAmounts workspace;
};

// sampling.hpp:10-28
struct SamplingOptions {
  double temperature{0.0};
  double top_p{1.0};
  std::uint64_t top_k{0};
  std::uint64_t seed{0};
  bool return_logprobs{false};
  std::uint32_t top_logprobs{0};
};
struct TokenLogProbability {
  std::uint64_t token_id;
  double logprob;
};
struct SampledToken {
  std::uint64_t id{};
  std::optional<double> logprob{};
  std::vector<TokenLogProbability> top_logprobs{};
};

// stage_backend.hpp:20-58
struct BoundaryActivation {
  std::size_t tokens;
  std::size_t width;
  std::vector<std::byte> payload;  // row-major little-endian F16, tokens * width * 2 bytes
};
struct TokenInput {
  std::vector<std::uint64_t> ids;
};
using StageInput = std::variant<TokenInput, BoundaryActivation>;
struct PrefillProgress {};
using StageOutput = std::variant<BoundaryActivation, SampledToken, PrefillProgress>;

struct SequenceState {
  SamplingOptions sampling;
  bool prefilling{false};
  bool prefill_only{false};
  std::uint64_t generated_index{0};
  virtual ~SequenceState() = default;
};

struct DecodeBatchItem {
  StageInput input;
  std::size_t position;
  SequenceState* sequence;
  const std::atomic_bool* cancelled;
};

// timing.hpp:11-18: per-phase times of a profiled execution.
struct ComponentTiming {
  std::string component;
  std::optional<std::size_t> layer_index;
  double milliseconds;
};
struct ExecutionTiming {
  std::vector<ComponentTiming> components;
};

// stage_backend.hpp:62-67
[[nodiscard]] constexpr std::size_t query_rows(std::size_t tokens, std::size_t maximum_query_tokens) noexcept {
  return maximum_query_tokens == 0 || maximum_query_tokens > tokens ? tokens : maximum_query_tokens;
}

// stage_backend.hpp:69-107
class StageBackend {
 public:
  virtual ~StageBackend() = default;
  [[nodiscard]] virtual MemoryAmounts weight_memory() const = 0;
  [[nodiscard]] virtual std::size_t hidden_size() const = 0;
  [[nodiscard]] virtual std::size_t vocabulary_size() const = 0;
  [[nodiscard]] virtual std::size_t maximum_tokens() const = 0;
  [[nodiscard]] virtual SequenceMemory sequence_memory(std::size_t tokens,
                                                       std::size_t maximum_query_tokens) const = 0;
  [[nodiscard]] SequenceMemory sequence_memory(std::size_t tokens) const {
    return sequence_memory(tokens, tokens);
  }
  [[nodiscard]] virtual std::unique_ptr<SequenceState> allocate_sequence(std::size_t tokens) const = 0;
  [[nodiscard]] virtual StageOutput execute(StageInput input, std::size_t first_position,
                                            SequenceState& state,
                                            const std::atomic_bool& cancelled) const = 0;
  virtual bool supports_decode_batch() const { return false; }
  virtual std::vector<StageOutput> execute_decode_batch(std::vector<DecodeBatchItem> items) const {
    std::vector<StageOutput> outputs;
    for (auto& item : items)
      outputs.push_back(execute(std::move(item.input), item.position, *item.sequence, *item.cancelled));
    return outputs;
  }
  // Diagnostics for profiling processes (stage_backend.hpp:102-106); serving uses execute().
  [[nodiscard]] virtual StageOutput execute_profiled(StageInput, std::size_t, SequenceState&,
                                                     const std::atomic_bool&, ExecutionTiming&) const {
    throw std::logic_error("backend does not implement compute profiling");
  }
};

// backend_factory.hpp:24-26 and profiling.hpp:8-15: the factory's allocator and device
// diagnostics.
struct AllocatorMetrics {
  std::size_t active_bytes, cached_bytes, peak_bytes;
};
struct ProfilingDeviceInfo {
  std::string identity;
  std::string name;
  std::string backend_version;
  std::string driver_version;
  std::string allocator;
  std::optional<std::size_t> available_bytes;
};

// cpp/src/sampling.cpp:10-17: the options every sampled pass is checked against
// (INVALID_REQUEST otherwise). Stage passes sample on the device.
void validate_sampling(const SamplingOptions& options);

}  // namespace hllm_rocm::runtime
