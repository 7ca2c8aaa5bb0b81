// The MI355X stage as a StageBackend (cpp/include/hllm/runtime/stage_backend.hpp:69-107),
// implemented over the C ABI of include/hllm_rocm.h, and its factory
// (cpp/include/hllm/runtime/backend_factory.hpp:28-47). This is the adapter a reference
// worker binary links in place of its CPU or CUDA stage.
#pragma once

#include <memory>
#include <mutex>
#include <string>
#include <vector>

#include "dense_loader.hpp"
#include "hllm_rocm.h"
#include "runtime.hpp"
#include "scheduler.hpp"

namespace hllm_rocm::backend {

struct StageOptions {
  int device{0};
  std::size_t kv_cache_bytes{0};     // 0: 90% of free HBM after weights
  std::uint32_t kv_block_tokens{0};  // 0: 64
  std::uint32_t max_sequences{0};    // 0: 512
  std::uint32_t max_pass_rows{0};    // 0: 2048
};

// Translates a failed C-ABI call into the runtime's error categories.
void check(hllm_status status);

// The decode-batch contract (cpp/include/hllm/runtime/stage_backend.hpp:52-58,93-101): 1..64
// members, each one row (a token, or a boundary row `hidden` wide) of a distinct sequence that
// has started, is not prefilling and is not prefill-only (cpp/src/decode_batch.cpp:8-24), all
// with the same kind of input. INVALID_REQUEST otherwise.
void require_decode_batch(const std::vector<runtime::DecodeBatchItem>& items, std::size_t hidden);

class RocmStage final : public runtime::StageBackend, public worker::MixedPassBackend {
 public:
  // Creates the device stage for an admitted dense source and uploads its tensors.
  RocmStage(const model::DenseSource& source, const std::filesystem::path& root, const StageOptions& options);
  // Takes ownership of a stage built directly through the C ABI (finalized).
  RocmStage(hllm_rocm_stage* stage, const hllm_rocm_stage_config& config);
  ~RocmStage() override;
  RocmStage(const RocmStage&) = delete;
  RocmStage& operator=(const RocmStage&) = delete;

  runtime::MemoryAmounts weight_memory() const override;
  std::size_t hidden_size() const override { return config_.hidden_size; }
  std::size_t vocabulary_size() const override { return config_.vocabulary_size; }
  std::size_t maximum_tokens() const override { return config_.maximum_sequence_length; }
  runtime::SequenceMemory sequence_memory(std::size_t tokens, std::size_t maximum_query_tokens) const override;
  using runtime::StageBackend::sequence_memory;
  std::unique_ptr<runtime::SequenceState> allocate_sequence(std::size_t tokens) const override;
  // The pass honours `cancelled` between layers and once more when it completes; a pass
  // cancelled after it started fails its sequence (never resumed, cpp/src/cuda/stage.cpp:463-468).
  runtime::StageOutput execute(runtime::StageInput input, std::size_t first_position, runtime::SequenceState& state,
                               const std::atomic_bool& cancelled) const override;
  // execute() with HIP events between phases on the stage's stream: "embedding" or
  // "from-wire", one "layer" per owned layer, then "final_norm", "lm_head", "sampling" or
  // "to-wire" (cpp/src/cuda/stage.cpp:234-239). Outputs equal execute()'s bit for bit.
  runtime::StageOutput execute_profiled(runtime::StageInput input, std::size_t first_position,
                                        runtime::SequenceState& state, const std::atomic_bool& cancelled,
                                        runtime::ExecutionTiming& timing) const override;
  bool supports_decode_batch() const override { return true; }
  std::vector<runtime::StageOutput> execute_decode_batch(std::vector<runtime::DecodeBatchItem> items) const override;

  // One ragged pass over any mix of prefill chunks and one-token decode inputs of distinct
  // sequences (the reference contract runs these as separate passes). Outputs in item order.
  std::vector<runtime::StageOutput> execute_mixed(std::vector<runtime::DecodeBatchItem> items) const override;

  hllm_rocm_stage* handle() const { return stage_; }
  const hllm_rocm_stage_config& config() const { return config_; }

 private:
  struct Member {
    runtime::StageInput* input;
    std::size_t position;
    runtime::SequenceState* state;
  };
  // `cancelled`: checked inside the pass (single-sequence execution only; batches are not
  // preempted). `timing`: a profiled pass.
  std::vector<runtime::StageOutput> run(std::vector<Member>& members, bool batch_outputs,
                                        const std::atomic_bool* cancelled = nullptr,
                                        runtime::ExecutionTiming* timing = nullptr) const;

  hllm_rocm_stage* stage_{nullptr};
  hllm_rocm_stage_config config_{};
  mutable std::mutex mutex_;
};

struct BackendCapabilities {
  std::string kind;                  // "ROCM" (proto/profile.proto Backend needs this value)
  std::string primary_memory_domain; // "DEVICE"
  std::vector<std::string> architectures;
  std::vector<std::string> execution_dtypes;
  std::string detail;
  bool supports_mixed_precision{true};
};

class RocmBackendFactory {
 public:
  explicit RocmBackendFactory(StageOptions options = {}) : options_(options) {}
  BackendCapabilities capabilities() const;
  // backend_factory.hpp:31-39: the device memory the library holds on the factory's device
  // (no caching allocator: cached_bytes 0), boundary rows staged through pinned host memory,
  // a peak reset after the device's work completes, and the device's identity.
  std::optional<runtime::AllocatorMetrics> allocator_metrics() const;
  std::string boundary_transport_mode() const { return "pinned"; }
  bool profiling_reset_peak() const;
  runtime::ProfilingDeviceInfo profiling_device_info() const;
  // Validates the request and the memory budget, then returns a complete stage (nothing
  // is published on failure: the partially built stage is destroyed).
  std::unique_ptr<runtime::StageBackend> load(const model::LoadStageRequest& request,
                                              const std::filesystem::path& root,
                                              const runtime::MemoryAmounts& capacity) const;

 private:
  StageOptions options_;
};

}  // namespace hllm_rocm::backend
