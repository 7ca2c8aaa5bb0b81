// The worker's pass scheduler (cpp/include/hllm/worker/scheduler.hpp,
// cpp/src/worker/scheduler.cpp:27-133): callers block in execute() with their own input;
// the first caller able to dispatch leads one pass for itself and the queued decode
// members it claims. Prefills run alone in FIFO order; decodes are batched up to the
// configured size; after a streak of decode items a waiting prefill goes next. Cancelled
// or expired tickets are retired before they reach the backend.
#pragma once

#include <chrono>
#include <condition_variable>
#include <deque>
#include <exception>
#include <mutex>
#include <optional>

#include "runtime.hpp"

namespace hllm_rocm::worker {

struct SchedulerMetrics {
  std::size_t queued_prefills{};
  std::size_t queued_decodes{};
  std::size_t executing{};
  std::size_t completed_steps{};
  double queue_wait_ms{};
  std::size_t decode_batches{};
  std::size_t largest_decode_batch{};
};

class StageScheduler final {
 public:
  // Decode batches of 1..kMaximumDecodeBatch members. The reference caps batches at 8;
  // this worker's passes take up to 64 decode rows, the combine limit of the contract.
  static constexpr std::size_t kMaximumDecodeBatch = 64;
  static constexpr std::size_t kMaximumDecodeStreak = 8;

  void configure(std::size_t maximum_decode_batch, std::size_t decode_streak = kMaximumDecodeStreak);
  runtime::StageOutput execute(const runtime::StageBackend& backend, runtime::StageInput input,
                               std::size_t position, runtime::SequenceState& sequence,
                               const std::atomic_bool& cancelled,
                               std::chrono::system_clock::time_point deadline);
  SchedulerMetrics metrics() const;

 private:
  struct Ticket {
    runtime::DecodeBatchItem item;
    std::chrono::system_clock::time_point deadline;
    std::chrono::steady_clock::time_point queued;
    bool claimed{false}, done{false};
    std::optional<runtime::StageOutput> result;
    std::exception_ptr error;
  };
  Ticket* next() const;
  void retire(Ticket* ticket);

  mutable std::mutex mutex_;
  std::condition_variable ready_;
  std::deque<Ticket*> prefills_, decodes_;
  std::size_t maximum_decode_batch_{1};
  std::size_t decode_streak_limit_{kMaximumDecodeStreak};
  std::size_t executing_{0};
  std::size_t decode_streak_{0};
  std::size_t completed_steps_{0};
  double queue_wait_ms_{0};
  std::size_t decode_batches_{0}, largest_decode_batch_{0};
};

}  // namespace hllm_rocm::worker
