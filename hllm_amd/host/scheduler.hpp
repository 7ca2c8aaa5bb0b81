// Pass scheduling for one stage: RPC threads hand in their own stage inputs and block until
// their result is ready, as with the reference's StageScheduler
// (cpp/include/hllm/worker/scheduler.hpp; cpp/src/worker/scheduler.cpp:27-133), but passes are
// composed differently. A dispatcher thread owned by the scheduler builds each pass from two
// FIFO queues:
//
//  * every waiting decode (one token of a sequence that is not prefilling), up to
//    `maximum_decode_rows`;
//  * waiting prefill inputs in arrival order while their rows fit `prefill_row_budget`
//    (the first one always goes, whatever its size).
//
// A backend that runs mixed passes (MixedPassBackend: the ROCm stage) gets both in one pass.
// Any other backend gets the reference's pass kinds: a prefill alone or a decode batch,
// alternating while both queues hold work (the first such pass serves the older request).
//
// Guarantees kept from the reference: arrival order within each queue; neither queue starves
// the other; a request cancelled or past its deadline before dispatch never reaches the
// backend (CANCELLED / DEADLINE_EXCEEDED); a request whose pass is running gets that pass's
// result or failure, whatever happens to its cancellation flag meanwhile. Destroying the
// scheduler lets a running pass finish, fails the queued requests CANCELLED and returns
// once every caller has left execute().
#pragma once

#include <atomic>
#include <chrono>
#include <condition_variable>
#include <cstddef>
#include <deque>
#include <exception>
#include <mutex>
#include <optional>
#include <thread>
#include <vector>

#include "runtime.hpp"

namespace hllm_rocm::worker {

// A backend that runs prefill chunks and decode rows of different sequences in one pass;
// outputs in item order.
class MixedPassBackend {
 public:
  virtual ~MixedPassBackend() = default;
  virtual std::vector<runtime::StageOutput> execute_mixed(std::vector<runtime::DecodeBatchItem> items) const = 0;
};

struct PassPolicy {
  std::size_t maximum_decode_rows{64};   // decode rows per pass, 1..kMaximumDecodeRows
  std::size_t prefill_row_budget{512};   // prefill rows per mixed pass (chunked-prefill budget)
};

struct SchedulerMetrics {
  std::size_t queued_prefills{};
  std::size_t queued_decodes{};
  std::size_t executing{};          // requests in the running pass
  std::size_t completed_steps{};    // requests completed by a pass
  std::size_t passes{};
  std::size_t mixed_passes{};       // passes holding prefill and decode rows
  std::size_t decode_batches{};     // passes with more than one decode row
  std::size_t largest_decode_batch{};
  std::size_t largest_pass_rows{};
  double queue_wait_ms{};           // summed over dispatched requests
};

class StageScheduler final {
 public:
  // Rows of a decode batch the device passes take (the contract's combine limit).
  static constexpr std::size_t kMaximumDecodeRows = 64;

  StageScheduler();
  ~StageScheduler();
  StageScheduler(const StageScheduler&) = delete;
  StageScheduler& operator=(const StageScheduler&) = delete;

  // INVALID_REQUEST for a decode limit outside 1..64 or a zero prefill budget.
  void configure(const PassPolicy& policy);
  void configure(std::size_t maximum_decode_rows) { configure(PassPolicy{maximum_decode_rows, policy().prefill_row_budget}); }
  PassPolicy policy() const;

  // Blocks until the request's pass has run; returns its output or rethrows its failure.
  runtime::StageOutput execute(const runtime::StageBackend& backend, runtime::StageInput input,
                               std::size_t position, runtime::SequenceState& sequence,
                               const std::atomic_bool& cancelled,
                               std::chrono::system_clock::time_point deadline);
  SchedulerMetrics metrics() const;

  // Holds dispatch (queued requests wait) until resume(): for draining and for tests that
  // need several requests queued before a pass is built.
  void hold();
  void resume();

 private:
  struct Request;
  void dispatch_loop();
  bool retire_unready();  // under mutex_: completes cancelled / expired queued requests
  std::vector<Request*> plan(bool& mixed);
  void run(const std::vector<Request*>& pass, bool mixed);

  mutable std::mutex mutex_;
  std::condition_variable work_, done_;
  std::deque<Request*> prefill_queue_, decode_queue_;
  PassPolicy policy_{};
  bool held_{false}, stopping_{false};
  // Backends without mixed passes: the kind of the previous pass (alternation).
  enum class Kind { kNone, kPrefill, kDecode };
  Kind last_kind_{Kind::kNone};
  SchedulerMetrics totals_{};
  std::size_t executing_{0};
  std::size_t callers_{0};  // threads inside execute()
  std::thread dispatcher_;
};

}  // namespace hllm_rocm::worker
