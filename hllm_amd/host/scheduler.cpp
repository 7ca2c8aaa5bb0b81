#include "scheduler.hpp"

#include <algorithm>
#include <utility>

namespace hllm_rocm::worker {

using runtime::Error;
using Clock = std::chrono::steady_clock;

struct StageScheduler::Request {
  const runtime::StageBackend* backend{nullptr};
  runtime::DecodeBatchItem item;
  std::chrono::system_clock::time_point deadline;
  Clock::time_point queued;
  std::size_t rows{0};
  bool decode{false};
  bool claimed{false};   // taken into a pass: its result comes from that pass
  bool finished{false};
  std::optional<runtime::StageOutput> output;
  std::exception_ptr failure;
};

namespace {

std::size_t input_rows(const runtime::StageInput& input) {
  if (const auto* t = std::get_if<runtime::TokenInput>(&input)) return t->ids.size();
  return std::get<runtime::BoundaryActivation>(input).tokens;
}

}  // namespace

StageScheduler::StageScheduler() : dispatcher_([this] { dispatch_loop(); }) {}

// Shutdown: the running pass (if any) completes and delivers its results; requests still
// queued fail CANCELLED; destruction waits until every caller has left execute(), so no
// caller touches the scheduler's lock or condition variables after it is gone.
StageScheduler::~StageScheduler() {
  {
    std::scoped_lock lock(mutex_);
    stopping_ = true;
  }
  work_.notify_all();
  dispatcher_.join();
  std::unique_lock lock(mutex_);
  done_.wait(lock, [&] { return callers_ == 0; });
}

void StageScheduler::configure(const PassPolicy& policy) {
  if (policy.maximum_decode_rows == 0 || policy.maximum_decode_rows > kMaximumDecodeRows)
    throw Error::invalid_request("decode rows per pass must be between 1 and 64");
  if (policy.prefill_row_budget == 0) throw Error::invalid_request("the prefill row budget must be positive");
  std::scoped_lock lock(mutex_);
  policy_ = policy;
}

PassPolicy StageScheduler::policy() const {
  std::scoped_lock lock(mutex_);
  return policy_;
}

void StageScheduler::hold() {
  std::scoped_lock lock(mutex_);
  held_ = true;
}

void StageScheduler::resume() {
  {
    std::scoped_lock lock(mutex_);
    held_ = false;
  }
  work_.notify_all();
}

SchedulerMetrics StageScheduler::metrics() const {
  std::scoped_lock lock(mutex_);
  SchedulerMetrics m = totals_;
  m.queued_prefills = prefill_queue_.size();
  m.queued_decodes = decode_queue_.size();
  m.executing = executing_;
  return m;
}

runtime::StageOutput StageScheduler::execute(const runtime::StageBackend& backend, runtime::StageInput input,
                                             std::size_t position, runtime::SequenceState& sequence,
                                             const std::atomic_bool& cancelled,
                                             std::chrono::system_clock::time_point deadline) {
  Request r;
  r.backend = &backend;
  r.rows = input_rows(input);
  if (r.rows == 0) throw Error::invalid_request("empty stage input");
  // A decode continues a started sequence (cpp/src/worker/scheduler.cpp:48 classes position 0
  // and prefilling sequences as prefills); prefill-only sequences never join decode batches
  // (cpp/src/decode_batch.cpp:16-17).
  r.decode = r.rows == 1 && position != 0 && !sequence.prefilling && !sequence.prefill_only;
  r.item = runtime::DecodeBatchItem{std::move(input), position, &sequence, &cancelled};
  r.deadline = deadline;
  r.queued = Clock::now();
  std::unique_lock lock(mutex_);
  if (stopping_) throw Error::cancelled("the stage is shutting down");
  // Leaves under the lock (declared after it, destroyed before it): the destructor waits
  // for the last caller.
  struct Caller {
    StageScheduler& s;
    explicit Caller(StageScheduler& scheduler) : s(scheduler) { ++s.callers_; }
    ~Caller() {
      if (--s.callers_ == 0) s.done_.notify_all();
    }
  } caller(*this);
  (r.decode ? decode_queue_ : prefill_queue_).push_back(&r);
  work_.notify_one();
  // A queued request watches its own cancellation and deadline; once claimed it belongs to
  // its pass.
  while (!r.finished) {
    done_.wait_for(lock, std::chrono::milliseconds(2));
    if (r.finished || r.claimed) continue;
    const bool expired = std::chrono::system_clock::now() >= r.deadline;
    if (!cancelled.load() && !expired) continue;
    auto& queue = r.decode ? decode_queue_ : prefill_queue_;
    queue.erase(std::find(queue.begin(), queue.end(), &r));
    throw cancelled.load() ? Error::cancelled("request cancelled before dispatch")
                           : Error::deadline_exceeded("request deadline passed before dispatch");
  }
  if (r.failure) std::rethrow_exception(r.failure);
  return std::move(*r.output);
}

bool StageScheduler::retire_unready() {
  bool any = false;
  const auto now = std::chrono::system_clock::now();
  for (auto* queue : {&prefill_queue_, &decode_queue_}) {
    for (auto it = queue->begin(); it != queue->end();) {
      Request* r = *it;
      const bool cancelled = r->item.cancelled->load();
      if (!cancelled && now < r->deadline) {
        ++it;
        continue;
      }
      r->failure = std::make_exception_ptr(cancelled ? Error::cancelled("request cancelled before dispatch")
                                                     : Error::deadline_exceeded("request deadline passed before dispatch"));
      r->finished = true;
      it = queue->erase(it);
      any = true;
    }
  }
  return any;
}

std::vector<StageScheduler::Request*> StageScheduler::plan(bool& mixed) {
  // The pass serves the backend of the oldest waiting request.
  Request* oldest = nullptr;
  for (auto* queue : {&prefill_queue_, &decode_queue_})
    if (!queue->empty() && (!oldest || queue->front()->queued < oldest->queued)) oldest = queue->front();
  std::vector<Request*> pass;
  if (!oldest) return pass;
  const runtime::StageBackend* backend = oldest->backend;
  auto take = [&](std::deque<Request*>& queue, std::size_t limit, std::size_t row_budget) {
    std::size_t rows = 0, taken = 0;
    for (auto it = queue.begin(); it != queue.end() && taken < limit;) {
      Request* r = *it;
      if (r->backend != backend) {
        ++it;
        continue;
      }
      if (taken > 0 && rows + r->rows > row_budget) break;  // arrival order: no skipping ahead
      rows += r->rows;
      ++taken;
      pass.push_back(r);
      it = queue.erase(it);
    }
  };
  mixed = dynamic_cast<const MixedPassBackend*>(backend) != nullptr;
  if (mixed) {
    take(decode_queue_, policy_.maximum_decode_rows, SIZE_MAX);
    take(prefill_queue_, SIZE_MAX, policy_.prefill_row_budget);
    return pass;
  }
  auto waiting = [&](const std::deque<Request*>& queue) {
    return std::any_of(queue.begin(), queue.end(), [&](Request* r) { return r->backend == backend; });
  };
  const bool prefills = waiting(prefill_queue_), decodes = waiting(decode_queue_);
  bool prefill_next = prefills;
  if (prefills && decodes)
    prefill_next = last_kind_ == Kind::kNone ? !oldest->decode : last_kind_ == Kind::kDecode;
  if (prefill_next) {
    take(prefill_queue_, 1, SIZE_MAX);
    last_kind_ = Kind::kPrefill;
  } else {
    take(decode_queue_, backend->supports_decode_batch() ? policy_.maximum_decode_rows : 1, SIZE_MAX);
    last_kind_ = Kind::kDecode;
  }
  return pass;
}

void StageScheduler::run(const std::vector<Request*>& pass, bool mixed) {
  try {
    const runtime::StageBackend& backend = *pass.front()->backend;
    std::vector<runtime::StageOutput> outputs;
    if (mixed) {
      std::vector<runtime::DecodeBatchItem> items;
      items.reserve(pass.size());
      for (Request* r : pass) items.push_back(std::move(r->item));
      outputs = dynamic_cast<const MixedPassBackend&>(backend).execute_mixed(std::move(items));
    } else if (pass.size() == 1) {
      runtime::DecodeBatchItem& it = pass.front()->item;
      outputs.push_back(backend.execute(std::move(it.input), it.position, *it.sequence, *it.cancelled));
    } else {
      std::vector<runtime::DecodeBatchItem> items;
      items.reserve(pass.size());
      for (Request* r : pass) items.push_back(std::move(r->item));
      outputs = backend.execute_decode_batch(std::move(items));
    }
    if (outputs.size() != pass.size()) throw Error::internal("a pass returned the wrong number of outputs");
    for (std::size_t i = 0; i < pass.size(); ++i) pass[i]->output = std::move(outputs[i]);
  } catch (...) {
    const std::exception_ptr failure = std::current_exception();
    for (Request* r : pass) r->failure = failure;
  }
}

void StageScheduler::dispatch_loop() {
  std::unique_lock lock(mutex_);
  for (;;) {
    work_.wait(lock, [&] { return stopping_ || (!held_ && (!prefill_queue_.empty() || !decode_queue_.empty())); });
    if (stopping_) {
      for (auto* queue : {&prefill_queue_, &decode_queue_}) {
        for (Request* r : *queue) {
          r->failure = std::make_exception_ptr(Error::cancelled("the stage is shutting down"));
          r->finished = true;
        }
        queue->clear();
      }
      done_.notify_all();
      return;
    }
    if (retire_unready()) done_.notify_all();
    bool mixed = false;
    const std::vector<Request*> pass = plan(mixed);
    if (pass.empty()) continue;
    const auto now = Clock::now();
    std::size_t rows = 0, decodes = 0;
    for (Request* r : pass) {
      r->claimed = true;
      rows += r->rows;
      decodes += r->decode ? 1 : 0;
      totals_.queue_wait_ms += std::chrono::duration<double, std::milli>(now - r->queued).count();
    }
    executing_ = pass.size();
    lock.unlock();
    run(pass, mixed);
    lock.lock();
    executing_ = 0;
    totals_.passes += 1;
    totals_.completed_steps += pass.size();
    totals_.mixed_passes += decodes > 0 && decodes < pass.size() ? 1 : 0;
    totals_.decode_batches += decodes > 1 ? 1 : 0;
    totals_.largest_decode_batch = std::max(totals_.largest_decode_batch, decodes);
    totals_.largest_pass_rows = std::max(totals_.largest_pass_rows, rows);
    for (Request* r : pass) r->finished = true;
    done_.notify_all();
  }
}

}  // namespace hllm_rocm::worker
