#include "scheduler.hpp"

#include <algorithm>
#include <array>

namespace hllm_rocm::worker {

using Clock = std::chrono::system_clock;

void StageScheduler::configure(std::size_t maximum_decode_batch, std::size_t decode_streak) {
  if (maximum_decode_batch == 0 || maximum_decode_batch > kMaximumDecodeBatch)
    throw runtime::Error::invalid_request("decode batch size must be between 1 and 64");
  if (decode_streak == 0) throw runtime::Error::invalid_request("decode streak must be positive");
  std::scoped_lock lock(mutex_);
  if (executing_ || !prefills_.empty() || !decodes_.empty())
    throw runtime::Error::internal("cannot reconfigure an active scheduler");
  maximum_decode_batch_ = maximum_decode_batch;
  decode_streak_limit_ = decode_streak;
}

// The ticket allowed to lead the next pass: the oldest prefill when no decode waits or
// the decode streak is spent, else the oldest decode.
StageScheduler::Ticket* StageScheduler::next() const {
  if (!prefills_.empty() && (decodes_.empty() || decode_streak_ >= decode_streak_limit_)) return prefills_.front();
  if (!decodes_.empty()) return decodes_.front();
  return nullptr;
}

// Marks a claimed ticket done with the reason it cannot run (deadline before cancel).
void StageScheduler::retire(Ticket* t) {
  try {
    if (Clock::now() >= t->deadline) throw runtime::Error::deadline_exceeded("deadline expired in native queue");
    throw runtime::Error::cancelled("request cancelled in native queue");
  } catch (...) {
    t->error = std::current_exception();
  }
  t->done = true;
}

runtime::StageOutput StageScheduler::execute(const runtime::StageBackend& backend, runtime::StageInput input,
                                             std::size_t position, runtime::SequenceState& sequence,
                                             const std::atomic_bool& cancelled, Clock::time_point deadline) {
  Ticket ticket{{std::move(input), position, &sequence, &cancelled}, deadline, std::chrono::steady_clock::now(),
                false, false, {}, {}};
  const bool batching = backend.supports_decode_batch();
  const bool prefill = position == 0 || sequence.prefilling;
  std::unique_lock lock(mutex_);
  auto& queue = prefill ? prefills_ : decodes_;
  queue.push_back(&ticket);
  while (!ticket.done) {
    if (!ticket.claimed && (cancelled.load() || Clock::now() >= deadline)) {
      queue.erase(std::find(queue.begin(), queue.end(), &ticket));
      ready_.notify_all();
      if (Clock::now() >= deadline) throw runtime::Error::deadline_exceeded("deadline expired in native queue");
      throw runtime::Error::cancelled("request cancelled in native queue");
    }
    if (ticket.claimed || executing_ || next() != &ticket) {
      ready_.wait_for(lock, std::chrono::milliseconds(5));
      continue;
    }
    // Lead a pass. Claiming does not allocate: claimed callers cannot leave.
    std::array<Ticket*, kMaximumDecodeBatch> claimed{};
    std::size_t count = 0;
    std::size_t limit = prefill || !batching ? 1 : maximum_decode_batch_;
    if (!prefill && !prefills_.empty()) limit = std::min(limit, decode_streak_limit_ - decode_streak_);
    while (!queue.empty() && count < limit) {
      Ticket* member = queue.front();
      queue.pop_front();
      member->claimed = true;
      if (member->item.cancelled->load() || Clock::now() >= member->deadline) {
        retire(member);
        continue;
      }
      claimed[count++] = member;
      queue_wait_ms_ +=
          std::chrono::duration<double, std::milli>(std::chrono::steady_clock::now() - member->queued).count();
    }
    if (count == 0) {
      ready_.notify_all();
      continue;
    }
    executing_ = count;
    decode_streak_ = prefill ? 0 : std::min(decode_streak_ + count, decode_streak_limit_);
    lock.unlock();
    std::vector<runtime::StageOutput> outputs;
    std::exception_ptr failure;
    try {
      if (count == 1) {
        runtime::DecodeBatchItem& item = claimed[0]->item;
        outputs.push_back(backend.execute(std::move(item.input), item.position, *item.sequence, *item.cancelled));
      } else {
        std::vector<runtime::DecodeBatchItem> items;
        items.reserve(count);
        for (std::size_t i = 0; i < count; ++i) items.push_back(std::move(claimed[i]->item));
        outputs = backend.execute_decode_batch(std::move(items));
        if (outputs.size() != count) throw runtime::Error::internal("batch output count mismatch");
      }
    } catch (...) {
      failure = std::current_exception();
    }
    lock.lock();
    for (std::size_t i = 0; i < count; ++i) {
      claimed[i]->error = failure;
      if (!failure) claimed[i]->result.emplace(std::move(outputs[i]));
      claimed[i]->done = true;
    }
    completed_steps_ += count;
    if (count > 1) {
      ++decode_batches_;
      largest_decode_batch_ = std::max(largest_decode_batch_, count);
    }
    executing_ = 0;
    ready_.notify_all();
  }
  if (ticket.error) std::rethrow_exception(ticket.error);
  return std::move(*ticket.result);
}

SchedulerMetrics StageScheduler::metrics() const {
  std::scoped_lock lock(mutex_);
  return {prefills_.size(), decodes_.size(), executing_, completed_steps_, queue_wait_ms_, decode_batches_,
          largest_decode_batch_};
}

}  // namespace hllm_rocm::worker
