// Host restatement of the reference's sampler (cpp/src/sampling.cpp:19-89) for the host
// tests: temperature in double precision, candidates sorted by probability (ties by lower
// token ID), top-k, then the smallest prefix whose mass reaches top_p of the total, and a
// SplitMix64 counter draw (seed + golden-ratio increment * (generated_index + 1)) scaled to
// the retained mass. The product samples on the device (hllm_amd/csrc/sampling.hip); this
// file is built into the host test program only, which checks it against the sampling
// vectors the device sampler is also checked against.
#include "host_sampling.hpp"

#include <algorithm>
#include <cmath>

namespace hllm_rocm::runtime {

namespace {
// Finalizer of Vigna's SplitMix64 applied to the request's counter.
std::uint64_t counter_bits(std::uint64_t seed, std::uint64_t index) {
  std::uint64_t z = seed + 0x9e3779b97f4a7c15ull * (index + 1);
  z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ull;
  z = (z ^ (z >> 27)) * 0x94d049bb133111ebull;
  return z ^ (z >> 31);
}
}  // namespace

std::uint64_t sample_logits(const float* logits, std::size_t count, const SamplingOptions& options,
                            std::uint64_t generated_index) {
  validate_sampling(options);
  if (count == 0) throw Error::internal("cannot sample empty logits");
  std::size_t best = 0;
  for (std::size_t i = 0; i < count; ++i) {
    if (!std::isfinite(logits[i])) throw Error::internal("cannot sample nonfinite logits");
    if (logits[i] > logits[best]) best = i;
  }
  if (options.temperature == 0.0) return best;
  struct Weighted {
    double p;
    std::uint64_t id;
  };
  std::vector<Weighted> order(count);
  const double top = logits[best];
  for (std::size_t i = 0; i < count; ++i)
    order[i] = {std::exp((static_cast<double>(logits[i]) - top) / options.temperature), i};
  std::sort(order.begin(), order.end(),
            [](const Weighted& a, const Weighted& b) { return a.p != b.p ? a.p > b.p : a.id < b.id; });
  if (options.top_k != 0 && options.top_k < order.size()) order.resize(options.top_k);
  double mass = 0.0;
  for (const Weighted& w : order) mass += w.p;
  const double threshold = mass * options.top_p;
  double kept = 0.0;
  std::size_t keep = 0;
  do {
    kept += order[keep++].p;
  } while (kept < threshold && keep < order.size());
  double target = static_cast<double>(counter_bits(options.seed, generated_index) >> 11) * 0x1.0p-53 * kept;
  for (std::size_t i = 0; i + 1 < keep; ++i) {
    target -= order[i].p;
    if (target < 0.0) return order[i].id;
  }
  return order[keep - 1].id;
}

SampledToken sample_token(const float* logits, std::size_t count, const SamplingOptions& options,
                          std::uint64_t generated_index) {
  SampledToken out{sample_logits(logits, count, options, generated_index)};
  if (!options.return_logprobs) return out;
  const double top = *std::max_element(logits, logits + count);
  double total = 0.0;
  for (std::size_t i = 0; i < count; ++i) total += std::exp(static_cast<double>(logits[i]) - top);
  const double log_total = std::log(total);
  out.logprob = static_cast<double>(logits[out.id]) - top - log_total;
  if (options.top_logprobs != 0) {
    std::vector<TokenLogProbability> all(count);
    for (std::size_t i = 0; i < count; ++i) all[i] = {i, static_cast<double>(logits[i]) - top - log_total};
    const std::size_t n = std::min<std::size_t>(count, options.top_logprobs);
    std::partial_sort(all.begin(), all.begin() + static_cast<std::ptrdiff_t>(n), all.end(),
                      [](const TokenLogProbability& a, const TokenLogProbability& b) {
                        return a.logprob != b.logprob ? a.logprob > b.logprob : a.token_id < b.token_id;
                      });
    all.resize(n);
    out.top_logprobs = std::move(all);
  }
  return out;
}

}  // namespace hllm_rocm::runtime
