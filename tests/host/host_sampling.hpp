// Host sampler used by the host tests only (tests/host/host_sampling.cpp).
#pragma once

#include <cstddef>
#include <cstdint>

#include "runtime.hpp"

namespace hllm_rocm::runtime {

std::uint64_t sample_logits(const float* logits, std::size_t count, const SamplingOptions& options,
                            std::uint64_t generated_index);
SampledToken sample_token(const float* logits, std::size_t count, const SamplingOptions& options,
                          std::uint64_t generated_index);

}  // namespace hllm_rocm::runtime
