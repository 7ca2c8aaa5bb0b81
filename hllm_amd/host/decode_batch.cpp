// Decode-batch packing of the stage contract (cpp/src/decode_batch.cpp:8-52): members are
// one-token inputs of independent, ready sequences, packed in item order.
#include <set>

#include "runtime.hpp"

namespace hllm_rocm::runtime {

StageInput combine_decode_inputs(const std::vector<DecodeBatchItem>& items) {
  if (items.empty() || items.size() > 64) throw Error::invalid_request("invalid decode batch size");
  const bool token_batch = std::holds_alternative<TokenInput>(items.front().input);
  std::set<const SequenceState*> seen;
  TokenInput ids;
  BoundaryActivation rows{items.size(), 0, {}};
  for (const DecodeBatchItem& item : items) {
    const bool ready = item.sequence && item.cancelled && item.position != 0 && !item.sequence->prefilling &&
                       !item.sequence->prefill_only;
    if (!ready || !seen.insert(item.sequence).second ||
        token_batch != std::holds_alternative<TokenInput>(item.input))
      throw Error::invalid_request("decode batch requires independent, ready decode sequences");
    if (token_batch) {
      const auto& in = std::get<TokenInput>(item.input);
      if (in.ids.size() != 1) throw Error::invalid_request("decode batch requires one token per sequence");
      ids.ids.push_back(in.ids[0]);
      continue;
    }
    const auto& in = std::get<BoundaryActivation>(item.input);
    if (in.tokens != 1 || in.width == 0 || in.payload.size() != in.width * 2 ||
        (rows.width != 0 && rows.width != in.width))
      throw Error::invalid_request("invalid decode batch boundary");
    rows.width = in.width;
    rows.payload.insert(rows.payload.end(), in.payload.begin(), in.payload.end());
  }
  if (token_batch) return ids;
  return rows;
}

std::vector<StageOutput> split_decode_boundary(BoundaryActivation output) {
  const std::size_t row_bytes = output.width * 2;
  if (output.width != 0 && output.tokens > output.payload.size() / row_bytes)
    throw Error::internal("invalid batched output boundary");
  if (output.payload.size() != output.tokens * row_bytes) throw Error::internal("invalid batched output boundary");
  std::vector<StageOutput> parts;
  parts.reserve(output.tokens);
  for (std::size_t i = 0; i < output.tokens; ++i) {
    const auto first = output.payload.begin() + static_cast<std::ptrdiff_t>(i * row_bytes);
    parts.push_back(BoundaryActivation{1, output.width, {first, first + static_cast<std::ptrdiff_t>(row_bytes)}});
  }
  return parts;
}

}  // namespace hllm_rocm::runtime
