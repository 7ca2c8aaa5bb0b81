// Device sampling of host logits without allocating: the rows are staged and sampled a few
// at a time through one file-scope device array (`scratch`), whose address is looked up
// once per device. For callers that cannot allocate device memory (code that must not call
// hipMalloc: serving loops, harnesses that forbid allocation). Same kernels and results as
// the allocating entry point.
#include <cmath>
#include <cstring>
#include <mutex>
#include <string>

#include "kernels.hpp"

namespace hllm_rocm {

void check_sampling(const hllm_rocm_item& it);

namespace {

constexpr uint64_t kStaticVocab = HLLM_ROCM_NOALLOC_MAX_VOCABULARY;
constexpr int kStaticGroup = 2;    // rows staged and sampled at a time
constexpr int kStaticChunks = 32;  // the sampler's largest first-pass split per row
constexpr int kStaticParts = 64;   // argmax partials per row
constexpr int kMaxDevices = 64;

constexpr uint64_t up256(uint64_t x) { return (x + 255) / 256 * 256; }

// Byte offsets of the areas of one group of rows inside the array.
struct Layout {
  static constexpr uint64_t G = kStaticGroup, V = kStaticVocab;
  static constexpr uint64_t logits = 0;
  static constexpr uint64_t weights = logits + up256(G * V * sizeof(float));
  static constexpr uint64_t buckets = weights + up256(G * V * sizeof(double));
  static constexpr uint64_t sorted = buckets + up256(G * ((V + 15) / 16 * 16));
  static constexpr uint64_t lists = sorted + up256(G * V * sizeof(uint32_t));
  static constexpr uint64_t hist = lists + up256(G * 4 * V * sizeof(uint32_t));
  static constexpr uint64_t cursor = hist + up256(G * 256 * 3 * sizeof(uint64_t));
  static constexpr uint64_t lse = cursor + up256(G * 256 * sizeof(uint32_t));
  static constexpr uint64_t candidates = lse + up256(G * kStaticChunks * sizeof(double));
  static constexpr uint64_t part_val = candidates + up256(G * kStaticChunks * 8 * sizeof(uint32_t));
  static constexpr uint64_t part_idx = part_val + up256(G * kStaticParts * sizeof(float));
  static constexpr uint64_t params = part_idx + up256(G * kStaticParts * sizeof(int32_t));
  static constexpr uint64_t tokens = params + up256(G * sizeof(SampleParams));
  // [logprob: G][top values: G * 5] doubles, then [top IDs: G * 5] int32
  static constexpr uint64_t out = tokens + up256(G * sizeof(int32_t));
  static constexpr uint64_t out_bytes = G * 6 * sizeof(double) + G * 5 * sizeof(int32_t);
  static constexpr uint64_t count = out + up256(out_bytes);
  static constexpr uint64_t flags = count + 256;
  static constexpr uint64_t total = flags + 256;
};
static_assert(Layout::total == HLLM_ROCM_NOALLOC_SCRATCH_BYTES, "scratch size in the header is stale");

// The sampler's workspace, the staged logits and the outputs of one group of rows. Each GPU
// holds its own copy until the process ends.
__device__ __align__(256) unsigned char scratch[Layout::total];

std::mutex g_lock;                     // one call at a time per process: they share the array
unsigned char* g_scratch[kMaxDevices];  // `scratch` on each device, looked up once

unsigned char* scratch_on(int device) {
  if (device < 0 || device >= kMaxDevices) fail(HLLM_INVALID_REQUEST, "device ordinal out of range");
  if (!g_scratch[device]) {
    void* p = nullptr;
    HIP_CHECK(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)));
    g_scratch[device] = static_cast<unsigned char*>(p);
  }
  return g_scratch[device];
}

}  // namespace

void sample_logits_noalloc(int32_t device, const float* logits, uint64_t rows, uint64_t V,
                           const hllm_rocm_item* options, uint64_t* tokens, double* logprobs,
                           uint64_t* top_ids, double* top_logprobs) {
  if (!logits || !options || !tokens || rows == 0 || V == 0) fail(HLLM_INVALID_REQUEST, "invalid sampling request");
  if (V > kStaticVocab)
    fail(HLLM_RESOURCE_EXHAUSTED, "vocabulary exceeds the allocation-free sampler's limit of " +
                                      std::to_string(kStaticVocab));
  if (rows > (1ull << 20)) fail(HLLM_RESOURCE_EXHAUSTED, "sampling request too large");
  for (uint64_t r = 0; r < rows; ++r) check_sampling(options[r]);
  std::lock_guard<std::mutex> lock(g_lock);
  HIP_CHECK(hipSetDevice(device));
  unsigned char* base = scratch_on(device);
  int cus = 256;
  HIP_CHECK(hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, device));
  // The first-pass split the allocating entry point uses for the same rows, so the
  // log-probability sums are taken in the same order.
  const int chunks = std::max(1, std::min(kStaticChunks, 4 * cus / (int)std::min<uint64_t>(rows, 64)));
  const hipStream_t stream = nullptr;
  auto at = [&](uint64_t offset) { return base + offset; };
  // The kernels expect these zero on entry; an earlier call may have ended early.
  HIP_CHECK(hipMemsetAsync(at(Layout::hist), 0, Layout::cursor - Layout::hist, stream));
  HIP_CHECK(hipMemsetAsync(at(Layout::cursor), 0, Layout::lse - Layout::cursor, stream));
  HIP_CHECK(hipMemsetAsync(at(Layout::flags), 0, sizeof(int32_t), stream));
  SampleArgs sa{};
  sa.vocab = (int)V;
  sa.logits = reinterpret_cast<const float*>(at(Layout::logits));
  sa.params = reinterpret_cast<const SampleParams*>(at(Layout::params));
  sa.tokens = reinterpret_cast<int32_t*>(at(Layout::tokens));
  sa.logprob = reinterpret_cast<double*>(at(Layout::out));
  sa.top_values = sa.logprob + kStaticGroup;
  sa.top_ids = reinterpret_cast<int32_t*>(sa.top_values + 5 * kStaticGroup);
  sa.weights = reinterpret_cast<double*>(at(Layout::weights));
  sa.buckets = at(Layout::buckets);
  sa.bucket_stride = sample_bucket_stride(V);
  sa.lists = reinterpret_cast<uint32_t*>(at(Layout::lists));
  sa.hist = reinterpret_cast<uint64_t*>(at(Layout::hist));
  sa.lse_parts = reinterpret_cast<double*>(at(Layout::lse));
  sa.sorted = reinterpret_cast<uint32_t*>(at(Layout::sorted));
  sa.cursor = reinterpret_cast<uint32_t*>(at(Layout::cursor));
  sa.candidates = reinterpret_cast<uint32_t*>(at(Layout::candidates));
  sa.group_rows = kStaticGroup;
  sa.chunks = chunks;
  alignas(8) unsigned char out[Layout::out_bytes];
  SampleParams params[kStaticGroup];
  int32_t group_tokens[kStaticGroup];
  int32_t flags = 0;
  for (uint64_t r0 = 0; r0 < rows; r0 += kStaticGroup) {
    const int32_t n = (int32_t)std::min<uint64_t>(kStaticGroup, rows - r0);
    for (int32_t j = 0; j < n; ++j) {
      const hllm_rocm_item& it = options[r0 + j];
      const bool lp = (it.flags & HLLM_ITEM_LOGPROBS) != 0;
      params[j] = {it.temperature, it.top_p, it.top_k, it.seed, it.generated_index, lp ? it.top_logprobs : 0u,
                   lp ? kSampleLogprobs : 0u};
    }
    HIP_CHECK(hipMemcpyAsync(at(Layout::logits), logits + r0 * V, n * V * sizeof(float), hipMemcpyHostToDevice,
                             stream));
    HIP_CHECK(hipMemcpyAsync(at(Layout::params), params, n * sizeof(SampleParams), hipMemcpyHostToDevice,
                             stream));
    HIP_CHECK(hipMemcpyAsync(at(Layout::count), &n, sizeof(n), hipMemcpyHostToDevice, stream));
    launch_argmax(stream, sa.logits, reinterpret_cast<const int32_t*>(at(Layout::count)), n, (int)V,
                  reinterpret_cast<float*>(at(Layout::part_val)), reinterpret_cast<int32_t*>(at(Layout::part_idx)),
                  kStaticParts, sa.tokens, reinterpret_cast<int32_t*>(at(Layout::flags)));
    sa.rows = n;
    launch_sample(stream, sa);
    HIP_CHECK(hipGetLastError());
    HIP_CHECK(hipMemcpyAsync(group_tokens, sa.tokens, n * sizeof(int32_t), hipMemcpyDeviceToHost, stream));
    HIP_CHECK(hipMemcpyAsync(out, at(Layout::out), sizeof(out), hipMemcpyDeviceToHost, stream));
    HIP_CHECK(hipMemcpyAsync(&flags, at(Layout::flags), sizeof(flags), hipMemcpyDeviceToHost, stream));
    HIP_CHECK(hipStreamSynchronize(stream));
    if (flags & 2) fail(HLLM_INTERNAL, "cannot sample nonfinite logits");
    const double* lp = reinterpret_cast<const double*>(out);
    const double* tv = lp + kStaticGroup;
    const int32_t* ti = reinterpret_cast<const int32_t*>(tv + 5 * kStaticGroup);
    for (int32_t j = 0; j < n; ++j) {
      const uint64_t r = r0 + j;
      tokens[r] = (uint64_t)group_tokens[j];
      if (!(params[j].flags & kSampleLogprobs)) continue;
      const uint64_t count = std::min<uint64_t>(params[j].top_logprobs, V);
      if (logprobs) logprobs[r] = lp[j];
      for (uint64_t k = 0; k < 5; ++k) {
        if (top_ids) top_ids[r * 5 + k] = k < count ? (uint64_t)ti[j * 5 + k] : UINT64_MAX;
        if (top_logprobs) top_logprobs[r * 5 + k] = k < count ? tv[j * 5 + k] : std::nan("");
      }
    }
  }
}

}  // namespace hllm_rocm
