// The stage runtime behind the C ABI: weights resident in HBM in the F-layout, a paged KV
// pool with a host-side block allocator, per-pass workspaces reserved up front, and the
// pass pipeline (pack -> embed/decode -> layers -> head/argmax or boundary encode).
#include <algorithm>
#include <cctype>
#include <atomic>
#include <cmath>
#include <cstdlib>
#include <cstring>
#include <map>
#include <memory>
#include <mutex>
#include <set>
#include <string>
#include <tuple>
#include <vector>

#include "gemm.hpp"
#include "kernels.hpp"

namespace hllm_rocm {
namespace {

thread_local std::string g_last_error;

uint64_t pad_to(uint64_t x, uint64_t m) { return (x + m - 1) / m * m; }

// Decode passes fuse QK-norm, RoPE and the K/V append into attention unless
// HLLM_ROCM_ROPE_FUSION=0 (the separate kernel, for comparisons).
bool rope_fusion_enabled() {
  static const bool on = [] {
    const char* v = std::getenv("HLLM_ROCM_ROPE_FUSION");
    return !(v && v[0] == '0');
  }();
  return on;
}

// Device memory the library holds, per device (the allocator metrics): bytes held now and
// the most held at once since the start or the last reset.
struct Ledger {
  std::mutex mutex;
  std::map<int, std::pair<uint64_t, uint64_t>> devices;  // device -> (active, peak)
  void add(int device, uint64_t n) {
    std::lock_guard<std::mutex> lock(mutex);
    auto& [active, peak] = devices[device];
    active += n;
    peak = std::max(peak, active);
  }
  void remove(int device, uint64_t n) {
    std::lock_guard<std::mutex> lock(mutex);
    devices[device].first -= n;
  }
};
Ledger& ledger() {
  static Ledger* l = new Ledger;  // never destroyed: stages may outlive static destruction
  return *l;
}

// Device allocation owned by the stage (RAII: a failed construction frees what it got).
struct DeviceMemory {
  void* ptr = nullptr;
  size_t bytes = 0;
  int device = 0;
  DeviceMemory() = default;
  DeviceMemory(const DeviceMemory&) = delete;
  DeviceMemory& operator=(const DeviceMemory&) = delete;
  ~DeviceMemory() { release(); }
  void release() {
    if (ptr) {
      (void)hipFree(ptr);
      ledger().remove(device, bytes);
    }
    ptr = nullptr;
    bytes = 0;
  }
  void allocate(size_t n, const char* what) {
    bytes = n;
    if (n == 0) return;
    HIP_CHECK(hipGetDevice(&device));
    const hipError_t e = hipMalloc(&ptr, n);
    if (e != hipSuccess) {
      ptr = nullptr;
      bytes = 0;
      fail(HLLM_RESOURCE_EXHAUSTED, std::string("device allocation failed: ") + what + " (" +
                                        std::to_string(n) + " bytes)");
    }
    ledger().add(device, n);
  }
  template <typename T>
  T* as() const {
    return static_cast<T*>(ptr);
  }
};

struct PinnedMemory {
  void* ptr = nullptr;
  PinnedMemory() = default;
  PinnedMemory(const PinnedMemory&) = delete;
  PinnedMemory& operator=(const PinnedMemory&) = delete;
  ~PinnedMemory() {
    if (ptr) (void)hipHostFree(ptr);
  }
  void allocate(size_t n) { HIP_CHECK(hipHostMalloc(&ptr, n == 0 ? 1 : n, hipHostMallocDefault)); }
  template <typename T>
  T* as() const {
    return static_cast<T*>(ptr);
  }
};

struct Matrix {  // an F-layout weight: hi parts and optional lo parts
  DeviceMemory hi, lo;
  uint64_t rows_padded = 0, cols_padded = 0;
  uint64_t cols = 0;  // the contraction length before padding
};

struct Layer {
  Matrix qkv, o, gate_up, down;
  DeviceMemory input_norm, post_norm, q_norm, k_norm;
};

struct Sequence {
  bool live = false;
  bool failed = false;
  // The sequence's previous pass sampled a token, which the device holds for a
  // device-fed input of its next pass.
  bool device_token = false;
  // A submitted pass uses the sequence (its KV blocks must not be handed out again).
  bool in_flight = false;
  // Released while in flight: the slot and blocks return to the pools when the pass completes.
  bool release_pending = false;
  uint64_t capacity = 0;
  uint64_t length = 0;
  std::vector<int32_t> blocks;
};

// Per-phase timing of a profiled pass (runtime::ExecutionTiming components,
// cpp/include/hllm/runtime/timing.hpp:11-18): events recorded on the stage's stream
// between phases, read once the pass completes.
struct PhaseMark {
  const char* component;
  int32_t layer;  // -1: not a layer
  hipEvent_t end;
};

// Expected tensor: shape and where it goes.
struct Target {
  std::vector<uint64_t> shape;
  Matrix* matrix = nullptr;
  DeviceMemory* vector = nullptr;
  int row_mode = 0;
  uint64_t row_offset = 0;
  bool loaded = false;
};

struct Profile {
  std::vector<std::pair<hipEvent_t, hipEvent_t>> events;
  uint64_t launches = 0;
  uint64_t bytes = 0;
  double flops = 0.0;
  bool owns_events = true;  // kernel records share the events of their family record
};

// The pass's cancellation flag or poll (either may be absent).
bool cancel_requested(const hllm_rocm_pass& pass) {
  return (pass.cancelled && *pass.cancelled) || (pass.cancel_poll && pass.cancel_poll(pass.cancel_context) != 0);
}

constexpr int kMaxSplits = 16;
constexpr int kSplitUnit = 256;
constexpr int kArgmaxParts = 64;
constexpr int kSampleBlocks = 64;  // workgroups of the sampler (one row each at a time)
constexpr size_t kMaxGraphs = 16;  // captured pass shapes kept (least recently used dropped)
constexpr uint64_t kStagingBytes = 64ull << 20;

}  // namespace

void check_sampling(const hllm_rocm_item& it);
void sample_logits_noalloc(int32_t device, const float* logits, uint64_t rows, uint64_t V,
                           const hllm_rocm_item* options, uint64_t* tokens, double* logprobs,
                           uint64_t* top_ids, double* top_logprobs);

class Stage {
 public:
  explicit Stage(const hllm_rocm_stage_config& c);
  ~Stage();
  void load_tensor(const std::string& name, uint32_t dtype, const uint64_t* shape, uint32_t rank,
                   const void* data, uint64_t bytes);
  void synthesize(const std::string& name, uint64_t seed, uint64_t tensor_id, float mean, float sigma,
                  uint32_t source_dtype);
  void finalize();
  hllm_rocm_memory weight_memory() const { return {0, weight_bytes_, 0, 0}; }
  void sequence_memory(uint64_t tokens, uint64_t max_query, hllm_rocm_memory* cache,
                       hllm_rocm_memory* workspace) const;
  uint32_t allocate_sequence(uint64_t tokens);
  void release_sequence(uint32_t handle);
  uint64_t sequence_length(uint32_t handle) const;
  void submit(const hllm_rocm_pass& pass, bool phases = false);
  void wait(hllm_rocm_phase_time* phases = nullptr, uint32_t capacity = 0, uint32_t* count = nullptr);
  void last_layout(uint32_t items, uint32_t rows, int32_t* cu, int32_t* pos, int32_t* slots);
  void sequence_blocks(uint32_t handle, int32_t* blocks, uint32_t capacity, uint32_t* count,
                       uint32_t* block_tokens);
  void read_kv(uint32_t handle, uint32_t layer, float* keys, float* values);
  void read_tensor(const std::string& name, float* out, uint64_t elements);
  void set_profiling(const std::string& families);
  void set_graphs(bool enabled) {
    std::lock_guard<std::mutex> lock(pass_mutex_);
    graphs_enabled_ = enabled;
  }
  void graph_stats(uint64_t* captured, uint64_t* replayed) {
    std::lock_guard<std::mutex> lock(pass_mutex_);
    if (captured) *captured = graph_captures_;
    if (replayed) *replayed = graph_replays_;
  }
  void profile_read(const std::string& record, double* ms, uint64_t* launches, uint64_t* bytes, double* flops);
  std::string profile_records();

 private:
  void check_sizes();
  Target& target(const std::string& name);
  void relayout(Target& t, const std::string& name, const void* device_src, uint32_t dtype,
                uint64_t seed, uint64_t tensor_id, float mean, float sigma, uint64_t row_base,
                uint64_t rows);
  void read_flags(const char* context);
  // `argmax_parts` > 0: the kEpiArgmax epilogue into argmax_val_ / argmax_idx_.
  int gemm(const char* family, const Matrix& w, const uint16_t* x_hi, const uint16_t* x_lo, int rows,
            int n, int epilogue, float* out, int ldo, uint16_t* out_hi, uint16_t* out_lo,
            uint64_t out_cols_padded,
           bool defer = false, int argmax_parts = 0);
  template <typename F>
  void timed(const char* family, uint64_t bytes, double flops, F&& launch);
  hipEvent_t take_event();
  void fail_pass(const std::vector<uint32_t>& sequences);
  // Ends the in-flight use of a pass's sequences (under seq_mutex_): clears the flag and
  // returns the slots and blocks of sequences released meanwhile.
  void retire_sequences(const std::vector<uint32_t>& sequences);
  void free_sequence(uint32_t handle);
  void mark_phase(const char* component, int32_t layer);

  hllm_rocm_stage_config c_;
  int device_ = 0;
  int cus_ = 256;
  hipStream_t stream_ = nullptr;
  int prec_ = kF16;
  bool kv_f32_ = false;
  bool w_f32_ = false;
  uint64_t H_, I_, Q_, K_, D_, V_, L_, Hp_, Ip_, QDp_, qkv_n_;
  uint64_t rows_max_, rows_padded_, items_max_;
  uint64_t weight_bytes_ = 0;
  bool finalized_ = false;

  std::vector<std::unique_ptr<Layer>> layers_;
  Matrix embedding_, head_;
  DeviceMemory final_norm_;
  std::map<std::string, Target> targets_;
  DeviceMemory rope_cos_, rope_sin_;

  // paged KV
  DeviceMemory kv_pool_;
  KvView kv_{};
  uint64_t blocks_total_ = 0;
  int table_width_ = 0;
  std::vector<int32_t> free_blocks_;
  std::vector<Sequence> sequences_;
  std::vector<uint32_t> free_slots_;
  DeviceMemory block_table_, last_token_;
  mutable std::mutex seq_mutex_;
  std::mutex pass_mutex_;

  // workspaces
  DeviceMemory h_, a0_hi_, a0_lo_, a1_hi_, a1_lo_, qkv_, q_, attn_partial_;
  // Per-pass inputs and outputs share one copy each way: items_dev_ holds the item list, then
  // the input tokens; tokens_ the sampled tokens, then the pass's error flags.
  DeviceMemory gemm_ws_, gemm_counters_, logits_, argmax_val_, argmax_idx_, tokens_;
  uint64_t argmax_capacity_ = 0;  // entries of argmax_val_ / argmax_idx_
  DeviceMemory items_dev_, pack_buf_, boundary_dev_, staging_, attn_work_;
  bool mfma_attention_ = false;
  uint64_t attn_work_max_ = 0;
  size_t gemm_ws_floats_ = 0;
  int gemm_counter_count_ = 0;
  PackOut pack_{};
  PinnedMemory pin_items_, pin_out_tokens_, pin_boundary_;
  size_t tokens_offset() const { return items_max_ * sizeof(ItemMeta); }
  int32_t* host_tokens_dev() const { return reinterpret_cast<int32_t*>(static_cast<char*>(items_dev_.ptr) + tokens_offset()); }
  int32_t* pin_tokens() const { return reinterpret_cast<int32_t*>(static_cast<char*>(pin_items_.ptr) + tokens_offset()); }
  int32_t* flags_dev() const { return tokens_.as<int32_t>() + items_max_; }
  int32_t* pin_flags() const { return pin_out_tokens_.as<int32_t>() + items_max_; }
  // sampler: per-row options, outputs [logprob: items][top values: items * 5][top IDs: items * 5]
  DeviceMemory sample_params_, sample_out_, sample_weights_, sample_lists_, sample_buckets_, sample_hist_,
      sample_lse_, sample_sorted_, sample_cursor_, sample_candidates_;
  PinnedMemory pin_sample_params_, pin_sample_out_;
  int sample_blocks_ = 0, sample_chunks_ = 1;

  // Passes whose shape repeats can be replayed from a captured HIP graph (off by default: on
  // MI355X the replay saves no measurable time on these passes, whose kernels, not their
  // launches, set the pace). Every launch parameter of a pass is a function of its shape:
  // items, rows, sampled rows, sampler, attention work items and splits, and the host-side
  // choices made per pass (the LM head's argmax-epilogue parts, the forced GEMM
  // configuration); all other per-pass values are read on the device. A shape is captured
  // the second time it is seen (the first run sets the kernels' attributes eagerly).
  struct PassShape {
    uint32_t items, rows, samples, sampler, attention_items, any_split;
    int32_t argmax_parts, gemm_config;
    bool operator<(const PassShape& o) const {
      return std::tie(items, rows, samples, sampler, attention_items, any_split, argmax_parts, gemm_config) <
             std::tie(o.items, o.rows, o.samples, o.sampler, o.attention_items, o.any_split, o.argmax_parts,
                      o.gemm_config);
    }
  };
  struct CapturedPass {
    hipGraph_t graph = nullptr;
    hipGraphExec_t exec = nullptr;
    uint64_t used = 0;
  };
  bool graphs_enabled_ = false;
  std::map<PassShape, CapturedPass> graphs_;
  std::set<PassShape> shapes_seen_;
  uint64_t graph_clock_ = 0, graph_captures_ = 0, graph_replays_ = 0;
  DeviceMemory attn_count_;
  DeviceMemory attn_arrivals_;  // [rows][kv_heads] split arrival counts, zero between launches
  bool attn_fold_ = true;

  // in-flight pass
  bool in_flight_ = false;
  hllm_rocm_pass pending_{};
  std::vector<uint32_t> pending_sequences_;
  std::vector<uint32_t> pending_lengths_;
  std::vector<int> pending_sample_items_;
  std::vector<int> pending_top_counts_;  // per sampled row: -1 without log-probabilities
  bool pending_sampler_ = false;
  uint64_t pending_rows_ = 0;
  // execute_profiled: the pass's start event and one mark per completed phase.
  bool phases_on_ = false;
  hipEvent_t phase_start_ = nullptr;
  std::vector<PhaseMark> phase_marks_;

  bool profiling_ = false;
  std::vector<std::string> profile_filter_;
  std::map<std::string, Profile> profiles_;
  std::vector<hipEvent_t> event_pool_;
};

// --------------------------------------------------------------------- construction

Stage::Stage(const hllm_rocm_stage_config& c) : c_(c) {
  if (c.abi_version != HLLM_ROCM_ABI_VERSION) fail(HLLM_INCOMPATIBLE_WORKER, "ABI version mismatch");
  check_sizes();
  device_ = c.device;
  HIP_CHECK(hipSetDevice(device_));
  HIP_CHECK(hipDeviceGetAttribute(&cus_, hipDeviceAttributeMultiprocessorCount, device_));
  HIP_CHECK(hipStreamCreateWithFlags(&stream_, hipStreamNonBlocking));

  H_ = c.hidden_size;
  I_ = c.intermediate_size;
  Q_ = c.attention_heads;
  K_ = c.key_value_heads;
  D_ = c.head_dimension;
  V_ = c.vocabulary_size;
  L_ = c.layer_end - c.layer_start;
  Hp_ = pad32(H_);
  Ip_ = pad32(I_);
  QDp_ = pad32(Q_ * D_);
  qkv_n_ = (Q_ + 2 * K_) * D_;
  const bool f32_exec = c.execution_dtype == HLLM_DTYPE_F32;
  w_f32_ = c.weight_dtype == HLLM_DTYPE_F32;
  prec_ = !f32_exec ? kF16 : (w_f32_ ? kSplitAB : kSplitA);
  kv_f32_ = f32_exec;
  rows_max_ = c.max_pass_rows ? c.max_pass_rows : 2048;
  rows_padded_ = gemm_padded_rows(rows_max_);
  const uint64_t seq_max = c.max_sequences ? c.max_sequences : 512;
  items_max_ = std::min<uint64_t>(std::max<uint64_t>(seq_max, 1), 1024);
  const int bt = c.kv_block_tokens ? (int)c.kv_block_tokens : 64;

  // ---- weights
  const size_t wel = w_f32_ ? 2 : 1;  // hi (+ lo) parts
  auto matrix = [&](Matrix& m, uint64_t rows, uint64_t cols, const char* what) {
    m.rows_padded = pad_to(rows, 256);  // whole GEMM weight tiles (at most 256 features)
    m.cols_padded = pad32(cols);
    m.cols = cols;
    const size_t bytes = m.rows_padded * m.cols_padded * 2;
    m.hi.allocate(bytes, what);
    HIP_CHECK(hipMemsetAsync(m.hi.ptr, 0, bytes, stream_));
    if (w_f32_) {
      m.lo.allocate(bytes, what);
      HIP_CHECK(hipMemsetAsync(m.lo.ptr, 0, bytes, stream_));
    }
    weight_bytes_ += rows * cols * 2 * wel;
  };
  auto vec = [&](DeviceMemory& v, uint64_t n, const char* what) {
    v.allocate(n * sizeof(float), what);
    weight_bytes_ += n * 2 * wel;
  };
  const std::string root = "model.layers.";
  for (uint64_t i = 0; i < L_; ++i) {
    layers_.push_back(std::make_unique<Layer>());
    Layer& l = *layers_.back();
    const std::string p = root + std::to_string(c.layer_start + i) + ".";
    matrix(l.qkv, qkv_n_, H_, "qkv");
    matrix(l.o, H_, Q_ * D_, "o_proj");
    matrix(l.gate_up, 2 * Ip_, H_, "gate_up");
    matrix(l.down, H_, Ip_, "down_proj");
    weight_bytes_ -= (2 * Ip_ - 2 * I_) * H_ * 2 * wel + H_ * (Ip_ - I_) * 2 * wel;
    vec(l.input_norm, H_, "norm");
    vec(l.post_norm, H_, "norm");
    targets_[p + "input_layernorm.weight"] = {{H_}, nullptr, &l.input_norm};
    targets_[p + "post_attention_layernorm.weight"] = {{H_}, nullptr, &l.post_norm};
    targets_[p + "self_attn.q_proj.weight"] = {{Q_ * D_, H_}, &l.qkv, nullptr, 0, 0};
    targets_[p + "self_attn.k_proj.weight"] = {{K_ * D_, H_}, &l.qkv, nullptr, 0, Q_ * D_};
    targets_[p + "self_attn.v_proj.weight"] = {{K_ * D_, H_}, &l.qkv, nullptr, 0, (Q_ + K_) * D_};
    targets_[p + "self_attn.o_proj.weight"] = {{H_, Q_ * D_}, &l.o, nullptr, 0, 0};
    targets_[p + "mlp.gate_proj.weight"] = {{I_, H_}, &l.gate_up, nullptr, 1, 0};
    targets_[p + "mlp.up_proj.weight"] = {{I_, H_}, &l.gate_up, nullptr, 2, 0};
    targets_[p + "mlp.down_proj.weight"] = {{H_, I_}, &l.down, nullptr, 0, 0};
    if (c.query_key_norm) {
      vec(l.q_norm, D_, "qk_norm");
      vec(l.k_norm, D_, "qk_norm");
      targets_[p + "self_attn.q_norm.weight"] = {{D_}, nullptr, &l.q_norm};
      targets_[p + "self_attn.k_norm.weight"] = {{D_}, nullptr, &l.k_norm};
    }
  }
  if (c.first_stage || (c.final_stage && c.tied_head)) {
    matrix(embedding_, V_, H_, "embedding");
    targets_["model.embed_tokens.weight"] = {{V_, H_}, &embedding_, nullptr, 0, 0};
  }
  if (c.final_stage) {
    vec(final_norm_, H_, "final_norm");
    targets_["model.norm.weight"] = {{H_}, nullptr, &final_norm_};
    if (!c.tied_head) {
      matrix(head_, V_, H_, "lm_head");
      targets_["lm_head.weight"] = {{V_, H_}, &head_, nullptr, 0, 0};
    }
  }

  // ---- RoPE tables, computed on the host with the CPU worker's float calls
  // (angle = position / powf(theta, 2i / D), cosf, sinf: cpp/src/cpu/llama.cpp:222-231).
  {
    const uint64_t half = D_ / 2, positions = c.maximum_sequence_length;
    std::vector<float> denominators(half), cs(positions * half), sn(positions * half);
    for (uint64_t i = 0; i < half; ++i) {
      denominators[i] = std::pow(c.rope_theta, static_cast<float>(2 * i) / static_cast<float>(D_));
    }
    for (uint64_t p = 0; p < positions; ++p) {
      for (uint64_t i = 0; i < half; ++i) {
        const float angle = static_cast<float>(p) / denominators[i];
        cs[p * half + i] = std::cos(angle);
        sn[p * half + i] = std::sin(angle);
      }
    }
    rope_cos_.allocate(cs.size() * sizeof(float), "rope");
    rope_sin_.allocate(sn.size() * sizeof(float), "rope");
    HIP_CHECK(hipMemcpy(rope_cos_.ptr, cs.data(), cs.size() * sizeof(float), hipMemcpyHostToDevice));
    HIP_CHECK(hipMemcpy(rope_sin_.ptr, sn.data(), sn.size() * sizeof(float), hipMemcpyHostToDevice));
  }

  // ---- workspaces
  const size_t R = rows_padded_;
  h_.allocate(R * H_ * sizeof(float), "hidden");
  const uint64_t a0_cols = Hp_, a1_cols = std::max(QDp_, Ip_);
  a0_hi_.allocate(R * a0_cols * 2, "operand");
  a1_hi_.allocate(R * a1_cols * 2, "operand");
  HIP_CHECK(hipMemsetAsync(a0_hi_.ptr, 0, a0_hi_.bytes, stream_));
  HIP_CHECK(hipMemsetAsync(a1_hi_.ptr, 0, a1_hi_.bytes, stream_));
  if (prec_ >= kSplitA) {
    a0_lo_.allocate(R * a0_cols * 2, "operand");
    a1_lo_.allocate(R * a1_cols * 2, "operand");
    HIP_CHECK(hipMemsetAsync(a0_lo_.ptr, 0, a0_lo_.bytes, stream_));
    HIP_CHECK(hipMemsetAsync(a1_lo_.ptr, 0, a1_lo_.bytes, stream_));
  }
  qkv_.allocate(R * qkv_n_ * sizeof(float), "qkv");
  q_.allocate(R * Q_ * D_ * sizeof(float), "q");
  attn_partial_.allocate(R * Q_ * kMaxSplits * (D_ + 2) * sizeof(float), "attention partials");
  gemm_ws_floats_ = 32ull << 20;
  gemm_ws_.allocate(gemm_ws_floats_ * sizeof(float), "gemm workspace");
  gemm_counter_count_ = 1 << 17;
  gemm_counters_.allocate(gemm_counter_count_ * sizeof(int32_t), "gemm counters");
  HIP_CHECK(hipMemsetAsync(gemm_counters_.ptr, 0, gemm_counters_.bytes, stream_));
  if (c.final_stage) {
    logits_.allocate(items_max_ * V_ * sizeof(float), "logits");
    // Candidates of the argmax kernels, or of the LM head's argmax epilogue (at most 64 rows,
    // one candidate per 64 or more features).
    argmax_capacity_ = std::max<uint64_t>(items_max_ * kArgmaxParts, 64 * ((V_ + 63) / 64));
    argmax_val_.allocate(argmax_capacity_ * sizeof(float), "argmax");
    argmax_idx_.allocate(argmax_capacity_ * sizeof(int32_t), "argmax");
    sample_blocks_ = (int)std::min<uint64_t>(items_max_, kSampleBlocks);
    sample_chunks_ = std::max(1, std::min(32, 4 * cus_ / sample_blocks_));
    sample_params_.allocate(items_max_ * sizeof(SampleParams), "sampling");
    sample_out_.allocate(items_max_ * (6 * sizeof(double) + 5 * sizeof(int32_t)), "sampling");
    sample_weights_.allocate((size_t)sample_blocks_ * V_ * sizeof(double), "sampling workspace");
    sample_buckets_.allocate((size_t)sample_blocks_ * sample_bucket_stride(V_), "sampling workspace");
    sample_lists_.allocate((size_t)sample_blocks_ * 4 * V_ * sizeof(uint32_t), "sampling workspace");
    sample_hist_.allocate((size_t)sample_blocks_ * 256 * 3 * sizeof(uint64_t), "sampling workspace");
    sample_lse_.allocate((size_t)sample_blocks_ * sample_chunks_ * sizeof(double), "sampling workspace");
    sample_sorted_.allocate((size_t)sample_blocks_ * V_ * sizeof(uint32_t), "sampling workspace");
    sample_cursor_.allocate((size_t)sample_blocks_ * 256 * sizeof(uint32_t), "sampling workspace");
    sample_candidates_.allocate((size_t)sample_blocks_ * sample_chunks_ * 8 * sizeof(uint32_t), "sampling workspace");
    HIP_CHECK(hipMemsetAsync(sample_hist_.ptr, 0, sample_hist_.bytes, stream_));
    HIP_CHECK(hipMemsetAsync(sample_cursor_.ptr, 0, sample_cursor_.bytes, stream_));
  }
  tokens_.allocate((items_max_ + 1) * sizeof(int32_t), "tokens");
  pack_.flags = flags_dev();
  items_dev_.allocate(tokens_offset() + R * sizeof(int32_t), "items");
  pack_buf_.allocate(((items_max_ + 1) + 5 * R + 2 * items_max_ + 1) * sizeof(int32_t), "pack");
  {
    int32_t* p = pack_buf_.as<int32_t>();
    pack_.cu_seqlens = p;
    p += items_max_ + 1;
    pack_.row_item = p;
    p += R;
    pack_.row_position = p;
    p += R;
    pack_.row_slot = p;
    p += R;
    pack_.row_token = p;
    p += R;
    pack_.sample_row = p;
    p += items_max_;
    pack_.sample_item = p;
    p += items_max_;
    pack_.sample_count = p;
    p += 1;
    pack_.row_splits = p;
  }
  mfma_attention_ = attention_uses_mfma((int)D_, kv_f32_);
  if (mfma_attention_) {
    // Upper bound of attention work items: per item, one per 64-vector block per split.
    const uint64_t group = Q_ / K_;
    const uint64_t qb = group >= 64 ? 1 : 64 / group;
    attn_work_max_ = (R / qb + items_max_) * kMaxSplits;
    attn_work_.allocate(attn_work_max_ * sizeof(AttnWork), "attention work");
    pack_.attn_work = attn_work_.as<AttnWork>();
    attn_count_.allocate(sizeof(int32_t), "attention work");
    pack_.attn_count = attn_count_.as<int32_t>();
    // Decode-like blocks merge their key splits in the attention kernel (the last split to
    // arrive) unless HLLM_ROCM_ATTN_FOLD=0 (the combine kernel, for comparisons). The counts
    // reset themselves, so they are cleared once here.
    if (const char* v = std::getenv("HLLM_ROCM_ATTN_FOLD")) attn_fold_ = v[0] != '0';
    attn_arrivals_.allocate(R * K_ * sizeof(int32_t), "attention arrivals");
    HIP_CHECK(hipMemsetAsync(attn_arrivals_.ptr, 0, attn_arrivals_.bytes, stream_));
    pack_.attn_fold = attn_fold_ ? 1 : 0;
    pack_.attn_group = (int)group;
    pack_.attn_max_splits = kMaxSplits;
    // Keys per split of decode-like attention blocks; HLLM_ROCM_ATTN_DECODE_SPLIT overrides
    // it for tuning (a multiple of 32).
    pack_.attn_decode_unit = 512;
    if (const char* v = std::getenv("HLLM_ROCM_ATTN_DECODE_SPLIT")) {
      const int unit = std::atoi(v);
      if (unit < 32 || unit % 32) fail(HLLM_INVALID_REQUEST, "HLLM_ROCM_ATTN_DECODE_SPLIT must be a multiple of 32");
      pack_.attn_decode_unit = unit;
    }
    pack_.attn_decode_split = pack_.attn_decode_unit;
    if (const char* v = std::getenv("HLLM_ROCM_ATTN_SPLIT_KEYS")) {
      const int keys = std::atoi(v);
      if (keys < 32 || keys % 32) fail(HLLM_INVALID_REQUEST, "HLLM_ROCM_ATTN_SPLIT_KEYS must be a multiple of 32");
      pack_.attn_decode_split = keys;
    }
  }
  if (!c.first_stage || !c.final_stage) boundary_dev_.allocate(R * H_ * 2, "boundary");
  pin_items_.allocate(tokens_offset() + R * sizeof(int32_t));
  pin_out_tokens_.allocate((items_max_ + 1) * sizeof(int32_t));
  pin_sample_params_.allocate(items_max_ * sizeof(SampleParams));
  pin_sample_out_.allocate(items_max_ * (6 * sizeof(double) + 5 * sizeof(int32_t)));
  pin_boundary_.allocate(R * H_ * 2);
  staging_.allocate(kStagingBytes, "load staging");

  // ---- paged KV pool (the rest of HBM unless sized explicitly)
  const size_t kv_el = kv_f32_ ? 4 : 2;
  const uint64_t block_bytes_all_layers = 2 * K_ * (uint64_t)bt * D_ * kv_el * L_;
  table_width_ = (int)((c.maximum_sequence_length + bt - 1) / bt);
  uint64_t kv_bytes = c.kv_cache_bytes;
  if (kv_bytes == 0) {
    size_t free_b = 0, total_b = 0;
    HIP_CHECK(hipStreamSynchronize(stream_));
    HIP_CHECK(hipMemGetInfo(&free_b, &total_b));
    kv_bytes = (uint64_t)(0.9 * (double)free_b);
  }
  blocks_total_ = kv_bytes / block_bytes_all_layers;
  if (blocks_total_ == 0) fail(HLLM_RESOURCE_EXHAUSTED, "KV cache budget holds no block");
  if (blocks_total_ * bt > 0x7fffffffull) blocks_total_ = 0x7fffffffull / bt;
  kv_pool_.allocate(blocks_total_ * block_bytes_all_layers, "KV cache");
  HIP_CHECK(hipMemsetAsync(kv_pool_.ptr, 0, kv_pool_.bytes, stream_));
  kv_.pool = kv_pool_.ptr;
  kv_.block_tokens = bt;
  kv_.kv_heads = (int)K_;
  kv_.head_dim = (int)D_;
  kv_.f32 = kv_f32_ ? 1 : 0;
  kv_.key_fragments = attention_uses_mfma((int)D_, kv_f32_) ? 1 : 0;
  kv_.layer_stride = blocks_total_ * 2 * K_ * bt * D_;
  free_blocks_.reserve(blocks_total_);
  for (uint64_t b = blocks_total_; b-- > 0;) free_blocks_.push_back((int32_t)b);
  sequences_.resize(seq_max);
  for (uint64_t s = seq_max; s-- > 0;) free_slots_.push_back((uint32_t)s);
  block_table_.allocate(seq_max * table_width_ * sizeof(int32_t), "block table");
  HIP_CHECK(hipMemsetAsync(block_table_.ptr, 0xff, block_table_.bytes, stream_));
  last_token_.allocate(seq_max * sizeof(int32_t), "last tokens");
  HIP_CHECK(hipMemsetAsync(last_token_.ptr, 0, last_token_.bytes, stream_));
  HIP_CHECK(hipStreamSynchronize(stream_));
}

Stage::~Stage() {
  if (stream_) {
    (void)hipStreamSynchronize(stream_);
    for (auto& [shape, g] : graphs_) {
      (void)hipGraphExecDestroy(g.exec);
      (void)hipGraphDestroy(g.graph);
    }
    for (auto& [name, p] : profiles_)
      if (p.owns_events)
        for (auto& e : p.events) event_pool_.push_back(e.first), event_pool_.push_back(e.second);
    for (const PhaseMark& m : phase_marks_) event_pool_.push_back(m.end);
    if (phase_start_) event_pool_.push_back(phase_start_);
    for (auto e : event_pool_) (void)hipEventDestroy(e);
    (void)hipStreamDestroy(stream_);
  }
}

void Stage::check_sizes() {
  const auto& c = c_;
  if (c.hidden_size == 0 || c.intermediate_size == 0 || c.attention_heads == 0 ||
      c.key_value_heads == 0 || c.head_dimension == 0 || c.maximum_sequence_length == 0 ||
      c.vocabulary_size == 0 || !(c.rms_norm_epsilon > 0.0f) || !std::isfinite(c.rms_norm_epsilon) ||
      !(c.rope_theta > 0.0f) || !std::isfinite(c.rope_theta)) {
    fail(HLLM_INCOMPATIBLE_WORKER, "unsupported dense model configuration");
  }
  if (c.attention_heads % c.key_value_heads != 0 || c.layer_start >= c.layer_end)
    fail(HLLM_INCOMPATIBLE_WORKER, "inconsistent attention heads or layer range");
  const uint64_t d = c.head_dimension;
  if (d < 4 || d > 256 || (d & (d - 1)) != 0)
    fail(HLLM_INCOMPATIBLE_WORKER, "head dimension must be a power of two in [4, 256]");
  if (c.attention_heads / c.key_value_heads > 8 || (c.attention_heads / c.key_value_heads) * d > 2048)
    fail(HLLM_INCOMPATIBLE_WORKER, "query heads per KV head must be at most 8");
  if (c.execution_dtype != HLLM_DTYPE_F16 && c.execution_dtype != HLLM_DTYPE_F32)
    fail(HLLM_INCOMPATIBLE_WORKER, "execution dtype must be F16 or F32");
  if (c.weight_dtype != HLLM_DTYPE_F16 &&
      !(c.weight_dtype == HLLM_DTYPE_F32 && c.execution_dtype == HLLM_DTYPE_F32))
    fail(HLLM_INCOMPATIBLE_WORKER, "unsupported resident/execution precision contract");
  if (c.maximum_sequence_length > (1u << 24) || c.vocabulary_size > 0x7fffffffull ||
      c.hidden_size > 8192 || c.intermediate_size > (1u << 18))
    fail(HLLM_INCOMPATIBLE_WORKER, "model dimensions exceed this worker's limits");
  if (c.kv_block_tokens && (c.kv_block_tokens & (c.kv_block_tokens - 1)))
    fail(HLLM_INVALID_REQUEST, "KV block tokens must be a power of two");
  if (c.kv_block_tokens && c.kv_block_tokens < 32)
    fail(HLLM_INVALID_REQUEST, "KV blocks hold at least 32 tokens");
  if (c.max_pass_rows > (1u << 16)) fail(HLLM_INVALID_REQUEST, "max pass rows too large");
}

// --------------------------------------------------------------------- loading

Target& Stage::target(const std::string& name) {
  if (finalized_) fail(HLLM_INVALID_REQUEST, "stage is already finalized");
  auto it = targets_.find(name);
  if (it == targets_.end()) fail(HLLM_INCOMPATIBLE_WORKER, "unsupported selected tensor: " + name);
  return it->second;
}

void Stage::read_flags(const char* context) {
  int32_t flags = 0;
  HIP_CHECK(hipMemcpyAsync(pin_flags(), flags_dev(), sizeof(int32_t), hipMemcpyDeviceToHost, stream_));
  HIP_CHECK(hipStreamSynchronize(stream_));
  flags = *pin_flags();
  if (flags & 1) fail(HLLM_INCOMPATIBLE_WORKER, std::string("non-finite weight: ") + context);
  if (flags & 4) fail(HLLM_INCOMPATIBLE_WORKER, std::string("weight is not representable as finite F16: ") + context);
}

void Stage::relayout(Target& t, const std::string& name, const void* device_src, uint32_t dtype,
                     uint64_t seed, uint64_t tensor_id, float mean, float sigma, uint64_t row_base,
                     uint64_t rows) {
  RelayoutArgs a{};
  a.src = device_src;
  a.src_dtype = dtype;
  a.seed = seed;
  a.tensor_id = tensor_id;
  a.mean = mean;
  a.sigma = sigma;
  a.rows = rows;
  a.row_base = row_base;
  a.cols = t.shape.size() == 2 ? t.shape[1] : t.shape[0];
  a.f16_resident = w_f32_ ? 0 : 1;
  a.flags = flags_dev();
  if (t.matrix) {
    a.dst_hi = t.matrix->hi.as<uint16_t>();
    a.dst_lo = w_f32_ ? t.matrix->lo.as<uint16_t>() : nullptr;
    a.dst_cols_padded = t.matrix->cols_padded;
    a.row_mode = t.row_mode;
    a.row_offset = t.row_offset;
  } else {
    a.dst_f32 = t.vector->as<float>();
    a.rows = 1;
  }
  (void)name;
  launch_relayout(stream_, a);
  HIP_CHECK(hipGetLastError());
}

void Stage::load_tensor(const std::string& name, uint32_t dtype, const uint64_t* shape, uint32_t rank,
                        const void* data, uint64_t bytes) {
  std::lock_guard<std::mutex> lock(pass_mutex_);
  Target& t = target(name);
  if (std::vector<uint64_t>(shape, shape + rank) != t.shape)
    fail(HLLM_INCOMPATIBLE_WORKER, "incorrect tensor shape: " + name);
  if (dtype != HLLM_DTYPE_F32 && dtype != HLLM_DTYPE_F16 && dtype != HLLM_DTYPE_BF16)
    fail(HLLM_INCOMPATIBLE_WORKER, "unsupported weight dtype: " + name);
  const uint64_t el = dtype == HLLM_DTYPE_F32 ? 4 : 2;
  const uint64_t rows = t.shape.size() == 2 ? t.shape[0] : 1;
  const uint64_t cols = t.shape.size() == 2 ? t.shape[1] : t.shape[0];
  if (bytes != rows * cols * el || !data) fail(HLLM_INCOMPATIBLE_WORKER, "truncated weight payload: " + name);
  HIP_CHECK(hipMemsetAsync(flags_dev(), 0, sizeof(int32_t), stream_));
  const uint64_t row_bytes = cols * el;
  const uint64_t chunk_rows = std::max<uint64_t>(1, kStagingBytes / row_bytes);
  if (row_bytes > kStagingBytes) fail(HLLM_INCOMPATIBLE_WORKER, "tensor row too large: " + name);
  for (uint64_t r0 = 0; r0 < rows; r0 += chunk_rows) {
    const uint64_t n = std::min(chunk_rows, rows - r0);
    HIP_CHECK(hipMemcpyAsync(staging_.ptr, static_cast<const char*>(data) + r0 * row_bytes,
                             n * row_bytes, hipMemcpyHostToDevice, stream_));
    relayout(t, name, staging_.ptr, dtype, 0, 0, 0.f, 0.f, r0, n);
    HIP_CHECK(hipStreamSynchronize(stream_));
  }
  read_flags(name.c_str());
  t.loaded = true;
}

void Stage::synthesize(const std::string& name, uint64_t seed, uint64_t tensor_id, float mean,
                       float sigma, uint32_t source_dtype) {
  std::lock_guard<std::mutex> lock(pass_mutex_);
  Target& t = target(name);
  if (source_dtype != HLLM_DTYPE_F32 && source_dtype != HLLM_DTYPE_F16)
    fail(HLLM_INVALID_REQUEST, "synthetic source dtype must be F32 or F16");
  HIP_CHECK(hipMemsetAsync(flags_dev(), 0, sizeof(int32_t), stream_));
  const uint64_t rows = t.shape.size() == 2 ? t.shape[0] : 1;
  relayout(t, name, nullptr, source_dtype, seed, tensor_id, mean, sigma, 0, rows);
  read_flags(name.c_str());
  t.loaded = true;
}

void Stage::finalize() {
  std::lock_guard<std::mutex> lock(pass_mutex_);
  for (auto& [name, t] : targets_) {
    if (!t.loaded) fail(HLLM_INCOMPATIBLE_WORKER, "missing required tensor: " + name);
  }
  HIP_CHECK(hipStreamSynchronize(stream_));
  staging_.release();
  finalized_ = true;
}

// --------------------------------------------------------------------- memory accounting

void Stage::sequence_memory(uint64_t tokens, uint64_t max_query, hllm_rocm_memory* cache,
                            hllm_rocm_memory* workspace) const {
  if (tokens == 0 || tokens > c_.maximum_sequence_length)
    fail(HLLM_INVALID_REQUEST, "request exceeds model context capacity");
  const uint64_t bt = kv_.block_tokens;
  const uint64_t kv_el = kv_f32_ ? 4 : 2;
  const uint64_t blocks = (tokens + bt - 1) / bt;
  const uint64_t rows = (max_query == 0 || max_query > tokens) ? tokens : max_query;
  // KV blocks come from the pool reserved at stage creation; the admission figure is the
  // HBM they occupy. Pass workspaces are reserved up front as well, so a request adds no
  // device workspace; the host holds its transport copies (request_transport_bytes,
  // cpp/include/hllm/runtime/stage_backend.hpp:36-40).
  if (cache) {
    *cache = {tokens * 3 * 8 + rows * H_ * 6, blocks * bt * 2 * K_ * D_ * kv_el * L_, 0, 0};
  }
  if (workspace) *workspace = {rows * H_ * 6 + 65536, 0, 0, 0};
}

uint32_t Stage::allocate_sequence(uint64_t tokens) {
  sequence_memory(tokens, tokens, nullptr, nullptr);
  std::lock_guard<std::mutex> lock(seq_mutex_);
  const uint64_t bt = kv_.block_tokens;
  const uint64_t blocks = (tokens + bt - 1) / bt;
  if (free_slots_.empty()) fail(HLLM_RESOURCE_EXHAUSTED, "no free sequence slot");
  if (free_blocks_.size() < blocks) fail(HLLM_RESOURCE_EXHAUSTED, "KV cache is full");
  const uint32_t slot = free_slots_.back();
  Sequence& s = sequences_[slot];
  s.blocks.assign(free_blocks_.end() - blocks, free_blocks_.end());
  std::vector<int32_t> row(table_width_, -1);
  std::copy(s.blocks.begin(), s.blocks.end(), row.begin());
  HIP_CHECK(hipMemcpy(block_table_.as<int32_t>() + (size_t)slot * table_width_, row.data(),
                      row.size() * sizeof(int32_t), hipMemcpyHostToDevice));
  free_blocks_.resize(free_blocks_.size() - blocks);
  free_slots_.pop_back();
  s.live = true;
  s.failed = false;
  s.device_token = false;
  s.in_flight = false;
  s.release_pending = false;
  s.capacity = tokens;
  s.length = 0;
  return slot;
}

void Stage::free_sequence(uint32_t handle) {
  Sequence& s = sequences_[handle];
  free_blocks_.insert(free_blocks_.end(), s.blocks.begin(), s.blocks.end());
  s = Sequence{};
  free_slots_.push_back(handle);
}

// SequenceState destruction may run while a pass that uses the sequence is in flight
// (cpp/src/worker/control_service.cpp:509-530): the handle is invalid at once, but its slot
// and KV blocks return to the pools only when that pass completes, so no later sequence
// inherits the pass's state or shares blocks the device is still writing.
void Stage::release_sequence(uint32_t handle) {
  std::lock_guard<std::mutex> lock(seq_mutex_);
  if (handle >= sequences_.size() || !sequences_[handle].live) fail(HLLM_INVALID_REQUEST, "unknown sequence");
  Sequence& s = sequences_[handle];
  if (s.in_flight) {
    s.live = false;
    s.release_pending = true;
    return;
  }
  free_sequence(handle);
}

void Stage::retire_sequences(const std::vector<uint32_t>& sequences) {
  for (uint32_t h : sequences) {
    Sequence& s = sequences_[h];
    s.in_flight = false;
    if (s.release_pending) free_sequence(h);
  }
}

uint64_t Stage::sequence_length(uint32_t handle) const {
  std::lock_guard<std::mutex> lock(seq_mutex_);
  if (handle >= sequences_.size() || !sequences_[handle].live) fail(HLLM_INVALID_REQUEST, "unknown sequence");
  return sequences_[handle].length;
}

// --------------------------------------------------------------------- diagnostics

void Stage::last_layout(uint32_t items, uint32_t rows, int32_t* cu, int32_t* pos, int32_t* slots) {
  std::lock_guard<std::mutex> lock(pass_mutex_);
  if (items > items_max_ || rows > rows_max_) fail(HLLM_INVALID_REQUEST, "layout request too large");
  HIP_CHECK(hipStreamSynchronize(stream_));
  if (cu) HIP_CHECK(hipMemcpy(cu, pack_.cu_seqlens, (items + 1) * sizeof(int32_t), hipMemcpyDeviceToHost));
  if (pos) HIP_CHECK(hipMemcpy(pos, pack_.row_position, rows * sizeof(int32_t), hipMemcpyDeviceToHost));
  if (slots) HIP_CHECK(hipMemcpy(slots, pack_.row_slot, rows * sizeof(int32_t), hipMemcpyDeviceToHost));
}

void Stage::sequence_blocks(uint32_t handle, int32_t* blocks, uint32_t capacity, uint32_t* count,
                            uint32_t* block_tokens) {
  std::lock_guard<std::mutex> lock(seq_mutex_);
  if (handle >= sequences_.size() || !sequences_[handle].live) fail(HLLM_INVALID_REQUEST, "unknown sequence");
  const auto& b = sequences_[handle].blocks;
  if (count) *count = (uint32_t)b.size();
  if (block_tokens) *block_tokens = (uint32_t)kv_.block_tokens;
  if (blocks) std::copy(b.begin(), b.begin() + std::min<size_t>(b.size(), capacity), blocks);
}

void Stage::read_tensor(const std::string& name, float* out, uint64_t elements) {
  std::lock_guard<std::mutex> lock(pass_mutex_);
  auto it = targets_.find(name);
  if (it == targets_.end() || !it->second.loaded) fail(HLLM_INVALID_REQUEST, "unknown or unloaded tensor: " + name);
  const Target& t = it->second;
  const uint64_t rows = t.shape.size() == 2 ? t.shape[0] : 1;
  const uint64_t cols = t.shape.size() == 2 ? t.shape[1] : t.shape[0];
  if (elements != rows * cols) fail(HLLM_INVALID_REQUEST, "element count mismatch");
  HIP_CHECK(hipStreamSynchronize(stream_));
  if (!t.matrix) {
    HIP_CHECK(hipMemcpy(out, t.vector->ptr, elements * sizeof(float), hipMemcpyDeviceToHost));
    return;
  }
  const Matrix& m = *t.matrix;
  std::vector<uint16_t> hi(m.rows_padded * m.cols_padded), lo;
  HIP_CHECK(hipMemcpy(hi.data(), m.hi.ptr, hi.size() * 2, hipMemcpyDeviceToHost));
  if (m.lo.ptr) {
    lo.resize(hi.size());
    HIP_CHECK(hipMemcpy(lo.data(), m.lo.ptr, lo.size() * 2, hipMemcpyDeviceToHost));
  }
  auto half_to_float = [](uint16_t b) {
    _Float16 h;
    std::memcpy(&h, &b, 2);
    return (float)h;
  };
  for (uint64_t r = 0; r < rows; ++r) {
    uint64_t dr = t.row_offset + r;
    if (t.row_mode == 1) dr = t.row_offset + (r / 32) * 64 + (r % 32);
    if (t.row_mode == 2) dr = t.row_offset + (r / 32) * 64 + 32 + (r % 32);
    for (uint64_t c = 0; c < cols; ++c) {
      const uint64_t at = flayout_index(dr, c, m.cols_padded);
      float v = half_to_float(hi[at]);
      if (!lo.empty()) v += half_to_float(lo[at]) * kLoUnscale;
      out[r * cols + c] = v;
    }
  }
}

void Stage::read_kv(uint32_t handle, uint32_t layer, float* keys, float* values) {
  std::lock_guard<std::mutex> lock(pass_mutex_);
  std::vector<int32_t> blocks;
  uint64_t length = 0;
  {
    std::lock_guard<std::mutex> sl(seq_mutex_);
    if (handle >= sequences_.size() || !sequences_[handle].live) fail(HLLM_INVALID_REQUEST, "unknown sequence");
    blocks = sequences_[handle].blocks;
    length = sequences_[handle].length;
  }
  if (layer >= L_) fail(HLLM_INVALID_REQUEST, "layer out of range");
  HIP_CHECK(hipStreamSynchronize(stream_));
  const uint64_t bt = kv_.block_tokens, el = kv_f32_ ? 4 : 2;
  const uint64_t head_elems = bt * D_;
  std::vector<char> block(2 * K_ * head_elems * el);
  for (uint64_t p0 = 0; p0 < length; p0 += bt) {
    const uint64_t b = (uint64_t)blocks[p0 / bt];
    const char* src = static_cast<const char*>(kv_pool_.ptr) +
                      (layer * kv_.layer_stride + b * 2 * K_ * head_elems) * el;
    HIP_CHECK(hipMemcpy(block.data(), src, block.size(), hipMemcpyDeviceToHost));
    for (uint64_t p = p0; p < std::min(length, p0 + bt); ++p)
      for (uint64_t which = 0; which < 2; ++which)
        for (uint64_t hd = 0; hd < K_; ++hd)
          for (uint64_t d = 0; d < D_; ++d) {
            // the block's elements as laid out by kv_key_index / kv_value_index
            const int o = (int)(p - p0);
            const uint64_t i = which ? kv_value_index(kv_, 0, 0, o, (int)hd, (int)d)
                                     : kv_key_index(kv_, 0, 0, o, (int)hd, (int)d);
            float v;
            if (kv_f32_) {
              std::memcpy(&v, block.data() + i * 4, 4);
            } else {
              _Float16 hv;
              std::memcpy(&hv, block.data() + i * 2, 2);
              v = (float)hv;
            }
            (which ? values : keys)[(p * K_ + hd) * D_ + d] = v;
          }
  }
}

// --------------------------------------------------------------------- profiling

hipEvent_t Stage::take_event() {
  if (event_pool_.empty()) {
    hipEvent_t e;
    HIP_CHECK(hipEventCreate(&e));
    return e;
  }
  hipEvent_t e = event_pool_.back();
  event_pool_.pop_back();
  return e;
}

template <typename F>
void Stage::timed(const char* family, uint64_t bytes, double flops, F&& launch) {
  // Filters are family prefixes ("*" = all) or "k:<kernel>" (that kernel only, whichever
  // family launches it).
  bool family_selected = false, kernel_filters = false;
  if (profiling_) {
    for (const auto& f : profile_filter_) {
      if (f.compare(0, 2, "k:") == 0)
        kernel_filters = true;
      else if (f == "*" || std::strncmp(family, f.c_str(), f.size()) == 0)
        family_selected = true;
    }
  }
  if (!family_selected && !kernel_filters) {
    launch();
    return;
  }
  // Events around every kernel the launch issues (the launchers report each one).
  struct Observer final : LaunchObserver {
    Stage* stage;
    const char* family;
    uint64_t bytes;
    double flops;
    bool all = false;  // every kernel of the launch, or only the filtered ones
    int kernels = 0;
    bool active = false;
    hipEvent_t start = nullptr;
    bool wanted(const char* kernel) const {
      if (all) return true;
      for (const auto& f : stage->profile_filter_)
        if (f.compare(0, 2, "k:") == 0 && f.compare(2, std::string::npos, kernel) == 0) return true;
      return false;
    }
    void before(const char* kernel) override {
      active = wanted(kernel);
      if (!active) return;
      start = stage->take_event();
      HIP_CHECK(hipEventRecord(start, stage->stream_));
    }
    void after(const char* kernel) override {
      if (!active) {
        ++kernels;
        return;
      }
      hipEvent_t stop = stage->take_event();
      HIP_CHECK(hipEventRecord(stop, stage->stream_));
      const bool first = kernels++ == 0;
      Profile& f = stage->profiles_[family];
      f.events.emplace_back(start, stop);
      if (first) {
        f.launches += 1;
        f.bytes += bytes;
        f.flops += flops;
      }
      for (const std::string& name : {std::string("k:") + kernel, std::string(family) + "/" + kernel}) {
        Profile& k = stage->profiles_[name];
        k.owns_events = false;
        k.events.emplace_back(start, stop);
        k.launches += 1;
        if (first) {
          k.bytes += bytes;
          k.flops += flops;
        }
      }
    }
  } observer;
  observer.stage = this;
  observer.all = family_selected;
  observer.family = family;
  observer.bytes = bytes;
  observer.flops = flops;
  LaunchObserver* previous = launch_observer;
  launch_observer = &observer;
  try {
    launch();
  } catch (...) {
    launch_observer = previous;
    throw;
  }
  launch_observer = previous;
}

void Stage::set_profiling(const std::string& families) {
  std::lock_guard<std::mutex> lock(pass_mutex_);
  HIP_CHECK(hipStreamSynchronize(stream_));
  for (auto& [name, p] : profiles_)
    if (p.owns_events)
      for (auto& e : p.events) event_pool_.push_back(e.first), event_pool_.push_back(e.second);
  profiles_.clear();
  profile_filter_.clear();
  size_t start = 0;
  while (start <= families.size()) {
    const size_t end = std::min(families.find(';', start), families.size());
    if (end > start) profile_filter_.push_back(families.substr(start, end - start));
    start = end + 1;
  }
  profiling_ = !profile_filter_.empty();
}

void Stage::profile_read(const std::string& record, double* ms, uint64_t* launches, uint64_t* bytes,
                         double* flops) {
  std::lock_guard<std::mutex> lock(pass_mutex_);
  HIP_CHECK(hipStreamSynchronize(stream_));
  const bool prefix = !record.empty() && record.back() == '*';
  const std::string stem = prefix ? record.substr(0, record.size() - 1) : record;
  double total = 0.0, f = 0.0;
  uint64_t n = 0, b = 0;
  for (auto& [name, p] : profiles_) {
    if (!(prefix ? name.compare(0, stem.size(), stem) == 0 : name == record)) continue;
    for (auto& e : p.events) {
      float t = 0.f;
      HIP_CHECK(hipEventElapsedTime(&t, e.first, e.second));
      total += t;
    }
    n += p.launches;
    b += p.bytes;
    f += p.flops;
  }
  *ms = total;
  *launches = n;
  *bytes = b;
  *flops = f;
}

std::string Stage::profile_records() {
  std::lock_guard<std::mutex> lock(pass_mutex_);
  std::string out;
  for (auto& [name, p] : profiles_) out += name + "\n";
  return out;
}

// --------------------------------------------------------------------- the pass

// Launches one projection; with `defer`, K-split partials are left in the workspace for the
// consumer and their count is returned (0: the epilogue has been applied).
int Stage::gemm(const char* family, const Matrix& w, const uint16_t* x_hi, const uint16_t* x_lo,
                int rows, int n, int epilogue, float* out, int ldo, uint16_t* out_hi,
                uint16_t* out_lo, uint64_t out_cols_padded, bool defer, int argmax_parts) {
  GemmArgs a{};
  a.defer_reduce = defer ? 1 : 0;
  a.w_hi = w.hi.as<uint16_t>();
  a.w_lo = w.lo.as<uint16_t>();
  a.x_hi = x_hi;
  a.x_lo = x_lo;
  a.M = rows;
  a.N = n;
  a.w_rows_padded = w.rows_padded;
  a.x_rows_padded = rows_padded_;
  a.Kp = w.cols_padded;
  a.workspace = gemm_ws_.as<float>();
  a.workspace_floats = gemm_ws_floats_;
  a.counters = gemm_counters_.as<int32_t>();
  a.counter_count = gemm_counter_count_;
  a.epilogue = epilogue;
  a.out = out;
  a.ldo = ldo;
  a.out_hi = out_hi;
  a.out_lo = out_lo;
  a.out_cols_padded = out_cols_padded;
  if (argmax_parts > 0) {
    a.argmax_val = argmax_val_.as<float>();
    a.argmax_idx = argmax_idx_.as<int32_t>();
    a.argmax_flags = flags_dev();
    a.argmax_parts = argmax_parts;
  }
  const uint64_t wbytes = (uint64_t)n * w.cols_padded * 2 * (w_f32_ ? 2 : 1);
  const uint64_t xbytes = (uint64_t)rows * w.cols_padded * 2 * (x_lo ? 2 : 1);
  const uint64_t obytes = epilogue == kEpiArgmax ? 0
                          : epilogue == kEpiSwiglu ? (uint64_t)rows * (n / 2) * 2 * (out_lo ? 2 : 1)
                                                   : (uint64_t)rows * n * 4 * (epilogue == kEpiResidual ? 2 : 1);
  const double flops = 2.0 * rows * n * w.cols;
  int parts = 0;
  timed(family, wbytes + xbytes + obytes, flops, [&] { parts = launch_gemm(stream_, a, prec_, rows, cus_); });
  return parts;
}

// A pass that failed after its work was enqueued: the device may have written part of the
// sequences' KV, so they are never resumed (cpp/src/cuda/stage.cpp:463-468), and their
// in-flight use ends here.
void Stage::fail_pass(const std::vector<uint32_t>& sequences) {
  (void)hipStreamSynchronize(stream_);
  std::lock_guard<std::mutex> lock(seq_mutex_);
  for (uint32_t s : sequences) {
    sequences_[s].failed = true;
    sequences_[s].device_token = false;
  }
  retire_sequences(sequences);
}

void Stage::mark_phase(const char* component, int32_t layer) {
  if (!phases_on_) return;
  hipEvent_t e = take_event();
  HIP_CHECK(hipEventRecord(e, stream_));
  phase_marks_.push_back({component, layer, e});
}

void Stage::submit(const hllm_rocm_pass& pass, bool phases) {
  std::unique_lock<std::mutex> lock(pass_mutex_);
  if (!finalized_) fail(HLLM_INVALID_REQUEST, "stage is not finalized");
  if (in_flight_) fail(HLLM_INVALID_REQUEST, "a pass is already in flight");
  const uint32_t n = pass.items;
  if (n == 0 || n > items_max_ || !pass.item) fail(HLLM_INVALID_REQUEST, "invalid pass size");
  // ---- validate the request on the host (inputs first, then the sequences' state) before
  // touching the device
  uint64_t rows = 0;
  std::vector<uint32_t> seqs(n);
  std::vector<int> sample_items;
  std::vector<int> top_counts;
  bool sampler = false;
  SampleParams* params = pin_sample_params_.as<SampleParams>();
  for (uint32_t i = 0; i < n; ++i) {
    const hllm_rocm_item& it = pass.item[i];
    if (it.query_tokens == 0 || it.query_tokens > c_.maximum_sequence_length ||
        it.first_position > c_.maximum_sequence_length)
      fail(HLLM_INVALID_REQUEST, "invalid sequence state, position or context capacity");
    // The device keeps the token sampled by the final stage, and only the first stage
    // embeds tokens: device-fed inputs need a stage that is both.
    if ((it.flags & HLLM_ITEM_TOKEN_FROM_DEVICE) && (!c_.first_stage || !c_.final_stage || it.query_tokens != 1))
      fail(HLLM_INVALID_REQUEST, "device-fed input needs one token on a stage that embeds and samples");
    if (it.flags & HLLM_ITEM_SAMPLE) {
      check_sampling(it);
      if (c_.final_stage) {
        const bool logprobs = (it.flags & HLLM_ITEM_LOGPROBS) != 0;
        params[sample_items.size()] = {it.temperature, it.top_p, it.top_k, it.seed, it.generated_index,
                                       logprobs ? it.top_logprobs : 0u, logprobs ? kSampleLogprobs : 0u};
        sampler |= it.temperature != 0.0 || logprobs;
        top_counts.push_back(logprobs ? (int)it.top_logprobs : -1);
        sample_items.push_back((int)i);
      }
    }
    seqs[i] = it.sequence;
    rows += it.query_tokens;
  }
  if (rows > rows_max_) fail(HLLM_RESOURCE_EXHAUSTED, "pass exceeds the stage's row budget");
  if (c_.first_stage && !pass.token_ids) fail(HLLM_INVALID_REQUEST, "stage zero requires tokens");
  if (!c_.first_stage && !pass.boundary_in) fail(HLLM_INVALID_REQUEST, "only stage zero accepts tokens");
  ItemMeta* meta = pin_items_.as<ItemMeta>();
  int32_t* host_tokens = pin_tokens();
  {
    uint64_t r = 0;
    for (uint32_t i = 0; i < n; ++i) {
      const hllm_rocm_item& it = pass.item[i];
      meta[i] = {it.sequence, it.query_tokens, (uint32_t)it.first_position, it.flags};
      for (uint32_t j = 0; j < it.query_tokens; ++j, ++r) {
        if (c_.first_stage) {
          const bool from_device = it.flags & HLLM_ITEM_TOKEN_FROM_DEVICE;
          const uint64_t id = from_device ? 0 : pass.token_ids[r];
          if (id >= V_) fail(HLLM_INVALID_REQUEST, "token ID exceeds vocabulary");
          host_tokens[r] = (int32_t)id;
        }
      }
    }
  }
  if (!c_.first_stage) {
    const uint64_t count = rows * H_;
    for (uint64_t i = 0; i < count; ++i) {
      if ((pass.boundary_in[i] & 0x7c00u) == 0x7c00u) fail(HLLM_INVALID_REQUEST, "non-finite activation");
    }
    std::memcpy(pin_boundary_.ptr, pass.boundary_in, count * 2);
  }
  if (cancel_requested(pass)) fail(HLLM_CANCELLED, "request cancelled");
  // Algorithmic attention bytes of one layer: every item's keys and values read once,
  // queries read and outputs written once.
  // FLOPs: 4 * D per (query head, attended key) pair (scores and the value sum).
  uint64_t attn_bytes = 0;
  double attn_flops = 0.0;
  {
    const uint64_t kv_el = kv_f32_ ? 4 : 2;
    for (uint32_t i = 0; i < n; ++i) {
      const double q = pass.item[i].query_tokens, first = (double)pass.item[i].first_position;
      attn_bytes += (pass.item[i].first_position + pass.item[i].query_tokens) * 2 * K_ * D_ * kv_el;
      attn_flops += 4.0 * Q_ * D_ * (q * first + q * (q + 1) / 2);
    }
    attn_bytes += rows * Q_ * D_ * (4 + 2);
  }
  int attn_work_count = 0;
  // Some block's keys split in two or more: the split combine runs after the attention.
  bool attn_any_split = false;
  if (mfma_attention_) {
    for (uint32_t i = 0; i < n; ++i) {
      const int work = attn_item_work((int)pass.item[i].query_tokens, (int)pass.item[i].first_position,
                                      (int)(Q_ / K_), kMaxSplits, pack_.attn_decode_unit, pack_.attn_decode_split);
      attn_work_count += work;
      attn_any_split |= attn_item_needs_combine((int)pass.item[i].query_tokens, (int)pass.item[i].first_position,
                                                (int)(Q_ / K_), kMaxSplits, pack_.attn_decode_unit, pack_.attn_decode_split,
                                                pack_.attn_fold);
    }
    if ((uint64_t)attn_work_count > attn_work_max_) fail(HLLM_INTERNAL, "attention work list overflow");
  }
  // Passes of single-token items (decode rows) at head dim 128 with F16 KV: QK-norm, RoPE and
  // the K/V append run inside the attention kernel (AttentionRope), one launch fewer per layer.
  bool fuse_rope = mfma_attention_ && !kv_f32_ && D_ == 128 && Q_ / K_ <= 16 && rope_fusion_enabled();
  for (uint32_t i = 0; i < n && fuse_rope; ++i) fuse_rope = pass.item[i].query_tokens == 1;

  // ---- device work. Every launch parameter below is a function of the pass shape (n, R,
  // S, sampler): the rest is read on the device. `capturing`: recorded into a graph.
  const int R = (int)rows;
  const int S = (int)sample_items.size();
  // One attention workgroup (per KV head) per work item: the hardware's dispatch balances
  // items of different lengths.
  const int attn_grid = attn_work_count;
  // Greedy passes that return no logits take each row's first maximum from the LM head's
  // epilogue (one candidate per workgroup; the logits are never written): its part count,
  // 0 when the logits are written and argmax kernels read them.
  int fused_parts = 0;
  if (c_.final_stage && S > 0 && !sampler && !pass.logits) {
    const Matrix& head = c_.tied_head ? embedding_ : head_;
    GemmArgs probe{};
    probe.M = S;
    probe.N = (int)V_;
    probe.w_rows_padded = head.rows_padded;
    probe.x_rows_padded = rows_padded_;
    probe.Kp = head.cols_padded;
    probe.epilogue = kEpiArgmax;
    fused_parts = gemm_argmax_parts(probe, prec_, S, cus_);
    if ((uint64_t)fused_parts * S > argmax_capacity_) fused_parts = 0;
  }
  auto enqueue = [&](bool capturing) {
    // The item list (all slots) and, on the first stage, the pass's tokens: one copy.
    HIP_CHECK(hipMemcpyAsync(items_dev_.ptr, meta, tokens_offset() + (c_.first_stage ? R * sizeof(int32_t) : 0),
                             hipMemcpyHostToDevice, stream_));
    timed("pack", 0, 0.0, [&] {
      launch_pack(stream_, items_dev_.as<ItemMeta>(), (int)n, host_tokens_dev(),
                  last_token_.as<int32_t>(), block_table_.as<int32_t>(), table_width_, kv_.block_tokens, pack_);
    });
    float* h = h_.as<float>();
    if (c_.first_stage) {
      timed("embed", (uint64_t)R * H_ * 6, 0.0, [&] {
        launch_embed(stream_, embedding_.hi.as<uint16_t>(), w_f32_ ? embedding_.lo.as<uint16_t>() : nullptr,
                     embedding_.cols_padded, pack_.row_token, R, (int)H_, h);
      });
    } else {
      HIP_CHECK(hipMemcpyAsync(boundary_dev_.ptr, pin_boundary_.ptr, (size_t)R * H_ * 2, hipMemcpyHostToDevice,
                               stream_));
      timed("boundary", (uint64_t)R * H_ * 6, 0.0,
            [&] { launch_boundary_decode(stream_, boundary_dev_.as<uint16_t>(), R, (int)H_, h); });
    }
    mark_phase(c_.first_stage ? "embedding" : "from-wire", -1);
    uint16_t* a0h = a0_hi_.as<uint16_t>();
    uint16_t* a0l = a0_lo_.as<uint16_t>();
    uint16_t* a1h = a1_hi_.as<uint16_t>();
    uint16_t* a1l = a1_lo_.as<uint16_t>();
    const float eps = c_.rms_norm_epsilon;
    const uint64_t a1_cols = std::max(QDp_, Ip_);
    (void)a1_cols;
    // K-split partials of a projection are summed by the kernel that consumes it: q/k/v's
    // by RoPE/append, o's and down's (residual adds) by the next RMSNorm. `pending` holds
    // the previous layer's down-projection partials until this layer's input norm.
    float* ws = gemm_ws_.as<float>();
    Partials pending{};
    for (uint64_t l = 0; l < L_; ++l) {
      if (!capturing && cancel_requested(pass)) fail(HLLM_CANCELLED, "request cancelled");
      Layer& w = *layers_[l];
      timed("norm", (uint64_t)R * H_ * 6, 0.0, [&] {
        launch_rmsnorm_flayout(stream_, h, (int)H_, nullptr, R, nullptr, w.input_norm.as<float>(), eps, a0h, a0l,
                               Hp_, pending);
      });
      pending = {};
      const int qkv_parts = gemm("gemm_qkv", w.qkv, a0h, a0l, R, (int)qkv_n_, kEpiStore, qkv_.as<float>(),
                                 (int)qkv_n_, nullptr, nullptr, 0, true);
      if (!fuse_rope) {
        timed("rope_append", (uint64_t)R * qkv_n_ * 6, 0.0, [&] {
          launch_qkv_rope_append(stream_, qkv_.as<float>(), R, (int)Q_, (int)K_, (int)D_,
                                 c_.query_key_norm ? w.q_norm.as<float>() : nullptr,
                                 c_.query_key_norm ? w.k_norm.as<float>() : nullptr, eps, rope_cos_.as<float>(),
                                 rope_sin_.as<float>(), pack_.row_position, pack_.row_slot, kv_, (int)l,
                                 q_.as<float>(), Partials{ws, qkv_parts, (uint64_t)R * qkv_n_});
        });
      }
      AttentionArgs at{};
      if (fuse_rope) {
        at.rope.qkv = qkv_.as<float>();
        at.rope.parts = Partials{ws, qkv_parts, (uint64_t)R * qkv_n_};
        at.rope.q_norm = c_.query_key_norm ? w.q_norm.as<float>() : nullptr;
        at.rope.k_norm = c_.query_key_norm ? w.k_norm.as<float>() : nullptr;
        at.rope.eps = eps;
        at.rope.rope_cos = rope_cos_.as<float>();
        at.rope.rope_sin = rope_sin_.as<float>();
        at.rope.row_slot = pack_.row_slot;
      }
      at.work = attn_work_.as<AttnWork>();
      at.work_count = attn_count_.as<int32_t>();
      at.work_grid = attn_grid;
      at.any_split = attn_any_split ? 1 : 0;
      at.row_splits = pack_.row_splits;
      at.fold = pack_.attn_fold;
      at.split_arrivals = attn_arrivals_.as<int32_t>();
      at.q = q_.as<float>();
      at.rows = R;
      at.q_heads = (int)Q_;
      at.kv_heads = (int)K_;
      at.head_dim = (int)D_;
      at.row_item = pack_.row_item;
      at.row_position = pack_.row_position;
      at.items = items_dev_.as<ItemMeta>();
      at.block_table = block_table_.as<int32_t>();
      at.table_width = table_width_;
      at.kv = kv_;
      at.layer = (int)l;
      at.scale = 1.0f / std::sqrt(static_cast<float>(D_));
      at.partial = attn_partial_.as<float>();
      at.max_splits = kMaxSplits;
      at.split_unit = kSplitUnit;
      at.out_hi = a1h;
      at.out_lo = a1l;
      at.out_cols_padded = QDp_;
      timed("attention", attn_bytes, attn_flops, [&] { launch_attention(stream_, at); });
      const int o_parts = gemm("gemm_o", w.o, a1h, a1l, R, (int)H_, kEpiResidual, h, (int)H_, nullptr, nullptr, 0,
                               true);
      timed("norm", (uint64_t)R * H_ * 6, 0.0, [&] {
        launch_rmsnorm_flayout(stream_, h, (int)H_, nullptr, R, nullptr, w.post_norm.as<float>(), eps, a0h, a0l,
                               Hp_, Partials{ws, o_parts, (uint64_t)R * H_});
      });
      gemm("gemm_gate_up", w.gate_up, a0h, a0l, R, (int)(2 * Ip_), kEpiSwiglu, nullptr, 0, a1h, a1l, Ip_);
      // The last layer's down partials are summed by the final norm, for the sampled rows it
      // gathers (nothing reads the other rows' residual afterwards); a boundary stage sums
      // them here (the boundary reads the whole stream).
      const bool defer_down = l + 1 < L_ || c_.final_stage;
      const int down_parts = gemm("gemm_down", w.down, a1h, a1l, R, (int)H_, kEpiResidual, h, (int)H_, nullptr,
                                  nullptr, 0, defer_down);
      pending = Partials{ws, down_parts, (uint64_t)R * H_};
      HIP_CHECK(hipGetLastError());
      mark_phase("layer", (int32_t)(c_.layer_start + l));
      if (pass.trace_hidden) {
        // The trace reads the completed residual stream: the pending partials are added
        // here, with the additions the next norm would make, so a traced pass computes
        // exactly what an untraced one does.
        launch_residual_sum(stream_, h, R, (int)H_, pending);
        pending = {};
        HIP_CHECK(hipMemcpyAsync(pass.trace_hidden + l * (size_t)R * H_, h, (size_t)R * H_ * sizeof(float),
                                 hipMemcpyDeviceToHost, stream_));
        HIP_CHECK(hipStreamSynchronize(stream_));
      }
    }
    if (c_.final_stage) {
      if (S > 0) {
        timed("norm", (uint64_t)S * H_ * 6, 0.0, [&] {
          launch_rmsnorm_flayout(stream_, h, (int)H_, pack_.sample_row, S, nullptr, final_norm_.as<float>(), eps,
                                 a0h, a0l, Hp_, pending);
        });
        mark_phase("final_norm", -1);
        const Matrix& head = c_.tied_head ? embedding_ : head_;
        // Without a sampler the argmax also records each sequence's last token (no separate
        // launch).
        if (fused_parts > 0) {
          gemm("gemm_lm_head", head, a0h, a0l, S, (int)V_, kEpiArgmax, nullptr, 0, nullptr, nullptr, 0, false,
               fused_parts);
          mark_phase("lm_head", -1);
          timed("argmax", 0, 0.0, [&] {
            launch_argmax_final(stream_, pack_.sample_count, S, fused_parts, argmax_val_.as<float>(),
                                argmax_idx_.as<int32_t>(), tokens_.as<int32_t>(), pack_.sample_item,
                                items_dev_.as<ItemMeta>(), last_token_.as<int32_t>());
          });
        } else {
          gemm("gemm_lm_head", head, a0h, a0l, S, (int)V_, kEpiStore, logits_.as<float>(), (int)V_, nullptr,
               nullptr, 0);
          mark_phase("lm_head", -1);
          timed("argmax", (uint64_t)S * V_ * 4, 0.0, [&] {
            launch_argmax(stream_, logits_.as<float>(), pack_.sample_count, S, (int)V_, argmax_val_.as<float>(),
                          argmax_idx_.as<int32_t>(), kArgmaxParts, tokens_.as<int32_t>(), flags_dev(),
                          sampler ? nullptr : pack_.sample_item, sampler ? nullptr : items_dev_.as<ItemMeta>(),
                          sampler ? nullptr : last_token_.as<int32_t>());
          });
        }
        if (sampler) {
          HIP_CHECK(hipMemcpyAsync(sample_params_.ptr, pin_sample_params_.ptr, S * sizeof(SampleParams),
                                   hipMemcpyHostToDevice, stream_));
          SampleArgs sa{};
          sa.logits = logits_.as<float>();
          sa.vocab = (int)V_;
          sa.rows = S;
          sa.params = sample_params_.as<SampleParams>();
          sa.tokens = tokens_.as<int32_t>();
          sa.logprob = sample_out_.as<double>();
          sa.top_values = sa.logprob + items_max_;
          sa.top_ids = reinterpret_cast<int32_t*>(sa.top_values + 5 * items_max_);
          sa.weights = sample_weights_.as<double>();
          sa.buckets = sample_buckets_.as<uint8_t>();
          sa.bucket_stride = sample_bucket_stride(V_);
          sa.lists = sample_lists_.as<uint32_t>();
          sa.hist = sample_hist_.as<uint64_t>();
          sa.lse_parts = sample_lse_.as<double>();
          sa.sorted = sample_sorted_.as<uint32_t>();
          sa.cursor = sample_cursor_.as<uint32_t>();
          sa.candidates = sample_candidates_.as<uint32_t>();
          sa.group_rows = sample_blocks_;
          sa.chunks = sample_chunks_;
          timed("sample", (uint64_t)S * V_ * 4, 0.0, [&] { launch_sample(stream_, sa); });
          HIP_CHECK(hipMemcpyAsync(pin_sample_out_.ptr, sample_out_.ptr, sample_out_.bytes, hipMemcpyDeviceToHost,
                                   stream_));
        }
        if (sampler)
          launch_record_tokens(stream_, tokens_.as<int32_t>(), pack_.sample_item, pack_.sample_count,
                               items_dev_.as<ItemMeta>(), last_token_.as<int32_t>());
        mark_phase("sampling", -1);
        if (pass.logits)
          HIP_CHECK(hipMemcpyAsync(pass.logits, logits_.ptr, (size_t)S * V_ * sizeof(float),
                                   hipMemcpyDeviceToHost, stream_));
      }
    } else {
      timed("boundary", (uint64_t)R * H_ * 6, 0.0, [&] {
        launch_boundary_encode(stream_, h, R, (int)H_, boundary_dev_.as<uint16_t>(), flags_dev());
      });
      HIP_CHECK(hipMemcpyAsync(pin_boundary_.ptr, boundary_dev_.ptr, (size_t)R * H_ * 2, hipMemcpyDeviceToHost,
                               stream_));
      mark_phase("to-wire", -1);
    }
    // The sampled tokens (final stage) and the error flags behind them: one copy.
    if (c_.final_stage && S > 0)
      HIP_CHECK(hipMemcpyAsync(pin_out_tokens_.ptr, tokens_.ptr, (items_max_ + 1) * sizeof(int32_t),
                               hipMemcpyDeviceToHost, stream_));
    else
      HIP_CHECK(hipMemcpyAsync(pin_flags(), flags_dev(), sizeof(int32_t), hipMemcpyDeviceToHost, stream_));
    HIP_CHECK(hipGetLastError());
  };
  // ---- the sequences' state, checked and claimed for this pass under one lock
  {
    std::lock_guard<std::mutex> sl(seq_mutex_);
    std::set<uint32_t> unique;
    for (uint32_t i = 0; i < n; ++i) {
      const hllm_rocm_item& it = pass.item[i];
      if (it.sequence >= sequences_.size() || !sequences_[it.sequence].live)
        fail(HLLM_INVALID_REQUEST, "unknown sequence");
      const Sequence& s = sequences_[it.sequence];
      if (s.failed || it.first_position != s.length ||
          it.query_tokens > s.capacity - std::min(s.capacity, s.length) || !unique.insert(it.sequence).second)
        fail(HLLM_INVALID_REQUEST, "invalid sequence state, position or context capacity");
      if ((it.flags & HLLM_ITEM_TOKEN_FROM_DEVICE) && !s.device_token)
        fail(HLLM_INVALID_REQUEST, "device-fed input needs a token sampled by the sequence's previous pass");
    }
    for (uint32_t s : seqs) sequences_[s].in_flight = true;
  }
  phases_on_ = phases;
  for (const PhaseMark& m : phase_marks_) event_pool_.push_back(m.end);
  phase_marks_.clear();
  if (phases && !phase_start_) phase_start_ = take_event();
  try {
    if (phases) HIP_CHECK(hipEventRecord(phase_start_, stream_));
    const PassShape shape{n, (uint32_t)R, (uint32_t)S, sampler ? 1u : 0u, (uint32_t)attn_grid,
                          attn_any_split ? 1u : 0u, fused_parts, forced_gemm_config()};
    const bool graphable = graphs_enabled_ && !profiling_ && !phases && !pass.logits && !pass.trace_hidden;
    auto found = graphable ? graphs_.find(shape) : graphs_.end();
    if (found != graphs_.end()) {
      found->second.used = ++graph_clock_;
      ++graph_replays_;
      HIP_CHECK(hipGraphLaunch(found->second.exec, stream_));
    } else if (graphable && shapes_seen_.count(shape)) {
      CapturedPass cp;
      HIP_CHECK(hipStreamBeginCapture(stream_, hipStreamCaptureModeThreadLocal));
      try {
        enqueue(true);
      } catch (...) {
        hipGraph_t dropped = nullptr;
        (void)hipStreamEndCapture(stream_, &dropped);
        if (dropped) (void)hipGraphDestroy(dropped);
        throw;
      }
      HIP_CHECK(hipStreamEndCapture(stream_, &cp.graph));
      const hipError_t e = hipGraphInstantiate(&cp.exec, cp.graph, nullptr, nullptr, 0);
      if (e != hipSuccess) {
        (void)hipGraphDestroy(cp.graph);
        graphs_enabled_ = false;  // this runtime cannot replay passes: run them eagerly
        enqueue(false);
      } else {
        if (graphs_.size() >= kMaxGraphs) {
          auto oldest = graphs_.begin();
          for (auto g = graphs_.begin(); g != graphs_.end(); ++g)
            if (g->second.used < oldest->second.used) oldest = g;
          (void)hipGraphExecDestroy(oldest->second.exec);
          (void)hipGraphDestroy(oldest->second.graph);
          graphs_.erase(oldest);
        }
        cp.used = ++graph_clock_;
        graphs_[shape] = cp;
        ++graph_captures_;
        ++graph_replays_;
        HIP_CHECK(hipGraphLaunch(cp.exec, stream_));
      }
    } else {
      if (graphable) {
        if (shapes_seen_.size() >= 4096) shapes_seen_.clear();
        shapes_seen_.insert(shape);
      }
      enqueue(false);
    }
  } catch (...) {
    fail_pass(seqs);
    throw;
  }
  in_flight_ = true;
  pending_ = pass;
  pending_sequences_ = seqs;
  pending_lengths_.assign(n, 0);
  for (uint32_t i = 0; i < n; ++i) pending_lengths_[i] = pass.item[i].query_tokens;
  pending_sample_items_ = sample_items;
  pending_top_counts_ = top_counts;
  pending_sampler_ = sampler;
  pending_rows_ = rows;
}

void Stage::wait(hllm_rocm_phase_time* phases, uint32_t capacity, uint32_t* count) {
  std::unique_lock<std::mutex> lock(pass_mutex_);
  if (!in_flight_) fail(HLLM_INVALID_REQUEST, "no pass in flight");
  in_flight_ = false;
  const hipError_t e = hipStreamSynchronize(stream_);
  if (e != hipSuccess) {
    fail_pass(pending_sequences_);
    check_hip(e, "pass");
  }
  // Cancellation is checked before each layer is enqueued and once more when the pass has
  // completed, before the sequences advance (cpp/src/cuda/stage.cpp:396,456): a pass
  // cancelled while it ran is discarded and its sequences are never resumed.
  if (cancel_requested(pending_)) {
    fail_pass(pending_sequences_);
    fail(HLLM_CANCELLED, "request cancelled");
  }
  if (count) *count = 0;
  if (phases_on_) {
    hipEvent_t previous = phase_start_;
    uint32_t k = 0;
    for (const PhaseMark& m : phase_marks_) {
      float ms = 0.f;
      HIP_CHECK(hipEventElapsedTime(&ms, previous, m.end));
      previous = m.end;
      if (phases && k < capacity) {
        hllm_rocm_phase_time& t = phases[k];
        std::memset(t.component, 0, sizeof(t.component));
        std::strncpy(t.component, m.component, sizeof(t.component) - 1);
        t.layer = m.layer;
        t.milliseconds = ms;
      }
      ++k;
    }
    if (count) *count = k;
    phases_on_ = false;
  }
  const int32_t flags = *pin_flags();
  if (flags & 2) {
    fail_pass(pending_sequences_);
    fail(HLLM_INTERNAL, "cannot sample nonfinite logits");
  }
  if (flags & 4) {
    fail_pass(pending_sequences_);
    fail(HLLM_INTERNAL, "activation is not representable as finite FP16");
  }
  const hllm_rocm_pass& pass = pending_;
  if (c_.final_stage && pass.tokens) {
    for (uint32_t i = 0; i < pass.items; ++i) pass.tokens[i] = UINT64_MAX;
    const int32_t* t = pin_out_tokens_.as<int32_t>();
    for (size_t j = 0; j < pending_sample_items_.size(); ++j) pass.tokens[pending_sample_items_[j]] = (uint64_t)t[j];
  }
  if (c_.final_stage && pending_sampler_) {
    const double* logprob = pin_sample_out_.as<double>();
    const double* top_values = logprob + items_max_;
    const int32_t* top_ids = reinterpret_cast<const int32_t*>(top_values + 5 * items_max_);
    for (size_t j = 0; j < pending_sample_items_.size(); ++j) {
      const int count = std::min(pending_top_counts_[j], (int)std::min<uint64_t>(V_, 5));
      if (count < 0) continue;
      const size_t item = (size_t)pending_sample_items_[j];
      if (pass.logprobs) pass.logprobs[item] = logprob[j];
      for (int r = 0; r < 5; ++r) {
        if (pass.top_ids) pass.top_ids[item * 5 + r] = r < count ? (uint64_t)top_ids[j * 5 + r] : UINT64_MAX;
        if (pass.top_logprobs)
          pass.top_logprobs[item * 5 + r] = r < count ? top_values[j * 5 + r] : std::nan("");
      }
    }
  }
  if (!c_.final_stage && pass.boundary_out) std::memcpy(pass.boundary_out, pin_boundary_.ptr, pending_rows_ * H_ * 2);
  std::lock_guard<std::mutex> sl(seq_mutex_);
  for (size_t i = 0; i < pending_sequences_.size(); ++i) {
    Sequence& s = sequences_[pending_sequences_[i]];
    s.length += pending_lengths_[i];
    s.device_token = false;
  }
  for (int item : pending_sample_items_) sequences_[pending_sequences_[item]].device_token = true;
  retire_sequences(pending_sequences_);
}

// The sampling options of one item, checked as runtime::validate_sampling
// (cpp/src/sampling.cpp:10-17) does.
void check_sampling(const hllm_rocm_item& it) {
  if (!(it.temperature >= 0.0 && it.temperature <= 100.0) || !(it.top_p > 0.0 && it.top_p <= 1.0) ||
      it.top_logprobs > 5 || (!(it.flags & HLLM_ITEM_LOGPROBS) && it.top_logprobs != 0))
    fail(HLLM_INVALID_REQUEST, "invalid sampling parameters");
}

hllm_rocm_allocator_metrics allocator_metrics(int32_t device) {
  int count = 0;
  HIP_CHECK(hipGetDeviceCount(&count));
  if (device < 0 || device >= count) fail(HLLM_INVALID_REQUEST, "device ordinal out of range");
  Ledger& l = ledger();
  std::lock_guard<std::mutex> lock(l.mutex);
  const auto it = l.devices.find(device);
  const auto [active, peak] = it == l.devices.end() ? std::pair<uint64_t, uint64_t>{0, 0} : it->second;
  return {active, 0, peak};
}

void reset_peak(int32_t device) {
  int count = 0;
  HIP_CHECK(hipGetDeviceCount(&count));
  if (device < 0 || device >= count) fail(HLLM_INVALID_REQUEST, "device ordinal out of range");
  int current = 0;
  HIP_CHECK(hipGetDevice(&current));
  HIP_CHECK(hipSetDevice(device));
  const hipError_t e = hipDeviceSynchronize();
  (void)hipSetDevice(current);
  check_hip(e, "device synchronize");
  Ledger& l = ledger();
  std::lock_guard<std::mutex> lock(l.mutex);
  auto& [active, peak] = l.devices[device];
  peak = active;
}

hllm_rocm_device_info device_info(int32_t device) {
  int count = 0;
  HIP_CHECK(hipGetDeviceCount(&count));
  if (device < 0 || device >= count) fail(HLLM_INVALID_REQUEST, "device ordinal out of range");
  hipDeviceProp_t p{};
  HIP_CHECK(hipGetDeviceProperties(&p, device));
  hllm_rocm_device_info out{};
  // ROCm reports the UUID as 16 ASCII hex digits (the unique ID of the GPU); other bytes are
  // written as hex.
  bool ascii = true;
  for (int i = 0; i < 16; ++i) ascii &= std::isxdigit(static_cast<unsigned char>(p.uuid.bytes[i])) != 0;
  static const char* hex = "0123456789abcdef";
  for (int i = 0; i < 16; ++i) {
    const unsigned char b = static_cast<unsigned char>(p.uuid.bytes[i]);
    if (ascii) {
      out.identity[i] = static_cast<char>(std::tolower(b));
    } else {
      out.identity[2 * i] = hex[b >> 4];
      out.identity[2 * i + 1] = hex[b & 15];
    }
  }
  std::strncpy(out.architecture, p.gcnArchName, sizeof(out.architecture) - 1);
  // The product name when the driver reports one, else the ISA name.
  const std::string arch(p.gcnArchName);
  const std::string name = p.name[0] ? std::string(p.name) : "AMD GPU " + arch.substr(0, arch.find(':'));
  std::strncpy(out.name, name.c_str(), sizeof(out.name) - 1);
  HIP_CHECK(hipRuntimeGetVersion(&out.runtime_version));
  HIP_CHECK(hipDriverGetVersion(&out.driver_version));
  out.compute_units = (uint32_t)p.multiProcessorCount;
  int current = 0;
  HIP_CHECK(hipGetDevice(&current));
  HIP_CHECK(hipSetDevice(device));
  size_t free_b = 0, total_b = 0;
  const hipError_t e = hipMemGetInfo(&free_b, &total_b);
  (void)hipSetDevice(current);
  check_hip(e, "memory info");
  out.available_bytes = free_b;
  out.total_bytes = total_b;
  return out;
}

// Best of five timed streaming reads of `bytes` (after a warm one), in GB/s.
double measure_read_bandwidth(int32_t device, uint64_t bytes) {
  if (bytes < (1u << 20) || bytes % 16 || bytes > (64ull << 30)) fail(HLLM_INVALID_REQUEST, "read probe size");
  HIP_CHECK(hipSetDevice(device));
  DeviceMemory buf, out;
  buf.allocate(bytes, "read probe");
  out.allocate(sizeof(float), "read probe");
  hipStream_t s = nullptr;
  HIP_CHECK(hipStreamCreate(&s));
  hipEvent_t e0 = nullptr, e1 = nullptr;
  double best = 0.0;
  try {
    HIP_CHECK(hipEventCreate(&e0));
    HIP_CHECK(hipEventCreate(&e1));
    HIP_CHECK(hipMemsetAsync(buf.ptr, 0, bytes, s));
    launch_read_probe(s, buf.ptr, bytes, out.as<float>());
    for (int i = 0; i < 5; ++i) {
      HIP_CHECK(hipEventRecord(e0, s));
      launch_read_probe(s, buf.ptr, bytes, out.as<float>());
      HIP_CHECK(hipEventRecord(e1, s));
      HIP_CHECK(hipEventSynchronize(e1));
      float ms = 0.f;
      HIP_CHECK(hipEventElapsedTime(&ms, e0, e1));
      best = std::max(best, bytes / (ms * 1e-3) / 1e9);
    }
  } catch (...) {
    if (e0) (void)hipEventDestroy(e0);
    if (e1) (void)hipEventDestroy(e1);
    (void)hipStreamDestroy(s);
    throw;
  }
  (void)hipEventDestroy(e0);
  (void)hipEventDestroy(e1);
  (void)hipStreamDestroy(s);
  return best;
}

// Best of five timed launches of the MFMA probe over every CU (eight workgroups of four
// waves per CU, eight independent accumulation chains per wave), in TFLOP/s.
double measure_mfma_rate(int32_t device, uint32_t shape) {
  if (shape != 16 && shape != 32) fail(HLLM_INVALID_REQUEST, "MFMA probe shape must be 16 or 32");
  HIP_CHECK(hipSetDevice(device));
  int cus = 256;
  HIP_CHECK(hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, device));
  DeviceMemory out;
  out.allocate(sizeof(float), "MFMA probe");
  hipStream_t s = nullptr;
  HIP_CHECK(hipStreamCreate(&s));
  hipEvent_t e0 = nullptr, e1 = nullptr;
  double best = 0.0;
  try {
    HIP_CHECK(hipEventCreate(&e0));
    HIP_CHECK(hipEventCreate(&e1));
    const int blocks = 8 * cus, iters = 2048;
    launch_mfma_probe(s, (int)shape, blocks, iters / 8, out.as<float>());
    for (int i = 0; i < 5; ++i) {
      HIP_CHECK(hipEventRecord(e0, s));
      const double flops = launch_mfma_probe(s, (int)shape, blocks, iters, out.as<float>());
      HIP_CHECK(hipEventRecord(e1, s));
      HIP_CHECK(hipEventSynchronize(e1));
      float ms = 0.f;
      HIP_CHECK(hipEventElapsedTime(&ms, e0, e1));
      best = std::max(best, flops / (ms * 1e-3) / 1e12);
    }
  } catch (...) {
    if (e0) (void)hipEventDestroy(e0);
    if (e1) (void)hipEventDestroy(e1);
    (void)hipStreamDestroy(s);
    throw;
  }
  (void)hipEventDestroy(e0);
  (void)hipEventDestroy(e1);
  (void)hipStreamDestroy(s);
  return best;
}

void sample_logits(int32_t device, const float* logits, uint64_t rows, uint64_t V, const hllm_rocm_item* options,
                   uint64_t* tokens, double* logprobs, uint64_t* top_ids, double* top_logprobs) {
  if (!logits || !options || !tokens || rows == 0 || V == 0) fail(HLLM_INVALID_REQUEST, "invalid sampling request");
  if (V > (1ull << 23) || rows > (1ull << 20)) fail(HLLM_RESOURCE_EXHAUSTED, "sampling request too large");
  std::vector<SampleParams> params(rows);
  for (uint64_t r = 0; r < rows; ++r) {
    const hllm_rocm_item& it = options[r];
    check_sampling(it);
    const bool lp = (it.flags & HLLM_ITEM_LOGPROBS) != 0;
    params[r] = {it.temperature, it.top_p, it.top_k, it.seed, it.generated_index, lp ? it.top_logprobs : 0u,
                 lp ? kSampleLogprobs : 0u};
  }
  HIP_CHECK(hipSetDevice(device));
  struct Stream {
    hipStream_t s = nullptr;
    ~Stream() {
      if (s) (void)hipStreamDestroy(s);
    }
  } st;
  HIP_CHECK(hipStreamCreate(&st.s));
  const int blocks = (int)std::min<uint64_t>(rows, kSampleBlocks);
  DeviceMemory d_logits, d_rows, d_tokens, d_flags, d_val, d_idx, d_params, d_out, d_w, d_lists, d_buckets, d_hist,
      d_lse, d_sorted, d_cursor, d_candidates;
  int cus = 256;
  HIP_CHECK(hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, device));
  const int chunks = std::max(1, std::min(32, 4 * cus / blocks));
  d_logits.allocate(rows * V * sizeof(float), "logits");
  d_rows.allocate(sizeof(int32_t), "sampling");
  d_tokens.allocate(rows * sizeof(int32_t), "sampling");
  d_flags.allocate(sizeof(int32_t), "sampling");
  d_val.allocate(rows * kArgmaxParts * sizeof(float), "argmax");
  d_idx.allocate(rows * kArgmaxParts * sizeof(int32_t), "argmax");
  d_params.allocate(rows * sizeof(SampleParams), "sampling");
  d_out.allocate(rows * (6 * sizeof(double) + 5 * sizeof(int32_t)), "sampling");
  d_w.allocate((size_t)blocks * V * sizeof(double), "sampling workspace");
  d_lists.allocate((size_t)blocks * 4 * V * sizeof(uint32_t), "sampling workspace");
  d_buckets.allocate((size_t)blocks * sample_bucket_stride(V), "sampling workspace");
  d_hist.allocate((size_t)blocks * 256 * 3 * sizeof(uint64_t), "sampling workspace");
  d_lse.allocate((size_t)blocks * chunks * sizeof(double), "sampling workspace");
  d_sorted.allocate((size_t)blocks * V * sizeof(uint32_t), "sampling workspace");
  d_cursor.allocate((size_t)blocks * 256 * sizeof(uint32_t), "sampling workspace");
  d_candidates.allocate((size_t)blocks * chunks * 8 * sizeof(uint32_t), "sampling workspace");
  HIP_CHECK(hipMemsetAsync(d_hist.ptr, 0, d_hist.bytes, st.s));
  HIP_CHECK(hipMemsetAsync(d_cursor.ptr, 0, d_cursor.bytes, st.s));
  const int32_t count = (int32_t)rows;
  HIP_CHECK(hipMemcpyAsync(d_logits.ptr, logits, d_logits.bytes, hipMemcpyHostToDevice, st.s));
  HIP_CHECK(hipMemcpyAsync(d_rows.ptr, &count, sizeof(count), hipMemcpyHostToDevice, st.s));
  HIP_CHECK(hipMemcpyAsync(d_params.ptr, params.data(), d_params.bytes, hipMemcpyHostToDevice, st.s));
  HIP_CHECK(hipMemsetAsync(d_flags.ptr, 0, sizeof(int32_t), st.s));
  launch_argmax(st.s, d_logits.as<float>(), d_rows.as<int32_t>(), (int)rows, (int)V, d_val.as<float>(),
                d_idx.as<int32_t>(), kArgmaxParts, d_tokens.as<int32_t>(), d_flags.as<int32_t>());
  SampleArgs sa{};
  sa.logits = d_logits.as<float>();
  sa.vocab = (int)V;
  sa.rows = (int)rows;
  sa.params = d_params.as<SampleParams>();
  sa.tokens = d_tokens.as<int32_t>();
  sa.logprob = d_out.as<double>();
  sa.top_values = sa.logprob + rows;
  sa.top_ids = reinterpret_cast<int32_t*>(sa.top_values + 5 * rows);
  sa.weights = d_w.as<double>();
  sa.buckets = d_buckets.as<uint8_t>();
  sa.bucket_stride = sample_bucket_stride(V);
  sa.lists = d_lists.as<uint32_t>();
  sa.hist = d_hist.as<uint64_t>();
  sa.lse_parts = d_lse.as<double>();
  sa.sorted = d_sorted.as<uint32_t>();
  sa.cursor = d_cursor.as<uint32_t>();
  sa.candidates = d_candidates.as<uint32_t>();
  sa.group_rows = blocks;
  sa.chunks = chunks;
  launch_sample(st.s, sa);
  HIP_CHECK(hipGetLastError());
  std::vector<int32_t> t(rows);
  std::vector<unsigned char> out(d_out.bytes);
  int32_t flags = 0;
  HIP_CHECK(hipMemcpyAsync(t.data(), d_tokens.ptr, rows * sizeof(int32_t), hipMemcpyDeviceToHost, st.s));
  HIP_CHECK(hipMemcpyAsync(out.data(), d_out.ptr, out.size(), hipMemcpyDeviceToHost, st.s));
  HIP_CHECK(hipMemcpyAsync(&flags, d_flags.ptr, sizeof(int32_t), hipMemcpyDeviceToHost, st.s));
  HIP_CHECK(hipStreamSynchronize(st.s));
  if (flags & 2) fail(HLLM_INTERNAL, "cannot sample nonfinite logits");
  const double* lp = reinterpret_cast<const double*>(out.data());
  const double* tv = lp + rows;
  const int32_t* ti = reinterpret_cast<const int32_t*>(tv + 5 * rows);
  for (uint64_t r = 0; r < rows; ++r) {
    tokens[r] = (uint64_t)t[r];
    if (!(params[r].flags & kSampleLogprobs)) continue;
    const uint64_t n = std::min<uint64_t>(params[r].top_logprobs, V);
    if (logprobs) logprobs[r] = lp[r];
    for (uint64_t k = 0; k < 5; ++k) {
      if (top_ids) top_ids[r * 5 + k] = k < n ? (uint64_t)ti[r * 5 + k] : UINT64_MAX;
      if (top_logprobs) top_logprobs[r * 5 + k] = k < n ? tv[r * 5 + k] : std::nan("");
    }
  }
}

}  // namespace hllm_rocm

// ========================================================================= C ABI

using hllm_rocm::Failure;
using hllm_rocm::Stage;

struct hllm_rocm_stage {
  std::unique_ptr<Stage> impl;
};

namespace {
template <typename F>
hllm_status guarded(F&& f) {
  try {
    f();
    return HLLM_OK;
  } catch (const Failure& e) {
    hllm_rocm::g_last_error = e.what();
    return e.status;
  } catch (const std::bad_alloc&) {
    hllm_rocm::g_last_error = "host allocation failed";
    return HLLM_RESOURCE_EXHAUSTED;
  } catch (const std::exception& e) {
    hllm_rocm::g_last_error = e.what();
    return HLLM_INTERNAL;
  } catch (...) {
    hllm_rocm::g_last_error = "unknown failure";
    return HLLM_INTERNAL;
  }
}
Stage& impl(hllm_rocm_stage* s) {
  if (!s || !s->impl) hllm_rocm::fail(HLLM_INVALID_REQUEST, "null stage");
  return *s->impl;
}
const Stage& impl(const hllm_rocm_stage* s) {
  if (!s || !s->impl) hllm_rocm::fail(HLLM_INVALID_REQUEST, "null stage");
  return *s->impl;
}
}  // namespace

extern "C" {

const char* hllm_rocm_last_error(void) { return hllm_rocm::g_last_error.c_str(); }
uint32_t hllm_rocm_abi_version(void) { return HLLM_ROCM_ABI_VERSION; }

hllm_status hllm_rocm_stage_create(const hllm_rocm_stage_config* config, hllm_rocm_stage** out) {
  return guarded([&] {
    if (!config || !out) hllm_rocm::fail(HLLM_INVALID_REQUEST, "null argument");
    *out = nullptr;
    auto s = std::make_unique<hllm_rocm_stage>();
    s->impl = std::make_unique<Stage>(*config);
    *out = s.release();
  });
}

void hllm_rocm_stage_destroy(hllm_rocm_stage* stage) { delete stage; }

hllm_status hllm_rocm_stage_load_tensor(hllm_rocm_stage* stage, const char* name, uint32_t dtype,
                                        const uint64_t* shape, uint32_t rank, const void* data, uint64_t bytes) {
  return guarded([&] {
    if (!name || (!shape && rank)) hllm_rocm::fail(HLLM_INVALID_REQUEST, "null argument");
    impl(stage).load_tensor(name, dtype, shape, rank, data, bytes);
  });
}

hllm_status hllm_rocm_stage_synthesize_tensor(hllm_rocm_stage* stage, const char* name, uint64_t seed,
                                              uint64_t tensor_id, float mean, float sigma, uint32_t source_dtype) {
  return guarded([&] {
    if (!name) hllm_rocm::fail(HLLM_INVALID_REQUEST, "null argument");
    impl(stage).synthesize(name, seed, tensor_id, mean, sigma, source_dtype);
  });
}

hllm_status hllm_rocm_stage_finalize(hllm_rocm_stage* stage) {
  return guarded([&] { impl(stage).finalize(); });
}

hllm_status hllm_rocm_stage_weight_memory(const hllm_rocm_stage* stage, hllm_rocm_memory* out) {
  return guarded([&] {
    if (!out) hllm_rocm::fail(HLLM_INVALID_REQUEST, "null argument");
    *out = impl(stage).weight_memory();
  });
}

hllm_status hllm_rocm_stage_sequence_memory(const hllm_rocm_stage* stage, uint64_t tokens,
                                            uint64_t maximum_query_tokens, hllm_rocm_memory* cache,
                                            hllm_rocm_memory* workspace) {
  return guarded([&] { impl(stage).sequence_memory(tokens, maximum_query_tokens, cache, workspace); });
}

hllm_status hllm_rocm_sequence_allocate(hllm_rocm_stage* stage, uint64_t tokens, uint32_t* sequence) {
  return guarded([&] {
    if (!sequence) hllm_rocm::fail(HLLM_INVALID_REQUEST, "null argument");
    *sequence = impl(stage).allocate_sequence(tokens);
  });
}

hllm_status hllm_rocm_sequence_release(hllm_rocm_stage* stage, uint32_t sequence) {
  return guarded([&] { impl(stage).release_sequence(sequence); });
}

hllm_status hllm_rocm_sequence_length(const hllm_rocm_stage* stage, uint32_t sequence, uint64_t* length) {
  return guarded([&] {
    if (!length) hllm_rocm::fail(HLLM_INVALID_REQUEST, "null argument");
    *length = impl(stage).sequence_length(sequence);
  });
}

hllm_status hllm_rocm_stage_submit(hllm_rocm_stage* stage, const hllm_rocm_pass* pass) {
  return guarded([&] {
    if (!pass) hllm_rocm::fail(HLLM_INVALID_REQUEST, "null argument");
    impl(stage).submit(*pass);
  });
}

hllm_status hllm_rocm_stage_wait(hllm_rocm_stage* stage) {
  return guarded([&] { impl(stage).wait(); });
}

hllm_status hllm_rocm_stage_execute(hllm_rocm_stage* stage, const hllm_rocm_pass* pass) {
  const hllm_status s = hllm_rocm_stage_submit(stage, pass);
  if (s != HLLM_OK) return s;
  return hllm_rocm_stage_wait(stage);
}

hllm_status hllm_rocm_stage_execute_profiled(hllm_rocm_stage* stage, const hllm_rocm_pass* pass,
                                             hllm_rocm_phase_time* phases, uint32_t capacity, uint32_t* count) {
  const hllm_status s = guarded([&] {
    if (!pass || !count || (capacity && !phases)) hllm_rocm::fail(HLLM_INVALID_REQUEST, "null argument");
    impl(stage).submit(*pass, true);
  });
  if (s != HLLM_OK) return s;
  return guarded([&] { impl(stage).wait(phases, capacity, count); });
}

hllm_status hllm_rocm_sample_logits(int32_t device, const float* logits, uint64_t rows, uint64_t vocabulary,
                                    const hllm_rocm_item* options, uint64_t* tokens, double* logprobs,
                                    uint64_t* top_ids, double* top_logprobs) {
  return guarded([&] {
    hllm_rocm::sample_logits(device, logits, rows, vocabulary, options, tokens, logprobs, top_ids, top_logprobs);
  });
}

hllm_status hllm_rocm_sample_logits_noalloc(int32_t device, const float* logits, uint64_t rows, uint64_t vocabulary,
                                            const hllm_rocm_item* options, uint64_t* tokens, double* logprobs,
                                            uint64_t* top_ids, double* top_logprobs) {
  return guarded([&] {
    hllm_rocm::sample_logits_noalloc(device, logits, rows, vocabulary, options, tokens, logprobs, top_ids,
                                     top_logprobs);
  });
}

hllm_status hllm_rocm_stage_set_graphs(hllm_rocm_stage* stage, uint32_t enabled) {
  return guarded([&] { impl(stage).set_graphs(enabled != 0); });
}

hllm_status hllm_rocm_stage_graph_stats(hllm_rocm_stage* stage, uint64_t* captured, uint64_t* replayed) {
  return guarded([&] { impl(stage).graph_stats(captured, replayed); });
}

hllm_status hllm_rocm_device_allocator_metrics(int32_t device, hllm_rocm_allocator_metrics* out) {
  return guarded([&] {
    if (!out) hllm_rocm::fail(HLLM_INVALID_REQUEST, "null output");
    *out = hllm_rocm::allocator_metrics(device);
  });
}

hllm_status hllm_rocm_device_reset_peak(int32_t device) {
  return guarded([&] { hllm_rocm::reset_peak(device); });
}

hllm_status hllm_rocm_device_query(int32_t device, hllm_rocm_device_info* out) {
  return guarded([&] {
    if (!out) hllm_rocm::fail(HLLM_INVALID_REQUEST, "null output");
    *out = hllm_rocm::device_info(device);
  });
}

hllm_status hllm_rocm_measure_mfma_rate(int32_t device, uint32_t shape, double* tflops) {
  return guarded([&] {
    if (!tflops) hllm_rocm::fail(HLLM_INVALID_REQUEST, "null output");
    *tflops = hllm_rocm::measure_mfma_rate(device, shape);
  });
}

hllm_status hllm_rocm_measure_read_bandwidth(int32_t device, uint64_t bytes, double* gb_s) {
  return guarded([&] {
    if (!gb_s) hllm_rocm::fail(HLLM_INVALID_REQUEST, "null output");
    *gb_s = hllm_rocm::measure_read_bandwidth(device, bytes);
  });
}

hllm_status hllm_rocm_set_gemm_config(int32_t config, int32_t* previous) {
  return guarded([&] {
    if (config < -1 || config > hllm_rocm::kGemmConfigs)
      hllm_rocm::fail(HLLM_INVALID_REQUEST, "GEMM configuration out of range");
    const int old = hllm_rocm::set_forced_gemm_config(config);
    if (previous) *previous = old;
  });
}

hllm_status hllm_rocm_stage_last_layout(hllm_rocm_stage* stage, uint32_t items, uint32_t rows,
                                        int32_t* cu_seqlens, int32_t* row_positions, int32_t* row_slots) {
  return guarded([&] { impl(stage).last_layout(items, rows, cu_seqlens, row_positions, row_slots); });
}

hllm_status hllm_rocm_sequence_blocks(hllm_rocm_stage* stage, uint32_t sequence, int32_t* blocks,
                                      uint32_t capacity, uint32_t* count, uint32_t* block_tokens) {
  return guarded([&] { impl(stage).sequence_blocks(sequence, blocks, capacity, count, block_tokens); });
}

hllm_status hllm_rocm_stage_read_tensor(hllm_rocm_stage* stage, const char* name, float* out, uint64_t elements) {
  return guarded([&] {
    if (!name || !out) hllm_rocm::fail(HLLM_INVALID_REQUEST, "null argument");
    impl(stage).read_tensor(name, out, elements);
  });
}

hllm_status hllm_rocm_sequence_read_kv(hllm_rocm_stage* stage, uint32_t sequence, uint32_t layer, float* keys,
                                       float* values) {
  return guarded([&] {
    if (!keys || !values) hllm_rocm::fail(HLLM_INVALID_REQUEST, "null argument");
    impl(stage).read_kv(sequence, layer, keys, values);
  });
}

hllm_status hllm_rocm_stage_profile(hllm_rocm_stage* stage, const char* families) {
  return guarded([&] { impl(stage).set_profiling(families ? families : ""); });
}

hllm_status hllm_rocm_stage_profile_read(hllm_rocm_stage* stage, const char* record, double* milliseconds,
                                         uint64_t* launches, uint64_t* bytes, double* flops) {
  return guarded([&] {
    if (!record || !milliseconds || !launches || !bytes || !flops)
      hllm_rocm::fail(HLLM_INVALID_REQUEST, "null argument");
    impl(stage).profile_read(record, milliseconds, launches, bytes, flops);
  });
}

hllm_status hllm_rocm_stage_profile_records(hllm_rocm_stage* stage, char* buffer, uint64_t capacity,
                                            uint64_t* needed) {
  return guarded([&] {
    if (!needed) hllm_rocm::fail(HLLM_INVALID_REQUEST, "null argument");
    const std::string names = impl(stage).profile_records();
    *needed = names.size() + 1;
    if (buffer && capacity) {
      const uint64_t n = std::min<uint64_t>(capacity - 1, names.size());
      std::memcpy(buffer, names.data(), n);
      buffer[n] = 0;
    }
  });
}

}  // extern "C"
