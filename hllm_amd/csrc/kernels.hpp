// Launchers for the stage's kernels. Every pointer is a device pointer unless named
// `host_*`; every launch goes to `stream`.
#pragma once

#include "common.hpp"

namespace hllm_rocm {

// Per-item metadata uploaded for each pass (host packs, device unpacks).
struct ItemMeta {
  uint32_t sequence;       // sequence slot (block-table row)
  uint32_t query_tokens;
  uint32_t first_position;
  uint32_t flags;          // HLLM_ITEM_*
};

// One attention work item: a block of query rows of one item against one split of the
// keys [key_begin, key_end) (times every KV head: grid y).
struct AttnWork {
  int32_t item;
  int32_t row0;       // packed row of the block's first query row
  int32_t rows;       // query rows in the block
  int32_t position0;  // position of the block's first query row
  int32_t split;      // split index of the block's key range
  int32_t splits;     // number of splits of the block's key range
  int32_t key_begin;
  int32_t key_end;
};

// Query rows per attention block: 64 query vectors (rows x query heads of one KV head),
// at least one row.
__host__ __device__ inline int attn_block_rows(int group) { return group >= 64 ? 1 : 64 / group; }

// Keys per split of prefill blocks (more than 16 query vectors).
constexpr int kAttnPrefillUnit = 1024;

// Splits of a block's `keys` key positions, 32-key aligned and non-empty: every
// `decode_unit` keys (a multiple of 32; 512 by default) for decode-like blocks (at most 16
// query vectors: the workgroup's four waves share the keys, and short splits balance rows
// of very different context lengths), every kAttnPrefillUnit keys for prefill blocks.
__host__ __device__ inline int attn_split_keys(int keys, int vectors, int max_splits, int decode_unit,
                                               int decode_split) {
  // Decode-like blocks of more than `decode_unit` keys split every `decode_split` keys.
  const int unit = vectors > 16 ? kAttnPrefillUnit : keys <= decode_unit ? decode_unit : decode_split;
  int splits = (keys + unit - 1) / unit;
  splits = splits < max_splits ? splits : max_splits;
  const int per = ((keys + splits - 1) / splits + 31) & ~31;
  return per;
}
// The work list is ordered by dispatch class: prefill blocks (more than 16 query vectors,
// each an MFMA-bound chain over its key tiles; within an item the blocks with the most keys
// first), then decode-like splits of at least half a decode unit of keys, then the rest.
// Workgroups are dispatched in list order, so the short items fill in behind the long ones.
constexpr int kAttnClasses = 3;
__host__ __device__ inline int attn_work_class(int per, int vectors, int decode_unit) {
  return vectors > 16 ? 0 : 2 * per >= decode_unit ? 1 : 2;
}
// Work items (block x key split) of one query item, per dispatch class.
__host__ __device__ inline void attn_item_work_classes(int query_tokens, int first_position, int group,
                                                       int max_splits, int decode_unit, int decode_split,
                                                       int (&count)[kAttnClasses]) {
  const int qb = attn_block_rows(group);
  for (int c = 0; c < kAttnClasses; ++c) count[c] = 0;
  for (int r0 = 0; r0 < query_tokens; r0 += qb) {
    const int rows = query_tokens - r0 < qb ? query_tokens - r0 : qb;
    const int keys = first_position + r0 + rows;
    const int per = attn_split_keys(keys, rows * group, max_splits, decode_unit, decode_split);
    count[attn_work_class(per, rows * group, decode_unit)] += (keys + per - 1) / per;
  }
}
__host__ __device__ inline int attn_item_work(int query_tokens, int first_position, int group,
                                              int max_splits, int decode_unit, int decode_split) {
  int count[kAttnClasses];
  attn_item_work_classes(query_tokens, first_position, group, max_splits, decode_unit, decode_split, count);
  return count[0] + count[1] + count[2];
}
// Whether a block of `vectors` query vectors whose keys are split merges its splits in the
// attention kernel (the last split's workgroup to arrive, decode-like blocks of at most 16
// vectors) rather than in the combine kernel.
__host__ __device__ inline bool attn_merges_in_kernel(int vectors, int fold) { return fold && vectors <= 16; }
// Whether some block of one query item leaves its splits to the combine kernel.
__host__ __device__ inline bool attn_item_needs_combine(int query_tokens, int first_position, int group,
                                                        int max_splits, int decode_unit, int decode_split,
                                                        int fold) {
  const int qb = attn_block_rows(group);
  for (int r0 = 0; r0 < query_tokens; r0 += qb) {
    const int rows = query_tokens - r0 < qb ? query_tokens - r0 : qb;
    const int keys = first_position + r0 + rows;
    const int per = attn_split_keys(keys, rows * group, max_splits, decode_unit, decode_split);
    if (per < keys && !attn_merges_in_kernel(rows * group, fold)) return true;
  }
  return false;
}

// Where each packed row of a pass comes from, built on the device from ItemMeta.
struct PackOut {
  int32_t* cu_seqlens;     // [items + 1] exclusive prefix sum of query_tokens
  int32_t* row_item;       // [rows]
  int32_t* row_position;   // [rows]
  int32_t* row_slot;       // [rows] physical KV slot: block * block_tokens + position % block_tokens
  int32_t* row_token;      // [rows] input token (first stage)
  int32_t* sample_row;     // [items] packed row of each sampling item, in item order (compacted)
  int32_t* sample_item;    // [items]
  int32_t* sample_count;   // [1]
  AttnWork* attn_work;     // attention work items (MFMA path), in item order
  int32_t* attn_count;     // [1] number of attention work items
  int32_t* row_splits;     // [rows] key splits of the row's attention block
  int32_t* flags;          // [1] the pass's error flags, cleared by the pack kernel
  int attn_group;          // query heads per KV head
  int attn_max_splits;
  int attn_decode_unit;    // decode-like blocks of at most this many keys are not split
  int attn_decode_split;   // keys per split of longer decode-like blocks (attn_split_keys)
  int attn_fold;           // decode-like blocks merge their splits in the attention kernel
};

// Paged KV pool: [layers][blocks][K, V][kv_heads][...] with keys as [block_tokens][head_dim]
// (a position's key contiguous; for the MFMA attention, 32-position tiles in operand order,
// see kv_key_index) and values transposed in 32-position sub-tiles as
// [block_tokens / 32][head_dim][32] (a dimension's values over 32 positions contiguous, and
// one 32-key attention tile's values one contiguous region): the operand layouts of the
// attention MFMAs. Blocks hold a multiple of 32 tokens.
struct KvView {
  void* pool;
  uint64_t layer_stride;   // elements per layer
  int32_t block_tokens;
  int32_t kv_heads;
  int32_t head_dim;
  int32_t f32;             // element type: 1 = F32, 0 = F16
  int32_t key_fragments;   // 1: each 32-position key tile in MFMA operand order (below)
};
// Keys of a block and head: [block_tokens][head_dim], or with key_fragments, per 32-position
// tile the A operands of v_mfma_f32_16x16x32_f16 one after another: operand (kk, h) (dims
// 32 kk .. 32 kk + 31 of rows 8 (c >> 2) + (c & 3) + 4 h, c = 0..15) is 1 KiB, lane
// 16 q + c holding dims 32 kk + 8 q .. + 7 of its row, so that one operand is one contiguous
// 1 KiB load per wave.
__host__ __device__ inline uint64_t kv_key_index(const KvView& kv, int layer, uint64_t block, int offset,
                                                 int head, int d) {
  const uint64_t head_base = (uint64_t)layer * kv.layer_stride + (block * 2 * kv.kv_heads + head) * kv.block_tokens * kv.head_dim;
  if (!kv.key_fragments) return head_base + (uint64_t)offset * kv.head_dim + d;
  const int r = offset & 31, h = (r >> 2) & 1, c = ((r >> 3) << 2) | (r & 3);
  return head_base + (uint64_t)(offset & ~31) * kv.head_dim +
         (uint64_t)((((d >> 5) * 2 + h) * 64 + ((d >> 3) & 3) * 16 + c) * 8 + (d & 7));
}
__host__ __device__ inline uint64_t kv_value_index(const KvView& kv, int layer, uint64_t block, int offset,
                                                   int head, int d) {
  return (uint64_t)layer * kv.layer_stride +
         ((block * 2 + 1) * kv.kv_heads + head) * (uint64_t)kv.block_tokens * kv.head_dim +
         ((uint64_t)(offset >> 5) * kv.head_dim + d) * 32 + (offset & 31);
}

// Streaming read of `bytes` (a multiple of 16) from p: a measured HBM read ceiling.
void launch_read_probe(hipStream_t stream, const void* p, size_t bytes, float* out);
// MFMA issue-rate probe (shape 16: 16x16x32 F16, 32: 32x32x16 F16); returns the FLOPs launched.
double launch_mfma_probe(hipStream_t stream, int shape, int blocks, int iters, float* out);
void launch_pack(hipStream_t stream, const ItemMeta* items, int n_items, const int32_t* host_tokens,
                 const int32_t* last_token, const int32_t* block_table, int table_width,
                 int block_tokens, PackOut out);

void launch_embed(hipStream_t stream, const uint16_t* table_hi, const uint16_t* table_lo,
                  uint64_t cols_padded, const int32_t* row_token, int rows, int hidden, float* h);

void launch_boundary_decode(hipStream_t stream, const uint16_t* in, int rows, int hidden, float* h);
void launch_boundary_encode(hipStream_t stream, const float* h, int rows, int hidden, uint16_t* out,
                            int32_t* flags);

// K-split partial outputs a projection left for its consumer: `parts` row-major matrices
// of the consumer's row width, `stride` floats apart, summed in order (0 = none).
struct Partials {
  const float* data = nullptr;
  int parts = 0;
  uint64_t stride = 0;
};

// y = (x * inv_rms) * w written to F-layout hi (+ lo when lo != nullptr); rows may be
// gathered through `row_index` (nullptr = identity) with `count` read from device
// memory when `device_rows` is non-null. With `residual` partials (identity rows only)
// the row is first updated in place: h += sum of the partials.
// h += the partials summed in split order from zero: the residual update the RMSNorm
// kernel makes with `residual` partials, with the same additions, for passes that read the
// residual stream between layers (traces).
void launch_residual_sum(hipStream_t stream, float* h, int rows, int hidden, Partials residual);

void launch_rmsnorm_flayout(hipStream_t stream, float* h, int hidden, const int32_t* row_index,
                            int rows, const int32_t* device_rows, const float* weight, float eps,
                            uint16_t* out_hi, uint16_t* out_lo, uint64_t cols_padded,
                            Partials residual = {});

// Per-head QK-norm (optional) + rotate-half RoPE from tables + paged KV append. `qkv` is
// [rows][(Q + 2K) * D] F32; q goes to `q_out` [rows][Q * D] F32.
// With `qkv_parts`, the projection is the sum of its K-split partials instead of `qkv`.
void launch_qkv_rope_append(hipStream_t stream, const float* qkv, int rows, int q_heads, int kv_heads,
                            int head_dim, const float* q_norm, const float* k_norm, float eps,
                            const float* rope_cos, const float* rope_sin, const int32_t* row_position,
                            const int32_t* row_slot, KvView kv, int layer, float* q_out,
                            Partials qkv_parts = {});

// Split-context GQA attention for every packed row against its sequence's paged cache
// (positions 0..row_position), then the split combine into F-layout A operands.
// Decode rows with the projection epilogue fused into attention (F16 KV, head dim 128, passes
// of single-token items): each item reads its row's q/k/v from the q/k/v projection output
// (`qkv` [rows][(Q + 2K) * D], or its K-split partials), applies QK-norm and RoPE itself, and
// the item that holds the row's own position appends the row's K/V to the cache and adds the
// row's own key to the softmax from registers. qkv == nullptr: q comes from `q`, K/V are in
// the cache already.
struct AttentionRope {
  const float* qkv = nullptr;
  Partials parts;
  const float* q_norm = nullptr;  // nullptr: no QK-norm
  const float* k_norm = nullptr;
  float eps = 0.0f;
  const float* rope_cos = nullptr;  // [positions][D / 2]
  const float* rope_sin = nullptr;
  const int32_t* row_slot = nullptr;
};

struct AttentionArgs {
  const float* q;              // [rows][Q][D]
  int rows, q_heads, kv_heads, head_dim;
  const AttnWork* work;        // MFMA path work list, its size (device) and the launch's
  const int32_t* work_count;   // workgroups along x, which loop over the list
  int work_grid;
  int any_split;               // some block's splits are left to the combine kernel
  const int32_t* row_splits;   // [rows] splits the combine kernel merges (1: none)
  int fold;                    // decode-like blocks merge their splits in the attention kernel
  int32_t* split_arrivals;     // [rows][kv_heads] arrival counts (zero between launches)
  const int32_t* row_item;
  const int32_t* row_position;
  const ItemMeta* items;
  const int32_t* block_table;
  int table_width;
  KvView kv;
  int layer;
  float scale;
  float* partial;              // [rows][Q][max_splits][D + 2]
  int max_splits;
  int split_unit;              // positions per split are a multiple of this
  uint16_t* out_hi;            // F-layout [rows][Q * D]
  uint16_t* out_lo;
  uint64_t out_cols_padded;
  AttentionRope rope;
};
void launch_attention(hipStream_t stream, const AttentionArgs& a);
// Whether launch_attention uses the MFMA kernel (and hence the pack kernel's work list).
bool attention_uses_mfma(int head_dim, bool kv_f32);

// Row-wise first maximum over `cols` F32 values per row (greedy sampling) and a
// non-finite flag (bit 1 of flags).
// The first maximum of each row over `parts` candidates [rows][parts] (launch_argmax's second
// kernel, for candidates a GEMM's argmax epilogue wrote).
void launch_argmax_final(hipStream_t stream, const int32_t* device_rows, int max_rows, int parts,
                         const float* part_val, const int32_t* part_idx, int32_t* tokens,
                         const int32_t* sample_item, const ItemMeta* items, int32_t* last_token);
// With `last_token` set, each row's token is also recorded as its sequence's last token
// (as launch_record_tokens does: sample_item maps sampled rows to items).
void launch_argmax(hipStream_t stream, const float* logits, const int32_t* device_rows, int max_rows,
                   int cols, float* part_val, int32_t* part_idx, int parts, int32_t* tokens,
                   int32_t* flags, const int32_t* sample_item = nullptr, const ItemMeta* items = nullptr,
                   int32_t* last_token = nullptr);

// Temperature / top-k / top-p sampling and log-probabilities of sampled rows whose item
// asks for either (runtime::sample_token, cpp/src/sampling.cpp:19-89); greedy rows without
// log-probabilities are left to the argmax. `tokens` holds each row's first maximum on
// entry and the sampled token on exit.
constexpr uint32_t kSampleLogprobs = 4;  // HLLM_ITEM_LOGPROBS
struct SampleParams {
  double temperature;
  double top_p;
  uint64_t top_k;
  uint64_t seed;
  uint64_t generated_index;
  uint32_t top_logprobs;
  uint32_t flags;
};
struct SampleArgs {
  const float* logits;          // [rows][vocab]
  int vocab;
  int rows;
  const SampleParams* params;   // [rows]
  int32_t* tokens;              // [rows]
  double* logprob;              // [rows]
  int32_t* top_ids;             // [rows][5]
  double* top_values;           // [rows][5]
  // Workspace for `group_rows` rows at a time (the rows are processed in groups):
  double* weights;              // [group_rows][vocab] probabilities
  uint8_t* buckets;             // [group_rows][bucket_stride] probability bucket per token
  uint64_t bucket_stride;       // a multiple of 16, >= vocab
  uint32_t* sorted;             // [group_rows][vocab] tokens grouped by bucket
  uint32_t* lists;              // [group_rows][4][vocab] token lists
  uint64_t* hist;               // [group_rows][256][3] zero between uses (the kernels clear it)
  uint32_t* cursor;             // [group_rows][256] zero between uses (the kernels clear it)
  double* lse_parts;            // [group_rows][chunks]
  uint32_t* candidates;         // [group_rows][chunks][8] log-probability candidates
  int group_rows;
  int chunks;                   // first-pass workgroups per row (at most 64)
};
// Workspace sizes for `group_rows` rows of `vocab` tokens.
inline uint64_t sample_bucket_stride(uint64_t vocab) { return (vocab + 15) / 16 * 16; }
void launch_sample(hipStream_t stream, const SampleArgs& a);

// Record sampled tokens as the sequences' last tokens (for HLLM_ITEM_TOKEN_FROM_DEVICE).
void launch_record_tokens(hipStream_t stream, const int32_t* tokens, const int32_t* sample_item,
                          const int32_t* sample_count, const ItemMeta* items, int32_t* last_token);

// Weight relayout: row-major [rows][cols] source (F32/F16/BF16 payload, or the seeded
// generator when `src == nullptr`) into F-layout hi (+ lo) at fused destination rows.
struct RelayoutArgs {
  const void* src;
  uint32_t src_dtype;          // hllm_dtype
  uint64_t seed, tensor_id;    // generator (src == nullptr)
  float mean, sigma;
  uint64_t rows, cols;         // this chunk's rows
  uint64_t row_base;           // tensor row of the chunk's first row
  uint16_t* dst_hi;
  uint16_t* dst_lo;            // nullptr unless F32 residency
  uint64_t dst_cols_padded;
  int row_mode;                // 0: dst_row = row_offset + r; 1: interleave 32-row blocks (gate); 2: (up)
  uint64_t row_offset;
  float* dst_f32;              // vectors (norm weights): F32 copy instead of F-layout
  int f16_resident;            // weights are held as F16 (vectors: rounded through F16)
  int32_t* flags;              // bit 0: non-finite source value, bit 2: not finite in F16
};
void launch_relayout(hipStream_t stream, const RelayoutArgs& a);

}  // namespace hllm_rocm
