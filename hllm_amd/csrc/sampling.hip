// Temperature / top-k / top-p sampling and log-probabilities on the device, following the
// reference sampler (cpp/src/sampling.cpp:19-89):
//   p_i = exp((l_i - max) / T) in double; candidates in descending p, equal p by lower
//   token ID; the first top_k of them; the shortest prefix whose mass reaches top_p of the
//   candidates' total; a SplitMix64 counter draw u in [0, 1) times that prefix's mass picks
//   the first candidate whose running mass exceeds it.
// Nothing is sorted by probability. A first kernel (many workgroups per row) computes
// every p_i, its bucket (its binary exponent: buckets are ordered like the probabilities)
// and each bucket's exact count and mass; a second one groups each row's tokens by bucket
// (a counting sort). A third kernel (one workgroup per row) finds from the histogram the
// bucket where each boundary (k-th candidate, top-p cut, draw) falls and the boundary
// token inside that bucket's slice by a radix descent over their rank (~bits(p) << 32 |
// id, ascending = reference order): an 8-bit digit histogram of counts and masses in LDS
// picks the digit bucket in which the running mass crosses the goal, its members are
// compacted, and the next digit below the list's highest differing bit is examined, until
// one token remains.
// Log-probabilities: the normaliser is summed per chunk and the chunks in order; the top
// tokens are chosen from each chunk's eight best by logit, re-ranked by log-probability
// (exact unless four tokens of one chunk with distinct logits round to the log-probability
// of a chosen one).
// Masses are sums of probabilities held as integers in units of 2^-80 (each probability is
// in [0, 1]; a vocabulary of up to 2^23 sums without overflow), so every sum is exact and
// independent of the order of the atomics: results are deterministic. The reference
// sums in sorted order in double; the two agree on the token except when the draw falls
// within the reference's rounding error (about 1e-16 relative per term) of a boundary.
#include "kernels.hpp"

namespace hllm_rocm {
namespace {

constexpr int kThreads = 512;
constexpr int kWaves = kThreads / 64;
constexpr int kFracBits = 40;  // a probability p is floor(p * 2^40) * 2^40 + (next 40 bits)
using u64 = unsigned long long;
using u128 = unsigned __int128;

struct Shared {
  uint32_t count[256];
  u64 hi[256], lo[256];
  u64 red[kWaves][4];
  double dred[kWaves];
  uint32_t list_n;
  int chosen;
  int never;
  u64 before_hi, before_lo;
  u64 scan_count;
};

// ---------------------------------------------------------------- exact masses

struct Fx {
  u64 hi, lo;
};
__device__ inline Fx to_fx(double x) {
  if (!(x > 0.0)) return {0, 0};
  const double s = fmin(x, 0x1p22) * 0x1p40;
  const double h = floor(s);
  return {(u64)h, (u64)floor((s - h) * 0x1p40)};
}
__device__ inline u128 fx_value(u64 hi, u64 lo) { return ((u128)hi << kFracBits) + lo; }
__device__ inline u128 fx_of(double x) {
  const Fx f = to_fx(x);
  return fx_value(f.hi, f.lo);
}
__device__ inline double fx_double(u128 v) {
  return ((double)(u64)(v >> 64) * 0x1p64 + (double)(u64)v) * 0x1p-80;
}

// ---------------------------------------------------------------- ranks

// Ascending rank = descending probability (p >= 0, so its bits order as its value).
__device__ inline u64 prob_key(double p) { return ~(u64)__double_as_longlong(p); }
__device__ inline u128 rank_of(double p, uint32_t id) { return ((u128)prob_key(p) << 32) | id; }
// Ascending key = descending value, with -0.0 equal to +0.0.
__device__ inline u64 descending_key(double x) {
  const u64 b = (u64)__double_as_longlong(x + 0.0);
  const u64 ascending = (b >> 63) ? ~b : (b | 0x8000000000000000ull);
  return ~ascending;
}

// ---------------------------------------------------------------- block reductions

__device__ inline int lane_id() { return threadIdx.x & 63; }

// Also returns the list length (sh.list_n), read between the barriers: every push before
// the call is counted, and a reset after the call cannot race the read.
__device__ inline uint32_t block_and_or(u128& a, u128& o, Shared& sh) {
  u64 v[4] = {(u64)a, (u64)(a >> 64), (u64)o, (u64)(o >> 64)};
#pragma unroll
  for (int m = 32; m > 0; m >>= 1) {
    v[0] &= __shfl_xor(v[0], m, 64);
    v[1] &= __shfl_xor(v[1], m, 64);
    v[2] |= __shfl_xor(v[2], m, 64);
    v[3] |= __shfl_xor(v[3], m, 64);
  }
  if (lane_id() == 0) {
#pragma unroll
    for (int k = 0; k < 4; ++k) sh.red[threadIdx.x >> 6][k] = v[k];
  }
  __syncthreads();
  u64 r[4] = {~0ull, ~0ull, 0ull, 0ull};
  for (int w = 0; w < kWaves; ++w) {
    r[0] &= sh.red[w][0];
    r[1] &= sh.red[w][1];
    r[2] |= sh.red[w][2];
    r[3] |= sh.red[w][3];
  }
  const uint32_t listed = sh.list_n;
  __syncthreads();
  a = ((u128)r[1] << 64) | r[0];
  o = ((u128)r[3] << 64) | r[2];
  return listed;
}

// Exact integer sums.
__device__ inline void block_sum2(u64& x, u64& y, Shared& sh) {
#pragma unroll
  for (int m = 32; m > 0; m >>= 1) {
    x += __shfl_xor(x, m, 64);
    y += __shfl_xor(y, m, 64);
  }
  if (lane_id() == 0) {
    sh.red[threadIdx.x >> 6][0] = x;
    sh.red[threadIdx.x >> 6][1] = y;
  }
  __syncthreads();
  x = 0;
  y = 0;
  for (int w = 0; w < kWaves; ++w) {
    x += sh.red[w][0];
    y += sh.red[w][1];
  }
  __syncthreads();
}

// Append `e` to `out` when `keep` (one LDS atomic per wave; list order is arbitrary).
__device__ inline void push(bool keep, uint32_t e, uint32_t* out, uint32_t* counter) {
  const u64 m = __ballot(keep);
  if (m == 0) return;
  const int leader = __builtin_ctzll(m);
  uint32_t base = 0;
  if (lane_id() == leader) base = atomicAdd(counter, (uint32_t)__popcll(m));
  base = __shfl(base, leader, 64);
  if (keep) out[base + __builtin_amdgcn_mbcnt_hi((uint32_t)(m >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)m, 0))] = e;
}

// ---------------------------------------------------------------- list traversal

// Visits the tokens of a list (nullptr: the identity list 0..n-1) kB per thread at a time,
// with every load of a batch (list entries, then their probabilities) issued before any
// is used: the traversals are latency-bound. f(token, probability) runs for each in order.
constexpr int kB = 4;
template <typename F>
__device__ inline void for_each_token(const uint32_t* list, uint32_t n, const double* w, F&& f) {
  for (uint32_t j0 = threadIdx.x; j0 < n; j0 += kThreads * kB) {
    uint32_t e[kB];
    double p[kB];
#pragma unroll
    for (int u = 0; u < kB; ++u) {
      const uint32_t j = min(j0 + (uint32_t)u * kThreads, n - 1);
      e[u] = list ? list[j] : j;
    }
#pragma unroll
    for (int u = 0; u < kB; ++u) p[u] = w[e[u]];
#pragma unroll
    for (int u = 0; u < kB; ++u)
      if (j0 + (uint32_t)u * kThreads < n) f(e[u], p[u]);
  }
}

// ---------------------------------------------------------------- radix descent

// Wave 0: the digit bucket in which `before` + the running mass first reaches `goal`
// (>= goal, or > goal when `strict`); when none does (or `never`), the last non-empty
// bucket. Writes the bucket and the mass (or count) of the buckets before it, and empties
// the output list for the compaction that follows.
template <bool kWeighted>
__device__ void choose_bucket(Shared& sh, u128 before, u128 goal, bool strict, bool never) {
  const int lane = threadIdx.x;
  if (lane == 0) sh.list_n = 0;
  uint32_t c[4];
  u64 h[4], l[4];
  u64 lh = 0, ll = 0;
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    const int d = lane * 4 + k;
    c[k] = sh.count[d];
    h[k] = kWeighted ? sh.hi[d] : 0ull;
    l[k] = kWeighted ? sh.lo[d] : (u64)c[k];
    lh += h[k];
    ll += l[k];
  }
  u64 eh = lh, el = ll;  // inclusive scan over lanes, then exclusive
#pragma unroll
  for (int off = 1; off < 64; off <<= 1) {
    const u64 th = __shfl_up(eh, off, 64), tl = __shfl_up(el, off, 64);
    if (lane >= off) {
      eh += th;
      el += tl;
    }
  }
  eh -= lh;
  el -= ll;
  int hit = -1, last = -1;
  u64 hit_h = 0, hit_l = 0, last_h = 0, last_l = 0;
  u64 rh = eh, rl = el;
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    const u128 incl = before + fx_value(rh + h[k], rl + l[k]);
    if (c[k] > 0) {
      last = k;
      last_h = rh;
      last_l = rl;
      if (hit < 0 && !never && (strict ? incl > goal : incl >= goal)) {
        hit = k;
        hit_h = rh;
        hit_l = rl;
      }
    }
    rh += h[k];
    rl += l[k];
  }
  const u64 hits = __ballot(hit >= 0);
  if (hits) {
    if (lane == __builtin_ctzll(hits)) {
      sh.chosen = lane * 4 + hit;
      sh.before_hi = hit_h;
      sh.before_lo = hit_l;
      sh.never = 0;
    }
    return;
  }
  const u64 any = __ballot(last >= 0);
  const int owner = any ? 63 - __builtin_clzll(any) : 0;
  if (lane == owner) {
    sh.chosen = last >= 0 ? lane * 4 + last : -1;
    sh.before_hi = last_h;
    sh.before_lo = last_l;
    sh.never = 1;
  }
}

struct Found {
  int id;        // -1: the list was empty
  u128 running;  // mass (or count) of the candidates up to and including it
};

// The candidate of `in` (nullptr: the identity list 0..n-1) at which the running mass
// (kWeighted) or count, taken in rank order, first reaches `goal` (>= goal, or > goal when
// `strict`); the last candidate when it never does. c_and / c_or: AND and OR of the
// candidates' ranks. buf_a / buf_b: two lists of n entries, neither of them `in`.
template <bool kWeighted>
__device__ Found descend(const uint32_t* in, uint32_t n, u128 c_and, u128 c_or, const double* w, u128 goal,
                         bool strict, uint32_t* buf_a, uint32_t* buf_b, Shared& sh) {
  u128 before = 0;
  bool never = false;
  const uint32_t* cur = in;
  uint32_t* out = buf_a;
  uint32_t* spare = buf_b;
  // Each pass fixes at least eight more of the 96 rank bits.
  for (int pass = 0; pass < 13 && n > 1; ++pass) {
    const u128 diff = c_and ^ c_or;
    const u64 dh = (u64)(diff >> 64), dl = (u64)diff;
    const int top = dh ? 127 - __builtin_clzll(dh) : (dl ? 63 - __builtin_clzll(dl) : 0);
    const int shift = top > 7 ? top - 7 : 0;
    for (int d = threadIdx.x; d < 256; d += kThreads) {
      sh.count[d] = 0;
      sh.hi[d] = 0;
      sh.lo[d] = 0;
    }
    __syncthreads();
    for_each_token(cur, n, w, [&](uint32_t e, double p) {
      const int d = (int)((uint32_t)(rank_of(p, e) >> shift) & 255u);
      atomicAdd(&sh.count[d], 1u);
      if (kWeighted) {
        const Fx f = to_fx(p);
        atomicAdd(&sh.hi[d], f.hi);
        atomicAdd(&sh.lo[d], f.lo);
      }
    });
    __syncthreads();
    if (threadIdx.x < 64) choose_bucket<kWeighted>(sh, before, goal, strict, never);
    __syncthreads();
    const int chosen = sh.chosen;
    before += fx_value(sh.before_hi, sh.before_lo);
    never = sh.never != 0;
    u128 a = ~(u128)0, o = 0;
    // Wave-uniform trip counts keep every lane at the ballots of push().
    for (uint32_t j0 = threadIdx.x & ~63u; j0 < n; j0 += kThreads * kB) {
      uint32_t e[kB];
      double p[kB];
#pragma unroll
      for (int u = 0; u < kB; ++u) {
        const uint32_t j = min(j0 + lane_id() + (uint32_t)u * kThreads, n - 1);
        e[u] = cur ? cur[j] : j;
      }
#pragma unroll
      for (int u = 0; u < kB; ++u) p[u] = w[e[u]];
#pragma unroll
      for (int u = 0; u < kB; ++u) {
        const u128 r = rank_of(p[u], e[u]);
        const bool keep = j0 + lane_id() + (uint32_t)u * kThreads < n && (int)((uint32_t)(r >> shift) & 255u) == chosen;
        push(keep, e[u], out, &sh.list_n);
        if (keep) {
          a &= r;
          o |= r;
        }
      }
    }
    n = block_and_or(a, o, sh);  // its barriers also publish the list
    c_and = a;
    c_or = o;
    cur = out;
    uint32_t* t = out;
    out = spare;
    spare = t;
  }
  Found f{-1, before};
  if (n >= 1) {
    f.id = (int)(cur ? cur[0] : 0u);
    f.running = before + (kWeighted ? fx_of(w[f.id]) : (u128)1);
  }
  return f;
}

// The candidates of `in` (nullptr: 0..n-1) ranked at or before `limit`, into `out`; returns
// their number, and the AND / OR of their ranks and their exact mass.
__device__ uint32_t compact_upto(const uint32_t* in, uint32_t n, const double* w, u128 limit, uint32_t* out,
                                 u128& c_and, u128& c_or, u128& mass, Shared& sh) {
  if (threadIdx.x == 0) sh.list_n = 0;
  __syncthreads();
  u128 a = ~(u128)0, o = 0;
  u64 hi = 0, lo = 0;
  for (uint32_t j0 = threadIdx.x & ~63u; j0 < n; j0 += kThreads * kB) {
    uint32_t e[kB];
    double p[kB];
#pragma unroll
    for (int u = 0; u < kB; ++u) {
      const uint32_t j = min(j0 + lane_id() + (uint32_t)u * kThreads, n - 1);
      e[u] = in ? in[j] : j;
    }
#pragma unroll
    for (int u = 0; u < kB; ++u) p[u] = w[e[u]];
#pragma unroll
    for (int u = 0; u < kB; ++u) {
      const u128 r = rank_of(p[u], e[u]);
      const bool keep = j0 + lane_id() + (uint32_t)u * kThreads < n && r <= limit;
      push(keep, e[u], out, &sh.list_n);
      if (keep) {
        a &= r;
        o |= r;
        const Fx f = to_fx(p[u]);
        hi += f.hi;
        lo += f.lo;
      }
    }
  }
  const uint32_t listed = block_and_or(a, o, sh);
  block_sum2(hi, lo, sh);
  c_and = a;
  c_or = o;
  mass = fx_value(hi, lo);
  return listed;
}

__device__ inline u64 counter_bits(u64 seed, u64 index) {
  u64 z = seed + 0x9e3779b97f4a7c15ull * (index + 1);
  z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ull;
  z = (z ^ (z >> 27)) * 0x94d049bb133111ebull;
  return z ^ (z >> 31);
}

__device__ inline bool rank_less(u64 ka, uint32_t ia, u64 kb, uint32_t ib) { return ka < kb || (ka == kb && ia < ib); }

// ---------------------------------------------------------------- probability buckets

// Bucket of a probability: 1023 - its binary exponent, so ascending buckets hold
// descending probabilities (every probability of bucket b exceeds every one of bucket
// b + 1); probabilities below 2^-254, and zero, share the last bucket.
constexpr int kBuckets = 256;
constexpr int kCandidates = 8;  // log-probability candidates kept per chunk
__device__ inline int bucket_of(double p) {
  const int e = (int)(((u64)__double_as_longlong(p) >> 52) & 0x7ff);
  const int b = 1023 - e;
  return b < 0 ? 0 : (b > kBuckets - 1 ? kBuckets - 1 : b);
}

// Per-thread list of the kCandidates best (key, id) pairs seen, ascending.
struct Best8 {
  u64 k[kCandidates];
  uint32_t i[kCandidates];
  __device__ void clear() {
#pragma unroll
    for (int q = 0; q < kCandidates; ++q) {
      k[q] = ~0ull;
      i[q] = ~0u;
    }
  }
  __device__ void offer(u64 key, uint32_t id) {
    if (!rank_less(key, id, k[kCandidates - 1], i[kCandidates - 1])) return;
#pragma unroll
    for (int q = kCandidates - 1; q > 0; --q) {
      const bool below = rank_less(key, id, k[q - 1], i[q - 1]);
      const bool here = !below && rank_less(key, id, k[q], i[q]);
      k[q] = below ? k[q - 1] : here ? key : k[q];
      i[q] = below ? i[q - 1] : here ? id : i[q];
    }
    if (rank_less(key, id, k[0], i[0])) {
      k[0] = key;
      i[0] = id;
    }
  }
  __device__ void pop() {
#pragma unroll
    for (int q = 0; q < kCandidates - 1; ++q) {
      k[q] = k[q + 1];
      i[q] = i[q + 1];
    }
    k[kCandidates - 1] = ~0ull;
    i[kCandidates - 1] = ~0u;
  }
};

// The block-wide smallest (key, id) of the threads' offers (scratch: two u64 per wave).
template <int kWavesInBlock>
__device__ inline void block_min_pair(u64& key, uint32_t& id, u64 (*scratch)[4]) {
#pragma unroll
  for (int m = 32; m > 0; m >>= 1) {
    const u64 ok = __shfl_xor(key, m, 64);
    const uint32_t oi = __shfl_xor(id, m, 64);
    if (rank_less(ok, oi, key, id)) {
      key = ok;
      id = oi;
    }
  }
  if (lane_id() == 0) {
    scratch[threadIdx.x >> 6][0] = key;
    scratch[threadIdx.x >> 6][1] = id;
  }
  __syncthreads();
  u64 bk = ~0ull;
  uint32_t bi = ~0u;
  for (int wv = 0; wv < kWavesInBlock; ++wv) {
    if (rank_less(scratch[wv][0], (uint32_t)scratch[wv][1], bk, bi)) {
      bk = scratch[wv][0];
      bi = (uint32_t)scratch[wv][1];
    }
  }
  __syncthreads();
  key = bk;
  id = bi;
}

// First pass, one chunk of one row's vocabulary per workgroup (grid: chunks x rows): the
// probabilities (kept for the later passes), each token's bucket, and the exact count and
// mass of every bucket, added to the row's histogram with integer atomics (so the sums do
// not depend on their order); for log-probabilities, the chunk's share of the normaliser
// and its kCandidates best tokens by (logit - max) descending, ID ascending.
constexpr int kPassThreads = 256;
constexpr int kPassWaves = kPassThreads / 64;
__global__ void __launch_bounds__(kPassThreads) sample_histogram_kernel(SampleArgs a, int row0) {
  __shared__ uint32_t cnt[kBuckets];
  __shared__ u64 hi[kBuckets], lo[kBuckets];
  __shared__ double dred[kPassWaves];
  __shared__ u64 pred[kPassWaves][4];
  const int r = blockIdx.y, s = row0 + r;
  if (s >= a.rows) return;
  const SampleParams p = a.params[s];
  const bool sampled = p.temperature > 0.0, logprobs = (p.flags & kSampleLogprobs) != 0;
  if (!sampled && !logprobs) return;
  const uint32_t V = (uint32_t)a.vocab;
  const float* lg = a.logits + (size_t)s * V;
  const double best = (double)lg[a.tokens[s]];
  const uint32_t per = (V + gridDim.x - 1) / gridDim.x;
  const uint32_t i0 = blockIdx.x * per, i1 = min(V, i0 + per);
  double* w = a.weights + (size_t)r * V;
  uint8_t* bk = a.buckets + (size_t)r * a.bucket_stride;
  for (int b = threadIdx.x; b < kBuckets; b += kPassThreads) {
    cnt[b] = 0;
    hi[b] = 0;
    lo[b] = 0;
  }
  __syncthreads();
  double lse = 0.0;
  Best8 top;
  top.clear();
  for (uint32_t i = i0 + threadIdx.x; i < i1; i += kPassThreads) {
    const double l = (double)lg[i] - best;
    if (sampled) {
      const double q = exp(l / p.temperature);
      w[i] = q;
      const int b = bucket_of(q);
      bk[i] = (uint8_t)b;
      const Fx f = to_fx(q);
      atomicAdd(&cnt[b], 1u);
      if (f.hi) atomicAdd(&hi[b], f.hi);
      if (f.lo) atomicAdd(&lo[b], f.lo);
    }
    if (logprobs) {
      lse += exp(l);
      top.offer(descending_key(l), i);
    }
  }
  __syncthreads();
  if (sampled) {
    u64* h = reinterpret_cast<u64*>(a.hist) + (size_t)r * kBuckets * 3;
    for (int b = threadIdx.x; b < kBuckets; b += kPassThreads) {
      if (cnt[b] == 0) continue;
      atomicAdd(&h[b * 3 + 0], (u64)cnt[b]);
      atomicAdd(&h[b * 3 + 1], hi[b]);
      atomicAdd(&h[b * 3 + 2], lo[b]);
    }
  }
  if (logprobs) {
    // fixed order: each wave's butterfly, then the waves in index order
#pragma unroll
    for (int m = 32; m > 0; m >>= 1) lse += __shfl_xor(lse, m, 64);
    if ((threadIdx.x & 63) == 0) dred[threadIdx.x >> 6] = lse;
    __syncthreads();
    if (threadIdx.x == 0) {
      double t = 0.0;
      for (int q = 0; q < kPassWaves; ++q) t += dred[q];
      a.lse_parts[(size_t)r * gridDim.x + blockIdx.x] = t;
    }
    uint32_t* out = a.candidates + ((size_t)r * gridDim.x + blockIdx.x) * kCandidates;
    for (int q = 0; q < kCandidates; ++q) {
      u64 key = top.k[0];
      uint32_t id = top.i[0];
      block_min_pair<kPassWaves>(key, id, pred);
      if (top.k[0] == key && top.i[0] == id) top.pop();
      if (threadIdx.x == 0) out[q] = id;  // ~0u past the chunk's end
    }
  }
}

// Wave 0: exclusive prefix of the 256 bucket counts into `off`.
__device__ inline void bucket_offsets(const uint32_t* cnt, uint32_t* off) {
  const int lane = threadIdx.x;
  uint32_t c[4], t = 0;
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    c[k] = cnt[lane * 4 + k];
    t += c[k];
  }
  uint32_t e = t;
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const uint32_t v = __shfl_up(e, o, 64);
    if (lane >= o) e += v;
  }
  e -= t;
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    off[lane * 4 + k] = e;
    e += c[k];
  }
}

// Second pass (grid: chunks x rows): a counting sort of each row's tokens by bucket into
// `sorted` (bucket b's tokens at [offset(b), offset(b) + count(b)), in no particular
// order; every use of a bucket is order-independent).
__global__ void __launch_bounds__(kPassThreads) sample_scatter_kernel(SampleArgs a, int row0) {
  __shared__ uint32_t off[kBuckets], local[kBuckets], base[kBuckets];
  const int r = blockIdx.y, s = row0 + r;
  if (s >= a.rows) return;
  if (!(a.params[s].temperature > 0.0)) return;
  const uint32_t V = (uint32_t)a.vocab;
  const uint32_t per = (V + gridDim.x - 1) / gridDim.x;
  const uint32_t i0 = blockIdx.x * per, i1 = min(V, i0 + per);
  const uint8_t* bk = a.buckets + (size_t)r * a.bucket_stride;
  const u64* h = reinterpret_cast<const u64*>(a.hist) + (size_t)r * kBuckets * 3;
  uint32_t* cursor = a.cursor + (size_t)r * kBuckets;
  uint32_t* sorted = a.sorted + (size_t)r * V;
  for (int b = threadIdx.x; b < kBuckets; b += kPassThreads) {
    local[b] = (uint32_t)h[b * 3];  // the row's counts, for the offsets
  }
  __syncthreads();
  if (threadIdx.x < 64) bucket_offsets(local, off);
  __syncthreads();
  for (int b = threadIdx.x; b < kBuckets; b += kPassThreads) local[b] = 0;
  __syncthreads();
  for (uint32_t i = i0 + threadIdx.x; i < i1; i += kPassThreads) atomicAdd(&local[bk[i]], 1u);
  __syncthreads();
  for (int b = threadIdx.x; b < kBuckets; b += kPassThreads) {
    base[b] = local[b] ? off[b] + atomicAdd(&cursor[b], local[b]) : 0;
    local[b] = 0;
  }
  __syncthreads();
  for (uint32_t i = i0 + threadIdx.x; i < i1; i += kPassThreads) {
    const int b = bk[i];
    sorted[base[b] + atomicAdd(&local[b], 1u)] = i;
  }
}

struct BucketPick {
  int bucket;    // the first bucket reaching the goal; `limit` when none below it does
  u64 count;     // tokens in the buckets before it
  u128 mass;     // their mass
};

// Wave 0: the first bucket b < limit at which the running count (or mass) of buckets
// 0..b reaches `goal` (>= goal, or > goal when `strict`). Result in LDS.
__device__ void scan_buckets(const uint32_t* cnt, const u64* hi, const u64* lo, int limit, u128 goal, bool counts,
                             bool strict, Shared& sh) {
  const int lane = threadIdx.x;
  u64 c[4], h[4], l[4];
  u64 lc = 0, lh = 0, ll = 0;
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    const int d = lane * 4 + k;
    const bool in = d < limit;
    c[k] = in ? cnt[d] : 0;
    h[k] = in ? hi[d] : 0;
    l[k] = in ? lo[d] : 0;
    lc += c[k];
    lh += h[k];
    ll += l[k];
  }
  u64 ec = lc, eh = lh, el = ll;
#pragma unroll
  for (int off = 1; off < 64; off <<= 1) {
    const u64 tc = __shfl_up(ec, off, 64), th = __shfl_up(eh, off, 64), tl = __shfl_up(el, off, 64);
    if (lane >= off) {
      ec += tc;
      eh += th;
      el += tl;
    }
  }
  ec -= lc;
  eh -= lh;
  el -= ll;
  int hit = -1;
  u64 hc = 0, hh = 0, hl = 0;
  u64 rc = ec, rh = eh, rl = el;
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    const u128 incl = counts ? (u128)(rc + c[k]) : fx_value(rh + h[k], rl + l[k]);
    if (hit < 0 && c[k] > 0 && (strict ? incl > goal : incl >= goal)) {
      hit = k;
      hc = rc;
      hh = rh;
      hl = rl;
    }
    rc += c[k];
    rh += h[k];
    rl += l[k];
  }
  const u64 hits = __ballot(hit >= 0);
  if (hits) {
    if (lane == __builtin_ctzll(hits)) {
      sh.chosen = lane * 4 + hit;
      sh.before_hi = hh;
      sh.before_lo = hl;
      sh.scan_count = hc;
    }
  } else if (lane == 63) {
    sh.chosen = limit;
    sh.before_hi = rh;
    sh.before_lo = rl;
    sh.scan_count = rc;
  }
}

__device__ BucketPick pick_bucket(const uint32_t* cnt, const u64* hi, const u64* lo, int limit, u128 goal, bool counts,
                                  bool strict, Shared& sh) {
  if (threadIdx.x < 64) scan_buckets(cnt, hi, lo, limit, goal, counts, strict, sh);
  __syncthreads();
  const BucketPick b{sh.chosen, sh.scan_count, fx_value(sh.before_hi, sh.before_lo)};
  __syncthreads();
  return b;
}

// AND / OR of the ranks of a list's tokens.
__device__ void list_ranks(const uint32_t* list, uint32_t n, const double* w, u128& c_and, u128& c_or, Shared& sh) {
  u128 an = ~(u128)0, o = 0;
  for_each_token(list, n, w, [&](uint32_t e, double p) {
    const u128 r = rank_of(p, e);
    an &= r;
    o |= r;
  });
  block_and_or(an, o, sh);
  c_and = an;
  c_or = o;
}

// Third pass, one row per workgroup: the token, by exact descents over the bucket slices
// where the top-k, top-p and draw boundaries fall; then log-probabilities.
__global__ void __launch_bounds__(kThreads) sample_select_kernel(SampleArgs a, int row0) {
  __shared__ Shared sh;
  __shared__ uint32_t bcnt[kBuckets], boff[kBuckets];
  __shared__ u64 bhi[kBuckets], blo[kBuckets];
  const int r = blockIdx.x, s = row0 + r;
  if (s >= a.rows) return;
  const SampleParams p = a.params[s];
  const bool sampled = p.temperature > 0.0, logprobs = (p.flags & kSampleLogprobs) != 0;
  if (!sampled && !logprobs) return;  // greedy: the first maximum stands
  const uint32_t V = (uint32_t)a.vocab;
  const float* lg = a.logits + (size_t)s * V;
  int token = a.tokens[s];
  const double best = (double)lg[token];
  if (sampled) {
    const double* w = a.weights + (size_t)r * V;
    const uint32_t* sorted = a.sorted + (size_t)r * V;
    uint32_t* L[4];
#pragma unroll
    for (int q = 0; q < 4; ++q) L[q] = a.lists + ((size_t)r * 4 + q) * V;
    // The row's histogram and sort cursors, cleared for their next use.
    u64* h = reinterpret_cast<u64*>(a.hist) + (size_t)r * kBuckets * 3;
    uint32_t* cursor = a.cursor + (size_t)r * kBuckets;
    for (int b = threadIdx.x; b < kBuckets; b += kThreads) {
      bcnt[b] = (uint32_t)h[b * 3 + 0];
      bhi[b] = h[b * 3 + 1];
      blo[b] = h[b * 3 + 2];
      h[b * 3 + 0] = 0;
      h[b * 3 + 1] = 0;
      h[b * 3 + 2] = 0;
      cursor[b] = 0;
    }
    __syncthreads();
    if (threadIdx.x < 64) bucket_offsets(bcnt, boff);
    __syncthreads();
    auto slice = [&](int b) { return sorted + boff[b]; };
    // 1. Candidates: the first top_k in rank order (all tokens when top_k is 0 or >= V).
    //    Buckets below kb are whole; bucket kb contributes the list `kl` (nk tokens).
    int kb = kBuckets;
    u128 kb_mass = 0;  // mass of the buckets before kb
    uint32_t* kl = nullptr;
    uint32_t nk = 0;
    u128 k_and = 0, k_or = 0, total;
    if (p.top_k != 0 && p.top_k < (u64)V) {
      const BucketPick kp = pick_bucket(bcnt, bhi, blo, kBuckets, (u128)p.top_k, true, false, sh);
      kb = kp.bucket;
      kb_mass = kp.mass;
      u128 an, o;
      const uint32_t n = bcnt[kb];
      list_ranks(slice(kb), n, w, an, o, sh);
      const Found kth = descend<false>(slice(kb), n, an, o, w, (u128)(p.top_k - kp.count), false, L[2], L[3], sh);
      u128 km = 0;
      if (kth.id >= 0) nk = compact_upto(slice(kb), n, w, rank_of(w[kth.id], (uint32_t)kth.id), L[0], k_and, k_or, km, sh);
      kl = L[0];
      total = kb_mass + km;
    } else {
      total = pick_bucket(bcnt, bhi, blo, kBuckets, ~(u128)0, false, false, sh).mass;
    }
    // 2. The top-p cut: the first candidate whose running mass reaches total * top_p.
    const u128 threshold = fx_of(fx_double(total) * p.top_p);
    const BucketPick cp = pick_bucket(bcnt, bhi, blo, kb, threshold, false, false, sh);
    const uint32_t* cl;  // the cut's bucket slice (or its candidates in bucket kb)
    uint32_t nc;
    int cut_bucket;
    u128 c_and, c_or, c_before, goal = threshold;
    if (cp.bucket < kb) {
      cut_bucket = cp.bucket;
      cl = slice(cut_bucket);
      nc = bcnt[cut_bucket];
      list_ranks(cl, nc, w, c_and, c_or, sh);
      c_before = cp.mass;
    } else if (kb < kBuckets) {
      cut_bucket = kb;
      cl = kl;
      nc = nk;
      c_and = k_and;
      c_or = k_or;
      c_before = kb_mass;
    } else {
      // Rounding put the threshold above the whole mass: every candidate is retained,
      // and the cut is the last one (the reference's loop runs to the end).
      cut_bucket = kBuckets - 1;
      while (cut_bucket > 0 && bcnt[cut_bucket] == 0) --cut_bucket;
      cl = slice(cut_bucket);
      nc = bcnt[cut_bucket];
      list_ranks(cl, nc, w, c_and, c_or, sh);
      c_before = total - fx_value(bhi[cut_bucket], blo[cut_bucket]);
      goal = ~(u128)0;
    }
    const Found cut =
        descend<true>(cl, nc, c_and, c_or, w, goal == ~(u128)0 ? goal : goal - c_before, false, L[2], L[3], sh);
    if (cut.id >= 0) {
      const u128 retained = c_before + cut.running;
      // 3. The draw: the first retained candidate whose running mass exceeds u * retained.
      const double target = (double)(counter_bits(p.seed, p.generated_index) >> 11) * 0x1.0p-53 * fx_double(retained);
      const u128 x = fx_of(target);
      const BucketPick pp = pick_bucket(bcnt, bhi, blo, cut_bucket, x, false, true, sh);
      Found pick{-1, 0};
      if (pp.bucket < cut_bucket) {
        u128 an, o;
        const uint32_t n = bcnt[pp.bucket];
        list_ranks(slice(pp.bucket), n, w, an, o, sh);
        pick = descend<true>(slice(pp.bucket), n, an, o, w, x - pp.mass, true, L[2], L[3], sh);
      } else {
        u128 an, o, m;
        const uint32_t n = compact_upto(cl, nc, w, rank_of(w[cut.id], (uint32_t)cut.id), L[1], an, o, m, sh);
        pick = descend<true>(L[1], n, an, o, w, x > c_before ? x - c_before : (u128)0, true, L[2], L[3], sh);
      }
      if (pick.id >= 0) token = pick.id;
    }
  }
  if (threadIdx.x == 0) a.tokens[s] = token;
  if (logprobs) {
    // log-softmax of the raw logits (no temperature, no cuts)
    double lse = 0.0;
    for (int c = 0; c < a.chunks; ++c) lse += a.lse_parts[(size_t)r * a.chunks + c];
    const double log_sum = log(lse);
    if (threadIdx.x == 0) a.logprob[s] = ((double)lg[token] - best) - log_sum;
    // The top_logprobs best tokens by (log-probability descending, ID ascending), from
    // the chunks' candidates (each chunk's best by logit): thread t holds candidate t.
    const int total_candidates = a.chunks * kCandidates;
    u64 key = ~0ull;
    uint32_t id = ~0u;
    if ((int)threadIdx.x < total_candidates) {
      const uint32_t c = a.candidates[(size_t)r * total_candidates + threadIdx.x];
      if (c < V) {
        id = c;
        key = descending_key(((double)lg[c] - best) - log_sum);
      }
    }
    const uint32_t rounds = min(p.top_logprobs, min(5u, V));
    for (uint32_t q = 0; q < rounds; ++q) {
      u64 bk2 = key;
      uint32_t bi = id;
      block_min_pair<kWaves>(bk2, bi, sh.red);
      if (key == bk2 && id == bi) {
        key = ~0ull;
        id = ~0u;
      }
      if (threadIdx.x == 0 && bi < V) {
        a.top_ids[(size_t)s * 5 + q] = (int32_t)bi;
        a.top_values[(size_t)s * 5 + q] = ((double)lg[bi] - best) - log_sum;
      }
    }
  }
}

}  // namespace

void launch_sample(hipStream_t stream, const SampleArgs& a) {
  if (a.rows <= 0 || a.group_rows <= 0) return;
  if (a.chunks * kCandidates > kThreads) fail(HLLM_INTERNAL, "too many sampling chunks");
  for (int row0 = 0; row0 < a.rows; row0 += a.group_rows) {
    const int n = std::min(a.group_rows, a.rows - row0);
    observed("sample_histogram_kernel",
             [&] { sample_histogram_kernel<<<dim3(a.chunks, n), kPassThreads, 0, stream>>>(a, row0); });
    observed("sample_scatter_kernel",
             [&] { sample_scatter_kernel<<<dim3(a.chunks, n), kPassThreads, 0, stream>>>(a, row0); });
    observed("sample_select_kernel", [&] { sample_select_kernel<<<n, kThreads, 0, stream>>>(a, row0); });
  }
}

}  // namespace hllm_rocm
