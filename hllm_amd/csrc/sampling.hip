// Temperature / top-k / top-p sampling and log-probabilities on the device, one workgroup
// per sampled row, following the reference sampler (cpp/src/sampling.cpp:19-89):
//   p_i = exp((l_i - max) / T) in double; candidates in descending p, equal p by lower
//   token ID; the first top_k of them; the shortest prefix whose mass reaches top_p of the
//   candidates' total; a SplitMix64 counter draw u in [0, 1) times that prefix's mass picks
//   the first candidate whose running mass exceeds it.
// Nothing is sorted. Each cut is found by a radix descent over the candidates' rank
// (~bits(p) << 32 | id, ascending = reference order): an 8-bit digit histogram of counts
// and masses in LDS picks the digit bucket in which the running mass crosses the goal, that
// bucket's members are compacted into a list, and the next digit below the list's highest
// differing bit is examined, until one candidate remains.
// Masses are sums of probabilities held as integers in units of 2^-80 (each probability is
// in [0, 1]; a vocabulary of up to 2^23 sums without overflow), so every sum is exact and
// independent of the order of the LDS atomics: results are deterministic. The reference
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

// A double sum in a fixed order: each wave's butterfly, then the waves in index order.
__device__ inline double block_sum(double v, Shared& sh) {
#pragma unroll
  for (int m = 32; m > 0; m >>= 1) v += __shfl_xor(v, m, 64);
  if (lane_id() == 0) sh.dred[threadIdx.x >> 6] = v;
  __syncthreads();
  double total = 0.0;
  for (int w = 0; w < kWaves; ++w) total += sh.dred[w];
  __syncthreads();
  return total;
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
    for (uint32_t j = threadIdx.x; j < n; j += kThreads) {
      const uint32_t e = cur ? cur[j] : j;
      const double p = w[e];
      const int d = (int)((uint32_t)(rank_of(p, e) >> shift) & 255u);
      atomicAdd(&sh.count[d], 1u);
      if (kWeighted) {
        const Fx f = to_fx(p);
        atomicAdd(&sh.hi[d], f.hi);
        atomicAdd(&sh.lo[d], f.lo);
      }
    }
    __syncthreads();
    if (threadIdx.x < 64) choose_bucket<kWeighted>(sh, before, goal, strict, never);
    __syncthreads();
    const int chosen = sh.chosen;
    before += fx_value(sh.before_hi, sh.before_lo);
    never = sh.never != 0;
    u128 a = ~(u128)0, o = 0;
    for (uint32_t j = threadIdx.x; j < n; j += kThreads) {
      const uint32_t e = cur ? cur[j] : j;
      const u128 r = rank_of(w[e], e);
      const bool keep = (int)((uint32_t)(r >> shift) & 255u) == chosen;
      push(keep, e, out, &sh.list_n);
      if (keep) {
        a &= r;
        o |= r;
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
  for (uint32_t j = threadIdx.x; j < n; j += kThreads) {
    const uint32_t e = in ? in[j] : j;
    const double p = w[e];
    const u128 r = rank_of(p, e);
    const bool keep = r <= limit;
    push(keep, e, out, &sh.list_n);
    if (keep) {
      a &= r;
      o |= r;
      const Fx f = to_fx(p);
      hi += f.hi;
      lo += f.lo;
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

__global__ void __launch_bounds__(kThreads) sample_kernel(SampleArgs a) {
  __shared__ Shared sh;
  const uint32_t V = (uint32_t)a.vocab;
  double* w = a.weights + (size_t)blockIdx.x * V;
  uint32_t* b0 = a.lists + (size_t)blockIdx.x * 3 * V;
  uint32_t* b1 = b0 + V;
  uint32_t* b2 = b1 + V;
  for (int s = blockIdx.x; s < a.rows; s += gridDim.x) {
    const SampleParams p = a.params[s];
    const bool want_logprobs = (p.flags & kSampleLogprobs) != 0;
    if (!(p.temperature > 0.0) && !want_logprobs) continue;  // greedy: the first maximum stands
    const float* lg = a.logits + (size_t)s * V;
    int token = a.tokens[s];
    const double best = (double)lg[token];
    if (p.temperature > 0.0) {
      u128 c_and = ~(u128)0, c_or = 0;
      u64 hi = 0, lo = 0;
      for (uint32_t i = threadIdx.x; i < V; i += kThreads) {
        const double q = exp(((double)lg[i] - best) / p.temperature);
        w[i] = q;
        const u128 r = rank_of(q, i);
        c_and &= r;
        c_or |= r;
        const Fx f = to_fx(q);
        hi += f.hi;
        lo += f.lo;
      }
      block_and_or(c_and, c_or, sh);  // barriers also publish w
      block_sum2(hi, lo, sh);
      u128 total = fx_value(hi, lo);
      const uint32_t* cand = nullptr;
      uint32_t cn = V;
      if (p.top_k != 0 && p.top_k < (u64)V) {
        const Found kth = descend<false>(nullptr, V, c_and, c_or, w, (u128)p.top_k, false, b0, b1, sh);
        if (kth.id >= 0) {
          cn = compact_upto(nullptr, V, w, rank_of(w[kth.id], (uint32_t)kth.id), b2, c_and, c_or, total, sh);
          cand = b2;
        }
      }
      const u128 threshold = fx_of(fx_double(total) * p.top_p);
      const Found cut = descend<true>(cand, cn, c_and, c_or, w, threshold, false, b0, b1, sh);
      if (cut.id >= 0) {
        const double retained = fx_double(cut.running);
        const double target = (double)(counter_bits(p.seed, p.generated_index) >> 11) * 0x1.0p-53 * retained;
        u128 pa, po, pm;
        const uint32_t pn = compact_upto(cand, cn, w, rank_of(w[cut.id], (uint32_t)cut.id), b0, pa, po, pm, sh);
        const Found pick = descend<true>(b0, pn, pa, po, w, fx_of(target), true, b1, b2, sh);
        if (pick.id >= 0) token = pick.id;
      }
    }
    if (threadIdx.x == 0) a.tokens[s] = token;
    if (want_logprobs) {
      // log-softmax of the raw logits (no temperature, no cuts)
      double sum = 0.0;
      for (uint32_t i = threadIdx.x; i < V; i += kThreads) sum += exp((double)lg[i] - best);
      const double log_sum = log(block_sum(sum, sh));
      if (threadIdx.x == 0) a.logprob[s] = ((double)lg[token] - best) - log_sum;
      // the best top_logprobs tokens by (log-probability descending, ID ascending):
      // per-thread sorted top 5, then one block-wide minimum per output
      u64 tk[5];
      uint32_t ti[5];
#pragma unroll
      for (int k = 0; k < 5; ++k) {
        tk[k] = ~0ull;
        ti[k] = ~0u;
      }
      for (uint32_t i = threadIdx.x; i < V; i += kThreads) {
        const u64 key = descending_key(((double)lg[i] - best) - log_sum);
        if (!rank_less(key, i, tk[4], ti[4])) continue;
#pragma unroll
        for (int k = 4; k > 0; --k) {
          const bool below = rank_less(key, i, tk[k - 1], ti[k - 1]);
          const bool here = !below && rank_less(key, i, tk[k], ti[k]);
          tk[k] = below ? tk[k - 1] : here ? key : tk[k];
          ti[k] = below ? ti[k - 1] : here ? i : ti[k];
        }
        if (rank_less(key, i, tk[0], ti[0])) {
          tk[0] = key;
          ti[0] = i;
        }
      }
      const uint32_t rounds = min(p.top_logprobs, min(5u, V));
      for (uint32_t r = 0; r < rounds; ++r) {
        u64 k = tk[0];
        uint32_t id = ti[0];
#pragma unroll
        for (int m = 32; m > 0; m >>= 1) {
          const u64 ok = __shfl_xor(k, m, 64);
          const uint32_t oi = __shfl_xor(id, m, 64);
          if (rank_less(ok, oi, k, id)) {
            k = ok;
            id = oi;
          }
        }
        if (lane_id() == 0) {
          sh.red[threadIdx.x >> 6][0] = k;
          sh.red[threadIdx.x >> 6][1] = id;
        }
        __syncthreads();
        u64 bk = ~0ull;
        uint32_t bi = ~0u;
        for (int wv = 0; wv < kWaves; ++wv) {
          if (rank_less(sh.red[wv][0], (uint32_t)sh.red[wv][1], bk, bi)) {
            bk = sh.red[wv][0];
            bi = (uint32_t)sh.red[wv][1];
          }
        }
        __syncthreads();
        if (tk[0] == bk && ti[0] == bi) {
#pragma unroll
          for (int q = 0; q < 4; ++q) {
            tk[q] = tk[q + 1];
            ti[q] = ti[q + 1];
          }
          tk[4] = ~0ull;
          ti[4] = ~0u;
        }
        if (threadIdx.x == 0 && bi < V) {
          a.top_ids[(size_t)s * 5 + r] = (int32_t)bi;
          a.top_values[(size_t)s * 5 + r] = ((double)lg[bi] - best) - log_sum;
        }
      }
    }
    __syncthreads();
  }
}

}  // namespace

void launch_sample(hipStream_t stream, const SampleArgs& a, int blocks) {
  if (a.rows <= 0 || blocks <= 0) return;
  observed("sample_kernel", [&] { sample_kernel<<<std::min(a.rows, blocks), kThreads, 0, stream>>>(a); });
}

}  // namespace hllm_rocm
