// Token sampler for gfx950: the step after the last layer's decode.
//
// One workgroup (1024 threads) per row of logits, passes over the row (L2 /
// MALL resident after the first):
//   x_i = (repetition penalty on seen tokens)(logit_i) / T   (T = 1 for greedy rows)
//   min_p:  keep x_i >= max + ln(min_p)             (p_i >= min_p * p_max)
//   top_k:  keep the k largest (exact radix select over order-preserving
//           32-bit keys, four 8-bit rounds, LDS histograms; ties kept)
//   top_p:  keep token i iff the mass strictly above it is < top_p * mass
//           (radix select over the same keys with 64-bit fixed-point mass
//           histograms -- integer sums, so the threshold is deterministic)
//   sample: argmax over kept i of x_i - ln(E_i), E_i ~ Exp(1) from a
//           counter-based hash of (seed, step, i) -- the exponential race,
//           an exact draw from softmax over the kept set; greedy rows take
//           argmax x_i. Ties go to the lowest index.
// Outputs: the token, its processed logprob (log-softmax over the kept set of
// the processed logits), the kept set as a bitmap and its size.
#include <cmath>
#include <type_traits>

#include "wkv_common.h"

namespace wkv {

constexpr int kSampleThreads = 1024;
constexpr float kGreedyEps = 1e-5f;  // temperatures below this sample greedily
// A score x - ln E is at most x + 16.636 (u <= 1 - 2^-24): a token more than
// kScoreReach below a score already drawn never wins the race (0.064 of margin
// for float rounding).
constexpr float kScoreReach = 16.7f;

// Order-preserving key of a float (larger float -> larger key); NaN maps below
// every real value so it is never kept.
__device__ __forceinline__ uint32_t order_key(float x) {
  if (x != x) return 0u;
  const uint32_t u = __float_as_uint(x);
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

// splitmix64 finaliser.
__device__ __forceinline__ uint64_t mix64(uint64_t z) {
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
  return z ^ (z >> 31);
}

// ln(E) of the Exp(1) variate of token i: u in [2^-24, 1 - 2^-24] from 23
// hash bits, exact in float32 (24 bits would round the top value to 1.0:
// E = 0 and an infinite race score for one token in 2^24). Both logarithms
// take the hardware log2 times ln 2: their arguments (u >= 2^-24, -ln u >=
// 6e-8) are never denormal, so logf's scaling and extended-precision fixups
// buy at most an ulp here.
__device__ __forceinline__ float log_exp_variate(uint64_t stream, int64_t i) {
  const uint64_t h = mix64(stream + static_cast<uint64_t>(i));
  // u = (m + 0.5) 2^-23 for the top 23 bits m, exactly: 1 + m 2^-23 from the
  // bits, minus 1 (exact), plus 2^-24 (exact at that magnitude).
  const uint32_t m = static_cast<uint32_t>(h >> 32) >> 9;
  const float u = (__uint_as_float(0x3F800000u | m) - 1.0f) + 5.9604644775390625e-8f;
  constexpr float kLn2 = 0.693147180559945309f;
  return __builtin_amdgcn_logf(-__builtin_amdgcn_logf(u) * kLn2) * kLn2;
}

template <typename T>
__device__ __forceinline__ float load_logit(const T *row, int64_t i);
template <>
__device__ __forceinline__ float load_logit<float>(const float *row, int64_t i) { return row[i]; }
template <>
__device__ __forceinline__ float load_logit<uint16_t>(const uint16_t *row, int64_t i) {
  return bf16_bits_to_f32(row[i]);
}

// Elements per thread per step: 8 consecutive logits, one or two 16-byte loads
// when the row allows it (`vec`), element loads otherwise; -inf past the end.
constexpr int kVec = 8;
// Chunks a pass keeps in flight per thread: the loads of kBatch chunks issue
// before the first is used (with one 16-byte load per thread at a time a pass
// over a row is bound by the load latency, not by HBM).
constexpr int kBatch = 4;

// One chunk's raw bits: 16 bytes of bf16, or 32 of fp32.
template <typename T>
struct Chunk;
template <>
struct Chunk<uint16_t> {
  u32x4 w;
};
template <>
struct Chunk<float> {
  floatx4 a, b;
};

template <typename T>
__device__ __forceinline__ Chunk<T> load_chunk(const T *p) {
  if constexpr (sizeof(T) == 2) {
    return Chunk<T>{*reinterpret_cast<const u32x4 *>(p)};
  } else {
    return Chunk<T>{*reinterpret_cast<const floatx4 *>(p), *reinterpret_cast<const floatx4 *>(p + 4)};
  }
}

template <typename T>
__device__ __forceinline__ void unpack_chunk(const Chunk<T> &c, float v[kVec]) {
  if constexpr (sizeof(T) == 2) {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      v[2 * j] = __uint_as_float(c.w[j] << 16);
      v[2 * j + 1] = __uint_as_float(c.w[j] & 0xffff0000u);
    }
  } else {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      v[j] = c.a[j];
      v[4 + j] = c.b[j];
    }
  }
}

template <typename T>
__device__ __forceinline__ void load8(float v[kVec], const T *row, int64_t base, int vocab, bool vec) {
  if (vec && base + kVec <= vocab) {
    unpack_chunk<T>(load_chunk<T>(row + base), v);
  } else {
#pragma unroll
    for (int j = 0; j < kVec; ++j) v[j] = base + j < vocab ? load_logit<T>(row, base + j) : -INFINITY;
  }
}

// Block-wide reductions over 1024 threads (16 waves) through a small LDS array.
__device__ __forceinline__ float block_max(float v, float *red) {
  v = wave_max(v);
  const int w = threadIdx.x >> 6;
  if ((threadIdx.x & 63) == 0) red[w] = v;
  __syncthreads();
  float r = red[0];
  for (int i = 1; i < kSampleThreads / 64; ++i) r = fmaxf(r, red[i]);
  __syncthreads();
  return r;
}

__device__ __forceinline__ float block_sum(float v, float *red) {
  v = wave_sum(v);
  const int w = threadIdx.x >> 6;
  if ((threadIdx.x & 63) == 0) red[w] = v;
  __syncthreads();
  float r = 0.f;
  for (int i = 0; i < kSampleThreads / 64; ++i) r += red[i];  // fixed order: deterministic
  __syncthreads();
  return r;
}

// (value, index) argmax, ties to the lowest index.
__device__ __forceinline__ void arg_better(float &v, int64_t &i, float ov, int64_t oi) {
  if (ov > v || (ov == v && oi < i)) {
    v = ov;
    i = oi;
  }
}

__device__ __forceinline__ void block_argmax(float &v, int64_t &idx, float *redv, int64_t *redi) {
  const auto step = [&](auto o) {
    constexpr int O = decltype(o)::value;
    arg_better(v, idx, lane_xor<O>(v), lane_xor<O>(idx));
  };
  step(std::integral_constant<int, 32>{});
  step(std::integral_constant<int, 16>{});
  step(std::integral_constant<int, 8>{});
  step(std::integral_constant<int, 4>{});
  step(std::integral_constant<int, 2>{});
  step(std::integral_constant<int, 1>{});
  const int w = threadIdx.x >> 6;
  if ((threadIdx.x & 63) == 0) {
    redv[w] = v;
    redi[w] = idx;
  }
  __syncthreads();
  v = redv[0];
  idx = redi[0];
  for (int i = 1; i < kSampleThreads / 64; ++i) arg_better(v, idx, redv[i], redi[i]);
  __syncthreads();
}

// 64-bit sums and scans over a wave and the 1024-thread block.
__device__ __forceinline__ unsigned long long wave_sum_u64(unsigned long long v) {
  return wave_reduce(v, [](unsigned long long a, unsigned long long b) { return a + b; });
}

__device__ __forceinline__ unsigned long long wave_incl_scan_u64(unsigned long long v, int lane) {
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const unsigned long long y = __shfl_up(v, o, 64);
    if (lane >= o) v += y;
  }
  return v;
}

// Exclusive scan of one value per thread in thread order; `total` gets the sum.
__device__ __forceinline__ unsigned long long block_exscan_u64(unsigned long long v, unsigned long long *red,
                                                               unsigned long long &total) {
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const unsigned long long incl = wave_incl_scan_u64(v, lane);
  if (lane == 63) red[w] = incl;
  __syncthreads();
  unsigned long long before = 0, all = 0;
  for (int i = 0; i < kSampleThreads / 64; ++i) {
    if (i < w) before += red[i];
    all += red[i];
  }
  __syncthreads();
  total = all;
  return before + incl - v;
}

// Radix-select step on a 256-bin histogram, searched from the top bin down:
// the largest j with above + sum(hist[j..255]) >= target, and the sum
// strictly above it (bin -1 when no j qualifies). Wave 0 computes it (four
// bins per lane and one wave scan) and writes it to *bin_out / *cum_out.
__device__ __forceinline__ void find_from_top(const unsigned long long *hist, unsigned long long above,
                                              unsigned long long target, uint32_t *bin_out,
                                              unsigned long long *cum_out) {
  if (threadIdx.x >= 64) return;
  const int lane = threadIdx.x;
  unsigned long long h[4], s = 0;
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    h[q] = hist[255 - 4 * lane - q];
    s += h[q];
  }
  unsigned long long c = above + wave_incl_scan_u64(s, lane) - s;  // mass of the bins above this lane's
  int bin = -1;
  unsigned long long cum = 0;
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    if (bin < 0 && c + h[q] >= target) {
      bin = 255 - 4 * lane - q;
      cum = c;
    }
    c += h[q];
  }
  const unsigned long long hit = __ballot(bin >= 0);
  if (hit == 0ull) {
    if (lane == 0) *bin_out = 0xffffffffu;
  } else if (lane == __ffsll(static_cast<long long>(hit)) - 1) {
    *bin_out = static_cast<uint32_t>(bin);
    *cum_out = cum;
  }
}

// Fast top_k / top_p. Every kept token the threshold can keep lies within a
// range below the row maximum known before the second pass (top_k: the bin of
// the k-th largest of the threads' maxima; top_p alone: a bound on the tail's
// weight), so one capture pass copies the kept tokens in that range -- at
// most kCand of them -- into an LDS list, the exact radix selects run over
// the list and the draw, mass and mask come from it too. Rows whose range
// holds more tokens take a histogram of the kept tokens by distance below the
// maximum (kBins bins of 1/kBinScale, the last one open-ended), whose block
// scan gives the threshold's bin, and a compaction pass of the kept tokens at
// or above it. Binning is monotone in the value, so the list holds every
// token the threshold can keep and the selects give the same keys as over the
// whole row; rows whose threshold still falls in the open bin or overflows
// the list take the full-row radix passes.
constexpr int kBins = 2048;
constexpr float kBinScale = 32.f;
constexpr int kCand = 4096;
// A token this many bins or more below the maximum (22.2 nats) weighs under
// one unit of fixed_mass: exactly 0.
constexpr int kMassBins = 711;
// Rows of up to kMaskWords * 32 tokens build their mask in LDS on the list path.
constexpr int kMaskWords = 8192;
// Draws a wave may hold back before making them 64 at a time (final pass).
constexpr int kQueue = 128;
// The same for the final pass's fast loop, which makes its draws after every
// fourth token slot: fewer than 64 pending, plus 64 per slot.
constexpr int kFastQueue = 64 + 4 * 64;
static_assert(kBins == 2 * kSampleThreads, "the threshold scan gives every thread two bins");

__device__ __forceinline__ unsigned long long fixed_mass(float x, float mx) {
  return static_cast<unsigned long long>(expf(x - mx) * 4294967296.f);
}

struct SampleArgs {
  const float *temperature;  // [B] or NULL (1.0)
  const int32_t *top_k;      // [B] or NULL; <= 0 or >= vocab: off
  const float *top_p;        // [B] or NULL; >= 1: off
  const float *min_p;        // [B] or NULL; <= 0: off
  const float *rep_penalty;  // [B] or NULL; 1: off
  const uint32_t *seen;      // [B, words] bitmap of prompt/output tokens or NULL
  const uint64_t *seeds;     // [B] or NULL (0)
  int64_t step;              // mixed into every row's random stream
  int64_t *tokens;           // [B]
  float *logprobs;           // [B] or NULL
  uint32_t *mask;            // [B, words] or NULL
  int32_t *counts;           // [B] or NULL
};

template <typename T>
__global__ __launch_bounds__(kSampleThreads) void sample_kernel(const T *__restrict__ logits, int64_t row_stride,
                                                                int vocab, SampleArgs a) {
  __shared__ float redv[kSampleThreads / 64];
  __shared__ int64_t redi[kSampleThreads / 64];
  __shared__ unsigned long long hist[256];
  __shared__ uint32_t sel_prefix;
  __shared__ unsigned long long sel_above;
  __shared__ unsigned long long red64[kSampleThreads / 64];
  __shared__ uint32_t fcnt[kBins];
  __shared__ unsigned long long fmass[kBins];  // also the final pass's draw queues
  static_assert(sizeof(fmass) >= (kSampleThreads / 64) * kQueue * 8, "the draw queues fit the mass bins");
  __shared__ float fq_x[kSampleThreads / 64][kFastQueue];  // the fast loop's draw queues (value, token)
  __shared__ int32_t fq_t[kSampleThreads / 64][kFastQueue];
  __shared__ uint32_t ckey[kCand];
  __shared__ float cx[kCand];
  __shared__ int32_t cidx[kCand];
  __shared__ uint32_t mbits[kMaskWords];
  __shared__ int ncand, sel_bin;
  __shared__ unsigned long long sel_n;
  const int b = blockIdx.x;
  const int tid = threadIdx.x;
  const T *row = logits + static_cast<int64_t>(b) * row_stride;
  const int words = (vocab + 31) / 32;
  const float temp = a.temperature ? a.temperature[b] : 1.f;
  const bool greedy = temp < kGreedyEps;
  const float inv_t = greedy ? 1.f : 1.f / temp;
  const float pen = a.rep_penalty ? a.rep_penalty[b] : 1.f;
  const uint32_t *seen = (a.seen && pen != 1.f) ? a.seen + static_cast<int64_t>(b) * words : nullptr;
  const bool vec = (row_stride % kVec) == 0 && (reinterpret_cast<uintptr_t>(logits) & 15u) == 0;
  auto x_of = [&](int64_t i) {
    float l = load_logit<T>(row, i);
    if (seen && ((seen[i >> 5] >> (i & 31)) & 1u)) l = l > 0.f ? l / pen : l * pen;
    return l * inv_t;
  };
  // The 8 processed logits at base .. base+7 (-inf past the end).
  auto processed = [&](float v[kVec], int64_t base) {
    if (seen) {
      const uint32_t w = seen[base >> 5] >> (base & 31);  // base is a multiple of 8: one word
#pragma unroll
      for (int j = 0; j < kVec; ++j)
        if ((w >> j) & 1u) v[j] = v[j] > 0.f ? v[j] / pen : v[j] * pen;
    }
#pragma unroll
    for (int j = 0; j < kVec; ++j) v[j] *= inv_t;
  };
  auto x8 = [&](float v[kVec], int64_t base) {
    load8<T>(v, row, base, vocab, vec);
    processed(v, base);
  };
  const int64_t step8 = static_cast<int64_t>(kSampleThreads) * kVec;
  // f(v, base) over this thread's chunks in row order, kBatch loads in flight.
  // With EVERY the trip count is uniform and f also sees the chunks past the
  // end (all -inf), so every lane of a wave makes the same calls.
  auto for_chunks = [&](auto every, auto &&f) {
    constexpr bool EVERY = decltype(every)::value;
    for (int64_t c0 = 0; c0 < vocab; c0 += kBatch * step8) {
      const int64_t t0 = c0 + static_cast<int64_t>(tid) * kVec;
      if (vec && c0 + kBatch * step8 <= vocab) {  // uniform: every chunk of the batch is whole
        Chunk<T> r[kBatch];
#pragma unroll
        for (int u = 0; u < kBatch; ++u) r[u] = load_chunk<T>(row + t0 + u * step8);
#pragma unroll
        for (int u = 0; u < kBatch; ++u) {
          float v[kVec];
          unpack_chunk<T>(r[u], v);
          processed(v, t0 + u * step8);
          f(v, t0 + u * step8);
        }
      } else {
        for (int u = 0; u < kBatch; ++u) {
          const int64_t base = t0 + u * step8;
          float v[kVec];
          if (base < vocab) {
            x8(v, base);
          } else {
            if (!EVERY) break;
#pragma unroll
            for (int j = 0; j < kVec; ++j) v[j] = -INFINITY;
          }
          f(v, base);
        }
      }
    }
  };
  using Every = std::true_type;
  using Own = std::false_type;

  // Pass 1: the row maximum. Each thread keeps its own (top_k's capture range)
  // and, for rows drawn by the full-row pass, where it is (the race's bound).
  const int topk = a.top_k ? a.top_k[b] : 0;
  const float tp = a.top_p ? a.top_p[b] : 1.f;
  const bool want_k = topk > 0 && topk < vocab;
  const bool want_p = tp < 1.f;
  const bool track = !greedy && !want_k && !want_p;
  float tmx = -INFINITY;
  int tmi = 0;
  if (track) {
    for_chunks(Own{}, [&](const float v[kVec], int64_t base) {
#pragma unroll
      for (int j = 0; j < kVec; ++j) {
        if (v[j] > tmx) {  // NaN never wins
          tmx = v[j];
          tmi = static_cast<int>(base) + j;
        }
      }
    });
  } else {
    for_chunks(Own{}, [&](const float v[kVec], int64_t) {
#pragma unroll
      for (int j = 0; j < kVec; ++j) tmx = fmaxf(tmx, v[j]);  // NaN never wins
    });
  }
  const float mx = block_max(tmx, redv);
  if (!(mx > -INFINITY)) {  // nothing finite: token 0, empty support
    if (tid == 0) {
      a.tokens[b] = 0;
      if (a.logprobs) a.logprobs[b] = -INFINITY;
      if (a.counts) a.counts[b] = 0;
    }
    if (a.mask)
      for (int wd = tid; wd < words; wd += kSampleThreads) a.mask[static_cast<int64_t>(b) * words + wd] = 0u;
    return;
  }
  // min_p as a key threshold: x >= max + ln(min_p).
  const float mp = a.min_p ? a.min_p[b] : 0.f;
  uint32_t key_lo = order_key(-3.402823466e38f);  // finite values only
  if (mp > 0.f) {
    uint32_t k = order_key(mx + logf(mp));
    if (k > order_key(mx)) k = order_key(mx);  // min_p above 1 still keeps the maximum
    key_lo = k > key_lo ? k : key_lo;
  }

  const int lane = tid & 63;
  bool fallback = false;
  bool listed = false;  // the LDS list holds every kept token the threshold can keep
  int n = 0;            // its length
  unsigned long long mtot = 0;  // the kept mass of the row (top_p alone)
  auto bin_of = [&](float x) {
    const float d = (mx - x) * kBinScale;  // NaN and -inf land in the open bin (and are not kept)
    return d < static_cast<float>(kBins - 1) ? static_cast<int>(d) : kBins - 1;
  };
  // Appends the kept tokens with `take` set to the list (one LDS atomic per
  // wave and slot); every lane of the wave that is still in the pass calls it.
  auto append = [&](bool take, float x, int64_t t) {
    const unsigned long long bal = __ballot(take);
    if (bal == 0ull) return;  // uniform: most slots of most passes
    const int first = __ffsll(static_cast<long long>(bal)) - 1;
    int at = 0;
    if (lane == first) at = atomicAdd(&ncand, __popcll(bal));
    at = __shfl(at, first, 64) + __builtin_amdgcn_mbcnt_hi(static_cast<uint32_t>(bal >> 32),
                                                            __builtin_amdgcn_mbcnt_lo(static_cast<uint32_t>(bal), 0u));
    if (take && at < kCand) {
      ckey[at] = order_key(x);
      cx[at] = x;
      cidx[at] = static_cast<int32_t>(t);
    }
  };
  if (want_k || want_p) {
    const bool hmass = want_p && !want_k;  // after top_k, top_p runs on the list
    for (int j = tid; j < kBins; j += kSampleThreads) {
      fcnt[j] = 0u;
      fmass[j] = 0ull;
    }
    if (tid == 0) {
      ncand = 0;
      sel_n = 0ull;
    }
    __syncthreads();

    // Capture range, in bins below the maximum, holding every token the
    // threshold can keep. top_k (k <= threads): the k largest of the threads'
    // maxima are k distinct tokens, so the row's k-th largest lies in or above
    // the bin of their k-th. top_p alone: tokens more than
    // r = ln(vocab / (1 - top_p)) + 1 below the maximum weigh at most
    // (1 - top_p) / e of the maximum's weight all together, so the mass above
    // the threshold is reached within r (the maximum's fixed-point weight is
    // exactly 2^32, whence the kept mass is at least that).
    int bcap = kBins - 1;
    if (want_k && topk <= kSampleThreads) {
      atomicAdd(&fcnt[bin_of(tmx)], 1u);
      __syncthreads();
      const unsigned long long c0 = fcnt[2 * tid], c1 = fcnt[2 * tid + 1];
      unsigned long long ctot;
      const unsigned long long cex = block_exscan_u64(c0 + c1, red64, ctot);
      const unsigned long long kk = static_cast<unsigned long long>(topk);
      if (tid == 0) sel_bin = kBins - 1;
      __syncthreads();
      if (cex < kk && kk <= cex + c0)
        sel_bin = 2 * tid;
      else if (cex + c0 < kk && kk <= cex + c0 + c1)
        sel_bin = 2 * tid + 1;
      fcnt[2 * tid] = 0u;
      fcnt[2 * tid + 1] = 0u;
      __syncthreads();
      bcap = sel_bin;
    } else if (!want_k) {
      const double tail = 1.0 - static_cast<double>(tp);
      if (tail > 1e-6) {
        const double r = (log(static_cast<double>(vocab) / tail) + 1.0) * static_cast<double>(kBinScale);
        bcap = r < static_cast<double>(kBins - 1) ? static_cast<int>(ceil(r)) : kBins - 1;
      }
    }

    // Capture pass: the kept tokens within the range go to the list and to
    // the threshold's histogram (for a list that overflows); the kept mass
    // sums over the whole row (a token kMassBins or more below the maximum
    // weighs under one fixed-point unit: exactly 0).
    const bool captured = bcap < kBins - 1;
    if (captured) {
      unsigned long long tmass = 0;
      // The bin tests as distance compares: with d = (mx - x) * kBinScale as
      // bin_of forms it (d >= 0: x <= mx; NaN and -inf fail every compare),
      // bin <= bcap <=> d < bcap + 1 and bin < kMassBins <=> d < kMassBins
      // (bcap + 1 <= kBins - 1). The key test is one float compare when the
      // threshold is a negative float (NEG; see the fast final loop below).
      // The bin and the key are formed only for the few tokens taken.
      const float bcap1 = static_cast<float>(bcap + 1);
      const float thr = __uint_as_float(~key_lo);  // with NEG: the keep threshold as a float
      // (one instance per mass flag and key test: a select on them would do both)
      auto capture = [&](auto with_mass, auto neg) {
        constexpr bool M = decltype(with_mass)::value;
        constexpr bool NEG = decltype(neg)::value;
        for_chunks(Own{}, [&](const float v[kVec], int64_t base) {
#pragma unroll
          for (int j = 0; j < kVec; ++j) {
            const float d = (mx - v[j]) * kBinScale;
            const bool kept = NEG ? v[j] >= thr : order_key(v[j]) >= key_lo;
            unsigned long long m = 0;
            if constexpr (M) {
              if (kept && d < static_cast<float>(kMassBins)) m = fixed_mass(v[j], mx);
              tmass += m;
            }
            const bool take = kept && d < bcap1;
            if (take) {
              const int bn = static_cast<int>(d);
              atomicAdd(&fcnt[bn], 1u);
              if constexpr (M) atomicAdd(&fmass[bn], m);
            }
            append(take, v[j], base + j);
          }
        });
      };
      const bool neg_thr = key_lo < 0x80000000u;
      if (hmass) {
        if (neg_thr)
          capture(std::true_type{}, std::true_type{});
        else
          capture(std::true_type{}, std::false_type{});
      } else {
        if (neg_thr)
          capture(std::false_type{}, std::true_type{});
        else
          capture(std::false_type{}, std::false_type{});
      }
      if (hmass) {
        const unsigned long long wm = wave_sum_u64(tmass);
        if (lane == 0) atomicAdd(&sel_n, wm);
      }
      __syncthreads();
      n = ncand;
      listed = n <= kCand;
      mtot = sel_n;
      __syncthreads();
    }

    if (!listed) {
      // The threshold's bin from the histogram -- the capture pass's, which
      // holds the threshold, or one pass over the whole row -- then a
      // compaction pass: every kept token at or above that bin.
      if (tid == 0) ncand = 0;
      if (!captured) {
        uint32_t tcnt = 0;
        unsigned long long tmass = 0;  // this thread's share of the open bin
        for_chunks(Own{}, [&](const float v[kVec], int64_t) {
#pragma unroll
          for (int j = 0; j < kVec; ++j) {
            if (order_key(v[j]) < key_lo) continue;
            const int bn = bin_of(v[j]);
            const unsigned long long m = hmass ? fixed_mass(v[j], mx) : 0ull;
            if (bn == kBins - 1) {
              ++tcnt;
              tmass += m;
            } else {
              atomicAdd(&fcnt[bn], 1u);
              if (hmass) atomicAdd(&fmass[bn], m);
            }
          }
        });
        const unsigned long long wc = wave_sum_u64(tcnt), wm = wave_sum_u64(tmass);
        if (lane == 0) {
          atomicAdd(&fcnt[kBins - 1], static_cast<uint32_t>(wc));
          if (hmass) atomicAdd(&fmass[kBins - 1], wm);
        }
      }
      __syncthreads();
      // Threshold bin from scans over the bins in value order (bin 0 = nearest the max).
      const unsigned long long c0 = fcnt[2 * tid], c1 = fcnt[2 * tid + 1];
      unsigned long long ctot;
      const unsigned long long cex = block_exscan_u64(c0 + c1, red64, ctot);
      unsigned long long m0 = 0, m1 = 0, mex = 0;
      if (hmass) {
        m0 = fmass[2 * tid];
        m1 = fmass[2 * tid + 1];
        unsigned long long htot;
        mex = block_exscan_u64(m0 + m1, red64, htot);
        if (!captured) mtot = htot;  // else the capture pass summed the whole row
      }
      if (tid == 0) sel_bin = -1;
      __syncthreads();
      if (want_k) {
        const unsigned long long kk = static_cast<unsigned long long>(topk);
        if (ctot >= kk) {  // else fewer than k kept tokens: the full-row path keeps them all
          if (cex < kk && kk <= cex + c0) {
            sel_bin = 2 * tid;
            sel_n = cex + c0;
          } else if (cex + c0 < kk && kk <= cex + c0 + c1) {
            sel_bin = 2 * tid + 1;
            sel_n = cex + c0 + c1;
          }
        }
      } else {
        const unsigned long long target =
            static_cast<unsigned long long>(ceil(static_cast<double>(tp) * static_cast<double>(mtot)));
        if (mex < target && target <= mex + m0) {
          sel_bin = 2 * tid;
          sel_n = cex + c0;
        } else if (mex + m0 < target && target <= mex + m0 + m1) {
          sel_bin = 2 * tid + 1;
          sel_n = cex + c0 + c1;
        }
      }
      __syncthreads();
      const int tb = sel_bin;
      const unsigned long long n_list = sel_n;
      fallback = tb < 0 || tb == kBins - 1 || n_list > static_cast<unsigned long long>(kCand);
      if (!fallback) {
        for_chunks(Own{}, [&](const float v[kVec], int64_t base) {
#pragma unroll
          for (int j = 0; j < kVec; ++j) append(order_key(v[j]) >= key_lo && bin_of(v[j]) <= tb, v[j], base + j);
        });
        __syncthreads();
        n = ncand < kCand ? ncand : kCand;  // == n_list
        listed = true;
      }
    }

    if (listed) {
      // top_k on the list: the k-th largest key (ties kept). Every list entry
      // is kept; a list shorter than k holds every kept token, all of which stay.
      if (want_k && n >= topk) {
        uint32_t prefix = 0, pmask = 0;
        unsigned long long remaining = static_cast<unsigned long long>(topk);
        for (int shift = 24; shift >= 0; shift -= 8) {
          for (int j = tid; j < 256; j += kSampleThreads) hist[j] = 0ull;
          __syncthreads();
          for (int i = tid; i < n; i += kSampleThreads) {
            const uint32_t k = ckey[i];
            if ((k & pmask) == prefix) atomicAdd(&hist[(k >> shift) & 255u], 1ull);
          }
          __syncthreads();
          find_from_top(hist, 0ull, remaining, &sel_prefix, &sel_above);  // found: the list holds >= k keys
          __syncthreads();
          remaining -= sel_above;
          prefix |= sel_prefix << shift;
          pmask |= 255u << shift;
          __syncthreads();
        }
        if (prefix > key_lo) key_lo = prefix;
      }
      // top_p on the list. After top_k the list holds every kept token (its
      // keys >= key_lo), so the kept mass sums over it; top_p alone keeps the
      // whole row's mass.
      if (want_p) {
        unsigned long long total = mtot;
        if (want_k) {
          unsigned long long part = 0;
          for (int i = tid; i < n; i += kSampleThreads)
            if (ckey[i] >= key_lo) part += fixed_mass(cx[i], mx);
          (void)block_exscan_u64(part, red64, total);
        }
        const unsigned long long target =
            static_cast<unsigned long long>(ceil(static_cast<double>(tp) * static_cast<double>(total)));
        uint32_t prefix = 0, pmask = 0;
        unsigned long long above = 0;
        for (int shift = 24; shift >= 0; shift -= 8) {
          for (int j = tid; j < 256; j += kSampleThreads) hist[j] = 0ull;
          __syncthreads();
          for (int i = tid; i < n; i += kSampleThreads) {
            const uint32_t k = ckey[i];
            if (k >= key_lo && (k & pmask) == prefix) atomicAdd(&hist[(k >> shift) & 255u], fixed_mass(cx[i], mx));
          }
          __syncthreads();
          find_from_top(hist, above, target, &sel_prefix, &sel_above);
          __syncthreads();
          prefix |= sel_prefix << shift;
          above = sel_above;
          pmask |= 255u << shift;
          __syncthreads();
        }
        if (prefix > key_lo) key_lo = prefix;
      }
    }
  }

  // top_k over the whole row: radix select of the k-th largest kept key.
  if (fallback && want_k) {
    uint32_t prefix = 0, pmask = 0;
    unsigned long long remaining = static_cast<unsigned long long>(topk);
    bool enough = true;
    for (int shift = 24; shift >= 0; shift -= 8) {
      for (int j = tid; j < 256; j += kSampleThreads) hist[j] = 0ull;
      __syncthreads();
      for (int64_t base = static_cast<int64_t>(tid) * kVec; base < vocab; base += step8) {
        float v[kVec];
        x8(v, base);
#pragma unroll
        for (int j = 0; j < kVec; ++j) {
          const uint32_t k = order_key(v[j]);
          if (k >= key_lo && (k & pmask) == prefix) atomicAdd(&hist[(k >> shift) & 255u], 1ull);
        }
      }
      __syncthreads();
      find_from_top(hist, 0ull, remaining, &sel_prefix, &sel_above);  // -1: fewer than k kept tokens
      __syncthreads();
      const int bin = static_cast<int>(sel_prefix);
      const unsigned long long above = sel_above;
      __syncthreads();
      if (bin < 0) {
        enough = false;
        break;
      }
      remaining -= above;
      prefix |= static_cast<uint32_t>(bin) << shift;
      pmask |= 255u << shift;
    }
    if (enough && prefix > key_lo) key_lo = prefix;
  }

  // top_p over the whole row: radix select over fixed-point mass
  // w_i = exp(x_i - max) * 2^32.
  if (fallback && want_p) {
    unsigned long long total = 0;
    {
      // total kept mass (integer: exact, order-independent)
      for (int j = tid; j < 256; j += kSampleThreads) hist[j] = 0ull;
      __syncthreads();
      unsigned long long part = 0;
      for (int64_t base = static_cast<int64_t>(tid) * kVec; base < vocab; base += step8) {
        float v[kVec];
        x8(v, base);
#pragma unroll
        for (int j = 0; j < kVec; ++j)
          if (order_key(v[j]) >= key_lo) part += static_cast<unsigned long long>(expf(v[j] - mx) * 4294967296.f);
      }
      atomicAdd(&hist[0], part);
      __syncthreads();
      total = hist[0];
      __syncthreads();
    }
    const unsigned long long target =
        static_cast<unsigned long long>(ceil(static_cast<double>(tp) * static_cast<double>(total)));
    uint32_t prefix = 0, pmask = 0;
    unsigned long long above = 0;
    for (int shift = 24; shift >= 0; shift -= 8) {
      for (int j = tid; j < 256; j += kSampleThreads) hist[j] = 0ull;
      __syncthreads();
      for (int64_t base = static_cast<int64_t>(tid) * kVec; base < vocab; base += step8) {
        float v[kVec];
        x8(v, base);
#pragma unroll
        for (int j = 0; j < kVec; ++j) {
          const uint32_t k = order_key(v[j]);
          if (k >= key_lo && (k & pmask) == prefix)
            atomicAdd(&hist[(k >> shift) & 255u], static_cast<unsigned long long>(expf(v[j] - mx) * 4294967296.f));
        }
      }
      __syncthreads();
      find_from_top(hist, above, target, &sel_prefix, &sel_above);  // target <= total: always found
      __syncthreads();
      prefix |= sel_prefix << shift;
      above = sel_above;
      pmask |= 255u << shift;
      __syncthreads();
    }
    if (prefix > key_lo) key_lo = prefix;
  }

  const uint64_t stream = mix64((a.seeds ? a.seeds[b] : 0ull) + static_cast<uint64_t>(a.step) * 0x9E3779B97F4A7C15ull);
  float best = -INFINITY;
  int64_t bi = 0x7fffffffffffffffll;
  int cnt = 0;
  float lz;  // ln of the kept mass, in units of the maximum's weight
  // The race's bound, raised by each thread's own draws as they come: a
  // token below bound - kScoreReach cannot reach it, so its draw is skipped.
  // It starts from the maximum's least possible score (ln E <= 2.812; the
  // maximum is always kept), or from the best score of the threads' kept
  // maxima where pass 1 kept them.
  float lim = -INFINITY;
  if (!greedy) {
    lim = mx - 2.9f;
    if (track) {
      const float s0 = order_key(tmx) >= key_lo ? tmx - log_exp_variate(stream, tmi) : -INFINITY;
      lim = fmaxf(lim, block_max(s0, redv));
    }
    lim -= kScoreReach;
  }
  auto race = [&](float x, int64_t t) {
    if (greedy) {
      arg_better(best, bi, x, t);
    } else if (x >= lim) {
      arg_better(best, bi, x - log_exp_variate(stream, t), t);
      lim = fmaxf(lim, best - kScoreReach);
    }
  };
  if (listed && words <= kMaskWords) {
    // Final step on the list, which holds every kept token: the kept mass in
    // fixed point (exact, so independent of the list's order), the draw, the
    // mask (assembled in LDS) and the support size.
    if (a.mask)
      for (int wd = tid; wd < words; wd += kSampleThreads) mbits[wd] = 0u;
    __syncthreads();
    unsigned long long zf = 0;
    for (int i = tid; i < n; i += kSampleThreads) {
      if (ckey[i] < key_lo) continue;
      const float x = cx[i];
      const int64_t t = cidx[i];
      zf += fixed_mass(x, mx);
      ++cnt;
      race(x, t);
      if (a.mask) atomicOr(&mbits[t >> 5], 1u << (t & 31));
    }
    unsigned long long ztot;
    (void)block_exscan_u64(zf, red64, ztot);  // its barriers also complete the mask
    lz = static_cast<float>(log(static_cast<double>(ztot)) - 22.180709777918249);  // - ln 2^32
    if (a.mask)
      for (int wd = tid; wd < words; wd += kSampleThreads) a.mask[static_cast<int64_t>(b) * words + wd] = mbits[wd];
  } else if (!greedy && key_lo < 0x80000000u) {
    // Final pass over the row, fast loop: the keep threshold is a negative
    // float t (the RL defaults keep every finite token, and most min_p rows
    // land here). Keys order negative floats (-0 included) as the floats do
    // and every non-negative float above them, and NaN fails both compares as
    // it fails the key test, so: kept <=> v >= t, and a race candidate (kept
    // and v >= lim) <=> v >= max(t, lim), one float compare each. The draws go
    // through a queue per wave, made 64 at a time after every fourth token
    // slot (lim only moves there): the token slots in between carry no draw
    // code, and the mass, counts and mask come out as in the general loop.
    const float thr = __uint_as_float(~key_lo);
    float clim = fmaxf(thr, lim);
    float *qx = &fq_x[tid >> 6][0];
    int32_t *qt = &fq_t[tid >> 6][0];
    int qn = 0;  // wave-uniform
    float z = 0.f;
    for_chunks(Every{}, [&](const float v[kVec], int64_t base) {
      uint32_t bits = 0;
#pragma unroll
      for (int j = 0; j < kVec; ++j) {
        const bool kept = v[j] >= thr;
        if (__ballot(kept) != 0ull) {  // uniform: something kept in this slot of the wave
          if (kept) {
            bits |= 1u << j;
            z += __expf(v[j] - mx);
          }
          const bool c = v[j] >= clim;
          const unsigned long long bal = __ballot(c);
          if (bal != 0ull) {  // uniform
            if (c) {
              const int at = qn + static_cast<int>(__builtin_amdgcn_mbcnt_hi(
                                      static_cast<uint32_t>(bal >> 32), __builtin_amdgcn_mbcnt_lo(static_cast<uint32_t>(bal), 0u)));
              qx[at] = v[j];
              qt[at] = static_cast<int32_t>(base) + j;
            }
            qn += __popcll(bal);
          }
        }
        if ((j & 3) == 3) {
          while (qn >= 64) {  // uniform
            qn -= 64;
            race(qx[qn + lane], qt[qn + lane]);
          }
          clim = fmaxf(thr, lim);
        }
      }
      cnt += __popc(bits);
      if (a.mask) {
        // four consecutive lanes hold the 32 bits of one mask word
        const uint32_t b1 = __shfl_down(bits, 1, 64), b2 = __shfl_down(bits, 2, 64), b3 = __shfl_down(bits, 3, 64);
        const int64_t wd = base >> 5;
        if ((tid & 3) == 0 && wd < words)
          a.mask[static_cast<int64_t>(b) * words + wd] = bits | (b1 << 8) | (b2 << 16) | (b3 << 24);
      }
    });
    if (lane < qn) race(qx[lane], qt[lane]);
    lz = logf(block_sum(z, redv));
  } else {
    // Final pass over the row. Every lane makes the same calls (chunks past
    // the end are all -inf, kept nowhere): the mask words below are assembled
    // across lanes.
    // The draws go through a queue per wave (in the top_p mass bins, idle by
    // now) and are made 64 at a time, one per lane: a draw taken in place would
    // hold the whole wave whenever any one lane needs it.
    float *qx = reinterpret_cast<float *>(fmass) + (tid >> 6) * (2 * kQueue);
    int32_t *qt = reinterpret_cast<int32_t *>(qx + kQueue);
    int qn = 0;  // wave-uniform
    float z = 0.f;
    for_chunks(Every{}, [&](const float v[kVec], int64_t base) {
      uint32_t bits = 0;
#pragma unroll
      for (int j = 0; j < kVec; ++j) {
        const bool kept = order_key(v[j]) >= key_lo;
        if (__ballot(kept) == 0ull) continue;  // uniform: nothing kept in this slot of the wave
        if (kept) {
          bits |= 1u << j;
          z += __expf(v[j] - mx);  // (relative error ~1e-6 at 100 below the maximum)
        }
        if (greedy) {
          if (kept) arg_better(best, bi, v[j], base + j);
          continue;
        }
        const bool c = kept && v[j] >= lim;
        const unsigned long long bal = __ballot(c);
        if (bal == 0ull) continue;  // uniform
        if (c) {
          const int at = qn + static_cast<int>(__builtin_amdgcn_mbcnt_hi(
                                  static_cast<uint32_t>(bal >> 32), __builtin_amdgcn_mbcnt_lo(static_cast<uint32_t>(bal), 0u)));
          qx[at] = v[j];
          qt[at] = static_cast<int32_t>(base) + j;
        }
        qn += __popcll(bal);  // < 64 before, < 128 after
        if (qn >= 64) {
          qn -= 64;
          race(qx[qn + lane], qt[qn + lane]);
        }
      }
      cnt += __popc(bits);
      if (a.mask) {
        // four consecutive lanes hold the 32 bits of one mask word
        const uint32_t b1 = __shfl_down(bits, 1, 64), b2 = __shfl_down(bits, 2, 64), b3 = __shfl_down(bits, 3, 64);
        const int64_t wd = base >> 5;
        if ((tid & 3) == 0 && wd < words)
          a.mask[static_cast<int64_t>(b) * words + wd] = bits | (b1 << 8) | (b2 << 16) | (b3 << 24);
      }
    });
    if (lane < qn) race(qx[lane], qt[lane]);
    lz = logf(block_sum(z, redv));
  }
  block_argmax(best, bi, redv, redi);
  const float c = block_sum(static_cast<float>(cnt), redv);
  if (tid == 0) {
    a.tokens[b] = bi;
    if (a.logprobs) a.logprobs[b] = (x_of(bi) - mx) - lz;
    if (a.counts) a.counts[b] = static_cast<int32_t>(c);
  }
}

}  // namespace wkv

using namespace wkv;

extern "C" int wkv_sample(const void *logits, int32_t logits_dtype, int64_t row_stride, int32_t batch, int32_t vocab,
                          const float *temperature, const int32_t *top_k, const float *top_p, const float *min_p,
                          const float *repetition_penalty, const uint32_t *seen_tokens, const uint64_t *seeds,
                          int64_t step, int64_t *out_tokens, float *out_logprobs, uint32_t *out_mask,
                          int32_t *out_counts, void *stream) {
  WKV_CHECK_ARG(batch >= 0, "batch must be >= 0");
  if (batch == 0) return WKV_OK;
  WKV_CHECK_ARG(vocab > 0 && vocab < (1 << 24), "vocab must be in [1, 2^24) (got %d)", vocab);
  WKV_CHECK_ARG(logits != nullptr && out_tokens != nullptr, "logits / out_tokens is NULL");
  WKV_CHECK_ARG(logits_dtype == 0 || logits_dtype == 1, "logits_dtype must be 0 (fp32) or 1 (bf16)");
  WKV_CHECK_ARG(row_stride >= vocab, "row_stride %lld < vocab %d", (long long)row_stride, vocab);
  SampleArgs a{temperature, top_k, top_p, min_p, repetition_penalty, seen_tokens, seeds, step,
               out_tokens, out_logprobs, out_mask, out_counts};
  auto s = static_cast<hipStream_t>(stream);
  if (logits_dtype == 0)
    sample_kernel<float><<<batch, kSampleThreads, 0, s>>>(static_cast<const float *>(logits), row_stride, vocab, a);
  else
    sample_kernel<uint16_t><<<batch, kSampleThreads, 0, s>>>(static_cast<const uint16_t *>(logits), row_stride,
                                                              vocab, a);
  WKV_CHECK_LAUNCH("sample");
  return WKV_OK;
}
