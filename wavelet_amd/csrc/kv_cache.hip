// Slot-mapped append (bf16, fp8-e4m3 with per-(block, head) scales, MLA latent),
// block-table gather and block copy for the paged KV cache.
//
// Cache layout (x = 16 / element bytes):
//   K [NB, H, D/x, BS, x]   V [NB, H, D, BS]   scales [NB, H]   MLA [NB, BS, W]
// These kernels move at most a few hundred KB per decode step; they are
// launch-latency bound, so they favour one simple pass with 16-byte vector
// accesses on the contiguous side over anything cleverer.
#include "wkv_common.h"
#include "kv_append_dev.h"

namespace wkv {

// ---------------------------------------------------------------------------
// bf16 append: one thread per (token, head, 8-element chunk).
template <int D>
__global__ __launch_bounds__(256) void append_bf16_kernel(uint16_t *__restrict__ kc, uint16_t *__restrict__ vc,
                                                          const uint16_t *__restrict__ key, int64_t kst,
                                                          int64_t ksh, const uint16_t *__restrict__ val,
                                                          int64_t vst, int64_t vsh,
                                                          const int64_t *__restrict__ slots, int64_t T, int H,
                                                          int BS, int64_t NB) {
  constexpr int C = D / 8;
  int64_t idx = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  if (idx >= T * H * C) return;
  const int c = static_cast<int>(idx % C);
  const int64_t th = idx / C;
  const int h = static_cast<int>(th % H);
  const int64_t t = th / H;
  const int64_t slot = slots[t];
  if (slot < 0) return;
  const int64_t blk = slot / BS;
  const int off = static_cast<int>(slot % BS);
  if (blk >= NB) return;  // out-of-range ids are never written (no fault)
  const u32x4 kv = *reinterpret_cast<const u32x4 *>(key + t * kst + h * ksh + c * 8);
  *reinterpret_cast<u32x4 *>(kc + (((blk * H + h) * C + c) * BS + off) * 8) = kv;
  const u32x4 vv = *reinterpret_cast<const u32x4 *>(val + t * vst + h * vsh + c * 8);
  uint16_t *vdst = vc + ((blk * H + h) * D + c * 8) * BS + off;
#pragma unroll
  for (int j = 0; j < 8; ++j) vdst[j * BS] = static_cast<uint16_t>(vv[j >> 1] >> (16 * (j & 1)));
}

// bf16 append of many tokens (a prompt): workgroup = 64 consecutive tokens x
// one head, rows read whole (16 bytes per thread, coalesced). K ([.., C, BS,
// 8]: a chunk's pieces of a block's tokens are contiguous) is stored from the
// registers as loaded: 16-byte pieces, 64-byte runs per store instruction
// where the slots are consecutive. V ([.., D, BS]: a row of the cache holds
// one d of a block's tokens) goes through LDS: the window's tokens go in
// groups of 8; a group whose 8 slots are consecutive and start 8-aligned in
// one block (every group of a prompt that starts on an 8-token boundary) is
// written as one 16-byte piece per d row, lanes along (d, group pair) so that
// a store instruction covers 32 whole 32-byte rows of a 16-token block; other
// groups (scattered slots, skipped tokens, a sequence starting mid-group, the
// ragged end) fall back to 2-byte stores per token. 17 KB of LDS at d=128:
// the whole prompt's workgroups are resident at once.
constexpr int kBulkTokens = 64;
constexpr int64_t kBulkMinTokens = 256;  // below this (a decode step's tokens) the per-chunk kernel spreads wider

template <int D>
__global__ __launch_bounds__(256) void append_bf16_bulk_kernel(uint16_t *__restrict__ kc, uint16_t *__restrict__ vc,
                                                               const uint16_t *__restrict__ key, int64_t kst,
                                                               int64_t ksh, const uint16_t *__restrict__ val,
                                                               int64_t vst, int64_t vsh,
                                                               const int64_t *__restrict__ slots, int64_t T, int H,
                                                               int BS, int64_t NB) {
  constexpr int C = D / 8;
  constexpr int RP = D * 2 + 8;        // V pitch in bytes per token row: rows 8 apart land 16 banks apart
  constexpr int NG = kBulkTokens / 8;  // token groups of the window
  __shared__ __attribute__((aligned(16))) uint8_t lv[kBulkTokens * RP];
  __shared__ int64_t gslot[NG];  // a group's first slot when its 8 slots are one aligned run, else -1
  const int64_t t0 = static_cast<int64_t>(blockIdx.x) * kBulkTokens;
  const int h = blockIdx.y;
  const int tid = threadIdx.x;
  // load: thread -> (token tid / C + k * (256 / C), chunk tid % C)
  {
    const int c = tid % C;
#pragma unroll
    for (int k = 0; k < kBulkTokens * C / 256; ++k) {
      const int t = tid / C + k * (256 / C);
      if (t0 + t < T) {
        const u32x4 kv = *reinterpret_cast<const u32x4 *>(key + (t0 + t) * kst + h * ksh + c * 8);
        const u32x4 vv = *reinterpret_cast<const u32x4 *>(val + (t0 + t) * vst + h * vsh + c * 8);
        const int64_t slot = slots[t0 + t];
        const int64_t blk = slot / BS;
        if (slot >= 0 && blk < NB)
          *reinterpret_cast<u32x4 *>(kc + (((blk * H + h) * C + c) * BS + slot % BS) * 8) = kv;
        uint32_t *w = reinterpret_cast<uint32_t *>(&lv[t * RP + c * 16]);
#pragma unroll
        for (int j = 0; j < 4; ++j) w[j] = vv[j];
      }
    }
    if (tid < NG) {
      const int64_t ta = t0 + 8 * tid;
      int64_t first = -1;
      if (ta + 7 < T && BS % 8 == 0) {
        first = slots[ta];
        const bool start = first >= 0 && first / BS < NB && (first % BS) % 8 == 0;
        bool run = start;
#pragma unroll
        for (int j = 1; j < 8; ++j) run = run && slots[ta + j] == first + j;
        if (!run) first = -1;
      }
      gslot[tid] = first;
    }
  }
  __syncthreads();
  // V: item i -> group pair gp = i / (2 D), d = (i / 2) % D, group 2 gp + i % 2
#pragma unroll
  for (int k = 0; k < NG * D / 256; ++k) {
    const int i = tid + 256 * k;
    const int g = 2 * (i / (2 * D)) + (i & 1);
    const int d = (i >> 1) % D;
    const int64_t first = gslot[g];
    if (first >= 0) {  // one aligned run: 8 tokens of row d in one 16-byte piece
      uint32_t w[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const uint32_t lo = *reinterpret_cast<const uint16_t *>(&lv[(8 * g + 2 * j) * RP + 2 * d]);
        const uint32_t hi = *reinterpret_cast<const uint16_t *>(&lv[(8 * g + 2 * j + 1) * RP + 2 * d]);
        w[j] = lo | (hi << 16);
      }
      const int64_t blk = first / BS;
      const int off = static_cast<int>(first % BS);
      *reinterpret_cast<u32x4 *>(vc + ((blk * H + h) * D + d) * BS + off) = u32x4{w[0], w[1], w[2], w[3]};
    } else {
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const int t = 8 * g + j;
        if (t0 + t >= T) break;
        const int64_t slot = slots[t0 + t];
        const int64_t blk = slot / BS;
        if (slot < 0 || blk >= NB) continue;
        vc[((blk * H + h) * D + d) * BS + slot % BS] = *reinterpret_cast<const uint16_t *>(&lv[t * RP + 2 * d]);
      }
    }
  }
}

template <int D>
__global__ __launch_bounds__(64) void append_fp8_kernel(uint8_t *__restrict__ kc, uint8_t *__restrict__ vc,
                                                        float *__restrict__ ks, float *__restrict__ vs,
                                                        const uint16_t *__restrict__ key, int64_t kst,
                                                        int64_t ksh, const uint16_t *__restrict__ val,
                                                        int64_t vst, int64_t vsh,
                                                        const int64_t *__restrict__ slots, int64_t T, int H,
                                                        int BS, int64_t NB) {
  const int64_t t = blockIdx.x;
  const int h = blockIdx.y;
  const int64_t slot = slots[t];
  if (slot < 0) return;
  const int64_t blk = slot / BS;
  if (blk >= NB) return;
  if (t > 0) {
    const int64_t prev = slots[t - 1];
    if (prev >= 0 && prev / BS == blk) return;  // not the first token of its run
  }
  int r = 1;
  while (t + r < T) {
    const int64_t nx = slots[t + r];
    if (nx < 0 || nx / BS != blk) break;
    ++r;
  }
  const int first = static_cast<int>(slot % BS);
  fp8_append_one<D, false>(kc, ks, key, kst, ksh, slots, t, r, blk, first, h, H, BS);
  fp8_append_one<D, true>(vc, vs, val, vst, vsh, slots, t, r, blk, first, h, H, BS);
}

// Bulk fp8 append (calls of 64 tokens or more): one workgroup of NW waves per
// (64-token window of the call, KV head). Its waves find the runs that start
// in the window and their lengths from ballots over the blocks of this
// window's and the next window's tokens (a run lies in one block, so with
// blocks of at most 64 tokens it ends within the next window); wave w appends
// the window's runs w, w + NW, ... -- K and V, with the same scale rule; a run
// that reaches past the window is still this window's. Runs are independent (a
// block is in at most one run of a call), so the waves need no
// synchronisation. A decode-shaped call (one token per sequence: 64 one-token
// runs per window) takes NW = 8: 256 tokens x 4 heads 58 us against 318 with
// one wave per window; a prompt (four 16-token blocks per window) NW = 4, one
// block per wave: 16,384 tokens x 8 heads 23.5 us (one wave per window 23.9,
// eight 30.1; kernel traces). A whole fresh 16-token block (the prompt case) takes
// fp8_append_block16: 16-byte loads and stores, hardware code conversion.
// Other runs: fp8_append_run_vec.
constexpr int kFp8BulkMinTokens = 64;
// Calls of this many tokens or more are taken as prompts (NW = 4), smaller
// ones as decode-shaped (NW = 8).
constexpr int64_t kFp8PromptTokens = 4096;
template <int D, int NW>
__global__ __launch_bounds__(64 * NW) void append_fp8_bulk_kernel(uint8_t *__restrict__ kc, uint8_t *__restrict__ vc,
                                                             float *__restrict__ ks, float *__restrict__ vs,
                                                             const uint16_t *__restrict__ key, int64_t kst,
                                                             int64_t ksh, const uint16_t *__restrict__ val,
                                                             int64_t vst, int64_t vsh,
                                                             const int64_t *__restrict__ slots, int64_t T, int H,
                                                             int BS, int64_t NB) {
  const int64_t t0 = static_cast<int64_t>(blockIdx.x) * 64;
  const int h = blockIdx.y;
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x >> 6));
  // block of token `tok` of the call (-1: past the call, a skipped slot or an
  // unmapped block); block ids are below 2^31 (num_blocks * num_kv_heads is)
  auto block_of = [&](int64_t tok) -> int {
    if (tok < 0 || tok >= T) return -1;
    const int64_t slot = slots[tok];
    return (slot >= 0 && slot / BS < NB) ? static_cast<int>(slot / BS) : -1;
  };
  const int ba = block_of(t0 + lane);
  const int bb = BS <= 64 ? block_of(t0 + 64 + lane) : -1;
  const int bp = block_of(t0 - 1);  // the token before the window
  // token j continues a run when it and token j - 1 lie in one block
  int pa = __shfl_up(ba, 1, 64), pb = __shfl_up(bb, 1, 64);
  const int last_a = __shfl(ba, 63, 64);
  if (lane == 0) {
    pa = bp;
    pb = last_a;
  }
  const bool start = ba >= 0 && pa != ba;
  uint64_t starts = __ballot(start);
  const uint64_t ca = __ballot(ba >= 0 && pa == ba), cb = __ballot(bb >= 0 && pb == bb);
  for (int k = 0; starts != 0ull; ++k) {  // uniform
    const int i = __ffsll(static_cast<long long>(starts)) - 1;
    starts &= starts - 1ull;
    if (k % NW != wave) continue;  // another wave's run
    const int64_t t = t0 + i;
    const int64_t slot = slots[t];
    const int64_t blk = slot / BS;
    int r;
    if (BS <= 64) {
      // 1 + the continuation bits after i: through the window, then into the next
      const uint64_t x = i < 63 ? (ca >> (i + 1)) : 0ull;
      const int n1 = __builtin_ctzll(~x);
      const int n2 = (n1 == 63 - i) ? (~cb == 0ull ? 64 : __builtin_ctzll(~cb)) : 0;
      r = 1 + n1 + n2;
    } else {
      r = 1;
      while (t + r < T) {
        const int64_t nx = slots[t + r];
        if (nx < 0 || nx / BS != blk) break;
        ++r;
      }
    }
    const int first = static_cast<int>(slot % BS);
    // a whole block at offsets 0..15 in token order (a slot mapping may order a
    // block's tokens otherwise: then the general path)
    if (BS == 16 && first == 0 && r == 16 && __all(slots[t + (lane & 15)] == slot + (lane & 15)) &&
        fp8_append_block16<D>(kc, vc, ks, vs, key, kst, ksh, val, vst, vsh, t, blk, h, H))
      continue;
    fp8_append_run_vec<D, false>(kc, ks, key, kst, ksh, slots, t, r, blk, first, h, H, BS);
    fp8_append_run_vec<D, true>(vc, vs, val, vst, vsh, slots, t, r, blk, first, h, H, BS);
  }
}

// ---------------------------------------------------------------------------
// Gather: one workgroup per (sequence, block index). Reads follow the
// physical order (coalesced); writes are 16-byte pieces of the contiguous
// [tokens, H, D] output.
template <int D, bool FP8, bool DEQUANT>
__global__ __launch_bounds__(256) void gather_kernel(const uint8_t *__restrict__ kc, const uint8_t *__restrict__ vc,
                                                     const float *__restrict__ ks, const float *__restrict__ vs,
                                                     const int32_t *__restrict__ bt, int64_t bt_stride, int Mb,
                                                     const int32_t *__restrict__ seq_lens,
                                                     const int64_t *__restrict__ cu, uint8_t *__restrict__ out_k,
                                                     uint8_t *__restrict__ out_v, int H, int BS, int64_t NB) {
  constexpr int ESZ = FP8 ? 1 : 2;        // stored element bytes
  constexpr int OSZ = DEQUANT ? 2 : ESZ;  // output element bytes
  constexpr int X = 16 / ESZ;             // elements per 16-byte K chunk
  constexpr int C = D / X;
  const int i = blockIdx.y, j = blockIdx.x;
  int L = seq_lens[i];
  L = L < Mb * BS ? L : Mb * BS;
  if (L <= 0 || j * BS >= L) return;
  const int64_t blk = bt[i * bt_stride + j];
  if (blk < 0 || blk >= NB) return;
  const int ntok = (L - j * BS) < BS ? (L - j * BS) : BS;
  const int64_t tok0 = cu[i] + static_cast<int64_t>(j) * BS;

  // K: work item = one 16-byte chunk (X elements of one token, one head).
  for (int w = threadIdx.x; w < H * C * ntok; w += 256) {
    const int o = w % ntok, hc = w / ntok, c = hc % C, h = hc / C;
    const u32x4 raw = *reinterpret_cast<const u32x4 *>(kc + ((((blk * H + h) * C + c) * BS + o) * 16));
    uint8_t *dst = out_k + (((tok0 + o) * H + h) * D + c * X) * OSZ;
    if constexpr (!DEQUANT) {
      *reinterpret_cast<u32x4 *>(dst) = raw;
    } else {
      const float s = ks[blk * H + h];
      u32x4 lo, hi;
#pragma unroll
      for (int q = 0; q < 16; q += 2) {
        const uint32_t b0 = (raw[q >> 2] >> (8 * (q & 3))) & 0xffu;
        const uint32_t b1 = (raw[q >> 2] >> (8 * ((q & 3) + 1))) & 0xffu;
        const uint32_t pk = f32_to_bf16_bits(e4m3_decode(b0) * s) | (f32_to_bf16_bits(e4m3_decode(b1) * s) << 16);
        if (q < 8) lo[q >> 1] = pk; else hi[(q - 8) >> 1] = pk;
      }
      reinterpret_cast<u32x4 *>(dst)[0] = lo;
      reinterpret_cast<u32x4 *>(dst)[1] = hi;
    }
  }
  // V: work item = 8 consecutive d of one token and head (stride BS in the cache).
  for (int w = threadIdx.x; w < H * (D / 8) * ntok; w += 256) {
    const int o = w % ntok, hg = w / ntok, g = hg % (D / 8), h = hg / (D / 8);
    const int64_t base = ((blk * H + h) * D + g * 8) * BS + o;
    uint8_t *dst = out_v + (((tok0 + o) * H + h) * D + g * 8) * OSZ;
    if constexpr (!FP8) {
      const uint16_t *src = reinterpret_cast<const uint16_t *>(vc);
      u32x4 pk;
#pragma unroll
      for (int q = 0; q < 4; ++q)
        pk[q] = static_cast<uint32_t>(src[base + (2 * q) * BS]) | (static_cast<uint32_t>(src[base + (2 * q + 1) * BS]) << 16);
      *reinterpret_cast<u32x4 *>(dst) = pk;
    } else if constexpr (!DEQUANT) {
      u32x2 pk;
#pragma unroll
      for (int q = 0; q < 2; ++q) {
        uint32_t wv = 0;
#pragma unroll
        for (int b = 0; b < 4; ++b) wv |= static_cast<uint32_t>(vc[base + (4 * q + b) * BS]) << (8 * b);
        pk[q] = wv;
      }
      *reinterpret_cast<u32x2 *>(dst) = pk;
    } else {
      const float s = vs[blk * H + h];
      u32x4 pk;
#pragma unroll
      for (int q = 0; q < 4; ++q)
        pk[q] = f32_to_bf16_bits(e4m3_decode(vc[base + (2 * q) * BS]) * s) |
                (f32_to_bf16_bits(e4m3_decode(vc[base + (2 * q + 1) * BS]) * s) << 16);
      *reinterpret_cast<u32x4 *>(dst) = pk;
    }
  }
}

// ---------------------------------------------------------------------------
// Whole-block copy (K, V, scales): one workgroup per (src, dst) pair.
__global__ __launch_bounds__(256) void copy_blocks_kernel(uint8_t *__restrict__ kc, uint8_t *__restrict__ vc,
                                                          float *__restrict__ ks, float *__restrict__ vs,
                                                          const int64_t *__restrict__ mapping, int64_t block_bytes,
                                                          int H, int64_t NB) {
  const int64_t src = mapping[2 * blockIdx.x], dst = mapping[2 * blockIdx.x + 1];
  if (src < 0 || dst < 0 || src >= NB || dst >= NB) return;
  const int64_t n16 = block_bytes / 16;
  const u32x4 *ks4 = reinterpret_cast<const u32x4 *>(kc + src * block_bytes);
  const u32x4 *vs4 = reinterpret_cast<const u32x4 *>(vc + src * block_bytes);
  u32x4 *kd4 = reinterpret_cast<u32x4 *>(kc + dst * block_bytes);
  u32x4 *vd4 = reinterpret_cast<u32x4 *>(vc + dst * block_bytes);
  for (int64_t w = threadIdx.x; w < n16; w += 256) {
    kd4[w] = ks4[w];
    vd4[w] = vs4[w];
  }
  if (ks != nullptr && threadIdx.x < H) {
    ks[dst * H + threadIdx.x] = ks[src * H + threadIdx.x];
    vs[dst * H + threadIdx.x] = vs[src * H + threadIdx.x];
  }
}

// ---------------------------------------------------------------------------
// MLA latent append: one thread per (token, 8-element chunk of the W-wide row).
__global__ __launch_bounds__(256) void mla_append_kernel(uint16_t *__restrict__ lat, const uint16_t *__restrict__ kvc,
                                                         int64_t kvc_st, const uint16_t *__restrict__ kpe,
                                                         int64_t kpe_st, const int64_t *__restrict__ slots,
                                                         int64_t T, int R, int P, int BS, int64_t NB) {
  const int W = R + P, C = W / 8;
  const int64_t idx = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  if (idx >= T * C) return;
  const int c = static_cast<int>(idx % C);
  const int64_t t = idx / C;
  const int64_t slot = slots[t];
  if (slot < 0 || slot / BS >= NB) return;
  const uint16_t *src = (c * 8 < R) ? kvc + t * kvc_st + c * 8 : kpe + t * kpe_st + (c * 8 - R);
  *reinterpret_cast<u32x4 *>(lat + slot * W + c * 8) = *reinterpret_cast<const u32x4 *>(src);
}

// ---------------------------------------------------------------------------
// MLA latent gather: one workgroup per (block j of sequence i). A block's
// rows are one contiguous run of BS rows in the cache, and the rows a
// sequence takes from it are one contiguous run of the output: a plain
// 16-byte copy of ntok * row_bytes.
__global__ __launch_bounds__(256) void mla_gather_kernel(const uint8_t *__restrict__ lat,
                                                         const int32_t *__restrict__ bt, int64_t bt_stride, int Mb,
                                                         const int32_t *__restrict__ seq_lens,
                                                         const int64_t *__restrict__ cu, uint8_t *__restrict__ out,
                                                         int row_bytes, int BS, int64_t NB) {
  const int i = blockIdx.y, j = blockIdx.x;
  int L = seq_lens[i];
  L = L < Mb * BS ? L : Mb * BS;
  if (L <= 0 || j * BS >= L) return;
  const int64_t blk = bt[i * bt_stride + j];
  if (blk < 0 || blk >= NB) return;
  const int ntok = (L - j * BS) < BS ? (L - j * BS) : BS;
  const int n16 = ntok * (row_bytes / 16);
  const u32x4 *src = reinterpret_cast<const u32x4 *>(lat + blk * BS * static_cast<int64_t>(row_bytes));
  u32x4 *dst = reinterpret_cast<u32x4 *>(out + (cu[i] + static_cast<int64_t>(j) * BS) * row_bytes);
  for (int w = threadIdx.x; w < n16; w += 256) dst[w] = src[w];
}

// Whole-block copy of an MLA latent cache: one workgroup per (src, dst) pair.
__global__ __launch_bounds__(256) void mla_copy_blocks_kernel(uint8_t *__restrict__ lat,
                                                              const int64_t *__restrict__ mapping,
                                                              int64_t block_bytes, int64_t NB) {
  const int64_t src = mapping[2 * blockIdx.x], dst = mapping[2 * blockIdx.x + 1];
  if (src < 0 || dst < 0 || src >= NB || dst >= NB) return;
  const int64_t n16 = block_bytes / 16;
  const u32x4 *s4 = reinterpret_cast<const u32x4 *>(lat + src * block_bytes);
  u32x4 *d4 = reinterpret_cast<u32x4 *>(lat + dst * block_bytes);
  for (int64_t w = threadIdx.x; w < n16; w += 256) d4[w] = s4[w];
}

static int check_kv_input(const void *p, int64_t st_t, int64_t st_h, const char *name) {
  WKV_CHECK_ARG(p != nullptr, "%s is NULL", name);
  WKV_CHECK_ARG(aligned16(p), "%s must be 16-byte aligned", name);
  WKV_CHECK_ARG(st_t % 8 == 0 && st_h % 8 == 0 && st_t >= 0 && st_h >= 0,
                "%s strides must be non-negative multiples of 8 (got %lld, %lld)", name, (long long)st_t,
                (long long)st_h);
  return WKV_OK;
}

}  // namespace wkv

using namespace wkv;

extern "C" int wkv_append(const wkv_cache_t *cache, const void *key, int64_t key_stride_t, int64_t key_stride_h,
                          const void *value, int64_t value_stride_t, int64_t value_stride_h,
                          const int64_t *slot_mapping, int64_t num_tokens, void *stream) {
  int rc = check_cache(cache, WKV_KV_BF16);
  if (rc) return rc;
  WKV_CHECK_ARG(num_tokens >= 0, "num_tokens must be >= 0");
  if (num_tokens == 0) return WKV_OK;
  WKV_CHECK_ARG(slot_mapping != nullptr, "slot_mapping is NULL");
  if ((rc = check_kv_input(key, key_stride_t, key_stride_h, "key"))) return rc;
  if ((rc = check_kv_input(value, value_stride_t, value_stride_h, "value"))) return rc;
  const int H = cache->num_kv_heads, D = cache->head_dim;
  const int64_t work = num_tokens * H * (D / 8);
  const dim3 grid(static_cast<unsigned>((work + 255) / 256));
  auto s = static_cast<hipStream_t>(stream);
  auto kc = static_cast<uint16_t *>(cache->k);
  auto vc = static_cast<uint16_t *>(cache->v);
  auto k = static_cast<const uint16_t *>(key);
  auto v = static_cast<const uint16_t *>(value);
  if (num_tokens >= kBulkMinTokens) {  // a prompt: the transposing kernel
    WKV_CHECK_ARG(H <= 65535, "num_kv_heads too large");
    const dim3 bgrid(static_cast<unsigned>((num_tokens + kBulkTokens - 1) / kBulkTokens), static_cast<unsigned>(H));
    if (D == 128)
      append_bf16_bulk_kernel<128><<<bgrid, 256, 0, s>>>(kc, vc, k, key_stride_t, key_stride_h, v, value_stride_t,
                                                         value_stride_h, slot_mapping, num_tokens, H,
                                                         cache->block_size, cache->num_blocks);
    else
      append_bf16_bulk_kernel<64><<<bgrid, 256, 0, s>>>(kc, vc, k, key_stride_t, key_stride_h, v, value_stride_t,
                                                        value_stride_h, slot_mapping, num_tokens, H,
                                                        cache->block_size, cache->num_blocks);
  } else if (D == 128)
    append_bf16_kernel<128><<<grid, 256, 0, s>>>(kc, vc, k, key_stride_t, key_stride_h, v, value_stride_t,
                                                 value_stride_h, slot_mapping, num_tokens, H, cache->block_size,
                                                 cache->num_blocks);
  else
    append_bf16_kernel<64><<<grid, 256, 0, s>>>(kc, vc, k, key_stride_t, key_stride_h, v, value_stride_t,
                                                value_stride_h, slot_mapping, num_tokens, H, cache->block_size,
                                                cache->num_blocks);
  WKV_CHECK_LAUNCH("wkv_append");
  return WKV_OK;
}

extern "C" int wkv_append_fp8(const wkv_cache_t *cache, const void *key, int64_t key_stride_t,
                              int64_t key_stride_h, const void *value, int64_t value_stride_t,
                              int64_t value_stride_h, const int64_t *slot_mapping, int64_t num_tokens,
                              void *stream) {
  int rc = check_cache(cache, WKV_KV_FP8_E4M3);
  if (rc) return rc;
  WKV_CHECK_ARG(num_tokens >= 0 && num_tokens < (1ll << 31), "num_tokens out of range");
  if (num_tokens == 0) return WKV_OK;
  WKV_CHECK_ARG(slot_mapping != nullptr, "slot_mapping is NULL");
  if ((rc = check_kv_input(key, key_stride_t, key_stride_h, "key"))) return rc;
  if ((rc = check_kv_input(value, value_stride_t, value_stride_h, "value"))) return rc;
  WKV_CHECK_ARG(cache->num_kv_heads <= 65535, "num_kv_heads too large");
  const int H = cache->num_kv_heads, D = cache->head_dim;
  const dim3 grid(static_cast<unsigned>(num_tokens), static_cast<unsigned>(H));
  auto s = static_cast<hipStream_t>(stream);
  auto kc = static_cast<uint8_t *>(cache->k);
  auto vc = static_cast<uint8_t *>(cache->v);
  auto k = static_cast<const uint16_t *>(key);
  auto v = static_cast<const uint16_t *>(value);
  // 16-byte source rows for the bulk kernel's vector loads
  const bool rows16 = aligned16(key) && aligned16(value) && key_stride_t % 8 == 0 && key_stride_h % 8 == 0 &&
                      value_stride_t % 8 == 0 && value_stride_h % 8 == 0;
  if (num_tokens >= kFp8BulkMinTokens && rows16) {
    const dim3 bgrid(static_cast<unsigned>((num_tokens + 63) / 64), static_cast<unsigned>(H));
#define WKV_FP8_BULK(Dv, NWv)                                                                                   \
  append_fp8_bulk_kernel<Dv, NWv><<<bgrid, 64 * NWv, 0, s>>>(kc, vc, cache->k_scale, cache->v_scale, k,         \
                                                             key_stride_t, key_stride_h, v, value_stride_t,    \
                                                             value_stride_h, slot_mapping, num_tokens, H,      \
                                                             cache->block_size, cache->num_blocks)
    const bool prompt = num_tokens >= kFp8PromptTokens;
    if (D == 128) {
      if (prompt) WKV_FP8_BULK(128, 4); else WKV_FP8_BULK(128, 8);
    } else {
      if (prompt) WKV_FP8_BULK(64, 4); else WKV_FP8_BULK(64, 8);
    }
#undef WKV_FP8_BULK
  } else if (D == 128)
    append_fp8_kernel<128><<<grid, 64, 0, s>>>(kc, vc, cache->k_scale, cache->v_scale, k, key_stride_t,
                                               key_stride_h, v, value_stride_t, value_stride_h, slot_mapping,
                                               num_tokens, H, cache->block_size, cache->num_blocks);
  else
    append_fp8_kernel<64><<<grid, 64, 0, s>>>(kc, vc, cache->k_scale, cache->v_scale, k, key_stride_t,
                                              key_stride_h, v, value_stride_t, value_stride_h, slot_mapping,
                                              num_tokens, H, cache->block_size, cache->num_blocks);
  WKV_CHECK_LAUNCH("wkv_append_fp8");
  return WKV_OK;
}

extern "C" int wkv_mla_append(const wkv_mla_cache_t *cache, const void *kv_c, int64_t kv_c_stride,
                              const void *k_pe, int64_t k_pe_stride, const int64_t *slot_mapping,
                              int64_t num_tokens, void *stream) {
  int rc = check_mla_cache(cache);
  if (rc) return rc;
  WKV_CHECK_ARG(num_tokens >= 0, "num_tokens must be >= 0");
  if (num_tokens == 0) return WKV_OK;
  WKV_CHECK_ARG(slot_mapping != nullptr, "slot_mapping is NULL");
  if ((rc = check_kv_input(kv_c, kv_c_stride, 0, "kv_c"))) return rc;
  if (cache->rope_dim > 0 && (rc = check_kv_input(k_pe, k_pe_stride, 0, "k_pe"))) return rc;
  const int C = (cache->kv_lora_rank + cache->rope_dim) / 8;
  const dim3 grid(static_cast<unsigned>((num_tokens * C + 255) / 256));
  mla_append_kernel<<<grid, 256, 0, static_cast<hipStream_t>(stream)>>>(
      static_cast<uint16_t *>(cache->latent), static_cast<const uint16_t *>(kv_c), kv_c_stride,
      static_cast<const uint16_t *>(k_pe), k_pe_stride, slot_mapping, num_tokens, cache->kv_lora_rank,
      cache->rope_dim, cache->block_size, cache->num_blocks);
  WKV_CHECK_LAUNCH("wkv_mla_append");
  return WKV_OK;
}

extern "C" int wkv_gather(const wkv_cache_t *cache, const int32_t *block_table, int64_t bt_stride,
                          int32_t max_blocks_per_seq, const int32_t *seq_lens, const int64_t *cu_seq_lens,
                          int32_t batch, void *out_k, void *out_v, int32_t dequant, void *stream) {
  int rc = check_cache(cache, -1);
  if (rc) return rc;
  WKV_CHECK_ARG(batch >= 0 && batch <= 65535, "batch must be in [0, 65535]");
  if (batch == 0 || max_blocks_per_seq == 0) return WKV_OK;
  WKV_CHECK_ARG(max_blocks_per_seq > 0 && bt_stride >= max_blocks_per_seq, "bad block table geometry");
  WKV_CHECK_ARG(block_table && seq_lens && cu_seq_lens, "block_table / seq_lens / cu_seq_lens is NULL");
  WKV_CHECK_ARG(out_k && out_v && aligned16(out_k) && aligned16(out_v), "outputs must be non-NULL and 16-byte aligned");
  WKV_CHECK_ARG(dequant == 0 || dequant == 1, "dequant must be 0 or 1");
  const bool fp8 = cache->kv_dtype == WKV_KV_FP8_E4M3;
  WKV_CHECK_ARG(!dequant || fp8, "dequant applies to fp8 caches only");
  const dim3 grid(static_cast<unsigned>(max_blocks_per_seq), static_cast<unsigned>(batch));
  auto s = static_cast<hipStream_t>(stream);
  auto kc = static_cast<const uint8_t *>(cache->k);
  auto vc = static_cast<const uint8_t *>(cache->v);
  auto ok = static_cast<uint8_t *>(out_k);
  auto ov = static_cast<uint8_t *>(out_v);
  const int H = cache->num_kv_heads, BS = cache->block_size;
  const int64_t NB = cache->num_blocks;
#define WKV_GATHER(Dv, F8, DQ)                                                                               \
  gather_kernel<Dv, F8, DQ><<<grid, 256, 0, s>>>(kc, vc, cache->k_scale, cache->v_scale, block_table, bt_stride, \
                                                 max_blocks_per_seq, seq_lens, cu_seq_lens, ok, ov, H, BS, NB)
  if (cache->head_dim == 128) {
    if (!fp8) WKV_GATHER(128, false, false);
    else if (!dequant) WKV_GATHER(128, true, false);
    else WKV_GATHER(128, true, true);
  } else {
    if (!fp8) WKV_GATHER(64, false, false);
    else if (!dequant) WKV_GATHER(64, true, false);
    else WKV_GATHER(64, true, true);
  }
#undef WKV_GATHER
  WKV_CHECK_LAUNCH("wkv_gather");
  return WKV_OK;
}

extern "C" int wkv_copy_blocks(const wkv_cache_t *cache, const int64_t *block_mapping, int64_t n, void *stream) {
  int rc = check_cache(cache, -1);
  if (rc) return rc;
  WKV_CHECK_ARG(n >= 0 && n < (1ll << 31), "n out of range");
  if (n == 0) return WKV_OK;
  WKV_CHECK_ARG(block_mapping != nullptr, "block_mapping is NULL");
  const int esz = cache->kv_dtype == WKV_KV_FP8_E4M3 ? 1 : 2;
  const int64_t block_bytes =
      static_cast<int64_t>(cache->num_kv_heads) * cache->head_dim * cache->block_size * esz;
  WKV_CHECK_ARG(cache->num_kv_heads <= 256, "copy_blocks supports at most 256 KV heads");
  const bool fp8 = cache->kv_dtype == WKV_KV_FP8_E4M3;
  copy_blocks_kernel<<<dim3(static_cast<unsigned>(n)), 256, 0, static_cast<hipStream_t>(stream)>>>(
      static_cast<uint8_t *>(cache->k), static_cast<uint8_t *>(cache->v), fp8 ? cache->k_scale : nullptr,
      fp8 ? cache->v_scale : nullptr, block_mapping, block_bytes, cache->num_kv_heads, cache->num_blocks);
  WKV_CHECK_LAUNCH("wkv_copy_blocks");
  return WKV_OK;
}

extern "C" int wkv_mla_gather(const wkv_mla_cache_t *cache, const int32_t *block_table, int64_t bt_stride,
                              int32_t max_blocks_per_seq, const int32_t *seq_lens, const int64_t *cu_seq_lens,
                              int32_t batch, void *out, void *stream) {
  int rc = check_mla_cache(cache);
  if (rc) return rc;
  WKV_CHECK_ARG(batch >= 0 && batch <= 65535, "batch must be in [0, 65535]");
  if (batch == 0 || max_blocks_per_seq == 0) return WKV_OK;
  WKV_CHECK_ARG(max_blocks_per_seq > 0 && bt_stride >= max_blocks_per_seq, "bad block table geometry");
  WKV_CHECK_ARG(block_table && seq_lens && cu_seq_lens, "block_table / seq_lens / cu_seq_lens is NULL");
  WKV_CHECK_ARG(out != nullptr && aligned16(out), "out must be non-NULL and 16-byte aligned");
  const int row_bytes = 2 * (cache->kv_lora_rank + cache->rope_dim);
  const dim3 grid(static_cast<unsigned>(max_blocks_per_seq), static_cast<unsigned>(batch));
  mla_gather_kernel<<<grid, 256, 0, static_cast<hipStream_t>(stream)>>>(
      static_cast<const uint8_t *>(cache->latent), block_table, bt_stride, max_blocks_per_seq, seq_lens, cu_seq_lens,
      static_cast<uint8_t *>(out), row_bytes, cache->block_size, cache->num_blocks);
  WKV_CHECK_LAUNCH("wkv_mla_gather");
  return WKV_OK;
}

extern "C" int wkv_mla_copy_blocks(const wkv_mla_cache_t *cache, const int64_t *block_mapping, int64_t n,
                                   void *stream) {
  int rc = check_mla_cache(cache);
  if (rc) return rc;
  WKV_CHECK_ARG(n >= 0 && n < (1ll << 31), "n out of range");
  if (n == 0) return WKV_OK;
  WKV_CHECK_ARG(block_mapping != nullptr, "block_mapping is NULL");
  const int64_t block_bytes =
      static_cast<int64_t>(cache->block_size) * (cache->kv_lora_rank + cache->rope_dim) * 2;
  mla_copy_blocks_kernel<<<dim3(static_cast<unsigned>(n)), 256, 0, static_cast<hipStream_t>(stream)>>>(
      static_cast<uint8_t *>(cache->latent), block_mapping, block_bytes, cache->num_blocks);
  WKV_CHECK_LAUNCH("wkv_mla_copy_blocks");
  return WKV_OK;
}
