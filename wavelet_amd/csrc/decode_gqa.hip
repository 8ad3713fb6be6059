// GQA paged decode attention for gfx950.
//
// One wavefront owns one (sequence, KV head, partition) work item and streams
// the partition's tokens in 16-token tiles straight from HBM into MFMA operand
// registers; there is no LDS staging because the cache layout already places
// each lane's operand in one 16-byte (K) or 8-byte (V) run:
//
//   K [NB, Hkv, D/x, BS, x]: for chunk c the 16 tokens of a tile are 256
//      contiguous bytes, so the four chunks a QK MFMA needs are one 1 KB
//      contiguous wave load.
//   V [NB, Hkv, D, BS]: one head_dim row holds the block's tokens
//      contiguously, which is the A-operand (row = d, k = token) of the PV
//      MFMA without any transpose.
//
// Per tile:   S^T[16 tok, 16 heads] = K[16 tok, D] . Q^T[D, 16 heads]
//             (D/32 x mfma_f32_16x16x32_bf16; the group's G <= 16 query
//             heads padded to 16 columns)
//             online softmax on S^T (lane = head column, 4 tokens per lane,
//             two cross-row shuffles for the tile max)
//             O^T[D, 16 heads] += V^T[D, 16 tok] . P^T[16 tok, 16 heads]
//             (D/16 x mfma_f32_16x16x16_bf16; the QK output registers are
//             exactly the B operand, so P never leaves the lane)
// fp8 caches are widened to bf16 in registers (exact) and their power-of-two
// per-(block, head) scales are folded into the scores (K) and into P (V).
// Long contexts are split into partitions (one wave each) whose partial
// results a second, small kernel merges by log-sum-exp. (Merging inside the
// main kernel needs device-scope release/acquire between waves of different
// XCDs; measured here, that costs far more than the extra launch.)
// The decode-step append can be fused in: the wave that owns a sequence's last
// partition first writes the new token into the cache, then attends over it.
#include <cmath>

#include "wkv_common.h"
#include "kv_append_dev.h"

namespace wkv {

typedef __attribute__((__vector_size__(4 * sizeof(short)))) short shortx4;

// Registers of one 16-token tile exactly as loaded (fp8 is widened at use, so
// issuing a tile never waits for its data).
template <int D, bool FP8>
struct Tile {
  static constexpr int NK = FP8 ? D / 64 : D / 32;  // 16-byte K loads per lane
  static constexpr int NPV = D / 16;                 // PV MFMAs per tile
  u32x4 k[NK];
  u32x2 v[FP8 ? 1 : NPV];      // bf16: 4 tokens x 1 d per PV MFMA
  u32x4 v4[FP8 ? NPV / 4 : 1];  // fp8: 16 tokens of one d row per load (transposed at use)
  int valid;                // tokens of the tile inside the sequence (0 = skip)
  float ksc, vsc;           // fp8 per-(block, head) scales (1 for bf16)
};

// e4m3fn codes -> bf16, exact (every e4m3 value is a bf16 value), with the
// hardware pair conversion v_cvt_scalef32_pk_bf16_fp8 at scale 1: bytes 0, 1
// (word 0) or 2, 3 (word 1) of a dword become the low and high bf16 halves.
template <bool WORD1>
__device__ __forceinline__ uint32_t fp8x2_to_bf16x2(uint32_t w) {
  return __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w, 1.0f, WORD1));
}

__device__ __forceinline__ bf16x8 fp8x8_to_bf16x8(uint32_t lo, uint32_t hi) {
  u32x4 r;
  r[0] = fp8x2_to_bf16x2<false>(lo);
  r[1] = fp8x2_to_bf16x2<true>(lo);
  r[2] = fp8x2_to_bf16x2<false>(hi);
  r[3] = fp8x2_to_bf16x2<true>(hi);
  return __builtin_bit_cast(bf16x8, r);
}

__device__ __forceinline__ shortx4 fp8x4_to_bf16x4(uint32_t w) {
  u32x2 r;
  r[0] = fp8x2_to_bf16x2<false>(w);
  r[1] = fp8x2_to_bf16x2<true>(w);
  return __builtin_bit_cast(shortx4, r);
}

// A pointer every lane holds the same value of, moved to scalar registers. A
// buffer resource must be; when the compiler cannot prove it (it sometimes
// computes a uniform address with vector instructions) it would otherwise
// wrap every load in a loop over the distinct values.
__device__ __forceinline__ const uint8_t *wave_uniform(const uint8_t *p) {
  const uint64_t v = reinterpret_cast<uint64_t>(p);
  const uint32_t lo = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(v));
  const uint32_t hi = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(v >> 32));
  return reinterpret_cast<const uint8_t *>((static_cast<uint64_t>(hi) << 32) | lo);
}

// 4x4 transpose of dwords across the four 16-lane rows of a wave: on entry
// row g holds X[g][0..3] in w[0..3]; on return row g holds X[0..3][g]. Two
// v_permlane32_swap (rows g <-> g^2) then two v_permlane16_swap (g <-> g^1).
__device__ __forceinline__ void transpose_rows4(uint32_t w[4]) {
#pragma unroll
  for (int a = 0; a < 2; ++a) {  // upper rows of w[a] <-> lower rows of w[a+2]
    const auto r = __builtin_amdgcn_permlane32_swap(w[a], w[a + 2], false, false);
    w[a] = r[0];
    w[a + 2] = r[1];
  }
#pragma unroll
  for (int b = 0; b < 4; b += 2) {  // odd rows of w[b] <-> even rows of w[b+1]
    const auto r = __builtin_amdgcn_permlane16_swap(w[b], w[b + 1], false, false);
    w[b] = r[0];
    w[b + 1] = r[1];
  }
}

// Buffer-resource word 3 for raw (unformatted, unswizzled) buffers on gfx9-family parts.
constexpr int kRawBufferWord3 = 0x00020000;

// Issues the loads of one 16-token tile (tokens [o0, o0+16) of block blk) as
// buffer loads: a wave-uniform resource (scalar registers) per (block, head)
// region, a per-lane byte offset that never changes (koff, voff) and a scalar
// offset per load, so no per-tile vector address arithmetic is needed.
template <int D, bool FP8>
__device__ __forceinline__ void load_tile(Tile<D, FP8> &t, const uint8_t *__restrict__ kc,
                                          const uint8_t *__restrict__ vc, int blk, int kvh, int Hkv, int BS,
                                          int o0, uint32_t koff, uint32_t voff) {
  constexpr int ESZ = FP8 ? 1 : 2;
  const int region = D * BS * ESZ;  // bytes of one (block, head) region of K, and of V
  // Region index in 32 bits (the host keeps num_blocks * num_kv_heads below
  // 2^31), in a scalar register, so the 64-bit address arithmetic stays scalar.
  const int ridx = __builtin_amdgcn_readfirstlane(blk * Hkv + kvh);
  const int64_t rbase = static_cast<int64_t>(ridx) * region;
  const uint8_t *kb = wave_uniform(kc + rbase + o0 * 16);
  const __amdgpu_buffer_rsrc_t kr = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t *>(kb), 0, region, kRawBufferWord3);
#pragma unroll
  for (int j = 0; j < Tile<D, FP8>::NK; ++j)
    t.k[j] = __builtin_amdgcn_raw_buffer_load_b128(kr, koff, j * 4 * BS * 16, 0);
  const uint8_t *vb = wave_uniform(vc + rbase + o0 * ESZ);
  const __amdgpu_buffer_rsrc_t vr = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t *>(vb), 0, region, kRawBufferWord3);
  if constexpr (FP8) {
    // Lane (m, g) loads d row 64j + 16g + m whole (16 tokens, 16 bytes): 1 KB
    // per wave load instead of 256 B -- 4-byte loads cap HBM near half its rate.
#pragma unroll
    for (int j = 0; j < Tile<D, FP8>::NPV / 4; ++j)
      t.v4[j] = __builtin_amdgcn_raw_buffer_load_b128(vr, voff, j * 64 * BS, 0);
  } else {
#pragma unroll
    for (int n = 0; n < Tile<D, FP8>::NPV; ++n)
      t.v[n] = __builtin_amdgcn_raw_buffer_load_b64(vr, voff, n * 16 * BS * 2, 0);
  }
}

template <int D, bool FP8>
struct DecodeState {
  floatx4 o[D / 16];
  float m;  // running max (log2 domain) of this lane's head column
  float l;  // this lane's share of the running denominator
};

// One tile of online-softmax attention.
template <int D, bool FP8>
__device__ __forceinline__ void attend_tile(DecodeState<D, FP8> &st, const Tile<D, FP8> &t, const bf16x8 *qop,
                                            float scale_log2, int grp) {
  floatx4 s = {0.f, 0.f, 0.f, 0.f};
  if constexpr (FP8) {
#pragma unroll
    for (int m = 0; m < D / 64; ++m) {
      s = __builtin_amdgcn_mfma_f32_16x16x32_bf16(fp8x8_to_bf16x8(t.k[m][0], t.k[m][1]), qop[2 * m], s, 0, 0, 0);
      s = __builtin_amdgcn_mfma_f32_16x16x32_bf16(fp8x8_to_bf16x8(t.k[m][2], t.k[m][3]), qop[2 * m + 1], s, 0, 0, 0);
    }
  } else {
#pragma unroll
    for (int j = 0; j < D / 32; ++j)
      s = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, t.k[j]), qop[j], s, 0, 0, 0);
  }
  const float s_mul = scale_log2 * t.ksc;
  float sv[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) sv[i] = s[i] * s_mul;
  if (t.valid < 16) {  // uniform: only a sequence's first and last tiles are partial
#pragma unroll
    for (int i = 0; i < 4; ++i)
      if (4 * grp + i >= t.valid) sv[i] = -INFINITY;
  }
  const float mt = row_max4(fmaxf(fmaxf(sv[0], sv[1]), fmaxf(sv[2], sv[3])));
  // st.m is the reference maximum (-inf until the first attended token).
  const bool move = mt > st.m + SOFTMAX_TAU;
  const float m_new = move ? mt : st.m;
  const float corr = (move && st.m != -INFINITY) ? fast_exp2(st.m - m_new) : 1.f;
  const float m_use = (m_new == -INFINITY) ? 0.f : m_new;
  float p[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) p[i] = fast_exp2(sv[i] - m_use);
  st.l = st.l * corr + ((p[0] + p[1]) + (p[2] + p[3]));
  st.m = m_new;
  if (__any(corr != 1.f)) {  // a reference maximum moved for some head: rescale
#pragma unroll
    for (int n = 0; n < D / 16; ++n) {
#pragma unroll
      for (int i = 0; i < 4; ++i) st.o[n][i] *= corr;
    }
  }
  u32x2 pb;
  pb[0] = pack_bf16x2(p[0] * t.vsc, p[1] * t.vsc);
  pb[1] = pack_bf16x2(p[2] * t.vsc, p[3] * t.vsc);
  const shortx4 pop = __builtin_bit_cast(shortx4, pb);
  // fp8 V: after the transpose, lane (m, g) holds tokens 4g..4g+3 of d row
  // 16n + m in v8[n] -- the PV MFMA's A operand, as the bf16 loads deliver it.
  uint32_t v8[FP8 ? D / 16 : 1];
  if constexpr (FP8) {
#pragma unroll
    for (int j = 0; j < D / 64; ++j) {
      uint32_t w[4] = {t.v4[j][0], t.v4[j][1], t.v4[j][2], t.v4[j][3]};
      transpose_rows4(w);
#pragma unroll
      for (int e = 0; e < 4; ++e) v8[4 * j + e] = w[e];
    }
  }
#pragma unroll
  for (int n = 0; n < D / 16; ++n) {
    shortx4 vop = FP8 ? fp8x4_to_bf16x4(v8[FP8 ? n : 0]) : __builtin_bit_cast(shortx4, t.v[FP8 ? 0 : n]);
    if (t.valid < 16) {
      // Never let a masked slot's V reach the accumulator (it may hold NaN).
#pragma unroll
      for (int e = 0; e < 4; ++e)
        if (4 * grp + e >= t.valid) vop[e] = 0;
    }
    st.o[n] = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(vop, pop, st.o[n], 0, 0, 0);
  }
}

// The new token of a fused append + decode step: token b of `key`/`value`
// belongs to sequence b and goes to slot slots[b] (-1 = none).
struct StepAppend {
  const uint16_t *key;
  int64_t kst, ksh;
  const uint16_t *val;
  int64_t vst, vsh;
  const int64_t *slots;
};

// The token a bf16 fused append is adding, as a one-token tile built from
// the step's inputs (spread one dword per lane in nk, nv) instead of the
// cache, so the wave never waits for its own cache write.
template <int D>
__device__ __forceinline__ void new_token_tile(Tile<D, false> &t, uint32_t nk, uint32_t nv, int col, int grp) {
  t.valid = 1;
  t.ksc = 1.f;
  t.vsc = 1.f;
#pragma unroll
  for (int j = 0; j < D / 32; ++j) {
#pragma unroll
    for (int qd = 0; qd < 4; ++qd) {
      const uint32_t x = __shfl(nk, 4 * (4 * j + grp) + qd, 64);
      t.k[j][qd] = col == 0 ? x : 0u;  // row 0 = the new token
    }
  }
#pragma unroll
  for (int n = 0; n < D / 16; ++n) {
    const uint32_t x = __shfl(nv, (col + 16 * n) >> 1, 64);
    const uint32_t h = (col & 1) ? (x >> 16) : (x & 0xffffu);
    t.v[n][0] = grp == 0 ? h : 0u;  // token 0 of lane group 0
    t.v[n][1] = 0u;
  }
}

// Tiles a wave keeps in registers: one being attended while the others load.
// A wave's bytes in flight are what bound these kernels (HBM latency under load
// is several microseconds), so the smaller tiles (fp8, head_dim 64) go deeper:
//   bf16, d=128: 3 x 8 KB (the tile registers already limit the wave to 2 per SIMD)
//   fp8 or d=64: DEPTH_SMALL x 4 KB
#ifndef WKV_GQA_DEPTH_SMALL
#define WKV_GQA_DEPTH_SMALL 3
#endif
template <int D, bool FP8>
constexpr int pipeline_depth() {
  return (D == 128 && !FP8) ? 3 : WKV_GQA_DEPTH_SMALL;
}

// The tile loop of one wave over tokens [t_begin, t_end) of a block list:
// `consume(tile)` attends each 16-token tile. `my_blk` holds, in lane i, the
// id of the range's i-th block (loaded by the caller; the host keeps a range
// within 64 blocks); each tile takes its id with a register readlane.
template <int D, bool FP8, typename Consume>
__device__ __forceinline__ void attend_range(Consume &&consume, const uint8_t *__restrict__ kc,
                                             const uint8_t *__restrict__ vc, const float *__restrict__ ks,
                                             const float *__restrict__ vs, int my_blk, int t_begin, int t_end,
                                             int kvh, int Hkv, int BS, int64_t NB, int lane, int col, int grp) {
  if (t_end <= t_begin) return;
  const int n_tiles = (t_end - t_begin + 15) / 16;
  const int blk_first = t_begin / BS;
  const int nblk = (t_end - 1) / BS - blk_first + 1;
  float my_ks = 1.f, my_vs = 1.f;
  if (lane >= nblk || my_blk < 0 || my_blk >= NB) my_blk = -1;  // -1: never read, its slots count as masked
  if constexpr (FP8) {
    if (my_blk >= 0) {
      my_ks = ks[static_cast<int64_t>(my_blk) * Hkv + kvh];
      my_vs = vs[static_cast<int64_t>(my_blk) * Hkv + kvh];
    }
  }
  const uint32_t koff = static_cast<uint32_t>((grp * BS + col) * 16);
  const uint32_t voff = static_cast<uint32_t>(FP8 ? (16 * grp + col) * BS : (col * BS + 4 * grp) * 2);

  // Issue tile i's loads unconditionally (an index past the end re-reads the
  // last tile, an L2 hit) so the compiler can count outstanding loads and
  // wait only for the tile about to be used: three tiles rotate, two in flight.
  auto issue = [&](Tile<D, FP8> &t, int i) {
    const int ii = i < n_tiles ? i : n_tiles - 1;
    const int ts = t_begin + 16 * ii;
    const int bi = ts / BS - blk_first;
    int blk = __builtin_amdgcn_readlane(my_blk, bi);
    t.valid = (i < n_tiles && blk >= 0) ? ((t_end - ts) < 16 ? (t_end - ts) : 16) : 0;
    if constexpr (FP8) {
      t.ksc = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(my_ks), bi));
      t.vsc = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(my_vs), bi));
    } else {
      t.ksc = 1.f;
      t.vsc = 1.f;
    }
    if (blk < 0) blk = 0;
    load_tile<D, FP8>(t, kc, vc, blk, kvh, Hkv, BS, ts % BS, koff, voff);
  };
  // Loads are issued unconditionally, which keeps the wait counts exact; a
  // tile past the end (or of an unmapped block) is skipped, uniformly, when its
  // turn comes. NT tiles rotate; while tile i is attended, i+1 .. i+NT-1 load.
  constexpr int NT = pipeline_depth<D, FP8>();
  Tile<D, FP8> t[NT];
  // The prologue's loads must go out in tile order: the wait before a tile
  // counts the loads issued after it, and the loop-entry state is merged with
  // the back edge's (the scheduler otherwise reorders these independent loads,
  // which forces every loop iteration's first tile to wait for all but one).
#pragma unroll
  for (int k = 0; k < NT - 1; ++k) {
    issue(t[k], k);
    __builtin_amdgcn_sched_barrier(0);
  }
  for (int i = 0; i < n_tiles; i += NT) {
#pragma unroll
    for (int k = 0; k < NT; ++k) {
      issue(t[(k + NT - 1) % NT], i + k + NT - 1);
      if (t[k].valid > 0) consume(t[k]);
    }
  }
}

// The Q^T operand of one lane: 8 d-values of the query row its column stands
// for, in the d order of load_tile's K operand (zeros when !valid; qp must
// still point at a readable row).
template <int D, bool FP8>
__device__ __forceinline__ void load_q(bf16x8 *qop, const uint16_t *qp, bool valid, int grp) {
#pragma unroll
  for (int j = 0; j < D / 32; ++j) {
    const int d0 = FP8 ? 16 * (4 * (j >> 1) + grp) + 8 * (j & 1) : 32 * j + 8 * grp;
    u32x4 w = *reinterpret_cast<const u32x4 *>(qp + d0);
    if (!valid) w = u32x4{0u, 0u, 0u, 0u};
    qop[j] = __builtin_bit_cast(bf16x8, w);
  }
}

// Attention of one wave over tokens [t_begin, t_end) of one sequence: returns
// the unnormalised output, running max and this lane's share of the sum.
template <int D, bool FP8>
__device__ __forceinline__ void attend_partition(DecodeState<D, FP8> &st, const uint8_t *__restrict__ kc,
                                                 const uint8_t *__restrict__ vc, const float *__restrict__ ks,
                                                 const float *__restrict__ vs, const bf16x8 *qop, int my_blk,
                                                 int t_begin, int t_end, int kvh, int Hkv, int BS, int64_t NB,
                                                 float scale_log2, int lane, int col, int grp) {
  attend_range<D, FP8>([&](Tile<D, FP8> &t) { attend_tile<D, FP8>(st, t, qop, scale_log2, grp); }, kc, vc, ks, vs,
                       my_blk, t_begin, t_end, kvh, Hkv, BS, NB, lane, col, grp);
}

// Tokens per partition for a context of n > 0 tokens cut into chunks of W
// partitions of at most P_tok tokens: the chunk count stays ceil(n / (W P_tok))
// (the merge relies on it) and the tokens are spread evenly over the chunks'
// waves, rounded up to a multiple of `unit` (<= P_tok rounded up to `unit`).
// A workgroup lasts as long as its longest wave; balanced, no wave idles while
// another streams a full partition.
__device__ __forceinline__ int balanced_partition(int n, int W, int P_tok, int unit) {
  const int nchunks = (n + W * P_tok - 1) / (W * P_tok);
  int p = (n + W * nchunks - 1) / (W * nchunks);
  p = (p + unit - 1) / unit * unit;
  return __builtin_amdgcn_readfirstlane(p);
}

// Grid: (chunk, KV head, sequence); W waves per workgroup, wave w of chunk c
// owns partition c*W + w of P_tok tokens. The waves of a workgroup merge
// their partials through LDS; a context longer than one chunk leaves one
// partial per chunk for merge_partials_kernel.
template <int D, bool FP8, bool APPEND, int W>
__global__ __launch_bounds__(64 * W) void decode_gqa_kernel(
    uint8_t *__restrict__ kc, uint8_t *__restrict__ vc, float *__restrict__ ks, float *__restrict__ vs,
    const uint16_t *__restrict__ q, int64_t q_sb, int64_t q_sh, uint16_t *__restrict__ out,
    float *__restrict__ part_o, float *__restrict__ part_ml, const int32_t *__restrict__ bt, int64_t bt_stride,
    int Mb, int max_seq, const int32_t *__restrict__ seq_lens, int Hq, int Hkv, int G, int BS, int64_t NB,
    float scale_log2, int P_tok, int max_chunks, StepAppend ap) {
  const int chunk = blockIdx.x, kvh = blockIdx.y, b = blockIdx.z;
  // The wave index is uniform across the wave; saying so keeps everything
  // derived from it (partition, block ids, buffer resources) in scalar registers.
  const int wave = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x >> 6));
  const int lane = threadIdx.x & 63, col = lane & 15, grp = lane >> 4;
  const int part = chunk * W + wave;
  int t_begin = part * P_tok;
  int blk_first = t_begin / BS;

  // Loads that do not depend on the context length go out together with it:
  // the block ids of a full-size partition (bounded by the block-table width) and q.
  int L = seq_lens[b];
  int my_blk = -1;
  if (blk_first + lane < Mb) my_blk = bt[b * bt_stride + blk_first + lane];
  // Q^T operand: lane holds 8 d-values of head `col` (zero for padded heads).
  bf16x8 qop[D / 32];
  load_q<D, FP8>(qop, q + b * q_sb + static_cast<int64_t>(kvh * G + (col < G ? col : 0)) * q_sh, col < G, grp);

  L = L < max_seq ? L : max_seq;  // max_seq <= block-table width * BS: every read stays in the table
  if (L <= 0) {
    if (chunk == 0 && wave == 0 && col < G) {  // empty context: zeros
      uint16_t *op = out + (static_cast<int64_t>(b) * Hq + kvh * G + col) * D;
#pragma unroll
      for (int n = 0; n < D / 16; ++n) *reinterpret_cast<u32x2 *>(op + 16 * n + 4 * grp) = u32x2{0u, 0u};
    }
    return;
  }
  const int nchunks = (L + W * P_tok - 1) / (W * P_tok);
  if (chunk >= nchunks) return;  // the whole workgroup leaves together
  // This sequence's partitions: balanced over the chunks' waves, in whole
  // blocks (the new token's block has one reader; with or without a fused
  // append the split, and so the summation order, is the same). At most
  // ceil(P_tok / BS) blocks each, which the host keeps within 64.
  const int P_seq = balanced_partition(L, W, P_tok, BS);
  if (P_seq != P_tok) {
    t_begin = part * P_seq;
    blk_first = t_begin / BS;
    my_blk = -1;
    if (blk_first + lane < Mb) my_blk = bt[b * bt_stride + blk_first + lane];
  }
  const int nparts = (L + P_seq - 1) / P_seq;
  const bool active = part < nparts;
  const bool owns_new = APPEND && part == nparts - 1;

  // Fused append; the new token's block lies wholly in this wave's partition
  // (the partition size is a multiple of the block size): no other wave reads it.
  // fp8: a scale change can re-encode the whole block, so append first and
  //      wait before the block is read back.
  // bf16: the wave attends the cache up to the new token and then the token
  //      itself from the step's inputs (held one dword per lane), writing it
  //      to the cache at the end; nothing waits on the write or the slot.
  uint32_t nk = 0, nv = 0;
  int64_t slot = -1;
  if constexpr (APPEND) {
    if (owns_new) {
      slot = ap.slots[b];
      if constexpr (FP8) {
        if (slot >= 0 && slot / BS < NB) {
          const int64_t blk = slot / BS;
          const int off = static_cast<int>(slot % BS);
          fp8_append_one<D, false>(kc, ks, ap.key, ap.kst, ap.ksh, ap.slots, b, 1, blk, off, kvh, Hkv, BS);
          fp8_append_one<D, true>(vc, vs, ap.val, ap.vst, ap.vsh, ap.slots, b, 1, blk, off, kvh, Hkv, BS);
        }
        __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "workgroup");
      } else {
        if (lane < D / 2) {
          nk = reinterpret_cast<const uint32_t *>(ap.key + b * ap.kst + kvh * ap.ksh)[lane];
          nv = reinterpret_cast<const uint32_t *>(ap.val + b * ap.vst + kvh * ap.vsh)[lane];
        }
      }
    }
  }

  DecodeState<D, FP8> st;
#pragma unroll
  for (int n = 0; n < D / 16; ++n) st.o[n] = floatx4{0.f, 0.f, 0.f, 0.f};
  st.m = -INFINITY;
  st.l = 0.f;
  if (active) {
    const int t_end = (t_begin + P_seq) < L ? (t_begin + P_seq) : L;
    const bool from_regs = APPEND && !FP8 && owns_new;  // last token comes from the inputs
    attend_partition<D, FP8>(st, kc, vc, ks, vs, qop, my_blk, t_begin, from_regs ? L - 1 : t_end, kvh, Hkv, BS,
                             NB, scale_log2, lane, col, grp);
    if constexpr (APPEND && !FP8) {
      if (owns_new) {
        Tile<D, FP8> tn;
        new_token_tile<D>(tn, nk, nv, col, grp);
        attend_tile<D, FP8>(st, tn, qop, scale_log2, grp);
        // The cache write: lane i holds dword i of the K row and of the V row
        // (d = 2i, 2i+1); nothing in this launch reads the slot back.
        if (slot >= 0 && slot / BS < NB && lane < D / 2) {
          const int64_t nblk_id = slot / BS;
          const int off = static_cast<int>(slot % BS);
          uint16_t *kd = reinterpret_cast<uint16_t *>(kc) +
                         (((nblk_id * Hkv + kvh) * (D / 8) + (lane >> 2)) * BS + off) * 8 + (lane & 3) * 2;
          *reinterpret_cast<uint32_t *>(kd) = nk;
          uint16_t *vd = reinterpret_cast<uint16_t *>(vc) + ((nblk_id * Hkv + kvh) * D + 2 * lane) * BS + off;
          vd[0] = static_cast<uint16_t>(nv & 0xffffu);
          vd[BS] = static_cast<uint16_t>(nv >> 16);
        }
      }
    }
  }
  float l = st.l + __shfl_xor(st.l, 16, 64);
  l += __shfl_xor(l, 32, 64);

  if constexpr (W == 1) {
    if (col >= G) return;
    const int hq = kvh * G + col;
    if (nchunks == 1) {
      const float inv = l > 0.f ? 1.f / l : 0.f;
      uint16_t *op = out + (static_cast<int64_t>(b) * Hq + hq) * D;
#pragma unroll
      for (int n = 0; n < D / 16; ++n) {
        u32x2 w;
        w[0] = f32_to_bf16_bits(st.o[n][0] * inv) | (f32_to_bf16_bits(st.o[n][1] * inv) << 16);
        w[1] = f32_to_bf16_bits(st.o[n][2] * inv) | (f32_to_bf16_bits(st.o[n][3] * inv) << 16);
        *reinterpret_cast<u32x2 *>(op + 16 * n + 4 * grp) = w;
      }
      return;
    }
    const int64_t row = (static_cast<int64_t>(b) * Hq + hq) * max_chunks + chunk;
    float *po = part_o + row * D;
#pragma unroll
    for (int n = 0; n < D / 16; ++n) *reinterpret_cast<floatx4 *>(po + 16 * n + 4 * grp) = st.o[n];
    if (grp == 0) {
      part_ml[2 * row] = st.m;
      part_ml[2 * row + 1] = l;
    }
  } else {
    // Merge the W waves' partials of every head through LDS.
    __shared__ float sm_o[W][16][D];
    __shared__ float sm_m[W][16], sm_l[W][16];
    if (col < G) {
#pragma unroll
      for (int n = 0; n < D / 16; ++n) *reinterpret_cast<floatx4 *>(&sm_o[wave][col][16 * n + 4 * grp]) = st.o[n];
      if (grp == 0) {
        sm_m[wave][col] = st.m;
        sm_l[wave][col] = l;
      }
    }
    __syncthreads();
    const bool final_out = nchunks == 1;
    for (int e = threadIdx.x; e < G * D; e += 64 * W) {
      const int h = e / D, d = e % D;
      float M = -INFINITY;
#pragma unroll
      for (int w = 0; w < W; ++w) M = fmaxf(M, sm_m[w][h]);
      const float m_use = (M == -INFINITY) ? 0.f : M;
      float num = 0.f, den = 0.f;
#pragma unroll
      for (int w = 0; w < W; ++w) {
        const float f = exp2f(sm_m[w][h] - m_use);
        num += f * sm_o[w][h][d];
        den += f * sm_l[w][h];
      }
      const int hq = kvh * G + h;
      if (final_out) {
        out[(static_cast<int64_t>(b) * Hq + hq) * D + d] =
            static_cast<uint16_t>(f32_to_bf16_bits(den > 0.f ? num / den : 0.f));
      } else {
        const int64_t row = (static_cast<int64_t>(b) * Hq + hq) * max_chunks + chunk;
        part_o[row * D + d] = num;
        if (d == 0) {
          part_ml[2 * row] = M;
          part_ml[2 * row + 1] = den;
        }
      }
    }
  }
}

// Log-sum-exp merge of split-K partials: one wave per (sequence, query head)
// row, whose partials sit at slots [0, n0) and [s1, s1 + n1) of the row's
// `slots` (Slots gives the counts; false = the decode kernel finished the row).
// The loads of the first slots go out before the counts are known (their
// addresses do not depend on them; unused slots are masked, never summed), so
// a row costs about one memory round trip.
template <int D, typename Slots>
__global__ __launch_bounds__(256) void merge_partials_kernel(const float *__restrict__ part_o,
                                                             const float *__restrict__ part_ml,
                                                             uint16_t *__restrict__ out, int rows, int Hq, int slots,
                                                             Slots sl) {
  constexpr int SPEC = 4;    // slots whose outputs are loaded speculatively
  constexpr int E = D / 64;  // d values per lane
  const int wave = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x >> 6));
  const int lane = threadIdx.x & 63;
  const int row = blockIdx.x * 4 + wave;
  if (row >= rows) return;
  const int64_t base = static_cast<int64_t>(row) * slots;
  float m_l = -INFINITY, l_l = 0.f;  // slot `lane`
  if (lane < slots) {
    m_l = part_ml[2 * (base + lane)];
    l_l = part_ml[2 * (base + lane) + 1];
  }
  float o_spec[SPEC][E];
#pragma unroll
  for (int p = 0; p < SPEC; ++p) {
#pragma unroll
    for (int e = 0; e < E; ++e) o_spec[p][e] = 0.f;
    if (p < slots) {
#pragma unroll
      for (int e = 0; e < E; ++e) o_spec[p][e] = part_o[(base + p) * D + E * lane + e];
    }
  }
  int n0, s1, n1;
  if (!sl(row / Hq, n0, s1, n1)) return;
  auto used = [&](int p) { return p < n0 || (p >= s1 && p < s1 + n1); };
  float M = used(lane) && lane < slots ? m_l : -INFINITY;
  for (int p = lane + 64; p < slots; p += 64)
    if (used(p)) M = fmaxf(M, part_ml[2 * (base + p)]);
  M = wave_max(M);
  const float m_use = (M == -INFINITY) ? 0.f : M;
  float den = used(lane) && lane < slots ? exp2f(m_l - m_use) * l_l : 0.f;
  for (int p = lane + 64; p < slots; p += 64)
    if (used(p)) den += exp2f(part_ml[2 * (base + p)] - m_use) * part_ml[2 * (base + p) + 1];
  den = wave_sum(den);
  float acc[E];
#pragma unroll
  for (int e = 0; e < E; ++e) acc[e] = 0.f;
#pragma unroll
  for (int p = 0; p < SPEC; ++p) {
    if (p < slots && used(p)) {
      const float w = exp2f(__shfl(m_l, p, 64) - m_use);
#pragma unroll
      for (int e = 0; e < E; ++e) acc[e] += w * o_spec[p][e];
    }
  }
  for (int p = SPEC; p < slots; ++p) {
    if (!used(p)) continue;
    const float w = exp2f(part_ml[2 * (base + p)] - m_use);
    const float *po = part_o + (base + p) * D + E * lane;
#pragma unroll
    for (int e = 0; e < E; ++e) acc[e] += w * po[e];
  }
  const float inv = den > 0.f ? 1.f / den : 0.f;
  uint16_t *op = out + static_cast<int64_t>(row) * D + E * lane;
  if constexpr (E == 2)
    *reinterpret_cast<uint32_t *>(op) = f32_to_bf16_bits(acc[0] * inv) | (f32_to_bf16_bits(acc[1] * inv) << 16);
  else
    op[0] = static_cast<uint16_t>(f32_to_bf16_bits(acc[0] * inv));
}

// Slots of decode_gqa_kernel's partials: one per chunk of W partitions; rows of
// a single chunk were written by the decode kernel itself.
struct PlainSlots {
  const int32_t *seq_lens;
  int max_seq;
  int chunk_tokens;  // W * P_tok
  __device__ bool operator()(int b, int &n0, int &s1, int &n1) const {
    int L = seq_lens[b];
    L = L < max_seq ? L : max_seq;
    n0 = L > 0 ? (L + chunk_tokens - 1) / chunk_tokens : 0;
    s1 = 0;
    n1 = 0;
    return n0 > 1;
  }
};

// ---------------------------------------------------------------------------
// Group-aware decode (GRPO groups): sequences g*gs .. g*gs+gs-1 form group g
// and store the group's first prefix tokens in the same physical blocks. One
// launch runs two kinds of workgroups:
//   prefix role: per (group, KV head, prefix partition), the shared blocks are
//     streamed once for all gs*G query rows of the group -- the MFMA columns
//     are (member, head) pairs instead of one sequence's heads, and the W waves
//     of the workgroup take different 16-row tiles of the same tokens, so each
//     tile is fetched from HBM once and served to the others from cache;
//   suffix role: per (sequence, KV head, chunk), the ordinary decode over the
//     sequence's private tokens (with the step's fused append).
// Both leave (m, l, o) partials; merge_partials_kernel combines them.
struct GroupGeom {
  const int32_t *prefix_lens;  // [n_groups] leading tokens the caller declares shared
  int gs;                      // sequences per group (the last group may be short)
  int nrt;                     // 16-row tiles of a group's gs * G query rows
  int nrtb;                    // workgroups per (group, KV head, partition): ceil(nrt / W)
  int p_pre;                   // most tokens per prefix partition (a block multiple)
  int npp;                     // prefix partitions: partial slots 0 .. npp-1
  int nsc;                     // suffix chunks: partial slots npp .. npp+nsc-1
  int n_suf_wgs;               // workgroups of the suffix role (they come first: the
                               // longest-running ones start in the first round)
  int append;                  // 1 when the suffix role appends the step's token
};

// Tokens of group g that the prefix role attends: the declared prefix, cut to
// what every member holds (excluding a token this step appends, whose block an
// fp8 append may rewrite), to the launch's npp partitions, and down to whole
// blocks (so suffix partitions stay block-aligned for the fused append).
// (The members' lengths are read lane-parallel and reduced across the wave: one
// memory round trip, not one per member.) Call with the whole wave active.
__device__ __forceinline__ int group_prefix(const GroupGeom &gg, const int32_t *__restrict__ seq_lens, int g,
                                            int batch, int max_seq, int BS) {
  const int lane = threadIdx.x & 63;
  const int b0 = g * gg.gs;
  const int b1 = (b0 + gg.gs) < batch ? (b0 + gg.gs) : batch;
  int pre = gg.prefix_lens[g];
  for (int b = b0 + lane; b < b1; b += 64) {
    int L = seq_lens[b];
    L = L < max_seq ? L : max_seq;
    L -= gg.append;
    pre = pre < L ? pre : L;
  }
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) {
    const int other = __shfl_xor(pre, o, 64);
    pre = pre < other ? pre : other;
  }
  const int cap = gg.npp * gg.p_pre;
  pre = pre < cap ? pre : cap;
  pre = pre > 0 ? pre : 0;
  return __builtin_amdgcn_readfirstlane(pre / BS * BS);
}

// Tokens per prefix partition of a group whose prefix is pre > 0 tokens: the
// ceil(pre / p_pre) partitions balanced, in whole blocks (<= p_pre).
__device__ __forceinline__ int prefix_partition(int pre, int p_pre, int BS) {
  const int n = (pre + p_pre - 1) / p_pre;
  int p = (pre + n - 1) / n;
  p = (p + BS - 1) / BS * BS;
  return __builtin_amdgcn_readfirstlane(p);
}

template <int D, bool FP8, bool APPEND, int W>
__global__ __launch_bounds__(64 * W) void decode_gqa_grouped_kernel(
    uint8_t *__restrict__ kc, uint8_t *__restrict__ vc, float *__restrict__ ks, float *__restrict__ vs,
    const uint16_t *__restrict__ q, int64_t q_sb, int64_t q_sh, float *__restrict__ part_o,
    float *__restrict__ part_ml, const int32_t *__restrict__ bt, int64_t bt_stride, int Mb, int max_seq,
    const int32_t *__restrict__ seq_lens, int batch, int Hq, int Hkv, int G, int BS, int64_t NB, float scale_log2,
    int P_tok, StepAppend ap, GroupGeom gg) {
  const int wave = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x >> 6));
  const int lane = threadIdx.x & 63, col = lane & 15, grp = lane >> 4;
  const int slots = gg.npp + gg.nsc;
  DecodeState<D, FP8> st;
#pragma unroll
  for (int n = 0; n < D / 16; ++n) st.o[n] = floatx4{0.f, 0.f, 0.f, 0.f};
  st.m = -INFINITY;
  st.l = 0.f;

  if (static_cast<int>(blockIdx.x) >= gg.n_suf_wgs) {
    // ---- prefix role: workgroup (group, KV head, row-tile block, partition)
    int r = static_cast<int>(blockIdx.x) - gg.n_suf_wgs;
    const int p = r % gg.npp;
    r /= gg.npp;
    const int kvh = r % Hkv;
    r /= Hkv;
    const int rt = (r % gg.nrtb) * W + wave;
    const int g = __builtin_amdgcn_readfirstlane(r / gg.nrtb);
    const int pre = group_prefix(gg, seq_lens, g, batch, max_seq, BS);
    if (pre <= 0 || rt >= gg.nrt) return;  // no barrier in this role: waves leave independently
    const int ppart = prefix_partition(pre, gg.p_pre, BS);
    const int t_begin = p * ppart;
    if (t_begin >= pre) return;
    const int t_end = (t_begin + ppart) < pre ? (t_begin + ppart) : pre;
    const int b0 = g * gg.gs;
    // This lane's column is query row rt*16 + col of the group: (member, head).
    const int row = rt * 16 + col;
    const int member = row / G, h = row - member * G;
    const int b = b0 + member;
    const bool valid = member < gg.gs && b < batch;
    const int blk_first = t_begin / BS;
    int my_blk = -1;
    if (blk_first + lane < Mb) my_blk = bt[b0 * bt_stride + blk_first + lane];
    bf16x8 qop[D / 32];
    load_q<D, FP8>(qop, q + (valid ? b : b0) * q_sb + static_cast<int64_t>(kvh * G + (valid ? h : 0)) * q_sh,
                   valid, grp);
    attend_partition<D, FP8>(st, kc, vc, ks, vs, qop, my_blk, t_begin, t_end, kvh, Hkv, BS, NB, scale_log2, lane,
                             col, grp);
    float l = st.l + __shfl_xor(st.l, 16, 64);
    l += __shfl_xor(l, 32, 64);
    if (!valid) return;
    const int64_t prow = (static_cast<int64_t>(b) * Hq + kvh * G + h) * slots + p;
    float *po = part_o + prow * D;
#pragma unroll
    for (int n = 0; n < D / 16; ++n) *reinterpret_cast<floatx4 *>(po + 16 * n + 4 * grp) = st.o[n];
    if (grp == 0) {
      part_ml[2 * prow] = st.m;
      part_ml[2 * prow + 1] = l;
    }
    return;
  }

  // ---- suffix role: workgroup (sequence, KV head, chunk of W partitions)
  int r = blockIdx.x;
  const int chunk = r % gg.nsc;
  r /= gg.nsc;
  const int kvh = r % Hkv;
  const int b = __builtin_amdgcn_readfirstlane(r / Hkv);
  const int pre = group_prefix(gg, seq_lens, b / gg.gs, batch, max_seq, BS);
  int L = seq_lens[b];
  L = L < max_seq ? L : max_seq;
  const int S = L - pre;  // this sequence's own tokens
  const int nchunks = S > 0 ? (S + W * P_tok - 1) / (W * P_tok) : 0;
  if (chunk >= nchunks) return;  // the whole workgroup leaves together
  const int P_seq = balanced_partition(S, W, P_tok, BS);
  const int part = chunk * W + wave;
  const int t_begin = pre + part * P_seq;
  const int blk_first = t_begin / BS;
  int my_blk = -1;
  if (blk_first + lane < Mb) my_blk = bt[b * bt_stride + blk_first + lane];
  bf16x8 qop[D / 32];
  load_q<D, FP8>(qop, q + b * q_sb + static_cast<int64_t>(kvh * G + (col < G ? col : 0)) * q_sh, col < G, grp);
  const int nparts = (S + P_seq - 1) / P_seq;
  const bool active = part < nparts;
  const bool owns_new = APPEND && part == nparts - 1;

  // Fused append, as in decode_gqa_kernel: the new token's block lies wholly in
  // the last suffix partition (pre and P_tok are block multiples).
  uint32_t nk = 0, nv = 0;
  int64_t slot = -1;
  if constexpr (APPEND) {
    if (owns_new) {
      slot = ap.slots[b];
      if constexpr (FP8) {
        if (slot >= 0 && slot / BS < NB) {
          const int64_t blk = slot / BS;
          const int off = static_cast<int>(slot % BS);
          fp8_append_one<D, false>(kc, ks, ap.key, ap.kst, ap.ksh, ap.slots, b, 1, blk, off, kvh, Hkv, BS);
          fp8_append_one<D, true>(vc, vs, ap.val, ap.vst, ap.vsh, ap.slots, b, 1, blk, off, kvh, Hkv, BS);
        }
        __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "workgroup");
      } else {
        if (lane < D / 2) {
          nk = reinterpret_cast<const uint32_t *>(ap.key + b * ap.kst + kvh * ap.ksh)[lane];
          nv = reinterpret_cast<const uint32_t *>(ap.val + b * ap.vst + kvh * ap.vsh)[lane];
        }
      }
    }
  }
  if (active) {
    const int t_end = (t_begin + P_seq) < L ? (t_begin + P_seq) : L;
    const bool from_regs = APPEND && !FP8 && owns_new;
    attend_partition<D, FP8>(st, kc, vc, ks, vs, qop, my_blk, t_begin, from_regs ? L - 1 : t_end, kvh, Hkv, BS,
                             NB, scale_log2, lane, col, grp);
    if constexpr (APPEND && !FP8) {
      if (owns_new) {
        Tile<D, FP8> tn;
        new_token_tile<D>(tn, nk, nv, col, grp);
        attend_tile<D, FP8>(st, tn, qop, scale_log2, grp);
        if (slot >= 0 && slot / BS < NB && lane < D / 2) {
          const int64_t nblk_id = slot / BS;
          const int off = static_cast<int>(slot % BS);
          uint16_t *kd = reinterpret_cast<uint16_t *>(kc) +
                         (((nblk_id * Hkv + kvh) * (D / 8) + (lane >> 2)) * BS + off) * 8 + (lane & 3) * 2;
          *reinterpret_cast<uint32_t *>(kd) = nk;
          uint16_t *vd = reinterpret_cast<uint16_t *>(vc) + ((nblk_id * Hkv + kvh) * D + 2 * lane) * BS + off;
          vd[0] = static_cast<uint16_t>(nv & 0xffffu);
          vd[BS] = static_cast<uint16_t>(nv >> 16);
        }
      }
    }
  }
  float l = st.l + __shfl_xor(st.l, 16, 64);
  l += __shfl_xor(l, 32, 64);
  // Merge the W waves through LDS into this chunk's partial (slot npp + chunk).
  __shared__ float sm_o[W][16][D];
  __shared__ float sm_m[W][16], sm_l[W][16];
  if (col < G) {
#pragma unroll
    for (int n = 0; n < D / 16; ++n) *reinterpret_cast<floatx4 *>(&sm_o[wave][col][16 * n + 4 * grp]) = st.o[n];
    if (grp == 0) {
      sm_m[wave][col] = st.m;
      sm_l[wave][col] = l;
    }
  }
  __syncthreads();
  for (int e = threadIdx.x; e < G * D; e += 64 * W) {
    const int h = e / D, d = e % D;
    float M = -INFINITY;
#pragma unroll
    for (int w = 0; w < W; ++w) M = fmaxf(M, sm_m[w][h]);
    const float m_use = (M == -INFINITY) ? 0.f : M;
    float num = 0.f, den = 0.f;
#pragma unroll
    for (int w = 0; w < W; ++w) {
      const float f = exp2f(sm_m[w][h] - m_use);
      num += f * sm_o[w][h][d];
      den += f * sm_l[w][h];
    }
    const int64_t prow = (static_cast<int64_t>(b) * Hq + kvh * G + h) * slots + gg.npp + chunk;
    part_o[prow * D + d] = num;
    if (d == 0) {
      part_ml[2 * prow] = M;
      part_ml[2 * prow + 1] = den;
    }
  }
}

// Slots of a grouped decode's partials: the prefix partitions' [0, n_pre) and
// the suffix chunks' [npp, npp + n_suf), counted exactly as the kernel above
// cuts them; every row is merged.
struct GroupSlots {
  GroupGeom gg;
  const int32_t *seq_lens;
  int max_seq, batch, BS, chunk_tokens;  // chunk_tokens = W * P_tok
  __device__ bool operator()(int b, int &n0, int &s1, int &n1) const {
    const int pre = group_prefix(gg, seq_lens, b / gg.gs, batch, max_seq, BS);
    int L = seq_lens[b];
    L = L < max_seq ? L : max_seq;
    n0 = 0;
    if (pre > 0) {
      const int ppart = prefix_partition(pre, gg.p_pre, BS);
      n0 = (pre + ppart - 1) / ppart;
    }
    s1 = gg.npp;
    n1 = L > pre ? (L - pre + chunk_tokens - 1) / chunk_tokens : 0;
    return true;
  }
};

// Tokens per partition when the caller leaves it to the library: enough
// work items to give every CU a full complement of resident waves in about
// one round (fewer, longer waves amortise the per-wave prologue and the
// partial-result traffic), at least 128 tokens, a multiple of the block size
// (the fused append relies on it), and at most 64 blocks (one lane each).
static int choose_partition(int batch, int hkv, int max_seq_len, int BS, int D) {
  const int64_t target_waves = D == 128 ? 2048 : 4096;
  const int64_t items = static_cast<int64_t>(batch) * hkv;
  int64_t p = (items * max_seq_len + target_waves - 1) / target_waves;
  const int64_t unit = BS;  // a multiple of 16 already
  p = (p + unit - 1) / unit * unit;
  const int64_t lo = (128 + unit - 1) / unit * unit;
  int64_t hi = 1024 / unit * unit;
  if (hi < unit) hi = unit;
  if (hi > 64 * unit) hi = 64 * unit;
  if (p < lo) p = lo;
  if (p > hi) p = hi;
  return static_cast<int>(p);
}

}  // namespace wkv

using namespace wkv;

extern "C" int64_t wkv_decode_workspace_size(int32_t batch, int32_t num_q_heads, int32_t head_dim,
                                             int32_t max_seq_len, int32_t partition_size) {
  if (batch < 0 || num_q_heads <= 0 || head_dim <= 0 || max_seq_len < 0 || partition_size < 0) return -1;
  if (partition_size == 0) partition_size = 128;  // smallest partition the library picks by itself
  const int64_t max_parts = (static_cast<int64_t>(max_seq_len) + partition_size - 1) / partition_size;
  // partial outputs and (max, sum) per (sequence, query head, partition)
  return static_cast<int64_t>(batch) * num_q_heads * (max_parts > 0 ? max_parts : 1) * (head_dim + 2) * 4;
}

namespace wkv {

static int launch_decode(const wkv_cache_t *cache, const void *q, int64_t q_stride_b, int64_t q_stride_h, void *out,
                         int32_t num_q_heads, const int32_t *block_table, int64_t bt_stride,
                         int32_t max_blocks_per_seq, const int32_t *seq_lens, int32_t batch, int32_t max_seq_len,
                         float scale, int32_t partition_size, void *workspace, int64_t workspace_bytes,
                         const StepAppend *ap, void *stream) {
  int rc = check_cache(cache, -1);
  if (rc) return rc;
  WKV_CHECK_ARG(batch >= 0 && batch <= 65535, "batch must be in [0, 65535] (got %d)", batch);
  if (batch == 0) return WKV_OK;
  const int Hkv = cache->num_kv_heads, D = cache->head_dim, BS = cache->block_size;
  WKV_CHECK_ARG(num_q_heads > 0 && num_q_heads % Hkv == 0, "num_q_heads %d must be a multiple of num_kv_heads %d",
                num_q_heads, Hkv);
  const int G = num_q_heads / Hkv;
  if (G > 16) return fail(WKV_ERR_UNSUPPORTED, "query group size %d > 16 not supported", G);
  WKV_CHECK_ARG(static_cast<int64_t>(batch) * num_q_heads < INT32_MAX - 4, "batch * num_q_heads too large");
  WKV_CHECK_ARG(Hkv <= 65535, "num_kv_heads too large");
  WKV_CHECK_ARG(cache->num_blocks * Hkv <= INT32_MAX, "num_blocks * num_kv_heads must be below 2^31");
  WKV_CHECK_ARG(q != nullptr && aligned16(q), "q must be non-NULL and 16-byte aligned");
  WKV_CHECK_ARG(q_stride_b >= 0 && q_stride_h >= 0 && q_stride_b % 8 == 0 && q_stride_h % 8 == 0,
                "q strides must be non-negative multiples of 8");
  WKV_CHECK_ARG(out != nullptr && aligned16(out), "out must be non-NULL and 16-byte aligned");
  WKV_CHECK_ARG(block_table != nullptr && seq_lens != nullptr, "block_table / seq_lens is NULL");
  WKV_CHECK_ARG(max_blocks_per_seq > 0 && bt_stride >= max_blocks_per_seq, "bad block table geometry");
  WKV_CHECK_ARG(max_seq_len >= 0, "max_seq_len must be >= 0");
  WKV_CHECK_ARG(std::isfinite(scale), "scale must be finite");
  const int max_seq = max_seq_len < max_blocks_per_seq * BS ? max_seq_len : max_blocks_per_seq * BS;
  if (partition_size == 0) partition_size = choose_partition(batch, Hkv, max_seq, BS, D);
  WKV_CHECK_ARG(partition_size >= 16 && partition_size % 16 == 0, "partition_size must be a positive multiple of 16");
  WKV_CHECK_ARG((partition_size + BS - 17) / BS + 1 <= 64,
                "partition_size %d spans more than 64 blocks of %d tokens", partition_size, BS);
  if (ap != nullptr)
    WKV_CHECK_ARG(partition_size % BS == 0, "a fused append needs partition_size %d to be a multiple of block_size %d",
                  partition_size, BS);
  const int max_parts = max_seq > 0 ? (max_seq + partition_size - 1) / partition_size : 1;
  // Waves per workgroup: partitions of one context share a workgroup (and an
  // LDS merge) up to 4 at a time; longer contexts leave per-chunk partials.
  const int W = max_parts <= 1 ? 1 : (max_parts <= 2 ? 2 : 4);
  const int max_chunks = (max_parts + W - 1) / W;
  WKV_CHECK_ARG(max_chunks <= 65535, "too many partitions (%d)", max_parts);
  const int64_t need = wkv_decode_workspace_size(batch, num_q_heads, D, max_seq, partition_size * W);
  if (max_chunks > 1)
    WKV_CHECK_ARG(workspace != nullptr && aligned16(workspace) && workspace_bytes >= need,
                  "workspace too small: need %lld bytes, got %lld", (long long)need, (long long)workspace_bytes);
  float *part_o = static_cast<float *>(workspace);
  float *part_ml = part_o ? part_o + static_cast<int64_t>(batch) * num_q_heads * max_chunks * D : nullptr;
  const float scale_log2 = scale * 1.4426950408889634f;
  auto s = static_cast<hipStream_t>(stream);
  const dim3 grid(static_cast<unsigned>(max_chunks), static_cast<unsigned>(Hkv), static_cast<unsigned>(batch));
  auto kc = static_cast<uint8_t *>(cache->k);
  auto vc = static_cast<uint8_t *>(cache->v);
  auto qq = static_cast<const uint16_t *>(q);
  auto oo = static_cast<uint16_t *>(out);
  const bool fp8 = cache->kv_dtype == WKV_KV_FP8_E4M3;
  const StepAppend none{nullptr, 0, 0, nullptr, 0, 0, nullptr};
  const StepAppend apv = ap ? *ap : none;
#define WKV_DECODE(Dv, F8, AP, Wv)                                                                              \
  decode_gqa_kernel<Dv, F8, AP, Wv><<<grid, 64 * Wv, 0, s>>>(kc, vc, cache->k_scale, cache->v_scale, qq,       \
                                                             q_stride_b, q_stride_h, oo, part_o, part_ml,      \
                                                             block_table, bt_stride, max_blocks_per_seq,       \
                                                             max_seq, seq_lens,                                \
                                                             num_q_heads, Hkv, G, BS, cache->num_blocks,       \
                                                             scale_log2, partition_size, max_chunks, apv)
#define WKV_DECODE_W(Dv, F8, AP)   \
  do {                             \
    if (W == 1)                    \
      WKV_DECODE(Dv, F8, AP, 1);   \
    else if (W == 2)               \
      WKV_DECODE(Dv, F8, AP, 2);   \
    else                           \
      WKV_DECODE(Dv, F8, AP, 4);   \
  } while (0)
  if (D == 128) {
    if (fp8) { if (ap) WKV_DECODE_W(128, true, true); else WKV_DECODE_W(128, true, false); }
    else { if (ap) WKV_DECODE_W(128, false, true); else WKV_DECODE_W(128, false, false); }
  } else {
    if (fp8) { if (ap) WKV_DECODE_W(64, true, true); else WKV_DECODE_W(64, true, false); }
    else { if (ap) WKV_DECODE_W(64, false, true); else WKV_DECODE_W(64, false, false); }
  }
#undef WKV_DECODE_W
#undef WKV_DECODE
  WKV_CHECK_LAUNCH("paged decode");
  if (max_chunks > 1) {
    const int rows = batch * num_q_heads;
    const PlainSlots ps{seq_lens, max_seq, partition_size * W};
    if (D == 128)
      merge_partials_kernel<128><<<(rows + 3) / 4, 256, 0, s>>>(part_o, part_ml, oo, rows, num_q_heads, max_chunks, ps);
    else
      merge_partials_kernel<64><<<(rows + 3) / 4, 256, 0, s>>>(part_o, part_ml, oo, rows, num_q_heads, max_chunks, ps);
    WKV_CHECK_LAUNCH("paged decode merge");
  }
  return WKV_OK;
}

// Grouped decode: the prefix role's workgroups hold kGroupW waves (row tiles),
// the suffix role's as many partitions.
constexpr int kGroupW = 4;

static int grouped_partition(int32_t partition_size, int batch, int hkv, int max_seq, int BS, int D) {
  return partition_size != 0 ? partition_size : choose_partition(batch, hkv, max_seq, BS, D);
}

// Most tokens per prefix partition: about what the longest suffix gives each
// of its waves (prefix workgroups then last no longer than suffix ones), at
// least an eighth of the prefix (few partials), in whole blocks, within [BS, P].
static int64_t grouped_prefix_partition(int64_t max_seq, int64_t max_prefix, int64_t P, int64_t BS) {
  const int64_t pre = max_prefix < max_seq ? max_prefix : max_seq;
  int64_t p = (max_seq - pre + kGroupW - 1) / kGroupW;
  const int64_t eighth = (pre + 7) / 8;
  if (p < eighth) p = eighth;
  p = (p + BS - 1) / BS * BS;
  if (p > P) p = P;
  if (p < BS) p = BS;
  return p;
}

// Partial slots per (sequence, query head): prefix partitions, then suffix chunks.
static void grouped_slots(int64_t max_seq, int64_t max_prefix, int64_t P, int64_t BS, int64_t *npp, int64_t *nsc,
                          int64_t *p_pre) {
  const int64_t pre = max_prefix < max_seq ? max_prefix : max_seq;
  *p_pre = grouped_prefix_partition(max_seq, max_prefix, P, BS);
  *npp = (pre + *p_pre - 1) / *p_pre;
  *nsc = (max_seq + kGroupW * P - 1) / (kGroupW * P);
  if (*nsc < 1) *nsc = 1;
}

static int launch_grouped(const wkv_cache_t *cache, const StepAppend *ap, const void *q, int64_t q_stride_b,
                          int64_t q_stride_h, void *out, int32_t num_q_heads, const int32_t *block_table,
                          int64_t bt_stride, int32_t max_blocks_per_seq, const int32_t *seq_lens, int32_t batch,
                          int32_t max_seq_len, const int32_t *prefix_lens, int32_t group_size,
                          int32_t max_prefix_len, float scale, int32_t partition_size, void *workspace,
                          int64_t workspace_bytes, void *stream) {
  int rc = check_cache(cache, -1);
  if (rc) return rc;
  WKV_CHECK_ARG(batch >= 0 && batch <= 65535, "batch must be in [0, 65535] (got %d)", batch);
  if (batch == 0) return WKV_OK;
  const int Hkv = cache->num_kv_heads, D = cache->head_dim, BS = cache->block_size;
  WKV_CHECK_ARG(num_q_heads > 0 && num_q_heads % Hkv == 0, "num_q_heads %d must be a multiple of num_kv_heads %d",
                num_q_heads, Hkv);
  const int G = num_q_heads / Hkv;
  if (G > 16) return fail(WKV_ERR_UNSUPPORTED, "query group size %d > 16 not supported", G);
  WKV_CHECK_ARG(static_cast<int64_t>(batch) * num_q_heads < INT32_MAX - 4, "batch * num_q_heads too large");
  WKV_CHECK_ARG(Hkv <= 65535, "num_kv_heads too large");
  WKV_CHECK_ARG(cache->num_blocks * Hkv <= INT32_MAX, "num_blocks * num_kv_heads must be below 2^31");
  WKV_CHECK_ARG(q != nullptr && aligned16(q), "q must be non-NULL and 16-byte aligned");
  WKV_CHECK_ARG(q_stride_b >= 0 && q_stride_h >= 0 && q_stride_b % 8 == 0 && q_stride_h % 8 == 0,
                "q strides must be non-negative multiples of 8");
  WKV_CHECK_ARG(out != nullptr && aligned16(out), "out must be non-NULL and 16-byte aligned");
  WKV_CHECK_ARG(block_table != nullptr && seq_lens != nullptr, "block_table / seq_lens is NULL");
  WKV_CHECK_ARG(max_blocks_per_seq > 0 && bt_stride >= max_blocks_per_seq, "bad block table geometry");
  WKV_CHECK_ARG(max_seq_len >= 0, "max_seq_len must be >= 0");
  WKV_CHECK_ARG(std::isfinite(scale), "scale must be finite");
  WKV_CHECK_ARG(prefix_lens != nullptr, "prefix_lens is NULL");
  WKV_CHECK_ARG(group_size >= 1 && group_size <= batch, "group_size must be in [1, batch] (got %d)", group_size);
  WKV_CHECK_ARG(max_prefix_len >= 0, "max_prefix_len must be >= 0");
  const int max_seq = max_seq_len < max_blocks_per_seq * BS ? max_seq_len : max_blocks_per_seq * BS;
  const int P = grouped_partition(partition_size, batch, Hkv, max_seq, BS, D);
  WKV_CHECK_ARG(P >= 16 && P % BS == 0, "partition_size %d must be a positive multiple of block_size %d", P, BS);
  WKV_CHECK_ARG(P / BS <= 64, "partition_size %d spans more than 64 blocks of %d tokens", P, BS);
  const int n_groups = (batch + group_size - 1) / group_size;
  int64_t npp, nsc, p_pre;
  grouped_slots(max_seq, max_prefix_len, P, BS, &npp, &nsc, &p_pre);
  const int64_t slots = npp + nsc;
  GroupGeom gg;
  gg.prefix_lens = prefix_lens;
  gg.gs = group_size;
  gg.nrt = (group_size * G + 15) / 16;
  gg.nrtb = (gg.nrt + kGroupW - 1) / kGroupW;
  gg.p_pre = static_cast<int>(p_pre);
  gg.npp = static_cast<int>(npp);
  gg.nsc = static_cast<int>(nsc);
  gg.append = ap != nullptr ? 1 : 0;
  const int64_t n_pre = static_cast<int64_t>(n_groups) * Hkv * gg.nrtb * gg.npp;
  const int64_t n_suf = static_cast<int64_t>(batch) * Hkv * gg.nsc;
  WKV_CHECK_ARG(n_pre + n_suf <= INT32_MAX, "grouped decode grid too large");
  gg.n_suf_wgs = static_cast<int>(n_suf);
  const int64_t need = static_cast<int64_t>(batch) * num_q_heads * slots * (D + 2) * 4;
  WKV_CHECK_ARG(workspace != nullptr && aligned16(workspace) && workspace_bytes >= need,
                "workspace too small: need %lld bytes, got %lld", (long long)need, (long long)workspace_bytes);
  float *part_o = static_cast<float *>(workspace);
  float *part_ml = part_o + static_cast<int64_t>(batch) * num_q_heads * slots * D;
  const float scale_log2 = scale * 1.4426950408889634f;
  auto s = static_cast<hipStream_t>(stream);
  auto kc = static_cast<uint8_t *>(cache->k);
  auto vc = static_cast<uint8_t *>(cache->v);
  auto qq = static_cast<const uint16_t *>(q);
  const bool fp8 = cache->kv_dtype == WKV_KV_FP8_E4M3;
  const StepAppend none{nullptr, 0, 0, nullptr, 0, 0, nullptr};
  const StepAppend apv = ap ? *ap : none;
  const dim3 grid(static_cast<unsigned>(n_pre + n_suf));
#define WKV_GROUPED(Dv, F8, AP)                                                                                 \
  decode_gqa_grouped_kernel<Dv, F8, AP, kGroupW><<<grid, 64 * kGroupW, 0, s>>>(                                \
      kc, vc, cache->k_scale, cache->v_scale, qq, q_stride_b, q_stride_h, part_o, part_ml, block_table,         \
      bt_stride, max_blocks_per_seq, max_seq, seq_lens, batch, num_q_heads, Hkv, G, BS, cache->num_blocks,       \
      scale_log2, P, apv, gg)
  if (D == 128) {
    if (fp8) { if (ap) WKV_GROUPED(128, true, true); else WKV_GROUPED(128, true, false); }
    else { if (ap) WKV_GROUPED(128, false, true); else WKV_GROUPED(128, false, false); }
  } else {
    if (fp8) { if (ap) WKV_GROUPED(64, true, true); else WKV_GROUPED(64, true, false); }
    else { if (ap) WKV_GROUPED(64, false, true); else WKV_GROUPED(64, false, false); }
  }
#undef WKV_GROUPED
  WKV_CHECK_LAUNCH("grouped paged decode");
  auto oo = static_cast<uint16_t *>(out);
  const int rows = batch * num_q_heads;
  const GroupSlots gs{gg, seq_lens, max_seq, batch, BS, kGroupW * P};
  if (D == 128)
    merge_partials_kernel<128><<<(rows + 3) / 4, 256, 0, s>>>(part_o, part_ml, oo, rows, num_q_heads,
                                                              static_cast<int>(slots), gs);
  else
    merge_partials_kernel<64><<<(rows + 3) / 4, 256, 0, s>>>(part_o, part_ml, oo, rows, num_q_heads,
                                                             static_cast<int>(slots), gs);
  WKV_CHECK_LAUNCH("grouped paged decode merge");
  return WKV_OK;
}

}  // namespace wkv

extern "C" int64_t wkv_grouped_decode_workspace_size(int32_t batch, int32_t num_q_heads, int32_t head_dim,
                                                     int32_t max_seq_len, int32_t max_prefix_len,
                                                     int32_t partition_size) {
  if (batch < 0 || num_q_heads <= 0 || head_dim <= 0 || max_seq_len < 0 || max_prefix_len < 0 || partition_size < 0)
    return -1;
  // The smallest partition the library picks by itself, and the smallest block
  // (both give the most slots).
  if (partition_size == 0) partition_size = 128;
  int64_t npp, nsc, p_pre;
  wkv::grouped_slots(max_seq_len, max_prefix_len, partition_size, 16, &npp, &nsc, &p_pre);
  return static_cast<int64_t>(batch) * num_q_heads * (npp + nsc) * (head_dim + 2) * 4;
}

extern "C" int wkv_paged_decode_gqa_grouped(const wkv_cache_t *cache, const void *key, int64_t key_stride_t,
                                            int64_t key_stride_h, const void *value, int64_t value_stride_t,
                                            int64_t value_stride_h, const int64_t *slot_mapping, const void *q,
                                            int64_t q_stride_b, int64_t q_stride_h, void *out, int32_t num_q_heads,
                                            const int32_t *block_table, int64_t bt_stride,
                                            int32_t max_blocks_per_seq, const int32_t *seq_lens, int32_t batch,
                                            int32_t max_seq_len, const int32_t *prefix_lens, int32_t group_size,
                                            int32_t max_prefix_len, float scale, int32_t partition_size,
                                            void *workspace, int64_t workspace_bytes, void *stream) {
  using namespace wkv;
  StepAppend ap{};
  const bool append = key != nullptr || value != nullptr || slot_mapping != nullptr;
  if (append) {
    WKV_CHECK_ARG(key && value && aligned16(key) && aligned16(value),
                  "key/value must be non-NULL and 16-byte aligned (or all of key, value, slot_mapping NULL)");
    WKV_CHECK_ARG(key_stride_t >= 0 && key_stride_h >= 0 && value_stride_t >= 0 && value_stride_h >= 0 &&
                      (key_stride_t | key_stride_h | value_stride_t | value_stride_h) % 8 == 0,
                  "key/value strides must be non-negative multiples of 8");
    WKV_CHECK_ARG(slot_mapping != nullptr, "slot_mapping is NULL");
    ap = StepAppend{static_cast<const uint16_t *>(key), key_stride_t, key_stride_h,
                    static_cast<const uint16_t *>(value), value_stride_t, value_stride_h, slot_mapping};
  }
  return launch_grouped(cache, append ? &ap : nullptr, q, q_stride_b, q_stride_h, out, num_q_heads, block_table,
                        bt_stride, max_blocks_per_seq, seq_lens, batch, max_seq_len, prefix_lens, group_size,
                        max_prefix_len, scale, partition_size, workspace, workspace_bytes, stream);
}

extern "C" int wkv_paged_decode_gqa(const wkv_cache_t *cache, const void *q, int64_t q_stride_b,
                                    int64_t q_stride_h, void *out, int32_t num_q_heads,
                                    const int32_t *block_table, int64_t bt_stride, int32_t max_blocks_per_seq,
                                    const int32_t *seq_lens, int32_t batch, int32_t max_seq_len, float scale,
                                    int32_t partition_size, void *workspace, int64_t workspace_bytes, void *stream) {
  return launch_decode(cache, q, q_stride_b, q_stride_h, out, num_q_heads, block_table, bt_stride,
                       max_blocks_per_seq, seq_lens, batch, max_seq_len, scale, partition_size, workspace,
                       workspace_bytes, nullptr, stream);
}

extern "C" int wkv_append_paged_decode_gqa(const wkv_cache_t *cache, const void *key, int64_t key_stride_t,
                                           int64_t key_stride_h, const void *value, int64_t value_stride_t,
                                           int64_t value_stride_h, const int64_t *slot_mapping, const void *q,
                                           int64_t q_stride_b, int64_t q_stride_h, void *out, int32_t num_q_heads,
                                           const int32_t *block_table, int64_t bt_stride,
                                           int32_t max_blocks_per_seq, const int32_t *seq_lens, int32_t batch,
                                           int32_t max_seq_len, float scale, int32_t partition_size,
                                           void *workspace, int64_t workspace_bytes, void *stream) {
  WKV_CHECK_ARG(key && value && aligned16(key) && aligned16(value), "key/value must be non-NULL and 16-byte aligned");
  WKV_CHECK_ARG(key_stride_t >= 0 && key_stride_h >= 0 && value_stride_t >= 0 && value_stride_h >= 0 &&
                    (key_stride_t | key_stride_h | value_stride_t | value_stride_h) % 8 == 0,
                "key/value strides must be non-negative multiples of 8");
  WKV_CHECK_ARG(slot_mapping != nullptr, "slot_mapping is NULL");
  if (cache != nullptr && cache->kv_dtype == WKV_KV_FP8_E4M3)
    WKV_CHECK_ARG(cache->k_scale && cache->v_scale, "fp8 cache needs k_scale and v_scale");
  const StepAppend ap{static_cast<const uint16_t *>(key), key_stride_t, key_stride_h,
                      static_cast<const uint16_t *>(value), value_stride_t, value_stride_h, slot_mapping};
  return launch_decode(cache, q, q_stride_b, q_stride_h, out, num_q_heads, block_table, bt_stride,
                       max_blocks_per_seq, seq_lens, batch, max_seq_len, scale, partition_size, workspace,
                       workspace_bytes, &ap, stream);
}
