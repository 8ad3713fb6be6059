// The 16-token tile machinery shared by the GQA decode and prefill kernels
// (gfx950, wave64): loading a tile of the paged cache straight into MFMA
// operand registers, and one tile of online-softmax attention on them.
//
//   K [NB, Hkv, D/x, BS, x]: for chunk c the 16 tokens of a tile are 256
//      contiguous bytes, so the four chunks a QK MFMA needs are one 1 KB
//      contiguous wave load.
//   V [NB, Hkv, D, BS]: one head_dim row holds the block's tokens
//      contiguously, which is the A-operand (row = d, k = token) of the PV
//      MFMA without any transpose (fp8: after a 4x4 lane transpose).
//
// Per tile:   S^T[16 tok, 16 cols] = K[16 tok, D] . Q^T[D, 16 cols]
//             (D/32 x mfma_f32_16x16x32_bf16; a column is one query row)
//             online softmax on S^T (lane = column, 4 tokens per lane)
//             O^T[D, 16 cols] += V^T[D, 16 tok] . P^T[16 tok, 16 cols]
//             (D/16 x mfma_f32_16x16x16_bf16; the QK output registers are
//             exactly the B operand, so P never leaves the lane)
// fp8 caches are widened to bf16 in registers (exact) and their power-of-two
// per-(block, head) scales are folded into the scores (K) and into P (V).
#pragma once

#include <cmath>

#include "wkv_common.h"

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
  int ts;                   // position of the tile's first token
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

// Cache policy of a tile load: 0 = default; kStreamLoad sets the load's
// non-temporal bit (nt), for data read once. Measured on MI355X: a plain
// streaming read reaches 7.1 TB/s with nt and 6.4 without; the decode of
// unshared blocks gains 3-9%, while blocks that several sequences read
// (shared prefixes) lose their reuse in the caches and read 15% slower.
constexpr int kStreamLoad = 2;

// Issues the loads of one 16-token tile (tokens [o0, o0+16) of block blk) as
// buffer loads: a wave-uniform resource (scalar registers) per (block, head)
// region, a per-lane byte offset that never changes (koff, voff) and a scalar
// offset per load, so no per-tile vector address arithmetic is needed.
// live (wave-uniform) = false gives the resources zero records: every load is
// then out of range, returns zeros and reads no memory, yet is issued and
// counted like any other, so the pipeline's wait counts do not change.
template <int D, bool FP8, int AUX>
__device__ __forceinline__ void load_tile_as(Tile<D, FP8> &t, const uint8_t *__restrict__ kc,
                                             const uint8_t *__restrict__ vc, int blk, int kvh, int Hkv, int BS,
                                             int o0, uint32_t koff, uint32_t voff, bool live) {
  constexpr int ESZ = FP8 ? 1 : 2;
  const int region = D * BS * ESZ;  // bytes of one (block, head) region of K, and of V
  const int nrec = live ? region : 0;
  // Region index in 32 bits (the host keeps num_blocks * num_kv_heads below
  // 2^31), in a scalar register, so the 64-bit address arithmetic stays scalar.
  const int ridx = __builtin_amdgcn_readfirstlane(blk * Hkv + kvh);
  const int64_t rbase = static_cast<int64_t>(ridx) * region;
  const uint8_t *kb = wave_uniform(kc + rbase + o0 * 16);
  const __amdgpu_buffer_rsrc_t kr = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t *>(kb), 0, nrec, kRawBufferWord3);
#pragma unroll
  for (int j = 0; j < Tile<D, FP8>::NK; ++j)
    t.k[j] = __builtin_amdgcn_raw_buffer_load_b128(kr, koff, j * 4 * BS * 16, AUX);
  const uint8_t *vb = wave_uniform(vc + rbase + o0 * ESZ);
  const __amdgpu_buffer_rsrc_t vr = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t *>(vb), 0, nrec, kRawBufferWord3);
  if constexpr (FP8) {
    // Lane (m, g) loads d row 64j + 16g + m whole (16 tokens, 16 bytes): 1 KB
    // per wave load instead of 256 B -- 4-byte loads cap HBM near half its rate.
#pragma unroll
    for (int j = 0; j < Tile<D, FP8>::NPV / 4; ++j)
      t.v4[j] = __builtin_amdgcn_raw_buffer_load_b128(vr, voff, j * 64 * BS, AUX);
  } else {
#pragma unroll
    for (int n = 0; n < Tile<D, FP8>::NPV; ++n)
      t.v[n] = __builtin_amdgcn_raw_buffer_load_b64(vr, voff, n * 16 * BS * 2, AUX);
  }
}

// stream is wave-uniform: one scalar branch per tile.
template <int D, bool FP8>
__device__ __forceinline__ void load_tile(Tile<D, FP8> &t, const uint8_t *__restrict__ kc,
                                          const uint8_t *__restrict__ vc, int blk, int kvh, int Hkv, int BS,
                                          int o0, uint32_t koff, uint32_t voff, bool stream, bool live = true) {
  if (stream)
    load_tile_as<D, FP8, kStreamLoad>(t, kc, vc, blk, kvh, Hkv, BS, o0, koff, voff, live);
  else
    load_tile_as<D, FP8, 0>(t, kc, vc, blk, kvh, Hkv, BS, o0, koff, voff, live);
}

template <int D, bool FP8>
struct DecodeState {
  floatx4 o[D / 16];
  float m;  // running max (log2 domain) of this lane's head column
  float l;  // this lane's share of the running denominator
};

// One tile of online-softmax attention. CAUSAL: this lane's column sees only
// the tile's first `col_lim` tokens (a per-lane limit, 0..16; prefill's causal
// diagonal), on top of the tile's `valid`.
template <int D, bool FP8, bool CAUSAL = false>
__device__ __forceinline__ void attend_tile(DecodeState<D, FP8> &st, const Tile<D, FP8> &t, const bf16x8 *qop,
                                            float scale_log2, int grp, int col_lim = 16) {
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
  if constexpr (CAUSAL) {
    if (col_lim < 16) {
#pragma unroll
      for (int i = 0; i < 4; ++i)
        if (4 * grp + i >= col_lim) sv[i] = -INFINITY;
    }
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
    if (t.valid < 16) {
      // Never let a masked slot's V reach the accumulator (it may hold NaN):
      // code 0 is +0, widened to the bf16 zero. Byte e of every dword is
      // token 4 grp + e; one mask for all of them.
      const int keep = t.valid - 4 * grp;
      const uint32_t m = keep >= 4 ? 0xffffffffu : (keep <= 0 ? 0u : (1u << (8 * keep)) - 1u);
#pragma unroll
      for (int n = 0; n < D / 16; ++n) v8[n] &= m;
    }
  }
#pragma unroll
  for (int n = 0; n < D / 16; ++n) {
    shortx4 vop = FP8 ? fp8x4_to_bf16x4(v8[FP8 ? n : 0]) : __builtin_bit_cast(shortx4, t.v[FP8 ? 0 : n]);
    if (!FP8 && t.valid < 16) {
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

// Tiles a wave keeps in registers: one being attended while two load. Deeper
// rotations (4-6 tiles) measured slower on every decode workload: the extra
// registers cost occupancy, and a loads-only variant at depth 2 streams as
// fast as at depth 6 (the memory pipeline, not the wave's latency, binds).
template <int D, bool FP8>
constexpr int pipeline_depth() {
  return 3;
}

// The tile loop of one wave over tokens [t_begin, t_end) of a block list:
// `consume(tile)` attends each 16-token tile. `my_blk` holds, in lane i, the
// id of the range's i-th block (loaded by the caller; the host keeps a range
// within 64 blocks); each tile takes its id with a register readlane.
template <int D, bool FP8, typename Consume>
__device__ __forceinline__ void attend_range(Consume &&consume, const uint8_t *__restrict__ kc,
                                             const uint8_t *__restrict__ vc, const float *__restrict__ ks,
                                             const float *__restrict__ vs, int my_blk, int t_begin, int t_end,
                                             int kvh, int Hkv, int BS, int64_t NB, int lane, int col, int grp,
                                             bool stream) {
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

  // Issue tile i's loads unconditionally so the compiler can count
  // outstanding loads and wait only for the tile about to be used: three
  // tiles rotate, two in flight. A tile past the end (or of an unmapped
  // block) is issued with a zero-record resource: no memory is read for it
  // (re-reading the last tile instead cost 4% more HBM reads once the tiles
  // were loaded non-temporally, as the re-read no longer hit the L2).
  // Tile i's first token, its block (relative to blk_first) and its offset in
  // that block, kept as counters: issue() is called for i = 0, 1, 2, ... in
  // order, and a tile past the end keeps the last tile's position (its loads
  // read nothing). A division by the runtime block size per tile cost about
  // 20 scalar instructions.
  int c_ts = t_begin, c_bi = 0, c_off = t_begin - blk_first * BS;
  auto issue = [&](Tile<D, FP8> &t, int i) {
    const int ts = c_ts, bi = c_bi, o0 = c_off;
    if (i + 1 < n_tiles) {  // uniform: 16 tokens on, at most one block boundary (BS is a multiple of 16)
      c_ts += 16;
      c_off += 16;
      if (c_off >= BS) {
        c_off -= BS;
        ++c_bi;
      }
    }
    int blk = __builtin_amdgcn_readlane(my_blk, bi);
    const bool live = i < n_tiles && blk >= 0;
    t.valid = live ? ((t_end - ts) < 16 ? (t_end - ts) : 16) : 0;
    t.ts = ts;
    if constexpr (FP8) {
      t.ksc = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(my_ks), bi));
      t.vsc = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(my_vs), bi));
    } else {
      t.ksc = 1.f;
      t.vsc = 1.f;
    }
    if (blk < 0) blk = 0;
    load_tile<D, FP8>(t, kc, vc, blk, kvh, Hkv, BS, o0, koff, voff, stream, live);
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
                                                 float scale_log2, int lane, int col, int grp, bool stream) {
  attend_range<D, FP8>([&](Tile<D, FP8> &t) { attend_tile<D, FP8>(st, t, qop, scale_log2, grp); }, kc, vc, ks, vs,
                       my_blk, t_begin, t_end, kvh, Hkv, BS, NB, lane, col, grp, stream);
}

}  // namespace wkv
