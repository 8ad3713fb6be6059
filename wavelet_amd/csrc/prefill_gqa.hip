// GQA prefill / chunked-prefill attention over the paged cache (gfx950).
//
// Sequence b brings qlen_b = cu_seqlens_q[b+1] - cu_seqlens_q[b] new tokens
// at positions [L_b - qlen_b, L_b) (L_b = seq_lens[b]: cached context plus the
// new tokens, which the entry point appends to the cache first). New token j
// attends causally to positions [0, L_b - qlen_b + j] -- the bottom-right
// aligned mask of a varlen prefill over a paged context (a prefix-cache hit or
// an earlier chunk).
//
// Work decomposition: workgroup (query tile, KV head x head group, sequence)
// of four waves; wave w takes query head kvh*G + 4*hg + w, so the MFMA
// columns are consecutive query tokens of one head and the four waves of a
// workgroup stream the same key tiles. Every query tile of a (sequence, KV
// head) re-reads that head's keys, so the 1-D grid sends all of them to one
// XCD (the dispatcher deals workgroup i to XCD i mod 8): the keys are served
// from that XCD's L2 instead of being fetched by all eight. The latest (most
// expensive, causally) query tiles are dispatched first. Keys are copied once
// per workgroup into LDS by LDS-DMA, in 16-token tiles, four per step of 64
// keys; each wave holds 32 queries and runs 32x32x16 bf16 MFMAs. fp8 tiles
// are dequantized in LDS (exactly: power-of-two scales) by the wave that
// copied them, so both dtypes share the attention arithmetic. Tiles on the
// causal diagonal mask per lane (column). Every wave finishes its rows: no
// split-K, no workspace.
#include "gqa_tiles.h"
#include "lds_dma.h"

#include <cmath>

namespace wkv {

constexpr int kPrefillWaves = 4;

// Eight e4m3fn codes (bytes of lo, then hi) times a power-of-two scale as
// eight bf16 values, by the hardware pair conversion (exact: every such
// product is a bf16 value).
__device__ __forceinline__ u32x4 fp8x8_to_bf16_words(uint32_t lo, uint32_t hi, float sc) {
  return u32x4{__builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(lo, sc, false)),
               __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(lo, sc, true)),
               __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(hi, sc, false)),
               __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(hi, sc, true))};
}

// One 16-token key tile of one (block, KV head) in LDS, as the MFMAs read it
// (bf16; fp8 tiles are dequantized into the same layout): K as a bf16 cache
// holds it, [D/8 chunks][16 tokens][16 bytes]; V as [2 token octets][D rows]
// [8 tokens] (16-byte pieces, so a copy still moves whole pieces). A lane's
// MFMA operand is one 16-byte LDS read: 16 bytes of one token's K chunk, or
// the 8 tokens of one octet of one V row.
template <int D>
struct LdsTile {
  static constexpr int KB = D * 16 * 2;  // K bytes
  static constexpr int VB = D * 16 * 2;  // V bytes
};

// ---------------------------------------------------------------------------
// 32 queries per wave on 32x32x16 MFMAs, 64 keys per step (four 16-token
// tiles, one copied by each wave). Lane l holds query l % 32 in both
// accumulators. Per step and wave:
//   S^T for keys 0..31 and 32..63 of the step    two chains of D/16 MFMAs
//                                                 32x32x16 (one per half,
//                                                 interleaved: a chain never
//                                                 waits on itself)
//   one row maximum, one rescale test            over the 64 keys
//   P V^T                                        4 x D/32 MFMAs 32x32x16
//   copies of the wave's tile: V of the next     one buffer resource each,
//   step, K of the step after                    16-byte copies (the K copies
//                                                 under one M0)
// so the per-step costs (barriers, waits, loop and mask tests, the maximum's
// cross-lane swap) and the per-tile block lookup fall on 32 MFMAs. Row i of
// each half's S^T carries key kperm(i) of the half (rows 4..7 and 8..11 of
// each 16 swapped), so score r of lane l is key 16 (r/8) + 8 (l/32) + r % 8
// of the half -- the PV B operand as it stands -- and the row sum is taken
// on the packed bf16 probabilities the PV products consume (v_dot2c_f32_bf16
// against 1.0, two per instruction). A block id outside [0, num_blocks) reads block 0: no
// access leaves the cache, and that sequence's output is unspecified.
//
// Software pipeline, one workgroup barrier per step: while a wave finishes
// step s (its probabilities, then its PV products) it scores step s + 1, so
// its MFMAs and its softmax VALU work overlap inside the wave --
//   phase A: the QK products of step s + 1  ||  exponentials, packing and row
//            sum of step s
//   phase B: the PV products of step s      ||  mask, exponents against the
//            reference and their maximum of step s + 1 (the rare move of the
//            reference maximum rescales after the PV products)
// (interleaved by sched_group_barrier: an MFMA, then a few VALU, with the LDS
// operand reads four MFMAs ahead). The copies of a step are one step ahead:
// at the barrier of step s every wave's V of step s and K of step s + 1 have
// landed and every wave is done with step s - 1, whose slots take V of step
// s + 1 and K of step s + 2. LDS (bf16 tiles): K and V in two step slots
// each, 64 KB at d=128, two workgroups per CU at up to 256 VGPRs per wave.
// fp8 caches: the copies land in a staging area of the copying wave's own,
// and that wave dequantizes its tiles into the bf16 layout above with the
// hardware conversion at the (block, head) scale (a power of two: exact in
// bf16) after the wait and before the barrier of the step: its V tile of
// step s and its K tile of step s + 1. The attention arithmetic is the bf16
// one. LDS: 64 KB bf16 plus 8 + 8 KB staging at d=128.
template <int D, bool FP8>
__global__ __launch_bounds__(64 * kPrefillWaves, 2) void prefill_gqa_kernel(
    const uint8_t *__restrict__ kc, const uint8_t *__restrict__ vc, const float *__restrict__ ksc,
    const float *__restrict__ vsc, const uint16_t *__restrict__ q, int64_t q_st,
    int64_t q_sh, uint16_t *__restrict__ out, int64_t o_st, int64_t o_sh, const int32_t *__restrict__ cu_q,
    const int32_t *__restrict__ seq_lens, const int32_t *__restrict__ bt, int64_t bt_stride, int Mb, int max_seq,
    int Hkv, int G, int n_hg, int BS, int nb, float scale_log2, int n_qt, int n_items,
    const float *__restrict__ sinks) {
  using LT = LdsTile<D>;
  static_assert(kPrefillWaves == 4, "one tile per wave per 64-key step");
  static_assert(D % 64 == 0, "whole copies per lane");
  constexpr int KB = LT::KB, VB = LT::VB;   // bytes of one bf16 tile's K, V
  constexpr int ESZ = FP8 ? 1 : 2;          // cache bytes per element
  constexpr int NC = D * 16 * ESZ / 1024;   // 16-byte copies per lane of a tile's K (and of its V)
  constexpr int DV = D / 64;                // bf16 V copies per token octet
  constexpr int SB = FP8 ? D * 16 : 16;     // fp8 staging bytes per tile, K or V
  __shared__ __attribute__((aligned(16))) uint8_t ldsk[2 * 4 * KB];  // bf16 K: two step slots of four tiles
  __shared__ __attribute__((aligned(16))) uint8_t ldsv[2 * 4 * VB];  // bf16 V: two step slots
  __shared__ __attribute__((aligned(16))) uint8_t stgk[4 * SB];      // fp8 K as copied, a tile per wave
  __shared__ __attribute__((aligned(16))) uint8_t stgv[4 * SB];      // fp8 V as copied
  const int id = blockIdx.x;
  const int item = (id / (8 * n_qt)) * 8 + (id & 7);
  const int qt = __builtin_amdgcn_readfirstlane(n_qt - 1 - (id / 8) % n_qt);
  if (item >= n_items) return;
  const int b = __builtin_amdgcn_readfirstlane(item / (Hkv * n_hg));
  const int kvh = __builtin_amdgcn_readfirstlane((item / n_hg) % Hkv);
  const int hg = item % n_hg;
  const int wave = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x >> 6));
  const int lane = threadIdx.x & 63, n = lane & 31, hh = lane >> 5;
  const int q0 = cu_q[b];
  const int qlen = cu_q[b + 1] - q0;
  int L = seq_lens[b];
  L = L < max_seq ? L : max_seq;
  const int t0 = qt * 32;
  if (t0 >= qlen) return;  // the whole workgroup leaves together
  const int h_local = hg * kPrefillWaves + wave;
  const bool active = h_local < G;  // an idle wave still copies its tile of every step
  const int h = kvh * G + (active ? h_local : 0);
  const int ctx = L - qlen;
  // this lane's output row (query t0 + l % 32), formed before the key loop
  uint16_t *const op = out + static_cast<int64_t>(q0 + t0 + n) * o_st + static_cast<int64_t>(h) * o_sh;

  // Q^T operand j: lane l holds d = 16 j + 8 (l/32) .. + 7 of query t0 + l % 32.
  bf16x8 qb[D / 16];
  {
    const int tok = t0 + n;
    const bool valid = active && tok < qlen;
    const uint16_t *qp = q + static_cast<int64_t>(q0 + (tok < qlen ? tok : t0)) * q_st + static_cast<int64_t>(h) * q_sh;
#pragma unroll
    for (int j = 0; j < D / 16; ++j) {
      u32x4 w = *reinterpret_cast<const u32x4 *>(qp + 16 * j + 8 * hh);
      if (!valid) w = u32x4{0u, 0u, 0u, 0u};
      qb[j] = __builtin_bit_cast(bf16x8, w);
    }
  }
  floatx16 o[D / 32];
#pragma unroll
  for (int c = 0; c < D / 32; ++c)
#pragma unroll
    for (int r = 0; r < 16; ++r) o[c][r] = 0.f;
  float m_ref = -INFINITY, l_part = 0.f;

  const int last = (t0 + 32 < qlen ? t0 + 32 : qlen) - 1;
  const int kend = ctx + last + 1;  // keys [0, kend)
  const int n_tiles = kend > 0 ? (kend + 15) / 16 : 0;
  const int n_steps = (n_tiles + 3) / 4;
  const int region = D * BS * ESZ;
  const int min_pos = ctx + t0;  // the smallest query position of the workgroup

  // Copy k of lane l moves piece p = 64 k + l of the wave's tile's K or V
  // (LDS offset 16 p). K piece p (both dtypes: 16-byte chunks): chunk p >> 4,
  // token p & 15, at ((p >> 4) BS + (p & 15)) 16 of the (block, head) K region
  // = lane part ((l >> 4) BS + (l & 15)) 16 + copy part 64 BS k. bf16 V piece
  // p: row p % D, octet p / D, at (p % D) BS 2 + 16 (p / D) = lane part 2 BS l
  // + copy part 128 BS (k % DV) + 16 (k / DV). fp8 V piece p: row p, at p BS =
  // lane part BS l + copy part 64 BS k. The tile's first token o0 goes into
  // the base.
  const uint32_t lane_k = static_cast<uint32_t>(((lane >> 4) * BS + (lane & 15)) * 16);
  const uint32_t lane_v = static_cast<uint32_t>(lane * BS * ESZ);
  const uint32_t ldsk0 = lds_addr(ldsk), ldsv0 = lds_addr(ldsv);
  const uint32_t stgk0 = lds_addr(stgk), stgv0 = lds_addr(stgv);
  float ks_next = 1.f, vs_next = 1.f, vs_stage = 1.f;  // fp8 scales: last K issued, its V, the staged V
  const int32_t *btrow = bt + b * bt_stride;
  int bix = (16 * wave) / BS;
  int o0 = 16 * wave - bix * BS;
  const int dbix = 64 / BS, do0 = 64 - dbix * BS;
  int wbase = 0;  // the window: lane i holds the id of block wbase + i
  int win = load_i32_drained(btrow, lane, Mb);
  int64_t vbase = 0;  // V of the wave's tile of the step whose K went out last: cache offset
  auto has_tile = [&](int s) { return s < n_steps && 4 * s + wave < n_tiles; };  // uniform
  // K of the wave's tile of step s into K slot `slot` (fp8: into the staging area)
  auto issue_k = [&](int s, int slot) {
    if (has_tile(s)) {
      if (bix - wbase >= 64) {  // at most once per 64 blocks (its wait drains the copies in flight)
        wbase += 64;
        win = load_i32_drained(btrow, wbase + lane, Mb);
      }
      int blk = __builtin_amdgcn_readlane(win, bix - wbase);
      if (!(blk >= 0 && blk < nb)) blk = 0;
      const int64_t rb = static_cast<int64_t>(static_cast<uint64_t>(static_cast<uint32_t>(blk * Hkv + kvh)) *
                                              static_cast<uint32_t>(region));
      vbase = rb + o0 * ESZ;
      if constexpr (FP8) {
        ks_next = ksc[blk * Hkv + kvh];
        vs_next = vsc[blk * Hkv + kvh];
      }
      // copy part of K copy k: 64 BS k = 1024 k (its LDS offset, the instruction
      // offset) + k (64 BS - 1024)
      uint32_t kst = static_cast<uint32_t>(64 * BS);
      asm volatile("" : "+s"(kst));
      const __amdgpu_buffer_rsrc_t kr =
          __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t *>(kc + rb + o0 * 16), 0, region, kRawBufferWord3);
      const uint32_t dst = FP8 ? stgk0 + static_cast<uint32_t>(wave * SB)
                               : ldsk0 + static_cast<uint32_t>((4 * slot + wave) * KB);
      buffer_copy16_run_to_lds<NC>(kr, lane_k, kst - 1024u, dst);
    }
    o0 += do0;
    bix += dbix;
    if (o0 >= BS) {
      o0 -= BS;
      ++bix;
    }
  };
  // V of the wave's tile of step s (whose K went out last) into V slot `slot`
  auto issue_v = [&](int s, int slot) {
    if (has_tile(s)) {
      const __amdgpu_buffer_rsrc_t vr =
          __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t *>(vc + vbase), 0, region, kRawBufferWord3);
      if constexpr (FP8) {
        vs_stage = vs_next;
        const uint32_t dst = stgv0 + static_cast<uint32_t>(wave * SB);
        uint32_t vst = static_cast<uint32_t>(64 * BS);
        asm volatile("" : "+s"(vst));
#pragma unroll
        for (int k = 0; k < NC; ++k) buffer_copy16_to_lds(vr, lane_v, vst * k, dst + 1024 * k);
      } else {
        const uint32_t dst = ldsv0 + static_cast<uint32_t>((4 * slot + wave) * VB);
        uint32_t vst = static_cast<uint32_t>(128 * BS);
        asm volatile("" : "+s"(vst));
#pragma unroll
        for (int k = 0; k < NC; ++k)
          buffer_copy16_to_lds(vr, lane_v, vst * (k % DV) + 16 * (k / DV), dst + 1024 * k);
      }
    }
  };
  // fp8: the wave's K tile, staged, into bf16 K slot `slot` at scale sc.
  // Piece p = 64 i + l: chunk c = p >> 4 (16 d), token m = p & 15 -> bf16
  // chunks 2c, 2c + 1 of token m.
  auto convert_k = [&](float sc, int slot) {
#pragma unroll
    for (int i = 0; i < D / 64; ++i) {
      const int pc = 64 * i + lane;
      const u32x4 w = *reinterpret_cast<const u32x4 *>(stgk + wave * SB + pc * 16);
      uint8_t *dk = ldsk + (4 * slot + wave) * KB + ((2 * (pc >> 4)) * 16 + (pc & 15)) * 16;
      *reinterpret_cast<u32x4 *>(dk) = fp8x8_to_bf16_words(w[0], w[1], sc);
      *reinterpret_cast<u32x4 *>(dk + 256) = fp8x8_to_bf16_words(w[2], w[3], sc);
    }
  };
  // fp8: the wave's V tile, staged, into bf16 V slot `slot` at scale sc,
  // tokens at or past vt zeroed (the slots past the keys may hold NaN). Piece
  // p = 64 i + l: row p, 16 tokens -> octets 0, 1 of row p.
  auto convert_v = [&](float sc, int vt, int slot) {
#pragma unroll
    for (int i = 0; i < D / 64; ++i) {
      const int pc = 64 * i + lane;
      const u32x4 w = *reinterpret_cast<const u32x4 *>(stgv + wave * SB + pc * 16);
      u32x4 lo = fp8x8_to_bf16_words(w[0], w[1], sc), hi = fp8x8_to_bf16_words(w[2], w[3], sc);
      if (vt < 16) {
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          if (e >= vt) lo[e >> 1] &= (e & 1) ? 0x0000FFFFu : 0xFFFF0000u;
          if (8 + e >= vt) hi[e >> 1] &= (e & 1) ? 0x0000FFFFu : 0xFFFF0000u;
        }
      }
      uint8_t *dv = ldsv + (4 * slot + wave) * VB;
      *reinterpret_cast<u32x4 *>(dv + pc * 16) = lo;
      *reinterpret_cast<u32x4 *>(dv + (D + pc) * 16) = hi;
    }
  };
  // Step s's copies have landed (this wave's): make its V tile (and fp8: the
  // next step's K tile) ready in the bf16 slots -- fp8 conversion, slots of a
  // partial tile past the keys zeroed.
  // Before the last step every wave's tile of step s is whole and its K tile
  // of step s + 1 is converted whether or not it exists (a tile past the keys
  // is masked): the fp8 conversion then runs without branches, its four LDS
  // reads ahead of the conversions.
  auto land_body = [&](int s) {
    if constexpr (FP8) {
      u32x4 wv[D / 64], wk[D / 64];
#pragma unroll
      for (int i = 0; i < D / 64; ++i) {
        wv[i] = *reinterpret_cast<const u32x4 *>(stgv + wave * SB + (64 * i + lane) * 16);
        wk[i] = *reinterpret_cast<const u32x4 *>(stgk + wave * SB + (64 * i + lane) * 16);
      }
      uint8_t *dv = ldsv + (4 * (s & 1) + wave) * VB;
      uint8_t *dk = ldsk + (4 * ((s + 1) & 1) + wave) * KB;
#pragma unroll
      for (int i = 0; i < D / 64; ++i) {
        const int pc = 64 * i + lane;
        *reinterpret_cast<u32x4 *>(dv + pc * 16) = fp8x8_to_bf16_words(wv[i][0], wv[i][1], vs_stage);
        *reinterpret_cast<u32x4 *>(dv + (D + pc) * 16) = fp8x8_to_bf16_words(wv[i][2], wv[i][3], vs_stage);
        uint8_t *k = dk + ((2 * (pc >> 4)) * 16 + (pc & 15)) * 16;
        *reinterpret_cast<u32x4 *>(k) = fp8x8_to_bf16_words(wk[i][0], wk[i][1], ks_next);
        *reinterpret_cast<u32x4 *>(k + 256) = fp8x8_to_bf16_words(wk[i][2], wk[i][3], ks_next);
      }
    }
  };
  auto land = [&](int s) {
    int vt = kend - 64 * s - 16 * wave;  // keys of this wave's tile of step s
    vt = vt < 0 ? 0 : (vt > 16 ? 16 : vt);
    if constexpr (FP8) {
      if (vt > 0) convert_v(vs_stage, vt, s & 1);  // uniform
      if (has_tile(s + 1)) convert_k(ks_next, (s + 1) & 1);
    } else if (vt > 0 && vt < 16) {  // uniform; at most once per workgroup
#pragma unroll
      for (int i = 0; i < D / 32; ++i) {
        const int pc = 64 * i + lane;
        const int cnt = vt - 8 * (pc / D);
        u32x4 *ptr = reinterpret_cast<u32x4 *>(ldsv + (4 * (s & 1) + wave) * VB + pc * 16);
        u32x4 w = *ptr;
#pragma unroll
        for (int e = 0; e < 8; ++e)
          if (e >= cnt) w[e >> 1] &= (e & 1) ? 0x0000FFFFu : 0xFFFF0000u;
        *ptr = w;
      }
    }
  };
  const int kn = (n & 16) | (((n >> 2) & 3) == 1 ? (n & 3) + 8 : ((n >> 2) & 3) == 2 ? (n & 3) + 4 : (n & 15));
  const bf16x2 ones = __builtin_bit_cast(bf16x2, 0x3F803F80u);
  uint32_t pw[4][4];  // PV B operands of the step being finished: packed bf16 probabilities

  // S^T of step s (K slot s & 1) into (x0, x1)
  auto qk = [&](int s, floatx16 &x0, floatx16 &x1) {
#pragma unroll
    for (int r = 0; r < 16; ++r) x0[r] = x1[r] = 0.f;
    const uint8_t *lk = ldsk + ((s & 1) * 4 + (kn >> 4)) * KB + (kn & 15) * 16;
#pragma unroll
    for (int jj = 0; jj < D / 16; ++jj) {
      const bf16x8 a0 = __builtin_bit_cast(bf16x8, *reinterpret_cast<const u32x4 *>(lk + (2 * jj + hh) * 256));
      const bf16x8 a1 = __builtin_bit_cast(bf16x8, *reinterpret_cast<const u32x4 *>(lk + 2 * KB + (2 * jj + hh) * 256));
      x0 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a0, qb[jj], x0, 0, 0, 0);
      x1 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a1, qb[jj], x1, 0, 0, 0);
    }
  };
  // causal / end mask of step s's scores
  auto mask = [&](int s, floatx16 &x0, floatx16 &x1) {
    const int kb = 64 * s;
    if (!(kend >= kb + 64 && kb + 63 <= min_pos)) {  // uniform: masks in this step
      const int pos = min_pos + n;
      const int lim = (pos < kend - 1 ? pos : kend - 1) - kb - 8 * hh;
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        if (16 * (r / 8) + (r % 8) > lim) x0[r] = -INFINITY;
        if (32 + 16 * (r / 8) + (r % 8) > lim) x1[r] = -INFINITY;
      }
    }
  };
  // exponents against the reference maximum and their maximum
  auto expo = [&](floatx16 &x0, floatx16 &x1) {
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      x0[r] = __builtin_fmaf(x0[r], scale_log2, -m_ref);
      x1[r] = __builtin_fmaf(x1[r], scale_log2, -m_ref);
    }
    float mt0 = fmaxf(x0[0], x0[1]), mt1 = fmaxf(x1[0], x1[1]);
#pragma unroll
    for (int r = 2; r < 16; r += 2) {
      mt0 = fmaxf(fmaxf(mt0, x0[r]), x0[r + 1]);
      mt1 = fmaxf(fmaxf(mt1, x1[r]), x1[r + 1]);
    }
    float mt = fmaxf(mt0, mt1);
    const auto x = __builtin_amdgcn_permlane32_swap(__float_as_uint(mt), __float_as_uint(mt), false, false);
    return fmaxf(__uint_as_float(x[0]), __uint_as_float(x[1]));
  };
  // the rare move of the reference maximum (after the PV products of the steps before)
  auto rescale = [&](float mt, floatx16 &x0, floatx16 &x1) {
    const bool move = mt > SOFTMAX_TAU;
    if (__any(move)) {
      const float sh = move ? mt : 0.f;
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        x0[r] -= sh;
        x1[r] -= sh;
      }
      const float corr = fast_exp2(-sh);
      l_part *= corr;
      m_ref += sh;
#pragma unroll
      for (int c = 0; c < D / 32; ++c)
#pragma unroll
        for (int r = 0; r < 16; ++r) o[c][r] *= corr;
    }
  };
  // probabilities, packed as the PV operands, and their row sum
  auto probs = [&](floatx16 &x0, floatx16 &x1) {
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      x0[r] = fast_exp2(x0[r]);
      x1[r] = fast_exp2(x1[r]);
    }
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      const floatx16 &sv = t < 2 ? x0 : x1;
      const int e0 = 8 * (t & 1);
#pragma unroll
      for (int i = 0; i < 4; ++i) pw[t][i] = pack_bf16x2(sv[e0 + 2 * i], sv[e0 + 2 * i + 1]);
    }
    float ps = 0.f;
#pragma unroll
    for (int t = 0; t < 4; ++t)
#pragma unroll
      for (int i = 0; i < 4; ++i)
        ps = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, pw[t][i]), ones, ps, false);
    l_part += ps;
  };
  // P V^T of step s (V slot s & 1); tiles past the keys skipped when `partial`
  auto pv = [&](int s, bool partial) {
    const uint8_t *lv = ldsv + (s & 1) * 4 * VB + hh * D * 16 + n * 16;
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      if (partial && kend - 64 * s - 16 * t <= 0) continue;  // uniform
      const bf16x8 pb = __builtin_bit_cast(bf16x8, (u32x4{pw[t][0], pw[t][1], pw[t][2], pw[t][3]}));
#pragma unroll
      for (int c = 0; c < D / 32; ++c) {
        const u32x4 w = *reinterpret_cast<const u32x4 *>(lv + t * VB + 32 * c * 16);
        o[c] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, w), pb, o[c], 0, 0, 0);
      }
    }
  };
  // One step of the pipeline: finish step s (its scores in c0, c1 are
  // exponents against the reference) while scoring step s + 1 into n0, n1.
  auto body = [&](int s, floatx16 &c0, floatx16 &c1, floatx16 &n0, floatx16 &n1) {
    wait_vmcnt<0>();  // this wave's copies of step s's V and step s + 1's K
    land_body(s);
    barrier_lds();    // ... every wave's; every wave is done with step s - 1
    issue_v(s + 1, (s + 1) & 1);
    issue_k(s + 2, s & 1);
    {  // an idle wave computes on zero queries and stores nothing
      qk(s + 1, n0, n1);
      probs(c0, c1);
      // keeps the probabilities in this block (ahead of the mask's branch)
      asm volatile("" ::"v"(l_part), "v"(pw[0][0]), "v"(pw[0][1]), "v"(pw[0][2]), "v"(pw[0][3]), "v"(pw[1][0]),
                   "v"(pw[1][1]), "v"(pw[1][2]), "v"(pw[1][3]), "v"(pw[2][0]), "v"(pw[2][1]), "v"(pw[2][2]),
                   "v"(pw[2][3]), "v"(pw[3][0]), "v"(pw[3][1]), "v"(pw[3][2]), "v"(pw[3][3]));
      // the score products of step s + 1 interleaved with step s's probabilities
      __builtin_amdgcn_sched_group_barrier(0x100, 4, 0);  // LDS reads, four ahead
#pragma unroll
      for (int i = 0; i < 2 * D / 16; ++i) {
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // MFMA
        if (i + 4 < 2 * D / 16) __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);  // LDS read
        __builtin_amdgcn_sched_group_barrier(0x002, 4, 0);  // VALU
      }
      mask(s + 1, n0, n1);
      const float mt = expo(n0, n1);
      pv(s, false);
      // step s's PV products interleaved with step s + 1's exponents
      __builtin_amdgcn_sched_group_barrier(0x100, 4, 0);  // LDS reads, four ahead
#pragma unroll
      for (int i = 0; i < 4 * D / 32; ++i) {
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // MFMA
        if (i + 4 < 4 * D / 32) __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);  // LDS read
        __builtin_amdgcn_sched_group_barrier(0x002, 3, 0);  // VALU
      }
      rescale(mt, n0, n1);
    }
  };

  if (n_steps > 0) {
    issue_k(0, 0);
    if constexpr (FP8) {
      wait_vmcnt<0>();
      if (has_tile(0)) convert_k(ks_next, 0);
    }
    issue_v(0, 0);
    issue_k(1, 1);
    if constexpr (!FP8) {
      if (has_tile(1)) wait_vmcnt<2 * NC>(); else wait_vmcnt<NC>();  // K of step 0 landed
    }
    barrier_lds();
    floatx16 a0, a1, b0, b1;
    {
      qk(0, a0, a1);
      mask(0, a0, a1);
      // the reference maximum starts at the first step's row maximum (every
      // query sees key 0, so it is finite)
      float mt = fmaxf(a0[0], a1[0]);
#pragma unroll
      for (int r = 1; r < 16; ++r) mt = fmaxf(mt, fmaxf(a0[r], a1[r]));
      const auto x = __builtin_amdgcn_permlane32_swap(__float_as_uint(mt), __float_as_uint(mt), false, false);
      mt = fmaxf(__uint_as_float(x[0]), __uint_as_float(x[1])) * scale_log2;
      m_ref = mt == -INFINITY ? 0.f : mt;
      rescale(expo(a0, a1), a0, a1);
    }
    // the last step: its V, its probabilities, its PV products (tiles past the keys skipped)
    auto tail = [&](int s, floatx16 &c0, floatx16 &c1) {
      wait_vmcnt<0>();
      land(s);
      barrier_lds();
      probs(c0, c1);
      pv(s, true);
    };
    const int n_body = n_steps - 1;
    int s = 0;
    for (; s + 2 <= n_body; s += 2) {
      body(s, a0, a1, b0, b1);
      body(s + 1, b0, b1, a0, a1);
    }
    if (s < n_body) {
      body(s, a0, a1, b0, b1);
      tail(s + 1, b0, b1);
    } else {
      tail(s, a0, a1);
    }
  }
  const int tok = t0 + n;
  if (!active || tok >= qlen) return;
  float l = l_part;
  {
    const auto x = __builtin_amdgcn_permlane32_swap(__float_as_uint(l), __float_as_uint(l), false, false);
    l = __uint_as_float(x[0]) + __uint_as_float(x[1]);
  }
  // An attention sink (a zero-value logit of head h, natural-log units) adds
  // its weight against the row's reference maximum to the denominator.
  if (sinks != nullptr) l += exp2f(sinks[h] * 1.4426950408889634f - m_ref);
  const float inv = l > 0.f ? 1.f / l : 0.f;
#pragma unroll
  for (int c = 0; c < D / 32; ++c) {
#pragma unroll
    for (int g = 0; g < 4; ++g) {  // d = 32 c + 8 g + 4 hh + 0..3
      const u32x2 w = {pack_bf16x2(o[c][4 * g] * inv, o[c][4 * g + 1] * inv),
                       pack_bf16x2(o[c][4 * g + 2] * inv, o[c][4 * g + 3] * inv)};
      *reinterpret_cast<u32x2 *>(op + 32 * c + 8 * g + 4 * hh) = w;
    }
  }
}

}  // namespace wkv

using namespace wkv;

static int launch_prefill(const wkv_cache_t *cache, const void *key, int64_t key_stride_t, int64_t key_stride_h,
                          const void *value, int64_t value_stride_t, int64_t value_stride_h,
                          const int64_t *slot_mapping, int64_t num_tokens, const void *q, int64_t q_stride_t,
                          int64_t q_stride_h, void *out, int64_t out_stride_t, int64_t out_stride_h,
                          int32_t num_q_heads, const int32_t *cu_seqlens_q, const int32_t *seq_lens,
                          const int32_t *block_table, int64_t bt_stride, int32_t max_blocks_per_seq, int32_t batch,
                          int32_t max_query_len, int32_t max_seq_len, float scale, const float *sinks,
                          void *stream) {
  int rc = check_cache(cache, -1);
  if (rc) return rc;
  WKV_CHECK_ARG(batch >= 0 && batch <= 65535, "batch must be in [0, 65535] (got %d)", batch);
  WKV_CHECK_ARG(num_tokens >= 0, "num_tokens must be >= 0");
  if (key != nullptr || value != nullptr || slot_mapping != nullptr) {
    // The step's new tokens go into the cache first (same stream: the
    // attention launch below reads them back).
    rc = cache->kv_dtype == WKV_KV_FP8_E4M3
             ? wkv_append_fp8(cache, key, key_stride_t, key_stride_h, value, value_stride_t, value_stride_h,
                              slot_mapping, num_tokens, stream)
             : wkv_append(cache, key, key_stride_t, key_stride_h, value, value_stride_t, value_stride_h,
                          slot_mapping, num_tokens, stream);
    if (rc) return rc;
  }
  if (batch == 0 || max_query_len == 0) return WKV_OK;
  const int Hkv = cache->num_kv_heads, D = cache->head_dim, BS = cache->block_size;
  WKV_CHECK_ARG(num_q_heads > 0 && num_q_heads % Hkv == 0, "num_q_heads %d must be a multiple of num_kv_heads %d",
                num_q_heads, Hkv);
  const int G = num_q_heads / Hkv;
  WKV_CHECK_ARG(cache->num_blocks * Hkv <= INT32_MAX, "num_blocks * num_kv_heads must be below 2^31");
  WKV_CHECK_ARG(q != nullptr && aligned16(q), "q must be non-NULL and 16-byte aligned");
  WKV_CHECK_ARG(q_stride_t >= 0 && q_stride_h >= 0 && q_stride_t % 8 == 0 && q_stride_h % 8 == 0,
                "q strides must be non-negative multiples of 8");
  WKV_CHECK_ARG(out != nullptr && aligned16(out), "out must be non-NULL and 16-byte aligned");
  WKV_CHECK_ARG(out_stride_t >= 0 && out_stride_h >= 0 && out_stride_t % 4 == 0 && out_stride_h % 4 == 0,
                "out strides must be non-negative multiples of 4");
  WKV_CHECK_ARG(cu_seqlens_q != nullptr && seq_lens != nullptr && block_table != nullptr,
                "cu_seqlens_q / seq_lens / block_table is NULL");
  WKV_CHECK_ARG(max_blocks_per_seq > 0 && bt_stride >= max_blocks_per_seq, "bad block table geometry");
  WKV_CHECK_ARG(max_query_len > 0 && max_seq_len >= 0, "max_query_len must be > 0 and max_seq_len >= 0");
  WKV_CHECK_ARG(std::isfinite(scale), "scale must be finite");
  const int max_seq = max_seq_len < max_blocks_per_seq * BS ? max_seq_len : max_blocks_per_seq * BS;
  const bool fp8 = cache->kv_dtype == WKV_KV_FP8_E4M3;
  const int n_hg = (G + kPrefillWaves - 1) / kPrefillWaves;
  const int q_tile = 32;
  const int n_qt = (max_query_len + q_tile - 1) / q_tile;
  const int64_t n_items = static_cast<int64_t>(batch) * Hkv * n_hg;
  const int64_t n_wg = (n_items + 7) / 8 * 8 * n_qt;
  WKV_CHECK_ARG(n_wg <= INT32_MAX, "prefill grid too large");
  const dim3 grid(static_cast<unsigned>(n_wg));
  auto s = static_cast<hipStream_t>(stream);
  auto kc = static_cast<const uint8_t *>(cache->k);
  auto vc = static_cast<const uint8_t *>(cache->v);
  auto qq = static_cast<const uint16_t *>(q);
  auto oo = static_cast<uint16_t *>(out);
  const float scale_log2 = scale * 1.4426950408889634f;
#define WKV_PREFILL(Dv, F8)                                                                                       \
  prefill_gqa_kernel<Dv, F8><<<grid, 64 * kPrefillWaves, 0, s>>>(                                                \
      kc, vc, cache->k_scale, cache->v_scale, qq, q_stride_t, q_stride_h, oo, out_stride_t, out_stride_h,       \
      cu_seqlens_q, seq_lens, block_table, bt_stride, max_blocks_per_seq, max_seq, Hkv, G, n_hg, BS,           \
      static_cast<int>(cache->num_blocks), scale_log2, n_qt, static_cast<int>(n_items), sinks)
  if (D == 128) {
    if (fp8) WKV_PREFILL(128, true); else WKV_PREFILL(128, false);
  } else {
    if (fp8) WKV_PREFILL(64, true); else WKV_PREFILL(64, false);
  }
#undef WKV_PREFILL
  WKV_CHECK_LAUNCH("paged prefill");
  return WKV_OK;
}

extern "C" int wkv_prefill_gqa(const wkv_cache_t *cache, const void *key, int64_t key_stride_t, int64_t key_stride_h,
                               const void *value, int64_t value_stride_t, int64_t value_stride_h,
                               const int64_t *slot_mapping, int64_t num_tokens, const void *q, int64_t q_stride_t,
                               int64_t q_stride_h, void *out, int64_t out_stride_t, int64_t out_stride_h,
                               int32_t num_q_heads, const int32_t *cu_seqlens_q, const int32_t *seq_lens,
                               const int32_t *block_table, int64_t bt_stride, int32_t max_blocks_per_seq,
                               int32_t batch, int32_t max_query_len, int32_t max_seq_len, float scale, void *stream) {
  return launch_prefill(cache, key, key_stride_t, key_stride_h, value, value_stride_t, value_stride_h, slot_mapping,
                        num_tokens, q, q_stride_t, q_stride_h, out, out_stride_t, out_stride_h, num_q_heads,
                        cu_seqlens_q, seq_lens, block_table, bt_stride, max_blocks_per_seq, batch, max_query_len,
                        max_seq_len, scale, nullptr, stream);
}

extern "C" int wkv_prefill_gqa_sinks(const wkv_cache_t *cache, const void *key, int64_t key_stride_t,
                                     int64_t key_stride_h, const void *value, int64_t value_stride_t,
                                     int64_t value_stride_h, const int64_t *slot_mapping, int64_t num_tokens,
                                     const void *q, int64_t q_stride_t, int64_t q_stride_h, void *out,
                                     int64_t out_stride_t, int64_t out_stride_h, int32_t num_q_heads,
                                     const int32_t *cu_seqlens_q, const int32_t *seq_lens,
                                     const int32_t *block_table, int64_t bt_stride, int32_t max_blocks_per_seq,
                                     int32_t batch, int32_t max_query_len, int32_t max_seq_len, float scale,
                                     const float *sinks, void *stream) {
  WKV_CHECK_ARG(sinks != nullptr && reinterpret_cast<uintptr_t>(sinks) % 4 == 0, "sinks must be non-NULL fp32");
  return launch_prefill(cache, key, key_stride_t, key_stride_h, value, value_stride_t, value_stride_h, slot_mapping,
                        num_tokens, q, q_stride_t, q_stride_h, out, out_stride_t, out_stride_h, num_q_heads,
                        cu_seqlens_q, seq_lens, block_table, bt_stride, max_blocks_per_seq, batch, max_query_len,
                        max_seq_len, scale, sinks, stream);
}
