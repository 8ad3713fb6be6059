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
// Long contexts are split into partitions (one wave each); the last wave of a
// (sequence, KV head) to finish merges the partials by log-sum-exp, so one
// launch does the whole step.
#include <cmath>

#include "wkv_common.h"

namespace wkv {

typedef __attribute__((__vector_size__(4 * sizeof(short)))) short shortx4;

template <int D, bool FP8>
struct Tile {
  static constexpr int NQK = D / 32;  // QK MFMAs per tile
  static constexpr int NPV = D / 16;  // PV MFMAs per tile
  bf16x8 k[NQK];
  shortx4 v[NPV];
};

__device__ __forceinline__ bf16x8 fp8x8_to_bf16x8(uint32_t lo, uint32_t hi) {
  // Each e4m3 value is exactly representable in bf16: widen through fp32 and
  // keep the top half (truncation is exact here).
  u32x4 r;
  const uint32_t w[2] = {lo, hi};
#pragma unroll
  for (int q = 0; q < 2; ++q) {
    const floatx2 a = __builtin_amdgcn_cvt_pk_f32_fp8(w[q], false);
    const floatx2 b = __builtin_amdgcn_cvt_pk_f32_fp8(w[q], true);
    r[2 * q] = __builtin_amdgcn_perm(__float_as_uint(a[1]), __float_as_uint(a[0]), 0x07060302u);
    r[2 * q + 1] = __builtin_amdgcn_perm(__float_as_uint(b[1]), __float_as_uint(b[0]), 0x07060302u);
  }
  return __builtin_bit_cast(bf16x8, r);
}

__device__ __forceinline__ shortx4 fp8x4_to_bf16x4(uint32_t w) {
  const floatx2 a = __builtin_amdgcn_cvt_pk_f32_fp8(w, false);
  const floatx2 b = __builtin_amdgcn_cvt_pk_f32_fp8(w, true);
  u32x2 r;
  r[0] = __builtin_amdgcn_perm(__float_as_uint(a[1]), __float_as_uint(a[0]), 0x07060302u);
  r[1] = __builtin_amdgcn_perm(__float_as_uint(b[1]), __float_as_uint(b[0]), 0x07060302u);
  return __builtin_bit_cast(shortx4, r);
}

// Loads one 16-token tile (tokens [o0, o0+16) of block blk) into registers.
template <int D, bool FP8>
__device__ __forceinline__ void load_tile(Tile<D, FP8> &t, const uint8_t *__restrict__ kc,
                                          const uint8_t *__restrict__ vc, int64_t blk, int kvh, int Hkv, int BS,
                                          int o0, int col, int grp) {
  if constexpr (!FP8) {
    constexpr int C = D / 8;
    const uint8_t *kb = kc + (((blk * Hkv + kvh) * C) * BS + o0 + col) * 16;
#pragma unroll
    for (int j = 0; j < Tile<D, FP8>::NQK; ++j)
      t.k[j] = __builtin_bit_cast(bf16x8, *reinterpret_cast<const u32x4 *>(kb + (4 * j + grp) * BS * 16));
    const uint8_t *vb = vc + (((blk * Hkv + kvh) * D + col) * BS + o0 + 4 * grp) * 2;
#pragma unroll
    for (int n = 0; n < Tile<D, FP8>::NPV; ++n)
      t.v[n] = __builtin_bit_cast(shortx4, *reinterpret_cast<const u32x2 *>(vb + n * 16 * BS * 2));
  } else {
    constexpr int C = D / 16;
    const uint8_t *kb = kc + (((blk * Hkv + kvh) * C) * BS + o0 + col) * 16;
#pragma unroll
    for (int m = 0; m < D / 64; ++m) {
      const u32x4 raw = *reinterpret_cast<const u32x4 *>(kb + (4 * m + grp) * BS * 16);
      t.k[2 * m] = fp8x8_to_bf16x8(raw[0], raw[1]);
      t.k[2 * m + 1] = fp8x8_to_bf16x8(raw[2], raw[3]);
    }
    const uint8_t *vb = vc + ((blk * Hkv + kvh) * D + col) * BS + o0 + 4 * grp;
#pragma unroll
    for (int n = 0; n < Tile<D, FP8>::NPV; ++n)
      t.v[n] = fp8x4_to_bf16x4(*reinterpret_cast<const uint32_t *>(vb + n * 16 * BS));
  }
}

template <int D, bool FP8>
struct DecodeState {
  floatx4 o[D / 16];
  float m;  // running max (log2 domain) of this lane's head column
  float l;  // this lane's share of the running denominator
};

// One tile of online-softmax attention. `valid` = tokens of the tile that
// belong to the sequence (16 except in the last tile).
template <int D, bool FP8>
__device__ __forceinline__ void attend_tile(DecodeState<D, FP8> &st, Tile<D, FP8> &t, const bf16x8 *qop,
                                            float s_mul, float p_mul, int valid, int grp) {
  floatx4 s = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int j = 0; j < Tile<D, FP8>::NQK; ++j) s = __builtin_amdgcn_mfma_f32_16x16x32_bf16(t.k[j], qop[j], s, 0, 0, 0);
  float sv[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) sv[i] = (4 * grp + i < valid) ? s[i] * s_mul : -INFINITY;
  float mt = fmaxf(fmaxf(sv[0], sv[1]), fmaxf(sv[2], sv[3]));
  mt = fmaxf(mt, __shfl_xor(mt, 16, 64));
  mt = fmaxf(mt, __shfl_xor(mt, 32, 64));
  const float m_new = fmaxf(st.m, mt);
  const float m_use = (m_new == -INFINITY) ? 0.f : m_new;
  const float corr = exp2f(st.m - m_use);
  float p[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) p[i] = exp2f(sv[i] - m_use);
  st.l = st.l * corr + ((p[0] + p[1]) + (p[2] + p[3]));
  st.m = m_new;
#pragma unroll
  for (int n = 0; n < D / 16; ++n) {
#pragma unroll
    for (int i = 0; i < 4; ++i) st.o[n][i] *= corr;
  }
  u32x2 pb;
  pb[0] = f32_to_bf16_bits(p[0] * p_mul) | (f32_to_bf16_bits(p[1] * p_mul) << 16);
  pb[1] = f32_to_bf16_bits(p[2] * p_mul) | (f32_to_bf16_bits(p[3] * p_mul) << 16);
  const shortx4 pop = __builtin_bit_cast(shortx4, pb);
  if (valid < 16) {
    // Never let a masked slot's V reach the accumulator (it may hold NaN).
#pragma unroll
    for (int n = 0; n < D / 16; ++n) {
#pragma unroll
      for (int e = 0; e < 4; ++e)
        if (4 * grp + e >= valid) t.v[n][e] = 0;
    }
  }
#pragma unroll
  for (int n = 0; n < D / 16; ++n) st.o[n] = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(t.v[n], pop, st.o[n], 0, 0, 0);
}

template <int D, bool FP8>
__global__ __launch_bounds__(64) void decode_gqa_kernel(
    const uint8_t *__restrict__ kc, const uint8_t *__restrict__ vc, const float *__restrict__ ks,
    const float *__restrict__ vs, const uint16_t *__restrict__ q, int64_t q_sb, int64_t q_sh,
    uint16_t *__restrict__ out, float *__restrict__ part_o, float *__restrict__ part_ml,
    int *__restrict__ counters, const int32_t *__restrict__ bt, int64_t bt_stride, int max_seq, const int32_t *__restrict__ seq_lens,
    int Hq, int Hkv, int G, int BS, int64_t NB, float scale_log2, int P_tok, int max_parts) {
  const int part = blockIdx.x, kvh = blockIdx.y, b = blockIdx.z;
  const int lane = threadIdx.x, col = lane & 15, grp = lane >> 4;
  int L = seq_lens[b];
  L = L < max_seq ? L : max_seq;  // max_seq <= block-table width * BS: every read stays in the table
  const int nparts = L > 0 ? (L + P_tok - 1) / P_tok : 0;
  if (nparts == 0) {
    if (part == 0 && col < G) {  // empty context: zeros
      uint16_t *op = out + (static_cast<int64_t>(b) * Hq + kvh * G + col) * D;
#pragma unroll
      for (int n = 0; n < D / 16; ++n) *reinterpret_cast<u32x2 *>(op + 16 * n + 4 * grp) = u32x2{0u, 0u};
    }
    return;
  }
  if (part >= nparts) return;

  // Q^T operand: lane holds 8 d-values of head `col` (zero for padded heads).
  // The d order matches the K operand order of load_tile.
  bf16x8 qop[D / 32];
  {
    const uint16_t *qp = q + b * q_sb + static_cast<int64_t>(kvh * G + (col < G ? col : 0)) * q_sh;
#pragma unroll
    for (int j = 0; j < D / 32; ++j) {
      const int d0 = FP8 ? 16 * (4 * (j >> 1) + grp) + 8 * (j & 1) : 32 * j + 8 * grp;
      u32x4 w = *reinterpret_cast<const u32x4 *>(qp + d0);
      if (col >= G) w = u32x4{0u, 0u, 0u, 0u};
      qop[j] = __builtin_bit_cast(bf16x8, w);
    }
  }

  DecodeState<D, FP8> st;
#pragma unroll
  for (int n = 0; n < D / 16; ++n) st.o[n] = floatx4{0.f, 0.f, 0.f, 0.f};
  st.m = -INFINITY;
  st.l = 0.f;

  const int t_begin = part * P_tok;
  const int t_end = (t_begin + P_tok) < L ? (t_begin + P_tok) : L;
  const int32_t *btrow = bt + b * bt_stride;

  // Block id of a tile; an out-of-range id turns the tile into masked slots.
  auto tile_block = [&](int ts, int &valid) -> int64_t {
    int64_t blk = btrow[ts / BS];
    valid = (t_end - ts) < 16 ? (t_end - ts) : 16;
    if (blk < 0 || blk >= NB) {
      blk = 0;
      valid = 0;
    }
    return blk;
  };

  Tile<D, FP8> ta, tb;
  int va, vb;
  int64_t ba = tile_block(t_begin, va), bb = 0;
  load_tile<D, FP8>(ta, kc, vc, ba, kvh, Hkv, BS, t_begin % BS, col, grp);
  for (int ts = t_begin; ts < t_end; ts += 32) {
    const bool more = ts + 16 < t_end;
    if (more) {
      bb = tile_block(ts + 16, vb);
      load_tile<D, FP8>(tb, kc, vc, bb, kvh, Hkv, BS, (ts + 16) % BS, col, grp);
    }
    {
      const float ksc = FP8 ? ks[ba * Hkv + kvh] : 1.f;
      const float vsc = FP8 ? vs[ba * Hkv + kvh] : 1.f;
      attend_tile<D, FP8>(st, ta, qop, scale_log2 * ksc, vsc, va, grp);
    }
    if (!more) break;
    if (ts + 32 < t_end) {
      ba = tile_block(ts + 32, va);
      load_tile<D, FP8>(ta, kc, vc, ba, kvh, Hkv, BS, (ts + 32) % BS, col, grp);
    }
    {
      const float ksc = FP8 ? ks[bb * Hkv + kvh] : 1.f;
      const float vsc = FP8 ? vs[bb * Hkv + kvh] : 1.f;
      attend_tile<D, FP8>(st, tb, qop, scale_log2 * ksc, vsc, vb, grp);
    }
  }

  float l = st.l + __shfl_xor(st.l, 16, 64);
  l += __shfl_xor(l, 32, 64);
  const int hq = kvh * G + col;
  if (nparts == 1) {
    if (col < G) {
      const float inv = l > 0.f ? 1.f / l : 0.f;
      uint16_t *op = out + (static_cast<int64_t>(b) * Hq + hq) * D;
#pragma unroll
      for (int n = 0; n < D / 16; ++n) {
        u32x2 w;
        w[0] = f32_to_bf16_bits(st.o[n][0] * inv) | (f32_to_bf16_bits(st.o[n][1] * inv) << 16);
        w[1] = f32_to_bf16_bits(st.o[n][2] * inv) | (f32_to_bf16_bits(st.o[n][3] * inv) << 16);
        *reinterpret_cast<u32x2 *>(op + 16 * n + 4 * grp) = w;
      }
    }
    return;
  }
  if (col < G) {
    const int64_t row = (static_cast<int64_t>(b) * Hq + hq) * max_parts + part;
    float *po = part_o + row * D;
#pragma unroll
    for (int n = 0; n < D / 16; ++n) *reinterpret_cast<floatx4 *>(po + 16 * n + 4 * grp) = st.o[n];
    if (grp == 0) {
      part_ml[2 * row] = st.m;
      part_ml[2 * row + 1] = l;
    }
  }

  // The last partition of this (sequence, KV head) to finish merges all of
  // them by log-sum-exp: release the partials, take a ticket, and only the
  // holder of the final ticket acquires and reads them back.
  __threadfence();
  int ticket = 0;
  if (lane == 0) ticket = atomicAdd(&counters[b * Hkv + kvh], 1);
  ticket = __shfl(ticket, 0, 64);
  if (ticket != nparts - 1) return;
  __threadfence();
  for (int e = lane; e < G * (D / 4); e += 64) {
    const int h = e / (D / 4), d0 = (e % (D / 4)) * 4;
    const int64_t row0 = (static_cast<int64_t>(b) * Hq + kvh * G + h) * max_parts;
    float M = -INFINITY;
    for (int p = 0; p < nparts; ++p)
      M = fmaxf(M, __hip_atomic_load(&part_ml[2 * (row0 + p)], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT));
    const float m_use = (M == -INFINITY) ? 0.f : M;
    float den = 0.f, num[4] = {0.f, 0.f, 0.f, 0.f};
    for (int p = 0; p < nparts; ++p) {
      const float mp = __hip_atomic_load(&part_ml[2 * (row0 + p)], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      const float lp = __hip_atomic_load(&part_ml[2 * (row0 + p) + 1], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      const float w = exp2f(mp - m_use);
      den += w * lp;
      const float *po = part_o + (row0 + p) * D + d0;
#pragma unroll
      for (int i = 0; i < 4; ++i) num[i] += w * __hip_atomic_load(po + i, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    const float inv = den > 0.f ? 1.f / den : 0.f;
    u32x2 wv;
    wv[0] = f32_to_bf16_bits(num[0] * inv) | (f32_to_bf16_bits(num[1] * inv) << 16);
    wv[1] = f32_to_bf16_bits(num[2] * inv) | (f32_to_bf16_bits(num[3] * inv) << 16);
    *reinterpret_cast<u32x2 *>(out + (static_cast<int64_t>(b) * Hq + kvh * G + h) * D + d0) = wv;
  }
  if (lane == 0) counters[b * Hkv + kvh] = 0;  // leave the ticket counter zeroed for the next call
}

static int choose_partition(int batch, int hkv, int max_seq_len) {
  // Enough work items to fill 256 CUs several waves deep, but at least 256
  // tokens per item so the partial-result traffic stays a few percent.
  const int64_t items = static_cast<int64_t>(batch) * hkv;
  int p = 256;
  while (p < 2048 && items * ((max_seq_len + 2 * p - 1) / (2 * p)) >= 4096) p *= 2;
  return p;
}

}  // namespace wkv

using namespace wkv;

extern "C" int64_t wkv_decode_workspace_size(int32_t batch, int32_t num_q_heads, int32_t head_dim,
                                             int32_t max_seq_len, int32_t partition_size) {
  if (batch < 0 || num_q_heads <= 0 || head_dim <= 0 || max_seq_len < 0 || partition_size < 0) return -1;
  if (partition_size == 0) partition_size = 256;  // smallest partition the library picks by itself
  const int64_t max_parts = (static_cast<int64_t>(max_seq_len) + partition_size - 1) / partition_size;
  // partial outputs and (max, sum) per (sequence, query head, partition)
  return static_cast<int64_t>(batch) * num_q_heads * (max_parts > 0 ? max_parts : 1) * (head_dim + 2) * 4;
}

extern "C" int wkv_paged_decode_gqa(const wkv_cache_t *cache, const void *q, int64_t q_stride_b,
                                    int64_t q_stride_h, void *out, int32_t num_q_heads,
                                    const int32_t *block_table, int64_t bt_stride, int32_t max_blocks_per_seq,
                                    const int32_t *seq_lens, int32_t batch, int32_t max_seq_len, float scale,
                                    int32_t partition_size, void *workspace, int64_t workspace_bytes,
                                    int32_t *tickets, int64_t num_tickets, void *stream) {
  int rc = check_cache(cache, -1);
  if (rc) return rc;
  WKV_CHECK_ARG(batch >= 0 && batch <= 65535, "batch must be in [0, 65535] (got %d)", batch);
  if (batch == 0) return WKV_OK;
  const int Hkv = cache->num_kv_heads, D = cache->head_dim, BS = cache->block_size;
  WKV_CHECK_ARG(num_q_heads > 0 && num_q_heads % Hkv == 0, "num_q_heads %d must be a multiple of num_kv_heads %d",
                num_q_heads, Hkv);
  const int G = num_q_heads / Hkv;
  if (G > 16) return fail(WKV_ERR_UNSUPPORTED, "query group size %d > 16 not supported", G);
  WKV_CHECK_ARG(Hkv <= 65535, "num_kv_heads too large");
  WKV_CHECK_ARG(q != nullptr && aligned16(q), "q must be non-NULL and 16-byte aligned");
  WKV_CHECK_ARG(q_stride_b >= 0 && q_stride_h >= 0 && q_stride_b % 8 == 0 && q_stride_h % 8 == 0,
                "q strides must be non-negative multiples of 8");
  WKV_CHECK_ARG(out != nullptr && aligned16(out), "out must be non-NULL and 16-byte aligned");
  WKV_CHECK_ARG(block_table != nullptr && seq_lens != nullptr, "block_table / seq_lens is NULL");
  WKV_CHECK_ARG(max_blocks_per_seq > 0 && bt_stride >= max_blocks_per_seq, "bad block table geometry");
  WKV_CHECK_ARG(max_seq_len >= 0, "max_seq_len must be >= 0");
  WKV_CHECK_ARG(std::isfinite(scale), "scale must be finite");
  if (partition_size == 0) partition_size = choose_partition(batch, Hkv, max_seq_len);
  WKV_CHECK_ARG(partition_size >= 16 && partition_size % 16 == 0, "partition_size must be a positive multiple of 16");
  const int max_seq = max_seq_len < max_blocks_per_seq * BS ? max_seq_len : max_blocks_per_seq * BS;
  const int max_parts = max_seq > 0 ? (max_seq + partition_size - 1) / partition_size : 1;
  WKV_CHECK_ARG(max_parts <= 65535, "too many partitions (%d)", max_parts);
  const int64_t need = wkv_decode_workspace_size(batch, num_q_heads, D, max_seq, partition_size);
  if (max_parts > 1) {
    WKV_CHECK_ARG(workspace != nullptr && aligned16(workspace) && workspace_bytes >= need,
                  "workspace too small: need %lld bytes, got %lld", (long long)need, (long long)workspace_bytes);
    WKV_CHECK_ARG(tickets != nullptr && num_tickets >= static_cast<int64_t>(batch) * Hkv,
                  "tickets must hold batch * num_kv_heads = %lld zeroed int32 counters",
                  (long long)batch * Hkv);
  }
  float *part_o = static_cast<float *>(workspace);
  float *part_ml = part_o ? part_o + static_cast<int64_t>(batch) * num_q_heads * max_parts * D : nullptr;
  int *counters = tickets;
  const float scale_log2 = scale * 1.4426950408889634f;
  auto s = static_cast<hipStream_t>(stream);
  const dim3 grid(static_cast<unsigned>(max_parts), static_cast<unsigned>(Hkv), static_cast<unsigned>(batch));
  auto kc = static_cast<const uint8_t *>(cache->k);
  auto vc = static_cast<const uint8_t *>(cache->v);
  auto qq = static_cast<const uint16_t *>(q);
  auto oo = static_cast<uint16_t *>(out);
  const bool fp8 = cache->kv_dtype == WKV_KV_FP8_E4M3;
#define WKV_DECODE(Dv, F8)                                                                                   \
  decode_gqa_kernel<Dv, F8><<<grid, 64, 0, s>>>(kc, vc, cache->k_scale, cache->v_scale, qq, q_stride_b,    \
                                                q_stride_h, oo, part_o, part_ml, counters, block_table,   \
                                                bt_stride,                                                \
                                                max_seq, seq_lens, num_q_heads, Hkv, G, BS,               \
                                                cache->num_blocks, scale_log2, partition_size, max_parts)
  if (D == 128) {
    if (fp8) WKV_DECODE(128, true); else WKV_DECODE(128, false);
  } else {
    if (fp8) WKV_DECODE(64, true); else WKV_DECODE(64, false);
  }
#undef WKV_DECODE
  WKV_CHECK_LAUNCH("wkv_paged_decode_gqa");
  return WKV_OK;
}
