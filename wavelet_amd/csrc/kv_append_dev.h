// Device-side fp8 append shared by the append kernel and the fused append +
// decode kernel (one wave appends one run of one KV head).
#pragma once

#include "wkv_common.h"

namespace wkv {

// ---------------------------------------------------------------------------
// fp8 append of one run (tokens t..t+r-1, all in block blk, the first at
// offset `first`) for one head, by one wave: scale update, re-encode of the
// block's earlier entries when the scale grows, then the run's codes.
template <int D>
__device__ __forceinline__ int64_t fp8_k_index(int64_t blk, int h, int H, int BS, int off, int d) {
  return (((blk * H + h) * (D / 16) + (d >> 4)) * BS + off) * 16 + (d & 15);
}
template <int D>
__device__ __forceinline__ int64_t fp8_v_index(int64_t blk, int h, int H, int BS, int off, int d) {
  return ((blk * H + h) * D + d) * BS + off;
}

// Re-encodes the codes at offsets [0, first) of the (blk, h) region of K (IS_V
// false) or V at a grown scale: each code times `ratio`, an exact power of two
// below 1 (e4m3_encode(e4m3_decode(c) * ratio), code by code, as the oracle
// states it). The region is walked in 16-byte pieces, four per lane a pass,
// every load of a pass issued before its stores (a byte loop waits one memory
// round trip per byte). K [D/16][BS][16]: piece p holds token p % BS's 16
// d-values of one chunk; V [D][BS]: piece p holds tokens 16 (p % (BS/16)) ..
// + 15 of one d row. Pieces at or past `first` are not stored.
template <int D, bool IS_V>
__device__ __forceinline__ void fp8_reencode_block(uint8_t *__restrict__ cache, int64_t blk, int h, int H, int BS,
                                                   int first, float ratio) {
  const int lane = threadIdx.x & 63;
  u32x4 *base = reinterpret_cast<u32x4 *>(cache + (blk * H + h) * static_cast<int64_t>(D) * BS);
  const int np = D * BS / 16;
  constexpr int PL = 4;
  for (int p0 = 0; p0 < np; p0 += 64 * PL) {
    u32x4 w[PL];
#pragma unroll
    for (int k = 0; k < PL; ++k) {
      const int p = p0 + 64 * k + lane;
      if (p < np) w[k] = base[p];
    }
#pragma unroll
    for (int k = 0; k < PL; ++k) {
      const int p = p0 + 64 * k + lane;
      const int tok0 = IS_V ? 16 * (p % (BS / 16)) : p % BS;
      if (p >= np || tok0 >= first) continue;
      u32x4 o = w[k];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
#pragma unroll
        for (int b = 0; b < 4; ++b) {
          const int tok = IS_V ? tok0 + 4 * j + b : tok0;
          if (tok < first) {
            const uint32_t c = (o[j] >> (8 * b)) & 0xffu;
            const uint32_t n = e4m3_encode(e4m3_decode(c) * ratio);
            o[j] = (o[j] & ~(0xffu << (8 * b))) | (n << (8 * b));
          }
        }
      }
      base[p] = o;
    }
  }
}

template <int D, bool IS_V>
__device__ void fp8_append_one(uint8_t *__restrict__ cache, float *__restrict__ scales,
                               const uint16_t *__restrict__ src, int64_t st, int64_t sh,
                               const int64_t *__restrict__ slots, int64_t t, int r, int64_t blk, int first,
                               int h, int H, int BS) {
  const int lane = threadIdx.x & 63;  // the calling wave's lane (workgroups may hold several waves)
  float amax = 0.0f;
  for (int e = lane; e < r * D; e += 64) {
    const int tok = e / D, d = e % D;
    amax = fmaxf(amax, fabsf(bf16_bits_to_f32(src[(t + tok) * st + h * sh + d])));
  }
  amax = wave_max(amax);
  const float s_new = pow2_scale(amax);
  float s = s_new;
  if (first != 0) {
    const float s_old = scales[blk * H + h];
    s = (s_new > s_old) ? s_new : s_old;
    if (s > s_old) {
      // Byte by byte: with fp8_reencode_block here the fused decode kernel that
      // inlines this (one run of one token) measured 3-4% slower per launch
      // even in steps where no block grows (fp8 Qwen2.5-7B groups and Qwen3-4B
      // shapes, in-process A/B).
      const float ratio = s_old / s;  // exact power of two
      for (int e = lane; e < first * D; e += 64) {
        const int off = e / D, d = e % D;
        const int64_t a = IS_V ? fp8_v_index<D>(blk, h, H, BS, off, d) : fp8_k_index<D>(blk, h, H, BS, off, d);
        cache[a] = static_cast<uint8_t>(e4m3_encode(e4m3_decode(cache[a]) * ratio));
      }
    }
  }
  for (int e = lane; e < r * D; e += 64) {
    const int tok = e / D, d = e % D;
    const int off = static_cast<int>(slots[t + tok] % BS);
    const float x = bf16_bits_to_f32(src[(t + tok) * st + h * sh + d]);
    const int64_t a = IS_V ? fp8_v_index<D>(blk, h, H, BS, off, d) : fp8_k_index<D>(blk, h, H, BS, off, d);
    cache[a] = static_cast<uint8_t>(e4m3_quantize(x, s));
  }
  if (lane == 0) scales[blk * H + h] = s;
}

// The step token's K and V rows of one head as loaded (bf16 bits, d = lane +
// 64 i): loaded apart from the rest of the append so that a caller can issue
// them early and let their round trip overlap its own start (nothing here
// waits for them; the append below converts them).
template <int D>
struct Fp8TokenRows {
  uint32_t k[D / 64], v[D / 64];
};
template <int D>
__device__ __forceinline__ void fp8_token_rows_load(Fp8TokenRows<D> &r, const uint16_t *__restrict__ krow,
                                                    const uint16_t *__restrict__ vrow) {
  const int lane = threadIdx.x & 63;
#pragma unroll
  for (int i = 0; i < D / 64; ++i) {
    r.k[i] = krow[lane + 64 * i];
    r.v[i] = vrow[lane + 64 * i];
  }
}

// The step token's codes and the block's scales after its append, without
// writing anything: the same scale decision as fp8_append_token_kv (the
// token's power-of-two scale, or the block's own if that is not smaller),
// `grow` when the block's earlier codes would need re-encoding, and the
// token's K and V codes at the resulting scales, d = lane + 64 i.
template <int D>
struct Fp8TokenCodes {
  uint32_t k[D / 64], v[D / 64];
  float sk, sv;
  bool grow;
};
template <int D>
__device__ __forceinline__ Fp8TokenCodes<D> fp8_token_codes(const float *__restrict__ ks, const float *__restrict__ vs,
                                                            const Fp8TokenRows<D> &rows, int64_t blk, int off, int h,
                                                            int H) {
  constexpr int PER = D / 64;
  float xk[PER], xv[PER];
#pragma unroll
  for (int i = 0; i < PER; ++i) {
    xk[i] = bf16_bits_to_f32(static_cast<uint16_t>(rows.k[i]));
    xv[i] = bf16_bits_to_f32(static_cast<uint16_t>(rows.v[i]));
  }
  const int64_t si = blk * H + h;
  const float sk_old = off != 0 ? ks[si] : 0.f, sv_old = off != 0 ? vs[si] : 0.f;
  float ak = 0.f, av = 0.f;
#pragma unroll
  for (int i = 0; i < PER; ++i) {
    ak = fmaxf(ak, fabsf(xk[i]));
    av = fmaxf(av, fabsf(xv[i]));
  }
  ak = wave_max(ak);
  av = wave_max(av);
  Fp8TokenCodes<D> c;
  c.sk = pow2_scale(ak);
  c.sv = pow2_scale(av);
  c.grow = false;
  if (off != 0) {
    c.grow = c.sk > sk_old || c.sv > sv_old;
    if (!(c.sk > sk_old)) c.sk = sk_old;
    if (!(c.sv > sv_old)) c.sv = sv_old;
  }
#pragma unroll
  for (int i = 0; i < PER; ++i) {
    c.k[i] = e4m3_quantize(xk[i], c.sk);
    c.v[i] = e4m3_quantize(xv[i], c.sv);
  }
  return c;
}

// fp8 append of one token (the fused decode's step token) for one head, K and
// V together, from its loaded rows: both old scales are loaded at once and
// both rows reduced side by side, so the two appends cost one chain of memory
// round trips instead of two. The same codes, scales and re-encodes as
// fp8_append_one on each of K and V with a run of one token.
template <int D>
__device__ __forceinline__ void fp8_append_token_kv(uint8_t *__restrict__ kc, uint8_t *__restrict__ vc,
                                                    float *__restrict__ ks, float *__restrict__ vs,
                                                    const Fp8TokenRows<D> &rows, int64_t blk, int off, int h, int H,
                                                    int BS) {
  constexpr int PER = D / 64;  // elements of a row per lane: d = lane + 64 i
  const int lane = threadIdx.x & 63;
  float xk[PER], xv[PER];
#pragma unroll
  for (int i = 0; i < PER; ++i) {
    xk[i] = bf16_bits_to_f32(static_cast<uint16_t>(rows.k[i]));
    xv[i] = bf16_bits_to_f32(static_cast<uint16_t>(rows.v[i]));
  }
  const int64_t si = blk * H + h;
  const float sk_old = off != 0 ? ks[si] : 0.f, sv_old = off != 0 ? vs[si] : 0.f;
  float ak = 0.f, av = 0.f;
#pragma unroll
  for (int i = 0; i < PER; ++i) {
    ak = fmaxf(ak, fabsf(xk[i]));
    av = fmaxf(av, fabsf(xv[i]));
  }
  ak = wave_max(ak);
  av = wave_max(av);
  float sk = pow2_scale(ak), sv = pow2_scale(av);
  if (off != 0) {
    if (sk > sk_old) {  // the block's earlier K codes at the grown scale, byte by byte
      const float ratio = sk_old / sk;
      for (int e = lane; e < off * D; e += 64) {
        const int64_t a = fp8_k_index<D>(blk, h, H, BS, e / D, e % D);
        kc[a] = static_cast<uint8_t>(e4m3_encode(e4m3_decode(kc[a]) * ratio));
      }
    } else {
      sk = sk_old;
    }
    if (sv > sv_old) {
      const float ratio = sv_old / sv;
      for (int e = lane; e < off * D; e += 64) {
        const int64_t a = fp8_v_index<D>(blk, h, H, BS, e / D, e % D);
        vc[a] = static_cast<uint8_t>(e4m3_encode(e4m3_decode(vc[a]) * ratio));
      }
    } else {
      sv = sv_old;
    }
  }
#pragma unroll
  for (int i = 0; i < PER; ++i) {
    kc[fp8_k_index<D>(blk, h, H, BS, off, lane + 64 * i)] = static_cast<uint8_t>(e4m3_quantize(xk[i], sk));
    vc[fp8_v_index<D>(blk, h, H, BS, off, lane + 64 * i)] = static_cast<uint8_t>(e4m3_quantize(xv[i], sv));
  }
  if (lane == 0) {
    ks[si] = sk;
    vs[si] = sv;
  }
}

// The same append with 16-byte source loads and 16-byte K stores, and the
// quantisation as a product with 1 / scale (a power of two: x * (1 / s) and
// x / s round the same exact value, so the codes are identical). The source
// rows must be 16-byte aligned (the host checks). K: a lane quantises one
// (token, 16-d chunk) piece into 16 contiguous code bytes; V: one d row's
// byte per token, as before.
template <int D, bool IS_V>
__device__ void fp8_append_run_vec(uint8_t *__restrict__ cache, float *__restrict__ scales,
                                   const uint16_t *__restrict__ src, int64_t st, int64_t sh,
                                   const int64_t *__restrict__ slots, int64_t t, int r, int64_t blk, int first, int h,
                                   int H, int BS) {
  const int lane = threadIdx.x & 63;
  float amax = 0.0f;
  for (int e = lane; e < r * (D / 8); e += 64) {
    const int tok = e / (D / 8), g = e % (D / 8);
    const u32x4 w = *reinterpret_cast<const u32x4 *>(src + (t + tok) * st + h * sh + 8 * g);
#pragma unroll
    for (int j = 0; j < 4; ++j)
      amax = fmaxf(amax, fmaxf(fabsf(__uint_as_float(w[j] << 16)), fabsf(__uint_as_float(w[j] & 0xffff0000u))));
  }
  amax = wave_max(amax);
  const float s_new = pow2_scale(amax);
  float s = s_new;
  if (first != 0) {
    const float s_old = scales[blk * H + h];
    s = (s_new > s_old) ? s_new : s_old;
    if (s > s_old) {  // the block's earlier codes are re-encoded at the grown scale
      fp8_reencode_block<D, IS_V>(cache, blk, h, H, BS, first, s_old / s);  // exact power-of-two ratio
    }
  }
  const float inv = 1.0f / s;  // exact: s is a power of two in [2^-42, 2^119]
  auto q = [&](float x) {
    float v = x * inv;
    v = (v != v) ? v : fminf(fmaxf(v, -448.0f), 448.0f);
    return e4m3_encode(v);
  };
  if constexpr (!IS_V) {
    for (int e = lane; e < r * (D / 16); e += 64) {
      const int tok = e / (D / 16), c = e % (D / 16);
      const int off = static_cast<int>(slots[t + tok] % BS);
      const uint16_t *p = src + (t + tok) * st + h * sh + 16 * c;
      const u32x4 w0 = *reinterpret_cast<const u32x4 *>(p), w1 = *reinterpret_cast<const u32x4 *>(p + 8);
      u32x4 out;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const u32x4 &w = j < 2 ? w0 : w1;
        const uint32_t lo = w[(2 * j) & 3], hi = w[(2 * j + 1) & 3];
        out[j] = q(__uint_as_float(lo << 16)) | (q(__uint_as_float(lo & 0xffff0000u)) << 8) |
                 (q(__uint_as_float(hi << 16)) << 16) | (q(__uint_as_float(hi & 0xffff0000u)) << 24);
      }
      *reinterpret_cast<u32x4 *>(cache + fp8_k_index<D>(blk, h, H, BS, off, 16 * c)) = out;
    }
  } else {
    for (int e = lane; e < r * D; e += 64) {
      const int tok = e / D, d = e % D;
      const int off = static_cast<int>(slots[t + tok] % BS);
      const float x = bf16_bits_to_f32(src[(t + tok) * st + h * sh + d]);
      cache[fp8_v_index<D>(blk, h, H, BS, off, d)] = static_cast<uint8_t>(q(x));
    }
  }
  if (lane == 0) scales[blk * H + h] = s;
}

// Codes of a and b (after the clamp to +-448; never NaN here) in bytes
// 2 w, 2 w + 1 of `old`, by the hardware conversion: for every finite input
// bit-identical to e4m3_encode (checked on the GPU for all bf16 patterns at
// several scales). NaN is the one difference -- the hardware codes +NaN 0xFF
// where e4m3_encode gives 0x7F -- so callers keep NaN off this path.
template <bool W1>
__device__ __forceinline__ uint32_t e4m3_pack2(float a, float b, uint32_t old) {
  return static_cast<uint32_t>(__builtin_amdgcn_cvt_pk_fp8_f32(a, b, static_cast<int>(old), W1));
}

// Four bf16 pairs (words w0..w3, low half first) times inv, clamped, as 8 codes
// in two words.
__device__ __forceinline__ u32x2 e4m3_pack8(uint32_t w0, uint32_t w1, uint32_t w2, uint32_t w3, float inv) {
  auto lo = [&](uint32_t w) { return __builtin_amdgcn_fmed3f(__uint_as_float(w << 16) * inv, -448.f, 448.f); };
  auto hi = [&](uint32_t w) { return __builtin_amdgcn_fmed3f(__uint_as_float(w & 0xffff0000u) * inv, -448.f, 448.f); };
  u32x2 r;
  r[0] = e4m3_pack2<true>(lo(w1), hi(w1), e4m3_pack2<false>(lo(w0), hi(w0), 0u));
  r[1] = e4m3_pack2<true>(lo(w3), hi(w3), e4m3_pack2<false>(lo(w2), hi(w2), 0u));
  return r;
}

// fp8 append of a whole fresh block (16 tokens t..t+15 at offsets 0..15 of
// block blk, block_size 16) for one head, K and V, by one wave -- the prompt
// case. The block starts afresh (its scale is the run's), so nothing earlier
// is re-encoded. Returns false, having written nothing, when the block's
// inputs hold a NaN (the caller then takes fp8_append_run_vec, which codes NaN
// as e4m3_encode does). K: lane l quantises token l % 16, 16-d chunks
// l / 16 + 4 j, each one 16-byte store; V: lane l owns d rows RV l .. RV l +
// RV - 1 (RV = D / 64) and stores each row's 16 tokens as 16 bytes. Each
// block's absolute maximum is an integer maximum of bf16 magnitude bits (a
// NaN's bits exceed infinity's). Source rows 16-byte aligned (the host checks).
template <int D>
__device__ bool fp8_append_block16(uint8_t *__restrict__ kc, uint8_t *__restrict__ vc, float *__restrict__ ks,
                                   float *__restrict__ vs, const uint16_t *__restrict__ key, int64_t kst,
                                   int64_t ksh, const uint16_t *__restrict__ val, int64_t vst, int64_t vsh,
                                   int64_t t, int64_t blk, int h, int H) {
  constexpr int BS = 16, NC = D / 64, RV = D / 64;
  const int lane = threadIdx.x & 63;
  const int m = lane & 15;
  u32x4 kw[NC][2];
#pragma unroll
  for (int j = 0; j < NC; ++j) {
    const uint16_t *p = key + (t + m) * kst + h * ksh + 16 * ((lane >> 4) + 4 * j);
    kw[j][0] = *reinterpret_cast<const u32x4 *>(p);
    kw[j][1] = *reinterpret_cast<const u32x4 *>(p + 8);
  }
  uint32_t vw[BS];  // token i's RV values of this lane's rows (RV = 2: one word, RV = 1: the low half)
#pragma unroll
  for (int i = 0; i < BS; ++i) {
    const uint16_t *p = val + (t + i) * vst + h * vsh + RV * lane;
    if constexpr (RV == 2)
      vw[i] = *reinterpret_cast<const uint32_t *>(p);
    else
      vw[i] = *p;
  }
  uint32_t ka = 0u, va = 0u;  // largest magnitude bits, as bf16
#pragma unroll
  for (int j = 0; j < NC; ++j)
#pragma unroll
    for (int q = 0; q < 2; ++q)
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const uint32_t w = kw[j][q][e];
        ka = max(ka, max(w & 0x7fffu, (w >> 16) & 0x7fffu));
      }
#pragma unroll
  for (int i = 0; i < BS; ++i) va = max(va, max(vw[i] & 0x7fffu, (vw[i] >> 16) & 0x7fffu));
  ka = wave_reduce(ka, [](uint32_t a, uint32_t b) { return a > b ? a : b; });
  va = wave_reduce(va, [](uint32_t a, uint32_t b) { return a > b ? a : b; });
  if (ka > 0x7f80u || va > 0x7f80u) return false;  // uniform: a NaN somewhere
  const float sk = pow2_scale(__uint_as_float(ka << 16)), sv = pow2_scale(__uint_as_float(va << 16));
  const float ik = 1.0f / sk, iv = 1.0f / sv;  // exact: powers of two
#pragma unroll
  for (int j = 0; j < NC; ++j) {
    const u32x2 a = e4m3_pack8(kw[j][0][0], kw[j][0][1], kw[j][0][2], kw[j][0][3], ik);
    const u32x2 b = e4m3_pack8(kw[j][1][0], kw[j][1][1], kw[j][1][2], kw[j][1][3], ik);
    *reinterpret_cast<u32x4 *>(kc + fp8_k_index<D>(blk, h, H, BS, m, 16 * ((lane >> 4) + 4 * j))) =
        u32x4{a[0], a[1], b[0], b[1]};
  }
#pragma unroll
  for (int rr = 0; rr < RV; ++rr) {
    // row RV lane + rr: the rr-th half of every token's word, 16 tokens
    auto row = [&](int i) { return (vw[i] >> (16 * rr)) & 0xffffu; };
    auto pair = [&](int i) { return row(i) | (row(i + 1) << 16); };
    const u32x2 a = e4m3_pack8(pair(0), pair(2), pair(4), pair(6), iv);
    const u32x2 b = e4m3_pack8(pair(8), pair(10), pair(12), pair(14), iv);
    const u32x4 out = {a[0], a[1], b[0], b[1]};
    *reinterpret_cast<u32x4 *>(vc + fp8_v_index<D>(blk, h, H, BS, 0, RV * lane + rr)) = out;
  }
  if (lane == 0) {
    ks[blk * H + h] = sk;
    vs[blk * H + h] = sv;
  }
  return true;
}

}  // namespace wkv
