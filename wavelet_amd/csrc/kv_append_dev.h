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
      const float ratio = s_old / s;  // exact power of two
      for (int e = lane; e < first * D; e += 64) {
        const int off = e / D, d = e % D;
        const int64_t a = IS_V ? fp8_v_index<D>(blk, h, H, BS, off, d) : fp8_k_index<D>(blk, h, H, BS, off, d);
        cache[a] = static_cast<uint8_t>(e4m3_encode(e4m3_decode(cache[a]) * ratio));
      }
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

}  // namespace wkv
