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

}  // namespace wkv
