// Shared device helpers and host-side validation for libwkv (gfx950 only).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <cstdarg>
#include <cstdio>

#include "../../include/wkv.h"

namespace wkv {

// ---------------------------------------------------------------------------
// Vector types matching the MFMA builtin operand types.
typedef __attribute__((__vector_size__(8 * sizeof(__bf16)))) __bf16 bf16x8;
typedef __attribute__((__vector_size__(4 * sizeof(__bf16)))) __bf16 bf16x4;
typedef __attribute__((__vector_size__(2 * sizeof(__bf16)))) __bf16 bf16x2;
typedef __attribute__((__vector_size__(4 * sizeof(float)))) float floatx4;
typedef __attribute__((__vector_size__(2 * sizeof(float)))) float floatx2;
typedef __attribute__((__vector_size__(16 * sizeof(float)))) float floatx16;
typedef __attribute__((__vector_size__(4 * sizeof(uint32_t)))) uint32_t u32x4;
typedef __attribute__((__vector_size__(2 * sizeof(uint32_t)))) uint32_t u32x2;

// ---------------------------------------------------------------------------
// Host-side error state (thread-local message, set before returning non-zero).
void set_error(const char *fmt, ...);
int fail(int code, const char *fmt, ...);

#define WKV_CHECK_ARG(cond, ...)                      \
  do {                                                \
    if (!(cond)) return ::wkv::fail(WKV_ERR_INVALID, __VA_ARGS__); \
  } while (0)

#define WKV_CHECK_LAUNCH(what)                                                        \
  do {                                                                                \
    hipError_t e_ = hipGetLastError();                                                \
    if (e_ != hipSuccess)                                                             \
      return ::wkv::fail(WKV_ERR_LAUNCH, "%s: %s", what, hipGetErrorString(e_));     \
  } while (0)

inline bool aligned16(const void *p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

// Validates the parts of a cache descriptor every entry point relies on.
// want_dtype: a wkv_kv_dtype_t the entry point requires, or -1 for either.
int check_cache(const wkv_cache_t *c, int want_dtype);
int check_mla_cache(const wkv_mla_cache_t *c);

// ---------------------------------------------------------------------------
// bf16 <-> fp32 (bit level, RNE, NaN kept quiet) — matches torch's conversion.
__device__ __forceinline__ float bf16_bits_to_f32(uint32_t b) { return __uint_as_float(b << 16); }

__device__ __forceinline__ uint32_t f32_to_bf16_bits(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return (u >> 16) | 0x40u;
  return (u + 0x7fffu + ((u >> 16) & 1u)) >> 16;
}

// ---------------------------------------------------------------------------
// fp8 e4m3fn (OCP) encode, bit-identical to torch's fp32 -> float8_e4m3fn
// cast: RNE, no saturation (a value rounding above 448 becomes 0x7F | sign),
// NaN -> 0x7F | sign.
__device__ __forceinline__ uint32_t e4m3_encode(float x) {
  uint32_t bits = __float_as_uint(x);
  uint32_t sign = (bits >> 24) & 0x80u;
  uint32_t a = bits & 0x7fffffffu;
  if (a >= 0x43f00000u) return 0x7fu | sign;  // >= 480, inf, NaN
  if (a < 0x3c800000u) {                      // < 2^-6: multiples of 2^-9
    float q = rintf(__uint_as_float(a) * 512.0f);
    return static_cast<uint32_t>(q) | sign;
  }
  uint32_t e = (a >> 23) - 127u + 7u;  // biased e4m3 exponent, 1..15
  uint32_t mant = a & 0x7fffffu;
  uint32_t r = mant >> 20;
  uint32_t rem = mant & 0xfffffu;
  r += (rem > 0x80000u) || (rem == 0x80000u && (r & 1u));
  uint32_t code = (e << 3) + r;
  if (code > 0x7eu) code = 0x7fu;
  return code | sign;
}

__device__ __forceinline__ float e4m3_decode(uint32_t c) {
  uint32_t e = (c >> 3) & 0xfu, m = c & 7u;
  float mag;
  if (e == 0)
    mag = static_cast<float>(m) * 0.001953125f;  // 2^-9
  else if (e == 15 && m == 7)
    mag = __uint_as_float(0x7fc00000u);
  else
    mag = __uint_as_float(((e + 120u) << 23) | (m << 20));
  return (c & 0x80u) ? -mag : mag;
}

// Smallest power of two >= max(amax, 1e-10) / 448 (fp32 division), amax
// clamped to FLT_MAX first; the exponent is read from the bits, no log2.
__device__ __forceinline__ float pow2_scale(float amax) {
  float a = fminf(fmaxf(amax, 1e-10f), 3.402823466e38f);
  float r = a / 448.0f;
  uint32_t u = __float_as_uint(r);
  uint32_t e = u >> 23;            // r is normal: >= 2^-42
  if ((u & 0x7fffffu) != 0) e += 1;  // not a power of two: round the exponent up
  return __uint_as_float(e << 23);
}

// fp32 -> e4m3 after clamping to +-448 (NaN passes through to the NaN code).
__device__ __forceinline__ uint32_t e4m3_quantize(float x, float scale) {
  float v = x / scale;  // scale is a power of two: the quotient is exact
  v = (v != v) ? v : fminf(fmaxf(v, -448.0f), 448.0f);
  return e4m3_encode(v);
}

// ---------------------------------------------------------------------------
// Attention arithmetic shared by the decode kernels.

// 2^x on the hardware exp unit (v_exp_f32). Every argument these kernels pass
// is <= 0 (a score minus a reference maximum), where the only difference from
// exp2f is that results below 2^-126 flush to 0.
__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

// Two fp32 -> packed bf16 (RNE, NaN stays NaN) with the hardware conversion
// (v_cvt_pk_bf16_f32).
__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
  typedef __attribute__((__vector_size__(2 * sizeof(__bf16)))) __bf16 bf16x2_t;
  typedef __attribute__((__vector_size__(2 * sizeof(float)))) float f32x2_t;
  return __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2_t{lo, hi}), bf16x2_t));
}

// Maximum over the four 16-lane rows of a wave (lanes c, c + 16, c + 32,
// c + 48), with the cross-row swaps of gfx950 (no LDS round trip).
__device__ __forceinline__ float row_max4(float v) {
  const auto r32 = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  v = fmaxf(__uint_as_float(r32[0]), __uint_as_float(r32[1]));
  const auto r16 = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return fmaxf(__uint_as_float(r16[0]), __uint_as_float(r16[1]));
}

// Online softmax keeps a reference maximum per query head and rescales the
// running sum and output only when a tile's maximum exceeds it by more than
// 2^SOFTMAX_TAU: probabilities are exp2(s - ref) <= 2^SOFTMAX_TAU (well inside
// bf16's range, at its full precision), and a rescale -- a pass over every
// accumulator -- becomes rare.
constexpr float SOFTMAX_TAU = 8.f;

// ---------------------------------------------------------------------------
// Wavefront helpers (wave64).

// The value lane (lane ^ O) holds, for O a power of two below 64, with no
// address register (a ds_bpermute needs one per distance, which the compiler
// keeps live across a kernel): the cross-row swaps of gfx950 for 32 and 16
// (each returns {vdst, src} after the swap: the lane's own row in one, the
// partner row in the other), a DPP row rotate by 8 (within 16 lanes that is
// the xor), the LDS swizzle's bitmask mode for 4 and DPP quad permutes for 2
// and 1.
template <int O>
__device__ __forceinline__ uint32_t lane_xor(uint32_t x) {
  static_assert(O >= 1 && O <= 32 && (O & (O - 1)) == 0, "lane_xor: a power of two below 64");
  if constexpr (O == 32) {
    const auto r = __builtin_amdgcn_permlane32_swap(x, x, false, false);
    return (__lane_id() & 32) ? r[0] : r[1];
  } else if constexpr (O == 16) {
    const auto r = __builtin_amdgcn_permlane16_swap(x, x, false, false);
    return (__lane_id() & 16) ? r[0] : r[1];
  } else if constexpr (O == 8) {
    return static_cast<uint32_t>(__builtin_amdgcn_update_dpp(0, static_cast<int>(x), 0x128, 0xF, 0xF, false));
  } else if constexpr (O == 4) {
    return static_cast<uint32_t>(__builtin_amdgcn_ds_swizzle(static_cast<int>(x), (4 << 10) | 0x1F));
  } else if constexpr (O == 2) {
    return static_cast<uint32_t>(__builtin_amdgcn_update_dpp(0, static_cast<int>(x), 0x4E, 0xF, 0xF, false));
  } else {
    return static_cast<uint32_t>(__builtin_amdgcn_update_dpp(0, static_cast<int>(x), 0xB1, 0xF, 0xF, false));
  }
}

template <int O>
__device__ __forceinline__ float lane_xor(float x) {
  return __uint_as_float(lane_xor<O>(__float_as_uint(x)));
}

template <int O>
__device__ __forceinline__ int lane_xor(int x) {
  return static_cast<int>(lane_xor<O>(static_cast<uint32_t>(x)));
}

template <int O>
__device__ __forceinline__ unsigned long long lane_xor(unsigned long long x) {
  const uint32_t lo = lane_xor<O>(static_cast<uint32_t>(x)), hi = lane_xor<O>(static_cast<uint32_t>(x >> 32));
  return (static_cast<unsigned long long>(hi) << 32) | lo;
}

template <int O>
__device__ __forceinline__ int64_t lane_xor(int64_t x) {
  return static_cast<int64_t>(lane_xor<O>(static_cast<unsigned long long>(x)));
}

// f folded over the xor butterfly 32, 16, ..., 1: every lane ends with the
// same result, combined in the same order as a __shfl_xor loop.
template <class T, class F>
__device__ __forceinline__ T wave_reduce(T v, F f) {
  v = f(v, lane_xor<32>(v));
  v = f(v, lane_xor<16>(v));
  v = f(v, lane_xor<8>(v));
  v = f(v, lane_xor<4>(v));
  v = f(v, lane_xor<2>(v));
  return f(v, lane_xor<1>(v));
}

__device__ __forceinline__ float wave_max(float v) {
  return wave_reduce(v, [](float a, float b) { return fmaxf(a, b); });
}

__device__ __forceinline__ float wave_sum(float v) {
  return wave_reduce(v, [](float a, float b) { return a + b; });
}

}  // namespace wkv
