// GQA prefill / chunked-prefill attention over the paged cache (gfx950).
//
// Sequence b brings qlen_b = cu_seqlens_q[b+1] - cu_seqlens_q[b] new tokens
// at positions [L_b - qlen_b, L_b) (L_b = seq_lens[b]: cached context plus the
// new tokens, which the entry point appends to the cache first). New token j
// attends causally to positions [0, L_b - qlen_b + j] -- the bottom-right
// aligned mask of a varlen prefill over a paged context (a prefix-cache hit or
// an earlier chunk).
//
// Work decomposition: workgroup (16-token query tile, KV head x head group,
// sequence) of four waves; wave w takes query head kvh*G + 4*hg + w, so the
// MFMA columns are 16 consecutive query tokens of one head and the four waves
// of a workgroup stream the same key tiles (one HBM read, three cache hits).
// Keys are streamed in 16-token tiles by the decode kernels' tile loop
// (gqa_tiles.h), in ranges of 64 blocks; tiles on the causal diagonal mask per
// lane (column). Every wave finishes its rows: no split-K, no workspace.
#include "gqa_tiles.h"

namespace wkv {

constexpr int kPrefillWaves = 4;

template <int D, bool FP8>
__global__ __launch_bounds__(64 * kPrefillWaves) void prefill_gqa_kernel(
    const uint8_t *__restrict__ kc, const uint8_t *__restrict__ vc, const float *__restrict__ ks,
    const float *__restrict__ vs, const uint16_t *__restrict__ q, int64_t q_st, int64_t q_sh,
    uint16_t *__restrict__ out, int64_t o_st, int64_t o_sh, const int32_t *__restrict__ cu_q,
    const int32_t *__restrict__ seq_lens, const int32_t *__restrict__ bt, int64_t bt_stride, int Mb, int max_seq,
    int Hkv, int G, int n_hg, int BS, int64_t NB, float scale_log2) {
  const int qt = blockIdx.x, b = blockIdx.z;
  const int kvh = __builtin_amdgcn_readfirstlane(static_cast<int>(blockIdx.y) / n_hg);
  const int hg = static_cast<int>(blockIdx.y) - kvh * n_hg;
  const int wave = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x >> 6));
  const int lane = threadIdx.x & 63, col = lane & 15, grp = lane >> 4;
  const int q0 = cu_q[b];
  const int qlen = cu_q[b + 1] - q0;
  int L = seq_lens[b];
  L = L < max_seq ? L : max_seq;
  const int t0 = qt * 16;
  const int h_local = hg * kPrefillWaves + wave;
  if (t0 >= qlen || h_local >= G) return;  // no barrier in this kernel: waves leave independently
  const int h = kvh * G + h_local;
  const int ctx = L - qlen;  // position of new token 0 (negative only for inconsistent inputs)
  const int tok = t0 + col;
  const bool valid = tok < qlen;
  const int pos = ctx + tok;  // this column's position; it sees keys [0, pos]

  bf16x8 qop[D / 32];
  load_q<D, FP8>(qop, q + static_cast<int64_t>(q0 + (valid ? tok : t0)) * q_st + static_cast<int64_t>(h) * q_sh,
                 valid, grp);
  DecodeState<D, FP8> st;
#pragma unroll
  for (int n = 0; n < D / 16; ++n) st.o[n] = floatx4{0.f, 0.f, 0.f, 0.f};
  st.m = -INFINITY;
  st.l = 0.f;

  // Keys up to the tile's last query: [0, kend).
  const int last = (t0 + 16 < qlen ? t0 + 16 : qlen) - 1;
  const int kend = ctx + last + 1;
  const int span = 64 * BS;  // one attend_range: at most 64 blocks (one lane each)
  for (int r0 = 0; r0 < kend; r0 += span) {
    const int r1 = (r0 + span) < kend ? (r0 + span) : kend;
    const int blk_first = r0 / BS;
    int my_blk = -1;
    if (blk_first + lane < Mb) my_blk = bt[b * bt_stride + blk_first + lane];
    attend_range<D, FP8>(
        [&](Tile<D, FP8> &t) {
          int lim = pos - t.ts + 1;  // keys of the tile this column sees
          lim = lim < 0 ? 0 : (lim > 16 ? 16 : lim);
          attend_tile<D, FP8, true>(st, t, qop, scale_log2, grp, lim);
        },
        kc, vc, ks, vs, my_blk, r0, r1, kvh, Hkv, BS, NB, lane, col, grp);
  }
  float l = st.l + __shfl_xor(st.l, 16, 64);
  l += __shfl_xor(l, 32, 64);
  if (!valid) return;
  const float inv = l > 0.f ? 1.f / l : 0.f;
  uint16_t *op = out + static_cast<int64_t>(q0 + tok) * o_st + static_cast<int64_t>(h) * o_sh;
#pragma unroll
  for (int n = 0; n < D / 16; ++n) {
    u32x2 w;
    w[0] = f32_to_bf16_bits(st.o[n][0] * inv) | (f32_to_bf16_bits(st.o[n][1] * inv) << 16);
    w[1] = f32_to_bf16_bits(st.o[n][2] * inv) | (f32_to_bf16_bits(st.o[n][3] * inv) << 16);
    *reinterpret_cast<u32x2 *>(op + 16 * n + 4 * grp) = w;
  }
}

}  // namespace wkv

using namespace wkv;

extern "C" int wkv_prefill_gqa(const wkv_cache_t *cache, const void *key, int64_t key_stride_t, int64_t key_stride_h,
                               const void *value, int64_t value_stride_t, int64_t value_stride_h,
                               const int64_t *slot_mapping, int64_t num_tokens, const void *q, int64_t q_stride_t,
                               int64_t q_stride_h, void *out, int64_t out_stride_t, int64_t out_stride_h,
                               int32_t num_q_heads, const int32_t *cu_seqlens_q, const int32_t *seq_lens,
                               const int32_t *block_table, int64_t bt_stride, int32_t max_blocks_per_seq,
                               int32_t batch, int32_t max_query_len, int32_t max_seq_len, float scale, void *stream) {
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
  const int n_hg = (G + kPrefillWaves - 1) / kPrefillWaves;
  const int64_t gy = static_cast<int64_t>(Hkv) * n_hg;
  WKV_CHECK_ARG(gy <= 65535, "num_q_heads too large");
  const dim3 grid(static_cast<unsigned>((max_query_len + 15) / 16), static_cast<unsigned>(gy),
                  static_cast<unsigned>(batch));
  auto s = static_cast<hipStream_t>(stream);
  auto kc = static_cast<const uint8_t *>(cache->k);
  auto vc = static_cast<const uint8_t *>(cache->v);
  auto qq = static_cast<const uint16_t *>(q);
  auto oo = static_cast<uint16_t *>(out);
  const float scale_log2 = scale * 1.4426950408889634f;
  const bool fp8 = cache->kv_dtype == WKV_KV_FP8_E4M3;
#define WKV_PREFILL(Dv, F8)                                                                                       \
  prefill_gqa_kernel<Dv, F8><<<grid, 64 * kPrefillWaves, 0, s>>>(                                                \
      kc, vc, cache->k_scale, cache->v_scale, qq, q_stride_t, q_stride_h, oo, out_stride_t, out_stride_h,       \
      cu_seqlens_q, seq_lens, block_table, bt_stride, max_blocks_per_seq, max_seq, Hkv, G, n_hg, BS,           \
      cache->num_blocks, scale_log2)
  if (D == 128) {
    if (fp8) WKV_PREFILL(128, true); else WKV_PREFILL(128, false);
  } else {
    if (fp8) WKV_PREFILL(64, true); else WKV_PREFILL(64, false);
  }
#undef WKV_PREFILL
  WKV_CHECK_LAUNCH("paged prefill");
  return WKV_OK;
}
