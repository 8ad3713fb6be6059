// Weight-absorbed MLA paged decode for gfx950.
//
// Every query head reads the same latent entry c = [c_kv (R=512) | k_pe (64)],
// so a workgroup owns one (sequence, partition) for ALL heads and stages each
// 16-token latent tile once in LDS (HBM reads it exactly once). Its NW = H/16
// waves split the work two ways per tile:
//
//   QK  wave w: S^T[16 tok, heads 16w..16w+15] = C[16 tok, 576] . Q^T
//       (18 x mfma_f32_16x16x32_bf16, Q^T held in registers); online softmax
//       for its 16 heads; P^T (bf16) and the rescale factors go to LDS.
//   PV  wave w: O^T[d in its R/NW slice, all H heads] += C^T[d, 16 tok] . P^T
//       (mfma_f32_16x16x16_bf16; each wave reads only its d-slice of the tile
//       transposed out of LDS, and all of P^T).
//
// Two barriers per tile; partitions are merged by the log-sum-exp kernel.
#include <cmath>

#include "wkv_common.h"

namespace wkv {

typedef __attribute__((__vector_size__(4 * sizeof(short)))) short shortx4_m;

template <int D>
__global__ __launch_bounds__(D) void mla_merge_kernel(const float *__restrict__ part_o,
                                                      const float *__restrict__ part_ml, uint16_t *__restrict__ out,
                                                      const int32_t *__restrict__ seq_lens, int max_seq, int H,
                                                      int P_tok, int max_parts) {
  const int h = blockIdx.x, b = blockIdx.y, d = threadIdx.x;
  int L = seq_lens[b];
  L = L < max_seq ? L : max_seq;
  const int nparts = L > 0 ? (L + P_tok - 1) / P_tok : 0;
  if (nparts <= 1) return;
  const int64_t row0 = (static_cast<int64_t>(b) * H + h) * max_parts;
  float M = -INFINITY;
  for (int p = 0; p < nparts; ++p) M = fmaxf(M, part_ml[2 * (row0 + p)]);
  const float m_use = (M == -INFINITY) ? 0.f : M;
  float num = 0.f, den = 0.f;
  for (int p = 0; p < nparts; ++p) {
    const float w = exp2f(part_ml[2 * (row0 + p)] - m_use);
    den += w * part_ml[2 * (row0 + p) + 1];
    num += w * part_o[(row0 + p) * D + d];
  }
  out[(static_cast<int64_t>(b) * H + h) * D + d] = static_cast<uint16_t>(f32_to_bf16_bits(den > 0.f ? num / den : 0.f));
}

template <int NW>
struct MlaSmem {
  static constexpr int R = 512, W = 576, WP = W + 8;  // padded row (1168 B) spreads rows over banks
  static constexpr int H = 16 * NW;
  uint16_t tile[2][16][WP];
  uint16_t pt[H][16];  // P^T as [head][token], bf16
  float corr[H];
  float lsum[H];
};

template <int NW>
__global__ __launch_bounds__(64 * NW) void decode_mla_kernel(
    const uint16_t *__restrict__ lat, const uint16_t *__restrict__ qn, int64_t qn_sb, int64_t qn_sh,
    const uint16_t *__restrict__ qp, int64_t qp_sb, int64_t qp_sh, uint16_t *__restrict__ out,
    float *__restrict__ part_o, float *__restrict__ part_ml, const int32_t *__restrict__ bt, int64_t bt_stride,
    int max_seq, const int32_t *__restrict__ seq_lens, int BS, int64_t NB, float scale_log2, int P_tok,
    int max_parts) {
  using S = MlaSmem<NW>;
  constexpr int R = S::R, W = S::W, H = S::H;
  constexpr int DW = R / NW;        // PV d-slice per wave
  constexpr int NDT = DW / 16;      // d tiles per wave
  constexpr int NHT = NW;           // head tiles (16 heads each)
  constexpr int NCH = 16 * W / 8;   // 16-byte chunks per tile
  constexpr int TPB = 64 * NW;
  constexpr int CPT = (NCH + TPB - 1) / TPB;  // chunks per thread
  __shared__ S sm;

  const int part = blockIdx.x, b = blockIdx.y;
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, col = lane & 15, grp = lane >> 4;
  int L = seq_lens[b];
  L = L < max_seq ? L : max_seq;
  const int nparts = L > 0 ? (L + P_tok - 1) / P_tok : 0;
  if (nparts == 0) {
    if (part == 0) {
      for (int e = tid; e < H * R / 8; e += TPB)
        reinterpret_cast<u32x4 *>(out + static_cast<int64_t>(b) * H * R)[e] = u32x4{0u, 0u, 0u, 0u};
    }
    return;
  }
  if (part >= nparts) return;
  const int t_begin = part * P_tok;
  const int t_end = (t_begin + P_tok) < L ? (t_begin + P_tok) : L;
  const int32_t *btrow = bt + b * bt_stride;

  // Q^T operand for this wave's 16 heads.
  const int qh = 16 * wave + col;
  bf16x8 qop[W / 32];
#pragma unroll
  for (int j = 0; j < W / 32; ++j) {
    const uint16_t *src = (j < R / 32) ? qn + b * qn_sb + qh * qn_sh + 32 * j + 8 * grp
                                       : qp + b * qp_sb + qh * qp_sh + 32 * (j - R / 32) + 8 * grp;
    qop[j] = __builtin_bit_cast(bf16x8, *reinterpret_cast<const u32x4 *>(src));
  }

  floatx4 acc[NDT][NHT];
#pragma unroll
  for (int a = 0; a < NDT; ++a)
#pragma unroll
    for (int c = 0; c < NHT; ++c) acc[a][c] = floatx4{0.f, 0.f, 0.f, 0.f};
  float m_run = -INFINITY, l_run = 0.f;

  u32x4 stage[CPT];
  auto fetch = [&](int ts, int &valid) {
    int64_t blk = btrow[ts / BS];
    valid = (t_end - ts) < 16 ? (t_end - ts) : 16;
    if (blk < 0 || blk >= NB) {
      blk = 0;
      valid = 0;
    }
    const uint16_t *base = lat + (blk * BS + ts % BS) * W;
#pragma unroll
    for (int k = 0; k < CPT; ++k) {
      const int c = tid + k * TPB;
      if (c < NCH) stage[k] = *reinterpret_cast<const u32x4 *>(base + c * 8);
    }
  };
  auto commit = [&](int buf) {
#pragma unroll
    for (int k = 0; k < CPT; ++k) {
      const int c = tid + k * TPB;
      if (c < NCH) {
        const int tok = c / (W / 8), ch = c % (W / 8);
        *reinterpret_cast<u32x4 *>(&sm.tile[buf][tok][ch * 8]) = stage[k];
      }
    }
  };

  int valid_cur = 0, valid_next = 0;
  fetch(t_begin, valid_cur);
  commit(0);
  __syncthreads();
  int buf = 0;
  for (int ts = t_begin; ts < t_end; ts += 16) {
    const bool more = ts + 16 < t_end;
    if (more) fetch(ts + 16, valid_next);

    // ---- QK for this wave's 16 heads.
    floatx4 s = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int j = 0; j < W / 32; ++j) {
      const bf16x8 a = __builtin_bit_cast(bf16x8, *reinterpret_cast<const u32x4 *>(&sm.tile[buf][col][32 * j + 8 * grp]));
      s = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, qop[j], s, 0, 0, 0);
    }
    float sv[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) sv[i] = (4 * grp + i < valid_cur) ? s[i] * scale_log2 : -INFINITY;
    float mt = fmaxf(fmaxf(sv[0], sv[1]), fmaxf(sv[2], sv[3]));
    mt = fmaxf(mt, __shfl_xor(mt, 16, 64));
    mt = fmaxf(mt, __shfl_xor(mt, 32, 64));
    const float m_new = fmaxf(m_run, mt);
    const float m_use = (m_new == -INFINITY) ? 0.f : m_new;
    const float corr = exp2f(m_run - m_use);
    float p[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) p[i] = exp2f(sv[i] - m_use);
    l_run = l_run * corr + ((p[0] + p[1]) + (p[2] + p[3]));
    m_run = m_new;
    u32x2 pb;
    pb[0] = f32_to_bf16_bits(p[0]) | (f32_to_bf16_bits(p[1]) << 16);
    pb[1] = f32_to_bf16_bits(p[2]) | (f32_to_bf16_bits(p[3]) << 16);
    *reinterpret_cast<u32x2 *>(&sm.pt[qh][4 * grp]) = pb;
    if (grp == 0) sm.corr[qh] = corr;
    __syncthreads();

    // ---- PV for this wave's d-slice, all heads.
    shortx4_m vop[NDT];
#pragma unroll
    for (int a = 0; a < NDT; ++a) {
      const int d = wave * DW + 16 * a + col;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int tok = 4 * grp + e;
        vop[a][e] = (tok < valid_cur) ? static_cast<short>(sm.tile[buf][tok][d]) : static_cast<short>(0);
      }
    }
#pragma unroll
    for (int c = 0; c < NHT; ++c) {
      const shortx4_m pop = __builtin_bit_cast(shortx4_m, *reinterpret_cast<const u32x2 *>(&sm.pt[16 * c + col][4 * grp]));
      const float cr = sm.corr[16 * c + col];
#pragma unroll
      for (int a = 0; a < NDT; ++a) {
#pragma unroll
        for (int i = 0; i < 4; ++i) acc[a][c][i] *= cr;
        acc[a][c] = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(vop[a], pop, acc[a][c], 0, 0, 0);
      }
    }
    if (more) commit(buf ^ 1);
    __syncthreads();
    buf ^= 1;
    valid_cur = valid_next;
  }

  // ---- epilogue: per-head denominators through LDS.
  float l = l_run + __shfl_xor(l_run, 16, 64);
  l += __shfl_xor(l, 32, 64);
  if (grp == 0) {
    sm.lsum[qh] = l;
    sm.corr[qh] = m_run;  // reuse: running max per head
  }
  __syncthreads();
#pragma unroll
  for (int c = 0; c < NHT; ++c) {
    const int h = 16 * c + col;
    const float lh = sm.lsum[h];
#pragma unroll
    for (int a = 0; a < NDT; ++a) {
      const int d0 = wave * DW + 16 * a + 4 * grp;
      if (nparts == 1) {
        const float inv = lh > 0.f ? 1.f / lh : 0.f;
        u32x2 w;
        w[0] = f32_to_bf16_bits(acc[a][c][0] * inv) | (f32_to_bf16_bits(acc[a][c][1] * inv) << 16);
        w[1] = f32_to_bf16_bits(acc[a][c][2] * inv) | (f32_to_bf16_bits(acc[a][c][3] * inv) << 16);
        *reinterpret_cast<u32x2 *>(out + (static_cast<int64_t>(b) * H + h) * R + d0) = w;
      } else {
        const int64_t row = (static_cast<int64_t>(b) * H + h) * max_parts + part;
        *reinterpret_cast<floatx4 *>(part_o + row * R + d0) = acc[a][c];
      }
    }
    if (nparts > 1 && wave == 0 && grp == 0) {
      const int64_t row = (static_cast<int64_t>(b) * H + h) * max_parts + part;
      part_ml[2 * row] = sm.corr[h];
      part_ml[2 * row + 1] = lh;
    }
  }
}

static int choose_mla_partition(int batch, int max_seq_len) {
  // One workgroup per CU holds all heads; aim for >= 256 workgroups.
  int parts = batch > 0 ? (256 + batch - 1) / batch : 1;
  int p = (max_seq_len + parts - 1) / (parts > 0 ? parts : 1);
  p = (p + 63) / 64 * 64;
  return p < 64 ? 64 : p;
}

}  // namespace wkv

using namespace wkv;

extern "C" int64_t wkv_mla_workspace_size(int32_t batch, int32_t num_heads, int32_t kv_lora_rank,
                                          int32_t max_seq_len, int32_t partition_size) {
  if (batch < 0 || num_heads <= 0 || kv_lora_rank <= 0 || max_seq_len < 0 || partition_size < 0) return -1;
  if (partition_size == 0) partition_size = choose_mla_partition(batch, max_seq_len);
  const int64_t max_parts = (static_cast<int64_t>(max_seq_len) + partition_size - 1) / partition_size;
  return static_cast<int64_t>(batch) * num_heads * (max_parts > 0 ? max_parts : 1) * (kv_lora_rank + 2) * 4;
}

extern "C" int wkv_paged_decode_mla(const wkv_mla_cache_t *cache, const void *q_nope, int64_t qn_stride_b,
                                    int64_t qn_stride_h, const void *q_pe, int64_t qp_stride_b, int64_t qp_stride_h,
                                    void *out, int32_t num_heads, const int32_t *block_table, int64_t bt_stride,
                                    int32_t max_blocks_per_seq, const int32_t *seq_lens, int32_t batch,
                                    int32_t max_seq_len, float scale, int32_t partition_size, void *workspace,
                                    int64_t workspace_bytes, void *stream) {
  WKV_CHECK_ARG(cache != nullptr && cache->latent != nullptr && aligned16(cache->latent), "bad MLA cache");
  WKV_CHECK_ARG(cache->num_blocks > 0 && cache->block_size > 0 && cache->block_size % 16 == 0 &&
                    cache->block_size <= 256,
                "MLA block_size must be a multiple of 16 in [16, 256]");
  if (cache->kv_lora_rank != 512 || cache->rope_dim != 64)
    return fail(WKV_ERR_UNSUPPORTED, "MLA decode supports kv_lora_rank 512 + rope_dim 64 (got %d + %d)",
                cache->kv_lora_rank, cache->rope_dim);
  if (num_heads != 16 && num_heads != 32 && num_heads != 64 && num_heads != 128)
    return fail(WKV_ERR_UNSUPPORTED, "MLA decode supports 16, 32, 64 or 128 heads (got %d)", num_heads);
  WKV_CHECK_ARG(batch >= 0 && batch <= 65535, "batch must be in [0, 65535]");
  if (batch == 0) return WKV_OK;
  WKV_CHECK_ARG(q_nope && q_pe && aligned16(q_nope) && aligned16(q_pe), "q_nope/q_pe must be non-NULL, 16-byte aligned");
  WKV_CHECK_ARG(qn_stride_b >= 0 && qn_stride_h >= 0 && qp_stride_b >= 0 && qp_stride_h >= 0 &&
                    (qn_stride_b | qn_stride_h | qp_stride_b | qp_stride_h) % 8 == 0,
                "q strides must be non-negative multiples of 8");
  WKV_CHECK_ARG(out != nullptr && aligned16(out), "out must be non-NULL and 16-byte aligned");
  WKV_CHECK_ARG(block_table != nullptr && seq_lens != nullptr, "block_table / seq_lens is NULL");
  WKV_CHECK_ARG(max_blocks_per_seq > 0 && bt_stride >= max_blocks_per_seq, "bad block table geometry");
  WKV_CHECK_ARG(max_seq_len >= 0 && std::isfinite(scale), "bad max_seq_len or scale");
  const int BS = cache->block_size;
  if (partition_size == 0) partition_size = choose_mla_partition(batch, max_seq_len);
  WKV_CHECK_ARG(partition_size >= 16 && partition_size % 16 == 0, "partition_size must be a positive multiple of 16");
  const int max_seq = max_seq_len < max_blocks_per_seq * BS ? max_seq_len : max_blocks_per_seq * BS;
  const int max_parts = max_seq > 0 ? (max_seq + partition_size - 1) / partition_size : 1;
  WKV_CHECK_ARG(max_parts <= 65535, "too many partitions");
  const int64_t need = wkv_mla_workspace_size(batch, num_heads, 512, max_seq, partition_size);
  if (max_parts > 1)
    WKV_CHECK_ARG(workspace != nullptr && aligned16(workspace) && workspace_bytes >= need,
                  "workspace too small: need %lld bytes, got %lld", (long long)need, (long long)workspace_bytes);
  float *part_o = static_cast<float *>(workspace);
  float *part_ml = part_o ? part_o + static_cast<int64_t>(batch) * num_heads * max_parts * 512 : nullptr;
  const float scale_log2 = scale * 1.4426950408889634f;
  auto s = static_cast<hipStream_t>(stream);
  const dim3 grid(static_cast<unsigned>(max_parts), static_cast<unsigned>(batch));
  auto lat = static_cast<const uint16_t *>(cache->latent);
  auto qn = static_cast<const uint16_t *>(q_nope);
  auto qpp = static_cast<const uint16_t *>(q_pe);
  auto oo = static_cast<uint16_t *>(out);
#define WKV_MLA(NWv)                                                                                        \
  decode_mla_kernel<NWv><<<grid, 64 * NWv, 0, s>>>(lat, qn, qn_stride_b, qn_stride_h, qpp, qp_stride_b,   \
                                                   qp_stride_h, oo, part_o, part_ml, block_table, bt_stride, \
                                                   max_seq, seq_lens, BS, cache->num_blocks, scale_log2,   \
                                                   partition_size, max_parts)
  switch (num_heads) {
    case 16: WKV_MLA(1); break;
    case 32: WKV_MLA(2); break;
    case 64: WKV_MLA(4); break;
    default: WKV_MLA(8); break;
  }
#undef WKV_MLA
  WKV_CHECK_LAUNCH("wkv_paged_decode_mla");
  if (max_parts > 1) {
    mla_merge_kernel<512><<<dim3(static_cast<unsigned>(num_heads), static_cast<unsigned>(batch)), 512, 0, s>>>(
        part_o, part_ml, oo, seq_lens, max_seq, num_heads, partition_size, max_parts);
    WKV_CHECK_LAUNCH("wkv_paged_decode_mla merge");
  }
  return WKV_OK;
}
