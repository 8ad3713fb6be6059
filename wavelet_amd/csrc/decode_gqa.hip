// GQA paged decode attention for gfx950.
//
// One wavefront owns one (sequence, KV head, partition) work item and streams
// the partition's tokens in 16-token tiles straight from HBM into MFMA operand
// registers (gqa_tiles.h); the MFMA columns are the G <= 16 query heads of
// the KV head, padded to 16. Long contexts are split into partitions whose
// partial results are merged in LDS by the waves of a workgroup and, past one
// workgroup, by a second small kernel (log-sum-exp). (Merging across
// workgroups inside the main kernel needs device-scope release/acquire between
// waves of different XCDs; measured here, that costs far more than the extra
// launch.) The decode-step append can be fused in: the wave that owns a
// sequence's last partition first writes the new token into the cache, then
// attends over it.
#include <atomic>
#include <cmath>

#include "gqa_tiles.h"
#include "kv_append_dev.h"

namespace wkv {

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

// Weight of query head hq's attention sink in a softmax denominator whose
// terms are 2^(s - m_use) (log2 domain): the sink is an extra logit with a
// zero value vector (wavelet/trainer/models/deepseek_v4/attention.py:89-95),
// given in natural-log units like the scaled scores. No sinks: 0.
__device__ __forceinline__ float sink_weight(const float *sinks, int hq, float m_use) {
  return sinks != nullptr ? exp2f(sinks[hq] * 1.4426950408889634f - m_use) : 0.f;
}

// Grid: (chunk, KV head, sequence or dispatch rank); W waves per workgroup, wave w of chunk c
// owns partition c*W + w of P_tok tokens. The waves of a workgroup merge
// their partials through LDS; a context longer than one chunk leaves one
// partial per chunk for merge_partials_kernel.
// RP, the read policy of the K/V tiles -- a compile-time choice, as a per-tile
// one costs the tile pipeline its schedule:
//   kReadCached:   the default policy (blocks that several sequences read);
//   kReadStreamed: non-temporal loads (blocks read once);
//   kReadSplit:    GRPO groups of group_size consecutive sequences: the first
//     prefix_lens[b / group_size] tokens of sequence b -- the group's prompt,
//     whose blocks every member reads -- keep the default policy, so the
//     members' reads of one prompt block meet in the caches, and the member's
//     own tokens are streamed. The cut is a multiple of 16 tokens from the
//     partition start, so the tiles, and the result, are the plain call's.
constexpr int kReadCached = 0, kReadStreamed = 1, kReadSplit = 2;

// fp8: held to 128 VGPRs (four waves per SIMD, as before the fused append's
// tile patch, which took the grouped instances to 130 and three waves).
template <int D, bool FP8, bool APPEND, int W, int RP>
__global__ __launch_bounds__(64 * W) __attribute__((amdgpu_waves_per_eu(FP8 ? 4 : 1))) void decode_gqa_kernel(
    uint8_t *__restrict__ kc, uint8_t *__restrict__ vc, float *__restrict__ ks, float *__restrict__ vs,
    const uint16_t *__restrict__ q, int64_t q_sb, int64_t q_sh, uint16_t *__restrict__ out,
    float *__restrict__ part_o, float *__restrict__ part_ml, const int32_t *__restrict__ bt, int64_t bt_stride,
    int Mb, int max_seq, const int32_t *__restrict__ seq_lens, const int32_t *__restrict__ order, int Hq, int Hkv,
    int G, int BS, int64_t NB, float scale_log2, int P_tok, int max_chunks, StepAppend ap,
    const float *__restrict__ sinks, const int32_t *__restrict__ prefix_lens, int group_size, int max_prefix) {
  const int chunk = blockIdx.x, kvh = blockIdx.y;
  // The wave index is uniform across the wave; saying so keeps everything
  // derived from it (partition, block ids, buffer resources) in scalar registers.
  const int wave = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x >> 6));
  const int lane = threadIdx.x & 63, col = lane & 15, grp = lane >> 4;
  const int part = chunk * W + wave;
  int t_begin = part * P_tok;
  int blk_first = t_begin / BS;

  // Sequence: blockIdx.z, or the z-th entry of a dispatch order (longest
  // contexts first: the short ones then fill the gaps the long ones leave).
  // The loads of sequence blockIdx.z go out while the order entry is read
  // and are redone only when the entry names another sequence.
  int b = blockIdx.z;
  const int b_ord = order != nullptr ? order[b] : b;
  // Loads that do not depend on the context length go out together with it:
  // the block ids of a full-size partition (bounded by the block-table width) and q.
  int L = seq_lens[b];
  int my_blk = -1;
  if (blk_first + lane < Mb) my_blk = bt[b * bt_stride + blk_first + lane];
  // Q^T operand: lane holds 8 d-values of head `col` (zero for padded heads).
  bf16x8 qop[D / 32];
  load_q<D, FP8>(qop, q + b * q_sb + static_cast<int64_t>(kvh * G + (col < G ? col : 0)) * q_sh, col < G, grp);
  if (b_ord != b) {
    if (b_ord < 0 || b_ord >= static_cast<int>(gridDim.z)) return;  // not an entry of a permutation of the batch
    b = b_ord;
    L = seq_lens[b];
    my_blk = -1;
    if (blk_first + lane < Mb) my_blk = bt[b * bt_stride + blk_first + lane];
    load_q<D, FP8>(qop, q + b * q_sb + static_cast<int64_t>(kvh * G + (col < G ? col : 0)) * q_sh, col < G, grp);
  }

  // fp8 fused append: the step token's slot and K/V rows go out now, with the
  // loads above (every wave: which one appends is known only from the
  // length); the appending wave's chain then starts at the old scales.
  int64_t slot_pre = -1;
  Fp8TokenRows<D> rows_pre;
  if constexpr (APPEND && FP8) {
    slot_pre = ap.slots[b];
    fp8_token_rows_load<D>(rows_pre, ap.key + b * ap.kst + kvh * ap.ksh, ap.val + b * ap.vst + kvh * ap.vsh);
  }

  // The group's shared prompt: tokens [0, cut), read with the default policy.
  int cut = 0;
  if constexpr (RP == kReadSplit) {
    cut = prefix_lens[b / group_size];
    cut = cut < max_prefix ? cut : max_prefix;
  }
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
  // fp8: when the slot is the table's position L - 1 and the block's scales
  //      do not grow, the token's codes and the block's scales enter the tile
  //      that holds it in registers, exactly as a read of the cache after
  //      the append would bring them (so the output is the unfused call's),
  //      and the codes (and a new block's scales) are written after the
  //      tiles: stores count in the wave's in-order vmcnt, so written first
  //      they held up every tile load behind them (measured per fp8 Qwen3-4B
  //      layer: 92.9 -> 88.8 us). Otherwise (a scale grows and re-encodes the
  //      block, or the slot lies elsewhere) append first and wait before the
  //      block is read.
  // bf16: the wave attends the cache up to the new token and then the token
  //      itself from the step's inputs (held one dword per lane), writing it
  //      to the cache at the end; nothing waits on the write or the slot.
  uint32_t nk = 0, nv = 0;
  int64_t slot = -1;
  __shared__ uint8_t tok_code[(APPEND && FP8) ? W : 1][2][D];  // the fp8 token's K and V codes, per wave
  int patch_ts = -1, patch_p = 0;  // the tile holding the fp8 token, its row in the tile
  float psk = 1.f, psv = 1.f;      // the block's scales after the append
  bool late = false;               // the fp8 token's writes wait for the end
  if constexpr (APPEND) {
    if (owns_new) {
      if constexpr (FP8) {
        slot = slot_pre;
        if (slot >= 0 && slot / BS < NB) {
          const int64_t blk = slot / BS;
          const int off = static_cast<int>(slot % BS);
          const int tbl = __builtin_amdgcn_readlane(my_blk, (L - 1) / BS - blk_first);
          const Fp8TokenCodes<D> cd = fp8_token_codes<D>(ks, vs, rows_pre, blk, off, kvh, Hkv);
          if (tbl == blk && off == (L - 1) % BS && !cd.grow) {  // uniform
            late = true;
            psk = __int_as_float(__builtin_amdgcn_readfirstlane(__float_as_int(cd.sk)));  // uniform: scalar registers
            psv = __int_as_float(__builtin_amdgcn_readfirstlane(__float_as_int(cd.sv)));
#pragma unroll
            for (int i = 0; i < D / 64; ++i) {
              tok_code[wave][0][lane + 64 * i] = static_cast<uint8_t>(cd.k[i]);
              tok_code[wave][1][lane + 64 * i] = static_cast<uint8_t>(cd.v[i]);
            }
            patch_ts = t_begin + 16 * (((L - 1) - t_begin) >> 4);
            patch_p = (L - 1) - patch_ts;
          } else {
            fp8_append_token_kv<D>(kc, vc, ks, vs, rows_pre, blk, off, kvh, Hkv, BS);
            __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "workgroup");
          }
        }
      } else {
        slot = ap.slots[b];
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
    const int te = from_regs ? L - 1 : t_end;
    // Each tile, as loaded; the fp8 token's tile first takes the token's codes
    // (K: row patch_p of the tile, the lanes holding that token; V: byte
    // patch_p of every lane's d row) and the block's scales after the append.
    auto consume = [&](Tile<D, FP8> &t) __attribute__((always_inline)) {
      if constexpr (APPEND && FP8) {
        if (t.ts == patch_ts) {  // uniform; never for the other waves (-1)
          const uint32_t sh = 8u * static_cast<uint32_t>(patch_p & 3);
#pragma unroll
          for (int j = 0; j < Tile<D, FP8>::NK; ++j) {
            // dword by dword: one register of the tile loop's budget, not four
#pragma unroll
            for (int w = 0; w < 4; ++w) {
              const uint32_t kw = *reinterpret_cast<const uint32_t *>(&tok_code[wave][0][16 * (4 * j + grp) + 4 * w]);
              if (col == patch_p) t.k[j][w] = kw;
            }
            const uint32_t vq = tok_code[wave][1][lane + 64 * j];
#pragma unroll
            for (int w = 0; w < 4; ++w)
              if (w == (patch_p >> 2)) t.v4[j][w] = (t.v4[j][w] & ~(0xffu << sh)) | (vq << sh);
          }
          t.ksc = psk;
          t.vsc = psv;
        }
      }
      attend_tile<D, FP8>(st, t, qop, scale_log2, grp);
    };
    auto attend = [&](int mb, int t0, int t1, bool stream) __attribute__((always_inline)) {
      attend_range<D, FP8>(consume, kc, vc, ks, vs, mb, t0, t1, kvh, Hkv, BS, NB, lane, col, grp, stream);
    };
    if constexpr (RP == kReadSplit) {
      // [t_begin, c) of the shared prompt cached, [c, te) streamed; c - t_begin is
      // a multiple of 16, so both ranges hold the partition's own 16-token tiles.
      int c = cut - t_begin;
      c = t_begin + (c > 0 ? (c & ~15) : 0);
      if (c > t_begin) attend(my_blk, t_begin, te < c ? te : c, false);
      if (te > c) {
        // the streamed range's block ids, lane i = its i-th block
        const int sh = c / BS - blk_first;
        const int mb = sh > 0 ? __shfl(my_blk, (lane + sh) & 63, 64) : my_blk;
        attend(mb, c, te, true);
      }
    } else {
      attend(my_blk, t_begin, te, RP == kReadStreamed);
    }
    if constexpr (APPEND && FP8) {
      if (late) {  // the token's codes (staged by this wave above) and the block's scales
        const int64_t blk = slot / BS;
        const int off = static_cast<int>(slot % BS);
        if (col == 0) {
#pragma unroll
          for (int j = 0; j < Tile<D, FP8>::NK; ++j)
            *reinterpret_cast<u32x4 *>(kc + fp8_k_index<D>(blk, kvh, Hkv, BS, off, 16 * (4 * j + grp))) =
                *reinterpret_cast<const u32x4 *>(&tok_code[wave][0][16 * (4 * j + grp)]);
        }
#pragma unroll
        for (int i = 0; i < D / 64; ++i)
          vc[fp8_v_index<D>(blk, kvh, Hkv, BS, off, lane + 64 * i)] = tok_code[wave][1][lane + 64 * i];
        // A block's scales change only with its first token here (a growing
        // scale takes the append-first path): otherwise they are already stored.
        if (off == 0 && lane == 0) {
          ks[blk * Hkv + kvh] = psk;
          vs[blk * Hkv + kvh] = psv;
        }
      }
    }
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
      const float den = l + sink_weight(sinks, hq, st.m == -INFINITY ? 0.f : st.m);
      const float inv = den > 0.f ? 1.f / den : 0.f;
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
        den += sink_weight(sinks, hq, m_use);
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
                                                             Slots sl, const float *__restrict__ sinks) {
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
  den = wave_sum(den) + sink_weight(sinks, row % Hq, m_use);
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

// Tokens per partition when the caller leaves it to the library: about 2,048
// partition waves over the longest context -- every CU's resident slots in
// about one round, and no more (fewer, longer waves amortise the per-wave
// prologue and the partial-result traffic; measured, d=64 contexts of
// 256..2,048 tokens run 8% faster at 2,048 than at 4,096 waves) but at most
// an eighth of the longest context, at least 128 tokens, a multiple of the
// block size (the fused append relies on it), and at most 64 blocks (one
// lane each).
static int choose_partition(int batch, int hkv, int max_seq_len, int BS) {
  const int64_t target_waves = 2048;
  const int64_t items = static_cast<int64_t>(batch) * hkv;
  int64_t p = (items * max_seq_len + target_waves - 1) / target_waves;
  // An eighth of the longest context: every sequence gets eight waves, one
  // 8-wave workgroup while that fits (headline shape -1%, fp8 GRPO groups -3%
  // against the wave target alone).
  const int64_t eighth = (static_cast<int64_t>(max_seq_len) + 7) / 8;
  if (p > eighth) p = eighth;
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

// Waves per workgroup and chunks per sequence: partitions of one context
// share a workgroup (and an LDS merge) up to 8 at a time; longer contexts
// leave per-chunk partials. (8-wave workgroups for 8+ partitions: var-length
// Qwen3-4B -7%, Qwen2.5-0.5B -11% against 4.)
static void decode_shape(int max_seq, int partition_size, int *W, int *chunks) {
  const int max_parts = max_seq > 0 ? (max_seq + partition_size - 1) / partition_size : 1;
  *W = max_parts <= 1 ? 1 : (max_parts <= 2 ? 2 : (max_parts < 8 ? 4 : 8));
  *chunks = (max_parts + *W - 1) / *W;
}

}  // namespace wkv

using namespace wkv;

extern "C" int wkv_decode_plan(int32_t batch, int32_t num_kv_heads, int32_t max_seq_len, int32_t block_size,
                               int32_t partition_size, int32_t *out_partition, int32_t *out_waves,
                               int32_t *out_chunks) {
  WKV_CHECK_ARG(batch >= 0 && num_kv_heads > 0 && max_seq_len >= 0 && partition_size >= 0,
                "bad decode geometry");
  WKV_CHECK_ARG(block_size > 0 && block_size % 16 == 0, "block_size must be a positive multiple of 16");
  WKV_CHECK_ARG(out_partition && out_waves && out_chunks, "output pointer is NULL");
  const int p = partition_size != 0 ? partition_size : choose_partition(batch, num_kv_heads, max_seq_len, block_size);
  int W, chunks;
  decode_shape(max_seq_len, p, &W, &chunks);
  *out_partition = p;
  *out_waves = W;
  *out_chunks = chunks;
  return WKV_OK;
}

extern "C" int64_t wkv_decode_workspace_size(int32_t batch, int32_t num_q_heads, int32_t head_dim,
                                             int32_t max_seq_len, int32_t partition_size) {
  if (batch < 0 || num_q_heads <= 0 || head_dim <= 0 || max_seq_len < 0 || partition_size < 0) return -1;
  if (partition_size == 0) partition_size = 128;  // smallest partition the library picks by itself
  const int64_t max_parts = (static_cast<int64_t>(max_seq_len) + partition_size - 1) / partition_size;
  // partial outputs and (max, sum) per (sequence, query head, partition)
  return static_cast<int64_t>(batch) * num_q_heads * (max_parts > 0 ? max_parts : 1) * (head_dim + 2) * 4;
}

namespace wkv {

// Dispatch order for the decode kernels: the batch's sequence indices by
// context length, longest first, ties by index -- rank(i) = #{j : L_j > L_i,
// or L_j = L_i and j < i} is a permutation. O(batch^2) compares: a workgroup
// ranks 64 sequences, its four waves counting over a quarter of the batch
// each (scalar loads of L_j, every lane comparing with its own L_i), summed
// through LDS; 256 sequences take 5 us (8 with the classes below), 64 take 4 us,
// once per step.
// With n_cls > 1 (GRPO groups of group_size consecutive sequences; every class
// holds batch / n_cls sequences), group g belongs to class g % n_cls, each
// class is ranked longest first on its own, and rank r of class c is
// dispatched at position r * n_cls + c: every member of a group then lands at
// the same position modulo n_cls, which is what places a group's workgroups of
// one KV head on one XCD (see grouped_order_classes).
template <bool CLASSES>
__global__ __launch_bounds__(256) void decode_order_kernel(const int32_t *__restrict__ seq_lens, int batch,
                                                           int32_t *__restrict__ order, int group_size, int n_cls) {
  __shared__ int part_rank[4][64];
  const int lane = threadIdx.x & 63;
  const int part = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x >> 6));
  const int i = blockIdx.x * 64 + lane;
  const int ki = i < batch ? seq_lens[i] : 0;
  const int span = (batch + 3) / 4;
  const int j0 = part * span;
  const int j1 = j0 + span < batch ? j0 + span : batch;
  int rank = 0;
  if constexpr (!CLASSES) {
#pragma unroll 8
    for (int j = j0; j < j1; ++j) {
      const int kj = seq_lens[j];
      rank += (kj > ki || (kj == ki && j < i)) ? 1 : 0;
    }
  } else {
    const int ci = (i / group_size) % n_cls;
    // the class of sequence j is tracked incrementally (no division per step)
    int cj = (j0 / group_size) % n_cls, in_group = j0 % group_size;
#pragma unroll 8
    for (int j = j0; j < j1; ++j) {
      const int kj = seq_lens[j];
      rank += (cj == ci && (kj > ki || (kj == ki && j < i))) ? 1 : 0;
      if (++in_group == group_size) {
        in_group = 0;
        cj = cj + 1 == n_cls ? 0 : cj + 1;
      }
    }
  }
  part_rank[part][lane] = rank;
  __syncthreads();
  if (part == 0 && i < batch) {
    rank = part_rank[0][lane] + part_rank[1][lane] + part_rank[2][lane] + part_rank[3][lane];
    if constexpr (CLASSES)
      order[rank * n_cls + (i / group_size) % n_cls] = i;
    else
      order[rank] = i;
  }
}

// Workgroups are dispatched to the XCDs round-robin by linear workgroup id, and
// each XCD has its own L2. A decode workgroup (chunk, KV head, rank) has linear
// id chunk + chunks * (kvh + Hkv * rank), so the workgroups of ranks congruent
// modulo 8 / gcd(8, chunks * Hkv) run on the same XCDs, head by head: the
// number of order classes that keep a group's reads of its prompt in one L2.
// 1 (plain longest-first order) when the classes would not be of equal size.
constexpr int kXcds = 8;

static int grouped_order_classes(int batch, int group_size, int hkv, int max_seq, int BS, int partition_size) {
  const int P = partition_size != 0 ? partition_size : choose_partition(batch, hkv, max_seq, BS);
  int W, chunks;
  decode_shape(max_seq, P, &W, &chunks);
  int a = chunks * hkv % kXcds, g = kXcds;  // gcd(kXcds, chunks * hkv)
  while (a != 0) {
    const int t = g % a;
    g = a;
    a = t;
  }
  const int n_cls = kXcds / g;
  return batch % (group_size * n_cls) == 0 ? n_cls : 1;
}

static int launch_decode(const wkv_cache_t *cache, const void *q, int64_t q_stride_b, int64_t q_stride_h, void *out,
                         int32_t num_q_heads, const int32_t *block_table, int64_t bt_stride,
                         int32_t max_blocks_per_seq, const int32_t *seq_lens, int32_t batch, int32_t max_seq_len,
                         float scale, int32_t partition_size, void *workspace, int64_t workspace_bytes,
                         const StepAppend *ap, const int32_t *seq_order, void *stream,
                         bool static_scratch = false, const float *sinks = nullptr,
                         const int32_t *prefix_lens = nullptr, int group_size = 1, int max_prefix = 0) {
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
  if (partition_size == 0) partition_size = choose_partition(batch, Hkv, max_seq, BS);
  WKV_CHECK_ARG(partition_size >= 16 && partition_size % 16 == 0, "partition_size must be a positive multiple of 16");
  WKV_CHECK_ARG((partition_size + BS - 17) / BS + 1 <= 64,
                "partition_size %d spans more than 64 blocks of %d tokens", partition_size, BS);
  if (ap != nullptr)
    WKV_CHECK_ARG(partition_size % BS == 0, "a fused append needs partition_size %d to be a multiple of block_size %d",
                  partition_size, BS);
  int W, max_chunks;
  decode_shape(max_seq, partition_size, &W, &max_chunks);
  WKV_CHECK_ARG(max_chunks <= 65535, "too many partitions");
  const int64_t need = wkv_decode_workspace_size(batch, num_q_heads, D, max_seq, partition_size * W);
  if (max_chunks > 1 && static_scratch)
    WKV_CHECK_ARG(workspace_bytes >= need,
                  "this geometry needs %lld bytes of split-K scratch; the allocation-free entry point's static "
                  "scratch holds %lld (WKV_NOALLOC_SCRATCH_BYTES): use wkv_append_paged_decode_gqa with a workspace",
                  (long long)need, (long long)workspace_bytes);
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
  // Groups: the shared prompt cached, each member's own tokens streamed (per sequence, in the kernel).
  const int rp = prefix_lens != nullptr ? kReadSplit
                                        : ((cache->flags & WKV_CACHE_SHARED_BLOCKS) == 0 ? kReadStreamed : kReadCached);
#define WKV_DECODE_S(Dv, F8, AP, Wv, ST)                                                                         \
  decode_gqa_kernel<Dv, F8, AP, Wv, ST><<<grid, 64 * Wv, 0, s>>>(kc, vc, cache->k_scale, cache->v_scale, qq,     \
                                                                 q_stride_b, q_stride_h, oo, part_o, part_ml,    \
                                                                 block_table, bt_stride, max_blocks_per_seq,     \
                                                                 max_seq, seq_lens, seq_order,                   \
                                                                 num_q_heads, Hkv, G, BS, cache->num_blocks,     \
                                                                 scale_log2, partition_size, max_chunks, apv,    \
                                                                 sinks, prefix_lens, group_size, max_prefix)
#define WKV_DECODE(Dv, F8, AP, Wv)                     \
  do {                                                 \
    if (rp == kReadStreamed)                           \
      WKV_DECODE_S(Dv, F8, AP, Wv, kReadStreamed);     \
    else if (rp == kReadCached)                        \
      WKV_DECODE_S(Dv, F8, AP, Wv, kReadCached);       \
    else                                               \
      WKV_DECODE_S(Dv, F8, AP, Wv, kReadSplit);        \
  } while (0)
#define WKV_DECODE_W(Dv, F8, AP)   \
  do {                             \
    if (W == 1)                    \
      WKV_DECODE(Dv, F8, AP, 1);   \
    else if (W == 2)               \
      WKV_DECODE(Dv, F8, AP, 2);   \
    else if (W == 4)               \
      WKV_DECODE(Dv, F8, AP, 4);   \
    else                           \
      WKV_DECODE(Dv, F8, AP, 8);   \
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
#undef WKV_DECODE_S
  WKV_CHECK_LAUNCH("paged decode");
  if (max_chunks > 1) {
    const int rows = batch * num_q_heads;
    const PlainSlots ps{seq_lens, max_seq, partition_size * W};
    if (D == 128)
      merge_partials_kernel<128>
          <<<(rows + 3) / 4, 256, 0, s>>>(part_o, part_ml, oo, rows, num_q_heads, max_chunks, ps, sinks);
    else
      merge_partials_kernel<64>
          <<<(rows + 3) / 4, 256, 0, s>>>(part_o, part_ml, oo, rows, num_q_heads, max_chunks, ps, sinks);
    WKV_CHECK_LAUNCH("paged decode merge");
  }
  return WKV_OK;
}

}  // namespace wkv

extern "C" int64_t wkv_grouped_decode_workspace_size(int32_t batch, int32_t num_q_heads, int32_t head_dim,
                                                     int32_t max_seq_len, int32_t max_prefix_len,
                                                     int32_t partition_size) {
  if (max_prefix_len < 0) return -1;
  return wkv_decode_workspace_size(batch, num_q_heads, head_dim, max_seq_len, partition_size);
}

extern "C" int wkv_paged_decode_gqa_grouped(const wkv_cache_t *cache, const void *key, int64_t key_stride_t,
                                            int64_t key_stride_h, const void *value, int64_t value_stride_t,
                                            int64_t value_stride_h, const int64_t *slot_mapping, const void *q,
                                            int64_t q_stride_b, int64_t q_stride_h, void *out, int32_t num_q_heads,
                                            const int32_t *block_table, int64_t bt_stride,
                                            int32_t max_blocks_per_seq, const int32_t *seq_lens, int32_t batch,
                                            int32_t max_seq_len, const int32_t *prefix_lens, int32_t group_size,
                                            int32_t max_prefix_len, float scale, int32_t partition_size,
                                            void *workspace, int64_t workspace_bytes, const int32_t *seq_order,
                                            void *stream) {
  using namespace wkv;
  WKV_CHECK_ARG(batch >= 0 && batch <= 65535, "batch must be in [0, 65535] (got %d)", batch);
  if (batch == 0) return WKV_OK;
  WKV_CHECK_ARG(prefix_lens != nullptr, "prefix_lens is NULL");
  WKV_CHECK_ARG(group_size >= 1 && group_size <= batch, "group_size must be in [1, batch] (got %d)", group_size);
  WKV_CHECK_ARG(max_prefix_len >= 0, "max_prefix_len must be >= 0");
  StepAppend ap{};
  const bool append = key != nullptr || value != nullptr || slot_mapping != nullptr;
  if (append) {
    WKV_CHECK_ARG(key && value && aligned16(key) && aligned16(value),
                  "key/value must be non-NULL and 16-byte aligned (or all of key, value, slot_mapping NULL)");
    WKV_CHECK_ARG(key_stride_t >= 0 && key_stride_h >= 0 && value_stride_t >= 0 && value_stride_h >= 0 &&
                      (key_stride_t | key_stride_h | value_stride_t | value_stride_h) % 8 == 0,
                  "key/value strides must be non-negative multiples of 8");
    WKV_CHECK_ARG(slot_mapping != nullptr, "slot_mapping is NULL");
    if (cache != nullptr && cache->kv_dtype == WKV_KV_FP8_E4M3)
      WKV_CHECK_ARG(cache->k_scale && cache->v_scale, "fp8 cache needs k_scale and v_scale");
    ap = StepAppend{static_cast<const uint16_t *>(key), key_stride_t, key_stride_h,
                    static_cast<const uint16_t *>(value), value_stride_t, value_stride_h, slot_mapping};
  }
  return launch_decode(cache, q, q_stride_b, q_stride_h, out, num_q_heads, block_table, bt_stride,
                       max_blocks_per_seq, seq_lens, batch, max_seq_len, scale, partition_size, workspace,
                       workspace_bytes, append ? &ap : nullptr, seq_order, stream, false, nullptr, prefix_lens,
                       group_size, max_prefix_len);
}

extern "C" int wkv_decode_order(const int32_t *seq_lens, int32_t batch, int32_t *order, void *stream) {
  WKV_CHECK_ARG(batch >= 0 && batch <= 65535, "batch must be in [0, 65535] (got %d)", batch);
  if (batch == 0) return WKV_OK;
  WKV_CHECK_ARG(seq_lens != nullptr && order != nullptr, "seq_lens / order is NULL");
  decode_order_kernel<false>
      <<<(batch + 63) / 64, 256, 0, static_cast<hipStream_t>(stream)>>>(seq_lens, batch, order, 1, 1);
  WKV_CHECK_LAUNCH("decode order");
  return WKV_OK;
}

extern "C" int wkv_grouped_decode_order(const int32_t *seq_lens, int32_t batch, int32_t group_size,
                                        int32_t num_kv_heads, int32_t max_seq_len, int32_t block_size,
                                        int32_t partition_size, int32_t *order, void *stream) {
  using namespace wkv;
  WKV_CHECK_ARG(batch >= 0 && batch <= 65535, "batch must be in [0, 65535] (got %d)", batch);
  if (batch == 0) return WKV_OK;
  WKV_CHECK_ARG(seq_lens != nullptr && order != nullptr, "seq_lens / order is NULL");
  WKV_CHECK_ARG(group_size >= 1 && group_size <= batch, "group_size must be in [1, batch] (got %d)", group_size);
  WKV_CHECK_ARG(num_kv_heads > 0 && max_seq_len >= 0 && partition_size >= 0, "bad decode geometry");
  WKV_CHECK_ARG(block_size > 0 && block_size % 16 == 0, "block_size must be a positive multiple of 16");
  const int n_cls = grouped_order_classes(batch, group_size, num_kv_heads, max_seq_len, block_size, partition_size);
  if (n_cls == 1)
    decode_order_kernel<false>
        <<<(batch + 63) / 64, 256, 0, static_cast<hipStream_t>(stream)>>>(seq_lens, batch, order, 1, 1);
  else
    decode_order_kernel<true><<<(batch + 63) / 64, 256, 0, static_cast<hipStream_t>(stream)>>>(
        seq_lens, batch, order, group_size, n_cls);
  WKV_CHECK_LAUNCH("grouped decode order");
  return WKV_OK;
}

extern "C" int wkv_paged_decode_gqa(const wkv_cache_t *cache, const void *q, int64_t q_stride_b,
                                    int64_t q_stride_h, void *out, int32_t num_q_heads,
                                    const int32_t *block_table, int64_t bt_stride, int32_t max_blocks_per_seq,
                                    const int32_t *seq_lens, int32_t batch, int32_t max_seq_len, float scale,
                                    int32_t partition_size, void *workspace, int64_t workspace_bytes,
                                    const int32_t *seq_order, void *stream) {
  return launch_decode(cache, q, q_stride_b, q_stride_h, out, num_q_heads, block_table, bt_stride,
                       max_blocks_per_seq, seq_lens, batch, max_seq_len, scale, partition_size, workspace,
                       workspace_bytes, nullptr, seq_order, stream);
}

extern "C" int wkv_paged_decode_gqa_sinks(const wkv_cache_t *cache, const void *q, int64_t q_stride_b,
                                          int64_t q_stride_h, void *out, int32_t num_q_heads,
                                          const int32_t *block_table, int64_t bt_stride, int32_t max_blocks_per_seq,
                                          const int32_t *seq_lens, int32_t batch, int32_t max_seq_len, float scale,
                                          int32_t partition_size, void *workspace, int64_t workspace_bytes,
                                          const int32_t *seq_order, const float *sinks, void *stream) {
  WKV_CHECK_ARG(sinks != nullptr && reinterpret_cast<uintptr_t>(sinks) % 4 == 0, "sinks must be non-NULL fp32");
  return launch_decode(cache, q, q_stride_b, q_stride_h, out, num_q_heads, block_table, bt_stride,
                       max_blocks_per_seq, seq_lens, batch, max_seq_len, scale, partition_size, workspace,
                       workspace_bytes, nullptr, seq_order, stream, false, sinks);
}

extern "C" int wkv_append_paged_decode_gqa(const wkv_cache_t *cache, const void *key, int64_t key_stride_t,
                                           int64_t key_stride_h, const void *value, int64_t value_stride_t,
                                           int64_t value_stride_h, const int64_t *slot_mapping, const void *q,
                                           int64_t q_stride_b, int64_t q_stride_h, void *out, int32_t num_q_heads,
                                           const int32_t *block_table, int64_t bt_stride,
                                           int32_t max_blocks_per_seq, const int32_t *seq_lens, int32_t batch,
                                           int32_t max_seq_len, float scale, int32_t partition_size,
                                           void *workspace, int64_t workspace_bytes, const int32_t *seq_order,
                                           void *stream) {
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
                       workspace_bytes, &ap, seq_order, stream);
}

extern "C" int wkv_append_paged_decode_gqa_sinks(const wkv_cache_t *cache, const void *key, int64_t key_stride_t,
                                                 int64_t key_stride_h, const void *value, int64_t value_stride_t,
                                                 int64_t value_stride_h, const int64_t *slot_mapping, const void *q,
                                                 int64_t q_stride_b, int64_t q_stride_h, void *out,
                                                 int32_t num_q_heads, const int32_t *block_table, int64_t bt_stride,
                                                 int32_t max_blocks_per_seq, const int32_t *seq_lens, int32_t batch,
                                                 int32_t max_seq_len, float scale, int32_t partition_size,
                                                 void *workspace, int64_t workspace_bytes, const int32_t *seq_order,
                                                 const float *sinks, void *stream) {
  WKV_CHECK_ARG(sinks != nullptr && reinterpret_cast<uintptr_t>(sinks) % 4 == 0, "sinks must be non-NULL fp32");
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
                       workspace_bytes, &ap, seq_order, stream, false, sinks);
}

// ---------------------------------------------------------------------------
// Allocation-free fused decode: the split-K partials go to a file-scope device
// array instead of a caller workspace. Every GPU the library runs on holds its
// own copy (WKV_NOALLOC_SCRATCH_BYTES) until the process ends. Its address is
// looked up once per device, with that device current, and kept per device;
// host code passes that address, never the array's name (in host code the
// name is only a stand-in for the symbol). Nothing in the scratch has to start
// at zero: the merge reads only partials that the same call's decode kernel
// wrote. Calls that overlap on one GPU share the array and race.
static __device__ __align__(256) uint8_t scratch[WKV_NOALLOC_SCRATCH_BYTES];

namespace wkv {

constexpr int kMaxDevices = 64;
static std::atomic<void *> g_scratch_ptr[kMaxDevices];

// The scratch address on the calling thread's current device.
static int noalloc_scratch(void **ptr) {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return fail(WKV_ERR_LAUNCH, "hipGetDevice: %s", hipGetErrorString(e));
  if (dev < 0 || dev >= kMaxDevices) return fail(WKV_ERR_UNSUPPORTED, "device %d: at most %d devices", dev, kMaxDevices);
  void *p = g_scratch_ptr[dev].load(std::memory_order_acquire);
  if (p == nullptr) {
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || p == nullptr)
      return fail(WKV_ERR_LAUNCH, "hipGetSymbolAddress(scratch) on device %d: %s", dev, hipGetErrorString(e));
    g_scratch_ptr[dev].store(p, std::memory_order_release);
  }
  *ptr = p;
  return WKV_OK;
}

}  // namespace wkv

extern "C" int wkv_append_paged_decode_gqa_noalloc(const wkv_cache_t *cache, const void *key, int64_t key_stride_t,
                                                   int64_t key_stride_h, const void *value, int64_t value_stride_t,
                                                   int64_t value_stride_h, const int64_t *slot_mapping,
                                                   const void *q, int64_t q_stride_b, int64_t q_stride_h, void *out,
                                                   int32_t num_q_heads, const int32_t *block_table,
                                                   int64_t bt_stride, int32_t max_blocks_per_seq,
                                                   const int32_t *seq_lens, int32_t batch, int32_t max_seq_len,
                                                   float scale, int32_t partition_size, const int32_t *seq_order,
                                                   void *stream) {
  WKV_CHECK_ARG(key && value && aligned16(key) && aligned16(value), "key/value must be non-NULL and 16-byte aligned");
  WKV_CHECK_ARG(key_stride_t >= 0 && key_stride_h >= 0 && value_stride_t >= 0 && value_stride_h >= 0 &&
                    (key_stride_t | key_stride_h | value_stride_t | value_stride_h) % 8 == 0,
                "key/value strides must be non-negative multiples of 8");
  WKV_CHECK_ARG(slot_mapping != nullptr, "slot_mapping is NULL");
  if (cache != nullptr && cache->kv_dtype == WKV_KV_FP8_E4M3)
    WKV_CHECK_ARG(cache->k_scale && cache->v_scale, "fp8 cache needs k_scale and v_scale");
  void *ws = nullptr;
  const int rc = noalloc_scratch(&ws);
  if (rc) return rc;
  const StepAppend ap{static_cast<const uint16_t *>(key), key_stride_t, key_stride_h,
                      static_cast<const uint16_t *>(value), value_stride_t, value_stride_h, slot_mapping};
  return launch_decode(cache, q, q_stride_b, q_stride_h, out, num_q_heads, block_table, bt_stride,
                       max_blocks_per_seq, seq_lens, batch, max_seq_len, scale, partition_size, ws,
                       WKV_NOALLOC_SCRATCH_BYTES, &ap, seq_order, stream, true);
}
