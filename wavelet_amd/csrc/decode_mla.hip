// Weight-absorbed MLA paged decode for gfx950.
//
// Every query head reads the same latent row c = [c_kv (512) | k_pe (64)]
// (1152 bytes per token), so one workgroup owns one (sequence, partition) for
// ALL heads and HBM delivers each latent byte once.
//
// Memory pipeline. The partition is streamed in 32-token steps (36 KB). Each
// step is copied HBM -> LDS by global_load_lds_dwordx4 (lane i of a wave
// instruction lands at LDS base + 16 i), with no register staging, into one
// of four LDS buffers: the copy waves keep two steps in flight while the QK
// and PV waves compute on the other two. A copy wave waits only for its own
// copies of the step about to be used (s_waitcnt vmcnt(n)) and a barrier
// publishes everyone's. The copies and their waits are inline asm, so the
// compiler's own wait insertion never drains the copies in flight.
//
// LDS layout of a step: row t (token), 72 chunks of 16 bytes; chunk c of row
// t sits at slot c ^ swz(t), so the QK reads (16 rows, same chunk) run
// without bank conflicts.
//
// Per step (the wave roles are described at the kernel):
//   QK  S^T[32 tok, 16 heads of w] = C[32 tok, 576] . Q^T   (mfma_f32_16x16x32_bf16,
//       A = latent rows from LDS, B = Q^T resident in registers)
//       online softmax per head; P^T (bf16) and the rescale factors -> LDS.
//   PV  O^T[d-slice of w, all heads] += C^T[d, 32 tok] . P^T
//       (mfma_f32_16x16x32_bf16; A = ds_read_b64_tr_b16 of the same LDS rows:
//       lane l receives element l%4 of what lane 16(l/16) + 4k + (l%16)/4
//       loaded, i.e. 4 tokens of one d per read; B = P^T from LDS).
// The 8 tokens a lane contributes per PV MFMA are tokens {4g..4g+3} and
// {16+4g..16+4g+3} of the step (g = lane/16) -- exactly the 8 scores that
// lane holds after QK, so P is written to LDS in the same lane order it is
// read back.
// Partitions of one sequence are merged by the log-sum-exp kernel.
#include <cmath>

#include "lds_dma.h"
#include "wkv_common.h"

namespace wkv {
namespace mla {

constexpr int R = 512;           // kv_lora_rank
constexpr int PE = 64;           // rope dim
constexpr int W = R + PE;        // latent row, elements
constexpr int ROWB = W * 2;      // 1152 bytes per token
constexpr int CH = ROWB / 16;    // 72 chunks of 16 bytes per row
constexpr int STEP = 32;         // tokens per pipeline step
constexpr int STEPB = STEP * ROWB;  // 36,864 bytes per step buffer
constexpr int NDMA = STEPB / 1024;  // 36 wave-instructions (64 lanes x 16 B) per step
constexpr int HALF = 16 * ROWB;     // byte offset of tokens 16..31 within a step

// Chunk slot XOR of row t. A 16-byte LDS read is served 8 lanes per cycle
// (128 bytes), and a row (1152 = 9 x 128 bytes) starts on the same bank for
// every t, so the 8 rows an 8-lane group of the QK read touches (8 tokens, one
// chunk) must sit in 8 distinct 16-byte slots: slot = chunk ^ (t mod 8)
// (measured: as fast as a linear read; the transposed PV reads are unaffected).
__device__ __forceinline__ int swz(int t) { return t & 7; }

// Where the tokens of one step come from. A step covers tokens [ts, ts + 32)
// of the sequence, in at most two blocks: tokens [0, n_lo) of the step in
// the lo block, the rest in the hi block. A token is attended when it is in
// [0, lo_end) or [n_lo, hi_end) (inside the partition, block id in range);
// every other token copies the row of token `safe` (an attended token of the
// step), so the transposed PV reads only ever see finite, attended data. With
// no attended token at all the step is skipped.
struct StepSrc {
  const uint8_t *base_lo;  // + t * ROWB = row of lo-block token t
  const uint8_t *base_hi;  // + t * ROWB = row of hi-block token t (t >= n_lo)
  int n_lo, lo_end, hi_end, safe;
  bool any;   // some token attended
  bool full;  // all 32 tokens attended (no masking needed)
};

// Position of a step's first token: block index within the partition's
// block list and offset inside that block. Advanced 32 tokens at a time
// without a division (the block size is a runtime value; integer division by
// it would run on the vector unit): 32 tokens cross at most two block
// boundaries when the block size is a multiple of 16.
struct StepPos {
  int bi, off;
};

__device__ __forceinline__ void advance(StepPos &p, int BS) {
  p.off += STEP;
  if (p.off >= BS) {
    p.off -= BS;
    ++p.bi;
  }
  if (p.off >= BS) {
    p.off -= BS;
    ++p.bi;
  }
}

__device__ __forceinline__ StepSrc step_src(const uint16_t *lat, StepPos pos, int ts, int t_end, int BS, int my_blk,
                                            int NB) {
  // All uniform; readfirstlane keeps them (and what is derived) scalar even
  // where the compiler placed a loop-carried copy in a vector register.
  StepSrc s;
  const int valid = __builtin_amdgcn_readfirstlane((t_end - ts) < STEP ? (t_end - ts) : STEP);
  const int off = __builtin_amdgcn_readfirstlane(pos.off);
  s.n_lo = (BS - off) < STEP ? (BS - off) : STEP;
  const int bi = __builtin_amdgcn_readfirstlane(pos.bi);
  const int blo = __builtin_amdgcn_readlane(my_blk, bi);
  const int bhi = __builtin_amdgcn_readlane(my_blk, (bi + 1) & 63);
  const bool lo_ok = blo >= 0 && blo < NB;
  const bool hi_ok = bhi >= 0 && bhi < NB;
  s.lo_end = lo_ok ? (valid < s.n_lo ? valid : s.n_lo) : 0;
  s.hi_end = (hi_ok && valid > s.n_lo) ? valid : s.n_lo;
  s.safe = s.hi_end > s.n_lo ? s.hi_end - 1 : (s.lo_end > 0 ? s.lo_end - 1 : 0);
  s.any = s.lo_end > 0 || s.hi_end > s.n_lo;
  s.full = s.lo_end == s.n_lo && s.hi_end == STEP;
  const uint8_t *lat8 = reinterpret_cast<const uint8_t *>(lat);
  s.base_lo = lat8 + (static_cast<int64_t>(lo_ok ? blo : 0) * BS + off) * ROWB;
  s.base_hi = lat8 + (static_cast<int64_t>(hi_ok ? bhi : 0) * BS - s.n_lo) * ROWB;
  return s;
}

__device__ __forceinline__ bool token_ok(const StepSrc &s, int t) {
  return static_cast<bool>(static_cast<int>(t < s.lo_end) | (static_cast<int>(t >= s.n_lo) & static_cast<int>(t < s.hi_end)));
}



}  // namespace mla

// Profiling builds only (-DWKV_PHASE_CLOCKS, wavelet_amd.build --phase-clocks):
// every workgroup below kPhaseWgs sums the shader-clock cycles (s_memtime) of
// its step phases per role into 16 slots of g_mla_phase, read back with
// wkv_mla_phase_clocks (include/wkv_profile.h):
//   0 cycles, 1 wall ticks (100 MHz), 2 steps, 12 / 13 wall start / end;
//   copy waves: 3 barrier, 4 issue, 5 wait, 7 prologue;
//   PV waves:   8 barrier, 9 operand reads before the first MFMA, 10 MFMAs, 6 prologue;
//   QK waves:   11 barrier, 14 MFMAs (with their operand reads), 15 softmax.
// s_memtime is a scalar-memory read; waiting for it also waits for the wave's
// LDS reads in flight, so the stamps shift work across phase borders slightly.
constexpr int kPhaseWgs = 1024;
#ifdef WKV_PHASE_CLOCKS
__device__ unsigned long long g_mla_phase[kPhaseWgs * 16];
#define WKV_PHASE_INIT                                                                                 \
  const unsigned long long ph_t0 = __builtin_amdgcn_s_memtime(), ph_r0 = __builtin_amdgcn_s_memrealtime(); \
  unsigned long long ph_tp = ph_t0, ph_c[4] = {0, 0, 0, 0};
#define WKV_PHASE(i)                                         \
  {                                                          \
    const unsigned long long t_ = __builtin_amdgcn_s_memtime(); \
    ph_c[i] += t_ - ph_tp;                                   \
    ph_tp = t_;                                              \
  }
#define WKV_PHASE_STORE(s0, s1, s2, s3)                                            \
  if (lane == 0 && role_w == 0 && blockIdx.x < kPhaseWgs) {                        \
    unsigned long long *r_ = g_mla_phase + 16 * blockIdx.x;                        \
    const int sl_[4] = {s0, s1, s2, s3};                                           \
    for (int i_ = 0; i_ < 4; ++i_)                                                 \
      if (sl_[i_] >= 0) r_[sl_[i_]] = ph_c[i_];                                    \
  }
#define WKV_PHASE_TOTAL(n)                                                                             \
  if (lane == 0 && role_w == 0 && blockIdx.x < kPhaseWgs) {                                            \
    unsigned long long *r_ = g_mla_phase + 16 * blockIdx.x;                                            \
    const unsigned long long r1_ = __builtin_amdgcn_s_memrealtime();                                   \
    r_[0] = __builtin_amdgcn_s_memtime() - ph_t0;                                                      \
    r_[1] = r1_ - ph_r0;                                                                               \
    r_[2] = static_cast<unsigned long long>(n);                                                        \
    r_[12] = ph_r0;                                                                                    \
    r_[13] = r1_;                                                                                      \
  }
#else
#define WKV_PHASE_INIT
#define WKV_PHASE(i)
#define WKV_PHASE_STORE(s0, s1, s2, s3)
#define WKV_PHASE_TOTAL(n)
#endif

// The appended token of a fused append + decode step: row b of kv_c / k_pe
// belongs to sequence b (its position seq_lens[b] - 1) and goes to slot
// slots[b] (-1 = none). kvc == nullptr: attention only.
struct MlaAppend {
  const uint16_t *kvc;
  int64_t kvc_st;
  const uint16_t *kpe;
  int64_t kpe_st;
  const int64_t *slots;
};

// Weight of head h's attention sink in a denominator whose terms are
// 2^(s - m_use) (log2 domain): one more logit, natural-log units like the
// scaled scores, with a zero value vector
// (wavelet/trainer/models/deepseek_v4/attention.py:89-95). No sinks: 0.
__device__ __forceinline__ float mla_sink_weight(const float *sinks, int h, float m_use) {
  return sinks != nullptr ? exp2f(sinks[h] * 1.4426950408889634f - m_use) : 0.f;
}

// Log-sum-exp merge of the per-partition partials of one (sequence, head):
// 128 lanes per head, four output elements (one 8-byte partial load per
// partition) per lane, two heads per 256-thread workgroup. A partial is the
// partition's normalised output o_p (bf16) with its maximum m_p and sum l_p:
// out = sum_p 2^(m_p - M) l_p o_p / (sum_p 2^(m_p - M) l_p + sink weight).
__global__ __launch_bounds__(256) void mla_merge_kernel(const uint16_t *__restrict__ part_o,
                                                        const float *__restrict__ part_ml, uint16_t *__restrict__ out,
                                                        const int32_t *__restrict__ seq_lens, int max_seq, int H,
                                                        int P_tok, int max_parts, const float *__restrict__ sinks) {
  constexpr int R = mla::R;
  const int h = 2 * blockIdx.x + (threadIdx.x >> 7), b = blockIdx.y, d = 4 * (threadIdx.x & 127);
  if (h >= H) return;
  int L = seq_lens[b];
  L = L < max_seq ? L : max_seq;
  const int nparts = L > 0 ? (L + P_tok - 1) / P_tok : 0;
  if (nparts <= 1) return;
  const int64_t row0 = (static_cast<int64_t>(b) * H + h) * max_parts;
  float M = -INFINITY;
  for (int p = 0; p < nparts; ++p) M = fmaxf(M, part_ml[2 * (row0 + p)]);
  const float m_use = (M == -INFINITY) ? 0.f : M;
  floatx4 num = {0.f, 0.f, 0.f, 0.f};
  float den = 0.f;
  for (int p = 0; p < nparts; ++p) {
    const float wl = exp2f(part_ml[2 * (row0 + p)] - m_use) * part_ml[2 * (row0 + p) + 1];
    den += wl;
    const u32x2 o = *reinterpret_cast<const u32x2 *>(part_o + (row0 + p) * R + d);
#pragma unroll
    for (int i = 0; i < 4; ++i) num[i] += wl * __uint_as_float((o[i >> 1] >> (16 * (i & 1))) << 16);
  }
  den += mla_sink_weight(sinks, h, m_use);
  const float inv = den > 0.f ? 1.f / den : 0.f;
  u32x2 v;
  v[0] = f32_to_bf16_bits(num[0] * inv) | (f32_to_bf16_bits(num[1] * inv) << 16);
  v[1] = f32_to_bf16_bits(num[2] * inv) | (f32_to_bf16_bits(num[3] * inv) << 16);
  *reinterpret_cast<u32x2 *>(out + (static_cast<int64_t>(b) * H + h) * R + d) = v;
}

// A workgroup owns HW = 16 NQ of the H = HW * HG heads of one (sequence,
// partition) and runs 3 NQ waves in three roles, one of each per SIMD:
//   QK waves (w < NQ):  Q^T of heads 16 w .. 16 w + 15 in registers; compute
//       S for step s + 1, the online softmax, and write P^T and the rescale
//       factors of that step to LDS.
//   PV waves (NQ <= w < 2 NQ): the output accumulators of d-slice (w - NQ)
//       for all HW heads; rescale and accumulate O for step s.
//   copy waves (w >= 2 NQ): issue the LDS copies of step s + 3 and wait for
//       those of step s + 2.
// One barrier per step hands step s + 1's probabilities from the QK waves to
// the PV waves, which consume them one step later -- so on every SIMD the QK
// wave's softmax and bookkeeping overlap the PV wave's MFMAs and the two
// waves' MFMAs interleave. An LDS-DMA copy stalls the wave that issues it
// until the memory pipeline takes it (about 1,250 cycles per 36 KB step at
// full load, measured), so the copies have waves of their own, which hold
// no accumulators and stall without holding back an MFMA. Four 36 KB step
// buffers: the PV waves read step s, the QK waves step s + 1, and steps
// s + 2 and s + 3 are in flight.
//
// The 1-D grid is laid out for the dispatcher, which deals workgroup i to XCD
// i mod 8: work item k goes to XCD k mod 8, and its HG head groups are
// workgroups 8 HG (k / 8) + 8 g + (k mod 8), i.e. on the same XCD and
// dispatched back to back, so the second read of each latent tile is served
// by that XCD's L2. With a batch that is a multiple of 8 (seq_xcd), item k is
// (sequence k mod 8 + 8 (k / 8 / P), partition k / 8 mod P) for P partitions
// per sequence: every partition of a sequence sits on one XCD, so its q rows
// are fetched from memory once rather than once per partition (measured:
// 156 instead of 171 MB read per DeepSeek-V3 layer, same time); otherwise
// item k is (sequence k / P, partition k mod P), which spreads the
// partitions of a small batch over every XCD.
template <int NQ>
__global__ __launch_bounds__(192 * NQ, 1) void decode_mla_kernel(
    uint16_t *__restrict__ lat, const uint16_t *__restrict__ qn, int64_t qn_sb, int64_t qn_sh,
    const uint16_t *__restrict__ qp, int64_t qp_sb, int64_t qp_sh, uint16_t *__restrict__ out,
    uint16_t *__restrict__ part_o, float *__restrict__ part_ml, const int32_t *__restrict__ bt, int64_t bt_stride,
    int Mb, int max_seq, const int32_t *__restrict__ seq_lens, int BS, int64_t NB, float scale_log2, int P_tok,
    int max_parts, int H, int batch, MlaAppend ap, int seq_xcd, const float *__restrict__ sinks) {
  using namespace mla;
  constexpr int NHB = NQ;           // 16-head blocks of this workgroup
  constexpr int HW = 16 * NHB;      // heads of this workgroup
  constexpr int DSL = R / NQ;       // PV d-slice per PV wave
  constexpr int NDT = DSL / 16;     // PV d-tiles per PV wave
  constexpr int NIW = NDMA / NQ;    // copies every PV wave issues per step
  constexpr int NBUF = 4;
  static_assert(NDMA % NQ == 0 && DSL % 64 == 0, "copy split / d-slice");

  __shared__ __attribute__((aligned(16))) uint8_t buf[NBUF][STEPB];
  __shared__ __attribute__((aligned(16))) uint8_t pt[2][NHB * 1024];  // P^T per step parity, [hb][g][col][8 bf16]
  __shared__ __attribute__((aligned(16))) float corr_s[2][HW];        // rescale factors per step parity, [col][hb]
  __shared__ float lsum_s[HW];
  __shared__ float mrun_s[HW];

  // The decode divides by runtime values, which the compiler does on the
  // vector unit; readfirstlane returns the (uniform) results to scalar
  // registers so everything derived from them stays scalar.
  WKV_PHASE_INIT
  const int NBi = static_cast<int>(NB);  // the host bounds num_blocks to int32
  const int HG = H / HW;
  const int wg_r = __builtin_amdgcn_readfirstlane(static_cast<int>(blockIdx.x % (8 * HG)));
  const int item = __builtin_amdgcn_readfirstlane(static_cast<int>(8 * (blockIdx.x / (8 * HG)) + (wg_r & 7)));
  if (static_cast<int64_t>(item) >= static_cast<int64_t>(batch) * max_parts) return;  // padding of the last group of 8
  const int b = __builtin_amdgcn_readfirstlane(seq_xcd ? (item & 7) + 8 * ((item >> 3) / max_parts) : item / max_parts);
  const int part = __builtin_amdgcn_readfirstlane(seq_xcd ? (item >> 3) % max_parts : item % max_parts);
  const int hbase = HW * (wg_r >> 3);  // first head of this workgroup
  const int wave = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x >> 6));
  const int role = wave / NQ;          // 0: QK, 1: PV, 2: copies
  const int role_w = wave - NQ * role;  // QK: head block; PV: d-slice; copies: instruction set
  const int lane = threadIdx.x & 63, col = lane & 15, grp = lane >> 4;
  const int t_begin = part * P_tok;
  const int blk_first = __builtin_amdgcn_readfirstlane(t_begin / BS);
  const int off_first = t_begin - blk_first * BS;

  // Uniform across the workgroup: kept in scalar registers so that all the
  // per-step bookkeeping derived from it runs on the scalar unit.
  int L = __builtin_amdgcn_readfirstlane(seq_lens[b]);
  int my_blk = -1;  // lane i: id of the partition's i-th block
  if (blk_first + lane < Mb) my_blk = bt[b * bt_stride + blk_first + lane];
  // Pinned here so the compiler waits for the load now: its first use is in
  // the step loop, where that wait would also drain the copies in flight.
  asm volatile("" : "+v"(my_blk));
  L = L < max_seq ? L : max_seq;
  const int nparts = L > 0 ? (L + P_tok - 1) / P_tok : 0;
  if (nparts == 0) {
    if (part == 0) {
      for (int e = threadIdx.x; e < HW * R / 8; e += 192 * NQ)
        reinterpret_cast<u32x4 *>(out + (static_cast<int64_t>(b) * H + hbase) * R)[e] = u32x4{0u, 0u, 0u, 0u};
    }
    return;
  }
  if (part >= nparts) return;
  const int t_end = (t_begin + P_tok) < L ? (t_begin + P_tok) : L;
  const int nsteps = (t_end - t_begin + STEP - 1) / STEP;
  // Fused append: the partition holding position L - 1 attends the new token
  // from the inputs (its step s_new, row tn) and head group 0 writes it to
  // the cache; nothing in this launch reads that slot back.
  const bool fuse = ap.kvc != nullptr && part == nparts - 1;
  const int s_new = (L - 1 - t_begin) / STEP;
  const int tn = (L - 1 - t_begin) - STEP * s_new;

  // The three roles run separate loops with the same barrier sequence
  // (prologue, one per step, epilogue), so each role's registers are live
  // only in its own branch.
  if (role == 2) {
    // ---------------------------------------------------------- copy role
    // Copies: copy wave p issues the step's wave-instructions p, p + NQ, ...;
    // for each, the token of the step and its byte offset t * ROWB + chunk,
    // packed as (t << 16) | offset (offsets are < 2^16), fixed for every step.
    uint32_t cp_tok_off[NIW];
#pragma unroll
    for (int r = 0; r < NIW; ++r) {
      const int p = 64 * (role_w + NQ * r) + lane;
      const int t = p / CH;
      cp_tok_off[r] = (static_cast<uint32_t>(t) << 16) | static_cast<uint32_t>(t * ROWB + ((p - CH * t) ^ swz(t)) * 16);
    }
    StepPos ipos{0, off_first};  // the next step to copy
    auto issue = [&](int s) __attribute__((always_inline)) {
      const StepSrc src = step_src(lat, ipos, t_begin + STEP * s, t_end, BS, my_blk, NBi);
      advance(ipos, BS);
      const uint32_t dst0 = lds_addr(&buf[s & (NBUF - 1)][0]);
      const uint32_t lo_lim = static_cast<uint32_t>(src.n_lo) << 16;
      if (fuse && s == s_new) {
        // As the masked path, except that row tn (and every masked row that
        // would copy it) comes from the appended token's inputs.
        const uint8_t *kvc8 = reinterpret_cast<const uint8_t *>(ap.kvc + b * ap.kvc_st);
        const uint8_t *kpe8 = reinterpret_cast<const uint8_t *>(ap.kpe + b * ap.kpe_st);
#pragma unroll
        for (int r = 0; r < NIW; ++r) {
          const uint32_t to = cp_tok_off[r];
          const int t = static_cast<int>(to >> 16);
          const int tc = token_ok(src, t) ? t : src.safe;
          const int off = static_cast<int>(to & 0xffffu);
          const int c = (off - t * ROWB) >> 4;  // chunk of the row
          const uint8_t *g = (tc < src.n_lo ? src.base_lo : src.base_hi) + (off + (tc - t) * ROWB);
          if (tc == tn) g = c < R / 8 ? kvc8 + 16 * c : kpe8 + 16 * (c - R / 8);
          copy16_to_lds(g, dst0 + 1024 * (role_w + NQ * r));
        }
      } else if (src.full) {
#pragma unroll
        for (int r = 0; r < NIW; ++r) {
          const uint32_t to = cp_tok_off[r];
          copy16_to_lds((to < lo_lim ? src.base_lo : src.base_hi) + (to & 0xffffu), dst0 + 1024 * (role_w + NQ * r));
        }
      } else {
#pragma unroll
        for (int r = 0; r < NIW; ++r) {
          const uint32_t to = cp_tok_off[r];
          const int t = static_cast<int>(to >> 16);
          const int tc = token_ok(src, t) ? t : src.safe;
          // tc * ROWB + chunk offset, as a non-negative int (tc may be below t)
          copy16_to_lds(
              (tc < src.n_lo ? src.base_lo : src.base_hi) + (static_cast<int>(to & 0xffffu) + (tc - t) * ROWB),
              dst0 + 1024 * (role_w + NQ * r));
        }
      }
    };

    const int n_pre = nsteps < 3 ? nsteps : 3;  // steps copied before the loop
    for (int s = 0; s < n_pre; ++s) issue(s);
    // Step 0 landed once at most the later prologue copies are pending (the
    // counter holds 63: with one copy wave, wait for step 1 as well).
    if (n_pre == 3)
      wait_vmcnt<(2 * NIW < 64 ? 2 * NIW : NIW)>();
    else if (n_pre == 2)
      wait_vmcnt<NIW>();
    else
      wait_vmcnt<0>();
    barrier_lds();  // step 0 visible to the QK waves
    if (nsteps > 1) {
      if (n_pre == 3)  // step 1 landed
        wait_vmcnt<NIW>();
      else
        wait_vmcnt<0>();
    }
    WKV_PHASE(3)
    for (int s = 0; s < nsteps; ++s) {
      barrier_lds();  // step s + 1 landed, buffer of step s - 1 free
      WKV_PHASE(0)
      const bool more = s + 3 < nsteps;
      if (more) issue(s + 3);
      WKV_PHASE(1)
      // Step s + 2 must have landed before the next barrier.
      if (more)
        wait_vmcnt<NIW>();
      else
        wait_vmcnt<0>();
      WKV_PHASE(2)
    }
    WKV_PHASE_STORE(3, 4, 5, 7)
    __syncthreads();  // the epilogue barrier of the other roles
    return;
  }

  if (role == 1) {
    // ------------------------------------------------------------ PV role
    // Operand offsets. The transposed read of source lane (g, k, q) covers
    // row 4 g + k, elements d0 + 4 q .. + 3 of this wave's d-slice.
    const int tk = (lane >> 2) & 3, tq = lane & 3;
    const int trow = 4 * grp + tk;
    const int tr_row = trow * ROWB + role_w * DSL * 2 + (tq & 1) * 8;
    const int tr_x = (tq >> 1) ^ swz(trow);  // chunk of d-tile a: (2 (a & 3) + (tq >> 1)) ^ swz = (2 (a & 3)) ^ tr_x
    const int pt_w = ((grp * 16) + col) * 16;  // + hb * 1024
    floatx4 acc[NDT][NHB];
#pragma unroll
    for (int a = 0; a < NDT; ++a)
#pragma unroll
      for (int c = 0; c < NHB; ++c) acc[a][c] = floatx4{0.f, 0.f, 0.f, 0.f};
    StepPos ppos{0, off_first};  // the next step to accumulate

    auto pv_step = [&](int s) __attribute__((always_inline)) {
      const uint8_t *cur = &buf[s & (NBUF - 1)][0];
      const uint8_t *pts = &pt[s & 1][0];
      typedef __attribute__((__vector_size__(4 * sizeof(short)))) short s4;
      auto load_va = [&](int a) __attribute__((always_inline)) {
        const int o = tr_row + (((2 * (a & 3)) ^ tr_x) + 8 * (a >> 2)) * 16;
        const s4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) s4 *)(cur + o));
        const s4 hi =
            __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) s4 *)(cur + o + HALF));
        return __builtin_bit_cast(bf16x8, __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7));
      };
      // Every read the step starts with is issued before the first wait: the
      // first A operands, P^T and the rescale factors (one read). A-operand
      // reads then run PVPF d-tiles ahead of the MFMAs.
      constexpr int PVPF = 2;
      bf16x8 va[PVPF + 1];
#pragma unroll
      for (int a = 0; a < PVPF && a < NDT; ++a) va[a] = load_va(a);
      bf16x8 pb[NHB];
#pragma unroll
      for (int c = 0; c < NHB; ++c)
        pb[c] = __builtin_bit_cast(bf16x8, *reinterpret_cast<const u32x4 *>(pts + c * 1024 + pt_w));
      float cr[NHB];  // rescale factor of head 16 c + col
      if constexpr (NHB == 4) {
        const floatx4 v = *reinterpret_cast<const floatx4 *>(&corr_s[s & 1][col * NHB]);
#pragma unroll
        for (int c = 0; c < NHB; ++c) cr[c] = v[c];
      } else {
#pragma unroll
        for (int c = 0; c < NHB; ++c) cr[c] = corr_s[s & 1][col * NHB + c];
      }
      // The step's bookkeeping runs while those reads are in flight (a skipped
      // step leaves them unused).
      const StepSrc src = step_src(lat, ppos, t_begin + STEP * s, t_end, BS, my_blk, NBi);
      advance(ppos, BS);
      if (!src.any) return;
      bool moved = false;
#pragma unroll
      for (int c = 0; c < NHB; ++c) moved |= cr[c] != 1.f;
      if (__builtin_amdgcn_ballot_w64(moved)) {
#pragma unroll
        for (int a = 0; a < NDT; ++a)
#pragma unroll
          for (int c = 0; c < NHB; ++c)
#pragma unroll
            for (int i = 0; i < 4; ++i) acc[a][c][i] *= cr[c];
      }
      WKV_PHASE(1)
#pragma unroll
      for (int a = 0; a < NDT; ++a) {
        if (a + PVPF < NDT) va[(a + PVPF) % (PVPF + 1)] = load_va(a + PVPF);
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int c = 0; c < NHB; ++c)
          acc[a][c] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(va[a % (PVPF + 1)], pb[c], acc[a][c], 0, 0, 0);
      }
      WKV_PHASE(2)
    };

    WKV_PHASE(3)
    barrier_lds();  // step 0 landed
    for (int s = 0; s < nsteps; ++s) {
      barrier_lds();  // P(s) written, step s + 1 landed
      WKV_PHASE(0)
      pv_step(s);
    }
    WKV_PHASE_STORE(8, 9, 10, 6)
    WKV_PHASE_TOTAL(nsteps)
    __syncthreads();  // the QK waves' denominators and maxima are in LDS

    // ---- epilogue: the normalised output, or this partition's (bf16) partial.
#pragma unroll
    for (int c = 0; c < NHB; ++c) {
      const int hl = 16 * c + col, h = hbase + hl;
      const float lh = lsum_s[hl];
      // A whole sequence in one partition is finished here, sink included;
      // a partial carries (m, l) and the merge adds the sink.
      const float den = nparts == 1 ? lh + mla_sink_weight(sinks, h, mrun_s[hl] == -INFINITY ? 0.f : mrun_s[hl]) : lh;
      const float inv = den > 0.f ? 1.f / den : 0.f;
      uint16_t *dst = nparts == 1 ? out + (static_cast<int64_t>(b) * H + h) * R
                                  : part_o + ((static_cast<int64_t>(b) * H + h) * max_parts + part) * R;
#pragma unroll
      for (int a = 0; a < NDT; ++a) {
        u32x2 w;
        w[0] = pack_bf16x2(acc[a][c][0] * inv, acc[a][c][1] * inv);
        w[1] = pack_bf16x2(acc[a][c][2] * inv, acc[a][c][3] * inv);
        *reinterpret_cast<u32x2 *>(dst + role_w * DSL + 16 * a + 4 * grp) = w;
      }
      if (nparts > 1 && role_w == 0 && grp == 0) {
        const int64_t row = (static_cast<int64_t>(b) * H + h) * max_parts + part;
        part_ml[2 * row] = mrun_s[hl];
        part_ml[2 * row + 1] = lh;
      }
    }
    return;
  }

  // -------------------------------------------------------------- QK role
  // Q^T operand: lane holds 8 elements of head hbase + 16 w + col, k = 32 j + 8 grp.
  constexpr int NJ = W / 32;
  bf16x8 qop[NJ];
  {
    const int h = hbase + 16 * role_w + col;
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
      const uint16_t *src = (j < R / 32) ? qn + b * qn_sb + h * qn_sh + 32 * j + 8 * grp
                                         : qp + b * qp_sb + h * qp_sh + 32 * (j - R / 32) + 8 * grp;
      qop[j] = __builtin_bit_cast(bf16x8, *reinterpret_cast<const u32x4 *>(src));
    }
  }
  // Pin Q: the compiler waits for it here, not inside the loop.
#pragma unroll
  for (int j = 0; j < NJ; ++j) asm volatile("" : "+v"(qop[j]));
  if (fuse && hbase == 0 && role_w == 0) {  // the appended row -> its cache slot
    const int64_t slot = ap.slots[b];
    if (slot >= 0 && slot / BS < NB) {
      uint16_t *dst = lat + slot * W;
      for (int c = lane; c < CH; c += 64) {
        const uint16_t *src = c < R / 8 ? ap.kvc + b * ap.kvc_st + 8 * c : ap.kpe + b * ap.kpe_st + 8 * (c - R / 8);
        *reinterpret_cast<u32x4 *>(dst + 8 * c) = *reinterpret_cast<const u32x4 *>(src);
      }
    }
  }
  float m_run = -INFINITY, l_run = 0.f;  // reference maximum (log2 domain) and this lane's share of the sum
  StepPos qpos{0, off_first};  // the next step to score
  const int sq = swz(col);
  const int qk_gx = (grp ^ (sq & 3)) * 16 + col * ROWB;
  const int qk_jb = (sq >> 2) * 64;  // chunk bit 2 flips j's bit 0
  const int qk_even = qk_gx + qk_jb, qk_odd = qk_gx - qk_jb;
  const int pt_w = ((grp * 16) + col) * 16;

  auto qk_step = [&](int s) __attribute__((always_inline)) {
    const uint8_t *cur = &buf[s & (NBUF - 1)][0];
    // S^T for the 32 tokens; A-operand reads run QKPF k-steps ahead (a ring
    // of register slots; the scheduling fence keeps them there).
    // Even and odd k-steps accumulate separately: four independent chains.
    constexpr int QKPF = 2;
    floatx4 sc[2][2] = {{floatx4{0.f, 0.f, 0.f, 0.f}, floatx4{0.f, 0.f, 0.f, 0.f}},
                        {floatx4{0.f, 0.f, 0.f, 0.f}, floatx4{0.f, 0.f, 0.f, 0.f}}};
    bf16x8 ra[QKPF + 1][2];
    auto qk_load = [&](int j) __attribute__((always_inline)) {
      const int o = ((j & 1) ? qk_odd : qk_even) + 64 * j;
#pragma unroll
      for (int tt = 0; tt < 2; ++tt)
        ra[j % (QKPF + 1)][tt] = __builtin_bit_cast(bf16x8, *reinterpret_cast<const u32x4 *>(cur + o + tt * HALF));
    };
#pragma unroll
    for (int j = 0; j < QKPF; ++j) qk_load(j);
    // The step's bookkeeping runs while the first reads are in flight.
    const StepSrc src = step_src(lat, qpos, t_begin + STEP * s, t_end, BS, my_blk, NBi);
    advance(qpos, BS);
    if (!src.any) return;
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
      if (j + QKPF < NJ) qk_load(j + QKPF);
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int tt = 0; tt < 2; ++tt)
        sc[j & 1][tt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ra[j % (QKPF + 1)][tt], qop[j], sc[j & 1][tt], 0, 0, 0);
    }
    WKV_PHASE(1)
    // Online softmax; lane (col, grp) holds tokens 4 grp + i and 16 + 4 grp + i.
    float sv[8];
#pragma unroll
    for (int tt = 0; tt < 2; ++tt)
#pragma unroll
      for (int i = 0; i < 4; ++i) sv[4 * tt + i] = (sc[0][tt][i] + sc[1][tt][i]) * scale_log2;
    if (!src.full) {
#pragma unroll
      for (int tt = 0; tt < 2; ++tt)
#pragma unroll
        for (int i = 0; i < 4; ++i)
          if (!token_ok(src, 16 * tt + 4 * grp + i)) sv[4 * tt + i] = -INFINITY;
    }
    const float mt = row_max4(
        fmaxf(fmaxf(fmaxf(sv[0], sv[1]), fmaxf(sv[2], sv[3])), fmaxf(fmaxf(sv[4], sv[5]), fmaxf(sv[6], sv[7]))));
    const bool move = mt > m_run + SOFTMAX_TAU;
    const float m_new = move ? mt : m_run;
    const float cr = (move && m_run != -INFINITY) ? fast_exp2(m_run - m_new) : 1.f;
    const float m_use = (m_new == -INFINITY) ? 0.f : m_new;
    float p[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) p[i] = fast_exp2(sv[i] - m_use);
    m_run = m_new;
    // The packed words stay scalars: hipcc 7.2 hands a bit_cast of an element
    // of a 4-vector its first element.
    uint32_t pw[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) pw[i] = pack_bf16x2(p[2 * i], p[2 * i + 1]);
    *reinterpret_cast<u32x4 *>(&pt[s & 1][role_w * 1024 + pt_w]) = u32x4{pw[0], pw[1], pw[2], pw[3]};
    // The running sum takes the bf16 probabilities the PV products consume, so
    // numerator and denominator carry the same rounding (a head dominated by a
    // few tokens then normalises to their exact weights).
    const bf16x2 ones = __builtin_bit_cast(bf16x2, 0x3F803F80u);
    float psum = 0.f;
#pragma unroll
    for (int i = 0; i < 4; ++i) psum = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, pw[i]), ones, psum, false);
    l_run = l_run * cr + psum;
    if (grp == 0) corr_s[s & 1][col * NHB + role_w] = cr;
    WKV_PHASE(2)
  };

  barrier_lds();  // step 0 landed
  qk_step(0);
  for (int s = 0; s < nsteps; ++s) {
    barrier_lds();  // step s + 1 landed; the PV waves are done with P(s - 1)
    WKV_PHASE(0)
    if (s + 1 < nsteps) qk_step(s + 1);
  }
  WKV_PHASE_STORE(11, 14, 15, -1)
  {
    float l = l_run + __shfl_xor(l_run, 16, 64);
    l += __shfl_xor(l, 32, 64);
    if (grp == 0) {
      lsum_s[16 * role_w + col] = l;
      mrun_s[16 * role_w + col] = m_run;
    }
  }
  __syncthreads();
}

// Blocks a partition of p tokens can touch: partitions start on a multiple
// of the 32-token step, so at most BS - 32 tokens into a block (0 for BS 16).
static int mla_partition_blocks(int p, int BS) {
  const int lead = BS > mla::STEP ? BS - mla::STEP : 0;
  return (p + lead + BS - 1) / BS;
}

// Head groups per (sequence, partition): 128 heads run as two workgroups of
// 64 (12 waves, three per SIMD), every smaller count as one.
static int mla_head_groups(int num_heads) { return num_heads == 128 ? 2 : 1; }

// Tokens per partition when the caller leaves it to the library: one
// workgroup per CU in one round (256 CUs), a multiple of the 32-token step,
// touching at most 64 blocks (one lane of the block-id register each).
static int choose_mla_partition(int batch, int num_heads, int max_seq_len, int BS) {
  const int wg_per_part = batch * mla_head_groups(num_heads);
  int parts = wg_per_part > 0 ? (256 + wg_per_part - 1) / wg_per_part : 1;
  int p = (max_seq_len + parts - 1) / (parts > 0 ? parts : 1);
  p = (p + mla::STEP - 1) / mla::STEP * mla::STEP;
  if (p < mla::STEP) p = mla::STEP;
  while (p > mla::STEP && mla_partition_blocks(p, BS) > 64) p -= mla::STEP;
  return p;
}

}  // namespace wkv

using namespace wkv;

#ifdef WKV_PHASE_CLOCKS
extern "C" int wkv_mla_phase_clocks(unsigned long long *dst, int n) {
  if (dst == nullptr || n < 0 || n > kPhaseWgs * 16) return WKV_ERR_INVALID;
  return hipMemcpyFromSymbol(dst, HIP_SYMBOL(g_mla_phase), static_cast<size_t>(n) * 8) == hipSuccess ? WKV_OK
                                                                                                   : WKV_ERR_LAUNCH;
}
#endif

extern "C" int64_t wkv_mla_workspace_size(int32_t batch, int32_t num_heads, int32_t kv_lora_rank,
                                          int32_t max_seq_len, int32_t partition_size) {
  if (batch < 0 || num_heads <= 0 || kv_lora_rank <= 0 || max_seq_len < 0 || partition_size < 0) return -1;
  if (partition_size == 0) partition_size = mla::STEP;  // the smallest partition the library picks by itself
  const int64_t max_parts = (static_cast<int64_t>(max_seq_len) + partition_size - 1) / partition_size;
  // per (sequence, head, partition): the bf16 partial output, then its maximum and sum (fp32)
  return static_cast<int64_t>(batch) * num_heads * (max_parts > 0 ? max_parts : 1) * (kv_lora_rank * 2 + 8);
}

namespace wkv {

static int launch_mla(const wkv_mla_cache_t *cache, const void *q_nope, int64_t qn_stride_b, int64_t qn_stride_h,
                      const void *q_pe, int64_t qp_stride_b, int64_t qp_stride_h, void *out, int32_t num_heads,
                      const int32_t *block_table, int64_t bt_stride, int32_t max_blocks_per_seq,
                      const int32_t *seq_lens, int32_t batch, int32_t max_seq_len, float scale,
                      int32_t partition_size, void *workspace, int64_t workspace_bytes, const MlaAppend &ap,
                      const float *sinks, void *stream) {
  WKV_CHECK_ARG(cache != nullptr && cache->latent != nullptr && aligned16(cache->latent), "bad MLA cache");
  WKV_CHECK_ARG(cache->num_blocks > 0 && cache->num_blocks <= 0x7fffffff && cache->block_size > 0 &&
                    cache->block_size % 16 == 0 && cache->block_size <= 256,
                "MLA cache needs 1 <= num_blocks < 2^31 and block_size a multiple of 16 in [16, 256]");
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
  const int max_seq = max_seq_len < max_blocks_per_seq * BS ? max_seq_len : max_blocks_per_seq * BS;
  if (partition_size == 0) partition_size = choose_mla_partition(batch, num_heads, max_seq, BS);
  WKV_CHECK_ARG(partition_size >= mla::STEP && partition_size % mla::STEP == 0,
                "MLA partition_size must be a positive multiple of %d (got %d)", mla::STEP, partition_size);
  WKV_CHECK_ARG(mla_partition_blocks(partition_size, BS) <= 64,
                "MLA partition_size %d can span more than 64 blocks of %d tokens", partition_size, BS);
  const int max_parts = max_seq > 0 ? (max_seq + partition_size - 1) / partition_size : 1;
  WKV_CHECK_ARG(max_parts <= 65535, "too many partitions");
  const int64_t need = wkv_mla_workspace_size(batch, num_heads, 512, max_seq, partition_size);
  if (max_parts > 1)
    WKV_CHECK_ARG(workspace != nullptr && aligned16(workspace) && workspace_bytes >= need,
                  "workspace too small: need %lld bytes, got %lld", (long long)need, (long long)workspace_bytes);
  uint16_t *part_o = static_cast<uint16_t *>(workspace);
  float *part_ml = part_o ? reinterpret_cast<float *>(part_o + static_cast<int64_t>(batch) * num_heads * max_parts * 512)
                          : nullptr;
  const float scale_log2 = scale * 1.4426950408889634f;
  auto s = static_cast<hipStream_t>(stream);
  const int HG = mla_head_groups(num_heads);
  const int64_t items = static_cast<int64_t>(batch) * max_parts;
  const int64_t wgs = 8 * HG * ((items + 7) / 8);
  WKV_CHECK_ARG(wgs <= 0x7fffffff && items <= 0x7fffffff, "MLA grid too large");
  const dim3 grid(static_cast<unsigned>(wgs));
  auto lat = static_cast<uint16_t *>(cache->latent);
  auto qn = static_cast<const uint16_t *>(q_nope);
  auto qpp = static_cast<const uint16_t *>(q_pe);
  auto oo = static_cast<uint16_t *>(out);
#define WKV_MLA(NQv)                                                                                        \
  decode_mla_kernel<NQv><<<grid, 192 * NQv, 0, s>>>(lat, qn, qn_stride_b, qn_stride_h, qpp, qp_stride_b,          \
                                                    qp_stride_h, oo, part_o, part_ml, block_table, bt_stride,      \
                                                    max_blocks_per_seq, max_seq, seq_lens, BS, cache->num_blocks, \
                                                    scale_log2, partition_size, max_parts, num_heads, batch, ap,  \
                                                    batch % 8 == 0, sinks)
  switch (num_heads) {
    case 16: WKV_MLA(1); break;
    case 32: WKV_MLA(2); break;
    default: WKV_MLA(4); break;  // 64 heads, or 128 as two head groups
  }
#undef WKV_MLA
  WKV_CHECK_LAUNCH("wkv_paged_decode_mla");
  if (max_parts > 1) {
    mla_merge_kernel<<<dim3(static_cast<unsigned>((num_heads + 1) / 2), static_cast<unsigned>(batch)), 256, 0, s>>>(
        part_o, part_ml, oo, seq_lens, max_seq, num_heads, partition_size, max_parts, sinks);
    WKV_CHECK_LAUNCH("wkv_paged_decode_mla merge");
  }
  return WKV_OK;
}

}  // namespace wkv

extern "C" int wkv_paged_decode_mla(const wkv_mla_cache_t *cache, const void *q_nope, int64_t qn_stride_b,
                                    int64_t qn_stride_h, const void *q_pe, int64_t qp_stride_b, int64_t qp_stride_h,
                                    void *out, int32_t num_heads, const int32_t *block_table, int64_t bt_stride,
                                    int32_t max_blocks_per_seq, const int32_t *seq_lens, int32_t batch,
                                    int32_t max_seq_len, float scale, int32_t partition_size, void *workspace,
                                    int64_t workspace_bytes, void *stream) {
  const MlaAppend none{nullptr, 0, nullptr, 0, nullptr};
  return launch_mla(cache, q_nope, qn_stride_b, qn_stride_h, q_pe, qp_stride_b, qp_stride_h, out, num_heads,
                    block_table, bt_stride, max_blocks_per_seq, seq_lens, batch, max_seq_len, scale, partition_size,
                    workspace, workspace_bytes, none, nullptr, stream);
}

extern "C" int wkv_paged_decode_mla_sinks(const wkv_mla_cache_t *cache, const void *q_nope, int64_t qn_stride_b,
                                          int64_t qn_stride_h, const void *q_pe, int64_t qp_stride_b,
                                          int64_t qp_stride_h, void *out, int32_t num_heads,
                                          const int32_t *block_table, int64_t bt_stride, int32_t max_blocks_per_seq,
                                          const int32_t *seq_lens, int32_t batch, int32_t max_seq_len, float scale,
                                          int32_t partition_size, void *workspace, int64_t workspace_bytes,
                                          const float *sinks, void *stream) {
  WKV_CHECK_ARG(sinks != nullptr && reinterpret_cast<uintptr_t>(sinks) % 4 == 0, "sinks must be non-NULL fp32");
  const MlaAppend none{nullptr, 0, nullptr, 0, nullptr};
  return launch_mla(cache, q_nope, qn_stride_b, qn_stride_h, q_pe, qp_stride_b, qp_stride_h, out, num_heads,
                    block_table, bt_stride, max_blocks_per_seq, seq_lens, batch, max_seq_len, scale, partition_size,
                    workspace, workspace_bytes, none, sinks, stream);
}

extern "C" int wkv_append_paged_decode_mla(const wkv_mla_cache_t *cache, const void *kv_c, int64_t kv_c_stride,
                                           const void *k_pe, int64_t k_pe_stride, const int64_t *slot_mapping,
                                           const void *q_nope, int64_t qn_stride_b, int64_t qn_stride_h,
                                           const void *q_pe, int64_t qp_stride_b, int64_t qp_stride_h, void *out,
                                           int32_t num_heads, const int32_t *block_table, int64_t bt_stride,
                                           int32_t max_blocks_per_seq, const int32_t *seq_lens, int32_t batch,
                                           int32_t max_seq_len, float scale, int32_t partition_size,
                                           void *workspace, int64_t workspace_bytes, void *stream) {
  WKV_CHECK_ARG(kv_c && k_pe && aligned16(kv_c) && aligned16(k_pe), "kv_c/k_pe must be non-NULL and 16-byte aligned");
  WKV_CHECK_ARG(kv_c_stride >= 0 && k_pe_stride >= 0 && (kv_c_stride | k_pe_stride) % 8 == 0,
                "kv_c/k_pe row strides must be non-negative multiples of 8");
  WKV_CHECK_ARG(slot_mapping != nullptr, "slot_mapping is NULL");
  const MlaAppend ap{static_cast<const uint16_t *>(kv_c), kv_c_stride, static_cast<const uint16_t *>(k_pe),
                     k_pe_stride, slot_mapping};
  return launch_mla(cache, q_nope, qn_stride_b, qn_stride_h, q_pe, qp_stride_b, qp_stride_h, out, num_heads,
                    block_table, bt_stride, max_blocks_per_seq, seq_lens, batch, max_seq_len, scale, partition_size,
                    workspace, workspace_bytes, ap, nullptr, stream);
}

extern "C" int wkv_append_paged_decode_mla_sinks(const wkv_mla_cache_t *cache, const void *kv_c,
                                                 int64_t kv_c_stride, const void *k_pe, int64_t k_pe_stride,
                                                 const int64_t *slot_mapping, const void *q_nope,
                                                 int64_t qn_stride_b, int64_t qn_stride_h, const void *q_pe,
                                                 int64_t qp_stride_b, int64_t qp_stride_h, void *out,
                                                 int32_t num_heads, const int32_t *block_table, int64_t bt_stride,
                                                 int32_t max_blocks_per_seq, const int32_t *seq_lens, int32_t batch,
                                                 int32_t max_seq_len, float scale, int32_t partition_size,
                                                 void *workspace, int64_t workspace_bytes, const float *sinks,
                                                 void *stream) {
  WKV_CHECK_ARG(sinks != nullptr && reinterpret_cast<uintptr_t>(sinks) % 4 == 0, "sinks must be non-NULL fp32");
  WKV_CHECK_ARG(kv_c && k_pe && aligned16(kv_c) && aligned16(k_pe), "kv_c/k_pe must be non-NULL and 16-byte aligned");
  WKV_CHECK_ARG(kv_c_stride >= 0 && k_pe_stride >= 0 && (kv_c_stride | k_pe_stride) % 8 == 0,
                "kv_c/k_pe row strides must be non-negative multiples of 8");
  WKV_CHECK_ARG(slot_mapping != nullptr, "slot_mapping is NULL");
  const MlaAppend ap{static_cast<const uint16_t *>(kv_c), kv_c_stride, static_cast<const uint16_t *>(k_pe),
                     k_pe_stride, slot_mapping};
  return launch_mla(cache, q_nope, qn_stride_b, qn_stride_h, q_pe, qp_stride_b, qp_stride_h, out, num_heads,
                    block_table, bt_stride, max_blocks_per_seq, seq_lens, batch, max_seq_len, scale, partition_size,
                    workspace, workspace_bytes, ap, sinks, stream);
}
