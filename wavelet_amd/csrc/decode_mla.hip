// Weight-absorbed MLA paged decode for gfx950.
//
// Every query head reads the same latent row c = [c_kv (512) | k_pe (64)]
// (1152 bytes per token), so one workgroup owns one (sequence, partition) for
// ALL heads and HBM delivers each latent byte once.
//
// Memory pipeline. The partition is streamed in 32-token steps (36 KB). Each
// step is copied HBM -> LDS by global_load_lds_dwordx4 (lane i of a wave
// instruction lands at LDS base + 16 i), with no register staging, into one
// of three LDS buffers; two steps are in flight while the third is computed.
// A wave waits only for its own copies of the step about to be used
// (s_waitcnt vmcnt(n)) and a barrier publishes everyone's. The buffers are
// distinct __shared__ objects indexed statically, so the compiler can prove
// that reading one never aliases the copies still landing in the others.
//
// LDS layout of a step: row t (token), 72 chunks of 16 bytes; chunk c of row
// t sits at slot c ^ swz(t), so the QK reads (16 rows, same chunk) and the
// transposed PV reads (8 rows x 32 bytes) each cover all 64 banks once.
//
// Per step, with waves w = 0..NW-1 and HPB 16-head blocks per wave:
//   QK  S^T[32 tok, heads of w] = C[32 tok, 576] . Q^T   (mfma_f32_16x16x32_bf16,
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

// Chunk slot XOR of row t (t mod 16 matters). With 64 four-byte banks, a
// 16-byte read serves 16 lanes per cycle and an 8-byte read 32: rows of one
// parity share a 128-byte bank half (1152 = 4.5 x 256), so the slot XOR must
// differ across the 8 rows of each parity among 16 consecutive rows (QK: 16
// rows, one chunk each) and, in its upper two bits, across the 4 rows of each
// parity among 8 (transposed PV reads: 8 rows, an aligned chunk pair each).
__device__ __forceinline__ int swz(int t) { return (((t >> 1) & 3) << 1) | ((t >> 3) & 1); }

// The copies, the waits for them and the barriers are written as inline asm
// so the compiler's own wait-count insertion never sees an LDS write it would
// have to wait for: it cannot always prove that a read of one step buffer
// does not alias the copies still landing in the others, and then waits for
// every outstanding copy (vmcnt(0)), which would drain the pipeline. The
// "memory" clobbers keep the compiler from moving LDS accesses across them.
// M0 carries the LDS address of an LDS-DMA copy; nothing else in the kernel
// uses M0, and each copy sets it immediately before use.
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"
__device__ __forceinline__ void copy16_to_lds(const void *g, uint32_t lds) {
  asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %1, off" ::"s"(lds), "v"(g) : "memory", "m0");
}
#pragma clang diagnostic pop

// Waits until at most N of this wave's vector-memory operations are pending.
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}

// Workgroup barrier for LDS: this wave's LDS accesses complete, then s_barrier.
__device__ __forceinline__ void barrier_lds() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }

__device__ __forceinline__ uint32_t lds_addr(const void *p) {
  return static_cast<uint32_t>(reinterpret_cast<uintptr_t>((const __attribute__((address_space(3))) void *)p));
}

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

// 2^x on the hardware exp unit (v_exp_f32). Every argument here is <= 0 (a
// score minus a running maximum), where the only difference from exp2f is
// that results below 2^-126 flush to 0.
__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

// Two fp32 -> packed bf16 (RNE) with the hardware conversion (v_cvt_pk_bf16_f32).
__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
  typedef __attribute__((__vector_size__(2 * sizeof(__bf16)))) __bf16 bf16x2_t;
  typedef __attribute__((__vector_size__(2 * sizeof(float)))) float f32x2_t;
  return __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2_t{lo, hi}), bf16x2_t));
}

// Online softmax keeps a reference maximum per head and rescales the running
// sum and output only when a step's maximum exceeds it by more than 2^TAU:
// probabilities are exp2(s - ref) <= 2^TAU (exact in bf16's range and
// precision), and rescaling -- a pass over every accumulator -- becomes rare.
constexpr float TAU = 8.f;

}  // namespace mla

// Log-sum-exp merge of the per-partition partials of one (sequence, head):
// 128 lanes per head, four output elements (one 16-byte partial load per
// partition) per lane, two heads per 256-thread workgroup.
__global__ __launch_bounds__(256) void mla_merge_kernel(const float *__restrict__ part_o,
                                                        const float *__restrict__ part_ml, uint16_t *__restrict__ out,
                                                        const int32_t *__restrict__ seq_lens, int max_seq, int H,
                                                        int P_tok, int max_parts) {
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
    const float w = exp2f(part_ml[2 * (row0 + p)] - m_use);
    den += w * part_ml[2 * (row0 + p) + 1];
    const floatx4 o = *reinterpret_cast<const floatx4 *>(part_o + (row0 + p) * R + d);
#pragma unroll
    for (int i = 0; i < 4; ++i) num[i] += w * o[i];
  }
  const float inv = den > 0.f ? 1.f / den : 0.f;
  u32x2 v;
  v[0] = f32_to_bf16_bits(num[0] * inv) | (f32_to_bf16_bits(num[1] * inv) << 16);
  v[1] = f32_to_bf16_bits(num[2] * inv) | (f32_to_bf16_bits(num[3] * inv) << 16);
  *reinterpret_cast<u32x2 *>(out + (static_cast<int64_t>(b) * H + h) * R + d) = v;
}

// NW waves, HPB 16-head blocks per wave for QK: a workgroup owns HW = 16 *
// NW * HPB of the H = HW * HG heads. The 1-D grid is laid out for the
// dispatcher, which deals workgroup i to XCD i mod 8: work item k = (sequence,
// partition) goes to XCD k mod 8, and its HG head groups are workgroups
// 8 HG (k / 8) + 8 g + (k mod 8), i.e. on the same XCD and dispatched back
// to back, so the second read of each latent tile is served by that XCD's L2.
template <int NW, int HPB>
__global__ __launch_bounds__(64 * NW, 1) void decode_mla_kernel(
    const uint16_t *__restrict__ lat, const uint16_t *__restrict__ qn, int64_t qn_sb, int64_t qn_sh,
    const uint16_t *__restrict__ qp, int64_t qp_sb, int64_t qp_sh, uint16_t *__restrict__ out,
    float *__restrict__ part_o, float *__restrict__ part_ml, const int32_t *__restrict__ bt, int64_t bt_stride,
    int Mb, int max_seq, const int32_t *__restrict__ seq_lens, int BS, int64_t NB, float scale_log2, int P_tok,
    int max_parts, int H, int batch) {
  using namespace mla;
  constexpr int NHB = NW * HPB;     // head blocks of this workgroup
  constexpr int HW = 16 * NHB;      // heads of this workgroup
  constexpr int DSL = R / NW;       // PV d-slice per wave
  constexpr int NDT = DSL / 16;     // PV d-tiles per wave
  constexpr int NIW = NDMA / NW;    // copies every wave issues per step
  constexpr int NEXTRA = NDMA % NW; // waves < NEXTRA issue one more
  static_assert(DSL % 64 == 0, "d-slice must be a multiple of 64");

  __shared__ __attribute__((aligned(16))) uint8_t buf0[STEPB];
  __shared__ __attribute__((aligned(16))) uint8_t buf1[STEPB];
  __shared__ __attribute__((aligned(16))) uint8_t buf2[STEPB];
  __shared__ __attribute__((aligned(16))) uint8_t pt[NHB * 1024];  // P^T, [hb][g][col][8 bf16]
  __shared__ __attribute__((aligned(16))) uint8_t qpe_s[NHB * 2 * 1024];  // Q^T rope part, [hb][j][g][col][8]
  __shared__ float corr_s[HW];
  __shared__ float lsum_s[HW];
  __shared__ float mrun_s[HW];

  // The decode divides by runtime values, which the compiler does on the
  // vector unit; readfirstlane returns the (uniform) results to scalar
  // registers so everything derived from them stays scalar.
  const int NBi = static_cast<int>(NB);  // the host bounds num_blocks to int32
  const int HG = H / HW;
  const int wg_r = __builtin_amdgcn_readfirstlane(static_cast<int>(blockIdx.x % (8 * HG)));
  const int item = __builtin_amdgcn_readfirstlane(static_cast<int>(8 * (blockIdx.x / (8 * HG)) + (wg_r & 7)));
  if (static_cast<int64_t>(item) >= static_cast<int64_t>(batch) * max_parts) return;  // padding of the last group of 8
  const int b = __builtin_amdgcn_readfirstlane(item / max_parts);
  const int part = __builtin_amdgcn_readfirstlane(item % max_parts);
  const int hbase = HW * (wg_r >> 3);  // first head of this workgroup
  const int wave = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x >> 6));
  const int lane = threadIdx.x & 63, col = lane & 15, grp = lane >> 4;
  const int t_begin = part * P_tok;
  const int blk_first = __builtin_amdgcn_readfirstlane(t_begin / BS);
  const int off_first = t_begin - blk_first * BS;

  // Uniform across the workgroup: kept in scalar registers so that all the
  // per-step bookkeeping derived from it runs on the scalar unit.
  int L = __builtin_amdgcn_readfirstlane(seq_lens[b]);
  int my_blk = -1;  // lane i: id of the partition's i-th block
  if (blk_first + lane < Mb) my_blk = bt[b * bt_stride + blk_first + lane];
  L = L < max_seq ? L : max_seq;
  const int nparts = L > 0 ? (L + P_tok - 1) / P_tok : 0;
  if (nparts == 0) {
    if (part == 0) {
      for (int e = threadIdx.x; e < HW * R / 8; e += 64 * NW)
        reinterpret_cast<u32x4 *>(out + (static_cast<int64_t>(b) * H + hbase) * R)[e] = u32x4{0u, 0u, 0u, 0u};
    }
    return;
  }
  if (part >= nparts) return;
  const int t_end = (t_begin + P_tok) < L ? (t_begin + P_tok) : L;
  const int nsteps = (t_end - t_begin + STEP - 1) / STEP;

  // ---- copy issue: this wave's share of one step's 36 wave-instructions.
  // Per copy r of this wave: token t of the step and byte offset t * ROWB + chunk,
  // packed as (t << 16) | offset (offsets are < 2^16), fixed for every step.
  constexpr int NCP = NIW + (NEXTRA ? 1 : 0);
  uint32_t cp_tok_off[NCP];
#pragma unroll
  for (int r = 0; r < NCP; ++r) {
    const int p = 64 * (wave + NW * r) + lane;
    const int t = p / CH;
    cp_tok_off[r] = (static_cast<uint32_t>(t) << 16) | static_cast<uint32_t>(t * ROWB + ((p - CH * t) ^ swz(t)) * 16);
  }
  StepPos ipos{0, off_first};  // the next step to copy
  StepPos cpos{0, off_first};  // the next step to compute
  auto issue = [&](int s, uint8_t *dst) __attribute__((always_inline)) {
    const StepSrc src = step_src(lat, ipos, t_begin + STEP * s, t_end, BS, my_blk, NBi);
    advance(ipos, BS);
    const uint32_t dst0 = lds_addr(dst);
    const uint32_t lo_lim = static_cast<uint32_t>(src.n_lo) << 16;
    if (src.full) {
#pragma unroll
      for (int r = 0; r < NCP; ++r) {
        if (r < NIW || wave < NEXTRA) {
          const uint32_t to = cp_tok_off[r];
          copy16_to_lds((to < lo_lim ? src.base_lo : src.base_hi) + (to & 0xffffu), dst0 + 1024 * (wave + NW * r));
        }
      }
    } else {
#pragma unroll
      for (int r = 0; r < NCP; ++r) {
        if (r < NIW || wave < NEXTRA) {
          const uint32_t to = cp_tok_off[r];
          const int t = static_cast<int>(to >> 16);
          const int tc = token_ok(src, t) ? t : src.safe;
          // tc * ROWB + chunk offset, as a non-negative int (tc may be below t)
          copy16_to_lds((tc < src.n_lo ? src.base_lo : src.base_hi) + (static_cast<int>(to & 0xffffu) + (tc - t) * ROWB),
                        dst0 + 1024 * (wave + NW * r));
        }
      }
    }
  };

  // The first two steps' copies go out first, then Q. Q is then pinned
  // (an empty asm that reads every Q register) before the loop, so the
  // compiler waits for it here instead of inside the loop, where its count of
  // vector-memory operations (it cannot see the copies) would also wait for
  // every copy in flight.
  issue(0, buf0);
  if (nsteps > 1) issue(1, buf1);
  // ---- Q^T operands: lane holds 8 elements of head 16*hb + col, k = 32 j + 8 grp.
  // The c_kv part (j < 16) stays in registers; the rope part (j = 16, 17) is
  // parked in LDS (each wave reads back only its own heads) to leave the
  // registers to the accumulators and the LDS read pipeline.
  constexpr int NJQ = R / 32;
  bf16x8 qop[HPB][NJQ];
#pragma unroll
  for (int hb = 0; hb < HPB; ++hb) {
    const int hbg = wave * HPB + hb;
    const int h = hbase + 16 * hbg + col;
#pragma unroll
    for (int j = 0; j < NJQ; ++j)
      qop[hb][j] = __builtin_bit_cast(bf16x8, *reinterpret_cast<const u32x4 *>(qn + b * qn_sb + h * qn_sh + 32 * j + 8 * grp));
#pragma unroll
    for (int j = 0; j < PE / 32; ++j)
      *reinterpret_cast<u32x4 *>(qpe_s + (hbg * 2 + j) * 1024 + (grp * 16 + col) * 16) =
          *reinterpret_cast<const u32x4 *>(qp + b * qp_sb + h * qp_sh + 32 * j + 8 * grp);
  }
#pragma unroll
  for (int hb = 0; hb < HPB; ++hb)
#pragma unroll
    for (int j = 0; j < NJQ; ++j) asm volatile("" : "+v"(qop[hb][j]));

  // Per-lane LDS offsets. QK A operand: row (16 tt + col), chunk 4 j + grp.
  const int sq = swz(col);
  const int qk_gx = (grp ^ (sq & 3)) * 16 + col * ROWB;
  const int qk_jb = (sq >> 2) * 64;  // chunk bit 2 flips j's bit 0
  const int qk_even = qk_gx + qk_jb, qk_odd = qk_gx - qk_jb;
  // PV A operand (transposed read): source lane (g, k, q) reads row 4 g + k,
  // elements d0 + 4 q .. + 3 of its d-slice.
  const int tk = (lane >> 2) & 3, tq = lane & 3;
  const int trow = 4 * grp + tk;
  const int tsw = swz(trow);
  const int tr_row = trow * ROWB + wave * DSL * 2 + (tq & 1) * 8;
  const int tr_x = (tq >> 1) ^ tsw;  // chunk of d-tile a: (2 (a & 3) + (tq >> 1)) ^ tsw = (2 (a & 3)) ^ tr_x
  const int pt_w = ((grp * 16) + col) * 16;  // + hb * 1024

  floatx4 acc[NDT][NHB];
#pragma unroll
  for (int a = 0; a < NDT; ++a)
#pragma unroll
    for (int c = 0; c < NHB; ++c) acc[a][c] = floatx4{0.f, 0.f, 0.f, 0.f};
  float m_run[HPB], l_run[HPB];
#pragma unroll
  for (int hb = 0; hb < HPB; ++hb) {
    m_run[hb] = -INFINITY;
    l_run[hb] = 0.f;
  }

  auto step = [&](int s, const uint8_t *cur, uint8_t *nxt2) __attribute__((always_inline)) {
    // Own copies of step s have landed once at most the next step's remain.
    if (s + 1 < nsteps) {
      if (NEXTRA && wave < NEXTRA)
        wait_vmcnt<NIW + 1>();
      else
        wait_vmcnt<NIW>();
    } else {
      wait_vmcnt<0>();
    }
    barrier_lds();
    if (s + 2 < nsteps) issue(s + 2, nxt2);
    const int ts = t_begin + STEP * s;
    const StepSrc src = step_src(lat, cpos, ts, t_end, BS, my_blk, NBi);
    advance(cpos, BS);

    if (src.any) {
      // ---- QK for this wave's heads over the step's 32 tokens. The A-operand
      // reads run QKPF k-steps ahead of the MFMAs (a ring of register slots);
      // the scheduling fences keep the compiler from sinking them back to
      // their uses, which would leave one LDS round trip per MFMA.
      constexpr int NJ = W / 32;
      constexpr int QKPF = 2;
      floatx4 sc[2][HPB];
#pragma unroll
      for (int tt = 0; tt < 2; ++tt)
#pragma unroll
        for (int hb = 0; hb < HPB; ++hb) sc[tt][hb] = floatx4{0.f, 0.f, 0.f, 0.f};
      bf16x8 ra[QKPF + 1][2];
      auto qk_load = [&](int j) __attribute__((always_inline)) {
        const int o = ((j & 1) ? qk_odd : qk_even) + 64 * j;
#pragma unroll
        for (int tt = 0; tt < 2; ++tt)
          ra[j % (QKPF + 1)][tt] = __builtin_bit_cast(bf16x8, *reinterpret_cast<const u32x4 *>(cur + o + tt * HALF));
      };
#pragma unroll
      for (int j = 0; j < QKPF; ++j) qk_load(j);
#pragma unroll
      for (int j = 0; j < NJ; ++j) {
        if (j + QKPF < NJ) qk_load(j + QKPF);
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int hb = 0; hb < HPB; ++hb) {
          const bf16x8 qb = j < NJQ ? qop[hb][j < NJQ ? j : 0]
                                    : __builtin_bit_cast(bf16x8, *reinterpret_cast<const u32x4 *>(
                                          qpe_s + ((wave * HPB + hb) * 2 + (j - NJQ)) * 1024 + pt_w));
#pragma unroll
          for (int tt = 0; tt < 2; ++tt)
            sc[tt][hb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ra[j % (QKPF + 1)][tt], qb, sc[tt][hb], 0, 0, 0);
        }
      }
      // ---- online softmax; lane (col, grp) holds tokens 4 grp + i and 16 + 4 grp + i.
#pragma unroll
      for (int hb = 0; hb < HPB; ++hb) {
        float sv[8];
#pragma unroll
        for (int tt = 0; tt < 2; ++tt)
#pragma unroll
          for (int i = 0; i < 4; ++i) sv[4 * tt + i] = sc[tt][hb][i] * scale_log2;
        if (!src.full) {
#pragma unroll
          for (int tt = 0; tt < 2; ++tt)
#pragma unroll
            for (int i = 0; i < 4; ++i)
              if (!token_ok(src, 16 * tt + 4 * grp + i)) sv[4 * tt + i] = -INFINITY;
        }
        float mt = fmaxf(fmaxf(fmaxf(sv[0], sv[1]), fmaxf(sv[2], sv[3])), fmaxf(fmaxf(sv[4], sv[5]), fmaxf(sv[6], sv[7])));
        mt = fmaxf(mt, __shfl_xor(mt, 16, 64));
        mt = fmaxf(mt, __shfl_xor(mt, 32, 64));
        // m_run is the reference maximum (-inf until the first attended token).
        const bool move = mt > m_run[hb] + TAU;
        const float m_new = move ? mt : m_run[hb];
        const float cr = (move && m_run[hb] != -INFINITY) ? fast_exp2(m_run[hb] - m_new) : 1.f;
        const float m_use = (m_new == -INFINITY) ? 0.f : m_new;
        float p[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) p[i] = fast_exp2(sv[i] - m_use);
        l_run[hb] = l_run[hb] * cr + (((p[0] + p[1]) + (p[2] + p[3])) + ((p[4] + p[5]) + (p[6] + p[7])));
        m_run[hb] = m_new;
        u32x4 pb;
#pragma unroll
        for (int i = 0; i < 4; ++i) pb[i] = pack_bf16x2(p[2 * i], p[2 * i + 1]);
        const int hbg = wave * HPB + hb;
        *reinterpret_cast<u32x4 *>(pt + hbg * 1024 + pt_w) = pb;
        if (grp == 0) corr_s[col * NHB + hbg] = cr;
      }
    }
    barrier_lds();
    if (src.any) {
      // ---- PV: rescale, then O^T[d-slice, all heads] += C^T . P^T. The
      // smaller operand set (d-tiles or head blocks) is held in registers.
      typedef __attribute__((__vector_size__(4 * sizeof(short)))) short s4;
      auto load_va = [&](int a) __attribute__((always_inline)) {
        const int o = tr_row + (((2 * (a & 3)) ^ tr_x) + 8 * (a >> 2)) * 16;
        const s4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) s4 *)(cur + o));
        const s4 hi =
            __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) s4 *)(cur + o + HALF));
        return __builtin_bit_cast(bf16x8, __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7));
      };
      float crs[NHB];  // rescale factors of heads 16 c + col, one LDS read batch
#pragma unroll
      for (int c = 0; c < NHB; ++c) crs[c] = corr_s[col * NHB + c];
      auto rescale = [&](int c) __attribute__((always_inline)) {
        const float cr = crs[c];
        if (__builtin_amdgcn_ballot_w64(cr != 1.f)) {
#pragma unroll
          for (int a = 0; a < NDT; ++a)
#pragma unroll
            for (int i = 0; i < 4; ++i) acc[a][c][i] *= cr;
        }
      };
      auto load_p = [&](int c) __attribute__((always_inline)) {
        return __builtin_bit_cast(bf16x8, *reinterpret_cast<const u32x4 *>(pt + c * 1024 + pt_w));
      };
      if constexpr (NDT <= NHB) {
        bf16x8 va[NDT];
#pragma unroll
        for (int a = 0; a < NDT; ++a) va[a] = load_va(a);
#pragma unroll
        for (int c = 0; c < NHB; ++c) {
          rescale(c);
          const bf16x8 pb = load_p(c);
#pragma unroll
          for (int a = 0; a < NDT; ++a)
            acc[a][c] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(va[a], pb, acc[a][c], 0, 0, 0);
        }
      } else {
        bf16x8 pb[NHB];
#pragma unroll
        for (int c = 0; c < NHB; ++c) {
          rescale(c);
          pb[c] = load_p(c);
        }
#pragma unroll
        for (int a = 0; a < NDT; ++a) {
          const bf16x8 va = load_va(a);
#pragma unroll
          for (int c = 0; c < NHB; ++c)
            acc[a][c] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(va, pb[c], acc[a][c], 0, 0, 0);
        }
      }
    }
  };

  for (int s = 0; s < nsteps; s += 3) {
    step(s, buf0, buf2);
    if (s + 1 < nsteps) step(s + 1, buf1, buf0);
    if (s + 2 < nsteps) step(s + 2, buf2, buf1);
  }

  // ---- epilogue: per-head denominators and maxima through LDS.
#pragma unroll
  for (int hb = 0; hb < HPB; ++hb) {
    float l = l_run[hb] + __shfl_xor(l_run[hb], 16, 64);
    l += __shfl_xor(l, 32, 64);
    if (grp == 0) {
      const int h = 16 * (wave * HPB + hb) + col;
      lsum_s[h] = l;
      mrun_s[h] = m_run[hb];
    }
  }
  __syncthreads();
#pragma unroll
  for (int c = 0; c < NHB; ++c) {
    const int hl = 16 * c + col, h = hbase + hl;
    const float lh = lsum_s[hl];
#pragma unroll
    for (int a = 0; a < NDT; ++a) {
      const int d0 = wave * DSL + 16 * a + 4 * grp;
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
      part_ml[2 * row] = mrun_s[hl];
      part_ml[2 * row + 1] = lh;
    }
  }
}

// Blocks a partition of p tokens can touch: partitions start on a multiple
// of the 32-token step, so at most BS - 32 tokens into a block (0 for BS 16).
static int mla_partition_blocks(int p, int BS) {
  const int lead = BS > mla::STEP ? BS - mla::STEP : 0;
  return (p + lead + BS - 1) / BS;
}

// Head groups per (sequence, partition): 128 heads run as two workgroups of
// 64 (4 waves, one per SIMD), every smaller count as one.
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

extern "C" int64_t wkv_mla_workspace_size(int32_t batch, int32_t num_heads, int32_t kv_lora_rank,
                                          int32_t max_seq_len, int32_t partition_size) {
  if (batch < 0 || num_heads <= 0 || kv_lora_rank <= 0 || max_seq_len < 0 || partition_size < 0) return -1;
  if (partition_size == 0) partition_size = mla::STEP;  // the smallest partition the library picks by itself
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
  float *part_o = static_cast<float *>(workspace);
  float *part_ml = part_o ? part_o + static_cast<int64_t>(batch) * num_heads * max_parts * 512 : nullptr;
  const float scale_log2 = scale * 1.4426950408889634f;
  auto s = static_cast<hipStream_t>(stream);
  const int HG = mla_head_groups(num_heads);
  const int64_t items = static_cast<int64_t>(batch) * max_parts;
  const int64_t wgs = 8 * HG * ((items + 7) / 8);
  WKV_CHECK_ARG(wgs <= 0x7fffffff && items <= 0x7fffffff, "MLA grid too large");
  const dim3 grid(static_cast<unsigned>(wgs));
  auto lat = static_cast<const uint16_t *>(cache->latent);
  auto qn = static_cast<const uint16_t *>(q_nope);
  auto qpp = static_cast<const uint16_t *>(q_pe);
  auto oo = static_cast<uint16_t *>(out);
#define WKV_MLA(NWv, HPBv)                                                                                       \
  decode_mla_kernel<NWv, HPBv><<<grid, 64 * NWv, 0, s>>>(lat, qn, qn_stride_b, qn_stride_h, qpp, qp_stride_b,   \
                                                         qp_stride_h, oo, part_o, part_ml, block_table, bt_stride, \
                                                         max_blocks_per_seq, max_seq, seq_lens, BS,              \
                                                         cache->num_blocks, scale_log2, partition_size, max_parts, \
                                                         num_heads, batch)
  switch (num_heads) {
    case 16: WKV_MLA(1, 1); break;
    case 32: WKV_MLA(2, 1); break;
    default: WKV_MLA(4, 1); break;  // 64 heads, or 128 as two head groups
  }
#undef WKV_MLA
  WKV_CHECK_LAUNCH("wkv_paged_decode_mla");
  if (max_parts > 1) {
    mla_merge_kernel<<<dim3(static_cast<unsigned>((num_heads + 1) / 2), static_cast<unsigned>(batch)), 256, 0, s>>>(
        part_o, part_ml, oo, seq_lens, max_seq, num_heads, partition_size, max_parts);
    WKV_CHECK_LAUNCH("wkv_paged_decode_mla merge");
  }
  return WKV_OK;
}
