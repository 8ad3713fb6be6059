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
// of a workgroup stream the same key tiles. Every query tile of a (sequence,
// KV head) re-reads that head's keys, so the 1-D grid sends all of them to
// one XCD (the dispatcher deals workgroup i to XCD i mod 8): the keys are
// served from that XCD's L2 instead of being fetched by all eight. The
// latest (most expensive, causally) query tiles are dispatched first.
// Keys are streamed in 16-token tiles copied once per workgroup into LDS by
// LDS-DMA. bf16 caches: four buffers, a pair of tiles attended at once
// (attend_pair: one row maximum per 32 keys, 16x16x32 PV products) while the
// next pair is in flight. fp8 caches: three buffers, two tiles in flight while
// the waves attend the third with the decode kernels' tile arithmetic
// (gqa_tiles.h). Tiles on the causal diagonal mask per lane (column). Every
// wave finishes its rows: no split-K, no workspace.
#include "gqa_tiles.h"
#include "lds_dma.h"

#include <type_traits>

namespace wkv {

constexpr int kPrefillWaves = 4;

// One 16-token key tile of one (block, KV head) in LDS: K as the cache holds
// it, [D/x chunks][16 tokens][16 bytes]; fp8 V as the cache holds it, [D rows]
// [16 tokens]; bf16 V as [2 token octets][D rows][8 tokens] (16-byte pieces,
// so the copy still moves whole pieces). A lane's MFMA operand is one LDS read
// (K: 16 bytes of chunk 4j+grp, token col; bf16 V: tokens 4grp..4grp+3 of row
// 16n+col, 8 bytes at a 16-byte stride across the lanes -- at the cache's
// 32-byte row stride those reads conflicted on the LDS banks; fp8 V: the whole
// row 64j+16grp+col).
template <int D, bool FP8>
struct LdsTile {
  static constexpr int ESZ = FP8 ? 1 : 2;
  static constexpr int KB = D * 16 * ESZ;  // K bytes
  static constexpr int VB = D * 16 * ESZ;  // V bytes
  static constexpr int BYTES = KB + VB;
  static constexpr int PIECES = BYTES / 16;  // 16-byte pieces
  static constexpr int PER_THREAD = (PIECES + 64 * kPrefillWaves - 1) / (64 * kPrefillWaves);
  static constexpr bool EVEN = PIECES % (64 * kPrefillWaves) == 0;  // else the last round is partial
  // A wave issues PER_THREAD copies per tile, or none (its waits count on it).
  static_assert(EVEN || PIECES < 64 * kPrefillWaves, "copies per wave: PER_THREAD or 0");
  static_assert(PIECES % 64 == 0, "whole wave instructions");
};

// Global address of 16-byte piece p of the tile (tokens o0..o0+15 of block
// blk, KV head kvh) and its LDS offset (= 16 p).
template <int D, bool FP8>
__device__ __forceinline__ const uint8_t *tile_piece(const uint8_t *kc, const uint8_t *vc, int64_t rbase, int o0,
                                                     int BS, int p) {
  using T = LdsTile<D, FP8>;
  if (p < T::KB / 16) {  // K chunk c, token m: 16 bytes at ((c*BS + o0 + m) * 16) of the region
    const int c = p >> 4, m = p & 15;
    return kc + rbase + (static_cast<int64_t>(c) * BS + o0 + m) * 16;
  }
  // V row d: the 16 tokens are 32 (bf16) or 16 (fp8) contiguous bytes;
  // bf16 piece v holds octet v / D of row v % D
  const int v = p - T::KB / 16;
  const int d = FP8 ? v : v % D, half = FP8 ? 0 : v / D;
  return vc + rbase + (static_cast<int64_t>(d) * BS + o0) * T::ESZ + half * 16;
}

// LDS tile buffers: fp8, one attended and two in flight; bf16, a pair
// attended and the next pair in flight.
template <bool FP8>
constexpr int prefill_bufs() {
  return FP8 ? 3 : 4;
}

// Zeroes the bf16 V values of the tile slots at or past `valid` (4 tokens
// 4 grp .. 4 grp + 3 of one d row): a slot outside the sequence may hold NaN.
__device__ __forceinline__ u32x2 mask_v4(u32x2 v, int valid, int grp) {
#pragma unroll
  for (int e = 0; e < 4; ++e)
    if (4 * grp + e >= valid) v[e >> 1] &= (e & 1) ? 0x0000FFFFu : 0xFFFF0000u;
  return v;
}

// Two 16-key tiles of bf16 online-softmax attention at once: one row maximum,
// one rescale test, and the PV products as 16x16x32 MFMAs over the 32 keys --
// half the PV instructions of two 16-key steps. The PV product's k slots
// 8 grp .. 8 grp + 3 hold tile a's keys 4 grp .. 4 grp + 3 and slots
// 8 grp + 4 .. 8 grp + 7 tile b's: P and V are packed the same way, and the
// sum over k does not depend on which key a slot carries. lim_a / lim_b: the
// keys of each tile this lane's column sees (0..16, the causal diagonal). The
// V operands are read from the tiles' LDS copies (lva, lvb) as each PV
// product needs them, so they are not held through the softmax.
template <int D>
__device__ __forceinline__ void attend_pair(DecodeState<D, false> &st, const Tile<D, false> &ta,
                                            const Tile<D, false> &tb, const uint8_t *lva, const uint8_t *lvb,
                                            const bf16x8 *qop, float scale_log2, int col, int grp, int lim_a,
                                            int lim_b) {
  floatx4 sa = {0.f, 0.f, 0.f, 0.f}, sb = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int j = 0; j < D / 32; ++j) {
    sa = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, ta.k[j]), qop[j], sa, 0, 0, 0);
    sb = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, tb.k[j]), qop[j], sb, 0, 0, 0);
  }
  const int ca = ta.valid < lim_a ? ta.valid : lim_a;
  const int cb = tb.valid < lim_b ? tb.valid : lim_b;
  float sv[8];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    sv[i] = 4 * grp + i < ca ? sa[i] * scale_log2 : -INFINITY;
    sv[4 + i] = 4 * grp + i < cb ? sb[i] * scale_log2 : -INFINITY;
  }
  const float mt = row_max4(fmaxf(fmaxf(fmaxf(sv[0], sv[1]), fmaxf(sv[2], sv[3])),
                                  fmaxf(fmaxf(sv[4], sv[5]), fmaxf(sv[6], sv[7]))));
  // st.m is the reference maximum (-inf until the first attended token).
  const bool move = mt > st.m + SOFTMAX_TAU;
  const float m_new = move ? mt : st.m;
  const float corr = (move && st.m != -INFINITY) ? fast_exp2(st.m - m_new) : 1.f;
  const float m_use = (m_new == -INFINITY) ? 0.f : m_new;
  float p[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) p[i] = fast_exp2(sv[i] - m_use);
  st.l = st.l * corr + (((p[0] + p[1]) + (p[2] + p[3])) + ((p[4] + p[5]) + (p[6] + p[7])));
  st.m = m_new;
  if (__any(corr != 1.f)) {  // a reference maximum moved for some head: rescale
#pragma unroll
    for (int n = 0; n < D / 16; ++n) {
#pragma unroll
      for (int i = 0; i < 4; ++i) st.o[n][i] *= corr;
    }
  }
  const u32x4 pb = {pack_bf16x2(p[0], p[1]), pack_bf16x2(p[2], p[3]), pack_bf16x2(p[4], p[5]),
                    pack_bf16x2(p[6], p[7])};
  const bf16x8 pop = __builtin_bit_cast(bf16x8, pb);
#pragma unroll
  for (int n = 0; n < D / 16; ++n) {
    const int off = ((grp >> 1) * D + 16 * n + col) * 16 + (grp & 1) * 8;
    u32x2 va = *reinterpret_cast<const u32x2 *>(lva + off), vb = *reinterpret_cast<const u32x2 *>(lvb + off);
    if (ta.valid < 16) va = mask_v4(va, ta.valid, grp);  // uniform: a partial tile
    if (tb.valid < 16) vb = mask_v4(vb, tb.valid, grp);
    const u32x4 v8 = {va[0], va[1], vb[0], vb[1]};
    st.o[n] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, v8), pop, st.o[n], 0, 0, 0);
  }
}

template <int D, bool FP8>
__global__ __launch_bounds__(64 * kPrefillWaves) void prefill_gqa_kernel(
    const uint8_t *__restrict__ kc, const uint8_t *__restrict__ vc, const float *__restrict__ ks,
    const float *__restrict__ vs, const uint16_t *__restrict__ q, int64_t q_st, int64_t q_sh,
    uint16_t *__restrict__ out, int64_t o_st, int64_t o_sh, const int32_t *__restrict__ cu_q,
    const int32_t *__restrict__ seq_lens, const int32_t *__restrict__ bt, int64_t bt_stride, int Mb, int max_seq,
    int Hkv, int G, int n_hg, int BS, int64_t NB, float scale_log2, int n_qt, int n_items) {
  using LT = LdsTile<D, FP8>;
  constexpr int NBUF = prefill_bufs<FP8>();
  __shared__ __attribute__((aligned(16))) uint8_t lds[NBUF][LT::BYTES];
  // Linear id = ((item / 8) * n_qt + (n_qt - 1 - qt)) * 8 + item % 8, item =
  // (sequence, KV head, head group): the XCD (id % 8) depends on the item only.
  const int id = blockIdx.x;
  const int item = (id / (8 * n_qt)) * 8 + (id & 7);
  const int qt = __builtin_amdgcn_readfirstlane(n_qt - 1 - (id / 8) % n_qt);
  if (item >= n_items) return;
  const int b = __builtin_amdgcn_readfirstlane(item / (Hkv * n_hg));
  const int kvh = __builtin_amdgcn_readfirstlane((item / n_hg) % Hkv);
  const int hg = item % n_hg;
  const int wave = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x >> 6));
  const int lane = threadIdx.x & 63, col = lane & 15, grp = lane >> 4;
  const int q0 = cu_q[b];
  const int qlen = cu_q[b + 1] - q0;
  int L = seq_lens[b];
  L = L < max_seq ? L : max_seq;
  const int t0 = qt * 16;
  if (t0 >= qlen) return;  // the whole workgroup leaves together
  const int h_local = hg * kPrefillWaves + wave;
  const bool active = h_local < G;  // an idle wave still loads its share of every tile
  const int h = kvh * G + (active ? h_local : 0);
  const int ctx = L - qlen;  // position of new token 0 (negative only for inconsistent inputs)
  const int tok = t0 + col;
  const bool valid = active && tok < qlen;
  const int pos = ctx + tok;  // this column's position; it sees keys [0, pos]

  bf16x8 qop[D / 32];
  load_q<D, FP8>(qop, q + static_cast<int64_t>(q0 + (tok < qlen ? tok : t0)) * q_st + static_cast<int64_t>(h) * q_sh,
                 valid, grp);
  DecodeState<D, FP8> st;
#pragma unroll
  for (int n = 0; n < D / 16; ++n) st.o[n] = floatx4{0.f, 0.f, 0.f, 0.f};
  st.m = -INFINITY;
  st.l = 0.f;

  // Keys up to the tile's last query: [0, kend), in 16-token tiles.
  const int last = (t0 + 16 < qlen ? t0 + 16 : qlen) - 1;
  const int kend = ctx + last + 1;
  const int n_tiles = kend > 0 ? (kend + 15) / 16 : 0;
  const int region = D * BS * LT::ESZ;
  // Tile i's block (a wave-uniform table read: a scalar load, which waits on
  // its own counter and never on the tile copies in flight), region base and
  // position.
  auto tile_src = [&](int i, int64_t &rbase, int &o0, int &blk_ok, float &ksc, float &vsc) {
    const int ts = 16 * i;
    const int bi = ts / BS;
    int blk = bi < Mb ? bt[b * bt_stride + bi] : -1;
    blk_ok = (blk >= 0 && blk < NB) ? 1 : 0;
    if (!blk_ok) blk = 0;
    rbase = static_cast<int64_t>(__builtin_amdgcn_readfirstlane(blk * Hkv + kvh)) * region;
    o0 = ts % BS;
    ksc = vsc = 1.f;
    if constexpr (FP8) {
      ksc = ks[static_cast<int64_t>(blk) * Hkv + kvh];
      vsc = vs[static_cast<int64_t>(blk) * Hkv + kvh];
    }
  };

  // Tiles are copied HBM -> LDS by LDS-DMA (no register staging): wave w's
  // k-th copy moves pieces 256 k + 64 w .. + 63, lane i piece 256 k + 64 w + i,
  // to LDS offset 16 * piece. Tile i + 2 is issued at the start of iteration i
  // into the buffer tile i - 1 left; before the barrier that publishes tile
  // i + 1 each wave waits for its own copies of it.
  const int wave_base = 64 * wave;
  int okr[NBUF];
  float kscr[NBUF], vscr[NBUF];
  auto issue = [&](int i, int bi) {
    int64_t rbase;
    int o0;
    tile_src(i, rbase, o0, okr[bi], kscr[bi], vscr[bi]);
    const uint32_t dst = lds_addr(&lds[bi][0]);
#pragma unroll
    for (int k = 0; k < LT::PER_THREAD; ++k) {
      const int p0 = 256 * k + wave_base;  // uniform: this wave instruction's first piece
      if (LT::EVEN || p0 < LT::PIECES)
        copy16_to_lds(tile_piece<D, FP8>(kc, vc, rbase, o0, BS, p0 + lane),
                      __builtin_amdgcn_readfirstlane(dst + 16 * p0));
    }
  };
  // Tile i from LDS buffer bi into registers (V too unless !WITH_V); its
  // column limit in `lim`.
  auto read_tile = [&](int i, int bi, Tile<D, FP8> &t, int &lim, auto with_v) {
    const uint8_t *lk = &lds[bi][0];
    const uint8_t *lv = &lds[bi][LT::KB];
#pragma unroll
    for (int j = 0; j < Tile<D, FP8>::NK; ++j)
      t.k[j] = *reinterpret_cast<const u32x4 *>(lk + ((4 * j + grp) * 16 + col) * 16);
    if constexpr (FP8) {
#pragma unroll
      for (int j = 0; j < Tile<D, FP8>::NPV / 4; ++j)
        t.v4[j] = *reinterpret_cast<const u32x4 *>(lv + (64 * j + 16 * grp + col) * 16);
    } else if constexpr (decltype(with_v)::value) {
#pragma unroll
      for (int n = 0; n < Tile<D, FP8>::NPV; ++n)
        t.v[n] = *reinterpret_cast<const u32x2 *>(lv + ((grp >> 1) * D + 16 * n + col) * 16 + (grp & 1) * 8);
    }
    const int ts = 16 * i;
    t.ts = ts;
    t.valid = (i < n_tiles && okr[bi]) ? ((kend - ts) < 16 ? (kend - ts) : 16) : 0;
    t.ksc = kscr[bi];
    t.vsc = vscr[bi];
    lim = pos - ts + 1;  // keys of the tile this column sees
    lim = lim < 0 ? 0 : (lim > 16 ? 16 : lim);
  };
  auto attend = [&](int i, int bi) {
    Tile<D, FP8> t;
    int lim;
    read_tile(i, bi, t, lim, std::true_type{});
    if (t.valid > 0) attend_tile<D, FP8, true>(st, t, qop, scale_log2, grp, lim);
  };

  if constexpr (!FP8) {
    // bf16: tiles in pairs. Pair j sits in buffers 2 (j & 1), +1; the next
    // pair's copies go out before this one is attended (its buffers were left
    // by pair j - 1 at the last barrier) and land before the next barrier.
    if (n_tiles > 0) {
      issue(0, 0);
      if (n_tiles > 1) issue(1, 1);
      wait_vmcnt<0>();
      barrier_lds();
      for (int j = 0; 2 * j < n_tiles; ++j) {
        const int cur = 2 * (j & 1), nxt = 2 - cur;
        if (2 * j + 2 < n_tiles) issue(2 * j + 2, nxt);
        if (2 * j + 3 < n_tiles) issue(2 * j + 3, nxt + 1);
        if (active) {
          Tile<D, FP8> ta, tb;
          int la, lb;
          read_tile(2 * j, cur, ta, la, std::false_type{});
          read_tile(2 * j + 1, cur + 1, tb, lb, std::false_type{});  // past the end: valid 0, all masked
          if (ta.valid > 0 || tb.valid > 0)
            attend_pair<D>(st, ta, tb, &lds[cur][LT::KB], &lds[cur + 1][LT::KB], qop, scale_log2, col, grp, la, lb);
        }
        wait_vmcnt<0>();  // the next pair landed
        barrier_lds();    // ... for every wave; every wave is done with this pair
      }
    }
  } else if (n_tiles > 0) {
    issue(0, 0);
    if (n_tiles > 1) {
      issue(1, 1);
      wait_vmcnt<LT::PER_THREAD>();  // tile 0 landed
    } else {
      wait_vmcnt<0>();
    }
    barrier_lds();
    int bi = 0;  // buffer of tile i
    for (int i = 0; i < n_tiles; ++i) {
      const int b2 = bi == 0 ? 2 : bi - 1;  // (i + 2) mod 3: the buffer tile i - 1 left
      const bool more = i + 2 < n_tiles;
      if (more) issue(i + 2, b2);
      if (active) attend(i, bi);
      if (more)
        wait_vmcnt<LT::PER_THREAD>();  // tile i + 1 landed, tile i + 2 may be in flight
      else
        wait_vmcnt<0>();
      barrier_lds();  // tile i + 1 visible; every wave is done with tile i
      bi = bi == 2 ? 0 : bi + 1;
    }
  }
  if (!valid) return;
  float l = st.l + __shfl_xor(st.l, 16, 64);
  l += __shfl_xor(l, 32, 64);
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

// ---------------------------------------------------------------------------
// Pair slots of the bf16 prefill's LDS ring: pairs of 16-token tiles in
// flight = slots - 1.
constexpr int kPrefillPairSlots = 2;

// Waits until at most min(t, T) tiles' copies (PT per tile) of this wave are
// pending (t uniform).
template <int PT, int T>
__device__ __forceinline__ void wait_tiles_pending(int t) {
  if constexpr (T > 0) {
    if (t >= T) {
      wait_vmcnt<T * PT>();
      return;
    }
    wait_tiles_pending<PT, T - 1>(t);
  } else {
    wait_vmcnt<0>();
  }
}

// bf16 caches: QB blocks of 32 queries per wave on 32x32x16 MFMAs.
//
// Workgroup (32 QB-token query tile, KV head x group of four query heads,
// sequence), four waves, one query head each; key tiles as above (pairs of
// 16-token LDS tiles, LDS-DMA, a ring of kPrefillPairSlots pairs), 32 keys per
// step. Per step and query block:
//   S^T[32 keys, 32 queries] = K Q^T     D/16 MFMAs 32x32x16 (A: 16 bytes of
//                                        one key row from LDS, B: Q^T held in
//                                        registers for the whole kernel)
//   O^T[D, 32 queries] += V^T P^T       2 D/32 MFMAs 32x32x16
// Every K read from LDS feeds the QB blocks' QK products, which form QB
// independent accumulation chains: with QB = 2 the matrix core has a second
// chain to work on while a product's result is pending, and the K reads and
// barriers per MFMA halve. Each block then runs its softmax and PV products
// (V read per block: P for one block at a time keeps the registers within two
// waves per SIMD).
// Lane l holds query l % 32 of each block in both accumulators: 16 scores
// (rows 8 (r/4) + 4 (l/32) + r % 4 of S^T) and 16 outputs per 32 d. S^T's row
// i carries key kperm(i) (rows 4..7 and 8..11 of each 16 swapped), so score r
// of lane l is key 16 (r/8) + 8 (l/32) + r % 8: the scores a lane holds after
// the softmax are exactly its PV B operand (element e of step s = score
// 8 s + e), and V^T's A operand -- keys 16 s + 8 (l/32) + 0..7 of one d row --
// is one 16-byte LDS read in the [octet][D][8 tokens] V layout. The softmax
// (per 1,024 scores about a hundred VALU instructions: the scale folded into
// the exponent's FMA, one row maximum across the two lane halves, lazy rescale
// as in the decode kernels) runs per block.
template <int D, int QB>
__global__ __launch_bounds__(64 * kPrefillWaves) void prefill_gqa32_kernel(
    const uint8_t *__restrict__ kc, const uint8_t *__restrict__ vc, const uint16_t *__restrict__ q, int64_t q_st,
    int64_t q_sh, uint16_t *__restrict__ out, int64_t o_st, int64_t o_sh, const int32_t *__restrict__ cu_q,
    const int32_t *__restrict__ seq_lens, const int32_t *__restrict__ bt, int64_t bt_stride, int Mb, int max_seq,
    int Hkv, int G, int n_hg, int BS, int64_t NB, float scale_log2, int n_qt, int n_items) {
  using LT = LdsTile<D, false>;
  static_assert(LT::EVEN, "every wave issues PER_THREAD copies per tile (the waits count on it)");
  constexpr int NPAIR = kPrefillPairSlots;
  constexpr int NBUF = 2 * NPAIR;
  constexpr int QT = 32 * QB;  // query tokens per workgroup
  __shared__ __attribute__((aligned(16))) uint8_t lds[NBUF][LT::BYTES];
  const int id = blockIdx.x;
  const int item = (id / (8 * n_qt)) * 8 + (id & 7);
  const int qt = __builtin_amdgcn_readfirstlane(n_qt - 1 - (id / 8) % n_qt);
  if (item >= n_items) return;
  const int b = __builtin_amdgcn_readfirstlane(item / (Hkv * n_hg));
  const int kvh = __builtin_amdgcn_readfirstlane((item / n_hg) % Hkv);
  const int hg = item % n_hg;
  const int wave = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x >> 6));
  const int lane = threadIdx.x & 63, n = lane & 31, hh = lane >> 5;
  const int q0 = cu_q[b];
  const int qlen = cu_q[b + 1] - q0;
  int L = seq_lens[b];
  L = L < max_seq ? L : max_seq;
  const int t0 = qt * QT;
  if (t0 >= qlen) return;  // the whole workgroup leaves together
  const int h_local = hg * kPrefillWaves + wave;
  const bool active = h_local < G;  // an idle wave still copies its share of every tile
  const int h = kvh * G + (active ? h_local : 0);
  const int ctx = L - qlen;

  // Q^T operand j of block qbi: lane l holds d = 16 j + 8 (l/32) .. + 7 of query 32 qbi + l % 32.
  bf16x8 qb[QB][D / 16];
#pragma unroll
  for (int qbi = 0; qbi < QB; ++qbi) {
    const int tok = t0 + 32 * qbi + n;
    const bool valid = active && tok < qlen;
    const uint16_t *qp = q + static_cast<int64_t>(q0 + (tok < qlen ? tok : t0)) * q_st + static_cast<int64_t>(h) * q_sh;
#pragma unroll
    for (int j = 0; j < D / 16; ++j) {
      u32x4 w = *reinterpret_cast<const u32x4 *>(qp + 16 * j + 8 * hh);
      if (!valid) w = u32x4{0u, 0u, 0u, 0u};
      qb[qbi][j] = __builtin_bit_cast(bf16x8, w);
    }
  }
  floatx16 o[QB][D / 32];
#pragma unroll
  for (int qbi = 0; qbi < QB; ++qbi)
#pragma unroll
    for (int c = 0; c < D / 32; ++c)
#pragma unroll
      for (int r = 0; r < 16; ++r) o[qbi][c][r] = 0.f;
  float m_ref[QB], l_part[QB];
#pragma unroll
  for (int qbi = 0; qbi < QB; ++qbi) {
    m_ref[qbi] = -INFINITY;
    l_part[qbi] = 0.f;
  }

  const int last = (t0 + QT < qlen ? t0 + QT : qlen) - 1;
  const int kend = ctx + last + 1;  // keys [0, kend)
  const int n_tiles = kend > 0 ? (kend + 15) / 16 : 0;
  const int region = D * BS * LT::ESZ;
  const int wave_base = 64 * wave;
  // This lane's piece of copy k of every tile sits at a fixed offset from the
  // (block, head) region plus the tile's first token; whether the piece is K or
  // V depends on the wave and k only.
  // pbase[k]: the cache (K or V) plus this lane's offset; the tile's first
  // token o0 adds o0 << oshift[k] (16-byte K rows, 2-byte V elements).
  const uint8_t *pbase[LT::PER_THREAD];
  int oshift[LT::PER_THREAD];
#pragma unroll
  for (int k = 0; k < LT::PER_THREAD; ++k) {
    const int p = 256 * k + wave_base + lane;
    if (256 * k + wave_base < LT::KB / 16) {  // K chunk c, token m: ((c BS + m) 16)
      pbase[k] = kc + ((p >> 4) * BS + (p & 15)) * 16;
      oshift[k] = 4;
    } else {  // V row d, octet o: (d BS) 2 + 16 o
      const int v = p - LT::KB / 16;
      pbase[k] = vc + (v % D) * BS * 2 + (v / D) * 16;
      oshift[k] = 1;
    }
  }
  // Block ids of blocks wbase .. wbase + 63 of the sequence, lane i holding
  // block wbase + i, picked per tile with readlane (no memory access per tile).
  const int32_t *btrow = bt + b * bt_stride;
  int wbase = 0;
  int win = load_i32_drained(btrow, lane, Mb);
  int okmask = 0;  // bit bi: buffer bi holds a mapped block
  // Tiles are issued in order 0, 1, 2, ...: the next one's block (within the
  // window) and first token in it advance by 16 tokens per call (BS is a
  // multiple of 16: one block per tile), with no division.
  int nbix = 0, no0 = 0;
  auto issue = [&](int bi) {
    const int o0 = no0;
    int bix = nbix;
    no0 += 16;
    if (no0 == BS) {
      no0 = 0;
      ++nbix;
    }
    if (bix == 64) {  // uniform: the next 64 blocks (once per 64 blocks; its wait drains the copies)
      wbase += 64;
      nbix -= 64;
      bix = 0;
      win = load_i32_drained(btrow, wbase + lane, Mb);
    }
    int blk = __builtin_amdgcn_readlane(win, bix);
    const bool ok = blk >= 0 && blk < NB;
    okmask = ok ? (okmask | (1 << bi)) : (okmask & ~(1 << bi));
    if (!ok) blk = 0;
    const int64_t rbase = static_cast<int64_t>(blk * Hkv + kvh) * region;
    const uint32_t dst = lds_addr(&lds[bi][0]);
#pragma unroll
    for (int k = 0; k < LT::PER_THREAD; ++k) {
      const int p0 = 256 * k + wave_base;  // uniform
      if (LT::EVEN || p0 < LT::PIECES)
        copy16_to_lds(pbase[k] + (rbase + (o0 << oshift[k])), __builtin_amdgcn_readfirstlane(dst + 16 * p0));
    }
  };
  // A row n of S^T carries key kperm(n) of the pair.
  const int kn = (n & 16) | (((n >> 2) & 3) == 1 ? (n & 3) + 8 : ((n >> 2) & 3) == 2 ? (n & 3) + 4 : (n & 15));

  if (n_tiles > 0) {
    // Pair p sits in buffers 2 (p mod NPAIR), +1. Pairs 0 .. NPAIR - 2 go out
    // first; step j issues pair j + NPAIR - 1 into the slot pair j - 1 left
    // (every wave was done with it at the last barrier), so a pair's copies
    // have NPAIR - 1 steps to land.
    for (int t = 0; t < 2 * (NPAIR - 1) && t < n_tiles; ++t) issue(t);
    wait_tiles_pending<LT::PER_THREAD, 2 * (NPAIR - 2)>((n_tiles < 2 * (NPAIR - 1) ? n_tiles : 2 * (NPAIR - 1)) -
                                                        (n_tiles < 2 ? n_tiles : 2));  // pair 0 landed
    barrier_lds();
    int cur = 0;  // buffer of pair j's first tile
    for (int j = 0; 2 * j < n_tiles; ++j) {
      const int nxt = cur == 0 ? NBUF - 2 : cur - 2;
      const int ti = 2 * (j + NPAIR - 1);
      if (ti < n_tiles) issue(nxt);
      if (ti + 1 < n_tiles) issue(nxt + 1);
      const int kb = 32 * j;  // position of the pair's first key
      // keys of each half the pair holds (0 when the half lies past kend or its block is unmapped)
      const int va = (((okmask >> cur) & 1) && kb < kend) ? (kend - kb < 16 ? kend - kb : 16) : 0;
      const int vb =
          (2 * j + 1 < n_tiles && ((okmask >> (cur + 1)) & 1)) ? (kend - kb - 16 < 16 ? kend - kb - 16 : 16) : 0;
      if (active && (va > 0 || vb > 0)) {
        floatx16 sacc[QB];
#pragma unroll
        for (int qbi = 0; qbi < QB; ++qbi)
#pragma unroll
          for (int r = 0; r < 16; ++r) sacc[qbi][r] = 0.f;
        const uint8_t *lk = &lds[kn < 16 ? cur : cur + 1][0] + (kn & 15) * 16;
#pragma unroll
        for (int jj = 0; jj < D / 16; ++jj) {
          const bf16x8 a = __builtin_bit_cast(bf16x8, *reinterpret_cast<const u32x4 *>(lk + (2 * jj + hh) * 256));
#pragma unroll
          for (int qbi = 0; qbi < QB; ++qbi)
            sacc[qbi] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, qb[qbi][jj], sacc[qbi], 0, 0, 0);
        }
        // Per block: softmax, then its PV products (its P never waits in registers
        // for the other block's softmax).
#pragma unroll
        for (int qbi = 0; qbi < QB; ++qbi) {
          // Score r of this lane (raw, unscaled): key kb + 16 (r/8) + 8 hh + r % 8;
          // the softmax works on the accumulator in place.
          floatx16 &sv = sacc[qbi];
          const int min_pos = ctx + t0 + 32 * qbi;  // the block's smallest query position
          if (!(va == 16 && vb == 16 && kb + 31 <= min_pos)) {  // uniform: masks in this pair
            const int pos = min_pos + n;  // this lane's query sees keys [0, pos]
#pragma unroll
            for (int r = 0; r < 16; ++r) {
              const int kr = 16 * (r / 8) + 8 * hh + (r % 8);  // key within the pair
              const bool ok = (kr < 16 ? kr < va : kr - 16 < vb) && kb + kr <= pos;
              if (!ok) sv[r] = -INFINITY;
            }
          }
          float mt = sv[0];
#pragma unroll
          for (int r = 1; r < 16; ++r) mt = fmaxf(mt, sv[r]);
          {
            const auto x = __builtin_amdgcn_permlane32_swap(__float_as_uint(mt), __float_as_uint(mt), false, false);
            mt = fmaxf(__uint_as_float(x[0]), __uint_as_float(x[1])) * scale_log2;  // the scale is positive
          }
          const bool move = mt > m_ref[qbi] + SOFTMAX_TAU;
          const float m_new = move ? mt : m_ref[qbi];
          const float corr = (move && m_ref[qbi] != -INFINITY) ? fast_exp2(m_ref[qbi] - m_new) : 1.f;
          const float m_use = (m_new == -INFINITY) ? 0.f : m_new;
          float ps = 0.f;
#pragma unroll
          for (int r = 0; r < 16; ++r) {
            sv[r] = fast_exp2(__builtin_fmaf(sv[r], scale_log2, -m_use));  // masked: -inf -> 0
            ps += sv[r];
          }
          l_part[qbi] = l_part[qbi] * corr + ps;
          m_ref[qbi] = m_new;
          if (__any(corr != 1.f)) {
#pragma unroll
            for (int c = 0; c < D / 32; ++c)
#pragma unroll
              for (int r = 0; r < 16; ++r) o[qbi][c][r] *= corr;
          }
#pragma unroll
          for (int st = 0; st < 2; ++st) {
            const int vv = st == 0 ? va : vb;
            if (vv == 0) continue;  // uniform: a half past the keys or unmapped (its P is zero)
            const u32x4 pw = {pack_bf16x2(sv[8 * st], sv[8 * st + 1]), pack_bf16x2(sv[8 * st + 2], sv[8 * st + 3]),
                              pack_bf16x2(sv[8 * st + 4], sv[8 * st + 5]),
                              pack_bf16x2(sv[8 * st + 6], sv[8 * st + 7])};
            const bf16x8 pb = __builtin_bit_cast(bf16x8, pw);
            const uint8_t *lv = &lds[cur + st][LT::KB] + hh * D * 16;  // octet hh: keys 8 hh .. 8 hh + 7
#pragma unroll
            for (int c = 0; c < D / 32; ++c) {
              u32x4 w = *reinterpret_cast<const u32x4 *>(lv + (32 * c + n) * 16);
              if (vv < 16) {  // uniform: slots past the keys may hold NaN
#pragma unroll
                for (int e = 0; e < 8; ++e)
                  if (8 * hh + e >= vv) w[e >> 1] &= (e & 1) ? 0x0000FFFFu : 0xFFFF0000u;
              }
              o[qbi][c] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, w), pb, o[qbi][c], 0, 0, 0);
            }
          }
        }
      }
      {
        // pair j + 1 landed (the tiles of pairs j + 2 .. j + NPAIR - 1 may be in flight) ...
        const int after = n_tiles - 2 * (j + 2);
        wait_tiles_pending<LT::PER_THREAD, 2 * (NPAIR - 2)>(after < 0 ? 0 : after);
      }
      barrier_lds();  // ... for every wave; every wave is done with pair j
      cur = cur == NBUF - 2 ? 0 : cur + 2;
    }
  }
#pragma unroll
  for (int qbi = 0; qbi < QB; ++qbi) {
    const int tok = t0 + 32 * qbi + n;
    if (!active || tok >= qlen) continue;
    float l = l_part[qbi];
    {
      const auto x = __builtin_amdgcn_permlane32_swap(__float_as_uint(l), __float_as_uint(l), false, false);
      l = __uint_as_float(x[0]) + __uint_as_float(x[1]);
    }
    const float inv = l > 0.f ? 1.f / l : 0.f;
    uint16_t *op = out + static_cast<int64_t>(q0 + tok) * o_st + static_cast<int64_t>(h) * o_sh;
#pragma unroll
    for (int c = 0; c < D / 32; ++c) {
#pragma unroll
      for (int g = 0; g < 4; ++g) {  // d = 32 c + 8 g + 4 hh + 0..3
        const u32x2 w = {pack_bf16x2(o[qbi][c][4 * g] * inv, o[qbi][c][4 * g + 1] * inv),
                         pack_bf16x2(o[qbi][c][4 * g + 2] * inv, o[qbi][c][4 * g + 3] * inv)};
        *reinterpret_cast<u32x2 *>(op + 32 * c + 8 * g + 4 * hh) = w;
      }
    }
  }
}

// bf16 caches, 64 keys per step (four 16-token tiles, one copied by each
// wave). Workgroup and lanes as in prefill_gqa32_kernel with one block of 32
// queries per wave; what changes is the step. Per step and wave:
//   S^T for keys 0..31 and 32..63 of the step    two chains of D/16 MFMAs
//                                                 32x32x16 (one per half,
//                                                 interleaved: a chain never
//                                                 waits on itself)
//   one row maximum, one rescale test            over the 64 keys
//   P V^T                                        4 x D/32 MFMAs 32x32x16
//   copies of the wave's tile: V of this step,  one buffer resource per
//   K of the next                                 cache, PIECES/64 copies with
//                                                 a uniform offset each
// so the per-step costs (barrier, waits, loop and mask tests, the maximum's
// cross-lane swap) and the per-tile block lookup fall on twice the MFMAs of
// a 32-key step. Each half keeps the key permutation of the 32-key kernel
// (score r of lane l is key 16 (r/8) + 8 (l/32) + r % 8 of the half, the PV
// B operand as it stands), and the row sum is taken on the packed bf16
// probabilities the PV products consume (v_dot2c_f32_bf16 against 1.0, two
// per instruction). A block id outside [0, num_blocks) reads block 0: no
// access leaves the cache, and that sequence's output is unspecified.
// LDS: K in two step slots (the next step's K lands during this step), V in
// one (a step's V is copied at its start and lands during its QK and
// softmax; a second barrier per step separates the softmax from the PV
// products): 48 KB at d=128, so three workgroups share a CU.
template <int D>
__global__ __launch_bounds__(64 * kPrefillWaves, 3) void prefill_gqa64_kernel(
    const uint8_t *__restrict__ kc, const uint8_t *__restrict__ vc, const uint16_t *__restrict__ q, int64_t q_st,
    int64_t q_sh, uint16_t *__restrict__ out, int64_t o_st, int64_t o_sh, const int32_t *__restrict__ cu_q,
    const int32_t *__restrict__ seq_lens, const int32_t *__restrict__ bt, int64_t bt_stride, int Mb, int max_seq,
    int Hkv, int G, int n_hg, int BS, int64_t NB, float scale_log2, int n_qt, int n_items) {
  using LT = LdsTile<D, false>;
  static_assert(kPrefillWaves == 4, "one tile per wave per 64-key step");
  static_assert(LT::PIECES % 64 == 0 && LT::KB % 1024 == 0 && D % 64 == 0, "whole copies per lane");
  constexpr int KB = LT::KB, VB = LT::VB;  // bytes of one tile's K, V
  constexpr int CPT = LT::PIECES / 64;     // 16-byte copies per lane per tile
  constexpr int NK = KB / 1024;            // of which the first NK are K
  constexpr int DV = D / 64;               // V copies per token octet
  __shared__ __attribute__((aligned(16))) uint8_t ldsk[2 * 4 * KB];  // K: two steps of four tiles
  __shared__ __attribute__((aligned(16))) uint8_t ldsv[4 * VB];      // V: one step
  const int id = blockIdx.x;
  const int item = (id / (8 * n_qt)) * 8 + (id & 7);
  const int qt = __builtin_amdgcn_readfirstlane(n_qt - 1 - (id / 8) % n_qt);
  if (item >= n_items) return;
  const int b = __builtin_amdgcn_readfirstlane(item / (Hkv * n_hg));
  const int kvh = __builtin_amdgcn_readfirstlane((item / n_hg) % Hkv);
  const int hg = item % n_hg;
  const int wave = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x >> 6));
  const int lane = threadIdx.x & 63, n = lane & 31, hh = lane >> 5;
  const int q0 = cu_q[b];
  const int qlen = cu_q[b + 1] - q0;
  int L = seq_lens[b];
  L = L < max_seq ? L : max_seq;
  const int t0 = qt * 32;
  if (t0 >= qlen) return;  // the whole workgroup leaves together
  const int h_local = hg * kPrefillWaves + wave;
  const bool active = h_local < G;  // an idle wave still copies its tile of every step
  const int h = kvh * G + (active ? h_local : 0);
  const int ctx = L - qlen;

  // Q^T operand j: lane l holds d = 16 j + 8 (l/32) .. + 7 of query t0 + l % 32.
  bf16x8 qb[D / 16];
  {
    const int tok = t0 + n;
    const bool valid = active && tok < qlen;
    const uint16_t *qp = q + static_cast<int64_t>(q0 + (tok < qlen ? tok : t0)) * q_st + static_cast<int64_t>(h) * q_sh;
#pragma unroll
    for (int j = 0; j < D / 16; ++j) {
      u32x4 w = *reinterpret_cast<const u32x4 *>(qp + 16 * j + 8 * hh);
      if (!valid) w = u32x4{0u, 0u, 0u, 0u};
      qb[j] = __builtin_bit_cast(bf16x8, w);
    }
  }
  floatx16 o[D / 32];
#pragma unroll
  for (int c = 0; c < D / 32; ++c)
#pragma unroll
    for (int r = 0; r < 16; ++r) o[c][r] = 0.f;
  float m_ref = -INFINITY, l_part = 0.f;

  const int last = (t0 + 32 < qlen ? t0 + 32 : qlen) - 1;
  const int kend = ctx + last + 1;  // keys [0, kend)
  const int n_tiles = kend > 0 ? (kend + 15) / 16 : 0;
  const int n_steps = (n_tiles + 3) / 4;
  const int region = D * BS * 2;

  // Copy k of lane l moves piece p = 64 k + l of the wave's tile (LDS offset
  // 16 p). K piece p: chunk p >> 4, token p & 15, at ((p >> 4) BS + (p & 15)) 16
  // of the (block, head) K region = lane part ((l >> 4) BS + (l & 15)) 16 +
  // copy part 64 BS k. V piece v = p - KB/16: row v % D, octet v / D, at
  // (v % D) BS 2 + 16 (v / D) = lane part 2 BS l + copy part 128 BS (k' % DV) +
  // 16 (k' / DV), k' = k - NK. The tile's first token o0 goes into the base.
  const uint32_t lane_k = static_cast<uint32_t>(((lane >> 4) * BS + (lane & 15)) * 16);
  const uint32_t lane_v = static_cast<uint32_t>(lane * BS * 2);
  const int nb = static_cast<int>(NB);  // num_blocks * num_kv_heads < 2^31 (checked by the host)
  const uint32_t ldsk0 = lds_addr(ldsk), ldsv0 = lds_addr(ldsv);
  // This wave's tile of step s is tile 4 s + wave: token 64 s + 16 wave, in
  // block bix at offset o0, both advanced by 64 tokens per step.
  const int32_t *btrow = bt + b * bt_stride;
  int bix = (16 * wave) / BS;
  int o0 = 16 * wave - bix * BS;
  const int dbix = 64 / BS, do0 = 64 - dbix * BS;
  int wbase = 0;  // the window: lane i holds the id of block wbase + i
  int win = load_i32_drained(btrow, lane, Mb);
  int64_t vbase = 0;  // V of the wave's tile of the step whose K went out last: cache offset
  // K of the wave's tile of step s into K slot `slot` (and its V offset kept for issue_v)
  auto issue_k = [&](int s, int slot) {
    if (4 * s + wave < n_tiles) {  // uniform
      if (bix - wbase >= 64) {     // at most once per 64 blocks (its wait drains the copies in flight)
        wbase += 64;
        win = load_i32_drained(btrow, wbase + lane, Mb);
      }
      int blk = __builtin_amdgcn_readlane(win, bix - wbase);
      if (!(blk >= 0 && blk < nb)) blk = 0;
      const int64_t rb = static_cast<int64_t>(blk * Hkv + kvh) * region;
      vbase = rb + o0 * 2;
      // copy part of K copy k: 64 BS k (recomputed here, not held in registers)
      uint32_t kst = static_cast<uint32_t>(64 * BS);
      asm volatile("" : "+s"(kst));
      const __amdgpu_buffer_rsrc_t kr =
          __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t *>(kc + rb + o0 * 16), 0, region, kRawBufferWord3);
      const uint32_t dst = ldsk0 + static_cast<uint32_t>((4 * slot + wave) * KB);
#pragma unroll
      for (int k = 0; k < NK; ++k) buffer_copy16_to_lds(kr, lane_k, kst * k, dst + 1024 * k);
    }
    o0 += do0;
    bix += dbix;
    if (o0 >= BS) {
      o0 -= BS;
      ++bix;
    }
  };
  // V of the wave's tile of step s (whose K went out last) into the V slot
  auto issue_v = [&](int s) {
    if (4 * s + wave < n_tiles) {
      const __amdgpu_buffer_rsrc_t vr =
          __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t *>(vc + vbase), 0, region, kRawBufferWord3);
      const uint32_t dst = ldsv0 + static_cast<uint32_t>(wave * VB);
      // copy part of V copy k' = k - NK: 128 BS (k' % DV) + 16 (k' / DV)
      uint32_t vst = static_cast<uint32_t>(128 * BS);
      asm volatile("" : "+s"(vst));
#pragma unroll
      for (int k = NK; k < CPT; ++k)
        buffer_copy16_to_lds(vr, lane_v, vst * ((k - NK) % DV) + 16 * ((k - NK) / DV), dst + 1024 * (k - NK));
    }
  };
  // Row n of each half's S^T carries key kperm(n) of the half.
  const int kn = (n & 16) | (((n >> 2) & 3) == 1 ? (n & 3) + 8 : ((n >> 2) & 3) == 2 ? (n & 3) + 4 : (n & 15));
  const bf16x2 ones = __builtin_bit_cast(bf16x2, 0x3F803F80u);

  if (n_steps > 0) {
    issue_k(0, 0);
    wait_vmcnt<0>();
    barrier_lds();
    for (int s = 0; s < n_steps; ++s) {
      const int cur = s & 1;
      issue_v(s);  // its slot was left at the last barrier
      const bool k_next = s + 1 < n_steps && 4 * (s + 1) + wave < n_tiles;  // uniform
      if (s + 1 < n_steps) issue_k(s + 1, cur ^ 1);
      const int kb = 64 * s;  // position of the step's first key
      uint32_t pw[4][4];      // PV B operands, packed bf16 probabilities
      if (active) {
        floatx16 s0, s1;
#pragma unroll
        for (int r = 0; r < 16; ++r) s0[r] = s1[r] = 0.f;
        const uint8_t *lk = ldsk + (cur * 4 + (kn >> 4)) * KB + (kn & 15) * 16;
#pragma unroll
        for (int jj = 0; jj < D / 16; ++jj) {
          const bf16x8 a0 = __builtin_bit_cast(bf16x8, *reinterpret_cast<const u32x4 *>(lk + (2 * jj + hh) * 256));
          const bf16x8 a1 = __builtin_bit_cast(bf16x8, *reinterpret_cast<const u32x4 *>(lk + 2 * KB + (2 * jj + hh) * 256));
          s0 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a0, qb[jj], s0, 0, 0, 0);
          s1 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a1, qb[jj], s1, 0, 0, 0);
        }
        const int min_pos = ctx + t0;  // the smallest query position of the workgroup
        if (!(kend >= kb + 64 && kb + 63 <= min_pos)) {  // uniform: masks in this step
          // keys of the step this lane's query sees: 0 .. lim (relative to kb and
          // to this lane's key octet); past kend nothing is seen
          const int pos = min_pos + n;
          const int lim = (pos < kend - 1 ? pos : kend - 1) - kb - 8 * hh;
#pragma unroll
          for (int r = 0; r < 16; ++r) {
            if (16 * (r / 8) + (r % 8) > lim) s0[r] = -INFINITY;
            if (32 + 16 * (r / 8) + (r % 8) > lim) s1[r] = -INFINITY;
          }
        }
        if (s == 0) {  // uniform: the reference maximum starts at the first step's row maximum
          // (every query sees key 0, so it is finite)
          float mt = fmaxf(s0[0], s1[0]);
#pragma unroll
          for (int r = 1; r < 16; ++r) mt = fmaxf(mt, fmaxf(s0[r], s1[r]));
          const auto x = __builtin_amdgcn_permlane32_swap(__float_as_uint(mt), __float_as_uint(mt), false, false);
          mt = fmaxf(__uint_as_float(x[0]), __uint_as_float(x[1])) * scale_log2;  // the scale is positive
          m_ref = mt == -INFINITY ? 0.f : mt;
        }
        // Exponents against the reference maximum; their maximum (of FMA results,
        // which max3 takes as they are) says whether it must move.
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          s0[r] = __builtin_fmaf(s0[r], scale_log2, -m_ref);  // masked: -inf
          s1[r] = __builtin_fmaf(s1[r], scale_log2, -m_ref);
        }
        // two chains of max3 over the 32 exponents
        float mt0 = fmaxf(s0[0], s0[1]), mt1 = fmaxf(s1[0], s1[1]);
#pragma unroll
        for (int r = 2; r < 16; r += 2) {
          mt0 = fmaxf(fmaxf(mt0, s0[r]), s0[r + 1]);
          mt1 = fmaxf(fmaxf(mt1, s1[r]), s1[r + 1]);
        }
        float mt = fmaxf(mt0, mt1);
        {
          const auto x = __builtin_amdgcn_permlane32_swap(__float_as_uint(mt), __float_as_uint(mt), false, false);
          mt = fmaxf(__uint_as_float(x[0]), __uint_as_float(x[1]));
        }
        const bool move = mt > SOFTMAX_TAU;
        if (__any(move)) {  // rare: some row's maximum rose past the reference by 2^SOFTMAX_TAU
          const float sh = move ? mt : 0.f;
#pragma unroll
          for (int r = 0; r < 16; ++r) {
            s0[r] -= sh;
            s1[r] -= sh;
          }
          const float corr = fast_exp2(-sh);
          l_part *= corr;
          m_ref += sh;
#pragma unroll
          for (int c = 0; c < D / 32; ++c)
#pragma unroll
            for (int r = 0; r < 16; ++r) o[c][r] *= corr;
        }
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          s0[r] = fast_exp2(s0[r]);  // masked: -inf -> 0
          s1[r] = fast_exp2(s1[r]);
        }
        // Tile t = 2 half + st takes scores 8 st .. 8 st + 7 of its half, packed
        // as four words. The words stay scalars until the MFMA operand is
        // built: the dot products read them one by one (with the words as
        // elements of a 4-vector, hipcc 7.2 fed every dot product of a vector
        // its first element).
#pragma unroll
        for (int t = 0; t < 4; ++t) {
          const floatx16 &sv = t < 2 ? s0 : s1;
          const int e0 = 8 * (t & 1);
#pragma unroll
          for (int i = 0; i < 4; ++i) pw[t][i] = pack_bf16x2(sv[e0 + 2 * i], sv[e0 + 2 * i + 1]);
        }
        float ps = 0.f;
#pragma unroll
        for (int t = 0; t < 4; ++t)
#pragma unroll
          for (int i = 0; i < 4; ++i)
            ps = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, pw[t][i]), ones, ps, false);
        l_part += ps;
      }
      if (k_next)
        wait_vmcnt<NK>();  // this step's V landed (the next step's K may be in flight)
      else
        wait_vmcnt<0>();
      {
        // The slots of a partial tile past the keys may hold NaN (0 x NaN in a
        // PV product is NaN): the wave that copied the tile zeroes them, so
        // the PV products read V as it stands.
        int vt = kend - kb - 16 * wave;  // keys of this wave's tile
        vt = vt < 0 ? 0 : (vt > 16 ? 16 : vt);
        if (vt > 0 && vt < 16) {  // uniform; at most once per workgroup
#pragma unroll
          for (int i = 0; i < D / 32; ++i) {
            const int pc = 64 * i + lane;  // V piece: octet pc / D, row pc % D (8 tokens)
            const int cnt = vt - 8 * (pc / D);  // tokens of the piece that are keys
            u32x4 *ptr = reinterpret_cast<u32x4 *>(ldsv + wave * VB + pc * 16);
            u32x4 w = *ptr;
#pragma unroll
            for (int e = 0; e < 8; ++e)
              if (e >= cnt) w[e >> 1] &= (e & 1) ? 0x0000FFFFu : 0xFFFF0000u;
            *ptr = w;
          }
        }
      }
      barrier_lds();  // ... for every wave
      if (active) {
        const uint8_t *lv = ldsv + hh * D * 16 + n * 16;  // octet hh: keys 8 hh .. 8 hh + 7 of a tile
#pragma unroll
        for (int t = 0; t < 4; ++t) {
          if (kend - kb - 16 * t <= 0) continue;  // uniform: a tile past the keys (its LDS buffer is stale)
          const bf16x8 pb = __builtin_bit_cast(bf16x8, (u32x4{pw[t][0], pw[t][1], pw[t][2], pw[t][3]}));
#pragma unroll
          for (int c = 0; c < D / 32; ++c) {
            const u32x4 w = *reinterpret_cast<const u32x4 *>(lv + t * VB + 32 * c * 16);
            o[c] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, w), pb, o[c], 0, 0, 0);
          }
        }
      }
      wait_vmcnt<0>();  // the next step's K landed
      barrier_lds();    // ... for every wave; every wave is done with this step's K and V
    }
  }
  const int tok = t0 + n;
  if (!active || tok >= qlen) return;
  float l = l_part;
  {
    const auto x = __builtin_amdgcn_permlane32_swap(__float_as_uint(l), __float_as_uint(l), false, false);
    l = __uint_as_float(x[0]) + __uint_as_float(x[1]);
  }
  const float inv = l > 0.f ? 1.f / l : 0.f;
  uint16_t *op = out + static_cast<int64_t>(q0 + tok) * o_st + static_cast<int64_t>(h) * o_sh;
#pragma unroll
  for (int c = 0; c < D / 32; ++c) {
#pragma unroll
    for (int g = 0; g < 4; ++g) {  // d = 32 c + 8 g + 4 hh + 0..3
      const u32x2 w = {pack_bf16x2(o[c][4 * g] * inv, o[c][4 * g + 1] * inv),
                       pack_bf16x2(o[c][4 * g + 2] * inv, o[c][4 * g + 3] * inv)};
      *reinterpret_cast<u32x2 *>(op + 32 * c + 8 * g + 4 * hh) = w;
    }
  }
}

// Query blocks of 32 per wave of the bf16 prefill. One: at d=128 two blocks
// need 256 VGPRs (two waves per SIMD, with spills) and measured 540 against
// 420 us per layer for one block at three waves per SIMD on 8 x 2,048-token
// Qwen3-4B prompts -- the waves that hide each other's latency matter more
// than a second MFMA chain per wave.
template <int D>
constexpr int prefill_query_blocks() {
  return 1;
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
  const bool fp8 = cache->kv_dtype == WKV_KV_FP8_E4M3;
  const int n_hg = (G + kPrefillWaves - 1) / kPrefillWaves;
  const int q_tile = fp8 ? 16 : 32 * (D == 128 ? prefill_query_blocks<128>() : prefill_query_blocks<64>());
  const int n_qt = (max_query_len + q_tile - 1) / q_tile;
  const int64_t n_items = static_cast<int64_t>(batch) * Hkv * n_hg;
  const int64_t n_wg = (n_items + 7) / 8 * 8 * n_qt;
  WKV_CHECK_ARG(n_wg <= INT32_MAX, "prefill grid too large");
  const dim3 grid(static_cast<unsigned>(n_wg));
  auto s = static_cast<hipStream_t>(stream);
  auto kc = static_cast<const uint8_t *>(cache->k);
  auto vc = static_cast<const uint8_t *>(cache->v);
  auto qq = static_cast<const uint16_t *>(q);
  auto oo = static_cast<uint16_t *>(out);
  const float scale_log2 = scale * 1.4426950408889634f;
#define WKV_PREFILL(Dv)                                                                                           \
  prefill_gqa_kernel<Dv, true><<<grid, 64 * kPrefillWaves, 0, s>>>(                                              \
      kc, vc, cache->k_scale, cache->v_scale, qq, q_stride_t, q_stride_h, oo, out_stride_t, out_stride_h,       \
      cu_seqlens_q, seq_lens, block_table, bt_stride, max_blocks_per_seq, max_seq, Hkv, G, n_hg, BS,           \
      cache->num_blocks, scale_log2, n_qt, static_cast<int>(n_items))
#define WKV_PREFILL32(Dv)                                                                                         \
  prefill_gqa64_kernel<Dv><<<grid, 64 * kPrefillWaves, 0, s>>>(                                                  \
      kc, vc, qq, q_stride_t, q_stride_h, oo, out_stride_t, out_stride_h, cu_seqlens_q, seq_lens, block_table,   \
      bt_stride, max_blocks_per_seq, max_seq, Hkv, G, n_hg, BS, cache->num_blocks, scale_log2, n_qt,             \
      static_cast<int>(n_items))
  if (D == 128) {
    if (fp8) WKV_PREFILL(128); else WKV_PREFILL32(128);
  } else {
    if (fp8) WKV_PREFILL(64); else WKV_PREFILL32(64);
  }
#undef WKV_PREFILL32
#undef WKV_PREFILL
  WKV_CHECK_LAUNCH("paged prefill");
  return WKV_OK;
}
