// bf16 MFMA kernels of BDH strict-tril attention for gfx950 (the hot path):
//
//   out[b,h,i,:] = sum_{j<i} <R_i, R_j> V_j,   R = RoPE(x) (or R = q, k given)
//
// Forward, two kernels per call (three with an absolute-position table):
//  1. k_rope_table (RoPE with the RoPE(x) copy): (cos, sin) of every (row,
//     pair) as two bf16 halves of one dword, stage-major.  The same table
//     serves every (b,h).  Without the copy the score kernel rotates rows
//     about their tile's centre and makes the same dwords itself from the
//     frequencies, which it keeps in LDS.
//  2. k_sy_scores: partial score tiles S = R R^T.
//     * 256x256 output tiles over the lower triangle of each (b,h) slab; with
//       Q = K the diagonal tiles go in pairs, each computing its 36 lower
//       32x32 blocks (four 9-block wave programs per tile).
//     * split-K: split s of n handles a contiguous range of 64-wide k-chunks,
//       walked from an offset set by the slab's group on its XCD; all items
//       of a slab run on one XCD (workgroup id % 8 selects the XCD), so the
//       tiles that load the same row blocks walk k in step and the second
//       load is an L2 hit.
//     * x streams HBM -> LDS through global_load_lds_dwordx4 into a ring of
//       32-wide k stages (5 slots issued four stages ahead; with RoPE 4 slots,
//       and a fifth for the next stage's table entries or the frequencies).  The 16-byte chunk
//       c of row r sits at position c ^ ((r >> 2) & 3) of its 64-byte LDS
//       row, which makes the MFMA fragment reads bank-conflict free.
//     * RoPE is applied in place in the stage before its MFMAs: each lane
//       rotates the chunks it loaded itself (per pair two v_dot2_f32_bf16,
//       products exact in fp32, and one v_cvt_pk_bf16_f32).
//     * A barrier between the two k16 halves of a stage, fragments of the
//       next half read before the current half's MFMAs.
//     * v_mfma_f32_32x32x16_bf16 with fp32 accumulators; the epilogue stores
//       the partial tiles [slab][tile][split] as bf16 in MFMA fragment order
//       (whole 1 KB fragment rows per store).
//  3. k_sy_sv: out = tril(sum over splits of S, -1) V, score blocks and V rows
//     staged in LDS, V read as MFMA fragments with ds_read_b64_tr_b16.
// Backward (bf16 self attention): k_dq_sy (dQ = G X; with RoPE, R^T applied
// to its fp32 sums in the epilogue) and k_dv_sy (dV from the score tiles of
// k_sy_scores), both with transposing LDS reads.
#include <algorithm>
#include <cstdlib>
#include <cstring>
#include <type_traits>
#include <utility>

#include "fwd.h"
#include "lds_dma.h"


namespace bdh {
namespace {

constexpr int kSyThreads = 512;
constexpr int kSyTile = 256;
constexpr int kSyBlk = kSyTile * 64;   // bytes of one row block per stage (256 rows x 32 bf16)
constexpr int kSySlot = 2 * kSyBlk;    // A and B row blocks
constexpr int kSyLdsSlots = 5;    // 160 KB: x ring of 5 (plain), or 4 x + table or frequencies (fused)
constexpr int kSyTileElems = kSyTile * kSyTile;

// Work item kinds.  kSyFull: tile (ta, tb), ta > tb, or any tile when Q != K;
// kSyDiag2: diagonal tiles ta and tb; kSyDiag1: diagonal tile ta alone (tb =
// ta: loaded twice, stored once).
enum : int { kSyFull = 0, kSyDiag2 = 1, kSyDiag1 = 2 };


struct SyArgs {
  const bf16_t* q;
  const bf16_t* k;
  int64_t q0, q1, q2;  // element strides of q over (b, h, t)
  int64_t k0, k1, k2;
  int H, T, N, nslab, ips, nchunk, nsplit, ntl;
  int t0 = 0;          // packed index of the first stored tile (row tiles from s0: s0 (s0 + 1) / 2)
  int s0 = 0;          // first row tile with work
  int per_split;       // work items per split of a slab
  int nfull;           // of which full tiles (the rest: diagonal pairs)
  const uint32_t* cs;  // RoPE table, stage-major [N/32][T][16] (cos, sin) dwords, or null
  const float* freqs = nullptr;  // relative RoPE: the N frequencies (cos, sin made in the kernel)
  bf16_t* part;        // [nslab][ntl][nsplit][256*256] partial score tiles (bf16)
  bf16_t* qr;          // optional RoPE(x) copy
  int64_t r0, r1, r2;
  bf16_t* g;           // G output [nslab][tpad][tpad] (G epilogue only)
  int64_t tpad;
  int tq;              // rows of the RoPE table
};

// Work item itx of a slab: split-major; within a split the full tiles row by
// row from row tile s0, then (Q = K) the diagonal tiles of row tiles s0.. in
// pairs, the last one alone when their count is odd.  Returned as one word,
// ta | tb << 8 | split << 16 | kind << 24, so a single scalar register stays
// live.  Uniform scalar loops (at most nsplit and nt steps).
template <bool SELF>
__device__ inline uint32_t sy_item(const SyArgs& a, int itx) {
  int r = itx, split = 0;
  while (r >= a.per_split) {
    r -= a.per_split;
    ++split;
  }
  int ta, tb, kind;
  if (!SELF || r < a.nfull) {
    int t = a.s0;
    while (r >= (SELF ? t : t + 1)) {  // row t holds t (Q = K) or t + 1 full tiles
      r -= SELF ? t : t + 1;
      ++t;
    }
    ta = t;
    tb = r;
    kind = kSyFull;
  } else {
    const int nt = (a.T + kSyTile - 1) / kSyTile;
    ta = a.s0 + 2 * (r - a.nfull);
    tb = ta + 1 < nt ? ta + 1 : ta;
    kind = tb == ta ? kSyDiag1 : kSyDiag2;
  }
  return __builtin_amdgcn_readfirstlane(uint32_t(ta) | (uint32_t(tb) << 8) | (uint32_t(split) << 16) |
                                        (uint32_t(kind) << 24));
}

__shared__ __attribute__((aligned(1024))) uint8_t sy_lds[kSyLdsSlots * kSySlot];  // 160 KB

// ---------------------------------------------------------------- asm helpers
// (LDS DMA, its waits and scalar pointers: lds_dma.h)
__device__ __forceinline__ void sy_barrier() {
  asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
  __builtin_amdgcn_s_barrier();
}
// The same barrier as one asm statement: the compiler moves no memory access
// across it in either direction (the ping-pong schedule relies on that).
__device__ __forceinline__ void sy_barrier_asm() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }

// RoPE of the four adjacent pairs of one 16-byte chunk: pair m is
// x.lo = x[2m], x.hi = x[2m+1] with cs = (cos, sin) and sw = (sin, cos) as bf16
// halves, giving (x0 c - x1 s, x0 s + x1 c) = (dot2(x, cs) with s negated,
// dot2(x, sw)), rounded to bf16 once (products exact in fp32).  The swapped
// entry sw serves every chunk that shares cs, so the rows' data are never
// swapped.  One asm block so the hazard spacing is explicit: a v_dot2 result
// is read no sooner than three wait states after it is written (s_nop 2).
// CONJ rotates by the negated angle, (x0 c + x1 s, -x0 s + x1 c): the sign
// modifier moves from the first dot product to the second.
#define SY_ROT_ASM(NA, NB)                                                                                   \
  asm("v_dot2_f32_bf16 %[a0], %[x0], %[c0], 0" NA "\n\t"                                                    \
      "v_dot2_f32_bf16 %[a1], %[x1], %[c1], 0" NA "\n\t"                                                    \
      "v_dot2_f32_bf16 %[a2], %[x2], %[c2], 0" NA "\n\t"                                                    \
      "v_dot2_f32_bf16 %[a3], %[x3], %[c3], 0" NA "\n\t"                                                    \
      "v_dot2_f32_bf16 %[b0], %[x0], %[w0], 0" NB "\n\t"                                                    \
      "v_dot2_f32_bf16 %[b1], %[x1], %[w1], 0" NB "\n\t"                                                    \
      "v_dot2_f32_bf16 %[b2], %[x2], %[w2], 0" NB "\n\t"                                                    \
      "v_dot2_f32_bf16 %[b3], %[x3], %[w3], 0" NB "\n\t"                                                    \
      "s_nop 2\n\t"                                                                                         \
      "v_cvt_pk_bf16_f32 %[y0], %[a0], %[b0]\n\t"                                                           \
      "v_cvt_pk_bf16_f32 %[y1], %[a1], %[b1]\n\t"                                                           \
      "v_cvt_pk_bf16_f32 %[y2], %[a2], %[b2]\n\t"                                                           \
      "v_cvt_pk_bf16_f32 %[y3], %[a3], %[b3]"                                                                 \
      : [y0] "=&v"(y0), [y1] "=&v"(y1), [y2] "=&v"(y2), [y3] "=&v"(y3), [a0] "=&v"(a0), [a1] "=&v"(a1),       \
        [a2] "=&v"(a2), [a3] "=&v"(a3), [b0] "=&v"(b0), [b1] "=&v"(b1), [b2] "=&v"(b2), [b3] "=&v"(b3)         \
      : [x0] "v"(x.x), [x1] "v"(x.y), [x2] "v"(x.z), [x3] "v"(x.w), [c0] "v"(cs.x), [c1] "v"(cs.y),           \
        [c2] "v"(cs.z), [c3] "v"(cs.w), [w0] "v"(sw.x), [w1] "v"(sw.y), [w2] "v"(sw.z), [w3] "v"(sw.w))
template <bool CONJ = false>
__device__ __forceinline__ u32x4 rot_chunk_w(u32x4 x, u32x4 cs, u32x4 sw) {
  uint32_t y0, y1, y2, y3;
  float a0, a1, a2, a3, b0, b1, b2, b3;
  if constexpr (CONJ)
    SY_ROT_ASM("", " neg_lo:[0,1,0]");
  else
    SY_ROT_ASM(" neg_hi:[0,1,0]", "");
  return u32x4{y0, y1, y2, y3};
}
#undef SY_ROT_ASM

// (sin, cos) from (cos, sin): the halves of each dword swapped
__device__ __forceinline__ u32x4 swap_halves(u32x4 t) {
  const uint32_t t0 = t.x, t1 = t.y, t2 = t.z, t3 = t.w;
  return u32x4{__builtin_amdgcn_alignbit(t0, t0, 16), __builtin_amdgcn_alignbit(t1, t1, 16),
               __builtin_amdgcn_alignbit(t2, t2, 16), __builtin_amdgcn_alignbit(t3, t3, 16)};
}
template <bool CONJ = false>
__device__ __forceinline__ u32x4 rot_chunk(u32x4 x, u32x4 cs) {
  return rot_chunk_w<CONJ>(x, cs, swap_halves(cs));
}

// Two pairs of the rotation above (dwords x0, x1 with entries c0, c1 and their
// swaps w0, w1), so a chunk's rotation can be split between two MFMAs.
#define SY_ROT2_ASM(NA, NB)                                                                          \
  asm("v_dot2_f32_bf16 %[a0], %[x0], %[c0], 0" NA "\n\t"                                            \
      "v_dot2_f32_bf16 %[a1], %[x1], %[c1], 0" NA "\n\t"                                            \
      "v_dot2_f32_bf16 %[b0], %[x0], %[w0], 0" NB "\n\t"                                            \
      "v_dot2_f32_bf16 %[b1], %[x1], %[w1], 0" NB "\n\t"                                            \
      "s_nop 2\n\t"                                                                                 \
      "v_cvt_pk_bf16_f32 %[y0], %[a0], %[b0]\n\t"                                                   \
      "v_cvt_pk_bf16_f32 %[y1], %[a1], %[b1]"                                                         \
      : [y0] "=&v"(y0), [y1] "=&v"(y1), [a0] "=&v"(a0), [a1] "=&v"(a1), [b0] "=&v"(b0), [b1] "=&v"(b1) \
      : [x0] "v"(x0), [x1] "v"(x1), [c0] "v"(c0), [c1] "v"(c1), [w0] "v"(w0), [w1] "v"(w1))
template <bool CONJ = false>
__device__ __forceinline__ void rot_pairs_w(uint32_t x0, uint32_t x1, uint32_t c0, uint32_t c1, uint32_t w0,
                                            uint32_t w1, uint32_t& y0, uint32_t& y1) {
  float a0, a1, b0, b1;
  if constexpr (CONJ)
    SY_ROT2_ASM("", " neg_lo:[0,1,0]");
  else
    SY_ROT2_ASM(" neg_hi:[0,1,0]", "");
}
#undef SY_ROT2_ASM

__device__ __forceinline__ f32x16 mma(bf16x8 a, bf16x8 b, f32x16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
}

// ------------------------------------------------------------------ kernels
// RoPE table, stage-major: the (cos, sin) of pair m at row t sits in dword
// ((m / 16) * T + t) * 16 + m % 16, so the table entries one k32 stage of the
// score kernel needs for a 256-row block are one contiguous 16 KB run.  Row t
// is position rope_start + t.  (The score kernel's relative mode makes its
// entries for half-integer distances itself, with rope_cs below.)
// phase = fp32(pos) * freq, then cos/sin of 2 pi frac(phase); v_cos/v_sin
// take the angle in revolutions, so frac(phase) goes in directly.  The values
// are rounded to bf16, far above the hardware functions' error.  One dword
// (cos | sin << 16); the table kernel and the score kernel's relative mode
// both make their entries here, so they are the same bits.
__device__ __forceinline__ uint32_t rope_cs(float pos, float freq) {
  const float ph = __fmul_rn(pos, freq);
  const float fr = __builtin_amdgcn_fractf(ph);  // ph - floor(ph): ph >= 0
  return pack_bf2(__builtin_amdgcn_cosf(fr), __builtin_amdgcn_sinf(fr));
}

__global__ __launch_bounds__(256) void k_rope_table(const float* __restrict__ freqs, int64_t rope_start,
                                                    int N2, int T, uint32_t* __restrict__ cs) {
  const int t = blockIdx.y, m = blockIdx.x * 256 + threadIdx.x;
  if (m >= N2) return;
  cs[(int64_t(m >> 4) * T + t) * 16 + (m & 15)] = rope_cs(float(rope_start + t), freqs[2 * m]);
}

// Diagonal tiles (Q = K) in pairs: the 36 lower 32x32 blocks of one diagonal
// tile are split into four wave programs of 9 blocks; waves 0-3 run them on
// the first tile of the pair and waves 4-7 on the second, so each SIMD issues
// 18 MFMAs per k16 step (a full tile: 16).  Because A and B are the same row
// block, the fragment of row block r serves as either operand.
struct SyDiagWave {
  int nf;        // fragments per k16 step
  int rows[6];   // their row blocks
  int bi[9], bj[9];  // output blocks (row block, column block)
};
constexpr SyDiagWave kSyDiag[4] = {
    {6, {0, 1, 4, 5, 6, 7}, {4, 4, 5, 5, 6, 6, 7, 7, 0}, {0, 1, 0, 1, 0, 1, 0, 1, 0}},
    {6, {2, 3, 4, 5, 6, 7}, {4, 4, 5, 5, 6, 6, 7, 7, 4}, {2, 3, 2, 3, 2, 3, 2, 3, 4}},
    {4, {0, 1, 2, 3, 0, 0}, {1, 1, 2, 2, 2, 3, 3, 3, 3}, {0, 1, 0, 1, 2, 0, 1, 2, 3}},
    {4, {4, 5, 6, 7, 0, 0}, {5, 5, 6, 6, 6, 7, 7, 7, 7}, {4, 5, 4, 5, 6, 4, 5, 6, 7}},
};
constexpr int sy_fidx(const SyDiagWave& d, int r) {
  for (int k = 0; k < d.nf; ++k)
    if (d.rows[k] == r) return k;
  return -1;
}
// Wave program WT: 0 = a 128x64 corner of a full tile (8 blocks), 1..4 = the
// diagonal programs above.  Fragment indices of the A and B operands of MFMA m.
// Compile-time loop: f(integral_constant<int, i>) for i = 0 .. N-1, so array
// indices derived from i are constants (registers, not scratch).
template <typename F, int... I>
__device__ __forceinline__ void sy_static_for_impl(F&& f, std::integer_sequence<int, I...>) {
  (f(std::integral_constant<int, I>()), ...);
}
template <int N, typename F>
__device__ __forceinline__ void sy_static_for(F&& f) {
  sy_static_for_impl(f, std::make_integer_sequence<int, N>());
}

template <int WT>
struct SyProg {
  static constexpr int nf = WT == 0 ? 6 : kSyDiag[WT - 1].nf;
  static constexpr int nm = WT == 0 ? 8 : 9;
  static constexpr int fa(int m) { return WT == 0 ? m >> 1 : sy_fidx(kSyDiag[WT - 1], kSyDiag[WT - 1].bi[m]); }
  static constexpr int fb(int m) { return WT == 0 ? 4 + (m & 1) : sy_fidx(kSyDiag[WT - 1], kSyDiag[WT - 1].bj[m]); }
  static constexpr int row(int k) { return WT == 0 ? 0 : kSyDiag[WT - 1].rows[k]; }
  static constexpr int bi(int m) { return WT == 0 ? 0 : kSyDiag[WT - 1].bi[m]; }
  static constexpr int bj(int m) { return WT == 0 ? 0 : kSyDiag[WT - 1].bj[m]; }
  // Relative RoPE layout: the row group held by group slot g, and whether
  // MFMA m runs with its operands swapped so its block stays below the
  // diagonal.
  static constexpr int grp(int g) { return g < 4 ? g : 11 - g; }
  static constexpr bool swp(int m, bool rel) { return rel && WT != 0 && grp(bi(m)) < grp(bj(m)); }
};

// Relative RoPE: chunk u of wave program wt turns by the negated angle (full
// tile B rows; diagonal rows below the centre), and reads table entry
// sy_rot_tidx (absolute tables: one entry per chunk).
template <bool REL>
constexpr bool sy_rot_conj(int wt, int u) { return REL && (wt == 0 ? u >= 2 : (u & 1) == 0); }
template <bool REL>
constexpr int sy_rot_tidx(int wt, int u) { return !REL ? u : (wt == 0 ? ((u == 1 || u == 2) ? 1 : 0) : 0); }

// Partial score tiles are stored in MFMA fragment order: a tile's 32 x 32
// block held by wave slot ws (the wave, or wave & 3 on diagonal tiles) as its
// m-th accumulator is fragment slot k = ws * nm + m (nm = 8 full, 9
// diagonal) of 1024 bf16: lane l's 16 values, pairs (2q, 2q + 1) packed into
// dword q, dwords 0-3 at element 8 l and dwords 4-7 at 512 + 8 l.  Value r of
// lane l is block element (8 (r / 4) + 4 (l / 32) + r % 4, l % 32).  Each
// wave writes its 2 KB slots with two 1 KB coalesced stores.
// sy_slot_of maps a block (rb, cb) of a tile to its slot: the inverse of the
// epilogue's block mapping (relative RoPE reorders row groups), built at
// compile time for full tiles and the lower blocks of diagonal tiles.
struct SySlotTab {
  uint8_t full[2][64];  // [relative][8 rb + cb]
  uint8_t diag[2][64];  // [relative][8 rb + cb], rb >= cb
};
constexpr SySlotTab sy_make_slots() {
  SySlotTab t{};
  for (int rel = 0; rel < 2; ++rel) {
    for (int ws = 0; ws < 8; ++ws)
      for (int m = 0; m < 8; ++m) {
        const int wm = ws >> 2, wn = ws & 3;
        const int rb = (rel && wm == 1) ? 7 - (m >> 1) : 4 * wm + (m >> 1);
        const int cb = (rel && wn >= 2) ? 11 - 2 * wn - (m & 1) : 2 * wn + (m & 1);
        t.full[rel][8 * rb + cb] = uint8_t(ws * 8 + m);
      }
    for (int ws = 0; ws < 4; ++ws)
      for (int m = 0; m < 9; ++m) {
        int gi = kSyDiag[ws].bi[m], gj = kSyDiag[ws].bj[m];
        if (rel) {
          gi = gi < 4 ? gi : 11 - gi;
          gj = gj < 4 ? gj : 11 - gj;
        }
        const int rb = gi > gj ? gi : gj, cb = gi > gj ? gj : gi;
        t.diag[rel][8 * rb + cb] = uint8_t(ws * 9 + m);
      }
  }
  return t;
}
constexpr SySlotTab kSySlots = sy_make_slots();
// element offset (in a partial tile) of the 16-byte piece `half` of lane l of
// block (rb, cb)
__device__ __forceinline__ int sy_piece(bool diag_tile, int rel, int rb, int cb, int l, int half) {
  const int k = diag_tile ? kSySlots.diag[rel][8 * rb + cb] : kSySlots.full[rel][8 * rb + cb];
  return k * 1024 + half * 512 + l * 8;
}
// rows (in the block) of the eight values of piece `half` of lane l, in
// order: value 2q' + e is row sy_piece_row(l, half, q', e)
__device__ __forceinline__ int sy_piece_row(int l, int half, int qq, int e) {
  const int r = 2 * (4 * half + qq) + e;
  return 8 * (r >> 2) + 4 * (l >> 5) + (r & 3);
}

// RM: 0 no RoPE; 1 RoPE at absolute positions (table row t = position
// rope_start + t); 2 RoPE relative to each tile's centre.  Scores depend only
// on position differences, so rotating the rows of tile (ta, tb) by their
// position minus c = (256 (ta + tb) + 255) / 2 leaves them unchanged; every
// row then needs the angle of a half-integer distance q + 0.5, q < 128 nt,
// and within a row block the row at LDS position P is block row P (P < 128)
// or 383 - P (P >= 128), so the two rows a lane loads per block share q: one
// table entry per lane and stage on diagonal items, two on full tiles (row
// a of A and row 255 - a of B, rotated by the negated angle).  The lane
// makes those entries from the stage's frequencies in LDS (rel_entry).
// GOUT (with Q = dO, K = V, one split): instead of partial tiles, write the
// backward's G = dS + dS^T, dS = tril(dO V^T, -1), into a.g.
// PAIR (relative RoPE): even stages issue the chunks of stages s + 2 and s + 3
// back to back, odd stages none, so the two 64-byte halves of each 128-byte
// line of a row are requested together.  For rows whose stride is a multiple
// of 64 KB (the model's (B, T, nh, N) x_sparse): their pieces share few L2
// sets, and a line fetched for one stage is gone before the next stage reads
// its other half.
// SCH (relative RoPE): 0 the lockstep schedule; 1 the ping-pong schedule of
// the two wave groups (see the main loop).  Both give the same bits.
template <int RM, bool SELF, bool GOUT = false, bool PAIR = false, int SCH = 0>
__global__ __launch_bounds__(kSyThreads, 1) void k_sy_scores(const SyArgs a) {
  constexpr bool ROPE = RM != 0;
  constexpr bool REL = RM == 2;
  static_assert(!PAIR || REL, "paired stages: relative RoPE");
  static_assert(SCH == 0 || (RM != 1 && !GOUT), "ping-pong schedule: relative RoPE or none");
  constexpr bool PP = SCH == 1;
  static_assert(!GOUT || (!SELF && !ROPE), "G epilogue: distinct operands, no RoPE");
  static_assert(!REL || SELF, "relative RoPE: self attention");
  const int bid = blockIdx.x;
  const int xcd = bid & 7, kk = bid >> 3;
  const int grp = kk / a.ips;
  const int slab = grp * 8 + xcd;
  if (slab >= a.nslab) return;
  const int itx = kk - grp * a.ips;
  const uint32_t item = sy_item<SELF>(a, itx);
  const int ta = item & 255, tb = (item >> 8) & 255, split = (item >> 16) & 255;
  const int kind = int(item >> 24);
  const bool diag = SELF && kind != kSyFull;
  const int b = slab / a.H, h = slab - b * a.H;
  const int tid = threadIdx.x, lane = tid & 63;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int S = a.nsplit;
  // k chunks (64 wide) of this split: the contiguous range [kc0, kc0 + nch)
  const int kc0 = (split * a.nchunk) / S;
  const int nch = ((split + 1) * a.nchunk) / S - kc0;
  const int nst = 2 * nch;

  const void* baseA = sgpr_ptr(a.q + b * a.q0 + h * a.q1);
  const void* baseB = SELF ? baseA : sgpr_ptr(a.k + b * a.k0 + h * a.k1);
  const void* tbase = sgpr_ptr(a.cs);
  const uint32_t lds0 = __builtin_amdgcn_readfirstlane((uint32_t)(uintptr_t)(lds_u8*)sy_lds);

  // Per DMA instruction u: the 16-byte chunk this lane moves (and rotates).
  // Instructions 0-1 fill the row block of tile row ta, 2-3 that of tb.
  uint32_t xoff[4], toff[4];
#pragma unroll
  for (int u = 0; u < 4; ++u) {
    const int q = (u * 8 + w) * 1024 + lane * 16;
    const int blk = q >> 14;
    const int ob = q & (kSyBlk - 1);
    const int row = ob >> 6;  // LDS row position
    const int c = ((ob >> 4) & 3) ^ ((row >> 2) & 3);
    const int brow = (REL && row >= 128) ? 383 - row : row;
    const int rg = (blk == 0 ? ta : tb) * kSyTile + brow;
    const int rc = rg < a.T ? rg : a.T - 1;
    xoff[u] = uint32_t((int64_t(rc) * (blk == 0 ? a.q2 : (SELF ? a.q2 : a.k2)) + 8 * c) * 2);
    toff[u] = uint32_t(rc * 64 + 16 * c);
  }
  // Relative positions of this lane's chunks (rho: LDS row of chunk 0):
  // diagonal items q = 127 - rho for all four chunks; full tiles
  // q = 128 (ta - tb - 1) + rho (chunks 0 and 3) and + 255 - rho (1 and 2);
  // the angle is that of q + 0.5.  The lane's chunk holds pairs 4 cq .. +3
  // of each stage.
  float qpos[2] = {0.f, 0.f};
  int rcq = 0;
  if constexpr (REL) {
    const int rho = 16 * w + (lane >> 2);
    rcq = (lane & 3) ^ ((lane >> 4) & 3);
    const int q0 = diag ? 127 - rho : 128 * (ta - tb - 1) + rho;
    const int q1 = diag ? q0 : 128 * (ta - tb - 1) + 255 - rho;
    qpos[0] = float(q0) + 0.5f;
    qpos[1] = float(q1) + 0.5f;
  }
  // MFMA fragment offsets within a row block for the two k16 halves of a
  // stage; lrev reads a 32-row group stored in reverse (REL upper half), so
  // the fragment rows come out in block order.
  uint32_t loff[2], lrev[2];
#pragma unroll
  for (int kk2 = 0; kk2 < 2; ++kk2) {
    const int c = (2 * kk2 + (lane >> 5)) ^ ((lane >> 2) & 3);
    loff[kk2] = uint32_t((lane & 31) * 64 + c * 16);
    const int ir = 31 - (lane & 31);
    const int cr = (2 * kk2 + (lane >> 5)) ^ ((ir >> 2) & 3);
    lrev[kk2] = uint32_t(ir * 64 + cr * 16);
  }
  // RoPE(x) copy: each row of a slab belongs to exactly one diagonal tile and
  // each k chunk to one split, so the diagonal items write it (the first row
  // block only for a single diagonal tile, which loads it twice).
  const bool write_qr = RM == 1 && a.qr != nullptr && diag;

  // Stage s reads half s & 1 of the split's chunk (s / 2 + krs) mod nch.  The
  // four slab groups on one XCD (slab / 8) start a quarter of the range apart,
  // so at any time the XCD's items read x at different offsets of their rows:
  // rows 16 KB or 64 KB apart at one offset fall on few memory channels.  C1
  // without RoPE 75 -> 66 us, the model's (B, T, nh, N) view at C2 501 ->
  // 245 us (plain) and 389 -> 355 us (fused, paired); against splits that
  // interleave 64-wide chunks, all started at offset 0.  Both items of a split
  // (the full tile and the diagonal pair) walk the same order, so the second
  // reader of a row piece finds it in L2.
  const int krs = ((slab >> 3) * (nch >> 2 > 0 ? nch >> 2 : 1)) % nch;
  auto kofs = [&](int s) {
    int c = (s >> 1) + krs;
    c = c >= nch ? c - nch : c;
    return (kc0 + c) * 64 + (s & 1) * 32;
  };
  // LDS: an x ring of NX slots, issued lead = NX - 1 stages ahead; with RoPE
  // four x slots and a fifth slot: absolute positions, the table entries of
  // the next stage; relative, the frequencies of this workgroup's stages
  // (16 pairs a stage, at most 512 stages), from which each lane makes its
  // cos/sin entries.
  constexpr int NX = ROPE ? 4 : 5;
  constexpr int lead = NX - 1;
  auto xslot_ofs = [&](int s) { return (s % NX) * kSySlot; };
  auto slot = [&](int s) { return sy_lds + xslot_ofs(s); };
  auto tslot_ofs = [&](int s) { return NX * kSySlot; };
  auto tslot = [&](int s) { return sy_lds + tslot_ofs(s); };
  const float* const pfl = reinterpret_cast<const float*>(sy_lds + NX * kSySlot);
  // (cos, sin) dwords of this lane's four pairs of stage st at position p:
  // the relative table's entries, made from the same arithmetic
  auto rel_entry = [&](int st, float p) {
    const float* f = pfl + st * 16 + 4 * rcq;
    const float f0 = f[0], f1 = f[1], f2 = f[2], f3 = f[3];
    return u32x4{rope_cs(p, f0), rope_cs(p, f1), rope_cs(p, f2), rope_cs(p, f3)};
  };
  // The DMA instructions of one stage: per-stage scalar bases, per-instruction
  // immediates (instruction u of wave w fills LDS bytes [(8u + w) KB, +1 KB)
  // of its slot).
  const uint32_t wl = lds0 + uint32_t(w) * 1024u;
  struct StageDma {
    uint32_t xm0, tm0, kx, kt;
  };
  // Stage st goes to the slots of st; stages past the end re-load the last
  // stage into slots that are no longer read, so every stage issues the same
  // instructions and every wait counts the same number of them.
  auto stage_dma = [&](int st) {
    StageDma d;
    const int ko = kofs(min(st, nst - 1));
    d.xm0 = wl + uint32_t(xslot_ofs(st));
    d.tm0 = wl + uint32_t(tslot_ofs(st));
    d.kx = uint32_t(ko * 2);
    d.kt = uint32_t(ko >> 5) * uint32_t(a.tq) * 64u;
    return d;
  };
  auto dma_x = [&](const StageDma& d, auto uc) {
    constexpr int u = decltype(uc)::value;
    dma16<u * 8192>(d.xm0, u < 2 ? baseA : baseB, xoff[u] + d.kx);
  };
  auto dma_t = [&](const StageDma& d, auto ic) {
    constexpr int i = decltype(ic)::value;
    dma16<i * 8192>(d.tm0, tbase, toff[i] + d.kt);
  };
  // RoPE in place of chunk u of stage s (this lane's own DMA chunk)
  // (the row and chunk of instruction u follow from the lane: row
  // (u & 1) * 128 + 16 w + lane / 4 of the block of tile row ta (u < 2) or tb,
  // chunk (lane & 3) ^ ((lane >> 4) & 3) of the 64-byte row)
  // (REL: wave program WT 0 is a full tile, whose B rows (chunks 2, 3) turn by
  // the negated angle; the others are diagonal tiles, whose rows below the
  // centre (chunks 0, 2) do.)
  const int vrot = w * 1024 + lane * 16;
  auto put_rot = [&](int s, auto uc, u32x4 y) {
    constexpr int u = decltype(uc)::value;
    *reinterpret_cast<u32x4*>(slot(s) + vrot + u * 8192) = y;
    if (write_qr && (kind == kSyDiag2 || u < 2)) {
      const int rg = (u < 2 ? ta : tb) * kSyTile + (u & 1) * 128 + 16 * w + (lane >> 2);
      const int c = (lane & 3) ^ ((lane >> 4) & 3);
      if (rg < a.T)
        *reinterpret_cast<u32x4*>(a.qr + b * a.r0 + h * a.r1 + int64_t(rg) * a.r2 + kofs(s) + 8 * c) = y;
    }
  };
  auto rot_store = [&](int s, auto wtc, auto uc, u32x4 x, u32x4 t) {
    constexpr bool conj = sy_rot_conj<REL>(decltype(wtc)::value, decltype(uc)::value);
    put_rot(s, uc, rot_chunk<conj>(x, t));
  };
  // (table entry of chunk u: its own (absolute); REL full tiles 0, 1, 1, 0;
  // REL diagonal tiles 0)
  auto rot_load = [&](int s, auto wtc, auto uc, u32x4& x, u32x4& t) {
    constexpr int u = decltype(uc)::value;
    x = *reinterpret_cast<const u32x4*>(slot(s) + vrot + u * 8192);
    if constexpr (REL)
      t = rel_entry(s, qpos[sy_rot_tidx<REL>(decltype(wtc)::value, u)]);
    else
      t = *reinterpret_cast<const u32x4*>(tslot(s) + vrot + sy_rot_tidx<REL>(decltype(wtc)::value, u) * 8192);
  };

  // The wave program selects one of five instantiations of the whole pipeline
  // (prologue, loop, epilogue), so each loop holds straight-line MFMA code; all
  // of them run the same stages and barriers.
  auto run = [&](auto wt_tag) {
    constexpr int WT = decltype(wt_tag)::value;
    using P = SyProg<WT>;
    constexpr int NF = P::nf, NM = P::nm;
    // Fragment addresses: a per-wave base (with the lane's offset) in a
    // register, the fragment's 32-row group slot g as an immediate.  Full
    // tile: A slots 4 wm + k at fbase[0], B slots 2 wn + j at fbase[1];
    // diagonal: slot P::row(k) of the wave's tile at fbase[0] (REL: slots
    // g >= 4 at fbase[1]).  With REL, slot g >= 4 holds the row group
    // 11 - g of the block, read through lrev.
    int fbase[2][2];  // [half][A, B]
    int tile_out;     // partial tile this wave writes (-1: none)
    if constexpr (WT == 0) {
      const int wm = w >> 2, wn = w & 3;
#pragma unroll
      for (int hf = 0; hf < 2; ++hf) {
        fbase[hf][0] = 4 * wm * 2048 + int((REL && wm == 1) ? lrev[hf] : loff[hf]);
        fbase[hf][1] = kSyBlk + 2 * wn * 2048 + int((REL && wn >= 2) ? lrev[hf] : loff[hf]);
      }
      tile_out = ta * (ta + 1) / 2 + tb - a.t0;
    } else {
#pragma unroll
      for (int hf = 0; hf < 2; ++hf) {
        fbase[hf][0] = (w >> 2) * kSyBlk + int(loff[hf]);
        fbase[hf][1] = (w >> 2) * kSyBlk + int(REL ? lrev[hf] : loff[hf]);
      }
      const int t = w < 4 ? ta : tb;
      tile_out = (w < 4 || kind == kSyDiag2) ? t * (t + 1) / 2 + t - a.t0 : -1;
    }
    f32x16 acc[NM];
#pragma unroll
    for (int i = 0; i < NM; ++i)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][r] = 0.f;
    bf16x8 f0[NF], f1[NF];
    auto mfma_m = [&](bf16x8(&f)[NF], auto mc) {
      constexpr int m = decltype(mc)::value;
      constexpr bool sw = P::swp(m, REL);
      acc[m] = mma(f[sw ? P::fb(m) : P::fa(m)], f[sw ? P::fa(m) : P::fb(m)], acc[m]);
    };
    auto read_frags = [&](bf16x8(&f)[NF], int s, int half) {
      const uint8_t* pa = slot(s) + fbase[half][0];
      const uint8_t* pb = slot(s) + fbase[half][1];
      sy_static_for<NF>([&](auto kc) {
        constexpr int k = decltype(kc)::value;
        if constexpr (WT == 0)
          f[k] = *reinterpret_cast<const bf16x8*>(k < 4 ? pa + k * 2048 : pb + (k - 4) * 2048);
        else
          f[k] = *reinterpret_cast<const bf16x8*>((P::row(k) >= 4 ? pb : pa) + P::row(k) * 2048);
      });
    };

    // ------------------------------------------------------------ prologue
    // Issue order is what the waits count on: operations complete in order.
    // Per stage each wave issues four x chunks of stage s + lead, two with
    // each half, and (RoPE) the four table chunks of stage s+2 first thing
    // after the mid-stage barrier.
    using I0 = std::integral_constant<int, 0>;
    using I1 = std::integral_constant<int, 1>;
    using I2 = std::integral_constant<int, 2>;
    using I3 = std::integral_constant<int, 3>;
    // REL: per stage k the order is x chunks 0-1, the NT table entries of k,
    // x chunks 2-3, so the table runs at the lead of x.
    constexpr int NT = WT == 0 ? 2 : 1;
    auto rotate_all = [&](int st) {
      sy_static_for<4>([&](auto uc) {
        u32x4 x, t;
        rot_load(st, wt_tag, uc, x, t);
        rot_store(st, wt_tag, uc, x, t);
      });
    };
    if constexpr (PP) {
      // Ping-pong.  Waves 0-3 (group 0) and 4-7 (group 1) hold one wave per
      // SIMD each and run the same program one barrier apart.  Per group and
      // stage j:
      //   MEM(j): read the fragments of stage j (both k16 halves); issue the
      //           DMA of stage j + 3 (PAIR: of j + 2 and j + 3 on even j);
      //           once this wave's chunks of stage j + 1 landed, make their
      //           cos/sin entries and rotate them in LDS
      //   barrier
      //   MMA(j): the MFMAs of stage j
      //   barrier
      // Group 1 passes one extra barrier first, so its MEM(j) runs beside
      // group 0's MMA(j) and its MMA(j) beside group 0's MEM(j + 1): on each
      // SIMD one wave's MFMAs cover the other's waits, VALU and LDS work.
      // Chunks are DMA'd and rotated as in the lockstep schedule (each wave
      // its own four), and every chunk of stage j + 1 is rotated one barrier
      // or more before either group reads fragments of it (group 0 rotates
      // it two intervals ahead, group 1 one).  The DMA of stage j + 3 goes to
      // the slot of stage j - 1, which group 1 last read in its MEM(j - 1),
      // the interval before group 0's MEM(j).
      const bool g1 = w >= 4;
      constexpr int L = NX - 1;  // stages issued ahead: 3 with RoPE, 4 without
      auto rotate_stage = [&](int st) {
        u32x4 x[4], t[NT];
        sy_static_for<4>([&](auto uc) {
          x[decltype(uc)::value] = *reinterpret_cast<const u32x4*>(slot(st) + vrot + decltype(uc)::value * 8192);
        });
        sy_static_for<NT>([&](auto ic) { t[decltype(ic)::value] = rel_entry(st, qpos[decltype(ic)::value]); });
        u32x4 tw[NT];
        sy_static_for<NT>([&](auto ic) { tw[decltype(ic)::value] = swap_halves(t[decltype(ic)::value]); });
        sy_static_for<4>([&](auto uc) {
          constexpr int u = decltype(uc)::value;
          constexpr int ti = sy_rot_tidx<REL>(WT, u);
          put_rot(st, uc, rot_chunk_w<sy_rot_conj<REL>(WT, u)>(x[u], t[ti], tw[ti]));
        });
      };
      if constexpr (PAIR) {
        const StageDma d0 = stage_dma(0), d1 = stage_dma(1);
        sy_static_for<4>([&](auto uc) {
          dma_x(d0, uc);
          dma_x(d1, uc);
        });
        sy_wait<1>();  // stage 0 landed (chunk 3 of stage 1 issued after it)
      } else {
        sy_static_for<L>([&](auto sc) {
          const StageDma d = stage_dma(decltype(sc)::value);
          sy_static_for<4>([&](auto uc) { dma_x(d, uc); });
        });
        sy_wait<4 * (L - 1)>();  // stage 0 landed (stages 1 .. L - 1 issued after it)
      }
      if constexpr (REL) rotate_stage(0);
      __builtin_amdgcn_sched_barrier(0);
      sy_barrier_asm();
      if (g1) sy_barrier_asm();
      __builtin_amdgcn_sched_barrier(0);
      for (int j = 0; j < nst; ++j) {
        bf16x8 fa[NF], fb[NF];
        read_frags(fa, j, 0);
        read_frags(fb, j, 1);
        if (j + 1 < nst) {
          // operations issued after this wave's chunks of stage j + 1: PAIR
          // even j, the eight of j + 2 and j + 3 just issued; PAIR odd j, chunk
          // 3 of j + 2; otherwise stages j + 2 .. j + L
          if constexpr (PAIR) {
            if ((j & 1) == 0) {
              const StageDma d = stage_dma(j + 2), d2 = stage_dma(j + 3);
              sy_static_for<4>([&](auto uc) {
                dma_x(d, uc);
                dma_x(d2, uc);
              });
              sy_wait<8>();
            } else {
              sy_wait<1>();
            }
          } else {
            const StageDma d = stage_dma(j + L);
            sy_static_for<4>([&](auto uc) { dma_x(d, uc); });
            sy_wait<4 * (L - 1)>();
          }
          if constexpr (REL) rotate_stage(j + 1);
        }
        __builtin_amdgcn_sched_barrier(0);
        sy_barrier_asm();
        __builtin_amdgcn_sched_barrier(0);
        sy_static_for<NM>([&](auto mc) { mfma_m(fa, mc); });
        sy_static_for<NM>([&](auto mc) { mfma_m(fb, mc); });
        __builtin_amdgcn_sched_barrier(0);
        sy_barrier_asm();
        __builtin_amdgcn_sched_barrier(0);
      }
      if (!g1) sy_barrier_asm();
      // the re-loads past the end must land before the workgroup's LDS is freed
      sy_wait<0>();
    } else {
      if constexpr (PAIR) {
        const StageDma d0 = stage_dma(0), d1 = stage_dma(1);
        sy_static_for<4>([&](auto uc) {
          dma_x(d0, uc);
          dma_x(d1, uc);
        });
        sy_wait<0>();  // stages 0 and 1 landed
        rotate_all(0);
        sy_barrier();
      } else if constexpr (REL) {
        for (int st = 0; st < lead - 1; ++st) {
          const StageDma d = stage_dma(st);
          sy_static_for<4>([&](auto uc) { dma_x(d, uc); });
        }
        const StageDma d = stage_dma(lead - 1);
        dma_x(d, I0());
        dma_x(d, I1());
        sy_wait<(lead - 2) * 4 + 2>();  // stage 0 landed
        rotate_all(0);
        sy_barrier();
        dma_x(d, I2());
        dma_x(d, I3());
      } else {
        for (int st = 0; st < lead - 1; ++st) {
          const StageDma d = stage_dma(st);
          sy_static_for<4>([&](auto uc) { dma_x(d, uc); });
        }
        const StageDma d = stage_dma(lead - 1);
        dma_x(d, I0());
        dma_x(d, I1());
        if constexpr (ROPE) {
          sy_static_for<4>([&](auto ic) { dma_t(stage_dma(0), ic); });
          sy_wait<0>();  // stage 0 and its table landed
          rotate_all(0);
          sy_barrier();
          sy_static_for<4>([&](auto ic) { dma_t(stage_dma(1), ic); });
          dma_x(d, I2());
          dma_x(d, I3());
        } else {
          dma_x(d, I2());
          dma_x(d, I3());
          sy_wait<(lead - 1) * 4>();  // stage 0 landed
          sy_barrier();
        }
      }
      read_frags(f0, 0, 0);

      // ------------------------------------------------------------ main loop
      // Stage s, per wave:
      //  A. read the second-half fragments of s; first-half MFMAs of s with x
      //     chunks 0-1 of stage s + lead issued between them; once this lane's
      //     part of stage s+1 (and its table) landed, the rotation of stage s+1
      //  B. barrier: stage s+1 is complete (loaded and rotated) in LDS
      //  C. read the first-half fragments of s+1; (absolute RoPE) issue the
      //     table of stage s+2; second-half MFMAs of s with x chunks 2-3 of
      //     stage s + lead.
      // The barrier sits between the halves, so after it the MFMA pipe runs the
      // second half while the next fragments load.  Stage s + lead goes to x
      // slot (s-1) % NX, last read before the previous barrier; the table slot
      // is rewritten after the barrier that follows its rotation.
      constexpr int KW = NM / 2 - 1;  // wait for stage s+1 after first-half MFMA KW
      // (without RoPE) operations issued after the awaited ones at that wait:
      // after x of s+1, x of s+2 .. s+lead-1 and chunks 0-1 of s + lead
      constexpr int NWAIT = (lead - 2) * 4 + 2;
      // RoPE: the wait for stage s+1 comes first, all four chunks and their
      // table entries are read at once, and half a chunk is rotated after each
      // of the first eight MFMAs (scheduling barriers keep that order, so the
      // rotation's VALU work runs under the MFMAs).  Operations issued after
      // the awaited ones: REL, stages s+2 .. s+lead-1 with their tables;
      // absolute, x chunks 2-3 of s+2 after the table of s+1.
      constexpr int NWAITR = REL ? (lead - 2) * 4 : 2;
      constexpr int NTD = REL ? NT : 4;  // distinct table entries per lane and stage
      for (int s = 0; s + 1 < nst; ++s) {
        read_frags(f1, s, 1);
        __builtin_amdgcn_sched_barrier(0);
        const StageDma d = stage_dma(PAIR ? s + 2 : s + lead);
        // PAIR: stage s + 3 goes to the slot of stage s - 1, whose last reads
        // came before the previous barrier
        const StageDma d2 = stage_dma(s + 3);
        const bool issue = !PAIR || (s & 1) == 0;
        if constexpr (ROPE) {
          if constexpr (PAIR) {
            // stage s+1 landed: even s, nothing issued after it (odd stages
            // issue none); odd s, chunk 3 of stage s+2 after it
            if (s & 1)
              sy_wait<1>();
            else
              sy_wait<0>();
          } else {
            sy_wait<NWAITR>();
          }
          u32x4 x[4], t[NTD];
          sy_static_for<4>([&](auto uc) {
            x[decltype(uc)::value] = *reinterpret_cast<const u32x4*>(slot(s + 1) + vrot + decltype(uc)::value * 8192);
          });
          sy_static_for<NTD>([&](auto ic) {
            constexpr int i = decltype(ic)::value;
            if constexpr (REL)
              t[i] = rel_entry(s + 1, qpos[i]);
            else
              t[i] = *reinterpret_cast<const u32x4*>(tslot(s + 1) + vrot + i * 8192);
          });
          // relative: the entries with their halves swapped, once per entry
          // (shared by two or four chunks); absolute: per chunk, below
          u32x4 tw[REL ? NTD : 1];
          if constexpr (REL)
            sy_static_for<NTD>([&](auto ic) { tw[decltype(ic)::value] = swap_halves(t[decltype(ic)::value]); });
          __builtin_amdgcn_sched_barrier(0);
          sy_static_for<NM>([&](auto mc) {
            constexpr int m = decltype(mc)::value;
            mfma_m(f0, mc);
            if constexpr (m == 0) {
              if (issue) {
                dma_x(d, I0());
                if constexpr (PAIR) dma_x(d2, I0());
              }
            }
            if constexpr (m == 2) {
              if (issue) {
                dma_x(d, I1());
                if constexpr (PAIR) dma_x(d2, I1());
              }
            }
            if constexpr (m < 8) {
              constexpr int u = m >> 1, hh = m & 1;
              constexpr bool conj = sy_rot_conj<REL>(WT, u);
              const u32x4 tt = t[sy_rot_tidx<REL>(WT, u)];
              const u32x4 ww = REL ? tw[REL ? sy_rot_tidx<REL>(WT, u) : 0] : swap_halves(tt);
              // (vector elements go through scalars: this clang lowers some
              // element accesses of u32x4 as element 0)
              if constexpr (hh == 0) {
                const uint32_t x0 = x[u].x, x1 = x[u].y, c0 = tt.x, c1 = tt.y, w0 = ww.x, w1 = ww.y;
                uint32_t y0, y1;
                rot_pairs_w<conj>(x0, x1, c0, c1, w0, w1, y0, y1);
                x[u].x = y0;
                x[u].y = y1;
              } else {
                const uint32_t x2 = x[u].z, x3 = x[u].w, c2 = tt.z, c3 = tt.w, w2 = ww.z, w3 = ww.w;
                uint32_t y2, y3;
                rot_pairs_w<conj>(x2, x3, c2, c3, w2, w3, y2, y3);
                x[u].z = y2;
                x[u].w = y3;
                put_rot(s + 1, std::integral_constant<int, u>(), x[u]);
              }
            }
            __builtin_amdgcn_sched_barrier(0);
          });
        } else {
          sy_static_for<NM>([&](auto mc) {
            constexpr int m = decltype(mc)::value;
            mfma_m(f0, mc);
            if constexpr (m == 0) dma_x(d, I0());
            if constexpr (m == 2) dma_x(d, I1());
            if constexpr (m == KW) sy_wait<NWAIT>();
          });
        }
        __builtin_amdgcn_sched_barrier(0);
        sy_barrier();
        read_frags(f0, s + 1, 0);
        if constexpr (ROPE && !REL) {
          const StageDma dt = stage_dma(s + 2);
          sy_static_for<4>([&](auto ic) { dma_t(dt, ic); });
        }
        __builtin_amdgcn_sched_barrier(0);
        sy_static_for<NM>([&](auto mc) {
          constexpr int m = decltype(mc)::value;
          mfma_m(f1, mc);
          if constexpr (m == 1) {
            if (issue) {
              dma_x(d, I2());
              if constexpr (PAIR) dma_x(d2, I2());
            }
          }
          if constexpr (m == 3) {
            if (issue) {
              dma_x(d, I3());
              if constexpr (PAIR) dma_x(d2, I3());
            }
          }
        });
      }
      // last stage: nothing left to load or rotate
      read_frags(f1, nst - 1, 1);
      sy_static_for<NM>([&](auto mc) { mfma_m(f0, mc); });
      sy_static_for<NM>([&](auto mc) { mfma_m(f1, mc); });
      // the re-loads past the end must land before the workgroup's LDS is freed
      sy_wait<0>();
    }

    // ------------------------------------------------------------ epilogue
    if constexpr (GOUT) {
      // Tile (ta, tb), ta >= tb, of dO V^T gives G's block (ta, tb) as stored
      // and block (tb, ta) transposed.  On a diagonal tile only the elements
      // below the diagonal count: blocks above it are written from their
      // mirror, and the 32x32 blocks on it are masked per element.  Rows and
      // columns at or past T are zero (G's padding); nothing at or past tpad
      // is written.  Each element of G below tpad has exactly one writer.
      bf16_t* g = a.g + int64_t(slab) * a.tpad * a.tpad;
      const int tpad = int(a.tpad);
      const bool dtile = ta == tb;
      sy_static_for<NM>([&](auto mc) {
        constexpr int m = decltype(mc)::value;
        const int rb = 4 * (w >> 2) + (m >> 1), cb = 2 * (w & 3) + (m & 1);
        if (dtile && rb < cb) return;
        const bool dblk = dtile && rb == cb;
        const int gc = tb * kSyTile + cb * 32 + (lane & 31);
#pragma unroll
        for (int q4 = 0; q4 < 4; ++q4) {
          const int gr0 = ta * kSyTile + rb * 32 + 8 * q4 + 4 * (lane >> 5);
          float v[4];
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const int gr = gr0 + e;
            v[e] = (gr < a.T && gc < a.T && gc < gr) ? acc[m][4 * q4 + e] : 0.f;
            if (gr < tpad && gc < tpad && (!dblk || gc <= gr)) g[int64_t(gr) * tpad + gc] = f2bf(v[e]);
          }
          if (gc < tpad && gr0 < tpad) {  // tpad % 4 == 0: all four rows in range
            bf16_t* gt = g + int64_t(gc) * tpad + gr0;
            if (!dblk) {
              uint32_t wv[2] = {pack_bf2(v[0], v[1]), pack_bf2(v[2], v[3])};
              *reinterpret_cast<uint2*>(gt) = make_uint2(wv[0], wv[1]);
            } else {
#pragma unroll
              for (int e = 0; e < 4; ++e)
                if (gc < gr0 + e) gt[e] = f2bf(v[e]);
            }
          }
        }
      });
      return;
    }
    if (tile_out < 0) return;
    // partial tile(s) as bf16 in fragment order (see sy_piece)
    const int wslot = WT == 0 ? w : (w & 3);
    bf16_t* dst = a.part + ((int64_t(slab) * a.ntl + tile_out) * S + split) * kSyTileElems + wslot * NM * 1024 +
                  lane * 8;
    sy_static_for<NM>([&](auto mc) {
      constexpr int m = decltype(mc)::value;
      uint32_t pk[8];
#pragma unroll
      for (int r = 0; r < 8; ++r) pk[r] = pack_bf2(acc[m][2 * r], acc[m][2 * r + 1]);
      *reinterpret_cast<u32x4*>(dst + m * 1024) = u32x4{pk[0], pk[1], pk[2], pk[3]};
      *reinterpret_cast<u32x4*>(dst + m * 1024 + 512) = u32x4{pk[4], pk[5], pk[6], pk[7]};
    });
  };
  if constexpr (REL) {
    // the frequencies of this workgroup's stages into the fifth slot (plain
    // loads and stores, before any DMA is in flight)
    float* const pf = reinterpret_cast<float*>(sy_lds + 4 * kSySlot);
    for (int i = tid; i < nst * 16; i += kSyThreads) pf[i] = a.freqs[kofs(i >> 4) + 2 * (i & 15)];
    __syncthreads();
  }
  if (!diag) {
    run(std::integral_constant<int, 0>());
  } else {
    switch (w & 3) {
      case 0: run(std::integral_constant<int, 1>()); break;
      case 1: run(std::integral_constant<int, 2>()); break;
      case 2: run(std::integral_constant<int, 3>()); break;
      default: run(std::integral_constant<int, 4>()); break;
    }
  }
}

// ------------------------------------------------ backward: dQ = G X
// dQ[slab] = G[slab] X[slab] for self attention (G = dS + dS^T, bf16, T x T
// padded to tpad with zeros), X (T x N) bf16 row-major.  The contraction runs
// over time, which is X's row index, so the B operand tiles are taken from X
// as stored: 32 rows x 256 columns per k32 stage, DMA'd row-major into LDS
// and read as MFMA B fragments with ds_read_b64_tr_b16.  Within each 16-lane
// group that instruction hands lane i element i % 4 of the 8-byte chunks
// addressed by group lanes i / 4 + 4 k (k = 0..3); so group lane q = 4 k + c
// addresses row k0 + k, columns nb + 4 c .. + 3 and lane i receives
// X[k0 .. k0 + 3][nb + i], half of a B fragment.
//  * 256 x 256 output tiles, full K per workgroup (no partials), every tile of
//    a slab on one XCD; the ring, barriers and waits are those of k_sy_scores
//    (full tile, no RoPE).
//  * A (G rows) uses the 64-byte-row swizzle of k_sy_scores; B rows are 512
//    bytes with 16-byte chunk c stored at c ^ 4 (row & 3), so the four rows of
//    one transposing read fall in different banks.
//  * KM (G exactly symmetric, as the score kernel's G epilogue writes it):
//    A[i][t] = G[t][i], so A is staged like B, 32 rows t x 512 bytes of
//    columns i per stage, and read with the same transposing loads.  Every
//    DMA row piece is then 512 bytes (four whole 128-byte lines) instead of
//    A's 64-byte halves of a line: a stage needs 256 line requests instead of
//    384, and the L1-to-L2 request stream, not the MFMAs, bounds this kernel.
//    The products are the same bits (the same G values, the same order).
typedef __attribute__((__vector_size__(4 * sizeof(__bf16)))) __bf16 bf16x4;
typedef __attribute__((address_space(3))) bf16x4 lds_bf16x4;

struct DqsArgs {
  const bf16_t* g;  // [slab][tpad][tpad]
  const bf16_t* x;
  int64_t x0, x1, x2;  // element strides of X over (b, h, t)
  void* o;
  int64_t o0, o1, o2;
  int H, T, N, tpad, nslab, nti, ntn;
  const float* freqs = nullptr;  // RoPE: the output is R^T(G X), positions rope_start + t
  int64_t rope_start = 0;
};

__device__ __forceinline__ bf16x4 lds_tr4(const uint8_t* p) {
  return __builtin_amdgcn_ds_read_tr16_b64_v4bf16((lds_bf16x4*)(p));
}
typedef __attribute__((address_space(3))) bf16x8 lds_bf16x8;
// An LDS byte address as an LDS pointer: reads at a wave-uniform slot base plus
// a per-lane offset take one VALU add, and constant offsets go into the
// instruction's offset field.
__device__ __forceinline__ const lds_u8* lds_at(uint32_t addr) {
  return reinterpret_cast<const lds_u8*>(size_t(addr));
}
__device__ __forceinline__ bf16x4 lds_tr4(const lds_u8* p) {
  return __builtin_amdgcn_ds_read_tr16_b64_v4bf16((lds_bf16x4*)(p));
}

// ROTB (with ROPE): X is x itself and each lane rotates the B chunks it
// loaded (positions rope_start + row) in LDS after they land and before the
// barrier that hands the stage to the fragment reads, with the table
// kernel's (cos, sin) entries and the score kernel's rotation, so the
// product sees the bits of the R(x) copy the absolute score pass writes.
template <typename TO, bool ROPE = false, bool ROTB = false, bool KM = false>
__global__ __launch_bounds__(kSyThreads, 1) void k_dq_sy(const DqsArgs a) {
  static_assert(!ROTB || ROPE, "B rotation: RoPE output");
  const int bid = blockIdx.x;
  const int xcd = bid & 7, kk = bid >> 3;
  const int tiles = a.nti * a.ntn;
  const int grp = kk / tiles;
  const int slab = grp * 8 + xcd;
  if (slab >= a.nslab) return;
  const int tt = kk - grp * tiles;
  const int tn = tt / a.nti, ti = tt - tn * a.nti;
  const int b = slab / a.H, h = slab - b * a.H;
  const int tid = threadIdx.x, lane = tid & 63;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int nst = a.tpad / 32;
  const int i0 = ti * kSyTile, n0 = tn * kSyTile;
  const void* gbase = sgpr_ptr(a.g + int64_t(slab) * a.tpad * a.tpad);
  const void* xbase = sgpr_ptr(a.x + b * a.x0 + h * a.x1);
  const uint32_t lds0 = __builtin_amdgcn_readfirstlane((uint32_t)(uintptr_t)(lds_u8*)sy_lds);

  // DMA chunks of this lane: A (G rows) instructions 0-1, B (X rows) 2-3
  uint32_t aoff[2], bcol[2];
  int brow[2];
#pragma unroll
  for (int u = 0; u < 2; ++u) {
    const int q = (u * 8 + w) * 1024 + lane * 16;
    const int rb = q >> 9, pb = (q >> 4) & 31, pc = pb ^ (4 * (rb & 3));
    if constexpr (KM) {
      // row rb of the stage, columns i0 + 8 pc ..; columns past tpad (output
      // rows past tpad): garbage, not stored
      aoff[u] = uint32_t((rb * a.tpad + min(i0 + 8 * pc, a.tpad - 8)) * 2);
    } else {
      const int row = q >> 6;
      const int c = ((q >> 4) & 3) ^ ((row >> 2) & 3);
      const int gi = min(i0 + row, a.tpad - 1);  // rows past tpad: garbage, not stored
      aoff[u] = uint32_t((gi * a.tpad + 8 * c) * 2);
    }
    brow[u] = rb;
    bcol[u] = uint32_t((n0 + 8 * pc) * 2);
  }
  // ring of NX slots: stage st in slot st % NX, tracked as rotating scalar
  // slot indices in the loop (a modulo of the stage index made the compiler
  // rebuild every fragment address per stage)
  constexpr int NX = 5, lead = NX - 1;
  auto slot_addr = [&](int k) { return lds0 + uint32_t(k * kSySlot); };
  struct StageDma {
    uint32_t m0, ka, krow;
  };
  const uint32_t wl = lds0 + uint32_t(w) * 1024u;
  auto stage_dma = [&](int st, int k) {
    StageDma d;
    d.m0 = wl + uint32_t(k * kSySlot);
    const int sc = min(st, nst - 1);
    d.ka = KM ? uint32_t(sc) * uint32_t(64 * a.tpad) : uint32_t(sc * 64);  // tpad^2 * 2 < 2^31
    d.krow = uint32_t(sc * 32);
    return d;
  };
  auto dma_a = [&](const StageDma& d, auto uc) {
    constexpr int u = decltype(uc)::value;
    dma16<u * 8192>(d.m0, gbase, aoff[u] + d.ka);
  };
  auto dma_b = [&](const StageDma& d, auto uc) {
    constexpr int u = decltype(uc)::value;
    const int row = min(int(d.krow) + brow[u], a.T - 1);  // rows past T meet zero G columns
    dma16<kSyBlk + u * 8192>(d.m0, xbase, uint32_t(int64_t(row) * a.x2 * 2) + bcol[u]);
  };

  // fragments: A rows 4 wm + i; B columns 64 wn + 32 jb, two transposing reads each
  const int wm = w >> 2, wn = w & 3;
  uint32_t loff[2];
#pragma unroll
  for (int k2 = 0; k2 < 2; ++k2) {
    const int c = (2 * k2 + (lane >> 5)) ^ ((lane >> 2) & 3);
    loff[k2] = uint32_t((lane & 31) * 64 + c * 16);
  }
  const int g4 = lane >> 4, q = lane & 15;
  // transposing-read address of 32 columns from col0 in a 32 x 512-byte block
  auto tr_off = [&](int col0) {
    const int col = col0 + 16 * (g4 & 1) + 4 * (q & 3);
    const int row = 8 * (g4 >> 1) + (q >> 2);
    return row * 512 + (((col >> 3) ^ (4 * (row & 3))) * 16) + ((col >> 2) & 1) * 8;
  };
  int boff[2];
#pragma unroll
  for (int jb = 0; jb < 2; ++jb) boff[jb] = kSyBlk + tr_off(64 * wn + 32 * jb);
  // KM: A rows 128 wm + 32 i as columns of the stage's A block
  int akm[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) akm[i] = KM ? tr_off(128 * wm + 32 * i) : 0;
  f32x16 acc[8];
#pragma unroll
  for (int i = 0; i < 8; ++i)
#pragma unroll
    for (int r = 0; r < 16; ++r) acc[i][r] = 0.f;
  // B rotation: this lane's two chunks of each stage (rows brow[u], pairs
  // from element bcol[u] / 2) and their frequencies
  float bfq[2][4];
  if constexpr (ROTB) {
#pragma unroll
    for (int u = 0; u < 2; ++u)
#pragma unroll
      for (int j = 0; j < 4; ++j) bfq[u][j] = a.freqs[(bcol[u] >> 1) + 2 * j];
  }
  auto rotate_b = [&](int st, int k) __attribute__((always_inline)) {
    if constexpr (ROTB) {
#pragma unroll
      for (int u = 0; u < 2; ++u) {
        uint8_t* const pc = sy_lds + k * kSySlot + kSyBlk + u * 8192 + w * 1024 + lane * 16;
        const u32x4 xv = *reinterpret_cast<const u32x4*>(pc);
        const float pos = float(a.rope_start + st * 32 + brow[u]);
        const u32x4 cs{rope_cs(pos, bfq[u][0]), rope_cs(pos, bfq[u][1]), rope_cs(pos, bfq[u][2]),
                       rope_cs(pos, bfq[u][3])};
        *reinterpret_cast<u32x4*>(pc) = rot_chunk<false>(xv, cs);
      }
    }
  };
  bf16x8 f0[6], f1[6];
  // sa: LDS address of the stage's slot (wave-uniform)
  auto read_frags = [&](bf16x8(&f)[6], uint32_t sa, int hf) {
    if constexpr (KM) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const lds_u8* pa = lds_at(sa + uint32_t(akm[i])) + hf * 16 * 512;
        const bf16x4 lo = lds_tr4(pa), hi = lds_tr4(pa + 4 * 512);
        f[i] = __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
      }
    } else {
      const lds_u8* pa = lds_at(sa + uint32_t(wm * 8192) + loff[hf]);
#pragma unroll
      for (int i = 0; i < 4; ++i) f[i] = *reinterpret_cast<const lds_bf16x8*>(pa + i * 2048);
    }
#pragma unroll
    for (int jb = 0; jb < 2; ++jb) {
      const lds_u8* pb = lds_at(sa + uint32_t(boff[jb])) + hf * 16 * 512;
      const bf16x4 lo = lds_tr4(pb), hi = lds_tr4(pb + 4 * 512);
      f[4 + jb] = __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
    }
  };
  using I0 = std::integral_constant<int, 0>;
  using I1 = std::integral_constant<int, 1>;

  // prologue: stages 0 .. lead-1, then stage 0 landed
  for (int st = 0; st < lead; ++st) {
    const StageDma d = stage_dma(st, st);
    dma_a(d, I0());
    dma_a(d, I1());
    dma_b(d, I0());
    dma_b(d, I1());
  }
  sy_wait<(lead - 1) * 4>();
  rotate_b(0, 0);
  sy_barrier();
  read_frags(f0, slot_addr(0), 0);
  // stage s: second-half fragment reads; first-half MFMAs with the A chunks of
  // stage s + lead; wait for stage s+1; barrier; first-half fragments of s+1;
  // second-half MFMAs with the B chunks of stage s + lead.  Slots: ks of
  // stage s, kn of s + 1, kl of s + lead (= s - 1 mod NX).
  int ks = 0;
  for (int s = 0; s + 1 < nst; ++s) {
    const int kn = ks == NX - 1 ? 0 : ks + 1, kl = ks == 0 ? NX - 1 : ks - 1;
    read_frags(f1, slot_addr(ks), 1);
    __builtin_amdgcn_sched_barrier(0);
    const StageDma d = stage_dma(s + lead, kl);
    sy_static_for<8>([&](auto mc) {
      constexpr int m = decltype(mc)::value;
      acc[m] = mma(f0[m >> 1], f0[4 + (m & 1)], acc[m]);
      if constexpr (m == 0) dma_a(d, I0());
      if constexpr (m == 2) dma_a(d, I1());
      if constexpr (m == 3) sy_wait<(lead - 2) * 4 + 2>();  // stage s+1 landed
    });
    __builtin_amdgcn_sched_barrier(0);
    rotate_b(s + 1, kn);
    sy_barrier();
    read_frags(f0, slot_addr(kn), 0);
    __builtin_amdgcn_sched_barrier(0);
    sy_static_for<8>([&](auto mc) {
      constexpr int m = decltype(mc)::value;
      acc[m] = mma(f1[m >> 1], f1[4 + (m & 1)], acc[m]);
      if constexpr (m == 1) dma_b(d, I0());
      if constexpr (m == 3) dma_b(d, I1());
    });
    ks = kn;
  }
  read_frags(f1, slot_addr(ks), 1);
  sy_static_for<8>([&](auto mc) {
    constexpr int m = decltype(mc)::value;
    acc[m] = mma(f0[m >> 1], f0[4 + (m & 1)], acc[m]);
  });
  sy_static_for<8>([&](auto mc) {
    constexpr int m = decltype(mc)::value;
    acc[m] = mma(f1[m >> 1], f1[4 + (m & 1)], acc[m]);
  });
  sy_wait<0>();  // the re-loads past the end land before the LDS is freed

  TO* o = static_cast<TO*>(a.o) + b * a.o0 + h * a.o1;
  // Element (m, r) of this lane: row i0 + 128 wm + rr(m, r) + 4 (lane >> 5),
  // column n0 + 64 wn + 32 (m & 1) + (lane & 31).  On a full row block (every
  // row below T; wave-uniform) each store's row base is a scalar pointer and
  // the lane's part a 32-bit offset (the host keeps 4 rows of out below 2^31
  // bytes), so the stores need no per-lane 64-bit address arithmetic and no
  // exec-mask branch; the last, partial row block keeps the per-row check.
  auto rr_of = [](int m, int r) { return 32 * (m >> 1) + 8 * (r >> 2) + (r & 3); };
  char* const ob = reinterpret_cast<char*>(o + int64_t(i0 + 128 * wm) * a.o2 + (n0 + 64 * wn));
  const int64_t o2b = a.o2 * int64_t(sizeof(TO));
  const uint32_t lofs = uint32_t(4 * (lane >> 5)) * uint32_t(o2b) + uint32_t((lane & 31) * sizeof(TO));
  auto epilogue = [&](auto fullc) __attribute__((always_inline)) {
    constexpr bool FULL = decltype(fullc)::value;
    auto put = [&](int m, int r, float y) __attribute__((always_inline)) {
      if constexpr (FULL) {
        char* const rp = ob + int64_t(rr_of(m, r)) * o2b + 32 * (m & 1) * int(sizeof(TO));
        *reinterpret_cast<TO*>(rp + lofs) = from_f<TO>(y);
      } else {
        const int row = i0 + 128 * wm + rr_of(m, r) + 4 * (lane >> 5);
        const int col = n0 + 64 * wn + 32 * (m & 1) + (lane & 31);
        if (row < a.T) o[int64_t(row) * a.o2 + col] = from_f<TO>(y);
      }
    };
    if constexpr (ROPE) {
      // R^T of the RoPE pair (2p, 2p + 1) = columns of lanes l and l ^ 1:
      // dx[2p] = g[2p] c + g[2p+1] s, dx[2p+1] = g[2p+1] c - g[2p] s, with the
      // (cos, sin) dword of rope_cs (the table kernel's bits) at position
      // rope_start + row, fp32 arithmetic, one rounding to TO
      // Lanes l and l ^ 1 share every (row, pair): each makes the dwords of the
      // values r with r % 2 == l % 2 and takes the others from its partner, and
      // partners swap values with a DPP quad permute (1, 0, 3, 2).
      const bool odd = (lane & 1) != 0;
      auto swap1 = [](uint32_t u) { return uint32_t(__builtin_amdgcn_mov_dpp(int(u), 0xB1, 0xF, 0xF, false)); };
      float fq[2];
#pragma unroll
      for (int u = 0; u < 2; ++u) fq[u] = a.freqs[(n0 + 64 * wn + 32 * u + (lane & 31)) & ~1];
#pragma unroll
      for (int m = 0; m < 8; ++m)
#pragma unroll
        for (int r = 0; r < 16; r += 2) {
          const int row0 = i0 + 128 * wm + rr_of(m, r) + 4 * (lane >> 5);
          // this lane makes the dword of value r + (lane & 1); the partner the other
          const uint32_t mine = rope_cs(float(a.rope_start + row0 + (odd ? 1 : 0)), fq[m & 1]);
          const uint32_t theirs = swap1(mine);
          const uint32_t cws[2] = {odd ? theirs : mine, odd ? mine : theirs};
#pragma unroll
          for (int e = 0; e < 2; ++e) {
            const float v = acc[m][r + e];
            const float pv = __uint_as_float(swap1(__float_as_uint(v)));
            const float c = __uint_as_float(cws[e] << 16), sn = __uint_as_float(cws[e] & 0xffff0000u);
            const float y = odd ? fmaf(v, c, -(pv * sn)) : fmaf(v, c, pv * sn);
            put(m, r + e, y);
          }
        }
    } else {
#pragma unroll
      for (int m = 0; m < 8; ++m)
#pragma unroll
        for (int r = 0; r < 16; ++r) put(m, r, acc[m][r]);
    }
  };
  if (i0 + kSyTile <= a.T)
    epilogue(std::true_type());
  else
    epilogue(std::false_type());
}

// ---------------------------------------- backward: dV from score tiles
// dV[b, hv, j, :] = sum over heads h and rows i > j of M_h[i, j] dO_h[i, :],
// M from the partial score tiles of k_sy_scores (split sum in fp32, one
// rounding to bf16).  Rows j in blocks of 64 per workgroup, all D (<= 256)
// columns.  The workgroup's items, (head, 64-row chunk of i >= j0), are
// dealt alternately to two groups of four waves; in a group wave w owns
// columns [64 w, +64).  Per item the M block (64 i x 64 j) and the dO block
// (64 i x 256 d) are staged row-major in the group's LDS, and both MFMA
// operands (M^T as A, dO as B, both contracting over i, their row index) are
// read with ds_read_b64_tr_b16.  A group's next item is loaded while it runs
// the current one's MFMAs.  The second group's fp32 sums are added to the
// first's through LDS at the end.  Two groups halve the longest workgroup's
// chain of items (the row block j0 = 0 has H * T / 64 of them) and keep two
// items' loads in flight per CU.
// Every row block of one (b, hv) reads the same dO rows, so those workgroups
// share an XCD (its L2): units u = (b Hv + hv) nrb + rb go to the XCDs in
// contiguous ranges of per_xcd, and each workgroup walks its i chunks from the
// last one down, the heads inside, so they read each dO chunk at about the
// same time.
struct DvsArgs {
  const bf16_t* part;  // [slab][ntl][nsplit][256*256]
  int ntl, nsplit;
  const bf16_t* dO;
  int64_t d0, d1, d2;
  void* o;
  int64_t o0, o1, o2;
  int H, Hv, T, D;
  int rel = 0;  // the tiles came from the relative-RoPE score kernel (fragment slot order)
  int nrb = 0, nbv = 0, per_xcd = 0;  // row blocks, B Hv, units per XCD (grid 8 per_xcd)
};

template <typename TO, int NS>
__global__ __launch_bounds__(512) void k_dv_sy(const DvsArgs a) {
  // two groups of four waves, each with its own staging blocks:
  // M [i][j] (16-byte chunk c at c ^ 2 (i & 3)) and dO [i][d] (chunk c at c ^ 4 (i & 3))
  constexpr int kBlk = 64 * 128 + 64 * 512;
  __shared__ __attribute__((aligned(16))) uint8_t dv_lds[2 * kBlk];
  // workgroup L runs on XCD L % 8 (round robin by linear id)
  const int L = blockIdx.x, u = (L & 7) * a.per_xcd + (L >> 3);
  if (u >= a.nrb * a.nbv) return;
  const int bv = u / a.nrb, rb = u - bv * a.nrb;
  const int b = bv / a.Hv, hv = bv - b * a.Hv;
  const int j0 = rb * 64;
  const int tid = threadIdx.x, grp = tid >> 8, gt = tid & 255, w = gt >> 6, lane = tid & 63;
  uint8_t* const mblk = dv_lds + grp * kBlk;
  uint8_t* const dblk = mblk + 64 * 128;
  const int h_lo = a.Hv == 1 ? 0 : hv, h_hi = a.Hv == 1 ? a.H : hv + 1;
  const int ic0 = j0 / 64, nic = (a.T + 63) / 64;  // chunks of i: i >= j0 (i > j)
  const int tj = j0 >> 8;
  // items it = (chunk nic - 1 - it / nhv, head h_lo + it % nhv); group g takes
  // items g, g + 2, ... (ng of them), both groups step together (nk steps)
  const int nhv = h_hi - h_lo;
  const int total = (nic - ic0) * nhv;
  const int ng = (total - grp + 1) / 2, nk = (total + 1) / 2;
  auto item_ic = [&](int it) { return nic - 1 - it / nhv; };

  // builder roles: M pieces (fragment-ordered partial tiles, see sy_piece):
  // piece e of this thread is 32 x 32 block mbi = (gt + 256 e) / 128 of the
  // 64 x 64 (i, j) chunk (rows i: mbi / 2, columns j: mbi % 2), lane
  // ((gt & 127) >> 1), half gt & 1; dO chunks e = gt + 256 u
  const int pl = (gt & 127) >> 1, ph = gt & 1;
  uint4 mp[NS][2];
  uint4 dp[8];
  // Steps past a group's last item load the workgroup's last item again (an
  // L2 hit, not used); splits past nsplit re-read the last split (not summed).
  auto load_chunk = [&](int itq) {
    const int it = min(itq, total - 1);
    const int ic = item_ic(it), h = h_lo + it - (nic - 1 - ic) * nhv;
    const int i0 = ic * 64;
    const int ti = i0 >> 8;
    const int slab = b * a.H + h;
    const bool dt = ti == tj;
    const bf16_t* p = a.part + ((int64_t(slab) * a.ntl + ti * (ti + 1) / 2 + tj) * a.nsplit) * kSyTileElems;
#pragma unroll
    for (int e = 0; e < 2; ++e) {
      const int mbi = (gt >> 7) + 2 * e;
      const int rbk = ((i0 & 255) >> 5) + (mbi >> 1), cbk = ((j0 & 255) >> 5) + (mbi & 1);
      // (no blocks above a diagonal tile's diagonal: read the diagonal block, masked below)
      const int off = sy_piece(dt, a.rel, rbk, dt && cbk > rbk ? rbk : cbk, pl, ph);
#pragma unroll
      for (int sp = 0; sp < NS; ++sp)
        mp[sp][e] = *reinterpret_cast<const uint4*>(p + int64_t(min(sp, a.nsplit - 1)) * kSyTileElems + off);
    }
    const bf16_t* dob = a.dO + b * a.d0 + h * a.d1;
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      const int e = gt + 256 * u, r = e >> 5, c = e & 31;
      const int ig = i0 + r;
      dp[u] = (ig < a.T && 8 * c < a.D) ? *reinterpret_cast<const uint4*>(dob + int64_t(ig) * a.d2 + 8 * c)
                                        : uint4{0u, 0u, 0u, 0u};
    }
  };
  auto store_chunk = [&](int it, bool live) {
    const int ic = item_ic(min(it, total - 1));
#pragma unroll
    for (int e = 0; e < 2; ++e) {
      float sacc[8];
#pragma unroll
      for (int q = 0; q < 8; ++q) sacc[q] = 0.f;
#pragma unroll
      for (int sp = 0; sp < NS; ++sp) {
        if (sp >= a.nsplit) break;  // uniform
        const uint32_t xw[4] = {mp[sp][e].x, mp[sp][e].y, mp[sp][e].z, mp[sp][e].w};
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          sacc[2 * q] += __uint_as_float(xw[q] << 16);
          sacc[2 * q + 1] += __uint_as_float(xw[q] & 0xffff0000u);
        }
      }
      const int mbi = (gt >> 7) + 2 * e;
      const int lj = (mbi & 1) * 32 + (pl & 31), gj = j0 + lj;
#pragma unroll
      for (int q = 0; q < 4; ++q)
#pragma unroll
        for (int u = 0; u < 2; ++u) {
          const int li = (mbi >> 1) * 32 + sy_piece_row(pl, ph, q, u), gi = ic * 64 + li;
          const float val = (live && gi < a.T && gi > gj) ? sacc[2 * q + u] : 0.f;
          *reinterpret_cast<bf16_t*>(mblk + li * 128 + (((lj >> 3) ^ (2 * (li & 3))) * 16) + (lj & 7) * 2) = f2bf(val);
        }
    }
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      const int e = gt + 256 * u, r = e >> 5, c = e & 31;
      *reinterpret_cast<uint4*>(dblk + r * 512 + ((c ^ (4 * (r & 3))) * 16)) = dp[u];
    }
  };
  // transposing fragment reads: group lane q addresses row kbase + 4 t + q / 4,
  // columns nb + 4 (q % 4)
  const int g4 = lane >> 4, q = lane & 15;
  int aoff[2], boff[2];
#pragma unroll
  for (int x = 0; x < 2; ++x) {
    const int row = 8 * (g4 >> 1) + (q >> 2);
    const int cm = 32 * x + 16 * (g4 & 1) + 4 * (q & 3);            // j column of M
    aoff[x] = row * 128 + (((cm >> 3) ^ (2 * (row & 3))) * 16) + ((cm >> 2) & 1) * 8;
    const int cd = 64 * w + 32 * x + 16 * (g4 & 1) + 4 * (q & 3);   // d column of dO
    boff[x] = row * 512 + (((cd >> 3) ^ (4 * (row & 3))) * 16) + ((cd >> 2) & 1) * 8;
  }
  f32x16 acc[2][2];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int c = 0; c < 2; ++c)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][c][r] = 0.f;

  load_chunk(grp);
  // step k: the group's item grp + 2 k into its blocks, then the load of item
  // grp + 2 (k + 1), then the MFMAs.  A group past its last item stages a
  // zero M block (its MFMAs add zeros).
  for (int k = 0; k < nk; ++k) {
    __syncthreads();  // the previous step's fragment reads are done
    store_chunk(grp + 2 * k, k < ng);
    load_chunk(grp + 2 * (k + 1));
    __syncthreads();
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) {
      bf16x8 fa[2], fb[2];
#pragma unroll
      for (int x = 0; x < 2; ++x) {
        const uint8_t* pa = mblk + aoff[x] + ks * 16 * 128;
        fa[x] = __builtin_shufflevector(lds_tr4(pa), lds_tr4(pa + 4 * 128), 0, 1, 2, 3, 4, 5, 6, 7);
        const uint8_t* pb = dblk + boff[x] + ks * 16 * 512;
        fb[x] = __builtin_shufflevector(lds_tr4(pb), lds_tr4(pb + 4 * 512), 0, 1, 2, 3, 4, 5, 6, 7);
      }
#pragma unroll
      for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int c = 0; c < 2; ++c) acc[i][c] = mma(fa[i], fb[c], acc[i][c]);
    }
  }
  // group 1's sums into group 0's
  __syncthreads();  // the blocks' last fragment reads are done
  float* const red = reinterpret_cast<float*>(dv_lds);  // [wave][value][lane], 64 KB
  if (grp == 1) {
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int c = 0; c < 2; ++c)
#pragma unroll
        for (int r = 0; r < 16; ++r) red[(w * 64 + (i * 2 + c) * 16 + r) * 64 + lane] = acc[i][c][r];
  }
  __syncthreads();
  if (grp == 1) return;
  TO* o = static_cast<TO*>(a.o) + b * a.o0 + hv * a.o1;
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int c = 0; c < 2; ++c)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int j = j0 + 32 * i + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
        const int d = 64 * w + 32 * c + (lane & 31);
        const float val = acc[i][c][r] + red[(w * 64 + (i * 2 + c) * 16 + r) * 64 + lane];
        if (j < a.T && d < a.D) o[int64_t(j) * a.o2 + d] = from_f<TO>(val);
      }
}

// dV from score tiles of one split through an LDS ring: the k_dv_sy work
// (64 rows j of dV[b, hv] per workgroup, all D <= 256 columns; the same
// units per XCD and the same item order) with every operand moved by DMA.
// Per item the four 32 x 32 blocks of M, as the score kernel stored them
// (MFMA accumulator order, 2 KB a block), and the 64 dO rows (512-byte rows,
// 16-byte chunk c at c ^ 4 (i & 3)) go to a ring of three stages, two items
// in flight while one is multiplied.  A stored accumulator half (1 KB) is an A
// operand of M^T as it stands: lane l holds column j = l % 32 and rows
// 16 hf + 8 (t / 4) + 4 (l / 32) + t % 4 of the block for t = 0..7, so the
// MFMA's contraction index 8 (l / 32) + t runs over those rows, and the B
// operand (dO) is read in the same row order (two transposing reads eight
// rows apart).  Waves 0-3 contract rows 0-31 of each item, waves 4-7 rows
// 32-63; wave w & 3 owns columns [64 (w & 3), +64) and both 32-row halves of
// j.  Entries with i <= j (the diagonal chunk, whose block above the diagonal
// is not stored: the diagonal block is read in its place) or i >= T are
// zeroed in the A registers.  At the end the two halves' sums meet in LDS and
// the 64 x D tile leaves in 16-byte stores.
constexpr int kDvStage = 8192 + 64 * 512;  // M blocks + dO rows
constexpr int kDvRing = 3;
constexpr int kDvPitch = 1056;  // output tile row pitch in bytes (rows 4 apart on other banks)

template <typename TO>
__global__ __launch_bounds__(512, 1) void k_dv_dma(const DvsArgs a) {
  __shared__ __attribute__((aligned(1024))) uint8_t dv_ring[kDvRing * kDvStage];
  const int L = blockIdx.x, u = (L & 7) * a.per_xcd + (L >> 3);
  if (u >= a.nrb * a.nbv) return;
  const int bv = u / a.nrb, rb = u - bv * a.nrb;
  const int b = bv / a.Hv, hv = bv - b * a.Hv;
  const int j0 = rb * 64, tj = j0 >> 8;
  const int tid = threadIdx.x, lane = tid & 63;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int h_lo = a.Hv == 1 ? 0 : hv, nhv = a.Hv == 1 ? a.H : 1;
  const int nic = (a.T + 63) / 64;
  const int total = (nic - rb) * nhv;
  const uint32_t lds0 = __builtin_amdgcn_readfirstlane((uint32_t)(uintptr_t)(lds_u8*)dv_ring);

  // DMA roles: wave w moves half w & 1 of M block (ib, jb) = (w >> 2, (w >> 1) & 1)
  // and dO rows 8 w + 2 v + lane / 32 (v = 0..3); chunks past D re-read the last one
  const int mhf = w & 1, cbk = ((j0 & 255) >> 5) + ((w >> 1) & 1), mib = w >> 2;
  int drow[4];
  uint32_t dcol[4];
#pragma unroll
  for (int v = 0; v < 4; ++v) {
    const int r = 8 * w + 2 * v + (lane >> 5);
    drow[v] = r;
    dcol[v] = uint32_t(min((lane & 31) ^ (4 * (r & 3)), a.D / 8 - 1) * 16);
  }
  auto issue = [&](int it, int slot) __attribute__((always_inline)) {
    const int c = it / nhv, ic = nic - 1 - c, h = h_lo + it - c * nhv;
    const int i0 = ic * 64, ti = i0 >> 8;
    const bool dt = ti == tj;
    const int rbk = ((i0 & 255) >> 5) + mib;
    const bf16_t* tile = a.part + (int64_t(b * a.H + h) * a.ntl + ti * (ti + 1) / 2 + tj) * kSyTileElems;
    const int off = sy_piece(dt, a.rel, rbk, dt && cbk > rbk ? rbk : cbk, lane, mhf);
    const uint32_t sb = lds0 + uint32_t(slot * kDvStage);
    dma16<0>(sb + uint32_t(w) * 1024u, sgpr_ptr(tile), uint32_t(off * 2));
    const void* dob = sgpr_ptr(a.dO + b * a.d0 + h * a.d1);
    const uint32_t dm0 = sb + 8192u + uint32_t(w) * 4096u;
    dma16<0>(dm0, dob, uint32_t(min(i0 + drow[0], a.T - 1)) * uint32_t(a.d2 * 2) + dcol[0]);
    dma16<1024>(dm0, dob, uint32_t(min(i0 + drow[1], a.T - 1)) * uint32_t(a.d2 * 2) + dcol[1]);
    dma16<2048>(dm0, dob, uint32_t(min(i0 + drow[2], a.T - 1)) * uint32_t(a.d2 * 2) + dcol[2]);
    dma16<3072>(dm0, dob, uint32_t(min(i0 + drow[3], a.T - 1)) * uint32_t(a.d2 * 2) + dcol[3]);
  };

  // fragments: A (M^T) halves of blocks (kq, jb); B (dO) rows 16 ks + 4 (l / 32)
  // + q / 4 and 8 below, columns 64 wc + 32 c + 16 ((l / 16) & 1) + 4 (q % 4)
  const int kq = w >> 2, wc = w & 3;
  const int g4 = lane >> 4, q = lane & 15;
  uint32_t boff[2];
#pragma unroll
  for (int c = 0; c < 2; ++c) {
    const int row = 4 * (g4 >> 1) + (q >> 2);
    const int col = 64 * wc + 32 * c + 16 * (g4 & 1) + 4 * (q & 3);
    boff[c] = uint32_t(8192 + row * 512 + (((col >> 3) ^ (4 * (row & 3))) * 16) + ((col >> 2) & 1) * 8);
  }
  f32x16 acc[2][2];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int c = 0; c < 2; ++c)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][c][r] = 0.f;

  issue(0, 0);
  if (total > 1) issue(1, 1);
  int slot = 0;
  for (int k = 0; k < total; ++k) {
    if (k + 1 < total) sy_wait<5>();  // item k landed, item k + 1 in flight
    else sy_wait<0>();
    __syncthreads();  // item k in every wave's view; item k - 1's stage is free
    if (k + 2 < total) issue(k + 2, slot == 0 ? 2 : slot - 1);
    const int ic = nic - 1 - k / nhv;
    const bool msk = ic == rb || ic * 64 + 64 > a.T;  // uniform
    const uint32_t sb = lds0 + uint32_t(slot * kDvStage);
#pragma unroll
    for (int hf = 0; hf < 2; ++hf) {
      const int ks = 2 * kq + hf;
      bf16x8 fa[2], fb[2];
#pragma unroll
      for (int jb = 0; jb < 2; ++jb) {
        fa[jb] = *reinterpret_cast<const lds_bf16x8*>(lds_at(sb + uint32_t(((2 * kq + jb) * 2 + hf) * 1024 + lane * 16)));
        if (msk) {
          u32x4 wv = __builtin_bit_cast(u32x4, fa[jb]);
          const int ib0 = ic * 64 + 16 * ks + 4 * (lane >> 5);
          const int gj = j0 + 32 * jb + (lane & 31);
#pragma unroll
          for (int p = 0; p < 4; ++p) {
            const int il = ib0 + 8 * (p >> 1) + 2 * (p & 1);
            const uint32_t keep = ((il > gj && il < a.T) ? 0xffffu : 0u) | ((il + 1 > gj && il + 1 < a.T) ? 0xffff0000u : 0u);
            wv[p] &= keep;
          }
          fa[jb] = __builtin_bit_cast(bf16x8, wv);
        }
      }
#pragma unroll
      for (int c = 0; c < 2; ++c) {
        const lds_u8* pb = lds_at(sb + boff[c] + uint32_t(ks * 16 * 512));
        fb[c] = __builtin_shufflevector(lds_tr4(pb), lds_tr4(pb + 8 * 512), 0, 1, 2, 3, 4, 5, 6, 7);
      }
#pragma unroll
      for (int jb = 0; jb < 2; ++jb)
#pragma unroll
        for (int c = 0; c < 2; ++c) acc[jb][c] = mma(fa[jb], fb[c], acc[jb][c]);
    }
    slot = slot == 2 ? 0 : slot + 1;
  }

  // the two row halves' sums into one fp32 tile [64 j][pitch], then 16-byte stores
  __syncthreads();  // every wave's last fragment reads are done (its DMA waited above)
  float* const tl = reinterpret_cast<float*>(dv_ring);
  constexpr int PF = kDvPitch / 4;
  auto tile_idx = [&](int jb, int c, int r) {
    return (32 * jb + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3)) * PF + 64 * wc + 32 * c + (lane & 31);
  };
  if (kq == 1) {
#pragma unroll
    for (int jb = 0; jb < 2; ++jb)
#pragma unroll
      for (int c = 0; c < 2; ++c)
#pragma unroll
        for (int r = 0; r < 16; ++r) tl[tile_idx(jb, c, r)] = acc[jb][c][r];
  }
  __syncthreads();
  if (kq == 0) {
#pragma unroll
    for (int jb = 0; jb < 2; ++jb)
#pragma unroll
      for (int c = 0; c < 2; ++c)
#pragma unroll
        for (int r = 0; r < 16; ++r) tl[tile_idx(jb, c, r)] += acc[jb][c][r];
  }
  __syncthreads();
  TO* o = static_cast<TO*>(a.o) + b * a.o0 + hv * a.o1;
  if constexpr (sizeof(TO) == 2) {
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      const int e = tid + 512 * v, row = e >> 5, cc = e & 31;
      if (j0 + row < a.T && 8 * cc < a.D) {
        const f32x4 x0 = *reinterpret_cast<const f32x4*>(tl + row * PF + 8 * cc);
        const f32x4 x1 = *reinterpret_cast<const f32x4*>(tl + row * PF + 8 * cc + 4);
        *reinterpret_cast<u32x4*>(o + int64_t(j0 + row) * a.o2 + 8 * cc) =
            u32x4{pack_bf2(x0[0], x0[1]), pack_bf2(x0[2], x0[3]), pack_bf2(x1[0], x1[1]), pack_bf2(x1[2], x1[3])};
      }
    }
  } else {
#pragma unroll
    for (int v = 0; v < 8; ++v) {
      const int e = tid + 512 * v, row = e >> 6, cc = e & 63;
      if (j0 + row < a.T && 4 * cc < a.D)
        *reinterpret_cast<f32x4*>(o + int64_t(j0 + row) * a.o2 + 4 * cc) =
            *reinterpret_cast<const f32x4*>(tl + row * PF + 4 * cc);
    }
  }
}

// ------------------------------------------------------------- score x V
// out rows [64 rb, +64) of one (b,h) slab, all D (<= 256) columns.  Keys go
// in chunks of 64.  The 512 threads first stage the chunk in LDS: the score
// block (64 rows x 64 keys: the split sum of the partial rows in fp32, the
// strict-lower mask, one rounding to bf16), each thread 8 keys of one row,
// and the V rows of the chunk (64 x D, rounded to bf16), row-major as stored.
// Wave w then multiplies keys [32 (w / 4), +32) of the chunk into columns
// [64 (w % 4), +64): 2 x 2 blocks of 32 x 32, two k16 steps; A fragments are
// plain reads, B fragments (V, contracting over its row index)
// ds_read_b64_tr_b16 reads.  The two wave groups' sums are added through LDS
// at the end.  The loads of the next PF chunks are in flight while a chunk is
// processed.  Score rows are 128 bytes with 16-byte chunk kc at
// kc ^ ((r >> 1) & 7); V rows 512 bytes with chunk c at c ^ 4 (r & 3): both
// conflict free.
struct SvArgs {
  const bf16_t* part;  // partial score tiles [slab][ntl][nsplit][256*256]
  View v;              // V (B, Hv, T, D)
  int ntl, nsplit, H, Hv, T, D;
  View o;
  int t0 = 0;          // packed index of the first stored tile
  int rb0 = 0;         // first 64-row block (queries at an offset)
  int past = 0;        // rows below past are not stored; row i is stored at i - past
  int rel = 0;         // the tiles came from the relative-RoPE score kernel (fragment slot order)
  int self = 1;        // Q = K: diagonal tiles hold their 36 lower blocks (else every tile is full)
  int nrbk = 1;        // row blocks per slab in this launch
  int nslab = 0;
  int o16 = 0;         // output rows 16-byte aligned in groups of eight columns
};

template <typename TO, typename TV, int NS>
__global__ __launch_bounds__(512, 1) void k_sy_sv(const SvArgs a) {
  // 64 KB: the score and V blocks during the chunk loop, then the second wave
  // group's sums [wave][value][lane] (two workgroups fit a CU)
  __shared__ __attribute__((aligned(16))) uint8_t sv_lds[4 * 64 * 64 * 4];
  uint8_t* const blk = sv_lds;               // 64 x 128 bytes
  uint8_t* const vblk = sv_lds + 64 * 128;   // 64 x 512 bytes
  float* const red = reinterpret_cast<float*>(sv_lds);
  constexpr int VL = sizeof(TV) == 2 ? 1 : 2;  // 16-byte loads per 8 V elements
  // Workgroups go to the XCDs round robin by linear id L.  The row blocks of
  // slab s run on XCD s % 8, the XCD whose L2 took the slab's partial tiles
  // in the score kernel (this kernel serves the few-slab shapes that split K,
  // whose tiles fit the L2s).  On each XCD the row blocks go longest first
  // (block rb has rb + 1 key chunks): the k-th workgroup of XCD x is slab
  // 8 (k % nsx) + x, block nrbk - 1 - k / nsx, so when the grid takes more than
  // one round of the CUs the last workgroups to start are the short ones.
  const int nrbk = a.nrbk, nsx = (a.nslab + 7) / 8;
  const int L = blockIdx.x, xcdv = L & 7, kk = L >> 3;
  const int slab = (kk % nsx) * 8 + xcdv;
  if (slab >= a.nslab) return;
  const int rb = nrbk - 1 - kk / nsx + a.rb0;
  const int b = slab / a.H, h = slab - b * a.H, hv = a.Hv == 1 ? 0 : h;
  const int tid = threadIdx.x, w = tid >> 6, lane = tid & 63;
  const int r0 = rb * 64;
  const int kend = min(a.T, r0 + 64);  // keys j < rows of this block
  const int nch = (kend + 63) / 64;
  const bf16_t* pslab = a.part + int64_t(slab) * a.ntl * a.nsplit * kSyTileElems;
  const TV* vb = static_cast<const TV*>(a.v.p) + b * a.v.s0 + hv * a.v.s1;

  // block builder: one 16-byte piece of the fragment-ordered partial tiles
  // per split: 32 x 32 block sbi = (rows srh, keys skh) of the 64 x 64 chunk,
  // lane pl, half ph (8 values of one key column); V rows vr0 + 16 u, 16-byte
  // chunk vc of each (u = 0..3)
  const int sbi = tid >> 7, srh = sbi >> 1, skh = sbi & 1, pl = (tid & 127) >> 1, ph = tid & 1;
  const int ti = r0 >> 8;  // the tile row of all rows of this block (64 | 256)
  const int vr0 = tid >> 5, vc = tid & 31;
  // Loads are unconditional, from clamped addresses: splits past nsplit
  // re-read the last split (not summed), V rows past T re-read row T - 1 (their
  // scores are zero), V chunks past D re-read the last chunk (their output
  // columns are not stored).
  const int vcc = min(vc, a.D / 8 - 1);

  // chunks in flight: three while a chunk's loads take at most 8 registers
  // of 16 bytes per thread, else two
  constexpr int PF = NS + 4 * VL <= 8 ? 3 : 2;
  uint4 pr[PF][NS];    // partial rows of the chunks in flight
  uint4 vr[PF][4][VL];  // V rows of the chunks in flight
  auto load_chunk = [&](int ck, auto slotc) __attribute__((always_inline)) {
    constexpr int k = decltype(slotc)::value;
    const int j0 = ck * 64;
    const int tj = j0 >> 8;
    const int tile = ti * (ti + 1) / 2 + tj - a.t0;
    const int rbk = ((r0 & 255) >> 5) + srh, cbk = ((j0 & 255) >> 5) + skh;
    // a diagonal tile has no blocks above its diagonal: read the diagonal block
    // instead (masked to zero in store_chunk)
    const bool dt = a.self && ti == tj;
    const bf16_t* p = pslab + int64_t(tile) * a.nsplit * kSyTileElems +
                      sy_piece(dt, a.rel, rbk, dt && cbk > rbk ? rbk : cbk, pl, ph);
#pragma unroll
    for (int sp = 0; sp < NS; ++sp)
      pr[k][sp] = *reinterpret_cast<const uint4*>(p + int64_t(min(sp, a.nsplit - 1)) * kSyTileElems);
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const TV* vp = vb + int64_t(min(j0 + vr0 + 16 * u, a.T - 1)) * a.v.s2 + 8 * vcc;
#pragma unroll
      for (int l = 0; l < VL; ++l) vr[k][u][l] = *reinterpret_cast<const uint4*>(vp + 4 * l);
    }
  };
  // split sum, mask (j < i < T), one rounding, into the row-major score
  // block; then the V block as bf16
  auto store_chunk = [&](int ck, auto slotc) __attribute__((always_inline)) {
    constexpr int k = decltype(slotc)::value;
    float sacc[8];
#pragma unroll
    for (int q = 0; q < 8; ++q) sacc[q] = 0.f;
#pragma unroll
    for (int sp = 0; sp < NS; ++sp) {
      if (sp >= a.nsplit) break;  // uniform
      const uint32_t xw[4] = {pr[k][sp].x, pr[k][sp].y, pr[k][sp].z, pr[k][sp].w};
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        sacc[2 * q] += __uint_as_float(xw[q] << 16);
        sacc[2 * q + 1] += __uint_as_float(xw[q] & 0xffff0000u);
      }
    }
    const int key = skh * 32 + (pl & 31), gj = ck * 64 + key;
#pragma unroll
    for (int q = 0; q < 4; ++q)
#pragma unroll
      for (int e = 0; e < 2; ++e) {
        const int lr = srh * 32 + sy_piece_row(pl, ph, q, e), gi = r0 + lr;
        const float val = (gi < a.T && gj < gi) ? sacc[2 * q + e] : 0.f;
        *reinterpret_cast<bf16_t*>(blk + lr * 128 + (((key >> 3) ^ ((lr >> 1) & 7)) * 16) + (key & 7) * 2) = f2bf(val);
      }
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int r = vr0 + 16 * u, c = vc;
      u32x4 y;
      if constexpr (VL == 1) {
        y = u32x4{vr[k][u][0].x, vr[k][u][0].y, vr[k][u][0].z, vr[k][u][0].w};
      } else {
        const uint32_t f[8] = {vr[k][u][0].x, vr[k][u][0].y, vr[k][u][0].z, vr[k][u][0].w,
                               vr[k][u][1].x, vr[k][u][1].y, vr[k][u][1].z, vr[k][u][1].w};
        y = u32x4{pack_bf2(__uint_as_float(f[0]), __uint_as_float(f[1])), pack_bf2(__uint_as_float(f[2]), __uint_as_float(f[3])),
                  pack_bf2(__uint_as_float(f[4]), __uint_as_float(f[5])), pack_bf2(__uint_as_float(f[6]), __uint_as_float(f[7]))};
      }
      *reinterpret_cast<u32x4*>(vblk + r * 512 + ((c ^ (4 * (r & 3))) * 16)) = y;
    }
  };
  // MFMA roles: key half kh of each chunk, output columns [64 wc, +64).
  // B fragments: group lane q addresses V row 16 ks + 8 (g / 2) + 4 t + q / 4,
  // columns 64 wc + 32 c + 16 (g % 2) + 4 (q % 4)
  const int kh = w >> 2, wc = w & 3;
  const int g4 = lane >> 4, q = lane & 15;
  int boff[2];
  int dcol[2];
  bool dok[2];
#pragma unroll
  for (int c = 0; c < 2; ++c) {
    const int row = 8 * (g4 >> 1) + (q >> 2);
    const int cd = 64 * wc + 32 * c + 16 * (g4 & 1) + 4 * (q & 3);
    boff[c] = row * 512 + (((cd >> 3) ^ (4 * (row & 3))) * 16) + ((cd >> 2) & 1) * 8;
    dcol[c] = 64 * wc + 32 * c + (lane & 31);
    dok[c] = dcol[c] < a.D;
  }

  f32x16 acc[2][2];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int c = 0; c < 2; ++c)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][c][r] = 0.f;

  // Every processed chunk issues the same loads (chunks past the last re-read
  // the last one, an L2 hit), and the first PF chunks issue in slot order (no
  // scheduling across the barriers), so the compiler's wait before a chunk's
  // store leaves the PF - 1 chunks behind it in flight; a conditional load, or
  // slots interleaved at the start, make it wait for all of them.
  sy_static_for<PF>([&](auto kc) {
    load_chunk(min(int(decltype(kc)::value), nch - 1), kc);
    __builtin_amdgcn_sched_barrier(0);
  });
  // chunk ck from slot kc: staged into the blocks, then the slot refilled with
  // chunk ck + PF, then the MFMAs
  auto do_chunk = [&](int ck, auto kc) __attribute__((always_inline)) {
    __syncthreads();  // the previous chunk's fragment reads are done
    store_chunk(ck, kc);
    load_chunk(min(ck + PF, nch - 1), kc);
    __syncthreads();
#pragma unroll
    for (int k2 = 0; k2 < 2; ++k2) {
      const int ks = 2 * kh + k2;
      bf16x8 fa[2], fb[2];
#pragma unroll
      for (int i = 0; i < 2; ++i) {
        const int row = 32 * i + (lane & 31);
        const int kc2 = 2 * ks + (lane >> 5);
        fa[i] = *reinterpret_cast<const bf16x8*>(blk + row * 128 + ((kc2 ^ ((row >> 1) & 7)) * 16));
      }
#pragma unroll
      for (int c = 0; c < 2; ++c) {
        const uint8_t* pb = vblk + boff[c] + ks * 16 * 512;
        fb[c] = __builtin_shufflevector(lds_tr4(pb), lds_tr4(pb + 4 * 512), 0, 1, 2, 3, 4, 5, 6, 7);
      }
#pragma unroll
      for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int c = 0; c < 2; ++c) acc[i][c] = mma(fa[i], fb[c], acc[i][c]);
    }
  };
  // Full groups of PF chunks in the loop, the rest after it: a chunk skipped
  // inside the loop would reach the back edge with fewer loads issued, and
  // the compiler's waits would then drain every slot.
  int c0 = 0;
  for (; c0 + PF <= nch; c0 += PF)
    sy_static_for<PF>([&](auto kc) { do_chunk(c0 + int(decltype(kc)::value), kc); });
  sy_static_for<PF>([&](auto kc) {
    if (c0 + int(decltype(kc)::value) < nch) do_chunk(c0 + int(decltype(kc)::value), kc);
  });
  // add the second key half's sums (waves 4-7) into the first's (waves 0-3)
  __syncthreads();  // the blocks' last fragment reads are done
  if (kh == 1) {
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int c = 0; c < 2; ++c)
#pragma unroll
        for (int r = 0; r < 16; ++r) red[(wc * 64 + (i * 2 + c) * 16 + r) * 64 + lane] = acc[i][c][r];
  }
  __syncthreads();
  if (kh == 1) return;
  TO* o = static_cast<TO*>(const_cast<void*>(a.o.p)) + b * a.o.s0 + h * a.o.s1;
  if (!a.o16) {
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int c = 0; c < 2; ++c)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int row = r0 + 32 * i + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
          const float val = acc[i][c][r] + red[(wc * 64 + (i * 2 + c) * 16 + r) * 64 + lane];
          if (row >= a.past && row < a.T && dok[c]) o[int64_t(row - a.past) * a.o.s2 + dcol[c]] = from_f<TO>(val);
        }
    return;
  }
  // 16-byte output rows: wave wc sums its 64 x 64 block into its own 16 KB of
  // the reduction buffer (only it reads that region from here on), row-major
  // fp32, then writes the block back out as eight consecutive columns a lane
  // (one 16-byte store of bf16, two of fp32) instead of one element a store.
  float vals[2][2][16];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int c = 0; c < 2; ++c)
#pragma unroll
      for (int r = 0; r < 16; ++r) vals[i][c][r] = acc[i][c][r] + red[(wc * 64 + (i * 2 + c) * 16 + r) * 64 + lane];
  float* const ob = red + wc * 64 * 64;  // [64 rows][64 columns] of this wave
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int c = 0; c < 2; ++c)
#pragma unroll
      for (int r = 0; r < 16; ++r)
        ob[(32 * i + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3)) * 64 + 32 * c + (lane & 31)] = vals[i][c][r];
  asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");  // this wave's own writes
  const int lc = (lane & 7) * 8;  // first of the lane's eight columns
  const bool cok = 64 * wc + lc < a.D;
#pragma unroll
  for (int pass = 0; pass < 8; ++pass) {
    const int lr = pass * 8 + (lane >> 3), row = r0 + lr;
    const f32x4 v0 = *reinterpret_cast<const f32x4*>(ob + lr * 64 + lc);
    const f32x4 v1 = *reinterpret_cast<const f32x4*>(ob + lr * 64 + lc + 4);
    if (row < a.past || row >= a.T || !cok) continue;
    TO* dst = o + int64_t(row - a.past) * a.o.s2 + 64 * wc + lc;
    const float f[8] = {v0[0], v0[1], v0[2], v0[3], v1[0], v1[1], v1[2], v1[3]};
    if constexpr (sizeof(TO) == 2) {
      *reinterpret_cast<u32x4*>(dst) = u32x4{pack_bf2(f[0], f[1]), pack_bf2(f[2], f[3]), pack_bf2(f[4], f[5]),
                                             pack_bf2(f[6], f[7])};
    } else {
      *reinterpret_cast<f32x4*>(dst) = v0;
      *reinterpret_cast<f32x4*>(dst + 4) = v1;
    }
  }
}

// score x V from score tiles of one split through an LDS ring, V in bf16:
// the k_sy_sv work (64 output rows of one slab per workgroup, all D <= 256
// columns, key chunks of 64, the same grid) with every operand moved by DMA,
// in the stage layout of k_dv_dma: per chunk the four 32 x 32 blocks of M as
// the score kernel stored them (MFMA accumulator order) and the 64 V rows
// (512-byte rows, chunk c at c ^ 4 (j & 3)), three chunks in the ring.  The
// A operand (M, rows i, contracting over keys j) comes out of the stored
// accumulator order by transposing reads: within a group of 16 lanes, lane
// s = 4 e + m reads the 8 bytes that hold rows 4 m .. 4 m + 3 (of the group's
// 16) of key jbase + e, which sit in stored lane jbase + e + 32 (m & 1), bytes
// 8 (m >> 1) ..; the read hands lane q row q's four consecutive keys.  Stored
// lane L' of half hf lands in LDS slot L' ^ 4 (L' / 32) ^ 8 hf (the DMA lane
// loads the stored lane that belongs in its slot), which puts the two 64-byte
// runs of a group and the two halves on different banks.  Waves 0-3 contract
// the chunk's keys 0-31, waves 4-7 keys 32-63; wave w & 3 owns columns
// [64 (w & 3), +64) and both 32-row halves.  Entries with j >= i or i >= T are
// zeroed in the A registers; the two key halves' sums meet in LDS and leave in
// 16-byte stores (rows below past not stored, row i at i - past).
template <typename TO>
__global__ __launch_bounds__(512, 1) void k_sv_dma(const SvArgs a) {
  __shared__ __attribute__((aligned(1024))) uint8_t sv_ring[kDvRing * kDvStage];
  const int nrbk = a.nrbk, nsx = (a.nslab + 7) / 8;
  const int L = blockIdx.x, xcdv = L & 7, kk = L >> 3;
  const int slab = xcdv * nsx + kk % nsx;
  if (slab >= a.nslab) return;
  const int rb = nrbk - 1 - kk / nsx + a.rb0;
  const int b = slab / a.H, h = slab - b * a.H, hv = a.Hv == 1 ? 0 : h;
  const int tid = threadIdx.x, lane = tid & 63;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int r0 = rb * 64, ti = r0 >> 8;
  const int nch = (min(a.T, r0 + 64) + 63) / 64;
  const bf16_t* pslab = a.part + int64_t(slab) * a.ntl * kSyTileElems;
  const void* vbase = sgpr_ptr(static_cast<const bf16_t*>(a.v.p) + b * a.v.s0 + hv * a.v.s1);
  const uint32_t lds0 = __builtin_amdgcn_readfirstlane((uint32_t)(uintptr_t)(lds_u8*)sv_ring);

  // DMA roles: wave w moves half w & 1 of M block (ib, jb) = (w >> 2, (w >> 1) & 1)
  // (DMA lane l takes stored lane l ^ 4 (l / 32) ^ 8 hf) and V rows 8 w + 2 v + lane / 32
  const int mhf = w & 1, mjb = (w >> 1) & 1;
  const int rbk = ((r0 & 255) >> 5) + (w >> 2);
  const int mlane = lane ^ (4 * (lane >> 5)) ^ (8 * mhf);
  int vrow[4];
  uint32_t vcol[4];
#pragma unroll
  for (int v = 0; v < 4; ++v) {
    const int r = 8 * w + 2 * v + (lane >> 5);
    vrow[v] = r;
    vcol[v] = uint32_t(min((lane & 31) ^ (4 * (r & 3)), a.D / 8 - 1) * 16);
  }
  const uint32_t vpitch = uint32_t(a.v.s2 * 2);
  auto issue = [&](int ck, int slot) __attribute__((always_inline)) {
    const int j0 = ck * 64, tj = j0 >> 8;
    const bool dt = a.self && ti == tj;
    const int cbk = ((j0 & 255) >> 5) + mjb;
    const bf16_t* tile = pslab + int64_t(ti * (ti + 1) / 2 + tj - a.t0) * kSyTileElems;
    const int off = sy_piece(dt, a.rel, rbk, dt && cbk > rbk ? rbk : cbk, mlane, mhf);
    const uint32_t sb = lds0 + uint32_t(slot * kDvStage);
    dma16<0>(sb + uint32_t(w) * 1024u, sgpr_ptr(tile), uint32_t(off * 2));
    const uint32_t vm0 = sb + 8192u + uint32_t(w) * 4096u;
    dma16<0>(vm0, vbase, uint32_t(min(j0 + vrow[0], a.T - 1)) * vpitch + vcol[0]);
    dma16<1024>(vm0, vbase, uint32_t(min(j0 + vrow[1], a.T - 1)) * vpitch + vcol[1]);
    dma16<2048>(vm0, vbase, uint32_t(min(j0 + vrow[2], a.T - 1)) * vpitch + vcol[2]);
    dma16<3072>(vm0, vbase, uint32_t(min(j0 + vrow[3], a.T - 1)) * vpitch + vcol[3]);
  };

  // fragment reads: A (M) transposing reads of stored blocks (ib, kh), key
  // steps kk, halves r of the eight keys; B (V) rows 16 ks + 8 (l / 32) + q / 4
  // and 4 below, columns 64 wc + 32 c + 16 ((l / 16) & 1) + 4 (q % 4)
  const int kh = w >> 2, wc = w & 3;
  const int g4 = lane >> 4, q = lane & 15;
  uint32_t aoff[2][2];
#pragma unroll
  for (int k2 = 0; k2 < 2; ++k2)
#pragma unroll
    for (int r = 0; r < 2; ++r) {
      const int hf = g4 & 1;
      const int sl = 16 * k2 + 8 * (g4 >> 1) + 4 * r + (q >> 2) + 32 * (q & 1);
      const int slot = sl ^ (4 * (sl >> 5)) ^ (8 * hf);
      aoff[k2][r] = uint32_t(kh * 2048 + hf * 1024 + slot * 16 + 8 * ((q >> 1) & 1));
    }
  uint32_t boff[2];
#pragma unroll
  for (int c = 0; c < 2; ++c) {
    const int row = 8 * (g4 >> 1) + (q >> 2);
    const int col = 64 * wc + 32 * c + 16 * (g4 & 1) + 4 * (q & 3);
    boff[c] = uint32_t(8192 + row * 512 + (((col >> 3) ^ (4 * (row & 3))) * 16) + ((col >> 2) & 1) * 8);
  }
  f32x16 acc[2][2];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int c = 0; c < 2; ++c)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][c][r] = 0.f;

  issue(0, 0);
  if (nch > 1) issue(1, 1);
  int slot = 0;
  for (int ck = 0; ck < nch; ++ck) {
    if (ck + 1 < nch) sy_wait<5>();  // chunk ck landed, chunk ck + 1 in flight
    else sy_wait<0>();
    __syncthreads();  // chunk ck in every wave's view; chunk ck - 1's stage is free
    if (ck + 2 < nch) issue(ck + 2, slot == 0 ? 2 : slot - 1);
    const bool msk = ck == rb || r0 + 64 > a.T;  // uniform
    const uint32_t sb = lds0 + uint32_t(slot * kDvStage);
#pragma unroll
    for (int k2 = 0; k2 < 2; ++k2) {
      const int ks = 2 * kh + k2;
      bf16x8 fa[2], fb[2];
#pragma unroll
      for (int ib = 0; ib < 2; ++ib) {
        const lds_u8* pa = lds_at(sb + uint32_t(ib * 4096));
        fa[ib] = __builtin_shufflevector(lds_tr4(pa + aoff[k2][0]), lds_tr4(pa + aoff[k2][1]), 0, 1, 2, 3, 4, 5, 6, 7);
        if (msk) {
          u32x4 wv = __builtin_bit_cast(u32x4, fa[ib]);
          const int gi = r0 + 32 * ib + 16 * (g4 & 1) + q;
          const int jb0 = ck * 64 + 16 * ks + 8 * (g4 >> 1);
#pragma unroll
          for (int p = 0; p < 4; ++p) {
            const int jl = jb0 + 4 * (p >> 1) + 2 * (p & 1);
            const bool iok = gi < a.T;
            const uint32_t keep = ((iok && jl < gi) ? 0xffffu : 0u) | ((iok && jl + 1 < gi) ? 0xffff0000u : 0u);
            wv[p] &= keep;
          }
          fa[ib] = __builtin_bit_cast(bf16x8, wv);
        }
      }
#pragma unroll
      for (int c = 0; c < 2; ++c) {
        const lds_u8* pb = lds_at(sb + boff[c] + uint32_t(ks * 16 * 512));
        fb[c] = __builtin_shufflevector(lds_tr4(pb), lds_tr4(pb + 4 * 512), 0, 1, 2, 3, 4, 5, 6, 7);
      }
#pragma unroll
      for (int ib = 0; ib < 2; ++ib)
#pragma unroll
        for (int c = 0; c < 2; ++c) acc[ib][c] = mma(fa[ib], fb[c], acc[ib][c]);
    }
    slot = slot == 2 ? 0 : slot + 1;
  }

  // the two key halves' sums into one fp32 tile [64 i][pitch], then 16-byte stores
  __syncthreads();  // every wave's last fragment reads are done (its DMA waited above)
  float* const tl = reinterpret_cast<float*>(sv_ring);
  constexpr int PF = kDvPitch / 4;
  auto tile_idx = [&](int ib, int c, int r) {
    return (32 * ib + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3)) * PF + 64 * wc + 32 * c + (lane & 31);
  };
  if (kh == 1) {
#pragma unroll
    for (int ib = 0; ib < 2; ++ib)
#pragma unroll
      for (int c = 0; c < 2; ++c)
#pragma unroll
        for (int r = 0; r < 16; ++r) tl[tile_idx(ib, c, r)] = acc[ib][c][r];
  }
  __syncthreads();
  if (kh == 0) {
#pragma unroll
    for (int ib = 0; ib < 2; ++ib)
#pragma unroll
      for (int c = 0; c < 2; ++c)
#pragma unroll
        for (int r = 0; r < 16; ++r) tl[tile_idx(ib, c, r)] += acc[ib][c][r];
  }
  __syncthreads();
  TO* o = static_cast<TO*>(const_cast<void*>(a.o.p)) + b * a.o.s0 + h * a.o.s1;
  if constexpr (sizeof(TO) == 2) {
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      const int e = tid + 512 * v, row = e >> 5, cc = e & 31, gi = r0 + row;
      if (gi >= a.past && gi < a.T && 8 * cc < a.D) {
        const f32x4 x0 = *reinterpret_cast<const f32x4*>(tl + row * PF + 8 * cc);
        const f32x4 x1 = *reinterpret_cast<const f32x4*>(tl + row * PF + 8 * cc + 4);
        *reinterpret_cast<u32x4*>(o + int64_t(gi - a.past) * a.o.s2 + 8 * cc) =
            u32x4{pack_bf2(x0[0], x0[1]), pack_bf2(x0[2], x0[3]), pack_bf2(x1[0], x1[1]), pack_bf2(x1[2], x1[3])};
      }
    }
  } else {
#pragma unroll
    for (int v = 0; v < 8; ++v) {
      const int e = tid + 512 * v, row = e >> 6, cc = e & 63, gi = r0 + row;
      if (gi >= a.past && gi < a.T && 4 * cc < a.D)
        *reinterpret_cast<f32x4*>(o + int64_t(gi - a.past) * a.o.s2 + 4 * cc) =
            *reinterpret_cast<const f32x4*>(tl + row * PF + 4 * cc);
    }
  }
}

template <typename TO, typename TV>
int launch_sy_sv(const SvArgs& sa, dim3 grid, hipStream_t s) {
  const int ns = sa.nsplit;
  // one instantiation per split bound: a wider one re-reads the last split
  // for every split past nsplit
  if (ns == 1)
    BDH_LAUNCH("k_sy_sv", (k_sy_sv<TO, TV, 1>), grid, dim3(512), 0, s, sa);
  else if (ns <= 2)
    BDH_LAUNCH("k_sy_sv", (k_sy_sv<TO, TV, 2>), grid, dim3(512), 0, s, sa);
  else if (ns <= 4)
    BDH_LAUNCH("k_sy_sv", (k_sy_sv<TO, TV, 4>), grid, dim3(512), 0, s, sa);
  else
    BDH_LAUNCH("k_sy_sv", (k_sy_sv<TO, TV, 8>), grid, dim3(512), 0, s, sa);
  return BDH_OK;
}

// ---------------------------------------------------------------- host plan
struct SyPlan {
  int nt = 0, ntl = 0, ips = 0, nchunk = 0, nsplit = 1;
  int s0 = 0, t0 = 0;  // first row tile and its packed index (queries at an offset)
  int per_split = 0, nfull = 0;
  size_t table_bytes = 0, part_bytes = 0, ws_bytes = 0;
  bool ok = false;
};

// Work items of one (b, h) slab: with Q = K the full tiles below the diagonal
// plus the diagonal tiles in pairs (each pair costs about one full tile and
// loads two row blocks, like a full tile), else every lower tile in full.
// Every item of a slab runs the same split count, and the items of one split
// the same stages in the same order: a full tile and the diagonal pair of
// the same two row blocks then load the same bytes at the same time and the
// second load is served by the XCD's L2.  The split count is the smallest
// that gives every CU a work item.  s0 > 0 keeps the row tiles from s0 on
// (queries at an offset); their tiles are stored from packed index t0.
SyPlan sy_plan(int64_t nslab, int64_t T, int64_t N, bool self, bool rope, int64_t Dv = 0, int max_split = 8,
               int s0 = 0) {
  SyPlan p;
  if (T <= 0 || N <= 0 || N % 64 != 0 || nslab <= 0 || s0 < 0 || (s0 > 0 && rope)) return p;
  p.nt = int((T + kSyTile - 1) / kSyTile);
  if (s0 >= p.nt) return p;
  p.s0 = s0;
  p.t0 = s0 * (s0 + 1) / 2;
  p.ntl = p.nt * (p.nt + 1) / 2 - p.t0;
  p.nchunk = int(N / 64);
  const int nrow = p.nt - s0;  // row tiles kept
  p.nfull = self ? p.ntl - nrow : p.ntl;
  const int per_split = self ? p.nfull + (nrow + 1) / 2 : p.ntl;
  // one item per CU if that takes at most 8 splits, else the fewest that fill
  // every CU once
  const int64_t per_pass = nslab * per_split;
  int S = int(std::max<int64_t>(1, std::min<int64_t>(max_split, 256 / per_pass)));
  S = std::min(S, p.nchunk);
  p.nsplit = S;
  p.per_split = per_split;
  p.ips = per_split * S;
  // table of T absolute positions (used when the RoPE(x) copy is asked for,
  // or more than 512 stages per workgroup; else cos/sin are made in the kernel)
  p.table_bytes = rope ? align_up(size_t(T) * size_t(N / 2) * 4, 256) : 0;
  p.part_bytes = size_t(nslab) * size_t(p.ntl) * size_t(S) * kSyTileElems * sizeof(bf16_t);
  (void)Dv;
  p.ws_bytes = p.table_bytes + p.part_bytes;
  p.ok = true;
  return p;
}

bool rows16(const bdh_tensor4* t) {
  if ((reinterpret_cast<uintptr_t>(t->data) & 15) != 0) return false;
  for (int i = 0; i < 3; ++i)
    if (t->size[i] > 1 && (t->stride[i] % 8) != 0) return false;
  return true;
}

bool vec4_rows_sy(const bdh_tensor4* t) {
  const int64_t es = esize(t->dtype);
  if ((reinterpret_cast<uintptr_t>(t->data) % (4 * es)) != 0) return false;
  for (int i = 0; i < 3; ++i)
    if (t->size[i] > 1 && t->stride[i] % 4 != 0) return false;
  return t->size[3] % 4 == 0;
}

}  // namespace

size_t sy_workspace(int64_t B, int64_t H, int64_t T, int64_t N, int64_t Dv, bool rope) {
  const SyPlan p = sy_plan(B * H, T, N, true, rope, Dv);
  const SyPlan p2 = sy_plan(B * H, T, N, false, rope, Dv);
  return p.ok ? std::max(p.ws_bytes, p2.ok ? p2.ws_bytes : size_t(0)) : 0;
}

namespace {

// Eligibility of the MFMA forward path, and its plan.
bool sy_cold_check(const bdh_tensor4* q, const bdh_tensor4* k, const bdh_tensor4* v, bool rope,
                   const bdh_tensor4* qr, SyPlan& p, bool& self, int s0 = 0) {
  const int64_t B = q->size[0], H = q->size[1], T = q->size[2], N = q->size[3];
  if (q->dtype != BDH_BF16 || k->dtype != BDH_BF16) return false;
  self = q->data == k->data && q->stride[0] == k->stride[0] && q->stride[1] == k->stride[1] &&
         q->stride[2] == k->stride[2];
  if (rope && !self) return false;
  if (T < 1 || N < 64 || N % 64 != 0 || !rows16(q) || !rows16(k)) return false;
  // score x V: 8-element (16 / 32-byte) V row chunks, 256 columns per launch
  if (v->size[3] % 8 != 0 || !rows16(v)) return false;
  if (((T - 1) * std::max(q->stride[2], k->stride[2]) + N) * 2 >= (int64_t(1) << 31)) return false;
  if (rope && T * N * 2 >= (int64_t(1) << 31)) return false;  // 32-bit offsets into a table
  if (T > 65535) return false;
  if (qr != nullptr && (qr->dtype != BDH_BF16 || !rows16(qr))) return false;
  const int64_t nslab = B * H;
  if (nslab > (int64_t(1) << 24)) return false;
  p = sy_plan(nslab, T, N, self, rope, v->size[3], 8, s0);
  if (!p.ok) return false;
  return 8 * ((nslab + 7) / 8) * p.ips < (int64_t(1) << 31);
}

}  // namespace

bool sy_rope_keeps_scores(const bdh_tensor4* x, const bdh_tensor4* v, size_t* tiles_offset, size_t* kept_bytes,
                          int* rel) {
  SyPlan p;
  bool self = false;
  // what sy_run does for the fused RoPE forward without the R(x) copy: the
  // tiles follow the table region of the workspace, in the relative layout
  // when a workgroup has at most 512 stages
  if (v->size[3] < 1 || v->size[3] > 256 || !sy_cold_check(x, x, v, true, nullptr, p, self) || !self) return false;
  const int max_stages = 2 * ((p.nchunk + p.nsplit - 1) / p.nsplit);
  if (tiles_offset) *tiles_offset = p.table_bytes;
  if (kept_bytes) *kept_bytes = p.table_bytes + p.part_bytes;
  if (rel) *rel = max_stages <= 512 ? 1 : 0;
  return true;
}

bool sy_keeps_scores(const bdh_tensor4* q, const bdh_tensor4* v, size_t* scores_bytes) {
  SyPlan p;
  bool self = false;
  // the backward from saved tiles (sy_bwd_dv) takes at most 256 columns of V
  if (v->size[3] < 1 || v->size[3] > 256 || !sy_cold_check(q, q, v, false, nullptr, p, self) || !self) return false;
  if (scores_bytes) *scores_bytes = p.part_bytes;
  return true;
}

namespace {

// Schedule of the relative-RoPE score kernel (BDH_SY_SCHEDULE): 0 lockstep
// (default), 1 ping-pong; both give the same bits.
int sy_schedule() {
  const char* e = std::getenv("BDH_SY_SCHEDULE");
  return e != nullptr && std::strcmp(e, "pingpong") == 0 ? 1 : 0;
}

// past > 0 (no RoPE): out holds rows past.. only, and the score tiles of the
// row tiles below past / 256 are neither computed nor stored.
int sy_run(const bdh_tensor4* q, const bdh_tensor4* k, const bdh_tensor4* v, const bdh_tensor4* out,
           const float* freqs, int64_t rope_start, const bdh_tensor4* qr, int64_t past, void* ws,
           size_t ws_bytes, hipStream_t s) {
  const int64_t B = q->size[0], H = q->size[1], T = q->size[2], N = q->size[3];
  const bool rope = freqs != nullptr;
  SyPlan p;
  bool self = false;
  if (past < 0 || past >= T || (past > 0 && rope)) return kNotEligible;
  if (!sy_cold_check(q, k, v, rope, qr, p, self, int(past / kSyTile))) return kNotEligible;
  const int64_t nslab = B * H;
  const int64_t Dv = v->size[3];
  const int64_t grid_scores = 8 * ((nslab + 7) / 8) * p.ips;
  // Without the RoPE(x) copy the scores rotate rows about their tile's
  // centre, and each lane makes its cos/sin entries from the frequencies,
  // which the workgroup keeps in LDS (16 a stage, at most 512 stages); the
  // copy, or more stages, use a table of absolute positions.
  const bool want_qr = qr != nullptr && numel4(qr) > 0;
  const int max_stages = 2 * ((p.nchunk + p.nsplit - 1) / p.nsplit);
  const bool rel = rope && !want_qr && max_stages <= 512;
  if (ws == nullptr || ws_bytes < p.ws_bytes) return BDH_ERR_WORKSPACE;

  uint8_t* wsb = static_cast<uint8_t*>(ws);
  uint32_t* table = rope && !rel ? reinterpret_cast<uint32_t*>(wsb) : nullptr;
  bf16_t* part = reinterpret_cast<bf16_t*>(wsb + p.table_bytes);
  const int tq = rope && !rel ? int(T) : 0;
  if (table != nullptr) {
    BDH_LAUNCH("k_rope_table", k_rope_table, dim3(unsigned((N / 2 + 255) / 256), unsigned(tq)), dim3(256), 0, s,
               freqs, rope_start, int(N / 2), tq, table);
  }
  SyArgs a;
  a.g = nullptr;
  a.tpad = 0;
  a.q = static_cast<const bf16_t*>(q->data);
  a.k = static_cast<const bf16_t*>(k->data);
  a.q0 = q->stride[0];
  a.q1 = q->stride[1];
  a.q2 = q->stride[2];
  a.k0 = k->stride[0];
  a.k1 = k->stride[1];
  a.k2 = k->stride[2];
  a.H = int(H);
  a.T = int(T);
  a.N = int(N);
  a.nslab = int(nslab);
  a.ips = p.ips;
  a.nchunk = p.nchunk;
  a.nsplit = p.nsplit;
  a.ntl = p.ntl;
  a.t0 = p.t0;
  a.cs = table;
  a.freqs = rel ? freqs : nullptr;
  a.tq = tq;
  a.part = part;
  a.qr = nullptr;
  a.r0 = a.r1 = a.r2 = 0;
  if (want_qr) {
    a.qr = static_cast<bf16_t*>(qr->data);
    a.r0 = qr->stride[0];
    a.r1 = qr->stride[1];
    a.r2 = qr->stride[2];
  }
  a.s0 = p.s0;
  a.per_split = p.per_split;
  a.nfull = p.nfull;
  const dim3 gs{unsigned(grid_scores)};
  // row strides of a multiple of 64 KB: paired stages (both halves of each
  // 128-byte line requested together)
  const bool pair = rel && (q->stride[2] * 2) % 65536 == 0;
  const int sch = sy_schedule();
  if (pair && sch == 1)
    BDH_LAUNCH("k_sy_scores_paired", (k_sy_scores<2, true, false, true, 1>), gs, dim3(kSyThreads), 0, s, a);
  else if (pair)
    BDH_LAUNCH("k_sy_scores_paired", (k_sy_scores<2, true, false, true>), gs, dim3(kSyThreads), 0, s, a);
  else if (rel && sch == 1)
    BDH_LAUNCH("k_sy_scores", (k_sy_scores<2, true, false, false, 1>), gs, dim3(kSyThreads), 0, s, a);
  else if (rel)
    BDH_LAUNCH("k_sy_scores", (k_sy_scores<2, true>), gs, dim3(kSyThreads), 0, s, a);
  else if (rope)
    BDH_LAUNCH("k_sy_scores", (k_sy_scores<1, true>), gs, dim3(kSyThreads), 0, s, a);
  else if (self && sch == 1)
    BDH_LAUNCH("k_sy_scores", (k_sy_scores<0, true, false, false, 1>), gs, dim3(kSyThreads), 0, s, a);
  else if (self)
    BDH_LAUNCH("k_sy_scores", (k_sy_scores<0, true>), gs, dim3(kSyThreads), 0, s, a);
  else if (sch == 1)
    BDH_LAUNCH("k_sy_scores", (k_sy_scores<0, false, false, false, 1>), gs, dim3(kSyThreads), 0, s, a);
  else
    BDH_LAUNCH("k_sy_scores", (k_sy_scores<0, false>), gs, dim3(kSyThreads), 0, s, a);
  if (numel4(out) == 0) return BDH_OK;

  // score x V
  SvArgs sa;
  sa.part = part;
  sa.v = view_of(v);
  sa.ntl = p.ntl;
  sa.nsplit = p.nsplit;
  sa.H = int(H);
  sa.Hv = int(v->size[1]);
  sa.T = int(T);
  sa.D = int(Dv);
  sa.o = view_of(out);
  sa.o.s1 = out->stride[1];
  sa.t0 = p.t0;
  sa.rb0 = int(past / 64);
  sa.past = int(past);
  sa.rel = rel ? 1 : 0;
  sa.self = self ? 1 : 0;
  sa.nrbk = int((T + 63) / 64 - sa.rb0);
  sa.nslab = int(nslab);
  {
    // 16-byte stores of eight output columns need every group of eight
    // columns 16-byte aligned (each launch's column offset is a multiple of 256)
    const int64_t es = esize(out->dtype);
    bool al = (reinterpret_cast<uintptr_t>(out->data) % 16) == 0;
    for (int i = 0; i < 3; ++i)
      if (out->size[i] > 1 && (out->stride[i] * es) % 16 != 0) al = false;
    sa.o16 = al ? 1 : 0;
  }
  const dim3 gsv(unsigned(8 * ((nslab + 7) / 8) * sa.nrbk));
  const bool o16 = out->dtype == BDH_BF16, v16 = v->dtype == BDH_BF16;
  // one launch per 256 columns of V (the score tiles are read again by each)
  for (int64_t d0 = 0; d0 < Dv; d0 += 256) {
    SvArgs sc = sa;
    sc.v.p = static_cast<const char*>(v->data) + d0 * esize(v->dtype);
    sc.o.p = static_cast<const char*>(out->data) + d0 * esize(out->dtype);
    sc.D = int(std::min<int64_t>(256, Dv - d0));
    // one split, bf16 V in 16-byte rows, 16-byte output rows, V offsets within
    // 32 bits: the DMA ring
    if (sc.nsplit == 1 && v16 && sc.o16 && rows16(v) && ((T - 1) * v->stride[2] + 256) * 2 < (int64_t(1) << 32)) {
      if (o16) BDH_LAUNCH("k_sv_dma", (k_sv_dma<bf16_t>), gsv, dim3(512), 0, s, sc);
      else BDH_LAUNCH("k_sv_dma", (k_sv_dma<float>), gsv, dim3(512), 0, s, sc);
      continue;
    }
    const int rc = o16 ? (v16 ? launch_sy_sv<bf16_t, bf16_t>(sc, gsv, s) : launch_sy_sv<bf16_t, float>(sc, gsv, s))
                       : (v16 ? launch_sy_sv<float, bf16_t>(sc, gsv, s) : launch_sy_sv<float, float>(sc, gsv, s));
    if (rc != BDH_OK) return rc;
  }
  return BDH_OK;
}

}  // namespace

int sy_cold(const bdh_tensor4* q, const bdh_tensor4* k, const bdh_tensor4* v, const bdh_tensor4* out,
            const float* freqs, int64_t rope_start, const bdh_tensor4* qr, void* ws, size_t ws_bytes,
            hipStream_t s) {
  return sy_run(q, k, v, out, freqs, rope_start, qr, 0, ws, ws_bytes, s);
}

// Backward of the fused RoPE op, first step: the score tiles of R(x) R(x)^T
// (absolute positions) with R(x) written to qr, without score x V.  The
// workspace holds the (cos, sin) table of the absolute positions first, then
// the score tiles.
size_t sy_rope_scores_workspace(int64_t B, int64_t H, int64_t T, int64_t N) {
  const SyPlan p = sy_plan(B * H, T, N, true, true, 0);
  return p.ok ? p.ws_bytes : 0;
}

int sy_rope_scores(const bdh_tensor4* x, const bdh_tensor4* v, const float* freqs, int64_t rope_start,
                   const bdh_tensor4* qr, void* ws, size_t ws_bytes, hipStream_t s, const void** tiles) {
  SyPlan p;
  bool self = false;
  if (qr == nullptr || !sy_cold_check(x, x, v, true, qr, p, self) || !self) return kNotEligible;
  bdh_tensor4 none = *v;  // shape of an empty output: no score x V
  none.size[2] = 0;
  const int rc = sy_run(x, x, v, &none, freqs, rope_start, qr, 0, ws, ws_bytes, s);
  if (rc == BDH_OK && tiles != nullptr) *tiles = static_cast<const char*>(ws) + p.table_bytes;
  return rc;
}

size_t sy_past_workspace(int64_t B, int64_t H, int64_t Tk, int64_t past, int64_t N, int64_t Dv) {
  if (past <= 0 || past >= Tk) return 0;
  const SyPlan p = sy_plan(B * H, Tk, N, true, false, Dv, 8, int(past / kSyTile));
  return p.ok ? p.ws_bytes : 0;
}

// q is rows past.. of k (same storage and strides): the self-attention plan
// over k, restricted to the new rows.
int sy_past(const bdh_tensor4* q, const bdh_tensor4* k, const bdh_tensor4* v, const bdh_tensor4* out,
            int64_t past, void* ws, size_t ws_bytes, hipStream_t s) {
  if (q->dtype != BDH_BF16 || k->dtype != BDH_BF16 || past <= 0) return kNotEligible;
  for (int i = 0; i < 3; ++i)
    if (q->stride[i] != k->stride[i]) return kNotEligible;
  if (q->data != static_cast<const char*>(k->data) + past * k->stride[2] * 2) return kNotEligible;
  return sy_run(k, k, v, out, nullptr, 0, nullptr, past, ws, ws_bytes, s);
}


// dQ = G X (self attention, bf16 X) on the MFMA path; with freqs, out =
// R^T(G X) at positions rope_start + t (x is then R(x)).  kNotEligible when
// the shapes fall outside it.
namespace {
template <bool KM>
int launch_dq(const DqsArgs& a, bool bf_out, bool rope, bool rot_b, dim3 gs, hipStream_t s) {
  if (rope && rot_b) {
    if (bf_out)
      BDH_LAUNCH("k_dq_sy", (k_dq_sy<bf16_t, true, true, KM>), gs, dim3(kSyThreads), 0, s, a);
    else
      BDH_LAUNCH("k_dq_sy", (k_dq_sy<float, true, true, KM>), gs, dim3(kSyThreads), 0, s, a);
  } else if (rope) {
    if (bf_out)
      BDH_LAUNCH("k_dq_sy", (k_dq_sy<bf16_t, true, false, KM>), gs, dim3(kSyThreads), 0, s, a);
    else
      BDH_LAUNCH("k_dq_sy", (k_dq_sy<float, true, false, KM>), gs, dim3(kSyThreads), 0, s, a);
  } else if (bf_out) {
    BDH_LAUNCH("k_dq_sy", (k_dq_sy<bf16_t, false, false, KM>), gs, dim3(kSyThreads), 0, s, a);
  } else {
    BDH_LAUNCH("k_dq_sy", (k_dq_sy<float, false, false, KM>), gs, dim3(kSyThreads), 0, s, a);
  }
  return BDH_OK;
}
}  // namespace

int sy_dq(const void* g, int64_t tpad, bool g_sym, const bdh_tensor4* x, const bdh_tensor4* out, hipStream_t s,
          const float* freqs, int64_t rope_start, bool rot_b) {
  const int64_t B = x->size[0], H = x->size[1], T = x->size[2], N = x->size[3];
  if (x->dtype != BDH_BF16 || N % kSyTile != 0 || T < 1 || !rows16(x)) return kNotEligible;
  if (out->size[0] != B || out->size[1] != H || out->size[2] != T || out->size[3] != N) return kNotEligible;
  if (tpad % 32 != 0 || tpad * tpad * 2 >= (int64_t(1) << 31)) return kNotEligible;
  if (((T - 1) * x->stride[2] + N) * 2 >= (int64_t(1) << 31)) return kNotEligible;
  if (out->stride[2] >= (int64_t(1) << 26)) return kNotEligible;  // 4 rows of out < 2^31 bytes
  const int64_t nslab = B * H;
  const int64_t nti = (T + kSyTile - 1) / kSyTile, ntn = N / kSyTile;
  const int64_t grid = 8 * ((nslab + 7) / 8) * nti * ntn;
  if (grid >= (int64_t(1) << 31) || nslab > (int64_t(1) << 24)) return kNotEligible;
  DqsArgs a;
  a.g = static_cast<const bf16_t*>(g);
  a.x = static_cast<const bf16_t*>(x->data);
  a.x0 = x->stride[0];
  a.x1 = x->stride[1];
  a.x2 = x->stride[2];
  a.o = out->data;
  a.o0 = out->stride[0];
  a.o1 = out->stride[1];
  a.o2 = out->stride[2];
  a.H = int(H);
  a.T = int(T);
  a.N = int(N);
  a.tpad = int(tpad);
  a.nslab = int(nslab);
  a.nti = int(nti);
  a.ntn = int(ntn);
  a.freqs = freqs;
  a.rope_start = rope_start;
  const dim3 gs{unsigned(grid)};
  if (g_sym) return launch_dq<true>(a, out->dtype == BDH_BF16, freqs != nullptr, rot_b, gs, s);
  return launch_dq<false>(a, out->dtype == BDH_BF16, freqs != nullptr, rot_b, gs, s);
}


// G = dS + dS^T with dS = tril(dO V^T, -1), bf16, into g [B*H][tpad][tpad]
// (zero padding): the score kernel on Q = dO, K = V with one split (K = D)
// and the G epilogue.  kNotEligible outside its shapes.
int sy_bwd_g(const bdh_tensor4* dout, const bdh_tensor4* v, void* g, int64_t tpad, hipStream_t s) {
  const int64_t B = dout->size[0], H = dout->size[1], T = dout->size[2], D = dout->size[3];
  const int64_t Hv = v->size[1];
  if (dout->dtype != BDH_BF16 || v->dtype != BDH_BF16) return kNotEligible;
  if (v->size[0] != B || v->size[2] != T || v->size[3] != D || (Hv != 1 && Hv != H)) return kNotEligible;
  if (T < 1 || T > 65535 || D < 64 || D % 64 != 0 || !rows16(dout) || !rows16(v)) return kNotEligible;
  if (tpad < T || tpad % 4 != 0 || tpad > 65536) return kNotEligible;
  if (((T - 1) * std::max(dout->stride[2], v->stride[2]) + D) * 2 >= (int64_t(1) << 31)) return kNotEligible;
  const int64_t nslab = B * H;
  if (nslab > (int64_t(1) << 24)) return kNotEligible;
  const SyPlan p = sy_plan(nslab, T, D, false, false, 0, 1);
  if (!p.ok || p.nsplit != 1) return kNotEligible;
  const int64_t grid = 8 * ((nslab + 7) / 8) * p.ips;
  if (grid >= (int64_t(1) << 31)) return kNotEligible;
  SyArgs a;
  a.g = nullptr;
  a.tpad = 0;
  a.q = static_cast<const bf16_t*>(dout->data);
  a.q0 = dout->stride[0];
  a.q1 = dout->stride[1];
  a.q2 = dout->stride[2];
  a.k = static_cast<const bf16_t*>(v->data);
  a.k0 = v->stride[0];
  a.k1 = Hv == 1 ? 0 : v->stride[1];
  a.k2 = v->stride[2];
  a.H = int(H);
  a.T = int(T);
  a.N = int(D);
  a.nslab = int(nslab);
  a.ips = p.ips;
  a.nchunk = p.nchunk;
  a.nsplit = 1;
  a.ntl = p.ntl;
  a.cs = nullptr;
  a.part = nullptr;
  a.qr = nullptr;
  a.r0 = a.r1 = a.r2 = 0;
  a.g = static_cast<bf16_t*>(g);
  a.tpad = tpad;
  a.tq = 0;
  a.s0 = p.s0;
  a.per_split = p.per_split;
  a.nfull = p.nfull;
  BDH_LAUNCH("k_sy_scores_g", (k_sy_scores<0, false, true>), dim3{unsigned(grid)}, dim3(kSyThreads), 0, s, a);
  return BDH_OK;
}

size_t sy_bwd_workspace(int64_t B, int64_t H, int64_t T, int64_t N) {
  const SyPlan p = sy_plan(B * H, T, N, true, false, 0);
  return p.ok ? p.part_bytes : 0;
}

// dV for bf16 self attention without RoPE: the score tiles M by k_sy_scores
// into ws (or saved by the forward), then k_dv_sy.  kNotEligible when the
// shapes fall outside it.
int sy_bwd_dv(const bdh_tensor4* q, const bdh_tensor4* v, const bdh_tensor4* dout, const bdh_tensor4* dv, void* ws,
              size_t ws_bytes, hipStream_t s, const void* saved, int rel) {
  const int64_t B = q->size[0], H = q->size[1], T = q->size[2], N = q->size[3];
  const int64_t Hv = v->size[1], D = v->size[3];
  if (q->dtype != BDH_BF16 || dout->dtype != BDH_BF16) return kNotEligible;
  if (T < 1 || N < 64 || N % 64 != 0 || T > 65535 || !rows16(q) || !rows16(dout)) return kNotEligible;
  if (D < 1 || D > 256 || D % 8 != 0) return kNotEligible;
  if (((T - 1) * q->stride[2] + N) * 2 >= (int64_t(1) << 31)) return kNotEligible;
  const int64_t nslab = B * H;
  if (nslab > (int64_t(1) << 24) || B * Hv > 65535) return kNotEligible;
  const SyPlan p = sy_plan(nslab, T, N, true, false, 0);
  if (!p.ok) return kNotEligible;
  const int64_t grid_scores = 8 * ((nslab + 7) / 8) * p.ips;
  if (grid_scores >= (int64_t(1) << 31)) return kNotEligible;
  // saved: the score tiles of the forward on the same q (its workspace),
  // used in place of a recompute
  if (saved == nullptr && (ws == nullptr || ws_bytes < p.part_bytes)) return BDH_ERR_WORKSPACE;
  bf16_t* part = saved ? static_cast<bf16_t*>(const_cast<void*>(saved)) : static_cast<bf16_t*>(ws);
  if (saved == nullptr) {
    SyArgs a;
    a.g = nullptr;
    a.tpad = 0;
    a.tq = 0;
    a.q = a.k = static_cast<const bf16_t*>(q->data);
    a.q0 = a.k0 = q->stride[0];
    a.q1 = a.k1 = q->stride[1];
    a.q2 = a.k2 = q->stride[2];
    a.H = int(H);
    a.T = int(T);
    a.N = int(N);
    a.nslab = int(nslab);
    a.ips = p.ips;
    a.nchunk = p.nchunk;
    a.nsplit = p.nsplit;
    a.ntl = p.ntl;
    a.cs = nullptr;
    a.part = part;
    a.qr = nullptr;
    a.r0 = a.r1 = a.r2 = 0;
    a.s0 = p.s0;
    a.per_split = p.per_split;
    a.nfull = p.nfull;
    BDH_LAUNCH("k_sy_scores", (k_sy_scores<0, true>), dim3{unsigned(grid_scores)}, dim3(kSyThreads), 0, s, a);
  }
  if (numel4(dv) == 0) return BDH_OK;
  DvsArgs d;
  d.part = part;
  d.ntl = p.ntl;
  d.nsplit = p.nsplit;
  d.dO = static_cast<const bf16_t*>(dout->data);
  d.d0 = dout->stride[0];
  d.d1 = dout->stride[1];
  d.d2 = dout->stride[2];
  d.o = dv->data;
  d.o0 = dv->stride[0];
  d.o1 = dv->stride[1];
  d.o2 = dv->stride[2];
  d.H = int(H);
  d.Hv = int(Hv);
  d.T = int(T);
  d.D = int(D);
  d.rel = saved != nullptr ? rel : 0;
  d.nrb = int((T + 63) / 64);
  d.nbv = int(B * Hv);
  d.per_xcd = int((int64_t(d.nrb) * d.nbv + 7) / 8);
  const dim3 gd(unsigned(8 * d.per_xcd));
  const bool o16 = dv->dtype == BDH_BF16;
  // one split, 16-byte output rows and dO offsets within 32 bits: the DMA ring
  if (p.nsplit == 1 && rows16(dv) && ((T - 1) * dout->stride[2] + D) * 2 < (int64_t(1) << 32)) {
    if (o16) BDH_LAUNCH("k_dv_dma", (k_dv_dma<bf16_t>), gd, dim3(512), 0, s, d);
    else BDH_LAUNCH("k_dv_dma", (k_dv_dma<float>), gd, dim3(512), 0, s, d);
  } else if (p.nsplit == 1) {
    if (o16) BDH_LAUNCH("k_dv_sy", (k_dv_sy<bf16_t, 1>), gd, dim3(512), 0, s, d);
    else BDH_LAUNCH("k_dv_sy", (k_dv_sy<float, 1>), gd, dim3(512), 0, s, d);
  } else if (p.nsplit <= 2) {
    if (o16) BDH_LAUNCH("k_dv_sy", (k_dv_sy<bf16_t, 2>), gd, dim3(512), 0, s, d);
    else BDH_LAUNCH("k_dv_sy", (k_dv_sy<float, 2>), gd, dim3(512), 0, s, d);
  } else if (p.nsplit <= 4) {
    if (o16) BDH_LAUNCH("k_dv_sy", (k_dv_sy<bf16_t, 4>), gd, dim3(512), 0, s, d);
    else BDH_LAUNCH("k_dv_sy", (k_dv_sy<float, 4>), gd, dim3(512), 0, s, d);
  } else {
    if (o16) BDH_LAUNCH("k_dv_sy", (k_dv_sy<bf16_t, 8>), gd, dim3(512), 0, s, d);
    else BDH_LAUNCH("k_dv_sy", (k_dv_sy<float, 8>), gd, dim3(512), 0, s, d);
  }
  return BDH_OK;
}

}  // namespace bdh
