// bf16 prefill forward of BDH strict-tril attention for gfx950 (the hot path):
//
//   out[b,h,i,:] = sum_{j<i} <R_i, R_j> V_j,   R = RoPE(x) (or R = q, k given)
//
// Three kernels per call:
//  1. k_rope_table  (RoPE only): (cos, sin) of every (position, pair) as two
//     bf16 halves of one dword, [T][N/2].  The same table serves every (b,h).
//  2. k_sy_scores: partial score tiles S = R R^T.
//     * 256x256 output tiles over the lower triangle of each (b,h) slab.  A
//       diagonal tile with Q = K loads one row block and computes only its
//       lower 32x32 blocks (each SIMD issues at most 10 MFMAs per k16 step,
//       against 16 for a full tile).
//     * split-K: split s of n handles the 64-wide k-chunks s, s+n, s+2n, ...,
//       so the splits and tiles of a slab walk k in step and the row blocks
//       re-read by neighbouring tiles are served by the XCD's L2.  Every item
//       of a slab runs on one XCD (workgroup id % 8 selects the XCD).
//     * x streams HBM -> LDS through global_load_lds_dwordx4 into a ring of
//       32-wide k stages (5 slots, issued four stages ahead; with RoPE 3 slots
//       plus a 2-slot ring for the table entries of the same stages at the
//       same offsets, issued two stages ahead).  The 16-byte chunk c of row r sits at position c ^ ((r >> 2) & 3)
//       of its 64-byte LDS row, which makes the MFMA fragment reads
//       bank-conflict free.
//     * RoPE is applied in place at the end of the stage before its MFMAs:
//       each lane rotates the chunks it loaded itself (per pair two
//       v_dot2_f32_bf16, products exact in fp32, one v_cvt_pk_bf16_f32 and one
//       v_alignbit_b32).  No vector-memory load of the main loop returns to
//       registers, so the only waits on it are the explicit ones below.
//     * v_mfma_f32_32x32x16_bf16 with fp32 accumulators; the epilogue stores
//       the partial tiles [slab][item][256][256] as bf16.
//  3. k_sy_vt + k_sy_sv: out = tril(sum over splits of S, -1) V.  V is
//     transposed once (bf16, contiguous along the contraction); each wave then
//     loads its MFMA fragments straight from global memory: the split sum of
//     the partial score rows (formed in fp32, masked, rounded to bf16) and V^T.
#include <algorithm>
#include <type_traits>

#include "fwd.h"

#pragma clang diagnostic ignored "-Winline-asm"

namespace bdh {
namespace {

constexpr int kSyThreads = 512;
constexpr int kSyTile = 256;
constexpr int kSyBlk = kSyTile * 64;   // bytes of one row block per stage (256 rows x 32 bf16)
constexpr int kSySlot = 2 * kSyBlk;    // A and B row blocks
constexpr int kSyLdsSlots = 5;    // 160 KB: x ring of 5 (plain) or 3 x + 2 RoPE table (fused)
constexpr int kSyMaxItems = 256;
constexpr int kSyMaxTiles = 128;
constexpr int kSyTileElems = kSyTile * kSyTile;

typedef __attribute__((address_space(3))) uint8_t lds_u8;

struct SyArgs {
  const bf16_t* q;
  const bf16_t* k;
  int64_t q0, q1, q2;  // element strides of q over (b, h, t)
  int64_t k0, k1, k2;
  int H, T, N, nslab, ips, nchunk;
  const uint32_t* cs;  // RoPE table [T][tpitch] (first N/2 used) or null
  int tpitch;          // table row pitch in dwords
  bf16_t* part;        // [nslab][ips][256*256] partial score tiles (bf16)
  bf16_t* qr;          // optional RoPE(x) copy
  int64_t r0, r1, r2;
  uint32_t items[kSyMaxItems];  // ti | tj << 8 | split << 16 | nsplit << 24
};

__shared__ __attribute__((aligned(1024))) uint8_t sy_lds[kSyLdsSlots * kSySlot];  // 160 KB

// ---------------------------------------------------------------- asm helpers
// The x stream and the table are moved by LDS DMA issued from inline asm, so
// the compiler neither counts them in its own vmcnt waits nor orders LDS
// accesses behind them; the kernel waits for them explicitly (sy_wait).
// A wave-uniform pointer made explicitly scalar (the asm takes it in SGPRs).
__device__ __forceinline__ const void* sgpr_ptr(const void* p) {
  const uint64_t v = reinterpret_cast<uint64_t>(p);
  const uint32_t lo = __builtin_amdgcn_readfirstlane(uint32_t(v));
  const uint32_t hi = __builtin_amdgcn_readfirstlane(uint32_t(v >> 32));
  return reinterpret_cast<const void*>((uint64_t(hi) << 32) | lo);
}

__device__ __forceinline__ void dma16(uint32_t lds, const void* gbase, uint32_t voff) {
  asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %1, %2"
               :
               : "s"(lds), "v"(voff), "s"(gbase)
               : "memory", "m0");
}

// Wait until at most n vector-memory operations of this wave are outstanding
// (they complete in issue order).
__device__ __forceinline__ void sy_wait(int n) {
  switch (n) {
    case 0: asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); break;
    case 2: asm volatile("s_waitcnt vmcnt(2)" ::: "memory"); break;
    case 4: asm volatile("s_waitcnt vmcnt(4)" ::: "memory"); break;
    case 6: asm volatile("s_waitcnt vmcnt(6)" ::: "memory"); break;
    case 8: asm volatile("s_waitcnt vmcnt(8)" ::: "memory"); break;
    case 10: asm volatile("s_waitcnt vmcnt(10)" ::: "memory"); break;
    case 12: asm volatile("s_waitcnt vmcnt(12)" ::: "memory"); break;
    default: asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); break;
  }
}

__device__ __forceinline__ void sy_barrier() {
  asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
  __builtin_amdgcn_s_barrier();
}

// RoPE of the four adjacent pairs of one 16-byte chunk: pair m is
// x.lo = x[2m], x.hi = x[2m+1] with cs = (cos, sin) as bf16 halves, giving
// (x0 c - x1 s, x1 c + x0 s) rounded to bf16 once (products exact in fp32).
// One asm block so the hazard spacing is explicit: a v_dot2 result is read
// no sooner than three wait states after it is written (s_nop 2).
__device__ __forceinline__ u32x4 rot_chunk(u32x4 x, u32x4 cs) {
  u32x4 y;
  uint32_t s0, s1, s2, s3;
  float a0, a1, a2, a3, b0, b1, b2, b3;
  asm("v_alignbit_b32 %[s0], %[x0], %[x0], 16\n\t"
      "v_alignbit_b32 %[s1], %[x1], %[x1], 16\n\t"
      "v_alignbit_b32 %[s2], %[x2], %[x2], 16\n\t"
      "v_alignbit_b32 %[s3], %[x3], %[x3], 16\n\t"
      "v_dot2_f32_bf16 %[a0], %[x0], %[c0], 0 neg_hi:[0,1,0]\n\t"
      "v_dot2_f32_bf16 %[a1], %[x1], %[c1], 0 neg_hi:[0,1,0]\n\t"
      "v_dot2_f32_bf16 %[a2], %[x2], %[c2], 0 neg_hi:[0,1,0]\n\t"
      "v_dot2_f32_bf16 %[a3], %[x3], %[c3], 0 neg_hi:[0,1,0]\n\t"
      "v_dot2_f32_bf16 %[b0], %[s0], %[c0], 0\n\t"
      "v_dot2_f32_bf16 %[b1], %[s1], %[c1], 0\n\t"
      "v_dot2_f32_bf16 %[b2], %[s2], %[c2], 0\n\t"
      "v_dot2_f32_bf16 %[b3], %[s3], %[c3], 0\n\t"
      "s_nop 2\n\t"
      "v_cvt_pk_bf16_f32 %[y0], %[a0], %[b0]\n\t"
      "v_cvt_pk_bf16_f32 %[y1], %[a1], %[b1]\n\t"
      "v_cvt_pk_bf16_f32 %[y2], %[a2], %[b2]\n\t"
      "v_cvt_pk_bf16_f32 %[y3], %[a3], %[b3]"
      : [y0] "=&v"(y.x), [y1] "=&v"(y.y), [y2] "=&v"(y.z), [y3] "=&v"(y.w),
        [s0] "=&v"(s0), [s1] "=&v"(s1), [s2] "=&v"(s2), [s3] "=&v"(s3),
        [a0] "=&v"(a0), [a1] "=&v"(a1), [a2] "=&v"(a2), [a3] "=&v"(a3),
        [b0] "=&v"(b0), [b1] "=&v"(b1), [b2] "=&v"(b2), [b3] "=&v"(b3)
      : [x0] "v"(x.x), [x1] "v"(x.y), [x2] "v"(x.z), [x3] "v"(x.w),
        [c0] "v"(cs.x), [c1] "v"(cs.y), [c2] "v"(cs.z), [c3] "v"(cs.w));
  return y;
}

__device__ __forceinline__ bf16x8 frag(const uint8_t* blk, int rb, uint32_t loff) {
  return *reinterpret_cast<const bf16x8*>(blk + rb * 2048 + loff);
}

__device__ __forceinline__ f32x16 mma(bf16x8 a, bf16x8 b, f32x16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
}

// ------------------------------------------------------------------ kernels
__global__ __launch_bounds__(256) void k_rope_table(const float* __restrict__ freqs, int64_t rope_start,
                                                    int N2, int pitch, uint32_t* __restrict__ cs) {
  const int t = blockIdx.y, m = blockIdx.x * 256 + threadIdx.x;
  if (m >= N2) return;
  // phase = fp32(pos) * freq, then cos/sin of 2 pi frac(phase); v_cos/v_sin
  // take the angle in revolutions, so frac(phase) goes in directly.  The
  // values are rounded to bf16, far above the hardware functions' error.
  const float ph = __fmul_rn(float(rope_start + t), freqs[2 * m]);
  const float fr = ph - floorf(ph);
  cs[int64_t(t) * pitch + m] = pack_bf2(__builtin_amdgcn_cosf(fr), __builtin_amdgcn_sinf(fr));
}

template <bool ROPE, bool SELF>
__global__ __launch_bounds__(kSyThreads, 1) void k_sy_scores(const SyArgs a) {
  const int bid = blockIdx.x;
  const int xcd = bid & 7, kk = bid >> 3;
  const int grp = kk / a.ips;
  const int slab = grp * 8 + xcd;
  if (slab >= a.nslab) return;
  const int itx = kk - grp * a.ips;
  const uint32_t item = a.items[itx];
  const int ti = item & 255, tj = (item >> 8) & 255, split = (item >> 16) & 255, nsplit = int(item >> 24);
  const bool diag = SELF && ti == tj;
  const int b = slab / a.H, h = slab - b * a.H;
  const int tid = threadIdx.x, lane = tid & 63;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int ndma = diag ? 2 : 4;  // 1 KB DMA instructions per wave per stage
  const int nch = (a.nchunk - split + nsplit - 1) / nsplit;
  const int nst = 2 * nch;

  const void* baseA = sgpr_ptr(a.q + b * a.q0 + h * a.q1);
  const void* baseB = SELF ? baseA : sgpr_ptr(a.k + b * a.k0 + h * a.k1);
  const void* tbase = sgpr_ptr(a.cs);
  const uint32_t lds0 = __builtin_amdgcn_readfirstlane((uint32_t)(uintptr_t)(lds_u8*)sy_lds);

  // Per DMA instruction u: the 16-byte chunk this lane moves (and rotates).
  uint32_t xoff[4], toff[4];
  int rowg[4], kch[4];
#pragma unroll
  for (int u = 0; u < 4; ++u) {
    const int q = (u * 8 + w) * 1024 + lane * 16;
    const int blk = q >> 14;
    const int ob = q & (kSyBlk - 1);
    const int row = ob >> 6;
    const int c = ((ob >> 4) & 3) ^ ((row >> 2) & 3);
    const int rg = (blk == 0 ? ti : tj) * kSyTile + row;
    const int rc = rg < a.T ? rg : a.T - 1;
    rowg[u] = rg;
    kch[u] = 8 * c;
    xoff[u] = uint32_t((int64_t(rc) * (blk == 0 ? a.q2 : (SELF ? a.q2 : a.k2)) + 8 * c) * 2);
    toff[u] = uint32_t(int64_t(rc) * a.tpitch * 4 + 16 * c);
  }
  // MFMA fragment offsets within a row block for the two k16 steps of a stage.
  uint32_t loff[2];
#pragma unroll
  for (int kk2 = 0; kk2 < 2; ++kk2) {
    const int c = (2 * kk2 + (lane >> 5)) ^ ((lane >> 2) & 3);
    loff[kk2] = uint32_t((lane & 31) * 64 + c * 16);
  }

  auto kofs = [&](int s) { return (split + nsplit * (s >> 1)) * 64 + (s & 1) * 32; };
  // x ring depth; issuing runs NX - 1 stages ahead of the MFMAs
  constexpr int NX = ROPE ? 3 : 5;
  auto slot = [&](int s) { return sy_lds + (s % NX) * kSySlot; };
  auto tslot = [&](int s) { return sy_lds + (NX + (s & 1)) * kSySlot; };
  auto rotate = [&](int s) {
    uint8_t* sl = slot(s);
    const int k0 = kofs(s);
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      if (u < ndma) {
        const int off = (u * 8 + w) * 1024 + lane * 16;
        u32x4* p = reinterpret_cast<u32x4*>(sl + off);
        const u32x4 x = *p;
        const u32x4 t = *reinterpret_cast<const u32x4*>(tslot(s) + off);
        const u32x4 y = rot_chunk(x, t);
        *p = y;
        if (a.qr != nullptr && diag && rowg[u] < a.T)
          *reinterpret_cast<u32x4*>(a.qr + b * a.r0 + h * a.r1 + int64_t(rowg[u]) * a.r2 + k0 + kch[u]) = y;
      }
    }
  };

  f32x16 acc[8];
#pragma unroll
  for (int i = 0; i < 8; ++i)
#pragma unroll
    for (int r = 0; r < 16; ++r) acc[i][r] = 0.f;

  // Wave tile: rows [128 wm, +128) x cols [64 wn, +64) = 4 x 2 blocks of 32x32.
  // On a diagonal tile only blocks with row block >= column block are needed;
  // the wave tiles then cost 7,3,0,0 (wm = 0) and 8,8,7,3 (wm = 1) MFMAs per
  // k16 step, and waves w and w+4 (one SIMD) are given tiles summing to at
  // most 10 (a full tile: 16).
  int wm = w >> 2, wn = w & 3;
  if (diag) {
    constexpr int kDiagWave[8] = {4, 5, 0, 6, 2, 3, 7, 1};  // wm * 4 + wn per wave
    const int t = kDiagWave[w];
    wm = t >> 2;
    wn = t & 3;
  }
  // Blocks (i, j) of the wave tile that lie on or below the diagonal:
  // 0 all 8, 1 i >= j (7), 2 i >= j + 2 (3), 3 none.
  const int wtype = !diag ? 0 : (4 * wm >= 2 * wn + 1) ? 0 : (4 * wm == 2 * wn) ? 1 : (4 * wm == 2 * wn - 2) ? 2 : 3;
  // The wave tile type selects one of four instantiations of the whole
  // pipeline (prologue, loop, epilogue), so each loop holds straight-line MFMA
  // code; all of them run the same stages and barriers.
  auto run = [&](auto wt_tag, auto diag_tag) {
    constexpr int WT = decltype(wt_tag)::value;
    constexpr bool DG = decltype(diag_tag)::value;  // == diag
    constexpr int NDMA = DG ? 2 : 4;
    // vector-memory operations per stage per wave, in issue order: the table
    // chunks (RoPE) then the x chunks
    constexpr int per_stage = ROPE ? 2 * NDMA : NDMA;
    auto dma_op = [&](int st, int i) {
      const uint32_t kb = uint32_t(kofs(st) * 2);
      if (ROPE && i < NDMA) {
        dma16(lds0 + uint32_t((NX + (st & 1)) * kSySlot + (i * 8 + w) * 1024), tbase, toff[i] + kb);
      } else {
        const int u = ROPE ? i - NDMA : i;
        dma16(lds0 + uint32_t((st % NX) * kSySlot + (u * 8 + w) * 1024), u < 2 ? baseA : baseB, xoff[u] + kb);
      }
    };
    // The MFMAs of stage s with the loads of stage `ahead` (if any) spread
    // between them: issuing them all at once stalls the wave on the load
    // queue while its MFMAs wait.  All fragments of the stage are read first
    // into distinct registers (sched_group_barrier fixes that order; left
    // alone the scheduler reuses a few registers and waits on each read right
    // before its MFMA).
    auto mma_stage = [&](int s, int ahead) {
      const uint8_t* A = slot(s);
      const uint8_t* B = DG ? A : A + kSyBlk;
      const bool issue = ahead < nst;
      // after MFMA number m of nm, issue the loads [m*P/nm, (m+1)*P/nm)
      auto loads_after = [&](int m, int nm) {
        if (!issue) return;
#pragma unroll
        for (int i = (m * per_stage) / nm; i < ((m + 1) * per_stage) / nm; ++i) dma_op(ahead, i);
      };
      if constexpr (WT == 0 || WT == 1) {
        bf16x8 fa[2][4], fb[2][2];
#pragma unroll
        for (int k2 = 0; k2 < 2; ++k2) {
#pragma unroll
          for (int i = 0; i < 4; ++i) fa[k2][i] = frag(A, 4 * wm + i, loff[k2]);
#pragma unroll
          for (int j = 0; j < 2; ++j) fb[k2][j] = frag(B, 2 * wn + j, loff[k2]);
        }
        constexpr int NM = WT == 0 ? 16 : 14;
        int m = 0;
#pragma unroll
        for (int k2 = 0; k2 < 2; ++k2)
#pragma unroll
          for (int i = 0; i < 4; ++i)
#pragma unroll
            for (int j = 0; j < 2; ++j)
              if (WT == 0 || i >= j) {
                acc[2 * i + j] = mma(fa[k2][i], fb[k2][j], acc[2 * i + j]);
                if (m == 0) {
                  __builtin_amdgcn_sched_group_barrier(0x100, 12, 0);
                  __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
                }
                loads_after(m, NM);
                ++m;
              }
      } else if constexpr (WT == 2) {
        bf16x8 fa[2][2], fb[2][2];
#pragma unroll
        for (int k2 = 0; k2 < 2; ++k2) {
#pragma unroll
          for (int i = 0; i < 2; ++i) fa[k2][i] = frag(A, 4 * wm + 2 + i, loff[k2]);
#pragma unroll
          for (int j = 0; j < 2; ++j) fb[k2][j] = frag(B, 2 * wn + j, loff[k2]);
        }
#pragma unroll
        for (int k2 = 0; k2 < 2; ++k2) {
          acc[4] = mma(fa[k2][0], fb[k2][0], acc[4]);
          if (k2 == 0) {
            __builtin_amdgcn_sched_group_barrier(0x100, 8, 0);
            __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
          }
          loads_after(3 * k2, 6);
          acc[6] = mma(fa[k2][1], fb[k2][0], acc[6]);
          loads_after(3 * k2 + 1, 6);
          acc[7] = mma(fa[k2][1], fb[k2][1], acc[7]);
          loads_after(3 * k2 + 2, 6);
        }
      } else {
        loads_after(0, 1);
      }
    };
    constexpr auto live = [](int i, int j) { return WT == 0 || (WT == 1 && i >= j) || (WT == 2 && i >= j + 2); };
    // ------------------------------------------------------------ prologue
    // Issue order is what the waits count on: operations complete in order.
    const int lead = NX - 1;
    for (int st = 0; st < lead && st < nst; ++st)
      for (int i = 0; i < per_stage; ++i) dma_op(st, i);
    sy_wait((min(nst, lead) - 1) * per_stage);  // stage 0 landed
    if (ROPE) rotate(0);
    sy_barrier();

    // ------------------------------------------------------------ main loop
    for (int s = 0; s < nst; ++s) {
      // the loads of stage s + lead go to x slot (s-1) % NX and (fused) table
      // slot s % 2, consumed before the last barrier
      mma_stage(s, s + lead);
      if (s + 1 < nst) {
        // stage s+1 landed (this wave's part): the stages issued after it may
        // still be in flight
        sy_wait((min(nst - 1, s + lead) - (s + 1)) * per_stage);
        if (ROPE) rotate(s + 1);
      }
      sy_barrier();
    }

    // ------------------------------------------------------------ epilogue
    bf16_t* dst = a.part + (int64_t(slab) * a.ips + itx) * kSyTileElems;
    // Partial tiles are stored as bf16 (halving their traffic; the scores are
    // bf16 MFMA operands of the score x V product anyway).  Lane pairs swap one
    // value so each lane writes two adjacent columns of one row.
    const bool even = (lane & 1) == 0;
    auto store_block = [&](const f32x16& c, int rb, int cb) {
#pragma unroll
      for (int r = 0; r < 16; r += 2) {
        const float send = even ? c[r + 1] : c[r];
        const float recv = __shfl_xor(send, 1, 64);
        const int row = rb * 32 + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3) + (even ? 0 : 1);
        const int col = cb * 32 + ((lane & 31) & ~1);
        const uint32_t w2 = even ? pack_bf2(c[r], recv) : pack_bf2(recv, c[r + 1]);
        *reinterpret_cast<uint32_t*>(dst + row * kSyTile + col) = w2;
      }
    };
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int j = 0; j < 2; ++j)
        if (live(i, j)) store_block(acc[2 * i + j], 4 * wm + i, 2 * wn + j);
  };
  using T0 = std::integral_constant<int, 0>;
  using F = std::integral_constant<bool, false>;
  using D = std::integral_constant<bool, SELF>;  // diagonal tiles exist only with Q = K
  if (!diag) {
    run(T0(), F());
  } else {
    switch (wtype) {
      case 0: run(T0(), D()); break;
      case 1: run(std::integral_constant<int, 1>(), D()); break;
      case 2: run(std::integral_constant<int, 2>(), D()); break;
      default: run(std::integral_constant<int, 3>(), D()); break;
    }
  }
}

// ------------------------------------------------------ score x V (direct)
// V^T, bf16: vt[bv][d][t] = v[b][hv][t][d] (bv = b * Hv + hv), t padded to tp
// with zeros.  The score x V product contracts over t, and MFMA operands are
// contiguous along the contraction, so V is transposed once per call.
template <typename TV>
__global__ __launch_bounds__(256) void k_sy_vt(View v, int Hv, int T, int D, int tp, bf16_t* __restrict__ vt) {
  __shared__ float tile[32][33];
  const int bv = blockIdx.z, b = bv / Hv, hv = bv - b * Hv;
  const int t0 = blockIdx.x * 32, d0 = blockIdx.y * 32;
  const TV* src = static_cast<const TV*>(v.p) + b * v.s0 + hv * v.s1;
  const int tx = threadIdx.x & 31, ty = threadIdx.x >> 5;  // 32 x 8
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    const int t = t0 + ty + 8 * r, d = d0 + tx;
    tile[ty + 8 * r][tx] = (t < T && d < D) ? to_f(src[int64_t(t) * v.s2 + d]) : 0.f;
  }
  __syncthreads();
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    const int d = d0 + ty + 8 * r, t = t0 + tx;
    if (d < D && t < tp) vt[(int64_t(bv) * D + d) * tp + t] = f2bf(tile[tx][ty + 8 * r]);
  }
}

struct SvArgs {
  const bf16_t* part;  // partial score tiles [slab][ips][256*256]
  const bf16_t* vt;    // [B*Hv][D][tp]
  int ips, sf, sd, H, Hv, T, D, tp;
  View o;
};

// out rows [32 rb, +32) of one (b,h) slab, all D: each wave owns 64 columns
// (two 32x32 MFMA blocks) and loads its fragments straight from global
// memory: A = the masked split sum of the partial score rows, B = V^T.  The
// loads of U k16 steps (every split, predicated) are issued before any of
// them is used, so a wave keeps U * (NS + 2) loads in flight.
template <typename TO, int NS, int U>
__global__ __launch_bounds__(256) void k_sy_sv(const SvArgs a) {
  const int rb = blockIdx.x, slab = blockIdx.y;
  const int b = slab / a.H, h = slab - b * a.H, hv = a.Hv == 1 ? 0 : h;
  const int w = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int row = rb * 32 + (lane & 31);
  const int kq = (lane >> 5) * 8;
  const bf16_t* pslab = a.part + int64_t(slab) * a.ips * kSyTileElems;
  const bf16_t* vtb = a.vt + (int64_t(b) * a.Hv + hv) * a.D * a.tp;
  f32x16 acc[2];
#pragma unroll
  for (int c = 0; c < 2; ++c)
#pragma unroll
    for (int r = 0; r < 16; ++r) acc[c][r] = 0.f;
  const int ti = min(row, a.T - 1) >> 8;
  const int kend = min(a.T, (rb + 1) * 32);  // keys j < rows of this block
  const bool lastrow_ok = row < a.T;
  int dcol[2];
  bool dok[2];
#pragma unroll
  for (int c = 0; c < 2; ++c) {
    dcol[c] = 64 * w + 32 * c + (lane & 31);
    dok[c] = dcol[c] < a.D;
  }
  for (int k0 = 0; k0 < kend; k0 += 16 * U) {
    uint4 ra[U][NS];
    bf16x8 rb2[U][2];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int j = k0 + 16 * u + kq;
      const bool in = k0 + 16 * u < kend;
      const bool av = in && lastrow_ok && j < row;
      const int tj = j >> 8;
      const int first = a.sf * (ti * (ti - 1) / 2 + tj) + a.sd * ti;
      const int ns = ti == tj ? a.sd : a.sf;
      const bf16_t* p = pslab + int64_t(first) * kSyTileElems + (row & 255) * kSyTile + (j & 255);
#pragma unroll
      for (int sp = 0; sp < NS; ++sp)
        ra[u][sp] = (av && sp < ns) ? *reinterpret_cast<const uint4*>(p + int64_t(sp) * kSyTileElems)
                                    : uint4{0u, 0u, 0u, 0u};
#pragma unroll
      for (int c = 0; c < 2; ++c)
        rb2[u][c] = (in && dok[c]) ? *reinterpret_cast<const bf16x8*>(vtb + int64_t(dcol[c]) * a.tp + j)
                                   : __builtin_bit_cast(bf16x8, u32x4{0u, 0u, 0u, 0u});
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      if (k0 + 16 * u >= kend) break;
      const int j = k0 + 16 * u + kq;
      float sacc[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) sacc[e] = 0.f;
#pragma unroll
      for (int sp = 0; sp < NS; ++sp) {
        const uint32_t xw[4] = {ra[u][sp].x, ra[u][sp].y, ra[u][sp].z, ra[u][sp].w};
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          sacc[2 * e] += __uint_as_float(xw[e] << 16);
          sacc[2 * e + 1] += __uint_as_float(xw[e] & 0xffff0000u);
        }
      }
      uint32_t pk[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const float lo = (j + 2 * e < row) ? sacc[2 * e] : 0.f;
        const float hi = (j + 2 * e + 1 < row) ? sacc[2 * e + 1] : 0.f;
        pk[e] = pack_bf2(lo, hi);
      }
      const bf16x8 fa = __builtin_bit_cast(bf16x8, *reinterpret_cast<const u32x4*>(pk));
#pragma unroll
      for (int c = 0; c < 2; ++c) acc[c] = mma(fa, rb2[u][c], acc[c]);
    }
  }
  TO* o = static_cast<TO*>(const_cast<void*>(a.o.p)) + b * a.o.s0 + h * a.o.s1;
#pragma unroll
  for (int c = 0; c < 2; ++c)
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int i = rb * 32 + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
      if (i < a.T && dok[c]) o[int64_t(i) * a.o.s2 + dcol[c]] = from_f<TO>(acc[c][r]);
    }
}

template <typename TO>
int launch_sy_sv(const SvArgs& sa, dim3 grid, hipStream_t s) {
  const int ns = std::max(sa.sf, sa.sd);
  if (ns <= 2)
    BDH_LAUNCH("k_sy_sv", (k_sy_sv<TO, 2, 4>), grid, dim3(256), 0, s, sa);
  else if (ns <= 4)
    BDH_LAUNCH("k_sy_sv", (k_sy_sv<TO, 4, 4>), grid, dim3(256), 0, s, sa);
  else
    BDH_LAUNCH("k_sy_sv", (k_sy_sv<TO, 8, 2>), grid, dim3(256), 0, s, sa);
  return BDH_OK;
}

// ---------------------------------------------------------------- host plan
// Table rows are padded by 256 bytes so the rows one DMA instruction reads
// (same pair offset, consecutive positions) fall on different L2 channels.
inline int sy_table_pitch(int64_t N) { return int(N / 2) + 64; }
// V^T rows hold the positions padded to a multiple of 32 (zeros beyond T).
inline int sy_vt_pitch(int64_t T) { return int((T + 31) / 32 * 32); }

struct SyPlan {
  int nt = 0, ntl = 0, ips = 0, nchunk = 0, sf = 1, sd = 1;
  size_t table_bytes = 0, part_bytes = 0, vt_bytes = 0, ws_bytes = 0;
  uint32_t items[kSyMaxItems];
  bool ok = false;
};

// Split factors: the smallest full-tile split that gives every CU a work item,
// diagonal tiles (36/64 of a full tile's MFMAs when Q = K) split in proportion.
SyPlan sy_plan(int64_t nslab, int64_t T, int64_t N, bool self, bool rope, int64_t Dv = 0) {
  SyPlan p;
  if (T <= 0 || N <= 0 || N % 64 != 0 || nslab <= 0) return p;
  p.nt = int((T + kSyTile - 1) / kSyTile);
  p.ntl = p.nt * (p.nt + 1) / 2;
  p.nchunk = int(N / 64);
  if (p.ntl > kSyMaxTiles) return p;
  const int nfull = p.ntl - p.nt, ndiag = p.nt;
  int sf = 1, sd = 1;
  for (sf = 1; sf <= 8; ++sf) {
    sd = self ? std::max(1, (sf * 36 + 32) / 64) : sf;
    if (nslab * (nfull * sf + ndiag * sd) >= 256) break;
  }
  if (sf > 8) sf = 8;
  sf = std::min(sf, p.nchunk);
  sd = std::min(sd, p.nchunk);
  p.sf = sf;
  p.sd = sd;
  int n = 0;
  for (int ti = 0; ti < p.nt; ++ti)
    for (int tj = 0; tj <= ti; ++tj) {
      const int t = ti * (ti + 1) / 2 + tj;
      const int ns = (ti == tj) ? sd : sf;
      if (n + ns > kSyMaxItems) return p;
      (void)t;
      for (int s = 0; s < ns; ++s)
        p.items[n++] = uint32_t(ti) | (uint32_t(tj) << 8) | (uint32_t(s) << 16) | (uint32_t(ns) << 24);
    }
  p.ips = n;
  p.table_bytes = rope ? align_up(size_t(T) * size_t(sy_table_pitch(N)) * 4, 256) : 0;
  p.part_bytes = size_t(nslab) * size_t(p.ips) * kSyTileElems * sizeof(bf16_t);
  // V^T for the score x V product: at most one copy per (b, h) slab
  p.vt_bytes = align_up(size_t(nslab) * size_t(Dv) * size_t(sy_vt_pitch(T)) * sizeof(bf16_t), 256);
  p.ws_bytes = p.table_bytes + p.part_bytes + p.vt_bytes;
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

int sy_cold(const bdh_tensor4* q, const bdh_tensor4* k, const bdh_tensor4* v, const bdh_tensor4* out,
            const float* freqs, int64_t rope_start, const bdh_tensor4* qr, void* ws, size_t ws_bytes,
            hipStream_t s) {
  const int64_t B = q->size[0], H = q->size[1], T = q->size[2], N = q->size[3];
  if (q->dtype != BDH_BF16 || k->dtype != BDH_BF16) return kNotEligible;
  const bool self = q->data == k->data && q->stride[0] == k->stride[0] && q->stride[1] == k->stride[1] &&
                    q->stride[2] == k->stride[2];
  const bool rope = freqs != nullptr;
  if (rope && !self) return kNotEligible;
  if (T < 1 || N < 64 || N % 64 != 0 || !rows16(q) || !rows16(k)) return kNotEligible;
  if (v->size[3] > 256) return kNotEligible;  // score x V: four waves x 64 columns
  if (((T - 1) * std::max(q->stride[2], k->stride[2]) + N) * 2 >= (int64_t(1) << 31)) return kNotEligible;
  if (rope && int64_t(T) * sy_table_pitch(N) * 4 >= (int64_t(1) << 31)) return kNotEligible;
  if (T > 65535) return kNotEligible;
  if (qr != nullptr && (qr->dtype != BDH_BF16 || !rows16(qr))) return kNotEligible;
  const int64_t nslab = B * H;
  if (nslab > (int64_t(1) << 24)) return kNotEligible;
  const int64_t Dv = v->size[3];
  SyPlan p = sy_plan(nslab, T, N, self, rope, Dv);
  if (!p.ok) return kNotEligible;
  const int64_t grid_scores = 8 * ((nslab + 7) / 8) * p.ips;
  if (grid_scores >= (int64_t(1) << 31)) return kNotEligible;
  if (ws == nullptr || ws_bytes < p.ws_bytes) return BDH_ERR_WORKSPACE;

  uint8_t* wsb = static_cast<uint8_t*>(ws);
  uint32_t* table = rope ? reinterpret_cast<uint32_t*>(wsb) : nullptr;
  bf16_t* part = reinterpret_cast<bf16_t*>(wsb + p.table_bytes);
  const int tpitch = sy_table_pitch(N);
  if (rope) {
    BDH_LAUNCH("k_rope_table", k_rope_table, dim3(unsigned((N / 2 + 255) / 256), unsigned(T)), dim3(256), 0, s,
               freqs, rope_start, int(N / 2), tpitch, table);
  }
  SyArgs a;
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
  a.cs = table;
  a.tpitch = tpitch;
  a.part = part;
  a.qr = nullptr;
  a.r0 = a.r1 = a.r2 = 0;
  if (qr != nullptr && numel4(qr) > 0) {
    a.qr = static_cast<bf16_t*>(qr->data);
    a.r0 = qr->stride[0];
    a.r1 = qr->stride[1];
    a.r2 = qr->stride[2];
  }
  for (int i = 0; i < p.ips; ++i) a.items[i] = p.items[i];
  const dim3 gs{unsigned(grid_scores)};
  if (rope)
    BDH_LAUNCH("k_sy_scores", (k_sy_scores<true, true>), gs, dim3(kSyThreads), 0, s, a);
  else if (self)
    BDH_LAUNCH("k_sy_scores", (k_sy_scores<false, true>), gs, dim3(kSyThreads), 0, s, a);
  else
    BDH_LAUNCH("k_sy_scores", (k_sy_scores<false, false>), gs, dim3(kSyThreads), 0, s, a);
  if (numel4(out) == 0) return BDH_OK;

  // score x V: V^T once, then the direct-load MFMA kernel
  const int tp = sy_vt_pitch(T);
  bf16_t* vt = reinterpret_cast<bf16_t*>(wsb + p.table_bytes + p.part_bytes);
  const int Hv = int(v->size[1]);
  const int D = int(Dv);
  {
    View vv = view_of(v);
    vv.s1 = v->stride[1];
    const dim3 gv(unsigned((tp + 31) / 32), unsigned((D + 31) / 32), unsigned(B * Hv));
    if (v->dtype == BDH_BF16)
      BDH_LAUNCH("k_sy_vt", k_sy_vt<bf16_t>, gv, dim3(256), 0, s, vv, Hv, int(T), D, tp, vt);
    else
      BDH_LAUNCH("k_sy_vt", k_sy_vt<float>, gv, dim3(256), 0, s, vv, Hv, int(T), D, tp, vt);
  }
  SvArgs sa;
  sa.part = part;
  sa.vt = vt;
  sa.ips = p.ips;
  sa.sf = p.sf;
  sa.sd = p.sd;
  sa.H = int(H);
  sa.Hv = Hv;
  sa.T = int(T);
  sa.D = D;
  sa.tp = tp;
  sa.o = view_of(out);
  sa.o.s1 = out->stride[1];
  const dim3 gsv(unsigned((T + 31) / 32), unsigned(nslab));
  return out->dtype == BDH_BF16 ? launch_sy_sv<bf16_t>(sa, gsv, s) : launch_sy_sv<float>(sa, gsv, s);
}

}  // namespace bdh
