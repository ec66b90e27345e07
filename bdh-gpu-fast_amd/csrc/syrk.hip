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
//     * x streams HBM -> LDS through global_load_lds_dwordx4 into a 4-slot
//       ring of 32-wide k stages (issued three stages ahead).  The 16-byte
//       chunk c of row r sits at position c ^ ((r >> 2) & 3) of its 64-byte LDS
//       row, which makes the MFMA fragment reads bank-conflict free.
//     * RoPE is applied in place: the table entries of stage s+1 are DMA'd
//       into a fifth slot while stage s runs its MFMAs; then each lane rotates
//       the chunks it loaded itself (per pair two v_dot2_f32_bf16, products
//       exact in fp32, one v_cvt_pk_bf16_f32 and one v_alignbit_b32).  No vector-memory load of
//       the main loop returns to registers, so the only waits on it are the
//       explicit ones below.
//     * v_mfma_f32_32x32x16_bf16 with fp32 accumulators; the epilogue stores
//       fp32 partial tiles [slab][item][256][256].
//  3. k_sy_score_v: out = tril(sum over splits of S, -1) V with the 128x128
//     MFMA tile engine (scores rounded to bf16 as MFMA operands).
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
constexpr int kSySlots = 4;       // x ring; one more slot holds the RoPE table
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
  const uint32_t* cs;  // RoPE table [T][N/2] or null
  float* part;         // [nslab][ips][256*256]
  bf16_t* qr;          // optional RoPE(x) copy
  int64_t r0, r1, r2;
  uint32_t items[kSyMaxItems];  // ti | tj << 8 | split << 16 | nsplit << 24
};

__shared__ __attribute__((aligned(1024))) uint8_t sy_lds[(kSySlots + 1) * kSySlot];  // 160 KB

// ---------------------------------------------------------------- asm helpers
// The x stream and the table are moved by LDS DMA issued from inline asm, so
// the compiler neither counts them in its own vmcnt waits nor orders LDS
// accesses behind them; the kernel waits for them explicitly (sy_wait).
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
    default: asm volatile("s_waitcnt vmcnt(8)" ::: "memory"); break;
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
                                                    int T, int N2, uint32_t* __restrict__ cs) {
  const int64_t idx = int64_t(blockIdx.x) * 256 + threadIdx.x;
  if (idx >= int64_t(T) * N2) return;
  const int t = int(idx / N2), m = int(idx % N2);
  // phase = fp32(pos) * freq; theta = fp32(phase - floor(phase)) * fp32(2 pi)
  const float ph = __fmul_rn(float(rope_start + t), freqs[2 * m]);
  const float th = __fmul_rn(ph - floorf(ph), 6.28318530717958647692f);
  float s, c;
  sincosf(th, &s, &c);
  cs[idx] = pack_bf2(c, s);
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

  const bf16_t* baseA = a.q + b * a.q0 + h * a.q1;
  const bf16_t* baseB = SELF ? baseA : a.k + b * a.k0 + h * a.k1;
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
    toff[u] = uint32_t((int64_t(rc) * a.N + 8 * c) * 2);
  }
  // MFMA fragment offsets within a row block for the two k16 steps of a stage.
  uint32_t loff[2];
#pragma unroll
  for (int kk2 = 0; kk2 < 2; ++kk2) {
    const int c = (2 * kk2 + (lane >> 5)) ^ ((lane >> 2) & 3);
    loff[kk2] = uint32_t((lane & 31) * 64 + c * 16);
  }

  auto kofs = [&](int s) { return (split + nsplit * (s >> 1)) * 64 + (s & 1) * 32; };
  auto slot = [&](int s) { return sy_lds + (s & 3) * kSySlot; };
  uint8_t* const tslot = sy_lds + kSySlots * kSySlot;
  auto dma_x = [&](int s) {
    const uint32_t kb = uint32_t(kofs(s) * 2);
    const uint32_t sb = lds0 + uint32_t((s & 3) * kSySlot);
#pragma unroll
    for (int u = 0; u < 4; ++u)
      if (u < ndma) dma16(sb + uint32_t((u * 8 + w) * 1024), u < 2 ? baseA : baseB, xoff[u] + kb);
  };
  // table entries of the chunks this lane moves, at the same offsets in the table slot
  auto dma_t = [&](int s) {
    const uint32_t kb = uint32_t(kofs(s) * 2);
    const uint32_t sb = lds0 + uint32_t(kSySlots * kSySlot);
#pragma unroll
    for (int u = 0; u < 4; ++u)
      if (u < ndma) dma16(sb + uint32_t((u * 8 + w) * 1024), a.cs, toff[u] + kb);
  };
  auto rotate = [&](int s) {
    uint8_t* sl = slot(s);
    const int k0 = kofs(s);
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      if (u < ndma) {
        const int off = (u * 8 + w) * 1024 + lane * 16;
        u32x4* p = reinterpret_cast<u32x4*>(sl + off);
        const u32x4 x = *p;
        const u32x4 t = *reinterpret_cast<const u32x4*>(tslot + off);
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
  auto run = [&](auto wt_tag) {
    constexpr int WT = decltype(wt_tag)::value;
    auto mma_stage = [&](int s) {
      const uint8_t* A = slot(s);
      const uint8_t* B = diag ? A : A + kSyBlk;
#pragma unroll
      for (int k2 = 0; k2 < 2; ++k2) {
        const uint32_t lo = loff[k2];
        if constexpr (WT == 0 || WT == 1) {
          bf16x8 fa[4], fb[2];
#pragma unroll
          for (int i = 0; i < 4; ++i) fa[i] = frag(A, 4 * wm + i, lo);
#pragma unroll
          for (int j = 0; j < 2; ++j) fb[j] = frag(B, 2 * wn + j, lo);
#pragma unroll
          for (int i = 0; i < 4; ++i)
#pragma unroll
            for (int j = 0; j < 2; ++j)
              if (WT == 0 || i >= j) acc[2 * i + j] = mma(fa[i], fb[j], acc[2 * i + j]);
        } else if constexpr (WT == 2) {
          bf16x8 fa[2], fb[2];
#pragma unroll
          for (int i = 0; i < 2; ++i) fa[i] = frag(A, 4 * wm + 2 + i, lo);
#pragma unroll
          for (int j = 0; j < 2; ++j) fb[j] = frag(B, 2 * wn + j, lo);
          acc[4] = mma(fa[0], fb[0], acc[4]);
          acc[6] = mma(fa[1], fb[0], acc[6]);
          acc[7] = mma(fa[1], fb[1], acc[7]);
        }
      }
    };
    constexpr auto live = [](int i, int j) { return WT == 0 || (WT == 1 && i >= j) || (WT == 2 && i >= j + 2); };
    // ------------------------------------------------------------ prologue
    // Issue order is what the waits count on: operations complete in order.
    if (ROPE) dma_t(0);
    dma_x(0);
    if (nst > 1) dma_x(1);
    if (nst > 2) dma_x(2);
    if (ROPE) {
      sy_wait((nst > 1 ? ndma : 0) + (nst > 2 ? ndma : 0));  // table and x of stage 0
      rotate(0);
    } else {
      sy_wait((nst > 1 ? ndma : 0) + (nst > 2 ? ndma : 0));  // x of stage 0
    }
    sy_barrier();

    // ------------------------------------------------------------ main loop
    for (int s = 0; s < nst; ++s) {
      // slot (s+3)&3 held stage s-1, whose MFMAs ended before the last barrier;
      // the table slot held stage s, rotated before it.
      if (ROPE && s + 1 < nst) dma_t(s + 1);
      if (s + 3 < nst) dma_x(s + 3);
      mma_stage(s);
      if (s + 1 < nst) {
        // ROPE: the table of stage s+1 (and everything issued before it, so the
        // x of stages <= s+2); plain: the x of stage s+1 of every wave.
        if (ROPE) {
          sy_wait(s + 3 < nst ? ndma : 0);
          rotate(s + 1);
        } else {
          sy_wait((s + 2 < nst ? ndma : 0) + (s + 3 < nst ? ndma : 0));
        }
      }
      sy_barrier();
    }

    // ------------------------------------------------------------ epilogue
    float* dst = a.part + (int64_t(slab) * a.ips + itx) * kSyTileElems;
    auto store_block = [&](const f32x16& c, int rb, int cb) {
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int row = rb * 32 + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
        const int col = cb * 32 + (lane & 31);
        dst[row * kSyTile + col] = c[r];
      }
    };
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int j = 0; j < 2; ++j)
        if (live(i, j)) store_block(acc[2 * i + j], 4 * wm + i, 2 * wn + j);
  };
  switch (wtype) {
    case 0: run(std::integral_constant<int, 0>()); break;
    case 1: run(std::integral_constant<int, 1>()); break;
    case 2: run(std::integral_constant<int, 2>()); break;
    default: run(std::integral_constant<int, 3>()); break;
  }
}

// ---------------------------------------------------------------- score x V
struct SyVArgs {
  const float* part;
  int ips;
  View v;
  int64_t H, Hv, T, Dv;
  bool vec4_v;
  View o;
  int sf, sd;  // splits of off-diagonal / diagonal tiles (items ordered tile by tile)
};

// A operand of out = tril(S, -1) V: rows i of the 128-row block R, k = j; the
// sum of a tile's split partials, masked to j < i, as bf16.
struct PartRows {
  static constexpr int BK = Mode<true>::BK, E = Mode<true>::E;
  static constexpr int CPR = BK / E;
  static constexpr int CPT = kTile * CPR / kNT;

  const float* slab = nullptr;
  int T = 0, sf = 1, sd = 1;
  int R = 0;
  float v[CPT][E];

  __device__ __forceinline__ void load(int k0) {
#pragma unroll
    for (int c = 0; c < CPT; ++c) {
      const int ch = threadIdx.x + c * kNT;
      const int row = ch / CPR, kc = (ch % CPR) * E;
      const int gi = R * kTile + row, gj = k0 + kc;
#pragma unroll
      for (int e = 0; e < E; ++e) v[c][e] = 0.f;
      if (gi < T && gj < gi) {
        const int ti = gi >> 8, tj = gj >> 8;
        // items of the lower tiles in row-major order: row r holds r tiles of
        // sf splits and one diagonal tile of sd splits
        const int first = sf * (ti * (ti - 1) / 2 + tj) + sd * ti;
        const float* p = slab + int64_t(first) * kSyTileElems + (gi & 255) * kSyTile + (gj & 255);
        const int ns = ti == tj ? sd : sf;
        for (int sp = 0; sp < ns; ++sp) {
          const float4 x0 = *reinterpret_cast<const float4*>(p + int64_t(sp) * kSyTileElems);
          const float4 x1 = *reinterpret_cast<const float4*>(p + int64_t(sp) * kSyTileElems + 4);
          v[c][0] += x0.x; v[c][1] += x0.y; v[c][2] += x0.z; v[c][3] += x0.w;
          v[c][4] += x1.x; v[c][5] += x1.y; v[c][6] += x1.z; v[c][7] += x1.w;
        }
      }
    }
  }

  __device__ __forceinline__ void store(LdsTile<true> dst, int k0) {
#pragma unroll
    for (int c = 0; c < CPT; ++c) {
      const int ch = threadIdx.x + c * kNT;
      const int row = ch / CPR, kc = (ch % CPR) * E;
      const int gi = R * kTile + row, gj = k0 + kc;
      float f[E];
#pragma unroll
      for (int e = 0; e < E; ++e) f[e] = (gj + e < gi) ? v[c][e] : 0.f;
      lds_put<true>(dst, row, kc, f);
    }
  }
};

template <typename TV, typename TO>
__global__ __launch_bounds__(kNT) void k_sy_score_v(const SyVArgs a) {
  __shared__ Smem<true> sm;
  const int R = blockIdx.x, Dt = blockIdx.y, slab = blockIdx.z;
  const int b = slab / int(a.H), h = slab % int(a.H);
  const int hv = a.Hv == 1 ? 0 : h;
  PartRows la;
  la.slab = a.part + int64_t(slab) * a.ips * kSyTileElems;
  la.T = int(a.T);
  la.sf = a.sf;
  la.sd = a.sd;
  la.R = R;
  NRows<TV, true, false> lb;
  lb.base = static_cast<const TV*>(a.v.p) + b * a.v.s0 + hv * a.v.s1;
  lb.rs = a.v.s2;
  lb.n0 = Dt * kTile;
  lb.ncols = int(a.Dv);
  lb.krows = int(a.T);
  lb.vec4 = a.vec4_v;
  f32x16 acc[2][2];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.f;
  const int ke = int(min(a.T, int64_t(R + 1) * kTile));
  mainloop<true, false>(sm, la, lb, false, 0, ke, acc, true);
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int wm = wave >> 1, wn = wave & 1;
  TO* o = static_cast<TO*>(const_cast<void*>(a.o.p)) + b * a.o.s0 + h * a.o.s1;
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        int row, col;
        acc_coord<false>(wm, wn, lane, i, j, r, row, col);
        const int gi = R * kTile + row, gd = Dt * kTile + col;
        if (gi < a.T && gd < a.Dv) o[int64_t(gi) * a.o.s2 + gd] = from_f<TO>(acc[i][j][r]);
      }
}

// ---------------------------------------------------------------- host plan
struct SyPlan {
  int nt = 0, ntl = 0, ips = 0, nchunk = 0, sf = 1, sd = 1;
  size_t table_bytes = 0, part_bytes = 0, ws_bytes = 0;
  uint32_t items[kSyMaxItems];
  bool ok = false;
};

// Split factors: the smallest full-tile split that gives every CU a work item,
// diagonal tiles (36/64 of a full tile's MFMAs when Q = K) split in proportion.
SyPlan sy_plan(int64_t nslab, int64_t T, int64_t N, bool self, bool rope) {
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
  p.table_bytes = rope ? align_up(size_t(T) * size_t(N / 2) * 4, 256) : 0;
  p.part_bytes = size_t(nslab) * size_t(p.ips) * kSyTileElems * sizeof(float);
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

template <typename TV, typename TO>
int launch_sy_sv(const SyVArgs& va, int64_t nslab, hipStream_t s) {
  dim3 grid(unsigned((va.T + kTile - 1) / kTile), unsigned((va.Dv + kTile - 1) / kTile), unsigned(nslab));
  BDH_LAUNCH("k_sy_score_v", (k_sy_score_v<TV, TO>), grid, dim3(kNT), 0, s, va);
  return BDH_OK;
}

}  // namespace

size_t sy_workspace(int64_t B, int64_t H, int64_t T, int64_t N, bool rope) {
  const SyPlan p = sy_plan(B * H, T, N, true, rope);
  const SyPlan p2 = sy_plan(B * H, T, N, false, rope);
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
  if (((T - 1) * std::max(q->stride[2], k->stride[2]) + N) * 2 >= (int64_t(1) << 31)) return kNotEligible;
  if (rope && int64_t(T) * N * 2 >= (int64_t(1) << 31)) return kNotEligible;
  if (qr != nullptr && (qr->dtype != BDH_BF16 || !rows16(qr))) return kNotEligible;
  const int64_t nslab = B * H;
  if (nslab > (int64_t(1) << 24)) return kNotEligible;
  SyPlan p = sy_plan(nslab, T, N, self, rope);
  if (!p.ok) return kNotEligible;
  if (ws == nullptr || ws_bytes < p.ws_bytes) return BDH_ERR_WORKSPACE;

  uint8_t* wsb = static_cast<uint8_t*>(ws);
  uint32_t* table = rope ? reinterpret_cast<uint32_t*>(wsb) : nullptr;
  float* part = reinterpret_cast<float*>(wsb + p.table_bytes);
  if (rope) {
    const int64_t n = T * (N / 2);
    BDH_LAUNCH("k_rope_table", k_rope_table, dim3(unsigned((n + 255) / 256)), dim3(256), 0, s, freqs, rope_start,
               int(T), int(N / 2), table);
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
  const int64_t grid = 8 * ((nslab + 7) / 8) * p.ips;
  if (grid >= (int64_t(1) << 31)) return kNotEligible;
  if (rope)
    BDH_LAUNCH("k_sy_scores", (k_sy_scores<true, true>), dim3(unsigned(grid)), dim3(kSyThreads), 0, s, a);
  else if (self)
    BDH_LAUNCH("k_sy_scores", (k_sy_scores<false, true>), dim3(unsigned(grid)), dim3(kSyThreads), 0, s, a);
  else
    BDH_LAUNCH("k_sy_scores", (k_sy_scores<false, false>), dim3(unsigned(grid)), dim3(kSyThreads), 0, s, a);
  if (numel4(out) == 0) return BDH_OK;

  SyVArgs va;
  va.part = part;
  va.ips = p.ips;
  va.v = view_of(v);
  va.H = H;
  va.Hv = v->size[1];
  va.T = T;
  va.Dv = v->size[3];
  va.vec4_v = vec4_rows_sy(v);
  va.o = view_of(out);
  va.o.s1 = out->stride[1];
  va.sf = p.sf;
  va.sd = p.sd;
  const bool vb = v->dtype == BDH_BF16, ob = out->dtype == BDH_BF16;
  if (vb) return ob ? launch_sy_sv<bf16_t, bf16_t>(va, nslab, s) : launch_sy_sv<bf16_t, float>(va, nslab, s);
  return ob ? launch_sy_sv<float, bf16_t>(va, nslab, s) : launch_sy_sv<float, float>(va, nslab, s);
}

}  // namespace bdh
