// 128x128 MFMA tile engine for gfx950 (CDNA4), shared by the forward,
// score x V and backward kernels.
//
// A workgroup is 256 threads = 4 wave64s arranged 2x2; each wave owns a 64x64
// sub-tile made of 2x2 blocks of 32x32 MFMA accumulators (16 fp32 registers
// per block per lane).  Both operands are staged in LDS in "K-contiguous"
// form, A as [row][k] and B as [col][k], double-buffered: the global loads of
// stage s+1 are issued before the MFMAs of stage s, and transformed (RoPE,
// masks, dtype conversion) and written to the other LDS buffer after them.
//
// bf16 mode: v_mfma_f32_32x32x16_bf16, K-stage 64, LDS pitch 72 elements
// (144 B: conflict-free 16-byte fragment reads).  fp32 mode:
// v_mfma_f32_32x32x2f32, K-stage 32, LDS pitch 33 floats (conflict-free
// 4-byte fragment reads).
//
// Accumulator layout of a 32x32 block (lane l, register r = 0..15):
//   row = 8*(r/4) + 4*(l/32) + r%4, col = l%32.
// With TRANS the operands are swapped in the MFMA, so the block holds C^T:
//   C[row = l%32][col = 8*(r/4) + 4*(l/32) + r%4].
#pragma once

#include <type_traits>

#include "common.h"

namespace bdh {

constexpr int kNT = 256;    // threads per workgroup
constexpr int kTile = 128;  // output tile edge
constexpr int kTileElems = kTile * kTile;

template <bool BF> struct Mode;
template <> struct Mode<true> {
  static constexpr int BK = 64;
  static constexpr int E = 8;  // k elements per 16-byte LDS chunk
  static constexpr int LDSW = BK + 8;
  typedef bf16_t lds_t;
};
template <> struct Mode<false> {
  static constexpr int BK = 32;
  static constexpr int E = 4;
  static constexpr int LDSW = BK + 1;
  typedef float lds_t;
};

template <bool BF> struct Smem {
  typedef typename Mode<BF>::lds_t T;
  T a[2][kTile][Mode<BF>::LDSW];
  T b[2][kTile][Mode<BF>::LDSW];
};

template <bool BF> using LdsTile = typename Mode<BF>::lds_t (*)[Mode<BF>::LDSW];
template <bool BF> using CLdsTile = const typename Mode<BF>::lds_t (*)[Mode<BF>::LDSW];

// Packed index of lower tile (ti >= tj).
__device__ __forceinline__ int lower_tile_index(int ti, int tj) { return ti * (ti + 1) / 2 + tj; }
__device__ __forceinline__ void lower_tile_coords(int t, int& ti, int& tj) {
  int i = int((sqrtf(8.0f * float(t) + 1.0f) - 1.0f) * 0.5f);
  while (i * (i + 1) / 2 > t) --i;
  while ((i + 1) * (i + 2) / 2 <= t) ++i;
  ti = i;
  tj = t - i * (i + 1) / 2;
}

// Write E floats of one LDS chunk.
template <bool BF>
__device__ __forceinline__ void lds_put(LdsTile<BF> dst, int row, int kc, const float* f) {
  if constexpr (BF) {
    uint4 w;
    w.x = pack_bf2(f[0], f[1]);
    w.y = pack_bf2(f[2], f[3]);
    w.z = pack_bf2(f[4], f[5]);
    w.w = pack_bf2(f[6], f[7]);
    *reinterpret_cast<uint4*>(&dst[row][kc]) = w;
  } else {
#pragma unroll
    for (int e = 0; e < 4; ++e) dst[row][kc + e] = f[e];
  }
}

// One LDS stage of MFMAs for this wave's 2x2 blocks.
template <bool BF, bool TRANS>
__device__ __forceinline__ void mma_stage(CLdsTile<BF> A, CLdsTile<BF> B, f32x16 (&acc)[2][2],
                                          int wm, int wn, int lane) {
  const int r = lane & 31;
  if constexpr (BF) {
    const int ko = (lane >> 5) * 8;
#pragma unroll
    for (int kk = 0; kk < Mode<true>::BK; kk += 16) {
      bf16x8 a[2], b[2];
#pragma unroll
      for (int i = 0; i < 2; ++i)
        a[i] = *reinterpret_cast<const bf16x8*>(&A[wm * 64 + i * 32 + r][kk + ko]);
#pragma unroll
      for (int j = 0; j < 2; ++j)
        b[j] = *reinterpret_cast<const bf16x8*>(&B[wn * 64 + j * 32 + r][kk + ko]);
#pragma unroll
      for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j) {
          if constexpr (TRANS)
            acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(b[j], a[i], acc[i][j], 0, 0, 0);
          else
            acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[i], b[j], acc[i][j], 0, 0, 0);
        }
    }
  } else {
    const int ko = lane >> 5;
#pragma unroll
    for (int kk = 0; kk < Mode<false>::BK; kk += 2) {
      float a[2], b[2];
#pragma unroll
      for (int i = 0; i < 2; ++i) a[i] = A[wm * 64 + i * 32 + r][kk + ko];
#pragma unroll
      for (int j = 0; j < 2; ++j) b[j] = B[wn * 64 + j * 32 + r][kk + ko];
#pragma unroll
      for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j) {
          if constexpr (TRANS)
            acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(b[j], a[i], acc[i][j], 0, 0, 0);
          else
            acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(a[i], b[j], acc[i][j], 0, 0, 0);
        }
    }
  }
}

// Double-buffered main loop over k in [kb, ke) (kb a multiple of BK; the
// loaders zero-fill past their own limits).  When b_is_a the B operand is the
// A tile itself (diagonal tiles of Q = K), so B is neither loaded nor stored.
// Inactive waves load and synchronise but issue no MFMAs.
template <bool BF, bool TRANS, class LA, class LB>
__device__ __forceinline__ void mainloop(Smem<BF>& sm, LA& la, LB& lb, bool b_is_a, int kb, int ke,
                                         f32x16 (&acc)[2][2], bool active) {
  constexpr int BK = Mode<BF>::BK;
  if (kb >= ke) return;
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int wm = wave >> 1, wn = wave & 1;
  la.load(kb);
  if (!b_is_a) lb.load(kb);
  la.store(sm.a[0], kb);
  if (!b_is_a) lb.store(sm.b[0], kb);
  __syncthreads();
  int buf = 0;
  for (int k0 = kb; k0 < ke; k0 += BK) {
    const bool next = k0 + BK < ke;
    if (next) {
      la.load(k0 + BK);
      if (!b_is_a) lb.load(k0 + BK);
    }
    if (active)
      mma_stage<BF, TRANS>(sm.a[buf], b_is_a ? sm.a[buf] : sm.b[buf], acc, wm, wn, lane);
    if (next) {
      la.store(sm.a[buf ^ 1], k0 + BK);
      if (!b_is_a) lb.store(sm.b[buf ^ 1], k0 + BK);
    }
    __syncthreads();
    buf ^= 1;
  }
}

// Tile-relative coordinates of accumulator element (block i,j; register r).
template <bool TRANS>
__device__ __forceinline__ void acc_coord(int wm, int wn, int lane, int i, int j, int r, int& row,
                                          int& col) {
  const int rr = 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
  if constexpr (TRANS) {
    row = wm * 64 + i * 32 + (lane & 31);
    col = wn * 64 + j * 32 + rr;
  } else {
    row = wm * 64 + i * 32 + rr;
    col = wn * 64 + j * 32 + (lane & 31);
  }
}

// ------------------------------------------------------------------------
// Loader: rows of a K-contiguous matrix, staged as LDS [row][k].
// ROPE rotates adjacent pairs along k with position pos0 + row.
// MASK 1 keeps k < row, MASK 2 keeps k > row (global indices), MASK 0 none.
// ------------------------------------------------------------------------
template <typename TIn, bool BF, bool ROPE, int MASK>
struct KRows {
  static constexpr int BK = Mode<BF>::BK, E = Mode<BF>::E;
  static constexpr int CPR = BK / E;               // chunks per row
  static constexpr int CPT = kTile * CPR / kNT;    // chunks per thread
  static constexpr bool RAW = BF && std::is_same<TIn, bf16_t>::value && !ROPE && MASK == 0;

  const TIn* base = nullptr;
  int64_t rs = 0;    // row stride (elements)
  int r0 = 0;        // first row of the tile
  int nrows = 0;     // rows < nrows are valid
  int rlo = 0;       // rows < rlo are zero; row gr reads source row gr - rlo
  int K = 0;         // k < K is valid
  bool vec = false;  // 16-byte row access is legal
  const float* freqs = nullptr;
  float pos0 = 0.f;
  // Optional copy of the rotated rows (fused forward, diagonal tiles).
  void* qr = nullptr;
  int64_t qr_rs = 0;
  bool qr_bf = false;

  TIn v[CPT][E];
  float fq[ROPE ? CPT : 1][ROPE ? E / 2 : 1];

  __device__ __forceinline__ void load(int k0) {
#pragma unroll
    for (int c = 0; c < CPT; ++c) {
      const int ch = threadIdx.x + c * kNT;
      const int row = ch / CPR, kc = (ch % CPR) * E;
      const int gr = r0 + row, gk = k0 + kc;
      const bool rok = gr >= rlo && gr < nrows;
      const TIn* p = base + int64_t(rok ? gr - rlo : 0) * rs + gk;
      if (rok && vec && gk + E <= K) {
        if constexpr (sizeof(TIn) * E == 16) {
          *reinterpret_cast<uint4*>(v[c]) = *reinterpret_cast<const uint4*>(p);
        } else if constexpr (sizeof(TIn) * E == 32) {
          reinterpret_cast<uint4*>(v[c])[0] = reinterpret_cast<const uint4*>(p)[0];
          reinterpret_cast<uint4*>(v[c])[1] = reinterpret_cast<const uint4*>(p)[1];
        } else {
          *reinterpret_cast<uint2*>(v[c]) = *reinterpret_cast<const uint2*>(p);
        }
      } else {
#pragma unroll
        for (int e = 0; e < E; ++e) v[c][e] = (rok && gk + e < K) ? p[e] : TIn(0);
      }
      if constexpr (ROPE) {
#pragma unroll
        for (int q = 0; q < E / 2; ++q) fq[c][q] = (gk + 2 * q < K) ? freqs[gk + 2 * q] : 0.f;
      }
    }
  }

  __device__ __forceinline__ void store(LdsTile<BF> dst, int k0) {
#pragma unroll
    for (int c = 0; c < CPT; ++c) {
      const int ch = threadIdx.x + c * kNT;
      const int row = ch / CPR, kc = (ch % CPR) * E;
      if constexpr (RAW) {
        *reinterpret_cast<uint4*>(&dst[row][kc]) = *reinterpret_cast<const uint4*>(v[c]);
      } else {
        const int gr = r0 + row, gk = k0 + kc;
        float f[E];
#pragma unroll
        for (int e = 0; e < E; ++e) f[e] = to_f(v[c][e]);
        if constexpr (ROPE) {
          const float pos = pos0 + float(gr);
#pragma unroll
          for (int q = 0; q < E / 2; ++q) {
            float cs, sn;
            rope_cs(pos, fq[c][q], cs, sn);
            const float x0 = f[2 * q], x1 = f[2 * q + 1];
            f[2 * q] = x0 * cs - x1 * sn;
            f[2 * q + 1] = x1 * cs + x0 * sn;
          }
          if (qr != nullptr && gr < nrows) store_qr(gr, gk, f);
        }
        if constexpr (MASK == 1) {
#pragma unroll
          for (int e = 0; e < E; ++e)
            if (!(gk + e < gr)) f[e] = 0.f;
        } else if constexpr (MASK == 2) {
#pragma unroll
          for (int e = 0; e < E; ++e)
            if (!(gk + e > gr)) f[e] = 0.f;
        }
        lds_put<BF>(dst, row, kc, f);
      }
    }
  }

  __device__ __forceinline__ void store_qr(int gr, int gk, const float* f) {
    if (qr_bf) {
      bf16_t* o = reinterpret_cast<bf16_t*>(qr) + int64_t(gr) * qr_rs + gk;
#pragma unroll
      for (int e = 0; e < E; ++e)
        if (gk + e < K) o[e] = f2bf(f[e]);
    } else {
      float* o = reinterpret_cast<float*>(qr) + int64_t(gr) * qr_rs + gk;
#pragma unroll
      for (int e = 0; e < E; ++e)
        if (gk + e < K) o[e] = f[e];
    }
  }
};

// ------------------------------------------------------------------------
// Loader: B operand from a [k][n] matrix (n contiguous), staged as LDS
// [n][k].  One unit of 4 columns x E k-rows per thread per stage.  ROPE
// rotates adjacent column pairs with position pos0 + k.
// ------------------------------------------------------------------------
template <typename TIn, bool BF, bool ROPE>
struct NRows {
  static constexpr int BK = Mode<BF>::BK, E = Mode<BF>::E;
  static_assert((kTile / 4) * (BK / E) == kNT, "one unit per thread");

  const TIn* base = nullptr;
  int64_t rs = 0;     // stride between k rows (elements)
  int n0 = 0;         // first column of the tile
  int ncols = 0;      // columns < ncols are valid
  int krows = 0;      // k rows < krows are valid
  bool vec4 = false;  // 4-element row access is legal
  const float* freqs = nullptr;
  float pos0 = 0.f;

  TIn v[E][4];
  float fq[2];

  __device__ __forceinline__ void load(int k0) {
    const int nq = threadIdx.x & 31, kg = threadIdx.x >> 5;
    const int gn = n0 + nq * 4;
#pragma unroll
    for (int e = 0; e < E; ++e) {
      const int gk = k0 + kg * E + e;
      const TIn* p = base + int64_t(gk) * rs + gn;
      if (gk < krows && vec4 && gn + 4 <= ncols) {
        if constexpr (sizeof(TIn) == 2)
          *reinterpret_cast<uint2*>(v[e]) = *reinterpret_cast<const uint2*>(p);
        else
          *reinterpret_cast<uint4*>(v[e]) = *reinterpret_cast<const uint4*>(p);
      } else {
#pragma unroll
        for (int x = 0; x < 4; ++x) v[e][x] = (gk < krows && gn + x < ncols) ? p[x] : TIn(0);
      }
    }
    if constexpr (ROPE) {
      fq[0] = gn < ncols ? freqs[gn] : 0.f;
      fq[1] = gn + 2 < ncols ? freqs[gn + 2] : 0.f;
    }
  }

  __device__ __forceinline__ void store(LdsTile<BF> dst, int k0) {
    const int nq = threadIdx.x & 31, kg = threadIdx.x >> 5;
    float f[4][E];
#pragma unroll
    for (int e = 0; e < E; ++e) {
      float x[4];
#pragma unroll
      for (int c = 0; c < 4; ++c) x[c] = to_f(v[e][c]);
      if constexpr (ROPE) {
        const float pos = pos0 + float(k0 + kg * E + e);
#pragma unroll
        for (int q = 0; q < 2; ++q) {
          float cs, sn;
          rope_cs(pos, fq[q], cs, sn);
          const float x0 = x[2 * q], x1 = x[2 * q + 1];
          x[2 * q] = x0 * cs - x1 * sn;
          x[2 * q + 1] = x1 * cs + x0 * sn;
        }
      }
#pragma unroll
      for (int c = 0; c < 4; ++c) f[c][e] = x[c];
    }
#pragma unroll
    for (int c = 0; c < 4; ++c) lds_put<BF>(dst, nq * 4 + c, kg * E, f[c]);
  }
};

// ------------------------------------------------------------------------
// Loader: A operand summed over split-K partial score tiles (fp32, packed
// lower tiles of 128x128 per slab).  DV=false (score x V): A row i, k = j,
// tile (R, C), keep j < i.  DV=true (dV): partials stored transposed, A row
// j, k = i, tile (C, R), keep i > j.
// ------------------------------------------------------------------------
template <bool BF, bool DV>
struct SplitRows {
  static constexpr int BK = Mode<BF>::BK, E = Mode<BF>::E;
  static constexpr int CPR = BK / E;
  static constexpr int CPT = kTile * CPR / kNT;

  const float* slab = nullptr;  // partials of this slab, split 0
  int64_t split_stride = 0;     // floats between splits
  int nsplit = 1;
  int R = 0;                    // A row-tile index
  int t0 = 0;                   // packed index of the first stored tile

  float v[CPT][E];

  __device__ __forceinline__ void load(int k0) {
    const int C = k0 / kTile;
    const int tile = (DV ? lower_tile_index(C, R) : lower_tile_index(R, C)) - t0;
    const float* t = slab + int64_t(tile) * kTileElems + (k0 % kTile);
#pragma unroll
    for (int c = 0; c < CPT; ++c) {
      const int ch = threadIdx.x + c * kNT;
      const int row = ch / CPR, kc = (ch % CPR) * E;
      const float* p = t + row * kTile + kc;
      float s[E];
#pragma unroll
      for (int e = 0; e < E; e += 4) *reinterpret_cast<float4*>(&s[e]) = *reinterpret_cast<const float4*>(p + e);
      for (int sp = 1; sp < nsplit; ++sp) {
        const float* ps = p + sp * split_stride;
#pragma unroll
        for (int e = 0; e < E; e += 4) {
          const float4 w = *reinterpret_cast<const float4*>(ps + e);
          s[e] += w.x;
          s[e + 1] += w.y;
          s[e + 2] += w.z;
          s[e + 3] += w.w;
        }
      }
#pragma unroll
      for (int e = 0; e < E; ++e) v[c][e] = s[e];
    }
  }

  __device__ __forceinline__ void store(LdsTile<BF> dst, int k0) {
#pragma unroll
    for (int c = 0; c < CPT; ++c) {
      const int ch = threadIdx.x + c * kNT;
      const int row = ch / CPR, kc = (ch % CPR) * E;
      const int gr = R * kTile + row, gk = k0 + kc;
      float f[E];
#pragma unroll
      for (int e = 0; e < E; ++e) {
        const bool keep = DV ? (gk + e > gr) : (gk + e < gr);
        f[e] = keep ? v[c][e] : 0.f;
      }
      lds_put<BF>(dst, row, kc, f);
    }
  }
};

}  // namespace bdh
