// Elementwise consumer of the attention in the BDH layer, for gfx950:
//   out = x * max(y, 0)
// the ReLU of encoder_v's output and the sparse product x * y that feeds the
// decoder.  The operands are 4-D strided views of equal sizes, so y can stay
// in the head-major layout a batched GEMM leaves ((nh, B, T, N) viewed as
// (B, T, nh, N)) while x and out are the token-major (B, T, nh, N) tensors.
//
// One workgroup of 256 threads covers 2048 elements of one row (the last
// dimension); rows are blockIdx.x, so there is no per-thread index division.
// With 16-byte aligned rows each thread moves 8 elements per operand.  The
// product is formed in fp32 and rounded once to the output dtype, the same
// value torch's bf16 / fp32 elementwise product gives.
#include "common.h"
#include "lds_dma.h"
#include "tile_gemm.h"


namespace bdh {

struct ReluMulArgs {
  View x, y, o;
  int64_t d1, d2, n;  // sizes of dims 1, 2 and 3
  int vec8;           // all views: 16-byte aligned 8-element chunks
};

template <typename T>
__device__ inline void load8(const T* p, float (&f)[8]) {
  if constexpr (sizeof(T) == 2) {
    const uint4 u = *reinterpret_cast<const uint4*>(p);
    const uint32_t w[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      f[2 * i] = __uint_as_float(w[i] << 16);
      f[2 * i + 1] = __uint_as_float(w[i] & 0xffff0000u);
    }
  } else {
    const float4 a = *reinterpret_cast<const float4*>(p);
    const float4 b = *reinterpret_cast<const float4*>(p + 4);
    f[0] = a.x; f[1] = a.y; f[2] = a.z; f[3] = a.w;
    f[4] = b.x; f[5] = b.y; f[6] = b.z; f[7] = b.w;
  }
}

template <typename T>
__device__ inline void store8(T* p, const float (&f)[8]) {
  if constexpr (sizeof(T) == 2) {
    uint4 u;
    u.x = pack_bf2(f[0], f[1]);
    u.y = pack_bf2(f[2], f[3]);
    u.z = pack_bf2(f[4], f[5]);
    u.w = pack_bf2(f[6], f[7]);
    *reinterpret_cast<uint4*>(p) = u;
  } else {
    *reinterpret_cast<float4*>(p) = make_float4(f[0], f[1], f[2], f[3]);
    *reinterpret_cast<float4*>(p + 4) = make_float4(f[4], f[5], f[6], f[7]);
  }
}

// max(v, 0) with NaN passed through, as torch's relu does
__device__ inline float relu_f(float v) { return v != v ? v : fmaxf(v, 0.f); }

template <typename TX, typename TY, typename TO>
__global__ __launch_bounds__(256) void k_relu_mul(ReluMulArgs a) {
  const int64_t row = blockIdx.x;
  const int64_t i2 = row % a.d2, r1 = row / a.d2;
  const int64_t i1 = r1 % a.d1, i0 = r1 / a.d1;
  const TX* xp = static_cast<const TX*>(a.x.p) + i0 * a.x.s0 + i1 * a.x.s1 + i2 * a.x.s2;
  const TY* yp = static_cast<const TY*>(a.y.p) + i0 * a.y.s0 + i1 * a.y.s1 + i2 * a.y.s2;
  TO* op = static_cast<TO*>(const_cast<void*>(a.o.p)) + i0 * a.o.s0 + i1 * a.o.s1 + i2 * a.o.s2;
  const int64_t c0 = (int64_t(blockIdx.y) * 256 + threadIdx.x) * 8;
  if (c0 >= a.n) return;
  if (a.vec8) {
    float fx[8], fy[8], fo[8];
    load8(xp + c0, fx);
    load8(yp + c0, fy);
#pragma unroll
    for (int i = 0; i < 8; ++i) fo[i] = fx[i] * relu_f(fy[i]);
    store8(op + c0, fo);
  } else {
    const int64_t e = c0 + 8 < a.n ? c0 + 8 : a.n;
    for (int64_t c = c0; c < e; ++c) op[c] = from_f<TO>(to_f(xp[c]) * relu_f(to_f(yp[c])));
  }
}

// ---------------------------------------------------------------------------
// encoder_v GEMM with the gated product as its epilogue:
//   out[b,t,h,n] = x[b,t,h,n] * relu(sum_k y[b,h,t,k] * wt[h,n,k])       (bf16)
// y is the LayerNorm of the attention output (B, nh, T, K), wt encoder_v
// transposed to (nh, N, K), so both operands are K-contiguous rows.  y never
// goes to HBM: the kernel reads x once and writes out once.
//
// Tiles of 256 rows (tokens) x 128 columns of one head, 8 waves of 64 x 64
// (2 x 2 MFMA 32x32x16 blocks), K in stages of 32 through a ring of three LDS
// buffers filled by LDS DMA two stages ahead (16-byte chunk c of row r at
// c ^ ((r >> 2) & 3), conflict-free fragment reads; no register staging).
// Two workgroups per CU, so one tile's epilogue overlaps another's main loop.  Tiles run column
// blocks fastest (the tiles in flight on an XCD share their A block and cover
// whole rows of one head), each XCD a contiguous range.
// Epilogue: relu(acc) rounded to bf16 (the value the unfused GEMM would
// store) goes to LDS, then 16-byte coalesced reads of x and stores of out.
constexpr int kGM = 256, kGN = 128, kGK = 32;
constexpr int kGStageA = kGM * 64, kGStageB = kGN * 64, kGStage = kGStageA + kGStageB;  // 24 KB
constexpr int kGOutRow = kGN * 2 + 16;  // padded LDS row of the output tile (bytes)
constexpr int kGRing = 3;
constexpr int kGLds = kGM * kGOutRow > kGRing * kGStage ? kGM * kGOutRow : kGRing * kGStage;

struct GatedArgs {
  const bf16_t* y;
  int64_t y0, y1, y2;  // (B, nh, T, K)
  const bf16_t* w;
  int64_t w1, w2;      // (1, nh, N, K)
  const bf16_t* x;
  int64_t x0, x1, x2;  // (B, T, nh, N)
  bf16_t* o;
  int64_t o0, o1, o2;
  int T, M, N, K, nmb, nnb;
  int64_t total, per_xcd;
};

__device__ __forceinline__ f32x16 mma_bf16(bf16x8 a, bf16x8 b, f32x16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
}
__device__ __forceinline__ int g_sw(int row, int c) { return row * 64 + ((c ^ ((row >> 2) & 3)) * 16); }

template <bool kMul>
__global__ __launch_bounds__(512, 2) void k_gated_gemm(const GatedArgs a) {
  __shared__ __attribute__((aligned(1024))) uint8_t g_lds[kGLds];
  const int bid = blockIdx.x, xcd = bid & 7, kk = bid >> 3;
  if (kk >= a.per_xcd) return;
  const int64_t t = int64_t(xcd) * a.per_xcd + kk;
  if (t >= a.total) return;
  // tile -> (head, row block, column block), column blocks fastest
  const int64_t per_head = int64_t(a.nmb) * a.nnb;
  const int h = int(t / per_head);
  const int g = int(t - int64_t(h) * per_head);
  const int mbi = g / a.nnb, nbi = g - mbi * a.nnb;
  const int m0 = mbi * kGM, n0 = nbi * kGN;
  const int tid = threadIdx.x, lane = tid & 63;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);

  // LDS DMA: instruction u of wave w fills bytes [(8u + w) KB, +1 KB) of a
  // stage: u = 0, 1 the A rows 16 (8u + w) + lane / 4, u = 2 the B rows
  // 16 w + lane / 4; the lane's 16-byte slot lane & 3 of the row holds chunk
  // (lane & 3) ^ ((row >> 2) & 3)
  const int dc = (lane & 3) ^ ((lane >> 4) & 3);
  uint32_t aoffd[2];
#pragma unroll
  for (int u = 0; u < 2; ++u) {
    const int m = min(m0 + 16 * (8 * u + w) + (lane >> 2), a.M - 1);
    const int b = m / a.T, tt = m - b * a.T;
    aoffd[u] = uint32_t((b * a.y0 + tt * a.y2 + dc * 8) * 2);
  }
  const uint32_t boffd = uint32_t((int64_t(min(n0 + 16 * w + (lane >> 2), a.N - 1)) * a.w2 + dc * 8) * 2);
  const void* ybase = sgpr_ptr(a.y + h * a.y1);
  const void* wbase = sgpr_ptr(a.w + h * a.w1);
  const uint32_t lds0 = __builtin_amdgcn_readfirstlane((uint32_t)(uintptr_t)(lds_u8*)g_lds);
  auto issue = [&](int s) __attribute__((always_inline)) {
    const uint32_t m0b = lds0 + uint32_t((s % kGRing) * kGStage) + uint32_t(w) * 1024u;
    const uint32_t kb = uint32_t(s * kGK * 2);
    dma16<0>(m0b, ybase, aoffd[0] + kb);
    dma16<8192>(m0b, ybase, aoffd[1] + kb);
    dma16<kGStageA>(m0b, wbase, boffd + kb);
  };

  // fragments: wave (wm, wn) owns rows 64 wm.., columns 64 wn..; lane row / column fr, k half fh
  const int wm = w >> 1, wn = w & 1, fr = lane & 31, fh = lane >> 5;
  int fa[2][2], fb[2][2];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      fa[i][j] = g_sw(64 * wm + 32 * i + fr, 2 * j + fh);
      fb[i][j] = kGStageA + g_sw(64 * wn + 32 * i + fr, 2 * j + fh);
    }
  f32x16 acc[2][2];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int c = 0; c < 2; ++c)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][c][r] = 0.f;

  const int nst = a.K / kGK;
  issue(0);
  if (nst > 1) {
    issue(1);
    sy_wait<3>();
  } else {
    sy_wait<0>();
  }
  __syncthreads();
  constexpr int kEp = (kGM * kGN / 8) / 512;
  const int cc = tid & 15, n = n0 + cc * 8;
  uint4 xr[kEp];
  auto load_x = [&](int e) __attribute__((always_inline)) {
    const int m = min(m0 + (tid >> 4) + 32 * e, a.M - 1);
    const int b = m / a.T, tt = m - b * a.T;
    xr[e] = *reinterpret_cast<const uint4*>(a.x + b * a.x0 + tt * a.x1 + h * a.x2 + min(n, a.N - 8));
  };
  for (int s = 0; s < nst; ++s) {
    // stage s + 2 goes to the slot of stage s - 1, which every wave finished
    // before the barrier that ended stage s - 1
    if (s + 2 < nst) issue(s + 2);
    // the epilogue's x chunks go out with the last stage, so their latency
    // runs under its MFMAs
    if constexpr (kMul) {
      if (s == nst - 1) {
#pragma unroll
        for (int e = 0; e < kEp; ++e) load_x(e);
      }
    }
    const uint8_t* base = g_lds + (s % kGRing) * kGStage;
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      bf16x8 va[2], vb[2];
#pragma unroll
      for (int i = 0; i < 2; ++i) {
        va[i] = *reinterpret_cast<const bf16x8*>(base + fa[i][j]);
        vb[i] = *reinterpret_cast<const bf16x8*>(base + fb[i][j]);
      }
#pragma unroll
      for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int c = 0; c < 2; ++c) acc[i][c] = mma_bf16(va[i], vb[c], acc[i][c]);
    }
    if (s + 1 < nst) {
      if (s + 2 < nst)
        sy_wait<3>();  // stage s + 1 landed (only s + 2 outstanding)
      else
        sy_wait<0>();
      __syncthreads();
    }
  }
  __syncthreads();  // every wave's last fragment reads done before the output tile reuses the LDS

  // epilogue: relu(acc) goes as bf16 into the LDS output tile, then the gated
  // product with the x chunks loaded during the last stage (from clamped
  // addresses).  Thread tid takes 16-byte chunk tid & 15 of rows
  // (tid >> 4) + 32 e.
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int c = 0; c < 2; ++c)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int row = 64 * wm + 32 * i + 8 * (r >> 2) + 4 * fh + (r & 3);
        const int col = 64 * wn + 32 * c + fr;
        *reinterpret_cast<bf16_t*>(g_lds + row * kGOutRow + col * 2) = f2bf(relu_f(acc[i][c][r]));
      }
  __syncthreads();
  if constexpr (!kMul) {
#pragma unroll
    for (int e = 0; e < kEp; ++e) {
      const int row = (tid >> 4) + 32 * e;
      const int m = m0 + row;
      const uint4 v = *reinterpret_cast<const uint4*>(g_lds + row * kGOutRow + cc * 16);
      if (m < a.M && n < a.N) {
        const int b = m / a.T, tt = m - b * a.T;
        *reinterpret_cast<uint4*>(a.o + b * a.o0 + tt * a.o1 + h * a.o2 + n) = v;
      }
    }
    return;
  }
#pragma unroll
  for (int e = 0; e < kEp; ++e) {
    const int row = (tid >> 4) + 32 * e;
    const int m = m0 + row;
    float fy[8], fo[8];
    load8(reinterpret_cast<const bf16_t*>(g_lds + row * kGOutRow + cc * 16), fy);
    const uint32_t xw[4] = {xr[e].x, xr[e].y, xr[e].z, xr[e].w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      fo[2 * i] = __uint_as_float(xw[i] << 16) * fy[2 * i];
      fo[2 * i + 1] = __uint_as_float(xw[i] & 0xffff0000u) * fy[2 * i + 1];
    }
    if (m < a.M && n < a.N) {
      const int b = m / a.T, tt = m - b * a.T;
      store8(a.o + b * a.o0 + tt * a.o1 + h * a.o2 + n, fo);
    }
  }
}

// ---------------------------------------------------------------------------
// Few-row GEMM with split K: out (M, D) = a (M, K) @ b (K, D), bf16 operands,
// fp32 accumulation, for the decoder product of a decode step (M = batch,
// K = nh*N = 32768, D = 256), where a library GEMM runs a handful of tiles
// down the whole K.  Each workgroup takes one 128 x 128 output tile over one
// K range (the 128-tile MFMA engine), writing fp32 partials [split][M][D];
// k_small_gemm_reduce sums the splits and casts to out's dtype.
struct SmallGemmArgs {
  const bf16_t* a;
  int64_t as;  // row stride of a
  const bf16_t* b;
  int64_t bs;  // row stride of b
  float* part;
  int M, K, D, kc;
  bool avec, bvec;
};

__global__ __launch_bounds__(kNT) void k_small_gemm(SmallGemmArgs a) {
  __shared__ Smem<true> sm;
  const int n0 = blockIdx.x * kTile, split = blockIdx.y, m0 = blockIdx.z * kTile;
  KRows<bf16_t, true, false, 0> la;
  la.base = a.a;
  la.rs = a.as;
  la.r0 = m0;
  la.nrows = a.M;
  la.K = a.K;
  la.vec = a.avec;
  NRows<bf16_t, true, false> lb;
  lb.base = a.b;
  lb.rs = a.bs;
  lb.n0 = n0;
  lb.ncols = a.D;
  lb.krows = a.K;
  lb.vec4 = a.bvec;
  f32x16 acc[2][2];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.f;
  const int kb = split * a.kc, ke = min(a.K, kb + a.kc);
  mainloop<true, false>(sm, la, lb, false, kb, ke, acc, true);
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int wm = wave >> 1, wn = wave & 1;
  float* dst = a.part + int64_t(split) * a.M * a.D;
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        int row, col;
        acc_coord<false>(wm, wn, lane, i, j, r, row, col);
        const int gm = m0 + row, gn = n0 + col;
        if (gm < a.M && gn < a.D) dst[int64_t(gm) * a.D + gn] = acc[i][j][r];
      }
}

// 256 outputs per workgroup (4 consecutive per lane, D % 4 == 0); four
// groups of 64 threads each sum every fourth split with 16-byte loads, four
// splits in flight, then combine through LDS.  Each output's sum runs in the
// order of the scalar kernel below (group g: splits g, g + 4, ...; then the
// groups in order), so both give the same bits.
template <typename TO>
__global__ __launch_bounds__(256) void k_small_gemm_reduce4(const float* part, int nsplit, int M, int D,
                                                            TO* out, int64_t os) {
  __shared__ float4 red4[4][64];
  const int l = threadIdx.x & 63, g = threadIdx.x >> 6;
  const int64_t MD = int64_t(M) * D;
  const int64_t idx = (int64_t(blockIdx.x) * 64 + l) * 4;
  float4 s = make_float4(0.f, 0.f, 0.f, 0.f);
  if (idx < MD) {
    const float* p = part + idx;
    int sp = g;
    for (; sp + 12 < nsplit; sp += 16) {
      const float4 v0 = *reinterpret_cast<const float4*>(p + int64_t(sp) * MD);
      const float4 v1 = *reinterpret_cast<const float4*>(p + int64_t(sp + 4) * MD);
      const float4 v2 = *reinterpret_cast<const float4*>(p + int64_t(sp + 8) * MD);
      const float4 v3 = *reinterpret_cast<const float4*>(p + int64_t(sp + 12) * MD);
      s.x += v0.x; s.y += v0.y; s.z += v0.z; s.w += v0.w;
      s.x += v1.x; s.y += v1.y; s.z += v1.z; s.w += v1.w;
      s.x += v2.x; s.y += v2.y; s.z += v2.z; s.w += v2.w;
      s.x += v3.x; s.y += v3.y; s.z += v3.z; s.w += v3.w;
    }
    for (; sp < nsplit; sp += 4) {
      const float4 v = *reinterpret_cast<const float4*>(p + int64_t(sp) * MD);
      s.x += v.x; s.y += v.y; s.z += v.z; s.w += v.w;
    }
  }
  red4[g][l] = s;
  __syncthreads();
  if (g == 0 && idx < MD) {
    const int64_t m = idx / D, d = idx - m * D;
    const float4 r0 = red4[0][l], r1 = red4[1][l], r2 = red4[2][l], r3 = red4[3][l];
    TO* o = out + m * os + d;
    o[0] = from_f<TO>(r0.x + r1.x + r2.x + r3.x);
    o[1] = from_f<TO>(r0.y + r1.y + r2.y + r3.y);
    o[2] = from_f<TO>(r0.z + r1.z + r2.z + r3.z);
    o[3] = from_f<TO>(r0.w + r1.w + r2.w + r3.w);
  }
}

// 64 outputs per workgroup; four groups of 64 threads each sum every fourth
// split (coalesced 256-byte rows), then combine through LDS.
template <typename TO>
__global__ __launch_bounds__(256) void k_small_gemm_reduce(const float* part, int nsplit, int M, int D,
                                                           TO* out, int64_t os) {
  __shared__ float red[4][64];
  const int l = threadIdx.x & 63, g = threadIdx.x >> 6;
  const int64_t MD = int64_t(M) * D;
  const int64_t idx = int64_t(blockIdx.x) * 64 + l;
  float s = 0.f;
  if (idx < MD)
    for (int sp = g; sp < nsplit; sp += 4) s += part[int64_t(sp) * MD + idx];
  red[g][l] = s;
  __syncthreads();
  if (g == 0 && idx < MD) {
    const int64_t m = idx / D, d = idx - m * D;
    out[m * os + d] = from_f<TO>(red[0][l] + red[1][l] + red[2][l] + red[3][l]);
  }
}

// ---------------------------------------------------------------------------
// LayerNorm over the last dim of rows (no affine, eps 1e-5, fp32 arithmetic),
// the model's _ln and _residual_ln (reference bdh.py:565-574, 731-750):
//   out = LN(y)              (x absent)
//   out = LN(x + LN(y))      (the layer's residual update)
// One wave per row, elements lane + 64 e (e < E, D = 64 E): coalesced, and
// the row stays in registers, so the mean and then the variance about it
// take two passes over registers and one over memory.  Rows are the first
// three dims of 4-D strided views.
struct LnArgs {
  View x, y, o;
  View o2 = {nullptr, 0, 0, 0};  // optional second output, bf16 (the same values rounded once)
  int64_t d1, d2, rows;
  int D;
};

template <int E>
__device__ __forceinline__ void ln_row(float (&v)[E], int D) {
  float s = 0.f;
#pragma unroll
  for (int e = 0; e < E; ++e) s += v[e];
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) s += __shfl_xor(s, off, 64);
  const float mean = s / float(D);
  float q = 0.f;
#pragma unroll
  for (int e = 0; e < E; ++e) {
    v[e] -= mean;
    q += v[e] * v[e];
  }
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) q += __shfl_xor(q, off, 64);
  const float r = rsqrtf(q / float(D) + 1e-5f);
#pragma unroll
  for (int e = 0; e < E; ++e) v[e] *= r;
}

template <typename TX, typename TY, typename TO, int E>
__global__ __launch_bounds__(256) void k_ln_rows(const LnArgs a) {
  const int64_t row = int64_t(blockIdx.x) * 4 + (threadIdx.x >> 6);
  if (row >= a.rows) return;
  const int lane = threadIdx.x & 63;
  const int64_t i2 = row % a.d2, t = row / a.d2, i1 = t % a.d1, i0 = t / a.d1;
  const TY* y = static_cast<const TY*>(a.y.p) + i0 * a.y.s0 + i1 * a.y.s1 + i2 * a.y.s2;
  float v[E];
#pragma unroll
  for (int e = 0; e < E; ++e) v[e] = to_f(y[lane + 64 * e]);
  ln_row<E>(v, a.D);
  if (a.x.p != nullptr) {
    const TX* x = static_cast<const TX*>(a.x.p) + i0 * a.x.s0 + i1 * a.x.s1 + i2 * a.x.s2;
#pragma unroll
    for (int e = 0; e < E; ++e) v[e] += to_f(x[lane + 64 * e]);
    ln_row<E>(v, a.D);
  }
  TO* o = static_cast<TO*>(const_cast<void*>(a.o.p)) + i0 * a.o.s0 + i1 * a.o.s1 + i2 * a.o.s2;
#pragma unroll
  for (int e = 0; e < E; ++e) o[lane + 64 * e] = from_f<TO>(v[e]);
  if (a.o2.p != nullptr) {
    bf16_t* o2 = static_cast<bf16_t*>(const_cast<void*>(a.o2.p)) + i0 * a.o2.s0 + i1 * a.o2.s1 + i2 * a.o2.s2;
#pragma unroll
    for (int e = 0; e < E; ++e) o2[lane + 64 * e] = f2bf(v[e]);
  }
}

struct SmallGemmPlan {
  int nsplit, kc;
  size_t ws_bytes;
};

inline SmallGemmPlan small_gemm_plan(int64_t M, int64_t K, int64_t D) {
  SmallGemmPlan p;
  const int64_t tiles = ((M + kTile - 1) / kTile) * ((D + kTile - 1) / kTile);
  const int64_t BK = Mode<true>::BK;
  int64_t S = tiles > 0 ? (256 + tiles - 1) / tiles : 1;
  S = std::max<int64_t>(1, std::min<int64_t>(S, (K + BK - 1) / BK));
  int64_t kc = (K + S - 1) / S;
  kc = std::max<int64_t>(BK, (kc + BK - 1) / BK * BK);
  p.kc = int(kc);
  p.nsplit = int((K + kc - 1) / kc);
  p.ws_bytes = size_t(p.nsplit) * size_t(M) * size_t(D) * sizeof(float);
  return p;
}

namespace {

template <typename TX, typename TY>
int launch_relu_mul(const ReluMulArgs& a, int32_t odt, dim3 grid, hipStream_t s) {
  if (odt == BDH_BF16)
    BDH_LAUNCH("k_relu_mul", (k_relu_mul<TX, TY, bf16_t>), grid, dim3(256), 0, s, a);
  else
    BDH_LAUNCH("k_relu_mul", (k_relu_mul<TX, TY, float>), grid, dim3(256), 0, s, a);
  return BDH_OK;
}

template <typename TX, typename TY, typename TO>
int launch_ln_rows(const LnArgs& a, dim3 grid, hipStream_t s) {
  switch (a.D / 64) {
    case 1: BDH_LAUNCH("k_ln_rows", (k_ln_rows<TX, TY, TO, 1>), grid, dim3(256), 0, s, a); break;
    case 2: BDH_LAUNCH("k_ln_rows", (k_ln_rows<TX, TY, TO, 2>), grid, dim3(256), 0, s, a); break;
    case 4: BDH_LAUNCH("k_ln_rows", (k_ln_rows<TX, TY, TO, 4>), grid, dim3(256), 0, s, a); break;
    case 8: BDH_LAUNCH("k_ln_rows", (k_ln_rows<TX, TY, TO, 8>), grid, dim3(256), 0, s, a); break;
    case 16: BDH_LAUNCH("k_ln_rows", (k_ln_rows<TX, TY, TO, 16>), grid, dim3(256), 0, s, a); break;
    default: return BDH_ERR_SHAPE;
  }
  return BDH_OK;
}

template <typename TX, typename TY>
int launch_ln_rows_o(const LnArgs& a, int32_t odt, dim3 grid, hipStream_t s) {
  return odt == BDH_BF16 ? launch_ln_rows<TX, TY, bf16_t>(a, grid, s) : launch_ln_rows<TX, TY, float>(a, grid, s);
}

}  // namespace
}  // namespace bdh

using namespace bdh;

namespace {
int layer_norm_rows(const bdh_tensor4* x, const bdh_tensor4* y, const bdh_tensor4* out, const bdh_tensor4* out2,
                    bdh_stream stream) {
  BDH_TRY(check_view(y));
  BDH_TRY(check_view(out));
  if (x != nullptr) BDH_TRY(check_view(x));
  for (int i = 0; i < 4; ++i)
    if (out->size[i] != y->size[i] || (x != nullptr && x->size[i] != y->size[i])) return BDH_ERR_SHAPE;
  if (views_overlap(out, y) || (x != nullptr && views_overlap(out, x))) return BDH_ERR_ALIAS;
  if (out2 != nullptr) {
    BDH_TRY(check_view(out2));
    if (out2->dtype != BDH_BF16) return BDH_ERR_DTYPE;
    for (int i = 0; i < 4; ++i)
      if (out2->size[i] != y->size[i]) return BDH_ERR_SHAPE;
    if (views_overlap(out2, y) || views_overlap(out2, out) || (x != nullptr && views_overlap(out2, x)))
      return BDH_ERR_ALIAS;
  }
  if (numel4(out) == 0) return BDH_OK;
  const int64_t D = y->size[3];
  if (D % 64 != 0 || D > 1024 || ((D / 64) & (D / 64 - 1)) != 0) return BDH_ERR_SHAPE;
  const int64_t rows = y->size[0] * y->size[1] * y->size[2];
  if ((rows + 3) / 4 >= (int64_t(1) << 31)) return BDH_ERR_SHAPE;
  auto view = [](const bdh_tensor4* t) {
    View v;
    v.p = t->data;
    v.s0 = t->stride[0];
    v.s1 = t->stride[1];
    v.s2 = t->stride[2];
    return v;
  };
  LnArgs a;
  a.x = x != nullptr ? view(x) : View{nullptr, 0, 0, 0};
  a.y = view(y);
  a.o = view(out);
  if (out2 != nullptr) a.o2 = view(out2);
  a.d1 = y->size[1];
  a.d2 = y->size[2];
  a.rows = rows;
  a.D = int(D);
  const dim3 grid{unsigned((rows + 3) / 4)};
  hipStream_t s = static_cast<hipStream_t>(stream);
  const bool xb = x != nullptr && x->dtype == BDH_BF16, yb = y->dtype == BDH_BF16;
  if (xb)
    return yb ? launch_ln_rows_o<bf16_t, bf16_t>(a, out->dtype, grid, s)
              : launch_ln_rows_o<bf16_t, float>(a, out->dtype, grid, s);
  return yb ? launch_ln_rows_o<float, bf16_t>(a, out->dtype, grid, s)
            : launch_ln_rows_o<float, float>(a, out->dtype, grid, s);
}
}  // namespace

extern "C" int bdh_layer_norm_rows(const bdh_tensor4* x, const bdh_tensor4* y, const bdh_tensor4* out,
                                   bdh_stream stream) {
  return layer_norm_rows(x, y, out, nullptr, stream);
}

extern "C" int bdh_layer_norm_rows2(const bdh_tensor4* x, const bdh_tensor4* y, const bdh_tensor4* out,
                                    const bdh_tensor4* out_bf16, bdh_stream stream) {
  if (out_bf16 == nullptr) return BDH_ERR_ARG;
  return layer_norm_rows(x, y, out, out_bf16, stream);
}

extern "C" int bdh_relu_mul(const bdh_tensor4* x, const bdh_tensor4* y, const bdh_tensor4* out,
                            bdh_stream stream) {
  BDH_TRY(check_view(x));
  BDH_TRY(check_view(y));
  BDH_TRY(check_view(out));
  for (int i = 0; i < 4; ++i)
    if (y->size[i] != x->size[i] || out->size[i] != x->size[i]) return BDH_ERR_SHAPE;
  if (views_overlap(out, y) || views_overlap(out, x)) return BDH_ERR_ALIAS;
  if (numel4(out) == 0) return BDH_OK;
  const int64_t rows = x->size[0] * x->size[1] * x->size[2];
  const int64_t ncol = (x->size[3] + 2047) / 2048;
  if (rows >= (int64_t(1) << 31) || ncol > 65535) return BDH_ERR_SHAPE;
  ReluMulArgs a;
  auto full = [](const bdh_tensor4* t) {
    View v;
    v.p = t->data;
    v.s0 = t->stride[0];
    v.s1 = t->stride[1];
    v.s2 = t->stride[2];
    return v;
  };
  a.x = full(x);
  a.y = full(y);
  a.o = full(out);
  a.d1 = x->size[1];
  a.d2 = x->size[2];
  a.n = x->size[3];
  auto al = [](const bdh_tensor4* t) {
    if ((reinterpret_cast<uintptr_t>(t->data) & 15) != 0 || t->size[3] % 8 != 0) return false;
    const int per = 16 / esize(t->dtype);
    for (int i = 0; i < 3; ++i)
      if (t->size[i] > 1 && t->stride[i] % per != 0) return false;
    return true;
  };
  a.vec8 = al(x) && al(y) && al(out);
  const dim3 grid{unsigned(rows), unsigned(ncol)};
  hipStream_t s = static_cast<hipStream_t>(stream);
  const bool xb = x->dtype == BDH_BF16, yb = y->dtype == BDH_BF16;
  if (xb) return yb ? launch_relu_mul<bf16_t, bf16_t>(a, out->dtype, grid, s)
                    : launch_relu_mul<bf16_t, float>(a, out->dtype, grid, s);
  return yb ? launch_relu_mul<float, bf16_t>(a, out->dtype, grid, s)
            : launch_relu_mul<float, float>(a, out->dtype, grid, s);
}

namespace bdh {
bool relu_enc_takes(int64_t K, int64_t N);
int relu_enc_launch(const bdh_tensor4* y, const bdh_tensor4* wt, const bdh_tensor4* x, const bdh_tensor4* out,
                    hipStream_t s);
}  // namespace bdh

// out = [x *] relu(y @ wt^T) per head (x null: the ReLU GEMM alone, k_relu_enc
// where it takes the shape); see k_gated_gemm.
static int gated_gemm_launch(const bdh_tensor4* y, const bdh_tensor4* wt, const bdh_tensor4* x,
                             const bdh_tensor4* out, bdh_stream stream) {
  BDH_TRY(check_view(y));
  BDH_TRY(check_view(wt));
  if (x != nullptr) BDH_TRY(check_view(x));
  BDH_TRY(check_view(out));
  const int64_t B = out->size[0], T = out->size[1], H = out->size[2], N = out->size[3], K = y->size[3];
  if (y->dtype != BDH_BF16 || wt->dtype != BDH_BF16 || out->dtype != BDH_BF16) return BDH_ERR_DTYPE;
  if (x != nullptr && x->dtype != BDH_BF16) return BDH_ERR_DTYPE;
  if (y->size[0] != B || y->size[1] != H || y->size[2] != T) return BDH_ERR_SHAPE;
  if (wt->size[0] != 1 || wt->size[1] != H || wt->size[2] != N || wt->size[3] != K) return BDH_ERR_SHAPE;
  if (x != nullptr)
    for (int i = 0; i < 4; ++i)
      if (out->size[i] != x->size[i]) return BDH_ERR_SHAPE;
  if ((x != nullptr && views_overlap(out, x)) || views_overlap(out, y) || views_overlap(out, wt))
    return BDH_ERR_ALIAS;
  if (numel4(out) == 0) return BDH_OK;
  if (K < kGK || K % kGK != 0 || N % 8 != 0) return BDH_ERR_SHAPE;
  // 16-byte rows: aligned bases, outer strides multiples of 8 elements
  auto rows16 = [](const bdh_tensor4* t) {
    if ((reinterpret_cast<uintptr_t>(t->data) & 15) != 0) return false;
    for (int i = 0; i < 3; ++i)
      if (t->size[i] > 1 && t->stride[i] % 8 != 0) return false;
    return true;
  };
  if (!rows16(y) || !rows16(wt) || (x != nullptr && !rows16(x)) || !rows16(out)) return BDH_ERR_STRIDE;
  const int64_t M = B * T;
  if (M >= (int64_t(1) << 31) || T >= (int64_t(1) << 31)) return BDH_ERR_SHAPE;
  // the DMA takes 32-bit byte offsets from the per-head bases of y and wt
  const int64_t y_span = (B - 1) * y->stride[0] + (T - 1) * y->stride[2] + K;
  const int64_t w_span = (N - 1) * wt->stride[2] + K;
  if (y_span * 2 > (int64_t(1) << 32) || w_span * 2 > (int64_t(1) << 32)) return BDH_ERR_SHAPE;
  GatedArgs a;
  a.y = static_cast<const bf16_t*>(y->data);
  a.y0 = y->stride[0];
  a.y1 = y->stride[1];
  a.y2 = y->stride[2];
  a.w = static_cast<const bf16_t*>(wt->data);
  a.w1 = wt->stride[1];
  a.w2 = wt->stride[2];
  a.x = x != nullptr ? static_cast<const bf16_t*>(x->data) : nullptr;
  a.x0 = x != nullptr ? x->stride[0] : 0;
  a.x1 = x != nullptr ? x->stride[1] : 0;
  a.x2 = x != nullptr ? x->stride[2] : 0;
  a.o = static_cast<bf16_t*>(out->data);
  a.o0 = out->stride[0];
  a.o1 = out->stride[1];
  a.o2 = out->stride[2];
  a.T = int(T);
  a.M = int(M);
  a.N = int(N);
  a.K = int(K);
  a.nmb = int((M + kGM - 1) / kGM);
  a.nnb = int((N + kGN - 1) / kGN);
  a.total = int64_t(a.nmb) * a.nnb * H;
  a.per_xcd = (a.total + 7) / 8;
  const int64_t grid = 8 * a.per_xcd;
  if (grid >= (int64_t(1) << 31)) return BDH_ERR_SHAPE;
  // The streaming kernel runs one workgroup per (head, 256 tokens) down all N
  // columns: it needs enough token blocks to fill the chip (a decode step's
  // few tokens take the tile kernel, whose grid spans the columns too).
  if (relu_enc_takes(K, N) && (M + 255) / 256 * H >= 128 && ((N - 1) * wt->stride[2] + K) * 2 < (int64_t(1) << 32))
    return relu_enc_launch(y, wt, x, out, static_cast<hipStream_t>(stream));
  if (x != nullptr)
    BDH_LAUNCH("k_gated_gemm", k_gated_gemm<true>, dim3(unsigned(grid)), dim3(512), 0,
               static_cast<hipStream_t>(stream), a);
  else
    BDH_LAUNCH("k_relu_gemm", k_gated_gemm<false>, dim3(unsigned(grid)), dim3(512), 0,
               static_cast<hipStream_t>(stream), a);
  return BDH_OK;
}

extern "C" int bdh_gated_gemm(const bdh_tensor4* y, const bdh_tensor4* wt, const bdh_tensor4* x,
                              const bdh_tensor4* out, bdh_stream stream) {
  if (x == nullptr) return BDH_ERR_ARG;
  return gated_gemm_launch(y, wt, x, out, stream);
}

// out = relu(y @ wt^T) per head as bf16; see k_gated_gemm.
extern "C" int bdh_relu_gemm(const bdh_tensor4* y, const bdh_tensor4* wt, const bdh_tensor4* out,
                             bdh_stream stream) {
  return gated_gemm_launch(y, wt, nullptr, out, stream);
}

extern "C" size_t bdh_small_gemm_workspace(int64_t M, int64_t K, int64_t D) {
  if (M <= 0 || K <= 0 || D <= 0) return 0;
  return small_gemm_plan(M, K, D).ws_bytes;
}

// out (1, 1, M, D) = a (1, 1, M, K) @ b (1, 1, K, D); see k_small_gemm.
extern "C" int bdh_small_gemm(const bdh_tensor4* a, const bdh_tensor4* b, const bdh_tensor4* out, void* workspace,
                              size_t workspace_bytes, bdh_stream stream) {
  BDH_TRY(check_view(a));
  BDH_TRY(check_view(b));
  BDH_TRY(check_view(out));
  if (a->dtype != BDH_BF16 || b->dtype != BDH_BF16) return BDH_ERR_DTYPE;
  for (const bdh_tensor4* t : {a, b, out})
    if (t->size[0] != 1 || t->size[1] != 1) return BDH_ERR_SHAPE;
  const int64_t M = a->size[2], K = a->size[3], D = b->size[3];
  if (b->size[2] != K || out->size[2] != M || out->size[3] != D) return BDH_ERR_SHAPE;
  if (views_overlap(out, a) || views_overlap(out, b)) return BDH_ERR_ALIAS;
  if (numel4(out) == 0) return BDH_OK;
  if (M >= (int64_t(1) << 24) || K >= (int64_t(1) << 30) || D >= (int64_t(1) << 24)) return BDH_ERR_SHAPE;
  if ((M * D + 63) / 64 >= (int64_t(1) << 31)) return BDH_ERR_SHAPE;
  const SmallGemmPlan p = small_gemm_plan(M, K, D);
  if (workspace == nullptr || workspace_bytes < p.ws_bytes) return BDH_ERR_WORKSPACE;
  if ((reinterpret_cast<uintptr_t>(workspace) & 3) != 0) return BDH_ERR_WORKSPACE;  // fp32 partials
  if ((M + kTile - 1) / kTile > 65535 || p.nsplit > 65535) return BDH_ERR_SHAPE;
  SmallGemmArgs g;
  g.a = static_cast<const bf16_t*>(a->data);
  g.as = a->stride[2];
  g.b = static_cast<const bf16_t*>(b->data);
  g.bs = b->stride[2];
  g.part = static_cast<float*>(workspace);
  g.M = int(M);
  g.K = int(K);
  g.D = int(D);
  g.kc = p.kc;
  g.avec = (reinterpret_cast<uintptr_t>(a->data) & 15) == 0 && a->stride[2] % 8 == 0 && K % 8 == 0;
  g.bvec = (reinterpret_cast<uintptr_t>(b->data) & 7) == 0 && b->stride[2] % 4 == 0 && D % 4 == 0;
  hipStream_t s = static_cast<hipStream_t>(stream);
  const dim3 grid{unsigned((D + kTile - 1) / kTile), unsigned(p.nsplit), unsigned((M + kTile - 1) / kTile)};
  BDH_LAUNCH("k_small_gemm", k_small_gemm, grid, dim3(kNT), 0, s, g);
  // the 16-byte reduce needs 16-byte aligned partial rows: D % 4 == 0 and an
  // aligned workspace (a caller may pass any pointer)
  if (D % 4 == 0 && (reinterpret_cast<uintptr_t>(workspace) & 15) == 0) {
    const unsigned rg4 = unsigned((M * D / 4 + 63) / 64);
    if (out->dtype == BDH_BF16)
      BDH_LAUNCH("k_small_gemm_reduce", k_small_gemm_reduce4<bf16_t>, dim3(rg4), dim3(256), 0, s, g.part,
                 p.nsplit, int(M), int(D), static_cast<bf16_t*>(out->data), out->stride[2]);
    else
      BDH_LAUNCH("k_small_gemm_reduce", k_small_gemm_reduce4<float>, dim3(rg4), dim3(256), 0, s, g.part,
                 p.nsplit, int(M), int(D), static_cast<float*>(out->data), out->stride[2]);
    return BDH_OK;
  }
  const unsigned rg = unsigned((M * D + 63) / 64);
  if (out->dtype == BDH_BF16)
    BDH_LAUNCH("k_small_gemm_reduce", k_small_gemm_reduce<bf16_t>, dim3(rg), dim3(256), 0, s, g.part, p.nsplit,
               int(M), int(D), static_cast<bf16_t*>(out->data), out->stride[2]);
  else
    BDH_LAUNCH("k_small_gemm_reduce", k_small_gemm_reduce<float>, dim3(rg), dim3(256), 0, s, g.part, p.nsplit,
               int(M), int(D), static_cast<float*>(out->data), out->stride[2]);
  return BDH_OK;
}
