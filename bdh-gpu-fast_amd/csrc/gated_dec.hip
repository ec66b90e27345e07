// The BDH layer's gated product chained into the decoder product, for gfx950:
//
//   y_mlp[m, d] = sum_h sum_n (x[m, h, n] * relu(sum_k y[m, h, k] wv[h, n, k])) dec[h N + n, d]
//
// (bdh_baseline.py:135-141: y_sparse = relu(yKV @ encoder_v), xy = x_sparse *
// y_sparse, yMLP = xy @ decoder), for K = D = 256 (the C2 model), bf16
// operands, fp32 accumulation.  The product xy (B*T x nh*N, 1.07 GB at C2)
// never exists: it is made in registers and consumed at once.
//
// k_gated_dec: one workgroup per (head h, block of 256 tokens), four waves,
// one per SIMD; wave w owns tokens 64 w .. 64 w + 63 of the block.
//  * The wave keeps its tokens' y rows in registers for the whole kernel, as
//    the B operand of  S1^T = Wv_chunk y^T  (32 n x 32 tokens per MFMA block).
//  * The head's N columns go in chunks of 32: per chunk the encoder_v rows
//    (32 x 256), the decoder rows (32 x 256) and the x block (256 tokens x
//    32) stream HBM/L2 -> LDS by LDS DMA into a ring of three 48 KB slots.
//  * S1^T's MFMA output leaves lane l with token l % 32 and 16 of the chunk's
//    n.  xy = x * relu(S1) is formed there (one bf16 rounding) and is at once
//    the A operand of  out += xy dec_chunk: the contraction over n runs in the
//    order those 16 values sit in (n = 16 kk + 4 (l / 32) + {0..3, 8..11} for
//    k16 step kk), and the decoder fragments are read with transposing LDS
//    loads from the same rows.  No LDS round trip for xy.
//  * The 64 x 256 fp32 output of each wave stays in accumulator registers
//    over all chunks; the heads' partials go to a workspace [h][m][D] and
//    k_head_sum adds them in head order (deterministic).
//  * Fragment addresses are a per-lane base XOR a compile-time offset (the
//    swizzles flip only bits the bases leave clear), which frees the address
//    registers for reads two steps ahead of their MFMAs, with scheduling
//    fences between the steps: C2 layer 646 -> 572 us (before, the compiler
//    read each fragment just before its MFMA and waited for it).
// Workgroups of one head run on the same XCD, so the head's weight chunks
// stream through that XCD's L2 once for its token blocks.
#include "common.h"
#include "lds_dma.h"

namespace bdh {

namespace {

constexpr int kGdK = 256, kGdD = 256;  // y features (encoder_v's K) and decoder columns
constexpr int kGdMT = 256;             // tokens per workgroup
constexpr int kGdNC = 32;              // n per chunk
constexpr int kGdWv = kGdNC * kGdK * 2, kGdDec = kGdNC * kGdD * 2, kGdX = kGdMT * kGdNC * 2;  // 16 KB each
constexpr int kGdSlot = kGdWv + kGdDec + kGdX;                                                    // 48 KB
constexpr int kGdRing = 3;

struct GatedDecArgs {
  const bf16_t* y;
  int64_t y0, y1, y2;  // (B, nh, T, K)
  const bf16_t* w;
  int64_t w1, w2;      // (1, nh, N, K)
  const bf16_t* x;
  int64_t x0, x1, x2;  // (B, T, nh, N)
  const bf16_t* dec;
  int64_t dr;          // (nh N, D): row stride
  float* part;         // [nh][M][D]
  int T, M, N, nh, ntb;
  int64_t total, per_xcd;
};

typedef __attribute__((__vector_size__(4 * sizeof(__bf16)))) __bf16 bf16x4;
typedef __attribute__((address_space(3))) bf16x4 lds_bf16x4;

__shared__ __attribute__((aligned(1024))) uint8_t gd_lds[kGdRing * kGdSlot];  // 144 KB

__device__ __forceinline__ f32x16 gd_mma(bf16x8 a, bf16x8 b, f32x16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
}
__device__ __forceinline__ bf16x4 gd_tr4(const uint8_t* p) {
  return __builtin_amdgcn_ds_read_tr16_b64_v4bf16((lds_bf16x4*)(p));
}

__global__ __launch_bounds__(256, 1) void k_gated_dec(const GatedDecArgs a) {
  const int bid = blockIdx.x, xcd = bid & 7, kk0 = bid >> 3;
  if (kk0 >= a.per_xcd) return;
  const int64_t t = int64_t(xcd) * a.per_xcd + kk0;
  if (t >= a.total) return;
  const int h = int(t / a.ntb), tb = int(t - int64_t(h) * a.ntb);
  const int m0 = tb * kGdMT;
  const int tid = threadIdx.x, lane = tid & 63;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int hl = lane >> 5, l32 = lane & 31;

  const void* wbase = sgpr_ptr(a.w + h * a.w1);
  const void* dbase = sgpr_ptr(a.dec + int64_t(h) * a.N * a.dr);
  const uint32_t lds0 = __builtin_amdgcn_readfirstlane((uint32_t)(uintptr_t)(lds_u8*)gd_lds);

  // ---- DMA roles: instruction i = 4 u + w (u = 0..11) fills LDS bytes
  // [i KB, +1 KB) of a slot: i < 16 encoder_v rows 2i, 2i+1 (512 B each, 16-byte
  // chunk c at c ^ (row & 31)); 16 <= i < 32 decoder rows 2(i-16) + {0,1}
  // (chunk c at c ^ 4 (row & 3)); i >= 32 x rows 16 (i-32) + lane / 4 (64 B,
  // chunk c at c ^ ((row / 4) & 3)).  Each lane fetches the global chunk its
  // LDS position holds.
  uint32_t goff[12];
#pragma unroll
  for (int u = 0; u < 12; ++u) {
    const int i = 4 * u + w;
    if (i < 16) {
      const int r = 2 * i + hl, c = l32 ^ (r & 31);
      goff[u] = uint32_t((int64_t(r) * a.w2 + 8 * c) * 2);
    } else if (i < 32) {
      const int r = 2 * (i - 16) + hl, c = l32 ^ (4 * (r & 3));
      goff[u] = uint32_t((int64_t(r) * a.dr + 8 * c) * 2);
    } else {
      goff[u] = 0;  // x rows: 64-bit addresses below
    }
  }
  // x chunk rows: a 64-bit base per lane (token rows may lie far apart)
  const bf16_t* xrow[4];
#pragma unroll
  for (int u = 8; u < 12; ++u) {
    const int i = 4 * u + w;
    const int r = 16 * (i - 32) + (lane >> 2), c = (lane & 3) ^ ((r >> 2) & 3);
    const int m = min(m0 + r, a.M - 1);
    const int b = m / a.T, tt = m - b * a.T;
    xrow[u - 8] = a.x + b * a.x0 + tt * a.x1 + int64_t(h) * a.x2 + 8 * c;
  }
  const uint32_t wl = lds0 + uint32_t(w) * 1024u;
  auto issue = [&](int ck, int slot) __attribute__((always_inline)) {
    const int cc = min(ck, a.N / kGdNC - 1);  // past the end: re-load the last chunk (not read)
    const uint32_t m0b = wl + uint32_t(slot * kGdSlot);
    const uint32_t kw = uint32_t(cc * kGdNC) * uint32_t(a.w2 * 2);
    const uint32_t kd = uint32_t(cc * kGdNC) * uint32_t(a.dr * 2);
    dma16<0 * 4096>(m0b, wbase, goff[0] + kw);
    dma16<1 * 4096>(m0b, wbase, goff[1] + kw);
    dma16<2 * 4096>(m0b, wbase, goff[2] + kw);
    dma16<3 * 4096>(m0b, wbase, goff[3] + kw);
    dma16<4 * 4096>(m0b, dbase, goff[4] + kd);
    dma16<5 * 4096>(m0b, dbase, goff[5] + kd);
    dma16<6 * 4096>(m0b, dbase, goff[6] + kd);
    dma16<7 * 4096>(m0b, dbase, goff[7] + kd);
    // x: per-lane 64-bit addresses, so a plain VGPR-addressed LDS DMA
#pragma unroll
    for (int u = 8; u < 12; ++u) {
      const bf16_t* src = xrow[u - 8] + cc * kGdNC;
      asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %1, off offset:0"
                   :
                   : "s"(m0b + uint32_t(u * 4096)), "v"(src)
                   : "memory", "m0");
    }
  };

  // ---- y fragments in registers: token block j (32 tokens), k16 step s
  bf16x8 yf[2][16];
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const int m = min(m0 + 64 * w + 32 * j + l32, a.M - 1);
    const int b = m / a.T, tt = m - b * a.T;
    const bf16_t* yp = a.y + b * a.y0 + h * a.y1 + tt * a.y2 + 8 * hl;
#pragma unroll
    for (int s = 0; s < 16; ++s) yf[j][s] = *reinterpret_cast<const bf16x8*>(yp + 16 * s);
  }
  // All y loads complete here, as the compiler sees it: its own waits for
  // them would otherwise sit inside the chunk loop, where a vmcnt(0) also
  // drains the operand DMA in flight.
  __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0)

  // ---- fragment addresses within a slot, as a per-lane base XOR a
  // compile-time offset (the swizzles only flip address bits the bases leave
  // clear), so no per-fragment address registers
  // encoder_v (A of S1^T): row l32, logical chunk 2 s + hl, at position
  // (2 s + hl) ^ l32 = 2 (s ^ (l32 / 2)) + (hl ^ (l32 % 2))
  const uint32_t wvb = uint32_t(l32 * 512 + 16 * (hl ^ (l32 & 1)) + 32 * (l32 >> 1));
  // decoder (B of out += xy dec): transposing reads of 4 rows, lane group g4
  // (16 lanes) lane q addresses row 16 kk + 4 (g4 / 2) + q / 4 (+ 8 for the
  // second read), columns 32 db + 16 (g4 % 2) + 4 (q % 4); the row's 16-byte
  // chunk c sits at c ^ 4 (row % 4), i.e. 64 db at 64 (db ^ (row % 4))
  const int g4 = lane >> 4, q = lane & 15;
  const int drow = 4 * (g4 >> 1) + (q >> 2);
  const uint32_t dvb = uint32_t(kGdWv + drow * 512 + 32 * (g4 & 1) + 16 * ((q & 3) >> 1) + 8 * (q & 1) +
                                64 * (drow & 3));
  // x (elementwise factor): token row 64 w + 32 j + l32, 8-byte piece p of
  // the logical 16-byte chunk p (at p ^ ((row / 4) % 4)), half hl
  const uint32_t xvb = uint32_t(kGdWv + kGdDec + (64 * w + l32) * 64 + 8 * hl + 16 * ((l32 >> 2) & 3));

  f32x16 acc[2][8];
#pragma unroll
  for (int j = 0; j < 2; ++j)
#pragma unroll
    for (int db = 0; db < 8; ++db)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[j][db][r] = 0.f;

  auto rd_w = [&](const uint8_t* sb, int s) __attribute__((always_inline)) {
    return *reinterpret_cast<const bf16x8*>(sb + (wvb ^ uint32_t(32 * s)));
  };
  auto rd_d = [&](const uint8_t* sb, int st) __attribute__((always_inline)) {
    const int k2 = st >> 3, db = st & 7;
    const uint8_t* pb = sb + (dvb ^ uint32_t(64 * db)) + k2 * 16 * 512;
    return __builtin_shufflevector(gd_tr4(pb), gd_tr4(pb + 8 * 512), 0, 1, 2, 3, 4, 5, 6, 7);
  };

  const int nck = a.N / kGdNC;
  issue(0, 0);
  issue(1, 1);
  int slot = 0;
  for (int ck = 0; ck < nck; ++ck) {
    sy_wait<12>();  // chunk ck landed (chunk ck + 1 may be in flight)
    __syncthreads();  // every wave's part of chunk ck landed; chunk ck - 1's reads done
    const int s2 = slot == 0 ? 2 : slot - 1;  // slot of chunk ck - 1 = slot of chunk ck + 2
    issue(ck + 2, s2);
    const uint8_t* sb = gd_lds + slot * kGdSlot;
    // S1^T (32 n x 32 tokens per block) over K = 256; the encoder_v fragment
    // of step s + 2 and the x pieces are read while steps s, s + 1 run
    u32x2 xv[2][4];
    bf16x8 wq[3];
    wq[0] = rd_w(sb, 0);
    wq[1] = rd_w(sb, 1);
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int p = 0; p < 4; ++p) xv[j][p] = *reinterpret_cast<const u32x2*>(sb + ((xvb + 2048 * j) ^ uint32_t(16 * p)));
    f32x16 s1[2];
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) s1[j][r] = 0.f;
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int s = 0; s < 16; ++s) {
      if (s + 2 < 16) wq[(s + 2) % 3] = rd_w(sb, s + 2);
      s1[0] = gd_mma(wq[s % 3], yf[0][s], s1[0]);
      s1[1] = gd_mma(wq[s % 3], yf[1][s], s1[1]);
      __builtin_amdgcn_sched_barrier(0);
    }
    // the first decoder fragments go out before the product's VALU work
    bf16x8 dq[3];
    dq[0] = rd_d(sb, 0);
    dq[1] = rd_d(sb, 1);
    // xy = x * relu(S1) as bf16, packed as the A fragments of the two k16 steps
    bf16x8 af[2][2];
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      uint32_t pk[8];
#pragma unroll
      for (int p = 0; p < 4; ++p) {
        const uint32_t x01 = xv[j][p].x, x23 = xv[j][p].y;
        const float e0 = __uint_as_float(x01 << 16) * fmaxf(s1[j][4 * p + 0], 0.f);
        const float e1 = __uint_as_float(x01 & 0xffff0000u) * fmaxf(s1[j][4 * p + 1], 0.f);
        const float e2 = __uint_as_float(x23 << 16) * fmaxf(s1[j][4 * p + 2], 0.f);
        const float e3 = __uint_as_float(x23 & 0xffff0000u) * fmaxf(s1[j][4 * p + 3], 0.f);
        pk[2 * p] = pack_bf2(e0, e1);
        pk[2 * p + 1] = pack_bf2(e2, e3);
      }
#pragma unroll
      for (int k2 = 0; k2 < 2; ++k2) {
        const u32x4 v{pk[4 * k2], pk[4 * k2 + 1], pk[4 * k2 + 2], pk[4 * k2 + 3]};
        af[j][k2] = __builtin_bit_cast(bf16x8, v);
      }
    }
    __builtin_amdgcn_sched_barrier(0);
    // out += xy dec_chunk, the fragment of step st + 2 read while st runs
#pragma unroll
    for (int st = 0; st < 16; ++st) {
      if (st + 2 < 16) dq[(st + 2) % 3] = rd_d(sb, st + 2);
      const int k2 = st >> 3, db = st & 7;
      acc[0][db] = gd_mma(af[0][k2], dq[st % 3], acc[0][db]);
      acc[1][db] = gd_mma(af[1][k2], dq[st % 3], acc[1][db]);
      __builtin_amdgcn_sched_barrier(0);
    }
    slot = slot == kGdRing - 1 ? 0 : slot + 1;
  }
  sy_wait<0>();  // the re-loads past the end landed before the LDS is released

  // ---- partial out of head h: rows m0 + 64 w + 32 j + 8 (r / 4) + 4 hl + r % 4
  float* const pp = a.part + (int64_t(h) * a.M) * kGdD;
#pragma unroll
  for (int j = 0; j < 2; ++j)
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int m = m0 + 64 * w + 32 * j + 8 * (r >> 2) + 4 * hl + (r & 3);
      if (m < a.M) {
#pragma unroll
        for (int db = 0; db < 8; ++db) pp[int64_t(m) * kGdD + 32 * db + l32] = acc[j][db][r];
      }
    }
}

// out[m, d] = sum over heads of part[h][m][d], heads in order; four columns a
// thread, 16-byte loads.
template <typename TO>
__global__ __launch_bounds__(256) void k_head_sum(const float* __restrict__ part, int nh, int64_t M, TO* out,
                                                  int64_t o_rs) {
  const int64_t e = (int64_t(blockIdx.x) * 256 + threadIdx.x) * 4;
  if (e >= M * kGdD) return;
  const int64_t m = e / kGdD, d = e - m * kGdD;
  f32x4 s = *reinterpret_cast<const f32x4*>(part + e);
  for (int hh = 1; hh < nh; ++hh) {
    const f32x4 v = *reinterpret_cast<const f32x4*>(part + int64_t(hh) * M * kGdD + e);
    s[0] += v[0];
    s[1] += v[1];
    s[2] += v[2];
    s[3] += v[3];
  }
  TO* op = out + m * o_rs + d;
  if constexpr (sizeof(TO) == 4) {
    *reinterpret_cast<f32x4*>(op) = s;
  } else {
    *reinterpret_cast<u32x2*>(op) = u32x2{pack_bf2(s[0], s[1]), pack_bf2(s[2], s[3])};
  }
}

}  // namespace

size_t gated_dec_workspace(int64_t nh, int64_t M) { return size_t(nh) * size_t(M) * kGdD * sizeof(float); }

}  // namespace bdh

using namespace bdh;

extern "C" size_t bdh_gated_decoder_workspace(int64_t nh, int64_t M) {
  if (nh <= 0 || M <= 0) return 0;
  return gated_dec_workspace(nh, M);
}

// y_mlp = (x * relu(y wt^T)) viewed (B, T, nh N) @ dec; see k_gated_dec.
extern "C" int bdh_gated_decoder(const bdh_tensor4* y, const bdh_tensor4* wt, const bdh_tensor4* x,
                                 const bdh_tensor4* dec, const bdh_tensor4* out, void* workspace,
                                 size_t workspace_bytes, bdh_stream stream) {
  BDH_TRY(check_view(y));
  BDH_TRY(check_view(wt));
  BDH_TRY(check_view(x));
  BDH_TRY(check_view(dec));
  BDH_TRY(check_view(out));
  const int64_t B = x->size[0], T = x->size[1], H = x->size[2], N = x->size[3], K = y->size[3];
  if (y->dtype != BDH_BF16 || wt->dtype != BDH_BF16 || x->dtype != BDH_BF16 || dec->dtype != BDH_BF16)
    return BDH_ERR_DTYPE;
  if (out->dtype != BDH_BF16 && out->dtype != BDH_F32) return BDH_ERR_DTYPE;
  if (y->size[0] != B || y->size[1] != H || y->size[2] != T) return BDH_ERR_SHAPE;
  if (wt->size[0] != 1 || wt->size[1] != H || wt->size[2] != N || wt->size[3] != K) return BDH_ERR_SHAPE;
  if (dec->size[0] != 1 || dec->size[1] != 1 || dec->size[2] != H * N) return BDH_ERR_SHAPE;
  if (out->size[0] != B || out->size[1] != T || out->size[2] != 1 || out->size[3] != dec->size[3])
    return BDH_ERR_SHAPE;
  if (K != kGdK || dec->size[3] != kGdD || N % kGdNC != 0) return BDH_ERR_SHAPE;
  if (views_overlap(out, x) || views_overlap(out, y) || views_overlap(out, wt) || views_overlap(out, dec))
    return BDH_ERR_ALIAS;
  if (numel4(out) == 0) return BDH_OK;
  auto rows16 = [](const bdh_tensor4* t) {
    if ((reinterpret_cast<uintptr_t>(t->data) & 15) != 0) return false;
    for (int i = 0; i < 3; ++i)
      if (t->size[i] > 1 && t->stride[i] % 8 != 0) return false;
    return true;
  };
  if (!rows16(y) || !rows16(wt) || !rows16(x) || !rows16(dec) || !rows16(out)) return BDH_ERR_STRIDE;
  // out rows (b, t) must be evenly spaced: row m = b T + t at m * stride1
  if (out->size[0] > 1 && out->stride[0] != out->size[1] * out->stride[1]) return BDH_ERR_STRIDE;
  if (out->size[1] == 1 && out->size[0] > 1 && out->stride[0] % 8 != 0) return BDH_ERR_STRIDE;
  const int64_t M = B * T;
  if (M >= (int64_t(1) << 31)) return BDH_ERR_SHAPE;
  // the DMA takes 32-bit byte offsets from the per-head bases of wt and dec
  if (((N - 1) * wt->stride[2] + K) * 2 >= (int64_t(1) << 32)) return BDH_ERR_SHAPE;
  if (((N - 1) * dec->stride[2] + kGdD) * 2 >= (int64_t(1) << 32)) return BDH_ERR_SHAPE;
  const size_t need = gated_dec_workspace(H, M);
  if (workspace == nullptr || workspace_bytes < need) return BDH_ERR_WORKSPACE;
  GatedDecArgs a;
  a.y = static_cast<const bf16_t*>(y->data);
  a.y0 = y->stride[0];
  a.y1 = y->stride[1];
  a.y2 = y->stride[2];
  a.w = static_cast<const bf16_t*>(wt->data);
  a.w1 = wt->stride[1];
  a.w2 = wt->stride[2];
  a.x = static_cast<const bf16_t*>(x->data);
  a.x0 = x->stride[0];
  a.x1 = x->stride[1];
  a.x2 = x->stride[2];
  a.dec = static_cast<const bf16_t*>(dec->data);
  a.dr = dec->stride[2];
  a.part = static_cast<float*>(workspace);
  a.T = int(T);
  a.M = int(M);
  a.N = int(N);
  a.nh = int(H);
  a.ntb = int((M + kGdMT - 1) / kGdMT);
  a.total = int64_t(a.ntb) * H;
  a.per_xcd = (a.total + 7) / 8;
  const int64_t grid = 8 * a.per_xcd;
  if (grid >= (int64_t(1) << 31)) return BDH_ERR_SHAPE;
  const hipStream_t s = static_cast<hipStream_t>(stream);
  BDH_LAUNCH("k_gated_dec", k_gated_dec, dim3(unsigned(grid)), dim3(256), 0, s, a);
  // out rows: (b, t) at b * stride0 + t * stride1; evenly spaced, so row m at m * stride1
  const int64_t o_rs = out->size[1] > 1 ? out->stride[1] : out->stride[0];
  const int64_t nthr = (M * kGdD / 4 + 255) / 256;
  if (out->dtype == BDH_F32)
    BDH_LAUNCH("k_head_sum", k_head_sum<float>, dim3(unsigned(nthr)), dim3(256), 0, s, a.part, int(H), M,
               static_cast<float*>(out->data), o_rs);
  else
    BDH_LAUNCH("k_head_sum", k_head_sum<bf16_t>, dim3(unsigned(nthr)), dim3(256), 0, s, a.part, int(H), M,
               static_cast<bf16_t*>(out->data), o_rs);
  return BDH_OK;
}
