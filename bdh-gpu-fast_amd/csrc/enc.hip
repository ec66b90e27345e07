// The BDH encoder with its ReLU, and the gated encoder_v product, for gfx950:
//
//   out[b, t, h, n] = max(sum_k y[b, h, t, k] * wt[h, n, k], 0)          (bf16)
//   out[b, t, h, n] = x[b, t, h, n] * max(sum_k y[b, h, t, k] wt[h, n, k], 0)
//
// (bdh.py:861-912, `_encoder_relu`: x @ encoder per head, then ReLU;
// bdh.py:914-945, `_encoder_v_relu` and the `x_bthn * y_bthn` of _mlp_merge),
// with K = 256 or 512 (the C2 and C5 models), bf16 operands, fp32
// accumulation, the GEMM's ReLU rounded to bf16 before the gate.
// The product has few K steps and a large output (B*T x nh*N: 1.07 GB at C2
// and C5), so the kernel is built around the output stream:
//
// k_relu_enc: one workgroup per (head h, block of 256 tokens), four waves,
// one per SIMD; wave w owns tokens 64 w .. 64 w + 63 of the block.
//  * The wave keeps its tokens' y rows in registers for the whole kernel, as
//    the B operand of  S^T = W_chunk y^T  (K = 256: 128 VGPRs, 512: 256).
//  * The head's N columns go in chunks (64 of them at K = 256, 32 at 512,
//    32 KB of encoder rows either way), streamed L2 -> LDS by LDS DMA into a
//    ring of three slots, two chunks ahead.  Each encoder fragment read from
//    LDS feeds two MFMAs (the wave's two 32-token blocks).
//  * The k16 steps go in groups of four; the encoder fragments of the next
//    group are read while the current group's MFMAs run (two register sets,
//    scheduling fences between the groups).
//  * relu(S) goes as bf16 into an LDS tile [token][n] (16-byte pieces
//    swizzled by token), written in shares between the next chunk's MFMA
//    groups from a second accumulator set; one chunk later the tile leaves
//    as 16-byte stores covering whole 128-byte (K = 256) or 64-byte pieces of
//    output rows.  Two tiles alternate.
//  * Gated form: each chunk's x pieces land by LDS DMA in the output tile
//    itself, and the epilogue multiplies in place.
//  * The token blocks of a head walk the chunks from evenly spread starting
//    chunks (see c0).
// Measured (one box; bit-identical outputs): the encoder at C2 (M = 16384,
// K = 256, 4 x 8192 columns) 330 us against 430 for hipBLASLt's GEMM with a
// ReLU epilogue, at C5 (M = 8192, K = 512, 8 x 8192) 585 against 668; the
// gated form 507 / 785 us against 628 / 800 for the tile kernel.  Without the
// output stores the encoder loop takes 233-248 / 440-510 us, with the MFMAs
// taken out 232 / 609 us; the MFMA work alone is 125 / 250 us at 2.1 GHz.
// The LDS (encoder fragments, tile writes and reads, the DMA) and the
// per-chunk barrier, not the matrix cores, set the pace.
// The workgroups of one head sit on the same XCD, so the head's encoder
// chunks stream through that XCD's L2 once for all its token blocks.
#include "common.h"
#include "lds_dma.h"

namespace bdh {

namespace {

constexpr int kEnMT = 256;         // tokens per workgroup
constexpr int kEnSlot = 32 * 1024;  // encoder rows per chunk (bytes)
constexpr int kEnRing = 3;

template <int K>
struct EnShape {
  static constexpr int NC = K == 256 ? 64 : 32;  // n per chunk
  static constexpr int ROWB = K * 2;             // bytes per encoder row
  static constexpr int NB = NC / 32;             // 32-row MFMA blocks per chunk
  static constexpr int KS = K / 16;              // k16 steps
  static constexpr int TROW = NC * 2;            // bytes per token row of an output tile
  static constexpr int TILE = kEnMT * TROW;      // output tile (bytes)
  static constexpr int TCH = TROW / 16;          // 16-byte pieces per tile row
  static constexpr int SPT = kEnMT * TCH / 256;  // tile pieces stored per thread
  static constexpr int LDS = kEnRing * kEnSlot + 2 * TILE;
};

struct EncArgs {
  const bf16_t* y;
  int64_t y0, y1, y2;  // (B, nh, T, K)
  const bf16_t* w;
  int64_t w1, w2;      // (1, nh, N, K)
  const bf16_t* x;
  int64_t x0, x1, x2;  // (B, T, nh, N): the gate (gated form)
  bf16_t* o;
  int64_t o0, o1, o2;  // (B, T, nh, N)
  int T, M, N, ntb;
  int64_t total, per_xcd;
};

template <typename F, int... I>
__device__ __forceinline__ void en_static_for_impl(F&& f, std::integer_sequence<int, I...>) {
  (f(std::integral_constant<int, I>()), ...);
}
template <int N, typename F>
__device__ __forceinline__ void en_static_for(F&& f) {
  en_static_for_impl(f, std::make_integer_sequence<int, N>());
}

__device__ __forceinline__ f32x16 en_mma(bf16x8 a, bf16x8 b, f32x16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
}

template <int K, bool MUL>
__global__ __launch_bounds__(256, 1) void k_relu_enc(const EncArgs a) {
  using S = EnShape<K>;
  __shared__ __attribute__((aligned(1024))) uint8_t en_lds[S::LDS];
  const int bid = blockIdx.x, xcd = bid & 7, kk0 = bid >> 3;
  if (kk0 >= a.per_xcd) return;
  const int64_t t = int64_t(xcd) * a.per_xcd + kk0;
  if (t >= a.total) return;
  const int h = int(t / a.ntb), tb = int(t - int64_t(h) * a.ntb);
  const int m0 = tb * kEnMT;
  const int tid = threadIdx.x, lane = tid & 63;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int hl = lane >> 5, l32 = lane & 31;

  const void* wbase = sgpr_ptr(a.w + h * a.w1);
  const uint32_t lds0 = __builtin_amdgcn_readfirstlane((uint32_t)(uintptr_t)(lds_u8*)en_lds);
  uint8_t* const tiles = en_lds + kEnRing * kEnSlot;

  // ---- DMA roles: instruction u (0..7) of wave w fills LDS bytes
  // [i KB, +1 KB) of a slot, i = 4 u + w: K = 256, encoder rows 2 i + l / 32
  // (512 B each); K = 512, row i (1 KB).  The lane's 16-byte position p of its
  // row holds the row's chunk p ^ (row & 31).
  uint32_t goff[8];
#pragma unroll
  for (int u = 0; u < 8; ++u) {
    const int i = 4 * u + w;
    const int r = K == 256 ? 2 * i + hl : i;
    const int p = K == 256 ? l32 : lane;
    goff[u] = uint32_t((int64_t(r) * a.w2 + 8 * (p ^ (r & 31))) * 2);
  }
  const uint32_t wl = lds0 + uint32_t(w) * 1024u;
  const int nck = a.N / S::NC;
  // The token blocks of a head start their walk over the chunks at evenly
  // spread chunks (the walk wraps around): at any moment the workgroups
  // write different column ranges of their rows, which spreads the output
  // stream over the memory channels (C2: 379 -> 330 us, C5: 700 -> 585 us
  // against all blocks starting at chunk 0).
  const int c0 = int((int64_t(tb) * nck / a.ntb) % nck);
  auto cmap = [&](int c) { c += c0; return c >= nck ? c - nck : c; };
  auto issue = [&](int ck, int slot) __attribute__((always_inline)) {
    const int cc = min(ck, nck - 1);  // past the end: re-load the last chunk (not read)
    const uint32_t m0b = wl + uint32_t(slot * kEnSlot);
    const uint32_t kw = uint32_t(cc * S::NC) * uint32_t(a.w2 * 2);
    dma16<0 * 4096>(m0b, wbase, goff[0] + kw);
    dma16<1 * 4096>(m0b, wbase, goff[1] + kw);
    dma16<2 * 4096>(m0b, wbase, goff[2] + kw);
    dma16<3 * 4096>(m0b, wbase, goff[3] + kw);
    dma16<4 * 4096>(m0b, wbase, goff[4] + kw);
    dma16<5 * 4096>(m0b, wbase, goff[5] + kw);
    dma16<6 * 4096>(m0b, wbase, goff[6] + kw);
    dma16<7 * 4096>(m0b, wbase, goff[7] + kw);
  };

  // ---- gated form: the x pieces of chunk c land by LDS DMA in output tile
  // c & 1, in the tile's own layout, and the epilogue multiplies in place.
  // Instruction u of wave w fills tile bytes [i KB, +1 KB), i = 4 u + w:
  // rows RPI i + l / TCH, the lane's position l % TCH holding piece
  // (l % TCH) ^ (row % TCH).  Those are the rows the wave's tile reads take
  // (rows tid / TCH + (256 / TCH) e), so the wave refills only rows it has
  // itself read.
  constexpr int RPI = 1024 / S::TROW, XI = S::TILE / 1024 / 4;
  const bf16_t* xrow[MUL ? XI : 1];
  if constexpr (MUL) {
#pragma unroll
    for (int u = 0; u < XI; ++u) {
      const int r = RPI * (4 * u + w) + lane / S::TCH;
      const int m = min(m0 + r, a.M - 1);
      const int b = m / a.T, tt = m - b * a.T;
      xrow[u] = a.x + b * a.x0 + tt * a.x1 + int64_t(h) * a.x2 + 8 * ((lane % S::TCH) ^ (r & (S::TCH - 1)));
    }
  }
  const uint32_t tl = lds0 + uint32_t(kEnRing * kEnSlot) + uint32_t(w) * 1024u;
  auto issue_x = [&](int ck) __attribute__((always_inline)) {
    const uint32_t m0b = tl + uint32_t((ck & 1) * S::TILE);
    const int64_t col = int64_t(cmap(ck)) * S::NC;
#pragma unroll
    for (int u = 0; u < XI; ++u) {
      const bf16_t* src = xrow[u] + col;
      asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %1, off offset:0"
                   :
                   : "s"(m0b + uint32_t(u * 4096)), "v"(src)
                   : "memory", "m0");
    }
  };

  // ---- y fragments in registers: token block j (32 tokens), k16 step s
  bf16x8 yf[2][S::KS];
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const int m = min(m0 + 64 * w + 32 * j + l32, a.M - 1);
    const int b = m / a.T, tt = m - b * a.T;
    const bf16_t* yp = a.y + b * a.y0 + h * a.y1 + tt * a.y2 + 8 * hl;
#pragma unroll
    for (int s = 0; s < S::KS; ++s) yf[j][s] = *reinterpret_cast<const bf16x8*>(yp + 16 * s);
  }
  // All y loads complete here, as the compiler sees it: its own waits for
  // them would otherwise sit inside the chunk loop, where a vmcnt(0) also
  // drains the operand DMA in flight.
  __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0)

  // encoder fragment (A of S^T): block i row 32 i + l32, logical chunk 2 s + hl
  const uint32_t wfo = uint32_t(l32 * S::ROWB);
  // tile stores: thread tid takes piece tid % TCH of rows tid / TCH + (256 / TCH) e
  constexpr int RSTEP = 256 / S::TCH;
  const int spc = tid % S::TCH;
  int64_t orow[S::SPT];
#pragma unroll
  for (int e = 0; e < S::SPT; ++e) {
    const int m = m0 + tid / S::TCH + RSTEP * e;
    const int mc = min(m, a.M - 1);
    const int b = mc / a.T, tt = mc - b * a.T;
    orow[e] = m < a.M ? b * a.o0 + tt * a.o1 + h * a.o2 + 8 * spc : -1;
  }
  auto tile_read = [&](uint4 (&tv)[S::SPT], int ck) __attribute__((always_inline)) {
    const uint8_t* tp = tiles + (ck & 1) * S::TILE;
    en_static_for<S::SPT>([&](auto ec) {
      constexpr int e = decltype(ec)::value;
      const int r = tid / S::TCH + RSTEP * e;
      tv[e] = *reinterpret_cast<const uint4*>(tp + r * S::TROW + 16 * (spc ^ (r & (S::TCH - 1))));
    });
  };
  auto tile_store = [&](const uint4 (&tv)[S::SPT], int ck) __attribute__((always_inline)) {
    en_static_for<S::SPT>([&](auto ec) {
      constexpr int e = decltype(ec)::value;
      if (orow[e] >= 0) *reinterpret_cast<uint4*>(a.o + orow[e] + int64_t(cmap(ck)) * S::NC) = tv[e];
    });
  };

  // k16 steps go in groups of G; the fragments of group g + 1 are read
  // while group g's MFMAs run (two register sets, scheduling fences between
  // the groups so the reads stay ahead of their use)
  constexpr int G = 4, NG = S::KS / G;
  typedef bf16x8 Frag[G][S::NB];
  auto read_group = [&](Frag& f, const uint8_t* sb, int g) __attribute__((always_inline)) {
    en_static_for<G>([&](auto qc) {
      constexpr int q = decltype(qc)::value;
      en_static_for<S::NB>([&](auto ic) {
        constexpr int i = decltype(ic)::value;
        const int st = g * G + q;
        f[q][i] = *reinterpret_cast<const bf16x8*>(sb + i * 32 * S::ROWB + wfo + 16 * ((2 * st + hl) ^ l32));
      });
    });
  };
  // relu(S) as bf16 into tile ck & 1: lane (l32, hl) of block (i, j) holds
  // token 64 w + 32 j + l32 and n = 32 i + 8 q + 4 hl + {0..3} for r = 4 q + {0..3};
  // those four n are 8 bytes of the token row's 16-byte piece 4 i + q.
  // Item it = (i, j, q) of NI; group g of a chunk writes items [g NI / NG, (g + 1) NI / NG).
  constexpr int NI = S::NB * 8;
  auto epi_item = [&](const f32x16 (&acc)[S::NB][2], uint8_t* tp, auto itc) __attribute__((always_inline)) {
    constexpr int it = decltype(itc)::value;
    constexpr int i = it / 8, j = (it / 4) & 1, q = it & 3;
    const int row = 64 * w + 32 * j + l32;
    uint8_t* const pp = tp + row * S::TROW + 16 * ((4 * i + q) ^ (row & (S::TCH - 1))) + 8 * hl;
    u32x2 v{pack_bf2(fmaxf(acc[i][j][4 * q], 0.f), fmaxf(acc[i][j][4 * q + 1], 0.f)),
            pack_bf2(fmaxf(acc[i][j][4 * q + 2], 0.f), fmaxf(acc[i][j][4 * q + 3], 0.f))};
    if constexpr (MUL) {
      // x * relu(S): relu(S) rounded to bf16 (the value the plain GEMM
      // stores), the product in fp32, rounded once more
      const u32x2 xv = *reinterpret_cast<const u32x2*>(pp);
      v.x = pack_bf2(__uint_as_float(xv.x << 16) * __uint_as_float(v.x << 16),
                     __uint_as_float(xv.x & 0xffff0000u) * __uint_as_float(v.x & 0xffff0000u));
      v.y = pack_bf2(__uint_as_float(xv.y << 16) * __uint_as_float(v.y << 16),
                     __uint_as_float(xv.y & 0xffff0000u) * __uint_as_float(v.y & 0xffff0000u));
    }
    *reinterpret_cast<u32x2*>(pp) = v;
  };

  // One chunk: wait for its operands, then (fenced) the tile reads of chunk
  // ck - 2, the first fragment group, that tile's stores, the DMA two chunks
  // ahead, and per group: the next group's fragment reads, the group's MFMAs
  // into acc, a share of chunk ck - 1's epilogue from prev.  The stores of
  // tile rows past M are skipped, so the wait for chunk ck counts only the
  // DMA of chunk ck + 1 after it: vmcnt(8) (older stores complete with it).
  auto chunk = [&](f32x16 (&acc)[S::NB][2], const f32x16 (&prev)[S::NB][2], int ck, int slot, bool has_prev)
      __attribute__((always_inline)) {
    sy_wait<8>();
    // every wave's part of chunk ck landed; chunk ck - 1's fragment reads,
    // chunk ck - 2's tile writes and chunk ck - 3's tile reads are done
    __syncthreads();
    const uint8_t* sb = en_lds + slot * kEnSlot;
    Frag f0, f1;
    if (ck >= 2) {
      uint4 tv[S::SPT];
      tile_read(tv, ck - 2);
      read_group(f0, sb, 0);
      tile_store(tv, ck - 2);
    } else {
      read_group(f0, sb, 0);
    }
    // after the stores: a global store behind the DMA asm would wait for it.
    // Gated form: chunk ck's x pieces into tile ck & 1, after this wave's
    // reads of its rows there (chunk ck - 2's tile, consumed by the stores)
    if constexpr (MUL) issue_x(ck);
    issue(ck + 2 < nck ? cmap(ck + 2) : nck - 1, slot == 0 ? 2 : slot - 1);  // into the slot of chunk ck - 1
    en_static_for<S::NB>([&](auto ic) {
      en_static_for<2>([&](auto jc) {
#pragma unroll
        for (int r = 0; r < 16; ++r) acc[decltype(ic)::value][decltype(jc)::value][r] = 0.f;
      });
    });
    uint8_t* tp = tiles + ((ck - 1) & 1) * S::TILE;
    __builtin_amdgcn_sched_barrier(0);
    en_static_for<NG>([&](auto gc) {
      constexpr int g = decltype(gc)::value;
      Frag& fc = (g & 1) ? f1 : f0;
      Frag& fn = (g & 1) ? f0 : f1;
      if constexpr (g + 1 < NG) read_group(fn, sb, g + 1);
      en_static_for<G>([&](auto qc) {
        constexpr int q = decltype(qc)::value;
        en_static_for<S::NB>([&](auto ic) {
          constexpr int i = decltype(ic)::value;
          acc[i][0] = en_mma(fc[q][i], yf[0][g * G + q], acc[i][0]);
          acc[i][1] = en_mma(fc[q][i], yf[1][g * G + q], acc[i][1]);
        });
      });
      if (has_prev) {
        en_static_for<NI / NG>([&](auto kc) {
          epi_item(prev, tp, std::integral_constant<int, g * (NI / NG) + decltype(kc)::value>());
        });
      }
      __builtin_amdgcn_sched_barrier(0);
    });
  };
  auto next = [](int slot) { return slot == kEnRing - 1 ? 0 : slot + 1; };

  f32x16 acc0[S::NB][2], acc1[S::NB][2];
  issue(cmap(0), 0);
  issue(nck > 1 ? cmap(1) : 0, 1);
  int slot = 0;
  chunk(acc0, acc1, 0, slot, false);
  slot = next(slot);
  int ck = 1;
  for (; ck + 1 < nck; ck += 2) {
    chunk(acc1, acc0, ck, slot, true);
    slot = next(slot);
    chunk(acc0, acc1, ck + 1, slot, true);
    slot = next(slot);
  }
  // chunk ck - 1's result is in acc0; one chunk may remain
  const bool odd = ck < nck;
  if (odd) chunk(acc1, acc0, ck, slot, true);
  sy_wait<8>();      // gated form: the x pieces of chunk nck - 1 landed
  __syncthreads();  // chunk nck - 2's tile writes are done
  if (nck >= 2) {
    uint4 tv[S::SPT];
    tile_read(tv, nck - 2);
    tile_store(tv, nck - 2);
  }
  {
    uint8_t* tp = tiles + ((nck - 1) & 1) * S::TILE;
    if (odd)
      en_static_for<NI>([&](auto kc) { epi_item(acc1, tp, kc); });
    else
      en_static_for<NI>([&](auto kc) { epi_item(acc0, tp, kc); });
  }
  __syncthreads();  // the last tile's writes are done
  {
    uint4 tv[S::SPT];
    tile_read(tv, nck - 1);
    tile_store(tv, nck - 1);
  }
  sy_wait<0>();  // the re-loads past the end landed before the LDS is released
}

}  // namespace

// relu(y wt^T) per head through k_relu_enc: K = 256 or 512, N a multiple of
// the chunk width; false when the shape is not one it takes.
bool relu_enc_takes(int64_t K, int64_t N) { return (K == 256 && N % 64 == 0) || (K == 512 && N % 32 == 0); }

int relu_enc_launch(const bdh_tensor4* y, const bdh_tensor4* wt, const bdh_tensor4* x, const bdh_tensor4* out,
                    hipStream_t s) {
  const int64_t B = out->size[0], T = out->size[1], H = out->size[2], N = out->size[3], K = y->size[3];
  EncArgs a;
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
  a.M = int(B * T);
  a.N = int(N);
  a.ntb = int((B * T + kEnMT - 1) / kEnMT);
  a.total = int64_t(a.ntb) * H;
  a.per_xcd = (a.total + 7) / 8;
  const int64_t grid = 8 * a.per_xcd;
  if (grid >= (int64_t(1) << 31)) return BDH_ERR_SHAPE;
  if (x != nullptr) {
    if (K == 256)
      BDH_LAUNCH("k_gated_enc", (k_relu_enc<256, true>), dim3(unsigned(grid)), dim3(256), 0, s, a);
    else
      BDH_LAUNCH("k_gated_enc", (k_relu_enc<512, true>), dim3(unsigned(grid)), dim3(256), 0, s, a);
  } else {
    if (K == 256)
      BDH_LAUNCH("k_relu_enc", (k_relu_enc<256, false>), dim3(unsigned(grid)), dim3(256), 0, s, a);
    else
      BDH_LAUNCH("k_relu_enc", (k_relu_enc<512, false>), dim3(unsigned(grid)), dim3(256), 0, s, a);
  }
  return BDH_OK;
}

}  // namespace bdh
