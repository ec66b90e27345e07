// Analytic backward of out = tril(Q K^T, -1) V for gfx950.
//
//   dS = tril(dO V^T, -1);   G = dS + dS^T (zero diagonal)
//   self (K is Q):   dQ = G Q            (= dS K + dS^T Q, the merged gradient)
//   distinct Q, K:   dQ = lower(G) K,  dK = upper(G) Q
//   dV = sum_h M_h^T dO_h,  M = tril(Q K^T, -1)  (heads summed when V broadcasts)
//
// Kernels:
//  1. k_scores (TRANS) recomputes M as split-K partial tiles stored transposed,
//     so rows of M^T are contiguous for the dV product.
//  2. k_bwd_g forms G tile by tile: below the diagonal dO_i V_j^T, above it
//     V_i dO_j^T (= dS^T), on diagonal tiles both, masked.
//  3. k_bwd_dq: G rows times X (X staged column-major into LDS).  With RoPE,
//     X = RoPE(x) is rotated while staging and the result is rotated back
//     (the transpose rotation) in the epilogue, giving dx directly.
//  4. k_bwd_dv: split-summed M^T rows times dO, accumulated over heads.
#include "fwd.h"

namespace bdh {

struct GArgs {
  View dO, v;
  int64_t H, Hv, T, Dv;
  bool vec_do, vec_v;
  void* g;       // [slab][tpad][tpad] in the compute dtype
  int64_t tpad;
};

template <bool BF>
__device__ __forceinline__ void zero_acc(f32x16 (&acc)[2][2]) {
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.f;
}

template <bool BF, typename TA, typename TB>
__device__ __forceinline__ void g_product(Smem<BF>& sm, const TA* a, int64_t ars, bool avec, int ar0,
                                          const TB* b, int64_t brs, bool bvec, int br0, int T, int Dv,
                                          f32x16 (&acc)[2][2]) {
  KRows<TA, BF, false, 0> la;
  la.base = a;
  la.rs = ars;
  la.r0 = ar0;
  la.nrows = T;
  la.K = Dv;
  la.vec = avec;
  KRows<TB, BF, false, 0> lb;
  lb.base = b;
  lb.rs = brs;
  lb.r0 = br0;
  lb.nrows = T;
  lb.K = Dv;
  lb.vec = bvec;
  zero_acc<BF>(acc);
  mainloop<BF, false>(sm, la, lb, false, 0, Dv, acc, true);
}

template <bool BF, typename TDO, typename TV>
__global__ __launch_bounds__(kNT) void k_bwd_g(GArgs a) {
  typedef typename Mode<BF>::lds_t TG;
  __shared__ Smem<BF> sm;
  const int ti = blockIdx.x, tj = blockIdx.y, slab = blockIdx.z;
  const int b = slab / a.H, h = slab % a.H;
  const int hv = a.Hv == 1 ? 0 : h;
  const TDO* dO = static_cast<const TDO*>(a.dO.p) + b * a.dO.s0 + h * a.dO.s1;
  const TV* v = static_cast<const TV*>(a.v.p) + b * a.v.s0 + hv * a.v.s1;
  TG* g = static_cast<TG*>(a.g) + int64_t(slab) * a.tpad * a.tpad;
  const int T = int(a.T), Dv = int(a.Dv);
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int wm = wave >> 1, wn = wave & 1;
  f32x16 acc[2][2];
  // pass 0: dO_i V_j^T (strictly below the diagonal); pass 1: V_i dO_j^T (above).
  for (int pass = 0; pass < 2; ++pass) {
    if (pass == 0 && ti < tj) continue;
    if (pass == 1 && ti > tj) continue;
    if (pass == 0)
      g_product<BF, TDO, TV>(sm, dO, a.dO.s2, a.vec_do, ti * kTile, v, a.v.s2, a.vec_v, tj * kTile, T, Dv,
                             acc);
    else
      g_product<BF, TV, TDO>(sm, v, a.v.s2, a.vec_v, ti * kTile, dO, a.dO.s2, a.vec_do, tj * kTile, T, Dv,
                             acc);
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int j = 0; j < 2; ++j)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          int row, col;
          acc_coord<false>(wm, wn, lane, i, j, r, row, col);
          const int gi = ti * kTile + row, gj = tj * kTile + col;
          // each element has exactly one writer: pass 0 owns gj <= gi, pass 1 owns gj > gi
          const bool mine = pass == 0 ? (gj <= gi) : (gj > gi);
          if (!mine) continue;
          const float val = (gj == gi) ? 0.f : acc[i][j][r];
          g[int64_t(gi) * a.tpad + gj] = from_f<TG>(val);
        }
  }
}

struct DqArgs {
  const void* g;
  int64_t tpad;
  View x;
  int64_t H, T, N;
  bool vec4_x;
  const float* freqs;
  int64_t rope_start;
  View o;
};

// MASK: 0 full G (self attention), 1 keep j < i (dQ = dS K), 2 keep j > i (dK = dS^T Q).
template <bool BF, typename TX, typename TO, int MASK, bool ROPE>
__global__ __launch_bounds__(kNT) void k_bwd_dq(DqArgs a) {
  typedef typename Mode<BF>::lds_t TG;
  __shared__ Smem<BF> sm;
  const int ti = blockIdx.x, tn = blockIdx.y, slab = blockIdx.z;
  const int b = slab / a.H, h = slab % a.H;
  const int T = int(a.T), N = int(a.N);

  KRows<TG, BF, false, MASK> la;
  la.base = static_cast<const TG*>(a.g) + int64_t(slab) * a.tpad * a.tpad;
  la.rs = a.tpad;
  la.r0 = ti * kTile;
  la.nrows = T;
  la.K = T;
  la.vec = true;
  NRows<TX, BF, ROPE> lb;
  lb.base = static_cast<const TX*>(a.x.p) + b * a.x.s0 + h * a.x.s1;
  lb.rs = a.x.s2;
  lb.n0 = tn * kTile;
  lb.ncols = N;
  lb.krows = T;
  lb.vec4 = a.vec4_x;
  lb.freqs = a.freqs;
  lb.pos0 = float(a.rope_start);

  int kb = 0, ke = T;
  if (MASK == 1) ke = min(T, (ti + 1) * kTile);
  if (MASK == 2) kb = ti * kTile;
  f32x16 acc[2][2];
  zero_acc<BF>(acc);
  mainloop<BF, false>(sm, la, lb, false, kb, ke, acc, true);

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
        const int gi = ti * kTile + row, gn = tn * kTile + col;
        float val = acc[i][j][r];
        if constexpr (ROPE) {
          // column pairs (2m, 2m+1) sit in lanes (2l, 2l+1): swap partners, rotate back.
          const float other = __shfl_xor(val, 1, 64);
          const bool even = (lane & 1) == 0;
          const int ge = gn & ~1;
          float cs = 1.f, sn = 0.f;
          if (ge < N) rope_cs(float(a.rope_start) + float(gi), a.freqs[ge], cs, sn);
          const float g0 = even ? val : other, g1 = even ? other : val;
          val = even ? (g0 * cs + g1 * sn) : (-g0 * sn + g1 * cs);
        }
        if (gi < T && gn < N) o[int64_t(gi) * a.o.s2 + gn] = from_f<TO>(val);
      }
}

struct DvArgs {
  const float* spT;
  int64_t split_stride;
  int nsplit;
  int ntl;
  View dO;
  int64_t H, Hv, T, Dv;
  bool vec4_do;
  View o;
};

template <bool BF, typename TDO, typename TO>
__global__ __launch_bounds__(kNT) void k_bwd_dv(DvArgs a) {
  __shared__ Smem<BF> sm;
  const int R = blockIdx.x, Dt = blockIdx.y, bv = blockIdx.z;
  const int b = bv / int(a.Hv), hv = bv % int(a.Hv);
  const int h_lo = a.Hv == 1 ? 0 : hv;
  const int h_hi = a.Hv == 1 ? int(a.H) : hv + 1;
  const int T = int(a.T);
  f32x16 acc[2][2];
  zero_acc<BF>(acc);
  for (int h = h_lo; h < h_hi; ++h) {
    const int slab = b * int(a.H) + h;
    SplitRows<BF, true> la;
    la.slab = a.spT + int64_t(slab) * a.ntl * kTileElems;
    la.split_stride = a.split_stride;
    la.nsplit = a.nsplit;
    la.R = R;
    NRows<TDO, BF, false> lb;
    lb.base = static_cast<const TDO*>(a.dO.p) + b * a.dO.s0 + h * a.dO.s1;
    lb.rs = a.dO.s2;
    lb.n0 = Dt * kTile;
    lb.ncols = int(a.Dv);
    lb.krows = T;
    lb.vec4 = a.vec4_do;
    mainloop<BF, false>(sm, la, lb, false, R * kTile, T, acc, true);
  }
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int wm = wave >> 1, wn = wave & 1;
  TO* o = static_cast<TO*>(const_cast<void*>(a.o.p)) + b * a.o.s0 + hv * a.o.s1;
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        int row, col;
        acc_coord<false>(wm, wn, lane, i, j, r, row, col);
        const int gj = R * kTile + row, gd = Dt * kTile + col;
        if (gj < T && gd < a.Dv) o[int64_t(gj) * a.o.s2 + gd] = from_f<TO>(acc[i][j][r]);
      }
}

// ---------------------------------------------------------------- host side
namespace {

struct BwdPlan {
  FwdPlan f;
  int64_t tpad;
  size_t g_off, ws_bytes;
  // bf16 with RoPE on the MFMA path: [table + score tiles | R(x) bf16 | G bf16]
  size_t r_sy = 0, r_qr = 0, r_g = 0, r_end = 0;
};

// saved: the score tiles come from the forward's workspace, so the first
// region is not needed.  rope (bf16): room for the MFMA route as well.
BwdPlan plan_bwd(int64_t B, int64_t H, int64_t T, int64_t K, bool bf, bool saved = false, bool rope = false) {
  BwdPlan p;
  p.f = plan_fwd(B, H, T, K, bf);
  p.tpad = p.f.nt * kTile;
  // the first region holds the generic M^T partials or the bf16 score tiles
  // of the MFMA path, whichever is larger
  p.g_off = saved ? 0 : align_up(std::max(p.f.ws_bytes, bf ? sy_bwd_workspace(B, H, T, K) : size_t(0)), 256);
  p.ws_bytes = p.g_off + size_t(B * H) * size_t(p.tpad) * size_t(p.tpad) * (bf ? 2 : 4);
  if (rope && bf) {
    p.r_sy = sy_rope_scores_workspace(B, H, T, K);
    if (p.r_sy > 0) {
      const size_t x_elems = size_t(B * H) * size_t(T) * size_t(K);
      p.r_qr = align_up(p.r_sy, 256);
      p.r_g = align_up(p.r_qr + x_elems * 2, 256);
      p.r_end = p.r_g + size_t(B * H) * size_t(p.tpad) * size_t(p.tpad) * 2;
      p.ws_bytes = std::max(p.ws_bytes, p.r_end);
    }
  }
  return p;
}

bool rows16b(const bdh_tensor4* t) {
  if ((reinterpret_cast<uintptr_t>(t->data) & 15) != 0) return false;
  for (int i = 0; i < 3; ++i)
    if (t->size[i] > 1 && (t->stride[i] * esize(t->dtype)) % 16 != 0) return false;
  return true;
}

// bf16 self attention with RoPE on the MFMA path: one absolute-position score
// kernel recomputes M's tiles and writes R(x) into the workspace; dV from the
// tiles, G from dO and V, then dx = R^T(G R(x)) from the dQ kernel, whose
// epilogue applies R^T to its fp32 sums.  kNotEligible (nothing launched)
// outside its shapes.
int rope_fast_bwd(const bdh_tensor4* x, const bdh_tensor4* v, const bdh_tensor4* dout, const bdh_tensor4* dx,
                  const bdh_tensor4* dv, const float* freqs, int64_t rope_start, void* ws, size_t ws_bytes,
                  const BwdPlan& p, hipStream_t s) {
  const int64_t B = x->size[0], H = x->size[1], T = x->size[2], N = x->size[3];
  const int64_t D = v->size[3];
  if (p.r_end == 0 || ws_bytes < p.r_end) return kNotEligible;
  if (dout->dtype != BDH_BF16 || v->dtype != BDH_BF16) return kNotEligible;
  if (D < 64 || D > 256 || D % 64 != 0 || N % 256 != 0 || T > 65535) return kNotEligible;
  if (!rows16b(dout) || !rows16b(v) || !rows16b(dx) || !rows16b(dv)) return kNotEligible;
  if (dx->dtype != BDH_BF16 && dx->dtype != BDH_F32) return kNotEligible;
  if (p.tpad % 32 != 0 || p.tpad * p.tpad * 2 >= (int64_t(1) << 31)) return kNotEligible;
  if (((T - 1) * std::max(dout->stride[2], v->stride[2]) + D) * 2 >= (int64_t(1) << 31)) return kNotEligible;
  char* w = static_cast<char*>(ws);
  bdh_tensor4 qr{};
  qr.data = w + p.r_qr;
  qr.size[0] = B;
  qr.size[1] = H;
  qr.size[2] = T;
  qr.size[3] = N;
  qr.stride[3] = 1;
  qr.stride[2] = N;
  qr.stride[1] = T * N;
  qr.stride[0] = H * T * N;
  qr.dtype = BDH_BF16;
  const void* tiles = nullptr;
  int rc = sy_rope_scores(x, v, freqs, rope_start, &qr, ws, p.r_sy, s, &tiles);
  if (rc != BDH_OK) return rc;  // kNotEligible before anything ran
  // the checks above cover the remaining steps; a step that still declines
  // is reported as an error rather than leaving partial results
  auto step = [](int r) { return r == kNotEligible ? int(BDH_ERR_SHAPE) : r; };
  if (numel4(dv) > 0) BDH_TRY(step(sy_bwd_dv(&qr, v, dout, dv, nullptr, 0, s, tiles)));
  if (numel4(dx) == 0) return BDH_OK;
  BDH_TRY(step(sy_bwd_g(dout, v, w + p.r_g, p.tpad, s)));
  return step(sy_dq(w + p.r_g, p.tpad, true, &qr, dx, s, freqs, rope_start));
}

// The fused RoPE op's backward from the score tiles its forward kept
// (relative layout when the forward rotated about the tile centres): dV from
// the kept tiles, G from dO and V, then dx = R^T(G R(x)) with the dQ kernel
// rotating x at absolute positions as it stages it, so R(x) is never
// written.  Workspace: G bf16.
size_t rope_saved_bwd_bytes(int64_t B, int64_t H, int64_t T, int64_t N, size_t* g_off, int64_t* tpad) {
  const BwdPlan p = plan_bwd(B, H, T, N, true, true, false);
  if (g_off) *g_off = 0;
  if (tpad) *tpad = p.tpad;
  return size_t(B * H) * size_t(p.tpad) * size_t(p.tpad) * 2;
}

int rope_saved_bwd(const bdh_tensor4* x, const bdh_tensor4* v, const bdh_tensor4* dout, const bdh_tensor4* dx,
                   const bdh_tensor4* dv, const float* freqs, int64_t rope_start, const void* scores,
                   size_t scores_bytes, void* ws, size_t ws_bytes, hipStream_t s) {
  const int64_t B = x->size[0], H = x->size[1], T = x->size[2], N = x->size[3];
  const int64_t D = v->size[3];
  size_t off = 0, kept = 0;
  int rel = 0;
  if (scores == nullptr || !sy_rope_keeps_scores(x, v, &off, &kept, &rel)) return BDH_ERR_ARG;
  if (scores_bytes < kept) return BDH_ERR_WORKSPACE;
  size_t g_off = 0;
  int64_t tpad = 0;
  const size_t need = rope_saved_bwd_bytes(B, H, T, N, &g_off, &tpad);
  if (ws == nullptr || ws_bytes < need) return BDH_ERR_WORKSPACE;
  // the shapes every step below takes (checked here, so no step declines
  // after another has run)
  if (dout->dtype != BDH_BF16 || v->dtype != BDH_BF16) return BDH_ERR_DTYPE;
  if (D < 64 || D > 256 || D % 64 != 0 || N % 256 != 0 || T > 65535) return BDH_ERR_SHAPE;
  if (!rows16b(dout) || !rows16b(v) || !rows16b(dx) || !rows16b(dv)) return BDH_ERR_STRIDE;
  if (dx->dtype != BDH_BF16 && dx->dtype != BDH_F32) return BDH_ERR_DTYPE;
  if (tpad % 32 != 0 || tpad * tpad * 2 >= (int64_t(1) << 31)) return BDH_ERR_SHAPE;
  if (((T - 1) * std::max(dout->stride[2], v->stride[2]) + D) * 2 >= (int64_t(1) << 31)) return BDH_ERR_SHAPE;
  char* w = static_cast<char*>(ws);
  auto step = [](int r) { return r == kNotEligible ? int(BDH_ERR_SHAPE) : r; };
  const void* tiles = static_cast<const char*>(scores) + off;
  if (numel4(dv) > 0) BDH_TRY(step(sy_bwd_dv(x, v, dout, dv, nullptr, 0, s, tiles, rel)));
  if (numel4(dx) == 0) return BDH_OK;
  BDH_TRY(step(sy_bwd_g(dout, v, w + g_off, tpad, s)));
  return step(sy_dq(w + g_off, tpad, true, x, dx, s, freqs, rope_start, true));
}

bool vec4_rows(const bdh_tensor4* t) {
  const int64_t es = esize(t->dtype);
  if ((reinterpret_cast<uintptr_t>(t->data) % (4 * es)) != 0) return false;
  for (int i = 0; i < 3; ++i)
    if (t->size[i] > 1 && t->stride[i] % 4 != 0) return false;
  return t->size[3] % 4 == 0;
}

template <bool BF, typename TDO, typename TV>
int launch_g(const GArgs& a, int64_t nt, int64_t BH, hipStream_t s) {
  dim3 grid((unsigned)(nt), unsigned(nt), unsigned(BH));
  BDH_LAUNCH("k_bwd_g", (k_bwd_g<BF, TDO, TV>), grid, dim3(kNT), 0, s, a);
  return BDH_OK;
}

template <bool BF>
int run_g(const GArgs& a, int64_t nt, int64_t BH, int32_t do_dt, int32_t v_dt, hipStream_t s) {
  const bool db = do_dt == BDH_BF16, vb = v_dt == BDH_BF16;
  if (db) return vb ? launch_g<BF, bf16_t, bf16_t>(a, nt, BH, s) : launch_g<BF, bf16_t, float>(a, nt, BH, s);
  return vb ? launch_g<BF, float, bf16_t>(a, nt, BH, s) : launch_g<BF, float, float>(a, nt, BH, s);
}

template <bool BF, typename TX, typename TO, int MASK, bool ROPE>
int launch_dq(const DqArgs& a, int64_t nt, int64_t BH, hipStream_t s) {
  dim3 grid((unsigned)(nt), unsigned((a.N + kTile - 1) / kTile), unsigned(BH));
  BDH_LAUNCH("k_bwd_dq", (k_bwd_dq<BF, TX, TO, MASK, ROPE>), grid, dim3(kNT), 0, s, a);
  return BDH_OK;
}

// X has the compute dtype (it is q or k); only the output dtype varies.
template <bool BF, int MASK, bool ROPE>
int run_dq(const DqArgs& a, int64_t nt, int64_t BH, int32_t o_dt, hipStream_t s) {
  typedef typename std::conditional<BF, bf16_t, float>::type TX;
  return o_dt == BDH_BF16 ? launch_dq<BF, TX, bf16_t, MASK, ROPE>(a, nt, BH, s)
                          : launch_dq<BF, TX, float, MASK, ROPE>(a, nt, BH, s);
}

template <bool BF, typename TDO, typename TO>
int launch_dv(const DvArgs& a, int64_t nt, int64_t BHv, hipStream_t s) {
  dim3 grid((unsigned)(nt), unsigned((a.Dv + kTile - 1) / kTile), unsigned(BHv));
  BDH_LAUNCH("k_bwd_dv", (k_bwd_dv<BF, TDO, TO>), grid, dim3(kNT), 0, s, a);
  return BDH_OK;
}

template <bool BF>
int run_dv(const DvArgs& a, int64_t nt, int64_t BHv, int32_t do_dt, int32_t o_dt, hipStream_t s) {
  const bool db = do_dt == BDH_BF16, ob = o_dt == BDH_BF16;
  if (db) return ob ? launch_dv<BF, bf16_t, bf16_t>(a, nt, BHv, s) : launch_dv<BF, bf16_t, float>(a, nt, BHv, s);
  return ob ? launch_dv<BF, float, bf16_t>(a, nt, BHv, s) : launch_dv<BF, float, float>(a, nt, BHv, s);
}

bool same4(const bdh_tensor4* a, const bdh_tensor4* b) {
  for (int i = 0; i < 4; ++i)
    if (a->size[i] != b->size[i]) return false;
  return true;
}

// Shared validation: q (B,H,T,N); k like q or NULL; v (B,1|H,T,Dv); dout (B,H,T,Dv);
// dq like q; dk like k (NULL iff k is NULL); dv like v.
int check_bwd(const bdh_tensor4* q, const bdh_tensor4* k, const bdh_tensor4* v, const bdh_tensor4* dout,
              const bdh_tensor4* dq, const bdh_tensor4* dk, const bdh_tensor4* dv) {
  BDH_TRY(check_view(q));
  BDH_TRY(check_view(v));
  BDH_TRY(check_view(dout));
  BDH_TRY(check_view(dq));
  BDH_TRY(check_view(dv));
  if ((k == nullptr) != (dk == nullptr)) return BDH_ERR_ARG;
  if (k) {
    BDH_TRY(check_view(k));
    BDH_TRY(check_view(dk));
    if (!same4(q, k) || !same4(k, dk)) return BDH_ERR_SHAPE;
    if (k->dtype != q->dtype) return BDH_ERR_DTYPE;
  }
  const int64_t B = q->size[0], H = q->size[1], T = q->size[2];
  if (v->size[0] != B || v->size[2] != T || (v->size[1] != 1 && v->size[1] != H)) return BDH_ERR_SHAPE;
  if (dout->size[0] != B || dout->size[1] != H || dout->size[2] != T || dout->size[3] != v->size[3])
    return BDH_ERR_SHAPE;
  if (!same4(dq, q) || !same4(dv, v)) return BDH_ERR_SHAPE;
  const bdh_tensor4* outs[3] = {dq, dk, dv};
  const bdh_tensor4* ins[4] = {q, k, v, dout};
  for (auto o : outs)
    for (auto i : ins)
      if (o && i && views_overlap(o, i)) return BDH_ERR_ALIAS;
  if (views_overlap(dq, dv) || (dk && (views_overlap(dk, dq) || views_overlap(dk, dv)))) return BDH_ERR_ALIAS;
  if (B * H > 65535 || T >= (int64_t(1) << 24) || q->size[3] >= (int64_t(1) << 30)) return BDH_ERR_SHAPE;
  return BDH_OK;
}

int run_bwd(const bdh_tensor4* q, const bdh_tensor4* k, const bdh_tensor4* v, const bdh_tensor4* dout,
            const bdh_tensor4* dq, const bdh_tensor4* dk, const bdh_tensor4* dv, const float* freqs,
            int64_t rope_start, void* ws, size_t ws_bytes, hipStream_t s, const void* saved = nullptr) {
  const int64_t B = q->size[0], H = q->size[1], T = q->size[2], N = q->size[3];
  const int64_t Hv = v->size[1], Dv = v->size[3];
  const bool bf = q->dtype == BDH_BF16;
  const bool self = (k == nullptr);
  const bool rope = freqs != nullptr;
  if (numel4(dq) == 0 && numel4(dv) == 0) return BDH_OK;
  if (saved != nullptr && !(self && bf && !rope)) return BDH_ERR_ARG;
  const BwdPlan p = plan_bwd(B, H, T, N, bf, saved != nullptr, rope && self);
  if (ws == nullptr || ws_bytes < p.ws_bytes) return BDH_ERR_WORKSPACE;
  const int64_t BH = B * H;

  if (self && bf && rope) {
    const int rc = rope_fast_bwd(q, v, dout, dq, dv, freqs, rope_start, ws, ws_bytes, p, s);
    if (rc != kNotEligible) return rc;
  }

  // bf16 self attention without RoPE: score tiles by the forward score kernel
  // (or saved by the forward) and dV from them (syrk.hip), in place of steps
  // 1 and 4 below
  int fast_dv = kNotEligible;
  if (self && bf && !rope) fast_dv = sy_bwd_dv(q, v, dout, dv, ws, p.g_off, s, saved);
  if (saved != nullptr && fast_dv == kNotEligible) return BDH_ERR_ARG;  // the saved tiles are unusable here
  if (fast_dv != kNotEligible && fast_dv != BDH_OK) return fast_dv;

  // 1. M^T partial tiles.
  ScoresArgs sa;
  sa.q = view_of(q);
  sa.q.s1 = q->stride[1];
  sa.k = self ? sa.q : view_of(k);
  if (!self) sa.k.s1 = k->stride[1];
  sa.H = H;
  sa.T = T;
  sa.K = N;
  sa.q_is_k = self ? 1 : 0;
  sa.vec_q = vec16_ok(q);
  sa.vec_k = self ? sa.vec_q : vec16_ok(k);
  sa.freqs = freqs;
  sa.rope_start = rope_start;
  sa.sp = static_cast<float*>(ws);
  sa.kc = p.f.kc;
  sa.ntl = int(p.f.ntl);
  sa.qr.p = nullptr;
  sa.qr_bf = false;
  if (fast_dv == kNotEligible) BDH_TRY(run_scores(sa, p.f, BH, bf, rope, true, s));

  // 2. G = dS + dS^T.
  GArgs ga;
  ga.dO = view_of(dout);
  ga.dO.s1 = dout->stride[1];
  ga.v = view_of(v);
  ga.H = H;
  ga.Hv = Hv;
  ga.T = T;
  ga.Dv = Dv;
  ga.vec_do = vec16_ok(dout);
  ga.vec_v = vec16_ok(v);
  ga.g = static_cast<char*>(ws) + p.g_off;
  ga.tpad = p.tpad;
  // bf16 G from bf16 dO and V: the MFMA score kernel with the G epilogue
  // (syrk.hip); otherwise the generic tile kernel
  const int gfast = bf ? sy_bwd_g(dout, v, ga.g, p.tpad, s) : kNotEligible;
  if (gfast != kNotEligible)
    BDH_TRY(gfast);
  else
    BDH_TRY(bf ? run_g<true>(ga, p.f.nt, BH, dout->dtype, v->dtype, s)
               : run_g<false>(ga, p.f.nt, BH, dout->dtype, v->dtype, s));

  // 3. dQ (merged for self attention), dK.
  DqArgs da;
  da.g = ga.g;
  da.tpad = p.tpad;
  da.H = H;
  da.T = T;
  da.N = N;
  da.freqs = freqs;
  da.rope_start = rope_start;
  if (numel4(dq) > 0) {
    // bf16 self attention without RoPE: the MFMA kernel with transposing LDS
    // reads (syrk.hip); otherwise the generic tile kernel below
    int fast = kNotEligible;
    if (self && bf && !rope) fast = sy_dq(ga.g, p.tpad, gfast != kNotEligible, q, dq, s);
    if (fast != kNotEligible) {
      BDH_TRY(fast);
    } else if (self) {
      da.x = view_of(q);
      da.x.s1 = q->stride[1];
      da.vec4_x = vec4_rows(q);
      da.o = view_of(dq);
      da.o.s1 = dq->stride[1];
      if (rope)
        BDH_TRY(bf ? run_dq<true, 0, true>(da, p.f.nt, BH, dq->dtype, s)
                   : run_dq<false, 0, true>(da, p.f.nt, BH, dq->dtype, s));
      else
        BDH_TRY(bf ? run_dq<true, 0, false>(da, p.f.nt, BH, dq->dtype, s)
                   : run_dq<false, 0, false>(da, p.f.nt, BH, dq->dtype, s));
    } else {
      da.x = view_of(k);
      da.x.s1 = k->stride[1];
      da.vec4_x = vec4_rows(k);
      da.o = view_of(dq);
      da.o.s1 = dq->stride[1];
      BDH_TRY(bf ? run_dq<true, 1, false>(da, p.f.nt, BH, dq->dtype, s)
                 : run_dq<false, 1, false>(da, p.f.nt, BH, dq->dtype, s));
      da.x = view_of(q);
      da.x.s1 = q->stride[1];
      da.vec4_x = vec4_rows(q);
      da.o = view_of(dk);
      da.o.s1 = dk->stride[1];
      BDH_TRY(bf ? run_dq<true, 2, false>(da, p.f.nt, BH, dk->dtype, s)
                 : run_dq<false, 2, false>(da, p.f.nt, BH, dk->dtype, s));
    }
  }

  // 4. dV.
  if (numel4(dv) > 0 && fast_dv == kNotEligible) {
    DvArgs va;
    va.spT = sa.sp;
    va.split_stride = BH * p.f.ntl * int64_t(kTileElems);
    va.nsplit = int(p.f.splits);
    va.ntl = int(p.f.ntl);
    va.dO = ga.dO;
    va.H = H;
    va.Hv = Hv;
    va.T = T;
    va.Dv = Dv;
    va.vec4_do = vec4_rows(dout);
    va.o = view_of(dv);
    va.o.s1 = dv->stride[1];
    BDH_TRY(bf ? run_dv<true>(va, p.f.nt, B * Hv, dout->dtype, dv->dtype, s)
               : run_dv<false>(va, p.f.nt, B * Hv, dout->dtype, dv->dtype, s));
  }
  return BDH_OK;
}

}  // namespace
}  // namespace bdh

using namespace bdh;

extern "C" size_t bdh_tril_score_v_bwd_workspace(int64_t B, int64_t H, int64_t Hv, int64_t T, int64_t Dk,
                                                 int64_t Dv, int32_t qk_dtype) {
  (void)Hv;
  (void)Dv;
  return plan_bwd(B, H, T, Dk, qk_dtype == BDH_BF16).ws_bytes;
}

extern "C" int bdh_tril_score_v_bwd(const bdh_tensor4* q, const bdh_tensor4* k, const bdh_tensor4* v,
                                    const bdh_tensor4* dout, const bdh_tensor4* dq, const bdh_tensor4* dk,
                                    const bdh_tensor4* dv, void* workspace, size_t workspace_bytes,
                                    bdh_stream stream) {
  BDH_TRY(check_bwd(q, k, v, dout, dq, dk, dv));
  return run_bwd(q, k, v, dout, dq, dk, dv, nullptr, 0, workspace, workspace_bytes,
                 static_cast<hipStream_t>(stream));
}

extern "C" int bdh_tril_score_v_keeps_scores(const bdh_tensor4* q, const bdh_tensor4* v, size_t* scores_bytes) {
  size_t nb = 0;
  const bool keep = check_view(q) == BDH_OK && check_view(v) == BDH_OK && v->size[0] == q->size[0] &&
                    v->size[2] == q->size[2] && (v->size[1] == 1 || v->size[1] == q->size[1]) &&
                    sy_keeps_scores(q, v, &nb);
  if (scores_bytes) *scores_bytes = keep ? nb : 0;
  return keep ? 1 : 0;
}

extern "C" size_t bdh_tril_score_v_bwd_saved_workspace(int64_t B, int64_t H, int64_t Hv, int64_t T, int64_t N,
                                                       int64_t Dv, int32_t x_dtype) {
  (void)Hv;
  (void)Dv;
  return plan_bwd(B, H, T, N, x_dtype == BDH_BF16, true).ws_bytes;
}

extern "C" int bdh_tril_score_v_bwd_saved(const bdh_tensor4* x, const bdh_tensor4* v, const bdh_tensor4* dout,
                                          const bdh_tensor4* dx, const bdh_tensor4* dv, const void* scores,
                                          size_t scores_bytes, void* workspace, size_t workspace_bytes,
                                          bdh_stream stream) {
  BDH_TRY(check_bwd(x, nullptr, v, dout, dx, nullptr, dv));
  size_t need = 0;
  if (scores == nullptr || !sy_keeps_scores(x, v, &need)) return BDH_ERR_ARG;
  if (scores_bytes < need) return BDH_ERR_WORKSPACE;
  return run_bwd(x, nullptr, v, dout, dx, nullptr, dv, nullptr, 0, workspace, workspace_bytes,
                 static_cast<hipStream_t>(stream), scores);
}

extern "C" size_t bdh_tril_rope_score_v_bwd_workspace(int64_t B, int64_t H, int64_t Hv, int64_t T,
                                                      int64_t N, int64_t Dv, int32_t x_dtype) {
  (void)Hv;
  (void)Dv;
  return plan_bwd(B, H, T, N, x_dtype == BDH_BF16, false, true).ws_bytes;
}

extern "C" int bdh_tril_rope_score_v_keeps_scores(const bdh_tensor4* x, const bdh_tensor4* v, size_t* scores_bytes) {
  size_t off = 0, kept = 0;
  int rel = 0;
  // the limits rope_saved_bwd applies to what the forward already knows (G's
  // padded T x T tile and V's row span), so tiles are kept only when the
  // saved backward will take them; dO is passed with contiguous rows
  int64_t tpad = 0;
  const int64_t T = x->size[2], D = v->size[3];
  rope_saved_bwd_bytes(x->size[0], x->size[1], T, x->size[3], nullptr, &tpad);
  const bool fits = tpad % 32 == 0 && tpad * tpad * 2 < (int64_t(1) << 31) &&
                    ((T - 1) * std::max(v->stride[2], D) + D) * 2 < (int64_t(1) << 31);
  const bool keep = check_view(x) == BDH_OK && check_view(v) == BDH_OK && v->size[0] == x->size[0] &&
                    v->size[2] == x->size[2] && (v->size[1] == 1 || v->size[1] == x->size[1]) &&
                    x->size[3] % 256 == 0 && v->size[3] % 64 == 0 && fits &&
                    sy_rope_keeps_scores(x, v, &off, &kept, &rel);
  if (scores_bytes) *scores_bytes = keep ? kept : 0;
  return keep ? 1 : 0;
}

extern "C" size_t bdh_tril_rope_score_v_bwd_saved_workspace(int64_t B, int64_t H, int64_t Hv, int64_t T,
                                                            int64_t N, int64_t Dv, int32_t x_dtype) {
  (void)Hv;
  (void)Dv;
  if (x_dtype != BDH_BF16) return 0;
  return rope_saved_bwd_bytes(B, H, T, N, nullptr, nullptr);
}

extern "C" int bdh_tril_rope_score_v_bwd_saved(const bdh_tensor4* x, const bdh_tensor4* v, const bdh_tensor4* dout,
                                               const float* freqs, int64_t rope_start, const bdh_tensor4* dx,
                                               const bdh_tensor4* dv, const void* scores, size_t scores_bytes,
                                               void* workspace, size_t workspace_bytes, bdh_stream stream) {
  BDH_TRY(check_bwd(x, nullptr, v, dout, dx, nullptr, dv));
  if (freqs == nullptr && x->size[3] > 0) return BDH_ERR_ARG;
  if (x->size[3] % 2 != 0) return BDH_ERR_SHAPE;
  if (rope_start < 0 || rope_start + x->size[2] > (int64_t(1) << 24)) return BDH_ERR_ARG;
  if (numel4(dx) == 0 && numel4(dv) == 0) return BDH_OK;
  return rope_saved_bwd(x, v, dout, dx, dv, freqs, rope_start, scores, scores_bytes, workspace, workspace_bytes,
                        static_cast<hipStream_t>(stream));
}

extern "C" int bdh_tril_rope_score_v_bwd(const bdh_tensor4* x, const bdh_tensor4* v, const bdh_tensor4* dout,
                                         const float* freqs, int64_t rope_start, const bdh_tensor4* dx,
                                         const bdh_tensor4* dv, void* workspace, size_t workspace_bytes,
                                         bdh_stream stream) {
  BDH_TRY(check_bwd(x, nullptr, v, dout, dx, nullptr, dv));
  if (freqs == nullptr && x->size[3] > 0) return BDH_ERR_ARG;
  if (x->size[3] % 2 != 0) return BDH_ERR_SHAPE;
  if (rope_start < 0 || rope_start + x->size[2] > (int64_t(1) << 24)) return BDH_ERR_ARG;
  return run_bwd(x, nullptr, v, dout, dx, nullptr, dv, freqs, rope_start, workspace, workspace_bytes,
                 static_cast<hipStream_t>(stream));
}
