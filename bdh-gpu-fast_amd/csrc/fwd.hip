// Cold strict-tril attention forward for gfx950:
//   out[b,h,i,:] = sum_{j<i} <Q_i, K_j> V_j,   optionally Q = K = RoPE(x).
//
// Two kernels per call:
//  1. k_scores: split-K partial score tiles S = Q K^T over the packed lower
//     tiles (ti >= tj) of every (b,h) slab.  With Q = K a diagonal tile loads
//     its rows once and uses them as both operands; the strictly-upper wave of
//     a diagonal tile issues no MFMAs.  RoPE is applied while staging each
//     tile from HBM into LDS (phase frac(pos*freq), v_sin/v_cos).
//  2. k_score_v: out = tril(sum_splits S, -1) V, reading the partial tiles of
//     the lower triangle only (fully masked tiles are never touched).
#include "fwd.h"

namespace bdh {

template <typename TIn, bool ROPE, bool TRANS>
__global__ __launch_bounds__(kNT) void k_scores(ScoresArgs a) {
  constexpr bool BF = std::is_same<TIn, bf16_t>::value;
  __shared__ Smem<BF> sm;
  int ti, tj;
  lower_tile_coords(int(blockIdx.x) + a.t0, ti, tj);
  const int slab = blockIdx.y;
  const int b = slab / a.H, h = slab % a.H;
  const int split = blockIdx.z;
  const int kb = int(split * a.kc);
  const int ke = int(min(a.K, int64_t(kb) + a.kc));

  KRows<TIn, BF, ROPE, 0> la, lb;
  la.base = static_cast<const TIn*>(a.q.p) + b * a.q.s0 + h * a.q.s1;
  la.rs = a.q.s2;
  la.r0 = ti * kTile;
  la.nrows = int(a.T);
  la.rlo = int(a.past);  // query rows are global rows past ..
  la.K = int(a.K);
  la.vec = a.vec_q;
  lb.base = static_cast<const TIn*>(a.k.p) + b * a.k.s0 + h * a.k.s1;
  lb.rs = a.k.s2;
  lb.r0 = tj * kTile;
  lb.nrows = int(a.T);
  lb.K = int(a.K);
  lb.vec = a.vec_k;
  if constexpr (ROPE) {
    la.freqs = lb.freqs = a.freqs;
    la.pos0 = lb.pos0 = float(a.rope_start);
    if (ti == tj && a.qr.p != nullptr) {
      la.qr = const_cast<void*>(a.qr.p);
      la.qr = static_cast<char*>(la.qr) + (b * a.qr.s0 + h * a.qr.s1) * (a.qr_bf ? 2 : 4);
      la.qr_rs = a.qr.s2;
      la.qr_bf = a.qr_bf;
    }
  }
  const bool b_is_a = (ti == tj) && a.q_is_k && a.past == 0;
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int wm = wave >> 1, wn = wave & 1;
  // In a diagonal tile the wave at (rows 0-63, cols 64-127) sees only j > i.
  const bool active = !(ti == tj && wm == 0 && wn == 1);

  f32x16 acc[2][2];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.f;

  mainloop<BF, TRANS>(sm, la, lb, b_is_a, kb, ke, acc, active);

  if (!active) return;
  float* dst = a.sp + (int64_t(split) * gridDim.y + slab) * a.ntl * kTileElems +
               int64_t(blockIdx.x) * kTileElems;
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        int row, col;
        acc_coord<TRANS>(wm, wn, lane, i, j, r, row, col);
        // TRANS stores the tile transposed ([col][row]) so rows of S^T are contiguous.
        if constexpr (TRANS)
          dst[col * kTile + row] = acc[i][j][r];
        else
          dst[row * kTile + col] = acc[i][j][r];
      }
}

template <bool BF, typename TV, typename TO>
__global__ __launch_bounds__(kNT) void k_score_v(ScoreVArgs a) {
  __shared__ Smem<BF> sm;
  const int R = int(blockIdx.x) + a.s0, Dt = blockIdx.y, slab = blockIdx.z;
  const int b = slab / a.H, h = slab % a.H;
  const int hv = a.Hv == 1 ? 0 : h;

  SplitRows<BF, false> la;
  la.slab = a.sp + int64_t(slab) * a.ntl * kTileElems;
  la.split_stride = a.split_stride;
  la.nsplit = a.nsplit;
  la.R = R;
  la.t0 = a.t0;
  NRows<TV, BF, false> lb;
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
  mainloop<BF, false>(sm, la, lb, false, 0, ke, acc, true);

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
        if (gi >= a.past && gi < a.T && gd < a.Dv) o[int64_t(gi - a.past) * a.o.s2 + gd] = from_f<TO>(acc[i][j][r]);
      }
}

// ---------------------------------------------------------------- host side
// past > 0: only the row tiles from past / 128 on (their packed lower tiles
// are the suffix from t0 = s0 (s0 + 1) / 2); ntl counts the tiles launched.
FwdPlan plan_fwd(int64_t B, int64_t H, int64_t T, int64_t K, bool bf, int64_t past) {
  FwdPlan p;
  const int64_t BK = bf ? Mode<true>::BK : Mode<false>::BK;
  p.nt = (T + kTile - 1) / kTile;
  p.s0 = past / kTile;
  p.t0 = p.s0 * (p.s0 + 1) / 2;
  p.ntl = p.nt * (p.nt + 1) / 2 - p.t0;
  const int64_t wgs = B * H * p.ntl;
  int64_t splits = 1;
  if (wgs > 0 && wgs < kTargetWorkgroups) splits = (kTargetWorkgroups + wgs - 1) / wgs;
  const int64_t max_splits = K / 512 > 1 ? K / 512 : 1;
  if (splits > max_splits) splits = max_splits;
  int64_t kc = K > 0 ? (K + splits - 1) / splits : 0;
  kc = (kc + BK - 1) / BK * BK;
  if (kc == 0) kc = BK;
  p.kc = kc;
  p.splits = K > 0 ? (K + kc - 1) / kc : 1;
  p.ws_bytes = size_t(p.splits) * size_t(B * H) * size_t(p.ntl) * kTileElems * sizeof(float);
  return p;
}

template <typename TIn, bool ROPE, bool TRANS>
int launch_scores(const ScoresArgs& a, const FwdPlan& p, int64_t BH, hipStream_t s) {
  if (p.ntl == 0) return BDH_OK;
  dim3 grid((unsigned)(p.ntl), unsigned(BH), unsigned(p.splits));
  BDH_LAUNCH("k_scores", (k_scores<TIn, ROPE, TRANS>), grid, dim3(kNT), 0, s, a);
  return BDH_OK;
}

int run_scores(const ScoresArgs& a, const FwdPlan& p, int64_t BH, bool bf, bool rope, bool trans,
               hipStream_t s) {
  if (bf) {
    if (rope) return trans ? launch_scores<bf16_t, true, true>(a, p, BH, s)
                           : launch_scores<bf16_t, true, false>(a, p, BH, s);
    return trans ? launch_scores<bf16_t, false, true>(a, p, BH, s)
                 : launch_scores<bf16_t, false, false>(a, p, BH, s);
  }
  if (rope) return trans ? launch_scores<float, true, true>(a, p, BH, s)
                         : launch_scores<float, true, false>(a, p, BH, s);
  return trans ? launch_scores<float, false, true>(a, p, BH, s)
               : launch_scores<float, false, false>(a, p, BH, s);
}

template <bool BF, typename TV, typename TO>
int launch_score_v(const ScoreVArgs& a, int64_t nt, int64_t BH, hipStream_t s) {
  if (nt - a.s0 <= 0) return BDH_OK;
  dim3 grid((unsigned)(nt - a.s0), unsigned((a.Dv + kTile - 1) / kTile), unsigned(BH));
  BDH_LAUNCH("k_score_v", (k_score_v<BF, TV, TO>), grid, dim3(kNT), 0, s, a);
  return BDH_OK;
}

int run_score_v(const ScoreVArgs& a, int64_t nt, int64_t BH, bool bf, int32_t v_dt, int32_t o_dt,
                hipStream_t s) {
  const bool vb = v_dt == BDH_BF16, ob = o_dt == BDH_BF16;
  if (bf) {
    if (vb) return ob ? launch_score_v<true, bf16_t, bf16_t>(a, nt, BH, s)
                      : launch_score_v<true, bf16_t, float>(a, nt, BH, s);
    return ob ? launch_score_v<true, float, bf16_t>(a, nt, BH, s)
              : launch_score_v<true, float, float>(a, nt, BH, s);
  }
  if (vb) return ob ? launch_score_v<false, bf16_t, bf16_t>(a, nt, BH, s)
                    : launch_score_v<false, bf16_t, float>(a, nt, BH, s);
  return ob ? launch_score_v<false, float, bf16_t>(a, nt, BH, s)
            : launch_score_v<false, float, float>(a, nt, BH, s);
}

static bool vec4_rows(const bdh_tensor4* t) {
  const int64_t es = esize(t->dtype);
  if ((reinterpret_cast<uintptr_t>(t->data) % (4 * es)) != 0) return false;
  for (int i = 0; i < 3; ++i)
    if (t->size[i] > 1 && t->stride[i] % 4 != 0) return false;
  return t->size[3] % 4 == 0;
}

// Validate q/k/v/out of the cold op (contract of kernels/cuda_attn.py:103-111
// and csrc/tril_attn_cpu.cpp:161-167).
static int check_cold(const bdh_tensor4* q, const bdh_tensor4* k, const bdh_tensor4* v,
                      const bdh_tensor4* out) {
  BDH_TRY(check_view(q));
  BDH_TRY(check_view(k));
  BDH_TRY(check_view(v));
  BDH_TRY(check_view(out));
  for (int i = 0; i < 4; ++i)
    if (q->size[i] != k->size[i]) return BDH_ERR_SHAPE;
  if (q->dtype != k->dtype) return BDH_ERR_DTYPE;
  if (v->size[0] != q->size[0] || v->size[2] != q->size[2]) return BDH_ERR_SHAPE;
  if (v->size[1] != 1 && v->size[1] != q->size[1]) return BDH_ERR_SHAPE;
  if (out->size[0] != q->size[0] || out->size[1] != q->size[1] || out->size[2] != q->size[2] ||
      out->size[3] != v->size[3])
    return BDH_ERR_SHAPE;
  if (views_overlap(out, q) || views_overlap(out, k) || views_overlap(out, v)) return BDH_ERR_ALIAS;
  const int64_t lim = int64_t(1) << 30;
  for (int i = 0; i < 4; ++i)
    if (q->size[i] >= lim || v->size[i] >= lim) return BDH_ERR_SHAPE;
  if (q->size[0] * q->size[1] > 65535) return BDH_ERR_SHAPE;
  return BDH_OK;
}

static int run_cold(const bdh_tensor4* q, const bdh_tensor4* k, const bdh_tensor4* v,
                    const bdh_tensor4* out, const float* freqs, int64_t rope_start,
                    const bdh_tensor4* qr, void* ws, size_t ws_bytes, hipStream_t s) {
  const int64_t B = q->size[0], H = q->size[1], T = q->size[2], K = q->size[3];
  const int64_t Dv = v->size[3];
  if (numel4(out) == 0 && (qr == nullptr || numel4(qr) == 0)) return BDH_OK;
  const bool bf = q->dtype == BDH_BF16;
  if (bf && T > 0) {
    const int rc = sy_cold(q, k, v, out, freqs, rope_start, qr, ws, ws_bytes, s);
    if (rc != kNotEligible) return rc;
  }
  const FwdPlan p = plan_fwd(B, H, T, K, bf);
  if (ws == nullptr || ws_bytes < p.ws_bytes) return BDH_ERR_WORKSPACE;
  if (T == 0) return BDH_OK;

  ScoresArgs sa;
  sa.q = view_of(q);
  sa.k = view_of(k);
  sa.q.s1 = q->stride[1];
  sa.k.s1 = k->stride[1];
  sa.H = H;
  sa.T = T;
  sa.K = K;
  sa.q_is_k = (q->data == k->data && q->stride[0] == k->stride[0] && q->stride[1] == k->stride[1] &&
               q->stride[2] == k->stride[2]);
  sa.vec_q = vec16_ok(q);
  sa.vec_k = vec16_ok(k);
  sa.freqs = freqs;
  sa.rope_start = rope_start;
  sa.sp = static_cast<float*>(ws);
  sa.kc = p.kc;
  sa.ntl = int(p.ntl);
  sa.qr.p = nullptr;
  sa.qr_bf = false;
  if (qr != nullptr) {
    sa.qr = view_of(qr);
    sa.qr.s1 = qr->stride[1];
    sa.qr_bf = qr->dtype == BDH_BF16;
  }
  BDH_TRY(run_scores(sa, p, B * H, bf, freqs != nullptr, false, s));
  if (numel4(out) == 0) return BDH_OK;

  ScoreVArgs va;
  va.sp = sa.sp;
  va.split_stride = (B * H) * p.ntl * int64_t(kTileElems);
  va.nsplit = int(p.splits);
  va.ntl = int(p.ntl);
  va.v = view_of(v);
  va.H = H;
  va.Hv = v->size[1];
  va.T = T;
  va.Dv = Dv;
  va.vec4_v = vec4_rows(v);
  va.o = view_of(out);
  va.o.s1 = out->stride[1];
  return run_score_v(va, p.nt, B * H, bf, v->dtype, out->dtype, s);
}

// Queries at an offset (chunked prefill): q (B,H,T,N) are global rows
// past .. past+T-1 over k (B,H,past+T,N), v (B,1|H,past+T,Dv); out (B,H,T,Dv).
static int check_past(const bdh_tensor4* q, const bdh_tensor4* k, const bdh_tensor4* v,
                      const bdh_tensor4* out, int64_t past) {
  BDH_TRY(check_view(q));
  BDH_TRY(check_view(k));
  BDH_TRY(check_view(v));
  BDH_TRY(check_view(out));
  const int64_t B = q->size[0], H = q->size[1], T = q->size[2], N = q->size[3];
  if (past < 0) return BDH_ERR_ARG;
  if (k->size[0] != B || k->size[1] != H || k->size[2] != past + T || k->size[3] != N) return BDH_ERR_SHAPE;
  if (q->dtype != k->dtype) return BDH_ERR_DTYPE;
  if (v->size[0] != B || v->size[2] != past + T || (v->size[1] != 1 && v->size[1] != H)) return BDH_ERR_SHAPE;
  if (out->size[0] != B || out->size[1] != H || out->size[2] != T || out->size[3] != v->size[3])
    return BDH_ERR_SHAPE;
  if (views_overlap(out, q) || views_overlap(out, k) || views_overlap(out, v)) return BDH_ERR_ALIAS;
  const int64_t lim = int64_t(1) << 30;
  for (int i = 0; i < 4; ++i)
    if (k->size[i] >= lim || v->size[i] >= lim || q->size[i] >= lim) return BDH_ERR_SHAPE;
  if (B * H > 65535) return BDH_ERR_SHAPE;
  return BDH_OK;
}

static int run_past(const bdh_tensor4* q, const bdh_tensor4* k, const bdh_tensor4* v, const bdh_tensor4* out,
                    int64_t past, void* ws, size_t ws_bytes, hipStream_t s) {
  const int64_t B = q->size[0], H = q->size[1], T = q->size[2], K = q->size[3];
  const int64_t Tk = past + T;
  if (numel4(out) == 0) return BDH_OK;
  const bool bf = q->dtype == BDH_BF16;
  const FwdPlan p = plan_fwd(B, H, Tk, K, bf, past);
  if (ws == nullptr || ws_bytes < p.ws_bytes) return BDH_ERR_WORKSPACE;

  ScoresArgs sa;
  sa.q = view_of(q);
  sa.k = view_of(k);
  sa.q.s1 = q->stride[1];
  sa.k.s1 = k->stride[1];
  sa.H = H;
  sa.T = Tk;
  sa.K = K;
  sa.q_is_k = 0;
  sa.vec_q = vec16_ok(q);
  sa.vec_k = vec16_ok(k);
  sa.freqs = nullptr;
  sa.rope_start = 0;
  sa.sp = static_cast<float*>(ws);
  sa.kc = p.kc;
  sa.ntl = int(p.ntl);
  sa.qr.p = nullptr;
  sa.qr_bf = false;
  sa.past = past;
  sa.t0 = int(p.t0);
  BDH_TRY(run_scores(sa, p, B * H, bf, false, false, s));

  ScoreVArgs va;
  va.sp = sa.sp;
  va.split_stride = (B * H) * p.ntl * int64_t(kTileElems);
  va.nsplit = int(p.splits);
  va.ntl = int(p.ntl);
  va.v = view_of(v);
  va.H = H;
  va.Hv = v->size[1];
  va.T = Tk;
  va.Dv = v->size[3];
  va.vec4_v = vec4_rows(v);
  va.o = view_of(out);
  va.o.s1 = out->stride[1];
  va.past = past;
  va.s0 = int(p.s0);
  va.t0 = int(p.t0);
  return run_score_v(va, p.nt, B * H, bf, v->dtype, out->dtype, s);
}

}  // namespace bdh

using namespace bdh;

extern "C" size_t bdh_tril_score_v_past_workspace(int64_t B, int64_t H, int64_t T, int64_t past, int64_t Dk,
                                                  int64_t Dv, int32_t qk_dtype) {
  if (past <= 0) return bdh_tril_score_v_workspace(B, H, T, Dk, Dv, qk_dtype);
  const size_t generic = plan_fwd(B, H, past + T, Dk, qk_dtype == BDH_BF16, past).ws_bytes;
  const size_t fast = qk_dtype == BDH_BF16 ? sy_past_workspace(B, H, past + T, past, Dk, Dv) : 0;
  return generic > fast ? generic : fast;
}

extern "C" int bdh_tril_score_v_past(const bdh_tensor4* q, const bdh_tensor4* k, const bdh_tensor4* v,
                                     const bdh_tensor4* out, int64_t past, void* workspace,
                                     size_t workspace_bytes, bdh_stream stream) {
  BDH_TRY(check_past(q, k, v, out, past));
  if (past == 0) return bdh_tril_score_v(q, k, v, out, workspace, workspace_bytes, stream);
  if (numel4(out) == 0) return BDH_OK;
  const int rc = sy_past(q, k, v, out, past, workspace, workspace_bytes, static_cast<hipStream_t>(stream));
  if (rc != kNotEligible) return rc;
  return run_past(q, k, v, out, past, workspace, workspace_bytes, static_cast<hipStream_t>(stream));
}

extern "C" size_t bdh_tril_score_v_workspace(int64_t B, int64_t H, int64_t T, int64_t Dk,
                                             int64_t Dv, int32_t qk_dtype) {
  const size_t generic = plan_fwd(B, H, T, Dk, qk_dtype == BDH_BF16).ws_bytes;
  // bf16 operands may take the fast path (with a RoPE table when fused).
  const size_t fast = qk_dtype == BDH_BF16 ? sy_workspace(B, H, T, Dk, Dv, true) : 0;
  return generic > fast ? generic : fast;
}

extern "C" int bdh_tril_score_v(const bdh_tensor4* q, const bdh_tensor4* k, const bdh_tensor4* v,
                                const bdh_tensor4* out, void* workspace, size_t workspace_bytes,
                                bdh_stream stream) {
  BDH_TRY(check_cold(q, k, v, out));
  return run_cold(q, k, v, out, nullptr, 0, nullptr, workspace, workspace_bytes,
                  static_cast<hipStream_t>(stream));
}

extern "C" int bdh_tril_rope_score_v(const bdh_tensor4* x, const bdh_tensor4* v,
                                     const bdh_tensor4* out, const float* freqs,
                                     int64_t rope_start, const bdh_tensor4* qr_out,
                                     void* workspace, size_t workspace_bytes,
                                     bdh_stream stream) {
  BDH_TRY(check_cold(x, x, v, out));
  if (freqs == nullptr && x->size[3] > 0) return BDH_ERR_ARG;
  if (x->size[3] % 2 != 0) return BDH_ERR_SHAPE;
  if (rope_start < 0 || rope_start + x->size[2] > (int64_t(1) << 24)) return BDH_ERR_ARG;
  if (qr_out != nullptr) {
    BDH_TRY(check_view(qr_out));
    for (int i = 0; i < 4; ++i)
      if (qr_out->size[i] != x->size[i]) return BDH_ERR_SHAPE;
    if (views_overlap(qr_out, x) || views_overlap(qr_out, v) || views_overlap(qr_out, out))
      return BDH_ERR_ALIAS;
  }
  return run_cold(x, x, v, out, freqs, rope_start, qr_out, workspace, workspace_bytes,
                  static_cast<hipStream_t>(stream));
}
