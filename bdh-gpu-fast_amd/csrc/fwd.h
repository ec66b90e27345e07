// Forward-kernel arguments and launch helpers shared by fwd.hip and bwd.hip.
#pragma once

#include "tile_gemm.h"

namespace bdh {

// Split-K is chosen so that one launch has about this many workgroups.
constexpr int64_t kTargetWorkgroups = 1024;

struct FwdPlan {
  int64_t nt = 0;      // 128-row tiles per slab
  int64_t s0 = 0;      // first row tile computed (queries at an offset)
  int64_t t0 = 0;      // packed index of its first tile
  int64_t ntl = 0;     // packed lower tiles per slab, from t0 on
  int64_t splits = 1;  // split-K factor
  int64_t kc = 0;      // k extent of one split (multiple of the K stage)
  size_t ws_bytes = 0; // partial score tiles
};

struct ScoresArgs {
  View q, k;
  int64_t H, T, K;
  int q_is_k;
  bool vec_q, vec_k;
  const float* freqs;
  int64_t rope_start;
  float* sp;  // partial tiles [split][slab][tile - t0][128*128]
  int64_t kc;
  int ntl;
  View qr;    // optional RoPE(x) output (diagonal tiles write it)
  bool qr_bf;
  // Queries at an offset (chunked prefill): query row i is global row
  // past + i over keys [0, T); the launch covers the packed lower tiles from
  // t0 on (row tiles >= past / 128).  0 for the ordinary op.
  int64_t past = 0;
  int t0 = 0;
};

struct ScoreVArgs {
  const float* sp;
  int64_t split_stride;
  int nsplit;
  int ntl;
  View v;
  int64_t H, Hv, T, Dv;
  bool vec4_v;
  View o;
  int64_t past = 0;  // output row i is global row past + i (chunked prefill)
  int s0 = 0, t0 = 0;  // first row tile; packed index of its first tile
};

// bf16 fast path of the cold op (syrk.hip).  sy_cold returns kNotEligible
// when the operands fall outside its constraints (the caller then uses the
// generic kernels), otherwise a BDH_* code.
constexpr int kNotEligible = -1;
size_t sy_workspace(int64_t B, int64_t H, int64_t T, int64_t N, int64_t Dv, bool rope);
int sy_cold(const bdh_tensor4* q, const bdh_tensor4* k, const bdh_tensor4* v, const bdh_tensor4* out,
            const float* freqs, int64_t rope_start, const bdh_tensor4* qr, void* ws, size_t ws_bytes,
            hipStream_t s);
// Queries at an offset on the same path, when q is rows past.. of k (same
// storage and strides, bf16): only the row tiles that hold new rows.
size_t sy_past_workspace(int64_t B, int64_t H, int64_t Tk, int64_t past, int64_t N, int64_t Dv);
int sy_past(const bdh_tensor4* q, const bdh_tensor4* k, const bdh_tensor4* v, const bdh_tensor4* out,
            int64_t past, void* ws, size_t ws_bytes, hipStream_t s);

// Backward dV on the MFMA path (syrk.hip): score tiles recomputed by the
// forward score kernel into ws (sy_bwd_workspace bytes), then dV from them.
size_t sy_bwd_workspace(int64_t B, int64_t H, int64_t T, int64_t N);
// saved: the score tiles left by the forward on the same q (its workspace), used
// instead of recomputing them (then ws may be NULL).
// rel: the saved tiles came from the relative-RoPE forward (their fragment
// slot order).
int sy_bwd_dv(const bdh_tensor4* q, const bdh_tensor4* v, const bdh_tensor4* dout, const bdh_tensor4* dv, void* ws,
              size_t ws_bytes, hipStream_t s, const void* saved = nullptr, int rel = 0);
// Whether bdh_tril_rope_score_v(x, x, v) without the R(x) copy runs the MFMA
// path: its score tiles then sit at *tiles_offset of its workspace, whose
// first *kept_bytes the backward from saved tiles needs, in the relative
// layout when *rel.
bool sy_rope_keeps_scores(const bdh_tensor4* x, const bdh_tensor4* v, size_t* tiles_offset, size_t* kept_bytes,
                          int* rel);
// Whether bdh_tril_score_v(q, q, v) runs the MFMA path; its workspace then
// starts with the score tiles (*scores_bytes of them) that sy_bwd_dv can reuse.
bool sy_keeps_scores(const bdh_tensor4* q, const bdh_tensor4* v, size_t* scores_bytes);
// Backward G = dS + dS^T (bf16, [B*H][tpad][tpad]) on the MFMA score kernel
// (syrk.hip): bf16 dO and V, D a multiple of 64.
int sy_bwd_g(const bdh_tensor4* dout, const bdh_tensor4* v, void* g, int64_t tpad, hipStream_t s);
// Backward dQ = G X on the MFMA path (syrk.hip): bf16 X, self attention.
// With freqs, out = R^T(G X) at positions rope_start + t (X = R(x)).
// rot_b (with freqs): x is x itself, rotated in the kernel as it is staged.
// g_sym: G is exactly symmetric (written by sy_bwd_g), so its rows stand in
// for its columns and both operands stream as whole 128-byte lines.
int sy_dq(const void* g, int64_t tpad, bool g_sym, const bdh_tensor4* x, const bdh_tensor4* out, hipStream_t s,
          const float* freqs = nullptr, int64_t rope_start = 0, bool rot_b = false);
// Backward of the fused RoPE op on the MFMA path (syrk.hip): the score tiles
// of R(x) R(x)^T with R(x) written to qr (absolute positions; ws starts with
// their (cos, sin) table, *tiles points at the tiles).
size_t sy_rope_scores_workspace(int64_t B, int64_t H, int64_t T, int64_t N);
int sy_rope_scores(const bdh_tensor4* x, const bdh_tensor4* v, const float* freqs, int64_t rope_start,
                   const bdh_tensor4* qr, void* ws, size_t ws_bytes, hipStream_t s, const void** tiles);

FwdPlan plan_fwd(int64_t B, int64_t H, int64_t T, int64_t K, bool bf, int64_t past = 0);
int run_scores(const ScoresArgs& a, const FwdPlan& p, int64_t BH, bool bf, bool rope, bool trans,
               hipStream_t s);

}  // namespace bdh
