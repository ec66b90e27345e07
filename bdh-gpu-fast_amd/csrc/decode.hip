// KV-cache decode step for gfx950: out = (q K_past^T) V_past.
//
// HBM-bound: every past key row (N = 8192 elements) is read exactly once per
// query row.  Work is split over the past (chunks of keys per workgroup) so a
// B*H = 256 row batch still fills the chip; partial outputs over chunks are
// summed by a second small kernel (the op is linear in the scores, so no
// renormalisation is needed).
//
// Three score kernels share that shape: k_decode_bf16 (bf16 q and keys,
// v_dot2 products), k_decode_f32q (fp32 arithmetic, fp32 or bf16 keys, q of
// either dtype) and k_decode_partial (any strides and widths).  Each wave64
// streams key rows with 16-byte loads, reduces the dot product across the wave
// with shuffles and records the score in LDS; then all 256 threads form the
// partial out[d] = sum_s score_s V[s,d] with coalesced V row reads.
#include <mutex>

#include "common.h"

namespace bdh {

constexpr int kDecNT = 256;
constexpr int kChunk = 32;  // keys per workgroup

struct DecodeArgs {
  View q, k, v;
  int64_t H, Tq, S, Dk, Dv, Hv;
  int vec_k;
  float* part;    // [nchunk][rows][Dv]
  int64_t rows;   // B*H*Tq
};

template <typename TK>
__device__ __forceinline__ float dot_row(const float* qs, const TK* kp, int64_t Dk, int lane, bool vec) {
  float acc = 0.f;
  if (vec) {
    constexpr int EK = 16 / sizeof(TK);
    int64_t e0 = int64_t(lane) * EK;
    constexpr int STEP = 64 * EK;
    // four 16-byte loads in flight per lane per iteration
    for (; e0 + 3 * STEP < Dk; e0 += 4 * STEP) {
      u32x4 w[4];
#pragma unroll
      for (int u = 0; u < 4; ++u) w[u] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(kp + e0 + u * STEP));
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const TK* x = reinterpret_cast<const TK*>(&w[u]);
        const float* qq = qs + e0 + u * STEP;
#pragma unroll
        for (int e = 0; e < EK; ++e) acc += qq[e] * to_f(x[e]);
      }
    }
    for (; e0 < Dk; e0 += STEP) {
      u32x4 w = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(kp + e0));
      const TK* x = reinterpret_cast<const TK*>(&w);
#pragma unroll
      for (int e = 0; e < EK; ++e) acc += qs[e0 + e] * to_f(x[e]);
    }
  } else {
    for (int64_t e = lane; e < Dk; e += 64) acc += qs[e] * to_f(kp[e]);
  }
  return wave_sum(acc);
}

template <typename TQ, typename TK, typename TV>
__global__ __launch_bounds__(kDecNT) void k_decode_partial(DecodeArgs a) {
  extern __shared__ float smem[];
  float* qs = smem;              // Dk
  float* sc = smem + a.Dk;       // kChunk scores
  const int64_t row = blockIdx.y;
  const int64_t t = row % a.Tq, bh = row / a.Tq;
  const int64_t h = bh % a.H, b = bh / a.H;
  const int64_t hv = a.Hv == 1 ? 0 : h;

  const TQ* qp = static_cast<const TQ*>(a.q.p) + b * a.q.s0 + h * a.q.s1 + t * a.q.s2;
  for (int64_t e = threadIdx.x; e < a.Dk; e += kDecNT) qs[e] = to_f(qp[e]);
  __syncthreads();

  const int64_t s0 = int64_t(blockIdx.x) * kChunk;
  const int64_t s1 = min(a.S, s0 + kChunk);
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const TK* kb = static_cast<const TK*>(a.k.p) + b * a.k.s0 + h * a.k.s1;
  for (int64_t s = s0 + wave; s < s1; s += kDecNT / 64) {
    const float d = dot_row<TK>(qs, kb + s * a.k.s2, a.Dk, lane, a.vec_k != 0);
    if (lane == 0) sc[s - s0] = d;
  }
  __syncthreads();

  const TV* vb = static_cast<const TV*>(a.v.p) + b * a.v.s0 + hv * a.v.s1;
  float* out = a.part + (int64_t(blockIdx.x) * a.rows + row) * a.Dv;
  for (int64_t d = threadIdx.x; d < a.Dv; d += kDecNT) {
    float o = 0.f;
    for (int64_t s = s0; s < s1; ++s) o += sc[s - s0] * to_f(vb[s * a.v.s2 + d]);
    out[d] = o;
  }
}

// bf16 q and K_past (the cache path): q is staged once as bf16 (16 KB at
// N = 8192); each wave scores two key rows at a time with eight 16-byte loads
// in flight per lane, accumulating v_dot2_f32_bf16 (exact bf16 products, fp32
// sums) against the staged q; then the 256 threads form the chunk's partial
// out[d] = sum_s score_s V[s,d].  Needs Dk a multiple of 2048.
constexpr int kDecChunkB = 64;  // keys per workgroup
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));

// (The dwords are copied to scalars before the bit cast: this clang lowers
// __builtin_bit_cast of a vector element such as k.y as element 0.)
__device__ __forceinline__ float dot2w(uint32_t k, uint32_t q, float acc) {
  return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, k), __builtin_bit_cast(bf16x2, q), acc, false);
}
__device__ __forceinline__ float dot8(u32x4 k, u32x4 q, float acc) {
  const uint32_t k0 = k.x, k1 = k.y, k2 = k.z, k3 = k.w;
  const uint32_t q0 = q.x, q1 = q.y, q2 = q.z, q3 = q.w;
  acc = dot2w(k0, q0, acc);
  acc = dot2w(k1, q1, acc);
  acc = dot2w(k2, q2, acc);
  return dot2w(k3, q3, acc);
}

template <typename TV>
__global__ __launch_bounds__(kDecNT) void k_decode_bf16(DecodeArgs a) {
  extern __shared__ float smem[];
  float* sc = smem;                                         // kDecChunkB scores
  u32x4* qs = reinterpret_cast<u32x4*>(smem + kDecChunkB);  // q as Dk / 8 chunks of 8 bf16
  const int64_t row = blockIdx.y;
  const int64_t t = row % a.Tq, bh = row / a.Tq;
  const int64_t h = bh % a.H, b = bh / a.H;
  const int64_t hv = a.Hv == 1 ? 0 : h;
  const bf16_t* qp = static_cast<const bf16_t*>(a.q.p) + b * a.q.s0 + h * a.q.s1 + t * a.q.s2;
  for (int64_t i = threadIdx.x; i < a.Dk / 8; i += kDecNT) qs[i] = *reinterpret_cast<const u32x4*>(qp + 8 * i);
  __syncthreads();

  const int64_t s0 = int64_t(blockIdx.x) * kDecChunkB;
  const int64_t s1 = min(a.S, s0 + kDecChunkB);
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const bf16_t* kb = static_cast<const bf16_t*>(a.k.p) + b * a.k.s0 + h * a.k.s1;
  const int nc = int(a.Dk / 512);  // 16-byte chunks per lane per key row
  // keys s0 + wave + 4 j of this wave, in pairs (s, s + 4)
  for (int64_t s = s0 + wave; s < s1; s += 8) {
    const bool two = s + 4 < s1;
    const bf16_t* k0 = kb + s * a.k.s2 + lane * 8;
    const bf16_t* k1 = kb + (two ? s + 4 : s) * a.k.s2 + lane * 8;
    float acc0 = 0.f, acc1 = 0.f;
    for (int c = 0; c < nc; c += 4) {
      u32x4 x0[4], x1[4];
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        x0[u] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(k0 + (c + u) * 512));
        x1[u] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(k1 + (c + u) * 512));
      }
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const u32x4 q = qs[(c + u) * 64 + lane];
        acc0 = dot8(x0[u], q, acc0);
        acc1 = dot8(x1[u], q, acc1);
      }
    }
    acc0 = wave_sum(acc0);
    acc1 = wave_sum(acc1);
    if (lane == 0) {
      sc[s - s0] = acc0;
      if (two) sc[s + 4 - s0] = acc1;
    }
  }
  __syncthreads();

  const TV* vb = static_cast<const TV*>(a.v.p) + b * a.v.s0 + hv * a.v.s1;
  float* out = a.part + (int64_t(blockIdx.x) * a.rows + row) * a.Dv;
  for (int64_t d = threadIdx.x; d < a.Dv; d += kDecNT) {
    float o = 0.f;
    for (int64_t s = s0; s < s1; ++s) o += sc[s - s0] * to_f(vb[s * a.v.s2 + d]);
    out[d] = o;
  }
}

// fp32 arithmetic against fp32 or bf16 keys, q of either dtype: the
// reference's decode computes in fp32 (its cache casts a 16-bit past up
// before the products), and widening bf16 to fp32 is exact, so reading a bf16
// cache in place gives the products of its fp32 cast copy without the copy.
// q is staged once per workgroup as fp32 in LDS, arranged so that the 16-byte
// key piece a lane loads (EK elements) meets its q values in EK / 4
// contiguous 16-byte LDS reads: float4 plane p of piece c sits at
// qs[(NP c + p) 64 + lane].  Each wave scores two key rows at a time with
// eight 16-byte loads in flight per lane; then the 256 threads form the
// chunk's partial out[d] = sum_s score_s V[s,d].  Needs Dk a multiple of
// 64 EK and 16-byte aligned q and key rows.
template <typename TK>
__device__ __forceinline__ float dot_piece(const u32x4& w, const float4* qs4, int np_stride, float acc) {
  if constexpr (sizeof(TK) == 4) {
    const float4 q = qs4[0];
    acc = fmaf(__uint_as_float(w.x), q.x, acc);
    acc = fmaf(__uint_as_float(w.y), q.y, acc);
    acc = fmaf(__uint_as_float(w.z), q.z, acc);
    return fmaf(__uint_as_float(w.w), q.w, acc);
  } else {
    const float4 qa = qs4[0], qb = qs4[np_stride];
    const uint32_t w0 = w.x, w1 = w.y, w2 = w.z, w3 = w.w;
    acc = fmaf(__uint_as_float(w0 << 16), qa.x, acc);
    acc = fmaf(__uint_as_float(w0 & 0xffff0000u), qa.y, acc);
    acc = fmaf(__uint_as_float(w1 << 16), qa.z, acc);
    acc = fmaf(__uint_as_float(w1 & 0xffff0000u), qa.w, acc);
    acc = fmaf(__uint_as_float(w2 << 16), qb.x, acc);
    acc = fmaf(__uint_as_float(w2 & 0xffff0000u), qb.y, acc);
    acc = fmaf(__uint_as_float(w3 << 16), qb.z, acc);
    return fmaf(__uint_as_float(w3 & 0xffff0000u), qb.w, acc);
  }
}

template <typename TQ, typename TK, typename TV>
__global__ __launch_bounds__(kDecNT) void k_decode_f32q(DecodeArgs a) {
  constexpr int EK = 16 / int(sizeof(TK));  // key elements per 16-byte piece
  constexpr int NP = EK / 4;                // float4 planes of q per piece
  extern __shared__ float smem[];
  float* sc = smem;                                         // kDecChunkB scores
  float4* qs = reinterpret_cast<float4*>(smem + kDecChunkB);  // Dk / 4 float4
  const int64_t row = blockIdx.y;
  const int64_t t = row % a.Tq, bh = row / a.Tq;
  const int64_t h = bh % a.H, b = bh / a.H;
  const int64_t hv = a.Hv == 1 ? 0 : h;
  const TQ* qp = static_cast<const TQ*>(a.q.p) + b * a.q.s0 + h * a.q.s1 + t * a.q.s2;
  for (int64_t i = threadIdx.x; i < a.Dk / 4; i += kDecNT) {
    const int64_t l = i & 63, cp = i >> 6;
    const int64_t e = ((cp / NP) * 64 + l) * EK + (cp % NP) * 4;
    float4 v;
    if constexpr (sizeof(TQ) == 4) {
      v = *reinterpret_cast<const float4*>(qp + e);
    } else {
      const u32x2 w = *reinterpret_cast<const u32x2*>(qp + e);
      const uint32_t w0 = w.x, w1 = w.y;
      v = make_float4(__uint_as_float(w0 << 16), __uint_as_float(w0 & 0xffff0000u), __uint_as_float(w1 << 16),
                      __uint_as_float(w1 & 0xffff0000u));
    }
    qs[i] = v;
  }
  __syncthreads();

  const int64_t s0 = int64_t(blockIdx.x) * kDecChunkB;
  const int64_t s1 = min(a.S, s0 + kDecChunkB);
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const TK* kb = static_cast<const TK*>(a.k.p) + b * a.k.s0 + h * a.k.s1;
  const int nc = int(a.Dk / (64 * EK));  // 16-byte pieces per lane per key row
  const float4* ql = qs + lane;
  // keys s0 + wave + 4 j of this wave, in pairs (s, s + 4)
  for (int64_t s = s0 + wave; s < s1; s += 8) {
    const bool two = s + 4 < s1;
    const TK* k0 = kb + s * a.k.s2 + lane * EK;
    const TK* k1 = kb + (two ? s + 4 : s) * a.k.s2 + lane * EK;
    float acc0 = 0.f, acc1 = 0.f;
    int c = 0;
    for (; c + 4 <= nc; c += 4) {
      u32x4 x0[4], x1[4];
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        x0[u] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(k0 + (c + u) * 64 * EK));
        x1[u] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(k1 + (c + u) * 64 * EK));
      }
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const float4* q = ql + (NP * (c + u)) * 64;
        acc0 = dot_piece<TK>(x0[u], q, 64, acc0);
        acc1 = dot_piece<TK>(x1[u], q, 64, acc1);
      }
    }
    for (; c < nc; ++c) {
      const u32x4 x0 = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(k0 + c * 64 * EK));
      const u32x4 x1 = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(k1 + c * 64 * EK));
      const float4* q = ql + (NP * c) * 64;
      acc0 = dot_piece<TK>(x0, q, 64, acc0);
      acc1 = dot_piece<TK>(x1, q, 64, acc1);
    }
    acc0 = wave_sum(acc0);
    acc1 = wave_sum(acc1);
    if (lane == 0) {
      sc[s - s0] = acc0;
      if (two) sc[s + 4 - s0] = acc1;
    }
  }
  __syncthreads();

  const TV* vb = static_cast<const TV*>(a.v.p) + b * a.v.s0 + hv * a.v.s1;
  float* out = a.part + (int64_t(blockIdx.x) * a.rows + row) * a.Dv;
  for (int64_t d = threadIdx.x; d < a.Dv; d += kDecNT) {
    float o = 0.f;
    for (int64_t s = s0; s < s1; ++s) o += sc[s - s0] * to_f(vb[s * a.v.s2 + d]);
    out[d] = o;
  }
}

template <typename TO>
__global__ __launch_bounds__(kDecNT) void k_decode_reduce(const float* part, int64_t nchunk, int64_t rows,
                                                          int64_t Dv, View o, int64_t H, int64_t Tq) {
  const int64_t idx = int64_t(blockIdx.x) * kDecNT + threadIdx.x;
  if (idx >= rows * Dv) return;
  const int64_t row = idx / Dv, d = idx % Dv;
  float s = 0.f;
  for (int64_t c = 0; c < nchunk; ++c) s += part[(c * rows + row) * Dv + d];
  const int64_t t = row % Tq, bh = row / Tq, h = bh % H, b = bh / H;
  TO* op = static_cast<TO*>(const_cast<void*>(o.p)) + b * o.s0 + h * o.s1 + t * o.s2;
  op[d] = from_f<TO>(s);
}

static int64_t n_chunks(int64_t S) { return S > 0 ? (S + kChunk - 1) / kChunk : 1; }

template <typename TQ, typename TK, typename TV>
static int launch_partial(const DecodeArgs& a, int64_t nchunk, hipStream_t s) {
  dim3 grid((unsigned)(nchunk), unsigned(a.rows));
  const size_t shm = size_t(a.Dk + kChunk) * sizeof(float);
  BDH_LAUNCH("k_decode_partial", (k_decode_partial<TQ, TK, TV>), grid, dim3(kDecNT), shm, s, a);
  return BDH_OK;
}

template <typename TQ, typename TK>
static int pick_v(const DecodeArgs& a, int64_t nchunk, int32_t vdt, hipStream_t s) {
  return vdt == BDH_BF16 ? launch_partial<TQ, TK, bf16_t>(a, nchunk, s)
                         : launch_partial<TQ, TK, float>(a, nchunk, s);
}

template <typename TQ>
static int pick_k(const DecodeArgs& a, int64_t nchunk, int32_t kdt, int32_t vdt, hipStream_t s) {
  return kdt == BDH_BF16 ? pick_v<TQ, bf16_t>(a, nchunk, vdt, s) : pick_v<TQ, float>(a, nchunk, vdt, s);
}

template <typename TQ, typename TK, typename TV>
static int launch_f32q_t(const DecodeArgs& a, int64_t nred, hipStream_t s) {
  const dim3 grid((unsigned)nred, unsigned(a.rows));
  const size_t shm = size_t(kDecChunkB) * sizeof(float) + size_t(a.Dk) * sizeof(float);
  BDH_LAUNCH("k_decode_f32q", (k_decode_f32q<TQ, TK, TV>), grid, dim3(kDecNT), shm, s, a);
  return BDH_OK;
}

template <typename TQ, typename TK>
static int launch_f32q_v(const DecodeArgs& a, int64_t nred, int32_t vdt, hipStream_t s) {
  return vdt == BDH_BF16 ? launch_f32q_t<TQ, TK, bf16_t>(a, nred, s) : launch_f32q_t<TQ, TK, float>(a, nred, s);
}

static int launch_f32q(const DecodeArgs& a, int64_t nred, int32_t qdt, int32_t kdt, int32_t vdt, hipStream_t s) {
  if (qdt == BDH_BF16)
    return kdt == BDH_BF16 ? launch_f32q_v<bf16_t, bf16_t>(a, nred, vdt, s) : launch_f32q_v<bf16_t, float>(a, nred, vdt, s);
  return kdt == BDH_BF16 ? launch_f32q_v<float, bf16_t>(a, nred, vdt, s) : launch_f32q_v<float, float>(a, nred, vdt, s);
}

}  // namespace bdh

using namespace bdh;

extern "C" size_t bdh_tril_decode_workspace(int64_t B, int64_t H, int64_t Tq, int64_t S, int64_t Dk,
                                            int64_t Dv) {
  (void)Dk;
  return size_t(n_chunks(S)) * size_t(B * H * Tq) * size_t(Dv) * sizeof(float);
}

namespace bdh {
namespace {

// Shape/dtype contract of decode (kernels/cuda_attn.py:114-131,
// csrc/tril_attn_cpu.cpp:214-223) and the launch plan: part_bytes is the
// partial-sum storage the chosen kernels need.
enum DecodeKind { kDecGeneric = 0, kDecBf16 = 1, kDecF32q = 2 };
struct DecodePlan {
  DecodeArgs a;
  DecodeKind kind = kDecGeneric;
  int64_t nred = 0;
  size_t part_bytes = 0;
};

int decode_plan(const bdh_tensor4* q, const bdh_tensor4* k, const bdh_tensor4* v, const bdh_tensor4* out,
                DecodePlan& p) {
  BDH_TRY(check_view(q));
  BDH_TRY(check_view(k));
  BDH_TRY(check_view(v));
  BDH_TRY(check_view(out));
  const int64_t B = q->size[0], H = q->size[1], Tq = q->size[2], Dk = q->size[3];
  const int64_t S = k->size[2], Dv = v->size[3];
  if (k->size[0] != B || k->size[1] != H || k->size[3] != Dk) return BDH_ERR_SHAPE;
  if (v->size[0] != B || v->size[2] != S) return BDH_ERR_SHAPE;
  if (v->size[1] != 1 && v->size[1] != H) return BDH_ERR_SHAPE;
  if (out->size[0] != B || out->size[1] != H || out->size[2] != Tq || out->size[3] != Dv)
    return BDH_ERR_SHAPE;
  if (views_overlap(out, q) || views_overlap(out, k) || views_overlap(out, v)) return BDH_ERR_ALIAS;
  if (B * H * Tq > 65535 || n_chunks(S) > int64_t(1) << 30) return BDH_ERR_SHAPE;
  if ((Dk + kChunk) * int64_t(sizeof(float)) > 64 * 1024) return BDH_ERR_SHAPE;
  DecodeArgs& a = p.a;
  a.q = view_of(q);
  a.q.s1 = q->stride[1];
  a.k = view_of(k);
  a.k.s1 = k->stride[1];
  a.v = view_of(v);
  a.H = H;
  a.Tq = Tq;
  a.S = S;
  a.Dk = Dk;
  a.Dv = Dv;
  a.Hv = v->size[1];
  a.vec_k = vec16_ok(k) ? 1 : 0;
  a.part = nullptr;
  a.rows = B * H * Tq;
  // streaming kernels (64-key chunks) where q and the key rows allow
  // 16-byte pieces; the generic kernel otherwise
  const bool vec = vec16_ok(q) && vec16_ok(k) && S > 0;
  if (vec && q->dtype == BDH_BF16 && k->dtype == BDH_BF16 && Dk % 2048 == 0 && Dk * 2 + kDecChunkB * 4 <= 64 * 1024)
    p.kind = kDecBf16;
  else if (vec && Dk % (64 * (k->dtype == BDH_BF16 ? 8 : 4)) == 0 && Dk * 4 + kDecChunkB * 4 <= 64 * 1024)
    p.kind = kDecF32q;
  else
    p.kind = kDecGeneric;
  p.nred = p.kind == kDecGeneric ? n_chunks(S) : (S + kDecChunkB - 1) / kDecChunkB;
  p.part_bytes = size_t(p.nred) * size_t(a.rows) * size_t(Dv) * sizeof(float);
  return BDH_OK;
}

// The partial kernels write every (chunk, row, column) of part, so part needs
// no clearing between calls.
int decode_run(const DecodePlan& p, const bdh_tensor4* q, const bdh_tensor4* k, const bdh_tensor4* v,
               const bdh_tensor4* out, float* part, hipStream_t st) {
  DecodeArgs a = p.a;
  a.part = part;
  if (p.kind == kDecBf16) {
    const dim3 grid((unsigned)p.nred, unsigned(a.rows));
    const size_t shm = size_t(kDecChunkB) * sizeof(float) + size_t(a.Dk) * 2;
    if (v->dtype == BDH_BF16)
      BDH_LAUNCH("k_decode_bf16", k_decode_bf16<bf16_t>, grid, dim3(kDecNT), shm, st, a);
    else
      BDH_LAUNCH("k_decode_bf16", k_decode_bf16<float>, grid, dim3(kDecNT), shm, st, a);
  } else if (p.kind == kDecF32q) {
    const int rc = launch_f32q(a, p.nred, q->dtype, k->dtype, v->dtype, st);
    if (rc != BDH_OK) return rc;
  } else {
    const int rc = q->dtype == BDH_BF16 ? pick_k<bf16_t>(a, p.nred, k->dtype, v->dtype, st)
                                        : pick_k<float>(a, p.nred, k->dtype, v->dtype, st);
    if (rc != BDH_OK) return rc;
  }
  View o = view_of(out);
  o.s1 = out->stride[1];
  const int64_t total = a.rows * a.Dv;
  dim3 grid((unsigned)((total + kDecNT - 1) / kDecNT));
  if (out->dtype == BDH_BF16)
    BDH_LAUNCH("k_decode_reduce", k_decode_reduce<bf16_t>, grid, dim3(kDecNT), 0, st, a.part, p.nred, a.rows,
               a.Dv, o, a.H, a.Tq);
  else
    BDH_LAUNCH("k_decode_reduce", k_decode_reduce<float>, grid, dim3(kDecNT), 0, st, a.part, p.nred, a.rows,
               a.Dv, o, a.H, a.Tq);
  return BDH_OK;
}

}  // namespace
}  // namespace bdh

extern "C" int bdh_tril_decode(const bdh_tensor4* q, const bdh_tensor4* k, const bdh_tensor4* v,
                               const bdh_tensor4* out, void* workspace, size_t workspace_bytes,
                               bdh_stream stream) {
  DecodePlan p;
  BDH_TRY(decode_plan(q, k, v, out, p));
  if (numel4(out) == 0) return BDH_OK;
  const size_t need = bdh_tril_decode_workspace(q->size[0], q->size[1], q->size[2], k->size[2], q->size[3],
                                                v->size[3]);
  if (workspace == nullptr || workspace_bytes < need) return BDH_ERR_WORKSPACE;
  return decode_run(p, q, k, v, out, static_cast<float*>(workspace), static_cast<hipStream_t>(stream));
}

// ------------------------------------------------------- no allocation
// The partial sums of bdh_tril_decode_noalloc live in this library-owned
// array: every GPU the library runs on holds its own copy (allocated when the
// code object loads on that device, kept until the process ends).  In host
// code `scratch` only names the symbol; its device address comes from
// hipGetSymbolAddress with the device current, once per device.
static __device__ __align__(256) uint8_t scratch[BDH_NOALLOC_SCRATCH_BYTES];

namespace {
constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices] = {};

// Device address of the current device's scratch array (looked up on the
// first call on that device), or nullptr when the lookup fails.
void* scratch_of_current_device() {
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return nullptr;
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (g_scratch_ptr[dev] == nullptr) {
    void* ptr = nullptr;
    if (hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch)) != hipSuccess || ptr == nullptr) return nullptr;
    g_scratch_ptr[dev] = ptr;
  }
  return g_scratch_ptr[dev];
}
}  // namespace

extern "C" int bdh_tril_decode_noalloc(const bdh_tensor4* q, const bdh_tensor4* k, const bdh_tensor4* v,
                                       const bdh_tensor4* out, bdh_stream stream) {
  DecodePlan p;
  BDH_TRY(decode_plan(q, k, v, out, p));
  if (numel4(out) == 0) return BDH_OK;
  if (p.part_bytes > size_t(BDH_NOALLOC_SCRATCH_BYTES)) return BDH_ERR_SCRATCH;
  void* part = scratch_of_current_device();
  if (part == nullptr) return BDH_ERR_LAUNCH;
  return decode_run(p, q, k, v, out, static_cast<float*>(part), static_cast<hipStream_t>(stream));
}
