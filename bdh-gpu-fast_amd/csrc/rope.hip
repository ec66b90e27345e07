// RoPE apply for gfx950: adjacent-pair rotation with caller-provided cos/sin
// tables (bdh_rope_rotate / bdh_rope_rotate_paired surface).
//
// Rounding follows the reference exactly (no FMA contraction):
//  - fp32 v: y0 = x0*c0 - x1*s0, y1 = x1*c1 + x0*s1 (fp32 products, fp32 add);
//  - bf16 v: every product is rounded to bf16, then the bf16 terms are added
//    and rounded again (kernels/rope.py:120-122);
//  - backward: dx0 = g0*c0 + g1*s1, dx1 = -g0*s0 + g1*c1 with the same
//    rounding rules (kernels/rope.py:543-556).
// The result is cast to the output dtype on store.
#include "common.h"

namespace bdh {

struct RopeArgs {
  View v, c, s, o;
  int64_t H, T, N;
  int64_t pairs;  // rows * N / 2
  int bwd;
  int vec8;       // every view 16-byte aligned per 8 elements (k_rope8)
  int64_t BH;     // B * H
  int bcast;      // cos/sin do not vary over batch and heads (k_rope8_bc)
  uint32_t nrr, ncb, total, per_xcd;  // k_rope8_bc work items: row runs x column blocks x T
};

template <typename TV, typename TC, typename TO>
__global__ __launch_bounds__(256) void k_rope(RopeArgs a) {
#pragma clang fp contract(off)
  const int64_t idx = int64_t(blockIdx.x) * 256 + threadIdx.x;
  if (idx >= a.pairs) return;
  const int64_t np = a.N / 2;
  const int64_t row = idx / np, p = idx % np;
  const int64_t t = row % a.T, bh = row / a.T, h = bh % a.H, b = bh / a.H;
  const TV* vp = static_cast<const TV*>(a.v.p) + b * a.v.s0 + h * a.v.s1 + t * a.v.s2 + 2 * p;
  const TC* cp = static_cast<const TC*>(a.c.p) + b * a.c.s0 + h * a.c.s1 + t * a.c.s2 + 2 * p;
  const TC* sp = static_cast<const TC*>(a.s.p) + b * a.s.s0 + h * a.s.s1 + t * a.s.s2 + 2 * p;
  TO* op = static_cast<TO*>(const_cast<void*>(a.o.p)) + b * a.o.s0 + h * a.o.s1 + t * a.o.s2 + 2 * p;
  const float x0 = to_f(vp[0]), x1 = to_f(vp[1]);
  const float c0 = to_f(cp[0]), c1 = to_f(cp[1]);
  const float s0 = to_f(sp[0]), s1 = to_f(sp[1]);
  float y0, y1;
  if constexpr (std::is_same<TV, bf16_t>::value) {
    if (a.bwd) {
      y0 = bf_round(bf_round(x0 * c0) + bf_round(x1 * s1));
      y1 = bf_round(bf_round((-x0) * s0) + bf_round(x1 * c1));
    } else {
      y0 = bf_round(bf_round(x0 * c0) + bf_round((-x1) * s0));
      y1 = bf_round(bf_round(x1 * c1) + bf_round(x0 * s1));
    }
  } else {
    if (a.bwd) {
      const float p0 = x0 * c0, p1 = x1 * s1, p2 = x0 * s0, p3 = x1 * c1;
      y0 = p0 + p1;
      y1 = -p2 + p3;
    } else {
      const float p0 = x0 * c0, p1 = x1 * s0, p2 = x1 * c1, p3 = x0 * s1;
      y0 = p0 - p1;
      y1 = p2 + p3;
    }
  }
  op[0] = from_f<TO>(y0);
  op[1] = from_f<TO>(y1);
}

// The same rotation, eight elements (four pairs) per thread with 16-byte
// accesses: grid (N / 2048, T, B * H), so no per-thread index division.
template <typename T>
struct Vec8 {
  T e[8];
};
template <typename T>
__device__ __forceinline__ Vec8<T> load8(const T* p) {
  Vec8<T> r;
  if constexpr (sizeof(T) == 2) {
    *reinterpret_cast<u32x4*>(r.e) = *reinterpret_cast<const u32x4*>(p);
  } else {
    reinterpret_cast<u32x4*>(r.e)[0] = reinterpret_cast<const u32x4*>(p)[0];
    reinterpret_cast<u32x4*>(r.e)[1] = reinterpret_cast<const u32x4*>(p)[1];
  }
  return r;
}
template <typename T>
__device__ __forceinline__ void store8(T* p, const Vec8<T>& r) {
  if constexpr (sizeof(T) == 2) {
    *reinterpret_cast<u32x4*>(p) = *reinterpret_cast<const u32x4*>(r.e);
  } else {
    reinterpret_cast<u32x4*>(p)[0] = reinterpret_cast<const u32x4*>(r.e)[0];
    reinterpret_cast<u32x4*>(p)[1] = reinterpret_cast<const u32x4*>(r.e)[1];
  }
}
// Streaming store (non-temporal: the rows are written once)
template <typename T>
__device__ __forceinline__ void store8_nt(T* p, const Vec8<T>& r) {
  u32x4* q = reinterpret_cast<u32x4*>(p);
  __builtin_nontemporal_store(reinterpret_cast<const u32x4*>(r.e)[0], q);
  if constexpr (sizeof(T) == 4) __builtin_nontemporal_store(reinterpret_cast<const u32x4*>(r.e)[1], q + 1);
}

template <typename TV, typename TC, typename TO>
__global__ __launch_bounds__(256) void k_rope8(RopeArgs a) {
#pragma clang fp contract(off)
  const int64_t e0 = (int64_t(blockIdx.x) * 256 + threadIdx.x) * 8;
  if (e0 >= a.N) return;
  const int64_t t = blockIdx.y, bh = blockIdx.z;
  const int64_t h = bh % a.H, b = bh / a.H;
  const Vec8<TV> x = load8(static_cast<const TV*>(a.v.p) + b * a.v.s0 + h * a.v.s1 + t * a.v.s2 + e0);
  const Vec8<TC> c = load8(static_cast<const TC*>(a.c.p) + b * a.c.s0 + h * a.c.s1 + t * a.c.s2 + e0);
  const Vec8<TC> sn = load8(static_cast<const TC*>(a.s.p) + b * a.s.s0 + h * a.s.s1 + t * a.s.s2 + e0);
  Vec8<TO> y;
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    const float x0 = to_f(x.e[2 * q]), x1 = to_f(x.e[2 * q + 1]);
    const float c0 = to_f(c.e[2 * q]), c1 = to_f(c.e[2 * q + 1]);
    const float s0 = to_f(sn.e[2 * q]), s1 = to_f(sn.e[2 * q + 1]);
    float y0, y1;
    if constexpr (std::is_same<TV, bf16_t>::value) {
      if (a.bwd) {
        y0 = bf_round(bf_round(x0 * c0) + bf_round(x1 * s1));
        y1 = bf_round(bf_round((-x0) * s0) + bf_round(x1 * c1));
      } else {
        y0 = bf_round(bf_round(x0 * c0) + bf_round((-x1) * s0));
        y1 = bf_round(bf_round(x1 * c1) + bf_round(x0 * s1));
      }
    } else {
      if (a.bwd) {
        const float p0 = x0 * c0, p1 = x1 * s1, p2 = x0 * s0, p3 = x1 * c1;
        y0 = p0 + p1;
        y1 = -p2 + p3;
      } else {
        const float p0 = x0 * c0, p1 = x1 * s0, p2 = x1 * c1, p3 = x0 * s1;
        y0 = p0 - p1;
        y1 = p2 + p3;
      }
    }
    y.e[2 * q] = from_f<TO>(y0);
    y.e[2 * q + 1] = from_f<TO>(y1);
  }
  store8(static_cast<TO*>(const_cast<void*>(a.o.p)) + b * a.o.s0 + h * a.o.s1 + t * a.o.s2 + e0, y);
}

// Tables broadcast over batch and heads (the model's case): work items
// (run of 16 (b, h) rows, column block of 2048, t); each thread loads its
// cos/sin once and rotates its eight elements in each row of the run, all
// sixteen loads in flight, non-temporal stores.  So the tables are read once
// per sixteen rows, and the grid spans the batch rows too (at C1: 98.6
// against 126 us with one workgroup per (column block, t) walking all B * H
// rows, four in flight).  Work items go to XCDs in contiguous ranges
// (workgroup i runs on XCD i % 8), so the row runs that share a table entry
// run on one XCD and read it from one L2.  C1, one box, a plain copy of x
// taking 98 us: 107.9-111.4 us with the runs of an entry on different XCDs,
// 97.1-98.4 with them on one, 96.0-96.5 with 16 rows a run instead of 8
// (32: 101.3); non-temporal loads of x cost 5 us more, plain stores 12 us.
constexpr int kRopeRows = 16;  // (b, h) rows per workgroup of k_rope8_bc

template <typename TV, typename TC, typename TO>
__global__ __launch_bounds__(256) void k_rope8_bc(RopeArgs a) {
#pragma clang fp contract(off)
  // 32-bit index arithmetic (the host checks the ranges): wave-uniform
  // 64-bit divisions would cost far more than this kernel's own work
  const uint32_t bid = blockIdx.x, L = (bid & 7) * a.per_xcd + (bid >> 3);
  if ((bid >> 3) >= a.per_xcd || L >= a.total) return;
  const uint32_t rr = L % a.nrr, q = L / a.nrr, cb = q % a.ncb, t = q / a.ncb;
  const int64_t e0 = (int64_t(cb) * 256 + threadIdx.x) * 8;
  if (e0 >= a.N) return;
  const Vec8<TC> c = load8(static_cast<const TC*>(a.c.p) + t * a.c.s2 + e0);
  const Vec8<TC> sn = load8(static_cast<const TC*>(a.s.p) + t * a.s.s2 + e0);
  float cf[8], sf[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    cf[e] = to_f(c.e[e]);
    sf[e] = to_f(sn.e[e]);
  }
  auto rot = [&](const Vec8<TV>& x) {
    Vec8<TO> y;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const float x0 = to_f(x.e[2 * q]), x1 = to_f(x.e[2 * q + 1]);
      const float c0 = cf[2 * q], c1 = cf[2 * q + 1], s0 = sf[2 * q], s1 = sf[2 * q + 1];
      float y0, y1;
      if constexpr (std::is_same<TV, bf16_t>::value) {
        if (a.bwd) {
          y0 = bf_round(bf_round(x0 * c0) + bf_round(x1 * s1));
          y1 = bf_round(bf_round((-x0) * s0) + bf_round(x1 * c1));
        } else {
          y0 = bf_round(bf_round(x0 * c0) + bf_round((-x1) * s0));
          y1 = bf_round(bf_round(x1 * c1) + bf_round(x0 * s1));
        }
      } else {
        if (a.bwd) {
          const float p0 = x0 * c0, p1 = x1 * s1, p2 = x0 * s0, p3 = x1 * c1;
          y0 = p0 + p1;
          y1 = -p2 + p3;
        } else {
          const float p0 = x0 * c0, p1 = x1 * s0, p2 = x1 * c1, p3 = x0 * s1;
          y0 = p0 - p1;
          y1 = p2 + p3;
        }
      }
      y.e[2 * q] = from_f<TO>(y0);
      y.e[2 * q + 1] = from_f<TO>(y1);
    }
    return y;
  };
  const TV* vp = static_cast<const TV*>(a.v.p) + t * a.v.s2 + e0;
  TO* op = static_cast<TO*>(const_cast<void*>(a.o.p)) + t * a.o.s2 + e0;
  const uint32_t H = uint32_t(a.H), BH = uint32_t(a.BH), bh0 = rr * kRopeRows;
  const uint32_t nrow = bh0 + kRopeRows < BH ? kRopeRows : BH - bh0;
  // row bh0 + u is (b, h) = ((bh0 + u) / H, (bh0 + u) % H), stepped from (b0, h0)
  uint32_t b = bh0 / H, h = bh0 - (bh0 / H) * H;
  if (nrow == kRopeRows) {
    int64_t vo[kRopeRows], oo[kRopeRows];
#pragma unroll
    for (int u = 0; u < kRopeRows; ++u) {
      vo[u] = b * a.v.s0 + h * a.v.s1;
      oo[u] = b * a.o.s0 + h * a.o.s1;
      if (++h == H) {
        h = 0;
        ++b;
      }
    }
    Vec8<TV> x[kRopeRows];
#pragma unroll
    for (int u = 0; u < kRopeRows; ++u) x[u] = load8(vp + vo[u]);
#pragma unroll
    for (int u = 0; u < kRopeRows; ++u) store8_nt(op + oo[u], rot(x[u]));
    return;
  }
  for (uint32_t u = 0; u < nrow; ++u) {
    store8_nt(op + b * a.o.s0 + h * a.o.s1, rot(load8(vp + b * a.v.s0 + h * a.v.s1)));
    if (++h == H) {
      h = 0;
      ++b;
    }
  }
}

// 16-byte alignment of every 8-element group of a view
static bool vec8_ok(const bdh_tensor4* t) {
  if ((reinterpret_cast<uintptr_t>(t->data) & 15) != 0) return false;
  for (int i = 0; i < 3; ++i)
    if (t->size[i] > 1 && (t->stride[i] % 8) != 0) return false;
  return t->size[3] % 8 == 0;
}

template <typename TV, typename TC, typename TO>
static int launch_rope(const RopeArgs& a, hipStream_t s) {
  // The broadcast kernel gains from its table reuse when there are many time
  // steps; at short T (a decode step: 4 column blocks at N = 8192) its few
  // workgroups leave the chip idle, so few time steps take the per-row kernel,
  // one workgroup per (column block, t, row).
  const int64_t bc_wgs = (a.N + 2047) / 2048 * a.T;
  if (a.vec8 && a.bcast && bc_wgs >= 512) {
    const int64_t nrr = (a.BH + kRopeRows - 1) / kRopeRows, ncb = (a.N + 2047) / 2048;
    const int64_t total = nrr * ncb * a.T, per_xcd = (total + 7) / 8;
    if (8 * per_xcd >= (int64_t(1) << 31)) return BDH_ERR_SHAPE;
    RopeArgs b = a;
    b.nrr = uint32_t(nrr);
    b.ncb = uint32_t(ncb);
    b.total = uint32_t(total);
    b.per_xcd = uint32_t(per_xcd);
    BDH_LAUNCH("k_rope", (k_rope8_bc<TV, TC, TO>), dim3(unsigned(8 * per_xcd)), dim3(256), 0, s, b);
    return BDH_OK;
  }
  if (a.vec8) {
    dim3 grid((unsigned)((a.N + 2047) / 2048), (unsigned)a.T, (unsigned)a.BH);
    BDH_LAUNCH("k_rope", (k_rope8<TV, TC, TO>), grid, dim3(256), 0, s, a);
    return BDH_OK;
  }
  dim3 grid((unsigned)((a.pairs + 255) / 256));
  BDH_LAUNCH("k_rope", (k_rope<TV, TC, TO>), grid, dim3(256), 0, s, a);
  return BDH_OK;
}

template <typename TV, typename TC>
static int pick_o(const RopeArgs& a, int32_t odt, hipStream_t s) {
  return odt == BDH_BF16 ? launch_rope<TV, TC, bf16_t>(a, s) : launch_rope<TV, TC, float>(a, s);
}

template <typename TV>
static int pick_c(const RopeArgs& a, int32_t cdt, int32_t odt, hipStream_t s) {
  return cdt == BDH_BF16 ? pick_o<TV, bf16_t>(a, odt, s) : pick_o<TV, float>(a, odt, s);
}

static View full_view(const bdh_tensor4* t) {
  View v;
  v.p = t->data;
  v.s0 = t->stride[0];
  v.s1 = t->stride[1];
  v.s2 = t->stride[2];
  return v;
}

}  // namespace bdh

using namespace bdh;

extern "C" int bdh_rope_rotate(const bdh_tensor4* v, const bdh_tensor4* cos, const bdh_tensor4* sin,
                               const bdh_tensor4* out, int32_t backward, bdh_stream stream) {
  BDH_TRY(check_view(v));
  BDH_TRY(check_view(cos));
  BDH_TRY(check_view(sin));
  BDH_TRY(check_view(out));
  if (cos->dtype != sin->dtype) return BDH_ERR_DTYPE;
  for (int i = 0; i < 4; ++i)
    if (cos->size[i] != v->size[i] || sin->size[i] != v->size[i] || out->size[i] != v->size[i])
      return BDH_ERR_SHAPE;
  if (v->size[3] % 2 != 0) return BDH_ERR_SHAPE;
  if (views_overlap(out, v) || views_overlap(out, cos) || views_overlap(out, sin)) return BDH_ERR_ALIAS;
  if (numel4(v) == 0) return BDH_OK;
  RopeArgs a;
  a.v = full_view(v);
  a.c = full_view(cos);
  a.s = full_view(sin);
  a.o = full_view(out);
  a.H = v->size[1];
  a.T = v->size[2];
  a.N = v->size[3];
  a.pairs = v->size[0] * v->size[1] * v->size[2] * (v->size[3] / 2);
  a.bwd = backward != 0;
  a.BH = v->size[0] * v->size[1];
  a.vec8 = vec8_ok(v) && vec8_ok(cos) && vec8_ok(sin) && vec8_ok(out) && a.T <= 65535 && a.BH <= 65535;
  auto flat = [](const bdh_tensor4* t) {
    return (t->size[0] <= 1 || t->stride[0] == 0) && (t->size[1] <= 1 || t->stride[1] == 0);
  };
  a.bcast = flat(cos) && flat(sin);
  hipStream_t s = static_cast<hipStream_t>(stream);
  return v->dtype == BDH_BF16 ? pick_c<bf16_t>(a, cos->dtype, out->dtype, s)
                              : pick_c<float>(a, cos->dtype, out->dtype, s);
}
