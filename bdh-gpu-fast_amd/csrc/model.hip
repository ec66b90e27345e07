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

namespace {

template <typename TX, typename TY>
int launch_relu_mul(const ReluMulArgs& a, int32_t odt, dim3 grid, hipStream_t s) {
  if (odt == BDH_BF16)
    BDH_LAUNCH("k_relu_mul", (k_relu_mul<TX, TY, bf16_t>), grid, dim3(256), 0, s, a);
  else
    BDH_LAUNCH("k_relu_mul", (k_relu_mul<TX, TY, float>), grid, dim3(256), 0, s, a);
  return BDH_OK;
}

}  // namespace
}  // namespace bdh

using namespace bdh;

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
