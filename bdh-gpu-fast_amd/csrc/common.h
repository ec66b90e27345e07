// Shared host/device helpers for the gfx950 BDH attention library.
#pragma once

#include <hip/hip_ext.h>
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "bdh_hip.h"

namespace bdh {

typedef __attribute__((__vector_size__(8 * sizeof(__bf16)))) __bf16 bf16x8;
typedef __attribute__((__vector_size__(16 * sizeof(float)))) float f32x16;
typedef __attribute__((__vector_size__(4 * sizeof(float)))) float f32x4;
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef uint16_t bf16_t;  // bf16 bits

// ---------------------------------------------------------------- scalars
__device__ __forceinline__ float to_f(float x) { return x; }
__device__ __forceinline__ float to_f(bf16_t h) { return __uint_as_float(uint32_t(h) << 16); }

// Round-to-nearest-even float -> bf16 bits (v_cvt_pk_bf16_f32 on gfx950).
__device__ __forceinline__ bf16_t f2bf(float x) {
  __bf16 b = (__bf16)x;
  return __builtin_bit_cast(bf16_t, b);
}
__device__ __forceinline__ float bf_round(float x) { return to_f(f2bf(x)); }
// Two floats to a bf16 pair (lo in bits 0-15), both rounded to nearest even:
// one v_cvt_pk_bf16_f32 (the scalar conversions above, packed by shifts and
// an or, took four instructions).
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef float f32x2_t __attribute__((ext_vector_type(2)));
__device__ __forceinline__ uint32_t pack_bf2(float lo, float hi) {
  const bf16x2_t b = __builtin_convertvector((f32x2_t{lo, hi}), bf16x2_t);
  return __builtin_bit_cast(uint32_t, b);
}

template <typename T> __device__ __forceinline__ T from_f(float x);
template <> __device__ __forceinline__ float from_f<float>(float x) { return x; }
template <> __device__ __forceinline__ bf16_t from_f<bf16_t>(float x) { return f2bf(x); }

// RoPE angle for (position, frequency): cos/sin of 2*pi*frac(fp32(pos)*freq).
// The phase product and its fractional part are computed exactly as the
// reference (one fp32 multiply, then phase - floor(phase)); v_sin/v_cos take
// the angle in revolutions, so no fp32(2*pi) rounding is added.
__device__ __forceinline__ void rope_cs(float pos, float freq, float& c, float& s) {
  const float ph = pos * freq;  // feeds v_fract only: nothing to contract with
  const float fr = __builtin_amdgcn_fractf(ph);
  c = __builtin_amdgcn_cosf(fr);
  s = __builtin_amdgcn_sinf(fr);
}

// Wave-wide (64 lanes) sum.
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}

// A strided 4-D view as seen by kernels: base pointer + element strides of the
// three outer dimensions (the last dimension is unit-stride).
struct View {
  const void* p;
  int64_t s0, s1, s2;
};

}  // namespace bdh

// ------------------------------------------------------------------ host
namespace bdh {

// Kernel launch bookkeeping shared by all entry points (profiling events).
// Profiling (bdh_profile_enable): the start and stop events of the next
// launch named `name`, or -1 (no events) when profiling is off.
int prof_begin(const char* name, hipEvent_t* start, hipEvent_t* stop);

inline int64_t numel4(const bdh_tensor4* t) {
  return t->size[0] * t->size[1] * t->size[2] * t->size[3];
}
inline int esize(int32_t dt) { return dt == BDH_BF16 ? 2 : 4; }
inline bool dtype_ok(int32_t dt) { return dt == BDH_F32 || dt == BDH_BF16; }

// Basic validity of a view: known dtype, data present when non-empty,
// unit stride on the last dimension (when it has more than one element).
inline int check_view(const bdh_tensor4* t) {
  if (!t) return BDH_ERR_ARG;
  if (!dtype_ok(t->dtype)) return BDH_ERR_DTYPE;
  for (int i = 0; i < 4; ++i)
    if (t->size[i] < 0) return BDH_ERR_SHAPE;
  if (numel4(t) > 0 && !t->data) return BDH_ERR_ARG;
  if (t->size[3] > 1 && t->stride[3] != 1) return BDH_ERR_STRIDE;
  return BDH_OK;
}

// True when 16-byte vector access of rows is legal: aligned base, outer
// strides and the row length multiples of the 16-byte element count.
inline bool vec16_ok(const bdh_tensor4* t) {
  const int per = 16 / esize(t->dtype);
  if ((reinterpret_cast<uintptr_t>(t->data) & 15) != 0) return false;
  for (int i = 0; i < 3; ++i)
    if (t->size[i] > 1 && (t->stride[i] % per) != 0) return false;
  return (t->size[3] % per) == 0;
}

inline View view_of(const bdh_tensor4* t) {
  View v;
  v.p = t->data;
  v.s0 = t->stride[0];
  v.s1 = t->size[1] == 1 ? 0 : t->stride[1];
  v.s2 = t->stride[2];
  return v;
}

// Byte ranges of two views overlap (conservative, by address span).
inline bool views_overlap(const bdh_tensor4* a, const bdh_tensor4* b) {
  if (!a || !b || numel4(a) == 0 || numel4(b) == 0) return false;
  auto span = [](const bdh_tensor4* t, uintptr_t& lo, uintptr_t& hi) {
    int64_t last = 0;
    for (int i = 0; i < 4; ++i) last += (t->size[i] - 1) * t->stride[i];
    lo = reinterpret_cast<uintptr_t>(t->data);
    hi = lo + uintptr_t(last + 1) * esize(t->dtype);
  };
  uintptr_t al, ah, bl, bh;
  span(a, al, ah);
  span(b, bl, bh);
  return al < bh && bl < ah;
}

inline size_t align_up(size_t x, size_t a) { return (x + a - 1) / a * a; }

}  // namespace bdh

#define BDH_TRY(...)                \
  do {                              \
    int _rc = (__VA_ARGS__);        \
    if (_rc != BDH_OK) return _rc;  \
  } while (0)

// Launch a kernel on `stream`.  When profiling is enabled the launch carries
// start and stop events that the runtime stamps when the kernel itself
// starts and ends (hipExtLaunchKernelGGL), so the recorded time is the
// kernel's execution, without the dispatch gaps around it.
#define BDH_LAUNCH(name, kernel, grid, block, shmem, stream, ...)                                   \
  do {                                                                                            \
    hipEvent_t _e0 = nullptr, _e1 = nullptr;                                                      \
    const int _slot = bdh::prof_begin(name, &_e0, &_e1);                                          \
    if (_slot >= 0)                                                                               \
      hipExtLaunchKernelGGL(kernel, grid, block, shmem, stream, _e0, _e1, 0, __VA_ARGS__);         \
    else                                                                                          \
      hipLaunchKernelGGL(kernel, grid, block, shmem, stream, __VA_ARGS__);                        \
    hipError_t _e = hipGetLastError();                                                            \
    if (_e != hipSuccess) return BDH_ERR_LAUNCH;                                                  \
  } while (0)
