// Shared device helpers for the Mamba3 SISO scan kernels (gfx950 / CDNA4).
//
// Wave64 everywhere: prefix scans and reductions are written for 64-lane
// wavefronts, MFMA tiles are 16x16 (v_mfma_f32_16x16x32_bf16 and
// v_mfma_f32_16x16x4_f32).  Transcendentals use the hardware units:
// v_exp_f32 (2^x), v_rcp_f32, and v_sin_f32 / v_cos_f32, which take their
// argument in revolutions (sin(2*pi*u)); angles are range-reduced to [0, 2pi)
// before use, so u lies in [0, 1).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace m3 {

typedef __bf16 bf16;
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

constexpr float kLog2e = 1.4426950408889634f;
constexpr float kPi = 3.14159265358979323846f;
constexpr float kTwoPi = 6.28318530717958647692f;
constexpr float kInvTwoPi = 0.15915494309189533577f;

// ---------------------------------------------------------------- math
__device__ __forceinline__ float exp2_fast(float x) { return __builtin_amdgcn_exp2f(x); }
__device__ __forceinline__ float exp_fast(float x) { return __builtin_amdgcn_exp2f(x * kLog2e); }
__device__ __forceinline__ float rcp_fast(float x) { return __builtin_amdgcn_rcpf(x); }

// tanh(x) = sign(x) (1 - e) / (1 + e), e = exp(-2|x|): no overflow for any x,
// absolute error ~1e-7 over the real line.
__device__ __forceinline__ float tanh_fast(float x) {
  float e = exp2_fast(-2.0f * kLog2e * fabsf(x));
  float t = (1.0f - e) * rcp_fast(1.0f + e);
  return copysignf(t, x);
}

__device__ __forceinline__ float sigmoid_fast(float x) { return rcp_fast(1.0f + exp_fast(-x)); }
__device__ __forceinline__ float silu_fast(float x) { return x * rcp_fast(1.0f + exp_fast(-x)); }

// theta - 2pi*floor(theta/2pi): the range reduction the reference applies to
// the cumulative rotation angle (mamba3_jax.py:143, mamba3.py:509); the
// quotient is formed with the reciprocal (differs only within an ulp of a
// multiple of 2pi, where both results are equivalent angles).
__device__ __forceinline__ float wrap_2pi(float th) { return th - kTwoPi * floorf(th * kInvTwoPi); }

// cos/sin of a wrapped angle in [0, 2pi) through the revolution-based units.
__device__ __forceinline__ void sincos_wrapped(float th, float* c, float* s) {
  float u = th * kInvTwoPi;
  *c = __builtin_amdgcn_cosf(u);
  *s = __builtin_amdgcn_sinf(u);
}

// ---------------------------------------------------------------- element IO
template <typename T> struct Elem;
template <> struct Elem<float> {
  __device__ __forceinline__ static float to_f(float x) { return x; }
  __device__ __forceinline__ static float from_f(float x) { return x; }
};
template <> struct Elem<bf16> {
  __device__ __forceinline__ static float to_f(bf16 x) { return (float)x; }
  __device__ __forceinline__ static bf16 from_f(float x) { return (bf16)x; }
};

// Eight consecutive elements held in registers in storage form.
template <typename T> struct Vec8;
template <> struct Vec8<bf16> {
  uint4 raw;
  __device__ __forceinline__ void zero() { raw = make_uint4(0, 0, 0, 0); }
  __device__ __forceinline__ void load(const bf16* p) { raw = *reinterpret_cast<const uint4*>(p); }
  __device__ __forceinline__ void raw_set(const uint4& r) { raw = r; }
  __device__ __forceinline__ void to_f(float f[8]) const {
    const uint32_t w[4] = {raw.x, raw.y, raw.z, raw.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      f[2 * i] = __uint_as_float(w[i] << 16);
      f[2 * i + 1] = __uint_as_float(w[i] & 0xffff0000u);
    }
  }
};
template <> struct Vec8<float> {
  float4 a, b;
  __device__ __forceinline__ void zero() { a = make_float4(0, 0, 0, 0); b = a; }
  __device__ __forceinline__ void load(const float* p) {
    a = reinterpret_cast<const float4*>(p)[0];
    b = reinterpret_cast<const float4*>(p)[1];
  }
  __device__ __forceinline__ void raw_set2(const uint4& r0, const uint4& r1) {
    a = make_float4(__uint_as_float(r0.x), __uint_as_float(r0.y), __uint_as_float(r0.z), __uint_as_float(r0.w));
    b = make_float4(__uint_as_float(r1.x), __uint_as_float(r1.y), __uint_as_float(r1.z), __uint_as_float(r1.w));
  }
  __device__ __forceinline__ void to_f(float f[8]) const {
    f[0] = a.x; f[1] = a.y; f[2] = a.z; f[3] = a.w;
    f[4] = b.x; f[5] = b.y; f[6] = b.z; f[7] = b.w;
  }
};

// Store eight floats as eight consecutive elements of T (16-byte aligned for bf16,
// 32-byte for float).
__device__ __forceinline__ void store8(bf16* p, const float f[8]) {
  bf16x8 v;
#pragma unroll
  for (int i = 0; i < 8; ++i) v[i] = (bf16)f[i];
  *reinterpret_cast<bf16x8*>(p) = v;
}
__device__ __forceinline__ void store8(float* p, const float f[8]) {
  reinterpret_cast<float4*>(p)[0] = make_float4(f[0], f[1], f[2], f[3]);
  reinterpret_cast<float4*>(p)[1] = make_float4(f[4], f[5], f[6], f[7]);
}

// ---------------------------------------------------------------- wave ops
// DPP lane move: lanes whose source is outside the row, or whose row/bank is
// masked off, receive 0.
template <int CTRL, int ROW_MASK = 0xf, int BANK_MASK = 0xf>
__device__ __forceinline__ float dpp0(float x) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), CTRL, ROW_MASK, BANK_MASK, true));
}
constexpr int kDppRowShr1 = 0x111, kDppRowShr2 = 0x112, kDppRowShr4 = 0x114, kDppRowShr8 = 0x118;
constexpr int kDppRowBcast15 = 0x142, kDppRowBcast31 = 0x143;
constexpr int kDppQuadXor1 = 0xB1;   // quad_perm [1,0,3,2]
constexpr int kDppQuadXor2 = 0x4E;   // quad_perm [2,3,0,1]
constexpr int kDppHalfMirror = 0x141, kDppMirror = 0x140;

// Inclusive prefix sum over the 64 lanes of a wavefront: Hillis-Steele inside
// each row of 16 lanes (row_shr 1, 2, 4, 8), then the row totals are carried
// with row_bcast:15 (into rows 1 and 3) and row_bcast:31 (into rows 2 and 3).
__device__ __forceinline__ float wave_incl_scan(float v) {
  v += dpp0<kDppRowShr1>(v);
  v += dpp0<kDppRowShr2>(v);
  v += dpp0<kDppRowShr4>(v);
  v += dpp0<kDppRowShr8>(v);
  v += dpp0<kDppRowBcast15, 0xa>(v);
  v += dpp0<kDppRowBcast31, 0xc>(v);
  return v;
}

// Four independent inclusive scans (the same operations as wave_incl_scan on each
// value), advanced step by step so that each value's DPP step fills the others' wait
// states instead of four chains running one after another.
__device__ __forceinline__ void wave_incl_scan4(float v[4]) {
#pragma unroll
  for (int j = 0; j < 4; ++j) v[j] += dpp0<kDppRowShr1>(v[j]);
#pragma unroll
  for (int j = 0; j < 4; ++j) v[j] += dpp0<kDppRowShr2>(v[j]);
#pragma unroll
  for (int j = 0; j < 4; ++j) v[j] += dpp0<kDppRowShr4>(v[j]);
#pragma unroll
  for (int j = 0; j < 4; ++j) v[j] += dpp0<kDppRowShr8>(v[j]);
#pragma unroll
  for (int j = 0; j < 4; ++j) v[j] += dpp0<kDppRowBcast15, 0xa>(v[j]);
#pragma unroll
  for (int j = 0; j < 4; ++j) v[j] += dpp0<kDppRowBcast31, 0xc>(v[j]);
}

// Sum over aligned groups of G consecutive lanes (G a power of two <= 64);
// every lane of the group receives the group sum.  Groups up to 16 lanes stay
// inside a DPP row; wider groups use cross-row shuffles.
template <int G>
__device__ __forceinline__ float group_sum(float v) {
  if (G >= 2) v += dpp0<kDppQuadXor1>(v);
  if (G >= 4) v += dpp0<kDppQuadXor2>(v);
  if (G >= 8) v += dpp0<kDppHalfMirror>(v);
  if (G >= 16) v += dpp0<kDppMirror>(v);
  if (G >= 32) v += __shfl_xor(v, 16, 64);
  if (G >= 64) v += __shfl_xor(v, 32, 64);
  return v;
}

}  // namespace m3
