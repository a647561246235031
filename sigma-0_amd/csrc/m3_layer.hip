// The Mamba3 mixer layer around the scan: the fused elementwise work between the
// two projections (src/base_model/models/mamba3.py, Mamba3SSM).
//
//   layer_pre_kernel   one projected row per workgroup (mamba3.py:203-268, the
//                      shared-B/C form of _preprocess): split [z, x, B, C, dd_dt,
//                      dd_A, trap, angles]; B and C RMS-normalised over d_state
//                      (statistics in float32, flax RMSNorm eps 1e-6); A =
//                      min(-softplus(dd_A), -A_floor), DT = softplus(dd_dt +
//                      dt_bias), ADT = A DT; Trap and the angle rates as given.
//                      Writes the scan's inputs in its layouts: Q = C, K = B
//                      (B, L, N), V = x, Z = z (B, L, H, P), ADT, DT, Trap (B, H, L)
//                      float32, angle rates (B, L, R) float32.
//   layer_post_kernel  one token per workgroup (mamba3.py:281-331, the norm of
//                      _post_norm_and_project): y * rsqrt(mean(y^2) + eps) *
//                      scale, rounded as the reference rounds it (the rsqrt in
//                      y's dtype, the scaled product in the GEMM's dtype).
// Both are one read and one write of every element: HBM-bound.
#include "m3_scan.h"

namespace m3 {
namespace {

constexpr int kLayerThreads = 256;

template <typename T>
__device__ __forceinline__ void load8v(const T* p, float f[8]) {
  Vec8<T> v;
  v.load(p);
  v.to_f(f);
}

__device__ __forceinline__ float softplus(float x) {      // logaddexp(x, 0), as jax.nn.softplus
  return fmaxf(x, 0.0f) + log1pf(expf(-fabsf(x)));
}

// Copy n elements from src to dst with the lanes of one wave, 16 bytes per lane when
// both rows are 16-byte aligned.
template <typename T>
__device__ __forceinline__ void wave_copy(T* dst, const T* src, int n, int lane) {
  constexpr int V = 16 / sizeof(T);
  if ((reinterpret_cast<uintptr_t>(dst) & 15) == 0 && (reinterpret_cast<uintptr_t>(src) & 15) == 0 && n % V == 0) {
    for (int i = lane; i < n / V; i += 64) reinterpret_cast<uint4*>(dst)[i] = reinterpret_cast<const uint4*>(src)[i];
  } else {
    for (int i = lane; i < n; i += 64) dst[i] = src[i];
  }
}

// A tile of kTileTok consecutive tokens of one batch row per workgroup: the row work
// (copies, BCNorm, angle rates) one wave per token, the per-head values with lanes
// along the tokens so that the (B, H, L) outputs are stored in whole rows.
constexpr int kTileTok = 64;

template <typename T>
__global__ __launch_bounds__(kLayerThreads)
void layer_pre_kernel(LayerPreArgs a) {
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int tiles = (a.L + kTileTok - 1) / kTileTok;
  const int b = blockIdx.x / tiles, l0 = (blockIdx.x % tiles) * kTileTok;
  const int nt = min(kTileTok, a.L - l0);
  const int DI = a.H * a.P, N = a.N, H = a.H, R = a.R;
  const int dproj = 2 * DI + 2 * N + 3 * H + R;
  const T* proj = reinterpret_cast<const T*>(a.proj);
  for (int j = wave; j < nt; j += kLayerThreads / 64) {
    const long tok = (long)b * a.L + l0 + j;
    const T* row = proj + tok * dproj;
    if (a.v) {   // null when the scan reads x and z in place from the projection
      wave_copy(reinterpret_cast<T*>(a.z) + tok * DI, row, DI, lane);
      wave_copy(reinterpret_cast<T*>(a.v) + tok * DI, row + DI, DI, lane);
    }
    // BCNorm over d_state (one scale per matrix, shared over heads)
    float ssb = 0.0f, ssc = 0.0f;
    for (int n = lane; n < N; n += 64) {
      const float xb = Elem<T>::to_f(row[2 * DI + n]), xc = Elem<T>::to_f(row[2 * DI + N + n]);
      ssb += xb * xb;
      ssc += xc * xc;
    }
    ssb = group_sum<64>(ssb);
    ssc = group_sum<64>(ssc);
    const float rb = rsqrtf(ssb / N + a.eps), rc = rsqrtf(ssc / N + a.eps);
    T* kq = reinterpret_cast<T*>(a.k) + tok * N;
    T* qq = reinterpret_cast<T*>(a.q) + tok * N;
    for (int n = lane; n < N; n += 64) {
      kq[n] = Elem<T>::from_f(Elem<T>::to_f(row[2 * DI + n]) * rb * a.b_scale[n]);
      qq[n] = Elem<T>::from_f(Elem<T>::to_f(row[2 * DI + N + n]) * rc * a.c_scale[n]);
    }
    const T* ar = row + 2 * DI + 2 * N + 3 * H;
    for (int r = lane; r < R; r += 64) a.ang[tok * R + r] = Elem<T>::to_f(ar[r]);
  }
  // per-head decay and trapezoid inputs, float32, (B, H, L): lanes along the tokens
  for (int i = tid; i < H * kTileTok; i += kLayerThreads) {
    const int h = i / kTileTok, j = i % kTileTok;
    if (j < nt) {
      const T* hd = proj + ((long)b * a.L + l0 + j) * dproj + 2 * DI + 2 * N;
      const float dt = softplus(Elem<T>::to_f(hd[h]) + a.dt_bias[h]);
      const float A = fminf(-softplus(Elem<T>::to_f(hd[H + h])), -a.A_floor);
      const long o = ((long)b * H + h) * a.L + l0 + j;
      a.dt[o] = dt;
      a.adt[o] = A * dt;
      a.trap[o] = Elem<T>::to_f(hd[2 * H + h]);
    }
  }
}

// One wave per token, four tokens per workgroup.
template <typename T>
__global__ __launch_bounds__(kLayerThreads)
void layer_post_kernel(LayerPostArgs a) {
  constexpr int V = 16 / sizeof(T);
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const long tok = (long)blockIdx.x * (kLayerThreads / 64) + wave;
  if (tok >= (long)a.B * a.L) return;                 // whole waves only: no barrier below
  const int D = a.D;
  const T* y = reinterpret_cast<const T*>(a.y) + tok * D;
  T* out = reinterpret_cast<T*>(a.out) + tok * D;
  const bool vec = D % V == 0 && (reinterpret_cast<uintptr_t>(y) & 15) == 0 &&
                   (reinterpret_cast<uintptr_t>(out) & 15) == 0;
  float ss = 0.0f;
  if (vec && sizeof(T) == 2) {
    for (int i = lane; i < D / 8; i += 64) {
      float f[8];
      load8v(y + 8 * i, f);
#pragma unroll
      for (int e = 0; e < 8; ++e) ss += f[e] * f[e];
    }
  } else {
    for (int i = lane; i < D; i += 64) {
      const float f = Elem<T>::to_f(y[i]);
      ss += f * f;
    }
  }
  ss = group_sum<64>(ss);
  const float ri = Elem<T>::to_f(Elem<T>::from_f(rsqrtf(ss / D + a.eps)));
  if (vec && sizeof(T) == 2) {
    for (int i = lane; i < D / 8; i += 64) {
      float f[8], o[8];
      load8v(y + 8 * i, f);
      const float4 s0 = reinterpret_cast<const float4*>(a.scale + 8 * i)[0];
      const float4 s1 = reinterpret_cast<const float4*>(a.scale + 8 * i)[1];
      const float sc[8] = {s0.x, s0.y, s0.z, s0.w, s1.x, s1.y, s1.z, s1.w};
#pragma unroll
      for (int e = 0; e < 8; ++e) o[e] = Elem<T>::to_f(Elem<T>::from_f(f[e] * ri)) * sc[e];
      store8(out + 8 * i, o);
    }
  } else {
    for (int i = lane; i < D; i += 64) {
      const T yn = Elem<T>::from_f(Elem<T>::to_f(y[i]) * ri);
      out[i] = Elem<T>::from_f(Elem<T>::to_f(yn) * a.scale[i]);
    }
  }
}

}  // namespace

hipError_t layer_pre_launch(const LayerPreArgs& a, bool bf16_io, hipStream_t st) {
  const dim3 grid((unsigned)((long)a.B * ((a.L + kTileTok - 1) / kTileTok)));
  if (bf16_io) hipLaunchKernelGGL(layer_pre_kernel<bf16>, grid, dim3(kLayerThreads), 0, st, a);
  else hipLaunchKernelGGL(layer_pre_kernel<float>, grid, dim3(kLayerThreads), 0, st, a);
  return hipGetLastError();
}

hipError_t layer_post_launch(const LayerPostArgs& a, bool bf16_io, hipStream_t st) {
  const dim3 grid((unsigned)(((long)a.B * a.L + kLayerThreads / 64 - 1) / (kLayerThreads / 64)));
  if (bf16_io) hipLaunchKernelGGL(layer_post_kernel<bf16>, grid, dim3(kLayerThreads), 0, st, a);
  else hipLaunchKernelGGL(layer_post_kernel<float>, grid, dim3(kLayerThreads), 0, st, a);
  return hipGetLastError();
}

}  // namespace m3
