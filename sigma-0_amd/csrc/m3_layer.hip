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

// A tile of up to 64 consecutive tokens of one batch row per workgroup (a.tile, a
// power of two chosen so the staging fits in LDS).  The workgroup first stages the
// tile's [B, C, dd_dt, dd_A, trap, angles] segments and the two norm scales into LDS,
// with every load issued before any is used (16-byte chunks when the rows allow).
// Then one wave per token normalises B and C and stores the angle rates, and lanes
// along the tokens compute the per-head decay, so that the (B, H, L) outputs are
// stored in whole rows.  Only the copies of z and x (the fallback route) read proj
// directly.
constexpr int kStageUnroll = 12;

template <typename T>
__global__ __launch_bounds__(kLayerThreads)
void layer_pre_kernel(LayerPreArgs a) {
  extern __shared__ __align__(16) unsigned char pre_smem[];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int TT = a.tile;
  const int tiles = (a.L + TT - 1) / TT;
  const int b = blockIdx.x / tiles, l0 = (blockIdx.x % tiles) * TT;
  const int nt = min(TT, a.L - l0);
  const int DI = a.H * a.P, N = a.N, H = a.H, R = a.R;
  const int seg = 2 * N + 3 * H + R;                   // staged elements per token
  const int dproj = 2 * DI + seg;
  const T* proj = reinterpret_cast<const T*>(a.proj);
  const long tok0 = (long)b * a.L + l0;
  const T* src0 = proj + tok0 * dproj + 2 * DI;         // the tile's first segment
  T* sseg = reinterpret_cast<T*>(pre_smem);             // [TT][seg]
  float* sscale = reinterpret_cast<float*>(pre_smem + (((size_t)TT * seg * sizeof(T) + 15) & ~(size_t)15));  // [2][N]

  if (a.vec) {    // rows, the segment offset and its length are multiples of 16 bytes
    constexpr int E = 16 / sizeof(T);
    const int cpt = seg / E, total = nt * cpt;
    const float rcpt = 1.0f / (float)cpt;
    for (int i0 = tid; i0 < total; i0 += kLayerThreads * kStageUnroll) {
      uint4 r[kStageUnroll];
#pragma unroll
      for (int u = 0; u < kStageUnroll; ++u) {
        const int i = i0 + u * kLayerThreads;
        // j = i / cpt without an integer division: i < 2^24, so the float quotient is
        // off by at most one, and the remainder's sign or size corrects it
        int j = (int)((float)i * rcpt), c = i - j * cpt;
        if (c < 0) { --j; c += cpt; }
        else if (c >= cpt) { ++j; c -= cpt; }
        r[u] = i < total ? *reinterpret_cast<const uint4*>(src0 + (long)j * dproj + c * E) : make_uint4(0, 0, 0, 0);
      }
#pragma unroll
      for (int u = 0; u < kStageUnroll; ++u) {
        const int i = i0 + u * kLayerThreads;
        if (i < total) reinterpret_cast<uint4*>(sseg)[i] = r[u];      // element j * seg + c * E
      }
    }
  } else {
    const int total = nt * seg;
    for (int i = tid; i < total; i += kLayerThreads) {
      const int j = i / seg, e = i - j * seg;
      sseg[i] = src0[(long)j * dproj + e];
    }
  }
  for (int n = tid; n < N; n += kLayerThreads) {
    sscale[n] = a.b_scale[n];
    sscale[N + n] = a.c_scale[n];
  }
  __syncthreads();

  for (int j = wave; j < nt; j += kLayerThreads / 64) {
    const long tok = tok0 + j;
    if (a.v) {   // null when the scan reads x and z in place from the projection
      const T* row = proj + tok * dproj;
      wave_copy(reinterpret_cast<T*>(a.z) + tok * DI, row, DI, lane);
      wave_copy(reinterpret_cast<T*>(a.v) + tok * DI, row + DI, DI, lane);
    }
    const T* s = sseg + j * seg;
    // BCNorm over d_state (one scale per matrix, shared over heads)
    float ssb = 0.0f, ssc = 0.0f;
    for (int n = lane; n < N; n += 64) {
      const float xb = Elem<T>::to_f(s[n]), xc = Elem<T>::to_f(s[N + n]);
      ssb += xb * xb;
      ssc += xc * xc;
    }
    ssb = group_sum<64>(ssb);
    ssc = group_sum<64>(ssc);
    const float rb = rsqrtf(ssb / N + a.eps), rc = rsqrtf(ssc / N + a.eps);
    T* kq = reinterpret_cast<T*>(a.k) + tok * N;
    T* qq = reinterpret_cast<T*>(a.q) + tok * N;
    for (int n = lane; n < N; n += 64) {
      kq[n] = Elem<T>::from_f(Elem<T>::to_f(s[n]) * rb * sscale[n]);
      qq[n] = Elem<T>::from_f(Elem<T>::to_f(s[N + n]) * rc * sscale[N + n]);
    }
    for (int r = lane; r < R; r += 64) a.ang[tok * R + r] = Elem<T>::to_f(s[2 * N + 3 * H + r]);
  }
  // per-head decay and trapezoid inputs, float32, (B, H, L): lanes along the tokens
  const int tt_shift = __builtin_ctz(TT);               // TT is a power of two
  for (int i = tid; i < H * TT; i += kLayerThreads) {
    const int h = i >> tt_shift, j = i & (TT - 1);
    if (j < nt) {
      const T* hd = sseg + j * seg + 2 * N;
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
                   (reinterpret_cast<uintptr_t>(out) & 15) == 0 && (reinterpret_cast<uintptr_t>(a.scale) & 15) == 0;
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

// LDS bytes of a tile of `tile` tokens (the layout of layer_pre_kernel).
size_t layer_pre_lds_bytes(int tile, int seg, int N, size_t es) {
  return (((size_t)tile * seg * es + 15) & ~(size_t)15) + 2 * (size_t)N * sizeof(float);
}

hipError_t layer_pre_launch(LayerPreArgs a, bool bf16_io, hipStream_t st) {
  const size_t es = bf16_io ? 2 : 4;
  const int seg = 2 * a.N + 3 * a.H + a.R;
  const long dproj = 2L * a.H * a.P + seg;
  a.tile = 64;
  while (a.tile > 1 && layer_pre_lds_bytes(a.tile, seg, a.N, es) > (size_t)kLayerPreLds) a.tile /= 2;
  if (layer_pre_lds_bytes(a.tile, seg, a.N, es) > (size_t)kLayerPreLds) return hipErrorInvalidValue;
  a.vec = (dproj * es) % 16 == 0 && (2L * a.H * a.P * es) % 16 == 0 && (seg * es) % 16 == 0 &&
          (reinterpret_cast<uintptr_t>(a.proj) & 15) == 0;
  const dim3 grid((unsigned)((long)a.B * ((a.L + a.tile - 1) / a.tile)));
  const size_t lds = layer_pre_lds_bytes(a.tile, seg, a.N, es);
  if (bf16_io) hipLaunchKernelGGL(layer_pre_kernel<bf16>, grid, dim3(kLayerThreads), lds, st, a);
  else hipLaunchKernelGGL(layer_pre_kernel<float>, grid, dim3(kLayerThreads), lds, st, a);
  return hipGetLastError();
}

hipError_t layer_post_launch(const LayerPostArgs& a, bool bf16_io, hipStream_t st) {
  const dim3 grid((unsigned)(((long)a.B * a.L + kLayerThreads / 64 - 1) / (kLayerThreads / 64)));
  if (bf16_io) hipLaunchKernelGGL(layer_post_kernel<bf16>, grid, dim3(kLayerThreads), 0, st, a);
  else hipLaunchKernelGGL(layer_post_kernel<float>, grid, dim3(kLayerThreads), 0, st, a);
  return hipGetLastError();
}

}  // namespace m3
