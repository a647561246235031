// The backbone block's elementwise work around the mixer on gfx950:
// SequenceLayer.__call__ (src/base_model/models/layers.py:108-160).
//   block_norm_kernel  flax nn.LayerNorm over d_model (layers.py:121-122, 150-151):
//                      mean and biased variance in float32, (x - mean) *
//                      rsqrt(var + eps) * scale + bias, from the float32 residual
//                      stream to the compute dtype (prenorm: the mixer's input) or
//                      to float32 (postnorm: the residual stream itself).
//   block_gelu_kernel  nn.gelu (tanh form) in the compute dtype: the GLU Dense's
//                      input (layers.py:127-137).
//   block_act_kernel   the activation epilogue and the residual add
//                      (layers.py:126-148): gelu, full_glu, half_glu1 or
//                      half_glu2 from the mixer output y and the Dense outputs,
//                      each product rounded to the compute dtype as a bf16
//                      layer rounds it, then out = skip + that, in float32.
// All three read and write each element once: HBM-bound, one wave per row for
// the norm (its statistics), eight elements per lane for the elementwise pair.
#include "../../include/mamba3_layer.h"
#include "m3_scan.h"

namespace m3 {
namespace {

constexpr int kBlockThreads = 256;

// 0.5 x (1 + tanh(u)) == x * sigmoid(2u): the tanh gelu with one exponential.
// u = sqrt(2/pi) (x + 0.044715 x^3); exp(-2u) -> inf for large negative x gives
// x * rcp(inf) = -0, the gelu's limit.
__device__ __forceinline__ float gelu_tanh(float x) {
  const float u2 = 1.5957691216057308f * fmaf(0.044715f * x * x, x, x);   // 2 sqrt(2/pi) (x + k x^3)
  return x * __builtin_amdgcn_rcpf(1.0f + __expf(-u2));
}

__device__ __forceinline__ float sigmoid_f(float x) { return __builtin_amdgcn_rcpf(1.0f + __expf(-x)); }

template <typename T>
__device__ __forceinline__ float rnd(float x) { return Elem<T>::to_f(Elem<T>::from_f(x)); }

// One wave per row.  The vector path holds the row in registers (D a multiple of 4,
// D <= 64 * 4 * kNormVec, 16-byte rows): one read, two register passes for the
// statistics, one write.  Otherwise the row is read from memory three times.
constexpr int kNormVec = 8;

template <typename T>
__device__ __forceinline__ void load4(const T* p, float f[4]);
template <>
__device__ __forceinline__ void load4<float>(const float* p, float f[4]) {
  const float4 v = *reinterpret_cast<const float4*>(p);
  f[0] = v.x; f[1] = v.y; f[2] = v.z; f[3] = v.w;
}
template <>
__device__ __forceinline__ void load4<bf16>(const bf16* p, float f[4]) {
  const bf16x4 v = *reinterpret_cast<const bf16x4*>(p);
#pragma unroll
  for (int i = 0; i < 4; ++i) f[i] = (float)v[i];
}

template <typename T>
__device__ __forceinline__ void store4(T* p, const float o[4]);
template <>
__device__ __forceinline__ void store4<float>(float* p, const float o[4]) {
  *reinterpret_cast<float4*>(p) = make_float4(o[0], o[1], o[2], o[3]);
}
template <>
__device__ __forceinline__ void store4<bf16>(bf16* p, const float o[4]) {
  bf16x4 v;
#pragma unroll
  for (int i = 0; i < 4; ++i) v[i] = (bf16)o[i];
  *reinterpret_cast<bf16x4*>(p) = v;
}

template <typename T>
__global__ __launch_bounds__(kBlockThreads)
void block_norm_kernel(BlockNormArgs a) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const long row = (long)blockIdx.x * (kBlockThreads / 64) + wave;
  if (row >= a.rows) return;                           // whole waves only: no barrier below
  const int D = a.D;
  const float* x = a.x + row * D;
  T* out = reinterpret_cast<T*>(a.out) + row * D;
  const float inv_d = 1.0f / (float)D;
  if (a.vec) {
    const int n4 = D / 4;
    float4 v[kNormVec];
    float s = 0.0f;
#pragma unroll
    for (int k = 0; k < kNormVec; ++k) {
      const int i = lane + 64 * k;
      v[k] = i < n4 ? reinterpret_cast<const float4*>(x)[i] : make_float4(0, 0, 0, 0);
      s += (v[k].x + v[k].y) + (v[k].z + v[k].w);
    }
    const float mean = group_sum<64>(s) * inv_d;
    float ss = 0.0f;
#pragma unroll
    for (int k = 0; k < kNormVec; ++k) {
      if (lane + 64 * k < n4) {
        const float dx = v[k].x - mean, dy = v[k].y - mean, dz = v[k].z - mean, dw = v[k].w - mean;
        ss += (dx * dx + dy * dy) + (dz * dz + dw * dw);
      }
    }
    const float rs = rsqrtf(group_sum<64>(ss) * inv_d + a.eps);
#pragma unroll
    for (int k = 0; k < kNormVec; ++k) {
      const int i = lane + 64 * k;
      if (i < n4) {
        const float4 sc = reinterpret_cast<const float4*>(a.scale)[i];
        const float4 bi = reinterpret_cast<const float4*>(a.bias)[i];
        const float o[4] = {fmaf((v[k].x - mean) * rs, sc.x, bi.x), fmaf((v[k].y - mean) * rs, sc.y, bi.y),
                            fmaf((v[k].z - mean) * rs, sc.z, bi.z), fmaf((v[k].w - mean) * rs, sc.w, bi.w)};
        store4<T>(out + 4 * i, o);
      }
    }
  } else {
    float s = 0.0f;
    for (int i = lane; i < D; i += 64) s += x[i];
    const float mean = group_sum<64>(s) * inv_d;
    float ss = 0.0f;
    for (int i = lane; i < D; i += 64) ss += (x[i] - mean) * (x[i] - mean);
    const float rs = rsqrtf(group_sum<64>(ss) * inv_d + a.eps);
    for (int i = lane; i < D; i += 64) out[i] = Elem<T>::from_f(fmaf((x[i] - mean) * rs, a.scale[i], a.bias[i]));
  }
}

// Eight elements per lane when n is a multiple of 8 and the arrays are 16-byte
// aligned (a.vec), else one.
template <typename T>
__global__ __launch_bounds__(kBlockThreads)
void block_gelu_kernel(BlockEltArgs a) {
  const long i = (long)blockIdx.x * kBlockThreads + threadIdx.x;
  const T* x = reinterpret_cast<const T*>(a.y);
  T* out = reinterpret_cast<T*>(a.out);
  if (a.vec) {
    if (8 * i >= a.n) return;
    float f[8], o[8];
    Vec8<T> v;
    v.load(x + 8 * i);
    v.to_f(f);
#pragma unroll
    for (int e = 0; e < 8; ++e) o[e] = gelu_tanh(f[e]);
    store8(out + 8 * i, o);
  } else if (i < a.n) {
    out[i] = Elem<T>::from_f(gelu_tanh(Elem<T>::to_f(x[i])));
  }
}

// v = the activation's output rounded to T; out = skip + v (out may be skip).
template <typename T>
__device__ __forceinline__ float block_act(int act, float y, float h1, float h2) {
  switch (act) {
    case M3_ACT_GELU: return rnd<T>(gelu_tanh(y));
    case M3_ACT_FULL_GLU: return rnd<T>(h1 * rnd<T>(sigmoid_f(h2)));
    case M3_ACT_HALF_GLU1: return rnd<T>(rnd<T>(gelu_tanh(y)) * rnd<T>(sigmoid_f(h2)));
    default: return rnd<T>(y * rnd<T>(sigmoid_f(h2)));         // M3_ACT_HALF_GLU2
  }
}

template <typename T>
__global__ __launch_bounds__(kBlockThreads)
void block_act_kernel(BlockEltArgs a) {
  const long i = (long)blockIdx.x * kBlockThreads + threadIdx.x;
  const T* y = reinterpret_cast<const T*>(a.y);
  const T* h1 = reinterpret_cast<const T*>(a.h1);
  const T* h2 = reinterpret_cast<const T*>(a.h2);
  float* out = reinterpret_cast<float*>(a.out);
  const int act = a.act;
  if (a.vec) {
    if (8 * i >= a.n) return;
    float fy[8], f1[8] = {}, f2[8] = {}, sk[8], o[8];
    Vec8<T> v;
    v.load(y + 8 * i);
    v.to_f(fy);
    if (act == M3_ACT_FULL_GLU) {
      v.load(h1 + 8 * i);
      v.to_f(f1);
    }
    if (act != M3_ACT_GELU) {
      v.load(h2 + 8 * i);
      v.to_f(f2);
    }
    Vec8<float> s;
    s.load(a.skip + 8 * i);
    s.to_f(sk);
#pragma unroll
    for (int e = 0; e < 8; ++e) o[e] = sk[e] + block_act<T>(act, fy[e], f1[e], f2[e]);
    store8(out + 8 * i, o);
  } else if (i < a.n) {
    const float f1 = act == M3_ACT_FULL_GLU ? Elem<T>::to_f(h1[i]) : 0.0f;
    const float f2 = act != M3_ACT_GELU ? Elem<T>::to_f(h2[i]) : 0.0f;
    out[i] = a.skip[i] + block_act<T>(act, Elem<T>::to_f(y[i]), f1, f2);
  }
}

// The epilogue and a LayerNorm of its result in one pass, one wave per row:
// s = skip + act (float32, stored to `out` when given), then LayerNorm(s) with
// (scale, bias) to `ln_out` in U.  The vector path (a.vec: D a multiple of 4, at most
// 64 * 4 * kNormVec, 16-byte rows) keeps the row in registers; the scalar path
// re-reads s from out, or recomputes it when out is null, so it needs no scratch.
template <typename T, typename U>
__global__ __launch_bounds__(kBlockThreads)
void block_act_norm_kernel(BlockActNormArgs a) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const long row = (long)blockIdx.x * (kBlockThreads / 64) + wave;
  if (row >= a.rows) return;                           // whole waves only: no barrier below
  const int D = a.D, act = a.act;
  const long base = row * D;
  const T* y = reinterpret_cast<const T*>(a.y) + base;
  const T* h1 = a.h1 ? reinterpret_cast<const T*>(a.h1) + base : nullptr;
  const T* h2 = a.h2 ? reinterpret_cast<const T*>(a.h2) + base : nullptr;
  const float* skip = a.skip + base;
  float* out = a.out ? a.out + base : nullptr;
  U* lo = reinterpret_cast<U*>(a.ln_out) + base;
  const float inv_d = 1.0f / (float)D;
  auto value = [&](int i) {
    const float f1 = act == M3_ACT_FULL_GLU ? Elem<T>::to_f(h1[i]) : 0.0f;
    const float f2 = act != M3_ACT_GELU ? Elem<T>::to_f(h2[i]) : 0.0f;
    return skip[i] + block_act<T>(act, Elem<T>::to_f(y[i]), f1, f2);
  };
  if (a.vec) {
    const int n4 = D / 4;
    float4 v[kNormVec];
    float s = 0.0f;
#pragma unroll
    for (int k = 0; k < kNormVec; ++k) {
      const int i = lane + 64 * k;
      v[k] = make_float4(0, 0, 0, 0);
      if (i < n4) {
        const float4 sk = reinterpret_cast<const float4*>(skip)[i];
        float fy[4], f1[4] = {}, f2[4] = {};
        load4(y + 4 * i, fy);
        if (act == M3_ACT_FULL_GLU) load4(h1 + 4 * i, f1);
        if (act != M3_ACT_GELU) load4(h2 + 4 * i, f2);
        v[k] = make_float4(sk.x + block_act<T>(act, fy[0], f1[0], f2[0]), sk.y + block_act<T>(act, fy[1], f1[1], f2[1]),
                           sk.z + block_act<T>(act, fy[2], f1[2], f2[2]), sk.w + block_act<T>(act, fy[3], f1[3], f2[3]));
        if (out) reinterpret_cast<float4*>(out)[i] = v[k];
      }
      s += (v[k].x + v[k].y) + (v[k].z + v[k].w);
    }
    const float mean = group_sum<64>(s) * inv_d;
    float ss = 0.0f;
#pragma unroll
    for (int k = 0; k < kNormVec; ++k) {
      if (lane + 64 * k < n4) {
        const float dx = v[k].x - mean, dy = v[k].y - mean, dz = v[k].z - mean, dw = v[k].w - mean;
        ss += (dx * dx + dy * dy) + (dz * dz + dw * dw);
      }
    }
    const float rs = rsqrtf(group_sum<64>(ss) * inv_d + a.eps);
#pragma unroll
    for (int k = 0; k < kNormVec; ++k) {
      const int i = lane + 64 * k;
      if (i < n4) {
        const float4 sc = reinterpret_cast<const float4*>(a.scale)[i];
        const float4 bi = reinterpret_cast<const float4*>(a.bias)[i];
        const float o[4] = {fmaf((v[k].x - mean) * rs, sc.x, bi.x), fmaf((v[k].y - mean) * rs, sc.y, bi.y),
                            fmaf((v[k].z - mean) * rs, sc.z, bi.z), fmaf((v[k].w - mean) * rs, sc.w, bi.w)};
        store4<U>(lo + 4 * i, o);
      }
    }
  } else {     // three passes over the row: s is stored to out when given (each lane
               // re-reads only its own elements, also when out is skip), else recomputed
    auto sum_at = [&](int i) { return out ? out[i] : value(i); };
    float s = 0.0f;
    for (int i = lane; i < D; i += 64) {
      const float x = value(i);
      if (out) out[i] = x;
      s += x;
    }
    const float mean = group_sum<64>(s) * inv_d;
    float ss = 0.0f;
    for (int i = lane; i < D; i += 64) {
      const float dx = sum_at(i) - mean;
      ss += dx * dx;
    }
    const float rs = rsqrtf(group_sum<64>(ss) * inv_d + a.eps);
    for (int i = lane; i < D; i += 64) lo[i] = Elem<U>::from_f(fmaf((sum_at(i) - mean) * rs, a.scale[i], a.bias[i]));
  }
}

// log_softmax over each row of V float32 logits, one wave per row: x - max -
// log(sum(exp(x - max))).  The vector path (V a multiple of 4, at most 64 * 4 *
// kSoftmaxVec, 16-byte rows) reads the row once into registers; otherwise three
// passes over memory.  out may be x.
constexpr int kSoftmaxVec = 16;

__global__ __launch_bounds__(kBlockThreads)
void log_softmax_kernel(const float* x, float* out, long rows, int V, int vec) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const long row = (long)blockIdx.x * (kBlockThreads / 64) + wave;
  if (row >= rows) return;                             // whole waves only: no barrier below
  const float* xr = x + row * V;
  float* orow = out + row * V;
  auto wave_max = [](float m) {
    for (int o = 32; o >= 1; o >>= 1) m = fmaxf(m, __shfl_xor(m, o, 64));
    return m;
  };
  if (vec) {
    const int n4 = V / 4;
    float4 v[kSoftmaxVec];
    float m = -INFINITY;
#pragma unroll
    for (int k = 0; k < kSoftmaxVec; ++k) {
      const int i = lane + 64 * k;
      v[k] = i < n4 ? reinterpret_cast<const float4*>(xr)[i] : make_float4(-INFINITY, -INFINITY, -INFINITY, -INFINITY);
      m = fmaxf(m, fmaxf(fmaxf(v[k].x, v[k].y), fmaxf(v[k].z, v[k].w)));
    }
    m = wave_max(m);
    float s = 0.0f;
#pragma unroll
    for (int k = 0; k < kSoftmaxVec; ++k)
      if (lane + 64 * k < n4) s += (expf(v[k].x - m) + expf(v[k].y - m)) + (expf(v[k].z - m) + expf(v[k].w - m));
    const float lse = m + logf(group_sum<64>(s));
#pragma unroll
    for (int k = 0; k < kSoftmaxVec; ++k) {
      const int i = lane + 64 * k;
      if (i < n4) reinterpret_cast<float4*>(orow)[i] = make_float4(v[k].x - lse, v[k].y - lse, v[k].z - lse, v[k].w - lse);
    }
  } else {
    float m = -INFINITY;
    for (int i = lane; i < V; i += 64) m = fmaxf(m, xr[i]);
    m = wave_max(m);
    float s = 0.0f;
    for (int i = lane; i < V; i += 64) s += expf(xr[i] - m);
    const float lse = m + logf(group_sum<64>(s));
    for (int i = lane; i < V; i += 64) orow[i] = xr[i] - lse;
  }
}

inline bool al16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

}  // namespace

hipError_t block_norm_launch(BlockNormArgs a, bool bf16_out, hipStream_t st) {
  a.vec = a.D % 4 == 0 && a.D <= 64 * 4 * kNormVec && al16(a.x) && al16(a.out) && al16(a.scale) && al16(a.bias);
  const dim3 grid((unsigned)((a.rows + kBlockThreads / 64 - 1) / (kBlockThreads / 64)));
  if (bf16_out) hipLaunchKernelGGL(block_norm_kernel<bf16>, grid, dim3(kBlockThreads), 0, st, a);
  else hipLaunchKernelGGL(block_norm_kernel<float>, grid, dim3(kBlockThreads), 0, st, a);
  return hipGetLastError();
}

hipError_t block_act_norm_launch(BlockActNormArgs a, bool bf16_io, bool bf16_ln, hipStream_t st) {
  const size_t es = bf16_io ? 2 : 4;
  a.vec = a.D % 4 == 0 && a.D <= 64 * 4 * kNormVec && (a.D * es) % 8 == 0 && al16(a.skip) && al16(a.scale) &&
          al16(a.bias) && (!a.out || al16(a.out)) && al16(a.ln_out) && al16(a.y) && (!a.h1 || al16(a.h1)) &&
          (!a.h2 || al16(a.h2));
  const dim3 grid((unsigned)((a.rows + kBlockThreads / 64 - 1) / (kBlockThreads / 64)));
  if (bf16_io && bf16_ln) hipLaunchKernelGGL((block_act_norm_kernel<bf16, bf16>), grid, dim3(kBlockThreads), 0, st, a);
  else if (bf16_io) hipLaunchKernelGGL((block_act_norm_kernel<bf16, float>), grid, dim3(kBlockThreads), 0, st, a);
  else if (bf16_ln) hipLaunchKernelGGL((block_act_norm_kernel<float, bf16>), grid, dim3(kBlockThreads), 0, st, a);
  else hipLaunchKernelGGL((block_act_norm_kernel<float, float>), grid, dim3(kBlockThreads), 0, st, a);
  return hipGetLastError();
}

hipError_t log_softmax_launch(const float* x, float* out, long rows, int V, hipStream_t st) {
  const int vec = V % 4 == 0 && V <= 64 * 4 * kSoftmaxVec && al16(x) && al16(out);
  const dim3 grid((unsigned)((rows + kBlockThreads / 64 - 1) / (kBlockThreads / 64)));
  hipLaunchKernelGGL(log_softmax_kernel, grid, dim3(kBlockThreads), 0, st, x, out, rows, V, vec);
  return hipGetLastError();
}

hipError_t block_elt_launch(BlockEltArgs a, bool gelu_only, bool bf16_io, hipStream_t st) {
  a.vec = a.n % 8 == 0 && al16(a.y) && al16(a.out) && (!a.h1 || al16(a.h1)) && (!a.h2 || al16(a.h2)) &&
          (!a.skip || al16(a.skip));
  const long lanes = a.vec ? a.n / 8 : a.n;
  const dim3 grid((unsigned)((lanes + kBlockThreads - 1) / kBlockThreads));
  if (gelu_only) {
    if (bf16_io) hipLaunchKernelGGL(block_gelu_kernel<bf16>, grid, dim3(kBlockThreads), 0, st, a);
    else hipLaunchKernelGGL(block_gelu_kernel<float>, grid, dim3(kBlockThreads), 0, st, a);
  } else {
    if (bf16_io) hipLaunchKernelGGL(block_act_kernel<bf16>, grid, dim3(kBlockThreads), 0, st, a);
    else hipLaunchKernelGGL(block_act_kernel<float>, grid, dim3(kBlockThreads), 0, st, a);
  }
  return hipGetLastError();
}

}  // namespace m3
