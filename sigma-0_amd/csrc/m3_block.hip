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
//
// Their backward, and that of the per-token head's log_softmax with the tokens'
// negative log-likelihood, as autodiff of the same code gives it, in float32
// arithmetic (the forward's roundings to the compute dtype pass gradients unchanged;
// the rounded values are the operands):
//   block_act_bwd_kernel   from da, the gradient of the block's output (float32, the
//                          residual stream's): with s = sigmoid(h2) rounded as the
//                          forward rounds it, dh2 = da u s (1 - s), u the gated factor
//                          (h1, gelu(y) rounded, y), and dd = da s, the gradient of the
//                          other factor (full_glu: h1; half_glu1: gelu(y); half_glu2:
//                          y); gelu: dd = da gelu'(y), which is dy
//   block_gelu_bwd_kernel  dy = (dg + [half_glu1] dd) gelu'(y) + [half_glu2] dd, with dg
//                          the Dense layers' input gradient (library GEMMs)
//   block_norm_bwd_kernel  LayerNorm's backward from its float32 input x, one wave per
//                          row, kNormBwdRows rows per workgroup: dx = dres + rs (w -
//                          mean(w) - xh mean(w xh)), w = dn scale, xh = (x - mean) rs;
//                          the scale's and bias's gradients (sums of dn xh and dn) as one
//                          partial row per workgroup, its waves' sums added in LDS in
//                          wave order, then summed over the rows in a fixed order
//   nll_kernel             one wave per token (lob_seq_model.py:530-542's log_softmax):
//                          loss = logsumexp(z) - z[target], and in place dz =
//                          (softmax(z) - onehot(target)) w
//
// split3_kernel writes the bfloat16 operands of a float32 product computed as three
// bf16 products with float32 accumulation (the head's decoder Dense and its
// gradients in a bf16 model): hi = bf16(x) rounded to nearest even, lo = bf16(x - hi),
// so that a b = a_hi b_hi + a_hi b_lo + a_lo b_hi up to the omitted a_lo b_lo and the
// rounding of lo (relative 2^-16 per element).  gfx950's matrix cores have no
// reduced-precision float32 type; bf16 runs at 16 times the float32 MFMA rate.
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

// d/dx of gelu_tanh: x s(u2), u2 = 2 sqrt(2/pi) (x + k x^3), gives s + x s (1 - s) u2'
// with u2' = 2 sqrt(2/pi) (1 + 3 k x^2).
__device__ __forceinline__ float gelu_tanh_grad(float x) {
  const float c = 1.5957691216057308f;
  const float s = __builtin_amdgcn_rcpf(1.0f + __expf(-c * fmaf(0.044715f * x * x, x, x)));
  return fmaf(x * s * (1.0f - s), c * fmaf(3.0f * 0.044715f * x, x, 1.0f), s);
}

template <typename T>
__device__ __forceinline__ void act_bwd(int act, float da, float y, float h1, float h2, float& dh2, float& dd) {
  if (act == M3_ACT_GELU) {
    dh2 = 0.0f;
    dd = da * gelu_tanh_grad(y);
    return;
  }
  const float s = rnd<T>(sigmoid_f(h2));
  const float u = act == M3_ACT_FULL_GLU ? h1 : (act == M3_ACT_HALF_GLU1 ? rnd<T>(gelu_tanh(y)) : y);
  dh2 = da * u * (s * (1.0f - s));
  dd = da * s;
}

template <typename T>
__global__ __launch_bounds__(kBlockThreads)
void block_act_bwd_kernel(BlockBwdArgs a) {
  const long i = (long)blockIdx.x * kBlockThreads + threadIdx.x;
  const T* y = reinterpret_cast<const T*>(a.y);
  const T* h1 = reinterpret_cast<const T*>(a.h1);
  const T* h2 = reinterpret_cast<const T*>(a.h2);
  T* dh2 = reinterpret_cast<T*>(a.dh2);
  T* dd = reinterpret_cast<T*>(a.dd);
  const int act = a.act;
  if (a.vec) {
    if (8 * i >= a.n) return;
    float da[8], fy[8], f1[8] = {}, f2[8] = {}, o2[8], od[8];
    Vec8<float> d;
    d.load(a.da + 8 * i);
    d.to_f(da);
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
#pragma unroll
    for (int e = 0; e < 8; ++e) act_bwd<T>(act, da[e], fy[e], f1[e], f2[e], o2[e], od[e]);
    if (act != M3_ACT_GELU) store8(dh2 + 8 * i, o2);
    store8(dd + 8 * i, od);
  } else if (i < a.n) {
    const float f1 = act == M3_ACT_FULL_GLU ? Elem<T>::to_f(h1[i]) : 0.0f;
    const float f2 = act != M3_ACT_GELU ? Elem<T>::to_f(h2[i]) : 0.0f;
    float o2, od;
    act_bwd<T>(act, a.da[i], Elem<T>::to_f(y[i]), f1, f2, o2, od);
    if (act != M3_ACT_GELU) dh2[i] = Elem<T>::from_f(o2);
    dd[i] = Elem<T>::from_f(od);
  }
}

template <typename T>
__global__ __launch_bounds__(kBlockThreads)
void block_gelu_bwd_kernel(BlockBwdArgs a) {
  const long i = (long)blockIdx.x * kBlockThreads + threadIdx.x;
  const T* dg = reinterpret_cast<const T*>(a.dg);
  const T* dd = reinterpret_cast<const T*>(a.dd_in);
  const T* y = reinterpret_cast<const T*>(a.y);
  T* dy = reinterpret_cast<T*>(a.dy);
  const float kg = a.act == M3_ACT_HALF_GLU1 ? 1.0f : 0.0f, ky = a.act == M3_ACT_HALF_GLU2 ? 1.0f : 0.0f;
  const bool use_dd = kg != 0.0f || ky != 0.0f;
  if (a.vec) {
    if (8 * i >= a.n) return;
    float fg[8], fd[8] = {}, fy[8], o[8];
    Vec8<T> v;
    v.load(dg + 8 * i);
    v.to_f(fg);
    if (use_dd) {
      v.load(dd + 8 * i);
      v.to_f(fd);
    }
    v.load(y + 8 * i);
    v.to_f(fy);
#pragma unroll
    for (int e = 0; e < 8; ++e) o[e] = fmaf(fmaf(kg, fd[e], fg[e]), gelu_tanh_grad(fy[e]), ky * fd[e]);
    store8(dy + 8 * i, o);
  } else if (i < a.n) {
    const float fd = use_dd ? Elem<T>::to_f(dd[i]) : 0.0f;
    dy[i] = Elem<T>::from_f(fmaf(fmaf(kg, fd, Elem<T>::to_f(dg[i])), gelu_tanh_grad(Elem<T>::to_f(y[i])), ky * fd));
  }
}

constexpr int kNormBwdRows = 16;          // rows per workgroup, block_norm_bwd

// CH: float4 pieces per lane, ceil(D / 256).  Dynamic LDS: 4 waves x 2 x D floats.
template <typename T, int CH>
__global__ __launch_bounds__(kBlockThreads)
void block_norm_bwd_kernel(BlockNormBwdArgs a) {
  extern __shared__ float red[];              // [wave][2][D]
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int D = a.D, n4 = D / 4;
  const float inv_d = 1.0f / (float)D;
  const long r0 = (long)blockIdx.x * kNormBwdRows;
  const long r1 = r0 + kNormBwdRows < a.rows ? r0 + kNormBwdRows : a.rows;
  float sc[CH][4], as[CH][4], ab[CH][4];
#pragma unroll
  for (int k = 0; k < CH; ++k) {
    const int i = lane + 64 * k;
    const float4 v = i < n4 ? reinterpret_cast<const float4*>(a.scale)[i] : make_float4(0, 0, 0, 0);
    sc[k][0] = v.x; sc[k][1] = v.y; sc[k][2] = v.z; sc[k][3] = v.w;
#pragma unroll
    for (int j = 0; j < 4; ++j) as[k][j] = ab[k][j] = 0.0f;
  }
  for (long r = r0 + wave; r < r1; r += kBlockThreads / 64) {
    const float* xr = a.x + r * D;
    const T* dnr = reinterpret_cast<const T*>(a.dn) + r * D;
    float xv[CH][4], dn[CH][4];
    float s = 0.0f;
#pragma unroll
    for (int k = 0; k < CH; ++k) {
      const int i = lane + 64 * k;
#pragma unroll
      for (int j = 0; j < 4; ++j) xv[k][j] = dn[k][j] = 0.0f;
      if (i < n4) {
        load4<float>(xr + 4 * i, xv[k]);
        load4<T>(dnr + 4 * i, dn[k]);
      }
      s += (xv[k][0] + xv[k][1]) + (xv[k][2] + xv[k][3]);
    }
    const float mean = group_sum<64>(s) * inv_d;
    float ss = 0.0f;
#pragma unroll
    for (int k = 0; k < CH; ++k)
      if (lane + 64 * k < n4)
#pragma unroll
        for (int j = 0; j < 4; ++j) ss += (xv[k][j] - mean) * (xv[k][j] - mean);
    const float rs = rsqrtf(group_sum<64>(ss) * inv_d + a.eps);
    float sw = 0.0f, swx = 0.0f;
#pragma unroll
    for (int k = 0; k < CH; ++k)
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        xv[k][j] = (xv[k][j] - mean) * rs;      // xh (0 past D: dn is 0 there)
        const float w = dn[k][j] * sc[k][j];
        sw += w;
        swx += w * xv[k][j];
        as[k][j] += dn[k][j] * xv[k][j];
        ab[k][j] += dn[k][j];
      }
    sw = group_sum<64>(sw) * inv_d;
    swx = group_sum<64>(swx) * inv_d;
    float* dxr = a.dx + r * D;
#pragma unroll
    for (int k = 0; k < CH; ++k) {
      const int i = lane + 64 * k;
      if (i < n4) {
        float o[4] = {0.0f, 0.0f, 0.0f, 0.0f};
        if (a.dres) load4<float>(a.dres + r * D + 4 * i, o);
#pragma unroll
        for (int j = 0; j < 4; ++j) o[j] += rs * (dn[k][j] * sc[k][j] - sw - xv[k][j] * swx);
        store4<float>(dxr + 4 * i, o);
      }
    }
  }
  // the workgroup's partial row: [scale | bias], the waves' sums added in wave order
#pragma unroll
  for (int k = 0; k < CH; ++k) {
    const int i = lane + 64 * k;
    if (i < n4)
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        red[(2 * wave) * D + 4 * i + j] = as[k][j];
        red[(2 * wave + 1) * D + 4 * i + j] = ab[k][j];
      }
  }
  __syncthreads();
  float* part = a.part + (long)blockIdx.x * 2 * D;
  for (int c = threadIdx.x; c < 2 * D; c += kBlockThreads) {
    const int side = c / D, col = c - side * D;
    part[c] = ((red[side * D + col] + red[(2 + side) * D + col]) + red[(4 + side) * D + col]) +
              red[(6 + side) * D + col];
  }
}

// One wave per row; the vector path (V a multiple of 4, at most 64 * 4 * kSoftmaxVec,
// 16-byte rows) keeps the row in registers, otherwise three passes over memory.
__global__ __launch_bounds__(kBlockThreads)
void nll_kernel(float* z, const int* targets, float* loss, long rows, int V, float w, int vec) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const long row = (long)blockIdx.x * (kBlockThreads / 64) + wave;
  if (row >= rows) return;                             // whole waves only: no barrier below
  float* zr = z + row * V;
  const int t = targets[row];
  const bool ok = t >= 0 && t < V;
  const float zt = ok ? zr[t] : NAN;                   // read before the row is overwritten
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
      v[k] = i < n4 ? reinterpret_cast<const float4*>(zr)[i] : make_float4(-INFINITY, -INFINITY, -INFINITY, -INFINITY);
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
      if (i < n4) {
        float4 o = make_float4(expf(v[k].x - lse) * w, expf(v[k].y - lse) * w, expf(v[k].z - lse) * w,
                               expf(v[k].w - lse) * w);
        if (ok && t / 4 == i) {
          const int j = t % 4;
          if (j == 0) o.x -= w; else if (j == 1) o.y -= w; else if (j == 2) o.z -= w; else o.w -= w;
        }
        reinterpret_cast<float4*>(zr)[i] = o;
      }
    }
    if (lane == 0) loss[row] = lse - zt;
  } else {
    float m = -INFINITY;
    for (int i = lane; i < V; i += 64) m = fmaxf(m, zr[i]);
    m = wave_max(m);
    float s = 0.0f;
    for (int i = lane; i < V; i += 64) s += expf(zr[i] - m);
    const float lse = m + logf(group_sum<64>(s));
    for (int i = lane; i < V; i += 64) zr[i] = expf(zr[i] - lse) * w - (ok && i == t ? w : 0.0f);
    if (lane == 0) loss[row] = lse - zt;
  }
}

inline bool al16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

// hi to a (and b when given), lo to c: rows of K elements at row stride ld; x is
// (rows, K) contiguous.  vec: eight elements per thread (K a multiple of 8, 16-byte
// aligned rows).
__global__ __launch_bounds__(kBlockThreads)
void split3_kernel(const float* x, bf16* a, bf16* b, bf16* c, long rows, int K, long ld, int vec) {
  const long i = (long)blockIdx.x * kBlockThreads + threadIdx.x;
  if (vec) {
    const int kv = K / 8;
    if (i >= rows * kv) return;
    const long r = i / kv;
    const int q = (int)(i - r * kv);
    const float4* src = reinterpret_cast<const float4*>(x + r * K + 8 * q);
    const float4 v0 = src[0], v1 = src[1];
    const float f[8] = {v0.x, v0.y, v0.z, v0.w, v1.x, v1.y, v1.z, v1.w};
    float hi[8], lo[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      hi[e] = (float)(bf16)f[e];
      lo[e] = f[e] - hi[e];
    }
    const long o = r * ld + 8 * q;
    store8(a + o, hi);
    if (b) store8(b + o, hi);
    store8(c + o, lo);
  } else {
    if (i >= rows * K) return;
    const long r = i / K;
    const int k = (int)(i - r * K);
    const float f = x[i];
    const bf16 h = (bf16)f;
    const long o = r * ld + k;
    a[o] = h;
    if (b) b[o] = h;
    c[o] = (bf16)(f - (float)h);
  }
}

}  // namespace

hipError_t split3_launch(const float* x, void* a, void* b, void* c, long rows, int K, long ld, hipStream_t st) {
  const int vec = K % 8 == 0 && ld % 8 == 0 && al16(x) && al16(a) && al16(c) && (!b || al16(b));
  const long work = vec ? rows * (K / 8) : rows * K;
  const dim3 grid((unsigned)((work + kBlockThreads - 1) / kBlockThreads));
  hipLaunchKernelGGL(split3_kernel, grid, dim3(kBlockThreads), 0, st, x, reinterpret_cast<bf16*>(a),
                     reinterpret_cast<bf16*>(b), reinterpret_cast<bf16*>(c), rows, K, ld, vec);
  return hipGetLastError();
}

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

hipError_t block_act_bwd_launch(BlockBwdArgs a, bool bf16_io, hipStream_t st) {
  a.vec = a.n % 8 == 0 && al16(a.da) && al16(a.y) && al16(a.dd) && (!a.h1 || al16(a.h1)) && (!a.h2 || al16(a.h2)) &&
          (!a.dh2 || al16(a.dh2));
  const long lanes = a.vec ? a.n / 8 : a.n;
  const dim3 grid((unsigned)((lanes + kBlockThreads - 1) / kBlockThreads));
  if (bf16_io) hipLaunchKernelGGL(block_act_bwd_kernel<bf16>, grid, dim3(kBlockThreads), 0, st, a);
  else hipLaunchKernelGGL(block_act_bwd_kernel<float>, grid, dim3(kBlockThreads), 0, st, a);
  return hipGetLastError();
}

hipError_t block_gelu_bwd_launch(BlockBwdArgs a, bool bf16_io, hipStream_t st) {
  a.vec = a.n % 8 == 0 && al16(a.dg) && al16(a.y) && al16(a.dy) && (!a.dd_in || al16(a.dd_in));
  const long lanes = a.vec ? a.n / 8 : a.n;
  const dim3 grid((unsigned)((lanes + kBlockThreads - 1) / kBlockThreads));
  if (bf16_io) hipLaunchKernelGGL(block_gelu_bwd_kernel<bf16>, grid, dim3(kBlockThreads), 0, st, a);
  else hipLaunchKernelGGL(block_gelu_bwd_kernel<float>, grid, dim3(kBlockThreads), 0, st, a);
  return hipGetLastError();
}

long block_norm_bwd_parts(long rows) { return (rows + kNormBwdRows - 1) / kNormBwdRows + kReduceSlices; }

hipError_t block_norm_bwd_launch(const BlockNormBwdArgs& a, float* dscale, float* dbias, bool bf16_io,
                                 hipStream_t st) {
  const long blocks = block_norm_bwd_parts(a.rows) - kReduceSlices;
  const int ch = (a.D / 4 + 63) / 64;
  const size_t lds = (size_t)(kBlockThreads / 64) * 2 * a.D * sizeof(float);
#define M3_NORM_BWD(CH)                                                                                            \
  if (ch == CH) {                                                                                                  \
    if (bf16_io) hipLaunchKernelGGL((block_norm_bwd_kernel<bf16, CH>), dim3((unsigned)blocks), dim3(kBlockThreads), \
                                    lds, st, a);                                                                   \
    else hipLaunchKernelGGL((block_norm_bwd_kernel<float, CH>), dim3((unsigned)blocks), dim3(kBlockThreads), lds,  \
                            st, a);                                                                                \
  }
  M3_NORM_BWD(1) M3_NORM_BWD(2) M3_NORM_BWD(3) M3_NORM_BWD(4)
  M3_NORM_BWD(5) M3_NORM_BWD(6) M3_NORM_BWD(7) M3_NORM_BWD(8)
#undef M3_NORM_BWD
  static_assert(kBlockNormBwdMaxD == 64 * 4 * 8, "block_norm_bwd instantiations");
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  return reduce_rows(a.part, blocks, 2 * a.D, a.part + blocks * 2 * a.D, dscale, a.D, dbias, a.D, nullptr, st);
}

hipError_t nll_launch(float* z, const int* targets, float* loss, long rows, int V, float w, hipStream_t st) {
  const int vec = V % 4 == 0 && V <= 64 * 4 * kSoftmaxVec && al16(z);
  const dim3 grid((unsigned)((rows + kBlockThreads / 64 - 1) / (kBlockThreads / 64)));
  hipLaunchKernelGGL(nll_kernel, grid, dim3(kBlockThreads), 0, st, z, targets, loss, rows, V, w, vec);
  return hipGetLastError();
}

}  // namespace m3
