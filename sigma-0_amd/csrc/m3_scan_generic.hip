// Generic Mamba3 SISO prefill: token-by-token recurrent form, any shape.
//
// Serves the shapes the chunked MFMA kernel does not tile (state widths that
// are not multiples of 32, head dims below 32, rope widths that are not a
// power of two, fp32 with d_state > 64).  It evaluates the same causal
// operator as the chunked scan through the decode recurrence (rnn_step,
// src/base_model/models/mamba3.py:498-562; the two forms agree by
// tests/integration/test_backbone_contracts.py:81-111): x = V, B = K, C = Q,
// trap = sigmoid(Trap), the rope angle accumulated token by token and range
// reduced mod 2pi.  One workgroup per (batch, head) keeps the P x N fp32 state
// in LDS.  Chunk size does not change the result and is ignored here.
#include "m3_scan.h"

namespace m3 {

constexpr int kGenThreads = 256;
constexpr int kGenMaxN = 512;
constexpr int kGenMaxP = 512;

template <typename T>
__global__ __launch_bounds__(kGenThreads)
void scan_generic_kernel(ScanArgs a) {
  extern __shared__ float sH[];  // P * N
  __shared__ float sTh[kGenMaxN / 2], sCos[kGenMaxN / 2], sSin[kGenMaxN / 2];
  __shared__ float sQ[kGenMaxN], sK[kGenMaxN], sKp[kGenMaxN];
  __shared__ float sX[kGenMaxP], sVp[kGenMaxP], sY[kGenMaxP];
  __shared__ float sPart[kGenThreads];   // G > 1: row p's partial dot products at p * G + g

  const int tid = threadIdx.x;
  const int bh = blockIdx.x;
  const int b = bh / a.H, h = bh % a.H;
  const int hq = h / (a.H / a.Hqk);
  const int N = a.N, P = a.P, R = a.R, L = a.L, H = a.H, HQ = a.Hqk;
  const T* Q = reinterpret_cast<const T*>(a.q);
  const T* K = reinterpret_cast<const T*>(a.k);
  const T* V = reinterpret_cast<const T*>(a.v);
  const T* Z = reinterpret_cast<const T*>(a.z);
  T* O = reinterpret_cast<T*>(a.out);
  const float* adt = a.adt + (long)bh * L;
  const float* dtp = a.dt + (long)bh * L;
  const float* trp = a.trap + (long)bh * L;
  const float Dh = a.D ? a.D[h] : 0.0f;

  for (int e = tid; e < P * N; e += kGenThreads) sH[e] = a.init_h ? a.init_h[(long)bh * P * N + e] : 0.0f;
  for (int r = tid; r < R; r += kGenThreads) sTh[r] = a.init_theta ? a.init_theta[(long)bh * R + r] : 0.0f;
  for (int n = tid; n < N; n += kGenThreads) sKp[n] = a.init_k ? a.init_k[(long)bh * N + n] : 0.0f;
  for (int p = tid; p < P; p += kGenThreads) sVp[p] = a.init_v ? a.init_v[(long)bh * P + p] : 0.0f;
  __syncthreads();

  // row-slice mapping for the state update: G threads per state row (thread p * G + g
  // takes columns g, g + G, ...).  With G > 1 every row has one pass (P * G <= the
  // block) and its G partial dot products are summed in a fixed order, so the result
  // does not depend on thread timing; with G = 1 a thread owns whole rows.
  int G = kGenThreads / P;
  if (G < 1) G = 1;
  int gpow = 1;
  while (gpow * 2 <= G) gpow *= 2;
  G = gpow;
  const int rows_per_pass = kGenThreads / G;
  const int g = tid % G;

  for (int t = 0; t < L; ++t) {
    const float dtv = dtp[t];
    const float lam = sigmoid_fast(trp[t]);
    const float dec = exp_fast(adt[t]);
    const long tok = (long)b * L + t;
    // A: angle update, biased q/k, x
    for (int r = tid; r < R; r += kGenThreads) {
      const long arow = a.ang_shared ? tok : tok * H + h;      // shared rates: (B, L, R)
      const float th = wrap_2pi(sTh[r] + tanh_fast(a.ang[arow * R + r]) * kPi * dtv);
      sTh[r] = th;
      sincos_wrapped(th, &sCos[r], &sSin[r]);
    }
    for (int n = tid; n < N; n += kGenThreads) {
      sQ[n] = Elem<T>::to_f(Q[(tok * HQ + hq) * N + n]) + a.qbias[(long)h * N + n];
      sK[n] = Elem<T>::to_f(K[(tok * HQ + hq) * N + n]) + a.kbias[(long)h * N + n];
    }
    for (int p = tid; p < P; p += kGenThreads) sX[p] = Elem<T>::to_f(V[(tok * H + h) * P + p]);
    __syncthreads();
    // B: rotate the first R pairs
    for (int j = tid; j < R; j += kGenThreads) {
      const float c = sCos[j], s = sSin[j];
      const float q0 = sQ[2 * j], q1 = sQ[2 * j + 1], k0 = sK[2 * j], k1 = sK[2 * j + 1];
      sQ[2 * j] = q0 * c - q1 * s; sQ[2 * j + 1] = q0 * s + q1 * c;
      sK[2 * j] = k0 * c - k1 * s; sK[2 * j + 1] = k0 * s + k1 * c;
    }
    __syncthreads();
    // C: h = d h + (1-lam) dt d (v_prev (x) k_prev) + lam dt (x (x) k_rot); y = q_rot . h
    const float c_prev = (1.0f - lam) * dtv * dec;
    const float c_cur = lam * dtv;
    for (int p = tid / G; p < P; p += rows_per_pass) {
      const float vp = sVp[p], xp = sX[p];
      float part = 0.0f;
      for (int n = g; n < N; n += G) {
        float v = dec * sH[p * N + n];
        v = v + c_prev * (vp * sKp[n]);
        v = v + c_cur * (xp * sK[n]);
        sH[p * N + n] = v;
        part += sQ[n] * v;
      }
      if (G == 1) sY[p] = part;
      else sPart[tid] = part;
    }
    __syncthreads();
    // D: output, carries
    for (int p = tid; p < P; p += kGenThreads) {
      float acc = 0.0f;
      if (G == 1) acc = sY[p];
      else
        for (int j = 0; j < G; ++j) acc += sPart[p * G + j];
      float y = acc + Dh * sX[p];
      if (Z) y *= silu_fast(Elem<T>::to_f(Z[(tok * H + h) * P + p]));
      O[(tok * H + h) * P + p] = Elem<T>::from_f(y);
      sVp[p] = sX[p];
    }
    for (int n = tid; n < N; n += kGenThreads) sKp[n] = sK[n];
    __syncthreads();
  }

  if (a.fin_h) {
    for (int e = tid; e < P * N; e += kGenThreads) a.fin_h[(long)bh * P * N + e] = sH[e];
    for (int r = tid; r < R; r += kGenThreads) a.fin_theta[(long)bh * R + r] = sTh[r];
    for (int n = tid; n < N; n += kGenThreads) a.fin_k[(long)bh * N + n] = sKp[n];
    for (int p = tid; p < P; p += kGenThreads) a.fin_v[(long)bh * P + p] = sVp[p];
  }
}

bool scan_generic_supported(int N, int P, int R) {
  return N >= 2 && N <= kGenMaxN && (N % 2) == 0 && P >= 1 && P <= kGenMaxP &&
         R >= 0 && 2 * R <= N && (long)P * N * 4 <= 64 * 1024;
}

hipError_t scan_generic_launch(const ScanArgs& a, bool bf16_io, hipStream_t st) {
  const size_t smem = (size_t)a.P * a.N * sizeof(float);
  dim3 grid(a.B * a.H), block(kGenThreads);
  if (bf16_io) {
    hipLaunchKernelGGL(scan_generic_kernel<bf16>, grid, block, smem, st, a);
  } else {
    hipLaunchKernelGGL(scan_generic_kernel<float>, grid, block, smem, st, a);
  }
  return hipGetLastError();
}

}  // namespace m3
