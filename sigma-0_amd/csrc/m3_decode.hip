// Single-token Mamba3 decode state update (bandwidth-bound).
//
// Restates the recurrence of rnn_step, src/base_model/models/mamba3.py:498-562,
// for a whole batch at once (the model vmaps it over batch,
// lob_seq_model.py:747-751):
//   theta += tanh(angle_t) * pi * dt_t            (wrapped mod 2pi by default)
//   B_rot  = rope(B_t + B_bias, theta)   C_rot = rope(C_t + C_bias, theta)
//   h      = d h + (1 - trap) dt d (v_prev (x) k_prev) + trap dt (x_t (x) B_rot),  d = e^{adt}
//   y      = (C_rot . h + D x_t [+ gamma (C_rot . B_rot) x_t]) * silu(z_t)
//   carry <- (theta, h, B_rot, x_t)
//
// Layout in HBM (all row-major, contiguous): theta (B,H,R) f32, h (B,H,P,N) f32,
// k_prev (B,H,N) f32, v_prev (B,H,P) f32, x/z (B,H,P), B_t/C_t (B,H,N) in the
// input dtype, adt/dt/trap (B,H) f32 with trap post-sigmoid, angle (B,H,R) f32,
// B_bias/C_bias (H,N) f32, D (H,) f32, y (B,H,P) in the output dtype.
//
// One 512-thread workgroup per (b, h).  The P*N fp32 state is streamed as
// float4 with consecutive threads on consecutive 16-byte words, so each wave
// reads and writes whole 1 KiB spans, with non-temporal loads and stores (the
// state is touched once per step and is larger than the caches); those loads are
// issued before the small per-head preamble (angles, rope, carries) so HBM
// latency overlaps it.  The output dot C_rot . h reduces over the N/4 lanes
// holding one state row.
//
// The mixer layer's decode (LAYER: m3_layer_decode_step) runs the same update with
// the step inputs formed from the token's in_proj row, as m3_layer_pre forms them for
// the scan (mamba3.py:203-268, the shared-B/C form of _preprocess): z and x are the
// head's columns, B and C are RMS-normalised over d_state (waves 0 and 1, the sums in
// m3_layer_pre's order) and rounded to the I/O type, dt = softplus(dd_dt + dt_bias),
// A = min(-softplus(dd_A), -A_floor), trap = sigmoid(trap field), and the angle rates
// are the row's, shared by the heads.  One launch then replaces m3_layer_pre and the
// per-head copies of B, C and the rates that the decode contract takes.
#include "m3_scan.h"

namespace m3 {



template <typename T>
__device__ __forceinline__ float ld_f(const void* p, long i) {
  return Elem<T>::to_f(reinterpret_cast<const T*>(p)[i]);
}

__device__ __forceinline__ float softplus_f(float x) {      // logaddexp(x, 0), as jax.nn.softplus
  return fmaxf(x, 0.0f) + log1pf(expf(-fabsf(x)));
}

constexpr int kDecThreads = 512;
constexpr int kDecMaxP = 256;
constexpr int kDecMaxN = 256;

// ROWL = N/4 lanes per state row (a power of two <= 64); MAXV = ceil(P*N/4/256)
// float4 words per thread for the largest P*N this instantiation serves.
template <typename TI, typename TO, int ROWL, int MAXV, bool LAYER>
__global__ __launch_bounds__(kDecThreads)
void decode_step_kernel(DecodeArgs a) {
  const int tid = threadIdx.x;
  const int bh = blockIdx.x;
  const int hh = bh % a.H;
  const int N = a.N, P = a.P, R = a.R;
  const int nvec = P * N / 4;

  __shared__ float sCos[kDecMaxN / 2], sSin[kDecMaxN / 2];
  __shared__ float sB[kDecMaxN], sKp[kDecMaxN], sC[kDecMaxN];
  __shared__ float sX[kDecMaxP], sVp[kDecMaxP], sY[kDecMaxP];
  __shared__ float sQK[kDecThreads / 64];   // legacy_double: per-wave sums of the QK dot
  __shared__ float sScal[3];                // LAYER: the head's dt, decay and trap (wave 2)

  // 1. issue the state loads first
  f32x4* hrow = reinterpret_cast<f32x4*>(a.h + (long)bh * P * N);
  f32x4 hv[MAXV];
#pragma unroll
  for (int i = 0; i < MAXV; ++i) {
    const int v = tid + i * kDecThreads;
    if (v < nvec) hv[i] = __builtin_nontemporal_load(hrow + v);
  }

  // 2. preamble: carries and step inputs into LDS, angle update
  const long bhN = (long)bh * N, bhP = (long)bh * P, bhR = (long)bh * R;
  float dtv = 0.0f, trv = 0.0f, dec = 0.0f;
  // theta += tanh(rate) pi dt, wrapped; its cos and sin for the rope of step 3
  auto angle = [&](int r, float rate) {
    float th = a.theta[bhR + r] + tanh_fast(rate) * kPi * dtv;
    if (a.wrapped) th = wrap_2pi(th);
    a.theta[bhR + r] = th;
    float c, s;
    if (a.wrapped) {
      sincos_wrapped(th, &c, &s);
    } else {
      c = cosf(th);
      s = sinf(th);
    }
    sCos[r] = c;
    sSin[r] = s;
  };
  // LAYER: the token's projection row [z | x | B | C | dd_dt | dd_A | trap | rates]
  const TI* row = nullptr;
  long ox = 0, oz = 0, oang = 0;          // offsets of x_h, z_h and the rates in row
  if constexpr (LAYER) {
    const int H = a.H, DI = H * P;
    row = reinterpret_cast<const TI*>(a.proj) + (long)(bh / H) * (2L * DI + 2 * N + 3 * H + R);
    oz = (long)hh * P;
    ox = DI + oz;
    oang = 2L * DI + 2 * N + 3 * H;
    const int wave = tid >> 6, lane = tid & 63;
    if (wave == 2) {   // the head's scalars (the other waves read them after the barrier), angles
      const TI* hd = row + 2L * DI + 2 * N;
      dtv = softplus_f(Elem<TI>::to_f(hd[hh]) + a.dt_bias[hh]);
      const float A = fminf(-softplus_f(Elem<TI>::to_f(hd[H + hh])), -a.A_floor);
      dec = exp_fast(A * dtv);
      trv = 1.0f / (1.0f + expf(-Elem<TI>::to_f(hd[2 * H + hh])));
      if (lane == 0) {
        sScal[0] = dtv;
        sScal[1] = dec;
        sScal[2] = trv;
      }
      for (int r = lane; r < R; r += 64) angle(r, Elem<TI>::to_f(row[oang + r]));
    } else if (wave < 2) {   // BCNorm: wave 0 B (the key), wave 1 C (the query); N <= 256
      const TI* src = row + 2L * DI + wave * N;
      const float* sc = wave ? a.c_scale : a.b_scale;
      float xv[kDecMaxN / 64], scv[kDecMaxN / 64];
#pragma unroll
      for (int i = 0; i < kDecMaxN / 64; ++i) {     // one round of loads, kept in registers
        const int n = lane + 64 * i;
        xv[i] = n < N ? Elem<TI>::to_f(src[n]) : 0.0f;
        scv[i] = n < N ? sc[n] : 0.0f;
      }
      float ss = 0.0f;
#pragma unroll
      for (int i = 0; i < kDecMaxN / 64; ++i) ss += xv[i] * xv[i];
      ss = group_sum<64>(ss);
      const float rn = rsqrtf(ss / N + a.eps);
      float* dst = wave ? sC : sB;
#pragma unroll
      for (int i = 0; i < kDecMaxN / 64; ++i) {
        const int n = lane + 64 * i;
        if (n < N) dst[n] = Elem<TI>::to_f(Elem<TI>::from_f(xv[i] * rn * scv[i]));
      }
    }
  } else {
    dtv = a.dt[bh];
    trv = a.trap[bh];
    dec = exp_fast(a.adt[bh]);
  }
  for (int n = tid; n < N; n += kDecThreads) sKp[n] = a.kprev[bhN + n];
  for (int p = tid; p < P; p += kDecThreads) {
    sVp[p] = a.vprev[bhP + p];
    sX[p] = LAYER ? Elem<TI>::to_f(row[ox + p]) : ld_f<TI>(a.x, bhP + p);
  }
  if constexpr (!LAYER) {
    for (int r = tid; r < R; r += kDecThreads) angle(r, a.ang[bhR + r]);
  }
  // step 3's global inputs, requested before the barrier (none depends on step 2):
  // thread j < N/2 owns the pair (2j, 2j + 1); N/2 <= 128 < kDecThreads
  const int j = tid, n0 = 2 * j;
  const bool own = j < N / 2;
  float bb0 = 0.0f, bb1 = 0.0f, cb0 = 0.0f, cb1 = 0.0f, bt0 = 0.0f, bt1 = 0.0f, ct0 = 0.0f, ct1 = 0.0f;
  if (own) {
    bb0 = a.bbias[(long)hh * N + n0];
    bb1 = a.bbias[(long)hh * N + n0 + 1];
    cb0 = a.cbias[(long)hh * N + n0];
    cb1 = a.cbias[(long)hh * N + n0 + 1];
    if constexpr (!LAYER) {
      bt0 = ld_f<TI>(a.bt, bhN + n0);
      bt1 = ld_f<TI>(a.bt, bhN + n0 + 1);
      ct0 = ld_f<TI>(a.ct, bhN + n0);
      ct1 = ld_f<TI>(a.ct, bhN + n0 + 1);
    }
  }
  __syncthreads();
  if constexpr (LAYER) {
    dtv = sScal[0];
    dec = sScal[1];
    trv = sScal[2];
  }

  // 3. rotated key/query for this step; new carries
  float qk_part = 0.0f;
  if (own) {
    // LAYER: the normalised B and C are in sB / sC (this thread's two entries)
    float b0 = (LAYER ? sB[n0] : bt0) + bb0;
    float b1 = (LAYER ? sB[n0 + 1] : bt1) + bb1;
    float c0 = (LAYER ? sC[n0] : ct0) + cb0;
    float c1 = (LAYER ? sC[n0 + 1] : ct1) + cb1;
    if (j < R) {
      const float cs = sCos[j], sn = sSin[j];
      float t0 = b0 * cs - b1 * sn, t1 = b0 * sn + b1 * cs;
      b0 = t0; b1 = t1;
      t0 = c0 * cs - c1 * sn; t1 = c0 * sn + c1 * cs;
      c0 = t0; c1 = t1;
    }
    sB[n0] = b0; sB[n0 + 1] = b1;
    sC[n0] = c0; sC[n0 + 1] = c1;
    a.kprev[bhN + n0] = b0;
    a.kprev[bhN + n0 + 1] = b1;
    qk_part += c0 * b0 + c1 * b1;
  }
  if (a.legacy_double) {
    // butterfly sum within the wave, then the waves' sums in order: deterministic
    for (int o = 32; o > 0; o >>= 1) qk_part += __shfl_xor(qk_part, o);
    if ((tid & 63) == 0) sQK[tid >> 6] = qk_part;
  }
  for (int p = tid; p < P; p += kDecThreads) a.vprev[bhP + p] = sX[p];
  __syncthreads();

  // 4. state update + output partial dot over n
  const float c_prev = (1.0f - trv) * dtv * dec;   // (1 - trap) * dt * decay
  const float c_cur = trv * dtv;                   // trap * dt
#pragma unroll
  for (int i = 0; i < MAXV; ++i) {
    const int v = tid + i * kDecThreads;
    float part = 0.0f;
    int p = 0;
    if (v < nvec) {
      p = v / ROWL;
      const int n = (v % ROWL) * 4;
      const float vp = sVp[p], xp = sX[p];
      f32x4 hn = hv[i];
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        float t = dec * hn[q];
        t = t + c_prev * (vp * sKp[n + q]);
        t = t + c_cur * (xp * sB[n + q]);
        hn[q] = t;
        part += sC[n + q] * t;
      }
      __builtin_nontemporal_store(hn, hrow + v);
    }
    part = group_sum<ROWL>(part);
    if (v < nvec && (v % ROWL) == 0) sY[p] = part;
  }
  __syncthreads();

  // 5. output
  const float Dh = a.D ? a.D[hh] : 0.0f;
  float qk = 0.0f;
  if (a.legacy_double) {
    for (int w = 0; w < kDecThreads / 64; ++w) qk += sQK[w];
    qk *= dtv * trv;
  }
  for (int p = tid; p < P; p += kDecThreads) {
    float yv = sY[p] + Dh * sX[p];
    if (a.legacy_double) yv += qk * sX[p];
    if (LAYER) yv *= silu_fast(Elem<TI>::to_f(row[oz + p]));
    else if (a.z) yv *= silu_fast(ld_f<TI>(a.z, bhP + p));
    reinterpret_cast<TO*>(a.y)[bhP + p] = Elem<TO>::from_f(yv);
  }
}

template <typename TI, typename TO, int ROWL, bool LAYER>
static hipError_t launch_rowl(const DecodeArgs& a, hipStream_t st) {
  const int nvec = a.P * a.N / 4;
  const int per = (nvec + kDecThreads - 1) / kDecThreads;
  dim3 grid(a.B * a.H), block(kDecThreads);
  if (per <= 1) {
    hipLaunchKernelGGL((decode_step_kernel<TI, TO, ROWL, 1, LAYER>), grid, block, 0, st, a);
  } else if (per <= 2) {
    hipLaunchKernelGGL((decode_step_kernel<TI, TO, ROWL, 2, LAYER>), grid, block, 0, st, a);
  } else if (per <= 4) {
    hipLaunchKernelGGL((decode_step_kernel<TI, TO, ROWL, 4, LAYER>), grid, block, 0, st, a);
  } else if (per <= 8) {
    hipLaunchKernelGGL((decode_step_kernel<TI, TO, ROWL, 8, LAYER>), grid, block, 0, st, a);
  } else if (per <= 16) {
    hipLaunchKernelGGL((decode_step_kernel<TI, TO, ROWL, 16, LAYER>), grid, block, 0, st, a);
  } else {
    return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

template <typename TI, typename TO, bool LAYER = false>
static hipError_t launch_types(const DecodeArgs& a, hipStream_t st) {
  switch (a.N / 4) {
    case 1: return launch_rowl<TI, TO, 1, LAYER>(a, st);
    case 2: return launch_rowl<TI, TO, 2, LAYER>(a, st);
    case 4: return launch_rowl<TI, TO, 4, LAYER>(a, st);
    case 8: return launch_rowl<TI, TO, 8, LAYER>(a, st);
    case 16: return launch_rowl<TI, TO, 16, LAYER>(a, st);
    case 32: return launch_rowl<TI, TO, 32, LAYER>(a, st);
    case 64: return launch_rowl<TI, TO, 64, LAYER>(a, st);
    default: return hipErrorInvalidValue;
  }
}

hipError_t decode_step_launch(const DecodeArgs& a, bool in_bf16, bool out_bf16, hipStream_t st) {
  if (a.proj) {   // the layer's decode: one I/O type
    if (in_bf16 != out_bf16) return hipErrorInvalidValue;
    return in_bf16 ? launch_types<bf16, bf16, true>(a, st) : launch_types<float, float, true>(a, st);
  }
  if (in_bf16) {
    return out_bf16 ? launch_types<bf16, bf16>(a, st) : launch_types<bf16, float>(a, st);
  }
  return out_bf16 ? launch_types<float, bf16>(a, st) : launch_types<float, float>(a, st);
}

}  // namespace m3
