// Chunked Mamba3 SISO prefill scan on CDNA4 matrix cores.
//
// Computes the reference's mamba3_ssd_chunked_jax (phases 1-7,
// src/base_model/models/mamba3_jax.py:327-419) in one kernel:
//   phase 1  per-chunk decay prefix (wave64 scan), rotation-angle prefix
//            (wave64 scans over the chunk, carried across chunks and range
//            reduced mod 2pi), trapezoid weights, biases, QK-dot skip, rope,
//            key scaling                                        (:236-324)
//   phase 3  S^T = K_s Q_r^T on MFMA, causal decay mask in registers, then
//            Y_diag = M V on MFMA straight from the S^T accumulators (:371-393)
//   phase 4-6 Y_off = e^{A_cum} (Q_r h^T) on MFMA; h <- e^{A_end} h +
//            (K_s w)^T V on MFMA, h kept in fp32 accumulators      (:177-233)
//   phase 7  (Y_diag + Y_off + (D + QK) V) * silu(Z), 16-byte stores (:402-419)
//
// One workgroup (4 waves) per (batch, head) walks the chunks in order; the
// P x N fp32 state never leaves the CU.  While a chunk's matrix work runs,
// the next chunk's inputs are already in flight into registers, so every
// input byte is read from HBM exactly once and the output written once.
//
// MFMA tile conventions (32x32, verified lane layouts):
//   A (32 x K): lane i holds row i%32, k = (i/32)*KPL + [0, KPL)
//   B (K x 32): lane i holds col i%32, k = (i/32)*KPL + [0, KPL)
//   C (32x32):  lane i, reg r holds col i%32, row 8*(r/4) + 4*(i/32) + r%4
// bf16: v_mfma_f32_32x32x16_bf16 (KPL = 8); fp32: v_mfma_f32_32x32x2_f32 (KPL = 1).
// The S^T accumulator is reused as the A operand of M V by permuting the
// contraction index consistently in the V operand (fragVperm).
#include <type_traits>

#include "m3_scan.h"

namespace m3 {

template <typename T> struct MF;
template <> struct MF<bf16> {
  static constexpr int KSTEP = 16, KPL = 8, PAD = 8;
  typedef bf16x8 frag;
  __device__ __forceinline__ static f32x16 mma(frag a, frag b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
  }
  // row (row0 + lane%32), KPL contiguous elements at column k0 + (lane/32)*KPL
  __device__ __forceinline__ static frag ld(const bf16* buf, int ldm, int row0, int k0, int lane) {
    return *reinterpret_cast<const bf16x8*>(buf + (row0 + (lane & 31)) * ldm + k0 + (lane >> 5) * 8);
  }
  // k-step j of the S^T C tile as an A operand: C regs 8j .. 8j+7
  __device__ __forceinline__ static frag from_acc(const f32x16& c, int j) {
    frag f;
#pragma unroll
    for (int q = 0; q < 8; ++q) f[q] = (bf16)c[8 * j + q];
    return f;
  }
  // V operand matching from_acc's contraction order: row p of Vt holds V[:, p];
  // slots 0..3 <-> s = 16j + 4(lane/32) + 0..3, slots 4..7 <-> s + 8
  __device__ __forceinline__ static frag vperm(const bf16* vt, int ldv, int p0, int s0, int j, int lane) {
    const bf16* r = vt + (p0 + (lane & 31)) * ldv + s0 + 16 * j + 4 * (lane >> 5);
    const bf16x4 lo = *reinterpret_cast<const bf16x4*>(r);
    const bf16x4 hi = *reinterpret_cast<const bf16x4*>(r + 8);
    frag f;
    f[0] = lo[0]; f[1] = lo[1]; f[2] = lo[2]; f[3] = lo[3];
    f[4] = hi[0]; f[5] = hi[1]; f[6] = hi[2]; f[7] = hi[3];
    return f;
  }
  // A operand K^T: row n = n0 + lane%32, k = s = s0 + 8(lane/32) + q, read from row-major K[s][n]
  __device__ __forceinline__ static frag kt(const bf16* k, int ldk, int n0, int s0, int lane) {
    const bf16* c = k + (s0 + 8 * (lane >> 5)) * ldk + n0 + (lane & 31);
    frag f;
#pragma unroll
    for (int q = 0; q < 8; ++q) f[q] = c[q * ldk];
    return f;
  }
  // B operand w-scaled V for the state update: precomputed V^T * w in vwt
  __device__ __forceinline__ static frag vw(const bf16* vwt, const bf16*, const float*, int ldv, int p0, int s0, int lane) {
    return ld(vwt, ldv, p0, s0, lane);
  }
  // write rows n0 + 8g + 4(lane/32) + 0..3 of column p of a C tile into hb[p][n]
  __device__ __forceinline__ static void store_ht(bf16* hb, int ldh, int p, int n0, const f32x16& c, int lane) {
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      bf16x4 v;
      v[0] = (bf16)c[4 * g]; v[1] = (bf16)c[4 * g + 1]; v[2] = (bf16)c[4 * g + 2]; v[3] = (bf16)c[4 * g + 3];
      *reinterpret_cast<bf16x4*>(hb + p * ldh + n0 + 8 * g + 4 * (lane >> 5)) = v;
    }
  }
};

template <> struct MF<float> {
  static constexpr int KSTEP = 2, KPL = 1, PAD = 4;
  typedef float frag;
  __device__ __forceinline__ static f32x16 mma(frag a, frag b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x2f32(a, b, c, 0, 0, 0);
  }
  __device__ __forceinline__ static frag ld(const float* buf, int ldm, int row0, int k0, int lane) {
    return buf[(row0 + (lane & 31)) * ldm + k0 + (lane >> 5)];
  }
  __device__ __forceinline__ static frag from_acc(const f32x16& c, int j) { return c[j]; }
  // slot <-> s = 8(j/4) + 4(lane/32) + j%4
  __device__ __forceinline__ static frag vperm(const float* vt, int ldv, int p0, int s0, int j, int lane) {
    return vt[(p0 + (lane & 31)) * ldv + s0 + 8 * (j >> 2) + 4 * (lane >> 5) + (j & 3)];
  }
  __device__ __forceinline__ static frag kt(const float* k, int ldk, int n0, int s0, int lane) {
    return k[(s0 + (lane >> 5)) * ldk + n0 + (lane & 31)];
  }
  __device__ __forceinline__ static frag vw(const float*, const float* vt, const float* w, int ldv, int p0, int s0, int lane) {
    const int s = s0 + (lane >> 5);
    return vt[(p0 + (lane & 31)) * ldv + s] * w[s];
  }
  __device__ __forceinline__ static void store_ht(float* hb, int ldh, int p, int n0, const f32x16& c, int lane) {
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      *reinterpret_cast<float4*>(hb + p * ldh + n0 + 8 * g + 4 * (lane >> 5)) =
          make_float4(c[4 * g], c[4 * g + 1], c[4 * g + 2], c[4 * g + 3]);
    }
  }
};

// 16x16 tiles for the output path: v_mfma_f32_16x16x32_bf16 (KPL = 8) and
// v_mfma_f32_16x16x4_f32 (KPL = 1).  A: lane i holds row i%16, k = (i/16)*KPL + [0,KPL);
// B: col i%16, same k; C: lane i, reg r holds col i%16, row 4*(i/16) + r.
template <typename T> struct MF16;
template <> struct MF16<bf16> {
  static constexpr int KSTEP = 32;
  typedef bf16x8 frag;
  __device__ __forceinline__ static f32x4 mma(frag a, frag b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
  }
  __device__ __forceinline__ static frag ld(const bf16* buf, int ldm, int row0, int k0, int lane) {
    return *reinterpret_cast<const bf16x8*>(buf + (row0 + (lane & 15)) * ldm + k0 + (lane >> 4) * 8);
  }
  // steps over a pair of 16-row S^T tiles (32 values of s): slots 0..3 are the
  // first tile's regs (s = 4(lane/16) + 0..3), slots 4..7 the second's (s + 16)
  static constexpr int STEPS = 1;
  __device__ __forceinline__ static frag from_acc(const f32x4& c0, const f32x4& c1, int) {
    frag f;
    f[0] = (bf16)c0[0]; f[1] = (bf16)c0[1]; f[2] = (bf16)c0[2]; f[3] = (bf16)c0[3];
    f[4] = (bf16)c1[0]; f[5] = (bf16)c1[1]; f[6] = (bf16)c1[2]; f[7] = (bf16)c1[3];
    return f;
  }
  __device__ __forceinline__ static frag vperm(const bf16* vt, int ldv, int p0, int s0, int, int lane) {
    const bf16* r = vt + (p0 + (lane & 15)) * ldv + s0 + 4 * (lane >> 4);
    const bf16x4 lo = *reinterpret_cast<const bf16x4*>(r);
    const bf16x4 hi = *reinterpret_cast<const bf16x4*>(r + 16);
    frag f;
    f[0] = lo[0]; f[1] = lo[1]; f[2] = lo[2]; f[3] = lo[3];
    f[4] = hi[0]; f[5] = hi[1]; f[6] = hi[2]; f[7] = hi[3];
    return f;
  }
};
template <> struct MF16<float> {
  static constexpr int KSTEP = 4;
  typedef float frag;
  __device__ __forceinline__ static f32x4 mma(frag a, frag b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
  }
  __device__ __forceinline__ static frag ld(const float* buf, int ldm, int row0, int k0, int lane) {
    return buf[(row0 + (lane & 15)) * ldm + k0 + (lane >> 4)];
  }
  // step j (0..7) over a pair of tiles: j < 4 uses the first tile's reg j
  // (s = 4(lane/16) + j), j >= 4 the second's reg j-4 (s + 16)
  static constexpr int STEPS = 8;
  __device__ __forceinline__ static frag from_acc(const f32x4& c0, const f32x4& c1, int j) {
    return j < 4 ? c0[j] : c1[j - 4];
  }
  __device__ __forceinline__ static frag vperm(const float* vt, int ldv, int p0, int s0, int j, int lane) {
    return vt[(p0 + (lane & 15)) * ldv + s0 + 4 * (lane >> 4) + (j & 3) + (j >= 4 ? 16 : 0)];
  }
};

// Compile-time geometry of one instantiation.
template <typename T, int CS_, int N_, int P_, int R_, int NW_>
struct Geo {
  static constexpr bool BF = std::is_same<T, bf16>::value;
  static constexpr int CS = CS_, N = N_, P = P_, R = R_, NW = NW_, NT = 64 * NW_;
  static constexpr int NWY = NW / 2;                        // waves on output tiles; the rest on state tiles
  static constexpr int KSTEP = MF<T>::KSTEP;
  static constexpr int LB = CS / 32, PB = P / 32, NB = N / 32;
  static constexpr int LDQ = N + MF<T>::PAD;                // sQ, sK rows (elements)
  static constexpr int LDV = CS + MF<T>::PAD;               // sVt, sVwT rows
  static constexpr int LDH = N + MF<T>::PAD;                // sHB rows
  static constexpr int LDY = P + 4;                         // sY rows (fp32)
  static constexpr int LDC = R + 2;                         // cos/sin table rows (float2)
  static constexpr int QG = N / 8;                          // 8-wide vectors per Q/K row
  static constexpr int QROWS = NT / QG;                     // Q/K rows covered per pass
  static constexpr int QV = (CS + QROWS - 1) / QROWS;       // Q/K vectors per thread
  static constexpr int VV = (CS * (P / 8) + NT - 1) / NT;   // V/Z vectors per thread
  static constexpr int CPW = R / NW;                        // rotation columns per wave
  static constexpr int LB16 = CS / 16, PT = P / 16;          // 16-row query blocks, 16-col value tiles
  static constexpr int ST = (NB * PB + (NW - NWY) - 1) / (NW - NWY);  // state tiles per state wave
  static constexpr bool VWT = BF;                           // precomputed w-scaled V^T
  static constexpr int TS = BF ? 2 : 4;
  static constexpr int YB = CS * LDY * 4, CB = CS * LDC * 8;
  static constexpr int COMMON = 2 * CS * LDQ * TS + (VWT ? 2 : 1) * P * LDV * TS +
                                (YB > CB ? YB : CB) + 7 * CS * 4 + 64;
  static constexpr int HBB = P * LDH * TS;
  // two state-operand buffers (no barrier between the output and state-update
  // MFMAs) when they fit in the 160 KiB of LDS, else one
  static constexpr int NHB = (COMMON + 2 * HBB <= 160 * 1024 - 512) ? 2 : 1;
  static_assert(R == 0 || (R % NW == 0 && R % 4 == 0 && 2 * R <= N), "rotation width");
  static_assert(NT % QG == 0, "Q/K column groups");
};

template <typename G>
struct __attribute__((aligned(16))) Smem {
  typedef typename std::conditional<G::BF, bf16, float>::type T;
  T q[G::CS * G::LDQ];
  T k[G::CS * G::LDQ];
  T vt[G::P * G::LDV];
  T vwt[G::VWT ? G::P * G::LDV : 1];
  T hb[G::NHB][G::P * G::LDH];
  union __attribute__((aligned(16))) U {
    float y[G::CS * G::LDY];          // output tile before the gate (phase 3 -> 4)
    float2 cs[G::CS * G::LDC];        // cos/sin of the rotation angles (phase 1 -> 2)
  } u;
  alignas(16) float ac2[G::CS];    // A_cum * log2(e)
  float expa[G::CS];   // e^{A_cum}
  float w[G::CS];      // e^{A_end - A_cum}
  alignas(16) float g16[G::CS];  // e^{A_e - A_cum}, A_e = A_cum at the end of the token's 16-block
  float gam[G::CS];
  float scl[G::CS];
  float dtv[G::CS];
  float qk[G::CS];
  float qb[G::N];      // Q_bias, K_bias of this head
  float kb[G::N];
  float dec;
};

template <int CPW> struct AngRegs { float v[CPW > 0 ? CPW : 1]; };

template <typename T, int CS, int N, int P, int R, int NW>
__global__ __launch_bounds__(64 * NW, 1)
void scan_chunked_kernel(ScanArgs a) {
  typedef Geo<T, CS, N, P, R, NW> G;
  typedef MF<T> M;
  static_assert(sizeof(Smem<G>) <= 160 * 1024, "LDS budget");
  __shared__ Smem<G> sm;

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int bh = blockIdx.x;
  const int b = bh / a.H, h = bh % a.H;
  const int hq = h / (a.H / a.Hqk);
  const int L = a.L, H = a.H, HQ = a.Hqk;
  const int nc = (L + CS - 1) / CS;
  const T* gQ = reinterpret_cast<const T*>(a.q);
  const T* gK = reinterpret_cast<const T*>(a.k);
  const T* gV = reinterpret_cast<const T*>(a.v);
  const T* gZ = reinterpret_cast<const T*>(a.z);
  T* gO = reinterpret_cast<T*>(a.out);
  const float* gadt = a.adt + (long)bh * L;
  const float* gdt = a.dt + (long)bh * L;
  const float* gtr = a.trap + (long)bh * L;
  const float Dh = a.D ? a.D[h] : 0.0f;
  const bool has_z = gZ != nullptr;

  // ---- fixed per-thread mappings
  const int qg = tid % G::QG;            // Q/K column group (8 columns)
  const int qrow0 = tid / G::QG;         // Q/K row of pass 0
  for (int n = tid; n < N; n += G::NT) {
    sm.qb[n] = a.qbias[(long)h * N + n];
    sm.kb[n] = a.kbias[(long)h * N + n];
  }
  const long qk_base = ((long)b * L * HQ + hq) * N + 8 * qg;   // + t * HQ * N
  const long v_base = ((long)b * L * H + h) * P;                // + t * H * P + 8 * g8
  const long a_base = ((long)b * L * H + h) * R + wave * G::CPW;  // + t * H * R

  // ---- raw input registers (next chunk) and the current chunk's V/Z
  Vec8<T> rq[G::QV], rk[G::QV], rv[G::VV], rz[G::VV], cv[G::VV], cz[G::VV];
  AngRegs<G::CPW> ra;
  float s_adt = 0.f, s_dt = 0.f, s_tr = 0.f, s_dtn = 0.f, s_trn = 0.f;

  auto load_chunk = [&](int c) {
    const int t0 = c * CS;
#pragma unroll
    for (int i = 0; i < G::QV; ++i) {
      const int t = qrow0 + i * G::QROWS;
      if (t < CS && t0 + t < L) {
        const long off = qk_base + (long)(t0 + t) * HQ * N;
        rq[i].load(gQ + off);
        rk[i].load(gK + off);
      } else {
        rq[i].zero();
        rk[i].zero();
      }
    }
#pragma unroll
    for (int i = 0; i < G::VV; ++i) {
      const int v = tid + i * G::NT;
      const int t = v % CS, g8 = v / CS;
      if (g8 < P / 8 && t0 + t < L) {
        const long off = v_base + (long)(t0 + t) * H * P + 8 * g8;
        rv[i].load(gV + off);
        if (has_z) rz[i].load(gZ + off); else rz[i].zero();
      } else {
        rv[i].zero();
        rz[i].zero();
      }
    }
    if (G::CPW > 0) {
      const bool ok = lane < CS && t0 + lane < L;
      const float* src = a.ang + a_base + (long)(t0 + lane) * H * R;
#pragma unroll
      for (int j = 0; j < G::CPW; j += (G::CPW >= 4 ? 4 : G::CPW)) {
        if (G::CPW >= 4) {
          const float4 x = ok ? *reinterpret_cast<const float4*>(src + j) : make_float4(0, 0, 0, 0);
          ra.v[j] = x.x; ra.v[j + 1] = x.y; ra.v[j + 2] = x.z; ra.v[j + 3] = x.w;
        } else if (G::CPW == 2) {
          const float2 x = ok ? *reinterpret_cast<const float2*>(src) : make_float2(0, 0);
          ra.v[0] = x.x; ra.v[1] = x.y;
        } else {
          ra.v[0] = ok ? src[0] : 0.0f;
        }
      }
    }
    if (wave == 0) {
      const int t = t0 + lane;
      const bool ok = lane < CS && t < L;
      s_adt = ok ? gadt[t] : 0.f;
      s_dt = ok ? gdt[t] : 0.f;
      s_tr = ok ? gtr[t] : 0.f;
      const bool okn = lane == CS - 1 && t0 + CS < L;
      s_dtn = okn ? gdt[t0 + CS] : 0.f;
      s_trn = okn ? gtr[t0 + CS] : 0.f;
    }
  };

  // wave 0: decay prefix, trapezoid weights for the chunk whose scalars are in s_*
  auto scalar_stage = [&]() {
    const float sig = sigmoid_fast(s_tr);
    const float gam = s_dt * sig;
    const float u = s_dt * (1.0f - sig);                            // dt (1 - sigmoid), this token
    float un = __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(u), 0x130, 0xf, 0xf, false));  // wave_shl:1 -> next token
    if (lane == CS - 1) un = s_dtn * (1.0f - sigmoid_fast(s_trn));
    const float acum = wave_incl_scan(lane < CS ? s_adt : 0.0f);
    const float aend = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(acum), CS - 1));
    const float ablk = __shfl(acum, lane | 15, 64);
    if (lane < CS) {
      sm.ac2[lane] = acum * kLog2e;
      sm.expa[lane] = exp2_fast(acum * kLog2e);
      sm.w[lane] = exp2_fast((aend - acum) * kLog2e);
      sm.g16[lane] = exp2_fast((ablk - acum) * kLog2e);
      sm.gam[lane] = gam;
      sm.scl[lane] = gam + un;
      sm.dtv[lane] = s_dt;
    }
    if (lane == 0) sm.dec = exp2_fast(aend * kLog2e);
  };

  // ---- state accumulators (state waves): tiles z = (wave - NWY) * ST + m of h^T
  const bool ywave = wave < G::NWY;
  const int zw = (wave - G::NWY) * G::ST;
  f32x16 hacc[G::ST];
  float carry[G::CPW > 0 ? G::CPW : 1];
#pragma unroll
  for (int j = 0; j < G::CPW; ++j)
    carry[j] = a.init_theta ? a.init_theta[(long)bh * R + wave * G::CPW + j] : 0.0f;
  {
    // effective entering state: h0 + (1 - sigmoid(trap_0)) dt_0 (v0 (x) k0)
    const float cinit = (a.init_h && L > 0) ? (1.0f - sigmoid_fast(gtr[0])) * gdt[0] : 0.0f;
#pragma unroll
    for (int m = 0; m < G::ST; ++m) {
#pragma unroll
      for (int r = 0; r < 16; ++r) hacc[m][r] = 0.0f;
      const int z = zw + m;
      if (!ywave && z < G::NB * G::PB) {
        const int nb = z / G::PB, pb = z % G::PB;
        const int p = 32 * pb + (lane & 31);
        if (a.init_h) {
          const float v0 = a.init_v[(long)bh * P + p];
#pragma unroll
          for (int r = 0; r < 16; ++r) {
            const int n = 32 * nb + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
            hacc[m][r] = a.init_h[((long)bh * P + p) * N + n] + cinit * v0 * a.init_k[(long)bh * N + n];
          }
        }
        M::store_ht(sm.hb[0], G::LDH, p, 32 * nb, hacc[m], lane);
      }
    }
  }

  load_chunk(0);
  if (wave == 0) scalar_stage();
  __syncthreads();

  for (int c = 0; c < nc; ++c) {
    const int t0 = c * CS;
    const int hcur = c % G::NHB, hnext = (c + 1) % G::NHB;

    // ---- phase 1: rotation angles. lane = token, CPW columns per wave:
    // increments tanh(theta) pi dt, chunk prefix (DPP scan), carry, wrap, cos/sin
    if (G::CPW > 0) {
      const float dtl = lane < CS ? sm.dtv[lane] : 0.0f;
      float2 csv[G::CPW > 0 ? G::CPW : 1];
#pragma unroll
      for (int j = 0; j < G::CPW; ++j) {
        const float d = tanh_fast(ra.v[j]) * kPi * dtl;
        const float th = wrap_2pi(carry[j] + wave_incl_scan(d));
        carry[j] = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(th), CS - 1));
        sincos_wrapped(th, &csv[j].x, &csv[j].y);
      }
      if (lane < CS) {
        float2* dst = &sm.u.cs[lane * G::LDC + wave * G::CPW];
#pragma unroll
        for (int j = 0; j < G::CPW; j += 2) {
          if (G::CPW >= 2) {
            *reinterpret_cast<float4*>(dst + j) = make_float4(csv[j].x, csv[j].y, csv[j + 1].x, csv[j + 1].y);
          } else {
            dst[0] = csv[0];
          }
        }
      }
    }
    __syncthreads();

    // ---- phase 2: biases, QK skip, rope, key scale -> sQ, sK; V^T, (w V)^T
#pragma unroll
    for (int i = 0; i < G::QV; ++i) {
      const int t = qrow0 + i * G::QROWS;
      float qf[8], kf[8];
      rq[i].to_f(qf);
      rk[i].to_f(kf);
      const float4* qbp = reinterpret_cast<const float4*>(&sm.qb[8 * qg]);
      const float4* kbp = reinterpret_cast<const float4*>(&sm.kb[8 * qg]);
      const float4 qb0 = qbp[0], qb1 = qbp[1], kb0 = kbp[0], kb1 = kbp[1];
      const float qb[8] = {qb0.x, qb0.y, qb0.z, qb0.w, qb1.x, qb1.y, qb1.z, qb1.w};
      const float kb[8] = {kb0.x, kb0.y, kb0.z, kb0.w, kb1.x, kb1.y, kb1.z, kb1.w};
      float dot = 0.0f;
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        qf[e] += qb[e];
        kf[e] += kb[e];
        dot += qf[e] * kf[e];
      }
      dot = group_sum<G::QG>(dot);
      if (t < CS) {
        const bool real = t0 + t < L;
        if (qg == 0) sm.qk[t] = real ? dot * sm.gam[t] : 0.0f;
        if (4 * qg < R) {
          const float4* cp = reinterpret_cast<const float4*>(&sm.u.cs[t * G::LDC + 4 * qg]);
          const float4 c01 = cp[0], c23 = cp[1];
          const float cs4[4] = {c01.x, c01.z, c23.x, c23.z};
          const float sn4[4] = {c01.y, c01.w, c23.y, c23.w};
#pragma unroll
          for (int q = 0; q < 4; ++q) {
            const float q0 = qf[2 * q], q1 = qf[2 * q + 1];
            qf[2 * q] = q0 * cs4[q] - q1 * sn4[q];
            qf[2 * q + 1] = q0 * sn4[q] + q1 * cs4[q];
            const float k0 = kf[2 * q], k1 = kf[2 * q + 1];
            kf[2 * q] = k0 * cs4[q] - k1 * sn4[q];
            kf[2 * q + 1] = k0 * sn4[q] + k1 * cs4[q];
          }
        }
        if (a.fin_k && t0 + t == L - 1) {
#pragma unroll
          for (int e = 0; e < 8; ++e) a.fin_k[(long)bh * N + 8 * qg + e] = kf[e];
        }
        const float sc = sm.scl[t];
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          qf[e] = real ? qf[e] : 0.0f;
          kf[e] = real ? kf[e] * sc : 0.0f;
        }
        store8(&sm.q[t * G::LDQ + 8 * qg], qf);
        store8(&sm.k[t * G::LDQ + 8 * qg], kf);
      }
    }
#pragma unroll
    for (int i = 0; i < G::VV; ++i) {
      const int v = tid + i * G::NT;
      const int t = v % CS, g8 = v / CS;
      cv[i] = rv[i];
      cz[i] = rz[i];
      if (g8 < P / 8) {
        float vf[8];
        rv[i].to_f(vf);
        const float wt = sm.w[t];
#pragma unroll
        for (int q = 0; q < 8; ++q) {
          sm.vt[(8 * g8 + q) * G::LDV + t] = Elem<T>::from_f(vf[q]);
          if (G::VWT) sm.vwt[(8 * g8 + q) * G::LDV + t] = Elem<T>::from_f(vf[q] * wt);
        }
      }
    }
    __syncthreads();

    // ---- next chunk's inputs go in flight under the matrix work
    if (c + 1 < nc) load_chunk(c + 1);

    if (wave < G::LB16 && wave < G::NWY) {
      // ---- phases 3 + 6 for query rows l in [16 lb, 16 lb + 16), all value columns:
      //   Y = mask(K_s Q_r^T)^T V + e^{A_cum} Q_r h^T -> sY
      typedef MF16<T> W;
      const int lb = wave;
      const int l = 16 * lb + (lane & 15);
      const float al = sm.ac2[l];
      f32x4 yd[G::PT], yo[G::PT];
#pragma unroll
      for (int pt = 0; pt < G::PT; ++pt)
#pragma unroll
        for (int r = 0; r < 4; ++r) { yd[pt][r] = 0.0f; yo[pt][r] = 0.0f; }
      // Y_off: Q_r (16 x N) . h^T (N x P)
#pragma unroll
      for (int kk = 0; kk < N / W::KSTEP; ++kk) {
        const typename W::frag qf = W::ld(sm.q, G::LDQ, 16 * lb, kk * W::KSTEP, lane);
#pragma unroll
        for (int pt = 0; pt < G::PT; ++pt)
          yo[pt] = W::mma(qf, W::ld(sm.hb[hcur], G::LDH, 16 * pt, kk * W::KSTEP, lane), yo[pt]);
      }
      // Y_diag over key blocks sb <= lb, two 16-row blocks per step
#pragma unroll
      for (int sp = 0; sp < G::LB16; sp += 2) {
        if (sp <= lb) {
          f32x4 st[2];
#pragma unroll
          for (int u = 0; u < 2; ++u) {
            const int sb = sp + u;
#pragma unroll
            for (int r = 0; r < 4; ++r) st[u][r] = 0.0f;
            if (sb <= lb) {
#pragma unroll
              for (int kk = 0; kk < N / W::KSTEP; ++kk)
                st[u] = W::mma(W::ld(sm.k, G::LDQ, 16 * sb, kk * W::KSTEP, lane),
                               W::ld(sm.q, G::LDQ, 16 * lb, kk * W::KSTEP, lane), st[u]);
              const int s0 = 16 * sb + 4 * (lane >> 4);
              if (sb < lb) {
                // off-diagonal block: e^{A_l - A_s} = e^{A_l - A_e} e^{A_e - A_s}, both <= 1
                const float f = exp2_fast(fminf(al - sm.ac2[16 * sb + 15], 0.0f));
                const float4 g = *reinterpret_cast<const float4*>(&sm.g16[s0]);
                st[u][0] *= f * g.x; st[u][1] *= f * g.y; st[u][2] *= f * g.z; st[u][3] *= f * g.w;
              } else {
                // diagonal block: causal mask and per-element decay
                const float4 as = *reinterpret_cast<const float4*>(&sm.ac2[s0]);
                const float asv[4] = {as.x, as.y, as.z, as.w};
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                  const float v = st[u][r] * exp2_fast(fminf(al - asv[r], 0.0f));
                  st[u][r] = (s0 + r < l) ? v : 0.0f;
                }
              }
            }
          }
#pragma unroll
          for (int j = 0; j < W::STEPS; ++j) {
            const typename W::frag mf = W::from_acc(st[0], st[1], j);
#pragma unroll
            for (int pt = 0; pt < G::PT; ++pt)
              yd[pt] = W::mma(mf, W::vperm(sm.vt, G::LDV, 16 * pt, 16 * sp, j, lane), yd[pt]);
          }
        }
      }
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int lr = 16 * lb + 4 * (lane >> 4) + r;
        const float ea = sm.expa[lr];
#pragma unroll
        for (int pt = 0; pt < G::PT; ++pt)
          sm.u.y[lr * G::LDY + 16 * pt + (lane & 15)] = yd[pt][r] + ea * yo[pt][r];
      }
    }
    if (G::NHB == 1) __syncthreads();  // single state buffer: all reads of hb done
    if (!ywave) {
      // ---- phases 4-5: h <- e^{A_end} h + (K_s)^T (w V), state tiles interleaved
      const float dec = sm.dec;
#pragma unroll
      for (int m = 0; m < G::ST; ++m)
#pragma unroll
        for (int r = 0; r < 16; ++r) hacc[m][r] *= dec;
#pragma unroll
      for (int j = 0; j < CS / G::KSTEP; ++j) {
#pragma unroll
        for (int m = 0; m < G::ST; ++m) {
          const int z = zw + m;
          if (z < G::NB * G::PB) {
            const int nb = z / G::PB, pb = z % G::PB;
            hacc[m] = M::mma(M::kt(sm.k, G::LDQ, 32 * nb, j * G::KSTEP, lane),
                             M::vw(sm.vwt, sm.vt, sm.w, G::LDV, 32 * pb, j * G::KSTEP, lane), hacc[m]);
          }
        }
      }
#pragma unroll
      for (int m = 0; m < G::ST; ++m) {
        const int z = zw + m;
        if (z < G::NB * G::PB) {
          const int nb = z / G::PB, pb = z % G::PB;
          M::store_ht(sm.hb[hnext], G::LDH, 32 * pb + (lane & 31), 32 * nb, hacc[m], lane);
        }
      }
    }
    __syncthreads();

    // ---- phase 7: (Y + (D + QK) V) * silu(Z) -> out
#pragma unroll
    for (int i = 0; i < G::VV; ++i) {
      const int v = tid + i * G::NT;
      const int t = v % CS, g8 = v / CS;
      if (g8 < P / 8 && t0 + t < L) {
        float vf[8], zf[8], yv[8];
        cv[i].to_f(vf);
        cz[i].to_f(zf);
        const float4 y0 = *reinterpret_cast<const float4*>(&sm.u.y[t * G::LDY + 8 * g8]);
        const float4 y1 = *reinterpret_cast<const float4*>(&sm.u.y[t * G::LDY + 8 * g8 + 4]);
        yv[0] = y0.x; yv[1] = y0.y; yv[2] = y0.z; yv[3] = y0.w;
        yv[4] = y1.x; yv[5] = y1.y; yv[6] = y1.z; yv[7] = y1.w;
        const float dq = Dh + sm.qk[t];
#pragma unroll
        for (int q = 0; q < 8; ++q) {
          float o = yv[q] + dq * vf[q];
          if (has_z) o *= silu_fast(zf[q]);
          yv[q] = o;
        }
        store8(gO + v_base + (long)(t0 + t) * H * P + 8 * g8, yv);
        if (a.fin_v && t0 + t == L - 1) {
#pragma unroll
          for (int q = 0; q < 8; ++q) a.fin_v[(long)bh * P + 8 * g8 + q] = vf[q];
        }
      }
    }
    if (wave == 0 && c + 1 < nc) scalar_stage();
    __syncthreads();
  }

  if (a.fin_h) {
    if (!ywave) {
#pragma unroll
      for (int m = 0; m < G::ST; ++m) {
        const int z = zw + m;
        if (z < G::NB * G::PB) {
          const int nb = z / G::PB, pb = z % G::PB;
          const int p = 32 * pb + (lane & 31);
#pragma unroll
          for (int r = 0; r < 16; ++r) {
            const int n = 32 * nb + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
            a.fin_h[((long)bh * P + p) * N + n] = hacc[m][r];
          }
        }
      }
    }
    if (lane == 0) {
#pragma unroll
      for (int j = 0; j < G::CPW; ++j) a.fin_theta[(long)bh * R + wave * G::CPW + j] = carry[j];
    }
  }
}

// ------------------------------------------------------------------ dispatch
// (dtype, chunk, d_state, headdim, rotation width) instantiations; R is the
// model's rope_fraction 0.5 (R = N/4) or 1.0 (R = N/2) width, or 0.
#define M3_CHUNK_SHAPES(X)                                                                         \
  X(bf16, 64, 128, 64, 32) X(bf16, 64, 128, 64, 64) X(bf16, 64, 128, 64, 0)                        \
  X(bf16, 64, 128, 32, 32) X(bf16, 64, 64, 64, 16) X(bf16, 64, 64, 64, 32) \
  X(bf16, 64, 64, 32, 16) X(bf16, 64, 32, 32, 8) X(bf16, 64, 32, 64, 8)                            \
  X(bf16, 32, 128, 64, 32) X(bf16, 32, 64, 64, 16) X(bf16, 32, 64, 32, 16) X(bf16, 32, 128, 32, 32) \
  X(float, 64, 64, 64, 16) X(float, 64, 64, 64, 32) X(float, 64, 64, 32, 16) X(float, 32, 64, 64, 16) \
  X(float, 32, 64, 32, 16) X(float, 64, 32, 32, 8) X(float, 64, 32, 64, 8)

constexpr int kChunkWaves = 8;

bool scan_chunked_supported(bool bf16_io, int CS, int N, int P, int R) {
#define X(T, cs, n, p, r) \
  if ((std::is_same<T, bf16>::value == bf16_io) && CS == cs && N == n && P == p && R == r) return true;
  M3_CHUNK_SHAPES(X)
#undef X
  return false;
}

hipError_t scan_chunked_launch(const ScanArgs& a, bool bf16_io, hipStream_t st) {
#define X(T, cs, n, p, r)                                                                            \
  if ((std::is_same<T, bf16>::value == bf16_io) && a.CS == cs && a.N == n && a.P == p && a.R == r) { \
    hipLaunchKernelGGL((scan_chunked_kernel<T, cs, n, p, r, kChunkWaves>), dim3(a.B * a.H),          \
                       dim3(64 * kChunkWaves), 0, st, a);                                             \
    return hipGetLastError();                                                                         \
  }
  M3_CHUNK_SHAPES(X)
#undef X
  return hipErrorInvalidValue;
}

}  // namespace m3
