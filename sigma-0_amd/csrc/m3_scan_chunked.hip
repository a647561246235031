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
// One workgroup (8 waves) per (batch, head) walks the chunks in order; the
// P x N fp32 state never leaves the CU.  While a chunk's matrix work runs,
// the next chunk's inputs stream into LDS with direct-to-LDS loads (whole
// rows per instruction, stored XOR-swizzled), so every input byte is read
// from HBM exactly once and the output written once.
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
  // A operand (w K)^T: row n = n0 + lane%32, k = s = s0 + 8(lane/32) + q, read from
  // row-major K[s][n] and scaled by w[s] (the decay from token s to the chunk end)
  __device__ __forceinline__ static frag ktw(const bf16* k, const float* w, int ldk, int n0, int s0, int lane) {
    const int sb = s0 + 8 * (lane >> 5);
    const bf16* c = k + sb * ldk + n0 + (lane & 31);
    const float4 w0 = *reinterpret_cast<const float4*>(w + sb);
    const float4 w1 = *reinterpret_cast<const float4*>(w + sb + 4);
    const float wv[8] = {w0.x, w0.y, w0.z, w0.w, w1.x, w1.y, w1.z, w1.w};
    frag f;
#pragma unroll
    for (int q = 0; q < 8; ++q) f[q] = (bf16)((float)c[q * ldk] * wv[q]);
    return f;
  }
  // B operand V[s][p]: row p of V^T, s = s0 + 8(lane/32) + q
  __device__ __forceinline__ static frag vs(const bf16* vt, int ldv, int p0, int s0, int lane) {
    return ld(vt, ldv, p0, s0, lane);
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
  __device__ __forceinline__ static frag ktw(const float* k, const float* w, int ldk, int n0, int s0, int lane) {
    const int sv = s0 + (lane >> 5);
    return k[sv * ldk + n0 + (lane & 31)] * w[sv];
  }
  __device__ __forceinline__ static frag vs(const float* vt, int ldv, int p0, int s0, int lane) {
    return vt[(p0 + (lane & 31)) * ldv + s0 + (lane >> 5)];
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
  static constexpr int PB = P / 32, NB = N / 32;            // 32x32 state tiles
  static constexpr int LB16 = CS / 16, PT = P / 16;         // 16-row query blocks, 16-col value tiles
  static constexpr int TS = BF ? 2 : 4;
  static constexpr int LDQ = N + MF<T>::PAD;                // sQ, sK rows (elements)
  static constexpr int LDV = CS + MF<T>::PAD;               // sVt rows
  static constexpr int LDH = N + MF<T>::PAD;                // sHB rows
  static constexpr int LDY = P + 4;                         // sY rows (fp32)
  static constexpr int QG = N / 8, QGW = (QG + NW - 1) / NW;  // Q/K 8-column groups, per wave
  static constexpr int VG = P / 8, VGW = (VG + NW - 1) / NW;  // V/Z 8-column groups, per wave
  static constexpr int HT = (NB * PB + (NW - NWY) - 1) / (NW - NWY);  // state tiles per state wave
  // 16-byte staging slots per row: Q/K, V/Z, rotation rates
  static constexpr int SQ = N * TS / 16, SV = P * TS / 16, SA = R / 4 > 0 ? R / 4 : 1;
  static constexpr int GS = 8 * TS / 16;                    // slots per 8-element group (1 bf16, 2 f32)
  static constexpr int STAGE = (2 * CS * SQ + 2 * CS * SV + CS * SA) * 16 + 3 * (CS + 4) * 4;
  static constexpr int COMMON = 2 * CS * LDQ * TS + P * LDV * TS + CS * LDY * 4 + 8 * CS * 4 + 8 * N + 64 + STAGE;
  static constexpr int HBB = P * LDH * TS;
  // two state-operand buffers (no barrier between the output and state-update
  // MFMAs) when they fit in the 160 KiB of LDS, else one
  static constexpr int NHB = (COMMON + 2 * HBB <= 160 * 1024 - 512) ? 2 : 1;
  static_assert(CS <= 64, "one token per lane");
  static_assert(R % 4 == 0 && 2 * R <= N, "rotation width: a multiple of 4, at most N/2");
  static_assert((SQ & (SQ - 1)) == 0 && (SV & (SV - 1)) == 0 && (SA & (SA - 1)) == 0, "swizzle widths");
};

template <typename G>
struct __attribute__((aligned(16))) Smem {
  typedef typename std::conditional<G::BF, bf16, float>::type T;
  T q[G::CS * G::LDQ];
  T k[G::CS * G::LDQ];
  T vt[G::P * G::LDV];
  T hb[G::NHB][G::P * G::LDH];
  alignas(16) float y[G::CS * G::LDY];   // output tile before the gate (phase 3 -> 7)
  // raw inputs staged by direct-to-LDS loads: 16-byte slots, row t slot s stored at
  // t * S + (s ^ (t mod S)) so that a lane-per-row read is bank-conflict free
  alignas(16) uint4 rq[G::CS * G::SQ];
  alignas(16) uint4 rk[G::CS * G::SQ];
  alignas(16) uint4 rv[G::CS * G::SV];
  alignas(16) uint4 rz[G::CS * G::SV];
  alignas(16) uint4 ra[G::CS * G::SA];
  alignas(16) float rs[3][G::CS + 4];    // adt, dt, trap of the chunk; [CS] = the next token's
  alignas(16) float qb[G::N];            // biases of this head
  alignas(16) float kb[G::N];
  alignas(16) float ac2[G::CS];          // A_cum * log2(e)
  alignas(16) float g16[G::CS];          // e^{A_e - A_cum}, A_e = A_cum at the end of the token's 16-block
  alignas(16) float w[G::CS];            // e^{A_end - A_cum}
  float expa[G::CS];                     // e^{A_cum}
  float qk[2][G::CS];                    // QK skip term, accumulated over column groups (chunk parity)
  float dec;                             // e^{A_end}
};

// Direct-to-LDS loads (global_load_lds): the LDS slot is the instruction's base plus
// size * lane.  The LDS pointer is cast to the local address space here so that the
// builtin sees a local pointer rather than a flat one.
typedef __attribute__((address_space(3))) uint4 lds_uint4;
typedef __attribute__((address_space(3))) float lds_float;
__device__ __forceinline__ void lds_dma16(const void* g, lds_uint4* l) { __builtin_amdgcn_global_load_lds(g, l, 16, 0, 0); }
__device__ __forceinline__ void lds_dma4(const void* g, lds_float* l) { __builtin_amdgcn_global_load_lds(g, l, 4, 0, 0); }

// Direct-to-LDS staging of CS rows x S 16-byte slots.  Instruction j stages 64 slots:
// lane -> (row, physical slot) = (64j/S + lane/S, lane%S), fetching logical slot
// (lane%S) ^ (row%S), so each row is read whole (coalesced) and stored swizzled.  The
// lane part of the global offset repeats every PER instructions (row%S repeats), so a
// few 32-bit lane offsets plus a wave-uniform row base address every instruction.
template <int CS, int S>
__device__ __forceinline__ void stage_rows(lds_uint4* dst, const char* src, long stride, int rows_valid,
                                           int lane) {
  constexpr int RP = 64 / S;                               // rows per instruction
  constexpr int NJ = CS * S / 64;                          // instructions
  static_assert(CS * S % 64 == 0, "whole instructions");
  constexpr int PER = S * S / 64 > 1 ? S * S / 64 : 1;     // period of the lane pattern
  const int lrow = lane / S;
  uint32_t off[PER];
#pragma unroll
  for (int p = 0; p < PER; ++p) {
    const uint32_t row = p * RP + lrow;
    off[p] = row * (uint32_t)stride + 16u * ((lane % S) ^ (row & (S - 1)));
  }
  // the row base is made opaque so that the compiler keeps one wave-uniform base per
  // group of PER instructions instead of strength-reducing to 64-bit lane pointers
  const char* base = src;
  asm volatile("" : "+s"(base));
  if (rows_valid >= CS) {
#pragma unroll
    for (int m = 0; m < NJ / PER; ++m) {
      const char* bm = base + (long)m * (PER * RP) * stride;
#pragma unroll
      for (int p = 0; p < PER; ++p) lds_dma16(bm + off[p], dst + 64 * (m * PER + p));
    }
  } else {
#pragma unroll
    for (int m = 0; m < NJ / PER; ++m) {
      const char* bm = base + (long)m * (PER * RP) * stride;
#pragma unroll
      for (int p = 0; p < PER; ++p) {
        const int j = m * PER + p;
        if (j * RP + lrow < rows_valid) lds_dma16(bm + off[p], dst + 64 * j);
      }
    }
  }
}
template <int S>
__device__ __forceinline__ const uint4& staged(const uint4* buf, int row, int slot) {
  return buf[row * S + (slot ^ (row & (S - 1)))];
}

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
  __builtin_assume(wave >= 0 && wave < NW);
  const int bh = blockIdx.x;
  const int b = bh / a.H, h = bh % a.H;
  const int hq = h / (a.H / a.Hqk);
  const int L = a.L, H = a.H, HQ = a.Hqk;
  const int nc = (L + CS - 1) / CS;
  T* gO = reinterpret_cast<T*>(a.out);
  const float* gadt = a.adt + (long)bh * L;
  const float* gdt = a.dt + (long)bh * L;
  const float* gtr = a.trap + (long)bh * L;
  const float Dh = a.D ? a.D[h] : 0.0f;
  const bool has_z = a.z != nullptr;

  // ---- element offsets of row (b, t=0, head) in each input; rows advance by the stride
  const long qk_row = ((long)b * L * HQ + hq) * N, qk_stride = (long)HQ * N;
  const long v_row = ((long)b * L * H + h) * P, v_stride = (long)H * P;
  const long a_row = ((long)b * L * H + h) * R, a_stride = (long)H * R;
  for (int i = tid; i < N; i += G::NT) {
    sm.qb[i] = a.qbias[(long)h * N + i];
    sm.kb[i] = a.kbias[(long)h * N + i];
  }

  // ---- staging: the state waves stream the next chunk's inputs into LDS
  auto stage_main = [&](int c) {           // Q, K, V, rotation rates, scalars of chunk c
    const int t0 = c * CS;
    const int valid = L - t0;
    const char* q0 = reinterpret_cast<const char*>(reinterpret_cast<const T*>(a.q) + qk_row + (long)t0 * qk_stride);
    const char* k0 = reinterpret_cast<const char*>(reinterpret_cast<const T*>(a.k) + qk_row + (long)t0 * qk_stride);
    const char* v0 = reinterpret_cast<const char*>(reinterpret_cast<const T*>(a.v) + v_row + (long)t0 * v_stride);
    if (wave == G::NWY) stage_rows<CS, G::SQ>((lds_uint4*)sm.rq, q0, qk_stride * G::TS, valid, lane);
    if (wave == G::NWY + 1) stage_rows<CS, G::SQ>((lds_uint4*)sm.rk, k0, qk_stride * G::TS, valid, lane);
    if (wave == G::NWY + 2) {
      stage_rows<CS, G::SV>((lds_uint4*)sm.rv, v0, v_stride * G::TS, valid, lane);
      if (R > 0) {
        const char* a0 = reinterpret_cast<const char*>(a.ang + a_row + (long)t0 * a_stride);
        stage_rows<CS, G::SA>((lds_uint4*)sm.ra, a0, a_stride * 4, valid, lane);
      }
    }
    if (wave == G::NWY + 3) {
      if (lane < CS && lane < valid) {
        lds_dma4(gadt + t0 + lane, (lds_float*)&sm.rs[0][0]);
        lds_dma4(gdt + t0 + lane, (lds_float*)&sm.rs[1][0]);
        lds_dma4(gtr + t0 + lane, (lds_float*)&sm.rs[2][0]);
      }
      if (lane == 0 && t0 + CS < L) {
        lds_dma4(gdt + t0 + CS, (lds_float*)&sm.rs[1][CS]);
        lds_dma4(gtr + t0 + CS, (lds_float*)&sm.rs[2][CS]);
      }
    }
  };
  auto stage_z = [&](int c) {              // Z of chunk c
    if (has_z && wave == G::NWY + 3) {
      const int t0 = c * CS;
      const char* z0 = reinterpret_cast<const char*>(reinterpret_cast<const T*>(a.z) + v_row + (long)t0 * v_stride);
      stage_rows<CS, G::SV>((lds_uint4*)sm.rz, z0, v_stride * G::TS, L - t0, lane);
    }
  };

  // ---- state accumulators (state waves): tiles z = (wave - NWY) * HT + m of h^T
  const bool ywave = wave < G::NWY;
  const int zw = (wave - G::NWY) * G::HT;
  f32x16 hacc[G::HT];
  float carry[G::QGW][4];
#pragma unroll
  for (int k = 0; k < G::QGW; ++k)
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int r = 4 * (wave + NW * k) + j;
      carry[k][j] = (a.init_theta && r < R) ? a.init_theta[(long)bh * R + r] : 0.0f;
    }
  {
    // effective entering state: h0 + (1 - sigmoid(trap_0)) dt_0 (v0 (x) k0)
    const float cinit = (a.init_h && L > 0) ? (1.0f - sigmoid_fast(gtr[0])) * gdt[0] : 0.0f;
#pragma unroll
    for (int m = 0; m < G::HT; ++m) {
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
  // staging never holds uninitialised bits: rows past the sequence end are not loaded
  for (int i = tid; i < G::CS * G::SQ; i += G::NT) { sm.rq[i] = make_uint4(0, 0, 0, 0); sm.rk[i] = sm.rq[i]; }
  for (int i = tid; i < G::CS * G::SV; i += G::NT) { sm.rv[i] = make_uint4(0, 0, 0, 0); sm.rz[i] = sm.rv[i]; }
  for (int i = tid; i < G::CS * G::SA; i += G::NT) sm.ra[i] = make_uint4(0, 0, 0, 0);
  for (int i = tid; i < 3 * (G::CS + 4); i += G::NT) ((lds_float*)&sm.rs[0][0])[i] = 0.0f;
  if (tid < CS) sm.qk[0][tid] = 0.0f;
  __syncthreads();
  stage_main(0);
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();

  Vec8<T> cv[G::VGW];                      // this lane's V row slice, kept for the epilogue

  for (int c = 0; c < nc; ++c) {
    const int t0 = c * CS;
    const int hcur = c % G::NHB, hnext = (c + 1) % G::NHB;
    const bool tail = t0 + CS > L;              // chunk holds padding rows
    const bool tok = lane < CS && t0 + lane < L;
    const int tl = lane < CS ? lane : 0;        // staging row of this lane

    // ================= prep: lane = token =================
    // per-token decay prefix and trapezoid weights (every wave, registers)
    const float s_adt = tok ? sm.rs[0][tl] : 0.0f;
    const float s_dt = tok ? sm.rs[1][tl] : 0.0f;
    const float s_tr = tok ? sm.rs[2][tl] : 0.0f;
    const float sig = sigmoid_fast(s_tr);
    const float gam = s_dt * sig;
    const float u = s_dt * (1.0f - sig);                                   // dt (1 - sigmoid), this token
    float un = __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(u), 0x130, 0xf, 0xf, false));  // next token
    if (lane == CS - 1) un = (t0 + CS < L) ? sm.rs[1][CS] * (1.0f - sigmoid_fast(sm.rs[2][CS])) : 0.0f;
    const float scl = gam + un;
    const float acum = wave_incl_scan(lane < CS ? s_adt : 0.0f);
    const float aend = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(acum), CS - 1));
    if (wave == 0 && lane < CS) {
      const float ablk = __shfl(acum, lane | 15, 64);
      sm.ac2[lane] = acum * kLog2e;
      sm.expa[lane] = exp2_fast(acum * kLog2e);
      sm.g16[lane] = exp2_fast((ablk - acum) * kLog2e);
      sm.w[lane] = exp2_fast((aend - acum) * kLog2e);
      if (lane == 0) sm.dec = exp2_fast(aend * kLog2e);
    }
    // Q/K column groups: rotation angles, biases, QK skip partial, rope, key scale
    float dot = 0.0f;
#pragma unroll
    for (int k = 0; k < G::QGW; ++k) {
      const int g = wave + NW * k;
      if (g < G::QG) {
        float qf[8], kf[8];
        {
          Vec8<T> qv, kv;
          if constexpr (G::BF) {
            qv.raw_set(staged<G::SQ>(sm.rq, tl, g));
            kv.raw_set(staged<G::SQ>(sm.rk, tl, g));
          } else {
            qv.raw_set2(staged<G::SQ>(sm.rq, tl, 2 * g), staged<G::SQ>(sm.rq, tl, 2 * g + 1));
            kv.raw_set2(staged<G::SQ>(sm.rk, tl, 2 * g), staged<G::SQ>(sm.rk, tl, 2 * g + 1));
          }
          qv.to_f(qf);
          kv.to_f(kf);
        }
        {
          const float4* qb4 = reinterpret_cast<const float4*>(&sm.qb[8 * g]);
          const float4* kb4 = reinterpret_cast<const float4*>(&sm.kb[8 * g]);
          const float4 qa = qb4[0], qc = qb4[1], ka = kb4[0], kc = kb4[1];
          const float qbv[8] = {qa.x, qa.y, qa.z, qa.w, qc.x, qc.y, qc.z, qc.w};
          const float kbv[8] = {ka.x, ka.y, ka.z, ka.w, kc.x, kc.y, kc.z, kc.w};
#pragma unroll
          for (int e = 0; e < 8; ++e) {
            qf[e] += qbv[e];
            kf[e] += kbv[e];
            dot += qf[e] * kf[e];
          }
        }
        if (4 * g < R) {
          const uint4 rr = staged<G::SA>(sm.ra, tl, g);
          const float rav[4] = {__uint_as_float(rr.x), __uint_as_float(rr.y), __uint_as_float(rr.z),
                                __uint_as_float(rr.w)};
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            // theta = carry + prefix of tanh(rate) pi dt over the chunk, mod 2pi
            const float d = tok ? tanh_fast(rav[j]) * kPi * s_dt : 0.0f;
            const float th = wrap_2pi(carry[k][j] + wave_incl_scan(d));
            carry[k][j] = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(th), CS - 1));
            float cs, sn;
            sincos_wrapped(th, &cs, &sn);
            const float q0 = qf[2 * j], q1 = qf[2 * j + 1];
            qf[2 * j] = q0 * cs - q1 * sn;
            qf[2 * j + 1] = q0 * sn + q1 * cs;
            const float k0 = kf[2 * j], k1 = kf[2 * j + 1];
            kf[2 * j] = k0 * cs - k1 * sn;
            kf[2 * j + 1] = k0 * sn + k1 * cs;
          }
        }
        if (a.fin_k && t0 + lane == L - 1) {
#pragma unroll
          for (int e = 0; e < 8; ++e) a.fin_k[(long)bh * N + 8 * g + e] = kf[e];
        }
#pragma unroll
        for (int e = 0; e < 8; ++e) kf[e] *= scl;
        if (tail && !tok) {
#pragma unroll
          for (int e = 0; e < 8; ++e) { qf[e] = 0.0f; kf[e] = 0.0f; }
        }
        if (lane < CS) {
          store8(&sm.q[lane * G::LDQ + 8 * g], qf);
          store8(&sm.k[lane * G::LDQ + 8 * g], kf);
        }
      }
    }
    if (lane < CS) atomicAdd(&sm.qk[c & 1][lane], dot * gam);   // gam == 0 on padding rows
    // V column groups: V^T (this lane's slice is kept for the epilogue)
#pragma unroll
    for (int k = 0; k < G::VGW; ++k) {
      const int g = wave + NW * k;
      if (g < G::VG) {
        if constexpr (G::BF) cv[k].raw_set(staged<G::SV>(sm.rv, tl, g));
        else cv[k].raw_set2(staged<G::SV>(sm.rv, tl, 2 * g), staged<G::SV>(sm.rv, tl, 2 * g + 1));
        if (tail && !tok) cv[k].zero();
        if (lane < CS) {
          float vf[8];
          cv[k].to_f(vf);
#pragma unroll
          for (int q = 0; q < 8; ++q) sm.vt[(8 * g + q) * G::LDV + lane] = Elem<T>::from_f(vf[q]);
        }
      }
    }
    __syncthreads();

    // ---- staging for the epilogue of this chunk and the inputs of the next one
    stage_z(c);
    if (c + 1 < nc) stage_main(c + 1);

    if (wave == NW - 1 && lane < CS) sm.qk[(c + 1) & 1][lane] = 0.0f;   // read last by phase 7 of chunk c-1

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
          for (int u2 = 0; u2 < 2; ++u2) {
            const int sb = sp + u2;
#pragma unroll
            for (int r = 0; r < 4; ++r) st[u2][r] = 0.0f;
            if (sb <= lb) {
#pragma unroll
              for (int kk = 0; kk < N / W::KSTEP; ++kk)
                st[u2] = W::mma(W::ld(sm.k, G::LDQ, 16 * sb, kk * W::KSTEP, lane),
                                W::ld(sm.q, G::LDQ, 16 * lb, kk * W::KSTEP, lane), st[u2]);
              const int s0 = 16 * sb + 4 * (lane >> 4);
              if (sb < lb) {
                // off-diagonal block: e^{A_l - A_s} = e^{A_l - A_e} e^{A_e - A_s}, both <= 1
                const float f = exp2_fast(fminf(al - sm.ac2[16 * sb + 15], 0.0f));
                const float4 g4 = *reinterpret_cast<const float4*>(&sm.g16[s0]);
                st[u2][0] *= f * g4.x; st[u2][1] *= f * g4.y; st[u2][2] *= f * g4.z; st[u2][3] *= f * g4.w;
              } else {
                // diagonal block: causal mask and per-element decay
                const float4 as = *reinterpret_cast<const float4*>(&sm.ac2[s0]);
                const float asv[4] = {as.x, as.y, as.z, as.w};
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                  const float v = st[u2][r] * exp2_fast(fminf(al - asv[r], 0.0f));
                  st[u2][r] = (s0 + r < l) ? v : 0.0f;
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
          sm.y[lr * G::LDY + 16 * pt + (lane & 15)] = yd[pt][r] + ea * yo[pt][r];
      }
    }
    if (G::NHB == 1) __syncthreads();  // single state buffer: all reads of hb done
    if (!ywave) {
      // ---- phases 4-5: h <- e^{A_end} h + (w K_s)^T V, state tiles interleaved
      const float dec = sm.dec;
#pragma unroll
      for (int m = 0; m < G::HT; ++m)
#pragma unroll
        for (int r = 0; r < 16; ++r) hacc[m][r] *= dec;
#pragma unroll
      for (int j = 0; j < CS / G::KSTEP; ++j) {
#pragma unroll
        for (int m = 0; m < G::HT; ++m) {
          const int z = zw + m;
          if (z < G::NB * G::PB) {
            const int nb = z / G::PB, pb = z % G::PB;
            hacc[m] = M::mma(M::ktw(sm.k, sm.w, G::LDQ, 32 * nb, j * G::KSTEP, lane),
                             M::vs(sm.vt, G::LDV, 32 * pb, j * G::KSTEP, lane), hacc[m]);
          }
        }
      }
#pragma unroll
      for (int m = 0; m < G::HT; ++m) {
        const int z = zw + m;
        if (z < G::NB * G::PB) {
          const int nb = z / G::PB, pb = z % G::PB;
          M::store_ht(sm.hb[hnext], G::LDH, 32 * pb + (lane & 31), 32 * nb, hacc[m], lane);
        }
      }
    }
    __builtin_amdgcn_s_waitcnt(0);   // staged loads of this wave have landed in LDS
    __syncthreads();

    // ================= phase 7: lane = token, (Y + (D + QK) V) * silu(Z) -> out =================
    {
      const float dq = Dh + (lane < CS ? sm.qk[c & 1][lane] : 0.0f);
#pragma unroll
      for (int k = 0; k < G::VGW; ++k) {
        const int g = wave + NW * k;
        if (g < G::VG && tok) {
          float vf[8], zf[8], yv[8];
          cv[k].to_f(vf);
          Vec8<T> zv;
          if constexpr (G::BF) zv.raw_set(staged<G::SV>(sm.rz, tl, g));
          else zv.raw_set2(staged<G::SV>(sm.rz, tl, 2 * g), staged<G::SV>(sm.rz, tl, 2 * g + 1));
          zv.to_f(zf);
          const float4 y0 = *reinterpret_cast<const float4*>(&sm.y[lane * G::LDY + 8 * g]);
          const float4 y1 = *reinterpret_cast<const float4*>(&sm.y[lane * G::LDY + 8 * g + 4]);
          yv[0] = y0.x; yv[1] = y0.y; yv[2] = y0.z; yv[3] = y0.w;
          yv[4] = y1.x; yv[5] = y1.y; yv[6] = y1.z; yv[7] = y1.w;
#pragma unroll
          for (int q = 0; q < 8; ++q) {
            float o = yv[q] + dq * vf[q];
            if (has_z) o *= silu_fast(zf[q]);
            yv[q] = o;
          }
          store8(gO + v_row + (long)(t0 + lane) * v_stride + 8 * g, yv);
          if (a.fin_v && t0 + lane == L - 1) {
#pragma unroll
            for (int q = 0; q < 8; ++q) a.fin_v[(long)bh * P + 8 * g + q] = vf[q];
          }
        }
      }
    }
  }

  if (a.fin_h) {
    if (!ywave) {
#pragma unroll
      for (int m = 0; m < G::HT; ++m) {
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
      for (int k = 0; k < G::QGW; ++k)
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const int r = 4 * (wave + NW * k) + j;
          if (r < R) a.fin_theta[(long)bh * R + r] = carry[k][j];
        }
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
