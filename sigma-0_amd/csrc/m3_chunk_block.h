// Workgroup set-up, staging and chunk constants shared by the chunked prefill kernels
// (bf16 I/O in m3_scan_chunked.hip, float32 I/O in m3_scan_chunked_f32.hip).
//
// Both run one workgroup of 12 waves per (batch, head, sequence segment) over the
// segment's chunks in order, stage every chunk's rows by direct-to-LDS loads
// double-buffered by chunk parity, carry the state in the state waves' accumulators
// and compute the same per-token chunk constants on one wave.  What differs between
// them stays in each kernel: the geometry and LDS layout (64- against 32-token chunks,
// the float32 kernel's Y tiles), the wave roles (four query blocks on the output waves
// against three phase-3 items spread over three SIMDs) and the chunk loop built on them.
#pragma once

#include <type_traits>

#include "m3_chunk_common.h"

namespace m3 {

// Geometry common to the chunked kernels' instantiations: 12 waves (output waves 0-3,
// state waves 4-7, auxiliary waves 8-11), 16 x 16 MFMA tiles, the Q/K 8-column groups
// and the staging tiles' 16-byte slots per row.  Each kernel's Geo adds its LDS budget
// and its assignment of the column groups to the waves.
template <typename T, int CS_, int N_, int P_, int R_, int NW_>
struct GeoBase {
  static constexpr bool BF = std::is_same<T, bf16>::value;
  static constexpr int CS = CS_, N = N_, P = P_, R = R_, NW = NW_, NT = 64 * NW_;
  static constexpr int NWY = 4;                             // output waves 0..3
  static constexpr int NST = 4;                             // state waves 4..7
  static constexpr int NAUX = NW - NWY - NST;               // auxiliary waves 8..11
  static constexpr int KSTEP = MF16<T>::KSTEP;
  static constexpr int LB16 = CS / 16, PT = P / 16;         // 16-row query blocks, 16-col p-tiles
  static constexpr int NB16 = N / 16;                       // 16-row state tiles per p-tile
  static constexpr int SPT = NST / PT;                      // state waves per p-tile
  static constexpr int TS = BF ? 2 : 4;
  static constexpr int PAD = BF ? 8 : 4;
  static constexpr int LDQ = N + PAD;                       // sQ, sK (and the bf16 kernel's sH) rows
  static constexpr int QG = N / 8, QGW = 2;                 // Q/K 8-column groups, at most 2 per wave
  // 16-byte staging slots per row: Q/K, V, rotation rates
  static constexpr int SQ = N * TS / 16, SV = P * TS / 16, SA = R / 4 > 0 ? R / 4 : 1;
  static_assert(CS <= 64 && LB16 <= NWY, "one token per lane, one query block per output wave");
  static_assert(NAUX == 4, "12 waves");
  static_assert(QG <= 2 * NAUX + NWY + NST, "column groups per wave");
  static_assert(R % 4 == 0 && 2 * R <= N, "rotation width: a multiple of 4, at most N/2");
  static_assert((SQ & (SQ - 1)) == 0 && (SV & (SV - 1)) == 0 && (SA & (SA - 1)) == 0, "swizzle widths");
};

// The (batch, head, segment) of a workgroup, its tokens and the row bases of its
// inputs and output: element pointers to row (b, t = tb, head), rows advancing by the
// strides (elements, 32-bit; offsets along the sequence are formed in 64 bits).
template <typename T>
struct ChunkBlock {
  int bh, b, h, hq;
  int seg, nseg;
  int tb;                        // first token of the segment
  int L;                         // tokens of the segment
  int Lnx;                       // tokens from tb to the sequence end: a segment's last
                                 // trapezoid weight reads the next token's scalars
  int nc;                        // chunks of the segment
  long ch0;                      // chunk-state outputs (chunk_h / chunk_th) are indexed by
                                 // the chunk over the whole sequence: ch0 is the segment's first
  int ci_in, ci_out;             // carry slots: per (b, h) or per (b, h, segment)
  bool has_init, fin_here, has_z;
  float Dh;
  int qk_stride, v_stride, a_stride, vz_stride;
  const float *gadt, *gdt, *gtr; // the segment's per-token scalars
  T* gO;
  const T *q_base, *k_base, *v_base, *z_base;
  T* o_base;
  const float* ang_base;
};

template <typename T, int CS, int N, int P, int R>
__device__ __forceinline__ ChunkBlock<T> chunk_block(const ScanArgs& a) {
  ChunkBlock<T> k;
  k.bh = xcd_bh(blockIdx.x, gridDim.x, a.Hqk, a.H);
  k.b = k.bh / a.H;
  k.h = k.bh % a.H;
  k.hq = k.h / (a.H / a.Hqk);
  const int Lg = a.L, H = a.H, HQ = a.Hqk;
  k.seg = blockIdx.y;
  k.nseg = gridDim.y;
  k.tb = a.seg_len > 0 ? k.seg * a.seg_len : 0;
  k.L = a.seg_len > 0 ? min(Lg - k.tb, a.seg_len) : Lg;
  k.Lnx = Lg - k.tb;
  k.nc = (k.L + CS - 1) / CS;
  k.ch0 = (long)k.bh * ((Lg + CS - 1) / CS) + k.tb / CS;
  k.ci_in = a.init_per_seg ? k.bh * k.nseg + k.seg : k.bh;
  k.ci_out = a.fin_per_seg ? k.bh * k.nseg + k.seg : k.bh;
  k.has_init = a.init_per_seg || k.seg == 0;
  k.fin_here = a.fin_per_seg || k.seg == k.nseg - 1;
  k.has_z = a.z != nullptr;
  k.Dh = a.D ? a.D[k.h] : 0.0f;
  k.gO = reinterpret_cast<T*>(a.out);
  k.gadt = a.adt + (long)k.bh * Lg + k.tb;
  k.gdt = a.dt + (long)k.bh * Lg + k.tb;
  k.gtr = a.trap + (long)k.bh * Lg + k.tb;
  const int AH = a.ang_shared ? 1 : H;                 // angle rows per token
  k.qk_stride = HQ * N;
  k.v_stride = H * P;
  k.a_stride = AH * R;
  // V and Z rows: contiguous (B, L, H, P), or in place in wider rows
  k.vz_stride = a.vz_tok ? (int)a.vz_tok : k.v_stride;
  const long vz_batch = a.vz_bat ? a.vz_bat : (long)Lg * k.v_stride;
  k.q_base = reinterpret_cast<const T*>(a.q) + ((long)k.b * Lg * HQ + k.hq) * N + (long)k.tb * k.qk_stride;
  k.k_base = reinterpret_cast<const T*>(a.k) + ((long)k.b * Lg * HQ + k.hq) * N + (long)k.tb * k.qk_stride;
  const long vz_row = (long)k.b * vz_batch + (long)k.h * P + (long)k.tb * k.vz_stride;
  k.v_base = reinterpret_cast<const T*>(a.v) + vz_row;
  k.z_base = reinterpret_cast<const T*>(a.z) + vz_row;
  k.o_base = k.gO + ((long)k.b * Lg * H + k.h) * P + (long)k.tb * k.v_stride;
  k.ang_base = a.ang + ((long)k.b * Lg * AH + (a.ang_shared ? 0 : k.h)) * R + (long)k.tb * k.a_stride;
  return k;
}

// The head's biases into LDS (read by every chunk's preparation).
template <int N, int NT>
__device__ __forceinline__ void stage_biases(float* qb, float* kb, const ScanArgs& a, int h, int tid) {
  for (int i = tid; i < N; i += NT) {
    qb[i] = a.qbias[(long)h * N + i];
    kb[i] = a.kbias[(long)h * N + i];
  }
}

// ---- staging of chunk c (G: the kernel's geometry, Sm its LDS layout, which holds the
// staging tiles rq, rk (by c % NQK), rv, ra (by parity) and rs: adt, dt, trap, [CS] the
// next chunk's first token).  Rows past the segment end are not loaded.
// Q and K rows: waves WQ0 / WQ1 the two halves of Q's (no Q in the state-only pass),
// WK0 / WK1 of K's.
template <typename G, bool SO, int WQ0, int WQ1, int WK0, int WK1, typename Sm, typename T>
__device__ __forceinline__ void stage_qk_chunk(Sm& sm, const ChunkBlock<T>& cb, int c, int wave, int lane) {
  constexpr int CS = G::CS;
  const int t0 = c * CS;
  const int valid = cb.L - t0;
  constexpr int JQ = CS * G::SQ / 64;
  const char* q0 = reinterpret_cast<const char*>(cb.q_base + (long)t0 * cb.qk_stride);
  const char* k0 = reinterpret_cast<const char*>(cb.k_base + (long)t0 * cb.qk_stride);
  lds_uint4* dq = (lds_uint4*)sm.rq[c % G::NQK];
  lds_uint4* dk = (lds_uint4*)sm.rk[c % G::NQK];
  if (!SO && wave == WQ0) stage_rows<CS, G::SQ, 0, JQ / 2>(dq, q0, cb.qk_stride * G::TS, valid, lane);
  if (!SO && wave == WQ1) stage_rows<CS, G::SQ, JQ / 2, JQ>(dq, q0, cb.qk_stride * G::TS, valid, lane);
  if (wave == WK0) stage_rows<CS, G::SQ, 0, JQ / 2>(dk, k0, cb.qk_stride * G::TS, valid, lane);
  if (wave == WK1) stage_rows<CS, G::SQ, JQ / 2, JQ>(dk, k0, cb.qk_stride * G::TS, valid, lane);
}
// V rows: wave WV.
template <typename G, int WV, typename Sm, typename T>
__device__ __forceinline__ void stage_v_chunk(Sm& sm, const ChunkBlock<T>& cb, int c, int wave, int lane) {
  constexpr int CS = G::CS;
  const int t0 = c * CS;
  constexpr int JV = CS * G::SV / 64;
  if (wave == WV) {
    const char* v0 = reinterpret_cast<const char*>(cb.v_base + (long)t0 * cb.vz_stride);
    stage_rows<CS, G::SV, 0, JV>((lds_uint4*)sm.rv[c & 1], v0, cb.vz_stride * G::TS, cb.L - t0, lane);
  }
}
// The rotation rates and the adt, dt, trap scalars (and dt, trap of the next chunk's
// first token, for the last key scale): wave WA.
template <typename G, int WA, typename Sm, typename T>
__device__ __forceinline__ void stage_ars_chunk(Sm& sm, const ChunkBlock<T>& cb, int c, int wave, int lane) {
  constexpr int CS = G::CS, R = G::R;
  const int t0 = c * CS;
  const int valid = cb.L - t0;
  constexpr int JA = CS * G::SA / 64;
  if (wave == WA) {
    if (R > 0) {
      const char* a0 = reinterpret_cast<const char*>(cb.ang_base + (long)t0 * cb.a_stride);
      stage_rows<CS, G::SA, 0, JA>((lds_uint4*)sm.ra[c & 1], a0, cb.a_stride * 4, valid, lane);
    }
    // the bases are made opaque here so that no derived pointer is hoisted out of the
    // chunk loop (and spilled)
    const float* pa = cb.gadt + t0;
    const float* pd = cb.gdt + t0;
    const float* pt = cb.gtr + t0;
    asm volatile("" : "+s"(pa), "+s"(pd), "+s"(pt));
    if (lane < CS && lane < valid) {
      lds_dma4(pa, 4u * lane, (lds_float*)&sm.rs[c & 1][0][0]);
      lds_dma4(pd, 4u * lane, (lds_float*)&sm.rs[c & 1][1][0]);
      lds_dma4(pt, 4u * lane, (lds_float*)&sm.rs[c & 1][2][0]);
    }
    if (lane == 0 && t0 + CS < cb.Lnx) {
      lds_dma4(pd, 4u * CS, (lds_float*)&sm.rs[c & 1][1][CS]);
      lds_dma4(pt, 4u * CS, (lds_float*)&sm.rs[c & 1][2][CS]);
    }
  }
}

// The staging tiles never hold uninitialised bits (rows past the sequence end are not
// loaded, and the preparation reads whole tiles).
template <typename G, typename Sm>
__device__ __forceinline__ void zero_staging(Sm& sm, int tid) {
  for (int i = tid; i < G::NQK * G::CS * G::SQ; i += G::NT) {
    (&sm.rq[0][0])[i] = make_uint4(0, 0, 0, 0);
    (&sm.rk[0][0])[i] = make_uint4(0, 0, 0, 0);
  }
  for (int i = tid; i < 2 * G::CS * G::SV; i += G::NT) (&sm.rv[0][0])[i] = make_uint4(0, 0, 0, 0);
  for (int i = tid; i < 2 * G::CS * G::SA; i += G::NT) (&sm.ra[0][0])[i] = make_uint4(0, 0, 0, 0);
  for (int i = tid; i < 2 * 3 * (G::CS + 4); i += G::NT) (&sm.rs[0][0][0])[i] = 0.0f;
}

// The effective state entering the segment, h0 + (1 - sigmoid(trap_0)) dt_0 (v0 (x) k0)
// from the carry (zero without one), as a state wave's accumulator tiles: column pcol
// of h^T, rows 16 nb + g4 + r.
template <typename G, typename T>
__device__ __forceinline__ void entering_state(f32x4 (&hs)[G::NB16], const ScanArgs& a, const ChunkBlock<T>& cb,
                                               bool swave, int pcol, int g4) {
  constexpr int N = G::N, P = G::P;
  const bool own = a.init_h && cb.has_init && swave;
  const float cinit = own ? (1.0f - sigmoid_fast(cb.gtr[0])) * cb.gdt[0] : 0.0f;
  const float v0 = own ? a.init_v[(long)cb.ci_in * P + pcol] : 0.0f;
#pragma unroll
  for (int nb = 0; nb < G::NB16; ++nb)
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int n = 16 * nb + g4 + r;
      hs[nb][r] = own ? a.init_h[((long)cb.ci_in * P + pcol) * N + n] + cinit * v0 * a.init_k[(long)cb.ci_in * N + n]
                      : 0.0f;
    }
}

// Per-token constants of a chunk (lane = token; lanes past CS take token 0's values,
// unused), from its scalars staged in rs and dt already read (s_dt, 0 past the end):
// gamma = dt sigmoid(trap), the key scale gamma_t + dt_{t+1} (1 - sigmoid(trap_{t+1}))
// (the last token reads the next chunk's first when there is one), the in-chunk prefix
// A_cum of adt and its value at the chunk end.
struct TokenScalars {
  float gam, scl, acum, aend;
};
template <int CS>
__device__ __forceinline__ TokenScalars token_scalars(const float (&rs)[3][CS + 4], float s_dt, bool tok, int tl,
                                                      int t0, int Lnx, int lane) {
  TokenScalars s;
  const float s_adt = tok ? rs[0][tl] : 0.0f;
  const float s_tr = tok ? rs[2][tl] : 0.0f;
  const float sig = sigmoid_fast(s_tr);
  s.gam = s_dt * sig;
  const float u = s_dt * (1.0f - sig);                                 // dt (1 - sigmoid), this token
  float un = __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(u), 0x130, 0xf, 0xf, false));  // next token
  if (lane == CS - 1) un = (t0 + CS < Lnx) ? rs[1][CS] * (1.0f - sigmoid_fast(rs[2][CS])) : 0.0f;
  s.scl = s.gam + un;
  s.acum = wave_incl_scan(lane < CS ? s_adt : 0.0f);
  s.aend = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(s.acum), CS - 1));
  return s;
}

// The final carry's k and v: k of the last token (kept in LDS by its preparation) and
// its v (still in the last chunk's staged rows).
template <typename G, typename Sm, typename T>
__device__ __forceinline__ void final_kv(const ScanArgs& a, Sm& sm, const ChunkBlock<T>& cb, int tid) {
  if (a.fin_k && cb.fin_here && cb.nc > 0) {
    for (int i = tid; i < G::N; i += G::NT) a.fin_k[(long)cb.ci_out * G::N + i] = sm.fink[i];
    for (int i = tid; i < G::P; i += G::NT)
      a.fin_v[(long)cb.ci_out * G::P + i] =
          Elem<T>::to_f(*staged_elem<G::SV, T>(sm.rv[(cb.nc - 1) & 1], cb.L - 1 - (cb.nc - 1) * G::CS, i));
  }
}

}  // namespace m3
