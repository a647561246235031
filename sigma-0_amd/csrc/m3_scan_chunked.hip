// Chunked Mamba3 SISO prefill scan on CDNA4 matrix cores.
//
// Computes the reference's mamba3_ssd_chunked_jax (phases 1-7,
// src/base_model/models/mamba3_jax.py:327-419) in one kernel:
//   phase 1  per-chunk decay prefix (wave64 scan), rotation-angle prefix
//            (wave64 scans over the chunk, carried across chunks and range
//            reduced mod 2pi), trapezoid weights, biases, QK-dot skip, rope
//                                                                (:236-324)
//   phase 3  S^T = K Q_r^T on MFMA, causal decay mask (with the keys' trapezoid
//            scale) in registers, then Y_diag^T = V^T M^T on MFMA straight from
//            the S^T accumulators                                 (:371-393)
//   phase 6  Y_off^T = h Q_r^T on MFMA from the state kept in LDS  (:224-233)
//   phase 4-5 h <- e^{A_end} h + K^T (w V) on MFMA, h in fp32 accumulators
//                                                                (:177-222)
//   phase 7  (Y_diag + e^{A_cum} Y_off + (D + QK) V) * silu(Z), in the registers of
//            the wave that formed Y                               (:402-419)
//
// One workgroup of 12 waves per (batch, head) walks the chunks in order; the P x N
// fp32 state never leaves the registers of the state waves.  Output waves 0-3 each
// own a 16-row query block: its S^T, Y_diag, Y_off, the gate and the output store.
// State waves 4-7 each own 16 columns of the value dimension (a p-tile):
// h^T[:, p-tile] (all N rows) as 16x16 accumulators and its update; in the
// preparation phase they copy the state entering the chunk into LDS (io type), where
// the output waves read it for Y_off.  Auxiliary waves 8-11 take the larger share of
// the preparation (the rope'd columns) and compute the next chunk's rotation angles
// while the others run the matrix work.  A chunk is two phases with a barrier after
// each:
//   preparation  lane = token: biases and rope into the Q/K tiles; the state into
//                LDS; Z of the chunk into registers; the direct-to-LDS loads of the
//                next chunk's Q and K
//   matrix       the loads of the next chunk's V and of the rates and scalars of the
//                chunk after, then the MFMA work, with V read straight from its
//                staged rows and K^T from the K tile by transposed LDS reads; the
//                gate and the output store
// The staged inputs are double-buffered by chunk parity, so every load has a whole
// chunk to land; every input byte is read from HBM once and the output written once.
#include <type_traits>

#include "m3_chunk_block.h"

namespace m3 {

// Compile-time geometry of one instantiation.
template <typename T, int CS_, int N_, int P_, int R_, int NW_>
struct Geo : GeoBase<T, CS_, N_, P_, R_, NW_> {
  typedef GeoBase<T, CS_, N_, P_, R_, NW_> B;
  // LDS bytes besides the Q/K staging.  The Q/K staging is double-buffered where it
  // fits; otherwise (rotation width N/2 at d_state 128) it is single-buffered and its
  // loads wait until the preparation phase has consumed it.
  static constexpr int FIXED = (2 * B::CS + B::P) * B::LDQ * B::TS + (2 * B::CS * B::SV + 2 * B::CS * B::SA) * 16 +
                               2 * 3 * (B::CS + 4) * 4 + 12 * B::N + 2 * 6 * B::CS * 4 + 64;
  static constexpr bool DBQK = FIXED + 4 * B::CS * B::SQ * 16 <= 160 * 1024 - 512;
  static constexpr int NQK = DBQK ? 2 : 1;
  static_assert(B::SPT >= 1 && B::NST % B::PT == 0, "state-wave split");
  // Q/K 8-column group k (< QGW) of a wave, or QG for none.  The first groups are the
  // rope columns, and their owner also computes their angles for the next chunk.  Full
  // pass: the auxiliary waves take the first groups, two each, so the angle work stays
  // off the matrix waves; the remaining groups go one per matrix wave.  State-only pass
  // (no Q and no Y, so the output waves have no matrix work): the output waves and then
  // the auxiliary waves take the first groups, one each, and the state waves two each
  // of the rest, which halves the angle work per wave.
  template <bool SO>
  __device__ static int qgroup(int wave, int k) {
    constexpr int NWY = B::NWY, NST = B::NST, NAUX = B::NAUX, QG = B::QG;
    int g;
    if constexpr (SO) {
      if (wave < NWY) g = k == 0 ? wave : QG;
      else if (wave >= NWY + NST) g = k == 0 ? NWY + (wave - NWY - NST) : QG;
      else g = NWY + NAUX + 2 * (wave - NWY) + k;
    } else {
      g = wave >= NWY + NST ? 2 * (wave - NWY - NST) + k : 2 * NAUX + wave + (NWY + NST) * k;
    }
    return g < QG ? g : QG;
  }
};

template <typename G>
struct __attribute__((aligned(16))) Smem {
  typedef typename std::conditional<G::BF, bf16, float>::type T;
  T q[G::CS * G::LDQ];                   // rope'd Q rows
  T k[G::CS * G::LDQ];                   // rope'd K rows (without the trapezoid scale)
  T h[G::P * G::LDQ];                    // the state entering the chunk, h[p][n]
  // raw inputs staged by direct-to-LDS loads, by chunk parity: 16-byte slots, row t slot
  // s stored at t * S + (s ^ (t mod S)) so that a lane-per-row read is bank-conflict free
  alignas(16) uint4 rq[G::NQK][G::CS * G::SQ];
  alignas(16) uint4 rk[G::NQK][G::CS * G::SQ];
  alignas(16) uint4 rv[2][G::CS * G::SV];
  // rotation rates and adt, dt, trap ([CS]: the next chunk's first token), by chunk
  // parity: chunk c+1's angles and weights are computed during chunk c's matrix phase
  alignas(16) uint4 ra[2][G::CS * G::SA];
  alignas(16) float rs[2][3][G::CS + 4];
  alignas(16) float qb[G::N];            // biases of this head
  alignas(16) float kb[G::N];
  // per-token chunk constants, by chunk parity.  The K tile holds the keys without
  // their trapezoid scale: the scale of key s is a factor of every term key s adds (to
  // S and to the state), so it is folded into that key's decay factors below.
  alignas(16) float ac2[2][G::CS];       // A_cum * log2(e)
  alignas(16) float g16[2][G::CS];       // scale_s e^{A_e - A_cum}, A_e = A_cum at the end of the key's 16-block
  alignas(16) float expa[2][G::CS];      // e^{A_cum}: the row scale of Y_off
  alignas(16) float gam[2][G::CS];       // gamma_l: the weight of the QK skip term on the S diagonal
  alignas(16) float scl[2][G::CS];       // trapezoid key scale gamma_t + dt_{t+1} (1 - sigmoid_{t+1})
  alignas(16) float wdec[2][G::CS];      // scale_s e^{A_end - A_cum}
  float dec[2];                          // e^{A_end}
  alignas(16) float fink[G::N];          // the last token's rope'd key (final carry), unscaled
};

// Four elements held as raw bits (bf16: 8 bytes, f32: 16 bytes) as floats.
__device__ __forceinline__ void raw4_to_f(const uint2& r, float f[4]) {
  f[0] = __uint_as_float(r.x << 16); f[1] = __uint_as_float(r.x & 0xffff0000u);
  f[2] = __uint_as_float(r.y << 16); f[3] = __uint_as_float(r.y & 0xffff0000u);
}
__device__ __forceinline__ void raw4_to_f(const uint4& r, float f[4]) {
  f[0] = __uint_as_float(r.x); f[1] = __uint_as_float(r.y); f[2] = __uint_as_float(r.z); f[3] = __uint_as_float(r.w);
}

// SO (state only): the pass that produces each segment's exit carry from a zero
// entering carry; it skips Q, Y_diag, Y_off, the gate and the output.
// SAVE (full pass): also write each chunk's entering state and angles (chunk_h,
// chunk_th), the residuals the backward reads instead of running the state-only pass.
template <typename T, int CS, int N, int P, int R, int NW, bool SO, bool SAVE = false>
__global__ __launch_bounds__(64 * NW, 1)
void scan_chunked_kernel(ScanArgs a) {
  typedef Geo<T, CS, N, P, R, NW> G;
  typedef MF16<T> W;
  static_assert(sizeof(Smem<G>) <= 160 * 1024, "LDS budget");
  __shared__ Smem<G> sm;
  if constexpr (SO) {
    if (a.so_skip_last && blockIdx.y + 1 == gridDim.y) return;   // before any barrier: the whole block
  }

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  __builtin_assume(wave >= 0 && wave < NW);
  const ChunkBlock<T> cb = chunk_block<T, CS, N, P, R>(a);
  const int L = cb.L, Lnx = cb.Lnx, nc = cb.nc;
  const long ch0 = cb.ch0;
  const int ci_in = cb.ci_in, ci_out = cb.ci_out;
  const bool has_init = cb.has_init, fin_here = cb.fin_here, has_z = cb.has_z;
  const float Dh = cb.Dh;
  const int v_stride = cb.v_stride, vz_stride = cb.vz_stride;
  const T* z_base = cb.z_base;
  T* o_base = cb.o_base;
  stage_biases<N, G::NT>(sm.qb, sm.kb, a, cb.h, tid);

  // ---- staging.  Q/K of chunk c into buffer c % NQK, V into parity c & 1, rotation
  // rates and scalars into parity c & 1.  A wave waits while the CU's load path drains
  // the loads queued ahead of its own, so they go to waves with slack: Q/K to the
  // output waves at the end of their preparation share (single-buffered Q/K: the
  // auxiliary waves, after the preparation barrier); V, rates and scalars to two state
  // waves at the start of the matrix phase.  Every issuing wave waits for its loads
  // before the chunk's closing barrier (the output waves before their gate).
  constexpr int kWQ0 = G::DBQK ? 0 : 8, kWQ1 = G::DBQK ? 1 : 9, kWK0 = G::DBQK ? 2 : 10, kWK1 = G::DBQK ? 3 : 11;
  // V and the rates: state waves 6 and 7 in the full pass (the output waves carry the
  // chunk's longest work there), output waves 0 and 1 in the state-only pass (idle
  // after the preparation, while the state waves' update ends the chunk)
  constexpr int kWV = SO ? 0 : 6, kWA = SO ? 1 : 7;
  auto stage_qk = [&](int c) { stage_qk_chunk<G, SO, kWQ0, kWQ1, kWK0, kWK1>(sm, cb, c, wave, lane); };
  auto stage_v = [&](int c) { stage_v_chunk<G, kWV>(sm, cb, c, wave, lane); };
  auto stage_ars = [&](int c) { stage_ars_chunk<G, kWA>(sm, cb, c, wave, lane); };

  // ---- roles: output waves own query block lb = wave (all p-tiles); state waves own
  // p-tile pr (h^T[:, 16 pr + lane%16], all N rows, as 16x16 accumulators)
  const bool ywave = wave < G::NWY;
  const bool swave = wave >= G::NWY && wave < G::NWY + G::NST;   // the rest are auxiliary
  const int sw = wave - G::NWY;
  const int pr = swave ? sw % G::PT : 0, part = swave ? sw / G::PT : 0;
  const int pcol = 16 * pr + (lane & 15);
  const int g4 = 4 * (lane >> 4);              // C-tile row offset of this lane
  f32x4 hs[G::NB16];
  entering_state<G>(hs, a, cb, swave, pcol, g4);
  float carry[G::QGW][4];
#pragma unroll
  for (int k = 0; k < G::QGW; ++k)
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int r = 4 * G::template qgroup<SO>(wave, k) + j;
      carry[k][j] = (a.init_theta && has_init && r < R) ? a.init_theta[(long)ci_in * R + r] * kInvTwoPi : 0.0f;  // revolutions
    }
  zero_staging<G>(sm, tid);

  // ---- Z of the chunk in the layout of an output wave's Y^T tiles: lane -> query row
  // 16 wave + lane%16 and, per p-tile, the 4 columns 16 pt + 4 (lane/16) + 0..3
  typedef typename std::conditional<G::BF, uint2, uint4>::type Z4;
  Z4 zr[G::PT];
  auto load_z = [&](int c) {
    const int l = 16 * wave + (lane & 15);
    if (has_z && ywave && 16 * wave < CS && c * CS + l < L) {
      const T* zp = z_base + (long)(c * CS + l) * vz_stride + g4;
#pragma unroll
      for (int pt = 0; pt < G::PT; ++pt) zr[pt] = *reinterpret_cast<const Z4*>(zp + 16 * pt);
    }
  };

  // ---- chunk constants and rotations of chunk cc, computed a chunk ahead: lane = token.
  // Wave kScalarWave writes the per-token constants to LDS; every wave keeps cos/sin of
  // the angles of its own rope pairs in registers.
  // (wave 8 shares a SIMD with the lightest output wave)
  constexpr int kScalarWave = G::NWY + G::NST;
  float p_cs[G::QGW][4], p_sn[G::QGW][4];
  float logdec = 0.0f;                     // state-only pass: sum of the chunks' log-decays
  // rope_c: whether the calling role's waves can own rope groups (a compile-time flag,
  // so that the loops of the other roles keep no angle registers live)
  auto pre = [&](int cc, auto rope_c) {
    constexpr bool RP = decltype(rope_c)::value;
    const int t0 = cc * CS;
    const int pb = cc & 1;
    const bool tok = lane < CS && t0 + lane < L;
    const int tl = lane < CS ? lane : 0;
    const float s_dt = tok ? sm.rs[pb][1][tl] : 0.0f;
    if (wave == kScalarWave) {
      const TokenScalars ts = token_scalars<CS>(sm.rs[pb], s_dt, tok, tl, t0, Lnx, lane);
      const float gam = ts.gam, scl = ts.scl, acum = ts.acum, aend = ts.aend;
      if (lane < CS) {
        const float ablk = __shfl(acum, lane | 15, 64);
        sm.scl[pb][lane] = scl;
        sm.wdec[pb][lane] = exp2_fast((aend - acum) * kLog2e) * scl;
        sm.ac2[pb][lane] = acum * kLog2e;
        sm.expa[pb][lane] = exp2_fast(acum * kLog2e);
        sm.g16[pb][lane] = exp2_fast((ablk - acum) * kLog2e) * scl;
        sm.gam[pb][lane] = gam;
        if (lane == 0) sm.dec[pb] = exp2_fast(aend * kLog2e);
        if constexpr (SO) logdec += aend;
      }
    }
#pragma unroll
    for (int k = 0; k < G::QGW; ++k) {
      const int g = G::template qgroup<SO>(wave, k);
      if (RP && g < G::QG && 4 * g < R) {
        const uint4 rr = staged<G::SA>(sm.ra[pb], tl, g);
        const float rav[4] = {__uint_as_float(rr.x), __uint_as_float(rr.y), __uint_as_float(rr.z),
                              __uint_as_float(rr.w)};
        const float hdt = 0.5f * s_dt;
        // angle in revolutions: carry + prefix of tanh(rate) pi dt / 2pi = tanh(rate) dt / 2,
        // with tanh(x) = 1 - 2 / (1 + e^{2x}); the fractional part is the reference's
        // mod-2pi wrap, and the hardware sin/cos take revolutions
        float d[4];
#pragma unroll
        for (int j = 0; j < 4; ++j)
          d[j] = fmaf(-s_dt, rcp_fast(1.0f + exp2_fast(2.0f * kLog2e * rav[j])), hdt);   // s_dt = 0 past the end
        wave_incl_scan4(d);
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const float th = __builtin_amdgcn_fractf(carry[k][j] + d[j]);
          // the angle entering chunk cc (revolutions), for the backward
          if constexpr (SO || SAVE) {
            if (a.chunk_th && lane == 0) a.chunk_th[(ch0 + cc) * R + 4 * g + j] = carry[k][j];
          }
          carry[k][j] = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(th), CS - 1));
          p_cs[k][j] = __builtin_amdgcn_cosf(th);
          p_sn[k][j] = __builtin_amdgcn_sinf(th);
        }
      }
    }
  };

  __syncthreads();
  stage_qk(0);
  stage_v(0);
  stage_ars(0);
  if (nc > 1) stage_ars(1);
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  pre(0, std::true_type{});
  __syncthreads();   // chunk 0's per-token constants (one wave writes them) before its preparation

  // ================= preparation, lane = token: this wave's Q/K column groups =========
  // (biases and rope into the Q/K tiles).  Rows past the sequence end hold stale
  // (finite) inputs: their key scale is 0, so they add nothing to S or h, and their
  // outputs are never stored.
  auto prep_groups = [&](int c, auto rope_c) {
    constexpr bool RP = decltype(rope_c)::value;
    const int t0 = c * CS;
    const bool tok = lane < CS && t0 + lane < L;
    const int tl = lane < CS ? lane : 0;        // staging row of this lane
    const uint4* sq = sm.rq[c % G::NQK];
    const uint4* sk = sm.rk[c % G::NQK];
#pragma unroll
    for (int k = 0; k < G::QGW; ++k) {
      const int g = G::template qgroup<SO>(wave, k);
      if (g < G::QG) {
        float qf[8], kf[8];
        {
          Vec8<T> qv, kv;
          if constexpr (G::BF) {
            qv.raw_set(staged<G::SQ>(sq, tl, g));
            kv.raw_set(staged<G::SQ>(sk, tl, g));
          } else {
            qv.raw_set2(staged<G::SQ>(sq, tl, 2 * g), staged<G::SQ>(sq, tl, 2 * g + 1));
            kv.raw_set2(staged<G::SQ>(sk, tl, 2 * g), staged<G::SQ>(sk, tl, 2 * g + 1));
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
          }
        }
        if (RP && 4 * g < R) {
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            const float cs = p_cs[k][j], sn = p_sn[k][j];
            const float q0 = qf[2 * j], q1 = qf[2 * j + 1];
            qf[2 * j] = q0 * cs - q1 * sn;
            qf[2 * j + 1] = q0 * sn + q1 * cs;
            const float k0 = kf[2 * j], k1 = kf[2 * j + 1];
            kf[2 * j] = k0 * cs - k1 * sn;
            kf[2 * j + 1] = k0 * sn + k1 * cs;
          }
        }
        if (tok && t0 + lane == L - 1) store8(&sm.fink[8 * g], kf);   // the final carry's key, written after the loop
        if (lane < CS) {
          if constexpr (!SO) store8(&sm.q[lane * G::LDQ + 8 * g], qf);
          store8(&sm.k[lane * G::LDQ + 8 * g], kf);
        }
      }
    }
  };

  // ---- query rows l in [16 lb, 16 lb + 16), all p-tiles (output wave lb).  The
  // products are formed transposed (Y^T = V^T M^T and h Q_r^T), so each lane holds 4
  // consecutive p of one query row: the gate and the store need no exchange.
  //   phase 3  Y_diag^T = V^T mask(K Q_r^T), the mask's diagonal carrying D + gamma QK
  //   phase 6  Y_off^T = h Q_r^T, scaled by the row's e^{A_cum}
  //   phase 7  (Y_diag + Y_off) silu(Z), stored
  // Instantiated per query block so every loop over key blocks is static.
  auto out_block = [&](auto lb_c, int c) {
    constexpr int lb = decltype(lb_c)::value;
    const int t0 = c * CS;
    const int pc = c & 1;
    const uint4* sv = sm.rv[pc];
    // lane-derived addresses are recomputed here, not kept live across the loop
    int ln = lane;
    asm volatile("" : "+v"(ln));
    const int g4l = 4 * (ln >> 4);
    const int l = 16 * lb + (ln & 15);
    const float al = sm.ac2[pc][l];
    const float gl = sm.gam[pc][l];
    constexpr int NK = N / W::KSTEP;
    f32x4 st[lb + 2];
#pragma unroll
    for (int sb = 0; sb < lb + 2; ++sb)
#pragma unroll
      for (int r = 0; r < 4; ++r) st[sb][r] = 0.0f;
    {
      // query fragments first (B operand of every S^T block), then the key blocks'
      // chains side by side
      typename W::frag qf[NK];
#pragma unroll
      for (int kk = 0; kk < NK; ++kk) qf[kk] = W::ld(sm.q, G::LDQ, 16 * lb, kk * W::KSTEP, ln);
#pragma unroll
      for (int kk = 0; kk < NK; ++kk)
#pragma unroll
        for (int sb = 0; sb <= lb; ++sb)
          st[sb] = W::mma(W::ld(sm.k, G::LDQ, 16 * sb, kk * W::KSTEP, ln), qf[kk], st[sb]);
    }
    // the V operands, requested before the mask arithmetic so that it covers their latency
    constexpr int NSP = lb / 2 + 1;
    typename W::frag vf[NSP][W::STEPS][G::PT];
#pragma unroll
    for (int i = 0; i < NSP; ++i)
#pragma unroll
      for (int j = 0; j < W::STEPS; ++j)
#pragma unroll
        for (int pt = 0; pt < G::PT; ++pt) vf[i][j][pt] = W::template vdiag<G::SV>(sv, 16 * pt, 32 * i, j, ln);
#pragma unroll
    for (int sb = 0; sb <= lb; ++sb) {
      const int s0 = 16 * sb + g4l;
      if (sb < lb) {
        // off-diagonal block: e^{A_l - A_s} = e^{A_l - A_e} e^{A_e - A_s}, both <= 1 (the
        // second carries the key scale)
        const float f = exp2_fast(fminf(al - sm.ac2[pc][16 * sb + 15], 0.0f));
        const float4 gg = *reinterpret_cast<const float4*>(&sm.g16[pc][s0]);
        st[sb][0] *= f * gg.x; st[sb][1] *= f * gg.y; st[sb][2] *= f * gg.z; st[sb][3] *= f * gg.w;
      } else {
        // diagonal block: causal decay times the key scale below the diagonal; on it,
        // D plus the QK skip gamma_l (q_l . k_l)
        const float4 as = *reinterpret_cast<const float4*>(&sm.ac2[pc][s0]);
        const float4 sc = *reinterpret_cast<const float4*>(&sm.scl[pc][s0]);
        const float asv[4] = {as.x, as.y, as.z, as.w};
        const float scv[4] = {sc.x, sc.y, sc.z, sc.w};
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const float v = st[sb][r] * exp2_fast(fminf(al - asv[r], 0.0f)) * scv[r];
          st[sb][r] = (s0 + r < l) ? v : (s0 + r == l ? Dh + st[sb][r] * gl : 0.0f);
        }
      }
    }
    f32x4 yd[G::PT];
#pragma unroll
    for (int pt = 0; pt < G::PT; ++pt)
#pragma unroll
      for (int r = 0; r < 4; ++r) yd[pt][r] = 0.0f;
#pragma unroll
    for (int i = 0; i < NSP; ++i) {
#pragma unroll
      for (int j = 0; j < W::STEPS; ++j) {
        const typename W::frag mf = W::from_acc(st[2 * i], st[2 * i + 1], j);
#pragma unroll
        for (int pt = 0; pt < G::PT; ++pt) yd[pt] = W::mma(vf[i][j][pt], mf, yd[pt]);
      }
    }
    // Y_off^T = h Q_r^T: the query fragments again (B), the state rows (A)
    f32x4 yo[G::PT];
#pragma unroll
    for (int pt = 0; pt < G::PT; ++pt)
#pragma unroll
      for (int r = 0; r < 4; ++r) yo[pt][r] = 0.0f;
#pragma unroll
    for (int kk = 0; kk < NK; ++kk) {
      const typename W::frag qk = W::ld(sm.q, G::LDQ, 16 * lb, kk * W::KSTEP, ln);
#pragma unroll
      for (int pt = 0; pt < G::PT; ++pt) yo[pt] = W::mma(W::ld(sm.h, G::LDQ, 16 * pt, kk * W::KSTEP, ln), qk, yo[pt]);
    }
    const float ea = sm.expa[pc][l];
    // this wave's staged loads (issued in the preparation phase) and Z have landed
    __builtin_amdgcn_s_waitcnt(0);
    if (t0 + l < L) {
      T* op = o_base + (long)(t0 + l) * v_stride + g4l;
#pragma unroll
      for (int pt = 0; pt < G::PT; ++pt) {
        float y4[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) y4[r] = fmaf(yo[pt][r], ea, yd[pt][r]);
        if (has_z) {
          float z4[4];
          raw4_to_f(zr[pt], z4);
#pragma unroll
          for (int r = 0; r < 4; ++r) y4[r] *= silu_fast(z4[r]);
        }
        store4(op + 16 * pt, y4);
      }
    }
  };

  // final carry, the parts held in registers: this wave's rope angles (and, for the
  // state-only pass's scalar wave, the total log-decay)
  auto fin_regs = [&](auto rope_c) {
    constexpr bool RP = decltype(rope_c)::value;
    if (RP && a.fin_theta && fin_here && lane == 0) {
#pragma unroll
      for (int k = 0; k < G::QGW; ++k)
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const int r = 4 * G::template qgroup<SO>(wave, k) + j;
          if (r < R) a.fin_theta[(long)ci_out * R + r] = carry[k][j] * kTwoPi;
        }
    }
    if constexpr (SO) {
      if (a.fin_logdec && fin_here && wave == kScalarWave && lane == 0) a.fin_logdec[ci_out] = logdec;
    }
  };

  // ---- the chunk loop, one per role: the roles share no loop-carried registers
  // (the state accumulators live only in the state waves' loop), and every loop passes
  // the same two barriers per chunk.  In the full pass the auxiliary waves own the
  // first 2 NAUX groups, so at rope widths up to 8 NAUX (the model's N/4 included) the
  // output and state waves own no rope group.
  const std::integral_constant<bool, SO || (R > 8 * G::NAUX)> rys{};
  if (ywave) {
    for (int c = 0; c < nc; ++c) {
      prep_groups(c, rys);
      // Z for this chunk's gate, then the loads of the next chunk's Q/K
      if (!SO) load_z(c);
      if (G::DBQK && c + 1 < nc) stage_qk(c + 1);
      __syncthreads();
      if constexpr (SO) {
        if (c + 1 < nc) stage_v(c + 1);
        if (c + 2 < nc) stage_ars(c + 2);
      }
      if constexpr (!SO) {
        if (wave == 0) out_block(std::integral_constant<int, 0>{}, c);
        if (wave == 1) out_block(std::integral_constant<int, 1>{}, c);
        if constexpr (G::LB16 > 2) {
          if (wave == 2) out_block(std::integral_constant<int, 2>{}, c);
          if (wave == 3) out_block(std::integral_constant<int, 3>{}, c);
        }
      }
      if (c + 1 < nc) pre(c + 1, rys);
      // staged loads have landed before the barrier (a wave with a query block waited
      // before its gate, so that the gate's stores are not waited for)
      if (SO || 16 * wave >= CS) __builtin_amdgcn_s_waitcnt(0);
      __syncthreads();
    }
    fin_regs(rys);
  } else if (swave) {
    for (int c = 0; c < nc; ++c) {
      const int pc = c & 1;
      prep_groups(c, rys);
      // the state entering this chunk, h[p][n] in the io type, for the output waves'
      // Y_off (the state waves of a p-tile hold it alike; the first writes it)
      if (!SO && part == 0) {
#pragma unroll
        for (int nb = 0; nb < G::NB16; ++nb) {
          const float hv[4] = {hs[nb][0], hs[nb][1], hs[nb][2], hs[nb][3]};
          store4(&sm.h[pcol * G::LDQ + 16 * nb + g4], hv);
        }
      }
      __syncthreads();
      if constexpr (!SO) {
        if (c + 1 < nc) stage_v(c + 1);
        if (c + 2 < nc) stage_ars(c + 2);
      }
      {
        // lane-derived addresses are recomputed here, not kept live across the loop
        int ln = lane;
        asm volatile("" : "+v"(ln));
        const uint4* sv = sm.rv[pc];
        const float dec = sm.dec[pc];
        float wv[CS / W::KSTEP][W::WN];
#pragma unroll
        for (int ks = 0; ks < CS / W::KSTEP; ++ks) W::load_w(&sm.wdec[pc][W::ktok(ks * W::KSTEP, ln)], wv[ks]);
        // ---- phases 4-5: h <- e^{A_end} h + K^T (w V) for my p-tile
        // the state entering chunk c, for the backward
        if constexpr (SO || SAVE) {
          if (a.chunk_h && part == 0) {
            T* dst = reinterpret_cast<T*>(a.chunk_h) + (ch0 + c) * P * N;
#pragma unroll
            for (int nb = 0; nb < G::NB16; ++nb) {
              const float hv[4] = {hs[nb][0], hs[nb][1], hs[nb][2], hs[nb][3]};
              store4(dst + saved_tile_off<N>(pr, nb, lane), hv);
            }
          }
        }
#pragma unroll
        for (int nb = 0; nb < G::NB16; ++nb)
#pragma unroll
          for (int r = 0; r < 4; ++r) hs[nb][r] *= dec;
#pragma unroll
        for (int ks = 0; ks < CS / W::KSTEP; ++ks) {
          const typename W::frag vb = W::scale(W::template vstate<G::SV>(sv, 16 * pr, ks * W::KSTEP, ln), wv[ks]);
#pragma unroll
          for (int nb = 0; nb < G::NB16; ++nb)
            hs[nb] = W::mma(W::kstate(sm.k, G::LDQ, ks * W::KSTEP, 16 * nb, ln), vb, hs[nb]);
        }
      }
      if (c + 1 < nc) pre(c + 1, rys);
      __builtin_amdgcn_s_waitcnt(0);
      __syncthreads();
    }
    fin_regs(rys);
    if (a.fin_h && fin_here && part == 0) {
#pragma unroll
      for (int nb = 0; nb < G::NB16; ++nb)
#pragma unroll
        for (int r = 0; r < 4; ++r) a.fin_h[((long)ci_out * P + pcol) * N + 16 * nb + g4 + r] = hs[nb][r];
    }
  } else {
    for (int c = 0; c < nc; ++c) {
      prep_groups(c, std::true_type{});
      __syncthreads();
      // single-buffered Q/K staging: every wave has read this chunk's rows
      if (!G::DBQK && c + 1 < nc) stage_qk(c + 1);
      if (c + 1 < nc) pre(c + 1, std::true_type{});
      __builtin_amdgcn_s_waitcnt(0);
      __syncthreads();
    }
    fin_regs(std::true_type{});
  }

  final_kv<G>(a, sm, cb, tid);
}

// ------------------------------------------------------------------ dispatch
// (dtype, chunk, d_state, headdim, rotation width) instantiations; R is the
// model's rope_fraction 0.5 (R = N/4) or 1.0 (R = N/2) width, or 0.
// float32 I/O has its own kernel (m3_scan_chunked_f32.hip).
#define M3_CHUNK_SHAPES(X)                                                                         \
  X(bf16, 64, 128, 64, 32) X(bf16, 64, 128, 64, 64) X(bf16, 64, 128, 64, 0)                        \
  X(bf16, 64, 128, 32, 32) X(bf16, 64, 64, 64, 16) X(bf16, 64, 64, 64, 32)                         \
  X(bf16, 64, 64, 32, 16) X(bf16, 64, 32, 32, 8) X(bf16, 64, 32, 64, 8)                            \
  X(bf16, 32, 128, 64, 32) X(bf16, 32, 64, 64, 16) X(bf16, 32, 64, 32, 16) X(bf16, 32, 128, 32, 32)

constexpr int kChunkWaves = 12;

// The chunked form is an exact rewrite of the token recurrence for every chunk size,
// so the kernel's blocking changes only the rounding, not the function computed:
// bf16 runs chunk sizes that are multiples of 64 as 64-token sub-chunks, fp32 (twice
// the LDS per token) multiples of 32 as 32-token sub-chunks.
static int kernel_chunk(bool bf16_io, int CS) {
  const int k = bf16_io ? 64 : 32;
  return (CS > k && CS % k == 0) ? k : CS;
}

bool scan_chunked_supported(bool bf16_io, int CS_, int N, int P, int R) {
  if (!bf16_io) return scan_chunked_f32_supported(CS_, N, P, R);
  const int CS = kernel_chunk(bf16_io, CS_);
#define X(T, cs, n, p, r) \
  if ((std::is_same<T, bf16>::value == bf16_io) && CS == cs && N == n && P == p && R == r) return true;
  M3_CHUNK_SHAPES(X)
#undef X
  return false;
}

// bf16 shapes whose full pass can also write the chunk states (the backward's shapes)
#define M3_SAVE_SHAPES(X) \
  X(bf16, 64, 128, 64, 32) X(bf16, 64, 128, 64, 64) X(bf16, 64, 128, 64, 0) X(bf16, 64, 64, 64, 16) X(bf16, 64, 64, 32, 16)

hipError_t scan_chunked_launch(const ScanArgs& a, bool bf16_io, hipStream_t st) {
  if (!bf16_io) return scan_chunked_f32_launch(a, st);
  const int CS = kernel_chunk(bf16_io, a.CS);
  const int nseg = a.seg_len > 0 ? (a.L + a.seg_len - 1) / a.seg_len : 1;
  if (a.chunk_h) {
#define X(T, cs, n, p, r)                                                                            \
  if (CS == cs && a.N == n && a.P == p && a.R == r) {                                                \
    hipLaunchKernelGGL((scan_chunked_kernel<T, cs, n, p, r, kChunkWaves, false, true>), dim3(a.B * a.H, nseg), \
                       dim3(64 * kChunkWaves), 0, st, a);                                             \
    return hipGetLastError();                                                                         \
  }
    M3_SAVE_SHAPES(X)
#undef X
    return hipErrorInvalidValue;
  }
#define X(T, cs, n, p, r)                                                                            \
  if ((std::is_same<T, bf16>::value == bf16_io) && CS == cs && a.N == n && a.P == p && a.R == r) {   \
    hipLaunchKernelGGL((scan_chunked_kernel<T, cs, n, p, r, kChunkWaves, false>), dim3(a.B * a.H, nseg), \
                       dim3(64 * kChunkWaves), 0, st, a);                                             \
    return hipGetLastError();                                                                         \
  }
  M3_CHUNK_SHAPES(X)
#undef X
  return hipErrorInvalidValue;
}

// The state-only pass: the sequence split's first pass (bf16, d_state 128, headdim
// 64) and the backward's chunk states (the backward's shapes; float32 at d_state 128
// runs the float32 kernel's state-only pass).
#define M3_STATE_SHAPES(X)                                                                  \
  X(bf16, 64, 128, 64, 32) X(bf16, 64, 128, 64, 64) X(bf16, 64, 128, 64, 0)                 \
  X(bf16, 64, 64, 64, 16) X(bf16, 64, 64, 32, 16) X(float, 32, 64, 64, 16) X(float, 32, 64, 32, 16)

bool scan_state_supported(bool bf16_io, int CS_, int N, int P, int R) {
  if (!bf16_io && scan_state_f32_supported(CS_, N, P, R)) return true;
  const int CS = kernel_chunk(bf16_io, CS_);
#define X(T, cs, n, p, r) \
  if ((std::is_same<T, bf16>::value == bf16_io) && CS == cs && N == n && P == p && R == r) return true;
  M3_STATE_SHAPES(X)
#undef X
  return false;
}

hipError_t scan_state_launch(const ScanArgs& a, bool bf16_io, hipStream_t st) {
  if (!bf16_io && scan_state_f32_supported(a.CS, a.N, a.P, a.R)) return scan_state_f32_launch(a, st);
  const int CS = kernel_chunk(bf16_io, a.CS);
  const int nseg = a.seg_len > 0 ? (a.L + a.seg_len - 1) / a.seg_len : 1;
#define X(T, cs, n, p, r)                                                                           \
  if ((std::is_same<T, bf16>::value == bf16_io) && CS == cs && a.N == n && a.P == p && a.R == r) {  \
    hipLaunchKernelGGL((scan_chunked_kernel<T, cs, n, p, r, kChunkWaves, true>), dim3(a.B * a.H, nseg), \
                       dim3(64 * kChunkWaves), 0, st, a);                                            \
    return hipGetLastError();                                                                        \
  }
  M3_STATE_SHAPES(X)
#undef X
  return hipErrorInvalidValue;
}

}  // namespace m3
