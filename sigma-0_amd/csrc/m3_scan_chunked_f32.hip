// Chunked Mamba3 SISO prefill scan with float32 I/O on CDNA4 matrix cores.
//
// The same operator as m3_scan_chunked.hip (the reference's mamba3_ssd_chunked_jax,
// phases 1-7, src/base_model/models/mamba3_jax.py:327-419), for the float32
// inputs the model hands its scan (mamba3.py:363-367 casts x, z, B and C to float32
// before mamba3_siso_triton), with float32 MFMA operands (v_mfma_f32_16x16x4_f32,
// float32 accumulation: exact float32 contractions) and 32-token chunks.
//
// The work is split differently from the bf16 kernel because a float32 MFMA costs
// 16 times a bf16 one per FLOP, so the matrix work must be spread over every SIMD:
// one workgroup of 12 waves per (batch, head) walks the chunks in order.  Output
// waves 0-2 each own one (query block, key block) item of Y_diag (an S^T block, the
// causal mask or the decay, M V over its keys), so three of the four SIMDs share it.
// State waves 4-7 each own 16 columns of the value dimension (a p-tile): h^T[:, p-tile]
// (all N rows) as 16x16 accumulators, that p-tile's Y_off = Q_r h^T and its state
// update.  Auxiliary waves 8-11 take the larger share of the preparation (the rope'd
// columns) and compute the next chunk's rotation angles while the others run the
// matrix work.  A chunk is two phases with a barrier after each:
//   preparation  lane = token: biases, rope and key scale into the Q/K tiles; the gate
//                and store of the previous chunk's Y; the direct-to-LDS loads of the
//                next chunk's Q and K
//   matrix       the loads of the next chunk's V and of the rates and scalars of the
//                chunk after, then the MFMA work
// The staged inputs are double-buffered by chunk parity; every input byte is read
// from HBM once and the output written once.
#include <type_traits>

#include "m3_chunk_block.h"

namespace m3 {
namespace chunked_f32 {

// Two inclusive scans over each 32-lane half of the wavefront on its own: the steps of
// wave_incl_scan without the carry from the lower half into the upper one.
__device__ __forceinline__ void half_incl_scan2(float v[2]) {
#pragma unroll
  for (int j = 0; j < 2; ++j) v[j] += dpp0<kDppRowShr1>(v[j]);
#pragma unroll
  for (int j = 0; j < 2; ++j) v[j] += dpp0<kDppRowShr2>(v[j]);
#pragma unroll
  for (int j = 0; j < 2; ++j) v[j] += dpp0<kDppRowShr4>(v[j]);
#pragma unroll
  for (int j = 0; j < 2; ++j) v[j] += dpp0<kDppRowShr8>(v[j]);
#pragma unroll
  for (int j = 0; j < 2; ++j) v[j] += dpp0<kDppRowBcast15, 0xa>(v[j]);
}

// Compile-time geometry of one instantiation.
template <typename T, int CS_, int N_, int P_, int R_, int NW_>
struct Geo : GeoBase<T, CS_, N_, P_, R_, NW_> {
  typedef GeoBase<T, CS_, N_, P_, R_, NW_> B;
  static constexpr int LDY = B::P + (B::BF ? 8 : 2);       // sY rows (io precision)
  // LDS bytes besides the Q/K staging.  The Q/K staging is double-buffered where it
  // fits; otherwise (rotation width N/2 at d_state 128) it is single-buffered and its
  // loads wait until the preparation phase has consumed it.
  static constexpr int FIXED = 2 * B::CS * B::LDQ * B::TS + 2 * B::CS * LDY * B::TS + 16 * LDY * B::TS +
                               (2 * B::CS * B::SV + 2 * B::CS * B::SA) * 16 + 2 * 3 * (B::CS + 4) * 4 + 8 * B::N +
                               2 * 6 * B::CS * 4 + 64;
  static constexpr bool DBQK = FIXED + 4 * B::CS * B::SQ * 16 <= 160 * 1024 - 512;
  static constexpr int NQK = DBQK ? 2 : 1;
  static_assert(B::SPT >= 1 && B::NST % B::PT == 0 && B::LB16 % B::SPT == 0, "state-wave split");
  // Q/K 8-column group k (< QGW) of a wave, or QG for none.  The first groups are the
  // rope columns, and their owner also computes their angles for the next chunk.  Full
  // pass: the output and auxiliary waves take the first groups, one each, so the angle
  // work stays off the state waves (the matrix phase ends with them); then the state
  // waves (which also run the gate in the preparation) and the auxiliary waves take
  // one each of the rest.  State-only pass
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
      if (wave < NWY) g = k == 0 ? wave : QG;
      else if (wave < NWY + NST) g = k == 0 ? NWY + NAUX + (wave - NWY) : QG;
      else g = k == 0 ? NWY + (wave - NWY - NST) : 2 * NWY + NAUX + (wave - NWY - NST);
    }
    return g < QG ? g : QG;
  }
};

template <typename G>
struct __attribute__((aligned(16))) Smem {
  typedef typename std::conditional<G::BF, bf16, float>::type T;
  T q[G::CS * G::LDQ];                   // rope'd Q rows
  T k[G::CS * G::LDQ];                   // rope'd, trapezoid-scaled K rows
  // Y before the gate, in two parts written by plain stores: the intra-chunk part
  // (output waves, by query block) and Q h^T (state waves, by p-tile; the gate applies
  // its e^{A_cum} row scale)
  alignas(16) T yd[G::CS * G::LDY];
  alignas(16) T yo[G::CS * G::LDY];
  alignas(16) T ydo[16 * G::LDY];        // the off-diagonal phase-3 item's part of rows 16..31
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
  // per-token chunk constants, by chunk parity
  alignas(16) float ac2[2][G::CS];       // A_cum * log2(e)
  alignas(16) float g16[2][G::CS];       // e^{A_e - A_cum}, A_e = A_cum at the end of the token's 16-block
  alignas(16) float expa[2][G::CS];      // e^{A_cum} (read by the gate, a chunk later)
  alignas(16) float dg[2][G::CS];        // gamma / scale: turns the S diagonal into the QK skip weight
  alignas(16) float scl[2][G::CS];       // trapezoid key scale gamma_t + dt_{t+1} (1 - sigmoid_{t+1})
  alignas(16) float wdec[2][G::CS];      // e^{A_end - A_cum}
  float dec[2];                          // e^{A_end}
  alignas(16) float fink[G::N];          // the last token's rope'd key (final carry), unscaled
};

// SO (state only): the pass that produces each segment's exit carry from a zero
// entering carry; it skips Q, Y_diag, Y_off, the gate and the output.
// SAVE (full pass): also write each chunk's entering state and angles (chunk_h,
// chunk_th), the residuals the backward reads instead of running the state-only pass,
// and with Z the output before the gate (out_v).
template <typename T, int CS, int N, int P, int R, int NW, bool SO, bool SAVE = false>
__global__ __launch_bounds__(64 * NW, 1)
void scan_chunked_f32_kernel(ScanArgs a) {
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
  T* gO = cb.gO;
  stage_biases<N, G::NT>(sm.qb, sm.kb, a, cb.h, tid);

  // ---- staging.  Q/K of chunk c into buffer c % NQK, V into parity c & 1, rotation
  // rates and scalars into parity c & 1.  A wave waits while the CU's load path drains
  // the loads queued ahead of its own, so they go to waves with slack: Q/K to the
  // output waves at the end of their preparation share (single-buffered Q/K: the
  // auxiliary waves, after the preparation barrier); V, rates and scalars to output
  // waves 0 and 1 (the two lightest query blocks) at the start of the matrix phase.
  constexpr int kWQ0 = G::DBQK ? 0 : 8, kWQ1 = G::DBQK ? 1 : 9, kWK0 = G::DBQK ? 2 : 10, kWK1 = G::DBQK ? 3 : 11;
  constexpr int kWV = 0, kWA = 1;
  auto stage_qk = [&](int c) { stage_qk_chunk<G, SO, kWQ0, kWQ1, kWK0, kWK1>(sm, cb, c, wave, lane); };
  auto stage_v = [&](int c) { stage_v_chunk<G, kWV>(sm, cb, c, wave, lane); };
  auto stage_ars = [&](int c) { stage_ars_chunk<G, kWA>(sm, cb, c, wave, lane); };

  // ---- gate (phase 7): thread -> (row, 8-column group) of a chunk's Y tile
  // (the state waves' threads: their share of the preparation is the lightest)
  constexpr int GROUPS = CS * (P / 8);
  static_assert(GROUPS <= 64 * G::NST, "the gate on the state waves' threads");
  const int gtid = tid - 64 * G::NWY;
  const int erow = max(gtid, 0) / (P / 8), egrp = max(gtid, 0) % (P / 8);
  const bool eact = gtid >= 0 && gtid < GROUPS;
  Vec8<T> zr;                              // Z of the chunk waiting for its gate
  zr.zero();
  auto load_z = [&](int c) {
    if (has_z && eact && c * CS + erow < L) zr.load(z_base + (long)(c * CS + erow) * vz_stride + 8 * egrp);
  };
  auto gate = [&](int c) {                 // Y of chunk c -> out
    if (eact && c * CS + erow < L) {
      const int off = erow * G::LDY + 8 * egrp;
      Vec8<T> ya, yb;
      ya.load(&sm.yd[off]);
      yb.load(&sm.yo[off]);
      const float ea = sm.expa[c & 1][erow];   // the e^{A_cum} row scale of Q h^T
      float o[8], ob[8];
      ya.to_f(o);
      yb.to_f(ob);
#pragma unroll
      for (int q = 0; q < 8; ++q) o[q] = fmaf(ob[q], ea, o[q]);
      if (erow >= 16) {                    // rows 16..31: the off-diagonal phase-3 item
        Vec8<T> yc;
        float oc[8];
        yc.load(&sm.ydo[(erow - 16) * G::LDY + 8 * egrp]);
        yc.to_f(oc);
#pragma unroll
        for (int q = 0; q < 8; ++q) o[q] += oc[q];
      }
      if constexpr (SAVE) {
        // the training forward: the output before the gate, for the backward's dZ
        if (has_z && a.out_v)
          store8(reinterpret_cast<T*>(a.out_v) + (o_base - gO) + (long)(c * CS + erow) * v_stride + 8 * egrp, o);
      }
      if (has_z) {
        float zf[8];
        zr.to_f(zf);
#pragma unroll
        for (int q = 0; q < 8; ++q) o[q] *= silu_fast(zf[q]);
      }
      store8(o_base + (long)(c * CS + erow) * v_stride + 8 * egrp, o);
    }
  };

  // ---- roles: output waves own query block lb = wave (all p-tiles); state waves own
  // p-tile pr (h^T[:, 16 pr + lane%16], all N rows, as 16x16 accumulators) and the
  // query blocks lb = part (mod SPT) of Y_off
  const bool ywave = wave < G::NWY;
  const bool swave = wave >= G::NWY && wave < G::NWY + G::NST;   // the rest are auxiliary
  const int sw = wave - G::NWY;
  const int pr = swave ? sw % G::PT : 0, part = swave ? sw / G::PT : 0;
  const int pcol = 16 * pr + (lane & 15);
  const int g4 = 4 * (lane >> 4);              // C-tile row offset of this lane
  f32x4 hs[G::NB16];
  entering_state<G>(hs, a, cb, swave, pcol, g4);
  // The Q/K column groups are worked on with two lanes per token: lane = token tkn
  // (< CS = 32) in half hf of the wave, which takes columns 8 g + 4 hf .. + 3 of group
  // g, i.e. its rope pairs 4 g + 2 hf + {0, 1}.
  static_assert(CS == 32, "two lanes per token");
  const int tkn = lane & (CS - 1), hf = lane / CS;
  float carry[G::QGW][2];                      // angles of this lane's two pairs, revolutions
#pragma unroll
  for (int k = 0; k < G::QGW; ++k)
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const int r = 4 * G::template qgroup<SO>(wave, k) + 2 * hf + j;
      carry[k][j] = (a.init_theta && has_init && r < R) ? a.init_theta[(long)ci_in * R + r] * kInvTwoPi : 0.0f;
    }
  zero_staging<G>(sm, tid);

  // ---- chunk constants and rotations of chunk cc, computed a chunk ahead.  Wave
  // kScalarWave writes the per-token constants to LDS (lane = token); every wave keeps
  // cos/sin of the angles of its own rope pairs in registers (two lanes per token).
  // (full pass: the last auxiliary wave, on the one SIMD without a phase-3 item)
  constexpr int kScalarWave = SO ? G::NWY + G::NST : G::NW - 1;
  float p_cs[G::QGW][2], p_sn[G::QGW][2];
  float logdec = 0.0f;                     // state-only pass: sum of the chunks' log-decays
  auto pre = [&](int cc) {
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
        sm.wdec[pb][lane] = exp2_fast((aend - acum) * kLog2e);
        sm.ac2[pb][lane] = acum * kLog2e;
        sm.expa[pb][lane] = exp2_fast(acum * kLog2e);
        sm.g16[pb][lane] = exp2_fast((ablk - acum) * kLog2e);
        sm.dg[pb][lane] = scl != 0.0f ? gam * rcp_fast(scl) : 0.0f;
        if (lane == 0) sm.dec[pb] = exp2_fast(aend * kLog2e);
        if constexpr (SO) logdec += aend;
      }
    }
#pragma unroll
    for (int k = 0; k < G::QGW; ++k) {
      const int g = G::template qgroup<SO>(wave, k);
      if (g < G::QG && 4 * g < R) {
        // two lanes per token (tkn, hf): this lane's pairs 4 g + 2 hf + {0, 1}
        const bool ttok = t0 + tkn < L;
        const float h_dt = ttok ? sm.rs[pb][1][tkn] : 0.0f;
        const uint4 rr = staged<G::SA>(sm.ra[pb], tkn, g);
        const float rav[2] = {__uint_as_float(hf ? rr.z : rr.x), __uint_as_float(hf ? rr.w : rr.y)};
        const float hdt = 0.5f * h_dt;
        // angle in revolutions: carry + prefix of tanh(rate) pi dt / 2pi = tanh(rate) dt / 2,
        // with tanh(x) = 1 - 2 / (1 + e^{2x}); the fractional part is the reference's
        // mod-2pi wrap, and the hardware sin/cos take revolutions
        float d[2];
#pragma unroll
        for (int j = 0; j < 2; ++j)
          d[j] = fmaf(-h_dt, rcp_fast(1.0f + exp2_fast(2.0f * kLog2e * rav[j])), hdt);   // dt = 0 past the end
        half_incl_scan2(d);                    // over the tokens, in each half
#pragma unroll
        for (int j = 0; j < 2; ++j) {
          const float th = __builtin_amdgcn_fractf(carry[k][j] + d[j]);
          // the angle entering chunk cc (revolutions), for the backward
          if constexpr (SO || SAVE) {
            if (a.chunk_th && tkn == 0) a.chunk_th[(ch0 + cc) * R + 4 * g + 2 * hf + j] = carry[k][j];
          }
          const float c0 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(th), CS - 1));
          const float c1 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(th), 2 * CS - 1));
          carry[k][j] = hf ? c1 : c0;
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
  pre(0);
  __syncthreads();   // chunk 0's per-token constants (one wave writes them) before its preparation

  for (int c = 0; c < nc; ++c) {
    const int t0 = c * CS;
    const int pc = c & 1;
    const uint4* sq = sm.rq[c % G::NQK];
    const uint4* sk = sm.rk[c % G::NQK];
    const uint4* sv = sm.rv[pc];

    // ================= preparation =================
    // Rows past the sequence end hold stale (finite) inputs: their key scale is 0,
    // so they add nothing to S or h, and their outputs are never stored.
    // Q/K column groups, two lanes per token: biases, rope, key scale
    const float hscl = sm.scl[pc][tkn];
#pragma unroll
    for (int k = 0; k < G::QGW; ++k) {
      const int g = G::template qgroup<SO>(wave, k);
      if (g < G::QG) {
        const int col = 8 * g + 4 * hf;        // this lane's 4 columns
        const uint4 qr = staged<G::SQ>(sq, tkn, 2 * g + hf), kr = staged<G::SQ>(sk, tkn, 2 * g + hf);
        const float4 qb = *reinterpret_cast<const float4*>(&sm.qb[col]);
        const float4 kb = *reinterpret_cast<const float4*>(&sm.kb[col]);
        float qf[4] = {__uint_as_float(qr.x) + qb.x, __uint_as_float(qr.y) + qb.y, __uint_as_float(qr.z) + qb.z,
                       __uint_as_float(qr.w) + qb.w};
        float kf[4] = {__uint_as_float(kr.x) + kb.x, __uint_as_float(kr.y) + kb.y, __uint_as_float(kr.z) + kb.z,
                       __uint_as_float(kr.w) + kb.w};
        if (4 * g < R) {
#pragma unroll
          for (int j = 0; j < 2; ++j) {
            const float cs = p_cs[k][j], sn = p_sn[k][j];
            const float q0 = qf[2 * j], q1 = qf[2 * j + 1];
            qf[2 * j] = q0 * cs - q1 * sn;
            qf[2 * j + 1] = q0 * sn + q1 * cs;
            const float k0 = kf[2 * j], k1 = kf[2 * j + 1];
            kf[2 * j] = k0 * cs - k1 * sn;
            kf[2 * j + 1] = k0 * sn + k1 * cs;
          }
        }
        if (t0 + tkn == L - 1) store4(&sm.fink[col], kf);   // the final carry's key, written after the loop
#pragma unroll
        for (int e = 0; e < 4; ++e) kf[e] *= hscl;
        if constexpr (!SO) store4(&sm.q[tkn * G::LDQ + col], qf);
        store4(&sm.k[tkn * G::LDQ + col], kf);
      }
    }
    // gate of the previous chunk (its Y tiles were written before the last barrier),
    // then Z for this chunk's gate, then the loads of the next chunks: the gate's wait
    // for Z comes before any of them is in flight
    if (!SO && c > 0) gate(c - 1);
    if (!SO) load_z(c);
    if (G::DBQK && c + 1 < nc) stage_qk(c + 1);
    __syncthreads();

    // single-buffered Q/K staging: every wave has read this chunk's rows
    if (!G::DBQK && c + 1 < nc) stage_qk(c + 1);
    if (c + 1 < nc) stage_v(c + 1);
    if (c + 2 < nc) stage_ars(c + 2);

    // ---- phase 3 as (query block lb, key block sb <= lb) items, one per output wave:
    // three at 32-token chunks, on three SIMDs (each also holds a state wave).  An item
    // is the 16 x 16 block S^T of keys 16 sb.. against queries 16 lb.., masked -- decayed
    // off the diagonal block; on it causal, with D + gamma QK on the diagonal -- then
    // M V over those 16 keys for every p-tile.  The diagonal items write their rows of
    // Y_diag to yd, the off-diagonal one to ydo, which the gate adds.  The S^T operands
    // are read four k-steps at a time: in step s of a 16-wide block of the d_state axis,
    // k slot i/16 of lane i stands for column k0 + 4 (i/16) + s in both operands (the
    // dot product is the same sum in another order), one 16-byte read per operand per
    // four MFMAs.
    auto diag_item = [&](auto lb_c, auto sb_c) {
      constexpr int lb = decltype(lb_c)::value, sb = decltype(sb_c)::value;
      static_assert(sb <= lb, "causal items only");
      // lane-derived addresses are recomputed here, not kept live across the loop
      int ln = lane;
      asm volatile("" : "+v"(ln));
      const int g4l = 4 * (ln >> 4);
      const int l = 16 * lb + (ln & 15);
      const float al = sm.ac2[pc][l];
      const float* kr = &sm.k[(16 * sb + (ln & 15)) * G::LDQ + 4 * (ln >> 4)];
      const float* qr = &sm.q[(16 * lb + (ln & 15)) * G::LDQ + 4 * (ln >> 4)];
      f32x4 st = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
      for (int k0 = 0; k0 < N; k0 += 16) {
        const float4 ka = *reinterpret_cast<const float4*>(kr + k0);
        const float4 qa = *reinterpret_cast<const float4*>(qr + k0);
        st = W::mma(ka.x, qa.x, st);
        st = W::mma(ka.y, qa.y, st);
        st = W::mma(ka.z, qa.z, st);
        st = W::mma(ka.w, qa.w, st);
      }
      const int s0 = 16 * sb + g4l;
      if constexpr (sb < lb) {
        // off-diagonal block: e^{A_l - A_s} = e^{A_l - A_e} e^{A_e - A_s}, both <= 1
        const float f = exp2_fast(fminf(al - sm.ac2[pc][16 * sb + 15], 0.0f));
        const float4 gg = *reinterpret_cast<const float4*>(&sm.g16[pc][s0]);
        st[0] *= f * gg.x; st[1] *= f * gg.y; st[2] *= f * gg.z; st[3] *= f * gg.w;
      } else {
        // diagonal block: causal decay below the diagonal; on it, D plus the
        // QK skip gamma_l (q_l . k_l) (the stored key carries the scale)
        const float dgl = sm.dg[pc][l];
        const float4 as = *reinterpret_cast<const float4*>(&sm.ac2[pc][s0]);
        const float asv[4] = {as.x, as.y, as.z, as.w};
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const float v = st[r] * exp2_fast(fminf(al - asv[r], 0.0f));
          st[r] = (s0 + r < l) ? v : (s0 + r == l ? Dh + st[r] * dgl : 0.0f);
        }
      }
      // M V: the A operand is the masked block itself (lane i, reg j: query l, key
      // 16 sb + 4 (i/16) + j), matched by V's rows
      f32x4 yd[G::PT];
#pragma unroll
      for (int pt = 0; pt < G::PT; ++pt)
#pragma unroll
        for (int r = 0; r < 4; ++r) yd[pt][r] = 0.0f;
#pragma unroll
      for (int j = 0; j < 4; ++j)
#pragma unroll
        for (int pt = 0; pt < G::PT; ++pt)
          yd[pt] = W::mma(st[j], W::template vdiag<G::SV>(sv, 16 * pt, 16 * sb, j, ln), yd[pt]);
      T* dst = sb == lb ? sm.yd + 16 * lb * G::LDY : sm.ydo;
#pragma unroll
      for (int pt = 0; pt < G::PT; ++pt)
#pragma unroll
        for (int r = 0; r < 4; r += 2)
          store_pair(&dst[(g4l + r) * G::LDY + 16 * pt + (ln & 15)],
                     &dst[(g4l + r + 1) * G::LDY + 16 * pt + (ln & 15)], yd[pt][r], yd[pt][r + 1]);
    };
    if (!SO && ywave) {                 // the state-only pass has no Y_diag
      static_assert(G::LB16 == 2 && G::NWY >= 3, "three phase-3 items on three output waves");
      if (wave == 0) diag_item(std::integral_constant<int, 0>{}, std::integral_constant<int, 0>{});
      if (wave == 1) diag_item(std::integral_constant<int, 1>{}, std::integral_constant<int, 1>{});
      if (wave == 2) diag_item(std::integral_constant<int, 1>{}, std::integral_constant<int, 0>{});
    } else if (swave) {
      // the state update's decay and per-token weights are read before this wave's
      // stores (a read issued after them would wait for them too)
      const float dec = sm.dec[pc];
      float wv[CS / W::KSTEP][W::WN];
      auto load_wv = [&]() {
#pragma unroll
        for (int ks = 0; ks < CS / W::KSTEP; ++ks) W::load_w(&sm.wdec[pc][W::ktok(ks * W::KSTEP, lane)], wv[ks]);
      };
      // ---- phase 6: Y_off = Q_r h^T for my p-tile, query blocks lb = part (mod SPT)
      if constexpr (!SO) {
      typename W::frag hf[G::BF ? N / 32 : 1];
      if constexpr (G::BF) {
#pragma unroll
        for (int q = 0; q < N / 32; ++q) hf[q] = W::hfrag(hs[2 * q], hs[2 * q + 1]);
      }
      constexpr int NLB = G::LB16 / G::SPT;
      f32x4 yo[NLB];
#pragma unroll
      for (int i = 0; i < NLB; ++i)
#pragma unroll
        for (int r = 0; r < 4; ++r) yo[i][r] = 0.0f;
      if constexpr (G::BF) {
        // per k-step the query blocks' fragments, then their chains side by side
#pragma unroll
        for (int q = 0; q < N / 32; ++q) {
          typename W::frag qa[NLB];
#pragma unroll
          for (int i = 0; i < NLB; ++i) qa[i] = W::qoff(sm.q, G::LDQ, 16 * (part + G::SPT * i), 32 * q, lane);
#pragma unroll
          for (int i = 0; i < NLB; ++i) yo[i] = W::mma(qa[i], hf[q], yo[i]);
        }
      } else {
#pragma unroll
        for (int nb = 0; nb < G::NB16; ++nb)
#pragma unroll
          for (int r = 0; r < 4; ++r)
#pragma unroll
            for (int i = 0; i < NLB; ++i) {
              const int l = 16 * (part + G::SPT * i) + (lane & 15);
              yo[i] = W::mma(sm.q[l * G::LDQ + 16 * nb + g4 + r], hs[nb][r], yo[i]);
            }
      }
      load_wv();
#pragma unroll
      for (int i = 0; i < NLB; ++i) {
        const int lb = part + G::SPT * i;
#pragma unroll
        for (int r = 0; r < 4; r += 2)
          store_pair(&sm.yo[(16 * lb + g4 + r) * G::LDY + pcol], &sm.yo[(16 * lb + g4 + r + 1) * G::LDY + pcol],
                     yo[i][r], yo[i][r + 1]);
      }
      } else {
        load_wv();
      }
      // ---- phases 4-5: h <- e^{A_end} h + K_s^T (w V) for my p-tile
      // the state entering chunk c, [p][n], for the backward
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
        const typename W::frag vb = W::scale(W::template vstate<G::SV>(sv, 16 * pr, ks * W::KSTEP, lane), wv[ks]);
#pragma unroll
        for (int nb = 0; nb < G::NB16; ++nb)
          hs[nb] = W::mma(W::kstate(sm.k, G::LDQ, ks * W::KSTEP, 16 * nb, lane), vb, hs[nb]);
      }
    }
    if (c + 1 < nc) pre(c + 1);
    __builtin_amdgcn_s_waitcnt(0);   // this wave's staged loads and gate stores are done
    __syncthreads();
  }
  if (!SO && nc > 0) gate(nc - 1);

  final_kv<G>(a, sm, cb, tid);
  if (a.fin_h && fin_here && swave && part == 0) {
#pragma unroll
    for (int nb = 0; nb < G::NB16; ++nb)
#pragma unroll
      for (int r = 0; r < 4; ++r) a.fin_h[((long)ci_out * P + pcol) * N + 16 * nb + g4 + r] = hs[nb][r];
  }
  if constexpr (SO) {
    if (a.fin_logdec && fin_here && wave == kScalarWave && lane == 0) a.fin_logdec[ci_out] = logdec;
  }
  if (a.fin_theta && fin_here && tkn == 0) {
#pragma unroll
    for (int k = 0; k < G::QGW; ++k)
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        const int r = 4 * G::template qgroup<SO>(wave, k) + 2 * hf + j;
        if (r < R) a.fin_theta[(long)ci_out * R + r] = carry[k][j] * kTwoPi;
      }
  }
}

}  // namespace chunked_f32

// ------------------------------------------------------------------ dispatch
// (chunk, d_state, headdim, rotation width) instantiations with float32 I/O; R is the
// model's rope_fraction 0.5 (R = N/4) or 1.0 (R = N/2) width.  Chunk sizes that are
// multiples of 32 run as 32-token sub-chunks (the chunked form is an exact rewrite of
// the token recurrence for every chunk size: only the rounding differs).
#define M3_F32_SHAPES(X)                                                                       \
  X(32, 128, 64, 32) X(32, 128, 64, 64) X(32, 64, 64, 16) X(32, 64, 64, 32) X(32, 64, 32, 16) \
  X(32, 32, 32, 8) X(32, 32, 64, 8)

constexpr int kF32Waves = 12;

static int f32_kernel_chunk(int CS) { return (CS > 32 && CS % 32 == 0) ? 32 : CS; }

bool scan_chunked_f32_supported(int CS_, int N, int P, int R) {
  const int CS = f32_kernel_chunk(CS_);
#define X(cs, n, p, r) \
  if (CS == cs && N == n && P == p && R == r) return true;
  M3_F32_SHAPES(X)
#undef X
  return false;
}

// shapes whose full pass can also write the chunk states (the backward's float32 shapes)
#define M3_F32_SAVE_SHAPES(X) X(32, 128, 64, 32) X(32, 128, 64, 64) X(32, 64, 64, 16) X(32, 64, 32, 16)

// the state-only pass of this kernel (the backward's chunk states) at the backward's
// float32 d_state-128 shapes
#define M3_F32_STATE_SHAPES(X) X(32, 128, 64, 32) X(32, 128, 64, 64)

bool scan_state_f32_supported(int CS_, int N, int P, int R) {
  const int CS = f32_kernel_chunk(CS_);
#define X(cs, n, p, r) \
  if (CS == cs && N == n && P == p && R == r) return true;
  M3_F32_STATE_SHAPES(X)
#undef X
  return false;
}

hipError_t scan_state_f32_launch(const ScanArgs& a, hipStream_t st) {
  const int CS = f32_kernel_chunk(a.CS);
  const int nseg = a.seg_len > 0 ? (a.L + a.seg_len - 1) / a.seg_len : 1;
#define X(cs, n, p, r)                                                                               \
  if (CS == cs && a.N == n && a.P == p && a.R == r) {                                                \
    hipLaunchKernelGGL((chunked_f32::scan_chunked_f32_kernel<float, cs, n, p, r, kF32Waves, true>),  \
                       dim3(a.B * a.H, nseg), dim3(64 * kF32Waves), 0, st, a);                       \
    return hipGetLastError();                                                                        \
  }
  M3_F32_STATE_SHAPES(X)
#undef X
  return hipErrorInvalidValue;
}

hipError_t scan_chunked_f32_launch(const ScanArgs& a, hipStream_t st) {
  const int CS = f32_kernel_chunk(a.CS);
  const int nseg = a.seg_len > 0 ? (a.L + a.seg_len - 1) / a.seg_len : 1;
  if (a.chunk_h) {
#define X(cs, n, p, r)                                                                                 \
  if (CS == cs && a.N == n && a.P == p && a.R == r) {                                                  \
    hipLaunchKernelGGL((chunked_f32::scan_chunked_f32_kernel<float, cs, n, p, r, kF32Waves, false, true>), \
                       dim3(a.B * a.H, nseg), dim3(64 * kF32Waves), 0, st, a);                         \
    return hipGetLastError();                                                                          \
  }
    M3_F32_SAVE_SHAPES(X)
#undef X
    return hipErrorInvalidValue;
  }
#define X(cs, n, p, r)                                                                                 \
  if (CS == cs && a.N == n && a.P == p && a.R == r) {                                                  \
    hipLaunchKernelGGL((chunked_f32::scan_chunked_f32_kernel<float, cs, n, p, r, kF32Waves, false>),   \
                       dim3(a.B * a.H, nseg), dim3(64 * kF32Waves), 0, st, a);                         \
    return hipGetLastError();                                                                          \
  }
  M3_F32_SHAPES(X)
#undef X
  return hipErrorInvalidValue;
}

}  // namespace m3
