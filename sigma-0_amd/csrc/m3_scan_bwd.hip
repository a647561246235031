// Backward of the chunked Mamba3 SISO scan on CDNA4 matrix cores.
//
// Gradients of every input of mamba3_siso_triton (the reference's custom_vjp,
// src/base_model/models/mamba3_ops.py:821-902, output order (dQ, dK, dV, dADT, dDT,
// dTrap, dQ_bias, dK_bias, dAngles, dD, dZ)).  With q~ = rot(q + qb), k~ = scale
// rot(k + kb), A the running sum of adt and dy = dOut silu(z):
//
//   y_t   = sum_{s<t} (q~_t . k~_s) e^{A_t - A_s} v_s + (D + gamma_t (q^.k^)_t) v_t
//   dv_s  = sum_{t>s} (q~_t . k~_s) e^{A_t - A_s} dy_t + (D + QK_s) dy_s
//   dq~_t = sum_{s<t} e^{A_t - A_s} (dy_t . v_s) k~_s
//   dk~_s = sum_{t>s} e^{A_t - A_s} (dy_t . v_s) q~_t
//   dA_t  = q~_t . dq~_t - k~_t . dk~_t,   dadt = reverse cumsum of dA
//
// and the chain through rope, bias, trapezoid weights and the angle cumsum.  The
// chunk-level form needs, for every chunk c, the state h_c entering it and the
// adjoint state G_c = sum_{t after chunk c} e^{A_t - A_end(c)} dy_t (x) q~_t after it.
// h_c and the rope angle entering chunk c come from the chunked kernel's state-only
// pass (scan_state_launch with chunk_h/chunk_th) or, in the training pair, from the
// training forward's residuals.  Then one of two routes, picked by B*H (bwd_walk):
//
// * The reverse walk (B*H >= 80: one workgroup per (b, h) fills the chip).
//   scan_bwd_walk_kernel walks each (b, h) from its last chunk to its first with
//   G in MFMA accumulators for the whole walk; per chunk it forms S and dP, y (for
//   dZ) and dV, advances G, then runs the dq~/dk~ passes (software-pipelined:
//   products of one column block beside the chain rule of the previous) and the
//   per-token dA.  It carries the reverse cumsums of dA and d(theta) from chunk to
//   chunk and sums the bias and D gradients over the walk.
//   scan_bwd_walk_finish_kernel then applies the trapezoid and angle chains and
//   the blend of the reverse and forward sums to dADT, dAngles, dDT and dTrap,
//   and scan_bwd_reduce_kernel sums the bias and D partials over the batch.
// * The chunk-parallel route (few (b, h) pairs).  scan_adjoint_kernel walks each
//   (b, h) backwards and saves every G_c; scan_bwd_chunk_kernel, one workgroup per
//   (chunk, b, h), computes the chunk's terms from h_c and G_c on MFMA: dZ, dV, dQ,
//   dK, and per token dA, d(theta), d(scale), d(gamma) (kept in the dADT, dAngles,
//   dTrap, dDT outputs); scan_bwd_finish_kernel turns those into dADT, dAngles, dDT,
//   dTrap (reverse cumsums over the sequence, the trapezoid and angle chains), and
//   scan_bwd_reduce_kernel sums the bias and D gradients over batch and chunks.
// With Q/K shared over heads (GQA, the fused path) the per-head dQ/dK and dAngles
// are summed by scan_bwd_gqa_kernel and scan_bwd_angle_heads_kernel.  Every sum runs
// in a fixed order, so the gradients are deterministic.
#include <stdlib.h>
#include <string.h>

#include <algorithm>
#include <type_traits>

#include "m3_chunk_common.h"

namespace m3 {
namespace {

constexpr int kBwdWaves = 8;
constexpr int kBwdThreads = 64 * kBwdWaves;

// Angle increment of a token in revolutions, tanh(rate) pi dt / 2pi, with the same
// arithmetic as the forward kernel (so the saved chunk angles continue exactly).
__device__ __forceinline__ float angle_step(float rate, float dt) {
  const float rcp = rcp_fast(1.0f + exp2_fast(2.0f * kLog2e * rate));
  return fmaf(-dt, rcp, 0.5f * dt);
}

// Rotate the four rope pairs of 8-column group g by the token's angles th4 (inverse
// rotation with sgn = -1); pairs r >= R pass through.
template <int R>
__device__ __forceinline__ void rope8(float x[8], const float th4[4], int g, float sgn) {
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int r = 4 * g + j;
    if (r < R) {
      const float c = __builtin_amdgcn_cosf(th4[j]), s = sgn * __builtin_amdgcn_sinf(th4[j]);
      const float x0 = x[2 * j], x1 = x[2 * j + 1];
      x[2 * j] = x0 * c - x1 * s;
      x[2 * j + 1] = x0 * s + x1 * c;
    }
  }
}

// The same rotation with the pairs' cosines and sines given.
template <int R>
__device__ __forceinline__ void rot8(float x[8], const float cs[4], const float sn[4], int g, float sgn) {
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    if (4 * g + j < R) {
      const float c = cs[j], s = sgn * sn[j];
      const float x0 = x[2 * j], x1 = x[2 * j + 1];
      x[2 * j] = x0 * c - x1 * s;
      x[2 * j + 1] = x0 * s + x1 * c;
    }
  }
}

// rot8 for a lane that holds PRS of the group's four pairs (2 PRS columns); rope: the
// group's pairs are rope pairs (R is a multiple of 4, so all four or none are).
template <int PRS>
__device__ __forceinline__ void rotp(float* x, const float* cs, const float* sn, bool rope, float sgn) {
  if (!rope) return;
#pragma unroll
  for (int j = 0; j < PRS; ++j) {
    const float c = cs[j], s = sgn * sn[j];
    const float x0 = x[2 * j], x1 = x[2 * j + 1];
    x[2 * j] = x0 * c - x1 * s;
    x[2 * j + 1] = x0 * s + x1 * c;
  }
}

// Inclusive scans over the tokens of a chunk: over the 64 lanes (4 values: one lane
// per token) or over each 32-lane half (2 values: two lanes per token, the halves
// holding the same tokens and different pairs).
template <int PRS>
__device__ __forceinline__ void token_scan(float* v) {
  if constexpr (PRS == 4) {
    wave_incl_scan4(v);
  } else {
    static_assert(PRS == 2, "one or two lanes per token");
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
}

// The total of a token scan: the value in the last lane of the lane's token range.
template <int PRS>
__device__ __forceinline__ float token_scan_total(float v, int hf) {
  if constexpr (PRS == 4) {
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 63));
  } else {
    const float t0 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 31));
    const float t1 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 63));
    return hf ? t1 : t0;
  }
}

// Sum of a token's value over its TPL lanes (lanes l and l + 32 at two lanes per token).
template <int TPL>
__device__ __forceinline__ float token_pair_sum(float v) {
  if constexpr (TPL == 1) return v;
  else return v + __shfl_xor(v, 32, 64);
}

__device__ __forceinline__ float wave_sum(float v) { return group_sum<64>(v); }

// Reverse inclusive scan over the 64 lanes (lane i gets the sum over lanes >= i).
__device__ __forceinline__ float wave_rev_scan(float v, int lane) {
  v = __shfl(v, 63 - lane, 64);
  v = wave_incl_scan(v);
  return __shfl(v, 63 - lane, 64);
}

template <typename T>
__device__ __forceinline__ void load8(const T* p, float f[8]) {
  Vec8<T> v;
  v.load(p);
  v.to_f(f);
}

struct BwdArgs {
  ScanArgs s;                  // forward inputs and dims (s.CS: the kernel chunk)
  const void* dout;
  void* dq; void* dk; void* dv; void* dz;
  float* dadt; float* ddt; float* dtrap; float* dang; float* dqb; float* dkb; float* dD;
  const void* hs;              // [bh][nc][P][N] T: state entering each chunk
  void* gs;                    // [bh][nc][N][P] T: adjoint state after each chunk
  const float* th0;            // [bh][nc][R] revolutions: angle entering each chunk
  float* pqb; float* pkb;      // [bh][nc][N] partial bias gradients
  float* pd;                   // [bh][nc] partial D gradient
  void* dqh; void* dkh;        // GQA: per-head dQ, dK (B, L, H, N) in the I/O type, else null
  float* dsc;                  // [bh][L] d(scale) per token
  float* ctot;                 // [bh][nc][1 + R] chunk sums of dA and of d(theta) per pair
  int nc;
  const void* yv;              // (B, L, H, P) T: the output before the gate, saved by the
                               // training forward (the walk then forms dZ = y_v fz), or null
  // The walk split into segments of seg_nc chunks (nseg > 1: grid (B*H, nseg)), for few
  // (b, h) pairs.  Partials (pqb, pkb, pd, ctot) are then per (b, h, segment), and the
  // walk of segment i starts from gin[bh][i] ([p][n] f32), the adjoint state after it.
  // The adjoint-only pass runs adj_sub sub-segments per walk segment (more workgroups
  // in flight than the walk's one per segment).
  int nseg = 1, seg_nc = 0, adj_sub = 1;
  float* gin = nullptr;        // [bh][nseg][P][N] adjoint entering each segment from the right
  float* gloc = nullptr;       // [bh][nseg * adj_sub][P][N] each sub-segment's own adjoint
  float* dseg = nullptr;       // [bh][nseg * adj_sub] each sub-segment's total log-decay
  // Rows of V and Z (s.vz_tok, s.vz_bat) and of dV and dZ (dvz_tok, dvz_bat): element
  // offset b * bat + t * tok + h * P.  The launcher sets both, to the contiguous
  // (B, L, H, P) layout's L H P and H P where the caller gives none.  dOut and the
  // saved output before the gate stay contiguous.
  long dvz_tok = 0, dvz_bat = 0;
};

// Per-chunk token constants shared by the adjoint and gradient kernels: lane = token.
template <int CS>
__device__ __forceinline__ void chunk_scalars(const BwdArgs& a, int bh, int t0, int lane, float* ac, float* gam,
                                              float* scl, float* dtv, float* aend) {
  const int L = a.s.L;
  const bool tok = lane < CS && t0 + lane < L;
  const long base = (long)bh * L + t0;
  const float adt = tok ? a.s.adt[base + lane] : 0.0f;
  const float dt = tok ? a.s.dt[base + lane] : 0.0f;
  const float tr = tok ? a.s.trap[base + lane] : 0.0f;
  const float sg = 1.0f / (1.0f + expf(-tr));
  const float gm = dt * sg;
  float un = __shfl_down(dt * (1.0f - sg), 1, 64);                  // next token's dt (1 - sigmoid)
  if (lane == CS - 1) {
    const bool nxt = t0 + CS < L;
    const float dtn = nxt ? a.s.dt[base + CS] : 0.0f, trn = nxt ? a.s.trap[base + CS] : 0.0f;
    un = dtn * (1.0f - 1.0f / (1.0f + expf(-trn)));
  }
  const float acum = wave_incl_scan(lane < CS ? adt : 0.0f);
  const float ae = __shfl(acum, CS - 1, 64);
  if (lane < CS) {
    ac[lane] = acum;
    gam[lane] = gm;
    scl[lane] = tok ? gm + un : 0.0f;
    dtv[lane] = dt;
  }
  if (lane == 0) *aend = ae;
}

// Rope angles (revolutions) of this lane's token for the pairs 4g..4g+3 of column
// group g: the angle entering the chunk plus a wave scan of the increments.  The
// rates are requested first (group_rates) and used later, so that their load latency
// overlaps the other loads of the kernel.  Call with the whole wave (g uniform).
// Lanes past the sequence end read the last token's row (a valid address), so the
// load is unconditional and nothing waits on it until its use; their dt is 0, which
// makes their angle increments 0.
template <int CS, int R>
__device__ __forceinline__ float4 group_rates(const BwdArgs& a, int b, int h, int t0, int g, int lane) {
  float4 rt = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
  if constexpr (R > 0) {
    const int L = a.s.L, H = a.s.H;
    const int t = min(t0 + lane, L - 1);
    const long arow = a.s.ang_shared ? (long)b * L + t : ((long)b * L + t) * H + h;
    if (4 * g < R) rt = *reinterpret_cast<const float4*>(a.s.ang + arow * R + 4 * g);
  }
  return rt;
}
template <int CS, int R>
__device__ __forceinline__ void group_theta(const BwdArgs& a, int bh, int c, int g, float4 rt, float dt,
                                            float th4[4]) {
#pragma unroll
  for (int j = 0; j < 4; ++j) th4[j] = 0.0f;
  if constexpr (R > 0) {
    if (4 * g >= R) return;
    const float rv[4] = {rt.x, rt.y, rt.z, rt.w};
    const float* t0c = a.th0 + ((long)bh * a.nc + c) * R + 4 * g;
#pragma unroll
    for (int j = 0; j < 4; ++j)
      if (4 * g + j < R) th4[j] = __builtin_amdgcn_fractf(t0c[j] + wave_incl_scan(angle_step(rv[j], dt)));
  }
}

// ------------------------------------------------------------------ adjoint pass
template <typename T, int CS, int N, int P, int R>
struct AdjSmem {
  static constexpr int PAD = std::is_same<T, bf16>::value ? 8 : 4;
  alignas(16) T qt[CS][N + PAD];      // q~ of the chunk
  alignas(16) T dye[CS][P + PAD];     // e^{A_cum} dy
  float qb[N];                         // the head's Q bias
};

// One chunk's inputs of the adjoint pass, requested a chunk ahead of their use (lane
// = token; the wave's Q groups g = wave + 8 k and dOut/Z groups likewise).  Every load
// is unconditional, from a clamped valid address: lanes past the sequence end read the
// last token's row, and their values are ignored (dt = 0 there makes their angle
// increments 0, and their q~ and dy are stored as zeros).
template <typename T, int CS, int N, int P, int R>
struct AdjLoads {
  static constexpr int GQ = (N / 8 + kBwdWaves - 1) / kBwdWaves;
  static constexpr int GV = (P / 8 + kBwdWaves - 1) / kBwdWaves;
  Vec8<T> q[GQ], dy[GV], z[GV];
  float4 rt[GQ], th[GQ];
  float adt, dt;
  __device__ __forceinline__ void issue(const BwdArgs& a, int c, int bh, int wave, int lane) {
    const int L = a.s.L, H = a.s.H, HQ = a.s.Hqk, b = bh / H, h = bh % H, hq = h / (H / HQ);
    const int t = min(c * CS + (lane & (CS - 1)), L - 1);
    adt = a.s.adt[(long)bh * L + t];
    dt = a.s.dt[(long)bh * L + t];
#pragma unroll
    for (int k = 0; k < GQ; ++k) {
      const int g = min(wave + kBwdWaves * k, N / 8 - 1);
      q[k].load(reinterpret_cast<const T*>(a.s.q) + (((long)b * L + t) * HQ + hq) * N + 8 * g);
      rt[k] = th[k] = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
      if constexpr (R > 0) {
        const int gr = min(g, R / 4 - 1);
        const long arow = a.s.ang_shared ? (long)b * L + t : ((long)b * L + t) * H + h;
        rt[k] = *reinterpret_cast<const float4*>(a.s.ang + arow * R + 4 * gr);
        th[k] = *reinterpret_cast<const float4*>(a.th0 + ((long)bh * a.nc + c) * R + 4 * gr);
      }
    }
    const T* gdo = reinterpret_cast<const T*>(a.dout) + (((long)b * L + t) * H + h) * P;
    const T* gz = a.s.z ? reinterpret_cast<const T*>(a.s.z) + a.s.vz_bat * b + a.s.vz_tok * t + (long)h * P : gdo;
#pragma unroll
    for (int k = 0; k < GV; ++k) {
      const int g = min(wave + kBwdWaves * k, P / 8 - 1);
      dy[k].load(gdo + 8 * g);
      z[k].load(gz + 8 * g);
    }
  }
};

// SEG: the split walk's adjoint-only pass.  Block (bh, j) walks sub-segment j + adj_sub
// (sub-segment k of walk segment i is number i adj_sub + k; those of walk segment 0
// are never needed) from a zero adjoint and leaves its own adjoint state, sum over its
// tokens of e^{A_t - A(sub-segment start)} dy_t (x) q~_t, in gloc ([p][n] f32), and its
// total log-decay in dseg; no per-chunk states are stored.  Two blocks fit a CU.
template <typename T, int CS, int N, int P, int R, bool SEG>
__global__ __launch_bounds__(kBwdThreads, SEG ? 2 : 1)
void scan_adjoint_kernel(BwdArgs a) {
  typedef MF16<T> W;
  typedef AdjSmem<T, CS, N, P, R> S;
  typedef AdjLoads<T, CS, N, P, R> Loads;
  __shared__ S sm;
  constexpr int PAD = S::PAD, KS = W::KSTEP;
  constexpr int NTILE = (P / 16) * (N / 16), TPW = (NTILE + kBwdWaves - 1) / kBwdWaves;
  static_assert(R % 4 == 0, "rope pairs in whole 8-column groups");
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int bh = blockIdx.x, h = bh % a.s.H;
  const int L = a.s.L, nc = a.nc;
  // SEG: sub-segment j of the walk's segments; its chunks (none when a short last
  // walk segment leaves it empty)
  const int sub = SEG ? (int)blockIdx.y + a.adj_sub : 0;
  const int sub_nc = (a.seg_nc + a.adj_sub - 1) / a.adj_sub;
  const int s0 = (sub / a.adj_sub) * a.seg_nc, s1 = min(nc, s0 + a.seg_nc);
  const int c_lo = SEG ? min(s1, s0 + (sub % a.adj_sub) * sub_nc) : 0;
  const int c_hi = SEG ? min(s1, c_lo + sub_nc) : nc;
  const bool has_z = a.s.z != nullptr;
  T* gs = reinterpret_cast<T*>(a.gs);
  for (int i = tid; i < N; i += kBwdThreads) sm.qb[i] = a.s.qbias[(long)h * N + i];

  f32x4 G[TPW];
#pragma unroll
  for (int i = 0; i < TPW; ++i) G[i] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
  float logdec = 0.0f;                                 // SEG: the segment's total log-decay

  Loads cur;
  if (c_hi > c_lo) cur.issue(a, c_hi - 1, bh, wave, lane);
  __syncthreads();                                     // the biases
  for (int c = c_hi - 1; c >= c_lo; --c) {
    const int t0 = c * CS;
    // adjoint state beyond chunk c, [n][p]
    if constexpr (!SEG) {
#pragma unroll
      for (int i = 0; i < TPW; ++i) {
        const int tile = wave + kBwdWaves * i;
        if (tile < NTILE) {
          const int pt = tile / (N / 16), nt = tile % (N / 16);
          const int n = 16 * nt + (lane & 15), p = 16 * pt + 4 * (lane >> 4);
          const float gv[4] = {G[i][0], G[i][1], G[i][2], G[i][3]};
          store4(gs + (((long)bh * nc + c) * N + n) * P + p, gv);
        }
      }
    }
    // lane = token; every wave forms the chunk's decay prefix itself
    const bool tok = lane < CS && t0 + lane < L;
    const float dtl = tok ? cur.dt : 0.0f;
    const float acum = wave_incl_scan(tok ? cur.adt : 0.0f);
    const float aend = __shfl(acum, CS - 1, 64);
#pragma unroll
    for (int k = 0; k < Loads::GQ; ++k) {
      const int g = wave + kBwdWaves * k;
      if (g < N / 8) {
        float q[8], th4[4];
        cur.q[k].to_f(q);
#pragma unroll
        for (int j = 0; j < 4; ++j) th4[j] = 0.0f;
        if constexpr (R > 0) {
          if (4 * g < R) {
            // R is a multiple of 4: the group's four pairs all rotate; their angle
            // prefixes advance side by side
            const float rv[4] = {cur.rt[k].x, cur.rt[k].y, cur.rt[k].z, cur.rt[k].w};
            const float t0c[4] = {cur.th[k].x, cur.th[k].y, cur.th[k].z, cur.th[k].w};
            float st[4];
#pragma unroll
            for (int j = 0; j < 4; ++j) st[j] = angle_step(rv[j], dtl);
            wave_incl_scan4(st);
#pragma unroll
            for (int j = 0; j < 4; ++j) th4[j] = __builtin_amdgcn_fractf(t0c[j] + st[j]);
          }
        }
#pragma unroll
        for (int e = 0; e < 8; ++e) q[e] = tok ? q[e] + sm.qb[8 * g + e] : 0.0f;
        rope8<R>(q, th4, g, 1.0f);
        if (lane < CS) store8(&sm.qt[lane][8 * g], q);
      }
    }
    // the decay and gate factors with the walk's arithmetic
    const float ea = tok ? exp2_fast(acum * kLog2e) : 0.0f;
#pragma unroll
    for (int k = 0; k < Loads::GV; ++k) {
      const int g = wave + kBwdWaves * k;
      if (g < P / 8) {
        float dy[8], z[8];
        cur.dy[k].to_f(dy);
        cur.z[k].to_f(z);
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          if (has_z) dy[e] *= z[e] * sigmoid_fast(z[e]);
          dy[e] *= ea;
        }
        if (lane < CS) store8(&sm.dye[lane][8 * g], dy);
      }
    }
    // every use of this chunk's loads is above: request the next chunk's
    if (c > c_lo) cur.issue(a, c - 1, bh, wave, lane);
    __syncthreads();
    // G <- e^{A_end} G + sum_t e^{A_cum,t} dy_t (x) q~_t
    const float dec = exp2_fast(aend * kLog2e);
    logdec += aend;
#pragma unroll
    for (int i = 0; i < TPW; ++i) {
      const int tile = wave + kBwdWaves * i;
      if (tile < NTILE) {
        const int pt = tile / (N / 16), nt = tile % (N / 16);
        f32x4 acc = G[i] * dec;
#pragma unroll
        for (int k0 = 0; k0 < CS; k0 += KS)
          acc = W::mma(ld_tr(&sm.dye[0][0], P + PAD, k0, 16 * pt, lane), ld_tr(&sm.qt[0][0], N + PAD, k0, 16 * nt, lane),
                       acc);
        G[i] = acc;
      }
    }
    __syncthreads();
  }
  if constexpr (SEG) {
    const long slot = (long)bh * a.nseg * a.adj_sub + sub;
#pragma unroll
    for (int i = 0; i < TPW; ++i) {
      const int tile = wave + kBwdWaves * i;
      if (tile < NTILE) {
        const int pt = tile / (N / 16), nt = tile % (N / 16);
        const int n = 16 * nt + (lane & 15), p = 16 * pt + 4 * (lane >> 4);
#pragma unroll
        for (int r = 0; r < 4; ++r) a.gloc[(slot * P + p + r) * N + n] = G[i][r];
      }
    }
    if (tid == 0) a.dseg[slot] = logdec;
  }
}

// The split walk's combine, thread = adjoint element (p, n) of one (b, h): walking the
// sub-segments from the last, g_j = gloc_j + e^{dseg_j} g_{j+1} is the adjoint after
// sub-segment j - 1, so at the first sub-segment of walk segment i + 1 it is the
// adjoint entering walk segment i from the right (the last walk segment starts from
// zero and reads nothing).
__global__ __launch_bounds__(256)
void seg_adjoint_combine_kernel(BwdArgs a) {
  const int bh = blockIdx.y, PN = a.s.P * a.s.N, k = a.adj_sub;
  const int e = blockIdx.x * 256 + threadIdx.x;
  if (e >= PN) return;
  const long l0 = (long)bh * a.nseg * k, i0 = (long)bh * a.nseg;
  float g = 0.0f;
  for (int j = a.nseg * k - 1; j >= k; --j) {
    g = a.gloc[(l0 + j) * PN + e] + expf(a.dseg[l0 + j]) * g;
    if (j % k == 0) a.gin[(i0 + j / k - 1) * PN + e] = g;
  }
}

// ------------------------------------------------------------ per-chunk gradients
template <typename T, int CS, int N, int P, int R>
struct GradSmem {
  static constexpr int PAD = std::is_same<T, bf16>::value ? 8 : 4;
  static constexpr int NH = N / 2;     // dq~ / dk~ are formed half the columns at a time
  alignas(16) T qt[CS][N + PAD];       // q~
  alignas(16) T kt[CS][N + PAD];       // k~
  alignas(16) T v[CS][P + PAD];
  alignas(16) T dy[CS][P + PAD];
  alignas(16) T fz[CS][P + PAD];       // dOut sigmoid(z) (1 + z (1 - sigmoid(z))): dZ = y fz
  alignas(16) T h[P][N + PAD];         // state entering the chunk
  alignas(16) T gt[N][P + PAD];        // adjoint state after the chunk, [n][p]
  alignas(16) T sm[CS][CS + PAD];      // S masked and decayed
  alignas(16) T dpm[CS][CS + PAD];     // dP masked and decayed
  alignas(16) float res[CS][NH + 4];   // dq~ or dk~ of half the columns
  // bf16: what q~ (k~) lost to rounding, for half the columns: dq~ and dk~ take
  // their q~ / k~ operand as hi + lo (the angle gradient cancels to a small sum)
  alignas(16) T lo[CS][NH + PAD];
  float ac[CS], gam[CS], scl[CS], dtv[CS], qk[CS], dqk[CS];
  float pq[N / 8][CS];                 // per column group: q^.k^, then q~.dq~ - k~.dk~
  float ps[N / 8][CS];                 // per column group: dk~ . rot(k^)
  float pv[P / 8][CS];                 // per value group: dy.v
  float aend;
};

// The global inputs of one (chunk, b, h) item of the chunk-gradient kernel, loaded into
// registers: the two saved states, this thread's Q/K rows (two column groups) and
// V/dOut/Z rows (one value group), the rates of its rope pairs and dt.  Every load is
// unconditional, from a clamped valid address where a lane or wave has nothing to load
// (past the sequence end, beyond the column groups), so the compiler never waits on one
// before its use; the unused values are zeroed or ignored there.
template <typename T, int CS, int N, int P, int R>
struct ItemLoads {
  static constexpr int GH = N / 16;                                       // column groups per half
  static constexpr int HP = (P * N / 8 + kBwdThreads - 1) / kBwdThreads;  // 8-element state pieces per thread
  static constexpr int VGW = (P / 8 + kBwdWaves - 1) / kBwdWaves;         // value groups per wave
  Vec8<T> hpc[HP], gpc[HP], qraw[2], kraw[2], vraw[VGW], dyraw[VGW], zraw[VGW];
  float4 rates[2];
  float dtraw;
  __device__ __forceinline__ void issue(const BwdArgs& a, int c, int bh, int tid, int wave, int lane) {
    const int b = bh / a.s.H, h = bh % a.s.H, hq = h / (a.s.H / a.s.Hqk);
    const int L = a.s.L, H = a.s.H, HQ = a.s.Hqk, nc = a.nc, t0 = c * CS;
    const int tcl = min(t0 + lane, L - 1);
    const long qrow = (((long)b * L + tcl) * HQ + hq) * N;
    const long vrow = (((long)b * L + tcl) * H + h) * P;                 // dOut
    const long vzrow = a.s.vz_bat * b + a.s.vz_tok * tcl + (long)h * P;    // V, Z
    const T* hsrc = reinterpret_cast<const T*>(a.hs) + ((long)bh * nc + c) * P * N;
    const T* gsrc = reinterpret_cast<const T*>(a.gs) + ((long)bh * nc + c) * N * P;
#pragma unroll
    for (int k = 0; k < HP; ++k) {
      const int i = min(tid + k * kBwdThreads, P * N / 8 - 1);
      hpc[k].load(hsrc + 8 * i);
      gpc[k].load(gsrc + 8 * i);
    }
#pragma unroll
    for (int hh = 0; hh < 2; ++hh) {
      const int g = min(hh * GH + wave, N / 8 - 1);
      qraw[hh].load(reinterpret_cast<const T*>(a.s.q) + qrow + 8 * g);
      kraw[hh].load(reinterpret_cast<const T*>(a.s.k) + qrow + 8 * g);
      rates[hh] = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
      if constexpr (R > 0) {
        const long arow = a.s.ang_shared ? (long)b * L + tcl : ((long)b * L + tcl) * H + h;
        rates[hh] = *reinterpret_cast<const float4*>(a.s.ang + arow * R + 4 * min(g, R / 4 - 1));
      }
    }
    dtraw = a.s.dt[(long)bh * L + tcl];
    const T* gv = reinterpret_cast<const T*>(a.s.v);
    const T* gz = a.s.z ? reinterpret_cast<const T*>(a.s.z) : gv;
#pragma unroll
    for (int k = 0; k < VGW; ++k) {
      const int g = min(wave + k * kBwdWaves, P / 8 - 1);
      vraw[k].load(gv + vzrow + 8 * g);
      dyraw[k].load(reinterpret_cast<const T*>(a.dout) + vrow + 8 * g);
      zraw[k].load(gz + vzrow + 8 * g);
    }
  }
};

// One workgroup per (chunk, b, h) item.
template <typename T, int CS, int N, int P, int R>
__global__ __launch_bounds__(kBwdThreads, 1)
void scan_bwd_chunk_kernel(BwdArgs a) {
  typedef MF16<T> W;
  typedef GradSmem<T, CS, N, P, R> S;
  typedef ItemLoads<T, CS, N, P, R> Loads;
  static_assert(sizeof(S) <= 160 * 1024, "LDS budget");
  __shared__ S sm;
  constexpr int PAD = S::PAD, KS = W::KSTEP, NH = S::NH;
  constexpr int TB = CS / 16;                          // 16-token blocks
  constexpr int GH = NH / 8, HP = Loads::HP, VGW = Loads::VGW;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  __builtin_assume(wave >= 0 && wave < kBwdWaves);
  const int L = a.s.L, H = a.s.H, HQ = a.s.Hqk, nc = a.nc;
  const bool qkw = wave < GH;
  const int c = blockIdx.x, bh = blockIdx.y, b = bh / H, h = bh % H;
  Loads cur;
  cur.issue(a, c, bh, tid, wave, lane);
  const int hq = h / (H / HQ);
  const int t0 = c * CS;
  const T* gz = reinterpret_cast<const T*>(a.s.z);
  const float Dh = a.s.D ? a.s.D[h] : 0.0f;
  const bool tok = lane < CS && t0 + lane < L;
  const long qrow = (((long)b * L + t0 + lane) * HQ + hq) * N;   // this lane's token (stores)
  const float dtl = tok ? cur.dtraw : 0.0f;

  // ---- token constants and the two saved states into LDS
  if (wave == 0) chunk_scalars<CS>(a, bh, t0, lane, sm.ac, sm.gam, sm.scl, sm.dtv, &sm.aend);
#pragma unroll
  for (int k = 0; k < HP; ++k) {
    const int i = tid + k * kBwdThreads;
    if (i < P * N / 8) {
      // the state piece holds two 4-element groups of the saved tile order
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        int p, n;
        saved_pos<N>(2 * i + j, p, n);
        if constexpr (std::is_same<T, bf16>::value) {
          const uint2 w = j ? make_uint2(cur.hpc[k].raw.z, cur.hpc[k].raw.w) : make_uint2(cur.hpc[k].raw.x, cur.hpc[k].raw.y);
          *reinterpret_cast<uint2*>(&sm.h[p][n]) = w;
        } else {
          *reinterpret_cast<float4*>(&sm.h[p][n]) = j ? cur.hpc[k].b : cur.hpc[k].a;
        }
      }
      *reinterpret_cast<Vec8<T>*>(&sm.gt[i / (P / 8)][8 * (i % (P / 8))]) = cur.gpc[k];
    }
  }

  // ---- this thread's two column groups, one per half of the state columns (waves
  // < GH): q^ = q + qb, k^ = k + kb and the rope cos/sin of their pairs stay in
  // registers for every phase below.  Padding tokens hold zeros.
  float qh[2][8], kh[2][8], cs[2][4], sn[2][4];
#pragma unroll
  for (int hh = 0; hh < 2; ++hh) {
    const int g = hh * GH + wave;
#pragma unroll
    for (int e = 0; e < 8; ++e) qh[hh][e] = kh[hh][e] = 0.0f;
#pragma unroll
    for (int j = 0; j < 4; ++j) cs[hh][j] = 1.0f, sn[hh][j] = 0.0f;
    if (qkw) {
      float th4[4];
      group_theta<CS, R>(a, bh, c, g, cur.rates[hh], dtl, th4);
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        cs[hh][j] = __builtin_amdgcn_cosf(th4[j]);
        sn[hh][j] = __builtin_amdgcn_sinf(th4[j]);
      }
      if (tok) {
        cur.qraw[hh].to_f(qh[hh]);
        cur.kraw[hh].to_f(kh[hh]);
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          qh[hh][e] += a.s.qbias[(long)h * N + 8 * g + e];
          kh[hh][e] += a.s.kbias[(long)h * N + 8 * g + e];
        }
      }
    }
  }
  __syncthreads();   // the token constants (key scale below) and the saved states


  // ---- preparation, lane = token: q~, k~, v, dy and the row dot products
  if (qkw) {
#pragma unroll
    for (int hh = 0; hh < 2; ++hh) {
      const int g = hh * GH + wave;
      float q[8], k[8], dot = 0.0f;
      const float sc = tok ? sm.scl[lane] : 0.0f;
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        q[e] = qh[hh][e];
        k[e] = kh[hh][e];
        dot += q[e] * k[e];
      }
      rot8<R>(q, cs[hh], sn[hh], g, 1.0f);
      rot8<R>(k, cs[hh], sn[hh], g, 1.0f);
#pragma unroll
      for (int e = 0; e < 8; ++e) k[e] *= sc;
      if (lane < CS) {
        store8(&sm.qt[lane][8 * g], q);
        store8(&sm.kt[lane][8 * g], k);
        sm.pq[g][lane] = dot;
      }
    }
  }
#pragma unroll
  for (int k = 0; k < VGW; ++k) {
    const int g = wave + k * kBwdWaves;
    if (g >= P / 8) continue;
    float v[8] = {0, 0, 0, 0, 0, 0, 0, 0}, dy[8] = {0, 0, 0, 0, 0, 0, 0, 0}, fz[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    float dot = 0.0f;
    if (tok) {
      cur.vraw[k].to_f(v);
      cur.dyraw[k].to_f(dy);
      if (gz) {
        float z[8];
        cur.zraw[k].to_f(z);
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const float sz = sigmoid_fast(z[e]);
          fz[e] = dy[e] * sz * (1.0f + z[e] * (1.0f - sz));
          dy[e] *= z[e] * sz;
        }
      }
#pragma unroll
      for (int e = 0; e < 8; ++e) dot += dy[e] * v[e];
    }
    if (lane < CS) {
      store8(&sm.v[lane][8 * g], v);
      store8(&sm.dy[lane][8 * g], dy);
      store8(&sm.fz[lane][8 * g], fz);
      sm.pv[g][lane] = dot;
    }
  }
  __syncthreads();
  if (wave == 0) {
    float qk = 0.0f, dqk = 0.0f;
    if (lane < CS) {
      for (int g = 0; g < N / 8; ++g) qk += sm.pq[g][lane];
      for (int g = 0; g < P / 8; ++g) dqk += sm.pv[g][lane];
      sm.qk[lane] = qk;
      sm.dqk[lane] = dqk;
    }
    const float tot = wave_sum(dqk);               // padding tokens hold dy = 0
    if (lane == 0 && a.pd) a.pd[(long)bh * nc + c] = tot;
  }

  // ---- S = q~ k~^T and dP = dy v^T, masked (s < t) and decayed e^{A_t - A_s}
  for (int i = wave; i < 2 * TB * TB; i += kBwdWaves) {
    const int which = i / (TB * TB), tt = (i % (TB * TB)) / TB, st = (i % (TB * TB)) % TB;
    f32x4 acc = {0.0f, 0.0f, 0.0f, 0.0f};
    if (st <= tt) {
      if (which == 0) {
        for (int k0 = 0; k0 < N; k0 += KS)
          acc = W::mma(W::ld(&sm.qt[0][0], N + PAD, 16 * tt, k0, lane), W::ld(&sm.kt[0][0], N + PAD, 16 * st, k0, lane),
                       acc);
      } else {
        for (int k0 = 0; k0 < P; k0 += KS)
          acc = W::mma(W::ld(&sm.dy[0][0], P + PAD, 16 * tt, k0, lane), W::ld(&sm.v[0][0], P + PAD, 16 * st, k0, lane),
                       acc);
      }
    }
    const int s = 16 * st + (lane & 15);
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int t = 16 * tt + 4 * (lane >> 4) + r;
      const float val = s < t ? acc[r] * exp2_fast((sm.ac[t] - sm.ac[s]) * kLog2e) : 0.0f;
      if (which == 0) sm.sm[t][s] = (T)val;
      else sm.dpm[t][s] = (T)val;
    }
  }
  __syncthreads();

  // ---- y (for dZ) and dV, per 16 x 16 tile of (token, value column)
  const float aend = sm.aend;
  for (int i = wave; i < 2 * TB * (P / 16); i += kBwdWaves) {
    const int which = i / (TB * (P / 16)), rt = (i % (TB * (P / 16))) / (P / 16), pt = i % (P / 16);
    f32x4 acc = {0.0f, 0.0f, 0.0f, 0.0f}, acc2 = {0.0f, 0.0f, 0.0f, 0.0f};
    if (which == 0) {
      if (!gz || !a.dz) continue;
      // y_t = sum_s Sm[t][s] v_s + e^{A_t} q~_t . h + (D + QK_t) v_t
      for (int k0 = 0; k0 < 16 * (rt + 1); k0 += KS)
        acc = W::mma(W::ld(&sm.sm[0][0], CS + PAD, 16 * rt, k0, lane), ld_tr(&sm.v[0][0], P + PAD, k0, 16 * pt, lane),
                     acc);
      for (int k0 = 0; k0 < N; k0 += KS)
        acc2 = W::mma(W::ld(&sm.qt[0][0], N + PAD, 16 * rt, k0, lane), W::ld(&sm.h[0][0], N + PAD, 16 * pt, k0, lane),
                      acc2);
      const int p = 16 * pt + (lane & 15);
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int t = 16 * rt + 4 * (lane >> 4) + r;
        if (t0 + t < L) {
          const long o = a.dvz_bat * b + a.dvz_tok * (t0 + t) + (long)h * P + p;
          const float y = acc[r] + exp2_fast(sm.ac[t] * kLog2e) * acc2[r] +
                          (Dh + sm.gam[t] * sm.qk[t]) * (float)sm.v[t][p];
          reinterpret_cast<T*>(a.dz)[o] = (T)(y * (float)sm.fz[t][p]);
        }
      }
    } else {
      // dv_s = sum_t Sm[t][s] dy_t + e^{A_end - A_s} G k~_s + (D + QK_s) dy_s
      for (int k0 = (16 * rt / KS) * KS; k0 < CS; k0 += KS)
        acc = W::mma(ld_tr(&sm.sm[0][0], CS + PAD, k0, 16 * rt, lane), ld_tr(&sm.dy[0][0], P + PAD, k0, 16 * pt, lane),
                     acc);
      for (int k0 = 0; k0 < N; k0 += KS)
        acc2 = W::mma(W::ld(&sm.kt[0][0], N + PAD, 16 * rt, k0, lane), ld_tr(&sm.gt[0][0], P + PAD, k0, 16 * pt, lane),
                      acc2);
      const int p = 16 * pt + (lane & 15);
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int s = 16 * rt + 4 * (lane >> 4) + r;
        if (t0 + s < L) {
          const float dv = acc[r] + exp2_fast((aend - sm.ac[s]) * kLog2e) * acc2[r] +
                           (Dh + sm.gam[s] * sm.qk[s]) * (float)sm.dy[s][p];
          reinterpret_cast<T*>(a.dv)[a.dvz_bat * b + a.dvz_tok * (t0 + s) + (long)h * P + p] = (T)dv;
        }
      }
    }
  }

  // ---- dq~ then dk~, half the columns at a time, each followed by its chain rule
  constexpr bool BF = std::is_same<T, bf16>::value;
  // unrolled: the register arrays above are indexed with compile-time halves only
#pragma unroll
  for (int pass = 0; pass < 4; ++pass) {
    const bool isq = pass < 2;
    const int n0 = (pass & 1) * NH;
    const int hh = pass & 1;
    // this thread's group of the half: raw values and rope by value selection
    float gq8[8], gk8[8], gcs[4], gsn[4];
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      gq8[e] = hh ? qh[1][e] : qh[0][e];
      gk8[e] = hh ? kh[1][e] : kh[0][e];
    }
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      gcs[j] = hh ? cs[1][j] : cs[0][j];
      gsn[j] = hh ? sn[1][j] : sn[0][j];
    }
    if constexpr (BF) {
      // rounding residual of the operand this pass multiplies: k~ (dq~) or q~ (dk~)
      if (qkw) {
        const int g = n0 / 8 + wave;
        float x[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) x[e] = isq ? gk8[e] : gq8[e];
        rot8<R>(x, gcs, gsn, g, 1.0f);
        const float sc = isq && tok ? sm.scl[lane] : 1.0f;
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          x[e] *= sc;
          x[e] -= (float)(bf16)x[e];
        }
        if (lane < CS) store8(&sm.lo[lane][8 * wave], x);
      }
      __syncthreads();
    }
    for (int i = wave; i < TB * (NH / 16); i += kBwdWaves) {
      const int rt = i / (NH / 16), nt = i % (NH / 16);
      f32x4 acc = {0.0f, 0.0f, 0.0f, 0.0f}, acc2 = {0.0f, 0.0f, 0.0f, 0.0f};
      if (isq) {
        // dq~_t = sum_s dPm[t][s] k~_s + e^{A_t} dy_t h
        for (int k0 = 0; k0 < 16 * (rt + 1); k0 += KS) {
          const typename W::frag fa = W::ld(&sm.dpm[0][0], CS + PAD, 16 * rt, k0, lane);
          acc = W::mma(fa, ld_tr(&sm.kt[0][0], N + PAD, k0, n0 + 16 * nt, lane), acc);
          if constexpr (BF) acc = W::mma(fa, ld_tr(&sm.lo[0][0], NH + PAD, k0, 16 * nt, lane), acc);
        }
        for (int k0 = 0; k0 < P; k0 += KS)
          acc2 = W::mma(W::ld(&sm.dy[0][0], P + PAD, 16 * rt, k0, lane),
                        ld_tr(&sm.h[0][0], N + PAD, k0, n0 + 16 * nt, lane), acc2);
      } else {
        // dk~_s = sum_t dPm[t][s] q~_t + e^{A_end - A_s} v_s G
        for (int k0 = (16 * rt / KS) * KS; k0 < CS; k0 += KS) {
          const typename W::frag fa = ld_tr(&sm.dpm[0][0], CS + PAD, k0, 16 * rt, lane);
          acc = W::mma(fa, ld_tr(&sm.qt[0][0], N + PAD, k0, n0 + 16 * nt, lane), acc);
          if constexpr (BF) acc = W::mma(fa, ld_tr(&sm.lo[0][0], NH + PAD, k0, 16 * nt, lane), acc);
        }
        for (int k0 = 0; k0 < P; k0 += KS)
          acc2 = W::mma(W::ld(&sm.v[0][0], P + PAD, 16 * rt, k0, lane),
                        W::ld(&sm.gt[0][0], P + PAD, n0 + 16 * nt, k0, lane), acc2);
      }
      const int nl = 16 * nt + (lane & 15);
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int t = 16 * rt + 4 * (lane >> 4) + r;
        const float w = exp2_fast((isq ? sm.ac[t] : aend - sm.ac[t]) * kLog2e);
        sm.res[t][nl] = acc[r] + w * acc2[r];
      }
    }
    __syncthreads();
    // chain rule, lane = token, one 8-column group per wave
    const int g = n0 / 8 + wave;
    if (qkw) {
      float dx[8] = {0, 0, 0, 0, 0, 0, 0, 0}, out[8] = {0, 0, 0, 0, 0, 0, 0, 0};
      float dot = 0.0f, dsc = 0.0f, dthf[4] = {0.0f, 0.0f, 0.0f, 0.0f};
      if (tok) {
#pragma unroll
        for (int e = 0; e < 8; ++e) dx[e] = sm.res[lane][8 * (g - n0 / 8) + e];
        const float sc = sm.scl[lane], gqk = sm.dqk[lane] * sm.gam[lane];
        float xr[8];                                      // q~ (pass Q) or rot(k^) (pass K)
#pragma unroll
        for (int e = 0; e < 8; ++e) xr[e] = isq ? gq8[e] : gk8[e];
        rot8<R>(xr, gcs, gsn, g, 1.0f);
        const float f = isq ? 1.0f : sc;                  // k~ = scale rot(k^)
        float dth[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          dot += f * xr[e] * dx[e];
          dsc += xr[e] * dx[e];
        }
#pragma unroll
        for (int j = 0; j < 4; ++j) dth[j] = f * (dx[2 * j + 1] * xr[2 * j] - dx[2 * j] * xr[2 * j + 1]);
        // d(q^) = rot^T dq~ + dQK gamma k^;  d(k^) = scale rot^T dk~ + dQK gamma q^
#pragma unroll
        for (int e = 0; e < 8; ++e) out[e] = f * dx[e];
        rot8<R>(out, gcs, gsn, g, -1.0f);
#pragma unroll
        for (int e = 0; e < 8; ++e) out[e] += gqk * (isq ? gk8[e] : gq8[e]);
        // angle gradient of the pairs of this group (finished by the finish kernel)
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const int r = 4 * g + j;
          if (r < R) {
            float* dst = a.dang + (((long)b * L + t0 + lane) * H + h) * R + r;
            dthf[j] = isq ? dth[j] : *dst + dth[j];
            *dst = dthf[j];
          }
        }
        // dQ / dK rows
        if (a.dqh) {
          T* dst = reinterpret_cast<T*>(isq ? a.dqh : a.dkh) + (((long)b * L + t0 + lane) * H + h) * N + 8 * g;
          store8(dst, out);
        } else {
          T* dst = reinterpret_cast<T*>(isq ? a.dq : a.dk) + qrow + 8 * g;
          store8(dst, out);
        }
      }
      if (lane < CS) {
        if (isq) sm.pq[g][lane] = dot;   // the same thread subtracts k~.dk~ in pass K
        else {
          sm.pq[g][lane] -= dot;
          sm.ps[g][lane] = dsc;
        }
      }
      // chunk sums of the finished angle gradient, for the reverse cumsum over chunks
      if (!isq) {
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          if (4 * g + j < R) {
            const float s = wave_sum(dthf[j]);
            if (lane == 0) a.ctot[((long)bh * nc + c) * (R + 1) + 1 + 4 * g + j] = s;
          }
        }
      }
      // bias gradient partials: column sums over the chunk's tokens
      float* pb = (isq ? a.pqb : a.pkb) + ((long)bh * nc + c) * N + 8 * g;
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const float s = wave_sum(out[e]);
        if (lane == 0) pb[e] = s;
      }
    }
    __syncthreads();
  }

  // ---- per token: dA and d(gamma) into the dADT and dDT outputs, d(scale) into the
  // workspace, and the chunk sum of dA
  if (wave == 0) {
    float da = 0.0f, ds = 0.0f;
    if (tok) {
      for (int g = 0; g < N / 8; ++g) {
        da += sm.pq[g][lane];
        ds += sm.ps[g][lane];
      }
      const long o = (long)bh * L + t0 + lane;
      a.dadt[o] = da;
      a.dsc[o] = ds;
      a.ddt[o] = sm.dqk[lane] * sm.qk[lane] + ds;
    }
    const float tot = wave_sum(da);
    if (lane == 0) a.ctot[((long)bh * nc + c) * (a.s.R + 1)] = tot;
  }
}

// ------------------------------------------------ reverse walk (adjoint fused in)
// One workgroup per (b, h) walks the chunks from the last to the first.  The adjoint
// state G (N x P, float32) stays in MFMA accumulators for the whole walk, as the
// forward keeps the state: each chunk writes G_c, the adjoint state after it, to LDS
// for its dV and dk~ products, then advances G <- e^{A_end} G + sum_t e^{A_cum,t}
// dy_t (x) q~_t with its own q~ and dy.  Against the chunk-parallel route this removes
// the adjoint pass (a second read of Q, dOut, Z and the rates) and the round trip of
// every G_c through the workspace.  The bias and D gradients are summed over the walk,
// and the reverse cumsums of dA and d(theta) over the sequence are carried from chunk
// to chunk: the walk writes the suffix sums themselves (and their totals), which
// scan_bwd_walk_finish_kernel turns into dADT, dAngles, dDT and dTrap.
//
// Memory access.  Every compute unit runs a walk at the same pace, so the chip's HBM
// traffic comes in per-chunk bursts; what limits a burst is the number of cache lines
// each load or store instruction touches.  Q, K, V, dOut and Z are therefore read as
// whole rows (consecutive lanes on consecutive 16-byte pieces of a row): V, dOut and
// Z are prepared in that layout directly, and Q and K pass through an LDS staging tile
// (XOR-swizzled 16-byte slots) to the token-per-lane layout of the rope.  dZ, dV, dQ,
// dK and dAngles are staged in LDS and written as whole rows.  The next chunk's loads
// are requested in four parts spread over the current chunk, behind whose work their
// latency hides.
// YV: also the saved output before the gate (the walk's training-pair variant)
template <typename T, int CS, int N, int P, int R, bool YV>
struct WalkLoads {
  static constexpr int GH = N / 16;                                       // column groups per half
  static constexpr int HP = (P * N / 8 + kBwdThreads - 1) / kBwdThreads;  // 8-element state pieces per thread
  static constexpr int QPT = (CS * N / 8 + kBwdThreads - 1) / kBwdThreads; // Q (K) row pieces per thread
  static constexpr int VPT = (CS * P / 8 + kBwdThreads - 1) / kBwdThreads; // V (dOut, Z) row pieces per thread
  static constexpr int HK = 8 * (int)sizeof(T) / 16;                     // 16-byte words per state piece
  typedef unsigned u32x4 __attribute__((ext_vector_type(4)));             // (a plain vector: kept in registers)
  u32x4 hpc[HP][HK];
  Vec8<T> qpc[QPT], kpc[QPT], vpc[VPT], dypc[VPT], zpc[VPT], ypc[VPT];
  float4 rates[2], th0[2];
  float adt, dt, trap, dtn, trapn;
  // Every load is unconditional, from a clamped valid address where a lane has nothing
  // to load (rows past the sequence end read the last token's row); those values are
  // ignored or zeroed at their use.
  template <int PART>
  __device__ __forceinline__ void issue(const BwdArgs& a, int c, int bh, int tid, int wave, int lane) {
    const int b = bh / a.s.H, h = bh % a.s.H, hq = h / (a.s.H / a.s.Hqk);
    const int L = a.s.L, H = a.s.H, HQ = a.s.Hqk, nc = a.nc, t0 = c * CS;
    if constexpr (PART == 0) {
      const T* hsrc = reinterpret_cast<const T*>(a.hs) + ((long)bh * nc + c) * P * N;
#pragma unroll
      for (int k = 0; k < HP; ++k) {
        const u32x4* src = reinterpret_cast<const u32x4*>(hsrc + 8 * min(tid + k * kBwdThreads, P * N / 8 - 1));
#pragma unroll
        for (int j = 0; j < HK; ++j) hpc[k][j] = src[j];
      }
      const long srow = (long)bh * L;
      // lane & (CS - 1): the token of a lane (two lanes per token at 32-token chunks)
      const int tcl = min(t0 + (lane & (CS - 1)), L - 1), tn = min(t0 + CS, L - 1);
      adt = a.s.adt[srow + tcl];
      dt = a.s.dt[srow + tcl];
      trap = a.s.trap[srow + tcl];
      dtn = a.s.dt[srow + tn];
      trapn = a.s.trap[srow + tn];
    } else if constexpr (PART == 1) {
#pragma unroll
      for (int k = 0; k < QPT; ++k) {
        const int p = min(tid + k * kBwdThreads, CS * N / 8 - 1);
        const long row = (((long)b * L + min(t0 + p / (N / 8), L - 1)) * HQ + hq) * N + 8 * (p % (N / 8));
        qpc[k].load(reinterpret_cast<const T*>(a.s.q) + row);
        kpc[k].load(reinterpret_cast<const T*>(a.s.k) + row);
      }
    } else if constexpr (PART == 2) {
      const T* gv = reinterpret_cast<const T*>(a.s.v) + a.s.vz_bat * b + (long)h * P;
      const T* gz = a.s.z ? reinterpret_cast<const T*>(a.s.z) + a.s.vz_bat * b + (long)h * P : gv;
#pragma unroll
      for (int k = 0; k < VPT; ++k) {
        const int p = min(tid + k * kBwdThreads, CS * P / 8 - 1);
        const long tk = min(t0 + p / (P / 8), L - 1);
        const int col = 8 * (p % (P / 8));
        const long row = (((long)b * L + tk) * H + h) * P + col;          // dOut, y_v
        const long vzr = a.s.vz_tok * tk + col;                           // V, Z
        vpc[k].load(gv + vzr);
        dypc[k].load(reinterpret_cast<const T*>(a.dout) + row);
        zpc[k].load(gz + vzr);
        if constexpr (YV) ypc[k].load(reinterpret_cast<const T*>(a.yv) + row);
      }
    } else {
      const int tcl = min(t0 + (lane & (CS - 1)), L - 1);
#pragma unroll
      for (int hh = 0; hh < 2; ++hh) {
        rates[hh] = th0[hh] = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
        if constexpr (R > 0) {
          const int gr = min(min(hh * GH + wave, N / 8 - 1), R / 4 - 1);
          const long arow = a.s.ang_shared ? (long)b * L + tcl : ((long)b * L + tcl) * H + h;
          rates[hh] = *reinterpret_cast<const float4*>(a.s.ang + arow * R + 4 * gr);
          th0[hh] = *reinterpret_cast<const float4*>(a.th0 + ((long)bh * nc + c) * R + 4 * gr);
        }
      }
    }
  }
  __device__ __forceinline__ void issue_all(const BwdArgs& a, int c, int bh, int tid, int wave, int lane) {
    issue<0>(a, c, bh, tid, wave, lane);
    issue<1>(a, c, bh, tid, wave, lane);
    issue<2>(a, c, bh, tid, wave, lane);
    issue<3>(a, c, bh, tid, wave, lane);
  }
};

// LDS of the walk.  The arrays live for the whole chunk except those in `u`, whose
// members are used in three windows separated by barriers: (A) the Q/K staging tiles
// (written at the top of the chunk, read in its preparation), (B) the masked S and the
// dZ/dV output tiles (S/dP to the dZ/dV stores), (C) the tiles of the dq~/dk~ passes:
// bf16 at d_state 128 two residual and two product tiles of the pipelined quarters
// (the residual tiles outside the output tiles, so that the first two are written
// while the dZ/dV rows are still being stored); other bf16 shapes the residual, the
// dq~ / dk~ results and the d(theta) output tile, apart in the same way; float the
// second product tile of its pipelined passes.  float keeps the LDS of d_state 128
// under the 160 KB limit with two more reuses: Q and K rows are staged in qt / kt
// themselves (the preparation reads each thread's own 8 raw elements and writes its
// q~ / k~ back to the same place), and its first product tile lives in fz's storage,
// dead after the y/dV phase.
template <typename T, int CS, int N, int P, int R>
struct WalkSmem {
  static constexpr bool BF = std::is_same<T, bf16>::value;
  static constexpr int PAD = BF ? 8 : 4;
  // Rows of 256 bytes (bf16, d_state 128) get 48 bytes of padding: a stride of 304 bytes
  // (48 mod 256) keeps both the 16-row MFMA operand reads and the transposed 4-row reads
  // of these tiles free of bank conflicts (272 bytes overlaps the transposed reads).
  static constexpr int PADN = BF && N == 128 ? 24 : PAD;
  static constexpr int NH = N / 2;
  static constexpr int SQ = N * (int)sizeof(T) / 16;        // 16-byte slots per Q/K row
  static constexpr int RH = NH / 2 + 4;                     // row of the dAngles tile (a half's pairs)
  static constexpr size_t SZ_Q = (size_t)CS * N * sizeof(T);
  static constexpr size_t SZ_SM = (size_t)CS * (CS + PAD) * sizeof(T);
  static constexpr size_t SZ_OUT = (size_t)2 * CS * (P + PAD) * sizeof(T);
  static constexpr size_t SZ_LO = BF ? (size_t)CS * (NH + PAD) * sizeof(T) : 0;
  static constexpr size_t SZ_RES = (size_t)CS * (NH + 4) * 4;
  static constexpr size_t SZ_DTH = (size_t)CS * RH * 4;
  static constexpr size_t OFF_K = SZ_Q, OFF_OUT = SZ_SM;
  // bf16: res may overlap the output tiles (it is first written after the residual
  // barrier)
  static constexpr size_t OFF_RES = SZ_LO;
  static constexpr size_t OFF_DTH = OFF_RES + SZ_RES;
  // bf16 at d_state 128: the dq~/dk~ passes run in quarters of 32 columns,
  // software-pipelined over two residual tiles (lo) and two product tiles, at u + 0,
  // u + 3 SZ_QT (residuals) and u + SZ_QT, u + 2 SZ_QT (products): the residuals of the
  // first two quarters are written while the dZ/dV rows are stored from the output
  // tiles, which lie in [SZ_SM, SZ_SM + SZ_OUT) = [SZ_QT, 3 SZ_QT).
  static constexpr bool QP = BF && N == 128;
  static constexpr int NQ = 32;                             // columns of a quarter
  static constexpr size_t SZ_QT = (size_t)CS * (NQ + 4) * 4;
  static_assert(!QP || (SZ_QT == (size_t)CS * (NH + PAD) * sizeof(T) && SZ_SM == SZ_QT &&
                        SZ_OUT == 2 * SZ_QT), "quarter tiles: a residual tile [CS][NH + PAD] bf16 per slot");
  static constexpr size_t U1 = BF ? 2 * SZ_Q : 0, U2 = SZ_SM + SZ_OUT,
                          U3 = QP ? 4 * SZ_QT : (BF ? OFF_DTH + SZ_DTH : 0);
  static_assert(BF || (SZ_RES <= (size_t)CS * (P + PAD) * sizeof(T) && SZ_DTH <= SZ_SM),
                "float: res fits fz's storage, the d(theta) tile the masked S's");
  static constexpr size_t U = U1 > U2 ? (U1 > U3 ? U1 : U3) : (U2 > U3 ? U2 : U3);
  alignas(16) T qt[CS][N + PADN];       // q~
  alignas(16) T kt[CS][N + PADN];       // k~
  alignas(16) T v[CS][P + PAD];
  alignas(16) T dy[CS][P + PAD];
  alignas(16) T fz[CS][P + PAD];       // dOut sigmoid(z) (1 + z (1 - sigmoid(z))): dZ = y fz
  alignas(16) T h[P][N + PADN];         // state entering the chunk
  alignas(16) T gt[N][P + PAD];        // adjoint state after the chunk, [n][p]
  alignas(16) T dpm[CS][CS + PAD];     // dP masked and decayed
  alignas(16) char u[U];
  alignas(16) float ac[CS];
  // e^{A_cum,t} and e^{A_end - A_cum,t}, formed once per chunk: the row factors of
  // Y_off (y), of dv's and dk~'s G terms, of dq~'s h term and of the adjoint update
  alignas(16) float ea[CS], eb[CS];
  float gam[CS], scl[CS], dtv[CS], qk[CS], dqk[CS];
  // per token, one row per column-group wave (its two groups): q^.k^, then
  // q~.dq~ - k~.dk~; dk~ . rot(k^)
  float pq[N / 16][CS];
  float ps[N / 16][CS];
  float qb[N], kb[N];                  // the head's biases
  float aend;
  __device__ __forceinline__ uint4* qstage() { return reinterpret_cast<uint4*>(u); }
  __device__ __forceinline__ uint4* kstage() { return reinterpret_cast<uint4*>(u + OFF_K); }
  __device__ __forceinline__ T* smk() { return reinterpret_cast<T*>(u); }                  // [CS][CS + PAD]
  __device__ __forceinline__ T* outs(int w) { return reinterpret_cast<T*>(u + OFF_OUT) + (size_t)w * CS * (P + PAD); }
  __device__ __forceinline__ T* lo() { return reinterpret_cast<T*>(u); }                   // [CS][NH + PAD]
  __device__ __forceinline__ float* res() {                                                  // [CS][NH + 4]
    if constexpr (BF) return reinterpret_cast<float*>(u + OFF_RES);
    else return reinterpret_cast<float*>(&fz[0][0]);
  }
  // quarter passes: residual tile i ([CS][NH + PAD] bf16, NQ columns used) and product
  // tile i ([CS][NQ + 4] float)
  __device__ __forceinline__ T* loq(int i) { return reinterpret_cast<T*>(u + (i ? 3 * SZ_QT : 0)); }
  __device__ __forceinline__ float* rq(int i) { return reinterpret_cast<float*>(u + (i ? 2 * SZ_QT : SZ_QT)); }
  // float: the second product tile of the pipelined passes (the staging and output
  // tiles are done by then)
  __device__ __forceinline__ float* res2() { return reinterpret_cast<float*>(u); }
  static_assert(BF || SZ_RES <= U, "float: the second product tile fits u");
  __device__ __forceinline__ float* dth() {                                                  // [CS][RH]
    if constexpr (BF) return reinterpret_cast<float*>(u + OFF_DTH);
    else return reinterpret_cast<float*>(u);
  }
};

__device__ __forceinline__ float lane63(float v) {
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 63));
}

// MFMA operand access of the walk.  bf16: MF16<bf16>, with transposed reads by ld_tr.
// float: each fragment holds four k-steps of v_mfma_f32_16x16x4_f32.  In step s of a
// 16-wide k block, the instruction's k slot i / 16 of lane i stands for k = k0 +
// 4 (i / 16) + s, in both operands of a product (the sum over k is the same in any
// order of its terms), so an operand stored with k contiguous is one 16-byte LDS read
// per four MFMAs, and a transposed operand is four reads from rows 4 apart, whose
// 4-row strides (528, 272 and 144 bytes, all 64 mod 256) put the 64 lanes on 64
// different banks.
template <typename T> struct WalkMma;
template <> struct WalkMma<bf16> : MF16<bf16> {
  __device__ __forceinline__ static frag ldt(const bf16* buf, int ld, int k0, int c0, int lane) {
    return ld_tr(buf, ld, k0, c0, lane);
  }
};
template <> struct WalkMma<float> {
  static constexpr int KSTEP = 16;
  typedef float4 frag;
  __device__ __forceinline__ static f32x4 mma(frag a, frag b, f32x4 c) {
    c = __builtin_amdgcn_mfma_f32_16x16x4f32(a.x, b.x, c, 0, 0, 0);
    c = __builtin_amdgcn_mfma_f32_16x16x4f32(a.y, b.y, c, 0, 0, 0);
    c = __builtin_amdgcn_mfma_f32_16x16x4f32(a.z, b.z, c, 0, 0, 0);
    return __builtin_amdgcn_mfma_f32_16x16x4f32(a.w, b.w, c, 0, 0, 0);
  }
  // rows row0 + lane%16 of a [row][k] tile, k = k0 + 4 (lane/16) + 0..3
  __device__ __forceinline__ static frag ld(const float* buf, int ldm, int row0, int k0, int lane) {
    return *reinterpret_cast<const float4*>(buf + (row0 + (lane & 15)) * ldm + k0 + 4 * (lane >> 4));
  }
  // column c0 + lane%16 of a [k][col] tile, the same k
  __device__ __forceinline__ static frag ldt(const float* buf, int ld, int k0, int c0, int lane) {
    const float* p = buf + (k0 + 4 * (lane >> 4)) * ld + c0 + (lane & 15);
    return make_float4(p[0], p[ld], p[2 * ld], p[3 * ld]);
  }
  static constexpr int WN = 4;
  __device__ __forceinline__ static int ktok(int k0, int lane) { return k0 + 4 * (lane >> 4); }
  __device__ __forceinline__ static frag scale(frag v, const float w[WN]) {
    return make_float4(v.x * w[0], v.y * w[1], v.z * w[2], v.w * w[3]);
  }
};

// YV: the training pair's variant that reads the saved output before the gate (a.yv)
// and forms dZ from it in the preparation instead of recomputing y.  SEGW: the walk
// split into segments (grid (B*H, nseg), each block one segment from its entering
// adjoint); without it the walk covers the whole sequence, compiled without the
// segment bounds.
// GQA: Q/K heads shared by several value heads (a.dqh set): the per-head dQ/dK go to
// the partials that scan_bwd_gqa_kernel sums; without it they go straight to dQ/dK.
template <typename T, int CS, int N, int P, int R, bool YV, bool SEGW, bool GQA>
__global__ __launch_bounds__(kBwdThreads, 1)
void scan_bwd_walk_kernel(BwdArgs a) {
  typedef WalkMma<T> W;
  typedef WalkSmem<T, CS, N, P, R> S;
  typedef WalkLoads<T, CS, N, P, R, YV> Loads;
  static_assert(sizeof(S) <= 160 * 1024, "LDS budget");
  __shared__ S sm;
  constexpr int PAD = S::PAD, PADN = S::PADN, KS = W::KSTEP, NH = S::NH, SQ = S::SQ, RH = S::RH;
  constexpr int TB = CS / 16;                          // 16-token blocks
  constexpr int GH = NH / 8, QPT = Loads::QPT, VPT = Loads::VPT;
  constexpr int NT = N / 16, NTILE = (P / 16) * NT, TPW = (NTILE + kBwdWaves - 1) / kBwdWaves;
  static_assert(kBwdWaves % NT == 0, "the adjoint tiles of a wave share one column tile");
  constexpr bool BF = S::BF;
  constexpr int HP = Loads::HP;
  // lanes per token (two at 32-token chunks: lanes l and l + 32), and per lane the
  // columns of an 8-column group and its rope pairs
  constexpr int TPL = 64 / CS, EL = 8 / TPL, PRS = 4 / TPL;
  static_assert(CS * TPL == 64, "64- or 32-token chunks");
  // float: the dq~/dk~ passes are software-pipelined and their chain rule stores its
  // rows itself; bf16 at d_state 128 the same in quarters of the columns (kQP); other
  // bf16 shapes keep the row stores from LDS after each pass
  constexpr bool kQP = S::QP;
  constexpr bool kDirect = !BF || kQP;
  // The per-token decay factors e^{A_t} and e^{A_end - A_t} are read from LDS (formed
  // once per chunk) and a wave's S and dP tiles of a block share theirs, except with
  // rope on every pair (R = N/2), whose instantiations are the tightest in registers:
  // there the loads kept live cost more in spills than the exponentials they replace.
  constexpr bool kHoist = 2 * R < N;
  auto exp_a = [&](int t) -> float {
    if constexpr (kHoist) return sm.ea[t];
    else return exp2_fast(sm.ac[t] * kLog2e);
  };
  auto exp_b = [&](int t, float ae) -> float {
    if constexpr (kHoist) return sm.eb[t];
    else return exp2_fast((ae - sm.ac[t]) * kLog2e);
  };
  const int wave = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
  __builtin_assume(wave >= 0 && wave < kBwdWaves);
  const int L = a.s.L, H = a.s.H, HQ = a.s.Hqk, nc = a.nc;
  const bool qkw = wave < GH;
  const int bh = blockIdx.x, b = bh / H, h = bh % H, hq = h / (H / HQ);
  // the chunks of this block's segment (the whole sequence without the split) and the
  // slot of its partial sums
  const int seg = SEGW ? (int)blockIdx.y : 0;
  const int c_lo = SEGW ? seg * a.seg_nc : 0, c_hi = SEGW ? min(nc, c_lo + a.seg_nc) : nc;
  const long ps = SEGW ? (long)bh * a.nseg + seg : bh;
  const T* gz = reinterpret_cast<const T*>(a.s.z);
  const float Dh = a.s.D ? a.s.D[h] : 0.0f;
  T* const smk = sm.smk();
  T* const lo = sm.lo();
  float* const res = sm.res();
  float* const dth = sm.dth();

  f32x4 G[TPW];                                        // adjoint state tiles [p][n]
#pragma unroll
  for (int i = 0; i < TPW; ++i) G[i] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
  if (SEGW && seg + 1 < a.nseg) {
    // the adjoint state after this segment, which the later segments leave
    const int lane = threadIdx.x & 63;
#pragma unroll
    for (int i = 0; i < TPW; ++i) {
      const int tile = wave + kBwdWaves * i;
      if (tile < NTILE) {
        const int n = 16 * (tile % NT) + (lane & 15), p = 16 * (tile / NT) + 4 * (lane >> 4);
#pragma unroll
        for (int r = 0; r < 4; ++r) G[i][r] = a.gin[(ps * P + p + r) * N + n];
      }
    }
  }
  // Bias gradients: per pass (q~ half 0, half 1, k~ half 0, half 1), thread (n, tg) sums
  // column n of the half over the tokens of its token group tg, over the whole walk.
  constexpr int TPG = CS * NH / kBwdThreads;           // tokens per group
  static_assert(TPG >= 1 && CS * NH % kBwdThreads == 0, "bias column sums: whole token groups");
  float bacc[4] = {0.0f, 0.0f, 0.0f, 0.0f};
  // (float) per pass, this lane's EL columns of the bias sums over its tokens
  float bq[4][EL];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int e = 0; e < EL; ++e) bq[i][e] = 0.0f;
  float cth[2][PRS];                                   // d(theta) over the later chunks, per pair
#pragma unroll
  for (int hh = 0; hh < 2; ++hh)
#pragma unroll
    for (int j = 0; j < PRS; ++j) cth[hh][j] = 0.0f;
  // The per-token dA of a chunk (sums over the column groups, reverse cumsum).  float:
  // on the last wave, beside wave 0's token constants at the top of the next chunk;
  // bf16 outside the quarter passes (a barrier follows it): wave 0, measured 1%
  // faster there.
  constexpr int kDaWave = BF && !S::QP ? 0 : kBwdWaves - 1;
  // the per-token d(scale) and dDT sums and stores, beside the dA's scan on another wave
  constexpr int kDsWave = BF && !S::QP ? 0 : kBwdWaves - 2;
  // the per-token q^.k^ sums and the D gradient, in the S/dP phase: float on a wave of
  // the dP tiles (which have half the S tiles' MFMAs at 32-token chunks)
  constexpr int kQkWave = BF ? 0 : kBwdWaves - 3;
  float cda = 0.0f, dsum = 0.0f;                       // wave kDaWave: dA over the later chunks; kQkWave: dD

  // One register set of loads: chunk c's inputs are consumed by the end of its
  // preparation, and chunk c - 1's are requested in parts during the rest of chunk c.
  Loads cur;
  {
    const int tid = threadIdx.x;
    cur.issue_all(a, c_hi - 1, bh, tid, wave, tid & 63);
    // the head's biases into LDS (read by every chunk's preparation)
    if (tid < N) {
      sm.qb[tid] = a.s.qbias[(long)h * N + tid];
      sm.kb[tid] = a.s.kbias[(long)h * N + tid];
    }
  }
  for (int c = c_hi - 1; c >= c_lo; --c) {
    // lane and thread indices made opaque per chunk, so that the compiler forms the
    // lane-dependent LDS and global addresses inside the chunk instead of hoisting them
    // all out of the walk and keeping each live in a register for the whole loop
    int tid = threadIdx.x;
    asm volatile("" : "+v"(tid));
    const int lane = tid & 63;
    const int tkn = lane & (CS - 1), hf = lane / CS;  // token of the lane and its half (two lanes per token)
    const int t0 = c * CS;
    const int nt = min(CS, L - t0);                   // tokens of this chunk
    const bool tok = tkn < nt;
    const float dtl = tok ? cur.dt : 0.0f;

    // ---- top: Q/K row pieces into the staging tiles, G_c and the saved state h_c
    // into LDS, the token constants
#pragma unroll
    for (int k = 0; k < QPT; ++k) {
      const int p = tid + k * kBwdThreads;
      if (p < CS * N / 8) {
        const int row = p / (N / 8), pc = p % (N / 8);
        if constexpr (BF) {
          // bf16: one 16-byte slot per piece, XOR-swizzled by row
          sm.qstage()[row * SQ + (pc ^ (row & (SQ - 1)))] = cur.qpc[k].raw;
          sm.kstage()[row * SQ + (pc ^ (row & (SQ - 1)))] = cur.kpc[k].raw;
        } else {
          // float: in place, in the row's own slots of q~ / k~ (member by member: a
          // copy of the whole struct goes through scratch memory)
          float4* dq = reinterpret_cast<float4*>(&sm.qt[row][8 * pc]);
          float4* dk = reinterpret_cast<float4*>(&sm.kt[row][8 * pc]);
          dq[0] = cur.qpc[k].a;
          dq[1] = cur.qpc[k].b;
          dk[0] = cur.kpc[k].a;
          dk[1] = cur.kpc[k].b;
        }
      }
    }
#pragma unroll
    for (int i = 0; i < TPW; ++i) {
      const int tile = wave + kBwdWaves * i;
      if (tile < NTILE) {
        const float gv[4] = {G[i][0], G[i][1], G[i][2], G[i][3]};
        store4(&sm.gt[16 * (tile % NT) + (lane & 15)][16 * (tile / NT) + 4 * (lane >> 4)], gv);
      }
    }
#pragma unroll
    for (int k = 0; k < HP; ++k) {
      const int i = tid + k * kBwdThreads;
      if (i < P * N / 8) {
        // the state piece holds two 4-element groups of the saved tile order
#pragma unroll
        for (int j = 0; j < 2; ++j) {
          int p, n;
          saved_pos<N>(2 * i + j, p, n);
          if constexpr (Loads::HK == 1) {
            typedef unsigned u32x2 __attribute__((ext_vector_type(2)));
            const typename Loads::u32x4 w = cur.hpc[k][0];
            *reinterpret_cast<u32x2*>(&sm.h[p][n]) = j ? u32x2{w[2], w[3]} : u32x2{w[0], w[1]};
          } else {
            *reinterpret_cast<typename Loads::u32x4*>(&sm.h[p][n]) = cur.hpc[k][j];
          }
        }
      }
    }
    if (wave == 0) {
      const float adt = tok ? cur.adt : 0.0f, tr = tok ? cur.trap : 0.0f;
      const float sg = 1.0f / (1.0f + expf(-tr));
      const float gm = dtl * sg;
      float un = __shfl_down(dtl * (1.0f - sg), 1, 64);             // next token's dt (1 - sigmoid)
      if (lane == CS - 1) {
        const bool nx = t0 + CS < L;
        const float dtn = nx ? cur.dtn : 0.0f, trn = nx ? cur.trapn : 0.0f;
        un = dtn * (1.0f - 1.0f / (1.0f + expf(-trn)));
      }
      const float acum = wave_incl_scan(lane < CS ? adt : 0.0f);
      const float ae = __shfl(acum, CS - 1, 64);
      if (lane < CS) {
        sm.ac[lane] = acum;
        sm.ea[lane] = exp2_fast(acum * kLog2e);
        sm.eb[lane] = exp2_fast((ae - acum) * kLog2e);
        sm.gam[lane] = gm;
        sm.scl[lane] = tok ? gm + un : 0.0f;
        sm.dtv[lane] = dtl;
      }
      if (lane == 0) sm.aend = ae;
    }
    __syncthreads();   // staging, token constants, G_c, h_c

    // ---- preparation.  Q/K, lane = token (two lanes per token at 32-token chunks,
    // each with EL of the group's 8 columns): this thread's two column groups (one per
    // half of the state columns): q^ = q + qb, k^ = k + kb and the rope cos/sin of
    // their pairs stay in registers for every phase below; q~ and k~ go to LDS.
    float qh[2][EL], kh[2][EL], cs[2][PRS], sn[2][PRS];
    float pqw = 0.0f;                                 // q^.k^ over the wave's two groups
#pragma unroll
    for (int hh = 0; hh < 2; ++hh) {
      const int g = hh * GH + wave;
      const int col = 8 * g + EL * hf;          // this lane's first column of the group
#pragma unroll
      for (int e = 0; e < EL; ++e) qh[hh][e] = kh[hh][e] = 0.0f;
#pragma unroll
      for (int j = 0; j < PRS; ++j) cs[hh][j] = 1.0f, sn[hh][j] = 0.0f;
      if (qkw) {
        float thp[PRS];
#pragma unroll
        for (int j = 0; j < PRS; ++j) thp[j] = 0.0f;
        if constexpr (R > 0) {
          if (4 * g < R) {
            // the rates and entering angles of this lane's pairs (a select per component:
            // an index by hf would put the arrays in scratch memory)
            const float4 rq = cur.rates[hh], tq = cur.th0[hh];
            float rv[PRS], tv[PRS];
            if constexpr (PRS == 4) {
              rv[0] = rq.x; rv[1] = rq.y; rv[2] = rq.z; rv[3] = rq.w;
              tv[0] = tq.x; tv[1] = tq.y; tv[2] = tq.z; tv[3] = tq.w;
            } else {
              rv[0] = hf ? rq.z : rq.x; rv[1] = hf ? rq.w : rq.y;
              tv[0] = hf ? tq.z : tq.x; tv[1] = hf ? tq.w : tq.y;
            }
#pragma unroll
            for (int j = 0; j < PRS; ++j) thp[j] = angle_step(rv[j], dtl);
            token_scan<PRS>(thp);
#pragma unroll
            for (int j = 0; j < PRS; ++j) thp[j] = __builtin_amdgcn_fractf(tv[j] + thp[j]);
          }
        }
#pragma unroll
        for (int j = 0; j < PRS; ++j) {
          cs[hh][j] = __builtin_amdgcn_cosf(thp[j]);
          sn[hh][j] = __builtin_amdgcn_sinf(thp[j]);
        }
        if (tok) {
          if constexpr (BF) {
            Vec8<T> qv, kv;
            qv.raw = staged<SQ>(sm.qstage(), lane, g);
            kv.raw = staged<SQ>(sm.kstage(), lane, g);
            qv.to_f(qh[hh]);
            kv.to_f(kh[hh]);
          } else {
            // the raw rows staged in place: this thread alone reads and then rewrites them
            load4(&sm.qt[tkn][col], qh[hh]);
            load4(&sm.kt[tkn][col], kh[hh]);
          }
#pragma unroll
          for (int e = 0; e < EL; ++e) {
            qh[hh][e] += sm.qb[col + e];
            kh[hh][e] += sm.kb[col + e];
          }
        }
        float q[EL], k[EL], dot = 0.0f;
        const float sc = tok ? sm.scl[tkn] : 0.0f;
#pragma unroll
        for (int e = 0; e < EL; ++e) {
          q[e] = qh[hh][e];
          k[e] = kh[hh][e];
          dot += q[e] * k[e];
        }
        rotp<PRS>(q, cs[hh], sn[hh], 4 * g < R, 1.0f);
        rotp<PRS>(k, cs[hh], sn[hh], 4 * g < R, 1.0f);
#pragma unroll
        for (int e = 0; e < EL; ++e) k[e] *= sc;
        dot = token_pair_sum<TPL>(dot);
        if constexpr (BF) {
          store8(&sm.qt[tkn][col], q);
          store8(&sm.kt[tkn][col], k);
        } else {
          store4(&sm.qt[tkn][col], q);
          store4(&sm.kt[tkn][col], k);
        }
        pqw += dot;
      }
    }
    // per-token partial sums: one row of pq per column-group wave
    if (qkw && hf == 0) sm.pq[wave][tkn] = pqw;
    // V, dOut, Z in row layout: dy = dOut silu(z), the dZ factor, and dy . v per token
#pragma unroll
    for (int k = 0; k < VPT; ++k) {
      const int p = tid + k * kBwdThreads;
      if (p < CS * P / 8) {                           // wave-uniform
        const int row = p / (P / 8), pc = p % (P / 8);
        float v[8] = {0, 0, 0, 0, 0, 0, 0, 0}, dy[8] = {0, 0, 0, 0, 0, 0, 0, 0}, fz[8] = {0, 0, 0, 0, 0, 0, 0, 0};
        float dot = 0.0f;
        if (row < nt) {
          cur.vpc[k].to_f(v);
          cur.dypc[k].to_f(dy);
          if (gz) {
            float z[8];
            cur.zpc[k].to_f(z);
#pragma unroll
            for (int e = 0; e < 8; ++e) {
              const float sz = sigmoid_fast(z[e]);
              fz[e] = dy[e] * sz * (1.0f + z[e] * (1.0f - sz));
              dy[e] *= z[e] * sz;
            }
            if (YV && a.dz) {
              // dZ = y_v fz, with y_v the training forward's saved output before the
              // gate (the reference's Out_v residual)
              float yv[8];
              cur.ypc[k].to_f(yv);
#pragma unroll
              for (int e = 0; e < 8; ++e) yv[e] *= fz[e];
              store8(reinterpret_cast<T*>(a.dz) + a.dvz_bat * b + a.dvz_tok * (t0 + row) + (long)h * P + 8 * pc, yv);
            }
          }
#pragma unroll
          for (int e = 0; e < 8; ++e) dot += dy[e] * v[e];
        }
        store8(&sm.v[row][8 * pc], v);
        store8(&sm.dy[row][8 * pc], dy);
        store8(&sm.fz[row][8 * pc], fz);
        dot = group_sum<P / 8>(dot);                   // the row's pieces sit in aligned lanes
        if (pc == 0) sm.dqk[row] = dot;
      }
    }
    __syncthreads();
    if (wave == kQkWave) {
      float qk = 0.0f;
      if (lane < CS) {
#pragma unroll
        for (int w = 0; w < GH; ++w) qk += sm.pq[w][lane];
        sm.qk[lane] = qk;
        dsum += sm.dqk[lane];                         // padding tokens hold dy = 0
      }
    }
    if (c > c_lo) cur.template issue<0>(a, c - 1, bh, tid, wave, lane);   // every use of chunk c's loads is above

    // ---- S = q~ k~^T and dP = dy v^T, masked (s < t) and decayed e^{A_t - A_s}.  Each
    // wave's tiles form a fixed number of iterations without branches (the tiles above
    // the diagonal are computed and masked like the others), so that their loads and
    // MFMA chains interleave.
    static_assert(2 * TB * TB % kBwdWaves == 0, "S/dP tiles: whole rounds");
    if constexpr (kHoist && TB * TB % kBwdWaves == 0) {
      // a wave takes whole (query block, key block) pairs: its S and dP tiles share the
      // decay factors, and the two MFMA chains interleave
#pragma unroll
      for (int j = 0; j < TB * TB / kBwdWaves; ++j) {
        const int i = wave + kBwdWaves * j;
        const int tt = i / TB, st = i % TB;
        // transposed tiles [s][t]: each lane holds 4 consecutive keys s of one query t
        f32x4 accs = {0.0f, 0.0f, 0.0f, 0.0f}, accp = accs;
#pragma unroll
        for (int k0 = 0; k0 < N; k0 += KS)
          accs = W::mma(W::ld(&sm.kt[0][0], N + PADN, 16 * st, k0, lane), W::ld(&sm.qt[0][0], N + PADN, 16 * tt, k0, lane),
                        accs);
#pragma unroll
        for (int k0 = 0; k0 < P; k0 += KS)
          accp = W::mma(W::ld(&sm.v[0][0], P + PAD, 16 * st, k0, lane), W::ld(&sm.dy[0][0], P + PAD, 16 * tt, k0, lane),
                        accp);
        const int t = 16 * tt + (lane & 15), s0 = 16 * st + 4 * (lane >> 4);
        const float at = sm.ac[t];
        float as[4], vs[4], vp[4];
        load4(&sm.ac[s0], as);
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const float e = exp2_fast((at - as[r]) * kLog2e);
          vs[r] = s0 + r < t ? accs[r] * e : 0.0f;
          vp[r] = s0 + r < t ? accp[r] * e : 0.0f;
        }
        store4(smk + t * (CS + PAD) + s0, vs);
        store4(&sm.dpm[0][0] + t * (CS + PAD) + s0, vp);
      }
    } else {
      // (32-token chunks: four pairs, so the S and dP tiles of a pair go to two waves)
#pragma unroll
      for (int j = 0; j < 2 * TB * TB / kBwdWaves; ++j) {
        const int i = wave + kBwdWaves * j;
        const int which = i / (TB * TB), tt = (i % (TB * TB)) / TB, st = (i % (TB * TB)) % TB;
        f32x4 acc = {0.0f, 0.0f, 0.0f, 0.0f};
        if (which == 0) {
#pragma unroll
          for (int k0 = 0; k0 < N; k0 += KS)
            acc = W::mma(W::ld(&sm.kt[0][0], N + PADN, 16 * st, k0, lane), W::ld(&sm.qt[0][0], N + PADN, 16 * tt, k0, lane),
                         acc);
        } else {
#pragma unroll
          for (int k0 = 0; k0 < P; k0 += KS)
            acc = W::mma(W::ld(&sm.v[0][0], P + PAD, 16 * st, k0, lane), W::ld(&sm.dy[0][0], P + PAD, 16 * tt, k0, lane),
                         acc);
        }
        const int t = 16 * tt + (lane & 15), s0 = 16 * st + 4 * (lane >> 4);
        T* dst = which == 0 ? smk : &sm.dpm[0][0];
        const float at = sm.ac[t];
        float as[4], val[4];
        load4(&sm.ac[s0], as);
#pragma unroll
        for (int r = 0; r < 4; ++r) val[r] = s0 + r < t ? acc[r] * exp2_fast((at - as[r]) * kLog2e) : 0.0f;
        store4(dst + t * (CS + PAD) + s0, val);
      }
    }
    __syncthreads();
    if (c > c_lo) cur.template issue<1>(a, c - 1, bh, tid, wave, lane);

    // ---- y (for dZ) and dV as transposed 16 x 16 tiles [p][token]: each lane holds 4
    // consecutive p of one token, written to the output tiles in LDS
    // The tiles' k ranges cover the whole chunk (the masked S is zero outside the causal
    // range), so each wave's tiles are fixed iterations without branches.
    const float aend = sm.aend;
    static_assert(2 * TB * (P / 16) % kBwdWaves == 0, "y/dV tiles: whole rounds");
    // two tiles of one value-column block pt (row blocks r0, r1) of y or dV: the A
    // fragments (v or dy columns, h rows or G columns of the block) are read once for both
    auto ypair = [&](int pt, int r0, int r1) {
      const int p = 16 * pt + 4 * (lane >> 4);
      // y_t = sum_s Sm[t][s] v_s + e^{A_t} h q~_t + (D + QK_t) v_t
      f32x4 c0 = {0.0f, 0.0f, 0.0f, 0.0f}, c1 = c0, d0 = c0, d1 = c0;
#pragma unroll
      for (int k0 = 0; k0 < CS; k0 += KS) {
        const typename W::frag fa = W::ldt(&sm.v[0][0], P + PAD, k0, 16 * pt, lane);
        c0 = W::mma(fa, W::ld(smk, CS + PAD, 16 * r0, k0, lane), c0);
        c1 = W::mma(fa, W::ld(smk, CS + PAD, 16 * r1, k0, lane), c1);
      }
#pragma unroll
      for (int k0 = 0; k0 < N; k0 += KS) {
        const typename W::frag fh = W::ld(&sm.h[0][0], N + PADN, 16 * pt, k0, lane);
        d0 = W::mma(fh, W::ld(&sm.qt[0][0], N + PADN, 16 * r0, k0, lane), d0);
        d1 = W::mma(fh, W::ld(&sm.qt[0][0], N + PADN, 16 * r1, k0, lane), d1);
      }
#pragma unroll
      for (int u2 = 0; u2 < 2; ++u2) {
        const int tl = 16 * (u2 ? r1 : r0) + (lane & 15);
        const f32x4 acc = u2 ? c1 : c0, acc2 = u2 ? d1 : d0;
        float vv[4], ff[4], o[4];
        load4(&sm.v[tl][p], vv);
        load4(&sm.fz[tl][p], ff);
        const float ea = exp_a(tl), dg = Dh + sm.gam[tl] * sm.qk[tl];
#pragma unroll
        for (int r = 0; r < 4; ++r) o[r] = (acc[r] + ea * acc2[r] + dg * vv[r]) * ff[r];
        store4(sm.outs(0) + tl * (P + PAD) + p, o);
      }
    };
    // (two_c false: row block r0 alone)
    auto dvpair = [&](int pt, int r0, int r1, auto two_c) {
      constexpr bool TWO = decltype(two_c)::value;
      const int p = 16 * pt + 4 * (lane >> 4);
      // dv_s = sum_t Sm[t][s] dy_t + e^{A_end - A_s} G^T k~_s + (D + QK_s) dy_s
      f32x4 c0 = {0.0f, 0.0f, 0.0f, 0.0f}, c1 = c0, d0 = c0, d1 = c0;
#pragma unroll
      for (int k0 = 0; k0 < CS; k0 += KS) {
        const typename W::frag fa = W::ldt(&sm.dy[0][0], P + PAD, k0, 16 * pt, lane);
        c0 = W::mma(fa, W::ldt(smk, CS + PAD, k0, 16 * r0, lane), c0);
        if (TWO) c1 = W::mma(fa, W::ldt(smk, CS + PAD, k0, 16 * r1, lane), c1);
      }
#pragma unroll
      for (int k0 = 0; k0 < N; k0 += KS) {
        const typename W::frag fg = W::ldt(&sm.gt[0][0], P + PAD, k0, 16 * pt, lane);
        d0 = W::mma(fg, W::ld(&sm.kt[0][0], N + PADN, 16 * r0, k0, lane), d0);
        if (TWO) d1 = W::mma(fg, W::ld(&sm.kt[0][0], N + PADN, 16 * r1, k0, lane), d1);
      }
#pragma unroll
      for (int u2 = 0; u2 < (TWO ? 2 : 1); ++u2) {
        const int tl = 16 * (u2 ? r1 : r0) + (lane & 15);
        const f32x4 acc = u2 ? c1 : c0, acc2 = u2 ? d1 : d0;
        float yy[4], o[4];
        load4(&sm.dy[tl][p], yy);
        const float ea = exp_b(tl, aend), dg = Dh + sm.gam[tl] * sm.qk[tl];
#pragma unroll
        for (int r = 0; r < 4; ++r) o[r] = acc[r] + ea * acc2[r] + dg * yy[r];
        store4(sm.outs(1) + tl * (P + PAD) + p, o);
      }
    };
    // y is needed for dZ alone; with the training forward's saved output before the
    // gate (a.yv) the preparation has written dZ already
    const bool need_y = gz && a.dz && !YV;
    if constexpr (TB * (P / 16) == 2 * kBwdWaves) {
      // both products per wave, two row blocks each
      const int pt = wave % (P / 16), r0 = wave / (P / 16), r1 = r0 + kBwdWaves / (P / 16);
      if (need_y) ypair(pt, r0, r1);
      dvpair(pt, r0, r1, std::true_type());
    } else if constexpr (TB == 2 && TB * (P / 16) == kBwdWaves) {
      // one product per wave, both row blocks: the first P/16 waves y, the others dV
      // (a y wave and a dV wave on each SIMD); without y, dV one row block per wave
      const int pt = wave % (P / 16);
      if (!need_y) {
        dvpair(pt, wave / (P / 16), 0, std::false_type());
      } else if (wave < P / 16) {
        ypair(pt, 0, 1);
      } else {
        dvpair(pt, 0, 1, std::true_type());
      }
    } else
#pragma unroll
    for (int j = 0; j < 2 * TB * (P / 16) / kBwdWaves; ++j) {
      const int i = wave + kBwdWaves * j;
      const int which = i / (TB * (P / 16)), rt = (i % (TB * (P / 16))) / (P / 16), pt = i % (P / 16);
      f32x4 acc = {0.0f, 0.0f, 0.0f, 0.0f}, acc2 = {0.0f, 0.0f, 0.0f, 0.0f};
      const int tl = 16 * rt + (lane & 15), p = 16 * pt + 4 * (lane >> 4);
      if (which == 0) {
        if (!need_y) continue;
        // y_t = sum_s Sm[t][s] v_s + e^{A_t} h q~_t + (D + QK_t) v_t
#pragma unroll
        for (int k0 = 0; k0 < CS; k0 += KS)
          acc = W::mma(W::ldt(&sm.v[0][0], P + PAD, k0, 16 * pt, lane), W::ld(smk, CS + PAD, 16 * rt, k0, lane), acc);
#pragma unroll
        for (int k0 = 0; k0 < N; k0 += KS)
          acc2 = W::mma(W::ld(&sm.h[0][0], N + PADN, 16 * pt, k0, lane), W::ld(&sm.qt[0][0], N + PADN, 16 * rt, k0, lane),
                        acc2);
        float vv[4], ff[4], o[4];
        load4(&sm.v[tl][p], vv);
        load4(&sm.fz[tl][p], ff);
        const float ea = exp_a(tl), dg = Dh + sm.gam[tl] * sm.qk[tl];
#pragma unroll
        for (int r = 0; r < 4; ++r) o[r] = (acc[r] + ea * acc2[r] + dg * vv[r]) * ff[r];
        store4(sm.outs(0) + tl * (P + PAD) + p, o);
      } else {
        // dv_s = sum_t Sm[t][s] dy_t + e^{A_end - A_s} G^T k~_s + (D + QK_s) dy_s
#pragma unroll
        for (int k0 = 0; k0 < CS; k0 += KS)
          acc = W::mma(W::ldt(&sm.dy[0][0], P + PAD, k0, 16 * pt, lane), W::ldt(smk, CS + PAD, k0, 16 * rt, lane), acc);
#pragma unroll
        for (int k0 = 0; k0 < N; k0 += KS)
          acc2 = W::mma(W::ldt(&sm.gt[0][0], P + PAD, k0, 16 * pt, lane), W::ld(&sm.kt[0][0], N + PADN, 16 * rt, k0, lane),
                        acc2);
        float yy[4], o[4];
        load4(&sm.dy[tl][p], yy);
        const float ea = exp_b(tl, aend), dg = Dh + sm.gam[tl] * sm.qk[tl];
#pragma unroll
        for (int r = 0; r < 4; ++r) o[r] = acc[r] + ea * acc2[r] + dg * yy[r];
        store4(sm.outs(1) + tl * (P + PAD) + p, o);
      }
    }
    __syncthreads();
    // ---- dZ and dV rows from the output tiles
    {
      T* const gdz = reinterpret_cast<T*>(a.dz);
      T* const gdv = reinterpret_cast<T*>(a.dv);
      for (int p = tid; p < 2 * CS * (P / 8); p += kBwdThreads) {
        const int w = p / (CS * (P / 8)), q = p % (CS * (P / 8)), row = q / (P / 8), pc = q % (P / 8);
        if (row < nt && (w == 1 || (gz && gdz && !YV))) {
          const long o = a.dvz_bat * b + a.dvz_tok * (t0 + row) + (long)h * P + 8 * pc;
          *reinterpret_cast<Vec8<T>*>((w ? gdv : gdz) + o) =
              *reinterpret_cast<const Vec8<T>*>(sm.outs(w) + row * (P + PAD) + 8 * pc);
        }
      }
    }
    // ---- advance the adjoint state to the one after chunk c - 1:
    // G <- e^{A_end} G + sum_t e^{A_cum,t} dy_t (x) q~_t (G_c is already in LDS)
    {
      const float dec = exp2_fast(aend * kLog2e);
      const int ntile = wave % NT;
      f32x4 acc[TPW];
#pragma unroll
      for (int i = 0; i < TPW; ++i) acc[i] = G[i] * dec;
#pragma unroll
      for (int k0 = 0; k0 < CS; k0 += KS) {
        float w[W::WN];
#pragma unroll
        for (int j = 0; j < W::WN; ++j) w[j] = exp_a(W::ktok(k0, lane) + j);
        const typename W::frag qf = W::scale(W::ldt(&sm.qt[0][0], N + PADN, k0, 16 * ntile, lane), w);
#pragma unroll
        for (int i = 0; i < TPW; ++i) {
          const int tile = wave + kBwdWaves * i;
          if (tile < NTILE) acc[i] = W::mma(W::ldt(&sm.dy[0][0], P + PAD, k0, 16 * (tile / NT), lane), qf, acc[i]);
        }
      }
#pragma unroll
      for (int i = 0; i < TPW; ++i) G[i] = acc[i];
    }
    if (c > c_lo) cur.template issue<2>(a, c - 1, bh, tid, wave, lane);

    // ---- dq~ then dk~, half the columns at a time, each followed by its chain rule
    // (passes: q~ half 0, q~ half 1, k~ half 0, k~ half 1)
    float dthq[2][PRS];                               // d(theta) from dq~, for pass K
#pragma unroll
    for (int hh = 0; hh < 2; ++hh)
#pragma unroll
      for (int j = 0; j < PRS; ++j) dthq[hh][j] = 0.0f;
    // this lane's q^ / k^ columns and rope pair of the pass's half
    float gq8[EL], gk8[EL], gcs[PRS], gsn[PRS];
    // per token over the wave's groups: q~.dq~ - k~.dk~ and dk~.rot(k^)
    float pacc = 0.0f, sacc = 0.0f;
    auto pass_regs = [&](int pass) {
      const int hh = pass & 1;
#pragma unroll
      for (int e = 0; e < EL; ++e) {
        gq8[e] = hh ? qh[1][e] : qh[0][e];
        gk8[e] = hh ? kh[1][e] : kh[0][e];
      }
#pragma unroll
      for (int j = 0; j < PRS; ++j) {
        gcs[j] = hh ? cs[1][j] : cs[0][j];
        gsn[j] = hh ? sn[1][j] : sn[0][j];
      }
    };
    // The products of a pass into rb [CS][NH + 4] (token rows): dq~ (passes 0, 1) or
    // dk~ (2, 3).  Each wave's tiles are fixed iterations; a tile's k range is that of
    // the wave's largest (dq~) or smallest (dk~) row block in the iteration, which
    // covers its own (the masked dP is zero outside the causal range), so the ranges
    // are compile-time constants once the loop is unrolled.
    auto pass_mfma = [&](int pass, float* rb) {
      const bool isq = pass < 2;
      const int n0 = (pass & 1) * NH;
      constexpr int NT2 = NH / 16, QT = TB * NT2, QJ = (QT + kBwdWaves - 1) / kBwdWaves;
#pragma unroll
      for (int j = 0; j < QJ; ++j) {
        const int i = wave + kBwdWaves * j;
        if (QT % kBwdWaves != 0 && i >= QT) continue;
        const int rt = i / NT2, ntl = i % NT2;
        const int rlo = min(kBwdWaves * j / NT2, TB - 1), rhi = min((kBwdWaves * j + kBwdWaves - 1) / NT2, TB - 1);
        const int kq = ((16 * (rhi + 1) + KS - 1) / KS) * KS, kk = (16 * rlo / KS) * KS;
        f32x4 acc = {0.0f, 0.0f, 0.0f, 0.0f}, acc2 = {0.0f, 0.0f, 0.0f, 0.0f};
        if (isq) {
          // dq~_t = sum_s dPm[t][s] k~_s + e^{A_t} dy_t h
#pragma unroll
          for (int k0 = 0; k0 < kq; k0 += KS) {
            const typename W::frag fa = W::ld(&sm.dpm[0][0], CS + PAD, 16 * rt, k0, lane);
            acc = W::mma(fa, W::ldt(&sm.kt[0][0], N + PADN, k0, n0 + 16 * ntl, lane), acc);
            if constexpr (BF) acc = W::mma(fa, W::ldt(lo, NH + PAD, k0, 16 * ntl, lane), acc);
          }
#pragma unroll
          for (int k0 = 0; k0 < P; k0 += KS)
            acc2 = W::mma(W::ld(&sm.dy[0][0], P + PAD, 16 * rt, k0, lane),
                          W::ldt(&sm.h[0][0], N + PADN, k0, n0 + 16 * ntl, lane), acc2);
        } else {
          // dk~_s = sum_t dPm[t][s] q~_t + e^{A_end - A_s} v_s G
#pragma unroll
          for (int k0 = kk; k0 < CS; k0 += KS) {
            const typename W::frag fa = W::ldt(&sm.dpm[0][0], CS + PAD, k0, 16 * rt, lane);
            acc = W::mma(fa, W::ldt(&sm.qt[0][0], N + PADN, k0, n0 + 16 * ntl, lane), acc);
            if constexpr (BF) acc = W::mma(fa, W::ldt(lo, NH + PAD, k0, 16 * ntl, lane), acc);
          }
#pragma unroll
          for (int k0 = 0; k0 < P; k0 += KS)
            acc2 = W::mma(W::ld(&sm.v[0][0], P + PAD, 16 * rt, k0, lane),
                          W::ld(&sm.gt[0][0], P + PAD, n0 + 16 * ntl, k0, lane), acc2);
        }
        const int nl = 16 * ntl + (lane & 15);
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int t = 16 * rt + 4 * (lane >> 4) + r;
          const float w = isq ? exp_a(t) : exp_b(t, aend);
          rb[t * (NH + 4) + nl] = acc[r] + w * acc2[r];
        }
      }
    };
    // The chain rule of a pass from its products in rb (row stride ldr, this wave's
    // group at column cofs), lane = token (two lanes per token at 32-token chunks, EL
    // columns each), one 8-column group per wave.  kDirect: the lanes store their
    // d(q^) / d(k^) columns and d(theta) pairs straight to the gradients and add up the
    // bias column sums in registers; otherwise they go back into rb and the d(theta)
    // tile, for row stores after a barrier.
    // (the chain rule's LDS reads, apart from its computation, so that a caller can
    // issue them ahead of other work)
    auto chain_load = [&](const float* rb, int ldr, int cofs, float* dx, float& sc, float& gqk) {
      const int rc = tkn * ldr + cofs + EL * hf;   // this lane's slots of rb
#pragma unroll
      for (int e = 0; e < EL; ++e) dx[e] = rb[rc + e];
      sc = sm.scl[tkn];
      gqk = sm.dqk[tkn] * sm.gam[tkn];
    };
    // Padding tokens (t >= nt) hold zeros in rb and in dQK, gamma and the scale, so
    // their results are zeros without a branch; only their stores are skipped.
    auto chain_compute = [&](int pass, const float* dx, float sc, float gqk) {
      const bool isq = pass < 2;
      const int n0 = (pass & 1) * NH;
      const int hh = pass & 1;
      const int g = n0 / 8 + wave;
      if constexpr (GH < kBwdWaves) {
        if (!qkw) return;
      }
      float out[EL], dthv[PRS];
      float dot = 0.0f, dsc = 0.0f;
      {
        float xr[EL];                                   // q~ (pass Q) or rot(k^) (pass K)
#pragma unroll
        for (int e = 0; e < EL; ++e) xr[e] = isq ? gq8[e] : gk8[e];
        rotp<PRS>(xr, gcs, gsn, 4 * g < R, 1.0f);
        const float f = isq ? 1.0f : sc;                // k~ = scale rot(k^)
#pragma unroll
        for (int e = 0; e < EL; ++e) {
          dot += f * xr[e] * dx[e];
          dsc += xr[e] * dx[e];
        }
#pragma unroll
        for (int j = 0; j < PRS; ++j) dthv[j] = f * (dx[2 * j + 1] * xr[2 * j] - dx[2 * j] * xr[2 * j + 1]);
        // d(q^) = rot^T dq~ + dQK gamma k^;  d(k^) = scale rot^T dk~ + dQK gamma q^
#pragma unroll
        for (int e = 0; e < EL; ++e) out[e] = f * dx[e];
        rotp<PRS>(out, gcs, gsn, 4 * g < R, -1.0f);
#pragma unroll
        for (int e = 0; e < EL; ++e) out[e] += gqk * (isq ? gk8[e] : gq8[e]);
      }
      dot = token_pair_sum<TPL>(dot);
      dsc = token_pair_sum<TPL>(dsc);
      if constexpr (kDirect) {
        if (tok) {
          const long row = (long)b * L + t0 + tkn;
          const int col = n0 + 8 * wave + EL * hf;
          if constexpr (GQA) {
            T* dst = reinterpret_cast<T*>(isq ? a.dqh : a.dkh) + (row * H + h) * N + col;
            if constexpr (EL == 4) store4(dst, out); else store8(dst, out);
          } else {
            T* dst = reinterpret_cast<T*>(isq ? a.dq : a.dk) + (row * HQ + hq) * N + col;
            if constexpr (EL == 4) store4(dst, out); else store8(dst, out);
          }
        }
        if constexpr (!BF) {
#pragma unroll
          for (int e = 0; e < EL; ++e) bq[pass][e] += out[e];   // 0 on padding tokens
        } else {
          // the 8 columns summed over the 64 lanes by halving exchanges: lane l keeps
          // column l / 8 of the group, summed over the lanes that share l % 8 (their
          // sum over the walk follows at its end).  v_permlane32_swap exchanges the
          // upper 32 lanes of its first operand with the lower 32 of its second, so the
          // sum of the two results holds column j in lanes 0-31 and column j + 4 in
          // lanes 32-63; v_permlane16_swap does the same with odd and even 16-lane rows.
          float v4[4], v2[2];
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(out[j]), __float_as_uint(out[j + 4]),
                                                            false, false);
            v4[j] = __uint_as_float(r[0]) + __uint_as_float(r[1]);
          }
#pragma unroll
          for (int j = 0; j < 2; ++j) {
            const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v4[j]), __float_as_uint(v4[j + 2]),
                                                            false, false);
            v2[j] = __uint_as_float(r[0]) + __uint_as_float(r[1]);
          }
          const bool b3 = lane & 8;
          constexpr int kDppRowRor8 = 0x128;   // lane l <- lane l ^ 8 of its row
          bacc[pass] += (b3 ? v2[1] : v2[0]) + dpp0<kDppRowRor8>(b3 ? v2[0] : v2[1]);
        }
      } else {
        // d(q^) / d(k^) back into the thread's own slots of the product tile (res),
        // for the row stores and the bias column sums
#pragma unroll
        for (int e = 0; e < EL; ++e) res[tkn * (NH + 4) + 8 * wave + EL * hf + e] = out[e];
      }
      if (isq) {
#pragma unroll
        for (int j = 0; j < PRS; ++j) dthq[hh][j] = dthv[j];
      } else if (4 * g < R) {
        // the token's d(theta) of each pair; its reverse cumsum over the sequence is
        // the chunk's suffix sum plus the later chunks' total (0 on padding tokens)
        float sv[PRS], d[PRS], f[PRS];
#pragma unroll
        for (int j = 0; j < PRS; ++j) f[j] = d[j] = dthq[hh][j] + dthv[j];
        token_scan<PRS>(f);
#pragma unroll
        for (int j = 0; j < PRS; ++j) {
          const float tot = token_scan_total<PRS>(f[j], hf);
          sv[j] = cth[hh][j] + tot - f[j] + d[j];
          cth[hh][j] += tot;
        }
        if constexpr (kDirect) {
          // pairs 4 g + PRS hf + j (4 g < R, R a multiple of 4)
          if (tok) {
            float* dst = a.dang + (((long)b * L + t0 + tkn) * H + h) * R + 4 * g + PRS * hf;
            if constexpr (PRS == 4) store4(dst, sv);
            else *reinterpret_cast<float2*>(dst) = make_float2(sv[0], sv[1]);
          }
        } else {
          if constexpr (PRS == 4) store4(dth + tkn * RH + 4 * wave, sv);
          else *reinterpret_cast<float2*>(dth + tkn * RH + 4 * wave + 2 * hf) = make_float2(sv[0], sv[1]);
        }
      }
      if (isq) {
        pacc += dot;
      } else {
        pacc -= dot;
        sacc += dsc;
      }
      // after the wave's last pass: its row of the per-token partial sums
      if (pass == 3 && hf == 0) {
        sm.pq[wave][tkn] = pacc;
        sm.ps[wave][tkn] = sacc;
      }
    };
    auto pass_chain = [&](int pass, const float* rb, int ldr, int cofs) {
      if constexpr (GH < kBwdWaves) {
        if (!qkw) return;
      }
      float dx[EL], sc, gqk;
      chain_load(rb, ldr, cofs, dx, sc, gqk);
      chain_compute(pass, dx, sc, gqk);
    };
    if constexpr (kQP) {
      // bf16, d_state 128: quarter q (0..7) is pass q / 2, columns 32 (q % 2) .. + 31 of
      // its half, whose 8-column groups belong to waves 4 (q % 2) .. + 3.  Software
      // pipeline, one barrier per quarter: the products of quarter q + 1 beside the chain
      // rule of quarter q and the rounding residual of quarter q + 2, over two product
      // and two residual tiles.
      // rounding residual of the operand of pass `pass`, k~ (dq~) or q~ (dk~), in this
      // wave's quarter (the waves of one half), into residual tile `slot`
      auto quarter_lo = [&](int pass, int slot) {
        const int hh = pass & 1;
        const bool isq = pass < 2;
        const int g = hh * GH + wave;
        float x[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) x[e] = isq ? kh[hh][e] : qh[hh][e];
        rotp<PRS>(x, cs[hh], sn[hh], 4 * g < R, 1.0f);
        const float sc = isq && tok ? sm.scl[lane] : 1.0f;
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          x[e] *= sc;
          x[e] -= (float)(bf16)x[e];
        }
        store8(sm.loq(slot) + lane * (NH + PAD) + 8 * (wave & 3), x);
      };
      // The products of quarter q into rb, tiles (row block rt, column tile ntl): with
      // `both`, the two tiles (rt, ntl) and (rt + 2, ntl) of rt = (wave % 4) / 2, ntl =
      // wave % 2 (the waves of one half cover the quarter), else the one tile (wave / 2,
      // wave % 2).  The two tiles share their k~ / q~, residual and h / G fragments, and
      // k blocks outside the causal range are skipped (the masked dP is zero there).
      auto quarter_mfma = [&](int q, float* rb, auto both) {
        constexpr bool B2 = decltype(both)::value;
        const int pass = q >> 1;
        const bool isq = pass < 2;
        const int c0 = (pass & 1) * NH + S::NQ * (q & 1) + 16 * (wave & 1);
        const int ra = B2 ? (wave & 3) >> 1 : wave >> 1;
        const T* lq = sm.loq(q & 1) + 16 * (wave & 1);
        f32x4 a0 = {0.0f, 0.0f, 0.0f, 0.0f}, a1 = a0, b0 = a0, b1 = a0;
#pragma unroll
        for (int k0 = 0; k0 < CS; k0 += KS) {
          // which tiles take this k block (B2: ra <= 1; dq~ block 0 both, block 1 the
          // lower tile; dk~ block 1 both, block 0 the upper tile)
          const bool ta = B2 ? (isq ? k0 == 0 : true) : (isq ? k0 < 16 * (ra + 1) : k0 + KS > 16 * ra);
          const bool tb = B2 && (isq ? true : k0 > 0);
          if (!ta && !tb) continue;
          const typename W::frag fo = W::ldt(isq ? &sm.kt[0][0] : &sm.qt[0][0], N + PADN, k0, c0, lane);
          const typename W::frag fl = W::ldt(lq, NH + PAD, k0, 0, lane);
          if (ta) {
            const typename W::frag fa = isq ? W::ld(&sm.dpm[0][0], CS + PAD, 16 * ra, k0, lane)
                                            : W::ldt(&sm.dpm[0][0], CS + PAD, k0, 16 * ra, lane);
            a0 = W::mma(fa, fo, a0);
            a0 = W::mma(fa, fl, a0);
          }
          if (tb) {
            const typename W::frag fb = isq ? W::ld(&sm.dpm[0][0], CS + PAD, 16 * (ra + 2), k0, lane)
                                            : W::ldt(&sm.dpm[0][0], CS + PAD, k0, 16 * (ra + 2), lane);
            a1 = W::mma(fb, fo, a1);
            a1 = W::mma(fb, fl, a1);
          }
        }
#pragma unroll
        for (int k0 = 0; k0 < P; k0 += KS) {
          // dq~: e^{A_t} dy_t h;  dk~: e^{A_end - A_s} v_s G
          const typename W::frag fs = isq ? W::ldt(&sm.h[0][0], N + PADN, k0, c0, lane)
                                          : W::ld(&sm.gt[0][0], P + PAD, c0, k0, lane);
          const T* xs = isq ? &sm.dy[0][0] : &sm.v[0][0];
          b0 = W::mma(W::ld(xs, P + PAD, 16 * ra, k0, lane), fs, b0);
          if (B2) b1 = W::mma(W::ld(xs, P + PAD, 16 * (ra + 2), k0, lane), fs, b1);
        }
        const int nl = 16 * (wave & 1) + (lane & 15);
#pragma unroll
        for (int u2 = 0; u2 < (B2 ? 2 : 1); ++u2) {
          const f32x4 acc = u2 ? a1 : a0, acc2 = u2 ? b1 : b0;
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            const int t = 16 * (ra + 2 * u2) + 4 * (lane >> 4) + r;
            const float w = isq ? exp_a(t) : exp_b(t, aend);
            rb[t * (S::NQ + 4) + nl] = acc[r] + w * acc2[r];
          }
        }
      };
      static_assert(!kQP || (CS == 64 && KS == 32 && GH == kBwdWaves && TB * (S::NQ / 16) == kBwdWaves),
                    "quarter passes: 8 product tiles and four groups per quarter, two k blocks");
      // quarters 0 and 1 (their residual tiles lie outside the output tiles that the
      // dZ/dV row stores above still read)
      quarter_lo(0, wave >> 2);
      __syncthreads();
      quarter_mfma(0, sm.rq(0), std::false_type());
      __syncthreads();
      // quarter q: the waves of half q % 2 run its chain rule and quarter q + 2's
      // residual, the other half quarter q + 1's products (a VALU wave and an MFMA wave
      // on each SIMD)
#pragma unroll
      for (int q = 0; q < 8; ++q) {
        if ((wave >> 2) == (q & 1)) {
          pass_regs(q >> 1);
          pass_chain(q >> 1, sm.rq(q & 1), S::NQ + 4, 8 * (wave & 3));
          if (q < 6) quarter_lo((q + 2) >> 1, q & 1);
        } else if (q < 7) {
          quarter_mfma(q + 1, sm.rq((q + 1) & 1), std::true_type());
        }
        if (q == 3 && c > c_lo) cur.template issue<3>(a, c - 1, bh, tid, wave, lane);
        // the tiles read above are written two quarters on; the last quarter's
        // per-token sums are read by the dA below
        __syncthreads();
      }
    } else if constexpr (!BF) {
      // Software pipeline, one barrier per pass: each wave's products of pass p + 1 go
      // into one tile while the chain rule of pass p reads the other, so that a SIMD's
      // two waves overlap MFMA and VALU work.
      float* const rbuf[2] = {res, sm.res2()};
      pass_mfma(0, rbuf[0]);
      __syncthreads();
#pragma unroll
      for (int pass = 0; pass < 4; ++pass) {
        // the chain rule's inputs first, so that its computation can interleave with
        // the products' MFMA chains (their tile stores would otherwise order them)
        float dx[EL], sc = 0.0f, gqk = 0.0f;
        if (qkw) chain_load(rbuf[pass & 1], NH + 4, 8 * wave, dx, sc, gqk);
        if (pass < 3) pass_mfma(pass + 1, rbuf[(pass + 1) & 1]);
        pass_regs(pass);
        chain_compute(pass, dx, sc, gqk);
        if (pass == 1 && c > c_lo) cur.template issue<3>(a, c - 1, bh, tid, wave, lane);
        // the tile read above is written by pass p + 2's products; the last pass's
        // per-token sums are read by the dA below
        __syncthreads();
      }
    } else {
#pragma unroll
      for (int pass = 0; pass < 4; ++pass) {
        const bool isq = pass < 2;
        const int n0 = (pass & 1) * NH;
        pass_regs(pass);
        if constexpr (BF) {
          // rounding residual of the operand this pass multiplies: k~ (dq~) or q~ (dk~)
          if (qkw) {
            const int g = n0 / 8 + wave;
            float x[8];
#pragma unroll
            for (int e = 0; e < 8; ++e) x[e] = isq ? gk8[e] : gq8[e];
            rotp<PRS>(x, gcs, gsn, 4 * g < R, 1.0f);
            const float sc = isq && tok ? sm.scl[lane] : 1.0f;
#pragma unroll
            for (int e = 0; e < 8; ++e) {
              x[e] *= sc;
              x[e] -= (float)(bf16)x[e];
            }
            if (lane < CS) store8(lo + lane * (NH + PAD) + 8 * wave, x);
          }
          __syncthreads();
        }
        pass_mfma(pass, res);
        __syncthreads();
        pass_chain(pass, res, NH + 4, 8 * wave);
        __syncthreads();
        // d(q^) / d(k^) rows of the half, the bias column sums, and (pass K) the half's
        // d(theta) rows
        {
          for (int p = tid; p < CS * (NH / 8); p += kBwdThreads) {
            const int row = p / (NH / 8), pc = p % (NH / 8);
            if (row < nt) {
              float o8[8];
#pragma unroll
              for (int e = 0; e < 8; ++e) o8[e] = res[row * (NH + 4) + 8 * pc + e];
              if constexpr (GQA) {
                store8(reinterpret_cast<T*>(isq ? a.dqh : a.dkh) + (((long)b * L + t0 + row) * H + h) * N + n0 + 8 * pc,
                       o8);
              } else {
                store8(reinterpret_cast<T*>(isq ? a.dq : a.dk) + (((long)b * L + t0 + row) * HQ + hq) * N + n0 + 8 * pc,
                       o8);
              }
            }
          }
          const int bn = tid % NH, btg = tid / NH;
#pragma unroll
          for (int i = 0; i < TPG; ++i) bacc[pass] += res[(btg * TPG + i) * (NH + 4) + bn];
          if (!isq) {
            const int R0 = (pass & 1) * (NH / 2);                 // first pair of the half
            const int RN = R - R0 < 0 ? 0 : (R - R0 < NH / 2 ? R - R0 : NH / 2);
            if (RN > 0) {
              for (int p = tid; p < CS * (RN / 4); p += kBwdThreads) {
                const int row = p / (RN / 4), q4 = p % (RN / 4);
                if (row < nt)
                  *reinterpret_cast<float4*>(a.dang + (((long)b * L + t0 + row) * H + h) * R + R0 + 4 * q4) =
                      *reinterpret_cast<const float4*>(dth + row * RH + 4 * q4);
              }
            }
          }
        }
        // (bf16) the next pass writes res and lo after its residual barrier
        if (pass == 1 && c > c_lo) cur.template issue<3>(a, c - 1, bh, tid, wave, lane);
      }
    }

    // ---- per token: dA (its reverse cumsum into dADT), d(gamma) into dDT, d(scale)
    // into the workspace
    // (lane = token here; lanes CS.. hold no token)
    if (wave == kDsWave && lane < nt) {
      float ds = 0.0f;
#pragma unroll
      for (int w = 0; w < GH; ++w) ds += sm.ps[w][lane];
      const long o = (long)bh * L + t0 + lane;
      a.dsc[o] = ds;
      a.ddt[o] = sm.dqk[lane] * sm.qk[lane] + ds;
    }
    if (wave == kDaWave) {
      const bool ltok = lane < nt;
      float da = 0.0f;
      if (ltok) {
#pragma unroll
        for (int w = 0; w < GH; ++w) da += sm.pq[w][lane];
      }
      const float f = wave_incl_scan(da);
      const float tot = lane63(f);
      if (ltok) a.dadt[(long)bh * L + t0 + lane] = cda + tot - f + da;
      cda += tot;
    }
    // the next chunk's staging overlaps res and the d(theta) tile read above (the
    // quarter passes end with a barrier and store their rows themselves)
    if constexpr (BF && !kQP) __syncthreads();
  }

  // ---- the walk's totals: bias and D gradients of this (b, h), and the sums over the
  // sequence of dA and of d(theta) per pair (rounding only: both are exactly zero)
  {
    const int tid = threadIdx.x, lane = tid & 63;
    if constexpr (kQP) {
      // lane l holds column l / 8 of the wave's group, summed over the lanes that share
      // l % 8
#pragma unroll
      for (int pass = 0; pass < 4; ++pass) {
        float v = bacc[pass];
        v += __shfl_xor(v, 1, 64);
        v += __shfl_xor(v, 2, 64);
        v += __shfl_xor(v, 4, 64);
        if ((lane & 7) == 0) (pass < 2 ? a.pqb : a.pkb)[ps * N + (pass & 1) * NH + 8 * wave + (lane >> 3)] = v;
      }
    } else if constexpr (kDirect) {
      // sums over the token lanes (the lanes of one hf hold the same columns)
      if (qkw) {
        const int tkn = lane & (CS - 1), hf = lane / CS;
#pragma unroll
        for (int pass = 0; pass < 4; ++pass)
#pragma unroll
          for (int e = 0; e < EL; ++e) {
            float v = bq[pass][e];
#pragma unroll
            for (int m = 1; m < CS; m <<= 1) v += __shfl_xor(v, m, 64);
            if (tkn == 0)
              (pass < 2 ? a.pqb : a.pkb)[ps * N + (pass & 1) * NH + 8 * wave + EL * hf + e] = v;
          }
      }
    } else {
      const int bn = tid % NH, btg = tid / NH;
#pragma unroll
      for (int pass = 0; pass < 4; ++pass) {
        __syncthreads();
        res[btg * (NH + 4) + bn] = bacc[pass];
        __syncthreads();
        if (tid < NH) {
          float s = 0.0f;
          for (int i = 0; i < kBwdThreads / NH; ++i) s += res[i * (NH + 4) + tid];
          (pass < 2 ? a.pqb : a.pkb)[ps * N + (pass & 1) * NH + tid] = s;
        }
      }
    }
    if (qkw) {
      const int tkn = lane & (CS - 1), hf = lane / CS;
#pragma unroll
      for (int hh = 0; hh < 2; ++hh)
#pragma unroll
        for (int j = 0; j < PRS; ++j) {
          const int r = 4 * (hh * GH + wave) + PRS * hf + j;
          if (r < R && tkn == 0) a.ctot[ps * (R + 1) + 1 + r] = cth[hh][j];
        }
    }
    if (wave == kQkWave) {
      const float tot = wave_sum(dsum);
      if (lane == 0 && a.pd) a.pd[ps] = tot;
    }
    if (wave == kDaWave && lane == 0) a.ctot[ps * (R + 1)] = cda;
  }
}

// Finishing pass of the walk, one workgroup per (chunk, b, h).  dADT and dAngles hold
// the reverse cumsums S_t of dA and d(theta), ctot their totals T over the sequence.
// The output depends on the angles and on A only through differences theta_t -
// theta_s and A_t - A_s (there is no initial carry), so the per-token d(theta) and dA
// sum to exactly zero over the sequence, for every pair.  S_t then carries the whole
// sequence's rounding error at t = 0, where the true value is 0.  S_t - T (L - t) / L
// is the blend (t / L) S_t - ((L - t) / L) F_t of the reverse sum and the negated
// forward sum F_t = T - S_t: the same value in exact arithmetic, and the
// minimum-variance combination of the two when the per-token errors are independent.
// Then dAngles = S pi dt (1 - tanh^2 rate), the angle part of dDT = pi sum_r S tanh,
// du_t = d(scale)_{t-1}, dDT = dgamma sigmoid + du (1 - sigmoid) + angle part and
// dTrap = (dgamma - du) dt sigmoid (1 - sigmoid).
// With the walk split into segments, dADT and dAngles hold each segment's own suffix
// sums and ctot each segment's totals: S_t adds the totals of the later segments
// (off), and T is the sum over all segments.
template <int CS>
__global__ __launch_bounds__(256)
void scan_bwd_walk_finish_kernel(BwdArgs a) {
  __shared__ float tot[65], off[65];
  __shared__ float dts[CS], angp[CS];
  const int tid = threadIdx.x;
  // grid (B*H, chunks): consecutive blocks take the heads of one chunk, so that the
  // blocks in flight read whole (token, all heads) rows of dAngles and the rates
  const int c = blockIdx.y, bh = blockIdx.x, b = bh / a.s.H, h = bh % a.s.H;
  const int L = a.s.L, H = a.s.H, R = a.s.R;
  const int t0 = c * CS, nt = min(CS, L - t0);
  if (tid <= R) {
    const int nseg = a.nseg, seg = nseg > 1 ? c / a.seg_nc : 0;
    const float* ct = a.ctot + (long)bh * nseg * (R + 1) + tid;
    float later = 0.0f;
    for (int j = nseg - 1; j > seg; --j) later += ct[(long)j * (R + 1)];
    float all = later;
    for (int j = seg; j >= 0; --j) all += ct[(long)j * (R + 1)];
    off[tid] = later;
    tot[tid] = all;
  }
  if (tid < CS) {
    dts[tid] = tid < nt ? a.s.dt[(long)bh * L + t0 + tid] : 0.0f;
    angp[tid] = 0.0f;
  }
  __syncthreads();
  if (R > 0) {
    // (token, 4 pairs) pieces; the R / 4 pieces of a token sit in consecutive lanes
    const int QR = R / 4;
    const long row0 = (((long)b * L + t0) * H + h) * R;
    const int AH = a.s.ang_shared ? 1 : H;
    const long arow0 = (((long)b * L + t0) * AH + (a.s.ang_shared ? 0 : h)) * R;
    for (int base = 0; base < CS * QR; base += 256) {
      const int i = base + tid, tt = i / QR, q = i % QR;
      float part = 0.0f;
      if (tt < nt) {
        const float w = (float)(L - t0 - tt) / (float)L;
        float4 s = *reinterpret_cast<const float4*>(a.dang + row0 + (long)tt * H * R + 4 * q);
        const float4 rt = *reinterpret_cast<const float4*>(a.s.ang + arow0 + (long)tt * AH * R + 4 * q);
        float sv[4] = {s.x, s.y, s.z, s.w};
        const float rv[4] = {rt.x, rt.y, rt.z, rt.w};
        const float f = kPi * dts[tt];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const float v = (sv[j] + off[1 + 4 * q + j]) - tot[1 + 4 * q + j] * w;
          const float tn = tanhf(rv[j]);
          sv[j] = v * f * (1.0f - tn * tn);
          part += v * tn;
        }
        *reinterpret_cast<float4*>(a.dang + row0 + (long)tt * H * R + 4 * q) = make_float4(sv[0], sv[1], sv[2], sv[3]);
      }
      // sum over the token's pieces (aligned groups of QR lanes)
      if (QR == 4) part = group_sum<4>(part);
      else if (QR == 8) part = group_sum<8>(part);
      else part = group_sum<16>(part);
      if (q == 0 && tt < nt) angp[tt] = part * kPi;
    }
    __syncthreads();
  }
  if (tid < nt) {
    const long o = (long)bh * L + t0 + tid;
    const int t = t0 + tid;
    const float dt = dts[tid];
    const float du = t > 0 ? a.dsc[o - 1] : 0.0f;
    const float dg = a.ddt[o];
    const float sg = 1.0f / (1.0f + expf(-a.s.trap[o]));
    a.dadt[o] = (a.dadt[o] + off[0]) - tot[0] * (float)(L - t) / (float)L;
    a.ddt[o] = dg * sg + du * (1.0f - sg) + angp[tid];
    a.dtrap[o] = (dg - du) * dt * sg * (1.0f - sg);
  }
}

// --------------------------------------------------------------- finishing scans
// One workgroup per (chunk, b, h), lane = token: dadt = reverse cumsum of dA; dPhi =
// reverse cumsum of d(theta), dAngles = dPhi pi dt (1 - tanh^2), the angle part of
// dDT = pi sum_r dPhi tanh; du_t = d(scale)_{t-1}; dDT = dgamma sigmoid + du
// (1 - sigmoid) + angle part; dTrap = (dgamma - du) dt sigmoid (1 - sigmoid).  The
// sums over later chunks come from the chunk totals.  The chunk's d(theta) and angle
// rate rows pass through LDS so that the (token, pair) tiles move coalesced.
constexpr int kFinWaves = 4;
template <int CS>
__global__ __launch_bounds__(64 * kFinWaves)
void scan_bwd_finish_kernel(BwdArgs a) {
  __shared__ float part[kFinWaves][64];
  __shared__ float carry[65];                // [0]: dA of the later chunks, [1 + r]: d(theta)
  __shared__ float total[65];                // the same over every chunk
  __shared__ float tdth[CS][65];             // d(theta), then dAngles, of (token, pair)
  __shared__ float tang[CS][65];             // angle rates
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int c = blockIdx.x, bh = blockIdx.y, b = bh / a.s.H, h = bh % a.s.H;
  const int L = a.s.L, H = a.s.H, R = a.s.R, nc = a.nc;
  const float kPi = 3.14159265358979323846f;
  // suffix sums of the chunk totals over chunks c+1.., and their sum over all chunks,
  // one value per wave pass
  for (int v = wave; v <= R; v += kFinWaves) {
    float s = 0.0f, s_all = 0.0f;
    for (int cc = lane; cc < nc; cc += 64) {
      const float x = a.ctot[((long)bh * nc + cc) * (R + 1) + v];
      s_all += x;
      if (cc > c) s += x;
    }
    s = wave_sum(s);
    s_all = wave_sum(s_all);
    if (lane == 0) {
      carry[v] = s;
      total[v] = s_all;
    }
  }
  __syncthreads();
  const int t = c * CS + lane;
  const bool tok = lane < CS && t < L;
  const long o = (long)bh * L + t;
  const float dt = tok ? a.s.dt[o] : 0.0f;
  // The output depends on the angles and on A only through differences theta_t -
  // theta_s and A_t - A_s (there is no initial carry), so the per-token d(theta) and
  // dA sum to exactly zero over the sequence, for every pair.  The reverse cumsum S_t
  // of the computed values then carries the whole sequence's rounding error at t = 0,
  // where the true value is 0.  S_t - T (L - t) / L, with T the computed total, is
  // the blend (t / L) S_t - ((L - t) / L) F_t of the reverse sum and the negated
  // forward sum F_t = T - S_t: the same value in exact arithmetic, and the
  // minimum-variance combination of the two when the per-token errors are independent.
  const float wfwd = (float)(L - t) / (float)L;
  const int nt = min(CS, L - c * CS);                                // tokens of this chunk
  const long row0 = (((long)b * L + c * CS) * H + h) * R;           // (token 0, pair 0)
  const int AH = a.s.ang_shared ? 1 : H;                             // angle-rate rows per token
  const long arow0 = (((long)b * L + c * CS) * AH + (a.s.ang_shared ? 0 : h)) * R;
  for (int i = tid; i < nt * R; i += 64 * kFinWaves) {
    const int tt = i / R, r = i % R;
    tdth[tt][r] = a.dang[row0 + (long)tt * H * R + r];
    tang[tt][r] = a.s.ang[arow0 + (long)tt * AH * R + r];
  }
  __syncthreads();
  float angp = 0.0f;
  for (int r = wave; r < R; r += kFinWaves) {
    const float d = tok ? tdth[lane][r] : 0.0f;
    const float sum = wave_rev_scan(d, lane) + carry[1 + r] - total[1 + r] * wfwd;
    if (tok) {
      const float tn = tanhf(tang[lane][r]);
      tdth[lane][r] = sum * kPi * dt * (1.0f - tn * tn);
      angp += sum * tn * kPi;
    }
  }
  part[wave][lane] = angp;
  __syncthreads();
  for (int i = tid; i < nt * R; i += 64 * kFinWaves) {
    const int tt = i / R, r = i % R;
    a.dang[row0 + (long)tt * H * R + r] = tdth[tt][r];
  }
  if (wave == 0) {
    const float dA = tok ? a.dadt[o] : 0.0f;
    const float sum = wave_rev_scan(dA, lane) + carry[0] - total[0] * wfwd;
    float angd = 0.0f;
    for (int w = 0; w < kFinWaves; ++w) angd += part[w][lane];
    if (tok) {
      const float du = t > 0 ? a.dsc[o - 1] : 0.0f;
      const float dg = a.ddt[o];
      const float sg = 1.0f / (1.0f + expf(-a.s.trap[o]));
      a.dadt[o] = sum;
      a.ddt[o] = dg * sg + du * (1.0f - sg) + angd;
      a.dtrap[o] = (dg - du) * dt * sg * (1.0f - sg);
    }
  }
}

// Bias and D gradients: sums over batch and chunks of the per-chunk partials.  Block
// (h, column block of 16): 16 partial sums per column in a fixed order, then a tree.
__global__ __launch_bounds__(256)
void scan_bwd_reduce_kernel(BwdArgs a) {
  __shared__ float red[2][256];
  const int h = blockIdx.x, tid = threadIdx.x, N = a.s.N, H = a.s.H, B = a.s.B, nc = a.nc;
  const int n = blockIdx.y * 16 + (tid & 15), part = tid >> 4;
  const int J = B * nc;
  float sq = 0.0f, sk = 0.0f;
  if (n < N)
    for (int j = part; j < J; j += 16) {
      const long i = (((long)(j / nc) * H + h) * nc + j % nc) * N + n;
      sq += a.pqb[i];
      sk += a.pkb[i];
    }
  red[0][tid] = sq;
  red[1][tid] = sk;
  __syncthreads();
  for (int w = 128; w >= 16; w >>= 1) {
    if (tid < w) {
      red[0][tid] += red[0][tid + w];
      red[1][tid] += red[1][tid + w];
    }
    __syncthreads();
  }
  if (tid < 16 && n < N) {
    a.dqb[(long)h * N + n] = red[0][tid];
    a.dkb[(long)h * N + n] = red[1][tid];
  }
  if (a.dD && blockIdx.y == 0) {
    __syncthreads();
    float s = 0.0f;
    for (int j = tid; j < J; j += 256) s += a.pd[((long)(j / nc) * H + h) * nc + j % nc];
    red[0][tid] = s;
    __syncthreads();
    for (int w = 128; w >= 1; w >>= 1) {
      if (tid < w) red[0][tid] += red[0][tid + w];
      __syncthreads();
    }
    if (tid == 0) a.dD[h] = red[0][0];
  }
}

// Shared angle rates: dAngles (B, L, R) = sum over heads of the per-head gradients.
// Thread = four consecutive pairs of one (b, t) (R is a multiple of 4); the heads are
// summed in order, eight 16-byte loads in flight.
__global__ __launch_bounds__(256) void scan_bwd_angle_heads_kernel(BwdArgs a, float* dang_out) {
  const int H = a.s.H, R4 = a.s.R / 4;
  const long total = (long)a.s.B * a.s.L * R4;
  for (long i = (long)blockIdx.x * blockDim.x + threadIdx.x; i < total; i += (long)gridDim.x * blockDim.x) {
    const long bt = i / R4;
    const float4* src = reinterpret_cast<const float4*>(a.dang) + bt * H * R4 + i % R4;
    float4 s = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    int h = 0;
    for (; h + 8 <= H; h += 8) {
      float4 v[8];
#pragma unroll
      for (int j = 0; j < 8; ++j) v[j] = src[(long)(h + j) * R4];
#pragma unroll
      for (int j = 0; j < 8; ++j) s = make_float4(s.x + v[j].x, s.y + v[j].y, s.z + v[j].z, s.w + v[j].w);
    }
    for (; h < H; ++h) {
      const float4 v = src[(long)h * R4];
      s = make_float4(s.x + v.x, s.y + v.y, s.z + v.z, s.w + v.w);
    }
    reinterpret_cast<float4*>(dang_out)[i] = s;
  }
}

// Four consecutive elements of the I/O type as floats (8 bytes of bf16, 16 of float).
__device__ __forceinline__ void load4f(const bf16* p, float f[4]) {
  const uint2 w = *reinterpret_cast<const uint2*>(p);
  f[0] = __uint_as_float(w.x << 16);
  f[1] = __uint_as_float(w.x & 0xffff0000u);
  f[2] = __uint_as_float(w.y << 16);
  f[3] = __uint_as_float(w.y & 0xffff0000u);
}
__device__ __forceinline__ void load4f(const float* p, float f[4]) {
  const float4 v = *reinterpret_cast<const float4*>(p);
  f[0] = v.x; f[1] = v.y; f[2] = v.z; f[3] = v.w;
}

// GQA: dQ, dK of a Q/K head = sum over the value heads that share it, in float32 over
// the per-head partials (in the I/O type: with bf16 I/O the partials exchanged are
// bf16, as the reference's fused path exchanges its per-head gradient tiles in its io
// dtype, mamba3_pallas.py:832-836).  Thread = eight consecutive columns of one
// (b, t, hq) row of both (16-byte loads and stores at bf16); the heads are summed in
// order, eight loads of each in flight.
template <typename T>
__global__ __launch_bounds__(256) void scan_bwd_gqa_kernel(BwdArgs a) {
  const int B = a.s.B, L = a.s.L, H = a.s.H, HQ = a.s.Hqk, N = a.s.N, N8 = N / 8, rep = H / HQ;
  const long total = (long)B * L * HQ * N8;
  for (long i = (long)blockIdx.x * blockDim.x + threadIdx.x; i < total; i += (long)gridDim.x * blockDim.x) {
    const int n8 = i % N8;
    const long row = i / N8;                     // (b, t, hq)
    const int hq = row % HQ;
    const long bt = row / HQ;
    const long s0 = (bt * H + (long)hq * rep) * N + 8 * n8;
    const T* q = reinterpret_cast<const T*>(a.dqh) + s0;
    const T* k = reinterpret_cast<const T*>(a.dkh) + s0;
    float sq[8] = {0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f}, sk[8] = {0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f};
    int j = 0;
    for (; j + 8 <= rep; j += 8) {
      Vec8<T> vq[8], vk[8];
#pragma unroll
      for (int u = 0; u < 8; ++u) {
        vq[u].load(q + (long)(j + u) * N);
        vk[u].load(k + (long)(j + u) * N);
      }
#pragma unroll
      for (int u = 0; u < 8; ++u) {
        float fq[8], fk[8];
        vq[u].to_f(fq);
        vk[u].to_f(fk);
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          sq[e] += fq[e];
          sk[e] += fk[e];
        }
      }
    }
    for (; j < rep; ++j) {
      Vec8<T> vq, vk;
      vq.load(q + (long)j * N);
      vk.load(k + (long)j * N);
      float fq[8], fk[8];
      vq.to_f(fq);
      vk.to_f(fk);
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        sq[e] += fq[e];
        sk[e] += fk[e];
      }
    }
    store8(reinterpret_cast<T*>(a.dq) + 8 * i, sq);
    store8(reinterpret_cast<T*>(a.dk) + 8 * i, sk);
  }
}

size_t al256(size_t x) { return (x + 255) & ~size_t(255); }

struct BwdWs {
  size_t hs, gs, th, pqb, pkb, pd, dsc, ctot, dqh, dkh, dangh, gin, gloc, dseg, split, total;
};

// Route of the backward.  The reverse walk runs one workgroup per (b, h), so it fills
// the chip only when B * H is large; below kWalkMinBH the chunk-parallel kernels (one
// workgroup per (chunk, b, h), with the adjoint pass before them) run instead.
// Measured (bf16, d_state 128, headdim 64): the routes tie at 64 pairs (1.08 / 1.05
// ms at L=4096), the one-segment walk wins at 96 (3.25 / 3.97 ms at config 5's B=4,
// L=12288, H=24) and 128 (1.12 / 1.54 ms), the chunks at 32 (2.11 / 1.60 ms at
// L=8192).  The environment variable M3_BWD_ROUTE = "walk" or "chunks" forces one of
// them (tests, measurements).
// Below kWalkTargetBlocks pairs the walk is split into sequence segments, each walked
// from the adjoint state that the later segments leave (an adjoint-only pass per
// segment and a reverse combine, the backward's form of the forward's sequence split),
// when the sequence holds at least two segments of kWalkMinSegChunks chunks and the
// split's modelled time (split_cost) is at most 0.8 of the one-segment walk's; below
// kWalkMinBH pairs whenever it can, and otherwise shorter sequences take the
// chunk-parallel route.  M3_BWD_ROUTE = "segments" forces the split walk (segments
// of at least two chunks), "walk" the one-segment walk.
constexpr long kWalkMinBH = 80;
constexpr int kWalkTargetBlocks = 256;
constexpr int kWalkMinSegChunks = 4;
constexpr int kWalkMaxRounds = 4;
struct BwdRoute {
  bool walk;
  int nseg, seg_nc;
  // sub-segments per walk segment of the adjoint-only pass: segments of 8 chunks or
  // more are cut in up to four
  int adj_sub() const { return nseg > 1 ? std::max(1, std::min(4, seg_nc / 8)) : 1; }
};
// Modelled time of the split walk, in half-chunks of one walk block.  The walk's n
// blocks of seg_nc chunks take ceil(n / 256) rounds of seg_nc chunks (12.6-13.0 us
// per chunk at 256 blocks, split or not); the adjoint-only pass runs two blocks per
// compute unit, each at about half a walk chunk's time per chunk (203 us for 896
// blocks of 16 chunks).  At config 5's layer shape (96 pairs, 192 chunks) the model
// picks 8 segments of 24 chunks: the backward took 1.66 against 2.76 ms with the
// one-segment walk, and 1.26 against 2.39 ms from the training forward's residuals.
long split_cost(long bh, const BwdRoute& r) {
  const long sub = r.adj_sub(), sub_nc = (r.seg_nc + sub - 1) / sub;
  const long walk_rounds = (bh * r.nseg + kWalkTargetBlocks - 1) / kWalkTargetBlocks;
  const long adj_rounds = (bh * (r.nseg - 1) * sub + 2 * kWalkTargetBlocks - 1) / (2 * kWalkTargetBlocks);
  return 2 * walk_rounds * r.seg_nc + adj_rounds * sub_nc;
}
BwdRoute bwd_route(int B, int H, int L, int CS) {
  const long bh = (long)B * H, nc = (L + CS - 1) / CS;
  // the segment count with the least modelled time (the fewest on ties), or one segment
  auto split = [&](int min_chunks) {
    const long smax = std::min<long>(nc / min_chunks, kWalkMaxRounds * kWalkTargetBlocks / std::max<long>(bh, 1));
    BwdRoute best{true, 1, (int)nc};
    long best_cost = 0;
    for (long s = 2; s <= smax; ++s) {
      const int seg_nc = (int)((nc + s - 1) / s);
      const BwdRoute r{true, (int)((nc + seg_nc - 1) / seg_nc), seg_nc};
      if (r.nseg < 2) continue;
      const long cost = split_cost(bh, r);
      if (best.nseg == 1 || cost < best_cost) {
        best = r;
        best_cost = cost;
      }
    }
    return best;
  };
  const char* e = getenv("M3_BWD_ROUTE");
  if (e && !strcmp(e, "walk")) return {true, 1, (int)nc};
  if (e && !strcmp(e, "chunks")) return {false, 1, (int)nc};
  if (e && !strcmp(e, "segments")) return split(2);
  if (bh >= kWalkTargetBlocks) return {true, 1, (int)nc};
  const BwdRoute r = split(kWalkMinSegChunks);
  if (bh >= kWalkMinBH) {
    // the one-segment walk: ceil(bh / 256) = 1 round of nc chunks (2 nc half-chunks)
    return r.nseg > 1 && 10 * split_cost(bh, r) <= 8 * 2 * nc ? r : BwdRoute{true, 1, (int)nc};
  }
  return r.nseg > 1 ? r : BwdRoute{false, 1, (int)nc};
}
bool bwd_walk(int B, int H, int L, int CS) { return bwd_route(B, H, L, CS).walk; }

// The chunk states and angles the backward reads: computed by its own state-only pass
// (in the workspace), or saved by the training forward (scan_bwd_saved_bytes, in the
// caller's buffer, the same layout).
size_t saved_h_bytes(bool bf16_io, int B, int L, int H, int N, int P) {
  const int CS = bf16_io ? 64 : 32;
  const long nc = (L + CS - 1) / CS;
  return al256((size_t)B * H * nc * P * N * (bf16_io ? 2 : 4));
}
size_t saved_th_bytes(bool bf16_io, int B, int L, int H, int R) {
  const int CS = bf16_io ? 64 : 32;
  const long nc = (L + CS - 1) / CS;
  return al256((size_t)B * H * nc * (R > 0 ? R : 1) * 4);
}

BwdWs bwd_layout(bool bf16_io, int B, int L, int H, int Hqk, int N, int P, int R, bool ang_shared,
                 bool saved = false) {
  const int CS = bf16_io ? 64 : 32;
  const BwdRoute route = bwd_route(B, H, L, CS);
  const bool walk = route.walk;
  const long nc = (L + CS - 1) / CS, bhc = (long)B * H * nc;
  const size_t ts = bf16_io ? 2 : 4;
  BwdWs w;
  size_t off = 0;
  auto take = [&](size_t bytes) { const size_t o = off; off += al256(bytes); return o; };
  w.hs = saved ? 0 : take(bhc * P * N * ts);
  w.gs = walk ? 0 : take(bhc * P * N * ts);     // the walk keeps the adjoint state on chip
  w.th = saved ? 0 : take(bhc * (R > 0 ? R : 1) * 4);
  w.pqb = take(bhc * N * 4);
  w.pkb = take(bhc * N * 4);
  w.pd = take(bhc * 4);
  w.dsc = take((size_t)B * H * L * 4);
  w.ctot = take(bhc * (R + 1) * 4);
  const bool gqa = Hqk < H;
  w.dqh = gqa ? take((size_t)B * L * H * N * ts) : 0;
  w.dkh = gqa ? take((size_t)B * L * H * N * ts) : 0;
  w.dangh = ang_shared && R > 0 ? take((size_t)B * L * H * R * 4) : 0;      // per-head dAngles
  // the split walk: the segments' adjoint states and log-decays
  const size_t bhs = (size_t)B * H * route.nseg, bhsub = bhs * route.adj_sub();
  w.gin = route.nseg > 1 ? take(bhs * P * N * 4) : 0;
  w.gloc = route.nseg > 1 ? take(bhsub * P * N * 4) : 0;
  w.dseg = route.nseg > 1 ? take(bhsub * 4) : 0;
  // the state-only pass split across compute units (few pairs, long sequences)
  const size_t sp = saved ? 0 : scan_split_ws_bytes(bf16_io, B, L, H, N, P, R, 64);
  w.split = sp ? take(sp) : 0;
  w.total = off;
  return w;
}

}  // namespace

// (dtype, kernel chunk, d_state, headdim, rotation width) of the backward
#define M3_BWD_SHAPES(X)                                                                    \
  X(bf16, 64, 128, 64, 32) X(bf16, 64, 128, 64, 64) X(bf16, 64, 128, 64, 0)                 \
  X(bf16, 64, 64, 64, 16) X(bf16, 64, 64, 32, 16) X(float, 32, 128, 64, 32) X(float, 32, 128, 64, 64)           \
  X(float, 32, 64, 64, 16) X(float, 32, 64, 32, 16)

bool scan_bwd_supported(bool bf16_io, int N, int P, int R) {
#define X(T, cs, n, p, r) \
  if ((std::is_same<T, bf16>::value == bf16_io) && N == n && P == p && R == r) return true;
  M3_BWD_SHAPES(X)
#undef X
  return false;
}

size_t scan_bwd_ws_bytes(bool bf16_io, int B, int L, int H, int Hqk, int N, int P, int R, bool ang_shared,
                         bool saved) {
  if (!scan_bwd_supported(bf16_io, N, P, R) || B <= 0 || L <= 0) return 0;
  return bwd_layout(bf16_io, B, L, H, Hqk, N, P, R, ang_shared, saved).total;
}

// The output before the gate (float32 I/O only: at bf16 the forward's extra writes
// cost more than the walk's y tiles, measured).
size_t saved_y_bytes(bool bf16_io, int B, int L, int H, int P) {
  return bf16_io ? 0 : al256((size_t)B * L * H * P * 4);
}

size_t scan_bwd_saved_bytes(bool bf16_io, int B, int L, int H, int N, int P, int R) {
  if (!scan_bwd_supported(bf16_io, N, P, R) || B <= 0 || L <= 0) return 0;
  return saved_h_bytes(bf16_io, B, L, H, N, P) + saved_th_bytes(bf16_io, B, L, H, R) +
         saved_y_bytes(bf16_io, B, L, H, P);
}

void scan_bwd_saved_ptrs(void* saved, bool bf16_io, int B, int L, int H, int N, int P, int R, void** h,
                         float** th, void** yv) {
  char* base = reinterpret_cast<char*>(saved);
  const size_t hb = saved_h_bytes(bf16_io, B, L, H, N, P), tb = saved_th_bytes(bf16_io, B, L, H, R);
  *h = saved;
  *th = R > 0 ? reinterpret_cast<float*>(base + hb) : nullptr;
  *yv = bf16_io ? nullptr : base + hb + tb;
}

// The walk, in its training-pair variant when the forward saved the output before the
// gate (float32 only: a.yv is never set for bf16), split into segments when a.nseg > 1.
template <typename T, int CS, int N, int P, int R, bool SEGW, bool GQA>
void launch_walk_seg(dim3 grid, hipStream_t st, const BwdArgs& a) {
  if constexpr (std::is_same<T, float>::value) {
    if (a.yv) {
      hipLaunchKernelGGL((scan_bwd_walk_kernel<T, CS, N, P, R, true, SEGW, GQA>), grid, dim3(kBwdThreads), 0, st,
                         a);
      return;
    }
  }
  hipLaunchKernelGGL((scan_bwd_walk_kernel<T, CS, N, P, R, false, SEGW, GQA>), grid, dim3(kBwdThreads), 0, st, a);
}
template <typename T, int CS, int N, int P, int R>
void launch_walk(dim3 grid, hipStream_t st, const BwdArgs& a) {
  const bool gqa = a.dqh != nullptr;
  if (a.nseg > 1) {
    if (gqa) launch_walk_seg<T, CS, N, P, R, true, true>(grid, st, a);
    else launch_walk_seg<T, CS, N, P, R, true, false>(grid, st, a);
  } else {
    if (gqa) launch_walk_seg<T, CS, N, P, R, false, true>(grid, st, a);
    else launch_walk_seg<T, CS, N, P, R, false, false>(grid, st, a);
  }
}

hipError_t scan_bwd_launch(const ScanBwd& g, bool bf16_io, void* ws, hipStream_t st, const void* saved) {
  const ScanArgs& s = g.fwd;
  const int CS = bf16_io ? 64 : 32;
  const BwdWs w = bwd_layout(bf16_io, s.B, s.L, s.H, s.Hqk, s.N, s.P, s.R, s.ang_shared != 0, saved != nullptr);
  const BwdRoute route = bwd_route(s.B, s.H, s.L, CS);
  char* base = reinterpret_cast<char*>(ws);
  BwdArgs a;
  a.s = s;
  a.s.CS = CS;
  if (a.s.vz_tok == 0) {
    a.s.vz_tok = (long)s.H * s.P;
    a.s.vz_bat = (long)s.L * s.H * s.P;
  }
  a.dvz_tok = g.dvz_tok ? g.dvz_tok : (long)s.H * s.P;
  a.dvz_bat = g.dvz_tok ? g.dvz_bat : (long)s.L * s.H * s.P;
  a.dout = g.dout;
  a.dq = g.dq; a.dk = g.dk; a.dv = g.dv; a.dz = g.dz;
  a.dadt = g.dadt; a.ddt = g.ddt; a.dtrap = g.dtrap;
  a.dang = w.dangh ? reinterpret_cast<float*>(base + w.dangh) : g.dang;   // per head, then summed
  a.dqb = g.dqb; a.dkb = g.dkb; a.dD = g.dD;
  a.yv = nullptr;
  if (saved) {
    void* sh;
    float* sth;
    void* syv;
    scan_bwd_saved_ptrs(const_cast<void*>(saved), bf16_io, s.B, s.L, s.H, s.N, s.P, s.R, &sh, &sth, &syv);
    a.hs = sh;
    a.th0 = sth;
    // the float32 walk reads the saved output before the gate (the chunk-parallel
    // route and bf16 recompute it)
    if (s.z && !bf16_io && route.walk) a.yv = syv;
  } else {
    a.hs = base + w.hs;
    a.th0 = reinterpret_cast<float*>(base + w.th);
  }
  a.gs = route.walk ? nullptr : base + w.gs;
  a.pqb = reinterpret_cast<float*>(base + w.pqb);
  a.pkb = reinterpret_cast<float*>(base + w.pkb);
  a.pd = reinterpret_cast<float*>(base + w.pd);
  a.dqh = w.dqh ? base + w.dqh : nullptr;
  a.dkh = w.dkh ? base + w.dkh : nullptr;
  a.dsc = reinterpret_cast<float*>(base + w.dsc);
  a.ctot = reinterpret_cast<float*>(base + w.ctot);
  a.nc = (s.L + CS - 1) / CS;
  a.nseg = route.nseg;
  a.seg_nc = route.seg_nc;
  a.adj_sub = route.adj_sub();
  if (route.nseg > 1) {
    a.gin = reinterpret_cast<float*>(base + w.gin);
    a.gloc = reinterpret_cast<float*>(base + w.gloc);
    a.dseg = reinterpret_cast<float*>(base + w.dseg);
  }

  // 1. chunk states and angles (the forward's state-only pass, split across compute
  // units for few pairs and long sequences), unless saved
  hipError_t e = hipSuccess;
  if (!saved) {
    ScanArgs p1 = s;
    p1.CS = CS;
    p1.seg_len = 0; p1.init_per_seg = 0; p1.fin_per_seg = 0;
    p1.init_theta = p1.init_h = p1.init_k = p1.init_v = nullptr;
    p1.fin_theta = p1.fin_h = p1.fin_k = p1.fin_v = nullptr;
    p1.fin_logdec = nullptr;
    p1.chunk_h = base + w.hs;
    p1.chunk_th = s.R > 0 ? reinterpret_cast<float*>(base + w.th) : nullptr;
    e = w.split ? scan_split_state_launch(p1, bf16_io, base + w.split, st) : scan_state_launch(p1, bf16_io, st);
    if (e != hipSuccess) return e;
  }

  const dim3 grid_bh(s.B * s.H), grid_c(a.nc, s.B * s.H);
  bool found = false;
  if (route.walk) {
#define X(T, cs, n, p, r)                                                                                  \
  if (!found && (std::is_same<T, bf16>::value == bf16_io) && s.N == n && s.P == p && s.R == r) {           \
    found = true;                                                                                          \
    if (a.nseg > 1) {                                                                                      \
      /* each later segment's own adjoint, then the adjoint entering every segment */                     \
      hipLaunchKernelGGL((scan_adjoint_kernel<T, cs, n, p, r, true>),                                      \
                         dim3(s.B * s.H, (a.nseg - 1) * a.adj_sub),                                        \
                         dim3(kBwdThreads), 0, st, a);                                                     \
      if ((e = hipGetLastError()) != hipSuccess) return e;                                                 \
      hipLaunchKernelGGL(seg_adjoint_combine_kernel, dim3((s.P * s.N + 255) / 256, s.B * s.H), dim3(256),   \
                         0, st, a);                                                                        \
      if ((e = hipGetLastError()) != hipSuccess) return e;                                                 \
    }                                                                                                      \
    launch_walk<T, cs, n, p, r>(dim3(s.B * s.H, a.nseg), st, a);                                           \
    if ((e = hipGetLastError()) != hipSuccess) return e;                                                   \
    if (a.dqh) {                                                                                           \
      hipLaunchKernelGGL((scan_bwd_gqa_kernel<T>), dim3(2048), dim3(256), 0, st, a);                       \
      if ((e = hipGetLastError()) != hipSuccess) return e;                                                 \
    }                                                                                                      \
  }
    M3_BWD_SHAPES(X)
#undef X
    if (!found) return hipErrorInvalidValue;
    const dim3 grid_hc(s.B * s.H, a.nc);
    if (CS == 64) hipLaunchKernelGGL(scan_bwd_walk_finish_kernel<64>, grid_hc, dim3(256), 0, st, a);
    else hipLaunchKernelGGL(scan_bwd_walk_finish_kernel<32>, grid_hc, dim3(256), 0, st, a);
    if ((e = hipGetLastError()) != hipSuccess) return e;
    if (w.dangh) {
      hipLaunchKernelGGL(scan_bwd_angle_heads_kernel, dim3(2048), dim3(256), 0, st, a, g.dang);
      if ((e = hipGetLastError()) != hipSuccess) return e;
    }
    BwdArgs ar = a;
    ar.nc = a.nseg;                              // one bias/D partial per (b, h, segment)
    hipLaunchKernelGGL(scan_bwd_reduce_kernel, dim3(s.H, (s.N + 15) / 16), dim3(256), 0, st, ar);
    return hipGetLastError();
  }
#define X(T, cs, n, p, r)                                                                                  \
  if (!found && (std::is_same<T, bf16>::value == bf16_io) && s.N == n && s.P == p && s.R == r) {           \
    found = true;                                                                                          \
    hipLaunchKernelGGL((scan_adjoint_kernel<T, cs, n, p, r, false>), grid_bh, dim3(kBwdThreads), 0, st, a); \
    if ((e = hipGetLastError()) != hipSuccess) return e;                                                   \
    hipLaunchKernelGGL((scan_bwd_chunk_kernel<T, cs, n, p, r>), grid_c, dim3(kBwdThreads), 0, st, a);      \
    if ((e = hipGetLastError()) != hipSuccess) return e;                                                   \
    if (a.dqh) {                                                                                           \
      hipLaunchKernelGGL((scan_bwd_gqa_kernel<T>), dim3(2048), dim3(256), 0, st, a);                       \
      if ((e = hipGetLastError()) != hipSuccess) return e;                                                 \
    }                                                                                                      \
  }
  M3_BWD_SHAPES(X)
#undef X
  if (!found) return hipErrorInvalidValue;
  if (CS == 64) hipLaunchKernelGGL(scan_bwd_finish_kernel<64>, grid_c, dim3(64 * kFinWaves), 0, st, a);
  else hipLaunchKernelGGL(scan_bwd_finish_kernel<32>, grid_c, dim3(64 * kFinWaves), 0, st, a);
  if ((e = hipGetLastError()) != hipSuccess) return e;
  if (w.dangh) {
    hipLaunchKernelGGL(scan_bwd_angle_heads_kernel, dim3(2048), dim3(256), 0, st, a, g.dang);
    if ((e = hipGetLastError()) != hipSuccess) return e;
  }
  hipLaunchKernelGGL(scan_bwd_reduce_kernel, dim3(s.H, (s.N + 15) / 16), dim3(256), 0, st, a);
  return hipGetLastError();
}

}  // namespace m3
