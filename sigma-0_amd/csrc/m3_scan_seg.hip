// Sequence split of the chunked prefill for few (batch, head) pairs.
//
// With B·H well below the CU count (config 3: B·H = 32 on 256 CUs) one block per
// (b, h) leaves most of the chip idle.  The recurrence is linear in its carry, so a
// sequence can be cut into S segments that run side by side:
//
//   pass 1  the state-only kernel runs every segment from a zero carry and leaves
//           its exit state h_i^0, rope angle advance Δθ_i and total log-decay ΣA_i,
//           with keys rotated by the segment's own angles (starting from zero).  A segment's last
//           token already carries the trapezoid's cross term with the next token
//           (its key scale reads the next token), so h_i^0 is complete;
//   pass 2  the combine chains the segments, one thread per state element: the state entering segment
//           i+1 is  h' = e^{ΣA_i} h + h_i^0 rot(θ)^T  and  θ' = θ + Δθ_i (mod 2π),
//           where rot(θ) turns the rope pairs (2r, 2r+1) of the state's d_state axis
//           by the entering angles (a rotation by θ + φ is rotation by φ, then θ).
//           Only segment 0 enters with a carry that lacks the cross term (a caller's
//           carry from an earlier prefill): there the first summand is
//           e^{ΣA_0} (h + c v ⊗ k) with c = (1 - sigmoid(trap)) dt of the first
//           token, as the kernel forms its entering state;
//   pass 3  the full kernel runs every segment from its entering carry; the carry
//           of segments 1.. has zero k and v, so the kernel adds no cross term again.
//
// This is the reference's sequence-parallel carry algebra (models/mamba3_seqpar.py:
// 67-110) applied across CUs of one GPU; the extra work is pass 1 (no Q, Y or gate).
#include "m3_scan.h"

namespace m3 {
namespace {

constexpr int kCombineThreads = 256;
constexpr int kTargetBlocks = 256;     // MI355X compute units
constexpr int kMinSegment = 256;       // tokens
constexpr int kMaxRounds = 4;          // rounds of blocks on the chip, at most

// Segment length for a (B, H, L) launch, or 0 for no split.  Segments are whole
// multiples of 128 tokens, so every interior segment ends on a kernel chunk.
// Time model: n blocks of len tokens take ceil(n / kTargetBlocks) rounds of len (one
// block per compute unit), and the state-only pass, which runs every segment but the
// last, half the full pass's time per token.  The segment count with the least
// modelled time is taken (the fewest on ties).  For 96 pairs (config 5's layer) that
// is eight segments, three whole rounds of 256 blocks, rather than two (192 blocks,
// and 96 in the state-only pass): in the 12-layer stack the layer's three launches
// took 375 against 417 us.  The model takes a block's time per chunk as fixed; with
// per-head B/C rows at the same shape, where the chip's memory traffic is larger, the
// full pass gained less (285 against 293 us) and the three launches took 1.5% longer
// (0.459 against 0.452 ms by bench.py).
int seg_len_for(int B, int H, int L) {
  const int bh = B * H;
  if (bh <= 0 || bh * 2 > kTargetBlocks || L < 2 * kMinSegment) return 0;
  const int smax = min(L / kMinSegment, kMaxRounds * kTargetBlocks / bh);
  int best = 0;
  long best_cost = 0;
  for (int s = 2; s <= smax; ++s) {
    const int len = ((L + s - 1) / s + 127) / 128 * 128;
    const long ns = (L + len - 1) / len;
    if (ns < 2) continue;
    const long rounds = (bh * ns + kTargetBlocks - 1) / kTargetBlocks;
    const long so_rounds = (bh * (ns - 1) + kTargetBlocks - 1) / kTargetBlocks;
    const long cost = (2 * rounds + so_rounds) * len;     // in half-token units of one block
    if (best == 0 || cost < best_cost) {
      best = len;
      best_cost = cost;
    }
  }
  return best;
}

struct Carries {
  float* h;   // (BH, S, P, N)
  float* k;   // (BH, S, N)   last rope'd key (pass 1 writes it; the combine does not need it)
  float* v;   // (BH, S, P)
  float* th;  // (BH, S, R)
  float* ld;  // (BH, S)      pass 1: the segment's total log-decay
};

size_t align256(size_t x) { return (x + 255) & ~size_t(255); }

// Carve the workspace: the local carries of pass 1, then the entering carries of pass 3.
size_t carve(char* base, long bhs, int N, int P, int R, Carries* loc, Carries* in) {
  size_t off = 0;
  auto take = [&](size_t n) {
    float* p = base ? reinterpret_cast<float*>(base + off) : nullptr;
    off += align256(n * sizeof(float));
    return p;
  };
  Carries* sets[2] = {loc, in};
  for (int set = 0; set < 2; ++set) {
    Carries* c = sets[set];
    Carries t;
    t.h = take((size_t)bhs * P * N);
    t.k = take((size_t)bhs * N);
    t.v = take((size_t)bhs * P);
    t.th = take((size_t)bhs * (R > 0 ? R : 1));
    t.ld = set == 0 ? take((size_t)bhs) : nullptr;
    if (c) *c = t;
  }
  return off;
}

// Grid (P*N / kCombineThreads, B*H): thread -> state element (p, n) of one (b, h),
// walking the segments in order.  Block x == 0 also writes the small carry parts
// (angles, zero k and v of segments 1..).
__global__ __launch_bounds__(kCombineThreads)
void seg_combine_kernel(ScanArgs a, int nseg, Carries loc, Carries in) {
  const int bh = blockIdx.y, tid = threadIdx.x;
  const int N = a.N, P = a.P, R = a.R;
  const long c0 = (long)bh * nseg;                 // carry slot of segment 0
  const int e = blockIdx.x * kCombineThreads + tid;
  if (blockIdx.x == 0) {
    for (int n = tid; n < N; n += kCombineThreads) {
      in.k[c0 * N + n] = a.init_k ? a.init_k[(long)bh * N + n] : 0.0f;
      for (int i = 1; i < nseg; ++i) in.k[(c0 + i) * N + n] = 0.0f;
    }
    for (int p = tid; p < P; p += kCombineThreads) {
      in.v[c0 * P + p] = a.init_v ? a.init_v[(long)bh * P + p] : 0.0f;
      for (int i = 1; i < nseg; ++i) in.v[(c0 + i) * P + p] = 0.0f;
    }
    for (int r = tid; r < R; r += kCombineThreads) {
      float th = a.init_theta ? a.init_theta[(long)bh * R + r] : 0.0f;
      in.th[c0 * R + r] = th;
      for (int i = 0; i + 1 < nseg; ++i) {
        const float x = th + loc.th[(c0 + i) * R + r];
        th = x - kTwoPi * floorf(x * kInvTwoPi);
        in.th[(c0 + i + 1) * R + r] = th;
      }
    }
  }
  if (e >= P * N) return;
  const int p = e / N, n = e % N, r = n >> 1;
  const bool rope = r < R;
  // segment 0 enters with the caller's carry, or zero; its cross term with the
  // previous token (c = (1 - sigmoid(trap_0)) dt_0) is added here, as the kernel
  // adds it to an entering carry
  float h = a.init_h ? a.init_h[(long)bh * P * N + e] : 0.0f;
  in.h[c0 * P * N + e] = h;
  if (a.init_h) {
    const float dt0 = a.dt[(long)bh * a.L], tr0 = a.trap[(long)bh * a.L];
    h += (1.0f - 1.0f / (1.0f + expf(-tr0))) * dt0 * a.init_v[(long)bh * P + p] * a.init_k[(long)bh * N + n];
  }
  float th = rope && a.init_theta ? a.init_theta[(long)bh * R + r] : 0.0f;
  // a segment's values (the element's rope pair of its exit state, its angle advance
  // and log-decay) are loaded one step ahead of their use, so that the loads overlap
  // the previous step's arithmetic instead of each step waiting for its own
  auto load_seg = [&](int i, float2& hp, float& dth, float& ld) {
    const long ci = c0 + i;
    hp = *reinterpret_cast<const float2*>(loc.h + ci * P * N + p * N + 2 * r);
    dth = rope ? loc.th[ci * R + r] : 0.0f;
    ld = loc.ld[ci];
  };
  float2 nhp = make_float2(0.0f, 0.0f);
  float ndth = 0.0f, nld = 0.0f;
  if (nseg > 1) load_seg(0, nhp, ndth, nld);
  for (int i = 0; i + 1 < nseg; ++i) {
    const float2 hp = nhp;
    const float dth = ndth, ld = nld;
    if (i + 2 < nseg) load_seg(i + 1, nhp, ndth, nld);
    float own = (n & 1) ? hp.y : hp.x;
    if (rope) {                          // segment-local key frame -> entering frame
      float sn, cs;
      sincosf(th, &sn, &cs);
      own = (n & 1) ? hp.x * sn + hp.y * cs : hp.x * cs - hp.y * sn;
      const float x = th + dth;
      th = x - kTwoPi * floorf(x * kInvTwoPi);
    }
    h = expf(ld) * h + own;
    in.h[(c0 + i + 1) * P * N + e] = h;
  }
}

}  // namespace

size_t scan_split_ws_bytes(bool bf16_io, int B, int L, int H, int N, int P, int R, int CS) {
  const int len = seg_len_for(B, H, L);
  // the model's shapes (d_state 128, headdim 64; bf16, and float32, the I/O the
  // model's mamba3_siso_triton call hands over) with a state-only pass; others run
  // one pass
  if (len == 0 || N != 128 || P != 64 || !scan_state_supported(bf16_io, 64, N, P, R) ||
      !scan_chunked_supported(bf16_io, CS, N, P, R))
    return 0;
  const long bhs = (long)B * H * ((L + len - 1) / len);
  return carve(nullptr, bhs, N, P, R, nullptr, nullptr);
}

hipError_t scan_split_launch(const ScanArgs& a, bool bf16_io, void* ws, hipStream_t st) {
  const int len = seg_len_for(a.B, a.H, a.L);
  const int nseg = (a.L + len - 1) / len;
  const long bhs = (long)a.B * a.H * nseg;
  Carries loc, in;
  carve(reinterpret_cast<char*>(ws), bhs, a.N, a.P, a.R, &loc, &in);

  ScanArgs p1 = a;                                   // pass 1: exit carries from a zero carry
  p1.seg_len = len;
  p1.init_theta = p1.init_h = p1.init_k = p1.init_v = nullptr;
  p1.fin_h = loc.h; p1.fin_k = loc.k; p1.fin_v = loc.v; p1.fin_theta = a.R > 0 ? loc.th : nullptr;
  p1.fin_logdec = loc.ld;
  p1.fin_per_seg = 1;
  p1.chunk_h = nullptr;                              // the saved residuals come from pass 3
  p1.chunk_th = nullptr;
  p1.out_v = nullptr;
  p1.CS = 64;                                        // 64-token (bf16) or 32-token (float32) sub-chunks
  p1.so_skip_last = 1;                               // no segment reads the last one's exit carry
  hipError_t e = scan_state_launch(p1, bf16_io, st);
  if (e != hipSuccess) return e;

  ScanArgs p2 = a;                                   // pass 2: entering carries
  p2.seg_len = len;
  hipLaunchKernelGGL(seg_combine_kernel, dim3((a.P * a.N + kCombineThreads - 1) / kCombineThreads, a.B * a.H),
                     dim3(kCombineThreads), 0, st, p2, nseg, loc, in);
  e = hipGetLastError();
  if (e != hipSuccess) return e;

  ScanArgs p3 = a;                                   // pass 3: the scan from the entering carries
  p3.seg_len = len;
  p3.init_h = in.h; p3.init_k = in.k; p3.init_v = in.v; p3.init_theta = a.R > 0 ? in.th : nullptr;
  p3.init_per_seg = 1;
  return scan_chunked_launch(p3, bf16_io, st);
}

hipError_t scan_split_state_launch(const ScanArgs& a, bool bf16_io, void* ws, hipStream_t st) {
  const int len = seg_len_for(a.B, a.H, a.L);
  const int nseg = (a.L + len - 1) / len;
  const long bhs = (long)a.B * a.H * nseg;
  Carries loc, in;
  carve(reinterpret_cast<char*>(ws), bhs, a.N, a.P, a.R, &loc, &in);

  ScanArgs p1 = a;                                   // pass 1: exit carries from a zero carry
  p1.seg_len = len;
  p1.init_theta = p1.init_h = p1.init_k = p1.init_v = nullptr;
  p1.fin_h = loc.h; p1.fin_k = loc.k; p1.fin_v = loc.v; p1.fin_theta = a.R > 0 ? loc.th : nullptr;
  p1.fin_logdec = loc.ld;
  p1.init_per_seg = 0;
  p1.fin_per_seg = 1;
  p1.chunk_h = nullptr;
  p1.chunk_th = nullptr;
  p1.so_skip_last = 1;                               // no segment reads the last one's exit carry
  hipError_t e = scan_state_launch(p1, bf16_io, st);
  if (e != hipSuccess) return e;

  ScanArgs p2 = a;                                   // pass 2: entering carries (none from the caller)
  p2.seg_len = len;
  p2.init_theta = p2.init_h = p2.init_k = p2.init_v = nullptr;
  hipLaunchKernelGGL(seg_combine_kernel, dim3((a.P * a.N + kCombineThreads - 1) / kCombineThreads, a.B * a.H),
                     dim3(kCombineThreads), 0, st, p2, nseg, loc, in);
  e = hipGetLastError();
  if (e != hipSuccess) return e;

  ScanArgs p3 = a;                                   // pass 3: the states entering every chunk
  p3.seg_len = len;
  p3.init_h = in.h; p3.init_k = in.k; p3.init_v = in.v; p3.init_theta = a.R > 0 ? in.th : nullptr;
  p3.init_per_seg = 1;
  p3.fin_theta = p3.fin_h = p3.fin_k = p3.fin_v = nullptr;
  p3.fin_logdec = nullptr;
  p3.fin_per_seg = 0;
  return scan_state_launch(p3, bf16_io, st);
}

}  // namespace m3
