// Sequence split of the chunked prefill for few (batch, head) pairs.
//
// With B·H well below the CU count (config 3: B·H = 32 on 256 CUs) one block per
// (b, h) leaves most of the chip idle.  The recurrence is linear in its carry, so a
// sequence can be cut into S segments that run side by side:
//
//   pass 1  the state-only kernel runs every segment from a zero carry and leaves
//           its exit state h_i^0 and rope angle advance Δθ_i, with keys rotated by
//           the segment's own angles (starting from zero).  A segment's last
//           token already carries the trapezoid's cross term with the next token
//           (its key scale reads the next token), so h_i^0 is complete;
//   pass 2  one block per (b, h) chains the segments: the state entering segment
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
constexpr int kMaxRope = 64;           // rope pairs: R <= d_state / 2 <= 64 for the split shapes

// Segment length for a (B, H, L) launch, or 0 for no split.  Segments are whole
// multiples of 128 tokens, so every interior segment ends on a kernel chunk.
int seg_len_for(int B, int H, int L) {
  const int bh = B * H;
  if (bh <= 0 || bh * 2 > kTargetBlocks || L < 2 * kMinSegment) return 0;
  const int s = min((kTargetBlocks + bh - 1) / bh, L / kMinSegment);
  if (s < 2) return 0;
  const int len = ((L + s - 1) / s + 127) / 128 * 128;
  return (L + len - 1) / len >= 2 ? len : 0;
}

struct Carries {
  float* h;   // (BH, S, P, N)
  float* k;   // (BH, S, N)   last rope'd key (pass 1 writes it; the combine does not need it)
  float* v;   // (BH, S, P)
  float* th;  // (BH, S, R)
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
  for (Carries* c : sets) {
    Carries t;
    t.h = take((size_t)bhs * P * N);
    t.k = take((size_t)bhs * N);
    t.v = take((size_t)bhs * P);
    t.th = take((size_t)bhs * (R > 0 ? R : 1));
    if (c) *c = t;
  }
  return off;
}

__global__ __launch_bounds__(kCombineThreads)
void seg_combine_kernel(ScanArgs a, int nseg, Carries loc, Carries in) {
  __shared__ float red[kCombineThreads];
  __shared__ float cs_[kMaxRope], sn_[kMaxRope];
  const int bh = blockIdx.x, tid = threadIdx.x;
  const int N = a.N, P = a.P, R = a.R, L = a.L, len = a.seg_len;
  const long c0 = (long)bh * nseg;                 // carry slot of segment 0
  // segment 0 enters with the caller's carry, or zero
  for (int e = tid; e < P * N; e += kCombineThreads) in.h[c0 * P * N + e] = a.init_h ? a.init_h[(long)bh * P * N + e] : 0.0f;
  for (int n = tid; n < N; n += kCombineThreads) in.k[c0 * N + n] = a.init_k ? a.init_k[(long)bh * N + n] : 0.0f;
  for (int p = tid; p < P; p += kCombineThreads) in.v[c0 * P + p] = a.init_v ? a.init_v[(long)bh * P + p] : 0.0f;
  for (int r = tid; r < R; r += kCombineThreads) in.th[c0 * R + r] = a.init_theta ? a.init_theta[(long)bh * R + r] : 0.0f;
  __syncthreads();
  const float* adt = a.adt + (long)bh * L;
  for (int i = 0; i + 1 < nseg; ++i) {
    const long ci = c0 + i, cn = ci + 1;
    const int t0 = i * len, t1 = min(L, t0 + len);
    // e^{sum of A dt over the segment}
    float sum = 0.0f;
    for (int t = t0 + tid; t < t1; t += kCombineThreads) sum += adt[t];
    red[tid] = sum;
    __syncthreads();
    for (int w = kCombineThreads / 2; w > 0; w >>= 1) {
      if (tid < w) red[tid] += red[tid + w];
      __syncthreads();
    }
    const float dec = expf(red[0]);
    // cross term of the first token with the previous one: only for the caller's
    // carry (segment 0); later carries hold zero k and v
    const float dt0 = a.dt[(long)bh * L + t0], tr0 = a.trap[(long)bh * L + t0];
    const float cross = i == 0 ? (1.0f - 1.0f / (1.0f + expf(-tr0))) * dt0 : 0.0f;
    for (int r = tid; r < R; r += kCombineThreads) sincosf(in.th[ci * R + r], &sn_[r], &cs_[r]);
    __syncthreads();
    const float* lh = loc.h + ci * P * N;
    for (int e = tid; e < P * N; e += kCombineThreads) {
      const int p = e / N, n = e % N, r = n >> 1;
      float own = lh[e];
      if (r < R) {                       // segment-local key frame -> entering frame
        const float h0 = lh[p * N + 2 * r], h1 = lh[p * N + 2 * r + 1];
        own = (n & 1) ? h0 * sn_[r] + h1 * cs_[r] : h0 * cs_[r] - h1 * sn_[r];
      }
      in.h[cn * P * N + e] = dec * (in.h[ci * P * N + e] + cross * in.v[ci * P + p] * in.k[ci * N + n]) + own;
    }
    for (int p = tid; p < P; p += kCombineThreads) in.v[cn * P + p] = 0.0f;
    for (int n = tid; n < N; n += kCombineThreads) in.k[cn * N + n] = 0.0f;
    for (int r = tid; r < R; r += kCombineThreads) {
      const float x = in.th[ci * R + r] + loc.th[ci * R + r];
      in.th[cn * R + r] = x - kTwoPi * floorf(x * kInvTwoPi);
    }
    __syncthreads();
  }
}

}  // namespace

size_t scan_split_ws_bytes(bool bf16_io, int B, int L, int H, int N, int P, int R, int CS) {
  const int len = seg_len_for(B, H, L);
  if (len == 0 || R > kMaxRope || !scan_state_supported(bf16_io, N, P, R) || !scan_chunked_supported(bf16_io, CS, N, P, R))
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
  p1.fin_per_seg = 1;
  hipError_t e = scan_state_launch(p1, st);
  if (e != hipSuccess) return e;

  ScanArgs p2 = a;                                   // pass 2: entering carries
  p2.seg_len = len;
  hipLaunchKernelGGL(seg_combine_kernel, dim3(a.B * a.H), dim3(kCombineThreads), 0, st, p2, nseg, loc, in);
  e = hipGetLastError();
  if (e != hipSuccess) return e;

  ScanArgs p3 = a;                                   // pass 3: the scan from the entering carries
  p3.seg_len = len;
  p3.init_h = in.h; p3.init_k = in.k; p3.init_v = in.v; p3.init_theta = a.R > 0 ? in.th : nullptr;
  p3.init_per_seg = 1;
  return scan_chunked_launch(p3, bf16_io, st);
}

}  // namespace m3
