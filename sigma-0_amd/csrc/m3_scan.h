// Internal declarations shared by the prefill kernels and the C ABI.
#pragma once

#include "m3_common.h"

namespace m3 {

// Arguments of one prefill launch.  Layouts (row-major, contiguous):
//   q, k   (B, L, Hqk, N)   io dtype      v, z, out (B, L, H, P) io dtype
//   adt, dt, trap (B, H, L) f32 (trap = pre-sigmoid logits)
//   ang    (B, L, H, R) f32 raw rotation rates
//   qbias, kbias (H, N) f32; D (H,) f32 or null; z may be null (no gate)
// Optional recurrent carry in/out (all four or none), the decode layout:
//   theta (B, H, R), h (B, H, P, N), k (B, H, N), v (B, H, P), all f32.
struct ScanArgs {
  const void* q; const void* k; const void* v;
  const float* adt; const float* dt; const float* trap;
  const float* qbias; const float* kbias; const float* ang; const float* D;
  const void* z; void* out;
  const float* init_theta; const float* init_h; const float* init_k; const float* init_v;
  float* fin_theta; float* fin_h; float* fin_k; float* fin_v;
  int B, L, H, Hqk, N, P, R, CS;
};

bool scan_generic_supported(int N, int P, int R);
hipError_t scan_generic_launch(const ScanArgs& a, bool bf16_io, hipStream_t st);

// Chunked MFMA kernel: returns true when (dtype, CS, N, P, R) has an instantiation.
bool scan_chunked_supported(bool bf16_io, int CS, int N, int P, int R);
hipError_t scan_chunked_launch(const ScanArgs& a, bool bf16_io, hipStream_t st);

// Arguments of one decode step (layouts in m3_decode.hip).
struct DecodeArgs {
  float* theta; float* h; float* kprev; float* vprev;
  const void* x; const void* z; const void* bt; const void* ct;
  const float* adt; const float* dt; const float* trap; const float* ang;
  const float* bbias; const float* cbias; const float* D;
  void* y;
  int B, H, N, P, R;
  int wrapped;        // 1: wrapped angle state (default), 0: legacy_unbounded
  int legacy_double;  // 1: add the explicit QK diagonal a second time
};

bool decode_supported(int N, int P, int R);
hipError_t decode_step_launch(const DecodeArgs& a, bool in_bf16, bool out_bf16, hipStream_t st);

}  // namespace m3
