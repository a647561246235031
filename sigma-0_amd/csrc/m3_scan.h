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
  // Sequence segments (chunked kernel only): with seg_len > 0 the grid's y index
  // is the segment and block (bh, seg) covers tokens [seg * seg_len,
  // min(L, (seg + 1) * seg_len)); seg_len is a multiple of 128.  Carries are one per
  // (b, h) (init used by segment 0, fin written by the last segment) or, with
  // init_per_seg / fin_per_seg, one per (b, h, segment) at index bh * nseg + seg.
  int seg_len = 0, init_per_seg = 0, fin_per_seg = 0;
  // State-only pass: the segment's total log-decay (sum of adt), one float per carry slot.
  float* fin_logdec = nullptr;
  // State-only pass for the backward: the state entering every chunk, [bh][chunk][P][N]
  // in the I/O type, and the rope angle entering every chunk, [bh][chunk][R], in
  // revolutions.
  void* chunk_h = nullptr;
  float* chunk_th = nullptr;
  // Angle rates shared over heads, (B, L, R), instead of (B, L, H, R): the fused
  // front end's layout (Q and K then come with Hqk = 1).
  int ang_shared = 0;
  // Token and batch strides (elements) of V and Z when they are read in place from
  // wider rows (the mixer layer's input projection); 0: the contiguous (B, L, H, P)
  // layout.  Honoured by the chunked kernels and the backward; the output stays
  // contiguous.
  long vz_tok = 0, vz_bat = 0;
  // With chunk_h (the training forward) and Z: the output before the gate, (B, L, H, P)
  // in the I/O type, which the backward multiplies into dZ instead of recomputing it
  // (last, so that the other members keep their kernel-argument offsets).
  void* out_v = nullptr;
  // State-only pass of a sequence split: the last segment's block exits at once (the
  // split reads the exit carries of the other segments only; the last segment's final
  // carry comes from the full pass).
  int so_skip_last = 0;
};

// Block order for launches whose heads share Q/K rows: blocks are handed to the 8
// XCDs round-robin, so block i runs (b, h) = (i % 8) * (G / 8) + i / 8 and the heads
// of one batch row share one XCD's L2.  Identity when nothing is shared.
__device__ __forceinline__ int xcd_bh(int i, int G, int Hqk, int H) {
  return (Hqk < H && G % 8 == 0) ? (i % 8) * (G / 8) + i / 8 : i;
}

bool scan_generic_supported(int N, int P, int R);
hipError_t scan_generic_launch(const ScanArgs& a, bool bf16_io, hipStream_t st);

// Chunked MFMA kernel: returns true when (dtype, CS, N, P, R) has an instantiation.
bool scan_chunked_supported(bool bf16_io, int CS, int N, int P, int R);
hipError_t scan_chunked_launch(const ScanArgs& a, bool bf16_io, hipStream_t st);
// Its float32-I/O kernel (m3_scan_chunked_f32.hip), reached through the two above.
bool scan_chunked_f32_supported(int CS, int N, int P, int R);
hipError_t scan_chunked_f32_launch(const ScanArgs& a, hipStream_t st);
// and its state-only pass (the backward's chunk states at float32, d_state 128)
bool scan_state_f32_supported(int CS, int N, int P, int R);
hipError_t scan_state_f32_launch(const ScanArgs& a, hipStream_t st);

// State-only pass of the chunked kernel (sequence split pass 1, backward chunk states).
bool scan_state_supported(bool bf16_io, int CS, int N, int P, int R);
hipError_t scan_state_launch(const ScanArgs& a, bool bf16_io, hipStream_t st);

// Backward: gradients of every input for a forward call described by fwd.
struct ScanBwd {
  ScanArgs fwd;
  const void* dout;                                    // like V, io dtype
  void* dq; void* dk; void* dv; void* dz;              // io dtype; dz null without Z
  float* dadt; float* ddt; float* dtrap; float* dang;  // like ADT, DT, Trap, Angles
  float* dqb; float* dkb; float* dD;                   // (H, N), (H, N), (H,) or null
  // Token and batch strides (elements) of dV and dZ when they are written into wider
  // rows (the mixer layer's in_proj gradient); 0: the contiguous (B, L, H, P) layout.
  // V and Z are read with fwd.vz_tok / fwd.vz_bat.
  long dvz_tok = 0, dvz_bat = 0;
};
bool scan_bwd_supported(bool bf16_io, int N, int P, int R);
// saved: the chunk states come from the training forward (no state-only pass)
size_t scan_bwd_ws_bytes(bool bf16_io, int B, int L, int H, int Hqk, int N, int P, int R, bool ang_shared,
                         bool saved = false);
// The training forward's residuals: the state entering every chunk of the backward's
// chunking ([bh][chunk][P][N], io type), its rope angle ([bh][chunk][R] f32,
// revolutions) and, for float32 I/O, the output before the gate ((B, L, H, P) f32;
// written when Z is given, else null); bytes, and the three arrays' addresses in a
// buffer of that size.
size_t scan_bwd_saved_bytes(bool bf16_io, int B, int L, int H, int N, int P, int R);
void scan_bwd_saved_ptrs(void* saved, bool bf16_io, int B, int L, int H, int N, int P, int R, void** h,
                         float** th, void** yv);
hipError_t scan_bwd_launch(const ScanBwd& g, bool bf16_io, void* ws, hipStream_t st, const void* saved = nullptr);

// Mamba3 mixer layer: the elementwise work around the scan.
struct LayerPreArgs {
  const void* proj;                        // (B, L, 2HP + 2N + 3H + R), io dtype
  const float* dt_bias; const float* b_scale; const float* c_scale;   // (H,), (N,), (N,)
  void* q; void* k;                        // (B, L, N) io dtype: normalised C and B
  void* v; void* z;                        // (B, L, H, P) io dtype
  float* adt; float* dt; float* trap;      // (B, H, L)
  float* ang;                              // (B, L, R)
  int B, L, H, P, N, R;
  float A_floor, eps;
  int tile, vec;                           // set by layer_pre_launch: tokens per workgroup, 16-byte staging
};
// Largest LDS staging of one token's [B, C, dd_dt, dd_A, trap, angles] plus the norm
// scales that layer_pre supports (bytes).
constexpr int kLayerPreLds = 64 * 1024;
struct LayerPostArgs {
  const void* y; const float* scale; void* out;   // (B, L, D), (D,), (B, L, D)
  int B, L, D;
  float eps;
};
hipError_t layer_pre_launch(LayerPreArgs a, bool bf16_io, hipStream_t st);
size_t layer_pre_lds_bytes(int tile, int seg, int N, size_t es);
hipError_t layer_post_launch(const LayerPostArgs& a, bool bf16_io, hipStream_t st);

// The layer's elementwise backward (m3_layer_bwd.hip).  Partial rows of the parameter
// gradients go to `part` (float32, layer_*_bwd_parts rows: the kernels' partial rows,
// then those of the slice sums), then are summed in order.
constexpr int kLayerPostBwdMaxD = 2048;    // layer_post_bwd: D a multiple of 8, at most this
constexpr int kLayerPreBwdMaxN = 256;      // layer_pre_bwd: d_state at most this
struct LayerPostBwdArgs {
  const void* y; const void* dn; const float* scale;   // (B, L, D) io, (B, L, D) io, (D,)
  void* dy;                                             // (B, L, D) io
  float* part;                                          // (parts, D)
  int B, L, D;
  float eps;
};
struct LayerPreBwdArgs {
  const void* proj;                                     // (B, L, 2HP + 2N + 3H + R) io
  const float* dt_bias; const float* b_scale; const float* c_scale;
  const void* dq; const void* dk;                       // d(normalised C), d(normalised B): (B, L, N) io
  const void* dv; const void* dz;                       // (B, L, H, P) io, or both null: in dproj already
  const float* dadt; const float* ddt; const float* dtrap;   // (B, H, L)
  const float* dang;                                    // (B, L, R)
  void* dproj;                                          // like proj
  float* part;                                          // (parts, 2N + H)
  int B, L, H, P, N, R;
  float A_floor, eps;
};
long layer_post_bwd_parts(int B, int L);
long layer_pre_bwd_parts(int B, int L);
// Partial rows (float32, `rows` of `cols`) summed in a fixed order: kReduceSlices
// slices of the rows side by side into mid (kReduceSlices rows of cols), then the
// slices' sums; column c goes to out0 (c < n0), out1 (c < n0 + n1) or out2.
constexpr int kReduceSlices = 16;
hipError_t reduce_rows(const float* part, long rows, int cols, float* mid, float* out0, int n0, float* out1, int n1,
                       float* out2, hipStream_t st);
hipError_t layer_post_bwd_launch(const LayerPostBwdArgs& a, float* dscale, bool bf16_io, hipStream_t st);
hipError_t layer_pre_bwd_launch(const LayerPreBwdArgs& a, float* d_b_scale, float* d_c_scale, float* d_dt_bias,
                                bool bf16_io, hipStream_t st);

// The backbone block's norm and elementwise kernels (m3_block.hip).  `vec` is set by
// the launchers (16-byte paths).
struct BlockNormArgs {
  const float* x; const float* scale; const float* bias; void* out;   // (rows, D), (D,), (D,), (rows, D)
  long rows; int D;
  float eps;
  int vec;
};
struct BlockEltArgs {
  const void* y; const void* h1; const void* h2; const float* skip; void* out;   // n elements each
  long n;
  int act;   // M3_ACT_*
  int vec;
};
struct BlockActNormArgs {
  const void* y; const void* h1; const void* h2; const float* skip;   // (rows, D)
  float* out;                                                         // (rows, D) float32 or null
  const float* scale; const float* bias; void* ln_out;                // (D,), (D,), (rows, D)
  long rows; int D;
  float eps;
  int act;   // M3_ACT_*
  int vec;
};
hipError_t block_norm_launch(BlockNormArgs a, bool bf16_out, hipStream_t st);
hipError_t block_act_norm_launch(BlockActNormArgs a, bool bf16_io, bool bf16_ln, hipStream_t st);
hipError_t log_softmax_launch(const float* x, float* out, long rows, int V, hipStream_t st);
hipError_t block_elt_launch(BlockEltArgs a, bool gelu_only, bool bf16_io, hipStream_t st);

// Their backward (m3_block.hip).  da: the gradient of the block's output (float32);
// y, h1, h2 as the forward read them; the element kernels write dh2 and dd (the
// gradient of the activation's other factor, or dy for gelu), then dy from the Dense
// layers' input gradient dg.  `vec` is set by the launchers.
struct BlockBwdArgs {
  const float* da; const void* y; const void* h1; const void* h2;   // n elements each
  const void* dg; const void* dd_in;                                // gelu backward's inputs
  void* dh2; void* dd; void* dy;                                    // outputs
  long n;
  int act;   // M3_ACT_*
  int vec;
};
// LayerNorm's backward from its float32 input x (rows, D), scale (D,), the output's
// gradient dn (rows, D, io type) and the residual path's gradient dres (or null):
// dx (rows, D) float32; the scale's and bias's gradients through `part`
// (block_norm_bwd_parts rows of 2 D floats).
constexpr int kBlockNormBwdMaxD = 2048;    // D a multiple of 4, at most this
struct BlockNormBwdArgs {
  const float* x; const float* scale; const void* dn; const float* dres;
  float* dx; float* part;
  long rows; int D;
  float eps;
};
hipError_t block_act_bwd_launch(BlockBwdArgs a, bool bf16_io, hipStream_t st);
hipError_t block_gelu_bwd_launch(BlockBwdArgs a, bool bf16_io, hipStream_t st);
long block_norm_bwd_parts(long rows);
hipError_t block_norm_bwd_launch(const BlockNormBwdArgs& a, float* dscale, float* dbias, bool bf16_io,
                                 hipStream_t st);
// log_softmax with each row's negative log-likelihood at its target: loss[row] =
// logsumexp(z) - z[target] and, in place, z = (softmax(z) - onehot(target)) w.  A
// target outside [0, V) gives a NaN loss and no one-hot term.
hipError_t nll_launch(float* z, const int* targets, float* loss, long rows, int V, float w, hipStream_t st);
hipError_t split3_launch(const float* x, void* a, void* b, void* c, long rows, int K, long ld, hipStream_t st);

// Sequence split across compute units: workspace bytes (0 = no split) and launch.
size_t scan_split_ws_bytes(bool bf16_io, int B, int L, int H, int N, int P, int R, int CS);
hipError_t scan_split_launch(const ScanArgs& a, bool bf16_io, void* ws, hipStream_t st);
// The backward's state-only pass (a.chunk_h / a.chunk_th, no initial carry) split the
// same way: the segments' exit carries, their combine, then every segment's state-only
// pass from its entering carry writes the states entering its chunks.  Workspace:
// scan_split_ws_bytes(bf16_io, B, L, H, N, P, R, 64).
hipError_t scan_split_state_launch(const ScanArgs& a, bool bf16_io, void* ws, hipStream_t st);

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
  // The mixer layer's decode (m3_layer_decode_step): with proj set, x, z, B, C, the
  // per-head dt/A/trap fields and the angle rates come from the token's projection row
  // (batch b's row of 2HP + 2N + 3H + R elements, the layout m3_layer_pre reads), B
  // and C RMS-normalised as m3_layer_pre does; x, z, bt, ct, adt, dt, trap and ang are
  // then unused.
  const void* proj = nullptr;
  const float* dt_bias = nullptr; const float* b_scale = nullptr; const float* c_scale = nullptr;
  float A_floor = 0.0f, eps = 0.0f;
};

bool decode_supported(int N, int P, int R);
hipError_t decode_step_launch(const DecodeArgs& a, bool in_bf16, bool out_bf16, hipStream_t st);

}  // namespace m3
