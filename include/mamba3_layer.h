/*
 * C ABI of the Mamba3 mixer layer's fused elementwise kernels (libmamba3_rocm.so).
 *
 * The layer (Mamba3SSM, src/base_model/models/mamba3.py) is
 *   proj = x @ in_proj                                  (library GEMM)
 *   m3_layer_pre: split, BCNorm, decay, trapezoid, angle rates
 *   m3_layer_scan: the scan, B/C shared over heads, x and z read in place from
 *                  proj (or m3_chunk_scan_fwd_shared of mamba3_scan.h on copies)
 *   m3_layer_post: output RMSNorm
 *   out = m3_layer_post(...) @ out_proj                 (library GEMM)
 * and, generating one token at a time, m3_layer_decode_step in place of
 * m3_layer_pre and the scan;
 * and its backward: m3_layer_post_bwd, m3_layer_scan_bwd (after m3_layer_scan_train,
 * the forward that saves the scan's residuals), m3_layer_pre_bwd, with the GEMMs'
 * gradients between them.
 * Same conventions as mamba3_scan.h: device pointers, io_dtype M3_DTYPE_F32 or
 * M3_DTYPE_BF16, asynchronous on `stream`, 0 or an M3_E* code (m3_last_error).
 */
#ifndef MAMBA3_LAYER_H
#define MAMBA3_LAYER_H

#include "mamba3_scan.h"

#ifdef __cplusplus
extern "C" {
#endif

/*
 * Replaces the JAX operations of Mamba3SSM._preprocess with shared_bc=True
 * (mamba3.py:203-268).  proj (B, L, 2HP + 2N + 3H + R) in io_dtype holds
 * [z, x, B, C, dd_dt, dd_A, trap, angles] per token.  Writes Q = RMSNorm(C)
 * and K = RMSNorm(B) (B, L, N) in io_dtype (statistics in float32, scales
 * C_norm_scale / B_norm_scale (N,), eps), V = x and Z = z (B, L, H, P) in io_dtype
 * (both null: not copied, for m3_layer_scan), DT = softplus(dd_dt + dt_bias),
 * ADT = min(-softplus(dd_A), -A_floor) * DT and Trap = trap as float32 (B, H, L),
 * and the angle rates as float32 (B, L, R).
 */
int m3_layer_pre(const void* proj, const float* dt_bias, const float* B_norm_scale, const float* C_norm_scale,
                 void* Q, void* K, void* V, void* Z, float* ADT, float* DT, float* Trap, float* Angles,
                 int B, int L, int H, int P, int N, int R, float A_floor, float eps, int io_dtype, void* stream);

/*
 * The layer's scan (_forward_pallas, mamba3.py:369-370, 413-425: Q = C and K = B (B, L, N),
 * angle rates (B, L, R)) reading x (V) and z (Z) in place from the projection
 * proj (B, L, d_in_proj), columns [HP, 2HP) and [0, HP), instead of from copies.
 * d_in_proj must be the projection's width 2HP + 2N + 3H + R, the layout m3_layer_pre
 * reads (M3_E_ARG otherwise).
 * Otherwise the arguments and result of m3_chunk_scan_fwd_shared (Out (B, L, H, P)
 * contiguous, the same workspace size from m3_chunk_scan_ws_bytes).  The rows and
 * the offset of x (H*P elements) must be multiples of 16 bytes (M3_E_ALIGN
 * otherwise; bf16: d_in_proj and H*P multiples of 8) and the shape must have a
 * chunked kernel (M3_E_UNSUPPORTED otherwise); the caller then copies x and z with
 * m3_layer_pre and uses m3_chunk_scan_fwd_shared.  The reference's layer slices x
 * and z out of the projection as views before its scan call (mamba3.py:212-219);
 * this entry point is that call without the copies a contiguous C ABI would need.
 */
int m3_layer_scan(const void* Q, const void* K, const void* proj, int d_in_proj,
                  const float* ADT, const float* DT, const float* Trap, const float* Angles,
                  const float* Q_bias, const float* K_bias, const float* D, void* Out,
                  int B, int L, int H, int N, int P, int R, int chunk_size, int io_dtype,
                  void* ws, size_t ws_bytes, void* stream);
/*
 * m3_layer_scan with the recurrent carry of m3_chunk_scan_fwd_carry (mamba3_scan.h):
 * initial (theta, ssm, k, v) in, final out, each all four or none, float32 in the
 * decode layout (theta (B,H,R) radians, ssm (B,H,P,N), k (B,H,N) the last token's
 * biased and rotated key, v (B,H,P) its x).  A prefill whose final carry
 * m3_decode_step continues token by token (Mamba3SSM.__call_rnn__,
 * mamba3.py:466-568), or a prefill in pieces.
 */
int m3_layer_scan_carry(const void* Q, const void* K, const void* proj, int d_in_proj,
                        const float* ADT, const float* DT, const float* Trap, const float* Angles,
                        const float* Q_bias, const float* K_bias, const float* D, void* Out,
                        const float* init_theta, const float* init_ssm, const float* init_k, const float* init_v,
                        float* fin_theta, float* fin_ssm, float* fin_k, float* fin_v,
                        int B, int L, int H, int N, int P, int R, int chunk_size, int io_dtype,
                        void* ws, size_t ws_bytes, void* stream);
/*
 * The layer's decode step (Mamba3SSM.__call_rnn__, mamba3.py:466-568, one token per
 * sequence): m3_layer_pre on the token followed by m3_decode_step, in one launch.
 * proj (B, 2HP + 2N + 3H + R) in io_dtype is the token's projection row, the layout
 * m3_layer_pre reads; B and C are normalised as m3_layer_pre normalises them (scales
 * B_norm_scale / C_norm_scale (N,), eps), dt, A (A_floor) likewise, trap = sigmoid of
 * the row's trap field (the reference's recurrent path applies it), the angle rates
 * shared by the heads.  The carry (theta, ssm, k, v), B_bias / C_bias (H, N), D (H,)
 * or NULL, angle_mode and diag_mode are m3_decode_step's; y (B, H, P) is written in
 * io_dtype (the input of m3_layer_post).  The same shape limits as m3_decode_step.
 */
int m3_layer_decode_step(const void* proj, const float* dt_bias, const float* B_norm_scale,
                         const float* C_norm_scale, const float* B_bias, const float* C_bias, const float* D,
                         float* theta, float* ssm, float* k, float* v, void* y, int B, int H, int P, int N, int R,
                         float A_floor, float eps, int io_dtype, int angle_mode, int diag_mode, void* stream);
/*
 * The layer's training pair with x and z in place: m3_chunk_scan_fwd_train_shared and
 * m3_chunk_scan_bwd_saved_shared of mamba3_scan.h (the fused path's chunk_scan_fwd_rule /
 * chunk_scan_bwd_rule, mamba3_pallas.py:602-645) with V and Z read from proj as
 * m3_layer_scan reads them, and the backward's dV and dZ written into the x and z
 * columns [HP, 2HP) and [0, HP) of d_proj (B, L, d_in_proj, io_dtype), which
 * m3_layer_pre_bwd then completes (called with dV = dZ = NULL).  Same layout
 * conditions and errors as m3_layer_scan, for proj and d_proj alike.
 * m3_layer_scan_train: saved of m3_chunk_scan_saved_bytes, workspace of
 * m3_chunk_scan_ws_bytes.  m3_layer_scan_bwd: with saved, the workspace of
 * m3_chunk_scan_bwd_saved_shared_ws_bytes; with saved = NULL the chunk states are
 * recomputed, workspace of m3_chunk_scan_bwd_shared_ws_bytes.  Z is always present
 * (the layer's gate).
 */
int m3_layer_scan_train(const void* Q, const void* K, const void* proj, int d_in_proj,
                        const float* ADT, const float* DT, const float* Trap, const float* Angles,
                        const float* Q_bias, const float* K_bias, const float* D, void* Out,
                        int B, int L, int H, int N, int P, int R, int chunk_size, int io_dtype,
                        void* saved, size_t saved_bytes, void* ws, size_t ws_bytes, void* stream);
int m3_layer_scan_bwd(const void* Q, const void* K, const void* proj, int d_in_proj,
                      const float* ADT, const float* DT, const float* Trap, const float* Angles,
                      const float* Q_bias, const float* K_bias, const float* D, const void* dOut,
                      void* dQ, void* dK, void* d_proj, float* dADT, float* dDT, float* dTrap,
                      float* dQ_bias, float* dK_bias, float* dAngles, float* dD,
                      int B, int L, int H, int N, int P, int R, int chunk_size, int io_dtype,
                      const void* saved, size_t saved_bytes, void* ws, size_t ws_bytes, void* stream);

/*
 * Replaces the RMSNorm of Mamba3SSM._post_norm_and_project (mamba3.py:281-312,
 * one device): out = (y * rsqrt(mean(y^2) + eps)) * scale over the last axis D,
 * with the reference's rounding (the rsqrt in y's dtype, the product in the
 * out-projection's dtype).  y, out (B, L, D) in io_dtype; scale (D,) float32.
 */
int m3_layer_post(const void* y, const float* scale, void* out, int B, int L, int D, float eps, int io_dtype,
                  void* stream);
/*
 * The layer's backward, the gradients autodiff of _post_norm_and_project and
 * _preprocess (mamba3.py:203-331) gives, in float32 arithmetic, deterministic
 * (parameter gradients summed over the tokens in a fixed order through the
 * workspace of the matching _ws_bytes call).  With the library GEMMs' gradients and
 * m3_chunk_scan_bwd_shared of mamba3_scan.h between them, they give the gradients of
 * x and every parameter of the layer.
 *
 * m3_layer_post's backward: from y (B, L, D) and d_out = dL/d(out) (B, L, D) in
 * io_dtype and scale (D,), dy = dL/dy (B, L, D) in io_dtype and d_scale (D,)
 * float32.  D a multiple of 8, at most 2048 (M3_E_UNSUPPORTED otherwise); y, d_out,
 * dy and ws 16-byte aligned (M3_E_ALIGN otherwise).
 */
size_t m3_layer_post_bwd_ws_bytes(int B, int L, int D);
int m3_layer_post_bwd(const void* y, const void* d_out, const float* scale, void* dy, float* d_scale, int B, int L,
                      int D, float eps, int io_dtype, void* ws, size_t ws_bytes, void* stream);
/*
 * m3_layer_pre's backward (autodiff of Mamba3SSM._preprocess, shared_bc,
 * src/base_model/models/mamba3.py:203-268): from proj and the parameters m3_layer_pre read, and the
 * gradients of its outputs -- dQ and dK of the normalised C and B (B, L, N), dV and
 * dZ (B, L, H, P), all in io_dtype (m3_chunk_scan_bwd_shared's dQ, dK, dV, dZ; dV and dZ
 * both NULL when m3_layer_scan_bwd wrote them into d_proj already), and
 * dADT, dDT, dTrap (B, H, L) and dAngles (B, L, R) float32 -- d_proj like proj (every
 * column written: the gradient of the in_proj output) and d_dt_bias (H,),
 * d_B_norm_scale, d_C_norm_scale (N,) float32.  The A_floor clip passes the gradient
 * where -softplus(dd_A) is below -A_floor and half of it on a tie.  d_state at most
 * 256 (M3_E_UNSUPPORTED otherwise).
 */
size_t m3_layer_pre_bwd_ws_bytes(int B, int L, int H, int N);
int m3_layer_pre_bwd(const void* proj, const float* dt_bias, const float* B_norm_scale, const float* C_norm_scale,
                     const void* dQ, const void* dK, const void* dV, const void* dZ, const float* dADT,
                     const float* dDT, const float* dTrap, const float* dAngles, void* d_proj, float* d_dt_bias,
                     float* d_B_norm_scale, float* d_C_norm_scale, int B, int L, int H, int P, int N, int R,
                     float A_floor, float eps, int io_dtype, void* ws, size_t ws_bytes, void* stream);

/*
 * The backbone block around the mixer: SequenceLayer.__call__
 * (src/base_model/models/layers.py:108-160).  A block on the float32 residual
 * stream x is
 *   prenorm:  y = mixer(m3_block_norm(x) -> compute dtype)
 *   postnorm: y = mixer(x)
 *   gelu:                 x = m3_block_act(y, -, -, skip = x)
 *   full_glu / half_glu*: g = m3_block_gelu(y); h1 = out1(g), h2 = out2(g) (GEMMs);
 *                         x = m3_block_act(y, h1, h2, skip = x)
 *   postnorm: x = m3_block_norm(x) -> float32
 */
#define M3_ACT_GELU 0      /* gelu(y)                    layers.py:139-140 */
#define M3_ACT_FULL_GLU 1  /* h1 * sigmoid(h2)           layers.py:126-129 */
#define M3_ACT_HALF_GLU1 2 /* gelu(y) * sigmoid(h2)      layers.py:130-133 */
#define M3_ACT_HALF_GLU2 3 /* y * sigmoid(h2)            layers.py:134-138 */

/*
 * flax nn.LayerNorm of the block (self.norm, layers.py:121-122 and 150-151): x
 * (B, L, D) float32 -> out (B, L, D) in out_dtype (M3_DTYPE_BF16 for the mixer's
 * input, M3_DTYPE_F32 for the postnorm residual; out may be x then).  Mean and
 * biased variance in float32, (x - mean) * rsqrt(var + eps) * scale + bias, scale
 * and bias (D,) float32.
 */
int m3_block_norm(const float* x, const float* scale, const float* bias, void* out, int B, int L, int D, float eps,
                  int out_dtype, void* stream);

/*
 * nn.gelu (approximate=True, the tanh form) of the mixer output, elementwise in
 * io_dtype: the GLU Dense layers' input (layers.py:127, 131, 136).  out may be x.
 */
int m3_block_gelu(const void* x, void* out, int B, int L, int D, int io_dtype, void* stream);

/*
 * The activation epilogue and the residual add (layers.py:126-148):
 * out = skip + act, float32, with act per `activation` (M3_ACT_*) from the mixer
 * output y and the Dense outputs h1 = out1(gelu(y)) (full_glu only) and
 * h2 = out2(gelu(y)) (all GLU forms), all in io_dtype; the sigmoid and the
 * products are rounded to io_dtype as a layer computing in it rounds them.
 * out may be skip.
 */
int m3_block_act(const void* y, const void* h1, const void* h2, const float* skip, float* out, int B, int L, int D,
                 int activation, int io_dtype, void* stream);

/*
 * m3_block_act followed by a LayerNorm of its result, in one pass over each row:
 * s = skip + act (stored to `out` (float32) when out is not NULL), then
 * ln_out = LayerNorm(s; scale, bias, eps) in ln_dtype.  Two uses:
 *   prenorm:  out = the next residual, ln_out = the next block's normalised mixer
 *             input (its scale and bias, ln_dtype the compute dtype);
 *   postnorm: out = NULL, ln_out = this block's LayerNorm of the sum in float32,
 *             the residual stream itself (layers.py:149-151).
 * ln_out must not alias skip or out; out may be skip.
 */
int m3_block_act_norm(const void* y, const void* h1, const void* h2, const float* skip, float* out,
                      const float* scale, const float* bias, void* ln_out, int B, int L, int D, float eps,
                      int activation, int io_dtype, int ln_dtype, void* stream);

/*
 * The per-token head's nn.log_softmax over the vocabulary, float32
 * (lob_seq_model.py:542): out = x - max - log(sum(exp(x - max))) per row of
 * x (B, L, V).  out may be x.
 */
int m3_log_softmax(const float* x, float* out, int B, int L, int V, void* stream);

/*
 * The backbone's backward around the mixer, as autodiff of SequenceLayer.__call__
 * (layers.py:108-160) and of the head's log_softmax (lob_seq_model.py:530-542) gives
 * it, in float32 arithmetic; the forward's roundings to io_dtype pass gradients
 * unchanged.  The Dense layers' gradients are library GEMMs between these calls.
 *
 * m3_block_act_bwd: from d_out (B, L, D) float32, the gradient of the activation's
 * output (the residual stream's gradient), and y, h1, h2 as m3_block_act read them:
 * with s = sigmoid(h2) rounded to io_dtype, dh2 = d_out u s (1 - s), u = h1
 * (full_glu), gelu(y) rounded (half_glu1) or y (half_glu2), and dd = d_out s, the
 * gradient of that other factor (h1, gelu(y), y); gelu: dd = d_out gelu'(y) is the
 * mixer output's gradient and dh2 is not written.  dh2, dd (B, L, D) in io_dtype.
 *
 * m3_block_gelu_bwd: after the GEMMs that give dg, the gradient of gelu(y) through the
 * Dense layers (full_glu: both): dy = (dg + dd) gelu'(y) (half_glu1), dg gelu'(y)
 * (full_glu, dd unused), dg gelu'(y) + dd (half_glu2).  All (B, L, D) io_dtype.
 *
 * m3_block_norm_bwd: LayerNorm's backward (eps as the forward's) from its float32
 * input x (B, L, D), scale (D,) and the output's gradient d_norm (B, L, D, io_dtype):
 * dx = d_res + the LayerNorm's input gradient (float32; d_res may be NULL), and the
 * scale's and bias's gradients (D,) float32, summed over the tokens in a fixed order
 * through the workspace of m3_block_norm_bwd_ws_bytes.  D a multiple of 4, at most
 * 2048 (M3_E_UNSUPPORTED otherwise); pointers 16-byte aligned (M3_E_ALIGN).
 *
 * m3_log_softmax_nll: per token, loss = logsumexp(z) - z[target] (float32, B*L
 * values) and, in place over the float32 logits z (B, L, V), the gradient of
 * weight * sum(loss): (softmax(z) - onehot(target)) * weight.  targets (B, L) int32;
 * one outside [0, V) gives a NaN loss and no one-hot term.
 */
int m3_block_act_bwd(const float* d_out, const void* y, const void* h1, const void* h2, void* dh2, void* dd, int B,
                     int L, int D, int activation, int io_dtype, void* stream);
int m3_block_gelu_bwd(const void* dg, const void* dd, const void* y, void* dy, int B, int L, int D, int activation,
                      int io_dtype, void* stream);
size_t m3_block_norm_bwd_ws_bytes(int B, int L, int D);
int m3_block_norm_bwd(const float* x, const float* scale, const void* d_norm, const float* d_res, float* dx,
                      float* d_scale, float* d_bias, int B, int L, int D, float eps, int io_dtype, void* ws,
                      size_t ws_bytes, void* stream);
int m3_log_softmax_nll(float* logits, const int* targets, float* loss, int B, int L, int V, float weight,
                       void* stream);

/*
 * No counterpart in the reference: the operands of a float32 product computed as
 * three bf16 products with float32 accumulation (a_hi b_hi + a_hi b_lo + a_lo b_hi,
 * the head's decoder Dense and its gradients in a bf16 model; relative error about
 * 1e-5 against 5e-4 for TF32, which gfx950's matrix cores do not have).  x (rows, K)
 * float32 contiguous; hi = bf16(x) (round to nearest even) is written to hi_a and, when
 * not NULL, to hi_b, and lo = bf16(x - hi) to lo: rows of K elements at row stride ld
 * (ld >= K), so that the three land side by side in one (rows, 3K) operand (ld = 3K,
 * pointers K apart) or stacked in one (3 rows, K) operand (ld = K, pointers rows * K
 * apart).
 */
int m3_split_bf16x3(const float* x, void* hi_a, void* hi_b, void* lo, long rows, int K, long ld, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* MAMBA3_LAYER_H */
