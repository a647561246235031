/*
 * mamba3_scan.h -- C ABI of the MI355X (gfx950) Mamba3 SISO state-scan operator.
 *
 * Plain pointers and sizes only.  Every device pointer is a HIP device
 * address; `stream` is a hipStream_t passed as void* (NULL = default stream).
 * All calls are asynchronous on `stream`, allocate nothing (a split prefill
 * takes a caller-owned workspace, or the library's own scratch array in
 * m3_chunk_scan_fwd_noalloc), keep no per-call state and may be issued
 * concurrently from several host threads (m3_chunk_scan_fwd_noalloc: see there).  Return
 * value: 0 on success, else an M3_E* code; m3_last_error() then describes it
 * (thread-local string).
 *
 * Shapes and layouts (row-major, contiguous) follow the reference call
 * signature mamba3_siso_triton(Q, K, V, ADT, DT, Trap, Q_bias, K_bias, Angles,
 * D, Z, chunk_size) of bold-lab-ai/sigma-0, src/base_model/models/
 * mamba3_ops.py:1116-1127 (batched form :1052-1110):
 *   Q, K    (B, L, Hqk, N)  io dtype, Hqk divides H (head h reads h / (H/Hqk))
 *   V, Z    (B, L, H, P)    io dtype (Z may be NULL: no gate)
 *   ADT, DT, Trap (B, H, L) float32 (Trap = pre-sigmoid logits)
 *   Q_bias, K_bias (H, N)   float32
 *   Angles  (B, L, H, R)    float32 raw rotation rates, 0 <= R <= N/2
 *   D       (H,)            float32 or NULL (no feedthrough)
 *   Out     (B, L, H, P)    io dtype
 */
#ifndef MAMBA3_SCAN_H_
#define MAMBA3_SCAN_H_

#include <stddef.h>

#ifdef __cplusplus
extern "C" {
#endif

#define M3_DTYPE_F32 0
#define M3_DTYPE_BF16 1

#define M3_OK 0
#define M3_E_ARG 1      /* invalid shape, dtype, mode or NULL pointer */
#define M3_E_ALIGN 2    /* a pointer is not 16-byte aligned */
#define M3_E_UNSUPPORTED 3
#define M3_E_LAUNCH 4   /* HIP launch error (message from hipGetErrorString) */

/* Kernel selected by m3_chunk_scan_fwd for a shape. */
#define M3_IMPL_NONE 0
#define M3_IMPL_CHUNKED_MFMA 1
#define M3_IMPL_GENERIC 2

/* ABI version (major * 100 + minor).  No counterpart in the reference (library plumbing). */
int m3_abi_version(void);

/* Message for the last failing call on this host thread ("" if none).  No counterpart in
 * the reference (library plumbing; the reference's FFI raises instead). */
const char* m3_last_error(void);

/* Which prefill kernel serves this shape (M3_IMPL_*), without launching.  No counterpart
 * in the reference (library plumbing). */
int m3_chunk_scan_impl(int io_dtype, int N, int P, int R, int chunk_size);

/*
 * Chunked prefill scan, forward.  Replaces the Triton forward launch of
 * mamba3_siso_triton (src/base_model/models/mamba3_ops.py:158-340, the
 * triton_call at :287-308; batched entry :1052-1110) and the CUDA phases 4-6
 * launch siso_state_scan_launch + reduce_y_off_launch
 * (src/base_model/kernels/mamba3_cuda/ffi/state_scan_ffi.cu:24-38) with one
 * launch covering phases 1-7 of mamba3_ssd_chunked_jax
 * (src/base_model/models/mamba3_jax.py:327-419).  Out = y (B, L, H, P).
 */
int m3_chunk_scan_fwd(const void* Q, const void* K, const void* V,
                      const float* ADT, const float* DT, const float* Trap,
                      const float* Q_bias, const float* K_bias, const float* Angles,
                      const float* D, const void* Z, void* Out,
                      int B, int L, int H, int Hqk, int N, int P, int R,
                      int chunk_size, int io_dtype, void* stream);

/*
 * Prefill with the recurrent carry in and out (prefill -> decode handoff).
 * The carry is the decode layout of Mamba3SSM.__call_rnn__ (mamba3.py:478-483,
 * layers.py:243-256 without the singleton dims), all float32:
 *   theta (B, H, R), ssm (B, H, P, N), k (B, H, N), v (B, H, P).
 * init_* may all be NULL (zero carry); fin_* may all be NULL (not returned).
 * Counterpart of the Triton kernel's HAS_INITIAL_STATES / RETURN_FINAL_STATES
 * paths (src/base_model/kernels/mamba3_triton/siso_fwd.py:76-77, 281-300,
 * 373-378), expressed in the decode carry.
 */
int m3_chunk_scan_fwd_carry(const void* Q, const void* K, const void* V,
                            const float* ADT, const float* DT, const float* Trap,
                            const float* Q_bias, const float* K_bias, const float* Angles,
                            const float* D, const void* Z, void* Out,
                            const float* init_theta, const float* init_ssm,
                            const float* init_k, const float* init_v,
                            float* fin_theta, float* fin_ssm, float* fin_k, float* fin_v,
                            int B, int L, int H, int Hqk, int N, int P, int R,
                            int chunk_size, int io_dtype, void* stream);

/*
 * Device workspace (bytes) that m3_chunk_scan_fwd_ws uses to split each sequence
 * into segments running on separate compute units; 0 when the shape runs as one
 * pass.  The split pays off when B*H is well below the compute-unit count
 * (single-sequence prefill, long context).  Hqk does not matter.  No counterpart in the
 * reference, whose long-context forward passes states in blocks inside its kernel
 * (src/base_model/models/mamba3_pallas.py:679-727).
 */
size_t m3_chunk_scan_ws_bytes(int B, int L, int H, int N, int P, int R, int chunk_size, int io_dtype);

/*
 * m3_chunk_scan_fwd_carry with a caller-owned device workspace of ws_bytes
 * (>= m3_chunk_scan_ws_bytes of the shape, 16-byte aligned).  With ws NULL or a
 * zero requirement it is exactly m3_chunk_scan_fwd_carry.  Otherwise it runs three
 * kernels on `stream`: every segment from a zero carry (state only), a combine of
 * the segments' exit carries into entering carries, and every segment's full scan
 * from its entering carry: the carry algebra of the reference's sequence-parallel
 * path (src/base_model/models/mamba3_seqpar.py:67-110) across the compute units of
 * one GPU.  The workspace is scratch for the call only.
 */
int m3_chunk_scan_fwd_ws(const void* Q, const void* K, const void* V,
                         const float* ADT, const float* DT, const float* Trap,
                         const float* Q_bias, const float* K_bias, const float* Angles,
                         const float* D, const void* Z, void* Out,
                         const float* init_theta, const float* init_ssm,
                         const float* init_k, const float* init_v,
                         float* fin_theta, float* fin_ssm, float* fin_k, float* fin_v,
                         int B, int L, int H, int Hqk, int N, int P, int R,
                         int chunk_size, int io_dtype, void* ws, size_t ws_bytes, void* stream);

/*
 * m3_chunk_scan_fwd_ws without the workspace argument: the split's scratch is a
 * device array of 67 MiB that the library holds for the life of the process, one
 * copy per GPU (its address is looked up on the first call with a stream of that
 * device, NULL meaning the current device; a failed lookup is reported and tried
 * again on the next call; make the first call on each device outside graph capture).  No
 * counterpart in the reference: this entry point is for callers that cannot
 * allocate (code under HIP graph capture, tight serving loops, harnesses that forbid
 * hipMalloc).  It allocates nothing and calls no allocating routine.  Shapes whose
 * split would need more than the 67 MiB (m3_chunk_scan_ws_bytes) are rejected with
 * M3_E_ARG; shapes that run as one pass need no scratch.  Every call on one GPU
 * shares that GPU's array: calls that overlap on one GPU (other streams, other host
 * threads) race and must be serialised by the caller.  Nothing in the array needs
 * to start at zero.
 */
int m3_chunk_scan_fwd_noalloc(const void* Q, const void* K, const void* V,
                              const float* ADT, const float* DT, const float* Trap,
                              const float* Q_bias, const float* K_bias, const float* Angles,
                              const float* D, const void* Z, void* Out,
                              const float* init_theta, const float* init_ssm,
                              const float* init_k, const float* init_v,
                              float* fin_theta, float* fin_ssm, float* fin_k, float* fin_v,
                              int B, int L, int H, int Hqk, int N, int P, int R,
                              int chunk_size, int io_dtype, void* stream);

/*
 * Device workspace (bytes) that m3_chunk_scan_bwd needs for a shape; 0 when the
 * backward has no kernel for (io_dtype, N, P, R).  About 2 * B*H*L*P*N/CS * the
 * element size (the state entering and the adjoint state after each chunk).  The
 * reference's custom_vjp backward (src/base_model/models/mamba3_ops.py:821-902) holds
 * its residuals in XLA buffers instead.
 */
size_t m3_chunk_scan_bwd_ws_bytes(int B, int L, int H, int Hqk, int N, int P, int R, int chunk_size,
                                  int io_dtype);

/*
 * Backward of m3_chunk_scan_fwd: the reference's custom_vjp backward of
 * mamba3_siso_triton (src/base_model/models/mamba3_ops.py:821-902, gradients in
 * the forward's argument order).  Inputs are the forward's inputs and dOut (like
 * V); outputs, written whole:
 *   dQ, dK (B,L,Hqk,N) and dV (B,L,H,P) in io_dtype (with Hqk < H, dQ and dK sum
 *   the value heads that share a Q/K head); dZ like Z (NULL when Z is NULL);
 *   dADT, dDT, dTrap (B,H,L), dAngles (B,L,H,R) float32 (dAngles may be NULL
 *   when R = 0); dQ_bias, dK_bias (H,N) and dD (H,) float32 (dD NULL when D is
 *   NULL), summed over the batch.
 * The chunk size does not change the gradients (the chunked form is exact).  The
 * workspace (>= m3_chunk_scan_bwd_ws_bytes, 16-byte aligned) is scratch for the
 * call.  Q, K, V, Z, Angles, dOut and every io-dtype gradient and dAngles must be
 * 16-byte aligned (M3_E_ALIGN otherwise).  Deterministic: no atomics, fixed
 * summation order.
 */
int m3_chunk_scan_bwd(const void* Q, const void* K, const void* V,
                      const float* ADT, const float* DT, const float* Trap,
                      const float* Q_bias, const float* K_bias, const float* Angles,
                      const float* D, const void* Z, const void* dOut,
                      void* dQ, void* dK, void* dV, float* dADT, float* dDT, float* dTrap,
                      float* dQ_bias, float* dK_bias, float* dAngles, float* dD, void* dZ,
                      int B, int L, int H, int Hqk, int N, int P, int R,
                      int chunk_size, int io_dtype, void* ws, size_t ws_bytes, void* stream);

/*
 * The training pair: the reference's mamba3_siso_fwd, which returns the output and
 * the residuals its backward reads (per-chunk SSM states among them;
 * src/base_model/models/mamba3_ops.py:788-818, siso_fwd_triton's SSM_States
 * :272-285), and mamba3_siso_bwd(saved, grad_output) (:821-902).
 *
 * m3_chunk_scan_saved_bytes: bytes of the residual buffer, the state entering every
 * chunk of the backward's chunking (64 tokens bf16, 32 float32; io dtype), its rope
 * angles (float32) and, for float32 I/O, the output before the gate (B x L x H x P,
 * the reference's Out_v residual; written when Z is given); 0 when the backward has
 * no kernel for the shape.
 *
 * m3_chunk_scan_fwd_train: m3_chunk_scan_fwd_ws that also writes the residuals into
 * `saved` (>= m3_chunk_scan_saved_bytes, 16-byte aligned).  No initial carry (the
 * backward differentiates from a zero state).  chunk_size must be a multiple of the
 * backward's chunk; shapes without a backward return M3_E_UNSUPPORTED.  Out is
 * bitwise that of m3_chunk_scan_fwd_ws.
 *
 * m3_chunk_scan_bwd_saved: m3_chunk_scan_bwd reading the residuals of the
 * m3_chunk_scan_fwd_train call on the same inputs instead of recomputing the chunk
 * states (and, float32 I/O with Z, dZ from the saved output before the gate); its
 * workspace is m3_chunk_scan_bwd_saved_ws_bytes.
 */
size_t m3_chunk_scan_saved_bytes(int B, int L, int H, int N, int P, int R, int io_dtype);
int m3_chunk_scan_fwd_train(const void* Q, const void* K, const void* V,
                            const float* ADT, const float* DT, const float* Trap,
                            const float* Q_bias, const float* K_bias, const float* Angles,
                            const float* D, const void* Z, void* Out,
                            int B, int L, int H, int Hqk, int N, int P, int R,
                            int chunk_size, int io_dtype, void* saved, size_t saved_bytes,
                            void* ws, size_t ws_bytes, void* stream);
size_t m3_chunk_scan_bwd_saved_ws_bytes(int B, int L, int H, int Hqk, int N, int P, int R, int chunk_size,
                                        int io_dtype);
int m3_chunk_scan_bwd_saved(const void* Q, const void* K, const void* V,
                            const float* ADT, const float* DT, const float* Trap,
                            const float* Q_bias, const float* K_bias, const float* Angles,
                            const float* D, const void* Z, const void* dOut,
                            void* dQ, void* dK, void* dV, float* dADT, float* dDT, float* dTrap,
                            float* dQ_bias, float* dK_bias, float* dAngles, float* dD, void* dZ,
                            int B, int L, int H, int Hqk, int N, int P, int R,
                            int chunk_size, int io_dtype, const void* saved, size_t saved_bytes,
                            void* ws, size_t ws_bytes, void* stream);

/*
 * The fused front end's contract: Q, K (B,L,N) and the angle rates (B,L,R) shared
 * over the H heads, the rest per head as in m3_chunk_scan_fwd.  Replaces the
 * reference's mamba3_ssd_chunked_pallas (src/base_model/models/mamba3_pallas.py:
 * 813-849, the model's shared_bc path, mamba3.py:356).  Same result as
 * m3_chunk_scan_fwd with Q, K and the angle rates repeated over heads.  The
 * workspace is as for m3_chunk_scan_fwd_ws (m3_chunk_scan_ws_bytes; NULL runs one
 * pass).  Blocks of heads that share a Q/K row are placed on one XCD so that its
 * L2 serves the sharing.
 */
int m3_chunk_scan_fwd_shared(const void* Q, const void* K, const void* V,
                             const float* ADT, const float* DT, const float* Trap,
                             const float* Q_bias, const float* K_bias, const float* Angles,
                             const float* D, const void* Z, void* Out,
                             int B, int L, int H, int N, int P, int R,
                             int chunk_size, int io_dtype, void* ws, size_t ws_bytes, void* stream);

/*
 * Backward of m3_chunk_scan_fwd_shared (the fused path's custom VJPs,
 * mamba3_pallas.py:292-410): dQ, dK (B,L,N) and dAngles (B,L,R) are summed over
 * heads; the rest as in m3_chunk_scan_bwd.
 */
size_t m3_chunk_scan_bwd_shared_ws_bytes(int B, int L, int H, int N, int P, int R, int chunk_size, int io_dtype);
int m3_chunk_scan_bwd_shared(const void* Q, const void* K, const void* V,
                             const float* ADT, const float* DT, const float* Trap,
                             const float* Q_bias, const float* K_bias, const float* Angles,
                             const float* D, const void* Z, const void* dOut,
                             void* dQ, void* dK, void* dV, float* dADT, float* dDT, float* dTrap,
                             float* dQ_bias, float* dK_bias, float* dAngles, float* dD, void* dZ,
                             int B, int L, int H, int N, int P, int R,
                             int chunk_size, int io_dtype, void* ws, size_t ws_bytes, void* stream);

/*
 * The training pair of the fused path's contract: m3_chunk_scan_fwd_train and
 * m3_chunk_scan_bwd_saved with Q, K (B,L,N) and the angle rates (B,L,R) shared over
 * heads, as m3_chunk_scan_fwd_shared / m3_chunk_scan_bwd_shared take them.  The
 * reference's fused chunk scan saves its residuals, the per-chunk states entering
 * each chunk among them, for its backward (chunk_scan_fwd_rule / chunk_scan_bwd_rule,
 * src/base_model/models/mamba3_pallas.py:602-645).  The residual buffer is
 * m3_chunk_scan_saved_bytes of the shape (per (batch, head), as without sharing);
 * the backward's workspace is m3_chunk_scan_bwd_saved_shared_ws_bytes.
 */
int m3_chunk_scan_fwd_train_shared(const void* Q, const void* K, const void* V,
                                   const float* ADT, const float* DT, const float* Trap,
                                   const float* Q_bias, const float* K_bias, const float* Angles,
                                   const float* D, const void* Z, void* Out,
                                   int B, int L, int H, int N, int P, int R,
                                   int chunk_size, int io_dtype, void* saved, size_t saved_bytes,
                                   void* ws, size_t ws_bytes, void* stream);
size_t m3_chunk_scan_bwd_saved_shared_ws_bytes(int B, int L, int H, int N, int P, int R, int chunk_size,
                                               int io_dtype);
int m3_chunk_scan_bwd_saved_shared(const void* Q, const void* K, const void* V,
                                   const float* ADT, const float* DT, const float* Trap,
                                   const float* Q_bias, const float* K_bias, const float* Angles,
                                   const float* D, const void* Z, const void* dOut,
                                   void* dQ, void* dK, void* dV, float* dADT, float* dDT, float* dTrap,
                                   float* dQ_bias, float* dK_bias, float* dAngles, float* dD, void* dZ,
                                   int B, int L, int H, int N, int P, int R,
                                   int chunk_size, int io_dtype, const void* saved, size_t saved_bytes,
                                   void* ws, size_t ws_bytes, void* stream);

/*
 * One decode step for a batch, in place on the carry.  Replaces the body of
 * rnn_step inside Mamba3SSM.__call_rnn__ (src/base_model/models/mamba3.py:498-562)
 * vmapped over batch (lob_seq_model.py:747-751):
 *   carry (in/out, float32): theta (B,H,R), ssm (B,H,P,N), k (B,H,N), v (B,H,P)
 *   step inputs: x, z (B,H,P) and Bt, Ct (B,H,N) in in_dtype (z may be NULL);
 *                adt, dt, trap (B,H) float32, trap AFTER the sigmoid
 *                (mamba3.py:489); angle (B,H,R) float32 raw rates
 *   B_bias, C_bias (H,N) float32; D (H,) float32 or NULL
 *   y (B,H,P) in out_dtype
 * angle_mode: 1 = "wrapped" (default), 0 = "legacy_unbounded"
 * diag_mode:  0 = "current" (default), 1 = "legacy_double"  (mamba3.py:28-45)
 */
int m3_decode_step(float* theta, float* ssm, float* k, float* v,
                   const void* x, const void* z, const void* Bt, const void* Ct,
                   const float* adt, const float* dt, const float* trap, const float* angle,
                   const float* B_bias, const float* C_bias, const float* D, void* y,
                   int B, int H, int N, int P, int R,
                   int in_dtype, int out_dtype, int angle_mode, int diag_mode, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* MAMBA3_SCAN_H_ */
