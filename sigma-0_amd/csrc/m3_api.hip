// C ABI of the Mamba3 scan operator: argument validation and kernel dispatch.
//
// Stateless: nothing is cached between calls (device properties included), so
// concurrent calls from several host threads and devices are safe.  Errors are
// reported through the return code plus a thread-local message, the C
// analogue of the reference handler's ffi::Error::Internal(cudaGetErrorString)
// (src/base_model/kernels/mamba3_cuda/ffi/state_scan_ffi.cu:64-66) and of its
// Python shape asserts (src/base_model/kernels/mamba3_triton/siso_fwd.py:466-482).
#include <stdarg.h>
#include <stdio.h>

#include <mutex>

#include "../../include/mamba3_layer.h"
#include "m3_scan.h"

namespace {

thread_local char g_err[512] = "";

int fail(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof(g_err), fmt, ap);
  va_end(ap);
  return code;
}

bool aligned16(const void* p) { return p == nullptr || (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

int check_launch(hipError_t e, const char* what) {
  if (e != hipSuccess) return fail(M3_E_LAUNCH, "%s: %s", what, hipGetErrorString(e));
  g_err[0] = '\0';
  return M3_OK;
}

int impl_for(int io_dtype, int N, int P, int R, int chunk_size) {
  const bool bf = io_dtype == M3_DTYPE_BF16;
  if (m3::scan_chunked_supported(bf, chunk_size, N, P, R)) return M3_IMPL_CHUNKED_MFMA;
  if (m3::scan_generic_supported(N, P, R)) return M3_IMPL_GENERIC;
  return M3_IMPL_NONE;
}

}  // namespace

namespace m3 {
bool decode_supported(int N, int P, int R) {
  const int rowl = N / 4;
  return N >= 4 && N <= 256 && (N % 4) == 0 && (rowl & (rowl - 1)) == 0 && P >= 1 &&
         P <= 256 && (long)P * N <= 16384 && R >= 0 && 2 * R <= N;
}
}  // namespace m3

extern "C" {

int m3_abi_version(void) { return 107; }

const char* m3_last_error(void) { return g_err; }

int m3_chunk_scan_impl(int io_dtype, int N, int P, int R, int chunk_size) {
  if (io_dtype != M3_DTYPE_F32 && io_dtype != M3_DTYPE_BF16) return M3_IMPL_NONE;
  return impl_for(io_dtype, N, P, R, chunk_size);
}

size_t m3_chunk_scan_ws_bytes(int B, int L, int H, int N, int P, int R, int chunk_size, int io_dtype) {
  if ((io_dtype != M3_DTYPE_F32 && io_dtype != M3_DTYPE_BF16) || B <= 0 || L <= 0 || H <= 0 || chunk_size <= 0)
    return 0;
  return m3::scan_split_ws_bytes(io_dtype == M3_DTYPE_BF16, B, L, H, N, P, R, chunk_size);
}

namespace {
int scan_fwd(const void* Q, const void* K, const void* V,
             const float* ADT, const float* DT, const float* Trap,
             const float* Q_bias, const float* K_bias, const float* Angles,
             const float* D, const void* Z, void* Out,
             const float* init_theta, const float* init_ssm,
             const float* init_k, const float* init_v,
             float* fin_theta, float* fin_ssm, float* fin_k, float* fin_v,
             int B, int L, int H, int Hqk, int N, int P, int R,
             int chunk_size, int io_dtype, void* ws, size_t ws_bytes, void* stream, bool ang_shared,
             long vz_tok = 0, long vz_bat = 0, void* saved = nullptr, size_t saved_bytes = 0) {
  if (io_dtype != M3_DTYPE_F32 && io_dtype != M3_DTYPE_BF16)
    return fail(M3_E_ARG, "io_dtype must be M3_DTYPE_F32 or M3_DTYPE_BF16, got %d", io_dtype);
  if (B < 0 || L < 0 || H <= 0 || Hqk <= 0 || N <= 0 || P <= 0 || R < 0 || chunk_size <= 0)
    return fail(M3_E_ARG, "non-positive dimension (B=%d L=%d H=%d Hqk=%d N=%d P=%d R=%d chunk=%d)",
                B, L, H, Hqk, N, P, R, chunk_size);
  if (H % Hqk != 0) return fail(M3_E_ARG, "nheads (%d) must be divisible by nheads_qk (%d)", H, Hqk);
  if (2 * R > N) return fail(M3_E_ARG, "num rope angles R=%d must be <= d_state/2 = %d", R, N / 2);
  const bool any_init = init_theta || init_ssm || init_k || init_v;
  const bool all_init = init_theta && init_ssm && init_k && init_v;
  const bool any_fin = fin_theta || fin_ssm || fin_k || fin_v;
  const bool all_fin = fin_theta && fin_ssm && fin_k && fin_v;
  if (any_init && !all_init) return fail(M3_E_ARG, "initial carry: pass all of theta, ssm, k, v or none");
  if (any_fin && !all_fin) return fail(M3_E_ARG, "final carry: pass all of theta, ssm, k, v or none");
  if (R > 0 && (init_theta == nullptr) && any_init) return fail(M3_E_ARG, "initial theta missing");
  if (B == 0 || L == 0) {
    g_err[0] = '\0';
    return M3_OK;  // empty batch or sequence: nothing to compute
  }
  if (!Q || !K || !V || !ADT || !DT || !Trap || !Q_bias || !K_bias || !Out || (R > 0 && !Angles))
    return fail(M3_E_ARG, "NULL required pointer");
  const void* vec_ptrs[] = {Q, K, V, Z, Out, Q_bias, K_bias};
  for (const void* p : vec_ptrs)
    if (!aligned16(p)) return fail(M3_E_ALIGN, "Q, K, V, Z, Out and the biases must be 16-byte aligned");
  const int impl = impl_for(io_dtype, N, P, R, chunk_size);
  if (impl == M3_IMPL_NONE)
    return fail(M3_E_UNSUPPORTED, "no kernel for d_state=%d headdim=%d R=%d (generic limits: N even <= 512, "
                "P <= 512, P*N*4 <= 64 KiB)", N, P, R);
  if (impl == M3_IMPL_CHUNKED_MFMA && !aligned16(Angles))
    return fail(M3_E_ALIGN, "Angles must be 16-byte aligned");  // staged as 16-byte rows
  if (vz_tok != 0 && impl != M3_IMPL_CHUNKED_MFMA)
    return fail(M3_E_UNSUPPORTED, "V and Z read in place (token stride %ld) need the chunked kernel", vz_tok);
  m3::ScanArgs a;
  a.q = Q; a.k = K; a.v = V; a.adt = ADT; a.dt = DT; a.trap = Trap;
  a.qbias = Q_bias; a.kbias = K_bias; a.ang = Angles; a.D = D; a.z = Z; a.out = Out;
  a.init_theta = init_theta; a.init_h = init_ssm; a.init_k = init_k; a.init_v = init_v;
  a.fin_theta = fin_theta; a.fin_h = fin_ssm; a.fin_k = fin_k; a.fin_v = fin_v;
  a.B = B; a.L = L; a.H = H; a.Hqk = Hqk; a.N = N; a.P = P; a.R = R; a.CS = chunk_size;
  a.ang_shared = ang_shared ? 1 : 0;
  a.vz_tok = vz_tok; a.vz_bat = vz_bat;
  const bool bf = io_dtype == M3_DTYPE_BF16;
  if (saved) {
    // the training forward: the backward's residuals (chunk states and angles)
    const int kbwd = bf ? 64 : 32;
    if (!m3::scan_bwd_supported(bf, N, P, R) || impl != M3_IMPL_CHUNKED_MFMA)
      return fail(M3_E_UNSUPPORTED, "no backward (saved states) for io_dtype=%d d_state=%d headdim=%d R=%d",
                  io_dtype, N, P, R);
    if (chunk_size % kbwd != 0)
      return fail(M3_E_UNSUPPORTED, "saved states need chunk_size a multiple of %d, got %d", kbwd, chunk_size);
    if (any_init) return fail(M3_E_ARG, "the training forward takes no initial carry");
    const size_t need = m3::scan_bwd_saved_bytes(bf, B, L, H, N, P, R);
    if (saved_bytes < need)
      return fail(M3_E_ARG, "saved-state buffer of %zu bytes, the shape needs %zu (m3_chunk_scan_saved_bytes)",
                  saved_bytes, need);
    if (!aligned16(saved)) return fail(M3_E_ALIGN, "saved-state buffer must be 16-byte aligned");
    void* yv;
    m3::scan_bwd_saved_ptrs(saved, bf, B, L, H, N, P, R, &a.chunk_h, &a.chunk_th, &yv);
    a.out_v = Z ? yv : nullptr;                      // null for bf16 I/O
  }
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  if (impl == M3_IMPL_CHUNKED_MFMA) {
    const size_t need = ws ? m3::scan_split_ws_bytes(bf, B, L, H, N, P, R, chunk_size) : 0;
    if (need > 0) {
      if (ws_bytes < need)
        return fail(M3_E_ARG, "workspace of %zu bytes, the split needs %zu (m3_chunk_scan_ws_bytes)", ws_bytes, need);
      if (!aligned16(ws)) return fail(M3_E_ALIGN, "workspace must be 16-byte aligned");
      return check_launch(m3::scan_split_launch(a, bf, ws, st), "split chunk scan");
    }
    return check_launch(m3::scan_chunked_launch(a, bf, st), "chunk scan");
  }
  return check_launch(m3::scan_generic_launch(a, bf, st), "generic scan");
}
}  // namespace

int m3_chunk_scan_fwd_ws(const void* Q, const void* K, const void* V,
                         const float* ADT, const float* DT, const float* Trap,
                         const float* Q_bias, const float* K_bias, const float* Angles,
                         const float* D, const void* Z, void* Out,
                         const float* init_theta, const float* init_ssm,
                         const float* init_k, const float* init_v,
                         float* fin_theta, float* fin_ssm, float* fin_k, float* fin_v,
                         int B, int L, int H, int Hqk, int N, int P, int R,
                         int chunk_size, int io_dtype, void* ws, size_t ws_bytes, void* stream) {
  return scan_fwd(Q, K, V, ADT, DT, Trap, Q_bias, K_bias, Angles, D, Z, Out, init_theta, init_ssm, init_k, init_v,
                  fin_theta, fin_ssm, fin_k, fin_v, B, L, H, Hqk, N, P, R, chunk_size, io_dtype, ws, ws_bytes, stream,
                  false);
}

int m3_chunk_scan_fwd_shared(const void* Q, const void* K, const void* V,
                             const float* ADT, const float* DT, const float* Trap,
                             const float* Q_bias, const float* K_bias, const float* Angles,
                             const float* D, const void* Z, void* Out,
                             int B, int L, int H, int N, int P, int R,
                             int chunk_size, int io_dtype, void* ws, size_t ws_bytes, void* stream) {
  return scan_fwd(Q, K, V, ADT, DT, Trap, Q_bias, K_bias, Angles, D, Z, Out, nullptr, nullptr, nullptr, nullptr,
                  nullptr, nullptr, nullptr, nullptr, B, L, H, 1, N, P, R, chunk_size, io_dtype, ws, ws_bytes, stream,
                  true);
}

}  // extern "C"

// ---- the allocation-free split prefill (m3_chunk_scan_fwd_noalloc)
// The sequence split's carry workspace lives in a device array that the library
// holds for the process, one copy per GPU, instead of memory from the caller.  Every
// split shape needs at most 1024 (batch, head, segment) carry slots (the split
// launches at most four rounds of 256 blocks), which at d_state 128, headdim 64 and
// R <= 64 is at most 69,208,064 bytes; the array holds 67 MiB.  Nothing in it needs to
// start at zero: the first kernel of a split call writes every carry slot that the
// later ones read.
namespace m3 {
constexpr size_t kNoallocScratchBytes = size_t(67) << 20;
__device__ __align__(256) char scratch[kNoallocScratchBytes];
}  // namespace m3

namespace {
constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices];   // null until a lookup on that device succeeded

// The array's device address on the device that `stream` belongs to (the current
// device for the null stream), looked up with that device current (each GPU holds
// its own copy at its own address).  Only a successful lookup is kept: a failed one
// is reported and tried again on the next call.  The first call on a device looks
// the address up, so it must not be made under stream capture.
int scratch_for_stream(hipStream_t stream, void** ptr) {
  int dev = -1;
  hipError_t e = stream ? hipStreamGetDevice(stream, &dev) : hipGetDevice(&dev);
  if (e != hipSuccess) return fail(M3_E_LAUNCH, "device of the stream: %s", hipGetErrorString(e));
  if (dev < 0 || dev >= kMaxDevices) return fail(M3_E_ARG, "device %d beyond the %d supported", dev, kMaxDevices);
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (g_scratch_ptr[dev] == nullptr) {
    int cur = -1;
    e = hipGetDevice(&cur);
    if (e != hipSuccess) return fail(M3_E_LAUNCH, "hipGetDevice: %s", hipGetErrorString(e));
    if (cur != dev && (e = hipSetDevice(dev)) != hipSuccess)
      return fail(M3_E_LAUNCH, "hipSetDevice(%d): %s", dev, hipGetErrorString(e));
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(m3::scratch));
    if (cur != dev) {
      const hipError_t e2 = hipSetDevice(cur);
      if (e == hipSuccess && e2 != hipSuccess)
        return fail(M3_E_LAUNCH, "hipSetDevice(%d): %s", cur, hipGetErrorString(e2));
    }
    if (e != hipSuccess)
      return fail(M3_E_LAUNCH, "hipGetSymbolAddress(scratch) on device %d: %s", dev, hipGetErrorString(e));
    g_scratch_ptr[dev] = p;
  }
  *ptr = g_scratch_ptr[dev];
  return M3_OK;
}
}  // namespace

extern "C" {

int m3_chunk_scan_fwd_noalloc(const void* Q, const void* K, const void* V,
                              const float* ADT, const float* DT, const float* Trap,
                              const float* Q_bias, const float* K_bias, const float* Angles,
                              const float* D, const void* Z, void* Out,
                              const float* init_theta, const float* init_ssm,
                              const float* init_k, const float* init_v,
                              float* fin_theta, float* fin_ssm, float* fin_k, float* fin_v,
                              int B, int L, int H, int Hqk, int N, int P, int R,
                              int chunk_size, int io_dtype, void* stream) {
  const size_t need = m3_chunk_scan_ws_bytes(B, L, H, N, P, R, chunk_size, io_dtype);
  if (need > m3::kNoallocScratchBytes)
    return fail(M3_E_ARG, "the split needs %zu bytes of scratch, the library holds %zu (m3_chunk_scan_fwd_ws "
                "takes a workspace of any size)", need, m3::kNoallocScratchBytes);
  void* ws = nullptr;
  if (need > 0) {
    const int rc = scratch_for_stream(reinterpret_cast<hipStream_t>(stream), &ws);
    if (rc != M3_OK) return rc;
  }
  return scan_fwd(Q, K, V, ADT, DT, Trap, Q_bias, K_bias, Angles, D, Z, Out, init_theta, init_ssm, init_k, init_v,
                  fin_theta, fin_ssm, fin_k, fin_v, B, L, H, Hqk, N, P, R, chunk_size, io_dtype, ws, need, stream,
                  false);
}

int m3_chunk_scan_fwd_carry(const void* Q, const void* K, const void* V,
                            const float* ADT, const float* DT, const float* Trap,
                            const float* Q_bias, const float* K_bias, const float* Angles,
                            const float* D, const void* Z, void* Out,
                            const float* init_theta, const float* init_ssm,
                            const float* init_k, const float* init_v,
                            float* fin_theta, float* fin_ssm, float* fin_k, float* fin_v,
                            int B, int L, int H, int Hqk, int N, int P, int R,
                            int chunk_size, int io_dtype, void* stream) {
  return m3_chunk_scan_fwd_ws(Q, K, V, ADT, DT, Trap, Q_bias, K_bias, Angles, D, Z, Out, init_theta, init_ssm,
                              init_k, init_v, fin_theta, fin_ssm, fin_k, fin_v, B, L, H, Hqk, N, P, R, chunk_size,
                              io_dtype, nullptr, 0, stream);
}

int m3_chunk_scan_fwd(const void* Q, const void* K, const void* V,
                      const float* ADT, const float* DT, const float* Trap,
                      const float* Q_bias, const float* K_bias, const float* Angles,
                      const float* D, const void* Z, void* Out,
                      int B, int L, int H, int Hqk, int N, int P, int R,
                      int chunk_size, int io_dtype, void* stream) {
  return m3_chunk_scan_fwd_carry(Q, K, V, ADT, DT, Trap, Q_bias, K_bias, Angles, D, Z, Out,
                                 nullptr, nullptr, nullptr, nullptr, nullptr, nullptr, nullptr, nullptr,
                                 B, L, H, Hqk, N, P, R, chunk_size, io_dtype, stream);
}

namespace {
size_t bwd_ws_bytes(int B, int L, int H, int Hqk, int N, int P, int R, int chunk_size, int io_dtype,
                    bool ang_shared) {
  if ((io_dtype != M3_DTYPE_F32 && io_dtype != M3_DTYPE_BF16) || B <= 0 || L <= 0 || H <= 0 || Hqk <= 0 ||
      H % Hqk != 0 || chunk_size <= 0)
    return 0;
  return m3::scan_bwd_ws_bytes(io_dtype == M3_DTYPE_BF16, B, L, H, Hqk, N, P, R, ang_shared);
}

int scan_bwd(const void* Q, const void* K, const void* V,
             const float* ADT, const float* DT, const float* Trap,
             const float* Q_bias, const float* K_bias, const float* Angles,
             const float* D, const void* Z, const void* dOut,
             void* dQ, void* dK, void* dV, float* dADT, float* dDT, float* dTrap,
             float* dQ_bias, float* dK_bias, float* dAngles, float* dD, void* dZ,
             int B, int L, int H, int Hqk, int N, int P, int R,
             int chunk_size, int io_dtype, void* ws, size_t ws_bytes, void* stream, bool ang_shared,
             const void* saved = nullptr, size_t saved_bytes = 0, long vz_tok = 0, long vz_bat = 0,
             long dvz_tok = 0, long dvz_bat = 0) {
  if (io_dtype != M3_DTYPE_F32 && io_dtype != M3_DTYPE_BF16)
    return fail(M3_E_ARG, "io_dtype must be M3_DTYPE_F32 or M3_DTYPE_BF16, got %d", io_dtype);
  if (B < 0 || L < 0 || H <= 0 || Hqk <= 0 || N <= 0 || P <= 0 || R < 0 || chunk_size <= 0)
    return fail(M3_E_ARG, "non-positive dimension (B=%d L=%d H=%d Hqk=%d N=%d P=%d R=%d chunk=%d)",
                B, L, H, Hqk, N, P, R, chunk_size);
  if (H % Hqk != 0) return fail(M3_E_ARG, "nheads (%d) must be divisible by nheads_qk (%d)", H, Hqk);
  if (2 * R > N) return fail(M3_E_ARG, "num rope angles R=%d must be <= d_state/2 = %d", R, N / 2);
  const bool bf = io_dtype == M3_DTYPE_BF16;
  if (!m3::scan_bwd_supported(bf, N, P, R))
    return fail(M3_E_UNSUPPORTED, "no backward kernel for io_dtype=%d d_state=%d headdim=%d R=%d", io_dtype, N, P, R);
  if (B == 0 || L == 0) {
    g_err[0] = '\0';
    return M3_OK;
  }
  if (!Q || !K || !V || !ADT || !DT || !Trap || !Q_bias || !K_bias || (R > 0 && !Angles) || !dOut || !dQ || !dK ||
      !dV || !dADT || !dDT || !dTrap || !dQ_bias || !dK_bias || (R > 0 && !dAngles))
    return fail(M3_E_ARG, "NULL required pointer");
  if ((Z == nullptr) != (dZ == nullptr)) return fail(M3_E_ARG, "pass dZ exactly when Z is given");
  const void* vec_ptrs[] = {Q, K, V, Z, dOut, dQ, dK, dV, dZ, Angles, dAngles};
  for (const void* p : vec_ptrs)
    if (!aligned16(p))
      return fail(M3_E_ALIGN, "Q, K, V, Z, Angles, dOut and their gradients must be 16-byte aligned");
  const size_t need = m3::scan_bwd_ws_bytes(bf, B, L, H, Hqk, N, P, R, ang_shared, saved != nullptr);
  if (ws == nullptr || ws_bytes < need)
    return fail(M3_E_ARG, "workspace of %zu bytes, the backward needs %zu (m3_chunk_scan_bwd%s_ws_bytes)", ws_bytes,
                need, saved ? "_saved" : "");
  if (!aligned16(ws)) return fail(M3_E_ALIGN, "workspace must be 16-byte aligned");
  if (saved) {
    const size_t sneed = m3::scan_bwd_saved_bytes(bf, B, L, H, N, P, R);
    if (saved_bytes < sneed)
      return fail(M3_E_ARG, "saved-state buffer of %zu bytes, the shape needs %zu (m3_chunk_scan_saved_bytes)",
                  saved_bytes, sneed);
    if (!aligned16(saved)) return fail(M3_E_ALIGN, "saved-state buffer must be 16-byte aligned");
  }
  m3::ScanBwd g;
  m3::ScanArgs& a = g.fwd;
  a.q = Q; a.k = K; a.v = V; a.adt = ADT; a.dt = DT; a.trap = Trap;
  a.qbias = Q_bias; a.kbias = K_bias; a.ang = Angles; a.D = D; a.z = Z; a.out = nullptr;
  a.init_theta = a.init_h = a.init_k = a.init_v = nullptr;
  a.fin_theta = a.fin_h = a.fin_k = a.fin_v = nullptr;
  a.B = B; a.L = L; a.H = H; a.Hqk = Hqk; a.N = N; a.P = P; a.R = R; a.CS = chunk_size;
  a.ang_shared = ang_shared ? 1 : 0;
  a.vz_tok = vz_tok; a.vz_bat = vz_bat;
  g.dvz_tok = dvz_tok; g.dvz_bat = dvz_bat;
  g.dout = dOut;
  g.dq = dQ; g.dk = dK; g.dv = dV; g.dz = dZ;
  g.dadt = dADT; g.ddt = dDT; g.dtrap = dTrap; g.dang = dAngles;
  g.dqb = dQ_bias; g.dkb = dK_bias; g.dD = D ? dD : nullptr;
  return check_launch(m3::scan_bwd_launch(g, bf, ws, reinterpret_cast<hipStream_t>(stream), saved), "scan backward");
}
}  // namespace

size_t m3_chunk_scan_saved_bytes(int B, int L, int H, int N, int P, int R, int io_dtype) {
  if ((io_dtype != M3_DTYPE_F32 && io_dtype != M3_DTYPE_BF16) || B <= 0 || L <= 0 || H <= 0) return 0;
  return m3::scan_bwd_saved_bytes(io_dtype == M3_DTYPE_BF16, B, L, H, N, P, R);
}

int m3_chunk_scan_fwd_train(const void* Q, const void* K, const void* V,
                            const float* ADT, const float* DT, const float* Trap,
                            const float* Q_bias, const float* K_bias, const float* Angles,
                            const float* D, const void* Z, void* Out,
                            int B, int L, int H, int Hqk, int N, int P, int R,
                            int chunk_size, int io_dtype, void* saved, size_t saved_bytes,
                            void* ws, size_t ws_bytes, void* stream) {
  if (saved == nullptr) return fail(M3_E_ARG, "NULL saved-state buffer");
  return scan_fwd(Q, K, V, ADT, DT, Trap, Q_bias, K_bias, Angles, D, Z, Out, nullptr, nullptr, nullptr, nullptr,
                  nullptr, nullptr, nullptr, nullptr, B, L, H, Hqk, N, P, R, chunk_size, io_dtype, ws, ws_bytes,
                  stream, false, 0, 0, saved, saved_bytes);
}

size_t m3_chunk_scan_bwd_saved_ws_bytes(int B, int L, int H, int Hqk, int N, int P, int R, int chunk_size,
                                        int io_dtype) {
  if ((io_dtype != M3_DTYPE_F32 && io_dtype != M3_DTYPE_BF16) || B <= 0 || L <= 0 || H <= 0 || Hqk <= 0 ||
      H % Hqk != 0 || chunk_size <= 0)
    return 0;
  return m3::scan_bwd_ws_bytes(io_dtype == M3_DTYPE_BF16, B, L, H, Hqk, N, P, R, false, true);
}

int m3_chunk_scan_bwd_saved(const void* Q, const void* K, const void* V,
                            const float* ADT, const float* DT, const float* Trap,
                            const float* Q_bias, const float* K_bias, const float* Angles,
                            const float* D, const void* Z, const void* dOut,
                            void* dQ, void* dK, void* dV, float* dADT, float* dDT, float* dTrap,
                            float* dQ_bias, float* dK_bias, float* dAngles, float* dD, void* dZ,
                            int B, int L, int H, int Hqk, int N, int P, int R,
                            int chunk_size, int io_dtype, const void* saved, size_t saved_bytes,
                            void* ws, size_t ws_bytes, void* stream) {
  if (saved == nullptr) return fail(M3_E_ARG, "NULL saved-state buffer");
  return scan_bwd(Q, K, V, ADT, DT, Trap, Q_bias, K_bias, Angles, D, Z, dOut, dQ, dK, dV, dADT, dDT, dTrap,
                  dQ_bias, dK_bias, dAngles, dD, dZ, B, L, H, Hqk, N, P, R, chunk_size, io_dtype, ws, ws_bytes,
                  stream, false, saved, saved_bytes);
}

size_t m3_chunk_scan_bwd_ws_bytes(int B, int L, int H, int Hqk, int N, int P, int R, int chunk_size,
                                  int io_dtype) {
  return bwd_ws_bytes(B, L, H, Hqk, N, P, R, chunk_size, io_dtype, false);
}

int m3_chunk_scan_bwd(const void* Q, const void* K, const void* V,
                      const float* ADT, const float* DT, const float* Trap,
                      const float* Q_bias, const float* K_bias, const float* Angles,
                      const float* D, const void* Z, const void* dOut,
                      void* dQ, void* dK, void* dV, float* dADT, float* dDT, float* dTrap,
                      float* dQ_bias, float* dK_bias, float* dAngles, float* dD, void* dZ,
                      int B, int L, int H, int Hqk, int N, int P, int R,
                      int chunk_size, int io_dtype, void* ws, size_t ws_bytes, void* stream) {
  return scan_bwd(Q, K, V, ADT, DT, Trap, Q_bias, K_bias, Angles, D, Z, dOut, dQ, dK, dV, dADT, dDT, dTrap,
                  dQ_bias, dK_bias, dAngles, dD, dZ, B, L, H, Hqk, N, P, R, chunk_size, io_dtype, ws, ws_bytes,
                  stream, false);
}

size_t m3_chunk_scan_bwd_shared_ws_bytes(int B, int L, int H, int N, int P, int R, int chunk_size, int io_dtype) {
  return bwd_ws_bytes(B, L, H, 1, N, P, R, chunk_size, io_dtype, true);
}

int m3_chunk_scan_bwd_shared(const void* Q, const void* K, const void* V,
                             const float* ADT, const float* DT, const float* Trap,
                             const float* Q_bias, const float* K_bias, const float* Angles,
                             const float* D, const void* Z, const void* dOut,
                             void* dQ, void* dK, void* dV, float* dADT, float* dDT, float* dTrap,
                             float* dQ_bias, float* dK_bias, float* dAngles, float* dD, void* dZ,
                             int B, int L, int H, int N, int P, int R,
                             int chunk_size, int io_dtype, void* ws, size_t ws_bytes, void* stream) {
  return scan_bwd(Q, K, V, ADT, DT, Trap, Q_bias, K_bias, Angles, D, Z, dOut, dQ, dK, dV, dADT, dDT, dTrap,
                  dQ_bias, dK_bias, dAngles, dD, dZ, B, L, H, 1, N, P, R, chunk_size, io_dtype, ws, ws_bytes,
                  stream, true);
}

int m3_chunk_scan_fwd_train_shared(const void* Q, const void* K, const void* V,
                                   const float* ADT, const float* DT, const float* Trap,
                                   const float* Q_bias, const float* K_bias, const float* Angles,
                                   const float* D, const void* Z, void* Out,
                                   int B, int L, int H, int N, int P, int R,
                                   int chunk_size, int io_dtype, void* saved, size_t saved_bytes,
                                   void* ws, size_t ws_bytes, void* stream) {
  if (saved == nullptr) return fail(M3_E_ARG, "NULL saved-state buffer");
  return scan_fwd(Q, K, V, ADT, DT, Trap, Q_bias, K_bias, Angles, D, Z, Out, nullptr, nullptr, nullptr, nullptr,
                  nullptr, nullptr, nullptr, nullptr, B, L, H, 1, N, P, R, chunk_size, io_dtype, ws, ws_bytes,
                  stream, true, 0, 0, saved, saved_bytes);
}

size_t m3_chunk_scan_bwd_saved_shared_ws_bytes(int B, int L, int H, int N, int P, int R, int chunk_size,
                                               int io_dtype) {
  if ((io_dtype != M3_DTYPE_F32 && io_dtype != M3_DTYPE_BF16) || B <= 0 || L <= 0 || H <= 0 || chunk_size <= 0)
    return 0;
  return m3::scan_bwd_ws_bytes(io_dtype == M3_DTYPE_BF16, B, L, H, 1, N, P, R, true, true);
}

int m3_chunk_scan_bwd_saved_shared(const void* Q, const void* K, const void* V,
                                   const float* ADT, const float* DT, const float* Trap,
                                   const float* Q_bias, const float* K_bias, const float* Angles,
                                   const float* D, const void* Z, const void* dOut,
                                   void* dQ, void* dK, void* dV, float* dADT, float* dDT, float* dTrap,
                                   float* dQ_bias, float* dK_bias, float* dAngles, float* dD, void* dZ,
                                   int B, int L, int H, int N, int P, int R,
                                   int chunk_size, int io_dtype, const void* saved, size_t saved_bytes,
                                   void* ws, size_t ws_bytes, void* stream) {
  if (saved == nullptr) return fail(M3_E_ARG, "NULL saved-state buffer");
  return scan_bwd(Q, K, V, ADT, DT, Trap, Q_bias, K_bias, Angles, D, Z, dOut, dQ, dK, dV, dADT, dDT, dTrap,
                  dQ_bias, dK_bias, dAngles, dD, dZ, B, L, H, 1, N, P, R, chunk_size, io_dtype, ws, ws_bytes,
                  stream, true, saved, saved_bytes);
}

int m3_decode_step(float* theta, float* ssm, float* k, float* v,
                   const void* x, const void* z, const void* Bt, const void* Ct,
                   const float* adt, const float* dt, const float* trap, const float* angle,
                   const float* B_bias, const float* C_bias, const float* D, void* y,
                   int B, int H, int N, int P, int R,
                   int in_dtype, int out_dtype, int angle_mode, int diag_mode, void* stream) {
  if ((in_dtype != M3_DTYPE_F32 && in_dtype != M3_DTYPE_BF16) ||
      (out_dtype != M3_DTYPE_F32 && out_dtype != M3_DTYPE_BF16))
    return fail(M3_E_ARG, "dtype must be M3_DTYPE_F32 or M3_DTYPE_BF16 (in=%d out=%d)", in_dtype, out_dtype);
  if (angle_mode != 0 && angle_mode != 1)
    return fail(M3_E_ARG, "angle_mode must be 1 (wrapped) or 0 (legacy_unbounded), got %d", angle_mode);
  if (diag_mode != 0 && diag_mode != 1)
    return fail(M3_E_ARG, "diag_mode must be 0 (current) or 1 (legacy_double), got %d", diag_mode);
  if (B < 0 || H <= 0 || N <= 0 || P <= 0 || R < 0)
    return fail(M3_E_ARG, "non-positive dimension (B=%d H=%d N=%d P=%d R=%d)", B, H, N, P, R);
  if (2 * R > N) return fail(M3_E_ARG, "num rope angles R=%d must be <= d_state/2 = %d", R, N / 2);
  if (!m3::decode_supported(N, P, R))
    return fail(M3_E_UNSUPPORTED, "decode needs d_state a multiple of 4 with d_state/4 a power of two "
                "<= 64, headdim <= 256 and headdim*d_state <= 16384 (got N=%d P=%d)", N, P);
  if (B == 0) {
    g_err[0] = '\0';
    return M3_OK;
  }
  if (!theta && R > 0) return fail(M3_E_ARG, "NULL angle state");
  if (!ssm || !k || !v || !x || !Bt || !Ct || !adt || !dt || !trap || !B_bias || !C_bias || !y ||
      (R > 0 && !angle))
    return fail(M3_E_ARG, "NULL required pointer");
  if (!aligned16(ssm)) return fail(M3_E_ALIGN, "ssm state must be 16-byte aligned");
  m3::DecodeArgs a;
  a.theta = theta; a.h = ssm; a.kprev = k; a.vprev = v;
  a.x = x; a.z = z; a.bt = Bt; a.ct = Ct; a.adt = adt; a.dt = dt; a.trap = trap; a.ang = angle;
  a.bbias = B_bias; a.cbias = C_bias; a.D = D; a.y = y;
  a.B = B; a.H = H; a.N = N; a.P = P; a.R = R;
  a.wrapped = angle_mode; a.legacy_double = diag_mode;
  return check_launch(m3::decode_step_launch(a, in_dtype == M3_DTYPE_BF16, out_dtype == M3_DTYPE_BF16,
                                             reinterpret_cast<hipStream_t>(stream)),
                      "decode step");
}

}  // extern "C"

extern "C" {

int m3_layer_pre(const void* proj, const float* dt_bias, const float* B_norm_scale, const float* C_norm_scale,
                 void* Q, void* K, void* V, void* Z, float* ADT, float* DT, float* Trap, float* Angles,
                 int B, int L, int H, int P, int N, int R, float A_floor, float eps, int io_dtype, void* stream) {
  if (io_dtype != M3_DTYPE_F32 && io_dtype != M3_DTYPE_BF16)
    return fail(M3_E_ARG, "io_dtype must be M3_DTYPE_F32 or M3_DTYPE_BF16, got %d", io_dtype);
  if (B < 0 || L < 0 || H <= 0 || P <= 0 || N <= 0 || R < 0)
    return fail(M3_E_ARG, "non-positive dimension (B=%d L=%d H=%d P=%d N=%d R=%d)", B, L, H, P, N, R);
  if (B == 0 || L == 0) {
    g_err[0] = '\0';
    return M3_OK;
  }
  if (!proj || !dt_bias || !B_norm_scale || !C_norm_scale || !Q || !K || !ADT || !DT || !Trap ||
      (R > 0 && !Angles))
    return fail(M3_E_ARG, "NULL required pointer");
  if ((V == nullptr) != (Z == nullptr)) return fail(M3_E_ARG, "V and Z: pass both or neither");
  const size_t es = io_dtype == M3_DTYPE_BF16 ? 2 : 4;
  if (m3::layer_pre_lds_bytes(1, 2 * N + 3 * H + R, N, es) > (size_t)m3::kLayerPreLds)
    return fail(M3_E_UNSUPPORTED, "one token's B, C, per-head and angle fields (%zu bytes) exceed the %d-byte staging",
                (size_t)(2 * N + 3 * H + R) * es, m3::kLayerPreLds);
  m3::LayerPreArgs a{};
  a.proj = proj; a.dt_bias = dt_bias; a.b_scale = B_norm_scale; a.c_scale = C_norm_scale;
  a.q = Q; a.k = K; a.v = V; a.z = Z; a.adt = ADT; a.dt = DT; a.trap = Trap; a.ang = Angles;
  a.B = B; a.L = L; a.H = H; a.P = P; a.N = N; a.R = R; a.A_floor = A_floor; a.eps = eps;
  return check_launch(m3::layer_pre_launch(a, io_dtype == M3_DTYPE_BF16, reinterpret_cast<hipStream_t>(stream)),
                      "layer pre");
}

int m3_layer_decode_step(const void* proj, const float* dt_bias, const float* B_norm_scale,
                         const float* C_norm_scale, const float* B_bias, const float* C_bias, const float* D,
                         float* theta, float* ssm, float* k, float* v, void* y, int B, int H, int P, int N, int R,
                         float A_floor, float eps, int io_dtype, int angle_mode, int diag_mode, void* stream) {
  if (io_dtype != M3_DTYPE_F32 && io_dtype != M3_DTYPE_BF16)
    return fail(M3_E_ARG, "io_dtype must be M3_DTYPE_F32 or M3_DTYPE_BF16, got %d", io_dtype);
  if (angle_mode != 0 && angle_mode != 1)
    return fail(M3_E_ARG, "angle_mode must be 1 (wrapped) or 0 (legacy_unbounded), got %d", angle_mode);
  if (diag_mode != 0 && diag_mode != 1)
    return fail(M3_E_ARG, "diag_mode must be 0 (current) or 1 (legacy_double), got %d", diag_mode);
  if (B < 0 || H <= 0 || N <= 0 || P <= 0 || R < 0)
    return fail(M3_E_ARG, "non-positive dimension (B=%d H=%d N=%d P=%d R=%d)", B, H, N, P, R);
  if (2 * R > N) return fail(M3_E_ARG, "num rope angles R=%d must be <= d_state/2 = %d", R, N / 2);
  if (!m3::decode_supported(N, P, R))
    return fail(M3_E_UNSUPPORTED, "decode needs d_state a multiple of 4 with d_state/4 a power of two "
                "<= 64, headdim <= 256 and headdim*d_state <= 16384 (got N=%d P=%d)", N, P);
  if (B == 0) {
    g_err[0] = '\0';
    return M3_OK;
  }
  if (!proj || !dt_bias || !B_norm_scale || !C_norm_scale || !B_bias || !C_bias || !ssm || !k || !v || !y ||
      (R > 0 && !theta))
    return fail(M3_E_ARG, "NULL required pointer");
  if (!aligned16(ssm)) return fail(M3_E_ALIGN, "ssm state must be 16-byte aligned");
  m3::DecodeArgs a{};
  a.theta = theta; a.h = ssm; a.kprev = k; a.vprev = v;
  a.bbias = B_bias; a.cbias = C_bias; a.D = D; a.y = y;
  a.B = B; a.H = H; a.N = N; a.P = P; a.R = R;
  a.wrapped = angle_mode; a.legacy_double = diag_mode;
  a.proj = proj; a.dt_bias = dt_bias; a.b_scale = B_norm_scale; a.c_scale = C_norm_scale;
  a.A_floor = A_floor; a.eps = eps;
  const bool bf = io_dtype == M3_DTYPE_BF16;
  return check_launch(m3::decode_step_launch(a, bf, bf, reinterpret_cast<hipStream_t>(stream)), "layer decode step");
}

}  // extern "C"

namespace {
// The in-place layout of the layer's scan entry points: projection rows exactly
// 2HP + 2N + 3H + R wide (the layout m3_layer_pre reads) and a multiple of 16 bytes;
// z in columns [0, HP) and x in [HP, 2HP).  On success *pz, *px point at row 0's z and
// x of `base` (proj, or d_proj for the gradients).
int layer_rows(const void* base, int d_in_proj, int H, int N, int P, int R, int io_dtype, const char** pz,
               const char** px) {
  if (io_dtype != M3_DTYPE_F32 && io_dtype != M3_DTYPE_BF16)
    return fail(M3_E_ARG, "io_dtype must be M3_DTYPE_F32 or M3_DTYPE_BF16, got %d", io_dtype);
  if (H <= 0 || P <= 0 || N <= 0 || R < 0)
    return fail(M3_E_ARG, "non-positive dimension (H=%d N=%d P=%d R=%d)", H, N, P, R);
  if ((long)d_in_proj != 2L * H * P + 2L * N + 3L * H + R)
    return fail(M3_E_ARG, "d_in_proj=%d is not the projection's width (2HP + 2N + 3H + R = %ld)", d_in_proj,
                2L * H * P + 2L * N + 3L * H + R);
  const long es = io_dtype == M3_DTYPE_BF16 ? 2 : 4;
  if (((long)d_in_proj * es) % 16 != 0)
    return fail(M3_E_ALIGN, "projection rows of %ld bytes: the in-place read of x and z needs a multiple of 16",
                (long)d_in_proj * es);
  if (!base) return fail(M3_E_ARG, "NULL required pointer");
  *pz = reinterpret_cast<const char*>(base);
  *px = *pz + (long)H * P * es;
  return M3_OK;
}
}  // namespace

extern "C" {

int m3_layer_scan(const void* Q, const void* K, const void* proj, int d_in_proj,
                  const float* ADT, const float* DT, const float* Trap, const float* Angles,
                  const float* Q_bias, const float* K_bias, const float* D, void* Out,
                  int B, int L, int H, int N, int P, int R, int chunk_size, int io_dtype,
                  void* ws, size_t ws_bytes, void* stream) {
  const char *pz, *pv;
  const int rc = layer_rows(proj, d_in_proj, H, N, P, R, io_dtype, &pz, &pv);
  if (rc != M3_OK) return rc;
  return scan_fwd(Q, K, pv, ADT, DT, Trap, Q_bias, K_bias, Angles, D, pz, Out, nullptr, nullptr, nullptr, nullptr,
                  nullptr, nullptr, nullptr, nullptr, B, L, H, 1, N, P, R, chunk_size, io_dtype, ws, ws_bytes, stream,
                  true, d_in_proj, (long)L * d_in_proj);
}

int m3_layer_scan_carry(const void* Q, const void* K, const void* proj, int d_in_proj,
                        const float* ADT, const float* DT, const float* Trap, const float* Angles,
                        const float* Q_bias, const float* K_bias, const float* D, void* Out,
                        const float* init_theta, const float* init_ssm, const float* init_k, const float* init_v,
                        float* fin_theta, float* fin_ssm, float* fin_k, float* fin_v,
                        int B, int L, int H, int N, int P, int R, int chunk_size, int io_dtype,
                        void* ws, size_t ws_bytes, void* stream) {
  const char *pz, *pv;
  const int rc = layer_rows(proj, d_in_proj, H, N, P, R, io_dtype, &pz, &pv);
  if (rc != M3_OK) return rc;
  return scan_fwd(Q, K, pv, ADT, DT, Trap, Q_bias, K_bias, Angles, D, pz, Out, init_theta, init_ssm, init_k, init_v,
                  fin_theta, fin_ssm, fin_k, fin_v, B, L, H, 1, N, P, R, chunk_size, io_dtype, ws, ws_bytes, stream,
                  true, d_in_proj, (long)L * d_in_proj);
}

int m3_layer_scan_train(const void* Q, const void* K, const void* proj, int d_in_proj,
                        const float* ADT, const float* DT, const float* Trap, const float* Angles,
                        const float* Q_bias, const float* K_bias, const float* D, void* Out,
                        int B, int L, int H, int N, int P, int R, int chunk_size, int io_dtype,
                        void* saved, size_t saved_bytes, void* ws, size_t ws_bytes, void* stream) {
  const char *pz, *pv;
  const int rc = layer_rows(proj, d_in_proj, H, N, P, R, io_dtype, &pz, &pv);
  if (rc != M3_OK) return rc;
  if (saved == nullptr) return fail(M3_E_ARG, "NULL saved-state buffer");
  return scan_fwd(Q, K, pv, ADT, DT, Trap, Q_bias, K_bias, Angles, D, pz, Out, nullptr, nullptr, nullptr, nullptr,
                  nullptr, nullptr, nullptr, nullptr, B, L, H, 1, N, P, R, chunk_size, io_dtype, ws, ws_bytes, stream,
                  true, d_in_proj, (long)L * d_in_proj, saved, saved_bytes);
}

int m3_layer_scan_bwd(const void* Q, const void* K, const void* proj, int d_in_proj,
                      const float* ADT, const float* DT, const float* Trap, const float* Angles,
                      const float* Q_bias, const float* K_bias, const float* D, const void* dOut,
                      void* dQ, void* dK, void* d_proj, float* dADT, float* dDT, float* dTrap,
                      float* dQ_bias, float* dK_bias, float* dAngles, float* dD,
                      int B, int L, int H, int N, int P, int R, int chunk_size, int io_dtype,
                      const void* saved, size_t saved_bytes, void* ws, size_t ws_bytes, void* stream) {
  const char *pz, *pv, *gz, *gv;
  int rc = layer_rows(proj, d_in_proj, H, N, P, R, io_dtype, &pz, &pv);
  if (rc != M3_OK) return rc;
  if ((rc = layer_rows(d_proj, d_in_proj, H, N, P, R, io_dtype, &gz, &gv)) != M3_OK) return rc;
  const long tok = d_in_proj, bat = (long)L * d_in_proj;
  return scan_bwd(Q, K, pv, ADT, DT, Trap, Q_bias, K_bias, Angles, D, pz, dOut, dQ, dK, const_cast<char*>(gv),
                  dADT, dDT, dTrap, dQ_bias, dK_bias, dAngles, dD, const_cast<char*>(gz), B, L, H, 1, N, P, R,
                  chunk_size, io_dtype, ws, ws_bytes, stream, true, saved, saved_bytes, tok, bat, tok, bat);
}

int m3_layer_post(const void* y, const float* scale, void* out, int B, int L, int D, float eps, int io_dtype,
                  void* stream) {
  if (io_dtype != M3_DTYPE_F32 && io_dtype != M3_DTYPE_BF16)
    return fail(M3_E_ARG, "io_dtype must be M3_DTYPE_F32 or M3_DTYPE_BF16, got %d", io_dtype);
  if (B < 0 || L < 0 || D <= 0) return fail(M3_E_ARG, "non-positive dimension (B=%d L=%d D=%d)", B, L, D);
  if (B == 0 || L == 0) {
    g_err[0] = '\0';
    return M3_OK;
  }
  if (!y || !scale || !out) return fail(M3_E_ARG, "NULL required pointer");
  m3::LayerPostArgs a;
  a.y = y; a.scale = scale; a.out = out; a.B = B; a.L = L; a.D = D; a.eps = eps;
  return check_launch(m3::layer_post_launch(a, io_dtype == M3_DTYPE_BF16, reinterpret_cast<hipStream_t>(stream)),
                      "layer post");
}

size_t m3_layer_post_bwd_ws_bytes(int B, int L, int D) {
  if (B <= 0 || L <= 0 || D <= 0) return 0;
  return (size_t)m3::layer_post_bwd_parts(B, L) * D * sizeof(float);
}

int m3_layer_post_bwd(const void* y, const void* d_out, const float* scale, void* dy, float* d_scale, int B, int L,
                      int D, float eps, int io_dtype, void* ws, size_t ws_bytes, void* stream) {
  if (io_dtype != M3_DTYPE_F32 && io_dtype != M3_DTYPE_BF16)
    return fail(M3_E_ARG, "io_dtype must be M3_DTYPE_F32 or M3_DTYPE_BF16, got %d", io_dtype);
  if (B < 0 || L < 0 || D <= 0) return fail(M3_E_ARG, "non-positive dimension (B=%d L=%d D=%d)", B, L, D);
  if (D % 8 != 0 || D > m3::kLayerPostBwdMaxD)
    return fail(M3_E_UNSUPPORTED, "D=%d: the backward takes multiples of 8 up to %d", D, m3::kLayerPostBwdMaxD);
  if (B == 0 || L == 0) {
    g_err[0] = '\0';
    return M3_OK;
  }
  if (!y || !d_out || !scale || !dy || !d_scale || !ws) return fail(M3_E_ARG, "NULL required pointer");
  if (ws_bytes < m3_layer_post_bwd_ws_bytes(B, L, D))
    return fail(M3_E_ARG, "workspace of %zu bytes, %zu needed", ws_bytes, m3_layer_post_bwd_ws_bytes(B, L, D));
  const size_t es = io_dtype == M3_DTYPE_BF16 ? 2 : 4;
  if ((reinterpret_cast<uintptr_t>(y) | reinterpret_cast<uintptr_t>(d_out) | reinterpret_cast<uintptr_t>(dy) |
       reinterpret_cast<uintptr_t>(ws)) % 16 != 0 || (D * es) % 16 != 0)
    return fail(M3_E_ALIGN, "y, d_out, dy and ws must be 16-byte aligned");
  m3::LayerPostBwdArgs a;
  a.y = y; a.dn = d_out; a.scale = scale; a.dy = dy; a.part = reinterpret_cast<float*>(ws);
  a.B = B; a.L = L; a.D = D; a.eps = eps;
  return check_launch(m3::layer_post_bwd_launch(a, d_scale, io_dtype == M3_DTYPE_BF16,
                                                reinterpret_cast<hipStream_t>(stream)), "layer post backward");
}

size_t m3_layer_pre_bwd_ws_bytes(int B, int L, int H, int N) {
  if (B <= 0 || L <= 0 || H <= 0 || N <= 0) return 0;
  return (size_t)m3::layer_pre_bwd_parts(B, L) * (2 * N + H) * sizeof(float);
}

int m3_layer_pre_bwd(const void* proj, const float* dt_bias, const float* B_norm_scale, const float* C_norm_scale,
                     const void* dQ, const void* dK, const void* dV, const void* dZ, const float* dADT,
                     const float* dDT, const float* dTrap, const float* dAngles, void* d_proj, float* d_dt_bias,
                     float* d_B_norm_scale, float* d_C_norm_scale, int B, int L, int H, int P, int N, int R,
                     float A_floor, float eps, int io_dtype, void* ws, size_t ws_bytes, void* stream) {
  if (io_dtype != M3_DTYPE_F32 && io_dtype != M3_DTYPE_BF16)
    return fail(M3_E_ARG, "io_dtype must be M3_DTYPE_F32 or M3_DTYPE_BF16, got %d", io_dtype);
  if (B < 0 || L < 0 || H <= 0 || P <= 0 || N <= 0 || R < 0)
    return fail(M3_E_ARG, "non-positive dimension (B=%d L=%d H=%d P=%d N=%d R=%d)", B, L, H, P, N, R);
  if (N > m3::kLayerPreBwdMaxN)
    return fail(M3_E_UNSUPPORTED, "d_state %d above the backward's %d", N, m3::kLayerPreBwdMaxN);
  if (B == 0 || L == 0) {
    g_err[0] = '\0';
    return M3_OK;
  }
  if (!proj || !dt_bias || !B_norm_scale || !C_norm_scale || !dQ || !dK || !dADT || !dDT || !dTrap ||
      (R > 0 && !dAngles) || !d_proj || !d_dt_bias || !d_B_norm_scale || !d_C_norm_scale || !ws)
    return fail(M3_E_ARG, "NULL required pointer");
  if ((dV == nullptr) != (dZ == nullptr))
    return fail(M3_E_ARG, "pass dV and dZ together (both NULL: already in d_proj's x and z columns)");
  if (ws_bytes < m3_layer_pre_bwd_ws_bytes(B, L, H, N))
    return fail(M3_E_ARG, "workspace of %zu bytes, %zu needed", ws_bytes, m3_layer_pre_bwd_ws_bytes(B, L, H, N));
  m3::LayerPreBwdArgs a;
  a.proj = proj; a.dt_bias = dt_bias; a.b_scale = B_norm_scale; a.c_scale = C_norm_scale;
  a.dq = dQ; a.dk = dK; a.dv = dV; a.dz = dZ; a.dadt = dADT; a.ddt = dDT; a.dtrap = dTrap; a.dang = dAngles;
  a.dproj = d_proj; a.part = reinterpret_cast<float*>(ws);
  a.B = B; a.L = L; a.H = H; a.P = P; a.N = N; a.R = R; a.A_floor = A_floor; a.eps = eps;
  return check_launch(m3::layer_pre_bwd_launch(a, d_B_norm_scale, d_C_norm_scale, d_dt_bias,
                                               io_dtype == M3_DTYPE_BF16, reinterpret_cast<hipStream_t>(stream)),
                      "layer pre backward");
}

int m3_block_norm(const float* x, const float* scale, const float* bias, void* out, int B, int L, int D, float eps,
                  int out_dtype, void* stream) {
  if (out_dtype != M3_DTYPE_F32 && out_dtype != M3_DTYPE_BF16)
    return fail(M3_E_ARG, "out_dtype must be M3_DTYPE_F32 or M3_DTYPE_BF16, got %d", out_dtype);
  if (B < 0 || L < 0 || D <= 0) return fail(M3_E_ARG, "non-positive dimension (B=%d L=%d D=%d)", B, L, D);
  if (B == 0 || L == 0) {
    g_err[0] = '\0';
    return M3_OK;
  }
  if (!x || !scale || !bias || !out) return fail(M3_E_ARG, "NULL required pointer");
  m3::BlockNormArgs a;
  a.x = x; a.scale = scale; a.bias = bias; a.out = out; a.rows = (long)B * L; a.D = D; a.eps = eps; a.vec = 0;
  return check_launch(m3::block_norm_launch(a, out_dtype == M3_DTYPE_BF16, reinterpret_cast<hipStream_t>(stream)),
                      "block norm");
}

int m3_block_act_norm(const void* y, const void* h1, const void* h2, const float* skip, float* out,
                      const float* scale, const float* bias, void* ln_out, int B, int L, int D, float eps,
                      int activation, int io_dtype, int ln_dtype, void* stream) {
  if (io_dtype != M3_DTYPE_F32 && io_dtype != M3_DTYPE_BF16)
    return fail(M3_E_ARG, "io_dtype must be M3_DTYPE_F32 or M3_DTYPE_BF16, got %d", io_dtype);
  if (ln_dtype != M3_DTYPE_F32 && ln_dtype != M3_DTYPE_BF16)
    return fail(M3_E_ARG, "ln_dtype must be M3_DTYPE_F32 or M3_DTYPE_BF16, got %d", ln_dtype);
  if (activation < M3_ACT_GELU || activation > M3_ACT_HALF_GLU2)
    return fail(M3_E_ARG, "activation must be one of M3_ACT_GELU..M3_ACT_HALF_GLU2, got %d", activation);
  if (B < 0 || L < 0 || D <= 0) return fail(M3_E_ARG, "non-positive dimension (B=%d L=%d D=%d)", B, L, D);
  if (B == 0 || L == 0) {
    g_err[0] = '\0';
    return M3_OK;
  }
  if (!y || !skip || !scale || !bias || !ln_out) return fail(M3_E_ARG, "NULL required pointer");
  if (activation == M3_ACT_FULL_GLU && !h1) return fail(M3_E_ARG, "full_glu needs h1 (the out1 Dense output)");
  if (activation != M3_ACT_GELU && !h2) return fail(M3_E_ARG, "the GLU activations need h2 (the out2 Dense output)");
  if (ln_out == (const void*)skip || (out && ln_out == (void*)out))
    return fail(M3_E_ARG, "ln_out must not alias skip or out");
  m3::BlockActNormArgs a{};
  a.y = y; a.h1 = h1; a.h2 = h2; a.skip = skip; a.out = out; a.scale = scale; a.bias = bias; a.ln_out = ln_out;
  a.rows = (long)B * L; a.D = D; a.eps = eps; a.act = activation;
  return check_launch(m3::block_act_norm_launch(a, io_dtype == M3_DTYPE_BF16, ln_dtype == M3_DTYPE_BF16,
                                                reinterpret_cast<hipStream_t>(stream)),
                      "block activation + norm");
}

int m3_log_softmax(const float* x, float* out, int B, int L, int V, void* stream) {
  if (B < 0 || L < 0 || V <= 0) return fail(M3_E_ARG, "non-positive dimension (B=%d L=%d V=%d)", B, L, V);
  if (B == 0 || L == 0) {
    g_err[0] = '\0';
    return M3_OK;
  }
  if (!x || !out) return fail(M3_E_ARG, "NULL required pointer");
  return check_launch(m3::log_softmax_launch(x, out, (long)B * L, V, reinterpret_cast<hipStream_t>(stream)),
                      "log_softmax");
}

int m3_block_gelu(const void* x, void* out, int B, int L, int D, int io_dtype, void* stream) {
  if (io_dtype != M3_DTYPE_F32 && io_dtype != M3_DTYPE_BF16)
    return fail(M3_E_ARG, "io_dtype must be M3_DTYPE_F32 or M3_DTYPE_BF16, got %d", io_dtype);
  if (B < 0 || L < 0 || D <= 0) return fail(M3_E_ARG, "non-positive dimension (B=%d L=%d D=%d)", B, L, D);
  if (B == 0 || L == 0) {
    g_err[0] = '\0';
    return M3_OK;
  }
  if (!x || !out) return fail(M3_E_ARG, "NULL required pointer");
  m3::BlockEltArgs a{};
  a.y = x; a.out = out; a.n = (long)B * L * D; a.act = M3_ACT_GELU;
  return check_launch(m3::block_elt_launch(a, true, io_dtype == M3_DTYPE_BF16, reinterpret_cast<hipStream_t>(stream)),
                      "block gelu");
}

int m3_block_act(const void* y, const void* h1, const void* h2, const float* skip, float* out, int B, int L, int D,
                 int activation, int io_dtype, void* stream) {
  if (io_dtype != M3_DTYPE_F32 && io_dtype != M3_DTYPE_BF16)
    return fail(M3_E_ARG, "io_dtype must be M3_DTYPE_F32 or M3_DTYPE_BF16, got %d", io_dtype);
  if (activation < M3_ACT_GELU || activation > M3_ACT_HALF_GLU2)
    return fail(M3_E_ARG, "activation must be one of M3_ACT_GELU..M3_ACT_HALF_GLU2, got %d", activation);
  if (B < 0 || L < 0 || D <= 0) return fail(M3_E_ARG, "non-positive dimension (B=%d L=%d D=%d)", B, L, D);
  if (B == 0 || L == 0) {
    g_err[0] = '\0';
    return M3_OK;
  }
  if (!y || !skip || !out) return fail(M3_E_ARG, "NULL required pointer");
  if (activation == M3_ACT_FULL_GLU && !h1) return fail(M3_E_ARG, "full_glu needs h1 (the out1 Dense output)");
  if (activation != M3_ACT_GELU && !h2) return fail(M3_E_ARG, "the GLU activations need h2 (the out2 Dense output)");
  m3::BlockEltArgs a{};
  a.y = y; a.h1 = h1; a.h2 = h2; a.skip = skip; a.out = out; a.n = (long)B * L * D; a.act = activation;
  return check_launch(m3::block_elt_launch(a, false, io_dtype == M3_DTYPE_BF16, reinterpret_cast<hipStream_t>(stream)),
                      "block activation");
}

int m3_block_act_bwd(const float* d_out, const void* y, const void* h1, const void* h2, void* dh2, void* dd, int B,
                     int L, int D, int activation, int io_dtype, void* stream) {
  if (io_dtype != M3_DTYPE_F32 && io_dtype != M3_DTYPE_BF16)
    return fail(M3_E_ARG, "io_dtype must be M3_DTYPE_F32 or M3_DTYPE_BF16, got %d", io_dtype);
  if (activation < M3_ACT_GELU || activation > M3_ACT_HALF_GLU2)
    return fail(M3_E_ARG, "activation must be one of M3_ACT_GELU..M3_ACT_HALF_GLU2, got %d", activation);
  if (B < 0 || L < 0 || D <= 0) return fail(M3_E_ARG, "non-positive dimension (B=%d L=%d D=%d)", B, L, D);
  if (B == 0 || L == 0) {
    g_err[0] = '\0';
    return M3_OK;
  }
  if (!d_out || !y || !dd) return fail(M3_E_ARG, "NULL required pointer");
  if (activation == M3_ACT_FULL_GLU && !h1) return fail(M3_E_ARG, "full_glu needs h1 (the out1 Dense output)");
  if (activation != M3_ACT_GELU && (!h2 || !dh2))
    return fail(M3_E_ARG, "the GLU activations need h2 and dh2 (the out2 Dense output and its gradient)");
  m3::BlockBwdArgs a{};
  a.da = d_out; a.y = y; a.h1 = activation == M3_ACT_FULL_GLU ? h1 : nullptr;
  a.h2 = activation != M3_ACT_GELU ? h2 : nullptr; a.dh2 = activation != M3_ACT_GELU ? dh2 : nullptr;
  a.dd = dd; a.n = (long)B * L * D; a.act = activation;
  return check_launch(m3::block_act_bwd_launch(a, io_dtype == M3_DTYPE_BF16, reinterpret_cast<hipStream_t>(stream)),
                      "block activation backward");
}

int m3_block_gelu_bwd(const void* dg, const void* dd, const void* y, void* dy, int B, int L, int D, int activation,
                      int io_dtype, void* stream) {
  if (io_dtype != M3_DTYPE_F32 && io_dtype != M3_DTYPE_BF16)
    return fail(M3_E_ARG, "io_dtype must be M3_DTYPE_F32 or M3_DTYPE_BF16, got %d", io_dtype);
  if (activation < M3_ACT_FULL_GLU || activation > M3_ACT_HALF_GLU2)
    return fail(M3_E_ARG, "the gelu backward follows a GLU activation (M3_ACT_FULL_GLU..M3_ACT_HALF_GLU2), got %d",
                activation);
  if (B < 0 || L < 0 || D <= 0) return fail(M3_E_ARG, "non-positive dimension (B=%d L=%d D=%d)", B, L, D);
  if (B == 0 || L == 0) {
    g_err[0] = '\0';
    return M3_OK;
  }
  if (!dg || !y || !dy || (activation != M3_ACT_FULL_GLU && !dd)) return fail(M3_E_ARG, "NULL required pointer");
  m3::BlockBwdArgs a{};
  a.dg = dg; a.dd_in = activation != M3_ACT_FULL_GLU ? dd : nullptr; a.y = y; a.dy = dy;
  a.n = (long)B * L * D; a.act = activation;
  return check_launch(m3::block_gelu_bwd_launch(a, io_dtype == M3_DTYPE_BF16, reinterpret_cast<hipStream_t>(stream)),
                      "block gelu backward");
}

size_t m3_block_norm_bwd_ws_bytes(int B, int L, int D) {
  if (B <= 0 || L <= 0 || D <= 0) return 0;
  return (size_t)m3::block_norm_bwd_parts((long)B * L) * 2 * D * sizeof(float);
}

int m3_block_norm_bwd(const float* x, const float* scale, const void* d_norm, const float* d_res, float* dx,
                      float* d_scale, float* d_bias, int B, int L, int D, float eps, int io_dtype, void* ws,
                      size_t ws_bytes, void* stream) {
  if (io_dtype != M3_DTYPE_F32 && io_dtype != M3_DTYPE_BF16)
    return fail(M3_E_ARG, "io_dtype must be M3_DTYPE_F32 or M3_DTYPE_BF16, got %d", io_dtype);
  if (B < 0 || L < 0 || D <= 0) return fail(M3_E_ARG, "non-positive dimension (B=%d L=%d D=%d)", B, L, D);
  if (D % 4 != 0 || D > m3::kBlockNormBwdMaxD)
    return fail(M3_E_UNSUPPORTED, "D=%d: the LayerNorm backward takes multiples of 4 up to %d", D,
                m3::kBlockNormBwdMaxD);
  if (B == 0 || L == 0) {
    g_err[0] = '\0';
    return M3_OK;
  }
  if (!x || !scale || !d_norm || !dx || !d_scale || !d_bias || !ws) return fail(M3_E_ARG, "NULL required pointer");
  if (ws_bytes < m3_block_norm_bwd_ws_bytes(B, L, D))
    return fail(M3_E_ARG, "workspace of %zu bytes, %zu needed", ws_bytes, m3_block_norm_bwd_ws_bytes(B, L, D));
  if (!aligned16(x) || !aligned16(scale) || !aligned16(d_norm) || (d_res && !aligned16(d_res)) || !aligned16(dx) ||
      !aligned16(ws))
    return fail(M3_E_ALIGN, "x, scale, d_norm, d_res, dx and ws must be 16-byte aligned");
  m3::BlockNormBwdArgs a;
  a.x = x; a.scale = scale; a.dn = d_norm; a.dres = d_res; a.dx = dx; a.part = reinterpret_cast<float*>(ws);
  a.rows = (long)B * L; a.D = D; a.eps = eps;
  return check_launch(m3::block_norm_bwd_launch(a, d_scale, d_bias, io_dtype == M3_DTYPE_BF16,
                                                reinterpret_cast<hipStream_t>(stream)), "LayerNorm backward");
}

int m3_log_softmax_nll(float* logits, const int* targets, float* loss, int B, int L, int V, float weight,
                       void* stream) {
  if (B < 0 || L < 0 || V <= 0) return fail(M3_E_ARG, "non-positive dimension (B=%d L=%d V=%d)", B, L, V);
  if (B == 0 || L == 0) {
    g_err[0] = '\0';
    return M3_OK;
  }
  if (!logits || !targets || !loss) return fail(M3_E_ARG, "NULL required pointer");
  return check_launch(m3::nll_launch(logits, targets, loss, (long)B * L, V, weight,
                                     reinterpret_cast<hipStream_t>(stream)), "log_softmax NLL");
}

int m3_split_bf16x3(const float* x, void* hi_a, void* hi_b, void* lo, long rows, int K, long ld, void* stream) {
  if (rows < 0 || K <= 0) return fail(M3_E_ARG, "non-positive dimension (rows=%ld K=%d)", rows, K);
  if (ld < K) return fail(M3_E_ARG, "row stride ld=%ld is below the row length K=%d", ld, K);
  if (rows == 0) {
    g_err[0] = '\0';
    return M3_OK;
  }
  if (!x || !hi_a || !lo) return fail(M3_E_ARG, "NULL required pointer");
  return check_launch(m3::split3_launch(x, hi_a, hi_b, lo, rows, K, ld, reinterpret_cast<hipStream_t>(stream)),
                      "split bf16x3");
}

}  // extern "C"
