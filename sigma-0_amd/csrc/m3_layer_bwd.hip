// Backward of the mixer layer's elementwise kernels (m3_layer.hip), as autodiff of
// Mamba3SSM._preprocess and _post_norm_and_project (src/base_model/models/
// mamba3.py:203-331) gives it, with float32 arithmetic:
//   layer_post_bwd_kernel  the output RMSNorm n = y r scale, r = rsqrt(mean(y^2) + eps):
//                          dy = r (dn scale) - r^3 y mean(dn scale y), one workgroup per
//                          kPostTok tokens, its waves on every fourth token (each loading
//                          its next token before working on the current one); the
//                          scale's gradient sum_t dn y r as one partial row per workgroup
//   layer_pre_bwd_kernel   d(proj) from the scan's gradients, one workgroup per tile of
//                          kPreTile tokens of one batch row: dZ and dV into the z and x
//                          columns (unless m3_layer_scan_bwd wrote them there) and BCNorm's
//                          backward into B and C (one wave per token, both rows' loads
//                          issued before their stores), the decay's chain
//                          rule into dd_dt and dd_A and dTrap into trap (lanes along the
//                          tokens, one head per wave at a time), dAngles into the angle
//                          columns; the norm scales' and dt_bias's gradients as one partial
//                          row per workgroup
//   reduce_slices_kernel,  the partial rows summed in a fixed order (the gradients are
//   reduce_final_kernel    deterministic): kReduceSlices slices of rows side by side,
//                          then the slices' sums
// Each is one read of its inputs and one write of its outputs: HBM-bound.
#include "m3_scan.h"

namespace m3 {
namespace {

constexpr int kBwdElThreads = 256;
constexpr int kPostTok = 16;            // tokens per workgroup, layer_post_bwd
constexpr int kPreTile = 64;            // tokens per workgroup, layer_pre_bwd (one per lane)
constexpr int kPreThreads = 512;        // layer_pre_bwd's workgroup: eight waves
constexpr int kPreHG = 32;              // layer_pre_bwd: heads per LDS-staged group
constexpr int kPostChunks = kLayerPostBwdMaxD / (64 * 8);   // 8-element chunks per lane, at most
constexpr int kPreCols = kLayerPreBwdMaxN / 64;             // B / C columns per lane

__device__ __forceinline__ float softplus_f(float x) {     // as layer_pre: logaddexp(x, 0)
  return fmaxf(x, 0.0f) + log1pf(expf(-fabsf(x)));
}

// Two rows of n elements, s0 -> d0 and s1 -> d1, by one wave: 16-byte pieces when all
// four are 16-byte aligned, every load of a lane issued before its stores.
template <typename T>
__device__ __forceinline__ void copy_two_rows(T* __restrict__ d0, const T* __restrict__ s0, T* __restrict__ d1,
                                              const T* __restrict__ s1, int n, int lane) {
  constexpr int V = 16 / sizeof(T);
  if (((reinterpret_cast<uintptr_t>(d0) | reinterpret_cast<uintptr_t>(s0) | reinterpret_cast<uintptr_t>(d1) |
        reinterpret_cast<uintptr_t>(s1)) & 15) == 0 && n % V == 0) {
    const int nv = n / V;
    const uint4* v0 = reinterpret_cast<const uint4*>(s0);
    const uint4* v1 = reinterpret_cast<const uint4*>(s1);
    uint4* w0 = reinterpret_cast<uint4*>(d0);
    uint4* w1 = reinterpret_cast<uint4*>(d1);
    for (int i = lane; i < nv; i += 4 * 64) {
      const bool k1 = i + 64 < nv, k2 = i + 128 < nv, k3 = i + 192 < nv;
      const uint4 a0 = v0[i], c0 = v1[i];
      uint4 a1 = {}, c1 = {}, a2 = {}, c2 = {}, a3 = {}, c3 = {};
      if (k1) { a1 = v0[i + 64]; c1 = v1[i + 64]; }
      if (k2) { a2 = v0[i + 128]; c2 = v1[i + 128]; }
      if (k3) { a3 = v0[i + 192]; c3 = v1[i + 192]; }
      w0[i] = a0;
      w1[i] = c0;
      if (k1) { w0[i + 64] = a1; w1[i + 64] = c1; }
      if (k2) { w0[i + 128] = a2; w1[i + 128] = c2; }
      if (k3) { w0[i + 192] = a3; w1[i + 192] = c3; }
    }
  } else {
    for (int i = lane; i < n; i += 64) {
      d0[i] = s0[i];
      d1[i] = s1[i];
    }
  }
}

// CH: 8-element chunks per lane, ceil(D / 512).
template <typename T, int CH>
__global__ __launch_bounds__(kBwdElThreads)
void layer_post_bwd_kernel(LayerPostBwdArgs a) {
  __shared__ float red[kBwdElThreads / 64][kLayerPostBwdMaxD];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const long rows = (long)a.B * a.L, t0 = (long)blockIdx.x * kPostTok;
  const long t1 = t0 + kPostTok < rows ? t0 + kPostTok : rows;
  const int D = a.D, nch = D / 8;
  const float invD = 1.0f / (float)D;
  float sc[CH][8], acc[CH][8];
#pragma unroll
  for (int j = 0; j < CH; ++j) {
    const int c = lane + 64 * j;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      sc[j][e] = c < nch ? a.scale[8 * c + e] : 0.0f;
      acc[j][e] = 0.0f;
    }
  }
  Vec8<T> ny[CH], nd[CH];                              // the wave's next token
  auto issue = [&](long t) {
    const T* yr = reinterpret_cast<const T*>(a.y) + t * D;
    const T* dr = reinterpret_cast<const T*>(a.dn) + t * D;
#pragma unroll
    for (int j = 0; j < CH; ++j) {
      const int c = lane + 64 * j;
      if (c < nch) {
        ny[j].load(yr + 8 * c);
        nd[j].load(dr + 8 * c);
      }
    }
  };
  constexpr int kW = kBwdElThreads / 64;
  if (t0 + wave < t1) issue(t0 + wave);
  for (long t = t0 + wave; t < t1; t += kW) {
    float yv[CH][8], dv[CH][8];
#pragma unroll
    for (int j = 0; j < CH; ++j) {
      ny[j].to_f(yv[j]);
      nd[j].to_f(dv[j]);
    }
    if (t + kW < t1) issue(t + kW);
    float ss = 0.0f, sd = 0.0f;
#pragma unroll
    for (int j = 0; j < CH; ++j) {
      if (lane + 64 * j < nch) {
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          ss += yv[j][e] * yv[j][e];
          sd += dv[j][e] * sc[j][e] * yv[j][e];
        }
      }
    }
    ss = group_sum<64>(ss);
    sd = group_sum<64>(sd);
    const float r = rsqrtf(ss * invD + a.eps);
    const float k = r * r * r * (sd * invD);
    T* out = reinterpret_cast<T*>(a.dy) + t * D;
#pragma unroll
    for (int j = 0; j < CH; ++j) {
      const int c = lane + 64 * j;
      if (c < nch) {
        float o[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          o[e] = r * (dv[j][e] * sc[j][e]) - k * yv[j][e];
          acc[j][e] += dv[j][e] * yv[j][e] * r;
        }
        store8(out + 8 * c, o);
      }
    }
  }
  // the workgroup's partial row: the four waves' sums added in wave order
#pragma unroll
  for (int j = 0; j < CH; ++j) {
    const int c = lane + 64 * j;
    if (c < nch)
#pragma unroll
      for (int e = 0; e < 8; ++e) red[wave][8 * c + e] = acc[j][e];
  }
  __syncthreads();
  float* part = a.part + (long)blockIdx.x * D;
  for (int c = threadIdx.x; c < D; c += kBwdElThreads) part[c] = ((red[0][c] + red[1][c]) + red[2][c]) + red[3][c];
}

template <typename T>
__global__ __launch_bounds__(kPreThreads)
void layer_pre_bwd_kernel(LayerPreBwdArgs a) {
  constexpr int kW = kPreThreads / 64;
  __shared__ float red[kW][2][kLayerPreBwdMaxN];
  __shared__ float sdd[kPreTile][2 * kPreHG + 1];     // a head group's dd_dt, dd_A per token
  __shared__ float sgo[kPreTile][3 * kPreHG + 1];     // and their gradients, with trap's
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int tiles = (a.L + kPreTile - 1) / kPreTile;
  const int b = blockIdx.x / tiles, t0 = (blockIdx.x % tiles) * kPreTile;
  const int nt = a.L - t0 < kPreTile ? a.L - t0 : kPreTile;
  const int H = a.H, N = a.N, R = a.R, di = H * a.P;
  const int dp = 2 * di + 2 * N + 3 * H + R;
  const int oB = 2 * di, oC = oB + N, oT = oC + N;      // dd_dt at oT, dd_A at oT + H, trap at oT + 2H,
  const long row0 = (long)b * a.L + t0;                  // angles at oT + 3H
  const T* proj = reinterpret_cast<const T*>(a.proj) + row0 * dp;
  T* dproj = reinterpret_cast<T*>(a.dproj) + row0 * dp;
  const int nparts = 2 * N + H;
  float* part = a.part + (long)blockIdx.x * nparts;

  // ---- one wave per token: dZ, dV into the z and x columns; BCNorm's backward
  float accB[kPreCols], accC[kPreCols];
#pragma unroll
  for (int k = 0; k < kPreCols; ++k) accB[k] = accC[k] = 0.0f;
  const float invN = 1.0f / (float)N;
  for (int i = wave; i < nt; i += kW) {
    const long row = row0 + i;
    T* dpr = dproj + (long)i * dp;
    const T* pr = proj + (long)i * dp;
    if (a.dz)   // else the scan's backward wrote them there
      copy_two_rows(dpr, reinterpret_cast<const T*>(a.dz) + row * di, dpr + di,
                    reinterpret_cast<const T*>(a.dv) + row * di, di, lane);
    // n = m rsqrt(mean m^2 + eps) scale  (B: K's, C: Q's).  Both sides' rows are loaded
    // before either side's stores (which could alias them as far as the compiler knows).
    float mv[2][kPreCols], dnv[2][kPreCols];
#pragma unroll
    for (int side = 0; side < 2; ++side) {
      const T* g = reinterpret_cast<const T*>(side ? a.dq : a.dk) + row * N;
      const int o = side ? oC : oB;
#pragma unroll
      for (int k = 0; k < kPreCols; ++k) {
        const int n = lane + 64 * k;
        mv[side][k] = n < N ? Elem<T>::to_f(pr[o + n]) : 0.0f;
        dnv[side][k] = n < N ? Elem<T>::to_f(g[n]) : 0.0f;
      }
    }
#pragma unroll
    for (int side = 0; side < 2; ++side) {
      const float* scale = side ? a.c_scale : a.b_scale;
      const int o = side ? oC : oB;
      const float* m = mv[side];
      const float* dn = dnv[side];
      float ds[kPreCols], ss = 0.0f, sd = 0.0f;
#pragma unroll
      for (int k = 0; k < kPreCols; ++k) {
        const int n = lane + 64 * k;
        ds[k] = n < N ? dn[k] * scale[n] : 0.0f;
        ss += m[k] * m[k];
        sd += ds[k] * m[k];
      }
      ss = group_sum<64>(ss);
      sd = group_sum<64>(sd);
      const float r = rsqrtf(ss * invN + a.eps);
      const float kk = r * r * r * (sd * invN);
#pragma unroll
      for (int k = 0; k < kPreCols; ++k) {
        const int n = lane + 64 * k;
        if (n < N) {
          dpr[o + n] = Elem<T>::from_f(r * ds[k] - kk * m[k]);
          // the scale's gradient: dn m r
          const float gs = dn[k] * m[k] * r;
          if (side) accC[k] += gs;
          else accB[k] += gs;
        }
      }
    }
  }
  // ---- lanes along the tokens, one head per wave at a time: DT = softplus(dd_dt +
  // dt_bias), A = min(-softplus(dd_A), -A_floor), ADT = A DT; trap passes through.  The
  // heads go in groups of kPreHG: the group's dd_dt and dd_A columns come in through
  // LDS and its three gradient columns go out through LDS, as row pieces.
  for (int h0 = 0; h0 < H; h0 += kPreHG) {
    const int hg = H - h0 < kPreHG ? H - h0 : kPreHG;
    __syncthreads();   // the previous group's sdd reads and sgo stores are done
    for (int e = tid; e < nt * 2 * hg; e += kPreThreads) {
      const int i = e / (2 * hg), j = e - i * 2 * hg;
      const int col = j < hg ? oT + h0 + j : oT + H + h0 + (j - hg);
      sdd[i][j] = Elem<T>::to_f(proj[(long)i * dp + col]);
    }
    __syncthreads();
    for (int hl = wave; hl < hg; hl += kW) {
      const int h = h0 + hl;
      float du = 0.0f;
      if (lane < nt) {
        const long hi = ((long)b * H + h) * a.L + t0 + lane;
        const float dadt = a.dadt[hi], ddt = a.ddt[hi], dtrap = a.dtrap[hi];
        const float u = sdd[lane][hl] + a.dt_bias[h];
        const float ddA = sdd[lane][hg + hl];
        const float DTv = softplus_f(u), sp = softplus_f(ddA);
        const float A = fminf(-sp, -a.A_floor);
        du = (ddt + dadt * A) * (1.0f / (1.0f + expf(-u)));
        // the clip passes the gradient below -A_floor, half of it on a tie (jax's min)
        const float gate = -sp < -a.A_floor ? 1.0f : (-sp == -a.A_floor ? 0.5f : 0.0f);
        const float dA = -(dadt * DTv) * gate * (1.0f / (1.0f + expf(-ddA)));
        sgo[lane][hl] = du;
        sgo[lane][hg + hl] = dA;
        sgo[lane][2 * hg + hl] = dtrap;
      }
      du = group_sum<64>(du);
      if (lane == 0) part[2 * N + h] = du;
    }
    __syncthreads();
    for (int e = tid; e < nt * 3 * hg; e += kPreThreads) {
      const int i = e / (3 * hg), j = e - i * 3 * hg;
      const int q = j / hg, jj = j - q * hg;           // 0: dd_dt, 1: dd_A, 2: trap
      dproj[(long)i * dp + oT + q * H + h0 + jj] = Elem<T>::from_f(sgo[i][j]);
    }
  }
  // ---- the angle rates' gradients into their columns
  for (int e = tid; e < nt * R; e += kPreThreads) {
    const int i = e / R, r = e % R;
    dproj[(long)i * dp + oT + 3 * H + r] = Elem<T>::from_f(a.dang[(row0 + i) * R + r]);
  }
  // ---- the norm scales' partial sums over the tile: the waves' rows added in order
#pragma unroll
  for (int k = 0; k < kPreCols; ++k) {
    const int n = lane + 64 * k;
    if (n < N) {
      red[wave][0][n] = accB[k];
      red[wave][1][n] = accC[k];
    }
  }
  __syncthreads();
  for (int n = tid; n < 2 * N; n += kPreThreads) {
    const int side = n / N, c = n % N;
    float s = 0.0f;
#pragma unroll
    for (int w = 0; w < kW; ++w) s += red[w][side][c];
    part[n] = s;
  }
}

// mid[y][c] = sum of part[r][c] over slice y of the rows (kReduceSlices slices): 64
// columns per workgroup, four row phases per column, added in a fixed order.
__global__ __launch_bounds__(kBwdElThreads)
void reduce_slices_kernel(const float* part, long rows, int cols, float* mid) {
  __shared__ float red[4][64];
  const int c = blockIdx.x * 64 + (threadIdx.x & 63), g = threadIdx.x >> 6;
  const long r0 = rows * blockIdx.y / kReduceSlices, r1 = rows * (blockIdx.y + 1) / kReduceSlices;
  float s = 0.0f;
  if (c < cols)
    for (long r = r0 + g; r < r1; r += 4) s += part[r * cols + c];
  red[g][threadIdx.x & 63] = s;
  __syncthreads();
  if (g == 0 && c < cols) mid[(long)blockIdx.y * cols + c] = red[0][threadIdx.x] + red[1][threadIdx.x] +
                                                             red[2][threadIdx.x] + red[3][threadIdx.x];
}
// out[c] = sum of mid[y][c] over the slices in order; column c goes to out0 (c < n0),
// out1 (c < n0 + n1) or out2.
__global__ __launch_bounds__(kBwdElThreads)
void reduce_final_kernel(const float* mid, int cols, float* out0, int n0, float* out1, int n1, float* out2) {
  const int c = blockIdx.x * kBwdElThreads + threadIdx.x;
  if (c >= cols) return;
  float s = 0.0f;
  for (int y = 0; y < kReduceSlices; ++y) s += mid[(long)y * cols + c];
  if (c < n0) out0[c] = s;
  else if (c < n0 + n1) out1[c - n0] = s;
  else out2[c - n0 - n1] = s;
}

}  // namespace

hipError_t reduce_rows(const float* part, long rows, int cols, float* mid, float* out0, int n0, float* out1, int n1,
                       float* out2, hipStream_t st) {
  hipLaunchKernelGGL(reduce_slices_kernel, dim3((cols + 63) / 64, kReduceSlices), dim3(kBwdElThreads), 0, st, part,
                     rows, cols, mid);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL(reduce_final_kernel, dim3((cols + kBwdElThreads - 1) / kBwdElThreads), dim3(kBwdElThreads), 0,
                     st, mid, cols, out0, n0, out1, n1, out2);
  return hipGetLastError();
}

long layer_post_bwd_parts(int B, int L) { return ((long)B * L + kPostTok - 1) / kPostTok + kReduceSlices; }
long layer_pre_bwd_parts(int B, int L) { return (long)B * ((L + kPreTile - 1) / kPreTile) + kReduceSlices; }

hipError_t layer_post_bwd_launch(const LayerPostBwdArgs& a, float* dscale, bool bf16_io, hipStream_t st) {
  const long runs = layer_post_bwd_parts(a.B, a.L) - kReduceSlices;   // the rest of the rows: the slices' sums
  const dim3 grid((unsigned)runs);
  const int ch = (a.D / 8 + 63) / 64;
  static_assert(kPostChunks == 4, "layer_post_bwd instantiations");
#define M3_POST_BWD(CH)                                                                                  \
  if (ch == CH) {                                                                                        \
    if (bf16_io) hipLaunchKernelGGL((layer_post_bwd_kernel<bf16, CH>), grid, dim3(kBwdElThreads), 0, st, a); \
    else hipLaunchKernelGGL((layer_post_bwd_kernel<float, CH>), grid, dim3(kBwdElThreads), 0, st, a);        \
  }
  M3_POST_BWD(1) M3_POST_BWD(2) M3_POST_BWD(3) M3_POST_BWD(4)
#undef M3_POST_BWD
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  return reduce_rows(a.part, runs, a.D, a.part + runs * a.D, dscale, a.D, nullptr, 0, nullptr, st);
}

hipError_t layer_pre_bwd_launch(const LayerPreBwdArgs& a, float* d_b_scale, float* d_c_scale, float* d_dt_bias,
                                bool bf16_io, hipStream_t st) {
  const long blocks = layer_pre_bwd_parts(a.B, a.L) - kReduceSlices;
  if (bf16_io) hipLaunchKernelGGL(layer_pre_bwd_kernel<bf16>, dim3((unsigned)blocks), dim3(kPreThreads), 0, st, a);
  else hipLaunchKernelGGL(layer_pre_bwd_kernel<float>, dim3((unsigned)blocks), dim3(kPreThreads), 0, st, a);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  const int cols = 2 * a.N + a.H;
  return reduce_rows(a.part, blocks, cols, a.part + blocks * cols, d_b_scale, a.N, d_c_scale, a.N, d_dt_bias, st);
}

}  // namespace m3
