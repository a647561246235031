// MFMA tile helpers, direct-to-LDS staging and small LDS store/load helpers shared
// by the chunked prefill kernels.
#pragma once

#include "m3_scan.h"

namespace m3 {

// Direct-to-LDS loads (global_load_lds): the LDS slot is M0 plus size * lane.  They
// are issued from inline assembly so that the compiler does not treat every later
// LDS access as possibly overlapping the in-flight writes (it would wait for all
// outstanding vector memory before the first LDS read of the matrix phase).  The
// kernel orders them itself: an s_waitcnt vmcnt(0) and a barrier separate each
// batch from the first reads of the staged rows.
// The compiler inserts no hazard wait states for instructions inside inline asm, so
// the asm carries its own: a vector memory instruction that reads an SGPR written by
// a VALU instruction needs 5 wait states (the compiler reloads spilled address SGPRs
// with v_readlane right before the asm), and the M0 write needs 1.  s_nop 4 gives 5.
// With fewer, the load can form its address from a stale SGPR half.
// The loads carry the non-temporal hint (nt): every staged byte is read once, and at
// the headline shape (bf16, B=8, L=4096, H=32) the hint took the kernel from 233 to
// 201 us in same-box runs (the same hint on the Z loads or the output stores made it
// slower).
typedef __attribute__((address_space(3))) uint4 lds_uint4;
typedef __attribute__((address_space(3))) float lds_float;
__device__ __forceinline__ uint32_t lds_addr(const lds_uint4* p) { return (uint32_t)(uintptr_t)p; }
__device__ __forceinline__ uint32_t lds_addr(const lds_float* p) { return (uint32_t)(uintptr_t)p; }
// Address = wave-uniform base (SGPRs) + 32-bit lane offset.
__device__ __forceinline__ void lds_dma16(const void* sbase, uint32_t voff, lds_uint4* l) {
  asm volatile("s_nop 4\n\tglobal_load_lds_dwordx4 %0, %1 nt" : : "v"(voff), "s"(sbase), "{m0}"(lds_addr(l)) : "memory");
}
__device__ __forceinline__ void lds_dma4(const void* sbase, uint32_t voff, lds_float* l) {
  asm volatile("s_nop 4\n\tglobal_load_lds_dword %0, %1 nt" : : "v"(voff), "s"(sbase), "{m0}"(lds_addr(l)) : "memory");
}

// Direct-to-LDS staging of instructions [J0, J1) of CS rows x S 16-byte slots.
// Instruction j stages 64 slots: lane -> (row, physical slot) = (64j/S + lane/S,
// lane%S), fetching logical slot (lane%S) ^ (row%S), so each row is read whole
// (coalesced) and stored swizzled.  The lane part of the global offset repeats every
// PER instructions (row%S repeats), so a few 32-bit lane offsets plus a wave-uniform
// row base address every instruction.
template <int CS, int S, int J0, int J1>
__device__ __forceinline__ void stage_rows(lds_uint4* dst, const char* src, int stride, int rows_valid,
                                           int lane) {
  constexpr int RP = 64 / S;                               // rows per instruction
  constexpr int PER = S * S / 64 > 1 ? S * S / 64 : 1;     // period of the lane pattern
  static_assert(CS * S % 64 == 0 && J1 <= CS * S / 64, "whole instructions");
  // the lane offsets are recomputed per call (a few VALU on the staging waves) rather
  // than kept live across the chunk loop
  int ln = lane;
  asm volatile("" : "+v"(ln));
  const int lrow = ln / S;
  uint32_t off[PER];
#pragma unroll
  for (int p = 0; p < PER; ++p) {
    const uint32_t row = p * RP + lrow;
    off[p] = row * (uint32_t)stride + 16u * ((ln % S) ^ (row & (S - 1)));
  }
  // the row base is made opaque so that the compiler keeps one wave-uniform base per
  // group of PER instructions instead of strength-reducing to 64-bit lane pointers; the
  // stride too, so that the per-group offsets are formed here (a few scalar operations)
  // instead of being hoisted out of the caller's loop and spilled
  const char* base = src;
  asm volatile("" : "+s"(base));
  int sstride = stride;
  asm volatile("" : "+s"(sstride));
  if (rows_valid >= CS) {
#pragma unroll
    for (int j = J0; j < J1; ++j)
      lds_dma16(base + (long)((j / PER) * (PER * RP)) * sstride, off[j % PER], dst + 64 * j);
  } else {
#pragma unroll
    for (int j = J0; j < J1; ++j)
      if (j * RP + lrow < rows_valid)
        lds_dma16(base + (long)((j / PER) * (PER * RP)) * sstride, off[j % PER], dst + 64 * j);
  }
}
template <int S>
__device__ __forceinline__ const uint4& staged(const uint4* buf, int row, int slot) {
  return buf[row * S + (slot ^ (row & (S - 1)))];
}
// Element (row, col) of a tile staged as above (rows of S 16-byte slots, swizzled).
template <int S, typename T>
__device__ __forceinline__ const T* staged_elem(const uint4* buf, int row, int col) {
  constexpr int E = 16 / (int)sizeof(T);
  return reinterpret_cast<const T*>(&buf[row * S + ((col / E) ^ (row & (S - 1)))]) + col % E;
}

typedef __attribute__((address_space(3))) bf16x4 lds_bf16x4;

// MFMA operand whose 16 rows (A) or columns (B) are columns c0.. of a row-major
// [k][col] LDS matrix: the transpose of what MF16::ld reads.  bf16: two
// ds_read_b64_tr_b16, each giving lane l the column c0 + l%16 of a 4 x 16 block
// (lane 4j+q addresses row j, columns 4q..4q+3).
__device__ __forceinline__ bf16x8 ld_tr(const bf16* buf, int ld, int k0, int c0, int lane) {
  const int g = lane >> 4, l = lane & 15;
  const bf16* p = buf + (k0 + 8 * g + (l >> 2)) * ld + c0 + 4 * (l & 3);
  const bf16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4bf16((lds_bf16x4*)p);
  const bf16x4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4bf16((lds_bf16x4*)(p + 4 * ld));
  bf16x8 f;
  f[0] = lo[0]; f[1] = lo[1]; f[2] = lo[2]; f[3] = lo[3];
  f[4] = hi[0]; f[5] = hi[1]; f[6] = hi[2]; f[7] = hi[3];
  return f;
}
__device__ __forceinline__ float ld_tr(const float* buf, int ld, int k0, int c0, int lane) {
  return buf[(k0 + (lane >> 4)) * ld + c0 + (lane & 15)];
}
// ld_tr from a staged (swizzled) [k][col] bf16 tile, with the rows chosen per lane
// group: lane l gets column c0 + l%16, k-slots 0..3 from rows r_lo + 0..3 and 4..7
// from rows r_hi + 0..3.
template <int S>
__device__ __forceinline__ bf16x8 staged_tr(const uint4* buf, int r_lo, int r_hi, int c0, int lane) {
  const int l = lane & 15;
  const int col = c0 + 4 * (l & 3);
  const bf16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4bf16((lds_bf16x4*)staged_elem<S, bf16>(buf, r_lo + (l >> 2), col));
  const bf16x4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4bf16((lds_bf16x4*)staged_elem<S, bf16>(buf, r_hi + (l >> 2), col));
  bf16x8 f;
  f[0] = lo[0]; f[1] = lo[1]; f[2] = lo[2]; f[3] = lo[3];
  f[4] = hi[0]; f[5] = hi[1]; f[6] = hi[2]; f[7] = hi[3];
  return f;
}

// Saved chunk states (the backward's residuals): each chunk's P x N state as 16 x 16
// tiles (p-tile pr, n-tile nb) at element offset (pr * N/16 + nb) * 256, each tile in
// the MFMA accumulator order (lane l, register r hold p = 16 pr + l % 16, n = 16 nb +
// 4 (l / 16) + r), so that the state waves store whole 512-byte (bf16) rows of it.
template <int N>
__device__ __forceinline__ int saved_tile_off(int pr, int nb, int lane) {
  return (pr * (N / 16) + nb) * 256 + 4 * lane;
}
// (p, n) of the four consecutive elements at offset 4 q of a saved chunk state.
template <int N>
__device__ __forceinline__ void saved_pos(int q, int& p, int& n) {
  const int tile = q >> 6, ln = q & 63;
  p = 16 * (tile / (N / 16)) + (ln & 15);
  n = 16 * (tile % (N / 16)) + 4 * (ln >> 4);
}

// Store 4 consecutive elements (8 bytes bf16, 16 bytes f32).
__device__ __forceinline__ void store4(bf16* p, const float* f) {
  bf16x4 v;
  v[0] = (bf16)f[0]; v[1] = (bf16)f[1]; v[2] = (bf16)f[2]; v[3] = (bf16)f[3];
  *reinterpret_cast<bf16x4*>(p) = v;
}
__device__ __forceinline__ void store4(float* p, const float* f) {
  *reinterpret_cast<float4*>(p) = make_float4(f[0], f[1], f[2], f[3]);
}
__device__ __forceinline__ void load4(const bf16* p, float* f) {
  const bf16x4 v = *reinterpret_cast<const bf16x4*>(p);
  f[0] = (float)v[0]; f[1] = (float)v[1]; f[2] = (float)v[2]; f[3] = (float)v[3];
}
__device__ __forceinline__ void load4(const float* p, float* f) {
  const float4 v = *reinterpret_cast<const float4*>(p);
  f[0] = v.x; f[1] = v.y; f[2] = v.z; f[3] = v.w;
}

// Two values to two 16-bit (or 32-bit) slots: one packed conversion, then the low and
// high halves written separately.
__device__ __forceinline__ void store_pair(bf16* p0, bf16* p1, float a, float b) {
  const bf16x2 v = {(bf16)a, (bf16)b};
  *p0 = v[0];
  *p1 = v[1];
}
__device__ __forceinline__ void store_pair(float* p0, float* p1, float a, float b) {
  *p0 = a;
  *p1 = b;
}

// 16x16 MFMA tiles: v_mfma_f32_16x16x32_bf16 (KPL = 8) and v_mfma_f32_16x16x4_f32
// (KPL = 1).  A: lane i holds row i%16, k = (i/16)*KPL + [0,KPL); B: col i%16, same k;
// C: lane i, reg r holds col i%16, row 4*(i/16) + r (verified lane layouts).
template <typename T> struct MF16;
// Operand access for the chunk kernel's MFMAs.  Q and K rows are stored in natural
// column order; V stays in its staged (swizzled) [token][p] rows and is read with
// transposed LDS reads, as is K for the state update, so no transposed copy is built.
template <> struct MF16<bf16> {
  static constexpr int KSTEP = 32;
  typedef bf16x8 frag;
  // B operand of Q h^T for state rows [32q, 32q + 32): the lane's regs of tiles 2q, 2q+1
  // (rows 32q + 4g + r and 32q + 16 + 4g + r, g = lane/16)
  __device__ __forceinline__ static frag hfrag(const f32x4& a, const f32x4& b) {
    frag f;
    f[0] = (bf16)a[0]; f[1] = (bf16)a[1]; f[2] = (bf16)a[2]; f[3] = (bf16)a[3];
    f[4] = (bf16)b[0]; f[5] = (bf16)b[1]; f[6] = (bf16)b[2]; f[7] = (bf16)b[3];
    return f;
  }
  __device__ __forceinline__ static f32x4 mma(frag a, frag b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
  }
  __device__ __forceinline__ static frag ld(const bf16* buf, int ldm, int row0, int k0, int lane) {
    return *reinterpret_cast<const bf16x8*>(buf + (row0 + (lane & 15)) * ldm + k0 + (lane >> 4) * 8);
  }
  // A operand of Q h^T: row row0 + lane%16, the columns matching hfrag's state rows
  __device__ __forceinline__ static frag qoff(const bf16* buf, int ldm, int row0, int k0, int lane) {
    const bf16* r = buf + (row0 + (lane & 15)) * ldm + k0 + 4 * (lane >> 4);
    const bf16x4 lo = *reinterpret_cast<const bf16x4*>(r);
    const bf16x4 hi = *reinterpret_cast<const bf16x4*>(r + 16);
    frag f;
    f[0] = lo[0]; f[1] = lo[1]; f[2] = lo[2]; f[3] = lo[3];
    f[4] = hi[0]; f[5] = hi[1]; f[6] = hi[2]; f[7] = hi[3];
    return f;
  }
  // steps over a pair of 16-row S^T tiles (32 values of s): slots 0..3 are the
  // first tile's regs (s = 4(lane/16) + 0..3), slots 4..7 the second's (s + 16)
  static constexpr int STEPS = 1;
  __device__ __forceinline__ static frag from_acc(const f32x4& c0, const f32x4& c1, int) {
    frag f;
    f[0] = (bf16)c0[0]; f[1] = (bf16)c0[1]; f[2] = (bf16)c0[2]; f[3] = (bf16)c0[3];
    f[4] = (bf16)c1[0]; f[5] = (bf16)c1[1]; f[6] = (bf16)c1[2]; f[7] = (bf16)c1[3];
    return f;
  }
  // B operand of M V (k = token, matching from_acc's slots), column p0 + lane%16
  template <int S>
  __device__ __forceinline__ static frag vdiag(const uint4* rv, int p0, int s0, int, int lane) {
    const int g4 = 4 * (lane >> 4);
    return staged_tr<S>(rv, s0 + g4, s0 + 16 + g4, p0, lane);
  }
  // B operand of K^T V (k = token t0 + 8(lane/16) + 0..7), column p0 + lane%16
  template <int S>
  __device__ __forceinline__ static frag vstate(const uint4* rv, int p0, int t0, int lane) {
    const int t = t0 + 8 * (lane >> 4);
    return staged_tr<S>(rv, t, t + 4, p0, lane);
  }
  // A operand of K^T V: rows n0 + lane%16 of K^T from the [token][n] rows
  __device__ __forceinline__ static frag kstate(const bf16* k, int ldq, int t0, int n0, int lane) {
    return ld_tr(k, ldq, t0, n0, lane);
  }
  // the per-token weights of vstate's k-slots (WN per lane, tokens from ktok), and
  // the scaling of a fragment by them
  static constexpr int WN = 8;
  __device__ __forceinline__ static int ktok(int t0, int lane) { return t0 + 8 * (lane >> 4); }
  __device__ __forceinline__ static void load_w(const float* w, float out[WN]) {
    const float4 a = *reinterpret_cast<const float4*>(w);
    const float4 b = *reinterpret_cast<const float4*>(w + 4);
    out[0] = a.x; out[1] = a.y; out[2] = a.z; out[3] = a.w;
    out[4] = b.x; out[5] = b.y; out[6] = b.z; out[7] = b.w;
  }
  __device__ __forceinline__ static frag scale(frag v, const float w[WN]) {
    frag f;
#pragma unroll
    for (int j = 0; j < 8; ++j) f[j] = (bf16)((float)v[j] * w[j]);
    return f;
  }
};
template <> struct MF16<float> {
  static constexpr int KSTEP = 4;
  typedef float frag;
  __device__ __forceinline__ static f32x4 mma(frag a, frag b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
  }
  __device__ __forceinline__ static frag ld(const float* buf, int ldm, int row0, int k0, int lane) {
    return buf[(row0 + (lane & 15)) * ldm + k0 + (lane >> 4)];
  }
  // step j (0..7) over a pair of tiles: j < 4 uses the first tile's reg j
  // (s = 4(lane/16) + j), j >= 4 the second's reg j-4 (s + 16)
  static constexpr int STEPS = 8;
  __device__ __forceinline__ static frag from_acc(const f32x4& c0, const f32x4& c1, int j) {
    return j < 4 ? c0[j] : c1[j - 4];
  }
  template <int S>
  __device__ __forceinline__ static frag vdiag(const uint4* rv, int p0, int s0, int j, int lane) {
    return *staged_elem<S, float>(rv, s0 + 4 * (lane >> 4) + (j & 3) + (j >= 4 ? 16 : 0), p0 + (lane & 15));
  }
  template <int S>
  __device__ __forceinline__ static frag vstate(const uint4* rv, int p0, int t0, int lane) {
    return *staged_elem<S, float>(rv, t0 + (lane >> 4), p0 + (lane & 15));
  }
  __device__ __forceinline__ static frag kstate(const float* k, int ldq, int t0, int n0, int lane) {
    return ld_tr(k, ldq, t0, n0, lane);
  }
  static constexpr int WN = 1;
  __device__ __forceinline__ static int ktok(int t0, int lane) { return t0 + (lane >> 4); }
  __device__ __forceinline__ static void load_w(const float* w, float out[WN]) { out[0] = w[0]; }
  __device__ __forceinline__ static frag scale(frag v, const float w[WN]) { return v * w[0]; }
};

}  // namespace m3
