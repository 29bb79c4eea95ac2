// MFMA fragment, LDS and lane-permute helpers shared by the chunked kernels
// (gfx950: v_mfma_f32_16x16x32_bf16, v_mfma_f32_16x16x4_f32, ds_read_b64_tr_b16).
//
// Operand conventions for the 16x16 MFMAs (lane l, q = l>>4, l16 = l&15):
//   A: row l16, 8 (bf16) or 1 (f32) k values of lane group q
//   B: column l16, the same k values
//   C/D: rows 4q+v (v = 0..3), column l16
// Only the A/B k assignment has to agree between the two operands, which lets a
// C-layout register tile serve directly as a B operand (see frag_perm/pack_b).
#pragma once
#include "common.hpp"

namespace hmx {

__device__ __forceinline__ f32x4 mfma16(bf16x8 a, bf16x8 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ f32x4 mfma16f(float a, float b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
}

// A (or B^T) fragment in natural k order: lane holds row r0+(l&15), k0+8(l>>4)..+7.
__device__ __forceinline__ bf16x8 frag(const bf16* base, int ld, int r0, int k0, int lane) {
  return *reinterpret_cast<const bf16x8*>(base + (r0 + (lane & 15)) * ld + k0 + 8 * (lane >> 4));
}

// A fragment whose k order matches a B operand built from two C-layout tiles:
// lane holds row r0+(l&15), k = k0+4q+{0..3} and k0+16+4q+{0..3}, q = l>>4.
__device__ __forceinline__ bf16x8 frag_perm(const bf16* base, int ld, int r0, int k0, int lane) {
  const bf16* p = base + (r0 + (lane & 15)) * ld + k0 + 4 * (lane >> 4);
  const bf16x4 a = *reinterpret_cast<const bf16x4*>(p);
  const bf16x4 b = *reinterpret_cast<const bf16x4*>(p + 16);
  return bf16x8{a[0], a[1], a[2], a[3], b[0], b[1], b[2], b[3]};
}

// Transposing LDS read (gfx950 ds_read_b64_tr_b16) of a row-major bf16 matrix
// M[row][col]: within each 16-lane group, lane i receives M[t0+j][c0+i] for
// j = 0..3 (4 consecutive rows of one column), where the group reads rows
// t0..t0+3 and columns c0..c0+15.  Each source lane s supplies the address of
// M[t0 + s/4][c0 + 4(s%4)].
typedef short s16x4 __attribute__((ext_vector_type(4)));
__device__ __forceinline__ bf16x4 ld_tr(const bf16* base, int ld, int t0, int c0, int lane) {
  const int s = lane & 15;
  const bf16* a = base + (t0 + (s >> 2)) * ld + c0 + 4 * (s & 3);
  const s16x4 r = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
      (__attribute__((address_space(3))) s16x4*)(a));
  return __builtin_bit_cast(bf16x4, r);
}

// B fragment of M[k=row][n=col] in natural k order (k = t0 + 8q + 0..7) from a
// row-major bf16 matrix: column c0 + (l&15).
__device__ __forceinline__ bf16x8 frag_t(const bf16* base, int ld, int t0, int c0, int lane) {
  const int tq = t0 + 8 * (lane >> 4);
  const bf16x4 a = ld_tr(base, ld, tq, c0, lane);
  const bf16x4 b = ld_tr(base, ld, tq + 4, c0, lane);
  return bf16x8{a[0], a[1], a[2], a[3], b[0], b[1], b[2], b[3]};
}

// A fragment of M^T (rows = columns of M, k = rows of M) in the permuted k
// order of frag_perm: k = t0+4q+{0..3} and t0+16+4q+{0..3}.
__device__ __forceinline__ bf16x8 frag_t_perm(const bf16* base, int ld, int t0, int c0, int lane) {
  const int tq = t0 + 4 * (lane >> 4);
  const bf16x4 a = ld_tr(base, ld, tq, c0, lane);
  const bf16x4 b = ld_tr(base, ld, tq + 16, c0, lane);
  return bf16x8{a[0], a[1], a[2], a[3], b[0], b[1], b[2], b[3]};
}

// B fragment from two vertically stacked C-layout 16x16 tiles (rows 0-15 in t0,
// rows 16-31 in t1); pairs with frag_perm.
__device__ __forceinline__ bf16x8 pack_b(const f32x4& t0, const f32x4& t1) {
  return bf16x8{(bf16)t0[0], (bf16)t0[1], (bf16)t0[2], (bf16)t0[3],
                (bf16)t1[0], (bf16)t1[1], (bf16)t1[2], (bf16)t1[3]};
}

// hi/lo split of two floats: hi = bf16(x) (one v_cvt_pk_bf16_f32), lo =
// bf16(x - hi), with hi widened back to fp32 exactly by a shift (low half) and
// a mask (high half) of the packed pair.  x ~= hi + lo to ~16 significant bits.
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
__device__ __forceinline__ void split2(float x0, float x1, bf16x2& hi, bf16x2& lo) {
  hi = bf16x2{(bf16)x0, (bf16)x1};
  const unsigned hb = __builtin_bit_cast(unsigned, hi);
  const float h0 = __builtin_bit_cast(float, hb << 16);
  const float h1 = __builtin_bit_cast(float, hb & 0xffff0000u);
  lo = bf16x2{(bf16)(x0 - h0), (bf16)(x1 - h1)};
}

// hi/lo split of the same pair: x ~= hi + lo with both in bf16.
__device__ __forceinline__ void pack_b_hilo(const f32x4& t0, const f32x4& t1, bf16x8& hi,
                                            bf16x8& lo) {
  bf16x2 h[4], l[4];
  split2(t0[0], t0[1], h[0], l[0]);
  split2(t0[2], t0[3], h[1], l[1]);
  split2(t1[0], t1[1], h[2], l[2]);
  split2(t1[2], t1[3], h[3], l[3]);
  hi = bf16x8{h[0][0], h[0][1], h[1][0], h[1][1], h[2][0], h[2][1], h[3][0], h[3][1]};
  lo = bf16x8{l[0][0], l[0][1], l[1][0], l[1][1], l[2][0], l[2][1], l[3][0], l[3][1]};
}

// Sum over the 16 lanes of a DPP row (VALU lane permutes, no LDS traffic).
__device__ __forceinline__ float row16_sum(float x) {
  auto dpp = [](float v, int ctrl) -> float {
    int r;
    switch (ctrl) {
      case 0: r = __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0xB1, 0xF, 0xF, false); break;
      case 1: r = __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x4E, 0xF, 0xF, false); break;
      case 2: r = __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x141, 0xF, 0xF, false); break;
      default: r = __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x140, 0xF, 0xF, false); break;
    }
    return __builtin_bit_cast(float, r);
  };
  x += dpp(x, 0);  // quad_perm [1,0,3,2]
  x += dpp(x, 1);  // quad_perm [2,3,0,1]
  x += dpp(x, 2);  // row_half_mirror
  x += dpp(x, 3);  // row_mirror
  return x;
}

// Maximum over the wave of non-negative floats (compared as their bit patterns,
// which order them; NaN and inf compare above every finite value): within each
// DPP row by lane permutes, then across the four rows in scalar registers.  The
// result is wave-uniform.
__device__ __forceinline__ float wave_max_nonneg(float x) {
  auto dpp = [](uint32_t v, int ctrl) -> uint32_t {
    int r;
    switch (ctrl) {
      case 0: r = __builtin_amdgcn_update_dpp(0, (int)v, 0xB1, 0xF, 0xF, false); break;
      case 1: r = __builtin_amdgcn_update_dpp(0, (int)v, 0x4E, 0xF, 0xF, false); break;
      case 2: r = __builtin_amdgcn_update_dpp(0, (int)v, 0x141, 0xF, 0xF, false); break;
      default: r = __builtin_amdgcn_update_dpp(0, (int)v, 0x140, 0xF, 0xF, false); break;
    }
    return (uint32_t)r;
  };
  uint32_t b = __builtin_bit_cast(uint32_t, x);
#pragma unroll
  for (int i = 0; i < 4; ++i) b = max(b, dpp(b, i));
  const uint32_t r0 = __builtin_amdgcn_readlane(b, 0), r1 = __builtin_amdgcn_readlane(b, 16);
  const uint32_t r2 = __builtin_amdgcn_readlane(b, 32), r3 = __builtin_amdgcn_readlane(b, 48);
  return __builtin_bit_cast(float, max(max(r0, r1), max(r2, r3)));
}

// The smallest e >= 0 with 2^-e m < 2^15 (m >= 0; inf and NaN act as 2^128):
// scaling operands bounded by m by 2^-e keeps them inside fp16's range with a
// factor-two margin, and the scaling is exact.  Integer work on a uniform m stays
// in scalar registers.
__device__ __forceinline__ int fp16_range_exp(float m) {
  const int k = (int)((__builtin_bit_cast(uint32_t, m) >> 23) & 0xff) - 126;   // m < 2^k
  return max(k, 15) - 15;
}
// 2^n as a float, for n in [-126, 127] (exact; no division or transcendental)
__device__ __forceinline__ float pow2f(int n) {
  return __builtin_bit_cast(float, (uint32_t)(127 + n) << 23);
}

// Inclusive prefix sum over lanes 0..31 (two DPP rows) with VALU lane shifts.
#define HMX_DPP_F(v, ctrl, rmask) \
  __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, (v)), (ctrl), \
                                                        (rmask), 0xF, true))
__device__ __forceinline__ float scan32(float x) {
  x += HMX_DPP_F(x, 0x111, 0xF);  // row_shr:1
  x += HMX_DPP_F(x, 0x112, 0xF);  // row_shr:2
  x += HMX_DPP_F(x, 0x114, 0xF);  // row_shr:4
  x += HMX_DPP_F(x, 0x118, 0xF);  // row_shr:8
  x += HMX_DPP_F(x, 0x142, 0xA);  // row_bcast:15 into rows 1 and 3
  return x;
}
#undef HMX_DPP_F

// ---------------------------------------------------------------------------
// fp16 operands (v_mfma_f32_16x16x32_f16 / 16x16x16f16, v_cvt_pk_f16_f32): the
// same fragment layouts as the bf16 helpers above, for 16-bit elements.
// ---------------------------------------------------------------------------
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ f32x4 mfma16h(f16x8 a, f16x8 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}

// 16x16x16: lane (q, l16) holds A[l16][4q..4q+3] and B[4q..4q+3][l16] - the C/D
// layout of a tile of A^T and of B, so C-layout tiles feed it directly.
__device__ __forceinline__ f32x4 mfma16h_k16(f16x4 a, f16x4 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x16f16(a, b, c, 0, 0, 0);
}

// round-to-nearest-even fp16 of a C-layout tile (two v_cvt_pk_f16_f32)
__device__ __forceinline__ f16x4 h4(const f32x4& x) {
  return f16x4{(f16)x[0], (f16)x[1], (f16)x[2], (f16)x[3]};
}

// operand from two vertically stacked C-layout tiles (k = 4q+v, then 16+4q+v)
__device__ __forceinline__ f16x8 h8(const f32x4& t0, const f32x4& t1) {
  return f16x8{(f16)t0[0], (f16)t0[1], (f16)t0[2], (f16)t0[3],
               (f16)t1[0], (f16)t1[1], (f16)t1[2], (f16)t1[3]};
}

template <typename T>
__device__ __forceinline__ f16x8 frag_h(const T* base, int ld, int r0, int k0, int lane) {
  return *reinterpret_cast<const f16x8*>(base + (r0 + (lane & 15)) * ld + k0 + 8 * (lane >> 4));
}

__device__ __forceinline__ f16x8 frag_perm_h(const f16* base, int ld, int r0, int k0, int lane) {
  const f16* p = base + (r0 + (lane & 15)) * ld + k0 + 4 * (lane >> 4);
  const f16x4 a = *reinterpret_cast<const f16x4*>(p);
  const f16x4 b = *reinterpret_cast<const f16x4*>(p + 16);
  return f16x8{a[0], a[1], a[2], a[3], b[0], b[1], b[2], b[3]};
}

__device__ __forceinline__ f16x4 ld_tr_h(const f16* base, int ld, int t0, int c0, int lane) {
  const int s = lane & 15;
  const f16* a = base + (t0 + (s >> 2)) * ld + c0 + 4 * (s & 3);
  const s16x4 r = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
      (__attribute__((address_space(3))) s16x4*)(a));
  return __builtin_bit_cast(f16x4, r);
}

__device__ __forceinline__ f16x8 frag_t_perm_h(const f16* base, int ld, int t0, int c0, int lane) {
  const int tq = t0 + 4 * (lane >> 4);
  const f16x4 a = ld_tr_h(base, ld, tq, c0, lane);
  const f16x4 b = ld_tr_h(base, ld, tq + 16, c0, lane);
  return f16x8{a[0], a[1], a[2], a[3], b[0], b[1], b[2], b[3]};
}

// Interleaved feature order for fp16 rows read as MFMA operands: within each
// 32-feature block, 4-feature chunk m of half h is stored at 8m + 4h.  One 128-bit
// read at 8q then returns features {4q..4q+3, 16+4q..16+4q+3}, the k order of a B
// operand built from two stacked C-layout tiles (frag_perm_h's order), which the
// natural order serves only with two 64-bit reads.  At a row stride of 72 dwords
// (8 mod 64 banks) these 128-bit row-fragment reads are bank-conflict-free.
__device__ __forceinline__ int icol(int f) {
  return (f & ~31) | ((f & 12) << 1) | ((f & 16) >> 2) | (f & 3);
}
// rows r0..r0+15 of an interleaved array, k = k0 + {4q+v, 16+4q+v}
__device__ __forceinline__ f16x8 frag_i(const f16* b, int ld, int r0, int k0, int lane) {
  return *reinterpret_cast<const f16x8*>(b + (r0 + (lane & 15)) * ld + k0 + 8 * (lane >> 4));
}
// frag_t_perm_h of an interleaved array: element (row c0 + l16, k) = b[t0 + k][c0 + l16]
__device__ __forceinline__ f16x4 ld_tr_i(const f16* b, int ld, int row, int c0, int lane) {
  const int s = lane & 15;
  const f16* a = b + (row + (s >> 2)) * ld + icol(c0 + 4 * (s & 3));
  const s16x4 r = __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) s16x4*)(a));
  return __builtin_bit_cast(f16x4, r);
}
__device__ __forceinline__ f16x8 frag_t_i(const f16* b, int ld, int t0, int c0, int lane) {
  const int tq = t0 + 4 * (lane >> 4);
  const f16x4 x = ld_tr_i(b, ld, tq, c0, lane);
  const f16x4 y = ld_tr_i(b, ld, tq + 16, c0, lane);
  return f16x8{x[0], x[1], x[2], x[3], y[0], y[1], y[2], y[3]};
}
// stores features f0..f0+7 (f0 a multiple of 8) of an interleaved row
__device__ __forceinline__ void store8_i(f16* row, int f0, const f16x8& y) {
  *reinterpret_cast<f16x4*>(row + icol(f0)) = f16x4{y[0], y[1], y[2], y[3]};
  *reinterpret_cast<f16x4*>(row + icol(f0 + 4)) = f16x4{y[4], y[5], y[6], y[7]};
}

// Workgroup barrier that orders LDS only: global loads issued before it stay in
// flight (the next chunk's prefetch), unlike __syncthreads().
__device__ __forceinline__ void lds_barrier() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}


}  // namespace hmx
