// MFMA fragment helpers for gfx950 (CDNA4) bf16 matrix cores.
//
// Lane layouts (verified on MI355X by comparing GPU products of small integers
// with the CPU product), with q = lane / 16 and r = lane % 16:
//   v_mfma_f32_16x16x32_bf16:  A[r][8q .. 8q+7],  B[8q .. 8q+7][r]
//   v_mfma_f32_16x16x16_bf16:  A[r][4q .. 4q+3],  B[4q .. 4q+3][r]
//   both:                      C[4q + v][r], v = 0..3
// Both operands are read as "row r, contiguous contraction elements": A from a
// row-major [i][k] array and B from a [j][k] (transposed) array.  Every LDS
// operand array in the kernels uses that layout.
#pragma once

#include "gdn_common.h"

namespace omx {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef short s16x4_t __attribute__((ext_vector_type(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
typedef unsigned int u32x2 __attribute__((ext_vector_type(2)));

// C += A(16x32) B(32x16)
__device__ __forceinline__ f32x4 mma16(u32x4 a, u32x4 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, a),
                                                  __builtin_bit_cast(bf16x8_t, b), c, 0, 0, 0);
}

// C += A(16x16) B(16x16)
__device__ __forceinline__ f32x4 mma16k16(u32x2 a, u32x2 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(__builtin_bit_cast(s16x4_t, a),
                                                    __builtin_bit_cast(s16x4_t, b), c, 0, 0, 0);
}

__device__ __forceinline__ f32x4 zero4() { return f32x4{0.f, 0.f, 0.f, 0.f}; }

__device__ __forceinline__ int lane_id() { return threadIdx.x & 63; }

// 16x32 operand fragment from a bf16 array with row stride `ld` (elements): row
// row0 + lane%16, contraction elements k0 + 8*(lane/16) .. +7.  16-byte aligned.
__device__ __forceinline__ u32x4 frag_bf16(const bf16_t* base, int ld, int row0, int k0) {
  const int l = lane_id();
  return *(const u32x4*)(base + (row0 + (l & 15)) * ld + k0 + 8 * (l >> 4));
}

// 16x16 operand fragment: row row0 + lane%16, elements k0 + 4*(lane/16) .. +3.
__device__ __forceinline__ u32x2 frag4_bf16(const bf16_t* base, int ld, int row0, int k0) {
  const int l = lane_id();
  return *(const u32x2*)(base + (row0 + (l & 15)) * ld + k0 + 4 * (l >> 4));
}

__device__ __forceinline__ float lo_part(float x) { return x - round_bf(x); }

// Transposed 16-bit LDS read (ds_read_b64_tr_b16).  Within each group of 16 lanes
// the lanes' 4-element rows (8 bytes at each lane's address) form a 16x4 block M,
// and lane 4a+b receives {M[a][b], M[a+4][b], M[a+8][b], M[a+12][b]} (mapping
// verified on MI355X).  Pointing source lane s at row base + s/4, column 4*(s%4)
// of a row-major array therefore hands each lane 4 consecutive rows of its own
// column: an MFMA operand whose contraction runs down the rows.
__device__ __forceinline__ u32x2 ds_read_tr(const bf16_t* p) {
  typedef __attribute__((address_space(3))) s16x4_t lds_s16x4;
  const s16x4_t v = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)p);
  return __builtin_bit_cast(u32x2, v);
}

// 16x32 operand whose contraction runs down the rows of a row-major [k][col]
// bf16 array (stride ld): lane (q, r) gets rows k0 + 8q .. +7 of column col0 + r.
__device__ __forceinline__ u32x4 frag_tr(const bf16_t* base, int ld, int k0, int col0) {
  const int l = lane_id(), q = l >> 4, s = l & 15;
  const bf16_t* p = base + (k0 + 8 * q + (s >> 2)) * ld + col0 + 4 * (s & 3);
  const u32x2 a = ds_read_tr(p), b = ds_read_tr(p + 4 * ld);
  return u32x4{a[0], a[1], b[0], b[1]};
}

// Four consecutive rows row0 + 4q .. +3 of column col0 + r (the MFMA C layout) of a
// row-major bf16 array, as 4 bf16 in two words.
__device__ __forceinline__ u32x2 rows4_tr(const bf16_t* base, int ld, int row0, int col0) {
  const int l = lane_id(), q = l >> 4, s = l & 15;
  return ds_read_tr(base + (row0 + 4 * q + (s >> 2)) * ld + col0 + 4 * (s & 3));
}

// Store a C fragment transposed as bf16 into a [col][row] array (row stride ld):
// the lane's 4 values (rows 4q..4q+3 of the tile) are contiguous there.
__device__ __forceinline__ void store_ct_bf16(bf16_t* base, int ld, int row0, int col0, f32x4 c) {
  const int l = lane_id();
  *(u32x2*)(base + (col0 + (l & 15)) * ld + row0 + 4 * (l >> 4)) =
      u32x2{pack_bf16(c[0], c[1]), pack_bf16(c[2], c[3])};
}

// As store_ct_bf16, storing hi and lo parts (c = hi + lo to ~2^-16) into two arrays.
__device__ __forceinline__ void store_ct_split(bf16_t* hi, bf16_t* lo, int ld, int row0, int col0,
                                               f32x4 c) {
  const int l = lane_id();
  const int off = (col0 + (l & 15)) * ld + row0 + 4 * (l >> 4);
  *(u32x2*)(hi + off) = u32x2{pack_bf16(c[0], c[1]), pack_bf16(c[2], c[3])};
  *(u32x2*)(lo + off) = u32x2{pack_bf16(lo_part(c[0]), lo_part(c[1])),
                              pack_bf16(lo_part(c[2]), lo_part(c[3]))};
}

// Order this wave's earlier LDS writes before its later LDS reads (lanes of one
// wave exchange data through LDS without a workgroup barrier).
__device__ __forceinline__ void wave_lds_fence() {
  __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0): this lane's LDS ops are complete
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

}  // namespace omx
