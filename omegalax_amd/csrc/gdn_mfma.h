// MFMA fragment helpers for gfx950 (CDNA4), v_mfma_f32_16x16x32_bf16.
//
// Lane layout of the 16x16x32 bf16 MFMA (verified on MI355X by comparing a GPU
// product of small integers with the CPU product): with q = lane / 16 and
// r = lane % 16,
//   A (16 x 32):  lane holds A[r][8q .. 8q+7]
//   B (32 x 16):  lane holds B[8q .. 8q+7][r]
//   C (16 x 16):  lane holds C[4q + v][r], v = 0..3
// Both operands are therefore read as "row r, 8 contiguous contraction
// elements": A from a row-major [i][k] array and B from a [j][k] (transposed)
// array.  Every LDS operand array in the kernels uses that layout.
#pragma once

#include "gdn_common.h"

namespace omx {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
typedef unsigned int u32x2 __attribute__((ext_vector_type(2)));

__device__ __forceinline__ f32x4 mma16(u32x4 a, u32x4 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, a),
                                                  __builtin_bit_cast(bf16x8_t, b), c, 0, 0, 0);
}

__device__ __forceinline__ f32x4 zero4() { return f32x4{0.f, 0.f, 0.f, 0.f}; }

__device__ __forceinline__ int lane_id() { return threadIdx.x & 63; }

// Operand fragment from a bf16 array with row stride `ld` (elements): row
// row0 + lane%16, contraction elements k0 + 8*(lane/16) .. +7.  16-byte aligned.
__device__ __forceinline__ u32x4 frag_bf16(const bf16_t* base, int ld, int row0, int k0) {
  const int l = lane_id();
  return *(const u32x4*)(base + (row0 + (l & 15)) * ld + k0 + 8 * (l >> 4));
}

__device__ __forceinline__ unsigned pack2(bf16_t lo, bf16_t hi) {
  return (unsigned)lo | ((unsigned)hi << 16);
}

// Split 8 floats into bf16 hi and lo parts (x = hi + lo to ~2^-16 relative).
__device__ __forceinline__ void split8(const float* x, u32x4& hi, u32x4& lo) {
  bf16_t h[8], l8[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    h[e] = f2bf(x[e]);
    l8[e] = f2bf(x[e] - bf2f(h[e]));
  }
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    hi[e] = pack2(h[2 * e], h[2 * e + 1]);
    lo[e] = pack2(l8[2 * e], l8[2 * e + 1]);
  }
}

// Store a C fragment transposed as bf16 into a [col][row] array (row stride ld):
// the lane's 4 values (rows 4q..4q+3 of the tile) are contiguous there.
__device__ __forceinline__ void store_ct_bf16(bf16_t* base, int ld, int row0, int col0, f32x4 c) {
  const int l = lane_id();
  u32x2 w;
  w[0] = pack2(f2bf(c[0]), f2bf(c[1]));
  w[1] = pack2(f2bf(c[2]), f2bf(c[3]));
  *(u32x2*)(base + (col0 + (l & 15)) * ld + row0 + 4 * (l >> 4)) = w;
}

// As store_ct_bf16, storing hi and lo parts into two arrays.
__device__ __forceinline__ void store_ct_split(bf16_t* hi, bf16_t* lo, int ld, int row0, int col0,
                                               f32x4 c) {
  const int l = lane_id();
  bf16_t h[4], r[4];
#pragma unroll
  for (int v = 0; v < 4; ++v) {
    h[v] = f2bf(c[v]);
    r[v] = f2bf(c[v] - bf2f(h[v]));
  }
  const int off = (col0 + (l & 15)) * ld + row0 + 4 * (l >> 4);
  *(u32x2*)(hi + off) = u32x2{pack2(h[0], h[1]), pack2(h[2], h[3])};
  *(u32x2*)(lo + off) = u32x2{pack2(r[0], r[1]), pack2(r[2], r[3])};
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
