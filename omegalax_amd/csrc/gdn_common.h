// Shared device helpers for the gfx950 GatedDeltaNet kernels.
//
// bf16 values travel as raw uint16_t; conversions round to nearest even, which
// is what a float32 -> bfloat16 cast does in the reference (jnp.astype).
// gfx950 converts in hardware (v_cvt_pk_bf16_f32).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace omx {

typedef uint16_t bf16_t;

__device__ __forceinline__ float bf2f(bf16_t h) { return __uint_as_float((uint32_t)h << 16); }

// float -> bf16, round to nearest even (one v_cvt_pk_bf16_f32 on gfx950)
__device__ __forceinline__ bf16_t f2bf(float f) { return __builtin_bit_cast(bf16_t, (__bf16)f); }

typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));

// two floats -> packed bf16 pair (first in the low half), one instruction on gfx950
__device__ __forceinline__ uint32_t pack_bf16(float lo, float hi) {
  return __builtin_bit_cast(uint32_t, bf16x2_t{(__bf16)lo, (__bf16)hi});
}

__device__ __forceinline__ float round_bf(float f) { return bf2f(f2bf(f)); }

// Buffer resource over `bytes` bytes at p (raw, stride 0): accesses through it take a
// 32-bit lane offset and a uniform scalar offset, with no per-lane address arithmetic.
// Loads at offsets past `bytes` return zeros and stores there are dropped, without a
// memory access: a range of 0 turns every access through the resource into a no-op.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t buf_rsrc(const void* p, unsigned bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(p), (short)0, (int)bytes, 0x00020000);
}

// Workgroup barrier that orders LDS accesses only: it does not wait for the wave's
// outstanding global loads and stores (__syncthreads does), so prefetches and result
// stores stay in flight across it.
__device__ __forceinline__ void lds_barrier() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

// bf16 lo parts of two floats whose bf16 hi parts are packed in h: (x0 - hi0, x1 - hi1)
// rounded to bf16.  Each difference is one bf16 dot product, x_k + (-1) hi_k + 0: the
// products are exact and the difference of two close floats is exact.
// The selectors (-1, 0) and (0, -1) are held in scalar registers: an inline float
// constant in a packed bf16 operand does not mean the bf16 pair.
__device__ __forceinline__ uint32_t pack_lo_pair(float x0, float x1, uint32_t h) {
  uint32_t m0, m1;
  asm("" : "=s"(m0) : "0"(0x0000BF80u));  // bf16 (-1, 0)
  asm("" : "=s"(m1) : "0"(0xBF800000u));  // bf16 (0, -1)
  const bf16x2_t hb = __builtin_bit_cast(bf16x2_t, h);
  const float l0 = __builtin_amdgcn_fdot2_f32_bf16(hb, __builtin_bit_cast(bf16x2_t, m0), x0, false);
  const float l1 = __builtin_amdgcn_fdot2_f32_bf16(hb, __builtin_bit_cast(bf16x2_t, m1), x1, false);
  return pack_bf16(l0, l1);
}

// w0 x0 + w1 x1 + w2 x2 + w3 x3 for bf16 weights and inputs held as packed pairs
// (w01 = (w0, w1), x01 = (x0, x1), ...), as two bf16 dot products (v_dot2_f32_bf16):
// the products are exact in fp32 and the sums are fp32.  The causal conv's tap sum, with
// x_d the input d tokens back and w_d its weight.
__device__ __forceinline__ float dot4_bf16(uint32_t w01, uint32_t w23, uint32_t x01,
                                           uint32_t x23) {
  const float s23 = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, x23),
                                                    __builtin_bit_cast(bf16x2_t, w23), 0.f, false);
  return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, x01),
                                         __builtin_bit_cast(bf16x2_t, w01), s23, false);
}

// Index of the partial sum of squares of (token t, value head h, 16-column slice s) in the
// layer prefill's [ceil(tokens / 64)][Hv][S][64] array (S slices per row): the 64 tokens
// of a block are contiguous for each (head, slice).
__device__ __forceinline__ long long ss_index(long long t, int h, int s, int Hv, int S) {
  return (((t >> 6) * Hv + h) * S + s) * 64 + (t & 63);
}

__device__ __forceinline__ float sigmoidf_(float x) { return 1.0f / (1.0f + __expf(-x)); }

// log(1 + e^x), the softplus of jax.nn.softplus; exact branch for large x.
__device__ __forceinline__ float softplusf_(float x) { return x > 20.0f ? x : log1pf(expf(x)); }

__device__ __forceinline__ float siluf_(float x) { return x / (1.0f + expf(-x)); }

// SiLU from the hardware exp2 and reciprocal (v_exp_f32, v_rcp_f32; about 2 ulp in
// fp32) for values that are rounded to bf16 or feed a bf16 output right after.
// Finite inputs only (x = -inf would give -inf * 0).
__device__ __forceinline__ float silu_fast(float x) {
  return x * __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(x * -1.4426950408889634f));
}

// Sum over the 64 lanes of a wavefront.
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}

// Sum over aligned groups of `width` lanes (width a power of two <= 64).
template <int WIDTH>
__device__ __forceinline__ float group_sum(float v) {
#pragma unroll
  for (int o = WIDTH / 2; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}

// lane permutation within rows of 16 lanes by a DPP control word (no LDS traffic)
template <int CTRL>
__device__ __forceinline__ float dpp_f(float v) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xf, 0xf, false));
}

// Sum over aligned groups of WIDTH (4, 8 or 16) lanes with DPP butterflies:
// quad_perm [1,0,3,2] and [2,3,0,1] sum each quad; row_half_mirror pairs the two
// quads of each 8-lane half; row_mirror pairs the two halves of each 16-lane row.
template <int WIDTH>
__device__ __forceinline__ float group_sum_dpp(float v) {
  static_assert(WIDTH == 4 || WIDTH == 8 || WIDTH == 16, "dpp group width");
  v += dpp_f<0xB1>(v);
  v += dpp_f<0x4E>(v);
  if constexpr (WIDTH >= 8) v += dpp_f<0x141>(v);
  if constexpr (WIDTH >= 16) v += dpp_f<0x140>(v);
  return v;
}

// DPP move restricted to the rows in ROW_MASK; other rows (and lanes whose source
// is outside the row) read 0.
template <int CTRL, int ROW_MASK>
__device__ __forceinline__ float dpp_rows(float v) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, ROW_MASK, 0xf, false));
}

// Inclusive prefix sum over the 64 lanes: shifts by 1, 2, 4, 8 within each row of
// 16 lanes, then lane 15 of rows 0 and 2 is added into rows 1 and 3 (row_bcast:15)
// and lane 31 into rows 2 and 3 (row_bcast:31).
__device__ __forceinline__ float wave_scan_dpp(float v) {
  v += dpp_rows<0x111, 0xf>(v);
  v += dpp_rows<0x112, 0xf>(v);
  v += dpp_rows<0x114, 0xf>(v);
  v += dpp_rows<0x118, 0xf>(v);
  v += dpp_rows<0x142, 0xa>(v);
  v += dpp_rows<0x143, 0xc>(v);
  return v;
}

}  // namespace omx
