// Shared definitions of the two chunked-prefill kernels: the chunk-parallel
// preparation kernel (gdn_prep.hip) and the recurrent scan (gdn_chunk.hip).
//
// The preparation kernel writes, for every (chunk, value head), a record that
// the scan reads back in one piece:
//   T diag(beta), with T = (I + L)^-1 the inverse of the chunk's unit lower-triangular
//       system (deltanet.py:100-113), as bf16 hi + lo MFMA A-operand fragments;
//   P = lower(scale (q_i . k_j) e^{G_i - G_j}) (deltanet.py:130-131), bf16 (hi + lo
//       for fp32 inputs), as A-operand fragments;
//   the gate vectors e^G, scale e^G, e^{G_last - G} and beta (fp32).
// The 64x64 lower-triangular T and P are stored as 16x32 A operands of the
// 16x16x32 MFMA whose contraction runs over two 16-token blocks 2p, 2p+1: for
// row block i and block pair p <= i/2, lane (q, r) = (lane / 16, lane % 16)
// holds 16 bytes, M[16i + r][32p + 4q .. +3] then M[16i + r][32p + 16 + 4q .. +3]
// (the 16x16 tiles (i, 2p) and (i, 2p+1), each in the 16x16x16 A layout).  The
// contraction order matches a B operand built from two C-layout tiles of the
// right-hand side.  The upper tiles (0, 1) and (2, 3) that complete the pairs of
// row blocks 0 and 2 are stored as zeros.  Six pairs, 1 KiB each, lanes in order.
#pragma once

#include "gdn_common.h"
#include "gdn_kernels.h"
#include "gdn_mfma.h"

namespace omx {

constexpr int kC = 64;      // chunk length (deltanet.py:59)
constexpr int kNT = 256;    // threads per workgroup in both kernels
constexpr int kLDT = kC + 8;   // row stride (elements) of 64-wide bf16 LDS arrays
constexpr int kLDD = 16 + 4;   // row stride of 16-wide LDS arrays
constexpr int MODE_BF16 = kModeBF16, MODE_F32 = kModeF32, MODE_LAYER = kModeLayer;

// record layout (bytes)
constexpr int kPairBytes = 64 * 16;            // one 16x32 A operand, all lanes
constexpr int kNPairs = 6;                     // (i, p): (0,0) (1,0) (2,0) (2,1) (3,0) (3,1)
constexpr int kRecT = 0;                       // 6 pairs x {hi, lo}
constexpr int kRecP = kRecT + 2 * kNPairs * kPairBytes;  // 6 pairs (hi)
constexpr int kRecG = kRecP + kNPairs * kPairBytes;      // 4 x 64 fp32 gate vectors
constexpr int kRecPL = kRecG + 4 * kC * 4;               // fp32 inputs, backward: P lo parts
constexpr int kRecBytesBF16 = kRecPL;                    // 19456
constexpr int kRecBytesF32 = kRecPL + kNPairs * kPairBytes;  // 25600
// rows of the gate block: e^G, scale e^G, e^{G_last - G} (its last entry, always 1, is
// replaced by e^{G_last}), beta
constexpr int kGateEG = 0, kGateEGS = 1, kGateEL = 2, kGateBeta = 3;

// backward extras per (chunk slot, value head), fp32 row-major 64x64 matrices:
// X^T (X = (I + L)^-1, upper triangular as stored), Lg = strict_lower(K K^T * Gamma)
// (L = diag(beta) Lg), P, then G.  Lg and P are written for fp32 inputs only: with bf16
// inputs the backward kernels form the Lg and P tiles they need from K, Q and G
constexpr int kXlpgMat = kC * kC;
constexpr int kXlpgX = 0, kXlpgLg = kXlpgMat, kXlpgP = 2 * kXlpgMat, kXlpgG = 3 * kXlpgMat;
constexpr int kXlpgFloats = 3 * kXlpgMat + kC;
static_assert(kXlpgFloats == kXlpgFloatsHost, "backward extras layout");

// Layer mode with dk = 128 (the scan's direct-load path): the value channels' conv +
// SiLU runs in the scan's helper wavefronts, so the prep forms the q and k rows only.
__host__ __device__ constexpr bool layer_v_in_scan(int dk) { return dk == 128; }

// Backward records (the recompute's prep and scan) carry P's lo parts with either input
// dtype: the layer backward's o, whose norm adjoint divides by its row RMS, is formed from
// split operands there.
__host__ __device__ constexpr int rec_bytes(int mode, bool bwd = false) {
  return mode == MODE_F32 || bwd ? kRecBytesF32 : kRecBytesBF16;
}
// base + off bytes; a uniform 64-bit base plus a 32-bit lane offset is one
// scalar-base memory instruction with no per-lane 64-bit address arithmetic
template <class T>
__device__ __forceinline__ T* at_bytes(T* base, unsigned off) {
  return (T*)((unsigned char*)base + off);
}
template <class T>
__device__ __forceinline__ const T* at_bytes(const T* base, unsigned off) {
  return (const T*)((const unsigned char*)base + off);
}


// index of the block pair (i, p), p <= i / 2
__host__ __device__ constexpr int pair_index(int i, int p) { return i + (i == 3) + p; }
// byte offsets of 16x16 tile (i, j), j <= i + (i even), in the record: its pair's
// 16 bytes per lane, first or second 8 (add 16 lane).  T lo parts follow T hi by one
// pair; P lo parts (fp32 inputs) sit at kRecPL - kRecP further.
__host__ __device__ constexpr int rec_t_off(int i, int j) {
  return kRecT + 2 * pair_index(i, j >> 1) * kPairBytes + 8 * (j & 1);
}
__host__ __device__ constexpr int rec_p_off(int i, int j) {
  return kRecP + pair_index(i, j >> 1) * kPairBytes + 8 * (j & 1);
}
// index of 16x16 tile (bi, bj), bj <= bi, of a lower-triangular 64x64 matrix
__host__ __device__ constexpr int tile_index(int bi, int bj) { return bi * (bi + 1) / 2 + bj; }

template <bool AS, bool BS>
__device__ __forceinline__ f32x4 mm(f32x4 acc, u32x4 ah, u32x4 al, u32x4 bh, u32x4 bl) {
  acc = mma16(ah, bh, acc);
  if constexpr (BS) acc = mma16(ah, bl, acc);
  if constexpr (AS) acc = mma16(al, bh, acc);
  return acc;
}

// acc += (ah + al)(bh + bl) without the lo*lo term, 16x16x16
__device__ __forceinline__ f32x4 mm3k16(f32x4 acc, u32x2 ah, u32x2 al, u32x2 bh, u32x2 bl) {
  acc = mma16k16(ah, bh, acc);
  acc = mma16k16(ah, bl, acc);
  acc = mma16k16(al, bh, acc);
  return acc;
}

template <bool SPLIT>
__device__ __forceinline__ void frag2(const bf16_t* base, int lo_off, int ld, int row0, int k0,
                                      u32x4& hi, u32x4& lo) {
  hi = frag_bf16(base, ld, row0, k0);
  if constexpr (SPLIT) lo = frag_bf16(base + lo_off, ld, row0, k0);
  else lo = hi;
}

// bf16 hi and lo parts of a C-layout tile, packed as a 16x16x16 B operand
__device__ __forceinline__ u32x2 pack_hi4(f32x4 x) {
  return u32x2{pack_bf16(x[0], x[1]), pack_bf16(x[2], x[3])};
}
__device__ __forceinline__ u32x2 pack_lo4(f32x4 x) {
  const u32x2 h = pack_hi4(x);
  return u32x2{pack_lo_pair(x[0], x[1], h[0]), pack_lo_pair(x[2], x[3], h[1])};
}

// Sum of n = 1, 2 or 4 consecutive 16-column partials as the pairwise tree ((a0 + a1) +
// (a2 + a3)) that a butterfly over the partials of a row forms, so that a row's total is
// the same however many partials a workgroup adds up first.
template <int N>
__device__ __forceinline__ float ss_tree(const float* a) {
  if constexpr (N == 1) return a[0];
  else if constexpr (N == 2) return a[0] + a[1];
  else return (a[0] + a[1]) + (a[2] + a[3]);
}

// Sums of squares of the rows of four 16x16 tiles held transposed (lane (q, r) holds
// row r, columns 4q .. 4q+3 of tile i in x[i]), reduce-scattered over the four lane rows
// of the wavefront (q = 0..3) so that lane (q, r) returns the sum of row r of tile q.
// Two cross-row swaps, no LDS traffic: v_permlane32_swap exchanges the upper 32 lanes of
// its first operand with the lower 32 lanes of its second, so after swapping (a, b) the
// two results summed give, in lanes q < 2, a's sum over rows q and q + 2 and, in lanes
// q >= 2, b's; v_permlane16_swap does the same for odd and even 16-lane rows.
// The four squares are summed by an explicit fma chain: written as a + b + c + d, the
// compiler may contract the first sum either way round (fma(x0, x0, x1^2) or
// fma(x1, x1, x0^2)), differently in different kernels, and the scans that fuse the
// norm must give the statistic of the ones that leave it to the epilogue kernel.
__device__ __forceinline__ float row_sq_scatter(const f32x4* x) {
  float ss[4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
    ss[i] = __builtin_fmaf(x[i][3], x[i][3],
                           __builtin_fmaf(x[i][2], x[i][2], __builtin_fmaf(x[i][1], x[i][1], x[i][0] * x[i][0])));
  const auto s02 = __builtin_amdgcn_permlane32_swap(__float_as_uint(ss[0]), __float_as_uint(ss[2]),
                                                    false, false);
  const auto s13 = __builtin_amdgcn_permlane32_swap(__float_as_uint(ss[1]), __float_as_uint(ss[3]),
                                                    false, false);
  // lanes q < 2: tiles 0 and 1 summed over rows q, q + 2; lanes q >= 2: tiles 2 and 3
  const float k0 = __uint_as_float(s02[0]) + __uint_as_float(s02[1]);
  const float k1 = __uint_as_float(s13[0]) + __uint_as_float(s13[1]);
  const auto t = __builtin_amdgcn_permlane16_swap(__float_as_uint(k0), __float_as_uint(k1), false,
                                                  false);
  return __uint_as_float(t[0]) + __uint_as_float(t[1]);
}

// unpack 8 input values (bf16 or fp32) from raw load words
template <bool F32>
__device__ __forceinline__ void unpack8(const u32x4* w, float* x) {
  if constexpr (F32) {
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      x[e] = __uint_as_float(w[0][e]);
      x[4 + e] = __uint_as_float(w[1][e]);
    }
  } else {
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      x[2 * e] = __uint_as_float(w[0][e] << 16);
      x[2 * e + 1] = __uint_as_float(w[0][e] & 0xffff0000u);
    }
  }
}

template <bool F32, class I>
__device__ __forceinline__ void load_raw(const void* base, I elem, u32x4* w) {
  if constexpr (F32) {
    const u32x4* p = (const u32x4*)((const float*)base + elem);
    w[0] = p[0];
    w[1] = p[1];
  } else {
    w[0] = *(const u32x4*)((const bf16_t*)base + elem);
  }
}

// 8 values -> packed bf16 words (hi, or the lo parts)
__device__ __forceinline__ u32x4 pack8(const float* x) {
  return u32x4{pack_bf16(x[0], x[1]), pack_bf16(x[2], x[3]), pack_bf16(x[4], x[5]),
               pack_bf16(x[6], x[7])};
}
__device__ __forceinline__ u32x4 pack8_lo(const float* x) {
  const u32x4 h = pack8(x);
  return u32x4{pack_lo_pair(x[0], x[1], h[0]), pack_lo_pair(x[2], x[3], h[1]),
               pack_lo_pair(x[4], x[5], h[2]), pack_lo_pair(x[6], x[7], h[3])};
}

// Sequence n's token range [s0, s1): packed by cu_seqlens (clamped to [0, T], so a
// malformed offsets array cannot index out of bounds) or batch row n.
__device__ __forceinline__ void seq_range(const int32_t* cu, int n, int T, long long& s0,
                                          long long& s1) {
  if (cu) {
    const long long lo = cu[n], hi = cu[n + 1];
    s0 = lo < 0 ? 0 : (lo > T ? T : lo);
    s1 = hi < s0 ? s0 : (hi > T ? T : hi);
  } else {
    s0 = (long long)n * T;
    s1 = s0 + T;
  }
}

// Work item of a workgroup of the scans (forward and reverse): sequence n, value head h
// and column block blk, from blockIdx.x.  The workgroups of one key head of one sequence
// (gqa value heads x nb blocks, which read the same q/k rows) form a group that runs on
// one XCD (the hardware deals workgroup i to XCD i % 8), so they share its L2.  When the
// group count is a multiple of 8, group ranks are dealt round-robin over the XCDs in the
// order of `order` (sequences longest first; null = index order): every XCD gets a share
// of every sequence and starts its longest chains first.  Otherwise each XCD takes a
// contiguous range of groups in index order.
struct ScanItem {
  int n, h, blk;
};
__device__ __forceinline__ ScanItem scan_item(const int32_t* order, int N, int Hk, int Hv,
                                              int nb) {
  const int gqa = Hv / Hk, G = gqa * nb, NG = N * Hk;
  const unsigned b = blockIdx.x, xcd = b % 8, slot = b / 8;
  int grp, member;
  if (NG % 8 == 0) {
    grp = 8 * (int)(slot / G) + (int)xcd;
    member = (int)(slot % G);
  } else {
    const unsigned nwg = gridDim.x, per = nwg / 8, rem = nwg % 8;
    const int wid = (int)(xcd * per + (xcd < rem ? xcd : rem) + slot);
    grp = wid / G;
    member = wid % G;
  }
  const int sr = grp / Hk;
  ScanItem it;
  it.n = order ? order[sr] : sr;
  it.h = (grp % Hk) * gqa + member / nb;
  it.blk = member % nb;
  return it;
}

}  // namespace omx
