// Causal depthwise conv + SiLU of the layer's input rows (deltanet.py:35-50, 243), shared
// by the chunk preparation (q, k and, for dk < 128, v channels) and the direct-load scan
// (v channels with dk = 128), so both round every value at the same points.
#pragma once

#include "gdn_chunk.h"
#include "gdn_common.h"
#include "gdn_kernels.h"

namespace omx {

// conv weights of channels ch0..ch0+7, cast to bf16 as at deltanet.py:243, as packed
// pairs: wp[e][0] = (w_0, w_1), wp[e][1] = (w_2, w_3) with w_d the weight of the input d
// tokens back (tap K-1-d); taps beyond K are 0
__device__ __forceinline__ void load_conv_w(const ChunkParams& p, int chu, int chl, uint32_t (*wp)[2]) {
  const int K = p.conv_k;
  const int ch0 = chu + chl;
  if (K == 4) {  // uniform: each channel's taps are one 16-byte row
    const float* wb = p.conv_w + (size_t)chu * 4;  // uniform base, lane channel offset
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const float4 w = *(const float4*)at_bytes(wb, 16u * (unsigned)(chl + e));
      wp[e][0] = pack_bf16(w.w, w.z);
      wp[e][1] = pack_bf16(w.y, w.x);
    }
    return;
  }
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    const float* w = p.conv_w + (size_t)(ch0 + e) * K;
    float wt[4];
#pragma unroll
    for (int d = 0; d < 4; ++d) wt[d] = d < K ? w[K - 1 - d] : 0.f;
    wp[e][0] = pack_bf16(wt[0], wt[1]);
    wp[e][1] = pack_bf16(wt[2], wt[3]);
  }
}

// Raw input row of 8 channels at token t before the sequence start s0: the conv cache
// (oldest slot first), or zeros (deltanet.py:46).
__device__ __forceinline__ u32x4 conv_history(const ChunkParams& p, int n, long long s0, long long t,
                                              int ch0) {
  u32x4 w{0u, 0u, 0u, 0u};
  const int K = p.conv_k;
  const int slot = (K - 1) - (int)(s0 - t);
  if (p.conv_state_in && slot >= 0) {
    const unsigned short* cs =
        (const unsigned short*)p.conv_state_in + ((size_t)n * p.conv_dim + ch0) * (K - 1) + slot;
#pragma unroll
    for (int e = 0; e < 4; ++e)
      w[e] = (unsigned)cs[(2 * e) * (K - 1)] | ((unsigned)cs[(2 * e + 1) * (K - 1)] << 16);
  }
  return w;
}

// Causal depthwise conv + SiLU (deltanet.py:35-50, 243) of one 8-channel group over
// chunk rows r0 .. r0+ROWS-1, streaming down the rows.  conv_load issues every input
// row once (rows r0-3 .. r0+ROWS-1); conv_compute consumes them.  Inputs and weights
// are bf16 (the weights cast as the reference casts them), the tap sum is two bf16 dot
// products per channel with fp32 sums, and the sum and the SiLU output are rounded to
// bf16 like the reference's bf16 ops; rows at or past nvalid give zeros.
// emit(m, y) receives row r0 + m as 8 packed bf16 values.
template <int ROWS>
__device__ __forceinline__ void conv_load(const ChunkParams& p, int n, long long s0, long long t0,
                                          int nvalid, int r0, int chu, int chl, u32x4* raw) {
  // Every row is one unconditional load from mixed_qkv (rows before the sequence start
  // load its first row), so all of them are in flight together; the rows before the
  // start, which only the first 3 of a sequence's first chunk can be, are replaced after.
  const bf16_t* base = (const bf16_t*)p.mixed_qkv + chu + chl;
  const int first = (int)(s0 - t0 > -3 ? s0 - t0 : -3);  // first row inside the sequence
#pragma unroll
  for (int k = 0; k < ROWS + 3; ++k) {
    int row = r0 - 3 + k;
    row = row < nvalid ? row : nvalid - 1;  // padded rows: in bounds, zeroed below
    row = row > first ? row : first;
    raw[k] = *(const u32x4*)(base + (t0 + row) * p.conv_dim);
  }
  if (r0 - 3 < first) {
#pragma unroll
    for (int k = 0; k < 3; ++k)
      if (r0 - 3 + k < first) raw[k] = conv_history(p, n, s0, t0 + r0 - 3 + k, chu + chl);
  }
}

// The pairs (x_t, x_{t-1}) of the 8 channels from input rows t (cur) and t-1 (prev):
// word c of pe holds channel 2c's pair, word c of po channel 2c+1's (v_perm_b32).
__device__ __forceinline__ void time_pairs(const u32x4& cur, const u32x4& prev, u32x4& pe, u32x4& po) {
#pragma unroll
  for (int c = 0; c < 4; ++c) {
    pe[c] = __builtin_amdgcn_perm(prev[c], cur[c], 0x05040100u);
    po[c] = __builtin_amdgcn_perm(prev[c], cur[c], 0x07060302u);
  }
}

template <int ROWS, class Emit>
__device__ __forceinline__ void conv_compute(const u32x4* raw, const uint32_t (*wp)[2], int nvalid,
                                             int r0, Emit emit) {
  // time pairs of rows m-2 and m-1 (a row's pair holds it and the row before)
  u32x4 pe2, po2, pe1, po1;
  time_pairs(raw[1], raw[0], pe2, po2);
  time_pairs(raw[2], raw[1], pe1, po1);
#pragma unroll
  for (int m = 0; m < ROWS; ++m) {
    u32x4 pe0, po0;
    time_pairs(raw[m + 3], raw[m + 2], pe0, po0);
    u32x4 y;
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      const float a0 = dot4_bf16(wp[2 * c][0], wp[2 * c][1], pe0[c], pe2[c]);
      const float a1 = dot4_bf16(wp[2 * c + 1][0], wp[2 * c + 1][1], po0[c], po2[c]);
      const uint32_t u = pack_bf16(a0, a1);  // the pre-activations, rounded to bf16
      y[c] = pack_bf16(silu_fast(__uint_as_float(u << 16)), silu_fast(__uint_as_float(u & 0xffff0000u)));
    }
    if (nvalid < kC) {  // uniform: a sequence's last chunk; its padded rows are zero
      if (r0 + m >= nvalid) y = u32x4{0u, 0u, 0u, 0u};
    }
    emit(m, y);
    pe2 = pe1;
    po2 = po1;
    pe1 = pe0;
    po1 = po0;
  }
}

// conv_load then conv_compute, with the window and weights local to the call
// (channels chu + chl .. +7: chu uniform, chl the lane's part)
template <int ROWS, class Emit>
__device__ __forceinline__ void conv_rows(const ChunkParams& p, int n, long long s0, long long t0,
                                          int nvalid, int r0, int chu, int chl, Emit emit) {
  u32x4 raw[ROWS + 3];
  uint32_t wp[8][2];
  load_conv_w(p, chu, chl, wp);
  conv_load<ROWS>(p, n, s0, t0, nvalid, r0, chu, chl, raw);
  conv_compute<ROWS>(raw, wp, nvalid, r0, emit);
}

}  // namespace omx
