// Gated RMSNorm epilogue of the layer prefill.
//
// deltanet.py:282-293 normalises each (token, value head) row of the fp32 core
// output: out = w * o * rsqrt(mean(o^2) + eps) * silu(z).  The chunked scan writes o
// in bf16 together with a few fp32 partial sums of squares of each row (formed from the
// fp32 o, in 64-token blocks: ss_index); this kernel takes the row's mean from those
// partials and applies the norm to the bf16 o.  Memory-bound: two bf16 reads and one
// bf16 write per element.  The mean divides by dv_mean, the caller's dv when the rows
// are zero-padded copies (their extra columns are zero and add nothing to the sums).
// A row is handled by a group of G lanes (G = dv / 8 rounded up to a power of two, at
// most 32), one thread per 8 columns (16-byte accesses); the group's first lanes hold one
// partial each and the row's sum is a butterfly over the group: the pairwise tree that
// the scan's partials continue (ss_tree), so a row's total does not depend on how many
// partials the scan formed.
#include "gdn_common.h"
#include "gdn_kernels.h"

namespace omx {

namespace {

// the norm of one row from its 8 columns of o and z (raw bf16 words) and the row's sum of
// squares; writes the 8 outputs
__device__ __forceinline__ void norm_row8(uint4 ow, uint4 zw, float ss, const float* norm_w, int c,
                                          float inv_dv, float eps, uint4* dst) {
  const uint32_t ov[4] = {ow.x, ow.y, ow.z, ow.w}, zv[4] = {zw.x, zw.y, zw.z, zw.w};
  const float rn = rsqrtf(__builtin_fmaf(ss, inv_dv, eps));  // as the scans that fuse the norm
  const float4 w0 = *(const float4*)(norm_w + c), w1 = *(const float4*)(norm_w + c + 4);
  const float w[8] = {w0.x, w0.y, w0.z, w0.w, w1.x, w1.y, w1.z, w1.w};
  uint32_t r[4];
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const float o0 = __uint_as_float(ov[e] << 16), o1 = __uint_as_float(ov[e] & 0xffff0000u);
    const float z0 = __uint_as_float(zv[e] << 16), z1 = __uint_as_float(zv[e] & 0xffff0000u);
    r[e] = pack_bf16(w[2 * e] * (o0 * rn) * silu_fast(z0), w[2 * e + 1] * (o1 * rn) * silu_fast(z1));
  }
  *dst = make_uint4(r[0], r[1], r[2], r[3]);
}

// One group of G lanes per row, rows in memory order; the group's first nss lanes read
// one partial each (the row's partials lie 64 floats apart in the ss_index layout).
template <int G>
__global__ __launch_bounds__(256) void norm_epilogue_kernel(const uint4* __restrict__ o_part,
                                                            const float* __restrict__ o_ss,
                                                            int nss,
                                                            const uint4* __restrict__ z,
                                                            const float* __restrict__ norm_w,
                                                            uint4* __restrict__ out,
                                                            long long tokens, int Hv, int dv,
                                                            float inv_dv, float eps) {
  // (token, head) of the group's row: the workgroup's first row by one scalar division,
  // then the group's offset from it (256 / G rows per workgroup)
  const long long row0 = (long long)blockIdx.x * (256 / G);
  long long t = row0 / Hv;
  int h = (int)(row0 - t * Hv) + (int)(threadIdx.x / G);
  while (h >= Hv) {
    h -= Hv;
    ++t;
  }
  const int j = (int)(threadIdx.x % G);  // octet of the row
  const int per_row = dv / 8;
  // whole groups stay in the loop for the shuffles; lanes past the row or the last
  // row contribute zeros
  const bool active = t < tokens && j < per_row;
  const long long i = (t * Hv + h) * per_row + j;
  uint4 ow = make_uint4(0u, 0u, 0u, 0u), zw = ow;
  float ss = 0.f;
  if (active) {
    ow = o_part[i];
    zw = z[i];
    if (j < nss) ss = o_ss[ss_index(t, h, j, Hv, nss)];
  }
#pragma unroll
  for (int m = 1; m < G; m <<= 1) ss += __shfl_xor(ss, m, G);
  if (active) norm_row8(ow, zw, ss, norm_w, 8 * j, inv_dv, eps, out + i);
}

template <int G>
hipError_t launch_g(const void* o_part, const float* o_ss, int nss, const void* z,
                    const float* norm_w, void* out, long long tokens, int Hv, int dv, int dv_mean,
                    float eps, hipStream_t stream) {
  const long long blocks = (tokens * Hv + 256 / G - 1) / (256 / G);
  if (blocks > 0xffffffffLL) return hipErrorInvalidValue;
  hipLaunchKernelGGL((norm_epilogue_kernel<G>), dim3((unsigned)blocks), dim3(256), 0, stream,
                     (const uint4*)o_part, o_ss, nss, (const uint4*)z, norm_w, (uint4*)out, tokens,
                     Hv, dv, 1.0f / (float)dv_mean, eps);
  return hipGetLastError();
}

}  // namespace

hipError_t launch_norm_epilogue(const void* o_part, const float* o_ss, int nss, const void* z,
                                const float* norm_w, void* out, long long tokens, int Hv, int dv,
                                int dv_mean, float eps, hipStream_t stream) {
  if (tokens == 0 || Hv == 0) return hipSuccess;
  const int per_row = dv / 8;
  if (dv % 16 != 0 || nss < 1 || 2 * nss > per_row) return hipErrorInvalidValue;
  if (per_row <= 8) return launch_g<8>(o_part, o_ss, nss, z, norm_w, out, tokens, Hv, dv, dv_mean, eps, stream);
  if (per_row <= 16) return launch_g<16>(o_part, o_ss, nss, z, norm_w, out, tokens, Hv, dv, dv_mean, eps, stream);
  if (per_row <= 32) return launch_g<32>(o_part, o_ss, nss, z, norm_w, out, tokens, Hv, dv, dv_mean, eps, stream);
  return hipErrorInvalidValue;
}

}  // namespace omx
