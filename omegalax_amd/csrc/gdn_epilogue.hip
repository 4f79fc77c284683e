// Gated RMSNorm epilogue of the layer prefill.
//
// deltanet.py:282-293 normalises each (token, value head) row of the fp32 core
// output: out = w * o * rsqrt(mean(o^2) + eps) * silu(z).  The chunked scan
// writes o in bf16; this kernel forms mean(o^2) from those values (the row's
// bf16 rounding moves the norm by at most 2^-9 relative) and applies the norm.
// Memory-bound: two bf16 reads and one bf16 write per element.  The mean divides by
// dv_mean, the caller's dv when the rows are zero-padded copies (their extra columns
// are zero and add nothing to the sum of squares).  A row is handled by
// a group of G lanes (G = dv / 8 rounded up to a power of two, at most 32), one
// thread per 8 columns (16-byte accesses); the row's sum of squares is a butterfly
// over the group.
#include "gdn_common.h"
#include "gdn_kernels.h"

namespace omx {

namespace {

template <int G>
__global__ __launch_bounds__(256) void norm_epilogue_kernel(const uint4* __restrict__ o_part,
                                                            const uint4* __restrict__ z,
                                                            const float* __restrict__ norm_w,
                                                            uint4* __restrict__ out,
                                                            long long rows, int dv, float inv_dv,
                                                            float eps) {
  const long long gid = (long long)blockIdx.x * 256 + threadIdx.x;
  const long long row = gid / G;
  const int j = (int)(gid % G);  // octet of the row
  const int per_row = dv / 8;
  // whole groups stay in the loop for the shuffles; lanes past the row or the last
  // row contribute zeros
  const bool active = row < rows && j < per_row;
  const long long i = row * per_row + j;
  uint4 ow = make_uint4(0u, 0u, 0u, 0u), zw = ow;
  if (active) {
    ow = o_part[i];
    zw = z[i];
  }
  const uint32_t ov[4] = {ow.x, ow.y, ow.z, ow.w}, zv[4] = {zw.x, zw.y, zw.z, zw.w};
  float o[8];
  float ss = 0.f;
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    o[2 * e] = __uint_as_float(ov[e] << 16);
    o[2 * e + 1] = __uint_as_float(ov[e] & 0xffff0000u);
    ss += o[2 * e] * o[2 * e] + o[2 * e + 1] * o[2 * e + 1];
  }
#pragma unroll
  for (int m = 1; m < G; m <<= 1) ss += __shfl_xor(ss, m, G);
  if (!active) return;
  const float rn = rsqrtf(ss * inv_dv + eps);
  const int c = 8 * j;
  const float4 w0 = *(const float4*)(norm_w + c), w1 = *(const float4*)(norm_w + c + 4);
  const float w[8] = {w0.x, w0.y, w0.z, w0.w, w1.x, w1.y, w1.z, w1.w};
  uint32_t r[4];
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const float z0 = __uint_as_float(zv[e] << 16), z1 = __uint_as_float(zv[e] & 0xffff0000u);
    r[e] = pack_bf16(w[2 * e] * (o[2 * e] * rn) * silu_fast(z0),
                     w[2 * e + 1] * (o[2 * e + 1] * rn) * silu_fast(z1));
  }
  out[i] = make_uint4(r[0], r[1], r[2], r[3]);
}

template <int G>
hipError_t launch_g(const void* o_part, const void* z, const float* norm_w, void* out,
                    long long rows, int dv, int dv_mean, float eps, hipStream_t stream) {
  const long long threads = rows * G;
  const unsigned grid = (unsigned)((threads + 255) / 256);
  hipLaunchKernelGGL((norm_epilogue_kernel<G>), dim3(grid), dim3(256), 0, stream,
                     (const uint4*)o_part, (const uint4*)z, norm_w, (uint4*)out, rows, dv,
                     1.0f / (float)dv_mean, eps);
  return hipGetLastError();
}

}  // namespace

hipError_t launch_norm_epilogue(const void* o_part, const void* z, const float* norm_w, void* out,
                                long long rows, int dv, int dv_mean, float eps,
                                hipStream_t stream) {
  if (rows == 0) return hipSuccess;
  const int per_row = dv / 8;
  if (per_row <= 8) return launch_g<8>(o_part, z, norm_w, out, rows, dv, dv_mean, eps, stream);
  if (per_row <= 16) return launch_g<16>(o_part, z, norm_w, out, rows, dv, dv_mean, eps, stream);
  if (per_row <= 32) return launch_g<32>(o_part, z, norm_w, out, rows, dv, dv_mean, eps, stream);
  return hipErrorInvalidValue;
}

}  // namespace omx
