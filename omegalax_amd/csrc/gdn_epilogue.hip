// Gated RMSNorm epilogue of the layer prefill.
//
// deltanet.py:282-293 normalises each (token, value head) row of the fp32 core
// output: out = w * o * rsqrt(mean(o^2) + eps) * silu(z).  The chunked scan
// spreads a row's dv columns over several wavefronts (and workgroups); each
// writes its columns of o (bf16) and its share of sum(o^2) (fp32, from the fp32
// o).  This kernel adds the nparts shares and applies the norm.  Memory-bound:
// two bf16 reads and one bf16 write per element, one thread per 8 columns
// (16-byte accesses).
#include "gdn_common.h"
#include "gdn_kernels.h"

namespace omx {

namespace {

__global__ __launch_bounds__(256) void norm_epilogue_kernel(const uint4* __restrict__ o_part,
                                                            const float* __restrict__ ss_part,
                                                            const uint4* __restrict__ z,
                                                            const float* __restrict__ norm_w,
                                                            uint4* __restrict__ out,
                                                            long long octets, int dv, int nparts,
                                                            float eps) {
  const long long i = (long long)blockIdx.x * 256 + threadIdx.x;
  if (i >= octets) return;
  const int per_row = dv / 8;
  const long long row = i / per_row;
  const int c = 8 * (int)(i % per_row);
  const uint4 ow = o_part[i], zw = z[i];
  float ss = 0.f;
  if ((nparts & 3) == 0) {  // the partial sums of a row are 16-byte aligned: float4 loads
    const float4* sp = (const float4*)(ss_part + row * nparts);
    for (int b = 0; b < nparts / 4; ++b) {
      const float4 v = sp[b];
      ss += (v.x + v.y) + (v.z + v.w);
    }
  } else {
    for (int b = 0; b < nparts; ++b) ss += ss_part[row * nparts + b];
  }
  const float rn = rsqrtf(ss / (float)dv + eps);
  const float4 w0 = *(const float4*)(norm_w + c), w1 = *(const float4*)(norm_w + c + 4);
  const float w[8] = {w0.x, w0.y, w0.z, w0.w, w1.x, w1.y, w1.z, w1.w};
  const uint32_t ov[4] = {ow.x, ow.y, ow.z, ow.w}, zv[4] = {zw.x, zw.y, zw.z, zw.w};
  uint32_t r[4];
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const float o0 = __uint_as_float(ov[e] << 16), o1 = __uint_as_float(ov[e] & 0xffff0000u);
    const float z0 = __uint_as_float(zv[e] << 16), z1 = __uint_as_float(zv[e] & 0xffff0000u);
    r[e] = pack_bf16(w[2 * e] * (o0 * rn) * silu_fast(z0), w[2 * e + 1] * (o1 * rn) * silu_fast(z1));
  }
  out[i] = make_uint4(r[0], r[1], r[2], r[3]);
}

}  // namespace

hipError_t launch_norm_epilogue(const void* o_part, const float* ss_part, const void* z,
                                const float* norm_w, void* out, long long rows, int dv, int nparts,
                                float eps, hipStream_t stream) {
  const long long octets = rows * (dv / 8);
  if (octets == 0) return hipSuccess;
  const unsigned grid = (unsigned)((octets + 255) / 256);
  hipLaunchKernelGGL(norm_epilogue_kernel, dim3(grid), dim3(256), 0, stream,
                     (const uint4*)o_part, ss_part, (const uint4*)z, norm_w, (uint4*)out, octets,
                     dv, nparts, eps);
  return hipGetLastError();
}

}  // namespace omx
