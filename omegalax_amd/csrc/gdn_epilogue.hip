// Gated RMSNorm epilogue for prefills whose dv is split across workgroups.
//
// deltanet.py:282-293 normalises each (token, value head) row of the fp32 core
// output: out = w * o * rsqrt(mean(o^2) + eps) * silu(z).  When the chunked
// kernel splits dv over nb workgroups, each writes its columns of o (bf16) and
// its share of sum(o^2) (fp32, from the fp32 o); this kernel adds the shares
// and applies the norm.  Memory-bound: two bf16 reads and one bf16 write per
// element, one thread per pair of columns.
#include "gdn_common.h"
#include "gdn_kernels.h"

namespace omx {

namespace {

__global__ __launch_bounds__(256) void norm_epilogue_kernel(const uint32_t* __restrict__ o_part,
                                                            const float* __restrict__ ss_part,
                                                            const uint32_t* __restrict__ z,
                                                            const float* __restrict__ norm_w,
                                                            uint32_t* __restrict__ out,
                                                            long long pairs, int dv, int nb,
                                                            float eps) {
  const long long i = (long long)blockIdx.x * 256 + threadIdx.x;
  if (i >= pairs) return;
  const int half = dv / 2;
  const long long row = i / half;
  const int c = 2 * (int)(i % half);
  float ss = 0.f;
  for (int b = 0; b < nb; ++b) ss += ss_part[row * nb + b];
  const float rn = rsqrtf(ss / (float)dv + eps);
  const uint32_t ow = o_part[i], zw = z[i];
  const float o0 = __uint_as_float(ow << 16), o1 = __uint_as_float(ow & 0xffff0000u);
  const float z0 = __uint_as_float(zw << 16), z1 = __uint_as_float(zw & 0xffff0000u);
  out[i] = pack_bf16(norm_w[c] * (o0 * rn) * siluf_(z0), norm_w[c + 1] * (o1 * rn) * siluf_(z1));
}

}  // namespace

hipError_t launch_norm_epilogue(const void* o_part, const float* ss_part, const void* z,
                                const float* norm_w, void* out, long long rows, int dv, int nb,
                                float eps, hipStream_t stream) {
  const long long pairs = rows * (dv / 2);
  if (pairs == 0) return hipSuccess;
  const unsigned grid = (unsigned)((pairs + 255) / 256);
  hipLaunchKernelGGL(norm_epilogue_kernel, dim3(grid), dim3(256), 0, stream,
                     (const uint32_t*)o_part, ss_part, (const uint32_t*)z, norm_w, (uint32_t*)out,
                     pairs, dv, nb, eps);
  return hipGetLastError();
}

}  // namespace omx
