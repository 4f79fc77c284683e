// Zero-padded copies for head dims the kernels are not compiled for.
//
// The chunked kernels take dk in {64, 128} (bf16) or {32, 64, 128} (fp32) and dv a
// multiple of 64.  Other head dims (the reference's smoke layout has dk = 16, dv = 32,
// config.py:94-101) run on copies padded with zeros to the next compiled size, which
// changes nothing that is returned: zero key/query entries leave every dot product and
// L2 norm unchanged (the scale stays the caller's dk^-1/2), zero value columns keep
// their state columns and outputs at zero, and the gated norm divides by the real dv.
// Results are then copied back out of the padded buffers.
//
// One kernel does both directions: it views src and dst as [R][G][E] arrays with their
// own row and group strides and writes every dst element (g < Gd, e < Ed) as the src
// element at (g, e) when g < Gs and e < Es, else zero.
#include "gdn_common.h"
#include "gdn_kernels.h"

namespace omx {

namespace {

template <typename E>
__global__ __launch_bounds__(256) void pad_copy_kernel(const E* __restrict__ src, E* __restrict__ dst,
                                                       long long R, int Gs, int Es, long long srs,
                                                       long long sgs, int Gd, int Ed, long long drs,
                                                       long long dgs) {
  const long long total = R * Gd * Ed;
  for (long long i = (long long)blockIdx.x * 256 + threadIdx.x; i < total;
       i += (long long)gridDim.x * 256) {
    const int e = (int)(i % Ed);
    const long long rg = i / Ed;
    const int g = (int)(rg % Gd);
    const long long r = rg / Gd;
    dst[r * drs + g * dgs + e] = (g < Gs && e < Es) ? src[r * srs + g * sgs + e] : E(0);
  }
}

}  // namespace

hipError_t launch_pad_copy(const PadView& s, const PadView& d, long long R, int esize,
                           hipStream_t stream) {
  const long long total = R * d.G * d.E;
  if (total == 0) return hipSuccess;
  const long long blocks = (total + 255) / 256;
  const unsigned grid = (unsigned)(blocks < 16384 ? blocks : 16384);
  if (esize == 4)
    hipLaunchKernelGGL(pad_copy_kernel<uint32_t>, dim3(grid), dim3(256), 0, stream,
                       (const uint32_t*)s.p, (uint32_t*)d.p, R, s.G, s.E, s.rs, s.gs, d.G, d.E,
                       d.rs, d.gs);
  else
    hipLaunchKernelGGL(pad_copy_kernel<uint16_t>, dim3(grid), dim3(256), 0, stream,
                       (const uint16_t*)s.p, (uint16_t*)d.p, R, s.G, s.E, s.rs, s.gs, d.G, d.E,
                       d.rs, d.gs);
  return hipGetLastError();
}

}  // namespace omx
