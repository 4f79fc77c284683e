// Internal launch interface between the C ABI (gdn_capi.cpp) and the kernels.
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

namespace omx {

// Decode step.  Layer mode reads mixed_qkv/z/a/b and the conv cache and writes
// the gated-norm output; core mode reads post-conv q/k/v plus g/beta and writes
// the fp32 core output o.
struct DecodeParams {
  // layer mode
  const void* mixed_qkv;  // [B, conv_dim] bf16
  const void* z;          // [B, Hv, dv] bf16
  const void* a;          // [B, Hv] bf16
  const void* b;          // [B, Hv] bf16
  const float* conv_w;    // [conv_dim, K]
  const float* A_log;     // [Hv]
  const float* dt_bias;   // [Hv]
  const float* norm_w;    // [dv]
  void* conv_state;       // [B, conv_dim, K-1] bf16, updated in place
  void* out;              // [B, Hv*dv] bf16
  // core mode
  const void* q;          // [B, Hk, dk]
  const void* k;          // [B, Hk, dk]
  const void* v;          // [B, Hv, dv]
  const float* g;         // [B, Hv]
  const float* beta;      // [B, Hv]
  float* o;               // [B, Hv, dv]
  // both
  float* state;           // [B, Hv, dk, dv] fp32, updated in place
  int B, Hk, Hv, dk, dv, conv_k;
  float scale, eps;
};

bool decode_dims_supported(int dk, int dv);
int decode_max_gqa();
hipError_t launch_decode(const DecodeParams& p, bool layer, bool in_bf16, hipStream_t stream);

}  // namespace omx
