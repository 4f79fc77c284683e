// Single-token cached decode step of the gated delta rule (gfx950).
//
// The reference has no Qwen3.5 decode (omegalax/models/qwen3_5/model.py:324-326,
// text/api.py:128-131).  Semantics follow transformers' causal_conv1d_update and
// torch_recurrent_gated_delta_rule; the gated norm follows deltanet.py:282-293.
//
// Work mapping: one workgroup of 256 threads per (sequence, key head).  The
// workgroup owns every channel of that key head's q/k and of its gqa value heads,
// so it can update the conv-state cache in place without racing another
// workgroup, and it loops over its value heads.  For one value head the fp32
// state S[dk][dv] (row-major, dv contiguous) is streamed once in and once out:
// thread t owns 4 consecutive columns (one float4 per row) of the rows
// rg, rg+RG, ... so one wavefront load covers whole contiguous rows.
// With the recurrence written as
//     kv = a S^T k,  delta = beta (v - kv),  o = a S^T q + (q.k) delta,
//     S' = a S + k delta^T
// both reductions over dk come from the same register-resident pass over S;
// S' is written back from the same registers.  Per sequence and step the kernel
// moves Hv*dk*dv*8 bytes of state plus the token's activations.
#include "gdn_common.h"
#include "gdn_kernels.h"

namespace omx {

namespace {

constexpr int kThreads = 256;
constexpr int kMaxConvK = 8;

typedef float v4f __attribute__((ext_vector_type(4)));

// State accesses: non-temporal (streamed past the caches) or ordinary.
template <bool NT>
__device__ __forceinline__ float4 load_st(const float* p) {
  if constexpr (NT) {
    const v4f v = __builtin_nontemporal_load((const v4f*)p);
    return make_float4(v[0], v[1], v[2], v[3]);
  } else {
    return *(const float4*)p;
  }
}
template <bool NT>
__device__ __forceinline__ void store_st(float* p, float4 x) {
  if constexpr (NT) __builtin_nontemporal_store(v4f{x.x, x.y, x.z, x.w}, (v4f*)p);
  else *(float4*)p = x;
}

// Prefetch shape of the layer path's small inputs (PRE): channels per thread and value
// heads per workgroup it covers.
constexpr int kPreChannels = 2, kPreHeads = 2;

template <int DK, int DV, bool LAYER, typename InT, bool NT, bool EARLY, bool PRE>
__global__ __launch_bounds__(kThreads) void decode_kernel(DecodeParams p) {
  constexpr int CG = DV / 4;            // column groups of 4
  constexpr int RG = kThreads / CG;     // row groups
  constexpr int R = (DK + RG - 1) / RG; // rows per thread
  static_assert(DV % 4 == 0 && CG <= kThreads, "dv layout");

  const int hk = blockIdx.x;
  const int b = blockIdx.y;
  const int tid = threadIdx.x;
  const int gqa = p.Hv / p.Hk;
  const int cg = tid % CG, rg = tid / CG;

  // With EARLY the state reads are issued first, so they stream in while the conv, the
  // norms and their barriers run; otherwise they follow the conv.  The next value head's
  // state is loaded while the current one is reduced and updated, so a workgroup keeps
  // two heads' state reads in flight.
  auto load_state = [&](int hh, float4* st) {
    const float* S = p.state + ((size_t)b * p.Hv + hk * gqa + hh) * DK * DV;
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const int row = rg + r * RG;
      if (row < DK) st[r] = load_st<NT>(S + (size_t)row * DV + 4 * cg);
      else st[r] = make_float4(0.f, 0.f, 0.f, 0.f);
    }
  };
  // PRE (layer path, K = 4, 2 dk + gqa dv <= 2 * 256 channels, gqa <= 2): the step's small
  // inputs -- this thread's conv channels (raw token, the three cached inputs, weights),
  // z, norm_w and the gate inputs -- are loaded before the state.  The memory counter
  // retires loads and stores in issue order, so a small load issued after the state
  // loads, or after a value head's state stores, would wait for all of them.
  const int conv_dim = 2 * p.Hk * DK + p.Hv * DV;
  auto conv_channel = [&](int i) {
    if (i < DK) return hk * DK + i;
    if (i < 2 * DK) return p.Hk * DK + hk * DK + (i - DK);
    return 2 * p.Hk * DK + hk * gqa * DV + (i - 2 * DK);
  };
  unsigned short pre_x[kPreChannels], pre_h[kPreChannels][3];
  float pre_w[kPreChannels][4], pre_z[kPreHeads], pre_a[kPreHeads], pre_b[kPreHeads];
  float pre_nw = 0.f;
  if constexpr (PRE) {
    const int nch = 2 * DK + gqa * DV;
    const unsigned short* xin = (const unsigned short*)p.mixed_qkv + (size_t)b * conv_dim;
#pragma unroll
    for (int m = 0; m < kPreChannels; ++m) {
      const int i = tid + m * kThreads;
      if (i < nch) {
        const int c = conv_channel(i);
        const unsigned short* cs = (const unsigned short*)p.conv_state + ((size_t)b * conv_dim + c) * 3;
        pre_x[m] = xin[c];
#pragma unroll
        for (int j = 0; j < 3; ++j) pre_h[m][j] = cs[j];
#pragma unroll
        for (int j = 0; j < 4; ++j) pre_w[m][j] = p.conv_w[(size_t)c * 4 + j];
      }
    }
#pragma unroll
    for (int hh = 0; hh < kPreHeads; ++hh) {
      const int h = hk * gqa + hh;
      if (hh < gqa) {
        if (tid < DV) pre_z[hh] = bf2f(((const bf16_t*)p.z)[((size_t)b * p.Hv + h) * DV + tid]);
        pre_a[hh] = bf2f(((const bf16_t*)p.a)[(size_t)b * p.Hv + h]);
        pre_b[hh] = bf2f(((const bf16_t*)p.b)[(size_t)b * p.Hv + h]);
      }
    }
    if (tid < DV) pre_nw = p.norm_w[tid];
  }
  float4 st[R], stn[R];
  if (EARLY) {
    load_state(0, st);
    if (gqa > 1) load_state(1, stn);
  }

  __shared__ __align__(16) float s_q[DK];
  __shared__ __align__(16) float s_k[DK];
  __shared__ __align__(16) float s_v[DV];
  __shared__ __align__(16) float s_red_kv[RG][DV + 1];
  __shared__ __align__(16) float s_red_qs[RG][DV + 1];
  __shared__ __align__(16) float s_delta[DV];
  __shared__ __align__(16) float s_o[DV];
  __shared__ float s_scal[8];

  // ---------------------------------------------------------------- q, k (and conv)
  if (PRE) {
    // the same arithmetic as below, on the prefetched registers (K = 4)
    const int nch = 2 * DK + gqa * DV;
#pragma unroll
    for (int m = 0; m < kPreChannels; ++m) {
      const int i = tid + m * kThreads;
      if (i >= nch) continue;
      const int c = conv_channel(i);
      bf16_t* cs = (bf16_t*)p.conv_state + ((size_t)b * conv_dim + c) * 3;
      float acc = 0.f;
#pragma unroll
      for (int j = 0; j < 3; ++j) acc += round_bf(pre_w[m][j]) * bf2f(pre_h[m][j]);
      acc += round_bf(pre_w[m][3]) * bf2f(pre_x[m]);
      const float y = round_bf(siluf_(round_bf(acc)));
      cs[0] = pre_h[m][1];
      cs[1] = pre_h[m][2];
      cs[2] = pre_x[m];
      if (i < DK) s_q[i] = y;
      else if (i < 2 * DK) s_k[i - DK] = y;
      else {
        const int vi = i - 2 * DK;
        s_red_kv[vi / DV][vi % DV] = y;
      }
    }
  } else if (LAYER) {
    const int nch = 2 * DK + gqa * DV;
    const int K = p.conv_k;
    for (int i = tid; i < nch; i += kThreads) {
      const int c = conv_channel(i);
      const bf16_t* xin = (const bf16_t*)p.mixed_qkv + (size_t)b * conv_dim;
      bf16_t* cs = (bf16_t*)p.conv_state + ((size_t)b * conv_dim + c) * (K - 1);
      float hist[kMaxConvK];
#pragma unroll
      for (int j = 0; j < kMaxConvK - 1; ++j) hist[j] = (j < K - 1) ? bf2f(cs[j]) : 0.f;
      const bf16_t xr = xin[c];
      float acc = 0.f;
#pragma unroll
      for (int j = 0; j < kMaxConvK; ++j) {
        if (j < K - 1) acc += round_bf(p.conv_w[(size_t)c * K + j]) * hist[j];
      }
      acc += round_bf(p.conv_w[(size_t)c * K + K - 1]) * bf2f(xr);
      const float y = round_bf(siluf_(round_bf(acc)));
      // shift the cache: drop the oldest input, append this token's raw input
#pragma unroll
      for (int j = 0; j < kMaxConvK - 2; ++j) {
        if (j < K - 2) cs[j] = f2bf(hist[j + 1]);
      }
      cs[K - 2] = xr;
      if (i < DK) s_q[i] = y;
      else if (i < 2 * DK) s_k[i - DK] = y;
      else {
        // value channels of head hh = (i - 2DK) / DV are parked in the reduction
        // buffer until their head's turn
        const int vi = i - 2 * DK;
        s_red_kv[vi / DV][vi % DV] = y;  // gqa * DV <= RG * (DV + 1) checked on the host
      }
    }
  } else {
    const InT* qp = (const InT*)p.q + ((size_t)b * p.Hk + hk) * DK;
    const InT* kp = (const InT*)p.k + ((size_t)b * p.Hk + hk) * DK;
    for (int i = tid; i < DK; i += kThreads) {
      if constexpr (sizeof(InT) == 2) {
        s_q[i] = bf2f(qp[i]);
        s_k[i] = bf2f(kp[i]);
      } else {
        s_q[i] = qp[i];
        s_k[i] = kp[i];
      }
    }
  }
  lds_barrier();

  // L2 norm of q and k at the input precision (deltanet.py:30-32, 65-66)
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63;
  if (wave < 2) {
    const float* src = wave == 0 ? s_q : s_k;
    float ss = 0.f;
    for (int i = lane; i < DK; i += 64) ss += src[i] * src[i];
    ss = wave_sum(ss);
    if (lane == 0) s_scal[wave] = rsqrtf(ss + 1e-6f);
  }
  lds_barrier();
  const bool round_act = LAYER || sizeof(InT) == 2;
  const float scale = p.scale;
  for (int i = tid; i < DK; i += kThreads) {
    float qn = s_q[i] * s_scal[0];
    float kn = s_k[i] * s_scal[1];
    if (round_act) { qn = round_bf(qn); kn = round_bf(kn); }
    s_q[i] = qn * scale;
    s_k[i] = kn;
  }
  lds_barrier();
  if (wave == 0) {
    float d = 0.f;
    for (int i = lane; i < DK; i += 64) d += s_q[i] * s_k[i];
    d = wave_sum(d);
    if (lane == 0) s_scal[2] = d;
  }
  // value channels out of the parking buffer
  float vpark[(DV * 8 + kThreads - 1) / kThreads];  // gqa <= 8
  if (LAYER) {
#pragma unroll
    for (int j = 0; j < (DV * 8 + kThreads - 1) / kThreads; ++j) {
      const int vi = tid + j * kThreads;
      vpark[j] = (vi < gqa * DV) ? s_red_kv[vi / DV][vi % DV] : 0.f;
    }
  }
  lds_barrier();
  const float qk = s_scal[2];
  if (!EARLY) {
    load_state(0, st);
    if (gqa > 1) load_state(1, stn);
  }

  for (int hh = 0; hh < gqa; ++hh) {
    const int h = hk * gqa + hh;
    if (hh > 0 && hh + 1 < gqa) load_state(hh + 1, stn);
    float alpha, beta;
    if (LAYER) {
      const float av = PRE ? pre_a[hh < kPreHeads ? hh : 0] : bf2f(((const bf16_t*)p.a)[(size_t)b * p.Hv + h]);
      const float bv = PRE ? pre_b[hh < kPreHeads ? hh : 0] : bf2f(((const bf16_t*)p.b)[(size_t)b * p.Hv + h]);
      const float g = -expf(p.A_log[h]) * softplusf_(av + p.dt_bias[h]);
      alpha = expf(g);
      beta = round_bf(sigmoidf_(bv));
      // this head's values from the parked registers
#pragma unroll
      for (int j = 0; j < (DV * 8 + kThreads - 1) / kThreads; ++j) {
        const int vi = tid + j * kThreads;
        if (vi >= hh * DV && vi < (hh + 1) * DV) s_v[vi - hh * DV] = vpark[j];
      }
    } else {
      alpha = expf(p.g[(size_t)b * p.Hv + h]);
      beta = p.beta[(size_t)b * p.Hv + h];
      const InT* vp = (const InT*)p.v + ((size_t)b * p.Hv + h) * DV;
      for (int i = tid; i < DV; i += kThreads) {
        if constexpr (sizeof(InT) == 2) s_v[i] = bf2f(vp[i]);
        else s_v[i] = vp[i];
      }
    }

    float* S = p.state + ((size_t)b * p.Hv + h) * DK * DV;
    float4 kv = make_float4(0.f, 0.f, 0.f, 0.f), qs = kv;
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const int row = rg + r * RG;
      const float kr = row < DK ? s_k[row] : 0.f;
      const float qr = row < DK ? s_q[row] : 0.f;
      kv.x += kr * st[r].x; kv.y += kr * st[r].y; kv.z += kr * st[r].z; kv.w += kr * st[r].w;
      qs.x += qr * st[r].x; qs.y += qr * st[r].y; qs.z += qr * st[r].z; qs.w += qr * st[r].w;
    }
    s_red_kv[rg][4 * cg + 0] = kv.x; s_red_kv[rg][4 * cg + 1] = kv.y;
    s_red_kv[rg][4 * cg + 2] = kv.z; s_red_kv[rg][4 * cg + 3] = kv.w;
    s_red_qs[rg][4 * cg + 0] = qs.x; s_red_qs[rg][4 * cg + 1] = qs.y;
    s_red_qs[rg][4 * cg + 2] = qs.z; s_red_qs[rg][4 * cg + 3] = qs.w;
    lds_barrier();
    if (tid < DV) {
      float skv = 0.f, sqs = 0.f;
#pragma unroll
      for (int r = 0; r < RG; ++r) { skv += s_red_kv[r][tid]; sqs += s_red_qs[r][tid]; }
      const float delta = beta * (s_v[tid] - alpha * skv);
      s_delta[tid] = delta;
      s_o[tid] = alpha * sqs + qk * delta;
    }
    lds_barrier();
    float4 dl = *(const float4*)(s_delta + 4 * cg);
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const int row = rg + r * RG;
      if (row < DK) {
        const float kr = s_k[row];
        float4 n;
        n.x = alpha * st[r].x + kr * dl.x;
        n.y = alpha * st[r].y + kr * dl.y;
        n.z = alpha * st[r].z + kr * dl.z;
        n.w = alpha * st[r].w + kr * dl.w;
        store_st<NT>(S + (size_t)row * DV + 4 * cg, n);
      }
    }
    if (LAYER) {
      // gated RMSNorm on the fp32 core output (deltanet.py:282-293)
      if (wave == 0) {
        float ss = 0.f;
        for (int i = lane; i < DV; i += 64) ss += s_o[i] * s_o[i];
        ss = wave_sum(ss);
        if (lane == 0) s_scal[3] = rsqrtf(ss / DV + p.eps);
      }
      lds_barrier();
      const float rn = s_scal[3];
      bf16_t* out = (bf16_t*)p.out + ((size_t)b * p.Hv + h) * DV;
      const bf16_t* z = (const bf16_t*)p.z + ((size_t)b * p.Hv + h) * DV;
      if (PRE) {
        if (tid < DV) out[tid] = f2bf(pre_nw * (s_o[tid] * rn) * siluf_(pre_z[hh < kPreHeads ? hh : 0]));
      } else {
        for (int i = tid; i < DV; i += kThreads) {
          const float n = p.norm_w[i] * (s_o[i] * rn);
          out[i] = f2bf(n * siluf_(bf2f(z[i])));
        }
      }
    } else {
      float* o = p.o + ((size_t)b * p.Hv + h) * DV;
      for (int i = tid; i < DV; i += kThreads) o[i] = s_o[i];
    }
    lds_barrier();
    if (hh + 1 < gqa) {
#pragma unroll
      for (int r = 0; r < R; ++r) st[r] = stn[r];
    }
  }
}

template <int DK, int DV, bool NT, bool EARLY>
void launch_cfg(const DecodeParams& p, bool layer, bool in_bf16, hipStream_t stream) {
  dim3 grid(p.Hk, p.B);
  const int gqa = p.Hv / p.Hk;
  const bool pre = p.conv_k == 4 && gqa <= kPreHeads && 2 * DK + gqa * DV <= kPreChannels * kThreads;
  if (layer && pre) {
    hipLaunchKernelGGL((decode_kernel<DK, DV, true, bf16_t, NT, EARLY, true>), grid, dim3(kThreads),
                       0, stream, p);
  } else if (layer) {
    hipLaunchKernelGGL((decode_kernel<DK, DV, true, bf16_t, NT, EARLY, false>), grid, dim3(kThreads),
                       0, stream, p);
  } else if (in_bf16) {
    hipLaunchKernelGGL((decode_kernel<DK, DV, false, bf16_t, NT, EARLY, false>), grid,
                       dim3(kThreads), 0, stream, p);
  } else {
    hipLaunchKernelGGL((decode_kernel<DK, DV, false, float, NT, EARLY, false>), grid,
                       dim3(kThreads), 0, stream, p);
  }
}

// The state is read once and written once per step and is not touched again until the
// layer's next token, after every other layer's state has streamed through: accesses are
// non-temporal so they do not evict the conv cache and the token rows from the caches.
// (Measured at C2 with the state rotated over 512 MiB, as in a multi-layer decode: B=64
// 72.8 us with ordinary accesses, 56.8 us streamed; B=256 198.5 vs 197.9 us.)  Issuing the
// state reads before the conv pays when the grid is at most two rounds of the chip's
// resident workgroups (B=64: 56.8 -> 54.5 us) and costs when it is more (B=256: 197.0 ->
// 209.4 us, the conv's small loads then queue behind a saturated stream).
constexpr long long kEarlyMaxWorkgroups = 2048;

template <int DK, int DV>
hipError_t launch_dims(const DecodeParams& p, bool layer, bool in_bf16, hipStream_t stream) {
  if ((long long)p.B * p.Hk <= kEarlyMaxWorkgroups) launch_cfg<DK, DV, true, true>(p, layer, in_bf16, stream);
  else launch_cfg<DK, DV, true, false>(p, layer, in_bf16, stream);
  return hipGetLastError();
}

}  // namespace

bool decode_dims_supported(int dk, int dv) {
  auto ok = [](int d) { return d == 16 || d == 32 || d == 64 || d == 128; };
  return ok(dk) && ok(dv);
}

int decode_max_gqa() { return 8; }

hipError_t launch_decode(const DecodeParams& p, bool layer, bool in_bf16, hipStream_t stream) {
#define OMX_DK_CASE(DKV)                                                        \
  if (p.dk == DKV) {                                                            \
    switch (p.dv) {                                                             \
      case 16: return launch_dims<DKV, 16>(p, layer, in_bf16, stream);         \
      case 32: return launch_dims<DKV, 32>(p, layer, in_bf16, stream);         \
      case 64: return launch_dims<DKV, 64>(p, layer, in_bf16, stream);         \
      case 128: return launch_dims<DKV, 128>(p, layer, in_bf16, stream);       \
    }                                                                           \
  }
  OMX_DK_CASE(16)
  OMX_DK_CASE(32)
  OMX_DK_CASE(64)
  OMX_DK_CASE(128)
#undef OMX_DK_CASE
  return hipErrorInvalidValue;
}

}  // namespace omx
