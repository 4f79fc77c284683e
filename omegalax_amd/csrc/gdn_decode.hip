// Single-token cached decode step of the gated delta rule (gfx950).
//
// The reference has no Qwen3.5 decode (omegalax/models/qwen3_5/model.py:324-326,
// text/api.py:128-131).  Semantics follow transformers' causal_conv1d_update and
// torch_recurrent_gated_delta_rule; the gated norm follows deltanet.py:282-293.
//
// Two kernels.  decode_stream_kernel (below decode_kernel) runs the layer step at the
// usual layouts (K = 4, gqa 1 or 2, dv 64 or 128): a fixed grid whose workgroups walk
// (sequence, key head) items with the next value head's state in flight, each wavefront
// owning a column slice of the state so that its reductions need no LDS.  decode_kernel
// covers every other shape and the core recurrent step.
//
// decode_kernel: one workgroup of 256 threads per (sequence, key head).  The
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
typedef unsigned int u32x4w __attribute__((ext_vector_type(4)));
typedef unsigned int u32x2w __attribute__((ext_vector_type(2)));

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

// The layer decode step as a stream over a fixed grid (the chip's resident workgroups):
// workgroup w walks the (sequence, key head) items w, w + G, w + 2G, ... (G = gridDim.x)
// and each item's GQA value heads ("units") in order.  Two register sets hold the state of
// the unit being updated and that of the next one, whose loads are in flight meanwhile;
// the next item's small inputs (its conv channels, z, a, b, A_log, dt_bias) are loaded while
// the current item's units run.  Every workgroup thus keeps a state read stream going from
// its first unit to its last, and the grid needs no second round.
//
// State layout in registers: wavefront w owns columns [DV/4 w, DV/4 (w + 1)) of a unit's
// state, and lane (rg, cg) = (lane / CGS, lane % CGS) the 4 columns DV/4 w + 4 cg .. +3 of
// rows rg + RGW r.  The reductions over dk (S^T k and S^T q) are then a lane's own rows
// summed and a butterfly over the wavefront's row groups (DPP and lane-swap moves, no LDS
// and no barrier), so each wavefront forms delta, o and its state update on its own and
// stores the state right away; the only barrier of a unit is the one the gated norm needs
// for its row statistic, after the state stores are issued.  Per item, one more barrier
// publishes the conv outputs (q, k, v rows in LDS); every wavefront forms the q and k norms
// and q.k from them itself.
//
// No memory operation sits under a per-thread branch, and every loop iteration issues the
// same ones (the vector memory counter retires loads and stores in issue order, and an
// instruction stream the compiler can count keeps its waits exact): accesses for an item
// past the workgroup's last go through buffer resources of range 0 (loads return zeros,
// stores are dropped, with no memory traffic), lanes without a channel or output store at
// an offset past the range, and small-input indices are clamped.
//
// Shapes: the layer path with K = 4, gqa 1 or 2, 2 dk + gqa dv <= 512 channels, dv 64 or
// 128 and dk a multiple of the row groups.
template <int DK, int DV, int GQA, bool NT>
__global__ __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(2, 2)))
void decode_stream_kernel(DecodeParams p) {
  constexpr int WC = DV / 4;                           // state columns of one wavefront
  constexpr int CGS = WC / 4;                          // column groups of 4 per wavefront
  constexpr int RGW = 64 / CGS, R = DK / RGW;          // row groups, rows per lane
  constexpr int NCH = 2 * DK + GQA * DV;               // conv channels of one item
  constexpr int NPC = (NCH + kThreads - 1) / kThreads; // channel slots per thread
  constexpr unsigned SB = DK * DV * 4;                 // bytes of one head's state
  constexpr int CP = NT ? 2 : 0;                       // cache policy of state accesses
  static_assert(DV == 64 || DV == 128, "stream decode dv");
  static_assert(DK % RGW == 0 && R >= 1, "stream decode rows");
  static_assert(NPC <= kPreChannels && (GQA == 1 || GQA == 2), "stream decode item shape");
  constexpr unsigned kDrop = 0x80000000u;              // a lane offset past every range

  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63;
  const int cg = lane % CGS, rg = lane / CGS;
  const int col = wave * WC + 4 * cg;                  // first of the lane's 4 columns
  const int G = gridDim.x;
  const int Hk = p.Hk, Hv = p.Hv;
  const int n_items = p.B * Hk;
  const int my_items = (n_items - (int)blockIdx.x + G - 1) / G;
  const int conv_dim = 2 * Hk * DK + Hv * DV;
  const float scale = p.scale, eps = p.eps;

  __shared__ __align__(16) float s_q[2][DK], s_k[2][DK], s_v[2][GQA][DV];
  __shared__ float s_ss[2][4];
  // normalised k and scaled q of the current item, one copy per wavefront, in the order its
  // lanes read them: row rg + RGW r at rg R + r (a lane's rows are contiguous)
  __shared__ __align__(16) float s_kn[4][DK], s_qn[4][DK];

  // item i of this workgroup (i >= my_items: a stand-in whose accesses are all no-ops)
  struct Item {
    int b, hk;
    bool ok;
  };
  auto item = [&](int i) {
    const int it = (int)blockIdx.x + (i < my_items ? i : 0) * G;
    return Item{it / Hk, it % Hk, i < my_items};
  };
  // channel of slot m of this thread (clamped to the item's last), and whether it is real
  auto channel = [&](int hk, int m, bool& real) {
    const int i0 = tid + m * kThreads;
    real = i0 < NCH;
    const int i = real ? i0 : NCH - 1;
    if (i < DK) return hk * DK + i;
    if (i < 2 * DK) return Hk * DK + hk * DK + (i - DK);
    return 2 * Hk * DK + hk * GQA * DV + (i - 2 * DK);
  };

  // state of value head hh of item i; lane offset of row rg + RGW r, columns col .. col + 3
  auto st_off = [&](int r) { return 4u * (unsigned)((rg + RGW * r) * DV + col); };
  auto state_rsrc = [&](const Item& t, int hh) {
    return buf_rsrc(p.state + ((size_t)t.b * Hv + t.hk * GQA + hh) * DK * DV, t.ok ? SB : 0u);
  };
  auto load_state = [&](int i, int hh, float4* st) {
    const auto r_ = state_rsrc(item(i), hh);
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const u32x4w w = __builtin_amdgcn_raw_buffer_load_b128(r_, st_off(r), 0, CP);
      st[r] = make_float4(__uint_as_float(w[0]), __uint_as_float(w[1]), __uint_as_float(w[2]),
                          __uint_as_float(w[3]));
    }
  };

  // small inputs of one item, in registers until its conv
  unsigned short px[NPC], ph[NPC][3];
  u32x4w pw[NPC];
  u32x2w pz[GQA];
  float pa[GQA], pb[GQA], pA[GQA], pdt[GQA];
  auto load_small = [&](int i) {
    const Item t = item(i);
    const auto xr = buf_rsrc((const bf16_t*)p.mixed_qkv + (size_t)t.b * conv_dim,
                             t.ok ? 2u * conv_dim : 0u);
    const auto cr = buf_rsrc((const bf16_t*)p.conv_state + (size_t)t.b * conv_dim * 3,
                             t.ok ? 6u * conv_dim : 0u);
    const auto wr = buf_rsrc(p.conv_w, 16u * conv_dim);
#pragma unroll
    for (int m = 0; m < NPC; ++m) {
      bool real;
      const unsigned c = (unsigned)channel(t.hk, m, real);
      px[m] = __builtin_amdgcn_raw_buffer_load_b16(xr, 2u * c, 0, 0);
#pragma unroll
      for (int j = 0; j < 3; ++j) ph[m][j] = __builtin_amdgcn_raw_buffer_load_b16(cr, 2u * (3u * c + j), 0, 0);
      pw[m] = __builtin_amdgcn_raw_buffer_load_b128(wr, 16u * c, 0, 0);
    }
    const size_t h0 = (size_t)t.b * Hv + t.hk * GQA;
    const auto zr = buf_rsrc((const bf16_t*)p.z + h0 * DV, t.ok ? 2u * GQA * DV : 0u);
    const auto ar = buf_rsrc((const bf16_t*)p.a + h0, t.ok ? 2u * GQA : 0u);
    const auto br = buf_rsrc((const bf16_t*)p.b + h0, t.ok ? 2u * GQA : 0u);
    // the heads' A_log and dt_bias with the rest: a load issued where they are used would
    // wait for every state load in flight before it
    const auto Ar = buf_rsrc(p.A_log + t.hk * GQA, 4u * GQA);
    const auto dr = buf_rsrc(p.dt_bias + t.hk * GQA, 4u * GQA);
#pragma unroll
    for (int hh = 0; hh < GQA; ++hh) {
      pz[hh] = __builtin_amdgcn_raw_buffer_load_b64(zr, 2u * (unsigned)col, 2 * hh * DV, 0);
      pa[hh] = bf2f(__builtin_amdgcn_raw_buffer_load_b16(ar, 0u, 2 * hh, 0));
      pb[hh] = bf2f(__builtin_amdgcn_raw_buffer_load_b16(br, 0u, 2 * hh, 0));
      pA[hh] = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(Ar, 0u, 4 * hh, 0));
      pdt[hh] = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(dr, 0u, 4 * hh, 0));
    }
  };
  const float4 nw = *(const float4*)(p.norm_w + col);

  // per-item values carried into its units
  float rq = 0.f, rk = 0.f, qk = 0.f, alpha_i[GQA], beta_i[GQA];
  float4 sz_i[GQA];

  auto conv_item = [&](int i) {
    const Item t = item(i);
    const int ib = i & 1;
    const auto cw = buf_rsrc((bf16_t*)p.conv_state + (size_t)t.b * conv_dim * 3,
                             t.ok ? 6u * conv_dim : 0u);
#pragma unroll
    for (int m = 0; m < NPC; ++m) {
      bool real;
      const unsigned c = (unsigned)channel(t.hk, m, real);
      const float w0 = __uint_as_float(pw[m][0]), w1 = __uint_as_float(pw[m][1]);
      const float w2 = __uint_as_float(pw[m][2]), w3 = __uint_as_float(pw[m][3]);
      float acc = round_bf(w0) * bf2f(ph[m][0]);
      acc += round_bf(w1) * bf2f(ph[m][1]);
      acc += round_bf(w2) * bf2f(ph[m][2]);
      acc += round_bf(w3) * bf2f(px[m]);
      const float y = round_bf(siluf_(round_bf(acc)));
      // shift the cache: drop the oldest input, append this token's raw input
      const unsigned co = real ? 2u * 3u * c : kDrop;
      __builtin_amdgcn_raw_buffer_store_b16(ph[m][1], cw, co, 0, 0);
      __builtin_amdgcn_raw_buffer_store_b16(ph[m][2], cw, co, 2, 0);
      __builtin_amdgcn_raw_buffer_store_b16(px[m], cw, co, 4, 0);
      const int i0 = tid + m * kThreads;
      if (real) {
        if (i0 < DK) s_q[ib][i0] = y;
        else if (i0 < 2 * DK) s_k[ib][i0 - DK] = y;
        else s_v[ib][(i0 - 2 * DK) / DV][(i0 - 2 * DK) % DV] = y;
      }
    }
#pragma unroll
    for (int hh = 0; hh < GQA; ++hh) {
      const float g = -expf(pA[hh]) * softplusf_(pa[hh] + pdt[hh]);
      alpha_i[hh] = expf(g);
      beta_i[hh] = round_bf(sigmoidf_(pb[hh]));
      sz_i[hh] = make_float4(siluf_(__uint_as_float(pz[hh][0] << 16)),
                             siluf_(__uint_as_float(pz[hh][0] & 0xffff0000u)),
                             siluf_(__uint_as_float(pz[hh][1] << 16)),
                             siluf_(__uint_as_float(pz[hh][1] & 0xffff0000u)));
    }
    load_small(i + 1);  // the next item's, in flight while this item's units run
    lds_barrier();
    // L2 norms of q and k at the input precision (deltanet.py:30-32, 65-66) and q.k, formed
    // by every wavefront from LDS
    float ssq = 0.f, ssk = 0.f;
    for (int j = lane; j < DK; j += 64) {
      ssq += s_q[ib][j] * s_q[ib][j];
      ssk += s_k[ib][j] * s_k[ib][j];
    }
    rq = rsqrtf(wave_sum(ssq) + 1e-6f);
    rk = rsqrtf(wave_sum(ssk) + 1e-6f);
    float d = 0.f;
    for (int j = lane; j < DK; j += 64) {
      const float qn = round_bf(s_q[ib][j] * rq) * scale, kn = round_bf(s_k[ib][j] * rk);
      const int pj = (j % RGW) * R + j / RGW;
      s_qn[wave][pj] = qn;
      s_kn[wave][pj] = kn;
      d += qn * kn;
    }
    qk = wave_sum(d);
  };

  // sum over the wavefront's row groups (lanes with the same cg), left in every lane:
  // rotations by 8 (and 4) within each 16-lane row, then the 16- and 32-lane swaps
  auto rows_sum = [&](float v) {
    v += dpp_f<0x128>(v);                           // row_ror:8
    if constexpr (CGS == 4) v += dpp_f<0x124>(v);   // row_ror:4
    const auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    v = __uint_as_float(a[0]) + __uint_as_float(a[1]);
    const auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return __uint_as_float(b[0]) + __uint_as_float(b[1]);
  };

  // unit (item i, value head hh) from the state in st; ub alternates between units
  auto run_unit = [&](int i, int hh, int ub, float4* st) {
    const Item t = item(i);
    const int ib = i & 1;
    const float alpha = alpha_i[hh], beta = beta_i[hh];
    // normalised k and scaled q of row rg + RGW r, read from this wavefront's copy where used
    auto k_row = [&](int r) { return s_kn[wave][rg * R + r]; };
    auto q_row = [&](int r) { return s_qn[wave][rg * R + r]; };
    float kv[4] = {0.f, 0.f, 0.f, 0.f}, qs[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const float kr = k_row(r), qr = q_row(r);
      kv[0] += kr * st[r].x; kv[1] += kr * st[r].y; kv[2] += kr * st[r].z; kv[3] += kr * st[r].w;
      qs[0] += qr * st[r].x; qs[1] += qr * st[r].y; qs[2] += qr * st[r].z; qs[3] += qr * st[r].w;
    }
    const float4 v4 = *(const float4*)(&s_v[ib][hh][col]);
    const float vv[4] = {v4.x, v4.y, v4.z, v4.w};
    float dl[4], o[4], ss = 0.f;
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      const float skv = rows_sum(kv[c]), sqs = rows_sum(qs[c]);
      dl[c] = beta * (vv[c] - alpha * skv);
      o[c] = alpha * sqs + qk * dl[c];
      ss += o[c] * o[c];
    }
    // S' = alpha S + k delta^T, stored as soon as formed (row offset in the lane offset:
    // the compiler lets a store of more than 64 bits with a register scalar offset have its
    // data registers overwritten right after issue, which gfx950 does not tolerate)
    const auto r_ = state_rsrc(t, hh);
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const float kr = k_row(r);
      const float nx = alpha * st[r].x + kr * dl[0], ny = alpha * st[r].y + kr * dl[1];
      const float nz = alpha * st[r].z + kr * dl[2], nw_ = alpha * st[r].w + kr * dl[3];
      __builtin_amdgcn_raw_buffer_store_b128(
          u32x4w{__float_as_uint(nx), __float_as_uint(ny), __float_as_uint(nz), __float_as_uint(nw_)},
          r_, st_off(r), 0, CP);
    }
    // gated RMSNorm on the fp32 core output (deltanet.py:282-293): the row statistic sums
    // the four wavefronts' column sums
    ss = group_sum_dpp<CGS>(ss);
    if (lane == 0) s_ss[ub][wave] = ss;
    lds_barrier();
    const float rn = rsqrtf((s_ss[ub][0] + s_ss[ub][1] + s_ss[ub][2] + s_ss[ub][3]) / DV + eps);
    const float4 sz = sz_i[hh];
    const auto orr = buf_rsrc((bf16_t*)p.out + ((size_t)t.b * Hv + t.hk * GQA + hh) * DV,
                              t.ok ? 2u * DV : 0u);
    const u32x2w ov{pack_bf16(nw.x * (o[0] * rn) * sz.x, nw.y * (o[1] * rn) * sz.y),
                    pack_bf16(nw.z * (o[2] * rn) * sz.z, nw.w * (o[3] * rn) * sz.w)};
    // one lane per column group stores (the row groups hold the same values)
    __builtin_amdgcn_raw_buffer_store_b64(ov, orr, rg == 0 ? 2u * (unsigned)col : kDrop, 0, 0);
  };

  if (my_items <= 0) return;
  float4 sa[R], sb[R];
  load_small(0);
  if constexpr (GQA == 2) {
    load_state(0, 0, sa);
    load_state(0, 1, sb);
    for (int i = 0; i < my_items; ++i) {
      conv_item(i);
      run_unit(i, 0, 0, sa);
      load_state(i + 1, 0, sa);
      run_unit(i, 1, 1, sb);
      load_state(i + 1, 1, sb);
    }
  } else {
    load_state(0, 0, sa);
    load_state(1, 0, sb);
    for (int i = 0; i < my_items; i += 2) {  // an odd count runs one stand-in item
      conv_item(i);
      run_unit(i, 0, 0, sa);
      load_state(i + 2, 0, sa);
      conv_item(i + 1);
      run_unit(i + 1, 0, 1, sb);
      load_state(i + 3, 0, sb);
    }
  }
}

// Grid of the stream kernel: as many workgroups as the chip holds at once (its occupancy,
// queried once per device), with the items dealt evenly (every workgroup gets the same
// count, or one less).  With at least 8 items per CU one workgroup per CU streams faster
// (C2 B=256, 4,096 items: 190-191 us against 195 us with two per CU; at B=64, 1,024 items,
// two per CU stay faster: 53.1-53.6 against 54.1-54.2 us).
template <int DK, int DV, int GQA, bool NT>
int stream_grid(int n_items) {
  static int per_cu[64] = {};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) dev = 0;
  if (per_cu[dev] == 0) {
    int v = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&v, decode_stream_kernel<DK, DV, GQA, NT>,
                                                     kThreads, 0) != hipSuccess || v <= 0)
      v = 1;
    per_cu[dev] = v;
  }
  int cus = 0;
  if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0)
    cus = 256;
  if (n_items >= 8 * cus) return cus;
  const long long cap = (long long)cus * per_cu[dev];
  const long long rounds = (n_items + cap - 1) / cap;
  return (int)((n_items + rounds - 1) / rounds);
}

template <int DK, int DV>
constexpr bool stream_dims() {
  return (DV == 64 || DV == 128) && DK % (64 / (DV / 16)) == 0;
}

template <int DK, int DV, int GQA, bool NT>
void launch_stream(const DecodeParams& p, hipStream_t stream) {
  const int n_items = p.B * p.Hk;
  hipLaunchKernelGGL((decode_stream_kernel<DK, DV, GQA, NT>),
                     dim3(stream_grid<DK, DV, GQA, NT>(n_items)), dim3(kThreads), 0, stream, p);
}

template <int DK, int DV, bool NT, bool EARLY>
void launch_cfg(const DecodeParams& p, bool layer, bool in_bf16, hipStream_t stream) {
  dim3 grid(p.Hk, p.B);
  const int gqa = p.Hv / p.Hk;
  const bool pre = p.conv_k == 4 && gqa <= kPreHeads && 2 * DK + gqa * DV <= kPreChannels * kThreads;
  if constexpr (stream_dims<DK, DV>()) {
    if (layer && pre) {
      if constexpr (2 * DK + 2 * DV <= kPreChannels * kThreads) {
        if (gqa == 2) {
          launch_stream<DK, DV, 2, NT>(p, stream);
          return;
        }
      }
      if (gqa == 1) {
        launch_stream<DK, DV, 1, NT>(p, stream);
        return;
      }
    }
  }
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
