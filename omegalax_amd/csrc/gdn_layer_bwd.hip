// Backward pass of the GatedDeltaNet layer prefill (omx_gdn_prefill_bwd): the parts
// around the chunked rule's backward (gdn_bwd.hip).
//
// Forward (deltanet.py:243-293, between the projections and out_proj):
//   u = conv(x, w) (causal depthwise, K = 4, bf16), y = silu(u) (bf16), y = [q | k | v];
//   beta = sigmoid(b) (bf16), g = -exp(A_log) softplus(a + dt_bias);
//   o = chunk_gated_delta_rule(q, k, v, g, beta) (fp32);
//   out = w_n * o * rsqrt(mean(o^2) + eps) * silu(z).
// Kernels here, in the order the backward runs them:
//   conv_silu_split_kernel  y from x and w, as the forward's prep computes it, into
//                           separate q, k, v rows for the rule's backward;
//   gates_kernel            g and beta per (token, value head);
//   norm_bwd_kernel         the gated RMSNorm's adjoint: do, dz and per-workgroup partial
//                           sums of dw_n (o comes from the rule's recompute scan);
//   gates_bwd_kernel        da, db and per-workgroup partial sums of dA_log, d dt_bias;
//   conv_bwd_kernel         du = dy silu'(u), dx (the transposed conv) and per-token-block
//                           partial sums of dw;
//   col_reduce_kernel       the partial sums in a fixed order (deterministic results).
// Dtype casts are differentiated as the identity, as autodiff does.
#include "gdn_chunk.h"
#include "gdn_kernels.h"

namespace omx {

namespace {

constexpr int NT = 256;

// Sequence bounds of token t: packed sequences (cu_seqlens, clamped by seq_range) or batch
// rows of length T.
__device__ __forceinline__ void token_seq(const int32_t* cu, int N, int T, long long t,
                                          long long& s0, long long& s1) {
  if (cu) {
    int lo = 0, hi = N;  // the last n with cu[n] <= t
    while (hi - lo > 1) {
      const int mid = (lo + hi) >> 1;
      if (cu[mid] <= t) lo = mid;
      else hi = mid;
    }
    seq_range(cu, lo, T, s0, s1);
  } else {
    s0 = (t / T) * T;
    s1 = s0 + T;
  }
}

// conv weights of channels c0 .. c0+7 cast to bf16 (deltanet.py:243): wt[e][d] multiplies
// the input d tokens back (tap K-1-d); K = 4
__device__ __forceinline__ void conv_w8(const float* w, int c0, float (*wt)[4]) {
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    const float4 x = *(const float4*)(w + (size_t)(c0 + e) * 4);
    wt[e][0] = round_bf(x.w);
    wt[e][1] = round_bf(x.z);
    wt[e][2] = round_bf(x.y);
    wt[e][3] = round_bf(x.x);
  }
}

__device__ __forceinline__ void load8(const bf16_t* p, float* x) {
  const u32x4 w = *(const u32x4*)p;
  unpack8<false>(&w, x);
}

__device__ __forceinline__ void zero8(float* x) {
#pragma unroll
  for (int e = 0; e < 8; ++e) x[e] = 0.f;
}

// the forward's conv pre-activation, computed and rounded to bf16 as there (the inputs
// and the weights wt are bf16 values, so the pairs pack exactly)
__device__ __forceinline__ float conv_u(const float* wt, float x0, float x1, float x2, float x3) {
  return round_bf(dot4_bf16(pack_bf16(wt[0], wt[1]), pack_bf16(wt[2], wt[3]), pack_bf16(x0, x1),
                            pack_bf16(x2, x3)));
}

// d silu(u) / du
__device__ __forceinline__ float silu_grad(float u) {
  // sigmoid from the hardware exp2 and reciprocal (about 2 ulp in fp32)
  const float s = __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(u * -1.4426950408889634f));
  return s * (1.0f + u * (1.0f - s));
}

// ---------------------------------------------------------------------------- forward pieces

// One thread per (16-token block, 8-channel group): the weights and the last three inputs
// stay in registers while it streams down the block's tokens (every input read once plus a
// 3-token halo).
constexpr int kConvFwdTB = 16;

__global__ __launch_bounds__(NT) void conv_silu_split_kernel(LayerBwdParams p) {
  const int G = p.conv_dim / 8;
  const long long nblk = (p.tokens + kConvFwdTB - 1) / kConvFwdTB;
  const long long idx = (long long)blockIdx.x * NT + threadIdx.x;
  if (idx >= nblk * G) return;
  const long long tb = (idx / G) * kConvFwdTB;
  const long long te = tb + kConvFwdTB < p.tokens ? tb + kConvFwdTB : p.tokens;
  const int c0 = 8 * (int)(idx % G);
  float wt[8][4];
  conv_w8(p.conv_w, c0, wt);
  const int kd = p.Hk * p.dk;
  bf16_t* dst;
  long long ld;
  if (c0 < kd) { dst = p.q + c0; ld = kd; }
  else if (c0 < 2 * kd) { dst = p.k + (c0 - kd); ld = kd; }
  else { dst = p.v + (c0 - 2 * kd); ld = (long long)p.Hv * p.dv; }
  long long s0, s1;
  token_seq(p.cu_seqlens, p.N, p.T, tb, s0, s1);
  float xs[4][8];  // inputs d tokens back
#pragma unroll
  for (int d = 1; d < 4; ++d) {
    if (tb - d >= s0) load8(p.x + (tb - d) * p.conv_dim + c0, xs[d]);
    else zero8(xs[d]);
  }
  // every row of the block is loaded before the first store: one memory round trip per
  // thread.  The loads are unconditional (rows past te reload row te - 1 and are never
  // used), so the compiler can count them and a wait for row m does not also wait for the
  // stores issued before it (the memory counter retires in order).
  u32x4 raw[kConvFwdTB];
#pragma unroll
  for (int m = 0; m < kConvFwdTB; ++m)
    raw[m] = *(const u32x4*)(p.x + (tb + m < te ? tb + m : te - 1) * p.conv_dim + c0);
#pragma unroll
  for (int m = 0; m < kConvFwdTB; ++m) {
    const long long t = tb + m;
    if (t >= te) break;
    if (t >= s1) {  // a new sequence starts at t: no history
      token_seq(p.cu_seqlens, p.N, p.T, t, s0, s1);
#pragma unroll
      for (int d = 1; d < 4; ++d) zero8(xs[d]);
      __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0): the lookup's loads end here
    }
    unpack8<false>(&raw[m], xs[0]);
    float y[8];
#pragma unroll
    for (int e = 0; e < 8; ++e)
      y[e] = round_bf(silu_fast(conv_u(wt[e], xs[0][e], xs[1][e], xs[2][e], xs[3][e])));
    *(u32x4*)(dst + t * ld) = pack8(y);
#pragma unroll
    for (int d = 3; d > 0; --d)
#pragma unroll
      for (int e = 0; e < 8; ++e) xs[d][e] = xs[d - 1][e];
  }
}

// one thread per (token, value head): g and beta as the forward's prep forms them
__global__ __launch_bounds__(NT) void gates_kernel(LayerBwdParams p) {
  const long long idx = (long long)blockIdx.x * NT + threadIdx.x;
  if (idx >= p.tokens * p.Hv) return;
  const int h = (int)(idx % p.Hv);
  p.g[idx] = -expf(p.A_log[h]) * softplusf_(bf2f(p.a[idx]) + p.dt_bias[h]);
  p.beta[idx] = round_bf(sigmoidf_(bf2f(p.b[idx])));
}

// ---------------------------------------------------------------------------- gated RMSNorm

// Persistent: each wavefront walks (token, value head) rows of dv <= 128 (lane l: columns
// 2l and 2l + 1, so o and dO move 8 bytes and z, dout, dz 4 bytes per lane).
// n = o r, r = (mean(o^2) + eps)^-1/2, out = w n silu(z):
//   dn = dout w silu(z), dz = dout w n silu'(z), dw = sum dout n silu(z),
//   do = r (dn - n mean(dn n)).
// sigmoid(z) comes from the hardware exp2 and reciprocal (about 2 ulp in fp32).
__global__ __launch_bounds__(NT) void norm_bwd_kernel(LayerBwdParams p) {
  __shared__ float sdw[NT / 64][128];
  const int l = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int dv = p.dv, c = 2 * l;
  const bool in = c < dv;  // dv is even
  const long long rows = p.tokens * p.Hv;
  const long long nw = (long long)gridDim.x * (NT / 64);
  float w[2], dw[2] = {0.f, 0.f};
#pragma unroll
  for (int e = 0; e < 2; ++e) w[e] = in ? p.norm_w[c + e] : 0.f;
  for (long long r = (long long)blockIdx.x * (NT / 64) + wave; r < rows; r += nw) {
    float o[2] = {0.f, 0.f}, z[2] = {0.f, 0.f}, go[2] = {0.f, 0.f};
    if (in) {
      const float2 ov = *(const float2*)(p.o + r * dv + c);
      const uint32_t zv = *(const uint32_t*)(p.z + r * dv + c);
      const uint32_t gv = *(const uint32_t*)(p.dout + r * dv + c);
      o[0] = ov.x; o[1] = ov.y;
      z[0] = __uint_as_float(zv << 16); z[1] = __uint_as_float(zv & 0xffff0000u);
      go[0] = __uint_as_float(gv << 16); go[1] = __uint_as_float(gv & 0xffff0000u);
    }
    float ss = o[0] * o[0] + o[1] * o[1];
#pragma unroll
    for (int s = 1; s < 64; s <<= 1) ss += __shfl_xor(ss, s);
    const float rr = rsqrtf(ss / (float)p.dv_mean + p.eps);
    float n[2], dn[2], dzv[2], dnn = 0.f;
#pragma unroll
    for (int e = 0; e < 2; ++e) {
      n[e] = o[e] * rr;
      const float sg = __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(z[e] * -1.4426950408889634f));
      const float sz = z[e] * sg;                       // silu(z)
      const float sgrad = sg * (1.0f + z[e] * (1.0f - sg));  // silu'(z)
      dn[e] = go[e] * w[e] * sz;
      dnn += dn[e] * n[e];
      dw[e] += go[e] * n[e] * sz;
      dzv[e] = go[e] * w[e] * n[e] * sgrad;
    }
#pragma unroll
    for (int s = 1; s < 64; s <<= 1) dnn += __shfl_xor(dnn, s);
    const float m = dnn / (float)p.dv_mean;
    if (in) {
      *(uint32_t*)(p.dz + r * dv + c) = pack_bf16(dzv[0], dzv[1]);
      *(float2*)(p.dO + r * dv + c) = float2{rr * (dn[0] - n[0] * m), rr * (dn[1] - n[1] * m)};
    }
  }
#pragma unroll
  for (int e = 0; e < 2; ++e)
    if (in) sdw[wave][c + e] = dw[e];
  __syncthreads();
  if (threadIdx.x < dv) {
    float s = 0.f;
#pragma unroll
    for (int v = 0; v < NT / 64; ++v) s += sdw[v][threadIdx.x];
    p.part_norm[(size_t)blockIdx.x * dv + threadIdx.x] = s;
  }
}

// ---------------------------------------------------------------------------- gates

// Workgroup w takes a contiguous token range; thread (j, h) = (tid / Hv, tid % Hv) walks its
// tokens j, j + R, ... (R = 256 / Hv) for value head h.
//   da = dg A sigmoid(a + dt_bias), A = -exp(A_log); db = dbeta sigmoid(b)(1 - sigmoid(b));
//   dA_log = sum dg g, d dt_bias = sum da.
__global__ __launch_bounds__(NT) void gates_bwd_kernel(LayerBwdParams p, long long per) {
  __shared__ float sacc[NT][2];
  const int Hv = p.Hv, tid = threadIdx.x;
  const int R = NT / Hv;
  const int h = tid % Hv, j = tid / Hv;
  float sA = 0.f, sdt = 0.f;
  if (j < R) {
    const float A = -expf(p.A_log[h]), dtb = p.dt_bias[h];
    const long long t0 = (long long)blockIdx.x * per;
    const long long t1 = t0 + per < p.tokens ? t0 + per : p.tokens;
    for (long long t = t0 + j; t < t1; t += R) {
      const long long i = t * Hv + h;
      const float dgv = p.dg[i];
      const float da = dgv * A * sigmoidf_(bf2f(p.a[i]) + dtb);
      const float sb = sigmoidf_(bf2f(p.b[i]));
      p.da[i] = f2bf(da);
      p.db[i] = f2bf(p.dbeta[i] * sb * (1.f - sb));
      sA += dgv * p.g[i];
      sdt += da;
    }
  }
  sacc[tid][0] = sA;
  sacc[tid][1] = sdt;
  __syncthreads();
  if (tid < Hv) {
    float a0 = 0.f, a1 = 0.f;
    for (int jj = 0; jj < R; ++jj) {
      a0 += sacc[jj * Hv + tid][0];
      a1 += sacc[jj * Hv + tid][1];
    }
    p.part_gates[(size_t)blockIdx.x * 2 * Hv + tid] = a0;
    p.part_gates[(size_t)blockIdx.x * 2 * Hv + Hv + tid] = a1;
  }
}

// ---------------------------------------------------------------------------- conv + SiLU

// One thread per (64-token block, 8-channel group).  du = dy silu'(u) with u recomputed;
// dx[s] = sum_d wt[d] du[s + d] over s + d inside s's sequence (the transposed conv);
// dwt[d] = sum_t du[t] x[t - d] (x = 0 before the sequence start), written per token block.
constexpr int kConvTB = 64;

__global__ __launch_bounds__(NT) void conv_bwd_kernel(LayerBwdParams p) {
  const int G = p.conv_dim / 8;
  const long long nblk = (p.tokens + kConvTB - 1) / kConvTB;
  const long long idx = (long long)blockIdx.x * NT + threadIdx.x;
  if (idx >= nblk * G) return;
  const long long blk = idx / G;
  const int c0 = 8 * (int)(idx % G);
  const int kd = p.Hk * p.dk;
  const long long vd = (long long)p.Hv * p.dv;
  const bf16_t* dys;
  long long dy_ld;
  int dy_c;
  if (c0 < kd) { dys = p.grad_q; dy_ld = kd; dy_c = c0; }
  else if (c0 < 2 * kd) { dys = p.grad_k; dy_ld = kd; dy_c = c0 - kd; }
  else { dys = p.grad_v; dy_ld = vd; dy_c = c0 - 2 * kd; }
  float wt[8][4];
  conv_w8(p.conv_w, c0, wt);
  const long long tb = blk * kConvTB;
  const long long te = tb + kConvTB < p.tokens ? tb + kConvTB : p.tokens;
  float dwt[8][4];
#pragma unroll
  for (int e = 0; e < 8; ++e)
#pragma unroll
    for (int d = 0; d < 4; ++d) dwt[e][d] = 0.f;
  // rolling windows: xs[d] = x[t - d]; dus[d] = du[t - d] (the last four du computed)
  float xs[4][8], dus[4][8];
#pragma unroll
  for (int d = 0; d < 4; ++d) {
    zero8(xs[d]);
    zero8(dus[d]);
  }
  long long cs0, cs1;  // sequence of the current token t
  token_seq(p.cu_seqlens, p.N, p.T, tb, cs0, cs1);
#pragma unroll
  for (int d = 1; d < 4; ++d)
    if (tb - d >= cs0) load8(p.x + (tb - d) * p.conv_dim + c0, xs[d]);
  // ends[d]: the end of token t - d's sequence (the rows a dx term may reach)
  long long ends[4] = {cs1, cs1, cs1, cs1};
  const long long tend = te + 3 < p.tokens ? te + 3 : p.tokens;
  // The next token's x and dy rows are loaded one iteration ahead, unconditionally (the
  // last iteration reloads its own row), and every iteration stores one dx row (see
  // below): no memory operation sits under a per-thread branch, which would leave the
  // count of outstanding operations unknown and make each wait for a load cover the
  // stores as well.  The loads before the loop have landed.
  u32x4 nx = *(const u32x4*)(p.x + tb * p.conv_dim + c0);
  u32x4 ndy = *(const u32x4*)(dys + tb * dy_ld + dy_c);
  __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0)
  for (long long t = tb; t < tend; ++t) {
    const u32x4 cx = nx, cdy = ndy;
    {
      const long long tn = t + 1 < tend ? t + 1 : t;
      nx = *(const u32x4*)(p.x + tn * p.conv_dim + c0);
      ndy = *(const u32x4*)(dys + tn * dy_ld + dy_c);
    }
    if (t >= cs1) {  // a new sequence starts at t: no history
      token_seq(p.cu_seqlens, p.N, p.T, t, cs0, cs1);
#pragma unroll
      for (int d = 1; d < 4; ++d) zero8(xs[d]);
      __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0): the lookup's loads end here
    }
#pragma unroll
    for (int d = 3; d > 0; --d) ends[d] = ends[d - 1];
    ends[0] = cs1;
    unpack8<false>(&cx, xs[0]);
    float dy[8];
    unpack8<false>(&cdy, dy);
    float du[8];
#pragma unroll
    for (int e = 0; e < 8; ++e)
      du[e] = dy[e] * silu_grad(conv_u(wt[e], xs[0][e], xs[1][e], xs[2][e], xs[3][e]));
    if (t < te) {
#pragma unroll
      for (int e = 0; e < 8; ++e)
#pragma unroll
        for (int d = 0; d < 4; ++d) dwt[e][d] += du[e] * xs[d][e];
    }
    // shift the du window; a sequence boundary cuts it (du of another sequence is 0 here)
#pragma unroll
    for (int d = 3; d > 0; --d)
#pragma unroll
      for (int e = 0; e < 8; ++e) dus[d][e] = dus[d - 1][e];
#pragma unroll
    for (int e = 0; e < 8; ++e) dus[0][e] = du[e];
    // dx[s] for s = t - 3 needs du[s .. s + 3] = dus[3 .. 0]; terms past s's sequence end
    // are dropped (tokens s + d >= end(s) belong to the next sequence)
    // (s < te always: t < te + 3.)  Rows s < tb (the first three iterations) store to
    // row tb instead, which this thread writes again later (here or in the tail below),
    // so the store need not sit under a branch.
    const long long s = t - 3;
    {
      const long long ss1 = ends[3];  // end of s's sequence
      float dx[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        float acc = 0.f;
#pragma unroll
        for (int d = 0; d < 4; ++d)
          if (s + d < ss1) acc += wt[e][d] * dus[3 - d][e];
        dx[e] = acc;
      }
      const long long sw = s >= tb ? s : tb;
      *(u32x4*)(p.dx + sw * p.conv_dim + c0) = pack8(dx);
    }
#pragma unroll
    for (int d = 3; d > 0; --d)
#pragma unroll
      for (int e = 0; e < 8; ++e) xs[d][e] = xs[d - 1][e];
  }
  // the block's last tokens whose du window runs past the end of all tokens
  for (long long s = (te - 3 > tb ? te - 3 : tb); s < te; ++s) {
    if (s + 3 < tend) continue;  // already written in the loop
    long long ss0, ss1;
    token_seq(p.cu_seqlens, p.N, p.T, s, ss0, ss1);
    const long long last = tend - 1;  // dus[0] holds du[last]
    float dx[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      float acc = 0.f;
#pragma unroll
      for (int d = 0; d < 4; ++d) {
        const long long tt = s + d;
        const int back = (int)(last - tt);
        if (tt < ss1 && tt <= last && back < 4) {
          float v = 0.f;
#pragma unroll
          for (int b = 0; b < 4; ++b)
            if (b == back) v = dus[b][e];
          acc += wt[e][d] * v;
        }
      }
      dx[e] = acc;
    }
    *(u32x4*)(p.dx + s * p.conv_dim + c0) = pack8(dx);
  }
  // partial dw in [c][k] order (k = 3 - d)
  float* part = p.part_conv + (size_t)blk * p.conv_dim * 4 + (size_t)c0 * 4;
#pragma unroll
  for (int e = 0; e < 8; ++e)
    *(float4*)(part + 4 * e) = float4{dwt[e][3], dwt[e][2], dwt[e][1], dwt[e][0]};
}

// out[c] = sum over rows r of part[r * stride + off + c], c < ncols: COLS columns per
// workgroup and NT / COLS row groups (rows r = rg mod NT/COLS), each summing its rows into
// four accumulators; the partial sums are combined in a fixed order, so the result does not
// depend on timing.
template <int COLS>
__global__ __launch_bounds__(NT) void col_reduce_kernel(const float* part, long long nrows,
                                                        int stride, int off, int ncols, float* out) {
  constexpr int RG = NT / COLS;
  __shared__ float s_part[RG][COLS];
  const int cl = threadIdx.x % COLS, rg = threadIdx.x / COLS;
  const int c = blockIdx.x * COLS + cl;
  float acc[4] = {0.f, 0.f, 0.f, 0.f};
  if (c < ncols) {
    long long r = rg;
    for (; r + 3 * RG < nrows; r += 4 * RG) {
#pragma unroll
      for (int u = 0; u < 4; ++u) acc[u] += part[(r + u * RG) * stride + off + c];
    }
    for (; r < nrows; r += RG) acc[0] += part[r * stride + off + c];
  }
  s_part[rg][cl] = (acc[0] + acc[1]) + (acc[2] + acc[3]);
  __syncthreads();
  if (rg == 0 && c < ncols) {
    float t = 0.f;
    for (int g = 0; g < RG; ++g) t += s_part[g][cl];
    out[c] = t;
  }
}

// narrow column groups (more row groups) for the few-column reductions
void launch_col_reduce(const float* part, long long nrows, int stride, int off, int ncols,
                       float* out, hipStream_t stream) {
  if (ncols <= 2048)
    hipLaunchKernelGGL((col_reduce_kernel<8>), dim3((ncols + 7) / 8), dim3(NT), 0, stream, part,
                       nrows, stride, off, ncols, out);
  else
    hipLaunchKernelGGL((col_reduce_kernel<32>), dim3((ncols + 31) / 32), dim3(NT), 0, stream, part,
                       nrows, stride, off, ncols, out);
}

}  // namespace

int layer_bwd_norm_blocks() { return 4096; }

long long layer_bwd_conv_blocks(long long tokens) { return (tokens + kConvTB - 1) / kConvTB; }

int layer_bwd_gate_blocks(long long tokens) {
  const long long b = (tokens + 255) / 256;
  return (int)(b < 1024 ? (b < 1 ? 1 : b) : 1024);
}

hipError_t launch_layer_fwd_pieces(const LayerBwdParams& p, hipStream_t stream) {
  const long long n1 = (p.tokens + kConvFwdTB - 1) / kConvFwdTB * (p.conv_dim / 8);
  if (n1 > 0) {
    hipLaunchKernelGGL(conv_silu_split_kernel, dim3((unsigned)((n1 + NT - 1) / NT)), dim3(NT), 0,
                       stream, p);
    const long long n2 = p.tokens * p.Hv;
    hipLaunchKernelGGL(gates_kernel, dim3((unsigned)((n2 + NT - 1) / NT)), dim3(NT), 0, stream, p);
  }
  return hipGetLastError();
}

hipError_t launch_layer_norm_bwd(const LayerBwdParams& p, hipStream_t stream) {
  hipLaunchKernelGGL(norm_bwd_kernel, dim3(layer_bwd_norm_blocks()), dim3(NT), 0, stream, p);
  launch_col_reduce(p.part_norm, layer_bwd_norm_blocks(), p.dv, 0, p.dv, p.d_norm_w, stream);
  return hipGetLastError();
}

hipError_t launch_layer_tail_bwd(const LayerBwdParams& p, hipStream_t stream) {
  const int gb = layer_bwd_gate_blocks(p.tokens);
  const long long per = (p.tokens + gb - 1) / gb;
  hipLaunchKernelGGL(gates_bwd_kernel, dim3(gb), dim3(NT), 0, stream, p, per);
  launch_col_reduce(p.part_gates, gb, 2 * p.Hv, 0, p.Hv, p.dA_log, stream);
  launch_col_reduce(p.part_gates, gb, 2 * p.Hv, p.Hv, p.Hv, p.d_dt_bias, stream);
  const long long nblk = layer_bwd_conv_blocks(p.tokens);
  const long long n = nblk * (p.conv_dim / 8);
  if (n > 0)
    hipLaunchKernelGGL(conv_bwd_kernel, dim3((unsigned)((n + NT - 1) / NT)), dim3(NT), 0, stream, p);
  launch_col_reduce(p.part_conv, nblk, p.conv_dim * 4, 0, p.conv_dim * 4, p.d_conv_w, stream);
  return hipGetLastError();
}

}  // namespace omx
