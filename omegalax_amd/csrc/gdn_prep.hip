// Chunk-parallel preparation for the chunked gated delta rule on gfx950.
//
// Everything in a chunk of chunk_gated_delta_rule (omegalax/models/qwen3_5/
// deltanet.py:53-153) that does not depend on the recurrent state is computed
// here, for all chunks at once, one workgroup per (chunk, key head):
//   * q, k rows: (layer path) causal depthwise conv + SiLU (deltanet.py:35-50,
//     243), then the L2 norm at input precision (:30-32, 65-66); written to the
//     workspace for the scan.  (layer path) v rows: conv + SiLU, written likewise.
//   * the Gram products K K^T and Q K^T of the key head, once for all gqa value
//     heads that share it (the repeat-interleave of :272-280);
//   * per value head: the gates (:248-250 on the layer path), G = cumsum(g)
//     (:98), L = strict_lower(beta_i (k_i.k_j) e^{G_i-G_j}) (:100-108),
//     T = (I + L)^-1 (:110-113), P = lower(scale (q_i.k_j) e^{G_i-G_j}) (:130-131).
// T is formed by blocks: each wavefront inverts one 16x16 diagonal block by
// forward substitution, then wavefront j runs down block column j,
//     T_ij = -T_ii sum_{k=j}^{i-1} L_ik T_kj,
// on 16x16x16 MFMAs with hi+lo bf16 operands (fp32-accurate products).  The
// outputs go to the per-(chunk, value head) record described in gdn_chunk.h.
#include "gdn_chunk.h"
#include "gdn_kernels.h"

namespace omx {

namespace {

constexpr int C = kC, NT = kNT, LDT = kLDT, LDD = kLDD;

template <int DK, int MODE>
struct PrepCfg {
  static constexpr bool IS = MODE == MODE_F32;  // q/k split hi+lo
  static constexpr int NS = IS ? 2 : 1;
  static constexpr int RAWW = IS ? 2 : 1;
  static constexpr int LDK = DK + 8;
  static constexpr int SEGS = DK / 8;
  static constexpr int NI_KQ = 2 * C * SEGS / NT;
  static_assert(NI_KQ * NT == 2 * C * SEGS && (C * SEGS) % NT == 0, "item split");
  static_assert(DK % 32 == 0 && DK <= 128, "dk");
};

// The 20 lower-triangular 16x16 tiles of K K^T (0..9, diagonal first) and Q K^T
// (10..19), each coded in 5 bits as qk << 4 | row block << 2 | col block and
// packed into two words, so a wave decodes its tiles with scalar shifts.
// Wavefront w takes tiles w, w+4, ..., w+16: slot 0 is its diagonal K K^T tile.
constexpr int kTileList[20] = {0x00, 0x05, 0x0A, 0x0F, 0x04, 0x08, 0x09, 0x0C, 0x0D, 0x0E,
                               0x10, 0x14, 0x15, 0x18, 0x19, 0x1A, 0x1C, 0x1D, 0x1E, 0x1F};
constexpr unsigned long long pack_tiles(int first, int count) {
  unsigned long long w = 0;
  for (int t = 0; t < count; ++t) w |= (unsigned long long)kTileList[first + t] << (5 * t);
  return w;
}
constexpr unsigned long long kTilesLo = pack_tiles(0, 12), kTilesHi = pack_tiles(12, 8);

__device__ __forceinline__ int tile_code(int t) {
  return t < 12 ? (int)((kTilesLo >> (5 * t)) & 31) : (int)((kTilesHi >> (5 * (t - 12))) & 31);
}

// Causal depthwise conv + SiLU of 8 consecutive channels ch0.. at token row r of
// the chunk (deltanet.py:35-50, 243): taps reach back K-1 tokens, into
// conv_state_in (or zeros) before the sequence start.  Inputs, weights (cast to
// bf16 as at :243), the conv sum and the SiLU output are rounded to bf16 like the
// reference's bf16 ops; the sum itself accumulates in fp32.
__device__ __forceinline__ void conv8(const ChunkParams& p, int n, long long s0, long long tok,
                                      int ch0, const float (*wt)[4], float* y) {
  const int K = p.conv_k;
  float acc[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) acc[e] = 0.f;
#pragma unroll
  for (int d = 0; d < 4; ++d) {  // token tok - d, weight tap K-1-d
    if (d >= K) break;           // uniform
    const long long t = tok - d;
    float xv[8];
    if (t >= s0) {
      const u32x4 w = *(const u32x4*)((const bf16_t*)p.mixed_qkv + t * p.conv_dim + ch0);
      unpack8<false>(&w, xv);
    } else {
#pragma unroll
      for (int e = 0; e < 8; ++e) xv[e] = 0.f;
      if (p.conv_state_in) {
        const int slot = (K - 1) - (int)(s0 - t);  // cache slot of time t (oldest first)
        const bf16_t* cs = (const bf16_t*)p.conv_state_in + ((size_t)n * p.conv_dim + ch0) * (K - 1);
#pragma unroll
        for (int e = 0; e < 8; ++e) xv[e] = bf2f(cs[e * (K - 1) + slot]);
      }
    }
#pragma unroll
    for (int e = 0; e < 8; ++e) acc[e] += wt[e][d] * xv[e];
  }
#pragma unroll
  for (int e = 0; e < 8; ++e) y[e] = round_bf(siluf_(round_bf(acc[e])));
}

// conv weights of channels ch0..ch0+7, cast to bf16: wt[e][d] multiplies token t - d
__device__ __forceinline__ void load_conv_w(const ChunkParams& p, int ch0, float (*wt)[4]) {
  const int K = p.conv_k;
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    const float* w = p.conv_w + (size_t)(ch0 + e) * K;
#pragma unroll
    for (int d = 0; d < 4; ++d) wt[e][d] = d < K ? round_bf(w[K - 1 - d]) : 0.f;
  }
}

// A C-layout tile (lane (q, r) holds rows 4q..4q+3 of column r) -> its A-operand
// fragment (lane (q, r) holds row r, columns 4q..4q+3), through the wave's
// scratch: stored transposed, read back with ds_read_b64_tr_b16.
__device__ __forceinline__ u32x2 to_afrag(bf16_t* scr, f32x4 x, bool lo) {
  const int l = lane_id();
  const f32x4 y = lo ? f32x4{lo_part(x[0]), lo_part(x[1]), lo_part(x[2]), lo_part(x[3])} : x;
  *(u32x2*)(scr + (l & 15) * LDD + 4 * (l >> 4)) = pack_hi4(y);
  wave_lds_fence();
  const u32x2 f = rows4_tr(scr, LDD, 0, 0);
  wave_lds_fence();  // the next tile may reuse the scratch
  return f;
}

__device__ __forceinline__ void put_tile(unsigned char* rec, int off, u32x2 f) {
  *(u32x2*)(rec + off + lane_id() * 8) = f;
}

template <int DK, int MODE>
__global__ __launch_bounds__(NT) void prep_kernel(ChunkParams p) {
  using Q_ = PrepCfg<DK, MODE>;
  constexpr int LDK = Q_::LDK, SEGS = Q_::SEGS;
  constexpr bool IS = Q_::IS, F32 = MODE == MODE_F32;
  __shared__ __align__(16) bf16_t sK[Q_::NS * C * LDK];   // K rows [token][dk] (hi, lo)
  __shared__ __align__(16) bf16_t sQ[Q_::NS * C * LDK];   // Q rows
  __shared__ __align__(16) bf16_t sLoT[2 * C * LDT];      // L^T off-diagonal blocks [m][i] (hi, lo)
  __shared__ __align__(16) bf16_t sTdT[2 * C * LDD];      // diagonal inverses, transposed (hi, lo)
  __shared__ __align__(16) float sLd[C * LDD];            // diagonal blocks of L (wave w: rows 16w..)
  __shared__ __align__(16) float sGw[4 * 2 * C];          // per wave: G log2(e), beta
  __shared__ __align__(16) bf16_t sX[4 * 16 * LDD];       // per wave: tile transposition
  constexpr int K_LO = C * LDK, LO_LO = C * LDT, TD_LO = C * LDD;

  const int tid = threadIdx.x, l = tid & 63, lq = l >> 4, lr = l & 15;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int hk = (int)(blockIdx.x % (unsigned)p.Hk);
  const int ci = (int)(blockIdx.x / (unsigned)p.Hk);  // global chunk index
  int n, c;
  if (p.chunk_off) {
    if (ci >= p.chunk_off[p.N]) return;  // past the last chunk (uniform)
    int lo = 0, hi = p.N;                // chunk_off[lo] <= ci < chunk_off[hi]
    while (hi - lo > 1) {
      const int mid = (lo + hi) >> 1;
      if (p.chunk_off[mid] <= ci) lo = mid;
      else hi = mid;
    }
    n = lo;
    c = ci - p.chunk_off[n];
  } else {
    n = ci / p.nch;
    c = ci % p.nch;
  }
  long long s0, s1;
  seq_range(p.cu_seqlens, n, p.T, s0, s1);
  const long long t0 = s0 + (long long)c * C;
  const int nvalid = (int)((s1 - t0) < C ? (s1 - t0) : C);
  const int gqa = p.Hv / p.Hk;

  // ---------------------------------------------------------------- q, k rows
  // a thread's items keep one 8-channel segment of k and one of q
  float wk[MODE == MODE_LAYER ? 8 : 1][4], wq[MODE == MODE_LAYER ? 8 : 1][4];
  if constexpr (MODE == MODE_LAYER) {
    const int seg = tid % SEGS;
    load_conv_w(p, p.Hk * DK + hk * DK + seg * 8, wk);
    load_conv_w(p, hk * DK + seg * 8, wq);
  }
#pragma unroll
  for (int k = 0; k < Q_::NI_KQ; ++k) {
    constexpr int PER = C * SEGS;
    const int which = (k * NT) / PER;  // 0 = k, 1 = q (compile time)
    const int rem = (k * NT) % PER + tid;
    const int r = rem / SEGS, seg = rem % SEGS;
    const long long tok = t0 + (r < nvalid ? r : nvalid - 1);  // padded rows: in bounds, zeroed
    float x[8];
    if constexpr (MODE == MODE_LAYER) {
      conv8(p, n, s0, tok, (which == 0 ? p.Hk * DK : 0) + hk * DK + seg * 8, which == 0 ? wk : wq, x);
    } else {
      u32x4 w[Q_::RAWW];
      load_raw<F32>(which == 0 ? p.k : p.q, tok * (which == 0 ? p.k_ld : p.q_ld) + (long long)hk * DK + seg * 8, w);
      unpack8<F32>(w, x);
    }
    const float keep = (float)(r < nvalid);
#pragma unroll
    for (int e = 0; e < 8; ++e) x[e] *= keep;
    if (p.qk_l2norm) {
      float ss = 0.f;
#pragma unroll
      for (int e = 0; e < 8; ++e) ss += x[e] * x[e];
      ss = group_sum_dpp<SEGS>(ss);
      const float inv = rsqrtf(ss + 1e-6f);
#pragma unroll
      for (int e = 0; e < 8; ++e) x[e] *= inv;
    }
    // bf16 inputs: the normalised row is rounded to bf16 (the reference normalises
    // in the input dtype); the pack below does the rounding
    bf16_t* dst = (which == 0 ? sK : sQ) + r * LDK + seg * 8;
    const u32x4 hw = pack8(x);
    *(u32x4*)dst = hw;
    if constexpr (IS) *(u32x4*)(dst + K_LO) = pack8_lo(x);
    void* out = which == 0 ? p.kn : p.qn;
    if (out && r < nvalid) {
      const long long o = (t0 + r) * (long long)p.Hk * DK + (long long)hk * DK + seg * 8;
      if constexpr (F32) {
        float4* d4 = (float4*)((float*)out + o);
        d4[0] = float4{x[0], x[1], x[2], x[3]};
        d4[1] = float4{x[4], x[5], x[6], x[7]};
      } else {
        *(u32x4*)((bf16_t*)out + o) = hw;
      }
    }
  }
  if constexpr (MODE == MODE_LAYER) {
    // v rows of the gqa value heads of this key head: conv + SiLU, bf16
    const int VS = gqa * p.DV / 8;  // 8-channel segments
    const int vch0 = 2 * p.Hk * DK + hk * gqa * p.DV;
    for (int it = tid; it < nvalid * VS; it += NT) {
      const int r = it / VS, sgi = it % VS;
      float y[8], wv[8][4];
      load_conv_w(p, vch0 + 8 * sgi, wv);
      conv8(p, n, s0, t0 + r, vch0 + 8 * sgi, wv, y);
      *(u32x4*)((bf16_t*)p.vc + (t0 + r) * (long long)p.Hv * p.DV + (long long)hk * gqa * p.DV +
                8 * sgi) = pack8(y);
    }
  }
  __syncthreads();

  // ---------------------------------------------------------------- Gram tiles
  f32x4 tacc[5];
#pragma unroll
  for (int ti = 0; ti < 5; ++ti) {
    const int code = tile_code(wave + 4 * ti);
    const bool qk = ti >= 3 || (ti == 2 && wave >= 2);
    const int bi = (code >> 2) & 3, bj = code & 3;
    tacc[ti] = zero4();
#pragma unroll
    for (int s = 0; s < DK / 32; ++s) {
      u32x4 ah, al, bh, bl;
      frag2<IS>(qk ? sQ : sK, K_LO, LDK, 16 * bi, 32 * s, ah, al);
      frag2<IS>(sK, K_LO, LDK, 16 * bj, 32 * s, bh, bl);
      tacc[ti] = mm<IS, IS>(tacc[ti], ah, al, bh, bl);
    }
  }

  float* gw = sGw + wave * 2 * C;  // this wave's G log2(e) [0, C) and beta [C, 2C)
  bf16_t* scr = sX + wave * 16 * LDD;
  const size_t rec_stride = (size_t)rec_bytes(MODE);

  for (int gg = 0; gg < gqa; ++gg) {
    const int h = hk * gqa + gg;
    unsigned char* rec = p.rec + ((size_t)ci * p.Hv + h) * rec_stride;

    // gates of value head h, one token per lane; every wave scans its own copy
    {
      float g = 0.f, bt = 0.f;
      if (l < nvalid) {
        const long long idx = (t0 + l) * p.Hv + h;
        if constexpr (MODE == MODE_LAYER) {
          // deltanet.py:248-250: beta in bf16, g in fp32
          g = -expf(p.A_log[h]) * softplusf_(bf2f(((const bf16_t*)p.a)[idx]) + p.dt_bias[h]);
          bt = round_bf(sigmoidf_(bf2f(((const bf16_t*)p.b)[idx])));
        } else {
          g = p.g[idx];
          bt = p.beta[idx];
        }
      }
      float G = g;
#pragma unroll
      for (int o = 1; o < 64; o <<= 1) {
        const float y = __shfl_up(G, o, 64);
        if (l >= o) G += y;
      }
      const float Gl = __shfl(G, 63, 64);
      const float eg = __expf(G);
      gw[l] = G * 1.4426950408889634f;
      gw[C + l] = bt;
      if (wave == 0) {
        float* rg = (float*)(rec + kRecG);
        rg[kGateBeta * C + l] = bt;
        rg[kGateBE * C + l] = bt * eg;
        rg[kGateEG * C + l] = eg;
        rg[kGateEL * C + l] = __expf(Gl - G);
      }
      wave_lds_fence();
    }

    // gate the wave's Gram tiles: L (strictly lower) and P (lower) blocks
    f32x4 Tw = zero4();  // this wave's diagonal inverse T_ww, C layout
#pragma unroll
    for (int ti = 0; ti < 5; ++ti) {
      const f32x4 acc = tacc[ti];
      const int code = tile_code(wave + 4 * ti);
      const bool qk = ti >= 3 || (ti == 2 && wave >= 2);
      const int bi = (code >> 2) & 3, bj = code & 3;
      const int m = 16 * bj + lr;
      const float Gm = gw[m];
      const float4 Gi = *(const float4*)(gw + 16 * bi + 4 * lq);
      const float gi[4] = {Gi.x, Gi.y, Gi.z, Gi.w};
      f32x4 val;
      if (!qk) {
        const float4 Bi = *(const float4*)(gw + C + 16 * bi + 4 * lq);
        const float bt[4] = {Bi.x, Bi.y, Bi.z, Bi.w};
        // branch-free: the exponent is clamped to <= 0 (masked entries would
        // overflow) and the strictly-lower mask multiplies the result
#pragma unroll
        for (int v = 0; v < 4; ++v) {
          const int i = 16 * bi + 4 * lq + v;
          const float dec = __builtin_amdgcn_exp2f(fminf(gi[v] - Gm, 0.f));
          val[v] = bt[v] * acc[v] * dec * (float)(i > m);
        }
        if (ti == 0) {
          // the diagonal block: T_ww = (I + L_ww)^-1 by forward substitution, one
          // column per lane (lanes 16..63 repeat the columns of lanes 0..15)
#pragma unroll
          for (int v = 0; v < 4; ++v) sLd[(16 * bi + 4 * lq + v) * LDD + lr] = val[v];
          wave_lds_fence();
          const int cc = l & 15;
          float x[16];
#pragma unroll
          for (int i = 0; i < 16; ++i) {
            const float* row = sLd + (16 * bi + i) * LDD;
            float a0 = (i == cc) ? 1.f : 0.f, a1 = 0.f;
#pragma unroll
            for (int mm2 = 0; mm2 < i; mm2 += 4) {
              const float4 r4 = *(const float4*)(row + mm2);
              a0 -= r4.x * x[mm2];
              if (mm2 + 1 < i) a1 -= r4.y * x[mm2 + 1];
              if (mm2 + 2 < i) a0 -= r4.z * x[mm2 + 2];
              if (mm2 + 3 < i) a1 -= r4.w * x[mm2 + 3];
            }
            x[i] = a0 + a1;
          }
          // C layout: lane (q, r) holds rows 4q..4q+3 of column r = its own column
#pragma unroll
          for (int v = 0; v < 4; ++v)
            Tw[v] = lq == 0 ? x[v] : (lq == 1 ? x[4 + v] : (lq == 2 ? x[8 + v] : x[12 + v]));
          if (l < 16) {
            // T_ww^T row cc = column cc of T_ww, hi and lo, for the other waves
            bf16_t* dh = sTdT + (16 * bi + cc) * LDD;
            bf16_t* dl = dh + TD_LO;
#pragma unroll
            for (int h8 = 0; h8 < 2; ++h8) {
              float hv[8];
#pragma unroll
              for (int e = 0; e < 8; ++e) hv[e] = x[8 * h8 + e];
              *(u32x4*)(dh + 8 * h8) = pack8(hv);
              *(u32x4*)(dl + 8 * h8) = pack8_lo(hv);
            }
          }
          const int tw = kRecT + 2 * tile_index(bi, bi) * kTileBytes;
          put_tile(rec, tw, to_afrag(scr, Tw, false));
          put_tile(rec, tw + kTileBytes, to_afrag(scr, Tw, true));
        } else {
          store_ct_split(sLoT, sLoT + LO_LO, LDT, 16 * bi, 16 * bj, val);
        }
      } else {
#pragma unroll
        for (int v = 0; v < 4; ++v) {
          const int i = 16 * bi + 4 * lq + v;
          const float dec = __builtin_amdgcn_exp2f(fminf(gi[v] - Gm, 0.f));
          val[v] = p.scale * acc[v] * dec * (float)(i >= m);
        }
        const int tix = tile_index(bi, bj);
        put_tile(rec, kRecP + tix * kTileBytes, to_afrag(scr, val, false));
        if constexpr (IS) put_tile(rec, kRecPL + tix * kTileBytes, to_afrag(scr, val, true));
      }
    }
    __syncthreads();  // L^T blocks and the diagonal inverses of all waves are in LDS

    // block column j = wave: T_ij = -T_ii sum_{k=j}^{i-1} L_ik T_kj, i = j+1..3
    {
      const int j = wave;
      u32x2 Th[4], Tl[4];  // B operands of the column's finished blocks T_kj
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        Th[k] = pack_hi4(Tw);
        Tl[k] = pack_lo4(Tw);
      }
#pragma unroll
      for (int i = 1; i < 4; ++i) {
        if (i <= j) continue;  // uniform
        f32x4 X = zero4();
#pragma unroll
        for (int k = 0; k < i; ++k) {
          if (k < j) continue;
          const u32x2 ah = rows4_tr(sLoT, LDT, 16 * k, 16 * i);
          const u32x2 al = rows4_tr(sLoT + LO_LO, LDT, 16 * k, 16 * i);
          X = mm3k16(X, ah, al, Th[k], Tl[k]);
        }
        // the A operand T_ii is negated (a sign flip is exact in bf16)
        const u32x2 th = rows4_tr(sTdT, LDD, 16 * i, 0) ^ 0x80008000u;
        const u32x2 tl = rows4_tr(sTdT + TD_LO, LDD, 16 * i, 0) ^ 0x80008000u;
        const f32x4 Tij = mm3k16(zero4(), th, tl, pack_hi4(X), pack_lo4(X));
        Th[i] = pack_hi4(Tij);
        Tl[i] = pack_lo4(Tij);
        const int off = kRecT + 2 * tile_index(i, j) * kTileBytes;
        put_tile(rec, off, to_afrag(scr, Tij, false));
        put_tile(rec, off + kTileBytes, to_afrag(scr, Tij, true));
      }
    }
    __syncthreads();  // sLoT / sTdT are rewritten for the next value head
  }
}

template <int DK, int MODE>
hipError_t launch_prep_cfg(const ChunkParams& p, hipStream_t stream) {
  const unsigned grid = (unsigned)p.n_rec * (unsigned)p.Hk;
  if (grid == 0) return hipSuccess;
  hipLaunchKernelGGL((prep_kernel<DK, MODE>), dim3(grid), dim3(NT), 0, stream, p);
  return hipGetLastError();
}

// chunk_off[n] = sum over m < n of ceil(len_m / 64), chunk_off[N] = the total, with
// each length taken from the clamped range seq_range gives.  One workgroup.
__global__ __launch_bounds__(1024) void chunk_plan_kernel(const int32_t* cu, int N, int T,
                                                          int32_t* off) {
  __shared__ int wsum[16];
  const int tid = threadIdx.x, l = tid & 63, w = tid >> 6;
  int carry = 0;
  for (int base = 0; base < N; base += 1024) {
    const int n = base + tid;
    int cnt = 0;
    if (n < N) {
      long long s0, s1;
      seq_range(cu, n, T, s0, s1);
      cnt = (int)((s1 - s0 + C - 1) / C);
    }
    int x = cnt;  // inclusive scan within the wave
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
      const int y = __shfl_up(x, o, 64);
      if (l >= o) x += y;
    }
    if (l == 63) wsum[w] = x;
    __syncthreads();
    int before = carry;
    for (int v = 0; v < w; ++v) before += wsum[v];
    if (n < N) off[n] = before + x - cnt;
    int total = 0;
    for (int v = 0; v < 16; ++v) total += wsum[v];
    carry += total;
    __syncthreads();
  }
  if (tid == 0) off[N] = carry;
}

}  // namespace

hipError_t launch_chunk_plan(const ChunkParams& p, hipStream_t stream) {
  hipLaunchKernelGGL(chunk_plan_kernel, dim3(1), dim3(1024), 0, stream, p.cu_seqlens, p.N, p.T,
                     p.chunk_off);
  return hipGetLastError();
}

hipError_t launch_prep(const ChunkParams& p, int mode, hipStream_t stream) {
  if (mode == MODE_F32) {
    if (p.dk == 64) return launch_prep_cfg<64, MODE_F32>(p, stream);
    if (p.dk == 32) return launch_prep_cfg<32, MODE_F32>(p, stream);
    return hipErrorInvalidValue;
  }
  if (mode == MODE_LAYER) {
    if (p.dk == 128) return launch_prep_cfg<128, MODE_LAYER>(p, stream);
    if (p.dk == 64) return launch_prep_cfg<64, MODE_LAYER>(p, stream);
    return hipErrorInvalidValue;
  }
  if (p.dk == 128) return launch_prep_cfg<128, MODE_BF16>(p, stream);
  if (p.dk == 64) return launch_prep_cfg<64, MODE_BF16>(p, stream);
  return hipErrorInvalidValue;
}

}  // namespace omx
