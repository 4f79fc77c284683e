// Chunked gated delta rule on gfx950: one kernel for the whole prefill.
//
// Follows chunk_gated_delta_rule (omegalax/models/qwen3_5/deltanet.py:53-153),
// restated for MFMA.  Per chunk of C = 64 tokens, with G the in-chunk cumsum of g
// (:98), L = strict_lower(beta_i (k_i.k_j) e^{G_i-G_j}) (:100-108) and
// T = (I + L)^-1 (the solve_triangular of :110-113):
//     V_new = T diag(beta) V - T diag(beta e^G) (K S)        (:115-116, :133-134)
//     O     = e^G (Q S) scale + P V_new,  P = lower(scale (q_i.k_j) e^{G_i-G_j})  (:130-137)
//     S    <- e^{G_last} S + K^T diag(e^{G_last - G}) V_new   (:139-142)
// (W S is evaluated as T diag(beta e^G) (K S), the same product reassociated.)
//
// Work mapping.  One workgroup per (sequence, value head, dv-block of BV = 16*NWC
// columns) walks that sequence's chunks in order.  Wavefront w owns state
// columns [16w, 16w+16) of the block: its fp32 slice S[dk][16] stays in MFMA
// accumulator registers for the whole sequence, and every product that touches
// it (K S, Q S, V_new, O, the state update) runs on that wavefront alone.  The
// per-chunk work that does not touch S -- staging K, Q, V in LDS, K K^T and Q K^T
// on MFMA, the 64x64 triangular inverse -- is shared by all wavefronts between
// workgroup barriers.
//
// Precision.  MFMA inputs are bf16 with fp32 accumulation.  q, k, v are bf16 on
// the layer path (exact), or fp32 split into hi+lo bf16 pairs (MODE_F32).  T and
// the state-update operand diag(e^{G_last-G}) V_new are always split hi+lo; with
// bf16 inputs S enters K S / Q S, and P, V_new enter P V_new, as single bf16
// (their rounding reaches only the bf16-tolerance output).
//
// Modes: MODE_BF16 / MODE_F32 read q, k, v, g, beta (core function) and store o
// in fp32; MODE_LAYER reads the raw in_proj outputs, applies the causal conv +
// SiLU + L2 norm and the gates in the load stage, and stores the gated-RMSNorm
// output in bf16 (deltanet.py:243-293); it needs BV == dv.
#include <type_traits>

#include "gdn_common.h"
#include "gdn_kernels.h"
#include "gdn_mfma.h"

namespace omx {

namespace {

constexpr int C = 64;        // chunk length (deltanet.py:59)
constexpr int LDT = C + 8;   // row stride (elements) of [x][token] bf16 arrays
constexpr int LDF = C + 4;   // row stride of the fp32 64x64 T array
constexpr int MODE_BF16 = 0, MODE_F32 = 1, MODE_LAYER = 2;

template <int DK, int NWC, int MODE>
struct Cfg {
  static constexpr int NT = 64 * NWC;               // threads
  static constexpr int BV = 16 * NWC;               // state columns per workgroup
  static constexpr bool IS = MODE == MODE_F32;      // q/k/v split hi+lo
  static constexpr bool OS = MODE == MODE_F32;      // output-path operands split
  static constexpr int NS = IS ? 2 : 1;
  static constexpr int LDK = DK + 8;                // row stride of [token][dk] arrays
  // shared arrays (bytes)
  static constexpr int SZ_K = NS * C * LDK * 2;
  static constexpr int SZ_KT = NS * DK * LDT * 2;
  static constexpr int SZ_VT = NS * BV * LDT * 2;
  static constexpr int SZ_T = C * LDF * 4;
  static constexpr int SZ_P = (OS ? 2 : 1) * C * LDT * 2;
  static constexpr int SZ_SC = 8 * C * 4;
  // per-wave scratch: S^T (start of phase B), then K S^T, then V_new^T + Vt^T hi/lo
  static constexpr int WS_S = NS * 16 * LDK * 2;
  static constexpr int WS_KS = NS * 16 * LDT * 2;
  static constexpr int WS_V = ((OS ? 2 : 1) + 2) * 16 * LDT * 2;
  static constexpr int WS = WS_S > WS_V ? (WS_S > WS_KS ? WS_S : WS_KS) : (WS_V > WS_KS ? WS_V : WS_KS);
  static constexpr int SZ_W = NWC * WS;
  // layer mode: raw conv history (K-1 = 3 rows of q|k|v-block) and norm partial sums
  static constexpr int HIST_W = 2 * DK + BV;
  static constexpr int SZ_H = MODE == MODE_LAYER ? 3 * HIST_W * 2 : 0;
  static constexpr int SZ_NP = MODE == MODE_LAYER ? C * NWC * 4 : 0;
  static constexpr int OFF_K = 0;
  static constexpr int OFF_Q = OFF_K + SZ_K;
  static constexpr int OFF_KT = OFF_Q + SZ_K;
  static constexpr int OFF_VT = OFF_KT + SZ_KT;
  static constexpr int OFF_T = OFF_VT + SZ_VT;
  static constexpr int OFF_P = OFF_T + SZ_T;
  static constexpr int OFF_SC = OFF_P + SZ_P;
  static constexpr int OFF_W = OFF_SC + SZ_SC;
  static constexpr int OFF_H = OFF_W + SZ_W;
  static constexpr int OFF_NP = OFF_H + SZ_H;
  static constexpr int TOTAL = OFF_NP + SZ_NP;
  static_assert(TOTAL <= 160 * 1024, "LDS budget");
  static_assert(SZ_W >= 32 * 33 * 4, "T-merge temp lives in the wave scratch");
  static_assert(DK % 32 == 0 && DK <= 128, "dk");
};

// lower-triangular 16x16 tiles of a 64x64 matrix, (row block, col block)
__constant__ int kTri[10][2] = {{0, 0}, {1, 0}, {1, 1}, {2, 0}, {2, 1},
                                {2, 2}, {3, 0}, {3, 1}, {3, 2}, {3, 3}};

template <bool AS, bool BS>
__device__ __forceinline__ f32x4 mm(f32x4 acc, u32x4 ah, u32x4 al, u32x4 bh, u32x4 bl) {
  acc = mma16(ah, bh, acc);
  if constexpr (BS) acc = mma16(ah, bl, acc);
  if constexpr (AS) acc = mma16(al, bh, acc);
  return acc;
}

// hi/lo fragment pair from a bf16 array pair (lo array at +lo_off elements).
template <bool SPLIT>
__device__ __forceinline__ void frag2(const bf16_t* base, int lo_off, int ld, int row0, int k0,
                                      u32x4& hi, u32x4& lo) {
  hi = frag_bf16(base, ld, row0, k0);
  if constexpr (SPLIT) lo = frag_bf16(base + lo_off, ld, row0, k0);
  else lo = hi;
}

// A fragment of T diag(colscale) (negated if NEG), split hi/lo: rows row0.., k0..
template <bool NEG>
__device__ __forceinline__ void frag_t(const float* sT, const float* colscale, int row0, int k0,
                                       u32x4& hi, u32x4& lo) {
  const int l = lane_id();
  const float* src = sT + (row0 + (l & 15)) * LDF + k0 + 8 * (l >> 4);
  const float* cs = colscale + k0 + 8 * (l >> 4);
  float x[8];
  const float4 a = *(const float4*)src, b = *(const float4*)(src + 4);
  const float4 ca = *(const float4*)cs, cb = *(const float4*)(cs + 4);
  x[0] = a.x * ca.x; x[1] = a.y * ca.y; x[2] = a.z * ca.z; x[3] = a.w * ca.w;
  x[4] = b.x * cb.x; x[5] = b.y * cb.y; x[6] = b.z * cb.z; x[7] = b.w * cb.w;
  if (NEG) {
#pragma unroll
    for (int e = 0; e < 8; ++e) x[e] = -x[e];
  }
  split8(x, hi, lo);
}

// Store 8 values as bf16 (and their lo parts) into a [token][dk] row and a
// [dk][token] column.
template <bool SPLIT>
__device__ __forceinline__ void stage_row(bf16_t* row_hi, int row_lo_off, bf16_t* colT,
                                          int colT_lo_off, const float* x) {
  bf16_t h[8], l8[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    h[e] = f2bf(x[e]);
    l8[e] = f2bf(x[e] - bf2f(h[e]));
  }
  if (row_hi) {
    *(u32x4*)row_hi = u32x4{pack2(h[0], h[1]), pack2(h[2], h[3]), pack2(h[4], h[5]), pack2(h[6], h[7])};
    if constexpr (SPLIT)
      *(u32x4*)(row_hi + row_lo_off) =
          u32x4{pack2(l8[0], l8[1]), pack2(l8[2], l8[3]), pack2(l8[4], l8[5]), pack2(l8[6], l8[7])};
  }
  if (colT) {
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      colT[e * LDT] = h[e];
      if constexpr (SPLIT) colT[e * LDT + colT_lo_off] = l8[e];
    }
  }
}

template <typename T_>
__device__ __forceinline__ void load8(const T_* p, float* x) {
  if constexpr (sizeof(T_) == 2) {
    const u32x4 w = *(const u32x4*)p;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      x[2 * e] = bf2f((bf16_t)(w[e] & 0xffffu));
      x[2 * e + 1] = bf2f((bf16_t)(w[e] >> 16));
    }
  } else {
    const float4 a = *(const float4*)p, b = *(const float4*)(p + 4);
    x[0] = a.x; x[1] = a.y; x[2] = a.z; x[3] = a.w;
    x[4] = b.x; x[5] = b.y; x[6] = b.z; x[7] = b.w;
  }
}

template <int DK, int NWC, int MODE>
__global__ __launch_bounds__(64 * NWC) void chunk_kernel(ChunkParams p) {
  using Q_ = Cfg<DK, NWC, MODE>;
  constexpr int NT = Q_::NT, BV = Q_::BV, LDK = Q_::LDK;
  constexpr bool IS = Q_::IS, OS = Q_::OS;
  using InT = typename std::conditional<MODE == MODE_F32, float, bf16_t>::type;
  __shared__ __align__(16) unsigned char smem[Q_::TOTAL];
  bf16_t* sK = (bf16_t*)(smem + Q_::OFF_K);
  bf16_t* sQ = (bf16_t*)(smem + Q_::OFF_Q);
  bf16_t* sKT = (bf16_t*)(smem + Q_::OFF_KT);
  bf16_t* sVT = (bf16_t*)(smem + Q_::OFF_VT);
  float* sT = (float*)(smem + Q_::OFF_T);
  bf16_t* sP = (bf16_t*)(smem + Q_::OFF_P);
  float* sG = (float*)(smem + Q_::OFF_SC);       // cumulative log decay G
  float* sBeta = sG + C;                          // beta
  float* sBE = sG + 2 * C;                        // beta e^G
  float* sEG = sG + 3 * C;                        // e^G
  float* sEL = sG + 4 * C;                        // e^{G_last - G}
  float* sX = (float*)(smem + Q_::OFF_W);         // T-merge temp (phase A only)
  constexpr int K_LO = C * LDK, KT_LO = DK * LDT, VT_LO = BV * LDT, P_LO = C * LDT;

  const int tid = threadIdx.x, wave = tid >> 6, l = tid & 63, lq = l >> 4, lr = l & 15;
  const int nb = p.nb;
  const int blk = blockIdx.x % nb;
  const int h = (blockIdx.x / nb) % p.Hv;
  const int n = blockIdx.x / (nb * p.Hv);
  const int gqa = p.Hv / p.Hk;
  const int hk = h / gqa;
  const int DV = p.DV;
  const int col0 = blk * BV;             // first state column of this workgroup

  // sequence token range [s0, s1) in global token indices
  long long s0, s1;
  if (p.cu_seqlens) {
    // clamp to [0, T] so a malformed offsets array can never index out of bounds
    const long long lo = p.cu_seqlens[n], hi = p.cu_seqlens[n + 1];
    s0 = lo < 0 ? 0 : (lo > p.T ? p.T : lo);
    s1 = hi < s0 ? s0 : (hi > p.T ? p.T : hi);
  } else {
    s0 = (long long)n * p.T;
    s1 = s0 + p.T;
  }
  const int nchunks = (int)((s1 - s0 + C - 1) / C);

  // zero T and P once: their strictly-upper 16x16 tiles are never written
  for (int i = tid; i < C * LDF; i += NT) sT[i] = 0.f;
  for (int i = tid; i < (OS ? 2 : 1) * C * LDT; i += NT) sP[i] = 0;

  // state slice S[dk][16w + (0..15)] in MFMA C layout: S[t][v] = S[16t + 4lq + v][16w + lr]
  f32x4 S[DK / 16];
  const size_t state_off = ((size_t)n * p.Hv + h) * DK * DV + col0 + 16 * wave + lr;
  if (p.initial_state) {
#pragma unroll
    for (int t = 0; t < DK / 16; ++t)
#pragma unroll
      for (int v = 0; v < 4; ++v) S[t][v] = p.initial_state[state_off + (size_t)(16 * t + 4 * lq + v) * DV];
  } else {
#pragma unroll
    for (int t = 0; t < DK / 16; ++t) S[t] = zero4();
  }

  const InT* qg = (const InT*)p.q;
  const InT* kg = (const InT*)p.k;
  const InT* vg = (const InT*)p.v;
  bf16_t* wscr = (bf16_t*)(smem + Q_::OFF_W + wave * Q_::WS);

  for (int j = 0; j < nchunks; ++j) {
    const long long t0 = s0 + (long long)j * C;
    const int nvalid = (int)((s1 - t0) < C ? (s1 - t0) : C);
    __syncthreads();  // previous chunk's readers are done with the shared arrays

    // ------------------------------------------------------------ A1: stage K, Q, V, gates
    {
      constexpr int SEGS = DK / 8;
      for (int it = tid; it < C * SEGS * 2; it += NT) {
        const int which = it / (C * SEGS);  // 0 = k, 1 = q
        const int r = (it / SEGS) % C, seg = it % SEGS;
        float x[8];
        if (r < nvalid) {
          const long long tok = t0 + r;
          const InT* src = which == 0 ? kg + tok * p.k_ld + (long long)hk * DK + seg * 8
                                      : qg + tok * p.q_ld + (long long)hk * DK + seg * 8;
          load8(src, x);
        } else {
#pragma unroll
          for (int e = 0; e < 8; ++e) x[e] = 0.f;
        }
        if (p.qk_l2norm) {
          float ss = 0.f;
#pragma unroll
          for (int e = 0; e < 8; ++e) ss += x[e] * x[e];
          ss = group_sum<SEGS>(ss);
          const float inv = rsqrtf(ss + 1e-6f);
#pragma unroll
          for (int e = 0; e < 8; ++e) x[e] = IS ? x[e] * inv : round_bf(x[e] * inv);
        }
        if (which == 0)
          stage_row<IS>(sK + r * LDK + seg * 8, K_LO, sKT + (seg * 8) * LDT + r, KT_LO, x);
        else
          stage_row<IS>(sQ + r * LDK + seg * 8, K_LO, nullptr, 0, x);
      }
      constexpr int VSEGS = BV / 8;
      for (int it = tid; it < C * VSEGS; it += NT) {
        const int r = it / VSEGS, seg = it % VSEGS;
        float x[8];
        if (r < nvalid) {
          load8(vg + (t0 + r) * p.v_ld + (long long)h * DV + col0 + seg * 8, x);
        } else {
#pragma unroll
          for (int e = 0; e < 8; ++e) x[e] = 0.f;
        }
        stage_row<IS>(nullptr, 0, sVT + (seg * 8) * LDT + r, VT_LO, x);
      }
      if (wave == 0) {
        float g = 0.f, bt = 0.f;
        if (l < nvalid) {
          g = p.g[(t0 + l) * p.Hv + h];
          bt = p.beta[(t0 + l) * p.Hv + h];
        }
        float G = g;
#pragma unroll
        for (int o = 1; o < 64; o <<= 1) {
          const float y = __shfl_up(G, o, 64);
          if (l >= o) G += y;
        }
        const float Gl = __shfl(G, 63, 64);
        const float eg = expf(G);
        sG[l] = G;
        sBeta[l] = bt;
        sBE[l] = bt * eg;
        sEG[l] = eg;
        sEL[l] = expf(Gl - G);
      }
    }
    __syncthreads();

    // ------------------------------------------------------------ A2: K K^T -> L, Q K^T -> P
    for (int tile = wave; tile < 20; tile += NWC) {
      const bool qk = tile >= 10;
      const int bi = kTri[tile % 10][0], bj = kTri[tile % 10][1];
      f32x4 acc = zero4();
#pragma unroll
      for (int s = 0; s < DK / 32; ++s) {
        u32x4 ah, al, bh, bl;
        frag2<IS>(qk ? sQ : sK, K_LO, LDK, 16 * bi, 32 * s, ah, al);
        frag2<IS>(sK, K_LO, LDK, 16 * bj, 32 * s, bh, bl);
        acc = mm<IS, IS>(acc, ah, al, bh, bl);
      }
      const int m = 16 * bj + lr;
      const float Gm = sG[m];
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        const int i = 16 * bi + 4 * lq + v;
        const float dec = expf(sG[i] - Gm);
        if (!qk) {
          sT[i * LDF + m] = (i > m) ? sBeta[i] * acc[v] * dec : 0.f;
        } else {
          const float pv = (i >= m) ? p.scale * acc[v] * dec : 0.f;
          const bf16_t ph = f2bf(pv);
          sP[i * LDT + m] = ph;
          if constexpr (OS) sP[P_LO + i * LDT + m] = f2bf(pv - bf2f(ph));
        }
      }
    }
    __syncthreads();

    // ------------------------------------------------------------ A3: T = (I + L)^-1
    // diagonal 16x16 blocks by forward substitution, one column per lane
    if (wave < 4 && l < 16) {
      const int b0 = 16 * wave, c = l;
      float x[16];
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        float acc = (i == c) ? 1.f : 0.f;
#pragma unroll
        for (int m = 0; m < i; ++m) acc -= sT[(b0 + i) * LDF + b0 + m] * x[m];
        x[i] = acc;
      }
#pragma unroll
      for (int i = 0; i < 16; ++i) sT[(b0 + i) * LDF + b0 + c] = x[i];
    }
    __syncthreads();
    // 16 -> 32: T_hl = -T_hh L_hl T_ll for (h, l) = (1, 0) and (3, 2)
    for (int it = tid; it < 512; it += NT) {
      const int pr = it >> 8, i = (it >> 4) & 15, c = it & 15;
      const int lo = 32 * pr, hi = lo + 16;
      float acc = 0.f;
      for (int m = c; m < 16; ++m) acc += sT[(hi + i) * LDF + lo + m] * sT[(lo + m) * LDF + lo + c];
      sX[pr * 16 * 17 + i * 17 + c] = acc;
    }
    __syncthreads();
    for (int it = tid; it < 512; it += NT) {
      const int pr = it >> 8, i = (it >> 4) & 15, c = it & 15;
      const int lo = 32 * pr, hi = lo + 16;
      float acc = 0.f;
      for (int m = 0; m <= i; ++m) acc += sT[(hi + i) * LDF + hi + m] * sX[pr * 16 * 17 + m * 17 + c];
      sT[(hi + i) * LDF + lo + c] = -acc;
    }
    __syncthreads();
    // 32 -> 64: T_[32:64][0:32] = -T_[32:64][32:64] L_[32:64][0:32] T_[0:32][0:32]
    for (int it = tid; it < 1024; it += NT) {
      const int i = it >> 5, c = it & 31;
      float acc = 0.f;
      for (int m = c; m < 32; ++m) acc += sT[(32 + i) * LDF + m] * sT[m * LDF + c];
      sX[i * 33 + c] = acc;
    }
    __syncthreads();
    for (int it = tid; it < 1024; it += NT) {
      const int i = it >> 5, c = it & 31;
      float acc = 0.f;
      for (int m = 0; m <= i; ++m) acc += sT[(32 + i) * LDF + 32 + m] * sX[m * 33 + c];
      sT[(32 + i) * LDF + c] = -acc;
    }
    __syncthreads();

    // ------------------------------------------------------------ B: this wave's 16 columns
    bf16_t* wS = wscr;                    // S^T [16][LDK] (hi, lo)
    bf16_t* wKS = wscr;                   // (K S)^T [16][LDT]
    bf16_t* wVN = wscr;                   // V_new^T [16][LDT] (hi, lo if OS)
    bf16_t* wVt = wscr + (OS ? 2 : 1) * 16 * LDT;  // Vt^T hi, then lo
    constexpr int WS_LO = 16 * LDK, W_LO = 16 * LDT;

    // B0: S^T into the scratch as the B operand of K S and Q S
#pragma unroll
    for (int t = 0; t < DK / 16; ++t) {
      if constexpr (IS) store_ct_split(wS, wS + WS_LO, LDK, 16 * t, 0, S[t]);
      else store_ct_bf16(wS, LDK, 16 * t, 0, S[t]);
    }
    wave_lds_fence();
    // B1/B2: K S and Q S for the 4 token tiles
    f32x4 KS[4], QS[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      KS[i] = zero4();
      QS[i] = zero4();
#pragma unroll
      for (int s = 0; s < DK / 32; ++s) {
        u32x4 bh, bl, ah, al;
        frag2<IS>(wS, WS_LO, LDK, 0, 32 * s, bh, bl);
        frag2<IS>(sK, K_LO, LDK, 16 * i, 32 * s, ah, al);
        KS[i] = mm<IS, IS>(KS[i], ah, al, bh, bl);
        frag2<IS>(sQ, K_LO, LDK, 16 * i, 32 * s, ah, al);
        QS[i] = mm<IS, IS>(QS[i], ah, al, bh, bl);
      }
    }
    wave_lds_fence();
    // B3: (K S)^T into the scratch (over S^T, whose reads are complete)
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      if constexpr (IS) store_ct_split(wKS, wKS + W_LO, LDT, 16 * i, 0, KS[i]);
      else store_ct_bf16(wKS, LDT, 16 * i, 0, KS[i]);
    }
    wave_lds_fence();
    // B4: V_new = T diag(beta) V - T diag(beta e^G) (K S); T is lower triangular
    f32x4 VN[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      VN[i] = zero4();
#pragma unroll
      for (int s = 0; s < 2; ++s) {
        if (s == 1 && i < 2) continue;
        u32x4 th, tl, bh, bl;
        frag_t<false>(sT, sBeta, 16 * i, 32 * s, th, tl);
        frag2<IS>(sVT + (16 * wave) * LDT, VT_LO, LDT, 0, 32 * s, bh, bl);
        VN[i] = mm<true, IS>(VN[i], th, tl, bh, bl);
        frag_t<true>(sT, sBE, 16 * i, 32 * s, th, tl);
        frag2<IS>(wKS, W_LO, LDT, 0, 32 * s, bh, bl);
        VN[i] = mm<true, IS>(VN[i], th, tl, bh, bl);
      }
    }
    wave_lds_fence();
    // B5: V_new^T and Vt^T = (diag(e^{G_last - G}) V_new)^T into the scratch
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      if constexpr (OS) store_ct_split(wVN, wVN + W_LO, LDT, 16 * i, 0, VN[i]);
      else store_ct_bf16(wVN, LDT, 16 * i, 0, VN[i]);
      f32x4 vt;
#pragma unroll
      for (int v = 0; v < 4; ++v) vt[v] = VN[i][v] * sEL[16 * i + 4 * lq + v];
      store_ct_split(wVt, wVt + W_LO, LDT, 16 * i, 0, vt);
    }
    wave_lds_fence();
    // B6: O = e^G (Q S) scale + P V_new
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      f32x4 o;
#pragma unroll
      for (int v = 0; v < 4; ++v) o[v] = p.scale * sEG[16 * i + 4 * lq + v] * QS[i][v];
#pragma unroll
      for (int s = 0; s < 2; ++s) {
        if (s == 1 && i < 2) continue;
        u32x4 ah, al, bh, bl;
        frag2<OS>(sP, P_LO, LDT, 16 * i, 32 * s, ah, al);
        frag2<OS>(wVN, W_LO, LDT, 0, 32 * s, bh, bl);
        o = mm<OS, OS>(o, ah, al, bh, bl);
      }
      if constexpr (MODE != MODE_LAYER) {
#pragma unroll
        for (int v = 0; v < 4; ++v) {
          const int r = 16 * i + 4 * lq + v;
          if (r < nvalid)
            p.o[((t0 + r) * p.Hv + h) * (long long)DV + col0 + 16 * wave + lr] = o[v];
        }
      }
    }
    // B7: S <- e^{G_last} S + K^T Vt
    const float gl = sEG[C - 1];
#pragma unroll
    for (int t = 0; t < DK / 16; ++t) {
#pragma unroll
      for (int v = 0; v < 4; ++v) S[t][v] *= gl;
#pragma unroll
      for (int s = 0; s < 2; ++s) {
        u32x4 ah, al, bh, bl;
        frag2<IS>(sKT, KT_LO, LDT, 16 * t, 32 * s, ah, al);
        frag2<true>(wVt, W_LO, LDT, 0, 32 * s, bh, bl);
        S[t] = mm<IS, true>(S[t], ah, al, bh, bl);
      }
    }
  }

  if (p.final_state) {
#pragma unroll
    for (int t = 0; t < DK / 16; ++t)
#pragma unroll
      for (int v = 0; v < 4; ++v) p.final_state[state_off + (size_t)(16 * t + 4 * lq + v) * DV] = S[t][v];
  }
}

template <int DK, int NWC, int MODE>
hipError_t launch_cfg(const ChunkParams& p, hipStream_t stream) {
  const unsigned grid = (unsigned)(p.N * p.Hv * p.nb);
  hipLaunchKernelGGL((chunk_kernel<DK, NWC, MODE>), dim3(grid), dim3(64 * NWC), 0, stream, p);
  return hipGetLastError();
}

}  // namespace

int chunk_block_cols(int dk, int dv, bool f32_inputs) {
  // columns per workgroup: the whole dv when the LDS budget allows it
  if (f32_inputs) return dv >= 64 ? 64 : dv;
  return dv >= 128 ? 128 : dv;
  (void)dk;
}

bool chunk_dims_supported(int dk, int dv, bool f32_inputs) {
  if (f32_inputs) return (dk == 32 || dk == 64) && (dv == 64 || dv == 128);
  return (dk == 64 || dk == 128) && (dv == 64 || dv == 128);
}

hipError_t launch_chunk(const ChunkParams& p, bool f32_inputs, hipStream_t stream) {
  const int bv = p.DV / p.nb;
  if (f32_inputs) {
    if (bv != 64) return hipErrorInvalidValue;
    if (p.dk == 64) return launch_cfg<64, 4, MODE_F32>(p, stream);
    if (p.dk == 32) return launch_cfg<32, 4, MODE_F32>(p, stream);
    return hipErrorInvalidValue;
  }
  if (p.dk == 128 && bv == 128) return launch_cfg<128, 8, MODE_BF16>(p, stream);
  if (p.dk == 128 && bv == 64) return launch_cfg<128, 4, MODE_BF16>(p, stream);
  if (p.dk == 64 && bv == 128) return launch_cfg<64, 8, MODE_BF16>(p, stream);
  if (p.dk == 64 && bv == 64) return launch_cfg<64, 4, MODE_BF16>(p, stream);
  return hipErrorInvalidValue;
}

}  // namespace omx
