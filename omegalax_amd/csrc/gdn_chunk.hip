// Chunked gated delta rule on gfx950: one kernel for the whole prefill.
//
// Follows chunk_gated_delta_rule (omegalax/models/qwen3_5/deltanet.py:53-153),
// restated for MFMA.  Per chunk of C = 64 tokens, with G the in-chunk cumsum of g
// (:98) and L = strict_lower(beta_i (k_i.k_j) e^{G_i-G_j}) (:100-108), the
// reference forms T = (I + L)^-1 by solve_triangular (:110-113) and then
// U = T diag(beta) V, W = T diag(beta e^G) K (:115-116).  Here the two products
// with T are merged into one triangular solve per chunk,
//     (I + L) V_new = diag(beta) V - diag(beta e^G) (K S)         (:133-134)
// done by block forward substitution over the four 16-token blocks; only the
// 16x16 diagonal blocks are inverted explicitly.  Then
//     O  = scale e^G (Q S) + P V_new,  P = lower(scale (q_i.k_j) e^{G_i-G_j})  (:130-137)
//     S <- e^{G_last} S + K^T diag(e^{G_last - G}) V_new           (:139-142)
//
// Work mapping.  One workgroup of 4 wavefronts per (sequence, value head,
// 64-column block of dv) walks that sequence's chunks in order.  Wavefront w
// owns state columns [16w, 16w+16) of the block: its fp32 slice S[dk][16] stays
// in MFMA accumulator registers for the whole sequence, and every product that
// touches it (K S, Q S, the solve, O, the state update) runs on that wavefront
// alone.  The per-chunk work that does not touch S -- staging K, Q, V in LDS,
// K K^T and Q K^T, the diagonal-block inverses -- is shared between workgroup
// barriers.  The next chunk's global loads are issued into registers before the
// state pipeline starts, so their latency hides behind it.
//
// Precision.  MFMA inputs are bf16 with fp32 accumulation.  q, k, v are bf16 on
// the layer path (exact), or fp32 split into hi+lo bf16 pairs (MODE_F32).  The
// solve's operands (L blocks, diagonal inverses, right-hand sides) and the
// state-update operand diag(e^{G_last-G}) V_new are always split hi+lo; with bf16
// inputs S enters K S / Q S, and P, V_new enter P V_new, as single bf16 (their
// rounding reaches only the bf16-tolerance output).
//
// Modes: MODE_BF16 / MODE_F32 read q, k, v, g, beta (core function) and store o
// in fp32.  MODE_LAYER reads the raw in_proj outputs, applies the causal conv +
// SiLU + L2 norm and the gates while staging (deltanet.py:243-250), and ends in
// the gated RMSNorm (deltanet.py:282-293): fused when one workgroup holds all of
// dv, otherwise through a bf16 o buffer and per-token partial sums of o^2 that
// the epilogue kernel (gdn_epilogue.hip) normalises.
#include <type_traits>

#include "gdn_common.h"
#include "gdn_kernels.h"
#include "gdn_mfma.h"

namespace omx {

namespace {

constexpr int C = 64;          // chunk length (deltanet.py:59)
constexpr int NWC = 4;         // column wavefronts per workgroup
constexpr int NT = 64 * NWC;   // threads per workgroup
constexpr int BV = 16 * NWC;   // state columns per workgroup
constexpr int LDT = C + 8;     // row stride (elements) of 64-wide bf16 arrays
constexpr int LDD = 16 + 4;    // row stride of 16-wide diagonal-block arrays
constexpr int MODE_BF16 = 0, MODE_F32 = 1, MODE_LAYER = 2;

template <int DK, int MODE>
struct Cfg {
  static constexpr bool IS = MODE == MODE_F32;  // q/k/v split hi+lo
  static constexpr bool OS = MODE == MODE_F32;  // output-path operands split
  static constexpr int NS = IS ? 2 : 1;
  static constexpr int RAWW = IS ? 2 : 1;       // u32x4 words per 8-element input segment
  static constexpr int LDK = DK + 8;            // row stride of [token][dk] arrays
  static constexpr int SEGS = DK / 8;           // 8-element segments per q/k row
  static constexpr int NI_KQ = 2 * C * SEGS / NT;
  static constexpr int NI_V = C * (BV / 8) / NT;
  // shared arrays (bytes)
  static constexpr int SZ_K = NS * C * LDK * 2;   // K rows [token][dk] (hi, lo)
  static constexpr int SZ_V = NS * C * LDT * 2;   // V rows [token][col]
  static constexpr int SZ_LO = 2 * C * LDT * 2;   // off-diagonal blocks of L (hi, lo)
  static constexpr int SZ_LD = C * LDD * 4;       // diagonal blocks of L, fp32
  static constexpr int SZ_TD = 2 * C * LDD * 2;   // inverses of the diagonal blocks (hi, lo)
  static constexpr int SZ_P = (OS ? 2 : 1) * C * LDT * 2;
  static constexpr int SZ_SC = 8 * C * 4;
  // per-wave scratch: S^T (K S, Q S), then Vt^T (hi, lo)
  static constexpr int WS_S = NS * 16 * LDK * 2;
  static constexpr int WS_U = 2 * 16 * LDT * 2;
  static constexpr int WS = WS_S > WS_U ? WS_S : WS_U;
  static constexpr int SZ_W = NWC * WS;
  static constexpr int HW = 2 * DK + BV;          // channels of this workgroup (q | k | v block)
  static constexpr int SZ_HIST = MODE == MODE_LAYER ? 3 * HW * 2 : 0;
  static constexpr int SZ_NP = MODE == MODE_LAYER ? C * NWC * 4 : 0;
  static constexpr int SZ_CW = MODE == MODE_LAYER ? 4 * HW * 4 : 0;  // conv weights [tap][ch]
  static constexpr int OFF_K = 0;
  static constexpr int OFF_Q = OFF_K + SZ_K;
  static constexpr int OFF_V = OFF_Q + SZ_K;
  static constexpr int OFF_LO = OFF_V + SZ_V;
  static constexpr int OFF_LD = OFF_LO + SZ_LO;
  static constexpr int OFF_TD = OFF_LD + SZ_LD;
  static constexpr int OFF_P = OFF_TD + SZ_TD;
  static constexpr int OFF_SC = OFF_P + SZ_P;
  static constexpr int OFF_W = OFF_SC + SZ_SC;
  static constexpr int OFF_HIST = OFF_W + SZ_W;
  static constexpr int OFF_NP = OFF_HIST + SZ_HIST;
  static constexpr int OFF_CW = OFF_NP + SZ_NP;
  static constexpr int TOTAL = OFF_CW + SZ_CW;
  static_assert(TOTAL <= 160 * 1024, "LDS budget");
  static_assert(DK % 32 == 0 && DK <= 128, "dk");
  static_assert(NI_KQ * NT == 2 * C * SEGS && NI_V * NT == C * (BV / 8), "item split");
};

// The 20 lower-triangular 16x16 tiles of K K^T (0..9, diagonal first) and Q K^T
// (10..19), each coded in 5 bits as qk << 4 | row block << 2 | col block and
// packed into two words, so a wave decodes its tiles with scalar shifts.
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

template <bool AS, bool BS>
__device__ __forceinline__ f32x4 mm(f32x4 acc, u32x4 ah, u32x4 al, u32x4 bh, u32x4 bl) {
  acc = mma16(ah, bh, acc);
  if constexpr (BS) acc = mma16(ah, bl, acc);
  if constexpr (AS) acc = mma16(al, bh, acc);
  return acc;
}

// acc += (ah + al)(bh + bl) without the lo*lo term, 16x16x16
__device__ __forceinline__ f32x4 mm3k16(f32x4 acc, u32x2 ah, u32x2 al, u32x2 bh, u32x2 bl) {
  acc = mma16k16(ah, bh, acc);
  acc = mma16k16(ah, bl, acc);
  acc = mma16k16(al, bh, acc);
  return acc;
}

template <bool SPLIT>
__device__ __forceinline__ void frag2(const bf16_t* base, int lo_off, int ld, int row0, int k0,
                                      u32x4& hi, u32x4& lo) {
  hi = frag_bf16(base, ld, row0, k0);
  if constexpr (SPLIT) lo = frag_bf16(base + lo_off, ld, row0, k0);
  else lo = hi;
}

// unpack 8 input values (bf16 or fp32) from raw prefetch words
template <bool F32>
__device__ __forceinline__ void unpack8(const u32x4* w, float* x) {
  if constexpr (F32) {
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      x[e] = __uint_as_float(w[0][e]);
      x[4 + e] = __uint_as_float(w[1][e]);
    }
  } else {
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      x[2 * e] = __uint_as_float(w[0][e] << 16);
      x[2 * e + 1] = __uint_as_float(w[0][e] & 0xffff0000u);
    }
  }
}

template <bool F32>
__device__ __forceinline__ void load_raw(const void* base, long long elem, u32x4* w) {
  if constexpr (F32) {
    const u32x4* p = (const u32x4*)((const float*)base + elem);
    w[0] = p[0];
    w[1] = p[1];
  } else {
    w[0] = *(const u32x4*)((const bf16_t*)base + elem);
  }
}

// 8 values -> packed bf16 words (hi, or the lo parts)
__device__ __forceinline__ u32x4 pack8(const float* x) {
  return u32x4{pack_bf16(x[0], x[1]), pack_bf16(x[2], x[3]), pack_bf16(x[4], x[5]),
               pack_bf16(x[6], x[7])};
}
__device__ __forceinline__ u32x4 pack8_lo(const float* x) {
  return u32x4{pack_bf16(lo_part(x[0]), lo_part(x[1])), pack_bf16(lo_part(x[2]), lo_part(x[3])),
               pack_bf16(lo_part(x[4]), lo_part(x[5])), pack_bf16(lo_part(x[6]), lo_part(x[7]))};
}

// write 8 values of one token into a [token][.] row and/or the transposed [.][token] column
template <bool SPLIT>
__device__ __forceinline__ void stage8(bf16_t* row, int row_lo, bf16_t* colT, int colT_lo,
                                       const float* x) {
  const u32x4 h = pack8(x);
  u32x4 lo{};
  if constexpr (SPLIT) lo = pack8_lo(x);
  if (row) {
    *(u32x4*)row = h;
    if constexpr (SPLIT) *(u32x4*)(row + row_lo) = lo;
  }
  if (colT) {
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      colT[(2 * e) * LDT] = (bf16_t)(h[e] & 0xffffu);
      colT[(2 * e + 1) * LDT] = (bf16_t)(h[e] >> 16);
      if constexpr (SPLIT) {
        colT[(2 * e) * LDT + colT_lo] = (bf16_t)(lo[e] & 0xffffu);
        colT[(2 * e + 1) * LDT + colT_lo] = (bf16_t)(lo[e] >> 16);
      }
    }
  }
}

// Per-thread register prefetch of one chunk's inputs.
template <int DK, int MODE>
struct Prefetch {
  using Q_ = Cfg<DK, MODE>;
  u32x4 kq[Q_::NI_KQ][Q_::RAWW];
  u32x4 v[Q_::NI_V][Q_::RAWW];
  float g0, g1;  // wave 0: g and beta (core) or a and b (layer) of token t0 + lane
};

template <int DK, int MODE>
__device__ __forceinline__ void prefetch(const ChunkParams& p, Prefetch<DK, MODE>& pf,
                                         long long t0, int nvalid, int hk, int h, int col0) {
  using Q_ = Cfg<DK, MODE>;
  constexpr bool F32 = MODE == MODE_F32;
  const int tid = threadIdx.x;
#pragma unroll
  for (int k = 0; k < Q_::NI_KQ; ++k) {
    const int it = tid + k * NT;
    const int which = it / (C * Q_::SEGS);  // 0 = k, 1 = q
    const int r = (it / Q_::SEGS) % C, seg = it % Q_::SEGS;
    // rows past the sequence end load the last valid row (in bounds); staging zeroes
    // them, so the loaded registers are not touched until the data is needed
    const long long tok = t0 + (r < nvalid ? r : nvalid - 1);
    if constexpr (MODE == MODE_LAYER) {
      const int ch = (which == 0 ? p.Hk * DK : 0) + hk * DK + seg * 8;
      load_raw<false>(p.mixed_qkv, tok * p.conv_dim + ch, pf.kq[k]);
    } else {
      const void* base = which == 0 ? p.k : p.q;
      const long long ld = which == 0 ? p.k_ld : p.q_ld;
      load_raw<F32>(base, tok * ld + (long long)hk * DK + seg * 8, pf.kq[k]);
    }
  }
#pragma unroll
  for (int k = 0; k < Q_::NI_V; ++k) {
    const int it = tid + k * NT;
    const int r = it / (BV / 8), seg = it % (BV / 8);
    const long long tok = t0 + (r < nvalid ? r : nvalid - 1);
    if constexpr (MODE == MODE_LAYER)
      load_raw<false>(p.mixed_qkv,
                      tok * p.conv_dim + 2 * p.Hk * DK + (long long)h * p.DV + col0 + seg * 8,
                      pf.v[k]);
    else
      load_raw<F32>(p.v, tok * p.v_ld + (long long)h * p.DV + col0 + seg * 8, pf.v[k]);
  }
  pf.g0 = 0.f;
  pf.g1 = 0.f;
  if (tid < 64 && tid < nvalid) {
    const long long idx = (t0 + tid) * p.Hv + h;
    if constexpr (MODE == MODE_LAYER) {
      pf.g0 = bf2f(((const bf16_t*)p.a)[idx]);
      pf.g1 = bf2f(((const bf16_t*)p.b)[idx]);
    } else {
      pf.g0 = p.g[idx];
      pf.g1 = p.beta[idx];
    }
  }
}

template <int DK, int MODE>
__global__ __launch_bounds__(NT) void chunk_kernel(ChunkParams p) {
  using Q_ = Cfg<DK, MODE>;
  constexpr int LDK = Q_::LDK, SEGS = Q_::SEGS;
  constexpr bool IS = Q_::IS, OS = Q_::OS;
  constexpr bool F32 = MODE == MODE_F32;
  // Each buffer is its own __shared__ object, so the compiler can tell their
  // accesses apart and overlap loads of one with stores to another.
  __shared__ __align__(16) bf16_t sK[Q_::SZ_K / 2];
  __shared__ __align__(16) bf16_t sQ[Q_::SZ_K / 2];
  __shared__ __align__(16) bf16_t sV[Q_::SZ_V / 2];
  __shared__ __align__(16) bf16_t sLoT[Q_::SZ_LO / 2];  // L^T off-diagonal blocks [m][i] (hi, lo)
  __shared__ __align__(16) float sLd[Q_::SZ_LD / 4];    // diagonal blocks of L, fp32
  __shared__ __align__(16) bf16_t sTdT[Q_::SZ_TD / 2];  // diagonal inverses, transposed (hi, lo)
  __shared__ __align__(16) bf16_t sPT[Q_::SZ_P / 2];    // P^T [m][i]
  __shared__ __align__(16) float sG2[Q_::SZ_SC / 4];    // cumulative log decay G, times log2(e)
  __shared__ __align__(16) bf16_t sWS[Q_::SZ_W / 2];    // per-wave scratch
  __shared__ __align__(16) bf16_t sHist[Q_::SZ_HIST / 2 + 8];  // layer: raw inputs of 3 previous tokens
  __shared__ __align__(16) float sNP[Q_::SZ_NP / 4 + 4];       // layer: [token][wave] sums of o^2
  __shared__ __align__(16) float sCW[Q_::SZ_CW / 4 + 4];       // layer: bf16-rounded conv weights
  float* sBeta = sG2 + C;                     // beta
  float* sBE = sG2 + 2 * C;                   // beta e^G
  float* sEG = sG2 + 3 * C;                   // e^G
  float* sEL = sG2 + 4 * C;                   // e^{G_last - G}
  constexpr int K_LO = C * LDK, V_LO = C * LDT, P_LO = C * LDT;
  constexpr int LO_LO = C * LDT, TD_LO = C * LDD;
  constexpr int HW = Q_::HW;

  // the wavefront index is uniform across the wave: readfirstlane puts it in an
  // SGPR so wave-dependent tile choices and branches stay scalar
  const int tid = threadIdx.x, l = tid & 63, lq = l >> 4, lr = l & 15;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  // XCD-aware numbering: workgroups are dealt round-robin over the 8 XCDs
  // (blockIdx % 8); renumber so that consecutive work items -- the gqa x nb
  // workgroups reading the same key head's q/k -- run on one XCD and share its L2.
  const unsigned nwg = gridDim.x, xcd = blockIdx.x % 8, slot = blockIdx.x / 8;
  const unsigned per = nwg / 8, rem = nwg % 8;
  const int wid = (int)(xcd * per + (xcd < rem ? xcd : rem) + slot);
  const int nb = p.nb;
  const int blk = wid % nb;
  const int h = (wid / nb) % p.Hv;
  const int n = wid / (nb * p.Hv);
  const int gqa = p.Hv / p.Hk;
  const int hk = h / gqa;
  const int DV = p.DV;
  const int col0 = blk * BV;

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

  // zero P once: its strictly-upper 16x16 tiles are never written
  for (int i = tid; i < (OS ? 2 : 1) * C * LDT / 2; i += NT) ((uint32_t*)sPT)[i] = 0u;
  if constexpr (MODE == MODE_LAYER) {
    // conv history before the first token: conv_state_in (oldest tap first) or zeros
    const int K = p.conv_k;
    for (int it = tid; it < 3 * HW; it += NT) {
      const int tap = it / HW, ci = it % HW;  // tap 0 holds time s0 - 3
      int ch;
      if (ci < DK) ch = hk * DK + ci;
      else if (ci < 2 * DK) ch = p.Hk * DK + hk * DK + (ci - DK);
      else ch = 2 * p.Hk * DK + h * DV + col0 + (ci - 2 * DK);
      bf16_t val = 0;
      const int slot = (K - 1) - (3 - tap);  // cache slot of time s0 - (3 - tap)
      if (p.conv_state_in && slot >= 0)
        val = ((const bf16_t*)p.conv_state_in)[((size_t)n * p.conv_dim + ch) * (K - 1) + slot];
      sHist[it] = val;
    }
    for (int it = tid; it < K * HW; it += NT) {
      const int tap = it / HW, ci = it % HW;
      int ch;
      if (ci < DK) ch = hk * DK + ci;
      else if (ci < 2 * DK) ch = p.Hk * DK + hk * DK + (ci - DK);
      else ch = 2 * p.Hk * DK + h * DV + col0 + (ci - 2 * DK);
      sCW[it] = round_bf(p.conv_w[(size_t)ch * K + tap]);  // cast to bf16 as at deltanet.py:243
    }
  }

  // state slice S[dk][16w + (0..15)] in MFMA C layout: S[t][v] = S[16t + 4lq + v][16w + lr]
  f32x4 S[DK / 16];
  const size_t state_off = ((size_t)n * p.Hv + h) * DK * DV + col0 + 16 * wave + lr;
  if (p.initial_state) {
#pragma unroll
    for (int t = 0; t < DK / 16; ++t)
#pragma unroll
      for (int v = 0; v < 4; ++v)
        S[t][v] = p.initial_state[state_off + (size_t)(16 * t + 4 * lq + v) * DV];
  } else {
#pragma unroll
    for (int t = 0; t < DK / 16; ++t) S[t] = zero4();
  }

  bf16_t* wscr = sWS + wave * (Q_::WS / 2);
  bf16_t* wS = wscr;                  // S^T [16][LDK] (hi, lo)
  bf16_t* wVt = wscr;                 // Vt^T [16][LDT] hi, then lo
  constexpr int WS_LO = 16 * LDK, W_LO = 16 * LDT;

  Prefetch<DK, MODE> pf;
  if (nchunks > 0) prefetch<DK, MODE>(p, pf, s0, (int)((s1 - s0) < C ? (s1 - s0) : C), hk, h, col0);

  for (int j = 0; j < nchunks; ++j) {
    const long long t0 = s0 + (long long)j * C;
    const int nvalid = (int)((s1 - t0) < C ? (s1 - t0) : C);
    __syncthreads();  // the previous chunk's readers are done with the shared arrays

    // ------------------------------------------------------------ A1: stage the chunk
    if (wave == 0) {
      float g = pf.g0, bt = pf.g1;
      if constexpr (MODE == MODE_LAYER) {
        // gates, deltanet.py:248-250: beta in bf16, g in fp32
        if (l < nvalid) {
          g = -expf(p.A_log[h]) * softplusf_(pf.g0 + p.dt_bias[h]);
          bt = round_bf(sigmoidf_(pf.g1));
        } else {
          g = 0.f;
          bt = 0.f;
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
      sG2[l] = G * 1.4426950408889634f;
      sBeta[l] = bt;
      sBE[l] = bt * eg;
      sEG[l] = eg;
      sEL[l] = __expf(Gl - G);
    }
    if constexpr (MODE != MODE_LAYER) {
      // K and Q rows (L2-normalised at input precision, deltanet.py:65-66), V rows
#pragma unroll
      for (int k = 0; k < Q_::NI_KQ; ++k) {
        const int it = tid + k * NT;
        const int which = it / (C * SEGS);
        const int r = (it / SEGS) % C, seg = it % SEGS;
        float x[8];
        unpack8<F32>(pf.kq[k], x);
        const float keep = (float)(r < nvalid);  // padded rows are zero
#pragma unroll
        for (int e = 0; e < 8; ++e) x[e] *= keep;
        if (p.qk_l2norm) {
          float ss = 0.f;
#pragma unroll
          for (int e = 0; e < 8; ++e) ss += x[e] * x[e];
          ss = group_sum_dpp<SEGS>(ss);
          const float inv = rsqrtf(ss + 1e-6f);
#pragma unroll
          for (int e = 0; e < 8; ++e) x[e] *= inv;  // bf16 inputs: the bf16 pack below rounds
        }
        stage8<IS>((which == 0 ? sK : sQ) + r * LDK + seg * 8, K_LO, nullptr, 0, x);
      }
#pragma unroll
      for (int k = 0; k < Q_::NI_V; ++k) {
        const int it = tid + k * NT;
        const int r = it / (BV / 8), seg = it % (BV / 8);
        float x[8];
        unpack8<F32>(pf.v[k], x);
        const float keep = (float)(r < nvalid);
#pragma unroll
        for (int e = 0; e < 8; ++e) x[e] *= keep;
        stage8<IS>(sV + r * LDT + seg * 8, V_LO, nullptr, 0, x);
      }
    } else {
      // raw rows: q -> sQ, k -> sK, v -> sV; the conv reads them next.  Padded rows
      // (copies of the last valid row) feed only padded outputs, which are zeroed.
#pragma unroll
      for (int k = 0; k < Q_::NI_KQ; ++k) {
        const int it = tid + k * NT;
        const int which = it / (C * SEGS);
        const int r = (it / SEGS) % C, seg = it % SEGS;
        *(u32x4*)((which == 0 ? sK : sQ) + r * LDK + seg * 8) = pf.kq[k][0];
      }
#pragma unroll
      for (int k = 0; k < Q_::NI_V; ++k) {
        const int it = tid + k * NT;
        const int r = it / (BV / 8), seg = it % (BV / 8);
        *(u32x4*)(sV + r * LDT + seg * 8) = pf.v[k][0];
      }
      __syncthreads();
      // causal depthwise conv (deltanet.py:35-50) + SiLU, each rounded to bf16 like the
      // reference's bf16 ops; the weights in sCW are already bf16 values (deltanet.py:243)
      const int K = p.conv_k;
      float ykq[Q_::NI_KQ][8], yv[Q_::NI_V][8];
#pragma unroll
      for (int k = 0; k < Q_::NI_KQ + Q_::NI_V; ++k) {
        const bool isv = k >= Q_::NI_KQ;
        const int it = tid + (isv ? k - Q_::NI_KQ : k) * NT;
        int r, seg, ci, ld;
        const bf16_t* rows;
        if (!isv) {
          const int which = it / (C * SEGS);
          r = (it / SEGS) % C;
          seg = it % SEGS;
          rows = which == 0 ? sK : sQ;
          ld = LDK;
          ci = (which == 0 ? DK : 0) + seg * 8;
        } else {
          r = it / (BV / 8);
          seg = it % (BV / 8);
          rows = sV;
          ld = LDT;
          ci = 2 * DK + seg * 8;
        }
        float acc[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) acc[e] = 0.f;
        for (int jt = 0; jt < K; ++jt) {
          const int rr = r - (K - 1) + jt;  // token row within the chunk
          float xv[8];
          const bf16_t* src = rr >= 0 ? rows + rr * ld + seg * 8 : sHist + (3 + rr) * HW + ci;
          const u32x4 w = *(const u32x4*)src;
          unpack8<false>(&w, xv);
          const float4 w0 = *(const float4*)(sCW + jt * HW + ci);
          const float4 w1 = *(const float4*)(sCW + jt * HW + ci + 4);
          acc[0] += w0.x * xv[0]; acc[1] += w0.y * xv[1]; acc[2] += w0.z * xv[2]; acc[3] += w0.w * xv[3];
          acc[4] += w1.x * xv[4]; acc[5] += w1.y * xv[5]; acc[6] += w1.z * xv[6]; acc[7] += w1.w * xv[7];
        }
        float* y = isv ? yv[k - Q_::NI_KQ] : ykq[k];
        const float keep = (float)(r < nvalid);  // padded rows are zero (branch-free)
#pragma unroll
        for (int e = 0; e < 8; ++e) y[e] = round_bf(siluf_(round_bf(acc[e]))) * keep;
      }
      __syncthreads();
      // history for the next chunk: raw inputs of tokens 61..63 (still in the prefetch)
#pragma unroll
      for (int k = 0; k < Q_::NI_KQ; ++k) {
        const int it = tid + k * NT;
        const int which = it / (C * SEGS);
        const int r = (it / SEGS) % C, seg = it % SEGS;
        if (r >= C - 3) *(u32x4*)(sHist + (r - (C - 3)) * HW + (which == 0 ? DK : 0) + seg * 8) = pf.kq[k][0];
      }
#pragma unroll
      for (int k = 0; k < Q_::NI_V; ++k) {
        const int it = tid + k * NT;
        const int r = it / (BV / 8), seg = it % (BV / 8);
        if (r >= C - 3) *(u32x4*)(sHist + (r - (C - 3)) * HW + 2 * DK + seg * 8) = pf.v[k][0];
      }
      // conv outputs: q, k rows L2-normalised (deltanet.py:65-66), v rows
#pragma unroll
      for (int k = 0; k < Q_::NI_KQ; ++k) {
        const int it = tid + k * NT;
        const int which = it / (C * SEGS);
        const int r = (it / SEGS) % C, seg = it % SEGS;
        float* x = ykq[k];
        float ss = 0.f;
#pragma unroll
        for (int e = 0; e < 8; ++e) ss += x[e] * x[e];
        ss = group_sum_dpp<SEGS>(ss);
        const float inv = rsqrtf(ss + 1e-6f);
#pragma unroll
        for (int e = 0; e < 8; ++e) x[e] *= inv;  // rounded to bf16 by the pack in stage8
        stage8<false>((which == 0 ? sK : sQ) + r * LDK + seg * 8, 0, nullptr, 0, x);
      }
#pragma unroll
      for (int k = 0; k < Q_::NI_V; ++k) {
        const int it = tid + k * NT;
        const int r = it / (BV / 8), seg = it % (BV / 8);
        stage8<false>(sV + r * LDT + seg * 8, 0, nullptr, 0, yv[k]);
      }
    }
    __syncthreads();

    // ------------------------------------------------------------ A2: K K^T -> L, Q K^T -> P
    // Wave w computes tiles w, w+4, ..., w+16 of kTileCode: first its diagonal K K^T
    // tile (w, w), which it inverts itself right away, then four more.  L and P are
    // written transposed (one vector store per lane) and read back through
    // ds_read_b64_tr_b16 as row-major operands.
    // Slot ti of wave w holds tile w + 4 ti: slot 0 is the wave's diagonal K K^T tile,
    // slot 1 an off-diagonal K K^T tile, slots 3 and 4 Q K^T tiles, and slot 2 is
    // K K^T for waves 0-1 and Q K^T for waves 2-3.
    f32x4 tacc[5];
#pragma unroll
    for (int ti = 0; ti < 5; ++ti) {  // all products first: no LDS stores in between
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
#pragma unroll
    for (int ti = 0; ti < 5; ++ti) {
      const f32x4 acc = tacc[ti];
      const int code = tile_code(wave + 4 * ti);
      const bool qk = ti >= 3 || (ti == 2 && wave >= 2);
      const int bi = (code >> 2) & 3, bj = code & 3;
      const int m = 16 * bj + lr;
      const float Gm = sG2[m];
      const float4 Gi = *(const float4*)(sG2 + 16 * bi + 4 * lq);
      const float gi[4] = {Gi.x, Gi.y, Gi.z, Gi.w};
      f32x4 val;
      if (!qk) {
        const float4 Bi = *(const float4*)(sBeta + 16 * bi + 4 * lq);
        const float bt[4] = {Bi.x, Bi.y, Bi.z, Bi.w};
        // branch-free: the exponent is clamped to <= 0 (the masked entries would
        // overflow) and the strictly-lower mask multiplies the result
#pragma unroll
        for (int v = 0; v < 4; ++v) {
          const int i = 16 * bi + 4 * lq + v;
          const float dec = __builtin_amdgcn_exp2f(fminf(gi[v] - Gm, 0.f));
          val[v] = bt[v] * acc[v] * dec * (float)(i > m);
        }
        if (ti == 0) {
          // this wave's diagonal block: T_ww = (I + L_ww)^-1 by forward substitution,
          // one column per lane (lanes 16..63 repeat the work and do not store)
#pragma unroll
          for (int v = 0; v < 4; ++v) sLd[(16 * bi + 4 * lq + v) * LDD + lr] = val[v];
          wave_lds_fence();
          const int c = l & 15;
          float x[16];
#pragma unroll
          for (int i = 0; i < 16; ++i) {
            const float* row = sLd + (16 * bi + i) * LDD;
            float a0 = (i == c) ? 1.f : 0.f, a1 = 0.f;
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
          if (l < 16) {
            // T_ww^T row c = column c of T_ww, hi and lo
            bf16_t* dh = sTdT + (16 * bi + c) * LDD;
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
        if constexpr (OS) store_ct_split(sPT, sPT + P_LO, LDT, 16 * bi, 16 * bj, val);
        else store_ct_bf16(sPT, LDT, 16 * bi, 16 * bj, val);
      }
    }

    // ------------------------------------------------------------ B1: K S, Q S, right-hand side
#pragma unroll
    for (int t = 0; t < DK / 16; ++t) {
      if constexpr (IS) store_ct_split(wS, wS + WS_LO, LDK, 16 * t, 0, S[t]);
      else store_ct_bf16(wS, LDK, 16 * t, 0, S[t]);
    }
    wave_lds_fence();
    f32x4 R[4], QS[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      f32x4 ks = zero4();
      QS[i] = zero4();
#pragma unroll
      for (int s = 0; s < DK / 32; ++s) {
        u32x4 bh, bl, ah, al;
        frag2<IS>(wS, WS_LO, LDK, 0, 32 * s, bh, bl);
        frag2<IS>(sK, K_LO, LDK, 16 * i, 32 * s, ah, al);
        ks = mm<IS, IS>(ks, ah, al, bh, bl);
        frag2<IS>(sQ, K_LO, LDK, 16 * i, 32 * s, ah, al);
        QS[i] = mm<IS, IS>(QS[i], ah, al, bh, bl);
      }
      // R = diag(beta) V - diag(beta e^G) K S at rows 16i + 4lq + v, column 16w + lr
      const int r0 = 16 * i + 4 * lq;
      const u32x2 vw = rows4_tr(sV, LDT, 16 * i, 16 * wave);
      float vv[4] = {__uint_as_float(vw[0] << 16), __uint_as_float(vw[0] & 0xffff0000u),
                     __uint_as_float(vw[1] << 16), __uint_as_float(vw[1] & 0xffff0000u)};
      if constexpr (IS) {
        const u32x2 vl = rows4_tr(sV + V_LO, LDT, 16 * i, 16 * wave);
        vv[0] += __uint_as_float(vl[0] << 16);
        vv[1] += __uint_as_float(vl[0] & 0xffff0000u);
        vv[2] += __uint_as_float(vl[1] << 16);
        vv[3] += __uint_as_float(vl[1] & 0xffff0000u);
      }
#pragma unroll
      for (int v = 0; v < 4; ++v) R[i][v] = sBeta[r0 + v] * vv[v] - sBE[r0 + v] * ks[v];
    }
    __syncthreads();  // L^T, P^T and the diagonal inverses complete

    // issue the next chunk's loads; they land during the rest of this chunk
    if (j + 1 < nchunks) {
      const long long tn = t0 + C;
      prefetch<DK, MODE>(p, pf, tn, (int)((s1 - tn) < C ? (s1 - tn) : C), hk, h, col0);
    }

    // ------------------------------------------------------------ B2: the solve, per wave
    // (I + L) U = R by block forward substitution on 16x16x16 MFMAs.  A C-layout
    // tile (lane (q, r) holds rows 4q..4q+3 of column r) is exactly the B operand
    // layout of that MFMA, so R and U feed the next products from registers.
    f32x4 U[4];
    u32x2 Uh[4], Ul[4];  // bf16 hi/lo of U blocks as B operands
#pragma unroll
    for (int b = 0; b < 4; ++b) {
      f32x4 acc = R[b];
#pragma unroll
      for (int jb = 0; jb < b; ++jb) {
        // acc -= L_b,jb U_jb: the A operand is negated (a sign flip is exact in bf16)
        const u32x2 ah = rows4_tr(sLoT, LDT, 16 * jb, 16 * b) ^ 0x80008000u;
        const u32x2 al = rows4_tr(sLoT + LO_LO, LDT, 16 * jb, 16 * b) ^ 0x80008000u;
        acc = mm3k16(acc, ah, al, Uh[jb], Ul[jb]);
      }
      const u32x2 rh = u32x2{pack_bf16(acc[0], acc[1]), pack_bf16(acc[2], acc[3])};
      const u32x2 rl = u32x2{pack_bf16(lo_part(acc[0]), lo_part(acc[1])),
                             pack_bf16(lo_part(acc[2]), lo_part(acc[3]))};
      const u32x2 th = rows4_tr(sTdT, LDD, 16 * b, 0);
      const u32x2 tl = rows4_tr(sTdT + TD_LO, LDD, 16 * b, 0);
      U[b] = mm3k16(zero4(), th, tl, rh, rl);
      Uh[b] = u32x2{pack_bf16(U[b][0], U[b][1]), pack_bf16(U[b][2], U[b][3])};
      Ul[b] = u32x2{pack_bf16(lo_part(U[b][0]), lo_part(U[b][1])),
                    pack_bf16(lo_part(U[b][2]), lo_part(U[b][3]))};
    }
    // Vt = diag(e^{G_last - G}) V_new for the state update
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      f32x4 vt;
      const float4 el = *(const float4*)(sEL + 16 * i + 4 * lq);
      vt[0] = U[i][0] * el.x; vt[1] = U[i][1] * el.y; vt[2] = U[i][2] * el.z; vt[3] = U[i][3] * el.w;
      store_ct_split(wVt, wVt + W_LO, LDT, 16 * i, 0, vt);
    }

    // ------------------------------------------------------------ B3: O = scale e^G (Q S) + P V_new
    f32x4 OUT[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      f32x4& o = OUT[i];
      const float4 eg = *(const float4*)(sEG + 16 * i + 4 * lq);
      o[0] = p.scale * eg.x * QS[i][0]; o[1] = p.scale * eg.y * QS[i][1];
      o[2] = p.scale * eg.z * QS[i][2]; o[3] = p.scale * eg.w * QS[i][3];
#pragma unroll
      for (int jb = 0; jb <= i; ++jb) {  // P is lower triangular
        const u32x2 ah = rows4_tr(sPT, LDT, 16 * jb, 16 * i);
        o = mma16k16(ah, Uh[jb], o);
        if constexpr (OS) {
          const u32x2 al = rows4_tr(sPT + P_LO, LDT, 16 * jb, 16 * i);
          o = mma16k16(ah, Ul[jb], o);
          o = mma16k16(al, Uh[jb], o);
        }
      }
      if constexpr (MODE != MODE_LAYER) {
        float* orow = p.o + (t0 * p.Hv + h) * (long long)DV + col0 + 16 * wave + lr;
        const long long rs = (long long)p.Hv * DV;  // row stride of o
        if (nvalid == C) {  // uniform: every row of a full chunk is stored
#pragma unroll
          for (int v = 0; v < 4; ++v) orow[(16 * i + 4 * lq + v) * rs] = o[v];
        } else {
#pragma unroll
          for (int v = 0; v < 4; ++v) {
            const int r = 16 * i + 4 * lq + v;
            if (r < nvalid) orow[r * rs] = o[v];
          }
        }
      } else {
#pragma unroll
        for (int v = 0; v < 4; ++v) {
          const float ss = group_sum_dpp<16>(o[v] * o[v]);
          if (lr == 0) sNP[(16 * i + 4 * lq + v) * NWC + wave] = ss;
        }
      }
    }

    // ------------------------------------------------------------ B4: S <- e^{G_last} S + K^T Vt
    wave_lds_fence();  // Vt^T stores above are visible to the wave's fragment loads
    const float gl = sEG[C - 1];
#pragma unroll
    for (int t = 0; t < DK / 16; ++t) {
#pragma unroll
      for (int v = 0; v < 4; ++v) S[t][v] *= gl;
#pragma unroll
      for (int s = 0; s < 2; ++s) {
        u32x4 ah, al, bh, bl;
        ah = frag_tr(sK, LDK, 32 * s, 16 * t);
        al = IS ? frag_tr(sK + K_LO, LDK, 32 * s, 16 * t) : ah;
        frag2<true>(wVt, W_LO, LDT, 0, 32 * s, bh, bl);
        S[t] = mm<IS, true>(S[t], ah, al, bh, bl);
      }
    }

    if constexpr (MODE == MODE_LAYER) {
      // gated RMSNorm epilogue (deltanet.py:282-293), fp32 like the reference
      __syncthreads();
      const int col = col0 + 16 * wave + lr;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
#pragma unroll
        for (int v = 0; v < 4; ++v) {
          const int r = 16 * i + 4 * lq + v;
          if (r < nvalid) {
            float ss = 0.f;
#pragma unroll
            for (int w2 = 0; w2 < NWC; ++w2) ss += sNP[r * NWC + w2];
            const size_t idx = ((size_t)(t0 + r) * p.Hv + h) * DV + col;
            if (nb == 1) {
              const float rn = rsqrtf(ss / (float)DV + p.eps);
              const float zz = bf2f(((const bf16_t*)p.z)[idx]);
              ((bf16_t*)p.out)[idx] = f2bf(p.norm_w[col] * (OUT[i][v] * rn) * siluf_(zz));
            } else {
              // unnormalised o in bf16 and this block's share of sum(o^2)
              ((bf16_t*)p.o_part)[idx] = f2bf(OUT[i][v]);
              if (wave == 0 && lr == 0) p.ss_part[((size_t)(t0 + r) * p.Hv + h) * nb + blk] = ss;
            }
          }
        }
      }
    }
  }

  if (p.final_state) {
#pragma unroll
    for (int t = 0; t < DK / 16; ++t)
#pragma unroll
      for (int v = 0; v < 4; ++v)
        p.final_state[state_off + (size_t)(16 * t + 4 * lq + v) * DV] = S[t][v];
  }

  if constexpr (MODE == MODE_LAYER) {
    // conv cache after the prefill: the last K-1 raw inputs of the sequence.  q/k
    // channels are written by the first value head of their key head only.
    if (p.conv_state_out) {
      const int K = p.conv_k;
      const bool own_qk = (h % gqa) == 0 && blk == 0;
      for (int it = tid; it < HW * (K - 1); it += NT) {
        const int ci = it / (K - 1), jj = it % (K - 1);
        if (ci < 2 * DK && !own_qk) continue;
        int ch;
        if (ci < DK) ch = hk * DK + ci;
        else if (ci < 2 * DK) ch = p.Hk * DK + hk * DK + (ci - DK);
        else ch = 2 * p.Hk * DK + h * DV + col0 + (ci - 2 * DK);
        const long long t = s1 - (K - 1) + jj;
        bf16_t val = 0;
        if (t >= s0) {
          val = ((const bf16_t*)p.mixed_qkv)[t * p.conv_dim + ch];
        } else if (p.conv_state_in) {
          const int slot = (K - 1) - (int)(s0 - t);
          val = ((const bf16_t*)p.conv_state_in)[((size_t)n * p.conv_dim + ch) * (K - 1) + slot];
        }
        ((bf16_t*)p.conv_state_out)[((size_t)n * p.conv_dim + ch) * (K - 1) + jj] = val;
      }
    }
  }
}

template <int DK, int MODE>
hipError_t launch_cfg(const ChunkParams& p, hipStream_t stream) {
  const unsigned grid = (unsigned)(p.N * p.Hv * p.nb);
  hipLaunchKernelGGL((chunk_kernel<DK, MODE>), dim3(grid), dim3(NT), 0, stream, p);
  return hipGetLastError();
}

}  // namespace

int chunk_block_cols() { return BV; }

bool chunk_dims_supported(int dk, int dv, bool f32_inputs) {
  if (dv % BV != 0 || dv > 256) return false;
  if (f32_inputs) return dk == 32 || dk == 64;
  return dk == 64 || dk == 128;
}

bool layer_dims_supported(int dk, int dv) { return chunk_dims_supported(dk, dv, false); }

hipError_t launch_chunk(const ChunkParams& p, bool f32_inputs, hipStream_t stream) {
  if (f32_inputs) {
    if (p.dk == 64) return launch_cfg<64, MODE_F32>(p, stream);
    if (p.dk == 32) return launch_cfg<32, MODE_F32>(p, stream);
    return hipErrorInvalidValue;
  }
  if (p.dk == 128) return launch_cfg<128, MODE_BF16>(p, stream);
  if (p.dk == 64) return launch_cfg<64, MODE_BF16>(p, stream);
  return hipErrorInvalidValue;
}

hipError_t launch_layer(const ChunkParams& p, hipStream_t stream) {
  if (p.dk == 128) return launch_cfg<128, MODE_LAYER>(p, stream);
  if (p.dk == 64) return launch_cfg<64, MODE_LAYER>(p, stream);
  return hipErrorInvalidValue;
}

}  // namespace omx
