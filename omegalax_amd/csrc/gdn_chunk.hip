// Recurrent scan of the chunked gated delta rule on gfx950.
//
// Follows chunk_gated_delta_rule (omegalax/models/qwen3_5/deltanet.py:53-153),
// restated for MFMA.  The chunk-parallel part -- conv, L2 norm, gates, and per
// chunk T = (I + L)^-1 and P (deltanet.py:98-113, 130-131) -- is done for all
// chunks beforehand by the preparation kernel (gdn_prep.hip), which leaves a
// record per (chunk, value head).  This kernel carries the state S across a
// sequence's chunks:
//     R     = diag(beta) V - diag(beta e^G) (K S)
//     V_new = T R                  (= U - W S of deltanet.py:115-116, 133-134)
//     O     = scale e^G (Q S) + P V_new                        (:130-137)
//     S    <- e^{G_last} S + K^T diag(e^{G_last - G}) V_new    (:139-142)
//
// Work mapping.  One workgroup of 4 wavefronts per (sequence, value head,
// 64-column block of dv) walks that sequence's chunks in order.  Wavefront w
// owns state columns [16w, 16w+16) of the block: its fp32 slice S[dk][16] stays
// in MFMA accumulator registers for the whole sequence, and every product that
// touches it runs on that wavefront alone, between two workgroup barriers per
// chunk that guard the shared staging arrays.  The next chunk's K, Q, V rows and
// record are loaded into registers while the current chunk computes.
//
// Precision.  MFMA inputs are bf16 with fp32 accumulation.  K, Q, V are bf16 on
// the bf16 and layer paths (exact), or fp32 split into hi+lo bf16 pairs
// (MODE_F32).  T and the right-hand side R enter V_new = T R as hi+lo pairs, and
// so does the state-update operand diag(e^{G_last-G}) V_new; with bf16 inputs S
// enters K S / Q S, and P, V_new enter P V_new, as single bf16.
//
// Modes: MODE_BF16 / MODE_F32 (core function) store o in fp32.  MODE_LAYER stores
// o in bf16 with each wavefront's partial sums of o^2 per token; the epilogue
// kernel (gdn_epilogue.hip) adds them and applies the gated RMSNorm
// (deltanet.py:282-293).
#include <type_traits>

#include "gdn_chunk.h"
#include "gdn_kernels.h"

namespace omx {

namespace {

constexpr int C = kC;
constexpr int NWC = 4;         // column wavefronts per workgroup
constexpr int NT = kNT;
constexpr int BV = 16 * NWC;   // state columns per workgroup
constexpr int LDT = kLDT;
static_assert(NT == 64 * NWC, "threads");

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
  static constexpr int REC = rec_bytes(MODE);
  static constexpr int NREC16 = REC / 16;
  static constexpr int NI_R = (NREC16 + NT - 1) / NT;
  // per-wave scratch: S^T (K S, Q S), then Vt^T (hi, lo)
  static constexpr int WS_S = NS * 16 * LDK * 2;
  static constexpr int WS_U = 2 * 16 * LDT * 2;
  static constexpr int WS = WS_S > WS_U ? WS_S : WS_U;
  static constexpr int TOTAL =
      2 * NS * C * LDK * 2 + NS * C * LDT * 2 + REC + NWC * WS;
  static_assert(TOTAL <= 160 * 1024, "LDS budget");
  static_assert(DK % 32 == 0 && DK <= 128, "dk");
  static_assert(NI_KQ * NT == 2 * C * SEGS && (C * SEGS) % NT == 0, "item split");
  static_assert(NI_V * NT == C * (BV / 8), "item split");
};

// Per-thread register prefetch of one chunk's inputs.
template <int DK, int MODE>
struct Prefetch {
  using Q_ = Cfg<DK, MODE>;
  u32x4 kq[Q_::NI_KQ][Q_::RAWW];
  u32x4 v[Q_::NI_V][Q_::RAWW];
  u32x4 rec[Q_::NI_R];
};

// Loads of one chunk, in four parts (PART = 0..3, or -1 for all) so that a chunk's
// prefetch can be spread over the previous chunk's compute phases: the four
// wavefronts of a CU issuing all their loads at once would queue them behind
// each other in the CU's memory pipeline.  Parts: record, v rows, k rows, q rows.
template <int DK, int MODE, int PART = -1>
__device__ __forceinline__ void prefetch(const ChunkParams& p, Prefetch<DK, MODE>& pf,
                                         long long t0, int nvalid, const unsigned char* rec,
                                         int hk, int h, int col0) {
  using Q_ = Cfg<DK, MODE>;
  constexpr bool F32 = MODE == MODE_F32;
  const int tid = threadIdx.x;
  if constexpr (PART == -1 || PART == 0) {
#pragma unroll
    for (int k = 0; k < Q_::NI_R; ++k) {
      const int it = tid + k * NT;
      if (Q_::NI_R * NT == Q_::NREC16 || it < Q_::NREC16) pf.rec[k] = ((const u32x4*)rec)[it];
    }
  }
  if constexpr (PART == -1 || PART == 1) {
#pragma unroll
    for (int k = 0; k < Q_::NI_V; ++k) {
      const int it = tid + k * NT;
      const int r = it / (BV / 8), seg = it % (BV / 8);
      const long long tok = t0 + (r < nvalid ? r : nvalid - 1);
      load_raw<F32>(p.vs, tok * p.vs_ld + (long long)h * p.DV + col0 + seg * 8, pf.v[k]);
    }
  }
#pragma unroll
  for (int k = 0; k < Q_::NI_KQ; ++k) {
    constexpr int PER = C * Q_::SEGS;
    const int which = (k * NT) / PER;  // 0 = k (part 2), 1 = q (part 3); folded when unrolled
    if (PART != -1 && PART != 2 + which) continue;
    const int rem = (k * NT) % PER + tid;
    const int r = rem / Q_::SEGS, seg = rem % Q_::SEGS;
    // rows past the sequence end load the last valid row (in bounds); staging zeroes
    // them, so the loaded registers are not touched until the data is needed
    const long long tok = t0 + (r < nvalid ? r : nvalid - 1);
    load_raw<F32>(which == 0 ? p.ks : p.qs,
                  tok * (which == 0 ? p.ks_ld : p.qs_ld) + (long long)hk * DK + seg * 8, pf.kq[k]);
  }
}

template <int DK, int MODE>
// One workgroup per CU is the design point (the state fills the register file), so the
// compiler may use the whole file instead of holding back for a second workgroup.
__global__ __launch_bounds__(NT) __attribute__((amdgpu_waves_per_eu(1, 1))) void scan_kernel(ChunkParams p) {
  using Q_ = Cfg<DK, MODE>;
  constexpr int LDK = Q_::LDK, SEGS = Q_::SEGS;
  constexpr bool IS = Q_::IS, OS = Q_::OS;
  constexpr bool F32 = MODE == MODE_F32;
  // Each buffer is its own __shared__ object, so the compiler can tell their
  // accesses apart and overlap loads of one with stores to another.
  __shared__ __align__(16) bf16_t sK[Q_::NS * C * LDK];
  __shared__ __align__(16) bf16_t sQ[Q_::NS * C * LDK];
  __shared__ __align__(16) bf16_t sV[Q_::NS * C * LDT];
  __shared__ __align__(16) unsigned char sRec[Q_::REC];     // the chunk's record
  __shared__ __align__(16) bf16_t sWS[NWC * Q_::WS / 2];    // per-wave scratch
  const float* sGate = (const float*)(sRec + kRecG);
  const float* sBeta = sGate + kGateBeta * C;  // beta
  const float* sBE = sGate + kGateBE * C;      // beta e^G
  const float* sEG = sGate + kGateEG * C;      // e^G
  const float* sEL = sGate + kGateEL * C;      // e^{G_last - G}
  constexpr int K_LO = C * LDK, V_LO = C * LDT;

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
  seq_range(p.cu_seqlens, n, p.T, s0, s1);
  const int nchunks = (int)((s1 - s0 + C - 1) / C);
  const int cbase = p.chunk_off ? p.chunk_off[n] : n * p.nch;
  // record of chunk j; the index is clamped so that inconsistent offsets stay in bounds
  auto rec_of = [&](int j) {
    const int ci = cbase + j < p.n_rec ? cbase + j : p.n_rec - 1;
    return p.rec + ((size_t)ci * p.Hv + h) * Q_::REC;
  };

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
  if (nchunks > 0)
    prefetch<DK, MODE>(p, pf, s0, (int)((s1 - s0) < C ? (s1 - s0) : C), rec_of(0), hk, h, col0);

  for (int j = 0; j < nchunks; ++j) {
    const long long t0 = s0 + (long long)j * C;
    const int nvalid = (int)((s1 - t0) < C ? (s1 - t0) : C);
    __syncthreads();  // the previous chunk's readers are done with the shared arrays

    // ------------------------------------------------------------ stage the chunk
    const bool full = nvalid == C;  // uniform: only a sequence's last chunk has padded rows
#pragma unroll
    for (int k = 0; k < Q_::NI_KQ; ++k) {
      constexpr int PER = C * SEGS;
      const int which = (k * NT) / PER;
      const int rem2 = (k * NT) % PER + tid;
      const int r = rem2 / SEGS, seg = rem2 % SEGS;
      bf16_t* dst = (which == 0 ? sK : sQ) + r * LDK + seg * 8;
      if constexpr (F32) {
        float x[8];
        unpack8<true>(pf.kq[k], x);
        const float keep = (float)(r < nvalid);  // padded rows are zero
#pragma unroll
        for (int e = 0; e < 8; ++e) x[e] *= keep;
        *(u32x4*)dst = pack8(x);
        *(u32x4*)(dst + K_LO) = pack8_lo(x);
      } else if (full) {
        *(u32x4*)dst = pf.kq[k][0];
      } else {
        const unsigned keep = r < nvalid ? 0xffffffffu : 0u;  // padded rows are zero
        *(u32x4*)dst = pf.kq[k][0] & keep;
      }
    }
#pragma unroll
    for (int k = 0; k < Q_::NI_V; ++k) {
      const int it = tid + k * NT;
      const int r = it / (BV / 8), seg = it % (BV / 8);
      bf16_t* dst = sV + r * LDT + seg * 8;
      if constexpr (F32) {
        float x[8];
        unpack8<true>(pf.v[k], x);
        const float keep = (float)(r < nvalid);
#pragma unroll
        for (int e = 0; e < 8; ++e) x[e] *= keep;
        *(u32x4*)dst = pack8(x);
        *(u32x4*)(dst + V_LO) = pack8_lo(x);
      } else if (full) {
        *(u32x4*)dst = pf.v[k][0];
      } else {
        const unsigned keep = r < nvalid ? 0xffffffffu : 0u;
        *(u32x4*)dst = pf.v[k][0] & keep;
      }
    }
#pragma unroll
    for (int k = 0; k < Q_::NI_R; ++k) {
      const int it = tid + k * NT;
      if (Q_::NI_R * NT == Q_::NREC16 || it < Q_::NREC16) ((u32x4*)sRec)[it] = pf.rec[k];
    }
    __syncthreads();

    // issue the next chunk's loads; they land during the rest of this chunk
    if (j + 1 < nchunks) {
      const long long tn = t0 + C;
      prefetch<DK, MODE>(p, pf, tn, (int)((s1 - tn) < C ? (s1 - tn) : C), rec_of(j + 1), hk, h,
                         col0);
    }

    // ------------------------------------------------------------ K S, Q S, right-hand side
    // S^T goes to the wave's scratch as the B operand of K S and Q S.  Every operand
    // that does not depend on S is read from LDS in one batch while it lands, so
    // the products below run back to back on registers.
#pragma unroll
    for (int t = 0; t < DK / 16; ++t) {
      if constexpr (IS) store_ct_split(wS, wS + WS_LO, LDK, 16 * t, 0, S[t]);
      else store_ct_bf16(wS, LDK, 16 * t, 0, S[t]);
    }
    constexpr int NSK = DK / 32;
    u32x4 kh[4][NSK], kl[4][NSK], qh[4][NSK], ql[4][NSK];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int s2 = 0; s2 < NSK; ++s2) {
        frag2<IS>(sK, K_LO, LDK, 16 * i, 32 * s2, kh[i][s2], kl[i][s2]);
        frag2<IS>(sQ, K_LO, LDK, 16 * i, 32 * s2, qh[i][s2], ql[i][s2]);
      }
    float vv[4][4];  // V at rows 16i + 4lq + v, column 16w + lr
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const u32x2 vw = rows4_tr(sV, LDT, 16 * i, 16 * wave);
      vv[i][0] = __uint_as_float(vw[0] << 16);
      vv[i][1] = __uint_as_float(vw[0] & 0xffff0000u);
      vv[i][2] = __uint_as_float(vw[1] << 16);
      vv[i][3] = __uint_as_float(vw[1] & 0xffff0000u);
      if constexpr (IS) {
        const u32x2 vl = rows4_tr(sV + V_LO, LDT, 16 * i, 16 * wave);
        vv[i][0] += __uint_as_float(vl[0] << 16);
        vv[i][1] += __uint_as_float(vl[0] & 0xffff0000u);
        vv[i][2] += __uint_as_float(vl[1] << 16);
        vv[i][3] += __uint_as_float(vl[1] & 0xffff0000u);
      }
    }
    wave_lds_fence();
    u32x4 sh[NSK], sl[NSK];
#pragma unroll
    for (int s2 = 0; s2 < NSK; ++s2) frag2<IS>(wS, WS_LO, LDK, 0, 32 * s2, sh[s2], sl[s2]);
    f32x4 KS[4], QS[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      KS[i] = zero4();
      QS[i] = zero4();
    }
#pragma unroll
    for (int s2 = 0; s2 < NSK; ++s2)
#pragma unroll
      for (int i = 0; i < 4; ++i) {  // eight independent accumulation chains
        KS[i] = mm<IS, IS>(KS[i], kh[i][s2], kl[i][s2], sh[s2], sl[s2]);
        QS[i] = mm<IS, IS>(QS[i], qh[i][s2], ql[i][s2], sh[s2], sl[s2]);
      }
    // T fragments for V_new = T R (read while the products run)
    u32x2 th[10], tl[10];
#pragma unroll
    for (int x = 0; x < 10; ++x) {
      const unsigned char* tp = sRec + kRecT + 2 * x * kTileBytes + 8 * l;
      th[x] = *(const u32x2*)tp;
      tl[x] = *(const u32x2*)(tp + kTileBytes);
    }
    // R = diag(beta) V - diag(beta e^G) K S at rows 16i + 4lq + v, column 16w + lr
    f32x4 R[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int r0 = 16 * i + 4 * lq;
      const float4 bt = *(const float4*)(sBeta + r0);
      const float4 be = *(const float4*)(sBE + r0);
      R[i][0] = bt.x * vv[i][0] - be.x * KS[i][0];
      R[i][1] = bt.y * vv[i][1] - be.y * KS[i][1];
      R[i][2] = bt.z * vv[i][2] - be.z * KS[i][2];
      R[i][3] = bt.w * vv[i][3] - be.w * KS[i][3];
    }

    // ------------------------------------------------------------ V_new = T R
    // A C-layout tile (lane (q, r) holds rows 4q..4q+3 of column r) is exactly the
    // B operand layout of the 16x16x16 MFMA, so R feeds the products from
    // registers; T comes as ready A-operand fragments.  The hi*hi, hi*lo and
    // lo*hi parts accumulate separately: twelve independent chains.
    u32x2 Rh[4], Rl[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      Rh[i] = pack_hi4(R[i]);
      Rl[i] = pack_lo4(R[i]);
    }
    f32x4 U[4];
    u32x2 Uh[4], Ul[4];  // bf16 hi/lo of V_new blocks as B operands
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      f32x4 a0 = zero4(), a1 = zero4(), a2 = zero4();
#pragma unroll
      for (int kb = 0; kb <= i; ++kb) {
        const int x = tile_index(i, kb);
        a0 = mma16k16(th[x], Rh[kb], a0);
        a1 = mma16k16(th[x], Rl[kb], a1);
        a2 = mma16k16(tl[x], Rh[kb], a2);
      }
      U[i] = a0 + a1 + a2;
      Uh[i] = pack_hi4(U[i]);
      Ul[i] = pack_lo4(U[i]);
    }
    // P fragments and the K^T fragments of the state update (read while V_new forms)
    u32x2 ph[10], pl[10];
#pragma unroll
    for (int x = 0; x < 10; ++x) {
      ph[x] = *(const u32x2*)(sRec + kRecP + x * kTileBytes + 8 * l);
      if constexpr (OS) pl[x] = *(const u32x2*)(sRec + kRecPL + x * kTileBytes + 8 * l);
      else pl[x] = ph[x];
    }
    u32x4 kth[DK / 16][2], ktl[DK / 16][2];
#pragma unroll
    for (int t = 0; t < DK / 16; ++t)
#pragma unroll
      for (int s2 = 0; s2 < 2; ++s2) {
        kth[t][s2] = frag_tr(sK, LDK, 32 * s2, 16 * t);
        ktl[t][s2] = IS ? frag_tr(sK + K_LO, LDK, 32 * s2, 16 * t) : kth[t][s2];
      }
    // Vt = diag(e^{G_last - G}) V_new for the state update
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      f32x4 vt;
      const float4 el = *(const float4*)(sEL + 16 * i + 4 * lq);
      vt[0] = U[i][0] * el.x; vt[1] = U[i][1] * el.y; vt[2] = U[i][2] * el.z; vt[3] = U[i][3] * el.w;
      store_ct_split(wVt, wVt + W_LO, LDT, 16 * i, 0, vt);
    }

    // ------------------------------------------------------------ O = scale e^G (Q S) + P V_new
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      f32x4 o;
      const float4 eg = *(const float4*)(sEG + 16 * i + 4 * lq);
      o[0] = p.scale * eg.x * QS[i][0]; o[1] = p.scale * eg.y * QS[i][1];
      o[2] = p.scale * eg.z * QS[i][2]; o[3] = p.scale * eg.w * QS[i][3];
#pragma unroll
      for (int jb = 0; jb <= i; ++jb) {  // P is lower triangular
        const int x = tile_index(i, jb);
        o = mma16k16(ph[x], Uh[jb], o);
        if constexpr (OS) {
          o = mma16k16(ph[x], Ul[jb], o);
          o = mma16k16(pl[x], Uh[jb], o);
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
        // unnormalised o in bf16 and this wave's share of sum(o^2) over its 16
        // columns; the epilogue kernel adds the shares and applies the norm
        const int col = col0 + 16 * wave + lr;
        const int nparts = nb * NWC;
#pragma unroll
        for (int v = 0; v < 4; ++v) {
          const float ss = group_sum_dpp<16>(o[v] * o[v]);
          const int r = 16 * i + 4 * lq + v;
          if (r < nvalid) {
            const size_t row = (size_t)(t0 + r) * p.Hv + h;
            ((bf16_t*)p.o_part)[row * DV + col] = f2bf(o[v]);
            if (lr == 0) p.ss_part[row * nparts + blk * NWC + wave] = ss;
          }
        }
      }
    }


    // ------------------------------------------------------------ S <- e^{G_last} S + K^T Vt
    wave_lds_fence();  // Vt^T stores above are visible to the wave's fragment loads
    u32x4 vth[2], vtl[2];
#pragma unroll
    for (int s2 = 0; s2 < 2; ++s2) frag2<true>(wVt, W_LO, LDT, 0, 32 * s2, vth[s2], vtl[s2]);
    const float gl = sEG[C - 1];
#pragma unroll
    for (int t = 0; t < DK / 16; ++t) {
#pragma unroll
      for (int v = 0; v < 4; ++v) S[t][v] *= gl;
#pragma unroll
      for (int s2 = 0; s2 < 2; ++s2) S[t] = mm<IS, true>(S[t], kth[t][s2], ktl[t][s2], vth[s2], vtl[s2]);
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
      constexpr int HW = 2 * DK + BV;  // q | k | this block's v channels
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
hipError_t launch_scan_cfg(const ChunkParams& p, hipStream_t stream) {
  const unsigned grid = (unsigned)(p.N * p.Hv * p.nb);
  hipLaunchKernelGGL((scan_kernel<DK, MODE>), dim3(grid), dim3(NT), 0, stream, p);
  return hipGetLastError();
}

}  // namespace

int chunk_block_cols() { return BV; }

int chunk_record_bytes(int mode) { return rec_bytes(mode); }

int layer_norm_parts(int dv) { return dv / BV * NWC; }

bool chunk_dims_supported(int dk, int dv, bool f32_inputs) {
  if (dv % BV != 0 || dv > 256) return false;
  if (f32_inputs) return dk == 32 || dk == 64;
  return dk == 64 || dk == 128;
}

bool layer_dims_supported(int dk, int dv) { return chunk_dims_supported(dk, dv, false); }

hipError_t launch_scan(const ChunkParams& p, int mode, hipStream_t stream) {
  if (mode == MODE_F32) {
    if (p.dk == 64) return launch_scan_cfg<64, MODE_F32>(p, stream);
    if (p.dk == 32) return launch_scan_cfg<32, MODE_F32>(p, stream);
    return hipErrorInvalidValue;
  }
  if (mode == MODE_LAYER) {
    if (p.dk == 128) return launch_scan_cfg<128, MODE_LAYER>(p, stream);
    if (p.dk == 64) return launch_scan_cfg<64, MODE_LAYER>(p, stream);
    return hipErrorInvalidValue;
  }
  if (p.dk == 128) return launch_scan_cfg<128, MODE_BF16>(p, stream);
  if (p.dk == 64) return launch_scan_cfg<64, MODE_BF16>(p, stream);
  return hipErrorInvalidValue;
}

}  // namespace omx
