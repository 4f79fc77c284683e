// Recurrent scan of the chunked gated delta rule on gfx950.
//
// Follows chunk_gated_delta_rule (omegalax/models/qwen3_5/deltanet.py:53-153),
// restated for MFMA.  The chunk-parallel part -- conv, L2 norm, gates, and per
// chunk T = (I + L)^-1 and P (deltanet.py:98-113, 130-131) -- is done for all
// chunks beforehand by the preparation kernel (gdn_prep.hip), which leaves a
// record per (chunk, value head).  This kernel carries the state S across a
// sequence's chunks:
//     R     = V - diag(e^G) (K S)
//     V_new = T diag(beta) R       (= U - W S of deltanet.py:115-116, 133-134)
//     O     = scale e^G (Q S) + P V_new                        (:130-137)
//     S    <- e^{G_last} S + K^T diag(e^{G_last - G}) V_new    (:139-142)
//
// Work mapping.  One workgroup per (sequence, value head, block of dv columns) walks
// that sequence's chunks in order; a block is 64 columns (4 compute wavefronts), or on
// the direct-load path 32 or 16 when 64-column blocks would leave CUs idle.  Wavefront w
// owns state columns [16w, 16w+16) of the block: its fp32 slice S[dk][16] stays in MFMA
// accumulator registers for the whole sequence, and every product that touches it runs
// on that wavefront alone.  All products are 16x16x32 MFMAs: the
// state's rows are kept in an order (state_row) in which two accumulator tiles
// side by side are the B operand of K S and Q S, and T, P arrive from the record
// as 16x32 operands over pairs of 16-token blocks whose contraction order matches
// two C-layout tiles of R or V_new side by side.  With bf16 inputs and dk = 128
// the next chunk's K, Q, V rows and record are loaded straight into the other of
// two LDS buffers while the current chunk computes (one workgroup barrier per
// chunk); otherwise they are staged through registers.  On the layer path with
// dk = 128 two helper wavefronts form the next chunk's V rows instead (conv + SiLU of
// mixed_qkv's value channels, deltanet.py:243), so the preparation kernel neither
// reads the value channels nor writes conv(v) to the workspace.
//
// Precision.  MFMA inputs are bf16 with fp32 accumulation.  K, Q, V are bf16 on
// the bf16 and layer paths (exact), or fp32 split into hi+lo bf16 pairs
// (MODE_F32).  T and the right-hand side R enter V_new = T R as hi+lo pairs, and
// so does the state-update operand diag(e^{G_last-G}) V_new; with bf16 inputs S
// enters K S / Q S, and P, V_new enter P V_new, as single bf16, except in the layer
// backward's recompute (BWD with p.o set), which forms o from hi+lo S, V_new and P.
//
// Modes: MODE_BF16 / MODE_F32 (core function) store o in fp32.  MODE_LAYER stores
// o in bf16; the epilogue kernel (gdn_epilogue.hip) applies the gated RMSNorm
// (deltanet.py:282-293).
#include <type_traits>

#include "gdn_chunk.h"
#include "gdn_conv.h"
#include "gdn_kernels.h"

namespace omx {

namespace {

constexpr int C = kC;
constexpr int LDT = kLDT;
constexpr int kBlockCols = 64;  // dv columns per block of the other kernels (nb = dv / 64)

// NWC_: 16-column state tiles (compute wavefronts) per workgroup.  Four on every path;
// the direct-load path also runs with two or one, so that sequences x heads x dv / 16 tiles
// fill the chip when 64-column workgroups would leave CUs idle.
template <int DK, int MODE, int NWC_ = 4, bool BWD_ = false>
struct Cfg {
  static constexpr int NWC = NWC_;
  static constexpr int BV = 16 * NWC;  // state columns per workgroup
  static constexpr int NT = 64 * NWC;  // compute threads
  static constexpr bool IS = MODE == MODE_F32;  // q/k/v split hi+lo
  static constexpr bool OS = MODE == MODE_F32;  // output-path operands split
  static constexpr int NS = IS ? 2 : 1;
  static constexpr int RAWW = IS ? 2 : 1;       // u32x4 words per 8-element input segment
  static constexpr int LDK = DK + 8;            // row stride of [token][dk] arrays
  static constexpr int SEGS = DK / 8;           // 8-element segments per q/k row
  static constexpr int NI_KQ = 2 * C * SEGS / NT;
  static constexpr int NI_V = C * (BV / 8) / NT;
  static constexpr int REC = rec_bytes(MODE, BWD_);
  static constexpr int NREC16 = REC / 16;
  // 16-byte pieces read per chunk: a backward scan that forms no o skips P's lo parts
  static constexpr int NREC16_NO_O = rec_bytes(MODE) / 16;
  static constexpr int NI_R = (NREC16 + NT - 1) / NT;
  // bf16 rows with dk = 128 are loaded straight from global memory into one of two
  // LDS buffers (no register staging): unpadded rows with XOR-swizzled 16-byte
  // segments.  fp32 inputs (split on staging) and dk = 64 stage through registers
  // into padded rows.
  static constexpr bool DIRECT = MODE != MODE_F32 && DK == 128;
  // (layer, direct loads) the value channels' conv + SiLU runs here, in NH helper
  // wavefronts that form the next chunk's V rows while the compute wavefronts scan
  static constexpr bool VCONV = MODE == MODE_LAYER && layer_v_in_scan(DK);
  static constexpr int NH = VCONV ? 2 : 0;
  // with direct loads one more wavefront issues them (and NH more form V); sharing SIMDs
  // with the compute wavefronts, each may then hold at most half the register file
  // loader wavefronts: two in the backward's bf16 recompute (the chunk after next's K/Q
  // rows in one's registers, its V rows and record in the other's, so that the loads are
  // not queued behind the state stores of the same step) and in the bf16 forward scan's
  // narrow workgroups (where the second loader takes a SIMD no compute wavefront uses:
  // C4 2.663-2.666 -> 2.605-2.639 ms), one elsewhere.  In the forward scan's 64-column
  // workgroups the second loader measured slower (C1 core call 0.311-0.319 against
  // 0.292-0.297 ms).
  static constexpr int NL = DIRECT ? (MODE == MODE_BF16 && (BWD_ || NWC_ < 4) ? 2 : 1) : 0;
  static constexpr int NTH = DIRECT ? NT + 64 * (NL + NH) : NT;
  static constexpr int WPE = (NTH / 64 + 3) / 4;
  static constexpr int NBUF = DIRECT ? 2 : 1;
  static constexpr int SZK = DIRECT ? C * DK : NS * C * LDK;  // elements of a K or Q buffer
  static constexpr int SZV = DIRECT ? C * BV : NS * C * LDT;  // elements of a V buffer
  static constexpr int TOTAL = NBUF * (2 * SZK * 2 + SZV * 2 + REC);
  static_assert(TOTAL <= 160 * 1024, "LDS budget");
  static_assert(!DIRECT || REC % 1024 == 0, "direct loads move the record in 1 KiB pieces");
  static_assert(DK % 32 == 0 && DK <= 128, "dk");
  static_assert(DIRECT || NWC == 4, "register staging runs four column wavefronts");
  static_assert(NI_KQ * NT == 2 * C * SEGS && (C * SEGS) % NT == 0, "item split");
  static_assert(NI_V * NT == C * (BV / 8), "item split");
  static_assert(!VCONV || DIRECT, "the helper wavefronts run beside the direct loads");
  static_assert(!VCONV || (BV / 8) * (C / (BV / 16)) == 64 * NH, "one V task per helper lane");
};

// Per-thread register prefetch of one chunk's inputs.
template <int DK, int MODE, bool BWD>
struct Prefetch {
  using Q_ = Cfg<DK, MODE, 4, BWD>;
  u32x4 kq[Q_::NI_KQ][Q_::RAWW];
  u32x4 v[Q_::NI_V][Q_::RAWW];
  u32x4 rec[Q_::NI_R];
};

// Loads of one chunk's k, q, v rows and record into registers.  Addresses are a
// chunk-uniform base (scalar registers) plus a per-thread 32-bit offset that does not
// change from chunk to chunk; only a sequence's last, partial chunk clamps its rows
// (rows past the end load the last valid row, in bounds, and staging zeroes them).
template <int DK, int MODE, bool BWD>
__device__ __forceinline__ void prefetch(const ChunkParams& p, Prefetch<DK, MODE, BWD>& pf,
                                         long long t0, int nvalid, const unsigned char* rec,
                                         int hk, int h, int col0) {
  using Q_ = Cfg<DK, MODE, 4, BWD>;
  constexpr int NT = Q_::NT, BV = Q_::BV;
  constexpr bool F32 = MODE == MODE_F32;
  using In = typename std::conditional<F32, float, bf16_t>::type;
  const int tid = threadIdx.x;
  const int nrec16 = BWD && !p.o ? Q_::NREC16_NO_O : Q_::NREC16;
#pragma unroll
  for (int k = 0; k < Q_::NI_R; ++k) {
    const int it = tid + k * NT;
    if (it < nrec16) pf.rec[k] = ((const u32x4*)rec)[it];
  }
  const unsigned ksl = (unsigned)p.ks_ld, qsl = (unsigned)p.qs_ld, vsl = (unsigned)p.vs_ld;
  const In* kb = (const In*)p.ks + t0 * p.ks_ld + (long long)hk * DK;
  const In* qb = (const In*)p.qs + t0 * p.qs_ld + (long long)hk * DK;
  const In* vb = (const In*)p.vs + t0 * p.vs_ld + (long long)h * p.DV + col0;
  const bool full = nvalid == C;
#pragma unroll
  for (int k = 0; k < Q_::NI_V; ++k) {
    const int it = tid + k * NT;
    const int r = it / (BV / 8), seg = it % (BV / 8);
    const unsigned rr = full ? r : (r < nvalid ? r : nvalid - 1);
    load_raw<F32>(vb, rr * vsl + seg * 8u, pf.v[k]);
  }
#pragma unroll
  for (int k = 0; k < Q_::NI_KQ; ++k) {
    constexpr int PER = C * Q_::SEGS;
    const int which = (k * NT) / PER;  // 0 = k, 1 = q (folded when unrolled)
    const int rem = (k * NT) % PER + tid;
    const int r = rem / Q_::SEGS, seg = rem % Q_::SEGS;
    const unsigned rr = full ? r : (r < nvalid ? r : nvalid - 1);
    if (which == 0) load_raw<F32>(kb, rr * ksl + seg * 8u, pf.kq[k]);
    else load_raw<F32>(qb, rr * qsl + seg * 8u, pf.kq[k]);
  }
}

// Swizzled layouts of the direct-loaded rows.  A K or Q row (dk = 128) is 16
// segments of 8 bf16; logical segment g of row r sits at physical segment
// g ^ swz_k(r).  swz_k is a bijection on 0..15, so the 16 rows of a 16-byte MFMA
// fragment read hit 16 different segments (all 64 banks), and swz_k(r) >> 1 is
// distinct over rows 0..7 and over rows 8..15, the rows one pass of the transposed
// 8-byte read (4 consecutive rows per 16 lanes) covers, so its 8 rows x 32 bytes
// also spread over all banks.  A V row of a 64-column block is 8 segments; swz_v(r) = r & 6
// makes the 8 rows x 32 bytes of a transposed read pass conflict-free the same way.  Rows
// of narrower blocks (SV = 4 or 2 segments) keep the bits of r & 6 that index a segment.
__device__ __forceinline__ int swz_k(int r) { return ((r & 7) << 1) | ((r >> 3) & 1); }
template <int SV>
__device__ __forceinline__ int swz_v(int r) { return r & 6 & (SV - 1); }

// element offset of (row, col) in a swizzled buffer with 8-element segments: K / Q rows
// (128 elements) or V rows (ROWLEN = the block's columns)
template <int ROWLEN>
__device__ __forceinline__ int swz_off(int row, int col) {
  const int g = col >> 3;
  const int sw = ROWLEN == 128 ? swz_k(row & 15) : swz_v<ROWLEN / 8>(row);
  return row * ROWLEN + ((g ^ sw) << 3) + (col & 7);
}

// 16x32 MFMA fragment (rows row0 + lane%16, elements k0 + 8 (lane/16) .. +7)
__device__ __forceinline__ u32x4 swz_frag(const bf16_t* base, int row0, int k0) {
  const int l = lane_id();
  return *(const u32x4*)(base + swz_off<128>(row0 + (l & 15), k0 + 8 * (l >> 4)));
}
// four consecutive rows row0 + 4q .. +3 of column col0 + r of a K buffer (as rows4_tr)
__device__ __forceinline__ u32x2 swz_rows4_k(const bf16_t* base, int row0, int col0) {
  const int l = lane_id(), q = l >> 4, s = l & 15;
  return ds_read_tr(base + swz_off<128>(row0 + 4 * q + (s >> 2), col0 + 4 * (s & 3)));
}
// four consecutive rows row0 + 4q .. +3 of column col0 + r of a V buffer (as rows4_tr)
template <int BV>
__device__ __forceinline__ u32x2 swz_rows4_v(const bf16_t* base, int row0, int col0) {
  const int l = lane_id(), q = l >> 4, s = l & 15;
  return ds_read_tr(base + swz_off<BV>(row0 + 4 * q + (s >> 2), col0 + 4 * (s & 3)));
}

// The state's row order: row r of state tile t is dk index
//   32 (t / 2) + 8 (r / 4) + 4 (t % 2) + r % 4,
// so that tiles 2 s2 and 2 s2 + 1 side by side are the 16x16x32 B operand over dk
// 32 s2 .. 32 s2 + 31 in natural order.  kt_rows4* read, for the state update, the
// A operand rows of tile t transposed out of a [token][dk] buffer: lane (q, r) gets
// tokens row0 + 4q .. +3 of dk column (row r of tile t); source lane s of each
// 16-lane group points at token row0 + 4q + s/4 and the 4 columns of row group s%4.
__device__ __forceinline__ int kt_col(int t, int s) { return 32 * (t >> 1) + 4 * (t & 1) + 8 * (s & 3); }
__device__ __forceinline__ u32x2 kt_rows4_swz(const bf16_t* base, int row0, int t) {
  const int l = lane_id(), q = l >> 4, s = l & 15;
  return ds_read_tr(base + swz_off<128>(row0 + 4 * q + (s >> 2), kt_col(t, s)));
}
__device__ __forceinline__ u32x2 kt_rows4(const bf16_t* base, int ld, int row0, int t) {
  const int l = lane_id(), q = l >> 4, s = l & 15;
  return ds_read_tr(base + (row0 + 4 * q + (s >> 2)) * ld + kt_col(t, s));
}
// dk index of element v of lane group q in state tile t
__device__ __forceinline__ int state_row(int t, int q, int v) { return 32 * (t >> 1) + 8 * q + 4 * (t & 1) + v; }

__device__ __forceinline__ u32x4 join(u32x2 a, u32x2 b) { return u32x4{a[0], a[1], b[0], b[1]}; }


// Issue one chunk's loads straight into an LDS buffer (global_load_lds_dwordx4: lane i
// of an instruction writes 16 bytes at the buffer offset + 16 i), all from the loader
// wavefront: 16 instructions each of K and Q rows, BV / 8 of V rows and one per KiB of
// the record.  Rows past the sequence end repeat the last valid row: every product they
// enter is multiplied by their zero beta, so they need no clearing.  Addresses are a
// uniform base plus a 32-bit lane byte offset (scalar-base loads).
typedef __attribute__((address_space(3))) void lds_void;
typedef __attribute__((address_space(3))) bf16_t lds_bf16;
typedef __attribute__((address_space(3))) unsigned char lds_u8;

// The buffers are passed as LDS-space pointers (cast where the __shared__ arrays are
// named), so no generic-to-LDS conversion happens here.
template <int DK, int MODE, int BV, bool BWD>
__device__ __forceinline__ void stage_all(const ChunkParams& p, long long t0, int nvalid,
                                          const unsigned char* rec, int hk, int h, int col0,
                                          lds_bf16* sK, lds_bf16* sQ, lds_bf16* sV, lds_u8* sRec) {
  typedef __attribute__((address_space(1))) void glob_void;
  constexpr int NRP = rec_bytes(MODE) / 1024, NRPX = rec_bytes(MODE, BWD) / 1024;
  constexpr bool VCONV = MODE == MODE_LAYER && layer_v_in_scan(DK);  // V rows: helper wavefronts
  // V rows: SV 16-byte segments per row, 64 / SV rows per instruction, SV instructions
  constexpr int SV = BV / 8, RPI = 64 / SV;
  const int l = lane_id();
  const bf16_t* kb = (const bf16_t*)p.ks + t0 * p.ks_ld + (long long)hk * DK;
  const bf16_t* qb = (const bf16_t*)p.qs + t0 * p.qs_ld + (long long)hk * DK;
  const bf16_t* vb = (const bf16_t*)p.vs + t0 * p.vs_ld + (long long)h * p.DV + col0;
  const unsigned kld = (unsigned)p.ks_ld, qld = (unsigned)p.qs_ld, vld = (unsigned)p.vs_ld;
  if (nvalid == C) {
    // K/Q instruction mi covers rows 4 mi + l/16, whose swizzle repeats every 4
    // instructions, and V instruction mi rows RPI mi + l/SV, whose swizzle does not depend
    // on mi: a few lane offsets plus uniform row steps
#pragma unroll
    for (int m0 = 0; m0 < 4; ++m0) {
      const unsigned row = 4u * m0 + (unsigned)(l >> 4);
      const unsigned g = (unsigned)((l & 15) ^ swz_k((int)row));
      const unsigned ko = 2u * (row * kld + 8u * g), qo = 2u * (row * qld + 8u * g);
#pragma unroll
      for (int mi = m0; mi < 16; mi += 4) {
        __builtin_amdgcn_global_load_lds((glob_void*)at_bytes(kb + (long long)(4 * (mi - m0)) * p.ks_ld, ko),
                                         (lds_void*)(sK + 512 * mi), 16, 0, 0);
        __builtin_amdgcn_global_load_lds((glob_void*)at_bytes(qb + (long long)(4 * (mi - m0)) * p.qs_ld, qo),
                                         (lds_void*)(sQ + 512 * mi), 16, 0, 0);
      }
    }
    if constexpr (!VCONV) {
      const unsigned vrow = (unsigned)(l / SV);
      const unsigned vo = 2u * (vrow * vld + 8u * (unsigned)((l % SV) ^ swz_v<SV>((int)vrow)));
#pragma unroll
      for (int mi = 0; mi < SV; ++mi)
        __builtin_amdgcn_global_load_lds((glob_void*)at_bytes(vb + (long long)(RPI * mi) * p.vs_ld, vo),
                                         (lds_void*)(sV + 512 * mi), 16, 0, 0);
    }
  } else {
    // a sequence's last, partial chunk: rows past its end repeat the last valid row
#pragma unroll
    for (int mi = 0; mi < 16; ++mi) {
      const int row = 4 * mi + (l >> 4);
      const unsigned rr = (unsigned)(row < nvalid ? row : nvalid - 1);
      const unsigned g = (unsigned)((l & 15) ^ swz_k(row & 15));
      __builtin_amdgcn_global_load_lds((glob_void*)at_bytes(kb, 2u * (rr * kld + 8u * g)),
                                       (lds_void*)(sK + 512 * mi), 16, 0, 0);
      __builtin_amdgcn_global_load_lds((glob_void*)at_bytes(qb, 2u * (rr * qld + 8u * g)),
                                       (lds_void*)(sQ + 512 * mi), 16, 0, 0);
    }
    if constexpr (!VCONV) {
#pragma unroll
      for (int mi = 0; mi < SV; ++mi) {
        const int row = RPI * mi + l / SV;
        const unsigned rr = (unsigned)(row < nvalid ? row : nvalid - 1);
        const unsigned g = (unsigned)((l % SV) ^ swz_v<SV>(row));
        __builtin_amdgcn_global_load_lds((glob_void*)at_bytes(vb, 2u * (rr * vld + 8u * g)),
                                         (lds_void*)(sV + 512 * mi), 16, 0, 0);
      }
    }
  }
#pragma unroll
  for (int mi = 0; mi < NRP; ++mi)
    __builtin_amdgcn_global_load_lds((glob_void*)(rec + 1024 * mi + 16 * l),
                                     (lds_void*)(sRec + 1024 * mi), 16, 0, 0);
  // (backward) P's lo parts, read where o is formed
  if constexpr (NRPX > NRP) {
    if (p.o) {
#pragma unroll
      for (int mi = NRP; mi < NRPX; ++mi)
        __builtin_amdgcn_global_load_lds((glob_void*)(rec + 1024 * mi + 16 * l),
                                         (lds_void*)(sRec + 1024 * mi), 16, 0, 0);
    }
  }
}

// Register staging of the bf16 path's two loaders (stage_all's addresses: lane l of
// piece mi holds the 16 bytes stage_all's instruction mi puts at the buffer offset +
// 16 l).  A chunk's pieces are loaded two chunk steps before the step that reads them and
// stored into their LDS buffer one step before it, so its loads have about two steps to
// land; split over two wavefronts, neither holds more than 132 VGPRs of rows.
struct KQRegs {
  u32x4 k[16], q[16];
};
template <int DK>
__device__ __forceinline__ void stage_kq(const ChunkParams& p, long long t0, int nvalid, int hk, KQRegs& r) {
  const int l = lane_id();
  const bf16_t* kb = (const bf16_t*)p.ks + t0 * p.ks_ld + (long long)hk * DK;
  const bf16_t* qb = (const bf16_t*)p.qs + t0 * p.qs_ld + (long long)hk * DK;
  const unsigned kld = (unsigned)p.ks_ld, qld = (unsigned)p.qs_ld;
  // rows past the sequence end repeat the last valid row, as in stage_all
#pragma unroll
  for (int mi = 0; mi < 16; ++mi) {
    const int row = 4 * mi + (l >> 4);
    const unsigned rr = (unsigned)(row < nvalid ? row : nvalid - 1);
    const unsigned g = (unsigned)((l & 15) ^ swz_k(row & 15));
    r.k[mi] = *(const u32x4*)at_bytes(kb, 2u * (rr * kld + 8u * g));
    r.q[mi] = *(const u32x4*)at_bytes(qb, 2u * (rr * qld + 8u * g));
  }
}
__device__ __forceinline__ void put_kq(const KQRegs& r, lds_bf16* sK, lds_bf16* sQ) {
  typedef __attribute__((address_space(3))) u32x4 lds_u32x4;
  const int l = lane_id();
#pragma unroll
  for (int mi = 0; mi < 16; ++mi) {
    *(lds_u32x4*)(sK + 512 * mi + 8 * l) = r.k[mi];
    *(lds_u32x4*)(sQ + 512 * mi + 8 * l) = r.q[mi];
  }
}
static_assert(kRecP % 1024 == 0 && kRecG % 1024 == 0, "P fills whole 1 KiB record pieces");
template <int MODE, int BV, bool BWD>
struct VRRegs {
  static constexpr int NV = BV / 8, NR = rec_bytes(MODE) / 1024, NRX = rec_bytes(MODE, BWD) / 1024;
  u32x4 v[NV], r[NRX];
};
template <int MODE, int BV, bool BWD>
__device__ __forceinline__ void stage_vr(const ChunkParams& p, long long t0, int nvalid,
                                         const unsigned char* rec, int h, int col0,
                                         VRRegs<MODE, BV, BWD>& r) {
  using R_ = VRRegs<MODE, BV, BWD>;
  constexpr int SV = BV / 8, RPI = 64 / SV;
  const int l = lane_id();
  const bf16_t* vb = (const bf16_t*)p.vs + t0 * p.vs_ld + (long long)h * p.DV + col0;
  const unsigned vld = (unsigned)p.vs_ld;
#pragma unroll
  for (int mi = 0; mi < SV; ++mi) {
    const int row = RPI * mi + l / SV;
    const unsigned rr = (unsigned)(row < nvalid ? row : nvalid - 1);
    const unsigned g = (unsigned)((l % SV) ^ swz_v<SV>(row));
    r.v[mi] = *(const u32x4*)at_bytes(vb, 2u * (rr * vld + 8u * g));
  }
  // P (hi parts) only where o is formed: the prep leaves it out of a recompute without o
  const bool with_p = !BWD || p.o;
#pragma unroll
  for (int mi = 0; mi < R_::NR; ++mi)
    if (with_p || mi < kRecP / 1024 || mi >= kRecG / 1024) r.r[mi] = *(const u32x4*)(rec + 1024 * mi + 16 * l);
  // (backward) P's lo parts, read where o is formed
  if constexpr (R_::NRX > R_::NR) {
    if (p.o) {
#pragma unroll
      for (int mi = R_::NR; mi < R_::NRX; ++mi) r.r[mi] = *(const u32x4*)(rec + 1024 * mi + 16 * l);
    }
  }
}
template <int MODE, int BV, bool BWD>
__device__ __forceinline__ void put_vr(const ChunkParams& p, const VRRegs<MODE, BV, BWD>& r, lds_bf16* sV,
                                       lds_u8* sRec) {
  using R_ = VRRegs<MODE, BV, BWD>;
  typedef __attribute__((address_space(3))) u32x4 lds_u32x4;
  const int l = lane_id();
#pragma unroll
  for (int mi = 0; mi < R_::NV; ++mi) *(lds_u32x4*)(sV + 512 * mi + 8 * l) = r.v[mi];
  const bool with_p = !BWD || p.o;
#pragma unroll
  for (int mi = 0; mi < R_::NR; ++mi)
    if (with_p || mi < kRecP / 1024 || mi >= kRecG / 1024) *(lds_u32x4*)(sRec + 1024 * mi + 16 * l) = r.r[mi];
  if constexpr (R_::NRX > R_::NR) {
    if (p.o) {
#pragma unroll
      for (int mi = R_::NR; mi < R_::NRX; ++mi) *(lds_u32x4*)(sRec + 1024 * mi + 16 * l) = r.r[mi];
    }
  }
}

// BWD (the backward pass's recompute): stores the state entering every chunk and V_new,
// and o only when p.o is set.
//
// FUSE (layer, direct loads, a grid the chip holds in one round): the gated RMSNorm
// (deltanet.py:282-293) is applied here and the scan writes the layer's output.  A row of
// o spans the nb workgroups of a value head (its column blocks), so its statistic needs
// their partial sums: each workgroup's loader publishes its rows' partial (the fp32 o's
// sum of squares over the block) for chunk c one step after the chunk, written through
// to memory (system scope) with a flag raised behind it, and one step later reads every
// block's partial (L2 bypassed), sums them in slot order with the pairwise tree the
// epilogue kernel uses and leaves 1/RMS per row in LDS.  Meanwhile the compute
// wavefronts keep their bf16 o rows in a four-chunk LDS ring and, three steps after the
// chunk, normalise and gate them: w (o rsqrt(mean + eps)) silu(z), the epilogue kernel's
// arithmetic, so the output is bit-identical to the unfused path's.  Every workgroup of
// the grid is resident at once, so a wait for another block's flag ends; it is bounded
// all the same.
template <int DK, int MODE, bool BWD = false, int NWC_ = 4, bool FUSE = false>
// One workgroup per CU is the design point (the state fills the register file): the
// compiler may use the whole file (half of it with a loader wavefront, which shares a
// SIMD) instead of holding back for a second workgroup.
__global__ __launch_bounds__((Cfg<DK, MODE, NWC_, BWD>::NTH)) __attribute__((amdgpu_waves_per_eu(Cfg<DK, MODE, NWC_, BWD>::WPE, Cfg<DK, MODE, NWC_, BWD>::WPE))) void scan_kernel(ChunkParams p) {
  using Q_ = Cfg<DK, MODE, NWC_, BWD>;
  constexpr int NWC = Q_::NWC, BV = Q_::BV, NT = Q_::NT;
  constexpr int LDK = Q_::LDK, SEGS = Q_::SEGS;
  constexpr bool IS = Q_::IS, OS = Q_::OS;
  constexpr bool F32 = MODE == MODE_F32;
  // Each buffer is its own __shared__ object, so the compiler can tell their
  // accesses apart and overlap loads of one with stores to another.
  constexpr bool DIRECT = Q_::DIRECT;
  // Buffer 0 and, with direct loads, buffer 1 are separate objects, and the chunk loop
  // below is unrolled by two so that every access names its buffer statically: the
  // compiler can then tell that the next chunk's loads into one buffer do not touch
  // the other, and does not wait for them before this chunk's LDS reads.
  __shared__ __align__(16) bf16_t sK0[Q_::SZK], sK1[DIRECT ? Q_::SZK : 8];
  __shared__ __align__(16) bf16_t sQ0[Q_::SZK], sQ1[DIRECT ? Q_::SZK : 8];
  __shared__ __align__(16) bf16_t sV0[Q_::SZV], sV1[DIRECT ? Q_::SZV : 8];
  __shared__ __align__(16) unsigned char sRec0[Q_::REC], sRec1[DIRECT ? Q_::REC : 16];
  // (layer, direct loads) the compute wavefronts' row sums of o^2, by chunk parity: chunk
  // j's are written after the barrier that opens chunk j + 1 (so no wavefront waits for
  // the write before a barrier); the loader adds them up after the barrier of chunk j + 2
  constexpr bool WG_SS = DIRECT && MODE == MODE_LAYER;
  __shared__ float sSS[WG_SS ? 2 : 1][WG_SS ? NWC : 1][C];
  float ss_prev = 0.f;  // this lane's row sum of the previous chunk, not yet in sSS
  static_assert(!FUSE || WG_SS, "the fused norm runs on the layer's direct-load scan");
  constexpr int kRing = 4;  // (FUSE) chunks of bf16 o kept per compute wavefront
  constexpr int kFin = 3;   // (FUSE) steps from a chunk to its normalisation
  // (FUSE) lane l's 4 x 4 bf16 o values of row block i of chunk c, wave w: sO[c % 4][w][i][l]
  __shared__ __align__(16) u32x2 sO[FUSE ? kRing : 1][FUSE ? NWC : 1][FUSE ? 4 : 1][64];
  __shared__ float sRN[FUSE ? 2 : 1][C];  // (FUSE) 1/RMS of each row of a chunk
  constexpr int K_LO = C * LDK, V_LO = C * LDT;

  const int tid = threadIdx.x, l = tid & 63, lq = l >> 4, lr = l & 15;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const bool loader = DIRECT && wave >= NWC && wave < NWC + Q_::NL;  // loads, computes nothing
  const bool helper = Q_::VCONV && wave >= NWC + Q_::NL;  // forms the V rows (layer, direct loads)
  const bool compute = wave < NWC;             // owns 16 state columns
  // XCD-aware work item (scan_item): a key head's workgroups share one XCD's L2, and
  // packed sequences start longest first
  const ScanItem item = scan_item(p.seq_order, p.N, p.Hk, p.Hv, p.nb);
  const int blk = item.blk, h = item.h, n = item.n;
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

  // state slice S[dk][16w + (0..15)] in MFMA C layout, rows in the state's row order:
  // S[t][v] = S[state_row(t, lq, v)][16w + lr]
  f32x4 S[DK / 16];
  const size_t state_off = ((size_t)n * p.Hv + h) * DK * DV + col0 + 16 * wave + lr;
  if (p.initial_state && compute) {
#pragma unroll
    for (int t = 0; t < DK / 16; ++t)
#pragma unroll
      for (int v = 0; v < 4; ++v)
        S[t][v] = p.initial_state[state_off + (size_t)state_row(t, lq, v) * DV];
  } else {
#pragma unroll
    for (int t = 0; t < DK / 16; ++t) S[t] = zero4();
  }


  // output addressing: row stride and the lane's constant offset within a chunk
  const int o_rs = p.Hv * DV;  // row stride of o
  // unsigned: a uniform 64-bit base plus a zero-extended 32-bit lane offset is one
  // scalar-base memory instruction with no per-lane 64-bit address arithmetic
  // (output tiles are transposed: lane (q, r) holds row r, columns 16w + 4q .. +3)
  const unsigned o_elem = (unsigned)lr * o_rs + 16u * wave + 4u * lq;
  const unsigned o_lane = 4u * o_elem, o_lane_h = 2u * o_elem;  // bytes: fp32 o, bf16 o

  Prefetch<DK, MODE, BWD> pf;
  if (nchunks > 0) {
    const int nv0 = (int)((s1 - s0) < C ? (s1 - s0) : C);
    if constexpr (DIRECT) {
      if (loader && wave == NWC) {
        stage_all<DK, MODE, BV, BWD>(p, s0, nv0, rec_of(0), hk, h, col0, (lds_bf16*)sK0, (lds_bf16*)sQ0,
                            (lds_bf16*)sV0, (lds_u8*)sRec0);
        __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0): landed before the first barrier
      }
    } else {
      prefetch<DK, MODE, BWD>(p, pf, s0, nv0, rec_of(0), hk, h, col0);
    }
  }

  // (FUSE) the normalisation of chunk c's rows on the compute wavefronts: o from the LDS
  // ring, 1/RMS of each row from sRN (left there by the loader), z loaded at the start of
  // the step; out = w (o rn) silu(z), stored through a buffer whose range ends at the
  // chunk's last valid row.  The row offsets are in the lane offsets, which the range
  // check covers (a scalar offset is not relied on to be checked).  c < 0 does nothing.
  u32x2 zf[4];
  const float4 nw4 = FUSE ? *(const float4*)(p.norm_w + col0 + 16 * wave + 4 * lq)
                          : make_float4(0.f, 0.f, 0.f, 0.f);
  auto chunk_rows = [&](int c, long long& tc) {
    tc = s0 + (long long)c * C;
    return (int)((s1 - tc) < C ? (s1 - tc) : C);
  };
  auto z_load = [&](int c) {
    if constexpr (FUSE) {
      if (c < 0) return;  // uniform
      long long tc;
      const int nvc = chunk_rows(c, tc);
      const auto zr = buf_rsrc((const bf16_t*)p.z + (tc * p.Hv + h) * (long long)DV + col0,
                               2u * nvc * o_rs);
#pragma unroll
      for (int i = 0; i < 4; ++i)
        zf[i] = __builtin_amdgcn_raw_buffer_load_b64(zr, o_lane_h + 2u * 16u * i * o_rs, 0, 0);
    }
  };
  auto finalize = [&](int c) {
    if constexpr (FUSE) {
      if (c < 0) return;  // uniform
      long long tc;
      const int nvc = chunk_rows(c, tc);
      const auto orr = buf_rsrc((bf16_t*)p.out + (tc * p.Hv + h) * (long long)DV + col0,
                                2u * nvc * o_rs);
      const float w[4] = {nw4.x, nw4.y, nw4.z, nw4.w};
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const u32x2 ow = sO[c % kRing][wave][i][l];
        const float rn = sRN[c & 1][16 * i + lr];
        uint32_t r[2];
#pragma unroll
        for (int e = 0; e < 2; ++e) {
          const float o0 = __uint_as_float(ow[e] << 16), o1 = __uint_as_float(ow[e] & 0xffff0000u);
          const float z0 = __uint_as_float(zf[i][e] << 16), z1 = __uint_as_float(zf[i][e] & 0xffff0000u);
          r[e] = pack_bf16(w[2 * e] * (o0 * rn) * silu_fast(z0), w[2 * e + 1] * (o1 * rn) * silu_fast(z1));
        }
        __builtin_amdgcn_raw_buffer_store_b64(u32x2{r[0], r[1]}, orr, o_lane_h + 2u * 16u * i * o_rs, 0, 0);
      }
    }
  };

  // one chunk on the compute wavefronts, from buffer (sK, sQ, sV, sRec)
  auto run_chunk = [&](const int j, bf16_t* sK, bf16_t* sQ, bf16_t* sV, unsigned char* sRec) {
    const long long t0 = s0 + (long long)j * C;
    const int nvalid = (int)((s1 - t0) < C ? (s1 - t0) : C);
    const float* sGate = (const float*)(sRec + kRecG);
    const float* sEG = sGate + kGateEG * C;    // e^G
    const float* sEGS = sGate + kGateEGS * C;  // scale e^G
    const float* sEL = sGate + kGateEL * C;    // e^{G_last - G}; e^{G_last} at C - 1
    if constexpr (DIRECT) {
      // the loader's loads of chunk j have landed (it waited before arriving), and
      // chunk j-1, the last reader of the other buffer, is finished everywhere
      lds_barrier();
      if constexpr (WG_SS && !FUSE) {
        if (j >= 1) sSS[(j - 1) & 1][wave][16 * lq + lr] = ss_prev;
      }
      // (FUSE) z of the chunk normalised at the end of this step, in flight meanwhile
      if constexpr (FUSE) z_load(j - kFin);
    } else {
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
    const int nrec16 = BWD && !p.o ? Q_::NREC16_NO_O : Q_::NREC16;
#pragma unroll
    for (int k = 0; k < Q_::NI_R; ++k) {
      const int it = tid + k * NT;
      if (it < nrec16) ((u32x4*)sRec)[it] = pf.rec[k];
    }
    __syncthreads();

    // issue the next chunk's loads; they land during the rest of this chunk
    if (j + 1 < nchunks) {
      const long long tn = t0 + C;
      prefetch<DK, MODE, BWD>(p, pf, tn, (int)((s1 - tn) < C ? (s1 - tn) : C), rec_of(j + 1), hk, h,
                         col0);
    }
    }

    if constexpr (BWD) {
      // the state entering chunk j, for the backward pass
      const int slot = cbase + j < p.n_rec ? cbase + j : p.n_rec - 1;
      // column-major per state ([dv][dk]): a lane's 4 rows of a tile are contiguous
      float* sd = p.states + ((size_t)slot * p.Hv + h) * DK * DV + (size_t)(col0 + 16 * wave + lr) * DK;
#pragma unroll
      for (int t = 0; t < DK / 16; ++t) *(f32x4*)(sd + state_row(t, lq, 0)) = S[t];
    }
    // ------------------------------------------------------------ K S, Q S, right-hand side
    // The B operand of K S and Q S over dk block s2 is the state itself: lane (q, r)
    // holds tiles 2 s2 and 2 s2 + 1, dk 32 s2 + 8q + (0..7) of column r (the state's
    // row order), packed to bf16 straight from the accumulators.  Every operand that
    // does not depend on S is read from LDS in one batch while the state update of
    // the previous chunk drains.
    constexpr int NSK = DK / 32;
    // On the direct-load path Q S is formed after the state update: it is off the chain
    // K S -> R -> T R -> S, and deferring its fragment reads halves the LDS traffic the
    // chunk's first products wait for.
    constexpr bool DEFER_QS = DIRECT && !IS;
    u32x4 kh[4][NSK], kl[4][NSK], qh[4][NSK], ql[4][NSK];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int s2 = 0; s2 < NSK; ++s2) {
        if constexpr (DIRECT) {
          kh[i][s2] = kl[i][s2] = swz_frag(sK, 16 * i, 32 * s2);
          if constexpr (!DEFER_QS) qh[i][s2] = ql[i][s2] = swz_frag(sQ, 16 * i, 32 * s2);
        } else {
          frag2<IS>(sK, K_LO, LDK, 16 * i, 32 * s2, kh[i][s2], kl[i][s2]);
          frag2<IS>(sQ, K_LO, LDK, 16 * i, 32 * s2, qh[i][s2], ql[i][s2]);
        }
      }
    float vv[4][4];  // V at rows 16i + 4lq + v, column 16w + lr
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const u32x2 vw = DIRECT ? swz_rows4_v<BV>(sV, 16 * i, 16 * wave) : rows4_tr(sV, LDT, 16 * i, 16 * wave);
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
    u32x4 sh[NSK], sl[NSK];
#pragma unroll
    for (int s2 = 0; s2 < NSK; ++s2) {
      sh[s2] = join(pack_hi4(S[2 * s2]), pack_hi4(S[2 * s2 + 1]));
      // (backward) the lo half also enters Q S, for the o that the norm's adjoint reads
      if constexpr (IS || BWD) sl[s2] = join(pack_lo4(S[2 * s2]), pack_lo4(S[2 * s2 + 1]));
      else sl[s2] = sh[s2];
    }
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
        if constexpr (!DEFER_QS) QS[i] = mm<IS, IS>(QS[i], sh[s2], sl[s2], qh[i][s2], ql[i][s2]);  // (Q S)^T
        if constexpr (BWD && !IS && !DEFER_QS)
          if (p.o) QS[i] = mma16(sl[s2], qh[i][s2], QS[i]);
      }
    if constexpr (DIRECT && !IS) {
      // all fragment reads go out back to back, then the state packs, then the
      // products: one LDS round trip for the phase instead of one per few products
      __builtin_amdgcn_sched_group_barrier(0x100, 4 * NSK + 4, 0);
      __builtin_amdgcn_sched_group_barrier(0x002, 4 * NSK, 0);
      __builtin_amdgcn_sched_group_barrier(0x008, 4 * NSK, 0);
    }
    // T operands of V_new = T R, one per block pair (read while the products run)
    u32x4 th[kNPairs], tl[kNPairs];
#pragma unroll
    for (int x = 0; x < kNPairs; ++x) {
      const unsigned char* tp = sRec + kRecT + 2 * x * kPairBytes + 16 * l;
      th[x] = *(const u32x4*)tp;
      tl[x] = *(const u32x4*)(tp + kPairBytes);
    }
    // R = V - diag(e^G) K S at rows 16i + 4lq + v, column 16w + lr (diag(beta) is
    // folded into the record's T)
    f32x4 R[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float4 eg = *(const float4*)(sEG + 16 * i + 4 * lq);
      R[i][0] = vv[i][0] - eg.x * KS[i][0];
      R[i][1] = vv[i][1] - eg.y * KS[i][1];
      R[i][2] = vv[i][2] - eg.z * KS[i][2];
      R[i][3] = vv[i][3] - eg.w * KS[i][3];
    }

    // ------------------------------------------------------------ V_new = T diag(beta) R
    // Two C-layout tiles of R (token blocks 2p, 2p+1) side by side are the B operand
    // of a 16x16x32 MFMA over that block pair, in the contraction order of the
    // record's T pairs.  hi*hi, hi*lo and lo*hi accumulate in one chain per row block.
    u32x4 Rh[2], Rl[2];
#pragma unroll
    for (int pp = 0; pp < 2; ++pp) {
      Rh[pp] = join(pack_hi4(R[2 * pp]), pack_hi4(R[2 * pp + 1]));
      Rl[pp] = join(pack_lo4(R[2 * pp]), pack_lo4(R[2 * pp + 1]));
    }
    f32x4 U[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      f32x4 a = zero4();
#pragma unroll
      for (int pp = 0; pp <= i / 2; ++pp) {
        const int x = pair_index(i, pp);
        a = mma16(th[x], Rh[pp], a);
        a = mma16(th[x], Rl[pp], a);
        a = mma16(tl[x], Rh[pp], a);
      }
      U[i] = a;
    }
    if constexpr (DIRECT && !IS) {
      // the T operands and gate rows are read in one batch ahead of the products
      __builtin_amdgcn_sched_group_barrier(0x100, 2 * kNPairs + 8, 1);
      __builtin_amdgcn_sched_group_barrier(0x002, 80, 1);
      __builtin_amdgcn_sched_group_barrier(0x008, 18, 1);
    }
    if constexpr (BWD) {
      // V_new for the backward pass, formed transposed (V_new^T = R^T (T diag(beta))^T:
      // the packed R serves as A operand and the record's T fragments as B operands), so
      // a lane holds 4 consecutive columns of one token row: one 16-byte store per row block
      float* vd = p.vnew + ((size_t)t0 * p.Hv + h) * DV + col0 + 16 * wave + 4 * lq;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        f32x4 ut = zero4();
#pragma unroll
        for (int pp = 0; pp <= i / 2; ++pp) {
          const int x = pair_index(i, pp);
          ut = mma16(Rh[pp], th[x], ut);
          ut = mma16(Rl[pp], th[x], ut);
          ut = mma16(Rh[pp], tl[x], ut);
        }
        if (16 * i + lr < nvalid) *(f32x4*)(vd + (size_t)(16 * i + lr) * p.Hv * DV) = ut;
      }
    }
    u32x4 Uh[2], Ul[2];  // bf16 hi/lo of V_new block pairs as B operands
#pragma unroll
    for (int pp = 0; pp < 2; ++pp) {
      Uh[pp] = join(pack_hi4(U[2 * pp]), pack_hi4(U[2 * pp + 1]));
      if constexpr (OS || BWD) Ul[pp] = join(pack_lo4(U[2 * pp]), pack_lo4(U[2 * pp + 1]));
    }
    // P operands and the K^T operands of the state update (read while V_new forms)
    u32x4 ph[kNPairs], pl[kNPairs];
#pragma unroll
    for (int x = 0; x < kNPairs; ++x) {
      ph[x] = *(const u32x4*)(sRec + kRecP + x * kPairBytes + 16 * l);
      if constexpr (OS) pl[x] = *(const u32x4*)(sRec + kRecPL + x * kPairBytes + 16 * l);
      else pl[x] = ph[x];
    }
    // K^T operands of the state update, 16x32 over token blocks 2p, 2p+1: lane (q, r)
    // holds K[32p + 4q .. +3][d] then K[32p + 16 + 4q .. +3][d] for the dk index d of
    // row r of state tile t (dk 32 (t/2) + 8 (r/4) + 4 (t%2) + r%4)
    u32x4 kth[DK / 16][2], ktl[DK / 16][2];
#pragma unroll
    for (int t = 0; t < DK / 16; ++t)
#pragma unroll
      for (int pp = 0; pp < 2; ++pp) {
        if constexpr (DIRECT) {
          kth[t][pp] = join(kt_rows4_swz(sK, 32 * pp, t), kt_rows4_swz(sK, 32 * pp + 16, t));
          ktl[t][pp] = kth[t][pp];
        } else {
          kth[t][pp] = join(kt_rows4(sK, LDK, 32 * pp, t), kt_rows4(sK, LDK, 32 * pp + 16, t));
          if constexpr (IS)
            ktl[t][pp] = join(kt_rows4(sK + K_LO, LDK, 32 * pp, t), kt_rows4(sK + K_LO, LDK, 32 * pp + 16, t));
          else ktl[t][pp] = kth[t][pp];
        }
      }
    // Vt = diag(e^{G_last - G}) V_new: its C-layout tiles side by side are the B
    // operands of the state update, so it stays in registers (hi and lo)
    u32x4 vth[2], vtl[2];
#pragma unroll
    for (int pp = 0; pp < 2; ++pp) {
      f32x4 vt[2];
#pragma unroll
      for (int hh = 0; hh < 2; ++hh) {
        const int i = 2 * pp + hh;
        const float4 el = *(const float4*)(sEL + 16 * i + 4 * lq);
        // row C - 1's factor is e^0 = 1; its slot holds e^{G_last}
        const float el3 = (i == 3 && lq == 3) ? 1.f : el.w;
        vt[hh][0] = U[i][0] * el.x; vt[hh][1] = U[i][1] * el.y;
        vt[hh][2] = U[i][2] * el.z; vt[hh][3] = U[i][3] * el3;
      }
      vth[pp] = join(pack_hi4(vt[0]), pack_hi4(vt[1]));
      vtl[pp] = join(pack_lo4(vt[0]), pack_lo4(vt[1]));
    }

    // ------------------------------------------------------------ S <- e^{G_last} S + K^T Vt
    const float gl = sEL[C - 1];  // e^{G_last}
#pragma unroll
    for (int t = 0; t < DK / 16; ++t) {
#pragma unroll
      for (int v = 0; v < 4; ++v) S[t][v] *= gl;
#pragma unroll
      for (int pp = 0; pp < 2; ++pp) {
        S[t] = mma16(kth[t][pp], vth[pp], S[t]);
        S[t] = mma16(kth[t][pp], vtl[pp], S[t]);
        if constexpr (IS) S[t] = mma16(ktl[t][pp], vth[pp], S[t]);
      }
    }

    // ------------------------------------------------------------ O = scale e^G (Q S) + P V_new
    // Computed transposed, O^T = S^T Q^T + V_new^T P^T: the packed state and V_new (B
    // operands above) serve as A operands and the Q and P fragments as B operands, since
    // both operand layouts hold "row r, contraction slots 8q .. 8q+7".  Lane (q, r) then
    // holds token 16i + r, columns 16w + 4q .. +3 of the wave's slice: one 16-byte (fp32)
    // or 8-byte (bf16) store per row block, and one gate factor per lane.
    if constexpr (BWD) {
      if (!p.o) return;  // the layer backward also needs o (for its norm's adjoint)
      // its o comes from split operands throughout (S, V_new and P hi and lo): the adjoint
      // scales by the row's 1 / RMS, which is large where o's terms nearly cancel
      if constexpr (!OS) {
#pragma unroll
        for (int x = 0; x < kNPairs; ++x) pl[x] = *(const u32x4*)(sRec + kRecPL + x * kPairBytes + 16 * l);
      }
    }
    if constexpr (DEFER_QS) {
      // (Q S)^T from the chunk's entering state, still held packed in sh
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int s2 = 0; s2 < NSK; ++s2) qh[i][s2] = swz_frag(sQ, 16 * i, 32 * s2);
#pragma unroll
      for (int s2 = 0; s2 < NSK; ++s2)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          QS[i] = mma16(sh[s2], qh[i][s2], QS[i]);
          if constexpr (BWD) QS[i] = mma16(sl[s2], qh[i][s2], QS[i]);
        }
    }
    f32x4 o[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float eg = sEGS[16 * i + lr];
#pragma unroll
      for (int v = 0; v < 4; ++v) o[i][v] = eg * QS[i][v];
#pragma unroll
      for (int pp = 0; pp <= i / 2; ++pp) {  // P is lower triangular
        const int x = pair_index(i, pp);
        o[i] = mma16(Uh[pp], ph[x], o[i]);
        if constexpr (OS || BWD) {
          o[i] = mma16(Ul[pp], ph[x], o[i]);
          o[i] = mma16(Uh[pp], pl[x], o[i]);
        }
      }
    }
    // row 16i + r of the chunk: a uniform row-block offset plus the lane's constant byte
    // offset; every row of a full chunk is stored (uniform)
    if constexpr (MODE != MODE_LAYER) {
      const auto ob = buf_rsrc(p.o + (t0 * p.Hv + h) * (long long)DV + col0, 4u * C * o_rs);
      auto store = [&](int i) {
        // row offset in the lane offset: a store of more than 64 bits with a register scalar
        // offset is one the compiler lets overwrite its data registers right after issue,
        // which gfx950 does not tolerate
        __builtin_amdgcn_raw_buffer_store_b128(
            u32x4{__float_as_uint(o[i][0]), __float_as_uint(o[i][1]), __float_as_uint(o[i][2]),
                  __float_as_uint(o[i][3])},
            ob, o_lane + 4u * 16u * i * o_rs, 0, 0);
      };
      if (nvalid == C) {
#pragma unroll
        for (int i = 0; i < 4; ++i) store(i);
      } else {
#pragma unroll
        for (int i = 0; i < 4; ++i)
          if (16 * i + lr < nvalid) store(i);
      }
    } else if constexpr (FUSE) {
      // unnormalised o in bf16 into the LDS ring, and the rows' sums of squares of the fp32
      // o into sSS for the loader (after the next barrier); finalize() normalises the chunk
      // kFin steps later
#pragma unroll
      for (int i = 0; i < 4; ++i)
        sO[j % kRing][wave][i][l] = u32x2{pack_bf16(o[i][0], o[i][1]), pack_bf16(o[i][2], o[i][3])};
      sSS[j & 1][wave][16 * lq + lr] = row_sq_scatter(o);
      finalize(j - kFin);
    } else {
      // unnormalised o in bf16; the epilogue kernel applies the norm, from the fp32 sums
      // of squares stored below
      const auto ob = buf_rsrc((bf16_t*)p.o_part + (t0 * p.Hv + h) * (long long)DV + col0, 2u * C * o_rs);
      auto store = [&](int i) {
        __builtin_amdgcn_raw_buffer_store_b64(
            u32x2{pack_bf16(o[i][0], o[i][1]), pack_bf16(o[i][2], o[i][3])}, ob, o_lane_h,
            2 * 16 * i * o_rs, 0);
      };
      if (nvalid == C) {
#pragma unroll
        for (int i = 0; i < 4; ++i) store(i);
      } else {
#pragma unroll
        for (int i = 0; i < 4; ++i)
          if (16 * i + lr < nvalid) store(i);
      }
      // sum of squares of each token row over the wave's 16 columns, from the fp32 o (the
      // statistic of the reference's fp32 norm, deltanet.py:282-293): lane (q, r) ends
      // with row 16q + r's sum (row_sq_scatter).  The partials are stored in 64-token
      // blocks (ss_index), so a chunk's partials of one slot are one contiguous store.
      // With direct loads the loader adds the workgroup's values up first (ss_tree);
      // otherwise each wavefront stores its own.
      const float mine = row_sq_scatter(o);
      if constexpr (WG_SS) {
        ss_prev = mine;
      } else if (16 * lq + lr < nvalid) {
        p.o_ss[ss_index(t0 + 16 * lq + lr, h, col0 / 16 + wave, p.Hv, p.ss_slots)] = mine;
      }
    }
  };

  if constexpr (DIRECT) {
    if (loader && Q_::NL == 2) {
      if constexpr (Q_::NL == 2) {
        // one barrier per chunk, as the compute wavefronts: after the barrier at the top of
        // chunk j, buffer (j + 1) % 2 is free and receives chunk j + 1 from the registers,
        // which then receive chunk j + 2.  The two loaders run separate loops, so neither
        // holds the other's rows.
        auto rows = [&](int c, long long& tc) {
          tc = s0 + (long long)c * C;
          return (int)((s1 - tc) < C ? (s1 - tc) : C);
        };
        if (wave == NWC) {  // the K and Q rows
          KQRegs r;
          long long tc;
          if (nchunks > 1) {
            const int nvc = rows(1, tc);
            stage_kq<DK>(p, tc, nvc, hk, r);
          }
          auto step = [&](int j, lds_bf16* nK, lds_bf16* nQ) {
            lds_barrier();
            if (j + 1 < nchunks) put_kq(r, nK, nQ);
            if (j + 2 < nchunks) {
              const int nvc = rows(j + 2, tc);
              stage_kq<DK>(p, tc, nvc, hk, r);
            }
          };
          for (int j = 0; j < nchunks; j += 2) {
            step(j, (lds_bf16*)sK1, (lds_bf16*)sQ1);
            if (j + 1 < nchunks) step(j + 1, (lds_bf16*)sK0, (lds_bf16*)sQ0);
          }
        } else {  // the V rows and the record
          VRRegs<MODE, BV, BWD> r;
          long long tc;
          if (nchunks > 1) {
            const int nvc = rows(1, tc);
            stage_vr<MODE, BV, BWD>(p, tc, nvc, rec_of(1), h, col0, r);
          }
          auto step = [&](int j, lds_bf16* nV, lds_u8* nRec) {
            lds_barrier();
            if (j + 1 < nchunks) put_vr<MODE, BV, BWD>(p, r, nV, nRec);
            if (j + 2 < nchunks) {
              const int nvc = rows(j + 2, tc);
              stage_vr<MODE, BV, BWD>(p, tc, nvc, rec_of(j + 2), h, col0, r);
            }
          };
          for (int j = 0; j < nchunks; j += 2) {
            step(j, (lds_bf16*)sV1, (lds_u8*)sRec1);
            if (j + 1 < nchunks) step(j + 1, (lds_bf16*)sV0, (lds_u8*)sRec0);
          }
        }
      }
    } else if (loader) {
      // one barrier per chunk, as the compute wavefronts: after the barrier at the top of
      // chunk j, buffer (j + 1) % 2 is free and receives chunk j + 1
      // (layer) lane l's row of chunk jj: the workgroup's partial, one per row, stored
      // after the wait for the next chunk's loads (the following wait covers it)
      auto store_ss = [&](int jj) {
        if constexpr (WG_SS) {
          const long long tj = s0 + (long long)jj * C;
          const int nvj = (int)((s1 - tj) < C ? (s1 - tj) : C);
          float v[NWC];
#pragma unroll
          for (int w = 0; w < NWC; ++w) v[w] = sSS[jj & 1][w][l];
          if (l < nvj) p.o_ss[ss_index(tj + l, h, blk, p.Hv, p.ss_slots)] = ss_tree<NWC>(v);
        }
      };
      // (FUSE) the row partials of chunk c in the exchange array: [slot][h][block][row]
      constexpr int NBX = 256 / BV;  // most column blocks a value head has at this width
      u32x2 xv[FUSE ? NBX : 1];
      int gave_up = 0;  // a bounded wait that ran out stops all later waits
      // ring entry of chunk c of block s: every block has read an entry before any block
      // writes it again, kXchRing chunks later (a block writes chunk c + 4's partial only
      // after it has seen every block's partial of chunk c + 2, which they publish after
      // they have read chunk c's)
      auto xch_rsrc = [&](int c, int s, unsigned bytes) {
        return buf_rsrc(p.ss_xch + 2 * ((((size_t)n * p.Hv + h) * p.ss_xch_slots + s) * kXchRing +
                                        c % kXchRing) * C,
                        bytes);
      };
      // this workgroup's partial of chunk c's row l (its waves' partials, in sSS since the
      // barrier that opened this step), written through to memory with tag c + 1
      auto publish = [&](int c) {
        if constexpr (FUSE) {
          long long tc;
          const int nvc = chunk_rows(c, tc);
          float v[NWC];
#pragma unroll
          for (int w = 0; w < NWC; ++w) v[w] = sSS[c & 1][w][l];
          __builtin_amdgcn_raw_buffer_store_b64(u32x2{__float_as_uint(ss_tree<NWC>(v)), (unsigned)c + 1u},
                                                xch_rsrc(c, blk, 8u * nvc), 8u * l, 0, 17);
        }
      };
      // every block's partial of chunk c's row l, read past the caches (system scope)
      auto gather = [&](int c) {
        if constexpr (FUSE) {
#pragma unroll
          for (int s = 0; s < NBX; ++s)
            if (s < p.nb) xv[s] = __builtin_amdgcn_raw_buffer_load_b64(xch_rsrc(c, s, 8u * C), 8u * l, 0, 17);
        }
      };
      // once every valid row's entries carry chunk c's tag: the row's sum over the blocks in the
      // pairwise order of the epilogue kernel's butterfly, and 1/RMS into sRN
      auto finish = [&](int c) {
        if constexpr (FUSE) {
          long long tc;
          const int nvc = chunk_rows(c, tc);
          auto ready = [&]() {
            bool r = true;
#pragma unroll
            for (int s = 0; s < NBX; ++s)
              if (s < p.nb) r = r && xv[s][1] == (unsigned)c + 1u;
            return l >= nvc || r;
          };
          for (int tries = 0; !gave_up && __ballot(!ready()) != 0ull; ++tries) {
            if (tries == (1 << 20)) {  // about a second: give up rather than hang
              gave_up = 1;
              break;
            }
            __builtin_amdgcn_s_sleep(4);
            gather(c);
            __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0)
          }
          float t[NBX];
#pragma unroll
          for (int s = 0; s < NBX; ++s) t[s] = s < p.nb ? __uint_as_float(xv[s][0]) : 0.f;
#pragma unroll
          for (int w = 1; w < NBX; w <<= 1)
#pragma unroll
            for (int s = 0; s + w < NBX; s += 2 * w) t[s] += t[s + w];
          // as the epilogue kernel; a wait that gave up (a partner block never ran, which a
          // grid the chip holds at once rules out unless other work kept CUs for a second)
          // leaves NaN rows rather than rows normalised by partial sums
          sRN[c & 1][l] = gave_up ? __builtin_nanf("") : rsqrtf(__builtin_fmaf(t[0], p.inv_dv, p.eps));
        }
      };
      auto load = [&](int j, lds_bf16* nK, lds_bf16* nQ, lds_bf16* nV, lds_u8* nRec) {
        lds_barrier();
        if (j + 1 < nchunks) {
          const long long tn = s0 + (long long)(j + 1) * C;
          const int nvn = (int)((s1 - tn) < C ? (s1 - tn) : C);
          stage_all<DK, MODE, BV, BWD>(p, tn, nvn, rec_of(j + 1), hk, h, col0, nK, nQ, nV, nRec);
        }
        if constexpr (FUSE) {
          // chunk j - 1's partial (its waves wrote sSS before this step's barrier), then
          // the partials of chunk j - 2 that every block published a step ago
          if (j >= 1 && j - 1 < nchunks) publish(j - 1);
          if (j >= 2 && j - 2 < nchunks) gather(j - 2);
        }
        __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0): landed before the next barrier
        if constexpr (FUSE) {
          if (j >= 2 && j - 2 < nchunks) finish(j - 2);
        } else {
          if (j >= 2) store_ss(j - 2);  // written after barrier j - 1, visible after barrier j
        }
      };
      for (int j = 0; j < nchunks; j += 2) {
        load(j, (lds_bf16*)sK1, (lds_bf16*)sQ1, (lds_bf16*)sV1, (lds_u8*)sRec1);
        if (j + 1 < nchunks) load(j + 1, (lds_bf16*)sK0, (lds_bf16*)sQ0, (lds_bf16*)sV0, (lds_u8*)sRec0);
      }
      if constexpr (FUSE) {  // the pipeline's drain: kFin more steps (no loads)
        if (nchunks > 0)
          for (int j = nchunks; j < nchunks + kFin; ++j)
            load(j, (lds_bf16*)sK0, (lds_bf16*)sQ0, (lds_bf16*)sV0, (lds_u8*)sRec0);
      } else if constexpr (WG_SS) {  // the last two chunks' row sums, as in the loop
        if (nchunks > 0) {
          lds_barrier();  // chunk n - 2's are visible; the buffer of n - 1's is free
          if (nchunks >= 2) store_ss(nchunks - 2);
          lds_barrier();  // chunk n - 1's are visible
          store_ss(nchunks - 1);
        }
      }
    } else if (helper) {
      if constexpr (Q_::VCONV) {
        // one barrier per chunk, as the loader: after the barrier at the top of chunk j,
        // V buffer (j + 1) % 2 is free and receives chunk j + 1's rows; chunk 0's are
        // formed before the first barrier
        // Conv + SiLU of the value channels chu .. chu + BV - 1 with the prep's arithmetic
        // (gdn_conv.h), stored in the swizzled layout the compute wavefronts read.  Helper
        // lane hl (0 .. 127) forms 8 channels of R = BV / 16 consecutive rows, with its
        // weights loaded once; rows past the sequence end are zero.  A chunk's input rows
        // are loaded one chunk step ahead (two register sets; loads past the last chunk
        // repeat it), so their latency is off the step.
        constexpr int SV = BV / 8, R = BV / 16;
        const int hl = tid - 64 * (NWC + Q_::NL);
        const int g = hl % SV, r0 = (hl / SV) * R;
        const int chu = 2 * p.Hk * DK + h * DV + col0;
        uint32_t wp[8][2];
        load_conv_w(p, chu, 8 * g, wp);
        auto nv_of = [&](int j) {
          const long long tj = s0 + (long long)j * C;
          return (int)((s1 - tj) < C ? (s1 - tj) : C);
        };
        auto load = [&](int j, u32x4* raw) {
          const int jj = j < nchunks ? j : nchunks - 1;
          conv_load<R>(p, n, s0, s0 + (long long)jj * C, nv_of(jj), r0, chu, 8 * g, raw);
        };
        auto form = [&](int j, const u32x4* raw, bf16_t* nV) {
          conv_compute<R>(raw, wp, nv_of(j), r0, [&](int m, const u32x4& y) {
            *(u32x4*)(nV + swz_off<BV>(r0 + m, 8 * g)) = y;
          });
        };
        u32x4 ra[R + 3], rb[R + 3];
        if (nchunks > 0) {
          load(0, ra);
          load(1, rb);
          form(0, ra, sV0);
        }
        for (int j = 0; j < nchunks; j += 2) {
          lds_barrier();
          if (j + 1 < nchunks) {
            load(j + 2, ra);
            form(j + 1, rb, sV1);
            lds_barrier();
            load(j + 3, rb);
            if (j + 2 < nchunks) form(j + 2, ra, sV0);
          }
        }
        if (nchunks > 0) {  // the loader's barriers after its loop
          lds_barrier();
          lds_barrier();
          if constexpr (FUSE) lds_barrier();
        }
      }
    } else {
      for (int j = 0; j < nchunks; j += 2) {
        run_chunk(j, sK0, sQ0, sV0, sRec0);
        if (j + 1 < nchunks) run_chunk(j + 1, sK1, sQ1, sV1, sRec1);
      }
      if constexpr (FUSE) {  // the drain: the last kFin chunks' normalisation
        if (nchunks > 0)
          for (int j = nchunks; j < nchunks + kFin; ++j) {
            lds_barrier();
            z_load(j - kFin);
            finalize(j - kFin);
          }
      } else if constexpr (WG_SS) {  // the loader's two barriers after its loop
        if (nchunks > 0) {
          lds_barrier();
          sSS[(nchunks - 1) & 1][wave][16 * lq + lr] = ss_prev;
          lds_barrier();
        }
      }
    }
  } else {
    for (int j = 0; j < nchunks; ++j) run_chunk(j, sK0, sQ0, sV0, sRec0);
  }

  if (p.final_state && compute) {
#pragma unroll
    for (int t = 0; t < DK / 16; ++t)
#pragma unroll
      for (int v = 0; v < 4; ++v)
        p.final_state[state_off + (size_t)state_row(t, lq, v) * DV] = S[t][v];
  }

  if constexpr (MODE == MODE_LAYER) {
    // conv cache after the prefill: the last K-1 raw inputs of the sequence.  q/k
    // channels are written by the first value head of their key head only.
    if (p.conv_state_out) {
      const int K = p.conv_k;
      const bool own_qk = (h % gqa) == 0 && blk == 0;
      constexpr int HW = 2 * DK + BV;  // q | k | this block's v channels
      for (int it = tid; it < HW * (K - 1); it += Q_::NTH) {
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

// The scan's workgroups cover Cfg::BV columns each; p.nb (the other kernels' 64-column
// blocks) is replaced by the scan's own count in a copy of the parameters.
template <int DK, int MODE, bool BWD = false, int NWC = 4, bool FUSE = false>
hipError_t launch_scan_cfg(const ChunkParams& p, hipStream_t stream) {
  using Q_ = Cfg<DK, MODE, NWC, BWD>;
  ChunkParams q = p;
  q.nb = p.DV / Q_::BV;
  // (layer) row-sum partials per (token, value head): one per workgroup with direct
  // loads, else one per wavefront
  q.ss_slots = Q_::DIRECT ? q.nb : p.DV / 16;
  const unsigned grid = (unsigned)(q.N * q.Hv * q.nb);
  hipLaunchKernelGGL((scan_kernel<DK, MODE, BWD, NWC, FUSE>), dim3(grid), dim3(Q_::NTH), 0, stream, q);
  return hipGetLastError();
}

// Compute units of the current device (queried once per device).
int device_cus() {
  static int cus[64] = {};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  if (cus[dev] == 0) {
    int v = 0;
    if (hipDeviceGetAttribute(&v, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || v <= 0)
      v = 256;
    cus[dev] = v;
  }
  return cus[dev];
}

// Column tiles per workgroup for the direct-load scan: 4 (64 columns) when that gives a
// workgroup per CU, else 2 or 1, the widest that still does.  The workgroups walk their
// sequences' chunks in order, so a grid smaller than the chip leaves CUs idle for the
// whole call; narrower workgroups also leave each CU's LDS to fewer wavefronts.
int scan_tiles_per_wg(const ChunkParams& p) {
  const long long tiles = (long long)p.N * p.Hv * (p.DV / 16);
  const long long cus = device_cus();
  if (tiles >= 4 * cus) return 4;
  if (tiles >= 2 * cus) return 2;
  return 1;
}

template <int DK, int MODE, bool FUSE = false>
hipError_t launch_scan_direct(const ChunkParams& p, hipStream_t stream) {
  switch (scan_tiles_per_wg(p)) {
    case 1: return launch_scan_cfg<DK, MODE, false, 1, FUSE>(p, stream);
    case 2: return launch_scan_cfg<DK, MODE, false, 2, FUSE>(p, stream);
    default: return launch_scan_cfg<DK, MODE, false, 4, FUSE>(p, stream);
  }
}

}  // namespace

int chunk_block_cols() { return kBlockCols; }

int layer_scan_blocks(const ChunkParams& p) {
  return p.dk == 128 ? p.DV / (16 * scan_tiles_per_wg(p)) : p.DV / kBlockCols;
}

// The layer scan applies the gated norm itself (FUSE) when it loads directly (dk = 128),
// the exchange array is there and its grid is one round of the chip: at one workgroup per
// CU (the scan's LDS), every workgroup is then resident together, so the waits for the
// other column blocks' partials end.
bool layer_scan_fuses_norm(const ChunkParams& p) {
  if (!p.ss_xch || !layer_v_in_scan(p.dk)) return false;
  const long long grid = (long long)p.N * p.Hv * layer_scan_blocks(p);
  return grid <= device_cus();
}

int layer_ss_slots(const ChunkParams& p) {
  return p.dk == 128 ? p.DV / (16 * scan_tiles_per_wg(p)) : p.DV / 16;
}

int chunk_record_bytes(int mode, bool bwd) { return rec_bytes(mode, bwd); }

bool chunk_dims_supported(int dk, int dv, bool f32_inputs) {
  if (dv % kBlockCols != 0 || dv > 256) return false;
  if (f32_inputs) return dk == 32 || dk == 64 || dk == 128;
  return dk == 64 || dk == 128;
}

bool layer_dims_supported(int dk, int dv) { return chunk_dims_supported(dk, dv, false); }

bool layer_scan_forms_v(int dk) { return layer_v_in_scan(dk); }

hipError_t launch_scan_bwd(const ChunkParams& p, int mode, hipStream_t stream) {
  if (mode == MODE_F32) {
    if (p.dk == 64) return launch_scan_cfg<64, MODE_F32, true>(p, stream);
    if (p.dk == 32) return launch_scan_cfg<32, MODE_F32, true>(p, stream);
    return hipErrorInvalidValue;
  }
  if (mode == MODE_BF16) {
    if (p.dk == 128) return launch_scan_cfg<128, MODE_BF16, true>(p, stream);
    if (p.dk == 64) return launch_scan_cfg<64, MODE_BF16, true>(p, stream);
  }
  return hipErrorInvalidValue;
}

hipError_t launch_scan(const ChunkParams& p, int mode, hipStream_t stream) {
  if (mode == MODE_F32) {
    if (p.dk == 64) return launch_scan_cfg<64, MODE_F32>(p, stream);
    if (p.dk == 32) return launch_scan_cfg<32, MODE_F32>(p, stream);
    if (p.dk == 128) return launch_scan_cfg<128, MODE_F32>(p, stream);
    return hipErrorInvalidValue;
  }
  if (mode == MODE_LAYER) {
    if (p.dk == 128) {
      if (layer_scan_fuses_norm(p)) return launch_scan_direct<128, MODE_LAYER, true>(p, stream);
      return launch_scan_direct<128, MODE_LAYER>(p, stream);
    }
    if (p.dk == 64) return launch_scan_cfg<64, MODE_LAYER>(p, stream);
    return hipErrorInvalidValue;
  }
  if (p.dk == 128) return launch_scan_direct<128, MODE_BF16>(p, stream);
  if (p.dk == 64) return launch_scan_cfg<64, MODE_BF16>(p, stream);
  return hipErrorInvalidValue;
}

}  // namespace omx
