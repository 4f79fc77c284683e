// Chunk-parallel preparation for the chunked gated delta rule on gfx950.
//
// Everything in a chunk of chunk_gated_delta_rule (omegalax/models/qwen3_5/
// deltanet.py:53-153) that does not depend on the recurrent state is computed
// here, for all chunks at once, one workgroup per (chunk, key head):
//   * q, k rows: (layer path) causal depthwise conv + SiLU (deltanet.py:35-50,
//     243), then the L2 norm at input precision (:30-32, 65-66); written to the
//     workspace for the scan.  (layer path, dk = 64) v rows: conv + SiLU, written
//     likewise; with dk = 128 the scan forms them from mixed_qkv itself.
//   * the Gram products K K^T and Q K^T of the key head, once for all gqa value
//     heads that share it (the repeat-interleave of :272-280);
//   * per value head: the gates (:248-250 on the layer path), G = cumsum(g)
//     (:98), L = strict_lower(beta_i (k_i.k_j) e^{G_i-G_j}) (:100-108),
//     T = (I + L)^-1 (:110-113), P = lower(scale (q_i.k_j) e^{G_i-G_j}) (:130-131).
// T is formed by blocks: each wavefront inverts one 16x16 diagonal block by the
// product (I + N)(I + N^2)(I + N^4)(I + N^8) with N = -L_ww, then wavefront j runs
// down block column j,
//     T_ij = -T_ii sum_{k=j}^{i-1} L_ik T_kj,
// on 16x16x16 MFMAs with hi+lo bf16 operands (fp32-accurate products).  The
// outputs go to the per-(chunk, value head) record described in gdn_chunk.h.
//
// Layouts without transposes.  An MFMA result tile C = A B sits in registers as
// lane (q, r) holding C[4q..4q+3][r]; read the other way round that is the
// A-operand fragment of C^T.  So every tile that must leave as an A fragment is
// computed transposed: the Gram tiles with the block roles swapped (K K^T is
// symmetric; (Q K^T)^T = K Q^T), and the off-diagonal T blocks a second time as
// T_ij^T = -X^T T_ii^T from the same two operands.
#include "gdn_chunk.h"
#include "gdn_conv.h"
#include "gdn_kernels.h"

namespace omx {

namespace {

constexpr int C = kC, NT = kNT;

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

// A 16x16 block in both MFMA layouts: fc = C layout (lane (q, r) holds rows
// 4q..4q+3 of column r), fa = A layout (lane (q, r) holds row r, columns 4q..4q+3),
// with the bf16 hi/lo packs of each.
struct Blk {
  f32x4 fa, fc;
  u32x2 ah, al, ch, cl;
  __device__ __forceinline__ void set(f32x4 a, f32x4 c) {
    fa = a;
    fc = c;
    ah = pack_hi4(a);
    al = pack_lo4(a);
    ch = pack_hi4(c);
    cl = pack_lo4(c);
  }
};

// X Y in both layouts: (X Y)_C from A(X) and C(Y); (X Y)_A = ((X Y)^T)_C = (Y^T X^T)_C,
// whose A operand is Y^T (= C(Y) read as A) and B operand X^T (= A(X) read as B)
__device__ __forceinline__ Blk blk_mul(const Blk& x, const Blk& y) {
  Blk r;
  r.set(mm3k16(zero4(), y.ch, y.cl, x.ah, x.al), mm3k16(zero4(), x.ah, x.al, y.ch, y.cl));
  return r;
}
__device__ __forceinline__ f32x4 blk_mul_c(const Blk& x, const Blk& y) {
  return mm3k16(zero4(), x.ah, x.al, y.ch, y.cl);
}

// beta of the columns 16 bj + 4 lq + (0..3) an A-layout tile holds (gw: G, then beta)
__device__ __forceinline__ f32x4 col_beta(const float* gw, int bj) {
  const float4 b = *(const float4*)(gw + kC + 16 * bj + 4 * (lane_id() >> 4));
  return f32x4{b.x, b.y, b.z, b.w};
}

// one 16x16 tile's A fragment into its half of a record pair (16 bytes per lane)
__device__ __forceinline__ void put_tile(__amdgpu_buffer_rsrc_t rec, int off, u32x2 f) {
  __builtin_amdgcn_raw_buffer_store_b64(f, rec, 16 * lane_id(), off, 0);
}

// L2 norm of a row spread over W lanes (8 values each), in fp32 like the
// reference's norm at input precision; the bf16 pack that follows rounds it.
template <int W>
__device__ __forceinline__ void l2norm8(float* x) {
  float ss = 0.f;
#pragma unroll
  for (int e = 0; e < 8; ++e) ss += x[e] * x[e];
  ss = group_sum_dpp<W>(ss);
  const float inv = rsqrtf(ss + 1e-6f);
#pragma unroll
  for (int e = 0; e < 8; ++e) x[e] *= inv;
}

// One (chunk, key head) task: chunk ci of sequence n (tokens [t0, t0 + nvalid)).
struct PrepTask {
  int ci, hk, n, nvalid;
  long long s0, t0;
};

// Entry i of a small read-only table (chunk offsets, sequence bounds) at a uniform
// index, read through the scalar unit: a constant-address-space load is a scalar load,
// which neither adds to nor waits on the vector memory counter (the table was written
// before this kernel started).
__device__ __forceinline__ int uniform_ld(const int32_t* a, int i) {
  return ((const __attribute__((address_space(4))) int32_t*)a)[i];
}

// Task index -> task.  Tasks are key-head major (task = hk * n_ci + ci), so the
// consecutive workgroups share the key head and its conv weights.
__device__ __forceinline__ PrepTask prep_task(const ChunkParams& p, int task, int n_ci) {
  PrepTask t;
  t.hk = task / n_ci;
  t.ci = task % n_ci;
  int c;
  if (p.chunk_off) {
    int lo = 0, hi = p.N;  // chunk_off[lo] <= ci < chunk_off[hi]
    while (hi - lo > 1) {
      const int mid = (lo + hi) >> 1;
      if (uniform_ld(p.chunk_off, mid) <= t.ci) lo = mid;
      else hi = mid;
    }
    t.n = lo;
    c = t.ci - uniform_ld(p.chunk_off, lo);
  } else {
    t.n = t.ci / p.nch;
    c = t.ci % p.nch;
  }
  long long s1;
  if (p.cu_seqlens) {  // as seq_range, from scalar loads
    const long long lo = uniform_ld(p.cu_seqlens, t.n), hi = uniform_ld(p.cu_seqlens, t.n + 1);
    t.s0 = lo < 0 ? 0 : (lo > p.T ? p.T : lo);
    s1 = hi < t.s0 ? t.s0 : (hi > p.T ? p.T : hi);
  } else {
    seq_range(nullptr, t.n, p.T, t.s0, s1);
  }
  t.t0 = t.s0 + (long long)c * C;
  t.nvalid = (int)((s1 - t.t0) < C ? (s1 - t.t0) : C);
  // the task is uniform over the workgroup: keep it in scalar registers (values read
  // from the offset arrays would otherwise sit in vector registers)
  t.ci = __builtin_amdgcn_readfirstlane(t.ci);
  t.hk = __builtin_amdgcn_readfirstlane(t.hk);
  t.n = __builtin_amdgcn_readfirstlane(t.n);
  t.nvalid = __builtin_amdgcn_readfirstlane(t.nvalid);
  t.s0 = ((long long)__builtin_amdgcn_readfirstlane((int)(t.s0 >> 32)) << 32) |
         (unsigned)__builtin_amdgcn_readfirstlane((int)t.s0);
  t.t0 = ((long long)__builtin_amdgcn_readfirstlane((int)(t.t0 >> 32)) << 32) |
         (unsigned)__builtin_amdgcn_readfirstlane((int)t.t0);
  return t;
}

constexpr int kGatePf = 4;  // value heads per key head whose gate inputs load with the rows

// Per-thread register load of the task's inputs: raw q/k rows (core modes)
// and the gate inputs of value head w of the task's first kGatePf (wavefront w,
// lane = token), with (layer) that head's A_log and dt_bias.
template <int DK, int MODE>
struct PrepIn {
  static constexpr int NRAW = MODE == MODE_LAYER ? 1 : PrepCfg<DK, MODE>::NI_KQ * PrepCfg<DK, MODE>::RAWW;
  u32x4 raw[NRAW];
  float ga, gb;
  float alog, dtb;
};
static_assert(kGatePf == NT / 64, "one value head's gate inputs per wavefront");

template <int DK, int MODE>
__device__ __forceinline__ void load_task_inputs(const ChunkParams& p, const PrepTask& t,
                                                 PrepIn<DK, MODE>& pf) {
  using Q_ = PrepCfg<DK, MODE>;
  constexpr int SEGS = Q_::SEGS;
  constexpr bool F32 = MODE == MODE_F32;
  const int tid = threadIdx.x, l = tid & 63;
  if constexpr (MODE == MODE_LAYER) {
    // the conv input windows are loaded where they are consumed (holding them
    // across the compute phase would halve the occupancy)
  } else {
    // uniform row-0 bases plus 32-bit lane byte offsets
    constexpr unsigned ES = F32 ? 4u : 2u;
    const unsigned char* kb = (const unsigned char*)p.k + (t.t0 * p.k_ld + (long long)t.hk * DK) * ES;
    const unsigned char* qb = (const unsigned char*)p.q + (t.t0 * p.q_ld + (long long)t.hk * DK) * ES;
#pragma unroll
    for (int k = 0; k < Q_::NI_KQ; ++k) {
      constexpr int PER = C * SEGS;
      const int which = (k * NT) / PER;  // 0 = k, 1 = q (compile time)
      const int rem = (k * NT) % PER + tid;
      const int r = rem / SEGS, seg = rem % SEGS;
      const unsigned rr = (unsigned)(r < t.nvalid ? r : t.nvalid - 1);  // padded rows: zeroed later
      const unsigned off = ES * (rr * (unsigned)(which == 0 ? p.k_ld : p.q_ld) + 8u * seg);
      const u32x4* src = (const u32x4*)at_bytes(which == 0 ? kb : qb, off);
      pf.raw[k * Q_::RAWW] = src[0];
      if constexpr (F32) pf.raw[k * Q_::RAWW + 1] = src[1];
    }
  }
  const int gqa = p.Hv / p.Hk;
  const int gg = tid >> 6;  // this wavefront's value head within the key head
  const long long g0 = t.t0 * p.Hv + (long long)t.hk * gqa;  // token t0, first value head
  pf.ga = 0.f;
  pf.gb = 0.f;
  pf.alog = 0.f;
  pf.dtb = 0.f;
  if constexpr (MODE == MODE_LAYER) {
    if (gg < gqa) {
      pf.alog = p.A_log[t.hk * gqa + gg];
      pf.dtb = p.dt_bias[t.hk * gqa + gg];
    }
  }
  if (gg < gqa && l < t.nvalid) {
    const unsigned lo = (unsigned)l * (unsigned)p.Hv;  // lane = token
    if constexpr (MODE == MODE_LAYER) {
      pf.ga = bf2f(*at_bytes((const bf16_t*)p.a + g0 + gg, 2u * lo));
      pf.gb = bf2f(*at_bytes((const bf16_t*)p.b + g0 + gg, 2u * lo));
    } else {
      pf.ga = *at_bytes(p.g + g0 + gg, 4u * lo);
      pf.gb = *at_bytes(p.beta + g0 + gg, 4u * lo);
    }
  }
}

// Each workgroup runs one task, whose first phase waits on its global loads; three
// resident workgroups per CU (the LDS limit) hide that latency.  A persistent variant
// that prefetched the next task into registers needed about 80 more registers, so
// only two fitted, and was slower.  fp32 inputs stage hi and lo rows, whose LDS allows
// two workgroups.
template <int DK, int MODE>
constexpr int prep_blocks_per_cu() { return MODE == MODE_F32 ? (DK == 128 ? 1 : 2) : 3; }

// A-layout 16x16 fp32 tile (lane (q, r) holds M[16 bi + r][16 bj + 4q .. +3]) into a
// row-major 64x64 matrix
__device__ __forceinline__ void put_f32_tile(float* m, int bi, int bj, f32x4 a) {
  const int l = lane_id();
  *(float4*)(m + (16 * bi + (l & 15)) * kC + 16 * bj + 4 * (l >> 4)) = float4{a[0], a[1], a[2], a[3]};
}

// BWD: also writes, per (chunk, value head), the fp32 matrices the backward pass reads
// (X^T with X = (I + L)^-1, Lg = strict_lower(K K^T * Gamma), P, and G; layout in
// gdn_chunk.h).
template <int DK, int MODE, bool BWD = false>
__global__ __launch_bounds__(NT, (prep_blocks_per_cu<DK, MODE>())) void prep_kernel(ChunkParams p) {
  using Q_ = PrepCfg<DK, MODE>;
  constexpr int LDK = Q_::LDK, SEGS = Q_::SEGS;
  constexpr bool IS = Q_::IS, F32 = MODE == MODE_F32;
  __shared__ __align__(16) bf16_t sK[Q_::NS * C * LDK];   // K rows [token][dk] (hi, lo)
  __shared__ __align__(16) bf16_t sQ[Q_::NS * C * LDK];   // Q rows
  __shared__ __align__(16) u32x2 sLf[10 * 2 * 64];        // L blocks as A fragments (hi, lo)
  __shared__ __align__(16) u32x2 sTd[4 * 2 * 64];         // diagonal inverses as A fragments (hi, lo)
  __shared__ __align__(16) float sGw[4 * 2 * C];          // per wave: G log2(e), beta
  __shared__ __align__(16) float sGin[kGatePf * 2 * C];   // gate inputs of kGatePf value heads
  __shared__ float sPar[kGatePf][2];                        // (layer) their A_log, dt_bias
  constexpr int K_LO = C * LDK;

  const int tid = threadIdx.x, l = tid & 63, lq = l >> 4, lr = l & 15;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int gqa = p.Hv / p.Hk;
  // tasks: (chunk, key head) pairs, one per workgroup (the grid may hold spare ones)
  const int n_ci = p.chunk_off ? uniform_ld(p.chunk_off, p.N) : p.n_rec;
  const int total = n_ci * p.Hk;
  const int task = (int)blockIdx.x;
  if (task >= total) return;  // uniform

  PrepIn<DK, MODE> pf;
  {
    const PrepTask tk = prep_task(p, task, n_ci);
    load_task_inputs<DK, MODE>(p, tk, pf);
    const int hk = tk.hk, ci = tk.ci, n = tk.n, nvalid = tk.nvalid;
    const long long s0 = tk.s0, t0 = tk.t0;

    // -------------------------------------------------------------- q, k, v rows
    if constexpr (MODE == MODE_LAYER) {
      // dk = 64: wave 0 forms the k rows, wave 1 the q rows, waves 2-3 the v channels of
      // the gqa value heads (16 rows per item).  dk = 128, where the scan forms v: waves
      // 0 and 2 the k rows (top and bottom half of the chunk), waves 1 and 3 the q rows.
      // Lane = 8-channel group g + SEGS * row part; each lane streams its rows, and the
      // SEGS lanes of a row are adjacent, so the row's L2 norm is a DPP sum.
      constexpr bool SPLIT = layer_v_in_scan(DK);
      if (SPLIT || wave < 2) {
        constexpr int RP = 64 / SEGS, ROWS = C / RP / (SPLIT ? 2 : 1);
        const int which = SPLIT ? (wave & 1) : wave;  // 0: k, 1: q
        const int g = l % SEGS, r0 = (SPLIT ? (wave >> 1) * (C / 2) : 0) + (l / SEGS) * ROWS;
        bf16_t* dst = (which == 0 ? sK : sQ) + 8 * g;
        // row t0 of this key head (uniform) plus the lane's byte offset; rows at or past
        // nvalid lie outside the resource's range and are dropped, so no store sits under
        // a branch (which would leave the count of outstanding memory operations unknown
        // and make the next wait for a load wait for every store too)
        const unsigned ostride = (unsigned)(p.Hk * DK);
        const auto gout = buf_rsrc((bf16_t*)(which == 0 ? p.kn : p.qn) + t0 * (long long)p.Hk * DK +
                                       (long long)hk * DK,
                                   2u * (unsigned)nvalid * ostride);
        conv_rows<ROWS>(p, n, s0, t0, nvalid, r0, (which == 0 ? p.Hk * DK : 0) + hk * DK, 8 * g,
                        [&](int m, const u32x4& yw) {
          float y[8];
          unpack8<false>(&yw, y);
          l2norm8<SEGS>(y);
          const u32x4 hw = pack8(y);
          const int r = r0 + m;
          *(u32x4*)(dst + r * LDK) = hw;
          __builtin_amdgcn_raw_buffer_store_b128(hw, gout, 2u * ((unsigned)r * ostride + 8u * g), 0, 0);
        });
      } else if constexpr (!layer_v_in_scan(DK)) {
        const int VG = gqa * p.DV / 8;  // 8-channel groups of v
        const int vch0 = 2 * p.Hk * DK + hk * gqa * p.DV;
        const unsigned vstride = (unsigned)(p.Hv * p.DV);
        // rows past nvalid are dropped by the range (no store under a branch)
        const auto vout = buf_rsrc((bf16_t*)p.vc + t0 * (long long)p.Hv * p.DV + (long long)hk * gqa * p.DV,
                                   2u * (unsigned)nvalid * vstride);
        for (int it = tid - 128; it < VG * 4; it += 128) {
          const int g = it % VG, r0 = (it / VG) * 16;
          if (r0 >= nvalid) continue;
          auto emit = [&](int m, const u32x4& y) {
            const int r = r0 + m;
            __builtin_amdgcn_raw_buffer_store_b128(y, vout, 2u * ((unsigned)r * vstride + 8u * g), 0, 0);
          };
          conv_rows<16>(p, n, s0, t0, nvalid, r0, vch0, 8 * g, emit);
        }
      }
    } else {
      // Every loaded register is consumed before the task's first global store:
      // the memory counter retires operations in issue order, so a register read after
      // a store would also wait for that store to complete.
      sGin[wave * 2 * C + l] = pf.ga;
      sGin[wave * 2 * C + C + l] = pf.gb;
      u32x4 hwk[Q_::NI_KQ];
#pragma unroll
      for (int k = 0; k < Q_::NI_KQ; ++k) {
        constexpr int PER = C * SEGS;
        const int which = (k * NT) / PER;  // 0 = k, 1 = q (compile time)
        const int rem = (k * NT) % PER + tid;
        const int r = rem / SEGS, seg = rem % SEGS;
        float x[8];
        unpack8<F32>(&pf.raw[k * Q_::RAWW], x);
        if (nvalid < C) {  // uniform: a sequence's last chunk; its padded rows are zero
          const float keep = (float)(r < nvalid);
#pragma unroll
          for (int e = 0; e < 8; ++e) x[e] *= keep;
        }
        if (p.qk_l2norm) l2norm8<SEGS>(x);
        // bf16 inputs: the normalised row is rounded to bf16 (the reference
        // normalises in the input dtype); the pack below does the rounding
        bf16_t* dst = (which == 0 ? sK : sQ) + r * LDK + seg * 8;
        const u32x4 hw = pack8(x);
        *(u32x4*)dst = hw;
        hwk[k] = hw;
        if constexpr (IS) *(u32x4*)(dst + K_LO) = pack8_lo(x);
        if constexpr (F32) {  // fp32 rows are stored as they form (no register copy)
          void* out = which == 0 ? p.kn : p.qn;
          if (out && (nvalid == C || r < nvalid)) {
            const long long o0 = t0 * (long long)p.Hk * DK + (long long)hk * DK;
            const unsigned lo = (unsigned)r * (unsigned)(p.Hk * DK) + 8u * seg;
            float4* d4 = (float4*)at_bytes((float*)out + o0, 4u * lo);
            d4[0] = float4{x[0], x[1], x[2], x[3]};
            d4[1] = float4{x[4], x[5], x[6], x[7]};
          }
        }
      }
      if constexpr (!F32) {
#pragma unroll
        for (int k = 0; k < Q_::NI_KQ; ++k) {
          constexpr int PER = C * SEGS;
          const int which = (k * NT) / PER;
          const int rem = (k * NT) % PER + tid;
          const int r = rem / SEGS, seg = rem % SEGS;
          void* out = which == 0 ? p.kn : p.qn;
          if (out && (nvalid == C || r < nvalid)) {
            // row t0 of this key head (uniform) plus the lane's byte offset
            const long long o0 = t0 * (long long)p.Hk * DK + (long long)hk * DK;
            const unsigned lo = (unsigned)r * (unsigned)(p.Hk * DK) + 8u * seg;
            *(u32x4*)at_bytes((bf16_t*)out + o0, 2u * lo) = hwk[k];
          }
        }
      }
    }
    if constexpr (MODE == MODE_LAYER) {
      sGin[wave * 2 * C + l] = pf.ga;
      sGin[wave * 2 * C + C + l] = pf.gb;
      if (l == 0) {
        sPar[wave][0] = pf.alog;
        sPar[wave][1] = pf.dtb;
      }
    }
    lds_barrier();

    // -------------------------------------------------------------- Gram tiles
    // Tile (bi, bj) is computed as (rows of block bj) x (rows of block bi)^T, so lane
    // (q, r) holds entry [16 bi + r][16 bj + 4q + v]: the A fragment of the tile.
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
        frag2<IS>(sK, K_LO, LDK, 16 * bj, 32 * s, ah, al);
        frag2<IS>(qk ? sQ : sK, K_LO, LDK, 16 * bi, 32 * s, bh, bl);
        tacc[ti] = mm<IS, IS>(tacc[ti], ah, al, bh, bl);
      }
    }

    float* gw = sGw + wave * 2 * C;  // this wave's G log2(e) [0, C) and beta [C, 2C)
    const size_t rec_stride = (size_t)rec_bytes(MODE, BWD);

    for (int gg = 0; gg < gqa; ++gg) {
      const int h = hk * gqa + gg;
      const auto rec = buf_rsrc(p.rec + ((size_t)ci * p.Hv + h) * rec_stride, (unsigned)rec_stride);
      float* xb = BWD ? p.xlpg + ((size_t)ci * p.Hv + h) * kXlpgFloats : nullptr;
      if constexpr (BWD) {
        // the lower tiles of X^T and (fp32 inputs) the upper tiles of Lg and P are zero
        for (int z = wave; z < (IS ? 18 : 6); z += 4) {
          const int mat = z / 6, u = z % 6;
          const int bi = u < 3 ? 0 : (u < 5 ? 1 : 2);
          const int bj = u < 3 ? u + 1 : (u < 5 ? u - 1 : 3);
          if (mat == 0) put_f32_tile(xb + kXlpgX, bj, bi, zero4());
          else if (IS) put_f32_tile(xb + mat * kXlpgMat, bi, bj, zero4());
        }
      }

      // gates of value head h, one token per lane; every wave scans its own copy.  The
      // inputs come from LDS only: a global load here, whose register the loop reuses,
      // would make every value head wait for all of the wavefront's outstanding memory
      // operations (this task's row and record stores).
      if (gg >= kGatePf && gg % kGatePf == 0) {  // uniform; only when gqa > kGatePf
        // the next kGatePf heads' gate inputs replace the staged ones (every wave has
        // passed the previous head's last barrier, so sGin is free)
        if (wave < kGatePf) {
          float ga = 0.f, gb = 0.f;
          if (gg + wave < gqa && l < nvalid) {
            const long long i0 = t0 * p.Hv + h + wave;
            const unsigned lo = (unsigned)l * (unsigned)p.Hv;
            if constexpr (MODE == MODE_LAYER) {
              ga = bf2f(*at_bytes((const bf16_t*)p.a + i0, 2u * lo));
              gb = bf2f(*at_bytes((const bf16_t*)p.b + i0, 2u * lo));
            } else {
              ga = *at_bytes(p.g + i0, 4u * lo);
              gb = *at_bytes(p.beta + i0, 4u * lo);
            }
          }
          sGin[wave * 2 * C + l] = ga;
          sGin[wave * 2 * C + C + l] = gb;
          if constexpr (MODE == MODE_LAYER) {
            if (l == 0 && gg + wave < gqa) {
              sPar[wave][0] = p.A_log[h + wave];
              sPar[wave][1] = p.dt_bias[h + wave];
            }
          }
        }
        lds_barrier();
      }
      {
        const int slot = gg % kGatePf;
        float g = sGin[slot * 2 * C + l];
        float bt = sGin[slot * 2 * C + C + l];
        if constexpr (MODE == MODE_LAYER) {
          // deltanet.py:248-250: beta in bf16, g in fp32 (padded tokens: both 0)
          const float keep = (float)(l < nvalid);
          g = -expf(sPar[slot][0]) * softplusf_(g + sPar[slot][1]) * keep;
          bt = round_bf(sigmoidf_(bt)) * keep;
        }
        const float G = wave_scan_dpp(g);
        if constexpr (BWD)
          if (wave == 0) xb[kXlpgG + l] = G;
        const float Gl = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(G), 63));
        const float eg = __expf(G);
        gw[l] = G * 1.4426950408889634f;
        gw[C + l] = bt;
        if (wave == 0) {
          auto put = [&](int row, float x) {
            __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(x), rec, 4 * l, kRecG + 4 * C * row, 0);
          };
          put(kGateEG, eg);
          put(kGateEGS, p.scale * eg);
          put(kGateEL, l == C - 1 ? __expf(Gl) : __expf(Gl - G));
          put(kGateBeta, bt);
        }
        wave_lds_fence();
      }
      // gate the wave's Gram tiles into L (strictly lower) and P (lower) blocks; lane
      // (q, r) holds row i = 16 bi + r, columns m = 16 bj + 4q + v
      f32x4 Tw = zero4();  // this wave's diagonal inverse T_ww, C layout
  #pragma unroll
      for (int ti = 0; ti < 5; ++ti) {
        const f32x4 acc = tacc[ti];
        const int code = tile_code(wave + 4 * ti);
        const bool qk = ti >= 3 || (ti == 2 && wave >= 2);
        const int bi = (code >> 2) & 3, bj = code & 3;
        const int i = 16 * bi + lr;
        const float Gi = gw[i];
        const float4 Gm4 = *(const float4*)(gw + 16 * bj + 4 * lq);
        const float Gm[4] = {Gm4.x, Gm4.y, Gm4.z, Gm4.w};
        f32x4 val;
        if (!qk) {
          const float bt = gw[C + i];
          // branch-free: the exponent is clamped to <= 0 (masked entries would
          // overflow) and the strictly-lower mask multiplies the result
          if constexpr (BWD) {
            f32x4 lg;
#pragma unroll
            for (int v = 0; v < 4; ++v) {
              const int m = 16 * bj + 4 * lq + v;
              lg[v] = acc[v] * __builtin_amdgcn_exp2f(fminf(Gi - Gm[v], 0.f)) * (float)(i > m);
              val[v] = bt * lg[v];
            }
            // (bf16 inputs: the gradient kernel forms its Lg tiles from K itself)
            if constexpr (IS) put_f32_tile(xb + kXlpgLg, bi, bj, lg);
          } else {
#pragma unroll
          for (int v = 0; v < 4; ++v) {
            const int m = 16 * bj + 4 * lq + v;
            val[v] = bt * acc[v] * __builtin_amdgcn_exp2f(fminf(Gi - Gm[v], 0.f)) * (float)(i > m);
          }
          }
          if (ti == 0) {
            // The diagonal block.  With N = -L_ww (strictly lower, so N^16 = 0),
            //   T_ww = (I + L_ww)^-1 = (I + N)(I + N^2)(I + N^4)(I + N^8),
            // formed in registers on 16x16x16 MFMAs in split precision.  Each product
            // is kept in two layouts: C (lane (q, r) holds rows 4q..4q+3 of column r,
            // the B operand of the next product) and A (the transpose of that: the A
            // operand), the A form computed as the transposed product (X Y)^T = Y^T X^T
            // from the same packed operands.
            Blk n1;
            f32x4 nc;  // C layout of N: entry (16bi + 4lq + v, 16bi + lr); K K^T is symmetric
            {
              const int m2 = 16 * bi + lr;
              const float Gm2 = gw[m2];
              const float4 Gi4 = *(const float4*)(gw + 16 * bi + 4 * lq);
              const float4 Bi4 = *(const float4*)(gw + C + 16 * bi + 4 * lq);
              const float gi2[4] = {Gi4.x, Gi4.y, Gi4.z, Gi4.w}, bt2[4] = {Bi4.x, Bi4.y, Bi4.z, Bi4.w};
#pragma unroll
              for (int v = 0; v < 4; ++v) {
                const int i2 = 16 * bi + 4 * lq + v;
                nc[v] = -bt2[v] * acc[v] * __builtin_amdgcn_exp2f(fminf(gi2[v] - Gm2, 0.f)) *
                        (float)(i2 > m2);
              }
            }
            n1.set(-val, nc);
            const Blk n2 = blk_mul(n1, n1), n4 = blk_mul(n2, n2);
            const f32x4 n8c = blk_mul_c(n4, n4);
            f32x4 eye;
#pragma unroll
            for (int v = 0; v < 4; ++v) eye[v] = (float)(4 * lq + v == lr);
            Blk x1, x2;
            {
              const Blk y = blk_mul(n1, n2);
              x1.set(eye + n1.fa + n2.fa + y.fa, eye + n1.fc + n2.fc + y.fc);
            }
            {
              const Blk z = blk_mul(x1, n4);
              x2.set(x1.fa + z.fa, x1.fc + z.fc);
            }
            const u32x2 n8h = pack_hi4(n8c), n8l = pack_lo4(n8c);
            const f32x4 Tc = x2.fc + mm3k16(zero4(), x2.ah, x2.al, n8h, n8l);
            const f32x4 Ta = x2.fa + mm3k16(zero4(), n8h, n8l, x2.ah, x2.al);
            Tw = Tc;
            const u32x2 th = pack_hi4(Ta), tl = pack_lo4(Ta);
            sTd[(2 * bi) * 64 + l] = th;  // A fragments of T_ww for the other waves
            sTd[(2 * bi + 1) * 64 + l] = tl;
            // the record holds T diag(beta): column 16 bi + 4 lq + v scaled by its beta
            const f32x4 Tb = Ta * col_beta(gw, bi);
            put_tile(rec, rec_t_off(bi, bi), pack_hi4(Tb));
            if constexpr (BWD) put_f32_tile(xb + kXlpgX, bi, bi, Tc);  // X^T: the C layout
            put_tile(rec, rec_t_off(bi, bi) + kPairBytes, pack_lo4(Tb));
            if ((bi & 1) == 0) {
              // the zero upper tile (bi, bi + 1) that completes row block bi's last pair
              const u32x2 z = {0u, 0u};
              put_tile(rec, rec_t_off(bi, bi + 1), z);
              put_tile(rec, rec_t_off(bi, bi + 1) + kPairBytes, z);
              if (!BWD || IS || p.o) put_tile(rec, rec_p_off(bi, bi + 1), z);
              if constexpr (IS || BWD)
                if (IS || p.o) put_tile(rec, rec_p_off(bi, bi + 1) + (kRecPL - kRecP), z);
            }
          } else {
            u32x2* d = sLf + 2 * 64 * tile_index(bi, bj) + l;
            d[0] = pack_hi4(val);
            d[64] = pack_lo4(val);
          }
        } else {
          const float sc = p.scale;
  #pragma unroll
          for (int v = 0; v < 4; ++v) {
            const int m = 16 * bj + 4 * lq + v;
            val[v] = sc * acc[v] * __builtin_amdgcn_exp2f(fminf(Gi - Gm[v], 0.f)) * (float)(i >= m);
          }
          // (a backward recompute that forms no o reads no P: bf16 inputs leave it out)
          if (!BWD || IS || p.o) put_tile(rec, rec_p_off(bi, bj), pack_hi4(val));
          // (bf16 inputs: the backward kernels form their P operands from K and Q)
          if constexpr (BWD && IS) put_f32_tile(xb + kXlpgP, bi, bj, val);
          // (backward) P's lo parts only where the scan forms o: the layer backward
          if constexpr (IS || BWD)
            if (IS || p.o) put_tile(rec, rec_p_off(bi, bj) + (kRecPL - kRecP), pack_lo4(val));
        }
      }
      lds_barrier();  // L blocks and the diagonal inverses of all waves are in LDS

      // block column j = wave: T_ij = -T_ii X, X = sum_{k=j}^{i-1} L_ik T_kj, i = j+1..3.
      // X is an MFMA result in C layout: the B operand here, and read the other way the
      // A operand of X^T, so T_ij^T = -X^T T_ii^T (the record's A fragment of T_ij)
      // comes from the same operands with the roles swapped.
      {
        const int j = wave;
        u32x2 Th[4], Tl[4];  // B operands (C layout) of the column's finished blocks T_kj
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
            const u32x2* f = sLf + 2 * 64 * tile_index(i, k) + l;
            X = mm3k16(X, f[0], f[64], Th[k], Tl[k]);
          }
          // the T_ii fragment is negated (a sign flip is exact in bf16)
          const u32x2 th = sTd[(2 * i) * 64 + l] ^ 0x80008000u;
          const u32x2 tl = sTd[(2 * i + 1) * 64 + l] ^ 0x80008000u;
          const u32x2 xh = pack_hi4(X), xl = pack_lo4(X);
          const f32x4 Tij = mm3k16(zero4(), th, tl, xh, xl);
          const f32x4 TijT = mm3k16(zero4(), xh, xl, th, tl);
          Th[i] = pack_hi4(Tij);
          Tl[i] = pack_lo4(Tij);
          const f32x4 Tb = TijT * col_beta(gw, j);  // T_ij diag(beta), A layout
          put_tile(rec, rec_t_off(i, j), pack_hi4(Tb));
          if constexpr (BWD) put_f32_tile(xb + kXlpgX, j, i, Tij);  // X^T: the C layout
          put_tile(rec, rec_t_off(i, j) + kPairBytes, pack_lo4(Tb));
        }
      }
      lds_barrier();  // sLf / sTd are rewritten for the next value head
    }
    // (layer) the task of a sequence's first chunk clears the exchange ring of the row
    // partials of the sequence's value heads under this key head (tag 0); the scan that
    // fuses the gated norm writes chunk c's entries with tag c + 1 (stores through a buffer
    // whose range ends at the ring: lanes past it are dropped).  The scan writes and reads
    // the ring at system scope, past the L2s, so the zeros are written through to memory
    // the same way (sc0 sc1) rather than left to the L2s' write-back: a previous call's
    // entries there carry the tags this call waits for.
    if constexpr (MODE == MODE_LAYER) {
      if (p.ss_xch && t0 == s0) {
        const int cnt = gqa * p.ss_xch_slots * kXchRing * C;  // {value, tag} pairs
        const auto xr = buf_rsrc(
            p.ss_xch + 2 * (((size_t)n * p.Hv + hk * gqa) * p.ss_xch_slots) * kXchRing * C,
            8u * (unsigned)cnt);
        for (int k = 0; k < cnt; k += NT)
          __builtin_amdgcn_raw_buffer_store_b64(u32x2{0u, 0u}, xr, 8u * (unsigned)(k + tid), 0, 17);
      }
    }
  }
}

template <int DK, int MODE, bool BWD = false>
hipError_t launch_prep_cfg(const ChunkParams& p, hipStream_t stream) {
  // one workgroup per (chunk slot, key head)
  const long long tasks = (long long)p.n_rec * p.Hk;
  if (tasks == 0) return hipSuccess;
  const unsigned grid = (unsigned)tasks;
  hipLaunchKernelGGL((prep_kernel<DK, MODE, BWD>), dim3(grid), dim3(NT), 0, stream, p);
  return hipGetLastError();
}

// The packed-sequence plan, one workgroup:
//  * cu_out, the offsets every later kernel reads: c[0] = 0, c[N] = T and, between,
//    c[n] = max(c[n-1], clamp(cu[n], 0, T)) (a running maximum), so the sequences are
//    ordered, disjoint and tile [0, T) whatever the caller's array holds.  For valid
//    offsets (0 = cu[0] <= ... <= cu[N] = T) c equals cu;
//  * off[n] = sum over m < n of ceil(len_m / 64), off[N] = the total chunk count;
//  * order: the sequences by chunk count, longest first (ties in index order), for at
//    most kOrderMax sequences (the identity beyond), so that the scans start the longest
//    chains first.
constexpr int kOrderMax = 1024;
__global__ __launch_bounds__(1024) void chunk_plan_kernel(const int32_t* cu, int N, int T,
                                                          int32_t* cu_out, int32_t* off,
                                                          int32_t* order) {
  __shared__ int wmax[16];
  __shared__ int wsum[16];
  __shared__ int scnt[kOrderMax];
  const int tid = threadIdx.x, l = tid & 63, w = tid >> 6;
  auto clamped = [&](int n) {
    if (n == 0) return 0;
    if (n >= N) return T;
    const int x = cu[n];
    return x < 0 ? 0 : (x > T ? T : x);
  };
  int carry_max = 0, carry = 0;
  for (int base = 0; base < N; base += 1024) {
    const int n = base + tid;
    int m = n < N ? clamped(n) : 0;  // inclusive running maximum within the wave
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
      const int y = __shfl_up(m, o, 64);
      if (l >= o) m = m > y ? m : y;
    }
    if (l == 63) wmax[w] = m;
    __syncthreads();
    int mb = carry_max;
    for (int v = 0; v < w; ++v) mb = mb > wmax[v] ? mb : wmax[v];
    const int c0 = m > mb ? m : mb;  // c[n]
    int cnt = 0;
    if (n < N) {
      const int x1 = clamped(n + 1);
      const int c1 = x1 > c0 ? x1 : c0;  // c[n + 1]
      cu_out[n] = c0;
      cnt = (c1 - c0 + C - 1) / C;
      if (n < kOrderMax) scnt[n] = cnt;
    }
    int x = cnt;  // inclusive scan of the chunk counts within the wave
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
    int total = 0, bmax = carry_max;
    for (int v = 0; v < 16; ++v) {
      total += wsum[v];
      bmax = bmax > wmax[v] ? bmax : wmax[v];
    }
    carry += total;
    carry_max = bmax;
    __syncthreads();
  }
  if (tid == 0) {
    off[N] = carry;
    cu_out[N] = T;
  }
  __syncthreads();  // scnt complete
  for (int n = tid; n < N; n += 1024) {
    int rank = n;
    if (N <= kOrderMax) {
      const int c = scnt[n];
      rank = 0;
      for (int m = 0; m < N; ++m) {
        const int cm = scnt[m];
        rank += (cm > c) || (cm == c && m < n);
      }
    }
    order[rank] = n;
  }
}

}  // namespace

hipError_t launch_chunk_plan(const ChunkParams& p, hipStream_t stream) {
  hipLaunchKernelGGL(chunk_plan_kernel, dim3(1), dim3(1024), 0, stream, p.cu_in, p.N, p.T,
                     const_cast<int32_t*>(p.cu_seqlens), p.chunk_off,
                     const_cast<int32_t*>(p.seq_order));
  return hipGetLastError();
}

hipError_t launch_prep_bwd(const ChunkParams& p, int mode, hipStream_t stream) {
  if (mode == MODE_F32) {
    if (p.dk == 64) return launch_prep_cfg<64, MODE_F32, true>(p, stream);
    if (p.dk == 32) return launch_prep_cfg<32, MODE_F32, true>(p, stream);
    return hipErrorInvalidValue;
  }
  if (mode == MODE_BF16) {
    if (p.dk == 128) return launch_prep_cfg<128, MODE_BF16, true>(p, stream);
    if (p.dk == 64) return launch_prep_cfg<64, MODE_BF16, true>(p, stream);
  }
  return hipErrorInvalidValue;
}

hipError_t launch_prep(const ChunkParams& p, int mode, hipStream_t stream) {
  if (mode == MODE_F32) {
    if (p.dk == 64) return launch_prep_cfg<64, MODE_F32>(p, stream);
    if (p.dk == 32) return launch_prep_cfg<32, MODE_F32>(p, stream);
    if (p.dk == 128) return launch_prep_cfg<128, MODE_F32>(p, stream);
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
