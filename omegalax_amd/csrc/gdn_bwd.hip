// Backward pass (VJP) of the chunked gated delta rule on gfx950.
//
// The reference trains through chunk_gated_delta_rule (omegalax/models/qwen3_5/
// deltanet.py:53-153) with JAX reverse-mode autodiff (trainers/vlm.py:157-195); this
// file computes that derivative.  Per chunk (G = in-chunk cumsum of g, Gamma_im =
// e^{G_i - G_m} for i >= m, X = (I + L)^-1 with L = diag(beta) Lg, Lg = strict_lower(
// K K^T * Gamma), P = lower(scale Q K^T * Gamma); deltanet.py:98-142):
//     V_new = X diag(beta) (V - diag(e^G) K S)               (:115-116, 133-134)
//     O     = scale diag(e^G) Q S + P V_new                   (:136-137)
//     S'    = e^{G_last} S + K^T diag(e^{G_last - G}) V_new   (:139-142)
// Three kernels, after the forward's preparation and scan have been rerun in their
// backward variants (which leave X, Lg, P, G per chunk and the state entering every
// chunk plus V_new):
//  1. rscan_kernel walks each sequence's chunks backwards carrying dS, the gradient of
//     the state leaving the chunk, in registers (one workgroup per (sequence, value head,
//     64 columns of dv), 16 columns per wavefront):
//         dV_new = P^T dO + diag(e^{G_last - G}) K dS
//         dS    <- e^{G_last} dS + scale Q^T diag(e^G) dO - K^T diag(e^G) diag(beta) X^T dV_new
//     and stores dS per chunk and dV_new.
//  2. cgrad_kernel forms, for every (chunk, value head) at once, the chunk-local
//     gradients of q, k (per value head), v, g and beta from S, dS, V_new, dV_new and
//     the chunk's matrices, differentiating :100-142 step by step (the derivation is the
//     one of the fp64 test oracle, oracle/gdn_vjp.py).
//  3. qk_final_kernel sums the per-value-head q/k gradients over each key head's value
//     heads (the adjoint of the repeat-interleave, :272-280) and applies the L2-norm
//     backward (:30-32), writing dq, dk at the input precision.
// All products are 16x16x32 bf16 MFMAs on operands split into bf16 hi + lo parts
// (hi*hi + hi*lo + lo*hi, fp32-accurate to ~2^-16); operands known to be exact bf16
// (bf16 q/k rows) skip their lo part.
#include <type_traits>

#include "gdn_chunk.h"
#include "gdn_kernels.h"

namespace omx {

namespace {

constexpr int C = kC;
constexpr int NT = kNT;

struct Op {
  u32x4 h, l;
};

// bf16 hi and lo parts of 8 values (x = hi + lo to ~2^-16 relative)
template <bool LO = true>
__device__ __forceinline__ Op split8(const float* x) {
  Op o;
  o.h = pack8(x);
  if constexpr (LO) o.l = pack8_lo(x);
  else o.l = o.h;
  return o;
}

// acc += A B: hi*hi, plus hi*lo when B has a lo part, plus lo*hi when A has one
template <bool AL, bool BL>
__device__ __forceinline__ f32x4 mm3(f32x4 acc, const Op& a, const Op& b) {
  acc = mma16(a.h, b.h, acc);
  if constexpr (BL) acc = mma16(a.h, b.l, acc);
  if constexpr (AL) acc = mma16(a.l, b.h, acc);
  return acc;
}

// B operand from two C-layout tiles side by side (block-pair contraction order)
__device__ __forceinline__ Op join_op(f32x4 a, f32x4 b) {
  Op o;
  o.h = u32x4{pack_bf16(a[0], a[1]), pack_bf16(a[2], a[3]), pack_bf16(b[0], b[1]),
              pack_bf16(b[2], b[3])};
  const u32x2 la = pack_lo4(a), lb = pack_lo4(b);
  o.l = u32x4{la[0], la[1], lb[0], lb[1]};
  return o;
}

__device__ __forceinline__ float ldx(const float* p) { return *p; }
__device__ __forceinline__ float ldx(const bf16_t* p) { return bf2f(*p); }

// Contraction index of operand slot e in lane group q: the natural order 8q + e, or the
// block-pair order (4q + e%4, then 16 + 4q + e%4) of two C-layout tiles side by side.
template <bool PAIR>
__device__ __forceinline__ int kslot(int q, int e) {
  return PAIR ? 4 * q + (e & 3) + 16 * (e >> 2) : 8 * q + e;
}

// operand row `row` of a row-major M[row][k], slots over k from k0
template <bool PAIR, class T>
__device__ __forceinline__ void frag_row(const T* m, int ld, int row, int k0, float* x) {
  const int q = lane_id() >> 4;
#pragma unroll
  for (int e = 0; e < 8; ++e) x[e] = ldx(m + row * ld + k0 + kslot<PAIR>(q, e));
}
// operand column `col` of a row-major M[k][col], slots over the rows from k0
template <bool PAIR, class T>
__device__ __forceinline__ void frag_col(const T* m, int ld, int col, int k0, float* x) {
  const int q = lane_id() >> 4;
#pragma unroll
  for (int e = 0; e < 8; ++e) x[e] = ldx(m + (k0 + kslot<PAIR>(q, e)) * ld + col);
}

// K / Q operand fragments from the staged rows: bf16 rows are exact bf16 (one vector or
// two transposed LDS reads, no lo part); fp32 rows are read element-wise and split.
// kq_row: row row0 + lane%16, slots over columns from k0; kq_col: column col0 + lane%16,
// slots over rows from k0.
template <bool PAIR>
__device__ __forceinline__ Op kq_row(const float* m, int ld, int row0, int k0) {
  float x[8];
  frag_row<PAIR>(m, ld, row0 + (lane_id() & 15), k0, x);
  return split8(x);
}
template <bool PAIR>
__device__ __forceinline__ Op kq_row(const bf16_t* m, int ld, int row0, int k0) {
  const int l = lane_id(), q = l >> 4;
  const bf16_t* pr = m + (row0 + (l & 15)) * ld + k0;
  Op o;
  if constexpr (PAIR) {
    const u32x2 a = *(const u32x2*)(pr + 4 * q), b = *(const u32x2*)(pr + 16 + 4 * q);
    o.h = u32x4{a[0], a[1], b[0], b[1]};
  } else {
    o.h = *(const u32x4*)(pr + 8 * q);
  }
  o.l = o.h;
  return o;
}
template <bool PAIR>
__device__ __forceinline__ Op kq_col(const float* m, int ld, int col0, int k0) {
  float x[8];
  frag_col<PAIR>(m, ld, col0 + (lane_id() & 15), k0, x);
  return split8(x);
}
template <bool PAIR>
__device__ __forceinline__ Op kq_col(const bf16_t* m, int ld, int col0, int k0) {
  Op o;
  if constexpr (PAIR) {
    const u32x2 a = rows4_tr(m, ld, k0, col0), b = rows4_tr(m, ld, k0 + 16, col0);
    o.h = u32x4{a[0], a[1], b[0], b[1]};
  } else {
    o.h = frag_tr(m, ld, k0, col0);
  }
  o.l = o.h;
  return o;
}

// global: 8 consecutive values of row `row` from column k0 + 8q (zero when row >= nvalid)
template <class T>
__device__ __forceinline__ void gfrag_row(const T* base, long long ld, int row, int nvalid, int k0,
                                          float* x) {
  const int q = lane_id() >> 4;
  if (row < nvalid) {
    const T* pr = base + (long long)row * ld + k0 + 8 * q;
    if constexpr (std::is_same<T, float>::value) {
      const float4 a = ((const float4*)pr)[0], b = ((const float4*)pr)[1];
      x[0] = a.x; x[1] = a.y; x[2] = a.z; x[3] = a.w;
      x[4] = b.x; x[5] = b.y; x[6] = b.z; x[7] = b.w;
    } else {
      const u32x4 w = *(const u32x4*)pr;
      unpack8<false>(&w, x);
    }
  } else {
#pragma unroll
    for (int e = 0; e < 8; ++e) x[e] = 0.f;
  }
}
// global: column `col`, rows k0 + 8q + e of a row-major fp32 array (stride ld)
__device__ __forceinline__ void gfrag_col(const float* base, long long ld, int col, int k0,
                                          float* x) {
  const int q = lane_id() >> 4;
#pragma unroll
  for (int e = 0; e < 8; ++e) x[e] = base[(long long)(k0 + 8 * q + e) * ld + col];
}

// Loads whose rows may lie past a sequence's end go through a buffer resource whose range
// ends at the last valid row: the hardware returns zeros beyond it.  So no load sits under
// a branch, which would leave the count of outstanding memory operations unknown and turn
// every later wait for one of them into a wait for all (the previous chunk's stores too).
// Byte offsets are 32-bit.
__device__ __forceinline__ float4 bload4(__amdgpu_buffer_rsrc_t r, unsigned off, const float*) {
  const u32x4 w = __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 0);
  return float4{__uint_as_float(w[0]), __uint_as_float(w[1]), __uint_as_float(w[2]),
                __uint_as_float(w[3])};
}
__device__ __forceinline__ u32x2 bload4(__amdgpu_buffer_rsrc_t r, unsigned off, const bf16_t*) {
  return __builtin_amdgcn_raw_buffer_load_b64(r, off, 0, 0);
}
// gfrag_col over a buffer resource of fp32 rows (zeros past its range)
__device__ __forceinline__ void gfrag_col_b(__amdgpu_buffer_rsrc_t r, unsigned ld, unsigned col,
                                            unsigned k0, float* x) {
  const unsigned q = (unsigned)lane_id() >> 4;
#pragma unroll
  for (int e = 0; e < 8; ++e)
    x[e] = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(r, 4u * ((k0 + 8u * q + e) * ld + col), 0, 0));
}

// 4 elements in registers (4 bf16 in two words, or 4 floats)
template <class T> struct Vec4;
template <> struct Vec4<float> { typedef float4 type; };
template <> struct Vec4<bf16_t> { typedef u32x2 type; };
__device__ __forceinline__ float4 load4(const float* src) { return *(const float4*)src; }
__device__ __forceinline__ void store4(float* dst, float4 x) { *(float4*)dst = x; }
// a float at the precision T (bf16 rounded to nearest even)
template <class T> __device__ __forceinline__ T from_f32(float x);
template <> __device__ __forceinline__ float from_f32<float>(float x) { return x; }
template <> __device__ __forceinline__ bf16_t from_f32<bf16_t>(float x) { return f2bf(x); }

__device__ __forceinline__ float4 to_f4(float4 x) { return x; }
__device__ __forceinline__ float4 to_f4(u32x2 x) {
  return float4{__uint_as_float(x[0] << 16), __uint_as_float(x[0] & 0xffff0000u),
                __uint_as_float(x[1] << 16), __uint_as_float(x[1] & 0xffff0000u)};
}
__device__ __forceinline__ void store4(bf16_t* dst, u32x2 x) { *(u32x2*)dst = x; }
// 8 consecutive elements (16 bytes of bf16, or two 16-byte fp32 loads) as floats
__device__ __forceinline__ void load8v(const bf16_t* p, float* x) {
  const u32x4 w = *(const u32x4*)p;
  unpack8<false>(&w, x);
}
__device__ __forceinline__ void load8v(const float* p, float* x) {
  const float4 a = *(const float4*)p, b = *(const float4*)(p + 4);
  x[0] = a.x; x[1] = a.y; x[2] = a.z; x[3] = a.w; x[4] = b.x; x[5] = b.y; x[6] = b.z; x[7] = b.w;
}

// Row sums of a C-layout tile (lane (q, r) holds rows 16 bi + 4q + v, v = 0..3, of
// column r) added into arr[row], without LDS traffic: a reduce-scatter over the 16 lanes of
// each row group with DPP moves.  Lanes r and r ^ 8 split the four rows between them
// (row_ror:8), lanes r and its mirror in the 8-lane half split the pair (row_half_mirror),
// then each quad sums (quad_perm); lane r with r % 4 == 0 ends with row 16 bi + 4q + r / 4.
__device__ __forceinline__ void add_rows(float* arr, int bi, f32x4 x) {
  const int l = lane_id(), r = l & 15;
  const bool up8 = (r & 8) != 0, up4 = (r & 4) != 0;
  const float k0 = up8 ? x[2] : x[0], k1 = up8 ? x[3] : x[1];
  const float g0 = up8 ? x[0] : x[2], g1 = up8 ? x[1] : x[3];
  const float a0 = k0 + dpp_f<0x128>(g0), a1 = k1 + dpp_f<0x128>(g1);
  const float kb = up4 ? a1 : a0, gb = up4 ? a0 : a1;
  float s = kb + dpp_f<0x141>(gb);
  s += dpp_f<0x4E>(s);
  s += dpp_f<0xB1>(s);
  if ((r & 3) == 0) arr[16 * bi + 4 * (l >> 4) + (r >> 2)] += s;
}
// Column sums of a C-layout tile (column 16 bj + r, summed over its 16 rows) added into
// arr[col]: the lane's four rows, then across the four row groups with the 16- and 32-lane
// swaps (lanes of row group 0 write).
__device__ __forceinline__ void add_cols(float* arr, int bj, f32x4 x) {
  const int l = lane_id();
  float s = x[0] + x[1] + x[2] + x[3];
  const auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(s), __float_as_uint(s), false, false);
  s = __uint_as_float(a[0]) + __uint_as_float(a[1]);
  const auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(s), __float_as_uint(s), false, false);
  s = __uint_as_float(b[0]) + __uint_as_float(b[1]);
  if ((l >> 4) == 0) arr[16 * bj + (l & 15)] += s;
}

// Sum over the 64 lanes, left in every lane (DPP within each row, then the row swaps).
__device__ __forceinline__ float wave_sum(float s) {
  s = group_sum_dpp<16>(s);
  const auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(s), __float_as_uint(s), false, false);
  s = __uint_as_float(a[0]) + __uint_as_float(a[1]);
  const auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(s), __float_as_uint(s), false, false);
  return __uint_as_float(b[0]) + __uint_as_float(b[1]);
}

__device__ __forceinline__ int rec_mode(bool f32) { return f32 ? MODE_F32 : MODE_BF16; }

// Split-matrix operands.  A 64-row fp32 matrix the backward kernels read as MFMA operands
// is kept in LDS as bf16 hi and lo planes (hi + lo is the value to ~2^-16 relative), split
// once when it is written, so no fragment read converts.  op_vec: lane (q, r) gets entries
// k0 + 8q .. +7 of storage row r0 + r (one 16-byte read per plane); op_tr: entries
// k0 + 8q .. +7 down storage column c0 + r (two transposed 8-byte reads per plane).
template <bool LO = true>
__device__ __forceinline__ Op op_vec(const bf16_t* h, const bf16_t* lo, int ld, int r0, int k0) {
  const int l = lane_id();
  const int off = (r0 + (l & 15)) * ld + k0 + 8 * (l >> 4);
  Op o;
  o.h = *(const u32x4*)(h + off);
  if constexpr (LO) o.l = *(const u32x4*)(lo + off);
  else o.l = o.h;
  return o;
}
template <bool LO = true>
__device__ __forceinline__ Op op_tr(const bf16_t* h, const bf16_t* lo, int ld, int c0, int k0) {
  Op o;
  o.h = frag_tr(h, ld, k0, c0);
  if constexpr (LO) o.l = frag_tr(lo, ld, k0, c0);
  else o.l = o.h;
  return o;
}
// A C-layout tile (lane (q, r): rows row0 + 4q .. +3 of column col0 + r) into column-major
// planes (storage [col][row]): one 8-byte write per plane.
__device__ __forceinline__ void put_ct(bf16_t* h, bf16_t* lo, int ld, int row0, int col0, f32x4 c) {
  const int l = lane_id();
  const int off = (col0 + (l & 15)) * ld + row0 + 4 * (l >> 4);
  *(u32x2*)(h + off) = pack_hi4(c);
  *(u32x2*)(lo + off) = pack_lo4(c);
}
// Four consecutive entries (one row, 4 columns from col) into row-major planes.
__device__ __forceinline__ void put_row4(bf16_t* h, bf16_t* lo, int off, f32x4 c) {
  *(u32x2*)(h + off) = pack_hi4(c);
  *(u32x2*)(lo + off) = pack_lo4(c);
}

// op_vec in the block-pair contraction order (kslot<true>): entries k0 + 4q .. +3 and
// k0 + 16 + 4q .. +3 of storage row r0 + r.
__device__ __forceinline__ Op op_pair(const bf16_t* h, const bf16_t* lo, int ld, int r0, int k0) {
  const int l = lane_id();
  const int off = (r0 + (l & 15)) * ld + k0 + 4 * (l >> 4);
  Op o;
  const u32x2 a = *(const u32x2*)(h + off), b = *(const u32x2*)(h + off + 16);
  const u32x2 c = *(const u32x2*)(lo + off), d = *(const u32x2*)(lo + off + 16);
  o.h = u32x4{a[0], a[1], b[0], b[1]};
  o.l = u32x4{c[0], c[1], d[0], d[1]};
  return o;
}
// op_tr in the block-pair contraction order (kslot<true>): entries k0 + 4q .. +3 and
// k0 + 16 + 4q .. +3 down storage column c0 + r
__device__ __forceinline__ Op op_tr_pair(const bf16_t* h, const bf16_t* lo, int ld, int c0, int k0) {
  const int l = lane_id(), q = l >> 4, s = l & 15;
  const int off = (k0 + 4 * q + (s >> 2)) * ld + c0 + 4 * (s & 3);
  const u32x2 a = ds_read_tr(h + off), b = ds_read_tr(h + off + 16 * ld);
  const u32x2 c = ds_read_tr(lo + off), d = ds_read_tr(lo + off + 16 * ld);
  Op o;
  o.h = u32x4{a[0], a[1], b[0], b[1]};
  o.l = u32x4{c[0], c[1], d[0], d[1]};
  return o;
}
// the fp32 values (hi + lo) of an operand's 8 slots
__device__ __forceinline__ void op_values(const Op& o, float* x) {
#pragma unroll
  for (int w = 0; w < 4; ++w) {
    x[2 * w] = __uint_as_float(o.h[w] << 16) + __uint_as_float(o.l[w] << 16);
    x[2 * w + 1] = __uint_as_float(o.h[w] & 0xffff0000u) + __uint_as_float(o.l[w] & 0xffff0000u);
  }
}

// ============================================================================ reverse scan

// index of the lower-triangular 16x16 tile (mb, nb), mb >= nb, of a 64x64 chunk matrix
__device__ __forceinline__ constexpr int ptile_index(int mb, int nb) { return mb * (mb + 1) / 2 + nb; }

// With bf16 inputs (LDR) four loader wavefronts beside the four compute wavefronts move
// each chunk's rows into one of two LDS buffers while the compute wavefronts work on the
// other, and form the chunk's P tiles once for all of them; the compute wavefronts issue
// no loads at all.  Two barriers per chunk: one opens the step (the chunk's rows are
// staged, the other buffer is free), one publishes the P tiles.  fp32 K and Q rows leave
// no room for a second buffer, so with fp32 inputs the compute wavefronts stage the rows
// themselves from a register prefetch two chunks deep.
template <int DK, bool F32>
__global__ __launch_bounds__(F32 ? NT : 2 * NT) void rscan_kernel(BwdParams p) {
  using KT = typename std::conditional<F32, float, bf16_t>::type;
  constexpr int LDK = DK + (F32 ? 4 : 8);
  constexpr int LDB = C + 8;  // stride (bf16) of a split plane
  constexpr bool LDR = !F32;
  // bf16 inputs form the P operands in registers (PREC) from the staged K and Q rows and G
  constexpr bool PREC = !F32;
  // Buffer 0 and (LDR) buffer 1 are separate objects, so the compiler can tell the
  // loaders' writes to one from the compute wavefronts' reads of the other.
  __shared__ __align__(16) KT sK0[C * LDK], sK1[LDR ? C * LDK : 8];
  __shared__ __align__(16) KT sQ0[C * LDK], sQ1[LDR ? C * LDK : 8];
  // dO (this block's 64 columns), X^T and (fp32 inputs) P, row-major, as bf16 hi / lo planes
  __shared__ __align__(16) bf16_t sDO0[2 * C * LDB], sDO1[LDR ? 2 * C * LDB : 8];
  __shared__ __align__(16) bf16_t sX0[2 * C * LDB], sX1[LDR ? 2 * C * LDB : 8];
  __shared__ __align__(16) bf16_t sP[PREC ? 8 : 2 * C * LDB];
  // (LDR) the chunk's ten lower-triangular 16x16 tiles of P, formed once by the loaders:
  // lane l of tile t holds its C-layout values as bf16 hi (2 words) then lo (2 words)
  __shared__ __align__(16) u32x4 sPT[LDR ? 10 : 1][64];
  __shared__ float sGl0[PREC ? C : 1], sGl1[LDR ? C : 1];
  __shared__ __align__(16) float sGate0[4 * C], sGate1[LDR ? 4 * C : 4];
  struct Buf {
    KT* K;
    KT* Q;
    bf16_t* DO;
    bf16_t* X;
    float* Gl;
    float* Gate;
  };
  const Buf B0{sK0, sQ0, sDO0, sX0, sGl0, sGate0};
  const Buf B1{sK1, sQ1, sDO1, sX1, sGl1, sGate1};
  bf16_t* const sPh = sP;
  bf16_t* const sPl = sP + C * LDB;

  const int tid = threadIdx.x, l = tid & 63, lq = l >> 4, lr = l & 15;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const bool loader = LDR && wave >= NT / 64;  // (LDR) waves 4-7: rows and P tiles only
  const int st = loader ? tid - NT : tid;       // index among the threads that stage rows
  const ScanItem item = scan_item(p.seq_order, p.N, p.Hk, p.Hv, p.nb);
  const int blk = item.blk, h = item.h, n = item.n;
  const int gqa = p.Hv / p.Hk, hk = h / gqa;
  const int DV = p.DV, col0 = 64 * blk, c = 16 * wave;
  long long s0, s1;
  seq_range(p.cu_seqlens, n, p.T, s0, s1);
  const int nchunks = (int)((s1 - s0 + C - 1) / C);
  const int cbase = p.chunk_off ? p.chunk_off[n] : n * p.nch;
  const size_t rec_stride = (size_t)rec_bytes(rec_mode(F32), true);
  const long long rs = (long long)p.Hv * DV;  // row stride of dO / dV_new

  // dS[t][v] = dS[16t + 4lq + v][col0 + c + lr]: gradient of the state leaving the chunk
  f32x4 dS[DK / 16];
  const size_t st_off = ((size_t)n * p.Hv + h) * DK * DV + col0 + c + lr;
  auto init_dS = [&]() {
#pragma unroll
    for (int t = 0; t < DK / 16; ++t)
#pragma unroll
      for (int v = 0; v < 4; ++v)
        dS[t][v] = p.dht ? p.dht[st_off + (size_t)(16 * t + 4 * lq + v) * DV] : 0.f;
  };
  // gradient of the initial state
  auto write_dh0 = [&]() {
    if (p.dh0) {
#pragma unroll
      for (int t = 0; t < DK / 16; ++t)
#pragma unroll
        for (int v = 0; v < 4; ++v) p.dh0[st_off + (size_t)(16 * t + 4 * lq + v) * DV] = dS[t][v];
    }
  };

  // Per-thread register copy of a chunk's inputs: K and Q rows, the chunk's dO columns,
  // X and P, and one gate value, loaded by the NT staging threads (the loaders, or with
  // fp32 inputs the compute wavefronts, two register sets deep) and stored into LDS a
  // chunk step later.
  constexpr int NKQ = 2 * C * (DK / 4) / NT;
  static_assert(NKQ * NT == 2 * C * (DK / 4), "item split");
  struct Pf {
    typename Vec4<KT>::type pkq[NKQ];
    float4 pdo[C * 16 / NT], pxp[(PREC ? 1 : 2) * C * 16 / NT];
    float pgate, pg;
  };
  // chunk jj into f; every call issues the same loads (a chunk before the sequence's first
  // reloads chunk 0, unused), so the loop's waits stay exact counts
  auto load_chunk = [&](int jj, Pf& f) {
    jj = jj < 0 ? 0 : jj;
    const long long tt = s0 + (long long)jj * C;
    const int nv = (int)((s1 - tt) < C ? (s1 - tt) : C);
    const int sl = cbase + jj < p.n_rec ? cbase + jj : p.n_rec - 1;
    // the chunk's valid rows only (zeros past them)
    const auto kr = buf_rsrc((const KT*)p.ks + tt * p.ks_ld + (long long)hk * DK,
                             (unsigned)(nv * p.ks_ld * (long long)sizeof(KT)));
    const auto qr = buf_rsrc((const KT*)p.qs + tt * p.qs_ld + (long long)hk * DK,
                             (unsigned)(nv * p.qs_ld * (long long)sizeof(KT)));
    const auto dr = buf_rsrc(p.dO + tt * rs + (long long)h * DV + col0, (unsigned)(4 * nv * rs));
    static_assert((C * DK / 4) % NT == 0, "a K / Q item's matrix follows from m alone");
#pragma unroll
    for (int m = 0; m < NKQ; ++m) {
      const int which = m * NT / (C * DK / 4);  // uniform: K items, then Q items
      const int rem = st + m * NT - which * (C * DK / 4);
      const int row = rem / (DK / 4), c4 = 4 * (rem % (DK / 4));
      const long long ld = which ? p.qs_ld : p.ks_ld;
      f.pkq[m] = bload4(which ? qr : kr, (unsigned)((row * ld + c4) * (long long)sizeof(KT)), (const KT*)nullptr);
    }
#pragma unroll
    for (int m = 0; m < C * 16 / NT; ++m) {
      const int it = st + m * NT;
      const int row = it >> 4, c4 = 4 * (it & 15);
      f.pdo[m] = bload4(dr, (unsigned)(4 * (row * rs + c4)), (const float*)nullptr);
    }
    const float* xb = p.xlpg + ((size_t)sl * p.Hv + h) * kXlpgFloats;
#pragma unroll
    for (int m = 0; m < (PREC ? 1 : 2) * C * 16 / NT; ++m) {
      const int it = st + m * NT;
      const int which = it / (C * 16), rem = it % (C * 16);
      f.pxp[m] = load4(xb + (which ? kXlpgP : kXlpgX) + (rem >> 4) * C + 4 * (rem & 15));
    }
    if constexpr (PREC) f.pg = xb[kXlpgG + (st & (C - 1))];
    f.pgate = ((const float*)(p.rec + ((size_t)sl * p.Hv + h) * rec_stride + kRecG))[st];
  };
  auto store_chunk = [&](const Pf& f, const Buf& bf) {
    bf16_t* const sDOh = bf.DO;
    bf16_t* const sDOl = bf.DO + C * LDB;
    bf16_t* const sXh = bf.X;
    bf16_t* const sXl = bf.X + C * LDB;
#pragma unroll
    for (int m = 0; m < NKQ; ++m) {
      const int it = st + m * NT;
      const int which = it / (C * DK / 4), rem = it % (C * DK / 4);
      const int row = rem / (DK / 4), c4 = 4 * (rem % (DK / 4));
      store4((which ? bf.Q : bf.K) + row * LDK + c4, f.pkq[m]);
    }
#pragma unroll
    for (int m = 0; m < C * 16 / NT; ++m) {
      const int it = st + m * NT;
      put_row4(sDOh, sDOl, (it >> 4) * LDB + 4 * (it & 15), f32x4{f.pdo[m].x, f.pdo[m].y, f.pdo[m].z, f.pdo[m].w});
    }
#pragma unroll
    for (int m = 0; m < (PREC ? 1 : 2) * C * 16 / NT; ++m) {
      const int it = st + m * NT;
      const int which = it / (C * 16), rem = it % (C * 16);
      const f32x4 v = f32x4{f.pxp[m].x, f.pxp[m].y, f.pxp[m].z, f.pxp[m].w};
      if (which) put_row4(sPh, sPl, (rem >> 4) * LDB + 4 * (rem & 15), v);
      else put_row4(sXh, sXl, (rem >> 4) * LDB + 4 * (rem & 15), v);
    }
    if constexpr (PREC)
      if (st < C) bf.Gl[st] = f.pg;
    bf.Gate[st] = f.pgate;
  };
  // (LDR) tile (mb, nb) of P = lower(scale Q K^T * Gamma) in the C layout, from the rows
  // staged in bf, with the preparation kernel's arithmetic:
  // scale * acc * 2^{min(G_m log2 e - G_n log2 e, 0)} * mask
  auto form_ptile = [&](int mb, int nb, const Buf& bf) {
    f32x4 acc = zero4();
#pragma unroll
    for (int s2 = 0; s2 < DK / 32; ++s2)
      acc = mma16(frag_bf16((const bf16_t*)bf.Q, LDK, 16 * mb, 32 * s2),
                  frag_bf16((const bf16_t*)bf.K, LDK, 16 * nb, 32 * s2), acc);
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      const int m = 16 * mb + 4 * lq + v, n = 16 * nb + lr;
      acc[v] = p.scale * acc[v] *
               __builtin_amdgcn_exp2f(fminf(bf.Gl[m] * 1.4426950408889634f - bf.Gl[n] * 1.4426950408889634f, 0.f)) *
               (float)(m >= n);
    }
    return acc;
  };
  // (LDR) the ten tiles, dealt over the four loaders (t = lw, lw + 4, lw + 8), into sPT
  auto form_ptiles = [&](const Buf& bf) {
    const int lw = wave - NT / 64;
    for (int t = lw; t < 10; t += 4) {  // uniform per wavefront
      const int mb = t < 1 ? 0 : t < 3 ? 1 : t < 6 ? 2 : 3;
      const int nb = t - mb * (mb + 1) / 2;
      const f32x4 x = form_ptile(mb, nb, bf);
      const u32x2 hi = pack_hi4(x), lo = pack_lo4(x);
      sPT[t][l] = u32x4{hi[0], hi[1], lo[0], lo[1]};
    }
  };
  // chunk j on the compute wavefronts, from the rows staged in bf
  auto compute = [&](const int j, const Buf& bf) {
    const long long t0 = s0 + (long long)j * C;
    const int nvalid = (int)((s1 - t0) < C ? (s1 - t0) : C);
    const int slot = cbase + j < p.n_rec ? cbase + j : p.n_rec - 1;
    const KT* const sK = bf.K;
    const KT* const sQ = bf.Q;
    const bf16_t* const sDOh = bf.DO;
    const bf16_t* const sDOl = bf.DO + C * LDB;
    const bf16_t* const sXh = bf.X;
    const bf16_t* const sXl = bf.X + C * LDB;
    const float* const sGate = bf.Gate;
    const float* sEG = sGate + kGateEG * C;
    const float* sEGS = sGate + kGateEGS * C;
    const float* sEL = sGate + kGateEL * C;  // e^{G_last - G}; e^{G_last} in the last slot
    const float* sB = sGate + kGateBeta * C;

    // gradient of the state leaving chunk j, for the chunk-local gradients
    {
      // column-major per state ([dv][dk]): a lane's 4 rows of a tile are contiguous
      float* dd = p.dstates + ((size_t)slot * p.Hv + h) * DK * DV + (size_t)(col0 + c + lr) * DK;
#pragma unroll
      for (int t = 0; t < DK / 16; ++t) *(f32x4*)(dd + 16 * t + 4 * lq) = dS[t];
    }

    // ---------------------------------------------------------------- K dS
    Op dsb[DK / 32];
#pragma unroll
    for (int s = 0; s < DK / 32; ++s) dsb[s] = join_op(dS[2 * s], dS[2 * s + 1]);
    f32x4 kds[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      f32x4 acc = zero4();
#pragma unroll
      for (int s = 0; s < DK / 32; ++s) {
        acc = mm3<F32, true>(acc, kq_row<true>(sK, LDK, 16 * i, 32 * s), dsb[s]);
      }
      kds[i] = acc;
    }
    // (LDR) the loaders' P tiles of this chunk are in sPT after this barrier
    if constexpr (LDR) lds_barrier();
    // ---------------------------------------------------------------- dV_new = P^T dO + e^{G_last-G} K dS
    f32x4 dvn[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      f32x4 acc = zero4();
#pragma unroll
      for (int p2 = i / 2; p2 < 2; ++p2) {  // P^T is upper triangular
        if constexpr (PREC) {
          // P^T rows 16i .. +15 over tokens 32 p2 .. +31 from the P tiles (2 p2, i) and
          // (2 p2 + 1, i) side by side (block-pair order; (2 p2, i) is above the diagonal,
          // zero, when 2 p2 < i), against dO read in the same order
          const u32x4 tb = sPT[ptile_index(2 * p2 + 1, i)][l];
          const u32x4 ta = 2 * p2 >= i ? sPT[ptile_index(2 * p2, i)][l] : u32x4{0u, 0u, 0u, 0u};
          Op pt;
          pt.h = u32x4{ta[0], ta[1], tb[0], tb[1]};
          pt.l = u32x4{ta[2], ta[3], tb[2], tb[3]};
          acc = mm3<true, true>(acc, pt, op_tr_pair(sDOh, sDOl, LDB, c, 32 * p2));
        } else {
          acc = mm3<true, true>(acc, op_tr(sPh, sPl, LDB, 16 * i, 32 * p2),
                                op_tr(sDOh, sDOl, LDB, c, 32 * p2));
        }
      }
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        const int row = 16 * i + 4 * lq + v;
        const float el = row == C - 1 ? 1.f : sEL[row];
        dvn[i][v] = acc[v] + el * kds[i][v];
      }
    }
    {
      // rows at or past nvalid lie outside the buffer range and are dropped: no branch
      const auto vd = buf_rsrc(p.dvnew + t0 * rs + (long long)h * DV + col0,
                               4u * (unsigned)nvalid * (unsigned)rs);
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int v = 0; v < 4; ++v)
          __builtin_amdgcn_raw_buffer_store_b32(
              __float_as_uint(dvn[i][v]), vd,
              4u * ((unsigned)(16 * i + 4 * lq + v) * (unsigned)rs + (unsigned)(c + lr)), 0, 0);
    }
    // ---------------------------------------------------------------- Y = diag(beta) X^T dV_new
    Op dvp[2];
#pragma unroll
    for (int pp = 0; pp < 2; ++pp) dvp[pp] = join_op(dvn[2 * pp], dvn[2 * pp + 1]);
    f32x4 y[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      f32x4 acc = zero4();
#pragma unroll
      for (int p2 = i / 2; p2 < 2; ++p2)  // X^T is upper triangular; X^T rows (stored transposed)
        acc = mm3<true, true>(acc, op_pair(sXh, sXl, LDB, 16 * i, 32 * p2), dvp[p2]);
#pragma unroll
      for (int v = 0; v < 4; ++v) y[i][v] = sB[16 * i + 4 * lq + v] * acc[v];
    }
    // ---------------------------------------------------------------- dS update
    Op b1[2], b2[2];
#pragma unroll
    for (int p2 = 0; p2 < 2; ++p2) {
      float x[8];
      op_values(op_tr(sDOh, sDOl, LDB, c, 32 * p2), x);
#pragma unroll
      for (int e = 0; e < 8; ++e) x[e] *= sEGS[32 * p2 + 8 * lq + e];
      b1[p2] = split8(x);
      f32x4 ya, yb;
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        ya[v] = -sEG[32 * p2 + 4 * lq + v] * y[2 * p2][v];
        yb[v] = -sEG[32 * p2 + 16 + 4 * lq + v] * y[2 * p2 + 1][v];
      }
      b2[p2] = join_op(ya, yb);
    }
    const float egl = sEL[C - 1];
#pragma unroll
    for (int t = 0; t < DK / 16; ++t) {
      f32x4 acc;
#pragma unroll
      for (int v = 0; v < 4; ++v) acc[v] = egl * dS[t][v];
#pragma unroll
      for (int p2 = 0; p2 < 2; ++p2) {
        acc = mm3<F32, true>(acc, kq_col<false>(sQ, LDK, 16 * t, 32 * p2), b1[p2]);
        acc = mm3<F32, true>(acc, kq_col<true>(sK, LDK, 16 * t, 32 * p2), b2[p2]);
      }
      dS[t] = acc;
    }
  };
  // Barriers here order LDS accesses only (lds_barrier): the global stores go to later
  // kernels and the staged rows come from per-thread registers, so neither the loads nor
  // the stores are waited for at a barrier.
  if constexpr (LDR) {
    // Chunk j is computed from one buffer while the loaders store chunk j - 1, loaded
    // during the step before, into the other and load chunk j - 2 (a chunk below the
    // sequence's first reloads chunk 0, unused): the barrier that opens a step finds the
    // next buffer filled and the previous one read.  The two roles run separate loops
    // with the same two barriers per step, so neither holds the other's registers.
    int j = nchunks - 1;
    if (loader) {
      Pf f;
      if (nchunks > 0) {
        load_chunk(nchunks - 1, f);
        store_chunk(f, B0);
        load_chunk(nchunks - 2, f);
      }
      // the P tiles of the chunk the compute wavefronts work on, published by the
      // step's second barrier, then the next chunk's rows
      auto lstep = [&](const Buf& cur, const Buf& nxt, const int jj) {
        lds_barrier();
        form_ptiles(cur);
        lds_barrier();
        store_chunk(f, nxt);
        load_chunk(jj - 2, f);
      };
      for (; j >= 1; j -= 2) {
        lstep(B0, B1, j);
        lstep(B1, B0, j - 1);
      }
      if (j == 0) lstep(B0, B1, 0);
    } else {
      init_dS();
      // the prologue's loads under the uniform p.dht test have landed
      __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0)
      auto cstep = [&](const int jj, const Buf& cur) {
        lds_barrier();
        compute(jj, cur);
      };
      for (; j >= 1; j -= 2) {
        cstep(j, B0);
        cstep(j - 1, B1);
      }
      if (j == 0) cstep(0, B0);
      write_dh0();
    }
  } else {
    init_dS();
    Pf pfa, pfb;
    if (nchunks > 0) {
      load_chunk(nchunks - 1, pfa);
      load_chunk(nchunks - 2, pfb);
    }
    // the prologue's loads (some under the uniform p.dht test) have landed: the loop's
    // waits then count only the loop's own memory operations
    __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0)
    // chunk j from the registers of cur, which then receive chunk jn (lands during this
    // chunk and the next)
    auto step = [&](const int jj, Pf& cur, const int jn) {
      lds_barrier();  // the previous chunk's readers are done
      store_chunk(cur, B0);
      load_chunk(jn, cur);
      lds_barrier();
      compute(jj, B0);
    };
    // chunks n-1, n-3, ... from pfa and n-2, n-4, ... from pfb, each set reloaded with the
    // chunk two below the one it held
    int j = nchunks - 1;
    for (; j >= 1; j -= 2) {
      step(j, pfa, j - 2);
      step(j - 1, pfb, j - 3);
    }
    if (j == 0) step(0, pfa, -2);
    write_dh0();
  }
}

// ============================================================================ chunk-local gradients

// Eight wavefronts (two per SIMD: the LDS holds one workgroup per CU).  Wavefront w owns
// dk column blocks w + 8m and dv column blocks w + 8m of the (chunk x head) gradients,
// and of the 64x64 chunk matrices row block w % 4, column blocks 2 (w / 4) and
// 2 (w / 4) + 1.
constexpr int CW = 8, CNT = 64 * CW;

template <int DK, int DV, bool F32>
__global__ __launch_bounds__(CNT) void cgrad_kernel(BwdParams p) {
  using KT = typename std::conditional<F32, float, bf16_t>::type;
  using In = KT;  // v has the input precision too
  constexpr int LDK = DK + (F32 ? 4 : 8);
  constexpr int LDB = C + 8;  // stride (bf16) of a split plane: 64 entries and a pad
  constexpr int NCB = DK / 16, NKB = (NCB + CW - 1) / CW;  // dk column blocks; per wavefront
  constexpr int NVB = DV / 16, NVW = (NVB + CW - 1) / CW;  // dv column blocks; per wavefront
  __shared__ __align__(16) KT sK[C * LDK];
  __shared__ __align__(16) KT sQ[C * LDK];
  // split planes (hi, lo): dW column-major [dk][token], dPg column-major
  __shared__ __align__(16) bf16_t sDW[2 * DK * LDB];
  __shared__ __align__(16) bf16_t sDP[2 * C * LDB];
  // X (row-major), dX and M1 / Qm (column-major), split; during the products over dv the
  // region stages their operand rows
  __shared__ __align__(16) bf16_t sR[3 * 2 * C * LDB];
  bf16_t* const sXh = sR;
  bf16_t* const sXl = sR + C * LDB;
  bf16_t* const sDXh = sR + 2 * C * LDB;
  bf16_t* const sDXl = sR + 3 * C * LDB;
  bf16_t* const sMh = sR + 4 * C * LDB;
  bf16_t* const sMl = sR + 5 * C * LDB;
  bf16_t* const sDWh = sDW;
  bf16_t* const sDWl = sDW + DK * LDB;
  bf16_t* const sDPh = sDP;
  bf16_t* const sDPl = sDP + C * LDB;
  __shared__ float sG[C], sBt[C];
  // per-wavefront partial row / column sums (deterministic: one writer per entry at a time)
  __shared__ float sRowG[CW][C], sColG[CW][C], sRowB[CW][C], sRowT[CW][C], sRP[CW][C];
  __shared__ float sRed[CW];

  const int tid = threadIdx.x, l = tid & 63, lq = l >> 4, lr = l & 15;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int Hv = p.Hv, h = blockIdx.x % Hv, ci = blockIdx.x / Hv;
  int n, cc;
  if (p.chunk_off) {
    if (ci >= p.chunk_off[p.N]) return;
    int lo = 0, hi = p.N;
    while (hi - lo > 1) {
      const int mid = (lo + hi) >> 1;
      if (p.chunk_off[mid] <= ci) lo = mid;
      else hi = mid;
    }
    n = lo;
    cc = ci - p.chunk_off[lo];
  } else {
    n = ci / p.nch;
    cc = ci % p.nch;
  }
  long long s0, s1;
  seq_range(p.cu_seqlens, n, p.T, s0, s1);
  const long long t0 = s0 + (long long)cc * C;
  const int nvalid = (int)((s1 - t0) < C ? (s1 - t0) : C);
  if (nvalid <= 0) return;
  const int gqa = Hv / p.Hk, hk = h / gqa;
  const size_t rec_stride = (size_t)rec_bytes(rec_mode(F32), true);
  const float* xb = p.xlpg + ((size_t)ci * Hv + h) * kXlpgFloats;
  const float* Sg = p.states + ((size_t)ci * Hv + h) * DK * DV;
  const float* dSg = p.dstates + ((size_t)ci * Hv + h) * DK * DV;
  const long long rs = (long long)Hv * DV;  // row stride of dO, V_new, dV_new, v
  const float* dOb = p.dO + t0 * rs + (long long)h * DV;
  const float* Vnb = p.vnew + t0 * rs + (long long)h * DV;
  const float* dVnb = p.dvnew + t0 * rs + (long long)h * DV;
  const In* vb = (const In*)p.v + t0 * rs + (long long)h * DV;
  const float scale = p.scale;

  // (the gates and the K, Q rows are staged just before the products over dv, together
  // with the first step's loads)
  auto eg = [&](int row) { return __expf(sG[row]); };
  auto el = [&](int row) { return row == C - 1 ? 1.f : __expf(sG[C - 1] - sG[row]); };
  auto gam = [&](int row, int col) {
    return row >= col ? __expf(fminf(sG[row] - sG[col], 0.f)) : 0.f;
  };
  float* rowG = sRowG[wave];
  float* colG = sColG[wave];
  float* rowB = sRowB[wave];
  float* rowT = sRowT[wave];
  float* rP = sRP[wave];

  // dq, dk accumulators of the wavefront's dk column blocks cb = wave + 4 kb
  f32x4 dq[NKB][4], dk[NKB][4];

  // ---------------------------------------------------------------- products over dv
  // One pass over dv in 32-column steps:
  //   X1 = diag(e^G) dO S^T, dW = -dV_new S^T, dkdec = V_new dS^T (the wavefront's dk
  //   column blocks), dP = (dO V_new^T) * tril and dXa = dV_new v^T (its row block bi,
  //   column blocks 2 half, 2 half + 1).
  // The step's dO, dV_new, V_new and v rows are staged in LDS as split planes (one
  // coalesced float4 per thread each, split once) and the state fragments come straight
  // from global memory; both are loaded into registers one step ahead.
  constexpr int LDR = 40;  // stride (bf16) of a staged 32-column slice plane
  static_assert(8 * C * LDR <= 6 * C * LDB, "the staged slices fit the X / dX / M1 region");
  bf16_t* const sDOh = sR;
  bf16_t* const sDOl = sR + C * LDR;
  bf16_t* const sDVh = sR + 2 * C * LDR;
  bf16_t* const sDVl = sR + 3 * C * LDR;
  bf16_t* const sVNh = sR + 4 * C * LDR;
  bf16_t* const sVNl = sR + 5 * C * LDR;
  bf16_t* const sVh = sR + 6 * C * LDR;  // v: exact in bf16 unless the inputs are fp32
  bf16_t* const sVl = sR + 7 * C * LDR;
  const int srow = tid >> 3, sc4 = 4 * (tid & 7);  // this thread's staged item
  float4 pf_do, pf_dv, pf_vn;
  typename Vec4<In>::type pf_v;
  // the chunk's valid rows of dO, dV_new, V_new and v (zeros past them)
  const unsigned rows_b = (unsigned)(nvalid * rs);  // elements
  const auto rDO = buf_rsrc(dOb, 4u * rows_b), rDV = buf_rsrc(dVnb, 4u * rows_b);
  const auto rVN = buf_rsrc(Vnb, 4u * rows_b), rV = buf_rsrc(vb, (unsigned)sizeof(In) * rows_b);
  auto load_rows = [&](int u) {
    const unsigned off = (unsigned)(srow * rs + 32 * u + sc4);
    pf_do = bload4(rDO, 4u * off, (const float*)nullptr);
    pf_dv = bload4(rDV, 4u * off, (const float*)nullptr);
    pf_vn = bload4(rVN, 4u * off, (const float*)nullptr);
    pf_v = bload4(rV, (unsigned)sizeof(In) * off, (const In*)nullptr);
  };
  auto f4 = [](float4 x) { return f32x4{x.x, x.y, x.z, x.w}; };
  auto store_rows = [&]() {
    const int o = srow * LDR + sc4;
    put_row4(sDOh, sDOl, o, f4(pf_do));
    put_row4(sDVh, sDVl, o, f4(pf_dv));
    put_row4(sVNh, sVNl, o, f4(pf_vn));
    if constexpr (F32) put_row4(sVh, sVl, o, f4(to_f4(pf_v)));
    else *(u32x2*)(sVh + o) = *(const u32x2*)&pf_v;
  };
  float sfr[NKB][8], dfr[NKB][8];  // state fragments (the states are column-major)
  float sds = 0.f;  // sum of dS_end * S over the state (each element is loaded once here)
  auto load_state = [&](int u) {
#pragma unroll
    for (int kb = 0; kb < NKB; ++kb) {
      // unconditional (a block past NCB reloads the last one, unused): see the dv loop
      const int cb = wave + CW * kb < NCB ? wave + CW * kb : NCB - 1;
      gfrag_col(Sg, DK, 16 * cb + lr, 32 * u, sfr[kb]);
      gfrag_col(dSg, DK, 16 * cb + lr, 32 * u, dfr[kb]);
    }
  };
  float4 pf_x[C * 16 / CNT];  // X, staged after the last step
  f32x4 dw[NKB][4], dp[2], dxa[2];
#pragma unroll
  for (int kb = 0; kb < NKB; ++kb)
#pragma unroll
    for (int i = 0; i < 4; ++i) dq[kb][i] = dk[kb][i] = dw[kb][i] = zero4();
#pragma unroll
  for (int j = 0; j < 2; ++j) dp[j] = dxa[j] = zero4();
  const int bi = wave & 3, half = wave >> 2;  // row block and column-block pair
  // P and Lg at this wavefront's tiles (bi, 2 half + jj), used elementwise after the
  // products over dv.  fp32 inputs read them from the preparation kernel's matrices; bf16
  // inputs form them after the products over dv from the staged K and Q rows.
  float pP[2][4], pLg[2][4];
  if constexpr (F32) {
#pragma unroll
    for (int jj = 0; jj < 2; ++jj)
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        const int o = (16 * bi + 4 * lq + v) * C + 16 * (2 * half + jj) + lr;
        pP[jj][v] = xb[kXlpgP + o];
        pLg[jj][v] = xb[kXlpgLg + o];
      }
  }
  // ---------------------------------------------------------------- stage
  // K and Q rows in 16-byte items, every load issued (with the first step's) before any
  // store, so the workgroup waits for one memory round trip rather than one per item
  {
    constexpr int EPI = 16 / (int)sizeof(KT);  // elements per item
    constexpr int PER = C * DK / EPI;          // items per matrix
    constexpr int NIT = 2 * PER / CNT;
    static_assert(NIT * CNT == 2 * PER, "staging split");
    // the chunk's valid rows only (zeros past them, no branch: see bload4)
    static_assert(PER % CNT == 0, "an item's matrix follows from m alone");
    const auto kr = buf_rsrc((const KT*)p.ks + t0 * p.ks_ld + (long long)hk * DK,
                             (unsigned)(nvalid * p.ks_ld * (long long)sizeof(KT)));
    const auto qr = buf_rsrc((const KT*)p.qs + t0 * p.qs_ld + (long long)hk * DK,
                             (unsigned)(nvalid * p.qs_ld * (long long)sizeof(KT)));
    u32x4 st[NIT];
#pragma unroll
    for (int m = 0; m < NIT; ++m) {
      const int which = m * CNT / PER;  // uniform: K items, then Q items
      const int rem = tid + m * CNT - which * PER;
      const int row = rem / (DK / EPI), c = EPI * (rem % (DK / EPI));
      const long long ld = which ? p.qs_ld : p.ks_ld;
      st[m] = __builtin_amdgcn_raw_buffer_load_b128(which ? qr : kr,
                                                    (unsigned)((row * ld + c) * (long long)sizeof(KT)), 0, 0);
    }
    load_rows(0);
    load_state(0);
    if (tid < C) {
      sG[tid] = xb[kXlpgG + tid];
      sBt[tid] = ((const float*)(p.rec + ((size_t)ci * Hv + h) * rec_stride + kRecG))[kGateBeta * C + tid];
    }
    sRowG[wave][l] = 0.f;
    sColG[wave][l] = 0.f;
    sRowB[wave][l] = 0.f;
    sRowT[wave][l] = 0.f;
    sRP[wave][l] = 0.f;
#pragma unroll
    for (int m = 0; m < NIT; ++m) {
      const int it = tid + m * CNT;
      const int which = it / PER, rem = it % PER;
      const int row = rem / (DK / EPI), c = EPI * (rem % (DK / EPI));
      *(u32x4*)((which ? sQ : sK) + row * LDK + c) = st[m];
    }
  }
  // (the barrier at the top of the first step orders the staging before every read)
  // not unrolled: with every fragment a plain LDS read, an unrolled loop lets the
  // scheduler hoist the reads of several steps and run out of registers
#pragma unroll 1
  for (int u = 0; u < DV / 32; ++u) {
    // (every barrier in this kernel orders LDS accesses only, as in the reverse scan)
    lds_barrier();  // the previous step's readers are done
    store_rows();
    Op bs[NKB], bd[NKB];
#pragma unroll
    for (int kb = 0; kb < NKB; ++kb) {
      bs[kb] = split8(sfr[kb]);
      bd[kb] = split8(dfr[kb]);
      if (wave + CW * kb < NCB) {
#pragma unroll
        for (int e = 0; e < 8; ++e) sds += sfr[kb][e] * dfr[kb][e];
      }
    }
    // The next step's loads, issued after this step's values are consumed (split and summed
    // above) and unconditionally (the last step reloads its own slices, unused; X's rows,
    // needed after the loop, load every step): loaded under a branch or hoisted above that
    // use, they would need other registers than the ones the loop carries, and the copies at
    // the end of the step would wait for them, turning the prefetch into a stall.
    __builtin_amdgcn_sched_barrier(0);
    {
      const int un = u + 1 < DV / 32 ? u + 1 : u;
      load_rows(un);
      load_state(un);
#pragma unroll
      for (int m = 0; m < C * 16 / CNT; ++m) {
        const int it = tid + m * CNT;
        pf_x[m] = load4(xb + kXlpgX + (it >> 4) * C + 4 * (it & 15));
      }
    }
    lds_barrier();
    const Op ow = op_vec(sDOh, sDOl, LDR, 16 * bi, 0);  // dO and dV_new rows of block bi
    const Op vw = op_vec(sDVh, sDVl, LDR, 16 * bi, 0);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const Op ao = op_vec(sDOh, sDOl, LDR, 16 * i, 0);
      const Op adv = op_vec(sDVh, sDVl, LDR, 16 * i, 0);
      const Op avn = op_vec(sVNh, sVNl, LDR, 16 * i, 0);
#pragma unroll
      for (int kb = 0; kb < NKB; ++kb) {
        if (wave + CW * kb >= NCB) continue;
        dq[kb][i] = mm3<true, true>(dq[kb][i], ao, bs[kb]);    // dO S^T
        dw[kb][i] = mm3<true, true>(dw[kb][i], adv, bs[kb]);   // dV_new S^T
        dk[kb][i] = mm3<true, true>(dk[kb][i], avn, bd[kb]);   // V_new dS^T
      }
      if ((i >> 1) == half) {
        const Op av = op_vec<F32>(sVh, sVl, LDR, 16 * i, 0);
        dxa[i & 1] = mm3<true, F32>(dxa[i & 1], vw, av);              // dV_new v^T
        if (i <= bi) dp[i & 1] = mm3<true, true>(dp[i & 1], ow, avn);  // dO V_new^T
      }
    }
  }
  lds_barrier();  // every read of the staged slices is done: the region now holds X
#pragma unroll
  for (int m = 0; m < C * 16 / CNT; ++m) {
    const int it = tid + m * CNT;
    put_row4(sXh, sXl, (it >> 4) * LDB + 4 * (it & 15), f4(pf_x[m]));
  }
  if constexpr (!F32) {
    // P = lower(scale Q K^T * Gamma) and Lg = strict_lower(K K^T * Gamma) at this
    // wavefront's tiles, with the preparation kernel's arithmetic (the exact bf16 products
    // summed by the same MFMA over the same dk blocks in the same order, then
    // scale * acc * 2^{min(G_i log2 e - G_m log2 e, 0)} * mask), so they are the values it
    // left in its matrices, without storing and reloading 32 KiB per (chunk, value head)
#pragma unroll
    for (int jj = 0; jj < 2; ++jj) {
      const int bj = 2 * half + jj;
      f32x4 kk = zero4(), qk = zero4();
#pragma unroll
      for (int s2 = 0; s2 < DK / 32; ++s2) {
        const u32x4 km = frag_bf16((const bf16_t*)sK, LDK, 16 * bj, 32 * s2);
        kk = mma16(frag_bf16((const bf16_t*)sK, LDK, 16 * bi, 32 * s2), km, kk);
        qk = mma16(frag_bf16((const bf16_t*)sQ, LDK, 16 * bi, 32 * s2), km, qk);
      }
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        const int row = 16 * bi + 4 * lq + v, col = 16 * bj + lr;
        const float e = __builtin_amdgcn_exp2f(
            fminf(sG[row] * 1.4426950408889634f - sG[col] * 1.4426950408889634f, 0.f));
        pLg[jj][v] = kk[v] * e * (float)(row > col);
        pP[jj][v] = scale * qk[v] * e * (float)(row >= col);
      }
    }
  }
#pragma unroll
  for (int kb = 0; kb < NKB; ++kb) {
    const int cb = wave + CW * kb;
    if (cb >= NCB) continue;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      f32x4 gx, rr;
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        const int row = 16 * i + 4 * lq + v, col = 16 * cb + lr;
        dq[kb][i][v] *= eg(row);                           // X1 = diag(e^G) dO S^T
        gx[v] = scale * ldx(sQ + row * LDK + col) * dq[kb][i][v];
        const float e = el(row);
        rr[v] = dk[kb][i][v] * ldx(sK + row * LDK + col) * e;  // dkdec * kdec
        dk[kb][i][v] *= e;
      }
      put_ct(sDWh, sDWl, LDB, 16 * i, 16 * cb, -dw[kb][i]);  // dW = -dV_new S^T
      add_rows(rowG, i, gx);
      add_rows(rP, i, rr);
    }
  }
#pragma unroll
  for (int jj = 0; jj < 2; ++jj) {
    const int bj = 2 * half + jj;
    f32x4 pdp, dpg;
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      const int row = 16 * bi + 4 * lq + v, col = 16 * bj + lr;
      const float d = row >= col ? dp[jj][v] : 0.f;
      pdp[v] = d * pP[jj][v];
      dpg[v] = d * gam(row, col);                          // dPg = dP * Gamma
    }
    put_ct(sDPh, sDPl, LDB, 16 * bi, 16 * bj, dpg);
    add_rows(rowG, bi, pdp);
    add_cols(colG, bj, -pdp);
  }
  // sum of dS_end * S over the state (the e^{G_last} S term of the state update)
  sds = wave_sum(sds);
  if (l == 0) sRed[wave] = sds;
  lds_barrier();

  // ---------------------------------------------------------------- dX = dU vb^T + dW kbe^T
  {
#pragma unroll
    for (int jj = 0; jj < 2; ++jj) {
      const int bj = 2 * half + jj;
      f32x4 acc = zero4();
#pragma unroll
      for (int s = 0; s < DK / 32; ++s)
        acc = mm3<true, F32>(acc, op_tr(sDWh, sDWl, LDB, 16 * bi, 32 * s),
                             kq_row<false>(sK, LDK, 16 * bj, 32 * s));
      const int col = 16 * bj + lr;
      const float bc = sBt[col], ec = eg(col);
      f32x4 dx;
#pragma unroll
      for (int v = 0; v < 4; ++v) dx[v] = bc * (dxa[jj][v] + ec * acc[v]);
      put_ct(sDXh, sDXl, LDB, 16 * bi, 16 * bj, dx);
    }
  }
  lds_barrier();

  // ---------------------------------------------------------------- dvb = X^T dU, dkbe = X^T dW
#pragma unroll
  for (int kv = 0; kv < NVW; ++kv) {
    const int cv = wave + CW * kv;
    if (cv >= NVB) continue;
    // the column's dV_new fragments (one per 32-token half, shared by every row block).
    // dvb is formed transposed, dvb^T = dV_new^T X (the fragments serve as A operands and
    // the X^T rows as B operands), so a lane holds 4 consecutive columns of one row: v is
    // read and dv written 4 columns at a time.
    Op bo[2];
    {
      float b[8];
      gfrag_col_b(rDV, (unsigned)rs, 16 * cv + lr, 0, b);
      bo[0] = split8(b);
      gfrag_col_b(rDV, (unsigned)rs, 16 * cv + lr, 32, b);
      bo[1] = split8(b);
    }
    typename Vec4<In>::type vv4[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int row = 16 * i + lr;
      vv4[i] = bload4(rV, (unsigned)sizeof(In) * (unsigned)(row * rs + 16 * cv + 4 * lq), (const In*)nullptr);
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      f32x4 acc = zero4();
#pragma unroll
      for (int p2 = i / 2; p2 < 2; ++p2)
        acc = mm3<true, true>(acc, bo[p2], op_vec(sXh, sXl, LDB, 16 * i, 32 * p2));
      const int row = 16 * i + lr;
      const float4 vf = to_f4(vv4[i]);
      const f32x4 vd = f32x4{vf.x * acc[0], vf.y * acc[1], vf.z * acc[2], vf.w * acc[3]};
      const float bt = sBt[row];
      if (row < nvalid) {
        In* dvo = (In*)p.dv + (t0 + row) * rs + (long long)h * DV + 16 * cv + 4 * lq;
        if constexpr (F32) *(float4*)dvo = float4{bt * acc[0], bt * acc[1], bt * acc[2], bt * acc[3]};
        else *(u32x2*)dvo = u32x2{pack_bf16(bt * acc[0], bt * acc[1]), pack_bf16(bt * acc[2], bt * acc[3])};
      }
      add_cols(rowB, i, vd);  // row 16 i + r of the chunk: the transposed tile's column r
    }
  }
#pragma unroll
  for (int kb = 0; kb < NKB; ++kb) {
    const int cb = wave + CW * kb;
    if (cb >= NCB) continue;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      f32x4 acc = zero4();
#pragma unroll
      for (int p2 = i / 2; p2 < 2; ++p2)
        acc = mm3<true, true>(acc, op_vec(sXh, sXl, LDB, 16 * i, 32 * p2),
                              op_vec(sDWh, sDWl, LDB, 16 * cb, 32 * p2));
      f32x4 kt;
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        const int row = 16 * i + 4 * lq + v, col = 16 * cb + lr;
        kt[v] = ldx(sK + row * LDK + col) * acc[v];
        dk[kb][i][v] += sBt[row] * eg(row) * acc[v];
      }
      add_rows(rowT, i, kt);
    }
  }
  // M1 = X^T dX
  {
#pragma unroll
    for (int jj = 0; jj < 2; ++jj) {
      const int bj = 2 * half + jj;
      f32x4 acc = zero4();
      for (int p2 = bi / 2; p2 < 2; ++p2)  // X^T is upper triangular
        acc = mm3<true, true>(acc, op_vec(sXh, sXl, LDB, 16 * bi, 32 * p2),
                              op_vec(sDXh, sDXl, LDB, 16 * bj, 32 * p2));
      put_ct(sMh, sMl, LDB, 16 * bi, 16 * bj, acc);
    }
  }
  lds_barrier();  // M1 complete (a row block's two halves come from two wavefronts)
  // ---------------------------------------------------------------- dL = -strict_lower(M1 X^T)
  {
    f32x4 dl[2];
#pragma unroll
    for (int jj = 0; jj < 2; ++jj) {
      const int bj = 2 * half + jj;
      f32x4 acc = zero4();
      if (bj <= bi) {
#pragma unroll
        for (int p2 = 0; p2 < 2; ++p2)  // B: rows of X
          if (p2 <= bj / 2)
            acc = mm3<true, true>(acc, op_tr(sMh, sMl, LDB, 16 * bi, 32 * p2),
                                  op_tr(sXh, sXl, LDB, 16 * bj, 32 * p2));
      }
      dl[jj] = acc;
    }
    lds_barrier();  // every read of M1 is complete before its rows are overwritten
#pragma unroll
    for (int jj = 0; jj < 2; ++jj) {
      const int bj = 2 * half + jj;
      f32x4 lb, ld, qm;
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        const int row = 16 * bi + 4 * lq + v, col = 16 * bj + lr;
        const float d = row > col ? -dl[jj][v] : 0.f;
        const float lg = pLg[jj][v];
        lb[v] = d * lg;
        ld[v] = d * sBt[row] * lg;                      // dL * L
        qm[v] = sBt[row] * d * gam(row, col);           // Qm = diag(beta) (dL * Gamma)
      }
      put_ct(sMh, sMl, LDB, 16 * bi, 16 * bj, qm);
      add_rows(rowB, bi, lb);
      add_rows(rowG, bi, ld);
      add_cols(colG, bj, -ld);
    }
  }
  lds_barrier();

  // ---------------------------------------------------------------- (Qm + Qm^T) k, dPg^T qs, dPg k
#pragma unroll
  for (int kb = 0; kb < NKB; ++kb) {
    const int cb = wave + CW * kb;
    if (cb >= NCB) continue;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      f32x4 a_k = dk[kb][i], a_q = dq[kb][i], a_t = zero4();
#pragma unroll
      for (int p2 = 0; p2 < 2; ++p2) {
        const Op bk = kq_col<false>(sK, LDK, 16 * cb, 32 * p2);
        // (Qm + Qm^T) k as Qm k + Qm^T k
        a_k = mm3<true, F32>(a_k, op_tr(sMh, sMl, LDB, 16 * i, 32 * p2), bk);
        a_k = mm3<true, F32>(a_k, op_vec(sMh, sMl, LDB, 16 * i, 32 * p2), bk);
        if (p2 <= i / 2)  // dPg is lower triangular
          a_q = mm3<true, F32>(a_q, op_tr(sDPh, sDPl, LDB, 16 * i, 32 * p2), bk);
        if (p2 >= i / 2)  // dPg^T is upper triangular
          a_t = mm3<true, F32>(a_t, op_vec(sDPh, sDPl, LDB, 16 * i, 32 * p2),
                               kq_col<false>(sQ, LDK, 16 * cb, 32 * p2));
      }
      // per value head rows at the input precision: the q/k finalisation sums them and
      // rounds to that precision anyway
      KT* dqo = (KT*)p.dqh + (t0 * Hv + h) * (long long)DK;
      KT* dko = (KT*)p.dkh + (t0 * Hv + h) * (long long)DK;
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        const int row = 16 * i + 4 * lq + v, col = 16 * cb + lr;
        if (row < nvalid) {
          dqo[(long long)row * Hv * DK + col] = from_f32<KT>(scale * a_q[v]);
          dko[(long long)row * Hv * DK + col] = from_f32<KT>(a_k[v] + scale * a_t[v]);
        }
      }
    }
  }
  lds_barrier();

  // ---------------------------------------------------------------- dG, dbeta, dg
  if (wave == 0) {
    const int i = l;
    float rg = 0.f, rt = 0.f, rb = 0.f, rp = 0.f;
#pragma unroll
    for (int w = 0; w < CW; ++w) {
      rg += sRowG[w][i] + sColG[w][i] - sRP[w][i];
      rt += sRowT[w][i];
      rb += sRowB[w][i];
      rp += sRP[w][i];
    }
    const float t = __expf(sG[i]) * rt;
    float dG = rg + sBt[i] * t;
    const float db = rb + t;
    const float rsum = wave_sum(rp);
    float sds = 0.f;
#pragma unroll
    for (int w = 0; w < CW; ++w) sds += sRed[w];
    if (i == C - 1) dG += rsum + __expf(sG[C - 1]) * sds;
    // dg_t = sum_{i >= t} dG_i (G = cumsum(g), deltanet.py:98)
    float x = dG;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
      const float y = __shfl_down(x, o);
      if (i + o < 64) x += y;
    }
    if (i < nvalid) {
      p.dg[(t0 + i) * Hv + h] = x;
      p.dbeta[(t0 + i) * Hv + h] = db;
    }
  }
}

// ============================================================================ q/k finalisation

// dk / 8 consecutive threads per (token, key head) row of dq or dk, 8 elements each: the
// sum over the key head's value heads, then (qk_l2norm) the L2-norm backward
// dx = r (dy - y (y . dy)), y = x r, r = rsqrt(sum x^2 + 1e-6) (deltanet.py:30-32; the bf16
// rounding of y is differentiated as the identity, as autodiff does for a dtype cast).
template <bool F32>
__global__ __launch_bounds__(NT) void qk_final_kernel(BwdParams p, long long rows) {
  using In = typename std::conditional<F32, float, bf16_t>::type;
  const int dk = p.dk, tpr = dk / 8, gqa = p.Hv / p.Hk;
  const long long gid = (long long)blockIdx.x * NT + threadIdx.x;
  const long long rid = gid / tpr;
  const int c8 = 8 * (int)(gid % tpr);
  if (rid >= 2 * rows) return;  // whole rows drop out together (tpr divides 64)
  const int which = (int)(rid / rows);
  const long long row = rid % rows;
  const long long token = row / p.Hk;
  const int hk = (int)(row % p.Hk);
  const In* src = (const In*)(which ? p.dkh : p.dqh) + (token * p.Hv + (long long)hk * gqa) * dk + c8;
  float d[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f}, x[8];
  for (int g = 0; g < gqa; ++g) {
    float w[8];
    load8v(src + (long long)g * dk, w);
#pragma unroll
    for (int e = 0; e < 8; ++e) d[e] += w[e];
  }
  load8v((const In*)(which ? p.k : p.q) + row * dk + c8, x);
  if (p.qk_l2norm) {
    float ss = 0.f;
#pragma unroll
    for (int e = 0; e < 8; ++e) ss += x[e] * x[e];
    for (int o = 1; o < tpr; o <<= 1) ss += __shfl_xor(ss, o);
    const float r = rsqrtf(ss + 1e-6f);
    float yd = 0.f;
#pragma unroll
    for (int e = 0; e < 8; ++e) yd += x[e] * r * d[e];
    for (int o = 1; o < tpr; o <<= 1) yd += __shfl_xor(yd, o);
#pragma unroll
    for (int e = 0; e < 8; ++e) d[e] = r * (d[e] - x[e] * r * yd);
  }
  In* out = (In*)(which ? p.dk_out : p.dq) + row * dk + c8;
  if constexpr (F32) {
    *(float4*)out = float4{d[0], d[1], d[2], d[3]};
    *(float4*)(out + 4) = float4{d[4], d[5], d[6], d[7]};
  } else {
    *(u32x4*)out = pack8(d);
  }
}

template <int DK, bool F32>
hipError_t launch_bwd_dk(const BwdParams& p, hipStream_t stream) {
  hipLaunchKernelGGL((rscan_kernel<DK, F32>), dim3((unsigned)(p.N * p.Hv * p.nb)), dim3(F32 ? NT : 2 * NT), 0,
                     stream, p);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  const unsigned grid = (unsigned)((long long)p.n_rec * p.Hv);
  if (grid > 0) {
    if (p.DV == 128)
      hipLaunchKernelGGL((cgrad_kernel<DK, 128, F32>), dim3(grid), dim3(CNT), 0, stream, p);
    else
      hipLaunchKernelGGL((cgrad_kernel<DK, 64, F32>), dim3(grid), dim3(CNT), 0, stream, p);
    e = hipGetLastError();
    if (e != hipSuccess) return e;
  }
  const long long rows = (long long)p.T * (p.cu_seqlens ? 1 : p.N) * p.Hk;
  if (rows > 0) {
    const long long threads = 2 * rows * (p.dk / 8);
    const unsigned g2 = (unsigned)((threads + NT - 1) / NT);
    hipLaunchKernelGGL((qk_final_kernel<F32>), dim3(g2), dim3(NT), 0, stream, p, rows);
    e = hipGetLastError();
  }
  return e;
}

}  // namespace

bool bwd_dims_supported(int dk, int dv, bool f32_inputs) {
  if (dv != 64 && dv != 128) return false;
  // fp32 inputs at dk = 128 would need 185 KiB of LDS in the gradient kernel
  if (f32_inputs) return dk == 32 || dk == 64;
  return dk == 64 || dk == 128;
}

hipError_t launch_bwd(const BwdParams& p, hipStream_t stream) {
  if (p.in_f32) {
    if (p.dk == 64) return launch_bwd_dk<64, true>(p, stream);
    if (p.dk == 32) return launch_bwd_dk<32, true>(p, stream);
    return hipErrorInvalidValue;
  }
  if (p.dk == 128) return launch_bwd_dk<128, false>(p, stream);
  if (p.dk == 64) return launch_bwd_dk<64, false>(p, stream);
  return hipErrorInvalidValue;
}

}  // namespace omx
