// in_proj_qkv with the causal conv + SiLU in its epilogue: a prototype of the
// projection-side fusion of the layer (deltanet.py:234-243: mixed_qkv = in_proj_qkv(x),
// then the depthwise conv over tokens and SiLU), measured against the library GEMM.
//
// out[m, n] = bf16(x[m, :] . W[n, :]) for x [M, D] and W [N, D] (the nn.Linear layout),
// fp32 accumulation, rounded to bf16 once as the reference's bf16 linear map rounds.
// With CONV the epilogue continues with the conv of that bf16 result over each sequence
// of T consecutive rows (no history: the rows before a sequence start are zeros,
// deltanet.py:46) and its SiLU, with the layer prep's arithmetic (gdn_conv.h: bf16
// weights and inputs, fp32 tap sums by two bf16 dot products, the sum and the SiLU
// rounded to bf16), and stores conv(x W^T) instead of x W^T.
//
// Tiles: 256 output rows x 256 columns per workgroup, the contraction in steps of 64
// (two per loop iteration: D a multiple of 128).  Eight wavefronts, two per SIMD, wave
// (wm, wn) owning rows 128 wm .. +127 and columns 64 wn .. +63 as 8 x 4 blocks of
// v_mfma_f32_16x16x32_bf16 with their 128 fp32 accumulators in VGPRs (VGPR-form MFMAs,
// each accumulating in place), formed transposed (C^T = W x^T) so a lane ends holding 4
// consecutive columns of one row.  (Four wavefronts of 128 x 128 need all 256 AGPRs for
// their accumulators, and the register allocator then moves them between AGPRs and
// VGPRs around every product instead of accumulating in place.)  Both operands are staged in LDS by
// direct global-to-LDS loads (global_load_lds_dwordx4, lane i writes 16 bytes at the
// buffer offset + 16 i), issued by every wavefront one step ahead into the other of two
// stage buffers; rows are 128 bytes of 8 segments, segment s of row r stored in slot
// s ^ (r & 7), so the 16-byte fragment reads of 8 consecutive rows hit 8 different bank
// groups.  The two stages are separate __shared__ objects, so the compiler can tell the
// loads into one from the reads of the other and does not wait for them.
//
// The conv needs the 3 rows before a tile's first row: with CONV the tile also forms a
// 16-row halo block (rows m0 - 16 .. m0 - 1), each wavefront taking two of its 16-column
// blocks, 6% more products.  The epilogue writes the bf16 tile (halo included) to LDS,
// over the stage buffers, and 512 threads each take 8 columns of 16 consecutive rows:
// the conv streams down the rows from registers, and every store is 16 bytes, 32
// threads covering a row's 512 contiguous bytes.  Without CONV the same tile is copied
// out unchanged (the plain GEMM, for measuring the GEMM itself).
//
// Workgroup order: the hardware deals workgroup ids round-robin over the 8 XCDs; ids are
// remapped so each XCD takes a contiguous range of tiles, walked 8 row panels at a time
// (N-tiles slower), so the tiles an XCD runs together share their x and W panels in its L2.
#include "gdn_common.h"
#include "gdn_conv.h"
#include "gdn_kernels.h"
#include "gdn_mfma.h"

namespace omx {

namespace {

typedef __attribute__((address_space(1))) void glob_void;
typedef __attribute__((address_space(3))) void lds_void;
typedef __attribute__((address_space(3))) unsigned char lds_u8;

constexpr int kBM = 256, kBN = 256, kBK = 64, kHalo = 16;
constexpr int kARows = kHalo + kBM;            // stage rows of x: the halo block first
constexpr int kAStage = kARows * kBK * 2;      // 34,816 bytes
constexpr int kBStage = kBN * kBK * 2;         // 32,768 bytes
constexpr int kOutStride = kBN * 2;            // bytes per row of the bf16 output tile
constexpr int kSplitRow = 144;                 // output-tile rows [0, 144) over stage 0
constexpr int cmax(int a, int b) { return a > b ? a : b; }
constexpr int kS0Bytes = cmax(kAStage + kBStage, kSplitRow * kOutStride);
constexpr int kS1Bytes = cmax(kAStage + kBStage, (kARows - kSplitRow) * kOutStride);
constexpr int kGroupM = 8;                     // row panels per group of the tile order

struct QkvParams {
  const bf16_t* x;
  const bf16_t* w;
  const float* conv_w;  // [N][4] fp32, taps oldest first (CONV)
  bf16_t* out;
  int M, N, D, T;       // T: rows per sequence (CONV)
  int tiles_m, tiles_n;
};

// 16-byte slot of segment s in stage row r, and of segment s in output-tile row r
__device__ __forceinline__ unsigned slot(int s, int r) { return (unsigned)(s ^ (r & 7)); }
__device__ __forceinline__ unsigned oslot(int s, int r) { return (unsigned)(s ^ (r & 31)); }

constexpr int kWaves = 8, kThreads = 64 * kWaves;
constexpr int kWR = 128, kWC = 64;  // a wavefront's rows and columns

template <bool CONV>
__global__ __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(2, 2)))
void qkv_proj_kernel(QkvParams p) {
  __shared__ __align__(16) unsigned char sS0[kS0Bytes];
  __shared__ __align__(16) unsigned char sS1[kS1Bytes];

  const int tid = threadIdx.x, l = tid & 63, lq = l >> 4, lr = l & 15;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave >> 2, wn = wave & 3;

  // tile of this workgroup: an XCD-contiguous range, then grouped row panels
  const int nwg = (int)gridDim.x, bid = (int)blockIdx.x;
  const int t = nwg % 8 == 0 ? (bid % 8) * (nwg / 8) + bid / 8 : bid;
  const int per_group = kGroupM * p.tiles_n;
  const int first_m = (t / per_group) * kGroupM;
  const int gsz = p.tiles_m - first_m < kGroupM ? p.tiles_m - first_m : kGroupM;
  const int tm = first_m + (t % per_group) % gsz, tn = (t % per_group) / gsz;
  const int m0 = tm * kBM, n0 = tn * kBN;

  // ---------------------------------------------------------------- staging
  // Stage row r of x (rows 0-15 the halo block) is x row m0 - 16 + r; of W, row n0 + r.
  // Instruction i covers stage rows 8i .. 8i+7: lane l takes row 8i + l/8 and slot l%8,
  // which holds segment (l%8) ^ (l/8), the same for every instruction, so one lane offset
  // and uniform row steps address all of them.  x is read through a buffer whose range
  // ends at row M: the halo rows before x (negative offsets wrap past the range) and rows
  // past M read zeros without a memory access.
  const unsigned ld = 2u * (unsigned)p.D;  // row stride in bytes
  const unsigned lo = (unsigned)(l >> 3) * ld + 16u * slot(l & 7, l >> 3);
  const auto xr = buf_rsrc(p.x, (unsigned)p.M * ld);
  const unsigned xo = (unsigned)(m0 - kHalo) * ld + lo;
  // W's rows all exist: the row step goes in the scalar offset, the lane offset is lo
  const auto wr = buf_rsrc(p.w + (size_t)n0 * p.D, (unsigned)kBN * ld);
  auto issue = [&](int kt, lds_u8* st) {
    const unsigned ko = 2u * kBK * (unsigned)kt;
    // 34 instructions of x with the halo (waves 0 and 1 take five, the others four and
    // repeat the last one, which writes the same bytes again), 32 without
#pragma unroll
    for (int j = 0; j < (CONV ? 5 : 4); ++j) {
      int i = kWaves * j + (CONV ? 0 : 2) + wave;
      i = i < kARows / 8 ? i : kARows / 8 - 1;
      __builtin_amdgcn_raw_ptr_buffer_load_lds(xr, (lds_void*)(st + 1024 * i), 16, xo + 8u * (unsigned)i * ld,
                                               ko, 0, 0);
    }
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int i = kWaves * j + wave;
      __builtin_amdgcn_raw_ptr_buffer_load_lds(wr, (lds_void*)(st + kAStage + 1024 * i), 16, lo,
                                               8u * (unsigned)i * ld + ko, 0, 0);
    }
  };

  // ---------------------------------------------------------------- products
  constexpr int RB = kWR / 16, CB = kWC / 16;  // 16 x 16 blocks per wavefront
  f32x4 acc[RB][CB];
  f32x4 acch[2];
#pragma unroll
  for (int i = 0; i < RB; ++i)
#pragma unroll
    for (int j = 0; j < CB; ++j) acc[i][j] = zero4();
#pragma unroll
  for (int j = 0; j < 2; ++j) acch[j] = zero4();

  // fragment rows: x rows 16 + 128 wm + 16 bi + lr, W rows 64 wn + 16 bj + lr; every
  // block row is a multiple of 8 past the lane's row, so the slot depends on lr only
  auto compute = [&](const unsigned char* st) {
    const unsigned char* sa = st + (unsigned)(kHalo + kWR * wm + lr) * 128u;
    const unsigned char* sb = st + kAStage + (unsigned)(kWC * wn + lr) * 128u;
    const unsigned char* sh = st + (unsigned)lr * 128u;
#pragma unroll
    for (int ks = 0; ks < kBK / 32; ++ks) {
      const unsigned so = 16u * slot(4 * ks + lq, lr);
      u32x4 a[RB], b[CB];
#pragma unroll
      for (int i = 0; i < RB; ++i) a[i] = *(const u32x4*)(sa + 16 * 128 * i + so);
#pragma unroll
      for (int j = 0; j < CB; ++j) b[j] = *(const u32x4*)(sb + 16 * 128 * j + so);
#pragma unroll
      for (int i = 0; i < RB; ++i)
#pragma unroll
        for (int j = 0; j < CB; ++j) acc[i][j] = mma16(b[j], a[i], acc[i][j]);
      if constexpr (CONV) {  // the halo block's columns 32 wm .. +31 of this wave's 64 (a
        // uniform branch: the fragments stay in registers, which a run-time index would not allow)
        const u32x4 ah = *(const u32x4*)(sh + so);
        if (wm == 0) {
#pragma unroll
          for (int j = 0; j < 2; ++j) acch[j] = mma16(b[j], ah, acch[j]);
        } else {
#pragma unroll
          for (int j = 0; j < 2; ++j) acch[j] = mma16(b[2 + j], ah, acch[j]);
        }
      }
    }
  };

  // an even number of steps (D a multiple of 128): both products of the unrolled loop
  // are unconditional, so the accumulators stay in place across it
  const int KT = p.D / kBK;
  issue(0, (lds_u8*)sS0);
  for (int kt = 0; kt < KT; kt += 2) {
    __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0): this wave's loads of step kt landed
    lds_barrier();                       // everyone's have; step kt - 1's buffer is free
    issue(kt + 1, (lds_u8*)sS1);
    compute(sS0);
    __builtin_amdgcn_s_waitcnt(0x0F70);
    lds_barrier();
    if (kt + 2 < KT) issue(kt + 2, (lds_u8*)sS0);  // uniform
    compute(sS1);
  }
  lds_barrier();  // every wave is done with the stage buffers

  // ---------------------------------------------------------------- bf16 tile in LDS
  // output-tile row r (0-15 the halo, 16-271 the tile) at stage 0 for r < 144, else
  // stage 1; lane (q, r) of block (bi, bj) holds row 16 + 128 wm + 16 bi + r, columns
  // 64 wn + 16 bj + 4q .. +3
  auto orow = [&](int r) -> unsigned char* {
    return r < kSplitRow ? sS0 + r * kOutStride : sS1 + (r - kSplitRow) * kOutStride;
  };
  auto put = [&](int r, int col, const f32x4& v) {
    *(u32x2*)(orow(r) + 16u * oslot(col >> 3, r) + 8u * ((col >> 2) & 1)) =
        u32x2{pack_bf16(v[0], v[1]), pack_bf16(v[2], v[3])};
  };
#pragma unroll
  for (int i = 0; i < RB; ++i)
#pragma unroll
    for (int j = 0; j < CB; ++j) put(kHalo + kWR * wm + 16 * i + lr, kWC * wn + 16 * j + 4 * lq, acc[i][j]);
  if constexpr (CONV) {
#pragma unroll
    for (int j = 0; j < 2; ++j) put(lr, kWC * wn + 16 * (2 * wm + j) + 4 * lq, acch[j]);
  }
  lds_barrier();

  // ---------------------------------------------------------------- epilogue
  // thread (g, rg): columns n0 + 8g .. +7 of tile rows 16 rg .. 16 rg + 15 (global rows
  // m0 + 16 rg + i); stores through a buffer whose range ends at row M
  constexpr int RPT = kBM / (kThreads / 32);  // rows per thread
  const int g = tid & 31, rg = tid >> 5;
  const auto ob = buf_rsrc(p.out + (size_t)m0 * p.N + n0, 2u * (unsigned)(p.M - m0) * (unsigned)p.N);
  const unsigned ost = 2u * (unsigned)p.N;
  auto tile_row = [&](int r) { return *(const u32x4*)(orow(r) + 16u * oslot(g, r)); };
  if constexpr (!CONV) {
#pragma unroll 4
    for (int i = 0; i < RPT; ++i) {
      const int r = kHalo + RPT * rg + i;
      __builtin_amdgcn_raw_buffer_store_b128(tile_row(r), ob, (unsigned)(RPT * rg + i) * ost + 16u * g, 0, 0);
    }
  } else {
    // weights of the 8 channels, cast to bf16 and paired as gdn_conv.h pairs them
    uint32_t wp[8][2];
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const float4 w = *(const float4*)(p.conv_w + (size_t)(n0 + 8 * g + e) * 4);
      wp[e][0] = pack_bf16(w.w, w.z);
      wp[e][1] = pack_bf16(w.y, w.x);
    }
    // row of the first output within its sequence; rows before a sequence start are zero
    const int mf = m0 + RPT * rg;
    int rs = mf % p.T;
    u32x4 x3 = tile_row(kHalo + RPT * rg - 3), x2 = tile_row(kHalo + RPT * rg - 2),
          x1 = tile_row(kHalo + RPT * rg - 1);
#pragma unroll 4
    for (int i = 0; i < RPT; ++i) {
      const u32x4 x0 = tile_row(kHalo + RPT * rg + i);
      u32x4 pe0, po0, pe2, po2;
      time_pairs(x0, x1, pe0, po0);  // (x_t, x_{t-1})
      time_pairs(x2, x3, pe2, po2);  // (x_{t-2}, x_{t-3})
      // first rows of a sequence: the taps before its start read zeros
      const uint32_t k0 = rs == 0 ? 0x0000ffffu : 0xffffffffu;
      const uint32_t k2 = rs <= 1 ? 0u : (rs == 2 ? 0x0000ffffu : 0xffffffffu);
      u32x4 y;
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        const float a0 = dot4_bf16(wp[2 * c][0], wp[2 * c][1], pe0[c] & k0, pe2[c] & k2);
        const float a1 = dot4_bf16(wp[2 * c + 1][0], wp[2 * c + 1][1], po0[c] & k0, po2[c] & k2);
        const uint32_t u = pack_bf16(a0, a1);
        y[c] = pack_bf16(silu_fast(__uint_as_float(u << 16)), silu_fast(__uint_as_float(u & 0xffff0000u)));
      }
      __builtin_amdgcn_raw_buffer_store_b128(y, ob, (unsigned)(RPT * rg + i) * ost + 16u * g, 0, 0);
      x3 = x2;
      x2 = x1;
      x1 = x0;
      rs = rs + 1 == p.T ? 0 : rs + 1;
    }
  }
}

}  // namespace

hipError_t launch_qkv_proj(const void* x, const void* w, const float* conv_w, void* out,
                           long long M, int N, int D, long long T, bool conv, hipStream_t stream) {
  if (M == 0) return hipSuccess;
  QkvParams p{};
  p.x = (const bf16_t*)x;
  p.w = (const bf16_t*)w;
  p.conv_w = conv_w;
  p.out = (bf16_t*)out;
  p.M = (int)M;
  p.N = N;
  p.D = D;
  p.T = (int)(conv ? T : M);
  p.tiles_m = (int)((M + kBM - 1) / kBM);
  p.tiles_n = N / kBN;
  const unsigned grid = (unsigned)(p.tiles_m * p.tiles_n);
  if (conv)
    hipLaunchKernelGGL(qkv_proj_kernel<true>, dim3(grid), dim3(kThreads), 0, stream, p);
  else
    hipLaunchKernelGGL(qkv_proj_kernel<false>, dim3(grid), dim3(kThreads), 0, stream, p);
  return hipGetLastError();
}

int qkv_proj_tile_cols() { return kBN; }
int qkv_proj_tile_depth() { return 2 * kBK; }

}  // namespace omx
