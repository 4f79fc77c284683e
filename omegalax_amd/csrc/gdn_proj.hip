// The layer's two per-head gate projections in one pass over the hidden rows.
//
// deltanet.py:240-241 computes b = in_proj_b(x) and a = in_proj_a(x): two bf16 linear
// maps [tokens, D] -> [tokens, Hv] with fp32 accumulation (nnx.Linear, dtype bf16).
// As two library GEMMs each N = Hv wide, every call reads the whole hidden state from
// HBM (64 MiB at C1) for a few MFLOP of work, twice.  This kernel reads each hidden row
// once and forms both outputs from it: a memory-bound skinny product.
//
// Work mapping: one workgroup per 64 token rows, wavefront w owning rows 16 (w % 4) ..
// +15 of contraction part w / 4 (one or two parts, the partial sums added at the end);
// each part runs its chunks of KC.  A chunk's weight rows (both matrices, 2 x 16 NT rows,
// rows past Hv zero) are staged once per part in LDS (rows padded by 16 bytes, so the 16
// rows of a fragment read fall in different banks) and shared by its four wavefronts;
// each lane loads its own token row's part straight into registers.  Both
// are read in the "row r, contraction slots 8q .. 8q+7" layout of a 16x16x32 MFMA
// operand, and the product is formed transposed, C^T = W X^T, so a lane ends holding 4
// consecutive output columns of one token row (one 8-byte store).  The contraction
// order inside a 64-wide step is permuted (lane q's slots of the two 32-wide halves are
// elements 16q .. 16q+7 and 16q+8 .. 16q+15), the same for both operands, so each lane
// reads 32 contiguous bytes of its row and a wavefront whole 128-byte lines.  The next
// chunk's weight and token loads are issued before the current chunk's products.
#include "gdn_common.h"
#include "gdn_kernels.h"
#include "gdn_mfma.h"

namespace omx {

namespace {

constexpr int kProjRows = 64;  // token rows per workgroup (four blocks of 16)

// Contraction parts per workgroup (four wavefronts each): two for up to 32 heads, which
// doubles the loads in flight per CU (measured at C1: 23.9 -> 21.2 us); one above, where
// two parts' weight buffers would leave one workgroup per CU (Hv=64: 87.6 -> 121.8 us).
template <int NT>
constexpr int proj_split() { return NT <= 2 ? 2 : 1; }

template <int NT, int KS>
struct ProjCfg {
  static constexpr int NTH = 256 * KS;             // four row blocks of 16 per part
  static constexpr int KC = NT >= 8 ? 128 : 256;   // contraction chunk (elements)
  static constexpr int NW = 32 * NT;               // staged weight rows (a then b)
  static constexpr int LDW = 2 * KC + 16;          // LDS row stride (bytes)
  static constexpr int WV = NW * KC / (8 * 256);   // 16-byte weight loads per thread
  static constexpr int XV = KC / 32;               // 16-byte token loads per lane
  static_assert(WV * 8 * 256 == NW * KC, "weight chunk split");
  static_assert(KS == 1 || 4 * 64 * 2 * NT * 16 <= NW * LDW, "partial sums fit a part's buffer");
};

template <int NT, int KS>
__global__ __launch_bounds__(256 * KS) void ab_proj_kernel(const bf16_t* __restrict__ x,
                                                          const bf16_t* __restrict__ wa,
                                                          const bf16_t* __restrict__ wb,
                                                          bf16_t* __restrict__ a,
                                                          bf16_t* __restrict__ b, long long M,
                                                          int D, int Hv, bool vec_out) {
  using Q_ = ProjCfg<NT, KS>;
  constexpr int KC = Q_::KC, NW = Q_::NW, LDW = Q_::LDW, WV = Q_::WV, XV = Q_::XV;
  __shared__ __align__(16) unsigned char sW[KS][NW * LDW];
  const int tid = threadIdx.x, l = tid & 63, lq = l >> 4, lr = l & 15;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int part = wave >> 2, tp = tid & 255;  // contraction part, thread within it
  const long long row0 = (long long)blockIdx.x * kProjRows + 16 * (wave & 3);
  // the lane's token row (rows past M load row M - 1, in bounds, and are not stored)
  const long long xr = row0 + lr < M ? row0 + lr : M - 1;
  const bf16_t* xrow = x + xr * D;
  const u32x4 z4 = {0u, 0u, 0u, 0u};
  const int nch = (D + KC - 1) / KC;
  const int nstep = (nch + KS - 1) / KS;  // part p takes chunks p, p + KS, ...
  unsigned char* const sWp = sW[part];

  // chunk c's loads: the weight rows this thread stages (row n, 16-byte segment s) and
  // the lane's token-row segments (D % 8 == 0).  Addresses are clamped and the values left
  // untouched until the next step uses them: a select here would make the compiler wait
  // for the loads right after issuing them, before the current chunk's products.  Weight
  // rows past Hv reload row Hv - 1 (they only feed output columns that are not stored);
  // elements past D reload element 0, finite, and meet zeros in x (xk below).
  u32x4 wreg[WV], xnext[XV];
  auto xk = [&](int c, int j) {  // step j / 2 (64 elements), half j % 2: 64 (j/2) + 16 q + 8 (j%2)
    return c * KC + 64 * (j >> 1) + 16 * lq + 8 * (j & 1);
  };
  auto load = [&](int c) {
    const int k0 = c * KC;
#pragma unroll
    for (int i = 0; i < WV; ++i) {
      const int it = tp + i * 256;
      const int n = it / (KC / 8), s = it % (KC / 8);
      const int m = n / (16 * NT), h = n % (16 * NT);  // matrix, row within it
      const int k = k0 + 8 * s;
      const bf16_t* src = (m == 0 ? wa : wb) + (long long)(h < Hv ? h : Hv - 1) * D + (k < D ? k : 0);
      wreg[i] = *(const u32x4*)src;
    }
#pragma unroll
    for (int j = 0; j < XV; ++j) {
      const int k = xk(c, j);
      xnext[j] = *(const u32x4*)(xrow + (k < D ? k : 0));
    }
  };

  f32x4 acc[2][NT];
#pragma unroll
  for (int m = 0; m < 2; ++m)
#pragma unroll
    for (int t = 0; t < NT; ++t) acc[m][t] = zero4();

  // every wavefront runs nstep steps, so all meet the same barriers; a part whose chunk is
  // past the end stages and multiplies nothing
  if (part < nch) load(part);
  for (int st = 0; st < nstep; ++st) {
    const int c = part + KS * st;
    const bool have = c < nch;
    u32x4 xcur[XV];
#pragma unroll
    for (int j = 0; j < XV; ++j) xcur[j] = xk(c, j) < D ? xnext[j] : z4;  // zeros past D
    lds_barrier();  // the previous step's fragment reads are done
    if (have) {
#pragma unroll
      for (int i = 0; i < WV; ++i) {
        const int it = tp + i * 256;
        const int n = it / (KC / 8), s = it % (KC / 8);
        *(u32x4*)(sWp + n * LDW + 16 * s) = wreg[i];
      }
      if (c + KS < nch) load(c + KS);
    }
    lds_barrier();  // the chunk's weight rows are in LDS
    if (have) {
#pragma unroll
      for (int j = 0; j < XV; ++j) {
        // weight fragment of tile t, matrix m: row 16 t + r, the same permuted slots
        const int kb = 2 * (64 * (j >> 1) + 16 * lq + 8 * (j & 1));  // byte offset in the row
#pragma unroll
        for (int m = 0; m < 2; ++m)
#pragma unroll
          for (int t = 0; t < NT; ++t) {
            const u32x4 wf = *(const u32x4*)(sWp + (m * 16 * NT + 16 * t + lr) * LDW + kb);
            acc[m][t] = mma16(wf, xcur[j], acc[m][t]);
          }
      }
    }
  }
  if constexpr (KS > 1) {
    // the other parts' partial sums, added into part 0's in a fixed order
    static_assert(KS == 2, "one exchange below");
    lds_barrier();  // every fragment read is done; part 1's buffer takes the sums
    f32x4* ex = (f32x4*)sW[1] + ((wave & 3) * 2 * NT) * 64 + l;
    if (part == 1) {
#pragma unroll
      for (int m = 0; m < 2; ++m)
#pragma unroll
        for (int t = 0; t < NT; ++t) ex[(m * NT + t) * 64] = acc[m][t];
    }
    lds_barrier();
    if (part != 0) return;
#pragma unroll
    for (int m = 0; m < 2; ++m)
#pragma unroll
      for (int t = 0; t < NT; ++t) acc[m][t] += ex[(m * NT + t) * 64];
  }

  // lane (q, r) holds token row row0 + r, output columns 16 t + 4q .. +3 of matrix m,
  // rounded to bf16 as the reference's bf16 linear map rounds its output; one 8-byte
  // store when the host found Hv % 4 == 0 and both outputs 8-byte aligned
  const long long row = row0 + lr;
  if (row >= M) return;
#pragma unroll
  for (int m = 0; m < 2; ++m) {
    bf16_t* out = (m == 0 ? a : b) + row * Hv;
#pragma unroll
    for (int t = 0; t < NT; ++t) {
      const int cc = 16 * t + 4 * lq;
      if (vec_out) {
        if (cc < Hv)
          *(uint2*)(out + cc) = make_uint2(pack_bf16(acc[m][t][0], acc[m][t][1]),
                                           pack_bf16(acc[m][t][2], acc[m][t][3]));
      } else {
#pragma unroll
        for (int v = 0; v < 4; ++v)
          if (cc + v < Hv) out[cc + v] = f2bf(acc[m][t][v]);
      }
    }
  }
}

template <int NT>
hipError_t launch_nt(const void* x, const void* wa, const void* wb, void* a, void* b, long long M,
                     int D, int Hv, hipStream_t stream) {
  constexpr int KS = proj_split<NT>();
  const long long blocks = (M + kProjRows - 1) / kProjRows;
  if (blocks > 0x7fffffffLL) return hipErrorInvalidValue;
  const bool vec_out = Hv % 4 == 0 && reinterpret_cast<uintptr_t>(a) % 8 == 0 &&
                       reinterpret_cast<uintptr_t>(b) % 8 == 0;
  hipLaunchKernelGGL((ab_proj_kernel<NT, KS>), dim3((unsigned)blocks), dim3(256 * KS), 0, stream,
                     (const bf16_t*)x, (const bf16_t*)wa, (const bf16_t*)wb, (bf16_t*)a,
                     (bf16_t*)b, M, D, Hv, vec_out);
  return hipGetLastError();
}

}  // namespace

int ab_proj_max_heads() { return 128; }

hipError_t launch_ab_proj(const void* x, const void* wa, const void* wb, void* a, void* b,
                          long long M, int D, int Hv, hipStream_t stream) {
  if (M == 0) return hipSuccess;
  if (D <= 0 || D % 8 != 0 || Hv < 1 || Hv > 128) return hipErrorInvalidValue;
  if (Hv <= 16) return launch_nt<1>(x, wa, wb, a, b, M, D, Hv, stream);
  if (Hv <= 32) return launch_nt<2>(x, wa, wb, a, b, M, D, Hv, stream);
  if (Hv <= 64) return launch_nt<4>(x, wa, wb, a, b, M, D, Hv, stream);
  return launch_nt<8>(x, wa, wb, a, b, M, D, Hv, stream);
}

}  // namespace omx
