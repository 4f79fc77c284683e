// C ABI of libomx_gdn.so: argument validation, workspace planning and launch.
//
// Every entry point validates its arguments on the host before the first HIP
// call, so an invalid request returns OMX_GDN_EINVAL (with a message from
// omx_gdn_last_error) on any machine, GPU or not.  No C++ exception crosses
// the ABI and nothing here synchronises the stream.
#include "omx_gdn.h"

#include <hip/hip_runtime.h>

#include <climits>
#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <mutex>
#include <string>

#include "gdn_kernels.h"

namespace {

thread_local std::string g_last_error;

int fail(int code, const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  g_last_error = buf;
  return code;
}

int ok() {
  g_last_error.clear();
  return OMX_GDN_OK;
}

int launch_status(hipError_t e, const char* what) {
  if (e != hipSuccess) return fail(OMX_GDN_ELAUNCH, "%s: HIP launch failed: %s", what, hipGetErrorString(e));
  return ok();
}

bool aligned(const void* p, size_t a) { return (reinterpret_cast<uintptr_t>(p) % a) == 0; }

size_t align_up(size_t x, size_t a) { return (x + a - 1) / a * a; }

#define REQUIRE(cond, ...) \
  do {                     \
    if (!(cond)) return fail(OMX_GDN_EINVAL, __VA_ARGS__); \
  } while (0)

// Workspace of the chunked prefill, offsets aligned to 256 bytes: the records of
// the preparation kernel (one per chunk slot and value head; a sequence adds at
// most one partial chunk, so ceil(tokens/64) + N slots cover any packing), the
// normalised k and q, (layer) the conv output of v (dk < 128: with dk = 128 the scan
// forms the v rows itself), the bf16 o and the partial
// sums of o^2 for the gated norm, and the plan of packed sequences (chunk offsets and
// the ordered copy of cu_seqlens the kernels read).
struct ChunkWs {
  size_t rec, kn, qn, vc, opart, oss, xch, off, cu, ord, total;
};

ChunkWs chunk_ws(int64_t B, int64_t T, int64_t Hk, int64_t Hv, int64_t dk, int64_t dv, int64_t N,
                 int mode, bool bwd = false) {
  ChunkWs w{};
  if (B < 0 || T < 0 || Hk < 0 || Hv < 0 || dk < 0 || dv < 0 || N < 0) return w;
  const size_t tokens = (size_t)(B * T);
  const size_t slots = (tokens + 63) / 64 + (size_t)N;
  const size_t elem = mode == omx::kModeF32 ? 4 : 2;
  size_t o = 0;
  w.rec = o;
  o += align_up(slots * (size_t)Hv * (size_t)omx::chunk_record_bytes(mode, bwd), 256);
  w.kn = o;
  o += align_up(tokens * (size_t)(Hk * dk) * elem, 256);
  w.qn = o;
  o += align_up(tokens * (size_t)(Hk * dk) * elem, 256);
  if (mode == omx::kModeLayer) {
    w.vc = o;
    if (!omx::layer_scan_forms_v((int)dk)) o += align_up(tokens * (size_t)(Hv * dv) * 2, 256);
    w.opart = o;
    o += align_up(tokens * (size_t)(Hv * dv) * 2, 256);
    w.oss = o;
    o += align_up((tokens + 63) / 64 * 64 * (size_t)Hv * (size_t)(dv / 16) * 4, 256);
    // the fused norm's exchange of row partials: {value, tag} per (sequence, value head,
    // column block, ring entry, row), for up to dv / 16 blocks
    w.xch = o;
    o += align_up((size_t)N * (size_t)Hv * (size_t)(dv / 16) * omx::kXchRing * 64 * 8, 256);
  }
  w.off = o;
  o += align_up((size_t)(N + 1) * 4, 256);
  w.cu = o;
  o += align_up((size_t)(N + 1) * 4, 256);
  w.ord = o;
  o += align_up((size_t)N * 4, 256);
  w.total = o;
  return w;
}

// Workspace of the backward pass: the forward's (records, normalised q/k, chunk
// offsets), then the prep's fp32 X, Lg, P, G per (chunk slot, value head), the state
// entering and the state gradient leaving every chunk, V_new and its gradient, and the
// per-value-head gradients of the normalised q and k.
struct BwdWs {
  ChunkWs f;
  size_t xlpg, states, dstates, vnew, dvnew, dqh, dkh, total;
};

BwdWs bwd_ws(int64_t B, int64_t T, int64_t Hk, int64_t Hv, int64_t dk, int64_t dv, int64_t N,
             int mode) {
  BwdWs w{};
  w.f = chunk_ws(B, T, Hk, Hv, dk, dv, N, mode, true);  // records with P's lo parts
  if (B < 0 || T < 0 || Hk < 0 || Hv < 0 || dk < 0 || dv < 0 || N < 0) return w;
  const size_t tokens = (size_t)(B * T);
  const size_t slots = (tokens + 63) / 64 + (size_t)N;
  size_t o = w.f.total;
  w.xlpg = o;
  o += align_up(slots * (size_t)Hv * omx::kXlpgFloatsHost * 4, 256);
  w.states = o;
  o += align_up(slots * (size_t)(Hv * dk * dv) * 4, 256);
  w.dstates = o;
  o += align_up(slots * (size_t)(Hv * dk * dv) * 4, 256);
  w.vnew = o;
  o += align_up(tokens * (size_t)(Hv * dv) * 4, 256);
  w.dvnew = o;
  o += align_up(tokens * (size_t)(Hv * dv) * 4, 256);
  w.dqh = o;
  o += align_up(tokens * (size_t)(Hv * dk) * 4, 256);
  w.dkh = o;
  o += align_up(tokens * (size_t)(Hv * dk) * 4, 256);
  w.total = o;
  return w;
}

int check_heads(const char* fn, int64_t Hk, int64_t Hv, int64_t dk, int64_t dv) {
  REQUIRE(Hk >= 1 && Hv >= 1, "%s: head counts must be positive (Hk=%lld, Hv=%lld)", fn,
          (long long)Hk, (long long)Hv);
  REQUIRE(Hv % Hk == 0, "%s: value heads (%lld) must be a multiple of key heads (%lld)", fn,
          (long long)Hv, (long long)Hk);
  REQUIRE(Hv <= 4096, "%s: too many value heads (%lld)", fn, (long long)Hv);
  REQUIRE(dk >= 1 && dv >= 1, "%s: head dims must be positive (dk=%lld, dv=%lld)", fn,
          (long long)dk, (long long)dv);
  return OMX_GDN_OK;
}

// Head dims a call runs at: the caller's when the kernels are compiled for them, else
// the smallest compiled dims that cover them (the call then runs on zero-padded copies,
// gdn_pad.hip); ok = false when none do.
struct HeadDims {
  int64_t dk, dv;
  bool pad, ok;
};
enum DimsKind { kCoreFwd, kLayerFwd, kCoreBwd, kLayerBwd };

HeadDims head_dims(DimsKind kind, int64_t dk, int64_t dv, bool f32) {
  auto compiled = [&](int64_t a, int64_t b) {
    switch (kind) {
      case kCoreFwd: return omx::chunk_dims_supported((int)a, (int)b, f32);
      case kLayerFwd: return omx::layer_dims_supported((int)a, (int)b);
      case kCoreBwd: return omx::bwd_dims_supported((int)a, (int)b, f32);
      default: return omx::bwd_dims_supported((int)a, (int)b, false);
    }
  };
  if (dk < 1 || dv < 1 || dk > 128 || dv > 256) return {dk, dv, false, compiled(dk, dv) && dk >= 1};
  if (compiled(dk, dv)) return {dk, dv, false, true};
  for (int64_t k2 = 32; k2 <= 128; k2 *= 2) {
    if (k2 < dk) continue;
    for (int64_t v2 = (dv + 63) / 64 * 64; v2 <= 256; v2 += 64)
      if (compiled(k2, v2)) return {k2, v2, true, true};
  }
  return {dk, dv, false, false};
}

// Sub-allocation of a workspace in 256-byte aligned pieces.
struct Arena {
  size_t off = 0;
  size_t take(size_t bytes) {
    const size_t at = off;
    off += align_up(bytes, 256);
    return at;
  }
};

omx::PadView pv(const void* p, int64_t G, int64_t E, int64_t rs, int64_t gs) {
  return omx::PadView{p, (int)G, (int)E, (long long)rs, (long long)gs};
}

// [R][G][E] -> [R][G2][E2] copy with zero fill (or the reverse, cropping)
hipError_t pad3(const void* src, int64_t G, int64_t E, void* dst, int64_t G2, int64_t E2,
                int64_t R, int esize, hipStream_t st) {
  return omx::launch_pad_copy(pv(src, G, E, G * E, E), pv(dst, G2, E2, G2 * E2, E2), R, esize, st);
}

// the channel blocks [q Hk*dk | k Hk*dk | v Hv*dv] of R rows of `per` values per channel
// (mixed_qkv: per = 1; conv weights: per = K; conv caches: per = K - 1), re-laid at
// (dk2, dv2) with zero channels (or cropped back)
hipError_t pad_channels(const void* src, int64_t dk, int64_t dv, void* dst, int64_t dk2,
                        int64_t dv2, int64_t Hk, int64_t Hv, int64_t R, int64_t per, int esize,
                        hipStream_t st) {
  const int64_t cs = 2 * Hk * dk + Hv * dv, cd = 2 * Hk * dk2 + Hv * dv2;
  hipError_t e = omx::launch_pad_copy(pv(src, 2 * Hk, dk * per, cs * per, dk * per),
                                      pv(dst, 2 * Hk, dk2 * per, cd * per, dk2 * per), R, esize, st);
  if (e != hipSuccess) return e;
  const char* s2 = (const char*)src + 2 * Hk * dk * per * esize;
  char* d2 = (char*)dst + 2 * Hk * dk2 * per * esize;
  return omx::launch_pad_copy(pv(s2, Hv, dv * per, cs * per, dv * per),
                              pv(d2, Hv, dv2 * per, cd * per, dv2 * per), R, esize, st);
}

}  // namespace

extern "C" {

const char* omx_gdn_last_error(void) { return g_last_error.c_str(); }

int omx_gdn_abi_version(void) { return 104; }

int omx_gdn_decode_step(const void* mixed_qkv, const void* z, const void* a, const void* b,
                        const float* conv_w, const float* A_log, const float* dt_bias,
                        const float* norm_w, float eps, void* conv_state, float* state,
                        void* out, int64_t B, int64_t Hk, int64_t Hv, int64_t dk, int64_t dv,
                        int64_t K, void* stream) {
  const char* fn = "omx_gdn_decode_step";
  int rc = check_heads(fn, Hk, Hv, dk, dv);
  if (rc) return rc;
  REQUIRE(B >= 0 && B <= 65535, "%s: batch %lld out of range [0, 65535]", fn, (long long)B);
  REQUIRE(K >= 2 && K <= 8, "%s: conv kernel size %lld not in [2, 8]", fn, (long long)K);
  REQUIRE(eps >= 0.f && eps < 1.f, "%s: eps %g out of range", fn, (double)eps);
  if (!omx::decode_dims_supported((int)dk, (int)dv))
    return fail(OMX_GDN_EUNSUPPORTED, "%s: head dims dk=%lld dv=%lld not compiled (16/32/64/128)",
                fn, (long long)dk, (long long)dv);
  if (Hv / Hk > omx::decode_max_gqa())
    return fail(OMX_GDN_EUNSUPPORTED, "%s: gqa factor %lld above %d", fn, (long long)(Hv / Hk),
                omx::decode_max_gqa());
  if (B == 0) return ok();
  REQUIRE(mixed_qkv && z && a && b && conv_w && A_log && dt_bias && norm_w && conv_state &&
              state && out,
          "%s: a required pointer is NULL", fn);
  REQUIRE(aligned(state, 16), "%s: state must be 16-byte aligned", fn);
  omx::DecodeParams p{};
  p.mixed_qkv = mixed_qkv; p.z = z; p.a = a; p.b = b; p.conv_w = conv_w; p.A_log = A_log;
  p.dt_bias = dt_bias; p.norm_w = norm_w; p.conv_state = conv_state; p.out = out;
  p.state = state;
  p.B = (int)B; p.Hk = (int)Hk; p.Hv = (int)Hv; p.dk = (int)dk; p.dv = (int)dv;
  p.conv_k = (int)K; p.scale = 1.0f / sqrtf((float)dk); p.eps = eps;
  return launch_status(omx::launch_decode(p, true, true, (hipStream_t)stream), fn);
}

int omx_gdn_recurrent_step(const void* q, const void* k, const void* v, int in_dtype,
                           const float* g, const float* beta, float* state, float* o, int64_t B,
                           int64_t Hk, int64_t Hv, int64_t dk, int64_t dv, float scale,
                           void* stream) {
  const char* fn = "omx_gdn_recurrent_step";
  int rc = check_heads(fn, Hk, Hv, dk, dv);
  if (rc) return rc;
  REQUIRE(in_dtype == OMX_GDN_F32 || in_dtype == OMX_GDN_BF16, "%s: unknown in_dtype %d", fn,
          in_dtype);
  REQUIRE(B >= 0 && B <= 65535, "%s: batch %lld out of range [0, 65535]", fn, (long long)B);
  if (!omx::decode_dims_supported((int)dk, (int)dv))
    return fail(OMX_GDN_EUNSUPPORTED, "%s: head dims dk=%lld dv=%lld not compiled (16/32/64/128)",
                fn, (long long)dk, (long long)dv);
  if (B == 0) return ok();
  REQUIRE(q && k && v && g && beta && state && o, "%s: a required pointer is NULL", fn);
  REQUIRE(aligned(state, 16), "%s: state must be 16-byte aligned", fn);
  omx::DecodeParams p{};
  p.q = q; p.k = k; p.v = v; p.g = g; p.beta = beta; p.o = o; p.state = state;
  p.B = (int)B; p.Hk = (int)Hk; p.Hv = (int)Hv; p.dk = (int)dk; p.dv = (int)dv;
  p.scale = scale; p.eps = 0.f;
  return launch_status(
      omx::launch_decode(p, false, in_dtype == OMX_GDN_BF16, (hipStream_t)stream), fn);
}

int omx_gdn_qkv_conv_proj(const void* x, const void* w, const float* conv_w, void* out,
                          int64_t M, int64_t D, int64_t N, int64_t T, int64_t K, int conv,
                          void* stream) {
  const char* fn = "omx_gdn_qkv_conv_proj";
  REQUIRE(M >= 0, "%s: row count %lld is negative", fn, (long long)M);
  REQUIRE(D > 0 && D % omx::qkv_proj_tile_depth() == 0,
          "%s: D=%lld must be a positive multiple of %d", fn, (long long)D,
          omx::qkv_proj_tile_depth());
  REQUIRE(N > 0 && N % omx::qkv_proj_tile_cols() == 0,
          "%s: N=%lld must be a positive multiple of %d", fn, (long long)N,
          omx::qkv_proj_tile_cols());
  // 32-bit byte offsets inside the kernel: x, W and out each under 2 GiB
  REQUIRE(M * D < ((int64_t)1 << 30) && N * D < ((int64_t)1 << 30) && M * N < ((int64_t)1 << 30),
          "%s: x, W or out exceeds 2 GiB (M=%lld D=%lld N=%lld)", fn, (long long)M, (long long)D,
          (long long)N);
  REQUIRE(conv == 0 || conv == 1, "%s: conv must be 0 or 1", fn);
  if (conv) {
    REQUIRE(K == 4, "%s: the conv epilogue takes K=4 taps (got %lld)", fn, (long long)K);
    REQUIRE(T >= 1 && M % T == 0, "%s: M=%lld must be a whole number of sequences of T=%lld rows",
            fn, (long long)M, (long long)T);
  }
  if (M == 0) return ok();
  REQUIRE(x && w && out && (!conv || conv_w), "%s: a required pointer is NULL", fn);
  REQUIRE(aligned(x, 16) && aligned(w, 16) && aligned(out, 16) && (!conv || aligned(conv_w, 16)),
          "%s: x, w, out and conv_w must be 16-byte aligned", fn);
  return launch_status(omx::launch_qkv_proj(x, w, conv_w, out, (long long)M, (int)N, (int)D,
                                            (long long)T, conv != 0, (hipStream_t)stream),
                       fn);
}

int omx_gdn_ab_proj(const void* x, const void* w_a, const void* w_b, void* a, void* b,
                    int64_t M, int64_t D, int64_t Hv, void* stream) {
  const char* fn = "omx_gdn_ab_proj";
  REQUIRE(M >= 0 && M <= (int64_t)1 << 40, "%s: row count %lld out of range", fn, (long long)M);
  REQUIRE(D > 0 && D % 8 == 0 && D <= (1 << 20), "%s: D=%lld must be a positive multiple of 8",
          fn, (long long)D);
  REQUIRE(Hv >= 1 && Hv <= omx::ab_proj_max_heads(), "%s: Hv=%lld out of range [1, %d]", fn,
          (long long)Hv, omx::ab_proj_max_heads());
  if (M == 0) return ok();
  REQUIRE(x && w_a && w_b && a && b, "%s: a required pointer is NULL", fn);
  REQUIRE(aligned(x, 16) && aligned(w_a, 16) && aligned(w_b, 16),
          "%s: x, w_a and w_b must be 16-byte aligned", fn);
  return launch_status(omx::launch_ab_proj(x, w_a, w_b, a, b, (long long)M, (int)D, (int)Hv,
                                           (hipStream_t)stream),
                       fn);
}

}  // extern "C"

// ---------------------------------------------------------------------------- prefill
namespace {

// Point the kernels at the workspace and launch: chunk plan (packed sequences),
// preparation over all chunks, then the scan; all on `stream`, in order.
void setup_chunked(omx::ChunkParams& p, const ChunkWs& ws, void* workspace, int mode) {
  char* base = (char*)workspace;
  p.nch = (p.T + 63) / 64;
  p.n_rec = p.cu_seqlens ? (int)((p.T + 63) / 64 + p.N) : p.N * p.nch;
  p.rec = (unsigned char*)(base + ws.rec);
  p.chunk_off = p.cu_seqlens ? (int32_t*)(base + ws.off) : nullptr;
  // the kernels after the plan read its ordered copy of the offsets
  p.cu_in = p.cu_seqlens;
  p.seq_order = p.cu_seqlens ? (const int32_t*)(base + ws.ord) : nullptr;
  if (p.cu_seqlens) p.cu_seqlens = (const int32_t*)(base + ws.cu);
  const bool norm = p.qk_l2norm || mode == omx::kModeLayer;
  p.kn = norm ? base + ws.kn : nullptr;
  p.qn = norm ? base + ws.qn : nullptr;
  if (norm) {
    p.ks = p.kn;
    p.qs = p.qn;
    p.ks_ld = p.qs_ld = (long long)p.Hk * p.dk;
  } else {
    p.ks = p.k;
    p.qs = p.q;
    p.ks_ld = p.k_ld;
    p.qs_ld = p.q_ld;
  }
  if (mode == omx::kModeLayer) {
    p.vc = omx::layer_scan_forms_v(p.dk) ? nullptr : base + ws.vc;
    p.vs = p.vc;
    p.vs_ld = (long long)p.Hv * p.DV;
    p.ss_xch = (unsigned*)(base + ws.xch);
    p.ss_xch_slots = omx::layer_scan_blocks(p);
  } else {
    p.vs = p.v;
    p.vs_ld = p.v_ld;
  }
}

hipError_t launch_chunked(omx::ChunkParams& p, const ChunkWs& ws, void* workspace, int mode,
                          hipStream_t stream) {
  setup_chunked(p, ws, workspace, mode);
  hipError_t e = hipSuccess;
  if (p.cu_seqlens) e = omx::launch_chunk_plan(p, stream);
  if (e == hipSuccess) e = omx::launch_prep(p, mode, stream);
  if (e == hipSuccess) e = omx::launch_scan(p, mode, stream);
  return e;
}

// The chunked rule at compiled head dims (omx_gdn_chunk_fwd pads other dims around it).
int chunk_fwd_core(const char* fn, const void* q, const void* k, const void* v, int in_dtype,
                   const float* g, const float* beta, const float* initial_state,
                   const int32_t* cu_seqlens, int64_t N, float* o, float* final_state, int64_t B,
                   int64_t T, int64_t Hk, int64_t Hv, int64_t dk, int64_t dv, int64_t chunk_size,
                   float scale, int qk_l2norm, void* workspace, size_t workspace_bytes,
                   void* stream) {
  int rc = check_heads(fn, Hk, Hv, dk, dv);
  if (rc) return rc;
  REQUIRE(in_dtype == OMX_GDN_F32 || in_dtype == OMX_GDN_BF16, "%s: unknown in_dtype %d", fn,
          in_dtype);
  REQUIRE(chunk_size == 64, "%s: chunk_size must be 64 (got %lld)", fn, (long long)chunk_size);
  REQUIRE(B >= 0 && T >= 0, "%s: negative shape (B=%lld, T=%lld)", fn, (long long)B, (long long)T);
  REQUIRE(B * T <= (int64_t)1 << 31, "%s: too many tokens (%lld)", fn, (long long)(B * T));
  REQUIRE(std::isfinite(scale), "%s: scale must be finite", fn);
  if (cu_seqlens) {
    REQUIRE(B == 1, "%s: cu_seqlens requires batch 1 (got %lld)", fn, (long long)B);
    REQUIRE(N >= 1 && N <= (1 << 20), "%s: sequence count %lld out of range", fn, (long long)N);
  } else {
    REQUIRE(N == B, "%s: without cu_seqlens N must equal B (%lld vs %lld)", fn, (long long)N,
            (long long)B);
  }
  const bool f32 = in_dtype == OMX_GDN_F32;
  if (!omx::chunk_dims_supported((int)dk, (int)dv, f32))
    return fail(OMX_GDN_EUNSUPPORTED,
                "%s: head dims dk=%lld dv=%lld not supported for %s inputs (dk <= 128, dv <= 256)",
                fn, (long long)dk, (long long)dv, f32 ? "fp32" : "bf16");
  const int mode = f32 ? omx::kModeF32 : omx::kModeBF16;
  const ChunkWs ws = chunk_ws(B, T, Hk, Hv, dk, dv, N, mode);
  REQUIRE(workspace_bytes >= ws.total, "%s: workspace of %zu bytes is smaller than the %zu needed",
          fn, workspace_bytes, ws.total);
  if (N == 0 || (B * T == 0 && !final_state)) return ok();
  REQUIRE(workspace && aligned(workspace, 16), "%s: workspace must be non-NULL and 16-byte aligned",
          fn);
  REQUIRE(o || B * T == 0, "%s: o is NULL", fn);
  if (B * T > 0) REQUIRE(q && k && v && g && beta, "%s: a required pointer is NULL", fn);
  const size_t al = f32 ? 16 : 16;
  REQUIRE(!q || (aligned(q, al) && aligned(k, al) && aligned(v, al)),
          "%s: q, k, v must be 16-byte aligned", fn);
  omx::ChunkParams p{};
  p.q = q; p.k = k; p.v = v;
  p.q_ld = Hk * dk; p.k_ld = Hk * dk; p.v_ld = Hv * dv;
  p.g = g; p.beta = beta; p.o = o;
  p.initial_state = initial_state; p.final_state = final_state; p.cu_seqlens = cu_seqlens;
  p.N = (int)N; p.T = (int)T; p.Hk = (int)Hk; p.Hv = (int)Hv; p.dk = (int)dk; p.DV = (int)dv;
  p.nb = (int)(dv / omx::chunk_block_cols());
  p.scale = scale; p.qk_l2norm = qk_l2norm ? 1 : 0;
  REQUIRE((int64_t)p.N * p.Hv * p.nb <= INT32_MAX, "%s: grid too large", fn);
  REQUIRE(((B * T + 63) / 64 + N) * Hk <= INT32_MAX, "%s: grid too large", fn);
  return launch_status(launch_chunked(p, ws, workspace, mode, (hipStream_t)stream), fn);
}

// Checks every entry point of the chunked path makes before looking at head dims.
int chunk_shape_check(const char* fn, int64_t Hk, int64_t Hv, int64_t dk, int64_t dv,
                      int64_t chunk_size, int64_t B, int64_t T, const int32_t* cu_seqlens,
                      int64_t N) {
  int rc = check_heads(fn, Hk, Hv, dk, dv);
  if (rc) return rc;
  REQUIRE(chunk_size == 64, "%s: chunk_size must be 64 (got %lld)", fn, (long long)chunk_size);
  REQUIRE(B >= 0 && T >= 0, "%s: negative shape (B=%lld, T=%lld)", fn, (long long)B, (long long)T);
  REQUIRE(B * T <= (int64_t)1 << 31, "%s: too many tokens (%lld)", fn, (long long)(B * T));
  if (cu_seqlens) {
    REQUIRE(B == 1, "%s: cu_seqlens requires batch 1 (got %lld)", fn, (long long)B);
    REQUIRE(N >= 1 && N <= (1 << 20), "%s: sequence count %lld out of range", fn, (long long)N);
  } else {
    REQUIRE(N == B, "%s: without cu_seqlens N must equal B (%lld vs %lld)", fn, (long long)N,
            (long long)B);
  }
  return OMX_GDN_OK;
}

// Workspace of a padded core forward: q, k, v, o, initial and final state at the padded
// dims, then the workspace of the call at those dims.
struct FwdPadWs {
  size_t q, k, v, o, s0, s1, inner, total;
};
FwdPadWs fwd_pad_ws(int64_t B, int64_t T, int64_t Hk, int64_t Hv, int64_t dk2, int64_t dv2,
                    int64_t N, bool f32) {
  FwdPadWs w{};
  if (B < 0 || T < 0 || N < 0) return w;
  const size_t tok = (size_t)(B * T), esz = f32 ? 4 : 2, st = (size_t)(N * Hv * dk2 * dv2) * 4;
  Arena a;
  w.q = a.take(tok * Hk * dk2 * esz);
  w.k = a.take(tok * Hk * dk2 * esz);
  w.v = a.take(tok * Hv * dv2 * esz);
  w.o = a.take(tok * Hv * dv2 * 4);
  w.s0 = a.take(st);
  w.s1 = a.take(st);
  w.inner = a.off;
  w.total = w.inner + chunk_ws(B, T, Hk, Hv, dk2, dv2, N, f32 ? omx::kModeF32 : omx::kModeBF16).total;
  return w;
}

}  // namespace

extern "C" {

size_t omx_gdn_chunk_fwd_workspace_size(int64_t B, int64_t T, int64_t Hk, int64_t Hv, int64_t dk,
                                        int64_t dv, int64_t N, int in_dtype) {
  const bool f32 = in_dtype == OMX_GDN_F32;
  const HeadDims hd = head_dims(kCoreFwd, dk, dv, f32);
  if (hd.pad) return fwd_pad_ws(B, T, Hk, Hv, hd.dk, hd.dv, N, f32).total;
  return chunk_ws(B, T, Hk, Hv, dk, dv, N, f32 ? omx::kModeF32 : omx::kModeBF16).total;
}

int omx_gdn_chunk_fwd(const void* q, const void* k, const void* v, int in_dtype, const float* g,
                      const float* beta, const float* initial_state, const int32_t* cu_seqlens,
                      int64_t N, float* o, float* final_state, int64_t B, int64_t T, int64_t Hk,
                      int64_t Hv, int64_t dk, int64_t dv, int64_t chunk_size, float scale,
                      int qk_l2norm, void* workspace, size_t workspace_bytes, void* stream) {
  const char* fn = "omx_gdn_chunk_fwd";
  const bool f32 = in_dtype == OMX_GDN_F32;
  const HeadDims hd = head_dims(kCoreFwd, dk, dv, f32);
  if (!hd.pad)
    return chunk_fwd_core(fn, q, k, v, in_dtype, g, beta, initial_state, cu_seqlens, N, o,
                          final_state, B, T, Hk, Hv, dk, dv, chunk_size, scale, qk_l2norm,
                          workspace, workspace_bytes, stream);
  // head dims the kernels are not compiled for: run on zero-padded copies
  int rc = chunk_shape_check(fn, Hk, Hv, dk, dv, chunk_size, B, T, cu_seqlens, N);
  if (rc) return rc;
  REQUIRE(in_dtype == OMX_GDN_F32 || in_dtype == OMX_GDN_BF16, "%s: unknown in_dtype %d", fn,
          in_dtype);
  const FwdPadWs w = fwd_pad_ws(B, T, Hk, Hv, hd.dk, hd.dv, N, f32);
  REQUIRE(workspace_bytes >= w.total, "%s: workspace of %zu bytes is smaller than the %zu needed",
          fn, workspace_bytes, w.total);
  if (N == 0 || (B * T == 0 && !final_state)) return ok();
  REQUIRE(workspace && aligned(workspace, 16), "%s: workspace must be non-NULL and 16-byte aligned",
          fn);
  if (B * T > 0) REQUIRE(q && k && v && g && beta && o, "%s: a required pointer is NULL", fn);
  char* base = (char*)workspace;
  hipStream_t st = (hipStream_t)stream;
  const int esz = f32 ? 4 : 2;
  const int64_t tok = B * T, dk2 = hd.dk, dv2 = hd.dv;
  hipError_t e = hipSuccess;
  if (tok > 0) {
    e = pad3(q, Hk, dk, base + w.q, Hk, dk2, tok, esz, st);
    if (e == hipSuccess) e = pad3(k, Hk, dk, base + w.k, Hk, dk2, tok, esz, st);
    if (e == hipSuccess) e = pad3(v, Hv, dv, base + w.v, Hv, dv2, tok, esz, st);
  }
  if (e == hipSuccess && initial_state)
    e = pad3(initial_state, dk, dv, base + w.s0, dk2, dv2, N * Hv, 4, st);
  if (e != hipSuccess) return launch_status(e, fn);
  rc = chunk_fwd_core(fn, base + w.q, base + w.k, base + w.v, in_dtype, g, beta,
                      initial_state ? (const float*)(base + w.s0) : nullptr, cu_seqlens, N,
                      (float*)(base + w.o), final_state ? (float*)(base + w.s1) : nullptr, B, T,
                      Hk, Hv, dk2, dv2, chunk_size, scale, qk_l2norm, base + w.inner,
                      workspace_bytes - w.inner, stream);
  if (rc) return rc;
  if (tok > 0) e = pad3(base + w.o, Hv, dv2, o, Hv, dv, tok, 4, st);
  if (e == hipSuccess && final_state)
    e = pad3(base + w.s1, dk2, dv2, final_state, dk, dv, N * Hv, 4, st);
  return launch_status(e, fn);
}

}  // extern "C"

namespace {

// The layer prefill at compiled head dims.  dk_real and dv_real are the caller's head dims
// (they differ from dk, dv when the buffers are zero-padded copies): q is scaled by
// dk_real^-1/2 and the gated norm's mean divides by dv_real.
int prefill_core(const char* fn, const void* mixed_qkv, const void* z, const void* a,
                 const void* b, const float* conv_w, const float* A_log, const float* dt_bias,
                 const float* norm_w, float eps, const int32_t* cu_seqlens, int64_t N,
                 const float* initial_state, float* final_state, const void* conv_state_in,
                 void* conv_state_out, void* out, int64_t B, int64_t T, int64_t Hk,
                 int64_t Hv, int64_t dk, int64_t dv, int64_t K, int64_t chunk_size,
                 void* workspace, size_t workspace_bytes, void* stream, int64_t dk_real,
                 int64_t dv_real, bool dry = false) {
  int rc = check_heads(fn, Hk, Hv, dk, dv);
  if (rc) return rc;
  REQUIRE(chunk_size == 64, "%s: chunk_size must be 64 (got %lld)", fn, (long long)chunk_size);
  REQUIRE(K >= 2 && K <= 4, "%s: conv kernel size %lld not in [2, 4]", fn, (long long)K);
  REQUIRE(B >= 0 && T >= 0, "%s: negative shape (B=%lld, T=%lld)", fn, (long long)B, (long long)T);
  REQUIRE(B * T <= (int64_t)1 << 31, "%s: too many tokens (%lld)", fn, (long long)(B * T));
  REQUIRE(eps >= 0.f && eps < 1.f, "%s: eps %g out of range", fn, (double)eps);
  if (cu_seqlens) {
    REQUIRE(B == 1, "%s: cu_seqlens requires batch 1 (got %lld)", fn, (long long)B);
    REQUIRE(N >= 1 && N <= (1 << 20), "%s: sequence count %lld out of range", fn, (long long)N);
  } else {
    REQUIRE(N == B, "%s: without cu_seqlens N must equal B (%lld vs %lld)", fn, (long long)N,
            (long long)B);
  }
  if (!omx::layer_dims_supported((int)dk, (int)dv))
    return fail(OMX_GDN_EUNSUPPORTED,
                "%s: head dims dk=%lld dv=%lld not supported (dk <= 128, dv <= 256)", fn,
                (long long)dk, (long long)dv);
  const ChunkWs ws = chunk_ws(B, T, Hk, Hv, dk, dv, N, omx::kModeLayer);
  const size_t need = ws.total;
  REQUIRE(workspace_bytes >= need, "%s: workspace of %zu bytes is smaller than the %zu needed", fn,
          workspace_bytes, need);
  if (N == 0) return ok();
  const int64_t tokens = B * T;
  if (tokens > 0)
    REQUIRE(mixed_qkv && z && a && b && out, "%s: an activation pointer is NULL", fn);
  REQUIRE(conv_w && A_log && dt_bias && norm_w, "%s: a parameter pointer is NULL", fn);
  REQUIRE(workspace && aligned(workspace, 16), "%s: workspace must be non-NULL and 16-byte aligned",
          fn);
  REQUIRE(!mixed_qkv || (aligned(mixed_qkv, 16) && aligned(z, 16) && aligned(out, 16)),
          "%s: mixed_qkv, z and out must be 16-byte aligned", fn);
  REQUIRE(aligned(norm_w, 16) && aligned(conv_w, 16), "%s: norm_w and conv_w must be 16-byte aligned",
          fn);
  REQUIRE(N * Hv * (dv / omx::chunk_block_cols()) <= INT32_MAX, "%s: grid too large", fn);
  REQUIRE(((B * T + 63) / 64 + N) * Hk <= INT32_MAX, "%s: grid too large", fn);
  if (dry) return ok();  // every host check passed; nothing is enqueued
  omx::ChunkParams p{};
  p.mixed_qkv = mixed_qkv; p.z = z; p.a = a; p.b = b;
  p.conv_w = conv_w; p.A_log = A_log; p.dt_bias = dt_bias; p.norm_w = norm_w;
  p.conv_state_in = conv_state_in; p.conv_state_out = conv_state_out; p.out = out;
  p.initial_state = initial_state; p.final_state = final_state; p.cu_seqlens = cu_seqlens;
  p.N = (int)N; p.T = (int)T; p.Hk = (int)Hk; p.Hv = (int)Hv; p.dk = (int)dk; p.DV = (int)dv;
  p.nb = (int)(dv / omx::chunk_block_cols());
  p.conv_k = (int)K;
  p.conv_dim = (int)(2 * Hk * dk + Hv * dv);
  p.scale = 1.0f / sqrtf((float)dk_real);
  p.eps = eps;
  p.qk_l2norm = 1;
  p.o_part = (char*)workspace + ws.opart;
  p.o_ss = (float*)((char*)workspace + ws.oss);
  p.inv_dv = 1.0f / (float)dv_real;
  hipError_t e = launch_chunked(p, ws, workspace, omx::kModeLayer, (hipStream_t)stream);
  // the scan applies the gated norm itself for one-round grids; else the epilogue kernel
  if (e == hipSuccess && !omx::layer_scan_fuses_norm(p))
    e = omx::launch_norm_epilogue(p.o_part, p.o_ss, omx::layer_ss_slots(p), z, norm_w, out,
                                  tokens, (int)Hv, (int)dv, (int)dv_real, eps,
                                  (hipStream_t)stream);
  return launch_status(e, fn);
}

// Workspace of a padded layer prefill: mixed_qkv, z, the output, conv weights, norm weight,
// initial and final state and the conv caches in and out at the padded dims (conv caches
// and weights sized for K = 4, the largest the prefill takes), then the call's workspace.
struct LayerPadWs {
  size_t x, z, out, cw, nw, s0, s1, c0, c1, inner, total;
};
LayerPadWs layer_pad_ws(int64_t B, int64_t T, int64_t Hk, int64_t Hv, int64_t dk2, int64_t dv2,
                        int64_t N) {
  LayerPadWs w{};
  if (B < 0 || T < 0 || N < 0) return w;
  const size_t tok = (size_t)(B * T), cd = (size_t)(2 * Hk * dk2 + Hv * dv2);
  const size_t st = (size_t)(N * Hv * dk2 * dv2) * 4;
  Arena a;
  w.x = a.take(tok * cd * 2);
  w.z = a.take(tok * Hv * dv2 * 2);
  w.out = a.take(tok * Hv * dv2 * 2);
  w.cw = a.take(cd * 4 * 4);
  w.nw = a.take(dv2 * 4);
  w.s0 = a.take(st);
  w.s1 = a.take(st);
  w.c0 = a.take((size_t)N * cd * 3 * 2);
  w.c1 = a.take((size_t)N * cd * 3 * 2);
  w.inner = a.off;
  w.total = w.inner + chunk_ws(B, T, Hk, Hv, dk2, dv2, N, omx::kModeLayer).total;
  return w;
}

size_t prefill_ws_bytes(int64_t B, int64_t T, int64_t Hk, int64_t Hv, int64_t dk, int64_t dv,
                        int64_t N) {
  const HeadDims hd = head_dims(kLayerFwd, dk, dv, false);
  if (hd.pad) return layer_pad_ws(B, T, Hk, Hv, hd.dk, hd.dv, N).total;
  return chunk_ws(B, T, Hk, Hv, dk, dv, N, omx::kModeLayer).total;
}

// Stand-in workspace address for a validate-only pass (`dry`): it is aligned and never
// dereferenced or handed to HIP, because a dry pass returns before enqueueing anything.
alignas(256) unsigned char g_dry_workspace[256];

// The layer prefill behind omx_gdn_prefill and omx_gdn_prefill_noalloc (`fn` names the
// entry point in error messages): at compiled head dims directly, else on zero-padded
// copies.  With `dry` it runs every host check and returns before the first HIP call
// (the workspace pointer is then not looked at).
int prefill_entry(const char* fn, const void* mixed_qkv, const void* z, const void* a,
                  const void* b, const float* conv_w, const float* A_log, const float* dt_bias,
                  const float* norm_w, float eps, const int32_t* cu_seqlens, int64_t N,
                  const float* initial_state, float* final_state, const void* conv_state_in,
                  void* conv_state_out, void* out, int64_t B, int64_t T, int64_t Hk,
                  int64_t Hv, int64_t dk, int64_t dv, int64_t K, int64_t chunk_size,
                  void* workspace, size_t workspace_bytes, void* stream, bool dry = false) {
  if (dry) workspace = g_dry_workspace;
  const HeadDims hd = head_dims(kLayerFwd, dk, dv, false);
  if (!hd.pad)
    return prefill_core(fn, mixed_qkv, z, a, b, conv_w, A_log, dt_bias, norm_w, eps, cu_seqlens,
                        N, initial_state, final_state, conv_state_in, conv_state_out, out, B, T,
                        Hk, Hv, dk, dv, K, chunk_size, workspace, workspace_bytes, stream, dk, dv,
                        dry);
  int rc = chunk_shape_check(fn, Hk, Hv, dk, dv, chunk_size, B, T, cu_seqlens, N);
  if (rc) return rc;
  REQUIRE(K >= 2 && K <= 4, "%s: conv kernel size %lld not in [2, 4]", fn, (long long)K);
  const LayerPadWs w = layer_pad_ws(B, T, Hk, Hv, hd.dk, hd.dv, N);
  REQUIRE(workspace_bytes >= w.total, "%s: workspace of %zu bytes is smaller than the %zu needed",
          fn, workspace_bytes, w.total);
  if (N == 0) return ok();
  const int64_t tok = B * T, dk2 = hd.dk, dv2 = hd.dv;
  if (tok > 0) REQUIRE(mixed_qkv && z && a && b && out, "%s: an activation pointer is NULL", fn);
  REQUIRE(conv_w && A_log && dt_bias && norm_w, "%s: a parameter pointer is NULL", fn);
  REQUIRE(workspace && aligned(workspace, 16), "%s: workspace must be non-NULL and 16-byte aligned",
          fn);
  char* base = (char*)workspace;
  // the inner call's checks (eps, conv size, grid limits) run before the first copy
  rc = prefill_core(fn, base + w.x, base + w.z, a, b, (const float*)(base + w.cw), A_log, dt_bias,
                    (const float*)(base + w.nw), eps, cu_seqlens, N, nullptr, nullptr, nullptr,
                    nullptr, base + w.out, B, T, Hk, Hv, dk2, dv2, K, chunk_size, base + w.inner,
                    workspace_bytes - w.inner, stream, dk, dv, true);
  if (rc || dry) return rc;
  hipStream_t st = (hipStream_t)stream;
  hipError_t e = hipSuccess;
  if (tok > 0) {
    e = pad_channels(mixed_qkv, dk, dv, base + w.x, dk2, dv2, Hk, Hv, tok, 1, 2, st);
    if (e == hipSuccess) e = pad3(z, Hv, dv, base + w.z, Hv, dv2, tok, 2, st);
  }
  if (e == hipSuccess) e = pad_channels(conv_w, dk, dv, base + w.cw, dk2, dv2, Hk, Hv, 1, K, 4, st);
  if (e == hipSuccess) e = pad3(norm_w, 1, dv, base + w.nw, 1, dv2, 1, 4, st);
  if (e == hipSuccess && initial_state)
    e = pad3(initial_state, dk, dv, base + w.s0, dk2, dv2, N * Hv, 4, st);
  if (e == hipSuccess && conv_state_in)
    e = pad_channels(conv_state_in, dk, dv, base + w.c0, dk2, dv2, Hk, Hv, N, K - 1, 2, st);
  if (e != hipSuccess) return launch_status(e, fn);
  rc = prefill_core(fn, base + w.x, base + w.z, a, b, (const float*)(base + w.cw), A_log, dt_bias,
                    (const float*)(base + w.nw), eps, cu_seqlens, N,
                    initial_state ? (const float*)(base + w.s0) : nullptr,
                    final_state ? (float*)(base + w.s1) : nullptr,
                    conv_state_in ? base + w.c0 : nullptr, conv_state_out ? base + w.c1 : nullptr,
                    base + w.out, B, T, Hk, Hv, dk2, dv2, K, chunk_size, base + w.inner,
                    workspace_bytes - w.inner, stream, dk, dv);
  if (rc) return rc;
  if (tok > 0) e = pad3(base + w.out, Hv, dv2, out, Hv, dv, tok, 2, st);
  if (e == hipSuccess && final_state)
    e = pad3(base + w.s1, dk2, dv2, final_state, dk, dv, N * Hv, 4, st);
  if (e == hipSuccess && conv_state_out)
    e = pad_channels(base + w.c1, dk2, dv2, conv_state_out, dk, dv, Hk, Hv, N, K - 1, 2, st);
  return launch_status(e, fn);
}

// The fixed scratch of omx_gdn_prefill_noalloc: a file-scope device array, so that entry
// point allocates nothing.  Each device holds its own copy (allocated when the library's
// code object is loaded there, kept until the process ends).  Host code never uses the
// array's name as an address: the per-device address comes from hipGetSymbolAddress.
constexpr size_t kNoAllocScratchBytes = size_t(64) << 20;
__device__ __align__(256) unsigned char scratch[kNoAllocScratchBytes];

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices] = {};

// The current device's scratch address (looked up once per device, with it current).
int scratch_for_current_device(const char* fn, void** out) {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return fail(OMX_GDN_ELAUNCH, "%s: hipGetDevice failed: %s", fn, hipGetErrorString(e));
  if (dev < 0 || dev >= kMaxDevices)
    return fail(OMX_GDN_EUNSUPPORTED, "%s: device index %d above %d", fn, dev, kMaxDevices - 1);
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    void* ptr = nullptr;
    e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !ptr)
      return fail(OMX_GDN_ELAUNCH, "%s: hipGetSymbolAddress of the scratch array failed on device %d: %s",
                  fn, dev, hipGetErrorString(e));
    g_scratch_ptr[dev] = ptr;
  }
  *out = g_scratch_ptr[dev];
  return OMX_GDN_OK;
}

}  // namespace

extern "C" {

size_t omx_gdn_prefill_workspace_size(int64_t B, int64_t T, int64_t Hk, int64_t Hv, int64_t dk,
                                      int64_t dv, int64_t N) {
  return prefill_ws_bytes(B, T, Hk, Hv, dk, dv, N);
}

int omx_gdn_prefill(const void* mixed_qkv, const void* z, const void* a, const void* b,
                    const float* conv_w, const float* A_log, const float* dt_bias,
                    const float* norm_w, float eps, const int32_t* cu_seqlens, int64_t N,
                    const float* initial_state, float* final_state, const void* conv_state_in,
                    void* conv_state_out, void* out, int64_t B, int64_t T, int64_t Hk,
                    int64_t Hv, int64_t dk, int64_t dv, int64_t K, int64_t chunk_size,
                    void* workspace, size_t workspace_bytes, void* stream) {
  return prefill_entry("omx_gdn_prefill", mixed_qkv, z, a, b, conv_w, A_log, dt_bias, norm_w,
                       eps, cu_seqlens, N, initial_state, final_state, conv_state_in,
                       conv_state_out, out, B, T, Hk, Hv, dk, dv, K, chunk_size, workspace,
                       workspace_bytes, stream);
}

size_t omx_gdn_prefill_noalloc_max_scratch(void) { return kNoAllocScratchBytes; }

int omx_gdn_prefill_noalloc(const void* mixed_qkv, const void* z, const void* a, const void* b,
                            const float* conv_w, const float* A_log, const float* dt_bias,
                            const float* norm_w, float eps, const int32_t* cu_seqlens, int64_t N,
                            const float* initial_state, float* final_state,
                            const void* conv_state_in, void* conv_state_out, void* out, int64_t B,
                            int64_t T, int64_t Hk, int64_t Hv, int64_t dk, int64_t dv, int64_t K,
                            int64_t chunk_size, void* stream) {
  const char* fn = "omx_gdn_prefill_noalloc";
  const size_t need = omx_gdn_prefill_workspace_size(B, T, Hk, Hv, dk, dv, N);
  REQUIRE(need <= kNoAllocScratchBytes,
          "%s: these shapes need %zu bytes of scratch, above the fixed %zu (call omx_gdn_prefill "
          "with a workspace instead)",
          fn, need, kNoAllocScratchBytes);
  // every argument check before the first HIP call (the device query below included)
  int rc = prefill_entry(fn, mixed_qkv, z, a, b, conv_w, A_log, dt_bias, norm_w, eps, cu_seqlens,
                         N, initial_state, final_state, conv_state_in, conv_state_out, out, B, T,
                         Hk, Hv, dk, dv, K, chunk_size, nullptr, kNoAllocScratchBytes, stream, true);
  if (rc) return rc;
  void* ws = nullptr;
  rc = scratch_for_current_device(fn, &ws);
  if (rc) return rc;
  return prefill_entry(fn, mixed_qkv, z, a, b, conv_w, A_log, dt_bias, norm_w, eps, cu_seqlens,
                       N, initial_state, final_state, conv_state_in, conv_state_out, out, B, T,
                       Hk, Hv, dk, dv, K, chunk_size, ws, kNoAllocScratchBytes, stream);
}

}  // extern "C"

// ---------------------------------------------------------------------------- backward
extern "C" {

}  // extern "C"

namespace {

// The rule's backward at compiled head dims (omx_gdn_chunk_bwd pads other dims around it).
int chunk_bwd_core(const char* fn, const void* q, const void* k, const void* v, int in_dtype,
                   const float* g, const float* beta, const float* initial_state,
                   const int32_t* cu_seqlens, int64_t N, const float* d_o,
                   const float* d_final_state, void* dq, void* dk, void* dv, float* dg,
                   float* dbeta, float* d_initial_state, int64_t B, int64_t T, int64_t Hk,
                   int64_t Hv, int64_t dk_dim, int64_t dv_dim, int64_t chunk_size, float scale,
                   int qk_l2norm, void* workspace, size_t workspace_bytes, void* stream) {
  int rc = check_heads(fn, Hk, Hv, dk_dim, dv_dim);
  if (rc) return rc;
  REQUIRE(in_dtype == OMX_GDN_F32 || in_dtype == OMX_GDN_BF16, "%s: unknown in_dtype %d", fn,
          in_dtype);
  REQUIRE(chunk_size == 64, "%s: chunk_size must be 64 (got %lld)", fn, (long long)chunk_size);
  REQUIRE(B >= 0 && T >= 0, "%s: negative shape (B=%lld, T=%lld)", fn, (long long)B, (long long)T);
  REQUIRE(B * T <= (int64_t)1 << 31, "%s: too many tokens (%lld)", fn, (long long)(B * T));
  REQUIRE(std::isfinite(scale), "%s: scale must be finite", fn);
  if (cu_seqlens) {
    REQUIRE(B == 1, "%s: cu_seqlens requires batch 1 (got %lld)", fn, (long long)B);
    REQUIRE(N >= 1 && N <= (1 << 20), "%s: sequence count %lld out of range", fn, (long long)N);
  } else {
    REQUIRE(N == B, "%s: without cu_seqlens N must equal B (%lld vs %lld)", fn, (long long)N,
            (long long)B);
  }
  const bool f32 = in_dtype == OMX_GDN_F32;
  if (!omx::bwd_dims_supported((int)dk_dim, (int)dv_dim, f32))
    return fail(OMX_GDN_EUNSUPPORTED,
                "%s: head dims dk=%lld dv=%lld not supported for %s inputs (dk <= 128, dv <= 128)",
                fn, (long long)dk_dim, (long long)dv_dim, f32 ? "fp32" : "bf16");
  const int mode = f32 ? omx::kModeF32 : omx::kModeBF16;
  const BwdWs ws = bwd_ws(B, T, Hk, Hv, dk_dim, dv_dim, N, mode);
  REQUIRE(workspace_bytes >= ws.total, "%s: workspace of %zu bytes is smaller than the %zu needed",
          fn, workspace_bytes, ws.total);
  if (N == 0) return ok();
  REQUIRE(workspace && aligned(workspace, 16), "%s: workspace must be non-NULL and 16-byte aligned",
          fn);
  if (B * T > 0) {
    REQUIRE(q && k && v && g && beta && d_o && dq && dk && dv && dg && dbeta,
            "%s: a required pointer is NULL", fn);
    REQUIRE(aligned(q, 16) && aligned(k, 16) && aligned(v, 16) && aligned(d_o, 16),
            "%s: q, k, v and d_o must be 16-byte aligned", fn);
  }
  omx::ChunkParams p{};
  p.q = q; p.k = k; p.v = v;
  p.q_ld = Hk * dk_dim; p.k_ld = Hk * dk_dim; p.v_ld = Hv * dv_dim;
  p.g = g; p.beta = beta; p.o = nullptr;
  p.initial_state = initial_state; p.final_state = nullptr; p.cu_seqlens = cu_seqlens;
  p.N = (int)N; p.T = (int)T; p.Hk = (int)Hk; p.Hv = (int)Hv; p.dk = (int)dk_dim;
  p.DV = (int)dv_dim;
  p.nb = (int)(dv_dim / omx::chunk_block_cols());
  p.scale = scale; p.qk_l2norm = qk_l2norm ? 1 : 0;
  REQUIRE((int64_t)p.N * p.Hv * p.nb <= INT32_MAX, "%s: grid too large", fn);
  REQUIRE(((B * T + 63) / 64 + N) * Hv <= INT32_MAX, "%s: grid too large", fn);
  char* base = (char*)workspace;
  setup_chunked(p, ws.f, workspace, mode);
  p.xlpg = (float*)(base + ws.xlpg);
  p.states = (float*)(base + ws.states);
  p.vnew = (float*)(base + ws.vnew);
  hipStream_t st = (hipStream_t)stream;
  hipError_t e = hipSuccess;
  if (p.cu_seqlens) e = omx::launch_chunk_plan(p, st);
  if (e == hipSuccess) e = omx::launch_prep_bwd(p, mode, st);
  if (e == hipSuccess) e = omx::launch_scan_bwd(p, mode, st);
  if (e != hipSuccess) return launch_status(e, fn);
  omx::BwdParams b{};
  b.ks = p.ks; b.qs = p.qs; b.ks_ld = p.ks_ld; b.qs_ld = p.qs_ld;
  b.v = v; b.dO = d_o; b.dht = d_final_state; b.rec = p.rec; b.xlpg = p.xlpg;
  b.states = p.states; b.vnew = p.vnew;
  b.dstates = (float*)(base + ws.dstates);
  b.dvnew = (float*)(base + ws.dvnew);
  b.dh0 = d_initial_state;
  b.dqh = base + ws.dqh;  // sized for fp32; bf16 inputs use the first half
  b.dkh = base + ws.dkh;
  b.dv = dv; b.dg = dg; b.dbeta = dbeta;
  b.q = q; b.k = k; b.dq = dq; b.dk_out = dk;
  b.cu_seqlens = p.cu_seqlens; b.chunk_off = p.chunk_off; b.seq_order = p.seq_order;
  b.N = p.N; b.T = p.T; b.Hk = p.Hk; b.Hv = p.Hv; b.dk = p.dk; b.DV = p.DV; b.nb = p.nb;
  b.nch = p.nch; b.n_rec = p.n_rec; b.in_f32 = f32 ? 1 : 0; b.qk_l2norm = p.qk_l2norm;
  b.scale = scale;
  return launch_status(omx::launch_bwd(b, st), fn);
}

// Workspace of a padded core backward: q, k, v, d_o, initial state, final-state cotangent,
// dq, dk, dv and the initial-state gradient at the padded dims, then the call's workspace.
struct BwdPadWs {
  size_t q, k, v, dO, s0, ds, gq, gk, gv, gs0, inner, total;
};
BwdPadWs bwd_pad_ws(int64_t B, int64_t T, int64_t Hk, int64_t Hv, int64_t dk2, int64_t dv2,
                    int64_t N, bool f32) {
  BwdPadWs w{};
  if (B < 0 || T < 0 || N < 0) return w;
  const size_t tok = (size_t)(B * T), esz = f32 ? 4 : 2, st = (size_t)(N * Hv * dk2 * dv2) * 4;
  Arena a;
  w.q = a.take(tok * Hk * dk2 * esz);
  w.k = a.take(tok * Hk * dk2 * esz);
  w.v = a.take(tok * Hv * dv2 * esz);
  w.dO = a.take(tok * Hv * dv2 * 4);
  w.s0 = a.take(st);
  w.ds = a.take(st);
  w.gq = a.take(tok * Hk * dk2 * esz);
  w.gk = a.take(tok * Hk * dk2 * esz);
  w.gv = a.take(tok * Hv * dv2 * esz);
  w.gs0 = a.take(st);
  w.inner = a.off;
  w.total = w.inner + bwd_ws(B, T, Hk, Hv, dk2, dv2, N, f32 ? omx::kModeF32 : omx::kModeBF16).total;
  return w;
}

}  // namespace

extern "C" {

size_t omx_gdn_chunk_bwd_workspace_size(int64_t B, int64_t T, int64_t Hk, int64_t Hv, int64_t dk,
                                        int64_t dv, int64_t N, int in_dtype) {
  const bool f32 = in_dtype == OMX_GDN_F32;
  const HeadDims hd = head_dims(kCoreBwd, dk, dv, f32);
  if (hd.pad) return bwd_pad_ws(B, T, Hk, Hv, hd.dk, hd.dv, N, f32).total;
  return bwd_ws(B, T, Hk, Hv, dk, dv, N, f32 ? omx::kModeF32 : omx::kModeBF16).total;
}

int omx_gdn_chunk_bwd(const void* q, const void* k, const void* v, int in_dtype, const float* g,
                      const float* beta, const float* initial_state, const int32_t* cu_seqlens,
                      int64_t N, const float* d_o, const float* d_final_state, void* dq, void* dk,
                      void* dv, float* dg, float* dbeta, float* d_initial_state, int64_t B,
                      int64_t T, int64_t Hk, int64_t Hv, int64_t dk_dim, int64_t dv_dim,
                      int64_t chunk_size, float scale, int qk_l2norm, void* workspace,
                      size_t workspace_bytes, void* stream) {
  const char* fn = "omx_gdn_chunk_bwd";
  const bool f32 = in_dtype == OMX_GDN_F32;
  const HeadDims hd = head_dims(kCoreBwd, dk_dim, dv_dim, f32);
  if (!hd.pad)
    return chunk_bwd_core(fn, q, k, v, in_dtype, g, beta, initial_state, cu_seqlens, N, d_o,
                          d_final_state, dq, dk, dv, dg, dbeta, d_initial_state, B, T, Hk, Hv,
                          dk_dim, dv_dim, chunk_size, scale, qk_l2norm, workspace,
                          workspace_bytes, stream);
  int rc = chunk_shape_check(fn, Hk, Hv, dk_dim, dv_dim, chunk_size, B, T, cu_seqlens, N);
  if (rc) return rc;
  REQUIRE(in_dtype == OMX_GDN_F32 || in_dtype == OMX_GDN_BF16, "%s: unknown in_dtype %d", fn,
          in_dtype);
  const BwdPadWs w = bwd_pad_ws(B, T, Hk, Hv, hd.dk, hd.dv, N, f32);
  REQUIRE(workspace_bytes >= w.total, "%s: workspace of %zu bytes is smaller than the %zu needed",
          fn, workspace_bytes, w.total);
  if (N == 0) return ok();
  REQUIRE(workspace && aligned(workspace, 16), "%s: workspace must be non-NULL and 16-byte aligned",
          fn);
  const int64_t tok = B * T, dk2 = hd.dk, dv2 = hd.dv;
  if (tok > 0)
    REQUIRE(q && k && v && g && beta && d_o && dq && dk && dv && dg && dbeta,
            "%s: a required pointer is NULL", fn);
  char* base = (char*)workspace;
  hipStream_t st = (hipStream_t)stream;
  const int esz = f32 ? 4 : 2;
  hipError_t e = hipSuccess;
  if (tok > 0) {
    e = pad3(q, Hk, dk_dim, base + w.q, Hk, dk2, tok, esz, st);
    if (e == hipSuccess) e = pad3(k, Hk, dk_dim, base + w.k, Hk, dk2, tok, esz, st);
    if (e == hipSuccess) e = pad3(v, Hv, dv_dim, base + w.v, Hv, dv2, tok, esz, st);
    if (e == hipSuccess) e = pad3(d_o, Hv, dv_dim, base + w.dO, Hv, dv2, tok, 4, st);
  }
  if (e == hipSuccess && initial_state)
    e = pad3(initial_state, dk_dim, dv_dim, base + w.s0, dk2, dv2, N * Hv, 4, st);
  if (e == hipSuccess && d_final_state)
    e = pad3(d_final_state, dk_dim, dv_dim, base + w.ds, dk2, dv2, N * Hv, 4, st);
  if (e != hipSuccess) return launch_status(e, fn);
  rc = chunk_bwd_core(fn, base + w.q, base + w.k, base + w.v, in_dtype, g, beta,
                      initial_state ? (const float*)(base + w.s0) : nullptr, cu_seqlens, N,
                      (const float*)(base + w.dO),
                      d_final_state ? (const float*)(base + w.ds) : nullptr, base + w.gq,
                      base + w.gk, base + w.gv, dg, dbeta,
                      d_initial_state ? (float*)(base + w.gs0) : nullptr, B, T, Hk, Hv, dk2, dv2,
                      chunk_size, scale, qk_l2norm, base + w.inner, workspace_bytes - w.inner,
                      stream);
  if (rc) return rc;
  if (tok > 0) {
    e = pad3(base + w.gq, Hk, dk2, dq, Hk, dk_dim, tok, esz, st);
    if (e == hipSuccess) e = pad3(base + w.gk, Hk, dk2, dk, Hk, dk_dim, tok, esz, st);
    if (e == hipSuccess) e = pad3(base + w.gv, Hv, dv2, dv, Hv, dv_dim, tok, esz, st);
  }
  if (e == hipSuccess && d_initial_state)
    e = pad3(base + w.gs0, dk2, dv2, d_initial_state, dk_dim, dv_dim, N * Hv, 4, st);
  return launch_status(e, fn);
}

}  // extern "C"

// ---------------------------------------------------------------------------- layer backward
namespace {

// Workspace of the layer backward: the rule's backward workspace, then the recomputed
// conv + SiLU output (q, k, v rows), g and beta, the rule's fp32 o and its cotangent, the
// rule's gradients of q, k, v, g and beta, and the partial sums of the parameter gradients.
struct LayerBwdWs {
  BwdWs c;
  size_t q, k, v, g, beta, o, dO, gq, gk, gv, dg, dbeta, pn, pg, pc, total;
};

LayerBwdWs layer_bwd_ws(int64_t B, int64_t T, int64_t Hk, int64_t Hv, int64_t dk, int64_t dv,
                        int64_t N) {
  LayerBwdWs w{};
  w.c = bwd_ws(B, T, Hk, Hv, dk, dv, N, omx::kModeBF16);
  if (B < 0 || T < 0 || Hk < 0 || Hv < 0 || dk < 0 || dv < 0 || N < 0) return w;
  const size_t tokens = (size_t)(B * T);
  const size_t kd = (size_t)(Hk * dk), vd = (size_t)(Hv * dv), conv_dim = 2 * kd + vd;
  size_t o = w.c.total;
  auto take = [&](size_t bytes) {
    const size_t at = o;
    o += align_up(bytes, 256);
    return at;
  };
  w.q = take(tokens * kd * 2);
  w.k = take(tokens * kd * 2);
  w.v = take(tokens * vd * 2);
  w.g = take(tokens * (size_t)Hv * 4);
  w.beta = take(tokens * (size_t)Hv * 4);
  w.o = take(tokens * vd * 4);
  w.dO = take(tokens * vd * 4);
  w.gq = take(tokens * kd * 2);
  w.gk = take(tokens * kd * 2);
  w.gv = take(tokens * vd * 2);
  w.dg = take(tokens * (size_t)Hv * 4);
  w.dbeta = take(tokens * (size_t)Hv * 4);
  w.pn = take((size_t)omx::layer_bwd_norm_blocks() * (size_t)dv * 4);
  w.pg = take((size_t)omx::layer_bwd_gate_blocks((long long)tokens) * 2 * (size_t)Hv * 4);
  w.pc = take((size_t)omx::layer_bwd_conv_blocks((long long)tokens) * conv_dim * 4 * 4);
  w.total = o;
  return w;
}

}  // namespace

extern "C" {

}  // extern "C"

namespace {

// The layer backward at compiled head dims; dk_real and dv_real as for prefill_core.
int prefill_bwd_core(const char* fn, const void* mixed_qkv, const void* z, const void* a,
                     const void* b, const float* conv_w, const float* A_log, const float* dt_bias,
                     const float* norm_w, float eps, const int32_t* cu_seqlens, int64_t N,
                     const float* initial_state, const void* d_out, const float* d_final_state,
                     void* d_mixed_qkv, void* dz, void* da, void* db, float* d_conv_w,
                     float* dA_log, float* d_dt_bias, float* d_norm_w, float* d_initial_state,
                     int64_t B, int64_t T, int64_t Hk, int64_t Hv, int64_t dk, int64_t dv,
                     int64_t K, int64_t chunk_size, void* workspace, size_t workspace_bytes,
                     void* stream, int64_t dk_real, int64_t dv_real) {
  int rc = check_heads(fn, Hk, Hv, dk, dv);
  if (rc) return rc;
  REQUIRE(chunk_size == 64, "%s: chunk_size must be 64 (got %lld)", fn, (long long)chunk_size);
  REQUIRE(K == 4, "%s: conv kernel size must be 4 (got %lld)", fn, (long long)K);
  REQUIRE(B >= 0 && T >= 0, "%s: negative shape (B=%lld, T=%lld)", fn, (long long)B, (long long)T);
  REQUIRE(B * T <= (int64_t)1 << 31, "%s: too many tokens (%lld)", fn, (long long)(B * T));
  REQUIRE(eps >= 0.f && eps < 1.f, "%s: eps %g out of range", fn, (double)eps);
  if (cu_seqlens) {
    REQUIRE(B == 1, "%s: cu_seqlens requires batch 1 (got %lld)", fn, (long long)B);
    REQUIRE(N >= 1 && N <= (1 << 20), "%s: sequence count %lld out of range", fn, (long long)N);
  } else {
    REQUIRE(N == B, "%s: without cu_seqlens N must equal B (%lld vs %lld)", fn, (long long)N,
            (long long)B);
  }
  if (!omx::bwd_dims_supported((int)dk, (int)dv, false) || Hv > 256)
    return fail(OMX_GDN_EUNSUPPORTED,
                "%s: dk=%lld dv=%lld Hv=%lld not supported (dk <= 128, dv <= 128, Hv <= 256)",
                fn, (long long)dk, (long long)dv, (long long)Hv);
  const LayerBwdWs ws = layer_bwd_ws(B, T, Hk, Hv, dk, dv, N);
  REQUIRE(workspace_bytes >= ws.total, "%s: workspace of %zu bytes is smaller than the %zu needed",
          fn, workspace_bytes, ws.total);
  if (N == 0) return ok();
  const int64_t tokens = B * T;
  REQUIRE(conv_w && A_log && dt_bias && norm_w && d_conv_w && dA_log && d_dt_bias && d_norm_w,
          "%s: a parameter or parameter-gradient pointer is NULL", fn);
  if (tokens > 0)
    REQUIRE(mixed_qkv && z && a && b && d_out && d_mixed_qkv && dz && da && db,
            "%s: an activation or activation-gradient pointer is NULL", fn);
  REQUIRE(workspace && aligned(workspace, 16), "%s: workspace must be non-NULL and 16-byte aligned",
          fn);
  REQUIRE(!mixed_qkv || (aligned(mixed_qkv, 16) && aligned(d_mixed_qkv, 16)),
          "%s: mixed_qkv and d_mixed_qkv must be 16-byte aligned", fn);
  REQUIRE(!z || (aligned(z, 16) && aligned(d_out, 16) && aligned(dz, 16)),
          "%s: z, d_out and dz must be 16-byte aligned", fn);
  REQUIRE(aligned(conv_w, 16), "%s: conv_w must be 16-byte aligned", fn);
  char* base = (char*)workspace;
  hipStream_t st = (hipStream_t)stream;
  omx::LayerBwdParams lp{};
  lp.x = (const uint16_t*)mixed_qkv; lp.conv_w = conv_w; lp.a = (const uint16_t*)a;
  lp.b = (const uint16_t*)b; lp.A_log = A_log; lp.dt_bias = dt_bias; lp.z = (const uint16_t*)z;
  lp.norm_w = norm_w; lp.dout = (const uint16_t*)d_out; lp.eps = eps;
  lp.q = (uint16_t*)(base + ws.q); lp.k = (uint16_t*)(base + ws.k); lp.v = (uint16_t*)(base + ws.v);
  lp.g = (float*)(base + ws.g); lp.beta = (float*)(base + ws.beta);
  lp.o = (const float*)(base + ws.o); lp.dO = (float*)(base + ws.dO);
  lp.grad_q = (uint16_t*)(base + ws.gq); lp.grad_k = (uint16_t*)(base + ws.gk);
  lp.grad_v = (uint16_t*)(base + ws.gv);
  lp.dg = (const float*)(base + ws.dg); lp.dbeta = (const float*)(base + ws.dbeta);
  lp.part_norm = (float*)(base + ws.pn); lp.part_gates = (float*)(base + ws.pg);
  lp.part_conv = (float*)(base + ws.pc);
  lp.dx = (uint16_t*)d_mixed_qkv; lp.dz = (uint16_t*)dz; lp.da = (uint16_t*)da;
  lp.db = (uint16_t*)db; lp.d_conv_w = d_conv_w; lp.dA_log = dA_log; lp.d_dt_bias = d_dt_bias;
  lp.d_norm_w = d_norm_w; lp.tokens = tokens;
  lp.N = (int)N; lp.T = (int)T; lp.Hk = (int)Hk; lp.Hv = (int)Hv; lp.dk = (int)dk; lp.dv = (int)dv;
  lp.conv_dim = (int)(2 * Hk * dk + Hv * dv);
  lp.dv_mean = (int)dv_real;
  omx::ChunkParams p{};
  p.q = lp.q; p.k = lp.k; p.v = lp.v;
  p.q_ld = Hk * dk; p.k_ld = Hk * dk; p.v_ld = Hv * dv;
  p.g = lp.g; p.beta = lp.beta; p.o = (float*)(base + ws.o);
  p.initial_state = initial_state; p.final_state = nullptr; p.cu_seqlens = cu_seqlens;
  p.N = (int)N; p.T = (int)T; p.Hk = (int)Hk; p.Hv = (int)Hv; p.dk = (int)dk; p.DV = (int)dv;
  p.nb = (int)(dv / omx::chunk_block_cols());
  p.scale = 1.0f / sqrtf((float)dk_real); p.qk_l2norm = 1;
  REQUIRE((int64_t)p.N * p.Hv * p.nb <= INT32_MAX, "%s: grid too large", fn);
  REQUIRE(((B * T + 63) / 64 + N) * Hv <= INT32_MAX, "%s: grid too large", fn);
  setup_chunked(p, ws.c.f, workspace, omx::kModeBF16);
  p.xlpg = (float*)(base + ws.c.xlpg);
  p.states = (float*)(base + ws.c.states);
  p.vnew = (float*)(base + ws.c.vnew);
  // the packed-sequence plan first: every kernel below reads its ordered offsets
  lp.cu_seqlens = p.cu_seqlens;
  hipError_t e = hipSuccess;
  if (p.cu_seqlens) e = omx::launch_chunk_plan(p, st);
  // forward recompute: conv + SiLU, gates, then the rule's prep and scan (keeping o)
  if (e == hipSuccess) e = omx::launch_layer_fwd_pieces(lp, st);
  if (e == hipSuccess) e = omx::launch_prep_bwd(p, omx::kModeBF16, st);
  if (e == hipSuccess) e = omx::launch_scan_bwd(p, omx::kModeBF16, st);
  // the gated norm's adjoint gives the rule's cotangent
  if (e == hipSuccess) e = omx::launch_layer_norm_bwd(lp, st);
  if (e != hipSuccess) return launch_status(e, fn);
  omx::BwdParams bp{};
  bp.ks = p.ks; bp.qs = p.qs; bp.ks_ld = p.ks_ld; bp.qs_ld = p.qs_ld;
  bp.v = lp.v; bp.dO = lp.dO; bp.dht = d_final_state; bp.rec = p.rec; bp.xlpg = p.xlpg;
  bp.states = p.states; bp.vnew = p.vnew;
  bp.dstates = (float*)(base + ws.c.dstates);
  bp.dvnew = (float*)(base + ws.c.dvnew);
  bp.dh0 = d_initial_state;
  bp.dqh = base + ws.c.dqh;
  bp.dkh = base + ws.c.dkh;
  bp.dv = lp.grad_v; bp.dg = (float*)(base + ws.dg); bp.dbeta = (float*)(base + ws.dbeta);
  bp.q = lp.q; bp.k = lp.k; bp.dq = lp.grad_q; bp.dk_out = lp.grad_k;
  bp.cu_seqlens = p.cu_seqlens; bp.chunk_off = p.chunk_off; bp.seq_order = p.seq_order;
  bp.N = p.N; bp.T = p.T; bp.Hk = p.Hk; bp.Hv = p.Hv; bp.dk = p.dk; bp.DV = p.DV; bp.nb = p.nb;
  bp.nch = p.nch; bp.n_rec = p.n_rec; bp.in_f32 = 0; bp.qk_l2norm = 1; bp.scale = p.scale;
  e = omx::launch_bwd(bp, st);
  // gates and conv + SiLU adjoints
  if (e == hipSuccess) e = omx::launch_layer_tail_bwd(lp, st);
  return launch_status(e, fn);
}

// Workspace of a padded layer backward: mixed_qkv, z, conv weights, norm weight, the output
// cotangent, initial state, final-state cotangent and the gradients of mixed_qkv, z, the
// conv and norm weights and the initial state at the padded dims, then the call's.
struct LayerBwdPadWs {
  size_t x, z, cw, nw, dout, s0, ds, gx, gz, gcw, gnw, gs0, inner, total;
};
LayerBwdPadWs layer_bwd_pad_ws(int64_t B, int64_t T, int64_t Hk, int64_t Hv, int64_t dk2,
                               int64_t dv2, int64_t N) {
  LayerBwdPadWs w{};
  if (B < 0 || T < 0 || N < 0) return w;
  const size_t tok = (size_t)(B * T), cd = (size_t)(2 * Hk * dk2 + Hv * dv2);
  const size_t st = (size_t)(N * Hv * dk2 * dv2) * 4;
  Arena a;
  w.x = a.take(tok * cd * 2);
  w.z = a.take(tok * Hv * dv2 * 2);
  w.cw = a.take(cd * 4 * 4);
  w.nw = a.take(dv2 * 4);
  w.dout = a.take(tok * Hv * dv2 * 2);
  w.s0 = a.take(st);
  w.ds = a.take(st);
  w.gx = a.take(tok * cd * 2);
  w.gz = a.take(tok * Hv * dv2 * 2);
  w.gcw = a.take(cd * 4 * 4);
  w.gnw = a.take(dv2 * 4);
  w.gs0 = a.take(st);
  w.inner = a.off;
  w.total = w.inner + layer_bwd_ws(B, T, Hk, Hv, dk2, dv2, N).total;
  return w;
}

}  // namespace

extern "C" {

size_t omx_gdn_prefill_bwd_workspace_size(int64_t B, int64_t T, int64_t Hk, int64_t Hv, int64_t dk,
                                          int64_t dv, int64_t N) {
  const HeadDims hd = head_dims(kLayerBwd, dk, dv, false);
  if (hd.pad) return layer_bwd_pad_ws(B, T, Hk, Hv, hd.dk, hd.dv, N).total;
  return layer_bwd_ws(B, T, Hk, Hv, dk, dv, N).total;
}

int omx_gdn_prefill_bwd(const void* mixed_qkv, const void* z, const void* a, const void* b,
                        const float* conv_w, const float* A_log, const float* dt_bias,
                        const float* norm_w, float eps, const int32_t* cu_seqlens, int64_t N,
                        const float* initial_state, const void* d_out,
                        const float* d_final_state, void* d_mixed_qkv, void* dz, void* da,
                        void* db, float* d_conv_w, float* dA_log, float* d_dt_bias,
                        float* d_norm_w, float* d_initial_state, int64_t B, int64_t T,
                        int64_t Hk, int64_t Hv, int64_t dk, int64_t dv, int64_t K,
                        int64_t chunk_size, void* workspace, size_t workspace_bytes,
                        void* stream) {
  const char* fn = "omx_gdn_prefill_bwd";
  const HeadDims hd = head_dims(kLayerBwd, dk, dv, false);
  if (!hd.pad || Hv > 256)
    return prefill_bwd_core(fn, mixed_qkv, z, a, b, conv_w, A_log, dt_bias, norm_w, eps,
                            cu_seqlens, N, initial_state, d_out, d_final_state, d_mixed_qkv, dz,
                            da, db, d_conv_w, dA_log, d_dt_bias, d_norm_w, d_initial_state, B, T,
                            Hk, Hv, dk, dv, K, chunk_size, workspace, workspace_bytes, stream, dk,
                            dv);
  int rc = chunk_shape_check(fn, Hk, Hv, dk, dv, chunk_size, B, T, cu_seqlens, N);
  if (rc) return rc;
  REQUIRE(K == 4, "%s: conv kernel size must be 4 (got %lld)", fn, (long long)K);
  const LayerBwdPadWs w = layer_bwd_pad_ws(B, T, Hk, Hv, hd.dk, hd.dv, N);
  REQUIRE(workspace_bytes >= w.total, "%s: workspace of %zu bytes is smaller than the %zu needed",
          fn, workspace_bytes, w.total);
  if (N == 0) return ok();
  const int64_t tok = B * T, dk2 = hd.dk, dv2 = hd.dv;
  REQUIRE(conv_w && A_log && dt_bias && norm_w && d_conv_w && dA_log && d_dt_bias && d_norm_w,
          "%s: a parameter or parameter-gradient pointer is NULL", fn);
  if (tok > 0)
    REQUIRE(mixed_qkv && z && a && b && d_out && d_mixed_qkv && dz && da && db,
            "%s: an activation or activation-gradient pointer is NULL", fn);
  REQUIRE(workspace && aligned(workspace, 16), "%s: workspace must be non-NULL and 16-byte aligned",
          fn);
  char* base = (char*)workspace;
  hipStream_t st = (hipStream_t)stream;
  hipError_t e = hipSuccess;
  if (tok > 0) {
    e = pad_channels(mixed_qkv, dk, dv, base + w.x, dk2, dv2, Hk, Hv, tok, 1, 2, st);
    if (e == hipSuccess) e = pad3(z, Hv, dv, base + w.z, Hv, dv2, tok, 2, st);
    if (e == hipSuccess) e = pad3(d_out, Hv, dv, base + w.dout, Hv, dv2, tok, 2, st);
  }
  if (e == hipSuccess) e = pad_channels(conv_w, dk, dv, base + w.cw, dk2, dv2, Hk, Hv, 1, K, 4, st);
  if (e == hipSuccess) e = pad3(norm_w, 1, dv, base + w.nw, 1, dv2, 1, 4, st);
  if (e == hipSuccess && initial_state)
    e = pad3(initial_state, dk, dv, base + w.s0, dk2, dv2, N * Hv, 4, st);
  if (e == hipSuccess && d_final_state)
    e = pad3(d_final_state, dk, dv, base + w.ds, dk2, dv2, N * Hv, 4, st);
  if (e != hipSuccess) return launch_status(e, fn);
  rc = prefill_bwd_core(fn, base + w.x, base + w.z, a, b, (const float*)(base + w.cw), A_log,
                        dt_bias, (const float*)(base + w.nw), eps, cu_seqlens, N,
                        initial_state ? (const float*)(base + w.s0) : nullptr, base + w.dout,
                        d_final_state ? (const float*)(base + w.ds) : nullptr, base + w.gx,
                        base + w.gz, da, db, (float*)(base + w.gcw), dA_log, d_dt_bias,
                        (float*)(base + w.gnw), d_initial_state ? (float*)(base + w.gs0) : nullptr,
                        B, T, Hk, Hv, dk2, dv2, K, chunk_size, base + w.inner,
                        workspace_bytes - w.inner, stream, dk, dv);
  if (rc) return rc;
  if (tok > 0) {
    e = pad_channels(base + w.gx, dk2, dv2, d_mixed_qkv, dk, dv, Hk, Hv, tok, 1, 2, st);
    if (e == hipSuccess) e = pad3(base + w.gz, Hv, dv2, dz, Hv, dv, tok, 2, st);
  }
  if (e == hipSuccess) e = pad_channels(base + w.gcw, dk2, dv2, d_conv_w, dk, dv, Hk, Hv, 1, K, 4, st);
  if (e == hipSuccess) e = pad3(base + w.gnw, 1, dv2, d_norm_w, 1, dv, 1, 4, st);
  if (e == hipSuccess && d_initial_state)
    e = pad3(base + w.gs0, dk2, dv2, d_initial_state, dk, dv, N * Hv, 4, st);
  return launch_status(e, fn);
}

}  // extern "C"
