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
// normalised k and q, (layer) the conv output of v, the bf16 o and the partial
// sums of o^2 for the gated norm, and the plan of packed sequences (chunk offsets and
// the ordered copy of cu_seqlens the kernels read).
struct ChunkWs {
  size_t rec, kn, qn, vc, opart, off, cu, total;
};

ChunkWs chunk_ws(int64_t B, int64_t T, int64_t Hk, int64_t Hv, int64_t dk, int64_t dv, int64_t N,
                 int mode) {
  ChunkWs w{};
  if (B < 0 || T < 0 || Hk < 0 || Hv < 0 || dk < 0 || dv < 0 || N < 0) return w;
  const size_t tokens = (size_t)(B * T);
  const size_t slots = (tokens + 63) / 64 + (size_t)N;
  const size_t elem = mode == omx::kModeF32 ? 4 : 2;
  size_t o = 0;
  w.rec = o;
  o += align_up(slots * (size_t)Hv * (size_t)omx::chunk_record_bytes(mode), 256);
  w.kn = o;
  o += align_up(tokens * (size_t)(Hk * dk) * elem, 256);
  w.qn = o;
  o += align_up(tokens * (size_t)(Hk * dk) * elem, 256);
  if (mode == omx::kModeLayer) {
    w.vc = o;
    o += align_up(tokens * (size_t)(Hv * dv) * 2, 256);
    w.opart = o;
    o += align_up(tokens * (size_t)(Hv * dv) * 2, 256);
  }
  w.off = o;
  o += align_up((size_t)(N + 1) * 4, 256);
  w.cu = o;
  o += align_up((size_t)(N + 1) * 4, 256);
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
  w.f = chunk_ws(B, T, Hk, Hv, dk, dv, N, mode);
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

}  // namespace

extern "C" {

const char* omx_gdn_last_error(void) { return g_last_error.c_str(); }

int omx_gdn_abi_version(void) { return 103; }

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
    p.vc = base + ws.vc;
    p.vs = p.vc;
    p.vs_ld = (long long)p.Hv * p.DV;
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

}  // namespace

extern "C" {

size_t omx_gdn_chunk_fwd_workspace_size(int64_t B, int64_t T, int64_t Hk, int64_t Hv, int64_t dk,
                                        int64_t dv, int64_t N, int in_dtype) {
  return chunk_ws(B, T, Hk, Hv, dk, dv, N,
                  in_dtype == OMX_GDN_F32 ? omx::kModeF32 : omx::kModeBF16).total;
}

int omx_gdn_chunk_fwd(const void* q, const void* k, const void* v, int in_dtype, const float* g,
                      const float* beta, const float* initial_state, const int32_t* cu_seqlens,
                      int64_t N, float* o, float* final_state, int64_t B, int64_t T, int64_t Hk,
                      int64_t Hv, int64_t dk, int64_t dv, int64_t chunk_size, float scale,
                      int qk_l2norm, void* workspace, size_t workspace_bytes, void* stream) {
  const char* fn = "omx_gdn_chunk_fwd";
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
    return fail(OMX_GDN_EUNSUPPORTED, "%s: head dims dk=%lld dv=%lld not compiled for %s inputs",
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

size_t omx_gdn_prefill_workspace_size(int64_t B, int64_t T, int64_t Hk, int64_t Hv, int64_t dk,
                                      int64_t dv, int64_t N) {
  return chunk_ws(B, T, Hk, Hv, dk, dv, N, omx::kModeLayer).total;
}

}  // extern "C"

namespace {

// The layer prefill behind omx_gdn_prefill and omx_gdn_prefill_noalloc (`fn` names the
// entry point in error messages).
int prefill_entry(const char* fn, const void* mixed_qkv, const void* z, const void* a,
                  const void* b, const float* conv_w, const float* A_log, const float* dt_bias,
                  const float* norm_w, float eps, const int32_t* cu_seqlens, int64_t N,
                  const float* initial_state, float* final_state, const void* conv_state_in,
                  void* conv_state_out, void* out, int64_t B, int64_t T, int64_t Hk,
                  int64_t Hv, int64_t dk, int64_t dv, int64_t K, int64_t chunk_size,
                  void* workspace, size_t workspace_bytes, void* stream) {
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
    return fail(OMX_GDN_EUNSUPPORTED, "%s: head dims dk=%lld dv=%lld not compiled", fn,
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
  omx::ChunkParams p{};
  p.mixed_qkv = mixed_qkv; p.z = z; p.a = a; p.b = b;
  p.conv_w = conv_w; p.A_log = A_log; p.dt_bias = dt_bias; p.norm_w = norm_w;
  p.conv_state_in = conv_state_in; p.conv_state_out = conv_state_out; p.out = out;
  p.initial_state = initial_state; p.final_state = final_state; p.cu_seqlens = cu_seqlens;
  p.N = (int)N; p.T = (int)T; p.Hk = (int)Hk; p.Hv = (int)Hv; p.dk = (int)dk; p.DV = (int)dv;
  p.nb = (int)(dv / omx::chunk_block_cols());
  p.conv_k = (int)K;
  p.conv_dim = (int)(2 * Hk * dk + Hv * dv);
  p.scale = 1.0f / sqrtf((float)dk);
  p.eps = eps;
  p.qk_l2norm = 1;
  p.o_part = (char*)workspace + ws.opart;
  REQUIRE((int64_t)p.N * p.Hv * p.nb <= INT32_MAX, "%s: grid too large", fn);
  REQUIRE(((B * T + 63) / 64 + N) * Hk <= INT32_MAX, "%s: grid too large", fn);
  hipError_t e = launch_chunked(p, ws, workspace, omx::kModeLayer, (hipStream_t)stream);
  if (e == hipSuccess)
    e = omx::launch_norm_epilogue(p.o_part, z, norm_w, out, tokens * Hv, (int)dv, eps,
                                  (hipStream_t)stream);
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
  void* ws = nullptr;
  const int rc = scratch_for_current_device(fn, &ws);
  if (rc) return rc;
  return prefill_entry(fn, mixed_qkv, z, a, b, conv_w, A_log, dt_bias, norm_w, eps, cu_seqlens,
                       N, initial_state, final_state, conv_state_in, conv_state_out, out, B, T,
                       Hk, Hv, dk, dv, K, chunk_size, ws, kNoAllocScratchBytes, stream);
}

}  // extern "C"

// ---------------------------------------------------------------------------- backward
extern "C" {

size_t omx_gdn_chunk_bwd_workspace_size(int64_t B, int64_t T, int64_t Hk, int64_t Hv, int64_t dk,
                                        int64_t dv, int64_t N, int in_dtype) {
  return bwd_ws(B, T, Hk, Hv, dk, dv, N,
                in_dtype == OMX_GDN_F32 ? omx::kModeF32 : omx::kModeBF16).total;
}

int omx_gdn_chunk_bwd(const void* q, const void* k, const void* v, int in_dtype, const float* g,
                      const float* beta, const float* initial_state, const int32_t* cu_seqlens,
                      int64_t N, const float* d_o, const float* d_final_state, void* dq, void* dk,
                      void* dv, float* dg, float* dbeta, float* d_initial_state, int64_t B,
                      int64_t T, int64_t Hk, int64_t Hv, int64_t dk_dim, int64_t dv_dim,
                      int64_t chunk_size, float scale, int qk_l2norm, void* workspace,
                      size_t workspace_bytes, void* stream) {
  const char* fn = "omx_gdn_chunk_bwd";
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
                "%s: head dims dk=%lld dv=%lld not compiled for %s inputs (bf16: dk 64/128, "
                "fp32: dk 32/64; dv 64/128)",
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
  b.cu_seqlens = p.cu_seqlens; b.chunk_off = p.chunk_off;
  b.N = p.N; b.T = p.T; b.Hk = p.Hk; b.Hv = p.Hv; b.dk = p.dk; b.DV = p.DV; b.nb = p.nb;
  b.nch = p.nch; b.n_rec = p.n_rec; b.in_f32 = f32 ? 1 : 0; b.qk_l2norm = p.qk_l2norm;
  b.scale = scale;
  return launch_status(omx::launch_bwd(b, st), fn);
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

size_t omx_gdn_prefill_bwd_workspace_size(int64_t B, int64_t T, int64_t Hk, int64_t Hv, int64_t dk,
                                          int64_t dv, int64_t N) {
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
                "%s: dk=%lld dv=%lld Hv=%lld not compiled (dk 64/128, dv 64/128, Hv <= 256)", fn,
                (long long)dk, (long long)dv, (long long)Hv);
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
  omx::ChunkParams p{};
  p.q = lp.q; p.k = lp.k; p.v = lp.v;
  p.q_ld = Hk * dk; p.k_ld = Hk * dk; p.v_ld = Hv * dv;
  p.g = lp.g; p.beta = lp.beta; p.o = (float*)(base + ws.o);
  p.initial_state = initial_state; p.final_state = nullptr; p.cu_seqlens = cu_seqlens;
  p.N = (int)N; p.T = (int)T; p.Hk = (int)Hk; p.Hv = (int)Hv; p.dk = (int)dk; p.DV = (int)dv;
  p.nb = (int)(dv / omx::chunk_block_cols());
  p.scale = 1.0f / sqrtf((float)dk); p.qk_l2norm = 1;
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
  bp.cu_seqlens = p.cu_seqlens; bp.chunk_off = p.chunk_off;
  bp.N = p.N; bp.T = p.T; bp.Hk = p.Hk; bp.Hv = p.Hv; bp.dk = p.dk; bp.DV = p.DV; bp.nb = p.nb;
  bp.nch = p.nch; bp.n_rec = p.n_rec; bp.in_f32 = 0; bp.qk_l2norm = 1; bp.scale = p.scale;
  e = omx::launch_bwd(bp, st);
  // gates and conv + SiLU adjoints
  if (e == hipSuccess) e = omx::launch_layer_tail_bwd(lp, st);
  return launch_status(e, fn);
}

}  // extern "C"
