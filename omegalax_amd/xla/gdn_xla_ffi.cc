// XLA FFI handlers over libomx_gdn's C ABI (include/omx_gdn.h), for calling the MI355X
// GatedDeltaNet kernels from JAX with jax.ffi.ffi_call on the ROCm platform.
//
// Built by omegalax_amd.build only when jaxlib's FFI headers are importable
// (jax.ffi.include_dir()); it is not part of libomx_gdn.so and nothing in this
// repository's torch path loads it.  JAX is absent from the image this was written in, so
// this file has never been compiled or run there: the handlers are untested source.
// Each handler checks only ranks and element types (the C ABI takes raw pointers and
// cannot see them); the C ABI checks shapes, pointers and attributes on the host and its
// error codes map to FFI errors (EINVAL -> InvalidArgument, EUNSUPPORTED ->
// Unimplemented, else Internal).
// Work is enqueued on XLA's stream; no handler synchronises or keeps state, so XLA may
// run them concurrently and re-run them under remat (model.py:202).
//
// The call site they replace is chunk_gated_delta_rule inside _full_deltanet
// (omegalax/models/qwen3_5/deltanet.py:281), which runs inside shard_map on per-device
// shapes; the layer-level handlers cover deltanet.py:243-293 and a decode step.
#include <cmath>
#include <cstdint>
#include <initializer_list>

#include <hip/hip_runtime.h>

#include "omx_gdn.h"
#include "xla/ffi/api/ffi.h"

namespace ffi = xla::ffi;

namespace {

ffi::Error status(int rc) {
  if (rc == OMX_GDN_OK) return ffi::Error::Success();
  if (rc == OMX_GDN_EINVAL) return ffi::Error::InvalidArgument(omx_gdn_last_error());
  if (rc == OMX_GDN_EUNSUPPORTED)
    return ffi::Error(ffi::ErrorCode::kUnimplemented, omx_gdn_last_error());
  return ffi::Error::Internal(omx_gdn_last_error());
}

// The C ABI reads q/k/v-style inputs as bf16 or fp32 only: any other element type (f16,
// f64, ...) is rejected here, as are operands whose type differs from the first one's,
// because the kernels would read them with the first operand's element size.
ffi::Error qkv_dtype(int* code, std::initializer_list<const ffi::AnyBuffer*> xs) {
  const ffi::DataType t = (*xs.begin())->element_type();
  if (t != ffi::DataType::BF16 && t != ffi::DataType::F32)
    return ffi::Error::InvalidArgument("q, k, v must be bf16 or f32");
  for (const ffi::AnyBuffer* x : xs)
    if (x->element_type() != t)
      return ffi::Error::InvalidArgument("q, k, v (and their gradients) must share one dtype");
  *code = t == ffi::DataType::BF16 ? OMX_GDN_BF16 : OMX_GDN_F32;
  return ffi::Error::Success();
}

// The layer entry points take bf16 activations (and conv caches) only.
ffi::Error all_bf16(std::initializer_list<const ffi::AnyBuffer*> xs) {
  for (const ffi::AnyBuffer* x : xs)
    if (x->element_type() != ffi::DataType::BF16)
      return ffi::Error::InvalidArgument("the layer's activations and conv caches must be bf16");
  return ffi::Error::Success();
}

// chunk_gated_delta_rule(q, k, v, g, beta, chunk_size) -> o (deltanet.py:53-153), with an
// optional initial state in and final state out (pass a [0]-sized buffer for none).
ffi::Error ChunkFwd(hipStream_t stream, ffi::AnyBuffer q, ffi::AnyBuffer k, ffi::AnyBuffer v,
                    ffi::Buffer<ffi::F32> g, ffi::Buffer<ffi::F32> beta,
                    ffi::Buffer<ffi::F32> initial_state, ffi::Result<ffi::Buffer<ffi::F32>> o,
                    ffi::Result<ffi::Buffer<ffi::F32>> final_state,
                    ffi::Result<ffi::AnyBuffer> workspace, int64_t chunk_size) {
  const auto qd = q.dimensions(), vd = v.dimensions();  // [B, T, Hk, dk], [B, T, Hv, dv]
  if (qd.size() != 4 || vd.size() != 4)
    return ffi::Error::InvalidArgument("q and v must be rank 4");
  const int64_t B = qd[0], T = qd[1], Hk = qd[2], dk = qd[3], Hv = vd[2], dv = vd[3];
  int code = 0;
  if (ffi::Error e = qkv_dtype(&code, {&q, &k, &v}); e.failure()) return e;
  const float* s0 = initial_state.element_count() ? initial_state.typed_data() : nullptr;
  float* s1 = final_state->element_count() ? final_state->typed_data() : nullptr;
  return status(omx_gdn_chunk_fwd(q.untyped_data(), k.untyped_data(), v.untyped_data(),
                                  code, g.typed_data(), beta.typed_data(), s0, nullptr,
                                  B, o->typed_data(), s1, B, T, Hk, Hv, dk, dv, chunk_size,
                                  1.0f / std::sqrt((float)dk), 1, workspace->untyped_data(),
                                  workspace->size_bytes(), stream));
}

// Its VJP: cotangent do of o -> dq, dk, dv (input dtype), dg, dbeta (fp32).
ffi::Error ChunkBwd(hipStream_t stream, ffi::AnyBuffer q, ffi::AnyBuffer k, ffi::AnyBuffer v,
                    ffi::Buffer<ffi::F32> g, ffi::Buffer<ffi::F32> beta, ffi::Buffer<ffi::F32> d_o,
                    ffi::Result<ffi::AnyBuffer> dq, ffi::Result<ffi::AnyBuffer> dk,
                    ffi::Result<ffi::AnyBuffer> dv, ffi::Result<ffi::Buffer<ffi::F32>> dg,
                    ffi::Result<ffi::Buffer<ffi::F32>> dbeta,
                    ffi::Result<ffi::AnyBuffer> workspace, int64_t chunk_size) {
  const auto qd = q.dimensions(), vd = v.dimensions();
  if (qd.size() != 4 || vd.size() != 4)
    return ffi::Error::InvalidArgument("q and v must be rank 4");
  const int64_t B = qd[0], T = qd[1], Hk = qd[2], dkd = qd[3], Hv = vd[2], dvd = vd[3];
  int code = 0;
  if (ffi::Error e = qkv_dtype(&code, {&q, &k, &v, &(*dq), &(*dk), &(*dv)}); e.failure()) return e;
  return status(omx_gdn_chunk_bwd(
      q.untyped_data(), k.untyped_data(), v.untyped_data(), code, g.typed_data(),
      beta.typed_data(), nullptr, nullptr, B, d_o.typed_data(), nullptr, dq->untyped_data(),
      dk->untyped_data(), dv->untyped_data(), dg->typed_data(), dbeta->typed_data(), nullptr, B,
      T, Hk, Hv, dkd, dvd, chunk_size, 1.0f / std::sqrt((float)dkd), 1,
      workspace->untyped_data(), workspace->size_bytes(), stream));
}

// GatedDeltaNet.__call__ between the projections and out_proj (deltanet.py:243-293).
ffi::Error Prefill(hipStream_t stream, ffi::AnyBuffer mixed_qkv, ffi::AnyBuffer z,
                   ffi::AnyBuffer a, ffi::AnyBuffer b, ffi::Buffer<ffi::F32> conv_w,
                   ffi::Buffer<ffi::F32> A_log, ffi::Buffer<ffi::F32> dt_bias,
                   ffi::Buffer<ffi::F32> norm_w, ffi::Result<ffi::AnyBuffer> out,
                   ffi::Result<ffi::AnyBuffer> workspace, int64_t num_k_heads, int64_t head_k_dim,
                   int64_t num_v_heads, int64_t head_v_dim, float eps) {
  const auto xd = mixed_qkv.dimensions(), wd = conv_w.dimensions();  // [B, T, C], [C, K]
  if (xd.size() != 3 || wd.size() != 2)
    return ffi::Error::InvalidArgument("mixed_qkv must be [B, T, C] and conv_w [C, K]");
  if (ffi::Error e = all_bf16({&mixed_qkv, &z, &a, &b, &(*out)}); e.failure()) return e;
  return status(omx_gdn_prefill(
      mixed_qkv.untyped_data(), z.untyped_data(), a.untyped_data(), b.untyped_data(),
      conv_w.typed_data(), A_log.typed_data(), dt_bias.typed_data(), norm_w.typed_data(), eps,
      nullptr, xd[0], nullptr, nullptr, nullptr, nullptr, out->untyped_data(), xd[0], xd[1],
      num_k_heads, num_v_heads, head_k_dim, head_v_dim, wd[1], 64, workspace->untyped_data(),
      workspace->size_bytes(), stream));
}

// Its VJP for the cotangent d_out of the output.
ffi::Error PrefillBwd(hipStream_t stream, ffi::AnyBuffer mixed_qkv, ffi::AnyBuffer z,
                      ffi::AnyBuffer a, ffi::AnyBuffer b, ffi::Buffer<ffi::F32> conv_w,
                      ffi::Buffer<ffi::F32> A_log, ffi::Buffer<ffi::F32> dt_bias,
                      ffi::Buffer<ffi::F32> norm_w, ffi::AnyBuffer d_out,
                      ffi::Result<ffi::AnyBuffer> dx, ffi::Result<ffi::AnyBuffer> dz,
                      ffi::Result<ffi::AnyBuffer> da, ffi::Result<ffi::AnyBuffer> db,
                      ffi::Result<ffi::Buffer<ffi::F32>> d_conv_w,
                      ffi::Result<ffi::Buffer<ffi::F32>> dA_log,
                      ffi::Result<ffi::Buffer<ffi::F32>> d_dt_bias,
                      ffi::Result<ffi::Buffer<ffi::F32>> d_norm_w,
                      ffi::Result<ffi::AnyBuffer> workspace, int64_t num_k_heads,
                      int64_t head_k_dim, int64_t num_v_heads, int64_t head_v_dim, float eps) {
  const auto xd = mixed_qkv.dimensions(), wd = conv_w.dimensions();
  if (xd.size() != 3 || wd.size() != 2)
    return ffi::Error::InvalidArgument("mixed_qkv must be [B, T, C] and conv_w [C, K]");
  if (ffi::Error e = all_bf16({&mixed_qkv, &z, &a, &b, &d_out, &(*dx), &(*dz), &(*da), &(*db)});
      e.failure())
    return e;
  return status(omx_gdn_prefill_bwd(
      mixed_qkv.untyped_data(), z.untyped_data(), a.untyped_data(), b.untyped_data(),
      conv_w.typed_data(), A_log.typed_data(), dt_bias.typed_data(), norm_w.typed_data(), eps,
      nullptr, xd[0], nullptr, d_out.untyped_data(), nullptr, dx->untyped_data(),
      dz->untyped_data(), da->untyped_data(), db->untyped_data(), d_conv_w->typed_data(),
      dA_log->typed_data(), d_dt_bias->typed_data(), d_norm_w->typed_data(), nullptr, xd[0],
      xd[1], num_k_heads, num_v_heads, head_k_dim, head_v_dim, wd[1], 64,
      workspace->untyped_data(), workspace->size_bytes(), stream));
}

// One cached decode step.  The caches are results aliased to the inputs
// (input_output_aliases={8: 1, 9: 2}); when XLA did not alias them they are copied first
// and updated in the results.
ffi::Error DecodeStep(hipStream_t stream, ffi::AnyBuffer mixed_qkv, ffi::AnyBuffer z,
                      ffi::AnyBuffer a, ffi::AnyBuffer b, ffi::Buffer<ffi::F32> conv_w,
                      ffi::Buffer<ffi::F32> A_log, ffi::Buffer<ffi::F32> dt_bias,
                      ffi::Buffer<ffi::F32> norm_w, ffi::AnyBuffer conv_state,
                      ffi::Buffer<ffi::F32> state, ffi::Result<ffi::AnyBuffer> out,
                      ffi::Result<ffi::AnyBuffer> conv_state_out,
                      ffi::Result<ffi::Buffer<ffi::F32>> state_out, int64_t num_k_heads,
                      int64_t head_k_dim, int64_t num_v_heads, int64_t head_v_dim, float eps) {
  const auto xd = mixed_qkv.dimensions(), wd = conv_w.dimensions();  // [B, C], [C, K]
  if (xd.size() != 2 || wd.size() != 2)
    return ffi::Error::InvalidArgument("mixed_qkv must be [B, C] and conv_w [C, K]");
  if (ffi::Error e = all_bf16({&mixed_qkv, &z, &a, &b, &conv_state, &(*out), &(*conv_state_out)});
      e.failure())
    return e;
  if (conv_state_out->untyped_data() != conv_state.untyped_data() &&
      hipMemcpyAsync(conv_state_out->untyped_data(), conv_state.untyped_data(),
                     conv_state.size_bytes(), hipMemcpyDeviceToDevice, stream) != hipSuccess)
    return ffi::Error::Internal("conv_state copy failed");
  if (state_out->untyped_data() != state.untyped_data() &&
      hipMemcpyAsync(state_out->untyped_data(), state.untyped_data(), state.size_bytes(),
                     hipMemcpyDeviceToDevice, stream) != hipSuccess)
    return ffi::Error::Internal("state copy failed");
  return status(omx_gdn_decode_step(
      mixed_qkv.untyped_data(), z.untyped_data(), a.untyped_data(), b.untyped_data(),
      conv_w.typed_data(), A_log.typed_data(), dt_bias.typed_data(), norm_w.typed_data(), eps,
      conv_state_out->untyped_data(), state_out->typed_data(), out->untyped_data(), xd[0],
      num_k_heads, num_v_heads, head_k_dim, head_v_dim, wd[1], stream));
}

// The gate projections (deltanet.py:240-241): x [M, D] bf16, w_a / w_b [Hv, D] bf16 ->
// a, b [M, Hv] bf16, one pass over x.
ffi::Error AbProj(hipStream_t stream, ffi::AnyBuffer x, ffi::AnyBuffer w_a, ffi::AnyBuffer w_b,
                  ffi::Result<ffi::AnyBuffer> a, ffi::Result<ffi::AnyBuffer> b) {
  const auto xd = x.dimensions(), wd = w_a.dimensions();
  if (xd.size() < 1 || wd.size() != 2) return ffi::Error::InvalidArgument("x [..., D], w [Hv, D]");
  if (ffi::Error e = all_bf16({&x, &w_a, &w_b, &(*a), &(*b)}); e.failure()) return e;
  const int64_t D = xd[xd.size() - 1], Hv = wd[0];
  const int64_t M = D ? (int64_t)x.element_count() / D : 0;
  return status(omx_gdn_ab_proj(x.untyped_data(), w_a.untyped_data(), w_b.untyped_data(),
                                a->untyped_data(), b->untyped_data(), M, D, Hv, stream));
}

}  // namespace

XLA_FFI_DEFINE_HANDLER_SYMBOL(OmxGdnChunkFwd, ChunkFwd,
                              ffi::Ffi::Bind()
                                  .Ctx<ffi::PlatformStream<hipStream_t>>()
                                  .Arg<ffi::AnyBuffer>()
                                  .Arg<ffi::AnyBuffer>()
                                  .Arg<ffi::AnyBuffer>()
                                  .Arg<ffi::Buffer<ffi::F32>>()
                                  .Arg<ffi::Buffer<ffi::F32>>()
                                  .Arg<ffi::Buffer<ffi::F32>>()
                                  .Ret<ffi::Buffer<ffi::F32>>()
                                  .Ret<ffi::Buffer<ffi::F32>>()
                                  .Ret<ffi::AnyBuffer>()
                                  .Attr<int64_t>("chunk_size"));

XLA_FFI_DEFINE_HANDLER_SYMBOL(OmxGdnChunkBwd, ChunkBwd,
                              ffi::Ffi::Bind()
                                  .Ctx<ffi::PlatformStream<hipStream_t>>()
                                  .Arg<ffi::AnyBuffer>()
                                  .Arg<ffi::AnyBuffer>()
                                  .Arg<ffi::AnyBuffer>()
                                  .Arg<ffi::Buffer<ffi::F32>>()
                                  .Arg<ffi::Buffer<ffi::F32>>()
                                  .Arg<ffi::Buffer<ffi::F32>>()
                                  .Ret<ffi::AnyBuffer>()
                                  .Ret<ffi::AnyBuffer>()
                                  .Ret<ffi::AnyBuffer>()
                                  .Ret<ffi::Buffer<ffi::F32>>()
                                  .Ret<ffi::Buffer<ffi::F32>>()
                                  .Ret<ffi::AnyBuffer>()
                                  .Attr<int64_t>("chunk_size"));

XLA_FFI_DEFINE_HANDLER_SYMBOL(OmxGdnPrefill, Prefill,
                              ffi::Ffi::Bind()
                                  .Ctx<ffi::PlatformStream<hipStream_t>>()
                                  .Arg<ffi::AnyBuffer>()
                                  .Arg<ffi::AnyBuffer>()
                                  .Arg<ffi::AnyBuffer>()
                                  .Arg<ffi::AnyBuffer>()
                                  .Arg<ffi::Buffer<ffi::F32>>()
                                  .Arg<ffi::Buffer<ffi::F32>>()
                                  .Arg<ffi::Buffer<ffi::F32>>()
                                  .Arg<ffi::Buffer<ffi::F32>>()
                                  .Ret<ffi::AnyBuffer>()
                                  .Ret<ffi::AnyBuffer>()
                                  .Attr<int64_t>("num_k_heads")
                                  .Attr<int64_t>("head_k_dim")
                                  .Attr<int64_t>("num_v_heads")
                                  .Attr<int64_t>("head_v_dim")
                                  .Attr<float>("eps"));

XLA_FFI_DEFINE_HANDLER_SYMBOL(OmxGdnPrefillBwd, PrefillBwd,
                              ffi::Ffi::Bind()
                                  .Ctx<ffi::PlatformStream<hipStream_t>>()
                                  .Arg<ffi::AnyBuffer>()
                                  .Arg<ffi::AnyBuffer>()
                                  .Arg<ffi::AnyBuffer>()
                                  .Arg<ffi::AnyBuffer>()
                                  .Arg<ffi::Buffer<ffi::F32>>()
                                  .Arg<ffi::Buffer<ffi::F32>>()
                                  .Arg<ffi::Buffer<ffi::F32>>()
                                  .Arg<ffi::Buffer<ffi::F32>>()
                                  .Arg<ffi::AnyBuffer>()
                                  .Ret<ffi::AnyBuffer>()
                                  .Ret<ffi::AnyBuffer>()
                                  .Ret<ffi::AnyBuffer>()
                                  .Ret<ffi::AnyBuffer>()
                                  .Ret<ffi::Buffer<ffi::F32>>()
                                  .Ret<ffi::Buffer<ffi::F32>>()
                                  .Ret<ffi::Buffer<ffi::F32>>()
                                  .Ret<ffi::Buffer<ffi::F32>>()
                                  .Ret<ffi::AnyBuffer>()
                                  .Attr<int64_t>("num_k_heads")
                                  .Attr<int64_t>("head_k_dim")
                                  .Attr<int64_t>("num_v_heads")
                                  .Attr<int64_t>("head_v_dim")
                                  .Attr<float>("eps"));

XLA_FFI_DEFINE_HANDLER_SYMBOL(OmxGdnDecodeStep, DecodeStep,
                              ffi::Ffi::Bind()
                                  .Ctx<ffi::PlatformStream<hipStream_t>>()
                                  .Arg<ffi::AnyBuffer>()
                                  .Arg<ffi::AnyBuffer>()
                                  .Arg<ffi::AnyBuffer>()
                                  .Arg<ffi::AnyBuffer>()
                                  .Arg<ffi::Buffer<ffi::F32>>()
                                  .Arg<ffi::Buffer<ffi::F32>>()
                                  .Arg<ffi::Buffer<ffi::F32>>()
                                  .Arg<ffi::Buffer<ffi::F32>>()
                                  .Arg<ffi::AnyBuffer>()
                                  .Arg<ffi::Buffer<ffi::F32>>()
                                  .Ret<ffi::AnyBuffer>()
                                  .Ret<ffi::AnyBuffer>()
                                  .Ret<ffi::Buffer<ffi::F32>>()
                                  .Attr<int64_t>("num_k_heads")
                                  .Attr<int64_t>("head_k_dim")
                                  .Attr<int64_t>("num_v_heads")
                                  .Attr<int64_t>("head_v_dim")
                                  .Attr<float>("eps"));

XLA_FFI_DEFINE_HANDLER_SYMBOL(OmxGdnAbProj, AbProj,
                              ffi::Ffi::Bind()
                                  .Ctx<ffi::PlatformStream<hipStream_t>>()
                                  .Arg<ffi::AnyBuffer>()
                                  .Arg<ffi::AnyBuffer>()
                                  .Arg<ffi::AnyBuffer>()
                                  .Ret<ffi::AnyBuffer>()
                                  .Ret<ffi::AnyBuffer>());
