/*
 * omx_gdn.h -- C ABI of the MI355X (gfx950) GatedDeltaNet library (libomx_gdn.so).
 *
 * Drop-in boundary for omegalax's Qwen3.5 gated-delta-rule path
 * (omegalax/models/qwen3_5/deltanet.py).  Every entry point takes raw device
 * pointers, sizes and a HIP stream (hipStream_t passed as void*; NULL = the
 * null stream), enqueues its kernels on that stream and returns without
 * synchronising.  The library never allocates device memory in these calls:
 * callers pass any scratch as `workspace` (size from the *_workspace_size
 * query).  Buffers are dense, row-major, in the layouts given per argument.
 *
 * Return value: OMX_GDN_OK (0) or a negative code; omx_gdn_last_error() then
 * returns a message for the calling thread.  Scalar arguments, pointers and
 * alignments are validated on the host before any HIP call, so a bad call returns
 * OMX_GDN_EINVAL without touching the GPU.  The contents of device arrays are not
 * read on the host (that would need a device-to-host copy and a synchronisation):
 * their preconditions are stated per argument, together with what the kernels do
 * when one is violated.
 *
 * dtype codes: OMX_GDN_F32 (float32) or OMX_GDN_BF16 (bfloat16 as uint16 bits).
 * Shapes: B batch, T tokens, Hk key heads, Hv value heads (Hv % Hk == 0; value
 * head h reads key head h / (Hv/Hk), the repeat-interleave of
 * deltanet.py:272-280), dk/dv head dims, K conv taps, conv_dim = 2*Hk*dk + Hv*dv.
 *
 * Head dims: the prefill entry points accept any 1 <= dk <= 128 and 1 <= dv <= 256
 * (dv <= 128 for the backward entry points).  Shapes the kernels are not compiled for
 * run on zero-padded copies at the next compiled dims, made in the workspace (the
 * *_workspace_size queries include them); the results equal the unpadded computation
 * (q is scaled by 1/sqrt of the caller's dk, the gated norm averages over the caller's
 * dv).  The decode entry points take dk, dv in {16, 32, 64, 128} and Hv/Hk <= 8.  Other
 * shapes return OMX_GDN_EUNSUPPORTED.
 */
#ifndef OMX_GDN_H
#define OMX_GDN_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define OMX_GDN_OK 0
#define OMX_GDN_EINVAL (-1)      /* bad shape, dtype, pointer or attribute */
#define OMX_GDN_EUNSUPPORTED (-2) /* valid request outside the compiled shapes */
#define OMX_GDN_ELAUNCH (-3)      /* a HIP launch failed */

#define OMX_GDN_F32 0
#define OMX_GDN_BF16 1

/* Message for the last failed call on this thread ("" if none). */
const char* omx_gdn_last_error(void);

/* Library ABI version (major * 100 + minor). */
int omx_gdn_abi_version(void);

/*
 * Chunked gated delta rule, the core of the prefill.
 * Replaces chunk_gated_delta_rule(q_BTHA, k_BTHA, v_BTHU, g_BTH, beta_BTH,
 * chunk_size=64) -> o_BTHU (deltanet.py:53-153), whose only caller is
 * _full_deltanet (deltanet.py:281).  Adds the semantics of transformers'
 * torch_chunk_gated_delta_rule: initial_state, final state and packed sequences.
 *
 *   q, k         [B, T, Hk, dk]  in_dtype (bf16 or f32); L2-normalised in the kernel
 *                                when qk_l2norm != 0 (deltanet.py:65-66), at the input
 *                                precision, then scaled by `scale` (deltanet.py:84-85)
 *   v            [B, T, Hv, dv]  in_dtype
 *   g            [B, T, Hv] f32  log decay (<= 0)
 *   beta         [B, T, Hv] f32
 *   initial_state [N, Hv, dk, dv] f32 or NULL (zeros, deltanet.py:118)
 *   cu_seqlens   int32 [N+1] device array or NULL.  When given, B must be 1 and
 *                sequence n spans tokens [cu[n], cu[n+1]); each sequence starts from
 *                its own initial state and chunks restart at its first token.
 *                Without it N = B.
 *                Precondition: 0 = cu[0] <= cu[1] <= ... <= cu[N] = T.  The kernels
 *                read the offsets as c[0] = 0, c[N] = T and c[n] = max(c[n-1],
 *                clamp(cu[n], 0, T)) in between (equal to cu when it is valid), so
 *                whatever the array holds the sequences are ordered, disjoint and
 *                cover every token: no output row is left unwritten, no two
 *                workgroups write one row, and no reduction reads an unwritten row.
 *   o            [B, T, Hv, dv] f32 (the reference returns fp32, deltanet.py:153)
 *   final_state  [N, Hv, dk, dv] f32 or NULL (the reference discards it, :146)
 *   chunk_size   must be 64.
 */
int omx_gdn_chunk_fwd(const void* q, const void* k, const void* v, int in_dtype,
                      const float* g, const float* beta, const float* initial_state,
                      const int32_t* cu_seqlens, int64_t N, float* o, float* final_state,
                      int64_t B, int64_t T, int64_t Hk, int64_t Hv, int64_t dk, int64_t dv,
                      int64_t chunk_size, float scale, int qk_l2norm, void* workspace,
                      size_t workspace_bytes, void* stream);

/*
 * Bytes of device workspace omx_gdn_chunk_fwd needs for these shapes and in_dtype
 * (N = number of sequences).  It holds the per-(chunk, value head) records of the
 * chunk-parallel preparation (the inverse T = (I + L)^-1 and P of each chunk,
 * deltanet.py:100-113, 130-131, and the chunk's gate vectors), the normalised
 * q and k, and the chunk offsets of packed sequences.  Pass it 16-byte aligned.
 */
size_t omx_gdn_chunk_fwd_workspace_size(int64_t B, int64_t T, int64_t Hk, int64_t Hv,
                                        int64_t dk, int64_t dv, int64_t N, int in_dtype);

/*
 * GatedDeltaNet prefill from the projection outputs to the gated-norm output.
 * Replaces the middle of GatedDeltaNet.__call__ (deltanet.py:243-293): causal
 * depthwise conv1d + SiLU (:243), gates beta = sigmoid(b), g = -exp(A_log) *
 * softplus(a + dt_bias) (:248-250), the split/GQA/L2-norm/chunked rule of
 * _full_deltanet (:261-281) and the inline gated RMSNorm (:282-293).  The
 * projections (:234-241) and out_proj (:305) stay with the caller.
 *
 *   mixed_qkv     [B, T, conv_dim] bf16  (in_proj_qkv output, token-major)
 *   z             [B, T, Hv, dv] bf16
 *   a, b          [B, T, Hv] bf16
 *   conv_w        [conv_dim, K] f32, 16-byte aligned (cast to bf16 as at deltanet.py:243)
 *   A_log, dt_bias [Hv] f32;  norm_w [dv] f32 (16-byte aligned);  eps (rms_norm_eps)
 *   cu_seqlens    as for omx_gdn_chunk_fwd (conv history also restarts per sequence)
 *   initial_state / final_state  [N, Hv, dk, dv] f32 or NULL
 *   conv_state_in  [N, conv_dim, K-1] bf16 or NULL: raw inputs preceding each
 *                  sequence (oldest first); NULL = zeros (deltanet.py:46)
 *   conv_state_out [N, conv_dim, K-1] bf16 or NULL: the last K-1 raw inputs of each
 *                  sequence (the decode cache after this prefill)
 *   out           [B, T, Hv*dv] bf16
 *
 * When the scan's grid fits the GPU in one round (at most one workgroup per CU, e.g.
 * B=4 T=4096 at Hv=32 d=128), its workgroups apply the gated norm themselves and
 * exchange each row's partial sums while they run, so they must run together: work on
 * other streams that holds CUs for more than about a second during the call leaves the
 * affected output rows NaN (a bounded wait that ran out) rather than a wrong value.
 */
int omx_gdn_prefill(const void* mixed_qkv, const void* z, const void* a, const void* b,
                    const float* conv_w, const float* A_log, const float* dt_bias,
                    const float* norm_w, float eps, const int32_t* cu_seqlens, int64_t N,
                    const float* initial_state, float* final_state, const void* conv_state_in,
                    void* conv_state_out, void* out, int64_t B, int64_t T, int64_t Hk,
                    int64_t Hv, int64_t dk, int64_t dv, int64_t K, int64_t chunk_size,
                    void* workspace, size_t workspace_bytes, void* stream);

/*
 * Bytes of device workspace omx_gdn_prefill needs (16-byte aligned): the chunk
 * records and normalised q/k as for omx_gdn_chunk_fwd, the conv output of v (dk < 128
 * after padding; with dk = 128 the scan forms the v rows from mixed_qkv itself), and
 * what the gated-norm epilogue reads: the unnormalised bf16 o and the fp32 sums of
 * squares of o per 16 columns of each row (unused when the scan applies the norm
 * itself), and the small exchange ring of row partials through which the scan's column
 * blocks share a row's statistic when it does.
 */
size_t omx_gdn_prefill_workspace_size(int64_t B, int64_t T, int64_t Hk, int64_t Hv, int64_t dk,
                                      int64_t dv, int64_t N);

/*
 * omx_gdn_prefill without a workspace argument: the same kernels, with their scratch
 * (the workspace omx_gdn_prefill_workspace_size gives) in a fixed device array of the
 * library, omx_gdn_prefill_noalloc_max_scratch() bytes (64 MiB) per GPU, held from the
 * library's first use on that GPU until the process ends.  No reference counterpart:
 * it is for callers that cannot allocate device memory (code under HIP graph capture,
 * tight serving loops, harnesses that forbid hipMalloc).  It calls no hipMalloc/hipFree
 * and no allocating library routine.
 *   Arguments, layouts and results are those of omx_gdn_prefill.  Shapes whose workspace
 * exceeds the fixed size are rejected with OMX_GDN_EINVAL (at the Qwen3.5 head layout,
 * Hk=16 Hv=32 d=128, about 2,400 tokens per call).  Every call on one GPU uses that
 * GPU's one array: calls that overlap on one GPU (other streams, other threads) race
 * and give undefined results; serialise them.  Nothing in the scratch needs to start
 * at zero: every region is written before it is read within a call, and the one region
 * read before this call writes it (the fused norm's exchange ring) is cleared by the
 * call's own kernels, not by a memset, so a call may be captured in a HIP graph.
 */
int omx_gdn_prefill_noalloc(const void* mixed_qkv, const void* z, const void* a, const void* b,
                            const float* conv_w, const float* A_log, const float* dt_bias,
                            const float* norm_w, float eps, const int32_t* cu_seqlens, int64_t N,
                            const float* initial_state, float* final_state,
                            const void* conv_state_in, void* conv_state_out, void* out,
                            int64_t B, int64_t T, int64_t Hk, int64_t Hv, int64_t dk, int64_t dv,
                            int64_t K, int64_t chunk_size, void* stream);

/* Bytes of the fixed scratch behind omx_gdn_prefill_noalloc. */
size_t omx_gdn_prefill_noalloc_max_scratch(void);

/*
 * One cached decode step for one token per sequence: conv-cache update + SiLU,
 * gates, q/k L2-norm, recurrent rule, gated RMSNorm.  No reference counterpart:
 * omegalax drops the cache for Qwen3.5 (model.py:324-326) and its decode API
 * raises (text/api.py:128-131).  Semantics follow transformers'
 * causal_conv1d_update and torch_recurrent_gated_delta_rule, with the
 * reference's fp32 gated norm (deltanet.py:282-293).
 *
 *   mixed_qkv  [B, conv_dim] bf16;  z [B, Hv, dv] bf16;  a, b [B, Hv] bf16
 *   conv_state [B, conv_dim, K-1] bf16, updated in place (oldest tap first)
 *   state      [B, Hv, dk, dv] f32, updated in place
 *   out        [B, Hv*dv] bf16
 */
int omx_gdn_decode_step(const void* mixed_qkv, const void* z, const void* a, const void* b,
                        const float* conv_w, const float* A_log, const float* dt_bias,
                        const float* norm_w, float eps, void* conv_state, float* state,
                        void* out, int64_t B, int64_t Hk, int64_t Hv, int64_t dk, int64_t dv,
                        int64_t K, void* stream);

/*
 * One token of the recurrent rule on post-conv inputs (core level).  Semantics of
 * transformers' torch_recurrent_gated_delta_rule with use_qk_l2norm_in_kernel=True
 * and T=1; equals omx_gdn_chunk_fwd on a one-token sequence.
 *
 *   q, k [B, Hk, dk], v [B, Hv, dv] in_dtype;  g, beta [B, Hv] f32
 *   state [B, Hv, dk, dv] f32 in place;  o [B, Hv, dv] f32
 */
int omx_gdn_recurrent_step(const void* q, const void* k, const void* v, int in_dtype,
                           const float* g, const float* beta, float* state, float* o, int64_t B,
                           int64_t Hk, int64_t Hv, int64_t dk, int64_t dv, float scale,
                           void* stream);

/*
 * Backward pass (VJP) of omx_gdn_chunk_fwd.  Replaces the reverse-mode derivative
 * JAX takes of chunk_gated_delta_rule (deltanet.py:53-153) when the reference trains
 * through it (value_and_grad in trainers/vlm.py:157-195, remat at model.py:202): given
 * the forward's inputs and the cotangents of o (and of the final state), returns the
 * gradients of every input.  Inputs have the meaning and layout of omx_gdn_chunk_fwd;
 * the forward is recomputed inside (nothing is kept between the two calls).
 *
 *   d_o            [B, T, Hv, dv] f32, cotangent of o
 *   d_final_state  [N, Hv, dk, dv] f32 or NULL (zeros)
 *   dq, dk         [B, T, Hk, dk] in_dtype: gradients of the raw q, k (through the
 *                  in-kernel L2 norm when qk_l2norm != 0, summed over each key head's
 *                  value heads)
 *   dv             [B, T, Hv, dv] in_dtype
 *   dg, dbeta      [B, T, Hv] f32
 *   d_initial_state [N, Hv, dk, dv] f32 or NULL
 * Compiled shapes: bf16 inputs dk 64/128, fp32 inputs dk 32/64; dv 64/128.  Other
 * dk <= 128 (<= 64 with fp32 inputs) and dv <= 128 run padded (see the head-dims note
 * at the top).
 */
int omx_gdn_chunk_bwd(const void* q, const void* k, const void* v, int in_dtype,
                      const float* g, const float* beta, const float* initial_state,
                      const int32_t* cu_seqlens, int64_t N, const float* d_o,
                      const float* d_final_state, void* dq, void* dk, void* dv, float* dg,
                      float* dbeta, float* d_initial_state, int64_t B, int64_t T, int64_t Hk,
                      int64_t Hv, int64_t dk_dim, int64_t dv_dim, int64_t chunk_size,
                      float scale, int qk_l2norm, void* workspace, size_t workspace_bytes,
                      void* stream);

/*
 * Bytes of device workspace omx_gdn_chunk_bwd needs (16-byte aligned): the forward's
 * workspace, the per-chunk fp32 X = (I + L)^-1, L, P and gates, the state entering and
 * the state gradient leaving every chunk, V_new and its gradient, and per-value-head
 * gradients of the normalised q and k.
 */
size_t omx_gdn_chunk_bwd_workspace_size(int64_t B, int64_t T, int64_t Hk, int64_t Hv,
                                        int64_t dk, int64_t dv, int64_t N, int in_dtype);

/*
 * Backward pass (VJP) of omx_gdn_prefill: the gradients the reference's SFT step takes
 * through GatedDeltaNet.__call__ between its projections and out_proj (deltanet.py:243-293,
 * differentiated by jax.value_and_grad in trainers/vlm.py:157-195), for the cotangent
 * d_out of the output (and d_final_state of the final state).  Inputs have the meaning and
 * layout of omx_gdn_prefill (no conv history: conv windows start from zeros); the forward
 * is recomputed inside.
 *
 *   d_out          [B, T, Hv*dv] bf16
 *   d_final_state  [N, Hv, dk, dv] f32 or NULL (zeros)
 *   d_mixed_qkv    [B, T, conv_dim] bf16;  dz [B, T, Hv, dv] bf16;  da, db [B, T, Hv] bf16
 *   d_conv_w       [conv_dim, K] f32;  dA_log, d_dt_bias [Hv] f32;  d_norm_w [dv] f32
 *   d_initial_state [N, Hv, dk, dv] f32 or NULL
 * mixed_qkv, d_mixed_qkv, z, d_out, dz and conv_w must be 16-byte aligned.
 * Compiled shapes: K = 4, dk 64/128, dv 64/128, Hv <= 256.  Other dk <= 128 and
 * dv <= 128 run padded (see the head-dims note at the top).
 */
int omx_gdn_prefill_bwd(const void* mixed_qkv, const void* z, const void* a, const void* b,
                        const float* conv_w, const float* A_log, const float* dt_bias,
                        const float* norm_w, float eps, const int32_t* cu_seqlens, int64_t N,
                        const float* initial_state, const void* d_out,
                        const float* d_final_state, void* d_mixed_qkv, void* dz, void* da,
                        void* db, float* d_conv_w, float* dA_log, float* d_dt_bias,
                        float* d_norm_w, float* d_initial_state, int64_t B, int64_t T,
                        int64_t Hk, int64_t Hv, int64_t dk, int64_t dv, int64_t K,
                        int64_t chunk_size, void* workspace, size_t workspace_bytes,
                        void* stream);

/*
 * Bytes of device workspace omx_gdn_prefill_bwd needs (16-byte aligned): that of
 * omx_gdn_chunk_bwd for bf16 inputs, plus the recomputed conv output, gates, the rule's
 * fp32 output and its cotangent, the rule's input gradients and partial sums of the
 * parameter gradients.
 */
size_t omx_gdn_prefill_bwd_workspace_size(int64_t B, int64_t T, int64_t Hk, int64_t Hv,
                                          int64_t dk, int64_t dv, int64_t N);

/*
 * in_proj_qkv (deltanet.py:234, nnx.Linear with bf16 compute: fp32 accumulation, bf16
 * output) with, for conv = 1, the causal depthwise conv + SiLU of deltanet.py:35-50, 243
 * applied in the GEMM's epilogue: out = SiLU(conv(bf16(x W^T))) with the layer prefill's
 * rounding points.  A prototype of the projection-side fusion, kept to measure it against
 * the library GEMM (bench.py --workload qkv_conv); the layer calls the library GEMM.
 *
 *   x      [M, D] bf16 token rows, D a multiple of 64
 *   w      [N, D] bf16 (the nn.Linear / HF weight layout, [out, in]), N a multiple of 256
 *   conv_w [N, K] fp32, K = 4 (conv = 1 only)
 *   out    [M, N] bf16: x W^T (conv = 0) or its conv + SiLU (conv = 1)
 *
 * With conv = 1 the rows are M / T sequences of T rows each, and every sequence starts
 * from zeros (no conv cache: deltanet.py:46).  x, w, out and conv_w 16-byte aligned; x,
 * W and out each under 2 GiB.
 */
int omx_gdn_qkv_conv_proj(const void* x, const void* w, const float* conv_w, void* out,
                          int64_t M, int64_t D, int64_t N, int64_t T, int64_t K, int conv,
                          void* stream);

/*
 * The layer's gate projections, b = in_proj_b(x) and a = in_proj_a(x)
 * (deltanet.py:240-241, nnx.Linear with bf16 compute: fp32 accumulation, bf16
 * output), formed in one pass over the hidden rows instead of two GEMMs that each
 * read all of x.  No bias (use_bias=False, deltanet.py:182-187).
 *
 *   x        [M, D] bf16 (M token rows, rows contiguous), D a multiple of 8
 *   w_a, w_b [Hv, D] bf16 (the nn.Linear / HF weight layout, [out, in])
 *   a, b     [M, Hv] bf16
 *
 * 1 <= Hv <= 128.  x, w_a and w_b must be 16-byte aligned; a and b need only bf16
 * (2-byte) alignment.
 */
int omx_gdn_ab_proj(const void* x, const void* w_a, const void* w_b, void* a, void* b,
                    int64_t M, int64_t D, int64_t Hv, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* OMX_GDN_H */
