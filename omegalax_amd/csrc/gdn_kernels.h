// Internal launch interface between the C ABI (gdn_capi.cpp) and the kernels.
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

namespace omx {

// Decode step.  Layer mode reads mixed_qkv/z/a/b and the conv cache and writes
// the gated-norm output; core mode reads post-conv q/k/v plus g/beta and writes
// the fp32 core output o.
struct DecodeParams {
  // layer mode
  const void* mixed_qkv;  // [B, conv_dim] bf16
  const void* z;          // [B, Hv, dv] bf16
  const void* a;          // [B, Hv] bf16
  const void* b;          // [B, Hv] bf16
  const float* conv_w;    // [conv_dim, K]
  const float* A_log;     // [Hv]
  const float* dt_bias;   // [Hv]
  const float* norm_w;    // [dv]
  void* conv_state;       // [B, conv_dim, K-1] bf16, updated in place
  void* out;              // [B, Hv*dv] bf16
  // core mode
  const void* q;          // [B, Hk, dk]
  const void* k;          // [B, Hk, dk]
  const void* v;          // [B, Hv, dv]
  const float* g;         // [B, Hv]
  const float* beta;      // [B, Hv]
  float* o;               // [B, Hv, dv]
  // both
  float* state;           // [B, Hv, dk, dv] fp32, updated in place
  int B, Hk, Hv, dk, dv, conv_k;
  float scale, eps;
};

// Chunked prefill (core function or fused layer).
// ring entries per (sequence, value head, column block) of ChunkParams::ss_xch
constexpr int kXchRing = 4;

struct ChunkParams {
  // core mode inputs: q/k [tokens, *, dk], v [tokens, *, DV] with row strides (elements)
  const void* q;
  const void* k;
  const void* v;
  long long q_ld, k_ld, v_ld;
  const float* g;         // [tokens, Hv]
  const float* beta;      // [tokens, Hv]
  float* o;               // [tokens, Hv, DV] fp32
  // layer mode inputs
  const void* mixed_qkv;  // [tokens, conv_dim] bf16
  const void* z;          // [tokens, Hv, DV] bf16
  const void* a;          // [tokens, Hv] bf16
  const void* b;          // [tokens, Hv] bf16
  const float* conv_w;    // [conv_dim, K]
  const float* A_log;
  const float* dt_bias;
  const float* norm_w;
  const void* conv_state_in;   // [N, conv_dim, K-1] bf16 or null
  void* conv_state_out;        // [N, conv_dim, K-1] bf16 or null
  void* out;                   // [tokens, Hv*DV] bf16
  void* o_part;                // unnormalised o [tokens, Hv, DV] bf16 (workspace)
  float* o_ss;                 // [ceil(tokens / 64), Hv, ss_slots, 64] fp32 (workspace):
                               // partial sums of squares of the fp32 o over a row
  int ss_slots;                // partials per (token, head) row (set by the scan's launcher)
  // (layer, scan with the gated norm fused) the workgroups' row partials of recent chunks,
  // [N][Hv][ss_xch_slots][kXchRing][64] pairs {fp32 bits, tag}: chunk c of a sequence uses
  // ring entry c % kXchRing with tag c + 1, written in one 8-byte store, so a reader that
  // sees its tag sees the value; zeroed by the preparation kernel (the task of each
  // sequence's first chunk)
  unsigned* ss_xch;
  int ss_xch_slots;            // partial slots per (chunk slot, value head) in ss_xch
  float inv_dv;                // 1 / the caller's dv (the norm's mean)
  // both
  const float* initial_state;  // [N, Hv, dk, DV] or null
  float* final_state;          // [N, Hv, dk, DV] or null
  const int32_t* cu_seqlens;   // [N+1] or null (then sequence n = batch row n of length T):
                               // the plan's ordered copy (workspace) once set up
  const int32_t* cu_in;        // the caller's cu_seqlens, read only by the plan kernel
  int N, T, Hk, Hv, dk, DV, nb, conv_k, conv_dim;
  float scale, eps;
  int qk_l2norm;
  // workspace written by the preparation kernel, read by the scan
  void* kn;                    // normalised k [tokens, Hk, dk] in the input precision, or null
  void* qn;                    // normalised q, likewise
  void* vc;                    // layer: conv + SiLU output of v [tokens, Hv, DV] bf16
  unsigned char* rec;          // per (chunk, value head) records, layout in gdn_chunk.h
  int32_t* chunk_off;          // cu_seqlens: [N+1] first chunk index of each sequence; else null
  const int32_t* seq_order;    // cu_seqlens: [N] sequences, longest first (the plan); else null
  int nch;                     // chunks per sequence without cu_seqlens
  int n_rec;                   // chunk slots the preparation kernel covers
  // the scan's k, q, v rows: kn/qn/vc or the raw inputs, with row strides (elements)
  const void* ks;
  const void* qs;
  const void* vs;
  long long ks_ld, qs_ld, vs_ld;
  // backward pass only (the backward variants of the two kernels write them)
  float* xlpg;                 // prep: per (chunk slot, value head) X^T, Lg, P [64][64], G [64]
  float* states;               // scan: the state entering each chunk [slot][Hv][DV][dk]
  float* vnew;                 // scan: V_new [tokens][Hv][DV]
};

// Backward pass of the chunked rule (gdn_bwd.hip): the reverse state-gradient scan,
// the chunk-parallel gradients and the q/k finalisation.
struct BwdParams {
  const void* ks;              // normalised (or raw) k rows [tokens][*][dk], input precision
  const void* qs;
  long long ks_ld, qs_ld;
  const void* v;               // [tokens][Hv][DV], input precision
  const float* dO;             // [tokens][Hv][DV]
  const float* dht;            // [N][Hv][dk][DV] or null
  const unsigned char* rec;    // prep records
  const float* xlpg;           // prep backward extras
  const float* states;         // state entering each chunk [slot][Hv][DV][dk]
  const float* vnew;           // V_new
  float* dstates;              // gradient of the state leaving each chunk [slot][Hv][DV][dk]
  float* dvnew;                // gradient of V_new [tokens][Hv][DV]
  float* dh0;                  // [N][Hv][dk][DV] or null
  void* dqh;                   // per value head gradient of the normalised q [tokens][Hv][dk],
                               // at the input precision (bf16 or fp32)
  void* dkh;                   // likewise k
  void* dv;                    // [tokens][Hv][DV], input precision
  float* dg;                   // [tokens][Hv]
  float* dbeta;                // [tokens][Hv]
  const void* q;               // raw q, k [tokens][Hk][dk] (L2-norm backward)
  const void* k;
  void* dq;                    // [tokens][Hk][dk], input precision
  void* dk_out;
  const int32_t* cu_seqlens;
  const int32_t* chunk_off;
  const int32_t* seq_order;
  int N, T, Hk, Hv, dk, DV, nb, nch, n_rec, in_f32, qk_l2norm;
  float scale;
};

// floats of the backward extras per (chunk slot, value head): X, Lg, P [64][64], G [64]
constexpr int kXlpgFloatsHost = 3 * 64 * 64 + 64;

// kernel modes of the chunked prefill (template arguments of both kernels)
constexpr int kModeBF16 = 0, kModeF32 = 1, kModeLayer = 2;

bool chunk_dims_supported(int dk, int dv, bool f32_inputs);
int chunk_block_cols();
bool layer_dims_supported(int dk, int dv);
// (layer) whether the scan forms the v rows itself (conv + SiLU), so the workspace holds
// no conv(v) rows
bool layer_scan_forms_v(int dk);
// bytes of one (chunk, value head) record for a mode
int chunk_record_bytes(int mode, bool bwd = false);
// cu_in -> the ordered offsets cu_seqlens and chunk_off (one workgroup); then the
// preparation kernel and the scan
hipError_t launch_chunk_plan(const ChunkParams& p, hipStream_t stream);
hipError_t launch_prep(const ChunkParams& p, int mode, hipStream_t stream);
hipError_t launch_scan(const ChunkParams& p, int mode, hipStream_t stream);
// backward variants: the prep also writes xlpg, the scan writes states and vnew (no o)
hipError_t launch_prep_bwd(const ChunkParams& p, int mode, hipStream_t stream);
hipError_t launch_scan_bwd(const ChunkParams& p, int mode, hipStream_t stream);
bool bwd_dims_supported(int dk, int dv, bool f32_inputs);
hipError_t launch_bwd(const BwdParams& p, hipStream_t stream);

// Backward of the layer prefill around the chunked rule's backward (gdn_layer_bwd.hip).
// bf16 arrays are raw uint16_t.
struct LayerBwdParams {
  // forward inputs
  const uint16_t* x;           // mixed_qkv [tokens][conv_dim]
  const float* conv_w;         // [conv_dim][4]
  const uint16_t* a;           // [tokens][Hv]
  const uint16_t* b;
  const float* A_log;          // [Hv]
  const float* dt_bias;
  const uint16_t* z;           // [tokens][Hv][dv]
  const float* norm_w;         // [dv]
  const uint16_t* dout;        // [tokens][Hv*dv], cotangent of the output
  float eps;
  // workspace: recomputed forward values and the rule's gradients
  uint16_t* q;                 // conv + SiLU output split: q, k [tokens][Hk*dk], v [tokens][Hv*dv]
  uint16_t* k;
  uint16_t* v;
  float* g;                    // [tokens][Hv]
  float* beta;
  const float* o;              // the rule's fp32 output [tokens][Hv][dv]
  float* dO;                   // its cotangent
  uint16_t* grad_q;            // gradients of q, k, v (bf16)
  uint16_t* grad_k;
  uint16_t* grad_v;
  const float* dg;             // [tokens][Hv]
  const float* dbeta;
  float* part_norm;            // partial sums [norm blocks][dv]
  float* part_gates;           // [gate blocks][2 Hv]
  float* part_conv;            // [conv blocks][conv_dim][4]
  // outputs
  uint16_t* dx;                // d mixed_qkv
  uint16_t* dz;
  uint16_t* da;
  uint16_t* db;
  float* d_conv_w;             // [conv_dim][4]
  float* dA_log;               // [Hv]
  float* d_dt_bias;            // [Hv]
  float* d_norm_w;             // [dv]
  const int32_t* cu_seqlens;
  long long tokens;
  int N, T, Hk, Hv, dk, dv, conv_dim;
  int dv_mean;                 // divisor of the norm's means (dv, or the real dv of padded rows)
};
int layer_bwd_norm_blocks();
long long layer_bwd_conv_blocks(long long tokens);
int layer_bwd_gate_blocks(long long tokens);
hipError_t launch_layer_fwd_pieces(const LayerBwdParams& p, hipStream_t stream);
hipError_t launch_layer_norm_bwd(const LayerBwdParams& p, hipStream_t stream);
hipError_t launch_layer_tail_bwd(const LayerBwdParams& p, hipStream_t stream);

// Gated RMSNorm of the layer prefill: out = w * o * rsqrt(mean(o^2) + eps) * silu(z) per
// (token, value head) row of dv (a multiple of 16, dv / 8 at most 32), with o the scan's
// bf16 o and the row's sum of squares the butterfly sum of its nss fp32 partials in o_ss
// (ss_index layout, formed by the scan from the fp32 o); the mean divides it by dv_mean.
hipError_t launch_norm_epilogue(const void* o_part, const float* o_ss, int nss, const void* z,
                                const float* norm_w, void* out, long long tokens, int Hv, int dv,
                                int dv_mean, float eps, hipStream_t stream);

// Row-sum partials per (token, value head) the layer scan writes for these parameters.
int layer_ss_slots(const ChunkParams& p);
// Column blocks (workgroups) per value head of the layer scan for these parameters.
int layer_scan_blocks(const ChunkParams& p);
// Whether the layer scan applies the gated norm itself for these parameters (then it
// writes p.out and the epilogue kernel is not needed); needs p.ss_xch.
bool layer_scan_fuses_norm(const ChunkParams& p);

// An [R][G][E] view of a buffer for launch_pad_copy: element pointer, group and element
// counts, row and group strides (elements).
struct PadView {
  const void* p;
  int G, E;
  long long rs, gs;
};
// dst[r][g][e] = (g < src.G && e < src.E) ? src[r][g][e] : 0 for g < dst.G, e < dst.E;
// esize 2 (bf16) or 4 (fp32) bytes (gdn_pad.hip)
hipError_t launch_pad_copy(const PadView& src, const PadView& dst, long long R, int esize,
                           hipStream_t stream);

bool decode_dims_supported(int dk, int dv);
int decode_max_gqa();
hipError_t launch_decode(const DecodeParams& p, bool layer, bool in_bf16, hipStream_t stream);

// The gate projections a = x W_a^T, b = x W_b^T (bf16, fp32 accumulation) in one pass
// over x [M, D] (gdn_proj.hip); D % 8 == 0, 1 <= Hv <= ab_proj_max_heads().
int ab_proj_max_heads();
// x W^T for x [M, D], W [N, D] bf16 (bf16 out), and with conv the causal conv + SiLU of
// that product over sequences of T rows in the epilogue (gdn_qkv.hip); N a multiple of
// qkv_proj_tile_cols(), D of qkv_proj_tile_depth().
hipError_t launch_qkv_proj(const void* x, const void* w, const float* conv_w, void* out,
                           long long M, int N, int D, long long T, bool conv, hipStream_t stream);
int qkv_proj_tile_cols();
int qkv_proj_tile_depth();

hipError_t launch_ab_proj(const void* x, const void* wa, const void* wb, void* a, void* b,
                          long long M, int D, int Hv, hipStream_t stream);

}  // namespace omx
