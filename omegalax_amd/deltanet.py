"""GatedDeltaNet on MI355X: Python mirror of omegalax's interface over libomx_gdn.

Reference interface (omegalax/models/qwen3_5/deltanet.py):
  * ``chunk_gated_delta_rule(q_BTHA, k_BTHA, v_BTHU, g_BTH, beta_BTH, chunk_size=64)``
    (:53-153) -- same positional signature and defaults, fp32 output; keyword-only
    extensions ``initial_state``, ``output_final_state``, ``cu_seqlens``.
  * ``GatedDeltaNet.__call__(hidden_BTD, attention_mask_BT=None)`` (:226-306) -- see
    ``omegalax_amd.layer``.
Tensors are torch tensors on the GPU (torch supplies device memory and the
current stream); every computation runs in libomx_gdn's HIP kernels.  There is
no fallback: a missing library or a CPU tensor raises.
"""
from __future__ import annotations

import torch

from . import _lib

__all__ = [
    "chunk_gated_delta_rule", "chunk_gated_delta_rule_bwd", "recurrent_gated_delta_rule_step",
    "gdn_prefill", "gdn_prefill_bwd",
    "gdn_decode_step", "GDNError",
]

GDNError = _lib.GDNError


def _ptr(t):
    return None if t is None else t.data_ptr()


def _stream(device):
    return torch.cuda.current_stream(device).cuda_stream


def _dev(*ts):
    dev = None
    for t in ts:
        if t is None:
            continue
        if not t.is_cuda:
            raise ValueError("omegalax_amd kernels need GPU tensors (got a CPU tensor)")
        if dev is None:
            dev = t.device
        elif t.device != dev:
            raise ValueError(f"tensors on different devices: {dev} vs {t.device}")
        if not t.is_contiguous():
            raise ValueError("omegalax_amd kernels need contiguous tensors")
    return dev


def _dtype_code(t):
    if t.dtype == torch.bfloat16:
        return _lib.BF16
    if t.dtype == torch.float32:
        return _lib.F32
    raise ValueError(f"unsupported dtype {t.dtype} (bf16 or fp32)")


def _f32(t):
    return None if t is None else t.to(torch.float32).contiguous()


def _cu_seqlens(cu, B, T, dev):
    """Packed-sequence offsets for the kernels: int32 [N+1] with B == 1.

    Valid offsets rise monotonically from cu[0] = 0 to cu[N] = T.  A device tensor is
    passed through without reading it on the host (no device-to-host copy, so the call
    can be captured into a HIP graph); the kernels read the offsets as their running
    maximum clamped to [0, T], with the first forced to 0 and the last to T, so every
    token belongs to exactly one sequence whatever the array holds.  A CPU tensor is
    checked on the host (ValueError when invalid) and copied to the device.
    Returns (offsets on ``dev``, N).
    """
    if cu.dtype != torch.int32 or cu.dim() != 1 or cu.numel() < 2:
        raise ValueError("cu_seqlens must be a 1-D int32 tensor with at least 2 entries")
    if B != 1:
        raise ValueError(f"cu_seqlens requires batch size 1, got {B}")
    if cu.is_cuda:
        if cu.device != dev:
            raise ValueError(f"tensors on different devices: {dev} vs {cu.device}")
        return cu.contiguous(), cu.numel() - 1
    h = cu
    if int(h[0]) != 0 or int(h[-1]) != T or bool((h[1:] < h[:-1]).any()):
        raise ValueError(f"cu_seqlens must rise monotonically from 0 to T={T}: {h.tolist()[:16]}")
    return cu.to(dev), cu.numel() - 1


def _workspace(nbytes, device):
    if nbytes == 0:
        return None
    return torch.empty(nbytes, dtype=torch.uint8, device=device)


def _prep_inputs(q_BTHA, k_BTHA, v_BTHU, g_BTH, beta_BTH, initial_state, cu_seqlens):
    q, k, v = q_BTHA.contiguous(), k_BTHA.contiguous(), v_BTHU.contiguous()
    if not (q.dtype == k.dtype == v.dtype):
        raise ValueError("q, k, v must share a dtype")
    g, beta = _f32(g_BTH), _f32(beta_BTH)
    dev = _dev(q, k, v, g, beta, initial_state)
    B, T, Hk, A = q.shape
    H, U = v.shape[2], v.shape[3]
    if k.shape != q.shape or v.shape[:2] != (B, T) or g.shape != (B, T, H) or beta.shape != (B, T, H):
        raise ValueError(f"shape mismatch: q{tuple(q.shape)} k{tuple(k.shape)} v{tuple(v.shape)} "
                         f"g{tuple(g.shape)} beta{tuple(beta.shape)}")
    N = B
    if cu_seqlens is not None:
        cu_seqlens, N = _cu_seqlens(cu_seqlens, B, T, dev)
    if initial_state is not None:
        initial_state = _f32(initial_state)
        if tuple(initial_state.shape) != (N, H, A, U):
            raise ValueError(f"initial_state must be {(N, H, A, U)}, got {tuple(initial_state.shape)}")
    return q, k, v, g, beta, initial_state, cu_seqlens, dev, (B, T, Hk, A, H, U, N)


def _chunk_fwd(q_BTHA, k_BTHA, v_BTHU, g_BTH, beta_BTH, chunk_size, initial_state,
               output_final_state, cu_seqlens, scale, use_qk_l2norm):
    q, k, v, g, beta, initial_state, cu_seqlens, dev, dims = _prep_inputs(
        q_BTHA, k_BTHA, v_BTHU, g_BTH, beta_BTH, initial_state, cu_seqlens)
    B, T, Hk, A, H, U, N = dims
    o = torch.empty((B, T, H, U), dtype=torch.float32, device=dev)
    fs = torch.empty((N, H, A, U), dtype=torch.float32, device=dev) if output_final_state else None
    sc = float(A ** -0.5) if scale is None else float(scale)
    L = _lib.lib()
    ws_bytes = L.omx_gdn_chunk_fwd_workspace_size(B, T, Hk, H, A, U, N, _dtype_code(q))
    ws = _workspace(ws_bytes, dev)
    _lib.call("omx_gdn_chunk_fwd", _ptr(q), _ptr(k), _ptr(v), _dtype_code(q), _ptr(g), _ptr(beta),
              _ptr(initial_state), _ptr(cu_seqlens), N, _ptr(o), _ptr(fs), B, T, Hk, H, A, U,
              int(chunk_size), sc, int(bool(use_qk_l2norm)), _ptr(ws), ws_bytes, _stream(dev))
    return o, fs


def chunk_gated_delta_rule_bwd(q_BTHA, k_BTHA, v_BTHU, g_BTH, beta_BTH, do_BTHU, chunk_size=64, *,
                               initial_state=None, d_final_state=None, cu_seqlens=None,
                               scale=None, use_qk_l2norm=True):
    """Gradients of ``chunk_gated_delta_rule`` at its inputs (the VJP JAX takes of
    deltanet.py:53-153 when the reference trains through it), on libomx_gdn.

    ``do_BTHU`` [B,T,H,U] is the cotangent of o, ``d_final_state`` [N,H,A,U] that of the
    final state (None = zeros).  Returns (dq, dk, dv, dg, dbeta, d_initial_state): dq/dk
    [B,T,Hk,A] and dv at the input dtype (gradients of the raw q/k, through the L2 norm
    and summed over each key head's value heads), dg/dbeta [B,T,H] fp32,
    d_initial_state [N,H,A,U] fp32.
    """
    q, k, v, g, beta, initial_state, cu_seqlens, dev, dims = _prep_inputs(
        q_BTHA, k_BTHA, v_BTHU, g_BTH, beta_BTH, initial_state, cu_seqlens)
    B, T, Hk, A, H, U, N = dims
    do = _f32(do_BTHU)
    _dev(do, d_final_state)
    if tuple(do.shape) != (B, T, H, U):
        raise ValueError(f"do must be {(B, T, H, U)}, got {tuple(do.shape)}")
    if d_final_state is not None:
        d_final_state = _f32(d_final_state)
        if tuple(d_final_state.shape) != (N, H, A, U):
            raise ValueError(f"d_final_state must be {(N, H, A, U)}")
    dq = torch.empty_like(q)
    dk = torch.empty_like(k)
    dv = torch.empty_like(v)
    dg = torch.empty((B, T, H), dtype=torch.float32, device=dev)
    db = torch.empty((B, T, H), dtype=torch.float32, device=dev)
    dh0 = torch.empty((N, H, A, U), dtype=torch.float32, device=dev)
    sc = float(A ** -0.5) if scale is None else float(scale)
    L = _lib.lib()
    ws_bytes = L.omx_gdn_chunk_bwd_workspace_size(B, T, Hk, H, A, U, N, _dtype_code(q))
    ws = _workspace(ws_bytes, dev)
    _lib.call("omx_gdn_chunk_bwd", _ptr(q), _ptr(k), _ptr(v), _dtype_code(q), _ptr(g), _ptr(beta),
              _ptr(initial_state), _ptr(cu_seqlens), N, _ptr(do), _ptr(d_final_state), _ptr(dq),
              _ptr(dk), _ptr(dv), _ptr(dg), _ptr(db), _ptr(dh0), B, T, Hk, H, A, U,
              int(chunk_size), sc, int(bool(use_qk_l2norm)), _ptr(ws), ws_bytes, _stream(dev))
    return dq, dk, dv, dg, db, dh0


class _ChunkGatedDeltaRule(torch.autograd.Function):
    """Autograd node of the chunked rule: forward omx_gdn_chunk_fwd, backward
    omx_gdn_chunk_bwd (the forward is recomputed there, as under the reference's remat,
    model.py:202)."""

    @staticmethod
    def forward(ctx, q, k, v, g, beta, initial_state, cu_seqlens, chunk_size, scale,
                use_qk_l2norm):
        o, fs = _chunk_fwd(q, k, v, g, beta, chunk_size, initial_state, True, cu_seqlens, scale,
                           use_qk_l2norm)
        ctx.save_for_backward(q, k, v, g, beta, initial_state, cu_seqlens)
        ctx.cfg = (chunk_size, scale, use_qk_l2norm)
        ctx.set_materialize_grads(False)
        return o, fs

    @staticmethod
    def backward(ctx, do, dfs):
        q, k, v, g, beta, initial_state, cu_seqlens = ctx.saved_tensors
        chunk_size, scale, use_qk_l2norm = ctx.cfg
        if do is None:
            do = torch.zeros(v.shape, dtype=torch.float32, device=v.device)
        dq, dk, dv, dg, db, dh0 = chunk_gated_delta_rule_bwd(
            q, k, v, g, beta, do, chunk_size, initial_state=initial_state, d_final_state=dfs,
            cu_seqlens=cu_seqlens, scale=scale, use_qk_l2norm=use_qk_l2norm)
        return (dq, dk, dv, dg, db, dh0 if initial_state is not None else None, None, None, None,
                None)


def chunk_gated_delta_rule(q_BTHA, k_BTHA, v_BTHU, g_BTH, beta_BTH, chunk_size=64, *,
                           initial_state=None, output_final_state=False, cu_seqlens=None,
                           scale=None, use_qk_l2norm=True):
    """Chunked gated delta rule (deltanet.py:53-153) on libomx_gdn.

    q/k [B,T,Hk,A] and v [B,T,H,U] (bf16 or fp32, same dtype); Hk may divide H
    (GQA, repeat-interleave semantics of deltanet.py:272-280) or equal it.
    g/beta [B,T,H].  Returns o [B,T,H,U] fp32, or (o, final_state) when
    ``output_final_state``.  ``cu_seqlens`` (int32 [N+1], B == 1) packs N
    sequences; ``initial_state`` is [N or B, H, A, U] fp32.  When gradients are
    enabled and an input requires them, the call is recorded for autograd and its
    backward runs omx_gdn_chunk_bwd.
    """
    needs_grad = torch.is_grad_enabled() and any(
        t is not None and t.requires_grad
        for t in (q_BTHA, k_BTHA, v_BTHU, g_BTH, beta_BTH, initial_state))
    if needs_grad:
        o, fs = _ChunkGatedDeltaRule.apply(q_BTHA, k_BTHA, v_BTHU, g_BTH, beta_BTH, initial_state,
                                           cu_seqlens, chunk_size, scale, use_qk_l2norm)
        return (o, fs) if output_final_state else o
    o, fs = _chunk_fwd(q_BTHA, k_BTHA, v_BTHU, g_BTH, beta_BTH, chunk_size, initial_state,
                       output_final_state, cu_seqlens, scale, use_qk_l2norm)
    return (o, fs) if output_final_state else o


def recurrent_gated_delta_rule_step(q, k, v, g, beta, state, *, scale=None):
    """One token of the recurrent rule, in place on ``state`` [B,H,A,U] fp32.

    q/k [B,Hk,A], v [B,H,U] (bf16 or fp32), g/beta [B,H].  Returns o [B,H,U] fp32.
    Semantics of transformers' torch_recurrent_gated_delta_rule (qk L2-norm in kernel).
    """
    q, k, v = q.contiguous(), k.contiguous(), v.contiguous()
    g, beta = _f32(g), _f32(beta)
    dev = _dev(q, k, v, g, beta, state)
    if state.dtype != torch.float32:
        raise ValueError("state must be fp32")
    B, Hk, A = q.shape
    H, U = v.shape[1], v.shape[2]
    if tuple(state.shape) != (B, H, A, U):
        raise ValueError(f"state must be {(B, H, A, U)}, got {tuple(state.shape)}")
    o = torch.empty((B, H, U), dtype=torch.float32, device=dev)
    sc = float(A ** -0.5) if scale is None else float(scale)
    _lib.call("omx_gdn_recurrent_step", _ptr(q), _ptr(k), _ptr(v), _dtype_code(q), _ptr(g),
              _ptr(beta), _ptr(state), _ptr(o), B, Hk, H, A, U, sc, _stream(dev))
    return o


def _gdn_prefill_fwd(mixed_qkv, z, a, b, conv_w, A_log, dt_bias, norm_w, *, num_k_heads, head_k_dim,
                     num_v_heads, head_v_dim, eps=1e-6, chunk_size=64, cu_seqlens=None,
                     initial_state=None, conv_state=None, output_final_state=False):
    """Prefill from projection outputs to the gated-norm output (deltanet.py:243-293).

    mixed_qkv [B,T,conv_dim] bf16, z [B,T,Hv,dv] bf16 (or [B,T,Hv*dv]), a/b [B,T,Hv] bf16,
    conv_w [conv_dim,K], A_log/dt_bias [Hv], norm_w [dv].  Returns out [B,T,Hv*dv] bf16,
    or (out, final_state, conv_state_out) when ``output_final_state``.
    """
    Hk, dk, Hv, dv = num_k_heads, head_k_dim, num_v_heads, head_v_dim
    x = mixed_qkv.contiguous()
    z = z.contiguous()
    a, b = a.contiguous(), b.contiguous()
    conv_w, A_log, dt_bias, norm_w = (_f32(t) for t in (conv_w, A_log, dt_bias, norm_w))
    dev = _dev(x, z, a, b, conv_w, A_log, dt_bias, norm_w, initial_state, conv_state)
    for name, t in (("mixed_qkv", x), ("z", z), ("a", a), ("b", b)):
        if t.dtype != torch.bfloat16:
            raise ValueError(f"{name} must be bf16")
    B, T, Cd = x.shape
    K = conv_w.shape[1]
    if Cd != 2 * Hk * dk + Hv * dv or conv_w.shape[0] != Cd:
        raise ValueError("mixed_qkv / conv_w channel count does not match the head layout")
    if z.numel() != B * T * Hv * dv or a.shape != (B, T, Hv) or b.shape != (B, T, Hv):
        raise ValueError("z/a/b shape does not match the head layout")
    N = B
    if cu_seqlens is not None:
        cu_seqlens, N = _cu_seqlens(cu_seqlens, B, T, dev)
    if initial_state is not None:
        initial_state = _f32(initial_state)
        if tuple(initial_state.shape) != (N, Hv, dk, dv):
            raise ValueError(f"initial_state must be {(N, Hv, dk, dv)}")
    if conv_state is not None:
        if conv_state.dtype != torch.bfloat16 or tuple(conv_state.shape) != (N, Cd, K - 1):
            raise ValueError(f"conv_state must be bf16 {(N, Cd, K - 1)}")
    out = torch.empty((B, T, Hv * dv), dtype=torch.bfloat16, device=dev)
    fs = cs = None
    if output_final_state:
        fs = torch.empty((N, Hv, dk, dv), dtype=torch.float32, device=dev)
        cs = torch.empty((N, Cd, K - 1), dtype=torch.bfloat16, device=dev)
    L = _lib.lib()
    ws_bytes = L.omx_gdn_prefill_workspace_size(B, T, Hk, Hv, dk, dv, N)
    ws = _workspace(ws_bytes, dev)
    _lib.call("omx_gdn_prefill", _ptr(x), _ptr(z), _ptr(a), _ptr(b), _ptr(conv_w), _ptr(A_log),
              _ptr(dt_bias), _ptr(norm_w), float(eps), _ptr(cu_seqlens), N, _ptr(initial_state),
              _ptr(fs), _ptr(conv_state), _ptr(cs), _ptr(out), B, T, Hk, Hv, dk, dv, K,
              int(chunk_size), _ptr(ws), ws_bytes, _stream(dev))
    return (out, fs, cs) if output_final_state else out


def gdn_prefill_bwd(mixed_qkv, z, a, b, conv_w, A_log, dt_bias, norm_w, d_out, *, num_k_heads,
                    head_k_dim, num_v_heads, head_v_dim, eps=1e-6, chunk_size=64,
                    cu_seqlens=None, initial_state=None, d_final_state=None):
    """Gradients of ``gdn_prefill`` (deltanet.py:243-293 between the projections and
    out_proj, as the reference's training step differentiates it) for the cotangent
    ``d_out`` [B,T,Hv*dv] of its output and ``d_final_state`` of the final state.

    Returns (d_mixed_qkv, dz, da, db) at the activations' bf16 and (d_conv_w, dA_log,
    d_dt_bias, d_norm_w, d_initial_state) in fp32.  Conv windows start from zeros (no conv
    history input).
    """
    Hk, dk, Hv, dv = num_k_heads, head_k_dim, num_v_heads, head_v_dim
    x = mixed_qkv.contiguous()
    z = z.contiguous()
    a, b = a.contiguous(), b.contiguous()
    d_out = d_out.to(torch.bfloat16).contiguous()
    conv_w, A_log, dt_bias, norm_w = (_f32(t) for t in (conv_w, A_log, dt_bias, norm_w))
    dev = _dev(x, z, a, b, conv_w, A_log, dt_bias, norm_w, initial_state, d_out, d_final_state)
    for name, t in (("mixed_qkv", x), ("z", z), ("a", a), ("b", b)):
        if t.dtype != torch.bfloat16:
            raise ValueError(f"{name} must be bf16")
    B, T, Cd = x.shape
    K = conv_w.shape[1]
    if Cd != 2 * Hk * dk + Hv * dv or conv_w.shape[0] != Cd:
        raise ValueError("mixed_qkv / conv_w channel count does not match the head layout")
    if z.numel() != B * T * Hv * dv or d_out.numel() != B * T * Hv * dv:
        raise ValueError("z / d_out size does not match the head layout")
    if a.shape != (B, T, Hv) or b.shape != (B, T, Hv):
        raise ValueError(f"a and b must be {(B, T, Hv)}, got {tuple(a.shape)}, {tuple(b.shape)}")
    N = B
    if cu_seqlens is not None:
        cu_seqlens, N = _cu_seqlens(cu_seqlens, B, T, dev)
    if initial_state is not None:
        initial_state = _f32(initial_state)
        if tuple(initial_state.shape) != (N, Hv, dk, dv):
            raise ValueError(f"initial_state must be {(N, Hv, dk, dv)}, got {tuple(initial_state.shape)}")
    if d_final_state is not None:
        d_final_state = _f32(d_final_state)
        if tuple(d_final_state.shape) != (N, Hv, dk, dv):
            raise ValueError(f"d_final_state must be {(N, Hv, dk, dv)}, got {tuple(d_final_state.shape)}")
    dx = torch.empty_like(x)
    dz = torch.empty_like(z)
    da = torch.empty_like(a)
    db = torch.empty_like(b)
    dconv = torch.empty_like(conv_w)
    dA = torch.empty_like(A_log)
    ddt = torch.empty_like(dt_bias)
    dnw = torch.empty_like(norm_w)
    dh0 = torch.empty((N, Hv, dk, dv), dtype=torch.float32, device=dev)
    L = _lib.lib()
    ws_bytes = L.omx_gdn_prefill_bwd_workspace_size(B, T, Hk, Hv, dk, dv, N)
    ws = _workspace(ws_bytes, dev)
    _lib.call("omx_gdn_prefill_bwd", _ptr(x), _ptr(z), _ptr(a), _ptr(b), _ptr(conv_w),
              _ptr(A_log), _ptr(dt_bias), _ptr(norm_w), float(eps), _ptr(cu_seqlens), N,
              _ptr(initial_state), _ptr(d_out), _ptr(d_final_state), _ptr(dx), _ptr(dz),
              _ptr(da), _ptr(db), _ptr(dconv), _ptr(dA), _ptr(ddt), _ptr(dnw), _ptr(dh0),
              B, T, Hk, Hv, dk, dv, K, int(chunk_size), _ptr(ws), ws_bytes, _stream(dev))
    return dx, dz, da, db, dconv, dA, ddt, dnw, dh0


class _GDNPrefill(torch.autograd.Function):
    """Autograd node of the layer prefill: forward omx_gdn_prefill, backward
    omx_gdn_prefill_bwd (which recomputes the forward)."""

    @staticmethod
    def forward(ctx, x, z, a, b, conv_w, A_log, dt_bias, norm_w, initial_state, cu_seqlens, cfg):
        out, fs, cs = _gdn_prefill_fwd(x, z, a, b, conv_w, A_log, dt_bias, norm_w,
                                       cu_seqlens=cu_seqlens, initial_state=initial_state,
                                       output_final_state=True, **cfg)
        ctx.save_for_backward(x, z, a, b, conv_w, A_log, dt_bias, norm_w, initial_state,
                              cu_seqlens)
        ctx.cfg = cfg
        ctx.set_materialize_grads(False)
        ctx.mark_non_differentiable(cs)
        return out, fs, cs

    @staticmethod
    def backward(ctx, d_out, d_fs, _d_cs):
        x, z, a, b, conv_w, A_log, dt_bias, norm_w, initial_state, cu_seqlens = ctx.saved_tensors
        if d_out is None:
            d_out = torch.zeros((x.shape[0], x.shape[1], ctx.cfg["num_v_heads"] * ctx.cfg["head_v_dim"]),
                                dtype=torch.bfloat16, device=x.device)
        dx, dz, da, db, dconv, dA, ddt, dnw, dh0 = gdn_prefill_bwd(
            x, z, a, b, conv_w, A_log, dt_bias, norm_w, d_out, cu_seqlens=cu_seqlens,
            initial_state=initial_state, d_final_state=d_fs, **ctx.cfg)
        return (dx, dz.view(z.shape), da, db, dconv, dA, ddt, dnw,
                dh0 if initial_state is not None else None, None, None)


def gdn_prefill(mixed_qkv, z, a, b, conv_w, A_log, dt_bias, norm_w, *, num_k_heads, head_k_dim,
                num_v_heads, head_v_dim, eps=1e-6, chunk_size=64, cu_seqlens=None,
                initial_state=None, conv_state=None, output_final_state=False):
    """Prefill from projection outputs to the gated-norm output (deltanet.py:243-293).

    mixed_qkv [B,T,conv_dim] bf16, z [B,T,Hv,dv] bf16 (or [B,T,Hv*dv]), a/b [B,T,Hv] bf16,
    conv_w [conv_dim,K], A_log/dt_bias [Hv], norm_w [dv].  Returns out [B,T,Hv*dv] bf16,
    or (out, final_state, conv_state_out) when ``output_final_state``.  When gradients are
    enabled and an input requires them (and no conv history is passed), the call is recorded
    for autograd; its backward runs omx_gdn_prefill_bwd.
    """
    cfg = dict(num_k_heads=num_k_heads, head_k_dim=head_k_dim, num_v_heads=num_v_heads,
               head_v_dim=head_v_dim, eps=eps, chunk_size=chunk_size)
    needs_grad = torch.is_grad_enabled() and any(
        t is not None and t.requires_grad
        for t in (mixed_qkv, z, a, b, conv_w, A_log, dt_bias, norm_w, initial_state))
    if needs_grad:
        if conv_state is not None:
            raise ValueError("gdn_prefill: gradients through a conv history are not supported")
        out, fs, cs = _GDNPrefill.apply(mixed_qkv, z, a, b, conv_w, A_log, dt_bias, norm_w,
                                        initial_state, cu_seqlens, cfg)
        return (out, fs, cs) if output_final_state else out
    return _gdn_prefill_fwd(mixed_qkv, z, a, b, conv_w, A_log, dt_bias, norm_w,
                            cu_seqlens=cu_seqlens, initial_state=initial_state,
                            conv_state=conv_state, output_final_state=output_final_state, **cfg)


# omx_gdn_ab_proj's limits (include/omx_gdn.h): D a multiple of 8, 1 <= Hv <= 128
AB_PROJ_MAX_HEADS = 128


def ab_proj_supported(D: int, Hv: int) -> bool:
    """Whether omx_gdn_ab_proj takes a hidden size D and Hv gate heads."""
    return D % 8 == 0 and 1 <= Hv <= AB_PROJ_MAX_HEADS


def _ab_proj_fwd(x, w_a, w_b):
    lead, D = x.shape[:-1], x.shape[-1]
    x2 = x.reshape(-1, D)
    if x2.dtype != torch.bfloat16 or w_a.dtype != torch.bfloat16 or w_b.dtype != torch.bfloat16:
        raise ValueError("gdn_ab_projections: x, w_a and w_b must be bf16")
    Hv = w_a.shape[0]
    if tuple(w_a.shape) != (Hv, D) or tuple(w_b.shape) != (Hv, D):
        raise ValueError(f"w_a and w_b must both be [Hv, {D}] (got {tuple(w_a.shape)}, "
                         f"{tuple(w_b.shape)})")
    if D % 8 != 0 or not 1 <= Hv <= AB_PROJ_MAX_HEADS:
        raise ValueError(f"gdn_ab_projections: the kernel takes D a multiple of 8 and 1 <= Hv <= "
                         f"{AB_PROJ_MAX_HEADS} (got D={D}, Hv={Hv})")
    # the kernel reads 16-byte pieces: a view whose storage offset breaks that alignment is
    # copied to a fresh (aligned) tensor
    x2, w_a, w_b = (t.contiguous() for t in (x2, w_a, w_b))
    x2, w_a, w_b = (t if t.data_ptr() % 16 == 0 else t.clone() for t in (x2, w_a, w_b))
    dev = _dev(x2, w_a, w_b)
    M = x2.shape[0]
    a = torch.empty((M, Hv), dtype=torch.bfloat16, device=dev)
    b = torch.empty((M, Hv), dtype=torch.bfloat16, device=dev)
    _lib.call("omx_gdn_ab_proj", _ptr(x2), _ptr(w_a), _ptr(w_b), _ptr(a), _ptr(b), M, D, Hv,
              _stream(dev))
    return a.reshape(*lead, Hv), b.reshape(*lead, Hv)


def qkv_conv_projection(x, w_qkv, conv_w=None, *, seq_len=None):
    """in_proj_qkv (deltanet.py:234) through the library's own GEMM kernel, and with
    ``conv_w`` [N, 4] the causal conv + SiLU (deltanet.py:35-50, 243) in its epilogue,
    over sequences of ``seq_len`` consecutive rows that start from zeros (no conv
    cache).  x [..., D] bf16, w_qkv [N, D] bf16; returns [..., N] bf16.  A forward-only
    prototype of the projection-side fusion (omx_gdn_qkv_conv_proj), measured against
    the library GEMM by ``bench.py --workload qkv_conv``; the layer itself uses F.linear.
    """
    lead, D = x.shape[:-1], x.shape[-1]
    x2 = x.reshape(-1, D).contiguous()
    w_qkv = w_qkv.contiguous()
    if x2.dtype != torch.bfloat16 or w_qkv.dtype != torch.bfloat16:
        raise ValueError("qkv_conv_projection: x and w_qkv must be bf16")
    N = w_qkv.shape[0]
    if w_qkv.shape[1] != D:
        raise ValueError(f"w_qkv must be [N, {D}] (got {tuple(w_qkv.shape)})")
    M = x2.shape[0]
    conv = conv_w is not None
    if conv:
        conv_w = _f32(conv_w)
        if tuple(conv_w.shape) != (N, 4):
            raise ValueError(f"conv_w must be [{N}, 4] (got {tuple(conv_w.shape)})")
        if seq_len is None:
            seq_len = x.shape[-2] if x.dim() >= 2 else M
    x2, w_qkv = (t if t.data_ptr() % 16 == 0 else t.clone() for t in (x2, w_qkv))
    dev = _dev(x2, w_qkv, conv_w)
    out = torch.empty((M, N), dtype=torch.bfloat16, device=dev)
    _lib.call("omx_gdn_qkv_conv_proj", _ptr(x2), _ptr(w_qkv), _ptr(conv_w), _ptr(out), M, D, N,
              int(seq_len or M), 4, int(conv), _stream(dev))
    return out.reshape(*lead, N)


class _ABProj(torch.autograd.Function):
    """Autograd node of the gate projections: forward omx_gdn_ab_proj; backward the
    linear maps' adjoints (dx = da W_a + db W_b, dW_a = da^T x, dW_b = db^T x) as bf16
    library GEMMs, as the two nn.Linear nodes they replace would run them."""

    @staticmethod
    def forward(ctx, x, w_a, w_b):
        ctx.save_for_backward(x, w_a, w_b)
        return _ab_proj_fwd(x, w_a, w_b)

    @staticmethod
    def backward(ctx, da, db):
        x, w_a, w_b = ctx.saved_tensors
        D = x.shape[-1]
        x2 = x.reshape(-1, D)
        da = torch.zeros_like(x2[:, :w_a.shape[0]]) if da is None else da.reshape(x2.shape[0], -1)
        db = torch.zeros_like(x2[:, :w_b.shape[0]]) if db is None else db.reshape(x2.shape[0], -1)
        dx = (da @ w_a + db @ w_b).reshape(x.shape) if ctx.needs_input_grad[0] else None
        dwa = da.t() @ x2 if ctx.needs_input_grad[1] else None
        dwb = db.t() @ x2 if ctx.needs_input_grad[2] else None
        return dx, dwa, dwb


def gdn_ab_projections(x, w_a, w_b):
    """(a, b) = (in_proj_a(x), in_proj_b(x)) of deltanet.py:240-241 in one pass over x.

    x [..., D] bf16, w_a / w_b [Hv, D] bf16 (nn.Linear weights).  Returns a, b [..., Hv]
    bf16, as the two bf16 linear maps give them (fp32 accumulation, rounded once).  When
    gradients are enabled and an input requires them, the call is recorded for autograd.
    """
    if torch.is_grad_enabled() and any(t.requires_grad for t in (x, w_a, w_b)):
        return _ABProj.apply(x, w_a, w_b)
    return _ab_proj_fwd(x, w_a, w_b)


def gdn_decode_step(mixed_qkv, z, a, b, conv_w, A_log, dt_bias, norm_w, conv_state, state, *,
                    num_k_heads, head_k_dim, num_v_heads, head_v_dim, eps=1e-6):
    """One cached decode step; updates ``conv_state`` and ``state`` in place.

    mixed_qkv [B,conv_dim] bf16, z [B,Hv,dv] bf16, a/b [B,Hv] bf16,
    conv_state [B,conv_dim,K-1] bf16, state [B,Hv,dk,dv] fp32.  Returns out [B,Hv*dv] bf16.
    """
    Hk, dk, Hv, dv = num_k_heads, head_k_dim, num_v_heads, head_v_dim
    x = mixed_qkv.contiguous()
    z, a, b = z.contiguous(), a.contiguous(), b.contiguous()
    conv_w, A_log, dt_bias, norm_w = (_f32(t) for t in (conv_w, A_log, dt_bias, norm_w))
    dev = _dev(x, z, a, b, conv_w, A_log, dt_bias, norm_w, conv_state, state)
    B, Cd = x.shape
    K = conv_w.shape[1]
    if Cd != 2 * Hk * dk + Hv * dv:
        raise ValueError("mixed_qkv channel count does not match the head layout")
    if tuple(conv_state.shape) != (B, Cd, K - 1) or conv_state.dtype != torch.bfloat16:
        raise ValueError(f"conv_state must be bf16 {(B, Cd, K - 1)}")
    if tuple(state.shape) != (B, Hv, dk, dv) or state.dtype != torch.float32:
        raise ValueError(f"state must be fp32 {(B, Hv, dk, dv)}")
    for name, t in (("mixed_qkv", x), ("z", z), ("a", a), ("b", b)):
        if t.dtype != torch.bfloat16:
            raise ValueError(f"{name} must be bf16")
    out = torch.empty((B, Hv * dv), dtype=torch.bfloat16, device=dev)
    _lib.call("omx_gdn_decode_step", _ptr(x), _ptr(z), _ptr(a), _ptr(b), _ptr(conv_w),
              _ptr(A_log), _ptr(dt_bias), _ptr(norm_w), float(eps), _ptr(conv_state),
              _ptr(state), _ptr(out), B, Hk, Hv, dk, dv, K, _stream(dev))
    return out
