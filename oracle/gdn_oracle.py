"""NumPy restatement of omegalax's Qwen3.5 gated-delta-rule path (test oracle).

TEST INFRASTRUCTURE ONLY: imported by ``tests/``, ``__graft_entry__.smoke()``
and the ``cpu_baseline`` leg of ``bench.py``; never by the product package.

Reference: /root/reference/omegalax/models/qwen3_5/deltanet.py (cited below as
``deltanet.py:LINE``) and norms.py.  The reference has no decode step, no
initial/final state and no ``cu_seqlens``; those semantics follow the
third-party torch functions that the reference's parity tests treat as ground
truth (transformers ``models/qwen3_5/modeling_qwen3_5.py``: ``causal_conv1d_update``,
``torch_chunk_gated_delta_rule``, ``torch_recurrent_gated_delta_rule``).

Every function computes in float64 unless ``dtype`` says otherwise.  Where the
reference rounds to the activation dtype (bf16 on the layer path), the caller
passes ``act_round=round_bf16`` so the oracle rounds at the same points.

Pinning (what checks each function; the tests live in tests/test_oracle.py):
  l2norm                    closed forms (unit vectors, zero vector, scaling) + HF fixture
  causal_depthwise_conv1d   brute force via np.convolve, impulse/identity/shift + HF fixture
  gates                     closed forms (softplus/sigmoid special values)
  chunk_gated_delta_rule    naive fp64 recurrence, chunk-size independence, T=1 closed
                            form, orthonormal-key retrieval, linearity, padding, varlen ==
                            per-sequence, HF torch_chunk_gated_delta_rule fixtures
  recurrent_gated_delta_rule brute-force matrix algebra on tiny cases + HF fixtures
  gated_rmsnorm             closed forms + HF Qwen3_5RMSNormGated fixture
  gdn_decode_step           decode-after-prefill == longer prefill; HF conv-update fixture
  gdn_prefill_layer         composition of the pinned pieces; split-prefill == full prefill
No function here is "parity unpinned".
"""
from __future__ import annotations

import numpy as np

__all__ = [
    "round_bf16", "l2norm", "causal_depthwise_conv1d", "silu", "sigmoid", "softplus",
    "gates", "chunk_gated_delta_rule", "recurrent_gated_delta_rule", "gated_rmsnorm",
    "gdn_prefill_layer", "gdn_decode_step", "split_mixed_qkv",
]


def round_bf16(x):
    """Round to the nearest bfloat16 value (ties to even), returned as float32.

    Values are first rounded to float32, as a bf16 cast from fp32 would see them.
    """
    a = np.array(x, dtype=np.float32, copy=True, order="C")
    u = a.view(np.uint32)
    nan = np.isnan(a)
    # uint32 arithmetic: a finite value's sum cannot wrap (it rounds up to inf at most);
    # NaNs, whose sum may wrap, are restored below
    r = (u >> 16) & 1
    r += 0x7FFF
    u += r
    u &= 0xFFFF0000
    if nan.any():
        a[nan] = np.nan
    return a


def _ident(x):
    return x


def sigmoid(x):
    return 1.0 / (1.0 + np.exp(-x))


def silu(x):
    return x * sigmoid(x)


def softplus(x):
    # log(1 + e^x) without overflow (jax.nn.softplus == logaddexp(x, 0)).
    return np.logaddexp(x, 0.0)


def l2norm(x, eps=1e-6, act_round=_ident):
    """``x * rsqrt(sum(x*x, -1) + eps)`` -- deltanet.py:30-32 (eps inside the sqrt)."""
    x64 = np.asarray(x, dtype=np.float64)
    inv = 1.0 / np.sqrt((x64 * x64).sum(-1, keepdims=True) + eps)
    return act_round(x64 * inv)


def causal_depthwise_conv1d(x_BTC, w_CK, history_BCk=None):
    """Depthwise causal conv1d in token-major layout -- deltanet.py:35-50.

    ``y[t, c] = sum_k w[c, k] * x[t - K + 1 + k, c]`` with zero left padding
    (deltanet.py:46), so ``w[:, K-1]`` multiplies the current token.  The
    reference works in (B, C, T) via transposes (deltanet.py:234, 244); this
    works in (B, T, C) directly.  ``history_BCk`` ([B, C, K-1], oldest first)
    replaces the zero padding, as the conv-state cache does in
    ``causal_conv1d_update`` (HF modeling_qwen3_5.py, causal_conv1d_update).
    """
    x = np.asarray(x_BTC, dtype=np.float64)
    w = np.asarray(w_CK, dtype=np.float64)
    B, T, C = x.shape
    K = w.shape[1]
    if history_BCk is None:
        hist = np.zeros((B, K - 1, C))
    else:
        hist = np.asarray(history_BCk, dtype=np.float64).transpose(0, 2, 1)
    xp = np.concatenate([hist, x], axis=1)  # [B, K-1+T, C]
    y = np.zeros_like(x)
    for k in range(K):
        y += w[None, None, :, k] * xp[:, k:k + T, :]
    return y


def gates(a_BTH, b_BTH, A_log_H, dt_bias_H, act_round=_ident):
    """beta = sigmoid(b) at activation dtype; g = -exp(A_log) * softplus(a + dt_bias).

    deltanet.py:248-250.  ``a`` is cast to fp32 before the add (:250), beta
    stays in the activation dtype (:248) and is rounded with ``act_round``.
    """
    b64 = np.asarray(b_BTH, dtype=np.float64)
    a64 = np.asarray(a_BTH, dtype=np.float64)
    beta = act_round(sigmoid(b64))
    A = -np.exp(np.asarray(A_log_H, dtype=np.float64))
    g = A * softplus(a64 + np.asarray(dt_bias_H, dtype=np.float64))
    return np.asarray(g, dtype=np.float64), np.asarray(beta, dtype=np.float64)


def _gqa_expand(x, H):
    """Repeat-interleave heads: v-head h reads k-head h // (H / Hk) (deltanet.py:272-280)."""
    Hk = x.shape[2]
    if Hk == H:
        return x
    if H % Hk:
        raise ValueError(f"value heads {H} not a multiple of key heads {Hk}")
    return np.repeat(x, H // Hk, axis=2)


def _chunk_core(q, k, v, g, beta, C, S0, dt):
    """Chunked gated delta rule on one batch, BH-major fp arrays.

    q, k [B,H,T,A]; v [B,H,T,U]; g, beta [B,H,T]; S0 [B,H,A,U].
    Follows deltanet.py:75-153 step for step; returns (o [B,H,T,U], S [B,H,A,U]).
    """
    B, H, T, A = k.shape
    U = v.shape[-1]
    pad = (C - T % C) % C  # deltanet.py:75-82: zero padding (g=0, beta=0 => no effect on S)
    if pad:
        q, k, v = (np.pad(x, ((0, 0), (0, 0), (0, pad), (0, 0))) for x in (q, k, v))
        beta, g = (np.pad(x, ((0, 0), (0, 0), (0, pad))) for x in (beta, g))
    Tt = T + pad
    q = q * dt.type(A ** -0.5)                                 # :84-85
    vb = v * beta[..., None]                                   # :87
    kb = k * beta[..., None]                                   # :88
    J = Tt // C
    qc, kc, kbc, vbc = (x.reshape(B, H, J, C, x.shape[-1]) for x in (q, k, kb, vb))  # :90-95
    gc = np.cumsum(g.reshape(B, H, J, C), axis=-1)             # :96-98
    tril = np.tril(np.ones((C, C), dtype=dt))
    diff = gc[..., :, None] - gc[..., None, :]
    decay = np.exp(diff * tril) * tril                         # :100-104
    attn = -(kbc @ np.swapaxes(kc, -1, -2) * decay)            # :107
    attn = np.where(np.triu(np.ones((C, C), dtype=bool)), 0.0, attn).astype(dt)  # :106,108
    lhs = np.eye(C, dtype=dt) - attn                           # :110-111
    # solve_triangular(lhs, I, lower=True) (:112-113) by forward substitution; lhs has a
    # unit diagonal, so row i of the inverse is e_i - sum_{m<i} lhs[i, m] * X[m].
    X = np.zeros_like(lhs)
    for i in range(C):
        acc = np.zeros(lhs.shape[:-2] + (C,), dtype=dt)
        acc[..., i] = 1.0
        if i:
            acc -= np.einsum("...m,...mc->...c", lhs[..., i, :i], X[..., :i, :])
        X[..., i, :] = acc / lhs[..., i, i][..., None]
    u = X @ vbc                                                # :115
    w = X @ (kbc * np.exp(gc)[..., None])                      # :116
    S = S0.astype(dt).copy()                                   # :118 (zero-init in the reference)
    strict_upper = np.triu(np.ones((C, C), dtype=bool), k=1)   # :119
    o = np.zeros((B, H, J, C, U), dtype=dt)
    for j in range(J):                                         # lax.scan, :121-148
        intra = qc[:, :, j] @ np.swapaxes(kc[:, :, j], -1, -2) * decay[:, :, j]   # :130
        intra = np.where(strict_upper, 0.0, intra)                                 # :131
        v_new = u[:, :, j] - w[:, :, j] @ S                                        # :133-134
        inter = np.exp(gc[:, :, j])[..., None] * (qc[:, :, j] @ S)                 # :136
        o[:, :, j] = inter + intra @ v_new                                         # :137
        g_last = gc[:, :, j, -1][..., None, None]                                  # :139
        kdec = kc[:, :, j] * np.exp(gc[:, :, j, -1:] - gc[:, :, j])[..., None]     # :140-141
        S = S * np.exp(g_last) + np.swapaxes(kdec, -1, -2) @ v_new                 # :142
    o = o.reshape(B, H, Tt, U)[:, :, :T]                       # :149-152
    return o, S


def chunk_gated_delta_rule(q_BTHA, k_BTHA, v_BTHU, g_BTH, beta_BTH, chunk_size=64, *,
                           initial_state=None, output_final_state=False, cu_seqlens=None,
                           dtype=np.float64, act_round=_ident, qk_l2norm=True):
    """Chunked gated delta rule -- deltanet.py:53-153, plus the HF extensions.

    Inputs are (B, T, H, dim).  q/k may carry fewer heads than v (GQA); they are
    expanded by repeat-interleave as deltanet.py:272-280 does before the call.
    q and k are L2-normalised at their input precision (deltanet.py:65-66;
    ``act_round`` models a bf16 input dtype) before the cast to ``dtype``.

    Extensions the reference lacks (semantics of HF torch_chunk_gated_delta_rule):
    ``initial_state`` [B or N, H, A, U]; ``output_final_state`` returns (o, S);
    ``cu_seqlens`` (int [N+1], requires B == 1) runs each packed sequence
    independently with its own initial state.
    Returns o [B, T, H, U] in ``dtype`` (the reference returns fp32, :153).
    """
    dt = np.dtype(dtype)
    H = v_BTHU.shape[2]
    q = _gqa_expand(np.asarray(q_BTHA, dtype=np.float64), H)
    k = _gqa_expand(np.asarray(k_BTHA, dtype=np.float64), H)
    if qk_l2norm:
        q = l2norm(q, act_round=act_round)
        k = l2norm(k, act_round=act_round)
    q, k, v = (np.asarray(x, dtype=np.float64).transpose(0, 2, 1, 3).astype(dt)
               for x in (q, k, v_BTHU))                       # :68
    beta = np.asarray(beta_BTH, dtype=np.float64).transpose(0, 2, 1).astype(dt)   # :69
    g = np.asarray(g_BTH, dtype=np.float64).transpose(0, 2, 1).astype(dt)         # :70
    B, _, T, A = k.shape
    U = v.shape[-1]
    if cu_seqlens is None:
        S0 = (np.zeros((B, H, A, U), dt) if initial_state is None
              else np.asarray(initial_state, dtype=np.float64).astype(dt))
        o, S = _chunk_core(q, k, v, g, beta, chunk_size, S0, dt)
    else:
        cu = np.asarray(cu_seqlens, dtype=np.int64)
        if B != 1:
            raise ValueError("cu_seqlens requires batch size 1")
        N = len(cu) - 1
        o = np.zeros((1, H, T, U), dt)
        S = np.zeros((N, H, A, U), dt)
        for n in range(N):
            s, e = int(cu[n]), int(cu[n + 1])
            S0 = (np.zeros((1, H, A, U), dt) if initial_state is None
                  else np.asarray(initial_state[n:n + 1], dtype=np.float64).astype(dt))
            if e == s:
                S[n] = S0[0]
                continue
            sl = slice(s, e)
            on, Sn = _chunk_core(q[:, :, sl], k[:, :, sl], v[:, :, sl], g[:, :, sl],
                                 beta[:, :, sl], chunk_size, S0, dt)
            o[:, :, sl] = on
            S[n] = Sn[0]
    o = o.transpose(0, 2, 1, 3)                                # :153
    return (o, S) if output_final_state else o


def recurrent_gated_delta_rule(q_BTHA, k_BTHA, v_BTHU, g_BTH, beta_BTH, *, initial_state=None,
                               act_round=_ident, qk_l2norm=True):
    """Token-by-token gated delta rule (the textbook recurrence), fp64.

    Semantics of HF torch_recurrent_gated_delta_rule with use_qk_l2norm_in_kernel:
      S <- e^g S;  kv = S^T k;  delta = beta (v - kv);  S <- S + k delta^T;  o = S^T (q/sqrt(A)).
    Returns (o [B,T,H,U], S [B,H,A,U]).
    """
    H = v_BTHU.shape[2]
    q = _gqa_expand(np.asarray(q_BTHA, dtype=np.float64), H)
    k = _gqa_expand(np.asarray(k_BTHA, dtype=np.float64), H)
    if qk_l2norm:
        q = l2norm(q, act_round=act_round)
        k = l2norm(k, act_round=act_round)
    q = np.asarray(q, np.float64)
    k = np.asarray(k, np.float64)
    v = np.asarray(v_BTHU, dtype=np.float64)
    g = np.asarray(g_BTH, dtype=np.float64)
    beta = np.asarray(beta_BTH, dtype=np.float64)
    B, T, _, A = k.shape
    U = v.shape[-1]
    S = (np.zeros((B, H, A, U)) if initial_state is None
         else np.asarray(initial_state, dtype=np.float64).copy())
    q = q * A ** -0.5
    o = np.zeros((B, T, H, U))
    for t in range(T):
        S = S * np.exp(g[:, t])[..., None, None]
        kv = np.einsum("bhau,bha->bhu", S, k[:, t])
        delta = (v[:, t] - kv) * beta[:, t][..., None]
        S = S + k[:, t][..., :, None] * delta[..., None, :]
        o[:, t] = np.einsum("bhau,bha->bhu", S, q[:, t])
    return o, S


def gated_rmsnorm(o_NU, z_NU, w_U, eps=1e-6, act_round=_ident):
    """Inline gated RMSNorm of deltanet.py:282-293 (semantics of norms.py:51-60).

    The core output is fp32, so the reference's ``dtype`` is fp32 and every step
    here is full precision; ``act_round`` rounds only the final result (what
    out_proj consumes after its bf16 promotion, deltanet.py:216-223, 305).
    """
    x = np.asarray(o_NU, dtype=np.float64)
    var = np.mean(x * x, axis=-1, keepdims=True)
    n = x / np.sqrt(var + eps)
    n = np.asarray(w_U, dtype=np.float64) * n
    return act_round(n * silu(np.asarray(z_NU, dtype=np.float64)))


def split_mixed_qkv(x_BTC, Hk, dk, Hv, dv):
    """Split the conv output into q [.., Hk, dk], k [.., Hk, dk], v [.., Hv, dv] (deltanet.py:268-271)."""
    kd = Hk * dk
    lead = x_BTC.shape[:-1]
    q = x_BTC[..., :kd].reshape(*lead, Hk, dk)
    k = x_BTC[..., kd:2 * kd].reshape(*lead, Hk, dk)
    v = x_BTC[..., 2 * kd:].reshape(*lead, Hv, dv)
    return q, k, v


def _conv_silu(x_BTC, conv_w, history, act_round):
    w = act_round(np.asarray(conv_w, dtype=np.float32))        # cast to act dtype (deltanet.py:243)
    y = act_round(causal_depthwise_conv1d(x_BTC, w, history))  # conv output in act dtype
    return act_round(silu(y))                                  # SiLU in act dtype (:243)


def gdn_prefill_layer(mixed_qkv, z, a, b, conv_w, A_log, dt_bias, norm_w, *, Hk, dk, Hv, dv,
                      eps=1e-6, chunk_size=64, cu_seqlens=None, initial_state=None,
                      conv_state=None, act_round=round_bf16, dtype=np.float64):
    """GDN prefill from projections to the gated-norm output: deltanet.py:243-293.

    mixed_qkv [B,T,conv_dim], z [B,T,Hv,dv], a/b [B,T,Hv] (activation-dtype values),
    conv_w [conv_dim, K], A_log/dt_bias [Hv], norm_w [dv].
    Optional: cu_seqlens (B == 1; conv history and state reset per sequence),
    initial_state [N,Hv,dk,dv], conv_state [N,conv_dim,K-1] (history before each sequence).
    ``dtype`` is the precision of the chunked core (float64 for checking, float32 for the
    CPU baseline, which is the reference's own precision).
    Returns (out [B,T,Hv*dv] rounded by act_round, final_state [N,Hv,dk,dv],
    conv_state_out [N,conv_dim,K-1]).
    """
    x = np.asarray(mixed_qkv, dtype=np.float64)
    B, T, Cd = x.shape
    K = conv_w.shape[1]
    if cu_seqlens is None:
        bounds = None
        xc = _conv_silu(x, conv_w, conv_state, act_round)
        xin = [x]
    else:
        cu = np.asarray(cu_seqlens, dtype=np.int64)
        xc = np.zeros_like(x)
        for n in range(len(cu) - 1):
            s, e = int(cu[n]), int(cu[n + 1])
            if e > s:
                h = None if conv_state is None else conv_state[n:n + 1]
                xc[:, s:e] = _conv_silu(x[:, s:e], conv_w, h, act_round)
        bounds = cu
    q, k, v = split_mixed_qkv(xc, Hk, dk, Hv, dv)
    g, beta = gates(a, b, A_log, dt_bias, act_round)
    o, S = chunk_gated_delta_rule(q, k, v, g, beta, chunk_size, initial_state=initial_state,
                                  output_final_state=True, cu_seqlens=cu_seqlens,
                                  act_round=act_round, dtype=dtype)
    out = gated_rmsnorm(o.reshape(-1, dv), np.asarray(z).reshape(-1, dv), norm_w, eps,
                        act_round).reshape(B, T, Hv * dv)
    # conv state after the prefill: the last K-1 raw inputs of each sequence (HF
    # update_conv_state keeps the tail of [history | x]).
    if bounds is None:
        hist = (np.zeros((B, Cd, K - 1)) if conv_state is None
                else np.asarray(conv_state, dtype=np.float64))
        full = np.concatenate([hist, x.transpose(0, 2, 1)], axis=2)
        conv_out = full[:, :, -(K - 1):]
    else:
        N = len(bounds) - 1
        conv_out = np.zeros((N, Cd, K - 1))
        for n in range(N):
            s, e = int(bounds[n]), int(bounds[n + 1])
            hist = (np.zeros((Cd, K - 1)) if conv_state is None
                    else np.asarray(conv_state[n], dtype=np.float64))
            full = np.concatenate([hist, x[0, s:e].T], axis=1)
            conv_out[n] = full[:, -(K - 1):]
    return out, S, conv_out


def gdn_decode_step(mixed_qkv, z, a, b, conv_w, A_log, dt_bias, norm_w, conv_state, state, *,
                    Hk, dk, Hv, dv, eps=1e-6, act_round=round_bf16):
    """One cached decode step for one token per sequence.

    The reference has no Qwen3.5 decode (model.py:324-326; text/api.py:128-131); this
    follows HF: conv-state update (causal_conv1d_update), recurrent step
    (torch_recurrent_gated_delta_rule with qk L2-norm in the kernel), then the
    reference's fp32 gated norm (deltanet.py:282-293).
    mixed_qkv [B,conv_dim], z [B,Hv,dv], a/b [B,Hv], conv_state [B,conv_dim,K-1],
    state [B,Hv,dk,dv].  Returns (out [B,Hv*dv], new conv_state, new state).
    """
    x = np.asarray(mixed_qkv, dtype=np.float64)[:, None, :]    # [B,1,C]
    xc = _conv_silu(x, conv_w, conv_state, act_round)
    new_conv = np.concatenate([np.asarray(conv_state, np.float64),
                               x.transpose(0, 2, 1)], axis=2)[:, :, 1:]
    q, k, v = split_mixed_qkv(xc, Hk, dk, Hv, dv)
    g, beta = gates(np.asarray(a)[:, None], np.asarray(b)[:, None], A_log, dt_bias, act_round)
    o, S = recurrent_gated_delta_rule(q, k, v, g, beta, initial_state=state, act_round=act_round)
    B = x.shape[0]
    out = gated_rmsnorm(o.reshape(-1, dv), np.asarray(z).reshape(-1, dv), norm_w, eps,
                        act_round).reshape(B, Hv * dv)
    return out, new_conv, S
