"""NumPy restatement of the VJP of omegalax's chunked gated delta rule (test oracle).

TEST INFRASTRUCTURE ONLY: imported by ``tests/``; never by the product package.

The reference trains through ``chunk_gated_delta_rule`` (deltanet.py:53-153) with
JAX reverse-mode autodiff (trainers/vlm.py:157-195 call ``value_and_grad``).  Its
VJP is therefore the exact derivative of that function.  This module writes the
reverse pass out by hand, in fp64, following the forward's steps in reverse
(the line numbers cite the forward step each part differentiates):

  forward per chunk (G = in-chunk cumsum of g, Gamma_il = e^{G_i - G_l}, i >= l):
    Lg = strict_lower(K K^T * Gamma)            L = diag(beta) Lg       (:100-108)
    X  = (I + L)^-1                                                     (:110-113)
    U  = X diag(beta) V,  W = X diag(beta e^G) K                        (:115-116)
    P  = lower(Qs K^T * Gamma)   (Qs = scale * q)                       (:130-131)
    V_new = U - W S                                                     (:133-134)
    O  = diag(e^G) Qs S + P V_new                                       (:136-137)
    S' = e^{G_last} S + K^T diag(e^{G_last - G}) V_new                  (:139-142)

  reverse (dS' = gradient of the state after the chunk; the scan runs backwards):
    dV_new = P^T dO + diag(e^{G_last-G}) K dS'
    dS     = e^{G_last} dS' + Qs^T diag(e^G) dO - W^T dV_new
  and per chunk, with S and dS' known, the gradients of q, k, v, g, beta (below).

Pinning (tests/test_vjp_oracle.py): central finite differences of the pinned
forward ``gdn_oracle.chunk_gated_delta_rule`` in every input (fp64, random
directions); torch autograd (CPU, fp64) of the token-by-token recurrence, an
independent formulation; chunk-size independence; closed forms (T = 1).
"""
from __future__ import annotations

import numpy as np

from . import gdn_oracle as O
from .gdn_oracle import _gqa_expand, _ident

__all__ = ["chunk_gated_delta_rule_bwd", "chunk_bwd_core", "gdn_prefill_layer_bwd"]


def _l2norm_fwd(x, eps, act_round):
    """(rounded normalised x, unrounded normalised x, 1/norm) -- deltanet.py:30-32."""
    x = np.asarray(x, np.float64)
    r = 1.0 / np.sqrt((x * x).sum(-1, keepdims=True) + eps)
    y = x * r
    return act_round(y), y, r


def _l2norm_bwd(dy, y, r):
    """VJP of y = x * rsqrt(sum x^2 + eps): dx = r (dy - y (y . dy)).

    The bf16 rounding of the normalised value (the reference computes _l2norm in
    the input dtype) is differentiated as the identity, as autodiff does for a
    dtype conversion.
    """
    return r * (dy - y * (y * dy).sum(-1, keepdims=True))


def chunk_bwd_core(q, k, v, g, beta, dO, C, S0, dST, keep=False):
    """Reverse pass of one batch of sequences, BH-major fp64 arrays.

    q, k [B,H,T,A] (normalised, unscaled); v, dO [B,H,T,U]; g, beta [B,H,T];
    S0, dST [B,H,A,U].  Returns dq, dk (of the normalised q, k), dv, dg, dbeta and
    dS0; with ``keep`` also a dict of the per-chunk intermediates.
    """
    B, H, T, A = k.shape
    U = v.shape[-1]
    pad = (C - T % C) % C                                       # :75-82
    if pad:
        q, k, v, dO = (np.pad(x, ((0, 0), (0, 0), (0, pad), (0, 0))) for x in (q, k, v, dO))
        beta, g = (np.pad(x, ((0, 0), (0, 0), (0, pad))) for x in (beta, g))
    Tt = T + pad
    J = Tt // C
    scale = A ** -0.5
    sh = lambda x: x.reshape(B, H, J, C, x.shape[-1])
    qs, kc, vc, dOc = sh(q * scale), sh(k), sh(v), sh(dO)
    bc = beta.reshape(B, H, J, C)
    G = np.cumsum(g.reshape(B, H, J, C), axis=-1)               # :96-98
    tril = np.tril(np.ones((C, C)))
    stril = np.tril(np.ones((C, C)), -1)
    Gam = np.exp((G[..., :, None] - G[..., None, :]) * tril) * tril   # :100-104
    eG = np.exp(G)
    Gl = G[..., -1]
    kT = np.swapaxes(kc, -1, -2)
    Lg = (kc @ kT) * Gam * stril                                # :107-108 without beta
    L = bc[..., :, None] * Lg
    X = np.linalg.inv(np.eye(C) + L)                            # :110-113
    Uc = X @ (bc[..., None] * vc)                               # :115
    W = X @ ((bc * eG)[..., None] * kc)                         # :116
    P = (qs @ kT) * Gam                                         # :130-131 (lower incl. diagonal)
    kdec = kc * np.exp(Gl[..., None] - G)[..., None]            # :140-141

    # forward state recompute: S_j is the state entering chunk j
    S = np.zeros((B, H, J, A, U))
    Vn = np.zeros((B, H, J, C, U))
    s = S0.copy()
    for j in range(J):
        S[:, :, j] = s
        Vn[:, :, j] = Uc[:, :, j] - W[:, :, j] @ s              # :133-134
        s = s * np.exp(Gl[:, :, j])[..., None, None] + np.swapaxes(kdec[:, :, j], -1, -2) @ Vn[:, :, j]

    # reverse state-gradient scan: dSe_j is the gradient of the state leaving chunk j
    dSe = np.zeros((B, H, J, A, U))
    dVn = np.zeros((B, H, J, C, U))
    ds = dST.copy()
    for j in reversed(range(J)):
        dSe[:, :, j] = ds
        dVn[:, :, j] = np.swapaxes(P[:, :, j], -1, -2) @ dOc[:, :, j] + kdec[:, :, j] @ ds
        ds = (ds * np.exp(Gl[:, :, j])[..., None, None]
              + np.swapaxes(qs[:, :, j] * eG[:, :, j][..., None], -1, -2) @ dOc[:, :, j]
              - np.swapaxes(W[:, :, j], -1, -2) @ dVn[:, :, j])
    dS0 = ds

    # chunk-local gradients (all chunks at once)
    St = np.swapaxes(S, -1, -2)
    dSeT = np.swapaxes(dSe, -1, -2)
    dG = np.zeros((B, H, J, C))
    # O = diag(e^G) Qs S: dQs, dG
    X1 = (eG[..., None] * dOc) @ St                              # (e^G dO) S^T   [C, A]
    dqs = X1.copy()
    dG += (qs * X1).sum(-1)
    # O += P V_new: dP (masked to P's support)
    dP = (dOc @ np.swapaxes(Vn, -1, -2)) * tril
    dPg = dP * Gam
    dqs += dPg @ kc
    dk = np.swapaxes(dPg, -1, -2) @ qs
    PdP = dP * P
    dG += PdP.sum(-1) - PdP.sum(-2)
    # S' = e^{G_last} S + kdec^T V_new
    dkdec = Vn @ dSeT                                            # [C, A]
    dk += dkdec * np.exp(Gl[..., None] - G)[..., None]
    r = (dkdec * kdec).sum(-1)
    dG -= r
    dG[..., -1] += r.sum(-1) + np.exp(Gl) * (dSe * S).sum((-1, -2))
    # V_new = U - W S
    dU = dVn
    dW = -(dVn @ St)
    # U = X diag(beta) V, W = X diag(beta e^G) K
    vb = bc[..., None] * vc
    kbe = (bc * eG)[..., None] * kc
    dX = dU @ np.swapaxes(vb, -1, -2) + dW @ np.swapaxes(kbe, -1, -2)
    XT = np.swapaxes(X, -1, -2)
    dvb = XT @ dU
    dkbe = XT @ dW
    dv = bc[..., None] * dvb
    dbeta = (vc * dvb).sum(-1)
    t = (kc * dkbe).sum(-1) * eG
    dbeta += t
    dG += bc * t
    dk += (bc * eG)[..., None] * dkbe
    # X = (I + L)^-1: dL = strict_lower(-X^T dX X^T)
    dL = -(XT @ dX @ XT) * stril
    # L = diag(beta) (K K^T * Gamma), strictly lower
    dLg = dL * Gam
    Qm = bc[..., :, None] * dLg
    dk += (Qm + np.swapaxes(Qm, -1, -2)) @ kc
    dbeta += (dL * Lg).sum(-1)
    LdL = dL * L
    dG += LdL.sum(-1) - LdL.sum(-2)
    # G = cumsum(g): dg_t = sum_{i >= t} dG_i
    dg = np.flip(np.cumsum(np.flip(dG, -1), -1), -1)

    un = lambda x: x.reshape(B, H, Tt, x.shape[-1])[:, :, :T]
    dq_n = un(dqs) * scale
    dk_n = un(dk)
    dv_ = un(dv)
    dg_ = dg.reshape(B, H, Tt)[:, :, :T]
    db_ = dbeta.reshape(B, H, Tt)[:, :, :T]
    out = (dq_n, dk_n, dv_, dg_, db_, dS0)
    if keep:
        return out + (dict(G=G, X=X, U=Uc, W=W, P=P, Lg=Lg, S=S, V_new=Vn, dS_end=dSe,
                           dV_new=dVn),)
    return out


def chunk_gated_delta_rule_bwd(q_BTHA, k_BTHA, v_BTHU, g_BTH, beta_BTH, do_BTHU, chunk_size=64, *,
                               initial_state=None, dht=None, cu_seqlens=None, act_round=_ident,
                               eps=1e-6, keep=False):
    """VJP of ``gdn_oracle.chunk_gated_delta_rule`` (deltanet.py:53-153 plus the HF
    extensions) at its inputs, for the cotangent ``do_BTHU`` of o and ``dht`` of the
    final state.

    q/k may carry fewer heads than v; their gradients are summed over each key
    head's value heads, the adjoint of the repeat-interleave at deltanet.py:272-280.
    Returns (dq [B,T,Hk,A], dk [B,T,Hk,A], dv [B,T,H,U], dg [B,T,H], dbeta [B,T,H],
    dh0 [B or N,H,A,U]) in fp64.
    """
    H = v_BTHU.shape[2]
    Hk = q_BTHA.shape[2]
    qr, qu, rq = _l2norm_fwd(q_BTHA, eps, act_round)
    kr, ku, rk = _l2norm_fwd(k_BTHA, eps, act_round)
    tr = lambda x: np.asarray(x, np.float64).transpose(0, 2, 1, 3)
    q = tr(_gqa_expand(qr, H))
    k = tr(_gqa_expand(kr, H))
    v = tr(v_BTHU)
    dO = tr(do_BTHU)
    beta = np.asarray(beta_BTH, np.float64).transpose(0, 2, 1)
    g = np.asarray(g_BTH, np.float64).transpose(0, 2, 1)
    B, _, T, A = k.shape
    U = v.shape[-1]
    keeps = []

    def run(sl, s0, dst):
        res = chunk_bwd_core(q[:, :, sl], k[:, :, sl], v[:, :, sl], g[:, :, sl], beta[:, :, sl],
                             dO[:, :, sl], chunk_size, s0, dst, keep=keep)
        if keep:
            keeps.append(res[-1])
        return res[:6]

    if cu_seqlens is None:
        S0 = np.zeros((B, H, A, U)) if initial_state is None else np.asarray(initial_state, np.float64)
        dST = np.zeros((B, H, A, U)) if dht is None else np.asarray(dht, np.float64)
        dq, dk, dv, dg, db, dh0 = run(slice(0, T), S0, dST)
    else:
        if B != 1:
            raise ValueError("cu_seqlens requires batch size 1")
        cu = np.asarray(cu_seqlens, np.int64)
        N = len(cu) - 1
        dq = np.zeros((1, H, T, A))
        dk = np.zeros((1, H, T, A))
        dv = np.zeros((1, H, T, U))
        dg = np.zeros((1, H, T))
        db = np.zeros((1, H, T))
        dh0 = np.zeros((N, H, A, U))
        for n in range(N):
            s, e = int(cu[n]), int(cu[n + 1])
            s0 = (np.zeros((1, H, A, U)) if initial_state is None
                  else np.asarray(initial_state[n:n + 1], np.float64))
            dst = np.zeros((1, H, A, U)) if dht is None else np.asarray(dht[n:n + 1], np.float64)
            if e == s:
                dh0[n] = dst[0]
                continue
            sl = slice(s, e)
            r = run(sl, s0, dst)
            dq[:, :, sl], dk[:, :, sl], dv[:, :, sl], dg[:, :, sl], db[:, :, sl] = r[:5]
            dh0[n] = r[5][0]
    back = lambda x: x.transpose(0, 2, 1, 3)
    dqn = back(dq)      # [B, T, H, A], gradient of the normalised (expanded) q
    dkn = back(dk)
    if H != Hk:
        dqn = dqn.reshape(B, T, Hk, H // Hk, A).sum(3)
        dkn = dkn.reshape(B, T, Hk, H // Hk, A).sum(3)
    dq_in = _l2norm_bwd(dqn, qu, rq)
    dk_in = _l2norm_bwd(dkn, ku, rk)
    out = (dq_in, dk_in, back(dv), dg.transpose(0, 2, 1), db.transpose(0, 2, 1), dh0)
    if keep:
        return out + (keeps,)
    return out


# ----------------------------------------------------------------------------- layer VJP

def _silu_grad(u):
    s = 1.0 / (1.0 + np.exp(-u))
    return s * (1.0 + u * (1.0 - s))


def gdn_prefill_layer_bwd(mixed_qkv, z, a, b, conv_w, A_log, dt_bias, norm_w, dout, *, Hk, dk, Hv,
                          dv, eps=1e-6, chunk_size=64, cu_seqlens=None, initial_state=None,
                          d_final_state=None, act_round=_ident):
    """VJP of ``gdn_oracle.gdn_prefill_layer`` (deltanet.py:243-293 between the projections
    and out_proj) for the cotangent ``dout`` [B,T,Hv*dv] of its output and ``d_final_state``
    of the final state.  Dtype casts are differentiated as the identity, as autodiff does.

    Steps, in reverse of the forward:
      gated RMSNorm (deltanet.py:282-293): n = o r, r = (mean(o^2) + eps)^-1/2,
        out = w n silu(z): dn = dout w silu(z), dz = dout w n silu'(z),
        dw = sum dout n silu(z), do = r (dn - n mean(dn n));
      the chunked rule (:261-281): ``chunk_gated_delta_rule_bwd``;
      gates (:248-250): beta = sigmoid(b) -> db = dbeta beta (1 - beta);
        g = A softplus(a + dt_bias), A = -exp(A_log) -> da = dg A sigmoid(a + dt_bias),
        d dt_bias = sum da, dA_log = sum dg g;
      conv + SiLU (:35-50, 243): y = silu(u), u = sum_k w[c,k] x[t-K+1+k] ->
        du = dy silu'(u), dx[s] = sum_k w[c,k] du[s+K-1-k], dw[c,k] = sum_t du[t] x[t-K+1+k],
        each sequence on its own (zero history).
    Returns (d_mixed_qkv, dz, da, db, d_conv_w, dA_log, d_dt_bias, d_norm_w, d_initial_state).
    """
    x = np.asarray(mixed_qkv, np.float64)
    B, T, Cd = x.shape
    w = act_round(np.asarray(conv_w, np.float32)).astype(np.float64)  # as the forward (:243)
    K = w.shape[1]
    seqs = ([(bb, 0, T) for bb in range(B)] if cu_seqlens is None else
            [(0, int(s), int(e)) for s, e in zip(cu_seqlens[:-1], cu_seqlens[1:])])
    # forward: conv pre-activation u and the rule's inputs
    u = np.zeros_like(x)
    for bb, s, e in seqs:
        if e > s:
            u[bb:bb + 1, s:e] = O.causal_depthwise_conv1d(x[bb:bb + 1, s:e], w)
    u = act_round(u)
    y = act_round(O.silu(u))
    q, k, v = O.split_mixed_qkv(y, Hk, dk, Hv, dv)
    g, beta = O.gates(a, b, A_log, dt_bias, act_round)
    o, _ = O.chunk_gated_delta_rule(q, k, v, g, beta, chunk_size, initial_state=initial_state,
                                    output_final_state=True, cu_seqlens=cu_seqlens,
                                    act_round=act_round)
    # gated RMSNorm
    o2 = o.reshape(-1, dv)
    z2 = np.asarray(z, np.float64).reshape(-1, dv)
    wn = np.asarray(norm_w, np.float64)
    d2 = np.asarray(dout, np.float64).reshape(-1, dv)
    r = 1.0 / np.sqrt(np.mean(o2 * o2, axis=-1, keepdims=True) + eps)
    n = o2 * r
    sz = O.silu(z2)
    dn = d2 * wn * sz
    dz = (d2 * wn * n * _silu_grad(z2)).reshape(np.shape(z))
    dnw = (d2 * n * sz).sum(0)
    do = r * (dn - n * np.mean(dn * n, axis=-1, keepdims=True))
    # the chunked rule
    dq, dk_, dv_, dg, dbeta, dh0 = chunk_gated_delta_rule_bwd(
        q, k, v, g, beta, do.reshape(B, T, Hv, dv), chunk_size, initial_state=initial_state,
        dht=d_final_state, cu_seqlens=cu_seqlens, act_round=act_round)
    # gates
    a64 = np.asarray(a, np.float64)
    b64 = np.asarray(b, np.float64)
    sb = O.sigmoid(b64)
    db = dbeta * sb * (1.0 - sb)
    A = -np.exp(np.asarray(A_log, np.float64))
    da = dg * A * O.sigmoid(a64 + np.asarray(dt_bias, np.float64))
    d_dt_bias = da.sum((0, 1))
    dA_log = (dg * g).sum((0, 1))
    # conv + SiLU
    dy = np.concatenate([dq.reshape(B, T, -1), dk_.reshape(B, T, -1), dv_.reshape(B, T, -1)], -1)
    du = dy * _silu_grad(u)
    dx = np.zeros_like(x)
    dw = np.zeros_like(w)
    for bb, s, e in seqs:
        L = e - s
        if L <= 0:
            continue
        xs, dus = x[bb, s:e], du[bb, s:e]
        xp = np.concatenate([np.zeros((K - 1, Cd)), xs], 0)      # x[t - K + 1 + k] = xp[t + k]
        for kk in range(K):
            dw[:, kk] += (dus * xp[kk:kk + L]).sum(0)
            # u[t] += w[k] x[t - K + 1 + k]: x[s'] feeds u[s' + K - 1 - k]
            sh = K - 1 - kk
            if sh < L:
                dx[bb, s:e - sh] += w[:, kk] * dus[sh:]
    return dx, dz, da, db, dw, dA_log, d_dt_bias, dnw, dh0
