"""Pins for the CPU oracle (oracle/gdn_oracle.py), all on the CPU.

Each check is chosen so that a plausible slip in the restatement (a dropped
decay term, a transposed product, a wrong mask diagonal, an off-by-one in the
conv window) fails at least one of them:
  * golden vectors written by transformers' torch functions (tests/golden/);
  * the textbook token-by-token recurrence vs the chunked WY/UT form;
  * closed forms (T=1, orthonormal keys, beta=0, zero inputs);
  * invariants (chunk-size independence, padding, linearity, varlen == per-sequence,
    decode-after-prefill == longer prefill, split prefill == full prefill).
"""
import os

import numpy as np
import pytest

from oracle import gdn_oracle as O

GOLD = os.path.join(os.path.dirname(__file__), "golden")


def _load(name):
    return dict(np.load(os.path.join(GOLD, name + ".npz")))


def rel(a, b):
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    return float(np.max(np.abs(a - b)) / max(np.max(np.abs(b)), 1e-30))


def _rand_case(seed, B=2, T=37, Hk=1, H=2, dk=8, dv=8, s0=True):
    rng = np.random.default_rng(seed)
    q = rng.standard_normal((B, T, Hk, dk))
    k = rng.standard_normal((B, T, Hk, dk))
    v = rng.standard_normal((B, T, H, dv))
    g = -rng.uniform(0.0, 0.5, (B, T, H))
    beta = rng.uniform(0.1, 0.9, (B, T, H))
    S0 = 0.3 * rng.standard_normal((B, H, dk, dv)) if s0 else None
    return q, k, v, g, beta, S0


# ----------------------------------------------------------------------------- golden vectors

@pytest.mark.parametrize("name", ["chunk_gqa_pad_c16", "chunk_gqa_pad_c64_s0", "chunk_d64_c64"])
def test_chunk_matches_hf_golden(name):
    d = _load(name)
    o, S = O.chunk_gated_delta_rule(d["q"], d["k"], d["v"], d["g"], d["beta"],
                                    int(d["chunk_size"]), initial_state=d.get("S0"),
                                    output_final_state=True)
    assert rel(o, d["o"]) < 2e-5
    assert rel(S, d["S"]) < 2e-5


def test_chunk_fp32_matches_hf_golden_closely():
    d = _load("chunk_gqa_pad_c64_s0")
    o, S = O.chunk_gated_delta_rule(d["q"], d["k"], d["v"], d["g"], d["beta"], 64,
                                    initial_state=d["S0"], output_final_state=True,
                                    dtype=np.float32)
    assert rel(o, d["o"]) < 1e-5 and rel(S, d["S"]) < 1e-5


def test_recurrent_matches_hf_golden():
    d = _load("recurrent_gqa_s0")
    o, S = O.recurrent_gated_delta_rule(d["q"], d["k"], d["v"], d["g"], d["beta"],
                                        initial_state=d["S0"])
    assert rel(o, d["o"]) < 1e-5
    assert rel(S, d["S"]) < 1e-5


def test_conv_matches_hf_golden():
    d = _load("conv_k4")
    x_BTC = d["x"].transpose(0, 2, 1)
    y = O.silu(O.causal_depthwise_conv1d(x_BTC, d["w"]))
    assert rel(y, d["y"].transpose(0, 2, 1)) < 1e-6
    # one cached step: history = state, new token x_step
    y1 = O.silu(O.causal_depthwise_conv1d(d["x_step"].transpose(0, 2, 1), d["w"], d["state"]))
    assert rel(y1, d["y_step"].transpose(0, 2, 1)) < 1e-6


def test_gated_norm_and_l2norm_match_hf_golden():
    d = _load("gated_norm")
    y = O.gated_rmsnorm(d["x"], d["z"], d["w"], 1e-6)
    assert rel(y, d["y"]) < 1e-6
    assert rel(O.l2norm(d["x"]), d["l2"]) < 1e-6


def test_decode_conv_state_shift_matches_hf_golden():
    d = _load("conv_k4")
    B, C, _ = d["state"].shape
    new = np.concatenate([d["state"], d["x_step"]], axis=2)[:, :, 1:]
    # gdn_decode_step's conv-state update must be the same shift HF applies in place
    Hk, dk, Hv, dv = 1, 8, 1, 8
    assert C == 2 * Hk * dk + Hv * dv
    z = np.zeros((B, Hv, dv))
    ab = np.zeros((B, Hv))
    _, new_conv, _ = O.gdn_decode_step(d["x_step"][:, :, 0], z, ab, ab, d["w"], np.zeros(Hv),
                                       np.zeros(Hv), np.ones(dv), d["state"],
                                       np.zeros((B, Hv, dk, dv)), Hk=Hk, dk=dk, Hv=Hv, dv=dv,
                                       act_round=lambda x: x)
    assert np.array_equal(new_conv, new)


# ----------------------------------------------------------------------------- closed forms

def test_round_bf16_known_values():
    x = np.array([1.0, 1.0 + 2 ** -8, 1.0 + 3 * 2 ** -8, -2.5, 3.0e38, 1e-40], np.float32)
    r = O.round_bf16(x)
    assert r[0] == 1.0
    assert r[1] == 1.0                       # tie -> even
    assert r[2] == 1.0 + 4 * 2 ** -8         # tie -> even (up)
    assert r[3] == -2.5
    assert np.isfinite(r[4])
    # bf16 keeps 7 fraction bits: 1 + 2^-7 + 2^-9 is below the half step, 1 + 2^-7 + 3*2^-9 above
    assert O.round_bf16(np.float32(1.0 + 2 ** -7 + 2 ** -9)) == np.float32(1.0 + 2 ** -7)
    assert O.round_bf16(np.float32(1.0 + 2 ** -7 + 3 * 2 ** -9)) == np.float32(1.0 + 2 ** -6)


def test_l2norm_closed_forms():
    e = np.zeros((3, 4))
    e[0, 1] = 1.0
    e[1] = [3.0, 4.0, 0.0, 0.0]
    out = O.l2norm(e)
    assert np.allclose(out[0], [0, 1 / np.sqrt(1 + 1e-6), 0, 0])
    assert np.allclose(out[1], np.array([0.6, 0.8, 0, 0]) * 5 / np.sqrt(25 + 1e-6))
    assert np.all(out[2] == 0.0)             # l2norm(0) = 0 (eps inside the sqrt)


def test_gates_closed_forms():
    g, beta = O.gates(np.zeros((1, 1, 2)), np.zeros((1, 1, 2)), np.log([1.0, 4.0]),
                      np.zeros(2))
    assert np.allclose(beta, 0.5)
    assert np.allclose(g[0, 0], [-np.log(2.0), -4 * np.log(2.0)])
    g2, beta2 = O.gates(np.full((1, 1, 1), -800.0), np.full((1, 1, 1), 800.0), np.zeros(1),
                        np.zeros(1))
    assert g2[0, 0, 0] == 0.0 or abs(g2[0, 0, 0]) < 1e-300   # softplus(-inf) -> 0: no decay
    assert beta2[0, 0, 0] == 1.0


def test_conv_brute_force_and_identity():
    rng = np.random.default_rng(3)
    x = rng.standard_normal((2, 11, 5))
    w = rng.standard_normal((5, 4))
    y = O.causal_depthwise_conv1d(x, w)
    for b in range(2):
        for c in range(5):
            # np.convolve flips the kernel: causal cross-correlation == convolve with w[::-1]
            ref = np.convolve(x[b, :, c], w[c, ::-1])[:11]
            assert np.allclose(y[b, :, c], ref)
    ident = np.zeros((5, 4))
    ident[:, 3] = 1.0
    assert np.allclose(O.causal_depthwise_conv1d(x, ident), x)
    shift = np.zeros((5, 4))
    shift[:, 2] = 1.0
    ys = O.causal_depthwise_conv1d(x, shift)
    assert np.allclose(ys[:, 1:], x[:, :-1]) and np.all(ys[:, 0] == 0)


def test_single_token_closed_form():
    """T=1: o = (q.k / sqrt(A)) * beta * (v - e^g S0^T k) + e^g S0^T q / sqrt(A)."""
    q, k, v, g, beta, S0 = _rand_case(5, B=1, T=1, Hk=2, H=2, dk=4, dv=3)
    o, S = O.chunk_gated_delta_rule(q, k, v, g, beta, 64, initial_state=S0,
                                    output_final_state=True)
    qn = q / np.linalg.norm(q, axis=-1, keepdims=True)
    kn = k / np.linalg.norm(k, axis=-1, keepdims=True)
    for h in range(2):
        a = np.exp(g[0, 0, h])
        qh, kh, S0h = qn[0, 0, h] / 2.0, kn[0, 0, h], S0[0, h]
        delta = beta[0, 0, h] * (v[0, 0, h] - a * S0h.T @ kh)
        S1 = a * S0h + np.outer(kh, delta)
        assert np.allclose(S[0, h], S1, atol=1e-6)
        assert np.allclose(o[0, 0, h], S1.T @ qh, atol=1e-6)


def test_orthonormal_keys_exact_retrieval():
    """g=0, beta=1, orthonormal keys, S0=0: S^T k_i = v_i for every stored pair."""
    dk, T = 8, 8
    rng = np.random.default_rng(7)
    Q, _ = np.linalg.qr(rng.standard_normal((dk, dk)))
    k = Q.T[None, :, None, :] * 5.0          # scale is removed by the L2 norm
    v = rng.standard_normal((1, T, 1, 4))
    _, S = O.chunk_gated_delta_rule(k, k, v, np.zeros((1, T, 1)), np.ones((1, T, 1)), 4,
                                    output_final_state=True)
    kn = Q.T / np.sqrt(1 + 1e-6 / 25.0)
    assert np.allclose(S[0, 0].T @ Q.T.T, (v[0, :, 0] / np.sqrt(1 + 1e-6 / 25.0)).T, atol=1e-5)
    del kn


def test_beta_zero_gives_zero():
    q, k, v, g, _, _ = _rand_case(9, s0=False)
    o, S = O.chunk_gated_delta_rule(q, k, v, g, np.zeros_like(g), 16, output_final_state=True)
    assert np.all(o == 0) and np.all(S == 0)


def test_brute_force_tiny_matrix_algebra():
    """T=3, d=2: unroll the recurrence by hand with explicit 2x2 matrices."""
    rng = np.random.default_rng(13)
    q, k, v = (rng.standard_normal((1, 3, 1, 2)) for _ in range(3))
    g = -rng.uniform(0, 1, (1, 3, 1))
    beta = rng.uniform(0, 1, (1, 3, 1))
    o, S = O.chunk_gated_delta_rule(q, k, v, g, beta, 2, output_final_state=True)
    qn = q[0, :, 0] / np.sqrt((q[0, :, 0] ** 2).sum(-1, keepdims=True) + 1e-6)
    kn = k[0, :, 0] / np.sqrt((k[0, :, 0] ** 2).sum(-1, keepdims=True) + 1e-6)
    St = np.zeros((2, 2))
    for t in range(3):
        a, b_ = np.exp(g[0, t, 0]), beta[0, t, 0]
        # S_t = a (I - b k k^T) S_{t-1} + b k v^T
        St = a * (np.eye(2) - b_ * np.outer(kn[t], kn[t])) @ St + b_ * np.outer(kn[t], v[0, t, 0])
        assert np.allclose(o[0, t, 0], St.T @ (qn[t] / np.sqrt(2.0)), atol=1e-10)
    assert np.allclose(S[0, 0], St, atol=1e-10)


# ----------------------------------------------------------------------------- invariants

@pytest.mark.parametrize("C", [1, 4, 16, 64])
def test_chunked_equals_recurrence(C):
    q, k, v, g, beta, S0 = _rand_case(1, T=37, Hk=1, H=2)
    o, S = O.chunk_gated_delta_rule(q, k, v, g, beta, C, initial_state=S0,
                                    output_final_state=True)
    o2, S2 = O.recurrent_gated_delta_rule(q, k, v, g, beta, initial_state=S0)
    assert rel(o, o2) < 1e-11 and rel(S, S2) < 1e-11


def test_linearity_in_v_and_state():
    q, k, v, g, beta, S0 = _rand_case(2)
    rng = np.random.default_rng(22)
    v2 = rng.standard_normal(v.shape)
    S02 = rng.standard_normal(S0.shape)
    f = lambda vv, ss: O.chunk_gated_delta_rule(q, k, vv, g, beta, 16, initial_state=ss,
                                                output_final_state=True)
    oa, Sa = f(v, S0)
    ob, Sb = f(v2, S02)
    oc, Sc = f(2.0 * v - 3.0 * v2, 2.0 * S0 - 3.0 * S02)
    assert rel(oc, 2 * oa - 3 * ob) < 1e-12 and rel(Sc, 2 * Sa - 3 * Sb) < 1e-12


def test_padding_does_not_change_state():
    q, k, v, g, beta, S0 = _rand_case(3, T=40)
    o1, S1 = O.chunk_gated_delta_rule(q, k, v, g, beta, 64, initial_state=S0,
                                      output_final_state=True)
    o2, S2 = O.chunk_gated_delta_rule(q, k, v, g, beta, 8, initial_state=S0,
                                      output_final_state=True)
    assert rel(o1, o2) < 1e-12 and rel(S1, S2) < 1e-12


def test_varlen_equals_per_sequence():
    rng = np.random.default_rng(4)
    lens = [5, 0, 33, 17, 64]
    cu = np.concatenate([[0], np.cumsum(lens)]).astype(np.int32)
    T = int(cu[-1])
    q, k, v, g, beta, _ = _rand_case(4, B=1, T=T)
    S0 = rng.standard_normal((len(lens), 2, 8, 8))
    o, S = O.chunk_gated_delta_rule(q, k, v, g, beta, 16, initial_state=S0,
                                    output_final_state=True, cu_seqlens=cu)
    for n in range(len(lens)):
        s, e = cu[n], cu[n + 1]
        on, Sn = O.recurrent_gated_delta_rule(q[:, s:e], k[:, s:e], v[:, s:e], g[:, s:e],
                                              beta[:, s:e], initial_state=S0[n:n + 1])
        assert rel(S[n], Sn[0]) < 1e-11
        if e > s:
            assert rel(o[:, s:e], on) < 1e-11


def _layer_case(seed, B, T, Hk=2, dk=8, Hv=4, dv=8, K=4):
    rng = np.random.default_rng(seed)
    Cd = 2 * Hk * dk + Hv * dv
    bf = O.round_bf16
    return dict(
        mixed_qkv=bf(rng.standard_normal((B, T, Cd))), z=bf(rng.standard_normal((B, T, Hv, dv))),
        a=bf(rng.standard_normal((B, T, Hv))), b=bf(rng.standard_normal((B, T, Hv))),
        conv_w=(0.3 * rng.standard_normal((Cd, K))).astype(np.float32),
        A_log=rng.uniform(0, np.log(16), Hv), dt_bias=rng.uniform(-2, 0, Hv),
        norm_w=1 + 0.1 * rng.standard_normal(dv)), dict(Hk=Hk, dk=dk, Hv=Hv, dv=dv)


def test_decode_after_prefill_equals_longer_prefill():
    d, dims = _layer_case(6, B=2, T=21)
    full, S_full, conv_full = O.gdn_prefill_layer(**d, **dims, chunk_size=8)
    n = 17
    part = {k_: (v_[:, :n] if k_ in ("mixed_qkv", "z", "a", "b") else v_) for k_, v_ in d.items()}
    _, S, conv = O.gdn_prefill_layer(**part, **dims, chunk_size=8)
    for t in range(n, 21):
        out, conv, S = O.gdn_decode_step(d["mixed_qkv"][:, t], d["z"][:, t], d["a"][:, t],
                                         d["b"][:, t], d["conv_w"], d["A_log"], d["dt_bias"],
                                         d["norm_w"], conv, S, **dims)
        assert rel(out, full[:, t]) < 1e-6
    assert rel(S, S_full) < 1e-11
    assert np.array_equal(conv, conv_full)


def test_split_prefill_with_carried_states_equals_full():
    d, dims = _layer_case(8, B=1, T=50)
    full, S_full, conv_full = O.gdn_prefill_layer(**d, **dims, chunk_size=16)
    cut = 23
    p1 = {k_: (v_[:, :cut] if k_ in ("mixed_qkv", "z", "a", "b") else v_) for k_, v_ in d.items()}
    p2 = {k_: (v_[:, cut:] if k_ in ("mixed_qkv", "z", "a", "b") else v_) for k_, v_ in d.items()}
    o1, S1, c1 = O.gdn_prefill_layer(**p1, **dims, chunk_size=16)
    o2, S2, c2 = O.gdn_prefill_layer(**p2, **dims, chunk_size=16, initial_state=S1,
                                     conv_state=c1)
    assert rel(np.concatenate([o1, o2], axis=1), full) < 1e-6
    assert rel(S2, S_full) < 1e-11 and np.array_equal(c2, conv_full)


def test_layer_varlen_equals_per_sequence():
    d, dims = _layer_case(10, B=1, T=45)
    cu = np.array([0, 7, 7, 30, 45], np.int32)
    N = len(cu) - 1
    rng = np.random.default_rng(1)
    S0 = rng.standard_normal((N, dims["Hv"], dims["dk"], dims["dv"]))
    Cd = d["mixed_qkv"].shape[-1]
    c0 = O.round_bf16(rng.standard_normal((N, Cd, 3)))
    out, S, conv = O.gdn_prefill_layer(**d, **dims, chunk_size=16, cu_seqlens=cu,
                                       initial_state=S0, conv_state=c0)
    for n in range(N):
        s, e = cu[n], cu[n + 1]
        p = {k_: (v_[:, s:e] if k_ in ("mixed_qkv", "z", "a", "b") else v_)
             for k_, v_ in d.items()}
        if e == s:
            assert np.array_equal(S[n], S0[n]) and np.array_equal(conv[n], c0[n])
            continue
        on, Sn, cn = O.gdn_prefill_layer(**p, **dims, chunk_size=16,
                                         initial_state=S0[n:n + 1], conv_state=c0[n:n + 1])
        assert rel(out[:, s:e], on) < 1e-7 and rel(S[n], Sn[0]) < 1e-11
        assert np.array_equal(conv[n], cn[0])
