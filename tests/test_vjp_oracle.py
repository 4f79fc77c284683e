"""Pins for the VJP oracle (oracle/gdn_vjp.py), all on the CPU.

* central finite differences of the pinned forward oracle, every input, random
  directions (a dropped term, a wrong sign or a transposed product in the hand-written
  reverse pass moves the directional derivative far beyond the fp64 difference error);
* torch autograd (CPU, fp64) through the token-by-token recurrence, a formulation that
  shares no code and no algebra with the chunked reverse pass;
* chunk-size independence of the gradients, varlen == per-sequence, and the T = 1
  closed form.
"""
import numpy as np
import pytest

from oracle import gdn_oracle as O
from oracle import gdn_vjp as V


def rel(a, b):
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    return float(np.max(np.abs(a - b)) / max(np.max(np.abs(b)), 1e-30))


def case(seed, B=1, T=11, Hk=1, H=2, dk=4, dv=3):
    rng = np.random.default_rng(seed)
    return dict(
        q=rng.standard_normal((B, T, Hk, dk)), k=rng.standard_normal((B, T, Hk, dk)),
        v=rng.standard_normal((B, T, H, dv)), g=-rng.uniform(0.05, 0.6, (B, T, H)),
        beta=rng.uniform(0.1, 0.95, (B, T, H)), S0=0.5 * rng.standard_normal((B, H, dk, dv)),
        do=rng.standard_normal((B, T, H, dv)), dht=rng.standard_normal((B, H, dk, dv)))


def loss(c, C, **over):
    x = {**c, **over}
    o, S = O.chunk_gated_delta_rule(x["q"], x["k"], x["v"], x["g"], x["beta"], C,
                                    initial_state=x["S0"], output_final_state=True)
    return float((o * c["do"]).sum() + (S * c["dht"]).sum())


@pytest.mark.parametrize("C", [4, 64])
@pytest.mark.parametrize("seed", [0, 1])
def test_vjp_oracle_matches_finite_differences(C, seed):
    c = case(seed)
    dq, dk, dv, dg, db, dh0 = V.chunk_gated_delta_rule_bwd(
        c["q"], c["k"], c["v"], c["g"], c["beta"], c["do"], C, initial_state=c["S0"], dht=c["dht"])
    grads = dict(q=dq, k=dk, v=dv, g=dg, beta=db, S0=dh0)
    rng = np.random.default_rng(100 + seed)
    eps = 1e-5
    for name, grad in grads.items():
        for _ in range(2):
            d = rng.standard_normal(c[name].shape)
            fd = (loss(c, C, **{name: c[name] + eps * d}) - loss(c, C, **{name: c[name] - eps * d})) / (2 * eps)
            an = float((grad * d).sum())
            assert abs(fd - an) <= 1e-7 * max(1.0, abs(fd)), (name, fd, an)


def _torch_recurrent_grads(c):
    torch = pytest.importorskip("torch")
    t = {n: torch.tensor(c[n], dtype=torch.float64, requires_grad=True)
         for n in ("q", "k", "v", "g", "beta", "S0")}
    H = c["v"].shape[2]
    Hk = c["q"].shape[2]
    rep = lambda x: x.repeat_interleave(H // Hk, dim=2)
    nq = rep(t["q"] / torch.sqrt((t["q"] ** 2).sum(-1, keepdim=True) + 1e-6))
    nk = rep(t["k"] / torch.sqrt((t["k"] ** 2).sum(-1, keepdim=True) + 1e-6))
    A = nq.shape[-1]
    S = t["S0"]
    outs = []
    for i in range(nq.shape[1]):
        S = S * torch.exp(t["g"][:, i])[..., None, None]
        kv = torch.einsum("bhau,bha->bhu", S, nk[:, i])
        delta = (t["v"][:, i] - kv) * t["beta"][:, i][..., None]
        S = S + nk[:, i][..., :, None] * delta[..., None, :]
        outs.append(torch.einsum("bhau,bha->bhu", S, nq[:, i] * A ** -0.5))
    o = torch.stack(outs, 1)
    L = (o * torch.tensor(c["do"])).sum() + (S * torch.tensor(c["dht"])).sum()
    L.backward()
    return {n: t[n].grad.numpy() for n in t}


@pytest.mark.parametrize("seed", [2, 3])
def test_vjp_oracle_matches_autograd_of_the_token_recurrence(seed):
    c = case(seed, B=2, T=70, Hk=2, H=4, dk=8, dv=5)
    ref = _torch_recurrent_grads(c)
    got = V.chunk_gated_delta_rule_bwd(c["q"], c["k"], c["v"], c["g"], c["beta"], c["do"], 16,
                                       initial_state=c["S0"], dht=c["dht"])
    for name, g in zip(("q", "k", "v", "g", "beta", "S0"), got):
        assert rel(g, ref[name]) < 1e-10, name


def test_vjp_oracle_chunk_size_independent():
    c = case(4, T=50, dk=6, dv=6)
    a = V.chunk_gated_delta_rule_bwd(c["q"], c["k"], c["v"], c["g"], c["beta"], c["do"], 8,
                                     initial_state=c["S0"], dht=c["dht"])
    b = V.chunk_gated_delta_rule_bwd(c["q"], c["k"], c["v"], c["g"], c["beta"], c["do"], 64,
                                     initial_state=c["S0"], dht=c["dht"])
    for x, y in zip(a, b):
        assert rel(x, y) < 1e-11


def test_vjp_oracle_varlen_equals_per_sequence():
    c = case(5, T=40)
    cu = [0, 13, 13, 40]
    S0 = np.concatenate([c["S0"]] * 3)
    dht = np.random.default_rng(9).standard_normal(S0.shape)
    got = V.chunk_gated_delta_rule_bwd(c["q"], c["k"], c["v"], c["g"], c["beta"], c["do"], 8,
                                       initial_state=S0, dht=dht, cu_seqlens=cu)
    for n in range(3):
        s, e = cu[n], cu[n + 1]
        if e == s:
            assert np.array_equal(got[5][n], dht[n])  # empty sequence: the state passes through
            continue
        sl = slice(s, e)
        one = V.chunk_gated_delta_rule_bwd(c["q"][:, sl], c["k"][:, sl], c["v"][:, sl], c["g"][:, sl],
                                           c["beta"][:, sl], c["do"][:, sl], 8,
                                           initial_state=S0[n:n + 1], dht=dht[n:n + 1])
        for x, y in zip(got[:5], one[:5]):
            assert rel(x[:, sl], y) < 1e-12
        assert rel(got[5][n], one[5][0]) < 1e-12


def test_vjp_oracle_single_token_closed_form():
    # T = 1, S0 = 0: o = beta (q.k) v * scale with unit q, k, so do -> dv = beta (q.k) scale do
    c = case(6, T=1, H=1, dk=4, dv=3)
    qn = c["q"] / np.sqrt((c["q"] ** 2).sum(-1, keepdims=True) + 1e-6)
    kn = c["k"] / np.sqrt((c["k"] ** 2).sum(-1, keepdims=True) + 1e-6)
    qk = float((qn * kn).sum()) * 4 ** -0.5
    got = V.chunk_gated_delta_rule_bwd(c["q"], c["k"], c["v"], c["g"], c["beta"], c["do"], 64)
    b = float(c["beta"].ravel()[0])
    assert np.allclose(got[2], b * qk * c["do"], rtol=1e-12, atol=1e-14)
    assert np.allclose(got[4].ravel(), qk * float((c["v"] * c["do"]).sum()), rtol=1e-12)
    assert np.allclose(got[3], 0.0, atol=1e-14)  # S0 = 0: the decay multiplies nothing


# ----------------------------------------------------------------------------- layer VJP

def layer_case(seed, B=1, T=13, Hk=1, dk=4, Hv=2, dv=4, K=4):
    rng = np.random.default_rng(seed)
    Cd = 2 * Hk * dk + Hv * dv
    return dict(
        x=rng.standard_normal((B, T, Cd)), z=rng.standard_normal((B, T, Hv, dv)),
        a=rng.standard_normal((B, T, Hv)), b=rng.standard_normal((B, T, Hv)),
        # conv weights with at most 10 fractional bits: the forward casts them to float32,
        # and w +- 2^-20 d with d = +-1 then stays exact there
        w=np.round(512 * rng.standard_normal((Cd, K))) / 1024, A_log=rng.uniform(-1.5, 0.5, Hv),
        dt=rng.uniform(-2, 0, Hv), nw=rng.uniform(0.5, 1.5, dv),
        S0=0.3 * rng.standard_normal((B, Hv, dk, dv)),
        dout=rng.standard_normal((B, T, Hv * dv)), dS=0.3 * rng.standard_normal((B, Hv, dk, dv)),
        dims=dict(Hk=Hk, dk=dk, Hv=Hv, dv=dv))


def layer_loss(c, C, cu=None, **over):
    x = {**c, **over}
    out, S, _ = O.gdn_prefill_layer(x["x"], x["z"], x["a"], x["b"], x["w"], x["A_log"], x["dt"],
                                    x["nw"], **c["dims"], chunk_size=C, cu_seqlens=cu,
                                    initial_state=x["S0"], act_round=lambda y: y)
    return float((out * c["dout"]).sum() + (S * c["dS"]).sum())


@pytest.mark.parametrize("C,cu", [(4, None), (64, None), (4, [0, 5, 5, 13])])
def test_layer_vjp_oracle_matches_finite_differences(C, cu):
    """Every input of the layer VJP against central differences of the pinned layer forward
    (conv_w goes through the forward's float32 cast, so its direction is +-1 with a 2^-20
    step, exact in float32)."""
    c = layer_case(3)
    if cu is not None:
        cu = np.asarray(cu)
        c["S0"] = 0.3 * np.random.default_rng(5).standard_normal((len(cu) - 1, 2, 4, 4))
        c["dS"] = 0.3 * np.random.default_rng(6).standard_normal((len(cu) - 1, 2, 4, 4))
    dx, dz, da, db, dw, dA, ddt, dnw, dh0 = V.gdn_prefill_layer_bwd(
        c["x"], c["z"], c["a"], c["b"], c["w"], c["A_log"], c["dt"], c["nw"], c["dout"],
        **c["dims"], chunk_size=C, cu_seqlens=cu, initial_state=c["S0"], d_final_state=c["dS"])
    grads = dict(x=dx, z=dz, a=da, b=db, w=dw, A_log=dA, dt=ddt, nw=dnw, S0=dh0)
    rng = np.random.default_rng(9)
    for name, grad in grads.items():
        eps, tol = (2.0 ** -20, 1e-7) if name == "w" else (1e-5, 1e-7)
        for _ in range(2):
            d = rng.standard_normal(np.shape(c[name]))
            if name == "w":
                d = np.sign(d)
            fd = (layer_loss(c, C, cu, **{name: c[name] + eps * d})
                  - layer_loss(c, C, cu, **{name: c[name] - eps * d})) / (2 * eps)
            an = float((grad * d).sum())
            assert abs(fd - an) <= tol * max(1.0, abs(fd)), (name, fd, an)
