"""Pins the oracle's layer composition (gdn_prefill_layer, gdn_decode_step) against
transformers' Qwen3_5GatedDeltaNet module run in float32 (fixtures from
tests/golden/make_golden.py).

In float32 the HF module computes what GatedDeltaNet.__call__ computes
(deltanet.py:226-306): mask, the four projections, conv + SiLU, the gates, the
q|k|v split with GQA repeat-interleave, the chunked rule and the gated RMSNorm,
then out_proj.  A wiring slip in the oracle -- a and b swapped, q and k swapped,
a z row paired with the wrong head, the wrong GQA mapping -- moves the output far
beyond the 1e-5 bound here (checked by the planted-mistake cases below).  The
parameters are read through omegalax_amd.layer.gdn_params_from_hf, so the
checkpoint key mapping (loader.py:173-190, 285-307) is pinned by the same data.
"""
import os

import numpy as np
import pytest

from oracle import gdn_oracle as O

torch = pytest.importorskip("torch")

GOLD = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
CASES = ["layer_d128", "layer_d64", "layer_smoke_d16"]
TOL = 1e-5


def rel(a, b):
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    return float(np.max(np.abs(a - b)) / max(np.max(np.abs(b)), 1e-30))


def load(name):
    from omegalax_amd.layer import gdn_params_from_hf
    d = dict(np.load(os.path.join(GOLD, name + ".npz")))
    D, Hk, Hv, dk, dv = (int(x) for x in d["dims"])
    p = gdn_params_from_hf({k: torch.from_numpy(v) for k, v in d.items()}, 0)
    # fp64 copies of the parameters (the mapping's linear weights are bf16 for the GPU
    # path; the oracle check takes the fixture's fp32 values straight from the file)
    base = "model.language_model.layers.0.linear_attn."
    w = {k[len(base):]: v.astype(np.float64) for k, v in d.items() if k.startswith(base)}
    return d, (D, Hk, Hv, dk, dv), p, w


def oracle_layer(w, dims, hidden, mask=None, wiring=None):
    D, Hk, Hv, dk, dv = dims
    h = np.asarray(hidden, np.float64)
    if mask is not None and h.shape[1] > 1:  # deltanet.py:227-228
        h = h * mask[:, :, None]
    B, T, _ = h.shape
    mixed = h @ w["in_proj_qkv.weight"].T
    z = (h @ w["in_proj_z.weight"].T).reshape(B, T, Hv, dv)
    a = h @ w["in_proj_a.weight"].T
    b = h @ w["in_proj_b.weight"].T
    if wiring == "swap_ab":
        a, b = b, a
    out, S, conv = O.gdn_prefill_layer(mixed, z, a, b, w["conv1d.weight"][:, 0, :], w["A_log"],
                                       w["dt_bias"], w["norm.weight"], Hk=Hk, dk=dk, Hv=Hv, dv=dv,
                                       eps=1e-6, act_round=O._ident)
    return out @ w["out_proj.weight"].T, S, conv


def test_fixture_mapping_round_trip():
    """gdn_params_from_hf reads every key the HF module holds, with conv1d.weight
    [C,1,K] squeezed to [C,K] (loader.py:289) and the linear weights in [out, in]."""
    from omegalax_amd.layer import gdn_params_to_hf
    d, (D, Hk, Hv, dk, dv), p, w = load("layer_d64")
    C = 2 * Hk * dk + Hv * dv
    assert tuple(p.in_proj_qkv.shape) == (C, D) and tuple(p.conv_w.shape) == (C, 4)
    assert tuple(p.out_proj.shape) == (D, Hv * dv) and tuple(p.norm_w.shape) == (dv,)
    np.testing.assert_array_equal(p.conv_w.numpy(), w["conv1d.weight"][:, 0, :].astype(np.float32))
    np.testing.assert_array_equal(p.A_log.numpy(), w["A_log"].astype(np.float32))
    back = gdn_params_to_hf(p, 0)
    assert set(back) == {k for k in d if k.startswith("model.")}
    for k, v in back.items():
        assert tuple(v.shape) == d[k].shape, k


@pytest.mark.parametrize("name", CASES)
def test_oracle_layer_prefill_matches_hf_module(name):
    d, dims, _, w = load(name)
    out, _, _ = oracle_layer(w, dims, d["hidden"], d["mask"].astype(np.float64))
    assert rel(out, d["out"]) < TOL


@pytest.mark.parametrize("name", CASES)
def test_oracle_layer_decode_matches_hf_cache(name):
    """prefill into the cache, then single-token steps (HF DynamicCache path)."""
    d, dims, _, w = load(name)
    D, Hk, Hv, dk, dv = dims
    out0, S, conv = oracle_layer(w, dims, d["hidden_prefill"])
    assert rel(out0, d["out_prefill"]) < TOL
    for s in range(d["hidden_decode"].shape[0]):
        h = d["hidden_decode"][s].astype(np.float64)
        mixed = h @ w["in_proj_qkv.weight"].T
        z = (h @ w["in_proj_z.weight"].T).reshape(-1, Hv, dv)
        a = h @ w["in_proj_a.weight"].T
        b = h @ w["in_proj_b.weight"].T
        o, conv, S = O.gdn_decode_step(mixed, z, a, b, w["conv1d.weight"][:, 0, :], w["A_log"],
                                       w["dt_bias"], w["norm.weight"], conv, S, Hk=Hk, dk=dk,
                                       Hv=Hv, dv=dv, eps=1e-6, act_round=O._ident)
        assert rel(o @ w["out_proj.weight"].T, d["out_decode"][s]) < TOL, s
    if "state_after_decode" in d:
        assert rel(S, d["state_after_decode"]) < TOL


def test_planted_wiring_mistake_is_caught():
    """The bound is tight enough to see a plausible wiring slip (a <-> b)."""
    d, dims, _, w = load("layer_d128")
    out, _, _ = oracle_layer(w, dims, d["hidden"], d["mask"].astype(np.float64), wiring="swap_ab")
    assert rel(out, d["out"]) > 100 * TOL


def test_planted_gqa_and_z_mistakes_are_caught():
    """q/k channel order and the z row a norm row pairs with are pinned too."""
    d, (D, Hk, Hv, dk, dv), _, w = load("layer_d128")
    kd = Hk * dk
    w2 = dict(w)
    W = w["in_proj_qkv.weight"]
    w2["in_proj_qkv.weight"] = np.concatenate([W[kd:2 * kd], W[:kd], W[2 * kd:]])  # q <-> k
    c = w["conv1d.weight"]
    w2["conv1d.weight"] = np.concatenate([c[kd:2 * kd], c[:kd], c[2 * kd:]])
    out, _, _ = oracle_layer(w2, (D, Hk, Hv, dk, dv), d["hidden"], d["mask"].astype(np.float64))
    assert rel(out, d["out"]) > 100 * TOL
    w3 = dict(w)
    Z = w["in_proj_z.weight"].reshape(Hv, dv, D)
    w3["in_proj_z.weight"] = Z[::-1].reshape(Hv * dv, D)  # z head order reversed
    out, _, _ = oracle_layer(w3, (D, Hk, Hv, dk, dv), d["hidden"], d["mask"].astype(np.float64))
    assert rel(out, d["out"]) > 100 * TOL


def test_planted_gqa_mapping_mistake_is_caught():
    """Value head h reads key head h // (Hv/Hk) (repeat-interleave, deltanet.py:272-280).
    Relabelling the value heads everywhere (v channels, z, a, b, A_log, dt_bias, out_proj)
    leaves the layer unchanged except for that mapping, so with the tiled mapping
    h -> h % Hk in its place the output must move; with the identity relabelling it must
    not."""
    d, (D, Hk, Hv, dk, dv), _, w = load("layer_d128")
    gqa = Hv // Hk
    kd = Hk * dk

    def relabel(perm):
        w2 = dict(w)
        W = w["in_proj_qkv.weight"]
        Wv = W[2 * kd:].reshape(Hv, dv, D)[perm].reshape(Hv * dv, D)
        w2["in_proj_qkv.weight"] = np.concatenate([W[:2 * kd], Wv])
        c = w["conv1d.weight"]
        cv = c[2 * kd:].reshape(Hv, dv, 1, 4)[perm].reshape(Hv * dv, 1, 4)
        w2["conv1d.weight"] = np.concatenate([c[:2 * kd], cv])
        w2["in_proj_z.weight"] = w["in_proj_z.weight"].reshape(Hv, dv, D)[perm].reshape(Hv * dv, D)
        for k in ("in_proj_a.weight", "in_proj_b.weight", "A_log", "dt_bias"):
            w2[k] = w[k][perm]
        w2["out_proj.weight"] = w["out_proj.weight"].reshape(D, Hv, dv)[:, perm].reshape(D, Hv * dv)
        return oracle_layer(w2, (D, Hk, Hv, dk, dv), d["hidden"], d["mask"].astype(np.float64))[0]

    assert rel(relabel(np.arange(Hv)), d["out"]) < TOL
    # value head slot s now holds original head perm[s]; the oracle gives it key head
    # s // gqa, which for this permutation is not perm[s] // gqa
    tiled = np.array([(s % Hk) * gqa + s // Hk for s in range(Hv)])
    assert any(tiled[s] // gqa != s // gqa for s in range(Hv))
    assert rel(relabel(tiled), d["out"]) > 100 * TOL
