"""GPU parity of the layer prefill's backward pass (omx_gdn_prefill_bwd) against the fp64
layer VJP oracle (oracle/gdn_vjp.gdn_prefill_layer_bwd, pinned by finite differences of the
layer forward in tests/test_vjp_oracle.py).

Tolerances (max-abs-normalised): 2e-2 for every gradient -- the activation gradients are
returned at bf16, and the parameter gradients are sums of products with the rule's bf16
input gradients; 1e-3 for the fp32 initial-state gradient.
"""
import sys

import numpy as np
import pytest

from oracle import gdn_oracle as O
from oracle import gdn_vjp as V
from omegalax_amd import workloads as W

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu

BF16_TOL = 2e-2
STATE_TOL = 1e-3
NAMES = ("dx", "dz", "da", "db", "dconv_w", "dA_log", "ddt_bias", "dnorm_w", "dh0")


def rel(a, b):
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    return float(np.max(np.abs(a - b)) / max(np.max(np.abs(b)), 1e-30))


def say(msg):
    print(msg, flush=True)
    sys.stdout.flush()


def np_(t):
    return t.detach().float().cpu().numpy()


def make(seed, B, T, Hk, Hv, dk, dv, N=None):
    d = W.layer_inputs(B, T, Hk, Hv, dk, dv, seed=seed)
    rng = np.random.default_rng(seed + 1)
    n = B if N is None else N
    d["S0"] = (0.02 * rng.standard_normal((n, Hv, dk, dv))).astype(np.float32)
    d["dout"] = O.round_bf16(rng.standard_normal((B, T, Hv * dv)))
    d["dS"] = (0.1 * rng.standard_normal((n, Hv, dk, dv))).astype(np.float32)
    return d


def run_gpu(d, dims, cu=None, s0=True):
    from omegalax_amd import gdn_prefill_bwd
    t = W.to_device({k_: v_ for k_, v_ in d.items() if k_ not in ("S0", "dout", "dS")})
    dev = lambda x: torch.from_numpy(np.ascontiguousarray(x)).cuda()
    out = gdn_prefill_bwd(
        t["mixed_qkv"], t["z"], t["a"], t["b"], t["conv_w"], t["A_log"], t["dt_bias"],
        t["norm_w"], dev(d["dout"]).bfloat16(), num_k_heads=dims["Hk"], head_k_dim=dims["dk"],
        num_v_heads=dims["Hv"], head_v_dim=dims["dv"],
        cu_seqlens=None if cu is None else dev(cu).int(),
        initial_state=dev(d["S0"]) if s0 else None, d_final_state=dev(d["dS"]))
    torch.cuda.synchronize()
    return [np_(x) for x in out]


def run_ref(d, dims, cu=None, s0=True):
    return V.gdn_prefill_layer_bwd(
        d["mixed_qkv"], d["z"], d["a"], d["b"], d["conv_w"], d["A_log"], d["dt_bias"],
        d["norm_w"], d["dout"], **dims, cu_seqlens=cu, initial_state=d["S0"] if s0 else None,
        d_final_state=d["dS"], act_round=O.round_bf16)


def check(got, ref):
    errs = {n: rel(a, b) for n, a, b in zip(NAMES, got, ref)}
    say("  " + " ".join(f"{k}={v:.2e}" for k, v in errs.items()))
    for n, e in errs.items():
        assert e < (STATE_TOL if n == "dh0" else BF16_TOL), (n, e)


@pytest.mark.parametrize("B,T,Hk,Hv,dk,dv", [
    (2, 100, 2, 4, 128, 128),
    (1, 200, 1, 2, 64, 64),
    (1, 130, 2, 2, 64, 128),
    (2, 3, 1, 2, 128, 64),
    (1, 100, 1, 6, 128, 64),
    (2, 33, 2, 4, 16, 32),       # the reference's smoke layout, on zero-padded copies
    (1, 90, 1, 2, 96, 48),
    (1, 40, 32, 256, 64, 64),    # Hv = 256, the most value heads the layer backward takes
])
def test_layer_bwd_matches_oracle(B, T, Hk, Hv, dk, dv):
    say(f"layer bwd B={B} T={T} Hk={Hk} Hv={Hv} dk={dk} dv={dv}")
    dims = dict(Hk=Hk, dk=dk, Hv=Hv, dv=dv)
    d = make(B * 100 + T, B, T, Hk, Hv, dk, dv)
    check(run_gpu(d, dims), run_ref(d, dims))


def test_layer_bwd_varlen():
    say("layer bwd varlen")
    lens = [70, 0, 1, 129, 64]
    cu = np.concatenate([[0], np.cumsum(lens)]).astype(np.int32)
    dims = dict(Hk=2, dk=128, Hv=4, dv=128)
    d = make(7, 1, int(cu[-1]), 2, 4, 128, 128, N=len(lens))
    check(run_gpu(d, dims, cu), run_ref(d, dims, cu))


def test_layer_autograd_routes_through_the_bwd_entry_point():
    """torch.autograd through gdn_prefill gives omx_gdn_prefill_bwd's gradients."""
    say("layer bwd autograd")
    from omegalax_amd import gdn_prefill
    dims = dict(Hk=2, dk=128, Hv=4, dv=128)
    d = make(11, 1, 150, 2, 4, 128, 128)
    t = W.to_device({k_: v_ for k_, v_ in d.items() if k_ not in ("S0", "dout", "dS")})
    names = ("mixed_qkv", "z", "a", "b", "conv_w", "A_log", "dt_bias", "norm_w")
    ins = [t[n].clone().requires_grad_() for n in names]
    S0 = torch.from_numpy(d["S0"]).cuda().requires_grad_()
    out, S, _ = gdn_prefill(*ins, num_k_heads=2, head_k_dim=128, num_v_heads=4, head_v_dim=128,
                            initial_state=S0, output_final_state=True)
    grads = torch.autograd.grad((out, S), ins + [S0],
                                (torch.from_numpy(d["dout"]).cuda().bfloat16(),
                                 torch.from_numpy(d["dS"]).cuda()))
    ref = run_gpu(d, dims)
    for g_, r_ in zip(grads, ref):
        assert np.array_equal(np_(g_).reshape(r_.shape), r_)


def test_layer_module_trains_end_to_end():
    """Gradients of every parameter and of the input through the layer module's forward
    (projections -> gdn_prefill -> out_proj, deltanet.py:226-306) under torch.autograd,
    against the chain rule around the fp64 layer VJP oracle."""
    say("layer module training step")
    from omegalax_amd import GDNConfig, GDNParams, gated_deltanet_forward
    Hk, dk, Hv, dv, D, B, T = 2, 128, 4, 128, 64, 1, 100
    cfg = GDNConfig(hidden_size=D, num_k_heads=Hk, head_k_dim=dk, num_v_heads=Hv, head_v_dim=dv)
    rng = np.random.default_rng(21)
    Cd = 2 * Hk * dk + Hv * dv
    w = {
        "in_proj_qkv": O.round_bf16(0.1 * rng.standard_normal((Cd, D))),
        "in_proj_z": O.round_bf16(0.1 * rng.standard_normal((Hv * dv, D))),
        "in_proj_b": O.round_bf16(0.1 * rng.standard_normal((Hv, D))),
        "in_proj_a": O.round_bf16(0.1 * rng.standard_normal((Hv, D))),
        "conv_w": (0.1 * rng.standard_normal((Cd, 4))).astype(np.float32),
        "dt_bias": rng.uniform(-2, 0, Hv).astype(np.float32),
        "A_log": rng.uniform(0, np.log(16), Hv).astype(np.float32),
        "norm_w": rng.uniform(0.5, 1.5, dv).astype(np.float32),
        "out_proj": O.round_bf16(0.05 * rng.standard_normal((D, Hv * dv))),
    }
    h = O.round_bf16(rng.standard_normal((B, T, D)))
    R = O.round_bf16(rng.standard_normal((B, T, D)))
    bf = ("in_proj_qkv", "in_proj_z", "in_proj_b", "in_proj_a", "out_proj")
    tw = {n: torch.from_numpy(v).cuda().to(torch.bfloat16 if n in bf else torch.float32)
          .requires_grad_() for n, v in w.items()}
    th = torch.from_numpy(h).cuda().bfloat16().requires_grad_()
    out = gated_deltanet_forward(GDNParams(**tw), cfg, th)
    (out.float() * torch.from_numpy(R).cuda()).sum().backward()
    # reference: forward with bf16-rounded projection outputs, then the chain rule
    f64 = {n: np.asarray(v, np.float64) for n, v in w.items()}
    mixed = O.round_bf16(h @ f64["in_proj_qkv"].T)
    z = O.round_bf16(h @ f64["in_proj_z"].T).reshape(B, T, Hv, dv)
    b = O.round_bf16(h @ f64["in_proj_b"].T)
    a = O.round_bf16(h @ f64["in_proj_a"].T)
    core, _, _ = O.gdn_prefill_layer(mixed, z, a, b, w["conv_w"], w["A_log"], w["dt_bias"],
                                     w["norm_w"], Hk=Hk, dk=dk, Hv=Hv, dv=dv)
    d_core = R @ f64["out_proj"]
    dmix, dz, da, db, dconv, dA, ddt, dnw, _ = V.gdn_prefill_layer_bwd(
        mixed, z, a, b, w["conv_w"], w["A_log"], w["dt_bias"], w["norm_w"], d_core, Hk=Hk,
        dk=dk, Hv=Hv, dv=dv, act_round=O.round_bf16)
    flat = lambda x: x.reshape(-1, x.shape[-1]) if x.ndim > 2 else x
    hf = h.reshape(-1, D)
    ref = {
        "out_proj": flat(R).T @ core.reshape(-1, Hv * dv),
        "in_proj_qkv": flat(dmix).T @ hf,
        "in_proj_z": dz.reshape(-1, Hv * dv).T @ hf,
        "in_proj_a": flat(da).T @ hf,
        "in_proj_b": flat(db).T @ hf,
        "conv_w": dconv, "A_log": dA, "dt_bias": ddt, "norm_w": dnw,
    }
    dh = (flat(dmix) @ f64["in_proj_qkv"] + dz.reshape(-1, Hv * dv) @ f64["in_proj_z"]
          + flat(da) @ f64["in_proj_a"] + flat(db) @ f64["in_proj_b"])
    errs = {n: rel(np_(tw[n].grad), r) for n, r in ref.items()}
    errs["hidden"] = rel(np_(th.grad).reshape(-1, D), dh)
    say("  " + " ".join(f"{k}={v:.2e}" for k, v in errs.items()))
    for n, e in errs.items():
        assert e < BF16_TOL, (n, e)


def test_layer_bwd_c1_heads_packed_persistent_rows():
    """The C1 head layout (Hk=16, Hv=32, d=128) with tokens * Hv = 19,200 rows, above the
    16,384 (token, value head) rows one pass of the norm adjoint's persistent grid covers, so
    its wavefronts take a second row; three packed sequences, one of a single token."""
    say("layer bwd C1 heads, T=600 packed in 3 sequences (norm adjoint's second pass)")
    lens = [200, 1, 399]
    cu = np.concatenate([[0], np.cumsum(lens)]).astype(np.int32)
    dims = dict(Hk=16, dk=128, Hv=32, dv=128)
    d = make(11, 1, int(cu[-1]), 16, 32, 128, 128, N=len(lens))
    got = run_gpu(d, dims, cu)
    say("  oracle (fp64, about 20 s)")
    check(got, run_ref(d, dims, cu))


def test_layer_bwd_reads_invalid_offsets_as_their_ordered_repair():
    """Offsets that break 0 = cu[0] <= ... <= cu[N] = T are read as c[0] = 0, c[N] = T,
    c[n] = running max of clamp(cu[n], 0, T): every token belongs to one sequence, so no
    gradient row is left unwritten and no parameter gradient sums one."""
    say("layer bwd with invalid offsets")
    T = 150
    bad = np.array([3, 70, 40, 120], np.int32)       # cu[0] > 0, a decrease, cu[N] < T
    fixed = np.array([0, 70, 70, T], np.int32)
    dims = dict(Hk=2, dk=128, Hv=4, dv=128)
    d = make(13, 1, T, 2, 4, 128, 128, N=3)
    got = run_gpu(d, dims, bad)
    want = run_gpu(d, dims, fixed)
    for n, a, b in zip(NAMES, got, want):
        assert np.all(np.isfinite(a)), n
        assert np.array_equal(a, b), n
    check(got, run_ref(d, dims, fixed))
