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
