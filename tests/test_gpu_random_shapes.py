"""GPU parity over seeded random layer shapes: prefill, then one cached decode step; and
the layer backward.

Each case draws its head layout (Hk, gqa, dk, dv, with dims the kernels are and are not
compiled for), a batch or a packed batch with initial states and conv history, runs
omx_gdn_prefill through the torch binding, continues every sequence by one decode step
from the returned caches, and compares both with the oracle (deltanet.py:243-293 for the
prefill; the HF cached step for the decode).  Tolerances: bf16 outputs 2e-2, fp32 state
1e-3 (max-abs-normalised); conv caches are raw data movement and must match bit for bit.
The backward cases compare omx_gdn_prefill_bwd with the fp64 layer VJP oracle.
"""
import sys

import numpy as np
import pytest

from oracle import gdn_oracle as O
from omegalax_amd import workloads as W

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu

STATE_TOL = 1e-3
BF16_TOL = 2e-2
DECODE_DIMS = (16, 32, 64, 128)  # head dims the decode kernel takes


def rel(a, b):
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    return float(np.max(np.abs(a - b)) / max(np.max(np.abs(b)), 1e-30))


def np_(t):
    return t.detach().float().cpu().numpy()


def draw_case(seed):
    rng = np.random.default_rng(seed)
    Hk = int(rng.choice([1, 2]))
    gqa = int(rng.choice([1, 2, 3, 4]))
    dk = int(rng.choice([16, 32, 48, 64, 96, 128]))
    dv = int(rng.choice([16, 32, 64, 80, 128, 192]))
    packed = bool(rng.integers(0, 2))
    if packed:
        lens = rng.integers(0, 140, size=int(rng.integers(1, 6)))
        lens[0] = max(int(lens[0]), 1)  # at least one token in the call
        B, N = 1, len(lens)
        cu = np.concatenate([[0], np.cumsum(lens)]).astype(np.int32)
        T = int(cu[-1])
    else:
        B = int(rng.integers(1, 3))
        N, cu = B, None
        T = int(rng.integers(1, 260))
    return rng, dict(Hk=Hk, dk=dk, Hv=Hk * gqa, dv=dv), B, T, N, cu


@pytest.mark.parametrize("seed", range(2100, 2112))
def test_random_layer_shape_prefill_then_decode(seed):
    from omegalax_amd import gdn_decode_step, gdn_prefill
    rng, dims, B, T, N, cu = draw_case(seed)
    print(f"random shape seed={seed} dims={dims} B={B} T={T} N={N} packed={cu is not None}",
          flush=True)
    sys.stdout.flush()
    Hk, dk, Hv, dv = dims["Hk"], dims["dk"], dims["Hv"], dims["dv"]
    conv_dim = 2 * Hk * dk + Hv * dv
    d = W.layer_inputs(B, T, **dims, seed=seed)
    S0 = (0.02 * rng.standard_normal((N, Hv, dk, dv))).astype(np.float32)
    conv0 = O.round_bf16(rng.standard_normal((N, conv_dim, 3)))
    t = W.to_device(d)
    out, S, conv = gdn_prefill(
        t["mixed_qkv"], t["z"], t["a"], t["b"], t["conv_w"], t["A_log"], t["dt_bias"],
        t["norm_w"], num_k_heads=Hk, head_k_dim=dk, num_v_heads=Hv, head_v_dim=dv,
        cu_seqlens=None if cu is None else torch.from_numpy(cu).cuda(),
        initial_state=torch.from_numpy(S0).cuda(),
        conv_state=torch.from_numpy(conv0).cuda().bfloat16(), output_final_state=True)
    torch.cuda.synchronize()
    ref, S_ref, conv_ref = O.gdn_prefill_layer(
        d["mixed_qkv"], d["z"], d["a"], d["b"], d["conv_w"], d["A_log"], d["dt_bias"],
        d["norm_w"], **dims, cu_seqlens=cu, initial_state=S0, conv_state=conv0)
    assert rel(np_(out), ref) < BF16_TOL
    assert rel(np_(S), S_ref) < STATE_TOL
    assert np.array_equal(np_(conv), conv_ref)

    if dk not in DECODE_DIMS or dv not in DECODE_DIMS:
        return  # the decode step is compiled for these head dims only
    # one more token per sequence from the returned caches
    x = O.round_bf16(rng.standard_normal((N, conv_dim)))
    z = O.round_bf16(rng.standard_normal((N, Hv, dv)))
    a = O.round_bf16(rng.standard_normal((N, Hv)))
    b = O.round_bf16(rng.standard_normal((N, Hv)))
    dev = lambda v: torch.from_numpy(v).to("cuda", torch.bfloat16)  # noqa: E731
    out1 = gdn_decode_step(dev(x), dev(z), dev(a), dev(b), t["conv_w"], t["A_log"],
                           t["dt_bias"], t["norm_w"], conv, S, num_k_heads=Hk, head_k_dim=dk,
                           num_v_heads=Hv, head_v_dim=dv)
    torch.cuda.synchronize()
    ref1, conv_ref1, S_ref1 = O.gdn_decode_step(x, z, a, b, d["conv_w"], d["A_log"],
                                                d["dt_bias"], d["norm_w"], conv_ref,
                                                S_ref.astype(np.float64), **dims)
    assert rel(np_(out1), ref1) < BF16_TOL
    assert rel(np_(S), S_ref1) < STATE_TOL
    assert np.array_equal(np_(conv), conv_ref1)


BWD_NAMES = ("dx", "dz", "da", "db", "dconv_w", "dA_log", "ddt_bias", "dnorm_w", "dh0")


@pytest.mark.parametrize("seed", range(2200, 2208))
def test_random_layer_shape_backward(seed):
    """The layer VJP (omx_gdn_prefill_bwd) against the fp64 VJP oracle on random shapes with
    head dims up to 128 (the backward's limit), packed or not, with initial states.
    Gradient tolerances: 2e-2 (bf16-returned activations and their parameter sums), 1e-3
    for the fp32 initial-state gradient."""
    from oracle import gdn_vjp as V
    from omegalax_amd import gdn_prefill_bwd
    rng = np.random.default_rng(seed)
    Hk = int(rng.choice([1, 2]))
    Hv = Hk * int(rng.choice([1, 2, 4]))
    dk = int(rng.choice([16, 32, 48, 64, 96, 128]))
    dv = int(rng.choice([16, 32, 64, 80, 128]))
    if bool(rng.integers(0, 2)):
        lens = rng.integers(0, 100, size=int(rng.integers(1, 5)))
        lens[0] = max(int(lens[0]), 1)
        cu = np.concatenate([[0], np.cumsum(lens)]).astype(np.int32)
        B, T, N = 1, int(cu[-1]), len(lens)
    else:
        cu = None
        B, T = int(rng.integers(1, 3)), int(rng.integers(1, 160))
        N = B
    print(f"random backward seed={seed} Hk={Hk} Hv={Hv} dk={dk} dv={dv} B={B} T={T} N={N} "
          f"packed={cu is not None}", flush=True)
    sys.stdout.flush()
    dims = dict(Hk=Hk, dk=dk, Hv=Hv, dv=dv)
    d = W.layer_inputs(B, T, **dims, seed=seed)
    S0 = (0.02 * rng.standard_normal((N, Hv, dk, dv))).astype(np.float32)
    dout = O.round_bf16(rng.standard_normal((B, T, Hv * dv)))
    dS = (0.1 * rng.standard_normal((N, Hv, dk, dv))).astype(np.float32)
    t = W.to_device(d)
    dev = lambda x: torch.from_numpy(np.ascontiguousarray(x)).cuda()  # noqa: E731
    got = gdn_prefill_bwd(
        t["mixed_qkv"], t["z"], t["a"], t["b"], t["conv_w"], t["A_log"], t["dt_bias"],
        t["norm_w"], dev(dout).bfloat16(), num_k_heads=Hk, head_k_dim=dk, num_v_heads=Hv,
        head_v_dim=dv, cu_seqlens=None if cu is None else dev(cu).int(),
        initial_state=dev(S0), d_final_state=dev(dS))
    torch.cuda.synchronize()
    ref = V.gdn_prefill_layer_bwd(
        d["mixed_qkv"], d["z"], d["a"], d["b"], d["conv_w"], d["A_log"], d["dt_bias"],
        d["norm_w"], dout, **dims, cu_seqlens=cu, initial_state=S0, d_final_state=dS,
        act_round=O.round_bf16)
    for name, g, r in zip(BWD_NAMES, got, ref):
        tol = STATE_TOL if name == "dh0" else BF16_TOL
        err = rel(np_(g), r)
        assert err < tol, (name, err)
