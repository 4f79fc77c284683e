"""GPU parity of the decode step and the core recurrent step against the oracle.

Tolerances (stated by the path's contract): fp32 state within 1e-3 relative
(max-abs-normalised), bf16 outputs within 2e-2; the conv cache is raw bf16
data movement and must match bit for bit.
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


def rel(a, b):
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    return float(np.max(np.abs(a - b)) / max(np.max(np.abs(b)), 1e-30))


def say(msg):
    print(msg, flush=True)
    sys.stdout.flush()


def np_(t):
    return t.detach().float().cpu().numpy()


@pytest.mark.parametrize("B,Hk,Hv,dk,dv", [
    (1, 1, 1, 16, 32), (3, 2, 4, 16, 32), (2, 2, 4, 64, 64), (2, 1, 8, 128, 128),
    (2, 2, 2, 32, 128), (4, 16, 32, 128, 128),
    (2, 2, 16, 128, 128),  # gqa 8, the largest the decode kernel takes, at d = 128
    (3, 1, 8, 16, 32),     # gqa 8 at the reference smoke layout's head dims
])
def test_decode_steps_match_oracle(B, Hk, Hv, dk, dv):
    from omegalax_amd import gdn_decode_step
    say(f"decode B={B} Hk={Hk} Hv={Hv} dk={dk} dv={dv}")
    d = W.decode_inputs(B, Hk, Hv, dk, dv, seed=77 + B + dk)
    t = W.to_device(d)
    rng = np.random.default_rng(5)
    conv_ref, S_ref = d["conv_state"], d["state"].astype(np.float64)
    dims = dict(Hk=Hk, dk=dk, Hv=Hv, dv=dv)
    for step in range(3):
        if step:
            for key in ("mixed_qkv", "z", "a", "b"):
                d[key] = O.round_bf16(rng.standard_normal(d[key].shape))
                t[key] = torch.from_numpy(d[key]).to("cuda", torch.bfloat16)
        out = gdn_decode_step(t["mixed_qkv"], t["z"], t["a"], t["b"], t["conv_w"], t["A_log"],
                              t["dt_bias"], t["norm_w"], t["conv_state"], t["state"],
                              num_k_heads=Hk, head_k_dim=dk, num_v_heads=Hv, head_v_dim=dv)
        torch.cuda.synchronize()
        ref, conv_ref, S_ref = O.gdn_decode_step(d["mixed_qkv"], d["z"], d["a"], d["b"],
                                                 d["conv_w"], d["A_log"], d["dt_bias"],
                                                 d["norm_w"], conv_ref, S_ref, **dims)
        assert rel(np_(out), ref) < BF16_TOL, f"step {step} out"
        assert rel(np_(t["state"]), S_ref) < STATE_TOL, f"step {step} state"
        assert np.array_equal(np_(t["conv_state"]), conv_ref), f"step {step} conv cache"


@pytest.mark.parametrize("B", [1, 8, 64, 128])
def test_decode_c2_full_size(B):
    """Config C2 (Hk=16, Hv=32, d=128) at B = 1, 8 (the sweep's small batches), 64 and 128
    (2,048 items: the smallest batch whose grid is one workgroup per CU with 8 items each):
    S [B,32,128,128] fp32 against the fp64 oracle, every sequence."""
    from omegalax_amd import gdn_decode_step
    say(f"decode C2 B={B}")
    d = W.decode_inputs(B)
    t = W.to_device(d)
    out = gdn_decode_step(t["mixed_qkv"], t["z"], t["a"], t["b"], t["conv_w"], t["A_log"],
                          t["dt_bias"], t["norm_w"], t["conv_state"], t["state"],
                          num_k_heads=16, head_k_dim=128, num_v_heads=32, head_v_dim=128)
    torch.cuda.synchronize()
    ref, conv_ref, S_ref = O.gdn_decode_step(d["mixed_qkv"], d["z"], d["a"], d["b"], d["conv_w"],
                                             d["A_log"], d["dt_bias"], d["norm_w"],
                                             d["conv_state"], d["state"].astype(np.float64),
                                             Hk=16, dk=128, Hv=32, dv=128)
    assert rel(np_(out), ref) < BF16_TOL
    assert rel(np_(t["state"]), S_ref) < STATE_TOL
    assert np.array_equal(np_(t["conv_state"]), conv_ref)


def test_decode_c2_b256_streamed_state():
    """Config C2 at B=256: S [256,32,128,128] fp32 is 512 MiB, above the size (192 MiB)
    where the kernel streams the state with non-temporal loads and stores.  Sequences
    are independent, so the fp64 oracle checks a sample of them (first, last and two
    inside), each against the whole-batch GPU call."""
    from omegalax_amd import gdn_decode_step
    say("decode C2 B=256 (non-temporal state path)")
    B = 256
    d = W.decode_inputs(B)
    t = W.to_device(d)
    assert t["state"].numel() * 4 > 192 << 20
    out = gdn_decode_step(t["mixed_qkv"], t["z"], t["a"], t["b"], t["conv_w"], t["A_log"],
                          t["dt_bias"], t["norm_w"], t["conv_state"], t["state"],
                          num_k_heads=16, head_k_dim=128, num_v_heads=32, head_v_dim=128)
    torch.cuda.synchronize()
    rows = np.array([0, 77, 200, 255])
    ref, conv_ref, S_ref = O.gdn_decode_step(d["mixed_qkv"][rows], d["z"][rows], d["a"][rows],
                                             d["b"][rows], d["conv_w"], d["A_log"],
                                             d["dt_bias"], d["norm_w"], d["conv_state"][rows],
                                             d["state"][rows].astype(np.float64),
                                             Hk=16, dk=128, Hv=32, dv=128)
    idx = torch.from_numpy(rows).cuda()
    assert rel(np_(out.index_select(0, idx)), ref) < BF16_TOL
    assert rel(np_(t["state"].index_select(0, idx)), S_ref) < STATE_TOL
    assert np.array_equal(np_(t["conv_state"].index_select(0, idx)), conv_ref)
    # every sequence was updated: no state row is left as it was
    S0 = torch.from_numpy(d["state"]).cuda()
    changed = (t["state"] != S0).flatten(1).any(dim=1)
    assert bool(changed.all())


@pytest.mark.parametrize("dtype", ["f32", "bf16"])
@pytest.mark.parametrize("B,Hk,Hv,dk,dv", [(2, 2, 4, 64, 64), (3, 16, 32, 128, 128),
                                           (1, 1, 3, 32, 16)])
def test_recurrent_step_matches_oracle(dtype, B, Hk, Hv, dk, dv):
    from omegalax_amd import recurrent_gated_delta_rule_step
    say(f"recurrent_step {dtype} B={B} Hk={Hk} Hv={Hv} dk={dk} dv={dv}")
    rng = np.random.default_rng(dk + dv + B)
    q = rng.standard_normal((B, Hk, dk)).astype(np.float32)
    k = rng.standard_normal((B, Hk, dk)).astype(np.float32)
    v = rng.standard_normal((B, Hv, dv)).astype(np.float32)
    if dtype == "bf16":
        q, k, v = O.round_bf16(q), O.round_bf16(k), O.round_bf16(v)
    g = -rng.uniform(0.01, 2.0, (B, Hv)).astype(np.float32)
    beta = rng.uniform(0.0, 1.0, (B, Hv)).astype(np.float32)
    S0 = (0.1 * rng.standard_normal((B, Hv, dk, dv))).astype(np.float32)
    tdt = torch.bfloat16 if dtype == "bf16" else torch.float32
    dev = lambda x, dt=torch.float32: torch.from_numpy(x).to("cuda", dt)
    S = dev(S0)
    o = recurrent_gated_delta_rule_step(dev(q, tdt), dev(k, tdt), dev(v, tdt), dev(g), dev(beta), S)
    torch.cuda.synchronize()
    act = O.round_bf16 if dtype == "bf16" else (lambda x: x)
    o_ref, S_ref = O.recurrent_gated_delta_rule(q[:, None], k[:, None], v[:, None], g[:, None],
                                                beta[:, None], initial_state=S0, act_round=act)
    tol = 1e-5 if dtype == "f32" else STATE_TOL
    assert rel(np_(o), o_ref[:, 0]) < tol
    assert rel(np_(S), S_ref) < tol
