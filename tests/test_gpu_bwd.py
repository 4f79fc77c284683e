"""GPU parity of the backward pass (VJP) of the chunked rule against the fp64 oracle.

The oracle (oracle/gdn_vjp.py) is the hand-written reverse pass of the pinned forward
restatement; it is itself pinned by finite differences and by torch autograd of the
token recurrence (tests/test_vjp_oracle.py).  Tolerances (max-abs-normalised):
gradients returned at bf16 (dq, dk, dv for bf16 inputs) 2e-2, the bf16 outputs' bar;
fp32 gradients (dg, dbeta, d_initial_state, and everything for fp32 inputs) 1e-3.
"""
import sys

import numpy as np
import pytest

from oracle import gdn_oracle as O
from oracle import gdn_vjp as V

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu

BF16_TOL = 2e-2
F32_TOL = 1e-3


def rel(a, b):
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    return float(np.max(np.abs(a - b)) / max(np.max(np.abs(b)), 1e-30))


def say(msg):
    print(msg, flush=True)
    sys.stdout.flush()


def np_(t):
    return t.detach().float().cpu().numpy()


def dev(x, dt=torch.float32):
    return torch.from_numpy(np.ascontiguousarray(x)).to("cuda", dt)


def make(seed, B, T, Hk, Hv, dk, dv, dtype, s0=True, N=None):
    rng = np.random.default_rng(seed)
    q = rng.standard_normal((B, T, Hk, dk)).astype(np.float32)
    k = rng.standard_normal((B, T, Hk, dk)).astype(np.float32)
    v = rng.standard_normal((B, T, Hv, dv)).astype(np.float32)
    if dtype == "bf16":
        q, k, v = O.round_bf16(q), O.round_bf16(k), O.round_bf16(v)
    a = rng.standard_normal((B, T, Hv)).astype(np.float32)
    A_log = rng.uniform(0, np.log(16), Hv)
    dt = rng.uniform(-2, 0, Hv)
    g = (-np.exp(A_log) * np.logaddexp(a + dt, 0)).astype(np.float32)
    beta = O.round_bf16(1 / (1 + np.exp(-rng.standard_normal((B, T, Hv)))))
    n = B if N is None else N
    S0 = (0.1 * rng.standard_normal((n, Hv, dk, dv))).astype(np.float32) if s0 else None
    do = rng.standard_normal((B, T, Hv, dv)).astype(np.float32)
    dht = (0.1 * rng.standard_normal((n, Hv, dk, dv))).astype(np.float32)
    return q, k, v, g, beta, S0, do, dht


def run_gpu(q, k, v, g, beta, S0, do, dht, dtype, cu=None):
    from omegalax_amd import chunk_gated_delta_rule_bwd
    tdt = torch.bfloat16 if dtype == "bf16" else torch.float32
    out = chunk_gated_delta_rule_bwd(
        dev(q, tdt), dev(k, tdt), dev(v, tdt), dev(g), dev(beta), dev(do), 64,
        initial_state=None if S0 is None else dev(S0),
        d_final_state=None if dht is None else dev(dht),
        cu_seqlens=None if cu is None else dev(cu, torch.int32))
    torch.cuda.synchronize()
    return [np_(t) for t in out]


def run_ref(q, k, v, g, beta, S0, do, dht, dtype, cu=None):
    act = O.round_bf16 if dtype == "bf16" else (lambda x: x)
    return V.chunk_gated_delta_rule_bwd(q, k, v, g, beta, do, 64, initial_state=S0, dht=dht,
                                        cu_seqlens=cu, act_round=act)


NAMES = ("dq", "dk", "dv", "dg", "dbeta", "dh0")


def check(got, ref, dtype, skip=()):
    errs = {}
    for name, a, b in zip(NAMES, got, ref):
        if name in skip:
            continue
        errs[name] = rel(a, b)
    say("  " + " ".join(f"{k}={v:.2e}" for k, v in errs.items()))
    for name, e in errs.items():
        tol = BF16_TOL if (dtype == "bf16" and name in ("dq", "dk", "dv")) else F32_TOL
        assert e < tol, (name, e, tol)


CASES = [
    # B, T, Hk, Hv, dk, dv, dtype
    (1, 64, 1, 1, 128, 128, "bf16"),
    (2, 100, 2, 4, 128, 128, "bf16"),
    (1, 1, 1, 2, 128, 128, "bf16"),
    (1, 257, 1, 2, 64, 64, "bf16"),
    (2, 130, 2, 2, 64, 128, "bf16"),
    (1, 200, 1, 1, 128, 64, "bf16"),
    (2, 150, 1, 2, 64, 64, "f32"),
    (1, 70, 2, 2, 32, 128, "f32"),
    (1, 120, 1, 6, 128, 64, "bf16"),  # gqa 6
    # head dims the kernels are not compiled for run on zero-padded copies: the
    # reference's smoke layout (config.py:94-101), and odd sizes
    (2, 100, 2, 4, 16, 32, "bf16"),
    (2, 100, 2, 4, 16, 32, "f32"),
    (1, 130, 1, 2, 96, 80, "bf16"),
]


@pytest.mark.parametrize("B,T,Hk,Hv,dk,dv,dtype", CASES)
def test_bwd_matches_oracle(B, T, Hk, Hv, dk, dv, dtype):
    say(f"bwd B={B} T={T} Hk={Hk} Hv={Hv} dk={dk} dv={dv} {dtype}")
    args = make(B * 1000 + T + dk, B, T, Hk, Hv, dk, dv, dtype)
    check(run_gpu(*args, dtype), run_ref(*args, dtype), dtype)


def test_bwd_without_state_cotangent_or_initial_state():
    say("bwd S0=None dht=None")
    q, k, v, g, beta, _, do, _ = make(5, 1, 180, 2, 4, 128, 128, "bf16", s0=False)
    check(run_gpu(q, k, v, g, beta, None, do, None, "bf16"),
          run_ref(q, k, v, g, beta, None, do, None, "bf16"), "bf16")


def test_bwd_varlen_matches_oracle():
    say("bwd varlen")
    lens = [70, 0, 1, 200, 64, 129]
    cu = np.concatenate([[0], np.cumsum(lens)]).astype(np.int32)
    T = int(cu[-1])
    q, k, v, g, beta, S0, do, dht = make(9, 1, T, 2, 4, 128, 128, "bf16", N=len(lens))
    check(run_gpu(q, k, v, g, beta, S0, do, dht, "bf16", cu),
          run_ref(q, k, v, g, beta, S0, do, dht, "bf16", cu), "bf16")


def test_bwd_c0_config():
    """Config C0's shapes and gate draws (fp32, B=2 T=512 H=4 d=64) against the fp64 oracle."""
    say("bwd C0")
    from omegalax_amd import workloads as W
    d = W.core_c0()
    rng = np.random.default_rng(77)
    do = rng.standard_normal(d["v"].shape).astype(np.float32)
    args = (d["q"], d["k"], d["v"], d["g"], d["beta"], None, do, None)
    check(run_gpu(*args, "f32"), run_ref(*args, "f32"), "f32", skip=("dh0",))


def test_autograd_routes_through_the_bwd_entry_point():
    """torch.autograd through chunk_gated_delta_rule gives the entry point's gradients."""
    say("bwd autograd")
    from omegalax_amd import chunk_gated_delta_rule
    q, k, v, g, beta, S0, do, dht = make(21, 1, 150, 2, 4, 128, 128, "bf16")
    ts = [dev(x, torch.bfloat16).requires_grad_() for x in (q, k, v)]
    gs = [dev(x).requires_grad_() for x in (g, beta, S0)]
    o, S = chunk_gated_delta_rule(*ts, gs[0], gs[1], 64, initial_state=gs[2],
                                  output_final_state=True)
    grads = torch.autograd.grad((o, S), ts + gs, (dev(do), dev(dht)))
    ref = run_gpu(q, k, v, g, beta, S0, do, dht, "bf16")
    for a, b in zip(grads, ref):
        assert np.array_equal(np_(a), b)


def test_bwd_long_memory_gates():
    """Long-memory gates (e^g in [0.9, 0.9999], config C4's regime) over 2048 tokens."""
    say("bwd long-memory T=2048")
    q, k, v, _, beta, S0, do, dht = make(31, 1, 2048, 1, 2, 128, 128, "bf16")
    g = np.log(np.random.default_rng(3).uniform(0.9, 0.9999, beta.shape)).astype(np.float32)
    check(run_gpu(q, k, v, g, beta, S0, do, dht, "bf16"),
          run_ref(q, k, v, g, beta, S0, do, dht, "bf16"), "bf16")


def test_bwd_4096_tokens_gqa():
    """64 chunks (C1's sequence length) with GQA and both state cotangents."""
    say("bwd T=4096")
    args = make(41, 1, 4096, 2, 4, 128, 128, "bf16")
    check(run_gpu(*args, "bf16"), run_ref(*args, "bf16"), "bf16")
