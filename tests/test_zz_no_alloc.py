"""GPU test of omx_gdn_prefill_noalloc, the prefill entry point that allocates nothing
(its scratch is a fixed device array of the library): called through the C ABI, its
outputs must equal omx_gdn_prefill's (same kernels, same inputs: bit for bit) on two
calls in a row, the second with a smaller input, so the second call runs on scratch
that still holds the first call's data."""
import sys

import numpy as np
import pytest

from omegalax_amd import _lib, workloads as W

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu


def say(msg):
    print(msg, flush=True)
    sys.stdout.flush()


def _ptr(t):
    return None if t is None else t.data_ptr()


def run(entry, t, dims, cu=None, S0=None, conv0=None):
    """One call of omx_gdn_prefill or omx_gdn_prefill_noalloc through the C ABI;
    returns (out, final_state, conv_state_out)."""
    Hk, dk, Hv, dv = dims["Hk"], dims["dk"], dims["Hv"], dims["dv"]
    B, T, Cd = t["mixed_qkv"].shape
    N = B if cu is None else cu.numel() - 1
    dev = t["mixed_qkv"].device
    out = torch.empty((B, T, Hv * dv), dtype=torch.bfloat16, device=dev)
    fs = torch.empty((N, Hv, dk, dv), dtype=torch.float32, device=dev)
    cs = torch.empty((N, Cd, 3), dtype=torch.bfloat16, device=dev)
    stream = torch.cuda.current_stream(dev).cuda_stream
    args = [_ptr(t["mixed_qkv"]), _ptr(t["z"]), _ptr(t["a"]), _ptr(t["b"]), _ptr(t["conv_w"]),
            _ptr(t["A_log"]), _ptr(t["dt_bias"]), _ptr(t["norm_w"]), 1e-6, _ptr(cu), N, _ptr(S0),
            _ptr(fs), _ptr(conv0), _ptr(cs), _ptr(out), B, T, Hk, Hv, dk, dv, 4, 64]
    if entry == "omx_gdn_prefill":
        L = _lib.lib()
        nbytes = L.omx_gdn_prefill_workspace_size(B, T, Hk, Hv, dk, dv, N)
        ws = torch.empty(nbytes, dtype=torch.uint8, device=dev)
        _lib.call(entry, *args, _ptr(ws), nbytes, stream)
    else:
        _lib.call(entry, *args, stream)
    torch.cuda.synchronize()
    return out, fs, cs


def case(B, T, dims, seed, packed=None):
    d = W.layer_inputs(B, T, **dims, seed=seed)
    t = W.to_device(d)
    rng = np.random.default_rng(seed + 1)
    cu = S0 = conv0 = None
    N = B
    if packed is not None:
        cu = torch.from_numpy(np.concatenate([[0], np.cumsum(packed)]).astype(np.int32)).cuda()
        N = len(packed)
    S0 = torch.from_numpy((0.02 * rng.standard_normal((N, dims["Hv"], dims["dk"], dims["dv"])))
                          .astype(np.float32)).cuda()
    Cd = 2 * dims["Hk"] * dims["dk"] + dims["Hv"] * dims["dv"]
    conv0 = torch.from_numpy(rng.standard_normal((N, Cd, 3)).astype(np.float32)).cuda().bfloat16()
    return t, cu, S0, conv0


def test_noalloc_prefill_equals_workspace_prefill_twice_shrinking():
    dims = dict(Hk=16, dk=128, Hv=32, dv=128)
    L = _lib.lib()
    assert L.omx_gdn_prefill_noalloc_max_scratch() == 64 << 20
    # first call: near the fixed size (C1 head layout, 3 packed sequences, 1,800 tokens)
    say("noalloc prefill call 1: T=1800 packed [700, 1, 1099], C1 head layout")
    t, cu, S0, conv0 = case(1, 1800, dims, 21, packed=[700, 1, 1099])
    need = L.omx_gdn_prefill_workspace_size(1, 1800, 16, 32, 128, 128, 3)
    assert need > 48 << 20  # the first call fills most of the scratch
    want = run("omx_gdn_prefill", t, dims, cu, S0, conv0)
    got = run("omx_gdn_prefill_noalloc", t, dims, cu, S0, conv0)
    for a, b in zip(got, want):
        assert torch.equal(a, b)
    # second call: smaller, different layout, over scratch the first call left behind
    say("noalloc prefill call 2: B=2 T=100, Hk=2 Hv=4 d=128")
    dims2 = dict(Hk=2, dk=128, Hv=4, dv=128)
    t, _, S0, conv0 = case(2, 100, dims2, 22)
    want = run("omx_gdn_prefill", t, dims2, None, S0, conv0)
    got = run("omx_gdn_prefill_noalloc", t, dims2, None, S0, conv0)
    for a, b in zip(got, want):
        assert torch.equal(a, b)


def test_noalloc_prefill_rejects_shapes_beyond_the_fixed_scratch():
    dims = dict(Hk=16, dk=128, Hv=32, dv=128)
    t, _, _, _ = case(1, 8, dims, 23)
    L = _lib.lib()
    args = [_ptr(t["mixed_qkv"]), _ptr(t["z"]), _ptr(t["a"]), _ptr(t["b"]), _ptr(t["conv_w"]),
            _ptr(t["A_log"]), _ptr(t["dt_bias"]), _ptr(t["norm_w"]), 1e-6, None, 1, None, None,
            None, None, 1, 1, 4096, 16, 32, 128, 128, 4, 64, None]
    rc = L.omx_gdn_prefill_noalloc(*args)
    assert rc == _lib.EINVAL
    assert "scratch" in L.omx_gdn_last_error().decode()


def test_noalloc_prefill_replays_under_hip_graph_capture():
    """The entry point records into a HIP graph (torch.cuda.CUDAGraph): one eager call looks
    the scratch address up, then a call is captured and the graph replayed three times on
    fresh inputs copied into the captured buffers, with eager work and synchronisations in
    between; every replay equals omx_gdn_prefill on the same inputs bit for bit.  The path
    issues no memset, copy or allocation, only kernel launches."""
    dims = dict(Hk=2, dk=128, Hv=4, dv=128)
    B, T, N = 1, 300, 2
    Hk, dk, Hv, dv = dims["Hk"], dims["dk"], dims["Hv"], dims["dv"]
    say(f"noalloc prefill graph capture: B={B} T={T} packed [120, 180], Hk=2 Hv=4 d=128")
    t, cu, S0, conv0 = case(B, T, dims, 31, packed=[120, 180])
    run("omx_gdn_prefill_noalloc", t, dims, cu, S0, conv0)  # eager: address lookup
    Cd = t["mixed_qkv"].shape[-1]
    out = torch.empty((B, T, Hv * dv), dtype=torch.bfloat16, device="cuda")
    fs = torch.empty((N, Hv, dk, dv), dtype=torch.float32, device="cuda")
    cs = torch.empty((N, Cd, 3), dtype=torch.bfloat16, device="cuda")
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        stream = torch.cuda.current_stream().cuda_stream
        _lib.call("omx_gdn_prefill_noalloc", _ptr(t["mixed_qkv"]), _ptr(t["z"]), _ptr(t["a"]),
                  _ptr(t["b"]), _ptr(t["conv_w"]), _ptr(t["A_log"]), _ptr(t["dt_bias"]),
                  _ptr(t["norm_w"]), 1e-6, _ptr(cu), N, _ptr(S0), _ptr(fs), _ptr(conv0), _ptr(cs),
                  _ptr(out), B, T, Hk, Hv, dk, dv, 4, 64, stream)
    for rep in range(3):
        say(f"  replay {rep}")
        t2, _, S2, c2 = case(B, T, dims, 40 + rep, packed=[120, 180])
        for k in ("mixed_qkv", "z", "a", "b"):
            t[k].copy_(t2[k])
        S0.copy_(S2)
        conv0.copy_(c2)
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        want = run("omx_gdn_prefill", t, dims, cu, S0, conv0)
        for a, b in zip((out, fs, cs), want):
            assert torch.equal(a, b)
