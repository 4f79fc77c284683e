"""GPU parity of the fused layer prefill (conv + gates + chunked rule + gated norm).

Reference semantics: deltanet.py:243-293 (oracle.gdn_prefill_layer).  Tolerances:
bf16 output 2e-2, fp32 state 1e-3 (max-abs-normalised); the conv cache is raw
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


def gpu_prefill(t, dims, cu=None, S0=None, conv0=None):
    from omegalax_amd import gdn_prefill
    out, S, conv = gdn_prefill(
        t["mixed_qkv"], t["z"], t["a"], t["b"], t["conv_w"], t["A_log"], t["dt_bias"], t["norm_w"],
        num_k_heads=dims["Hk"], head_k_dim=dims["dk"], num_v_heads=dims["Hv"],
        head_v_dim=dims["dv"],
        cu_seqlens=None if cu is None else torch.from_numpy(cu).cuda(),
        initial_state=None if S0 is None else torch.from_numpy(S0).cuda(),
        conv_state=None if conv0 is None else torch.from_numpy(conv0).cuda().bfloat16(),
        output_final_state=True)
    torch.cuda.synchronize()
    return out, S, conv


def ref_prefill(d, dims, cu=None, S0=None, conv0=None):
    return O.gdn_prefill_layer(d["mixed_qkv"], d["z"], d["a"], d["b"], d["conv_w"], d["A_log"],
                               d["dt_bias"], d["norm_w"], **dims, cu_seqlens=cu,
                               initial_state=S0, conv_state=conv0)


@pytest.mark.parametrize("B,T,Hk,Hv,dk,dv", [
    (2, 100, 2, 4, 128, 128),   # two batch rows, a partial last chunk
    (1, 64, 1, 1, 64, 64),      # exactly one chunk
    (2, 3, 1, 2, 64, 64),       # shorter than the conv window
    (1, 200, 2, 2, 64, 128),
    (1, 130, 1, 2, 128, 64),
    (1, 100, 1, 6, 128, 64),    # gqa 6: gate inputs restaged past the prefetched four
    (2, 33, 2, 4, 16, 32),      # the reference's smoke layout, on zero-padded copies
    (1, 150, 1, 2, 96, 80),
])
def test_layer_prefill_matches_oracle(B, T, Hk, Hv, dk, dv):
    say(f"layer B={B} T={T} Hk={Hk} Hv={Hv} dk={dk} dv={dv}")
    dims = dict(Hk=Hk, dk=dk, Hv=Hv, dv=dv)
    d = W.layer_inputs(B, T, Hk, Hv, dk, dv, seed=T + dk)
    t = W.to_device(d)
    out, S, conv = gpu_prefill(t, dims)
    ref, S_ref, conv_ref = ref_prefill(d, dims)
    assert rel(np_(out), ref) < BF16_TOL
    assert rel(np_(S), S_ref) < STATE_TOL
    assert np.array_equal(np_(conv), conv_ref)


@pytest.mark.parametrize("dk,dv", [(128, 128), (16, 32)])
def test_layer_varlen_with_carried_states(dk, dv):
    say(f"layer varlen dk={dk} dv={dv}")
    dims = dict(Hk=2, dk=dk, Hv=4, dv=dv)
    lens = [70, 0, 2, 129, 64]
    cu = np.concatenate([[0], np.cumsum(lens)]).astype(np.int32)
    T = int(cu[-1])
    d = W.layer_inputs(1, T, **dims, seed=5)
    rng = np.random.default_rng(6)
    N = len(lens)
    S0 = (0.02 * rng.standard_normal((N, 4, dk, dv))).astype(np.float32)
    conv_dim = 2 * 2 * dk + 4 * dv
    conv0 = O.round_bf16(rng.standard_normal((N, conv_dim, 3)))
    t = W.to_device(d)
    out, S, conv = gpu_prefill(t, dims, cu, S0, conv0)
    ref, S_ref, conv_ref = ref_prefill(d, dims, cu, S0, conv0)
    assert rel(np_(out), ref) < BF16_TOL
    assert rel(np_(S), S_ref) < STATE_TOL
    assert np.array_equal(np_(conv), conv_ref)


def test_layer_many_short_packed_sequences():
    """1,100 packed sequences of 0-4 tokens: past the 1,024 sequences whose start order the
    plan sorts (longest first), the scans take them in index order; every sequence restarts
    its conv window and state (from its own initial state), as the oracle runs each one."""
    say("layer 1100 short packed sequences")
    dims = dict(Hk=1, dk=64, Hv=2, dv=64)
    rng = np.random.default_rng(11)
    lens = rng.integers(0, 5, size=1100)
    cu = np.concatenate([[0], np.cumsum(lens)]).astype(np.int32)
    T = int(cu[-1])
    d = W.layer_inputs(1, T, **dims, seed=12)
    N = len(lens)
    S0 = (0.02 * rng.standard_normal((N, 2, 64, 64))).astype(np.float32)
    t = W.to_device(d)
    out, S, conv = gpu_prefill(t, dims, cu, S0)
    ref, S_ref, conv_ref = ref_prefill(d, dims, cu, S0)
    assert rel(np_(out), ref) < BF16_TOL
    assert rel(np_(S), S_ref) < STATE_TOL
    assert np.array_equal(np_(conv), conv_ref)


def test_layer_offsets_host_checked_or_read_as_ordered_repair():
    """cu_seqlens on the host is checked there (ValueError when invalid); on the device it
    is never read by the host, and the kernels read invalid offsets as c[0] = 0, c[N] = T,
    c[n] = running max of clamp(cu[n], 0, T): the result is then that of the repaired
    offsets, bit for bit, with every output row written."""
    from omegalax_amd import gdn_prefill
    say("layer offsets: host check and device repair")
    dims = dict(Hk=2, dk=128, Hv=4, dv=128)
    T = 150
    d = W.layer_inputs(1, T, **dims, seed=8)
    t = W.to_device(d)
    kw = dict(num_k_heads=2, head_k_dim=128, num_v_heads=4, head_v_dim=128,
              output_final_state=True)
    bad = np.array([3, 70, 40, 120], np.int32)
    fixed = np.array([0, 70, 70, T], np.int32)
    with pytest.raises(ValueError, match="monotonically"):
        gdn_prefill(t["mixed_qkv"], t["z"], t["a"], t["b"], t["conv_w"], t["A_log"],
                    t["dt_bias"], t["norm_w"], cu_seqlens=torch.from_numpy(bad), **kw)
    host = gdn_prefill(t["mixed_qkv"], t["z"], t["a"], t["b"], t["conv_w"], t["A_log"],
                       t["dt_bias"], t["norm_w"], cu_seqlens=torch.from_numpy(fixed), **kw)
    out, S, conv = gpu_prefill(t, dims, bad)
    out2, S2, conv2 = gpu_prefill(t, dims, fixed)
    for a, b, c in zip((out, S, conv), (out2, S2, conv2), host):
        assert bool(torch.isfinite(a.float()).all())
        assert torch.equal(a, b) and torch.equal(a, c)
    ref, S_ref, conv_ref = ref_prefill(d, dims, fixed)
    assert rel(np_(out), ref) < BF16_TOL
    assert rel(np_(S), S_ref) < STATE_TOL
    assert np.array_equal(np_(conv), conv_ref)


def test_prefill_then_decode_equals_longer_prefill():
    """prefill(x[:n]) + decode steps x[n], x[n+1], ... == prefill(x) (GPU vs GPU)."""
    from omegalax_amd import gdn_decode_step
    say("prefill -> decode handoff")
    dims = dict(Hk=2, dk=128, Hv=4, dv=128)
    T, n = 70, 66
    d = W.layer_inputs(2, T, **dims, seed=9)
    t = W.to_device(d)
    full, S_full, conv_full = gpu_prefill(t, dims)
    part = {k_: (v_[:, :n].contiguous() if k_ in ("mixed_qkv", "z", "a", "b") else v_)
            for k_, v_ in t.items()}
    _, S, conv = gpu_prefill(part, dims)
    for step in range(n, T):
        o = gdn_decode_step(t["mixed_qkv"][:, step].contiguous(), t["z"][:, step].contiguous(),
                            t["a"][:, step].contiguous(), t["b"][:, step].contiguous(),
                            t["conv_w"], t["A_log"], t["dt_bias"], t["norm_w"], conv, S,
                            num_k_heads=2, head_k_dim=128, num_v_heads=4, head_v_dim=128)
        torch.cuda.synchronize()
        assert rel(np_(o), np_(full[:, step])) < BF16_TOL, f"token {step}"
    assert rel(np_(S), np_(S_full)) < STATE_TOL
    assert np.array_equal(np_(conv), np_(conv_full))


def test_layer_c1_shape_batch_slice():
    """Config C1's shape (B=4, T=4096, Hk=16, Hv=32, d=128); batch row 0 against the oracle."""
    say("layer C1 shape")
    dims = dict(Hk=16, dk=128, Hv=32, dv=128)
    d = W.layer_inputs(4, 4096)
    t = W.to_device(d)
    out, S, conv = gpu_prefill(t, dims)
    d0 = {k_: (v_[:1] if k_ in ("mixed_qkv", "z", "a", "b") else v_) for k_, v_ in d.items()}
    ref, S_ref, conv_ref = ref_prefill(d0, dims)
    assert rel(np_(out[:1]), ref) < BF16_TOL
    assert rel(np_(S[:1]), S_ref) < STATE_TOL
    assert np.array_equal(np_(conv[:1]), conv_ref)
    # batch rows are independent: row 3 of the batched run equals a run on row 3 alone
    t3 = {k_: (v_[3:4].contiguous() if k_ in ("mixed_qkv", "z", "a", "b") else v_)
          for k_, v_ in t.items()}
    out3, S3, _ = gpu_prefill(t3, dims)
    assert torch.equal(out3, out[3:4]) and torch.equal(S3, S[3:4])


def key_head_slice(d, hk, Hk, dk, Hv, dv):
    """The inputs of key head hk and its gqa value heads alone (a layer with Hk=1): its q,
    k and value channels of mixed_qkv and conv_w, its heads of z, a, b, A_log, dt_bias.
    Key heads share nothing, so the slice's outputs are the full layer's on those heads.
    Returns (inputs, channel indices, value-head slice)."""
    gqa = Hv // Hk
    hs = slice(hk * gqa, (hk + 1) * gqa)
    ch = np.concatenate([np.arange(hk * dk, (hk + 1) * dk),
                         Hk * dk + np.arange(hk * dk, (hk + 1) * dk),
                         2 * Hk * dk + np.arange(hk * gqa * dv, (hk + 1) * gqa * dv)])
    sl = dict(mixed_qkv=d["mixed_qkv"][..., ch], z=d["z"][..., hs, :], a=d["a"][..., hs],
              b=d["b"][..., hs], conv_w=d["conv_w"][ch], A_log=d["A_log"][hs],
              dt_bias=d["dt_bias"][hs], norm_w=d["norm_w"])
    return sl, ch, hs


def test_layer_c3_full_size_packed_equals_separate():
    """Config C3 at full size: T=32768 packed as 8 Dirichlet-length sequences with carried
    initial states (C1 heads, B=1).  Each sequence's output, final state and conv cache from
    the packed call equal a separate call on that sequence (GPU vs GPU); the shortest
    sequence matches the oracle on every head, and the longest (the 10,779-token one) on the
    first and last key heads' value heads: its output, final state and conv cache."""
    say("layer C3 full size")
    dims = dict(Hk=16, dk=128, Hv=32, dv=128)
    d = W.varlen_inputs()
    cu = d["cu_seqlens"]
    S0 = d["initial_state"]
    t = W.to_device({k_: v_ for k_, v_ in d.items() if k_ not in ("cu_seqlens", "initial_state")})
    out, S, conv = gpu_prefill(t, dims, cu, S0)
    lens = np.diff(cu)
    for n in range(len(lens)):
        s, e = int(cu[n]), int(cu[n + 1])
        tn = {k_: (v_[:, s:e].contiguous() if k_ in ("mixed_qkv", "z", "a", "b") else v_)
              for k_, v_ in t.items()}
        o_n, S_n, c_n = gpu_prefill(tn, dims, None, S0[n:n + 1])
        assert rel(np_(o_n), np_(out[:, s:e])) < 1e-6, f"sequence {n}"
        assert rel(np_(S_n), np_(S[n:n + 1])) < 1e-6, f"sequence {n}"
        assert torch.equal(c_n, conv[n:n + 1])
    n = int(np.argmin(lens))
    s, e = int(cu[n]), int(cu[n + 1])
    dn = {k_: (v_[:, s:e] if k_ in ("mixed_qkv", "z", "a", "b") else v_)
          for k_, v_ in d.items() if k_ not in ("cu_seqlens", "initial_state")}
    ref, S_ref, conv_ref = ref_prefill(dn, dims, None, S0[n:n + 1])
    assert rel(np_(out[:, s:e]), ref) < BF16_TOL
    assert rel(np_(S[n:n + 1]), S_ref) < STATE_TOL
    assert np.array_equal(np_(conv[n:n + 1]), conv_ref)
    n = int(np.argmax(lens))
    s, e = int(cu[n]), int(cu[n + 1])
    Hk, dk, Hv, dv = dims["Hk"], dims["dk"], dims["Hv"], dims["dv"]
    out_h = np_(out[:, s:e]).reshape(1, e - s, Hv, dv)
    for hk in (0, Hk - 1):
        say(f"  longest sequence ({e - s} tokens), key head {hk}: fp64 oracle")
        dn = {k_: (v_[:, s:e] if k_ in ("mixed_qkv", "z", "a", "b") else v_)
              for k_, v_ in d.items() if k_ not in ("cu_seqlens", "initial_state")}
        sl, ch, hs = key_head_slice(dn, hk, Hk, dk, Hv, dv)
        sdims = dict(Hk=1, dk=dk, Hv=Hv // Hk, dv=dv)
        ref, S_ref, conv_ref = ref_prefill(sl, sdims, None, S0[n:n + 1, hs])
        assert rel(out_h[:, :, hs].reshape(ref.shape), ref) < BF16_TOL
        assert rel(np_(S[n:n + 1, hs]), S_ref) < STATE_TOL
        assert np.array_equal(np_(conv[n:n + 1])[:, ch], conv_ref)


def test_layer_fused_norm_equals_epilogue_kernel():
    """The layer scan applies the gated norm itself when its grid is one round of the chip
    (here B=32 at Hk=2, Hv=4, d=128: 256 workgroups of 64 columns) and leaves it to the
    epilogue kernel otherwise (B=64: 512).  Both form each row's statistic from the same
    partials in the same pairwise order and apply the same arithmetic, so the first 32
    sequences' outputs, final states and conv caches agree bit for bit; rows past a
    sequence's end (T=300 is not a multiple of 64) stay unwritten in both."""
    say("layer fused norm == epilogue kernel")
    dims = dict(Hk=2, dk=128, Hv=4, dv=128)
    d = W.layer_inputs(64, 300, **dims, seed=31)
    rng = np.random.default_rng(32)
    S0 = (0.02 * rng.standard_normal((64, 4, 128, 128))).astype(np.float32)
    t = W.to_device(d)
    out64, S64, c64 = gpu_prefill(t, dims, None, S0)
    t32 = {k_: (v_[:32].contiguous() if k_ in ("mixed_qkv", "z", "a", "b") else v_)
           for k_, v_ in t.items()}
    out32, S32, c32 = gpu_prefill(t32, dims, None, S0[:32])
    assert torch.equal(out32, out64[:32])
    assert torch.equal(S32, S64[:32]) and torch.equal(c32, c64[:32])
    # and the fused result against the oracle on one sequence
    d0 = {k_: (v_[5:6] if k_ in ("mixed_qkv", "z", "a", "b") else v_) for k_, v_ in d.items()}
    ref, S_ref, _ = ref_prefill(d0, dims, None, S0[5:6])
    assert rel(np_(out32[5:6]), ref) < BF16_TOL
    assert rel(np_(S32[5:6]), S_ref) < STATE_TOL


def test_layer_fused_norm_writes_nothing_past_the_last_token():
    """The scan that applies the norm itself stores a ragged last chunk through a buffer
    whose range ends at the sequence's last row.  At B=1, T=981 (C1's heads: 256
    workgroups, so the norm is fused) the call writes into an output with 64 guard rows
    after the last token: the guard rows keep their sentinel, and the first T rows equal
    the Python API's output."""
    from omegalax_amd import _lib
    from omegalax_amd.deltanet import _ptr, _stream, _workspace
    say("layer fused norm: guard rows past the last token")
    dims = dict(Hk=16, dk=128, Hv=32, dv=128)
    T, G = 981, 64
    d = W.layer_inputs(1, T, **dims, seed=41)
    t = W.to_device(d)
    ref, _, _ = gpu_prefill(t, dims)
    Hk, dk, Hv, dv = 16, 128, 32, 128
    x, z, a, b = (t[k_].contiguous() for k_ in ("mixed_qkv", "z", "a", "b"))
    conv_w, A_log, dt_bias, norm_w = (t[k_].float().contiguous()
                                      for k_ in ("conv_w", "A_log", "dt_bias", "norm_w"))
    out = torch.full((T + G, Hv * dv), -3.0, dtype=torch.bfloat16, device="cuda")
    sentinel = out[T:].clone()
    L = _lib.lib()
    ws_bytes = L.omx_gdn_prefill_workspace_size(1, T, Hk, Hv, dk, dv, 1)
    ws = _workspace(ws_bytes, out.device)
    _lib.call("omx_gdn_prefill", _ptr(x), _ptr(z), _ptr(a), _ptr(b), _ptr(conv_w), _ptr(A_log),
              _ptr(dt_bias), _ptr(norm_w), 1e-6, None, 1, None, None, None, None, _ptr(out), 1, T,
              Hk, Hv, dk, dv, conv_w.shape[1], 64, _ptr(ws), ws_bytes, _stream(out.device))
    torch.cuda.synchronize()
    assert torch.equal(out[T:], sentinel)
    assert torch.equal(out[:T], ref.reshape(T, Hv * dv))
