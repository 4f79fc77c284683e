"""GPU parity of the whole GatedDeltaNet layer against transformers'
Qwen3_5GatedDeltaNet fixtures (tests/golden/layer_*.npz, written in float32 on the
CPU by tests/golden/make_golden.py).

The parameters load through gdn_params_from_hf (the checkpoint mapping of
loader.py:173-190, 285-307), the layer runs in bf16 on the GPU
(omegalax_amd.layer: projections, gdn_prefill, out_proj; the cached decode path:
gated_deltanet_prefill_cache then gated_deltanet_decode), and its output is held to
* the oracle's layer with the reference's bf16 rounding points, on the GPU's own
  bf16 projection outputs: 2e-2 (max-abs-normalised) -- the parity bar;
* the fixture's fp32 output itself: 2e-2 at dk=dv=128.  At dk=dv=64 and at the
  reference's smoke layout dk=16, dv=32 (both with D=16) the oracle's exact-rounding
  bf16 emulation is itself 1.8e-2 and 4.7e-2 from the fp32 module, so the bounds there
  are 3e-2 and 7e-2: what any bf16 run of the reference would need.
"""
import os
import sys

import numpy as np
import pytest

from oracle import gdn_oracle as O

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu

GOLD = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
BF16_TOL = 2e-2
HF_TOL = {"layer_d128": 2e-2, "layer_d64": 3e-2, "layer_smoke_d16": 7e-2}


def rel(a, b):
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    return float(np.max(np.abs(a - b)) / max(np.max(np.abs(b)), 1e-30))


def say(msg):
    print(msg, flush=True)
    sys.stdout.flush()


def np_(t):
    return t.detach().float().cpu().numpy()


def load(name):
    from omegalax_amd.layer import GDNConfig, gdn_params_from_hf
    d = dict(np.load(os.path.join(GOLD, name + ".npz")))
    D, Hk, Hv, dk, dv = (int(x) for x in d["dims"])
    cfg = GDNConfig(hidden_size=D, num_k_heads=Hk, head_k_dim=dk, num_v_heads=Hv, head_v_dim=dv)
    p = gdn_params_from_hf({k: torch.from_numpy(v) for k, v in d.items()}, 0).to("cuda")
    return d, cfg, p


def oracle_from_projections(p, cfg, h):
    """The oracle layer (bf16 rounding points) on the GPU's bf16 projection outputs."""
    import torch.nn.functional as F
    B, T, _ = h.shape
    mixed, z, a, b = (F.linear(h, w) for w in (p.in_proj_qkv, p.in_proj_z, p.in_proj_a, p.in_proj_b))
    n, S, conv = O.gdn_prefill_layer(np_(mixed), np_(z).reshape(B, T, cfg.num_v_heads, cfg.head_v_dim),
                                     np_(a), np_(b), np_(p.conv_w), np_(p.A_log), np_(p.dt_bias),
                                     np_(p.norm_w), Hk=cfg.num_k_heads, dk=cfg.head_k_dim,
                                     Hv=cfg.num_v_heads, dv=cfg.head_v_dim)
    return np.asarray(n, np.float64).reshape(B, T, -1) @ np_(p.out_proj).astype(np.float64).T, S, conv


@pytest.mark.parametrize("name", sorted(HF_TOL))
def test_layer_forward_with_mask_matches_hf_fixture(name):
    from omegalax_amd.layer import gated_deltanet_forward
    say(f"HF layer fixture {name}: masked prefill")
    d, cfg, p = load(name)
    hidden = torch.from_numpy(d["hidden"]).bfloat16().cuda()
    mask = torch.from_numpy(d["mask"]).cuda()
    out = gated_deltanet_forward(p, cfg, hidden, mask)
    torch.cuda.synchronize()
    h = hidden * mask[:, :, None].to(hidden.dtype)
    ref, _, _ = oracle_from_projections(p, cfg, h)
    assert rel(np_(out), ref) < BF16_TOL
    assert rel(np_(out), d["out"]) < HF_TOL[name]


@pytest.mark.parametrize("name", sorted(HF_TOL))
def test_layer_cached_decode_matches_hf_fixture(name):
    """Prefill into the decode cache, then single-token steps, as HF's DynamicCache path
    ran them; the oracle continues from its own prefill with gdn_decode_step."""
    import torch.nn.functional as F
    from omegalax_amd.layer import gated_deltanet_decode, gated_deltanet_prefill_cache, make_gdn_cache
    say(f"HF layer fixture {name}: cached prefill + decode")
    d, cfg, p = load(name)
    h0 = torch.from_numpy(d["hidden_prefill"]).bfloat16().cuda()
    B = h0.shape[0]
    cache = make_gdn_cache(cfg, 1, B)[0]
    out0 = gated_deltanet_prefill_cache(p, cfg, h0, cache)
    torch.cuda.synchronize()
    ref0, S, conv = oracle_from_projections(p, cfg, h0)
    assert rel(np_(out0), ref0) < BF16_TOL
    assert rel(np_(out0), d["out_prefill"]) < HF_TOL[name]
    dims = dict(Hk=cfg.num_k_heads, dk=cfg.head_k_dim, Hv=cfg.num_v_heads, dv=cfg.head_v_dim)
    for s in range(d["hidden_decode"].shape[0]):
        h = torch.from_numpy(d["hidden_decode"][s]).bfloat16().cuda()
        out = gated_deltanet_decode(p, cfg, h, cache)
        torch.cuda.synchronize()
        mixed, z, a, b = (F.linear(h, w) for w in (p.in_proj_qkv, p.in_proj_z, p.in_proj_a, p.in_proj_b))
        n, conv, S = O.gdn_decode_step(np_(mixed), np_(z).reshape(B, cfg.num_v_heads, -1), np_(a),
                                       np_(b), np_(p.conv_w), np_(p.A_log), np_(p.dt_bias),
                                       np_(p.norm_w), conv, S, **dims)
        ref = np.asarray(n, np.float64) @ np_(p.out_proj).astype(np.float64).T
        assert rel(np_(out), ref) < BF16_TOL, s
        assert rel(np_(out), d["out_decode"][s]) < HF_TOL[name], s
    if "state_after_decode" in d:
        assert rel(np_(cache.recurrent_state), d["state_after_decode"]) < HF_TOL[name]
        assert rel(np_(cache.recurrent_state), S) < 1e-3
