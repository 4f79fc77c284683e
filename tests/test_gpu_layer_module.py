"""GPU parity of the GatedDeltaNet layer module (omegalax_amd.layer):

* the layer forward (projections as bf16 GEMMs, the fused kernel path between them)
  against the oracle's layer restatement on the same projection outputs
  (deltanet.py:226-306), with an attention mask;
* packed documents (segment ids) against the oracle's layer run on each document
  alone (state and conv window restart at every document), and against one GPU run
  per document;
* a right-padded prefill into the decode cache, then cached decode steps, against
  the oracle's prefill of each row's real tokens followed by the oracle's decode
  steps (gdn_decode_step), and against a full GPU prefill of each row.
Tolerance: bf16 outputs 2e-2 (max-abs-normalised).
"""
import sys

import numpy as np
import pytest

from oracle import gdn_oracle as O

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu

BF16_TOL = 2e-2


def rel(a, b):
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    return float(np.max(np.abs(a - b)) / max(np.max(np.abs(b)), 1e-30))


def say(msg):
    print(msg, flush=True)
    sys.stdout.flush()


def make(D=96, Hk=2, dk=128, Hv=4, dv=128, seed=0):
    from omegalax_amd.layer import GDNConfig, GDNParams
    rng = np.random.default_rng(seed)
    cfg = GDNConfig(hidden_size=D, num_k_heads=Hk, head_k_dim=dk, num_v_heads=Hv, head_v_dim=dv)
    C = cfg.conv_dim
    t = lambda s, *shape: torch.from_numpy((s * rng.standard_normal(shape)).astype(np.float32))
    p = GDNParams(in_proj_qkv=t(0.1, C, D).bfloat16(), in_proj_z=t(0.1, Hv * dv, D).bfloat16(),
                  in_proj_b=t(0.1, Hv, D).bfloat16(), in_proj_a=t(0.1, Hv, D).bfloat16(),
                  conv_w=t(0.3, C, 4), dt_bias=torch.from_numpy(rng.uniform(-2, 0, Hv).astype(np.float32)),
                  A_log=torch.from_numpy(np.log(rng.uniform(1, 16, Hv)).astype(np.float32)),
                  norm_w=1 + t(0.1, dv), out_proj=t(0.05, D, Hv * dv).bfloat16())
    return cfg, p.to("cuda")


def np_(t):
    return t.detach().float().cpu().numpy()


def test_layer_forward_matches_oracle_with_mask():
    import torch.nn.functional as F
    from omegalax_amd.layer import gated_deltanet_forward
    say("layer module forward B=2 T=100")
    cfg, p = make()
    B, T = 2, 100
    g = torch.Generator().manual_seed(1)
    hidden = torch.randn(B, T, cfg.hidden_size, generator=g).bfloat16().cuda()
    mask = torch.ones(B, T, dtype=torch.int32)
    mask[1, 80:] = 0  # right padding on row 1
    mask = mask.cuda()
    out = gated_deltanet_forward(p, cfg, hidden, mask)
    torch.cuda.synchronize()
    # the oracle from the same bf16 projection outputs
    h = hidden * mask[:, :, None].to(hidden.dtype)
    mixed, z, a, b = (F.linear(h, w) for w in (p.in_proj_qkv, p.in_proj_z, p.in_proj_a, p.in_proj_b))
    ref_n, _, _ = O.gdn_prefill_layer(np_(mixed), np_(z).reshape(B, T, cfg.num_v_heads, cfg.head_v_dim),
                                      np_(a), np_(b), np_(p.conv_w), np_(p.A_log), np_(p.dt_bias),
                                      np_(p.norm_w), Hk=cfg.num_k_heads, dk=cfg.head_k_dim,
                                      Hv=cfg.num_v_heads, dv=cfg.head_v_dim)
    ref = np.asarray(ref_n, np.float64).reshape(B, T, -1) @ np_(p.out_proj).astype(np.float64).T
    assert rel(np_(out), ref) < BF16_TOL


def oracle_rows(p, cfg, h_TD):
    """The oracle's layer (bf16 rounding points) on one sequence's bf16 projection
    outputs: returns (out [T, D] fp64, final state, conv state)."""
    import torch.nn.functional as F
    h = h_TD[None]
    T = h.shape[1]
    mixed, z, a, b = (F.linear(h, w) for w in (p.in_proj_qkv, p.in_proj_z, p.in_proj_a, p.in_proj_b))
    n, S, conv = O.gdn_prefill_layer(np_(mixed), np_(z).reshape(1, T, cfg.num_v_heads, cfg.head_v_dim),
                                     np_(a), np_(b), np_(p.conv_w), np_(p.A_log), np_(p.dt_bias),
                                     np_(p.norm_w), Hk=cfg.num_k_heads, dk=cfg.head_k_dim,
                                     Hv=cfg.num_v_heads, dv=cfg.head_v_dim)
    return np.asarray(n, np.float64)[0] @ np_(p.out_proj).astype(np.float64).T, S, conv


def oracle_decode(p, cfg, h_BD, conv, S):
    import torch.nn.functional as F
    mixed, z, a, b = (F.linear(h_BD, w) for w in (p.in_proj_qkv, p.in_proj_z, p.in_proj_a, p.in_proj_b))
    n, conv, S = O.gdn_decode_step(np_(mixed), np_(z).reshape(h_BD.shape[0], cfg.num_v_heads, -1),
                                   np_(a), np_(b), np_(p.conv_w), np_(p.A_log), np_(p.dt_bias),
                                   np_(p.norm_w), conv, S, Hk=cfg.num_k_heads, dk=cfg.head_k_dim,
                                   Hv=cfg.num_v_heads, dv=cfg.head_v_dim)
    return np.asarray(n, np.float64) @ np_(p.out_proj).astype(np.float64).T, conv, S


def test_packed_documents_equal_separate_runs():
    from omegalax_amd.layer import gated_deltanet_forward
    say("layer module packed documents")
    cfg, p = make(seed=2)
    B, T = 2, 48
    g = torch.Generator().manual_seed(3)
    hidden = torch.randn(B, T, cfg.hidden_size, generator=g).bfloat16().cuda()
    seg = torch.zeros(B, T, dtype=torch.int32)
    docs = [(0, 0, 20), (0, 20, 48), (1, 0, 7), (1, 7, 40), (1, 40, 48)]
    for i, (b, s, e) in enumerate(docs):
        seg[b, s:e] = i + 1
    out = gated_deltanet_forward(p, cfg, hidden, segment_ids_BT=seg.cuda())
    torch.cuda.synchronize()
    for b, s, e in docs:
        alone = gated_deltanet_forward(p, cfg, hidden[b:b + 1, s:e].contiguous())
        torch.cuda.synchronize()
        assert rel(np_(out[b, s:e]), np_(alone[0])) < BF16_TOL, (b, s, e)
        ref, _, _ = oracle_rows(p, cfg, hidden[b, s:e])
        assert rel(np_(out[b, s:e]), ref) < BF16_TOL, (b, s, e)


def test_right_padded_prefill_cache_then_decode_equals_full_prefill():
    from omegalax_amd.layer import (gated_deltanet_decode, gated_deltanet_forward,
                                    gated_deltanet_prefill_cache, make_gdn_cache)
    say("layer module cache: right-padded prefill + decode")
    cfg, p = make(seed=4)
    B, T, steps = 3, 40, 5
    lengths = torch.tensor([40, 23, 1], dtype=torch.int32)
    g = torch.Generator().manual_seed(5)
    full = torch.randn(B, T + steps, cfg.hidden_size, generator=g).bfloat16().cuda()
    # the prompt batch: row b's real tokens then padding
    prompt = torch.zeros(B, T, cfg.hidden_size, dtype=torch.bfloat16, device="cuda")
    for b in range(B):
        prompt[b, :lengths[b]] = full[b, :lengths[b]]
    cache = make_gdn_cache(cfg, 1, B)[0]
    out_p = gated_deltanet_prefill_cache(p, cfg, prompt, cache, lengths.cuda())
    outs = []
    for s in range(steps):
        tok = torch.stack([full[b, int(lengths[b]) + s] for b in range(B)])
        outs.append(gated_deltanet_decode(p, cfg, tok, cache))
    torch.cuda.synchronize()
    assert cache.lengths.tolist() == (lengths + steps).tolist()
    for b in range(B):
        n = int(lengths[b])
        ref = gated_deltanet_forward(p, cfg, full[b:b + 1, :n + steps].contiguous())
        torch.cuda.synchronize()
        assert rel(np_(out_p[b, :n]), np_(ref[0, :n])) < BF16_TOL, b
        if n < T:
            assert float(out_p[b, n:].abs().max()) == 0.0  # padded positions
        for s in range(steps):
            assert rel(np_(outs[s][b]), np_(ref[0, n + s])) < BF16_TOL, (b, s)
        # the oracle: prefill of the row's real tokens, then its decode steps
        o_ref, S, conv = oracle_rows(p, cfg, full[b, :n])
        assert rel(np_(out_p[b, :n]), o_ref) < BF16_TOL, b
        for s in range(steps):
            o_ref, conv, S = oracle_decode(p, cfg, full[b:b + 1, n + s], conv, S)
            assert rel(np_(outs[s][b]), o_ref[0]) < BF16_TOL, (b, s)
        assert rel(np_(cache.recurrent_state[b]), S[0]) < 1e-3, b
        assert np.array_equal(np_(cache.conv_state[b]), conv[0]), b
