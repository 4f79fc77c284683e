"""Write golden vectors for the GDN oracle from transformers' torch functions.

The reference (omegalax, JAX) cannot run in this container (JAX absent) and its
own tests hold no GDN fixtures.  Its parity tests treat transformers' Qwen3.5
torch implementation as ground truth (tests/test_qwen3_5_smoke.py:135-178), so
the fixtures here come from those third-party functions
(transformers/models/qwen3_5/modeling_qwen3_5.py):
  torch_chunk_gated_delta_rule, torch_recurrent_gated_delta_rule,
  causal_conv1d_fn, causal_conv1d_update, Qwen3_5RMSNormGated, l2norm.
All in float32 on the CPU.  The layer fixtures (``layer_*.npz``) run the whole
``Qwen3_5GatedDeltaNet`` module (projections, conv, gates, GQA, chunked rule, gated
norm, out_proj) with a padding mask, and its cached decode (``DynamicCache``:
prefill, then single-token steps through causal_conv1d_update and
torch_recurrent_gated_delta_rule).  In float32 HF's module computes what
deltanet.py:226-306 computes (its gated norm's casts are then identities), so these
pin the layer wiring: which channels are q, k and v, a -> g and b -> beta, and which
z a norm row pairs with.  Run once here (transformers 5.15.0); the .npz files are
committed and the tests read only those.

    python tests/golden/make_golden.py
"""
from __future__ import annotations

import os

import numpy as np
import torch
from transformers.models.qwen3_5 import modeling_qwen3_5 as hf

HERE = os.path.dirname(os.path.abspath(__file__))


def _g_beta(rng, B, T, H):
    b = rng.standard_normal((B, T, H)).astype(np.float32)
    a = rng.standard_normal((B, T, H)).astype(np.float32)
    A_log = rng.uniform(np.log(1.0), np.log(16.0), H).astype(np.float32)
    dt_bias = rng.uniform(-2.0, 0.0, H).astype(np.float32)
    beta = 1.0 / (1.0 + np.exp(-b.astype(np.float64)))
    g = -np.exp(A_log.astype(np.float64)) * np.logaddexp(a + dt_bias, 0.0)
    return g.astype(np.float32), beta.astype(np.float32)


def chunk_case(name, seed, B, T, Hk, H, dk, dv, C, with_s0):
    rng = np.random.default_rng(seed)
    q = rng.standard_normal((B, T, Hk, dk)).astype(np.float32)
    k = rng.standard_normal((B, T, Hk, dk)).astype(np.float32)
    v = rng.standard_normal((B, T, H, dv)).astype(np.float32)
    g, beta = _g_beta(rng, B, T, H)
    s0 = (0.1 * rng.standard_normal((B, H, dk, dv))).astype(np.float32) if with_s0 else None
    rep = H // Hk
    qt = torch.from_numpy(q).repeat_interleave(rep, dim=2)
    kt = torch.from_numpy(k).repeat_interleave(rep, dim=2)
    o, S = hf.torch_chunk_gated_delta_rule(
        qt, kt, torch.from_numpy(v), g=torch.from_numpy(g), beta=torch.from_numpy(beta),
        chunk_size=C, initial_state=None if s0 is None else torch.from_numpy(s0),
        output_final_state=True, use_qk_l2norm_in_kernel=True)
    out = dict(q=q, k=k, v=v, g=g, beta=beta, chunk_size=np.int64(C), o=o.numpy(), S=S.numpy())
    if s0 is not None:
        out["S0"] = s0
    np.savez_compressed(os.path.join(HERE, f"{name}.npz"), **out)


def recurrent_case(name, seed, B, T, Hk, H, dk, dv):
    rng = np.random.default_rng(seed)
    q = rng.standard_normal((B, T, Hk, dk)).astype(np.float32)
    k = rng.standard_normal((B, T, Hk, dk)).astype(np.float32)
    v = rng.standard_normal((B, T, H, dv)).astype(np.float32)
    g, beta = _g_beta(rng, B, T, H)
    s0 = (0.1 * rng.standard_normal((B, H, dk, dv))).astype(np.float32)
    rep = H // Hk
    o, S = hf.torch_recurrent_gated_delta_rule(
        torch.from_numpy(q).repeat_interleave(rep, dim=2),
        torch.from_numpy(k).repeat_interleave(rep, dim=2),
        torch.from_numpy(v), g=torch.from_numpy(g), beta=torch.from_numpy(beta),
        initial_state=torch.from_numpy(s0.copy()), output_final_state=True,
        use_qk_l2norm_in_kernel=True)
    np.savez_compressed(os.path.join(HERE, f"{name}.npz"), q=q, k=k, v=v, g=g, beta=beta,
                        S0=s0, o=o.numpy(), S=S.numpy())


def conv_case(name, seed, B, T, C, K):
    rng = np.random.default_rng(seed)
    x = rng.standard_normal((B, C, T)).astype(np.float32)
    w = (0.3 * rng.standard_normal((C, K))).astype(np.float32)
    y = hf.causal_conv1d_fn(torch.from_numpy(x), torch.from_numpy(w), None, activation="silu")
    state = rng.standard_normal((B, C, K - 1)).astype(np.float32)
    st = torch.from_numpy(state.copy())
    xt = rng.standard_normal((B, C, 1)).astype(np.float32)
    yu = hf.causal_conv1d_update(torch.from_numpy(xt), st, torch.from_numpy(w), None, "silu")
    np.savez_compressed(os.path.join(HERE, f"{name}.npz"), x=x, w=w, y=y.numpy(),
                        state=state, x_step=xt, y_step=yu.numpy(), state_after=st.numpy())


def norm_case(name, seed, N, D):
    rng = np.random.default_rng(seed)
    x = rng.standard_normal((N, D)).astype(np.float32)
    z = rng.standard_normal((N, D)).astype(np.float32)
    w = (1.0 + 0.1 * rng.standard_normal(D)).astype(np.float32)
    mod = hf.Qwen3_5RMSNormGated(D, eps=1e-6)
    with torch.no_grad():
        mod.weight.copy_(torch.from_numpy(w))
        y = mod(torch.from_numpy(x), torch.from_numpy(z))
    l2 = hf.l2norm(torch.from_numpy(x), dim=-1, eps=1e-6)
    np.savez_compressed(os.path.join(HERE, f"{name}.npz"), x=x, z=z, w=w, y=y.numpy(),
                        l2=l2.numpy())


LAYER_PREFIX = "model.language_model.layers.0.linear_attn."


def layer_case(name, seed, D, Hk, Hv, dk, dv, B, T, pad, T0, steps, save_state):
    """One Qwen3_5GatedDeltaNet layer in fp32: a masked prefill of [B, T] (row 1 has
    ``pad`` masked tokens at the front, row 0 ``pad`` at the back), and an unmasked
    prefill of T0 tokens into a DynamicCache followed by ``steps`` cached decode steps."""
    from transformers.cache_utils import DynamicCache
    from transformers.models.qwen3_5.configuration_qwen3_5 import Qwen3_5TextConfig
    cfg = Qwen3_5TextConfig(hidden_size=D, linear_num_key_heads=Hk, linear_num_value_heads=Hv,
                            linear_key_head_dim=dk, linear_value_head_dim=dv,
                            linear_conv_kernel_dim=4, num_hidden_layers=1,
                            layer_types=["linear_attention"], rms_norm_eps=1e-6, vocab_size=16,
                            intermediate_size=16, num_attention_heads=2, num_key_value_heads=1,
                            head_dim=16)
    rng = np.random.default_rng(seed)
    m = hf.Qwen3_5GatedDeltaNet(cfg, 0).float().eval()
    conv_dim = 2 * Hk * dk + Hv * dv
    n = lambda s, *shape: torch.from_numpy((s * rng.standard_normal(shape)).astype(np.float32))
    params = {
        "in_proj_qkv.weight": n(0.25, conv_dim, D), "in_proj_z.weight": n(0.25, Hv * dv, D),
        "in_proj_b.weight": n(0.25, Hv, D), "in_proj_a.weight": n(0.25, Hv, D),
        "conv1d.weight": n(0.3, conv_dim, 1, 4),
        "dt_bias": torch.from_numpy(rng.uniform(-2.0, 0.0, Hv).astype(np.float32)),
        "A_log": torch.from_numpy(np.log(rng.uniform(1.0, 16.0, Hv)).astype(np.float32)),
        "norm.weight": 1.0 + n(0.1, dv), "out_proj.weight": n(0.25 / np.sqrt(Hv), D, Hv * dv),
    }
    with torch.no_grad():
        sd = m.state_dict()
        for k_, v_ in params.items():
            assert sd[k_].shape == v_.shape, (k_, sd[k_].shape, v_.shape)
            sd[k_].copy_(v_)
    hidden = n(1.0, B, T, D)
    mask = torch.ones(B, T, dtype=torch.int64)
    if pad:
        mask[0, T - pad:] = 0
        if B > 1:
            mask[1, :pad] = 0
    hid0 = n(1.0, B, T0, D)
    hid_dec = n(1.0, steps, B, 1, D)
    with torch.no_grad():
        out = m(hidden, attention_mask=mask)
        cache = DynamicCache(config=cfg)
        out0 = m(hid0, cache_params=cache)
        outs = [m(hid_dec[s], cache_params=cache) for s in range(steps)]
    fx = {LAYER_PREFIX + k_: v_.numpy() for k_, v_ in params.items()}
    fx.update(dims=np.array([D, Hk, Hv, dk, dv], np.int64), hidden=hidden.numpy(),
              mask=mask.numpy().astype(np.int32), out=out.numpy(), hidden_prefill=hid0.numpy(),
              out_prefill=out0.numpy(), hidden_decode=hid_dec[:, :, 0].numpy(),
              out_decode=torch.stack(outs)[:, :, 0].numpy())
    if save_state:
        fx["state_after_decode"] = cache.layers[0].recurrent_states[0].numpy()
    np.savez_compressed(os.path.join(HERE, f"{name}.npz"), **fx)


def main():
    torch.set_num_threads(4)
    chunk_case("chunk_gqa_pad_c16", 11, B=1, T=100, Hk=1, H=2, dk=16, dv=32, C=16, with_s0=False)
    chunk_case("chunk_gqa_pad_c64_s0", 12, B=2, T=100, Hk=2, H=4, dk=16, dv=32, C=64,
               with_s0=True)
    chunk_case("chunk_d64_c64", 13, B=1, T=96, Hk=1, H=2, dk=64, dv=64, C=64, with_s0=True)
    recurrent_case("recurrent_gqa_s0", 21, B=2, T=5, Hk=2, H=4, dk=16, dv=32)
    conv_case("conv_k4", 31, B=2, T=20, C=24, K=4)
    norm_case("gated_norm", 41, N=16, D=32)
    layer_case("layer_d128", 51, D=16, Hk=2, Hv=4, dk=128, dv=128, B=2, T=100, pad=9, T0=67,
               steps=3, save_state=False)
    layer_case("layer_d64", 52, D=16, Hk=2, Hv=4, dk=64, dv=64, B=2, T=100, pad=0, T0=130,
               steps=3, save_state=True)
    # the reference's smoke layout (config.py:94-101): dk=16, dv=32
    layer_case("layer_smoke_d16", 53, D=16, Hk=2, Hv=4, dk=16, dv=32, B=2, T=33, pad=5, T0=16,
               steps=4, save_state=True)


if __name__ == "__main__":
    main()
