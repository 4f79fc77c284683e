"""Write golden vectors for the GDN oracle from transformers' torch functions.

The reference (omegalax, JAX) cannot run in this container (JAX absent) and its
own tests hold no GDN fixtures.  Its parity tests treat transformers' Qwen3.5
torch implementation as ground truth (tests/test_qwen3_5_smoke.py:135-178), so
the fixtures here come from those third-party functions
(transformers/models/qwen3_5/modeling_qwen3_5.py):
  torch_chunk_gated_delta_rule, torch_recurrent_gated_delta_rule,
  causal_conv1d_fn, causal_conv1d_update, Qwen3_5RMSNormGated, l2norm.
All in float32 on the CPU.  Run once here (transformers 5.15.0); the .npz files
are committed and the tests read only those.

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


def main():
    torch.set_num_threads(4)
    chunk_case("chunk_gqa_pad_c16", 11, B=1, T=100, Hk=1, H=2, dk=16, dv=32, C=16, with_s0=False)
    chunk_case("chunk_gqa_pad_c64_s0", 12, B=2, T=100, Hk=2, H=4, dk=16, dv=32, C=64,
               with_s0=True)
    chunk_case("chunk_d64_c64", 13, B=1, T=96, Hk=1, H=2, dk=64, dv=64, C=64, with_s0=True)
    recurrent_case("recurrent_gqa_s0", 21, B=2, T=5, Hk=2, H=4, dk=16, dv=32)
    conv_case("conv_k4", 31, B=2, T=20, C=24, K=4)
    norm_case("gated_norm", 41, N=16, D=32)


if __name__ == "__main__":
    main()
