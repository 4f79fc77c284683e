"""Seeded synthetic workloads for the GDN path (benchmark and test inputs).

Inputs are drawn with ``numpy.random.default_rng(1000 + config_index)`` in
float32 and rounded to bf16 where the workload says bf16, so the CPU oracle and
the GPU path see bit-identical values.  Arrays are returned as float32 numpy
arrays; ``to_device`` makes torch tensors of the requested dtypes.

Configs (head layout of Qwen3.5: 16 key heads, 32 or 64 value heads, d=128):
  C0 core fp32  B=2 T=512 H=4 d=64                        (parity config)
  C1 layer      B=4 T=4096 D=2048 Hk=16 Hv=32 d=128       (prefill bench)
  C2 decode     B in {1,8,64,256} Hk=16 Hv=32 d=128       (decode bench)
  C3 varlen     T=32768 in 8 packed sequences, S0 given   (layer, B=1)
  C4 core long  B=1 T=65536 Hk=16 Hv=64 d=128, e^g in [0.9, 0.9999]
"""
from __future__ import annotations

import numpy as np

from ._bf16 import round_bf16

CONV_K = 4


def _gates(rng, shape, H):
    """a, b ~ N(0,1); A_log ~ U(log 1, log 16); dt_bias ~ U(-2, 0) (deltanet.py:248-250)."""
    b = rng.standard_normal(shape).astype(np.float32)
    a = rng.standard_normal(shape).astype(np.float32)
    A_log = rng.uniform(np.log(1.0), np.log(16.0), H).astype(np.float32)
    dt_bias = rng.uniform(-2.0, 0.0, H).astype(np.float32)
    return a, b, A_log, dt_bias


def gates_f32(a, b, A_log, dt_bias, bf16_beta=True):
    """g = -exp(A_log) softplus(a + dt_bias) and beta = sigmoid(b), computed in float64."""
    beta = 1.0 / (1.0 + np.exp(-b.astype(np.float64)))
    if bf16_beta:
        beta = round_bf16(beta)
    g = -np.exp(A_log.astype(np.float64)) * np.logaddexp(a.astype(np.float64) + dt_bias, 0.0)
    return g.astype(np.float32), np.asarray(beta, np.float32)


def core_c0(seed=1000):
    """C0: chunked rule on fp32 inputs; q, k pre-normalised per head."""
    rng = np.random.default_rng(seed)
    B, T, H, d = 2, 512, 4, 64
    q = rng.standard_normal((B, T, H, d)).astype(np.float32)
    k = rng.standard_normal((B, T, H, d)).astype(np.float32)
    v = rng.standard_normal((B, T, H, d)).astype(np.float32)
    q /= np.linalg.norm(q, axis=-1, keepdims=True)
    k /= np.linalg.norm(k, axis=-1, keepdims=True)
    a, b, A_log, dt_bias = _gates(rng, (B, T, H), H)
    g, beta = gates_f32(a, b, A_log, dt_bias, bf16_beta=False)
    return dict(q=q, k=k, v=v, g=g, beta=beta)


def core_c4(T=65536, Hk=16, Hv=64, d=128, seed=1004):
    """C4: long-memory core inputs, bf16 q/k/v, e^g ~ U(0.9, 0.9999), beta = sigmoid(N(0,1))."""
    rng = np.random.default_rng(seed)
    B = 1
    q = round_bf16(rng.standard_normal((B, T, Hk, d), dtype=np.float32))
    k = round_bf16(rng.standard_normal((B, T, Hk, d), dtype=np.float32))
    v = round_bf16(rng.standard_normal((B, T, Hv, d), dtype=np.float32))
    g = np.log(rng.uniform(0.9, 0.9999, (B, T, Hv))).astype(np.float32)
    beta = round_bf16(1.0 / (1.0 + np.exp(-rng.standard_normal((B, T, Hv)))))
    return dict(q=q, k=k, v=v, g=g, beta=beta)


def layer_params(rng, Hk, Hv, dk, dv, K=CONV_K):
    conv_dim = 2 * Hk * dk + Hv * dv
    conv_w = (0.1 * rng.standard_normal((conv_dim, K))).astype(np.float32)
    A_log = rng.uniform(np.log(1.0), np.log(16.0), Hv).astype(np.float32)
    dt_bias = rng.uniform(-2.0, 0.0, Hv).astype(np.float32)
    norm_w = np.ones(dv, np.float32)
    return dict(conv_w=conv_w, A_log=A_log, dt_bias=dt_bias, norm_w=norm_w)


def module_params(D, Hk=16, Hv=32, dk=128, dv=128, seed=1001, K=CONV_K):
    """GatedDeltaNet parameters at hidden size D (config C1's draws): the projection
    weights N(0, 0.02) rounded to bf16, the conv, gate and norm parameters as layer_params.
    Returns numpy arrays keyed by the GDNParams field names."""
    rng = np.random.default_rng(seed)
    conv_dim = 2 * Hk * dk + Hv * dv
    w = lambda n, m: round_bf16(0.02 * rng.standard_normal((n, m), dtype=np.float32))
    p = dict(in_proj_qkv=w(conv_dim, D), in_proj_z=w(Hv * dv, D), in_proj_b=w(Hv, D),
             in_proj_a=w(Hv, D), out_proj=w(D, Hv * dv))
    p.update(layer_params(rng, Hk, Hv, dk, dv, K))
    return p


def layer_inputs(B, T, Hk=16, Hv=32, dk=128, dv=128, seed=1001, act_scale=1.0):
    """Projection outputs for the layer-level prefill (C1 layout by default).

    mixed_qkv/z/a/b are bf16 draws standing in for the bf16 projection outputs;
    ``act_scale`` scales mixed_qkv and z.
    """
    rng = np.random.default_rng(seed)
    conv_dim = 2 * Hk * dk + Hv * dv
    p = layer_params(rng, Hk, Hv, dk, dv)
    x = round_bf16(act_scale * rng.standard_normal((B, T, conv_dim), dtype=np.float32))
    z = round_bf16(act_scale * rng.standard_normal((B, T, Hv, dv), dtype=np.float32))
    a = round_bf16(rng.standard_normal((B, T, Hv), dtype=np.float32))
    b = round_bf16(rng.standard_normal((B, T, Hv), dtype=np.float32))
    return dict(mixed_qkv=x, z=z, a=a, b=b, **p)


def varlen_lengths(total=32768, n=8, min_len=256, seed=1003):
    """Dirichlet(1^n) split of total - n*min_len, largest-remainder integerised, + min_len."""
    rng = np.random.default_rng(seed)
    w = rng.dirichlet(np.ones(n))
    free = total - n * min_len
    raw = w * free
    base = np.floor(raw).astype(np.int64)
    rem = free - int(base.sum())
    order = np.argsort(-(raw - base), kind="stable")
    base[order[:rem]] += 1
    lens = base + min_len
    assert int(lens.sum()) == total
    return lens


def varlen_inputs(total=32768, n=8, Hk=16, Hv=32, dk=128, dv=128, seed=1003):
    lens = varlen_lengths(total, n, seed=seed)
    cu = np.concatenate([[0], np.cumsum(lens)]).astype(np.int32)
    d = layer_inputs(1, total, Hk, Hv, dk, dv, seed=seed + 7)
    rng = np.random.default_rng(seed + 11)
    d["initial_state"] = (0.02 * rng.standard_normal((n, Hv, dk, dv), dtype=np.float32))
    d["cu_seqlens"] = cu
    return d


def decode_inputs(B, Hk=16, Hv=32, dk=128, dv=128, seed=1002, K=CONV_K):
    """C2: one token per sequence plus conv cache and recurrent state."""
    rng = np.random.default_rng(seed)
    conv_dim = 2 * Hk * dk + Hv * dv
    p = layer_params(rng, Hk, Hv, dk, dv, K)
    x = round_bf16(rng.standard_normal((B, conv_dim), dtype=np.float32))
    z = round_bf16(rng.standard_normal((B, Hv, dv), dtype=np.float32))
    a = round_bf16(rng.standard_normal((B, Hv), dtype=np.float32))
    b = round_bf16(rng.standard_normal((B, Hv), dtype=np.float32))
    conv_state = round_bf16(rng.standard_normal((B, conv_dim, K - 1), dtype=np.float32))
    state = (0.02 * rng.standard_normal((B, Hv, dk, dv), dtype=np.float32))
    return dict(mixed_qkv=x, z=z, a=a, b=b, conv_state=conv_state, state=state, **p)


# dtype of each named array on the device
DEVICE_DTYPES = {
    "mixed_qkv": "bf16", "z": "bf16", "a": "bf16", "b": "bf16", "conv_state": "bf16",
    "state": "f32", "initial_state": "f32", "conv_w": "f32", "A_log": "f32", "dt_bias": "f32",
    "norm_w": "f32", "g": "f32", "beta": "f32", "cu_seqlens": "i32",
}


def to_device(arrs, device="cuda", qkv_dtype="bf16"):
    """numpy dict -> torch tensors on ``device`` (bf16/f32/i32 per DEVICE_DTYPES)."""
    import torch
    m = {"bf16": torch.bfloat16, "f32": torch.float32, "i32": torch.int32}
    out = {}
    for k_, v_ in arrs.items():
        dt = DEVICE_DTYPES.get(k_, qkv_dtype)
        out[k_] = torch.from_numpy(np.ascontiguousarray(v_)).to(device=device, dtype=m[dt])
    return out
