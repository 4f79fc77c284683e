"""JAX functions over the XLA FFI handlers of libomx_gdn_xla.so (gdn_xla_ffi.cc).

Drop-in for the reference's call of ``chunk_gated_delta_rule`` inside ``_full_deltanet``
(omegalax/models/qwen3_5/deltanet.py:281), with a ``jax.custom_vjp`` so that the
reference's ``value_and_grad`` training step (trainers/vlm.py:157-195) differentiates
through the HIP backward; and the layer-level prefill (deltanet.py:243-293) and a cached
decode step.  Workspaces are extra results sized by the library's own queries, so XLA
allocates them with the call's other buffers.  Importing this module needs JAX.
"""
from __future__ import annotations

import ctypes
import functools
import os

import jax
import jax.numpy as jnp

from .. import _lib

_XLA_LIB = os.path.join(os.path.dirname(_lib.LIB_PATH), "libomx_gdn_xla.so")
_TARGETS = ("OmxGdnChunkFwd", "OmxGdnChunkBwd", "OmxGdnPrefill", "OmxGdnPrefillBwd",
            "OmxGdnDecodeStep", "OmxGdnAbProj")


@functools.lru_cache(maxsize=None)
def register() -> None:
    """Register every handler with XLA for the ROCm platform (once)."""
    if not os.path.exists(_XLA_LIB):
        raise RuntimeError(f"{_XLA_LIB} is missing: build it with `python -m omegalax_amd.build` "
                           "in an environment with JAX")
    lib = ctypes.CDLL(_XLA_LIB)
    for name in _TARGETS:
        jax.ffi.register_ffi_target(name, jax.ffi.pycapsule(getattr(lib, name)), platform="ROCM")


def _code(x):
    return _lib.BF16 if x.dtype == jnp.bfloat16 else _lib.F32


def _chunk_fwd(q, k, v, g, beta):
    register()
    B, T, Hk, A = q.shape
    H, U = v.shape[2], v.shape[3]
    ws = _lib.lib().omx_gdn_chunk_fwd_workspace_size(B, T, Hk, H, A, U, B, _code(q))
    call = jax.ffi.ffi_call("OmxGdnChunkFwd",
                            (jax.ShapeDtypeStruct((B, T, H, U), jnp.float32),
                             jax.ShapeDtypeStruct((0,), jnp.float32),
                             jax.ShapeDtypeStruct((ws,), jnp.uint8)),
                            vmap_method="sequential")
    o, _, _ = call(q, k, v, g.astype(jnp.float32), beta.astype(jnp.float32),
                   jnp.zeros((0,), jnp.float32), chunk_size=64)
    return o


@jax.custom_vjp
def chunk_gated_delta_rule(q_BTHA, k_BTHA, v_BTHU, g_BTH, beta_BTH):
    """deltanet.py:53-153 on the MI355X kernels (chunk size 64); returns fp32 o."""
    return _chunk_fwd(q_BTHA, k_BTHA, v_BTHU, g_BTH, beta_BTH)


def _vjp_fwd(q, k, v, g, beta):
    return _chunk_fwd(q, k, v, g, beta), (q, k, v, g, beta)


def _vjp_bwd(res, do):
    q, k, v, g, beta = res
    B, T, Hk, A = q.shape
    H, U = v.shape[2], v.shape[3]
    ws = _lib.lib().omx_gdn_chunk_bwd_workspace_size(B, T, Hk, H, A, U, B, _code(q))
    call = jax.ffi.ffi_call("OmxGdnChunkBwd",
                            (jax.ShapeDtypeStruct(q.shape, q.dtype),
                             jax.ShapeDtypeStruct(k.shape, k.dtype),
                             jax.ShapeDtypeStruct(v.shape, v.dtype),
                             jax.ShapeDtypeStruct(g.shape, jnp.float32),
                             jax.ShapeDtypeStruct(beta.shape, jnp.float32),
                             jax.ShapeDtypeStruct((ws,), jnp.uint8)),
                            vmap_method="sequential")
    dq, dk, dv, dg, dbeta, _ = call(q, k, v, g.astype(jnp.float32), beta.astype(jnp.float32),
                                    do.astype(jnp.float32), chunk_size=64)
    return dq, dk, dv, dg.astype(g.dtype), dbeta.astype(beta.dtype)


chunk_gated_delta_rule.defvjp(_vjp_fwd, _vjp_bwd)


def gdn_prefill(mixed_qkv, z, a, b, conv_w, A_log, dt_bias, norm_w, *, num_k_heads, head_k_dim,
                num_v_heads, head_v_dim, eps=1e-6):
    """deltanet.py:243-293: projection outputs (bf16) -> gated-norm output [B, T, Hv*dv]."""
    register()
    B, T, _ = mixed_qkv.shape
    ws = _lib.lib().omx_gdn_prefill_workspace_size(B, T, num_k_heads, num_v_heads, head_k_dim,
                                                   head_v_dim, B)
    call = jax.ffi.ffi_call("OmxGdnPrefill",
                            (jax.ShapeDtypeStruct((B, T, num_v_heads * head_v_dim), jnp.bfloat16),
                             jax.ShapeDtypeStruct((ws,), jnp.uint8)),
                            vmap_method="sequential")
    out, _ = call(mixed_qkv, z, a, b, conv_w.astype(jnp.float32), A_log.astype(jnp.float32),
                  dt_bias.astype(jnp.float32), norm_w.astype(jnp.float32),
                  num_k_heads=num_k_heads, head_k_dim=head_k_dim, num_v_heads=num_v_heads,
                  head_v_dim=head_v_dim, eps=float(eps))
    return out


def gdn_decode_step(mixed_qkv, z, a, b, conv_w, A_log, dt_bias, norm_w, conv_state, state, *,
                    num_k_heads, head_k_dim, num_v_heads, head_v_dim, eps=1e-6):
    """One cached decode step; returns (out, conv_state, state), the caches donated and
    updated in place."""
    register()
    B = mixed_qkv.shape[0]
    call = jax.ffi.ffi_call("OmxGdnDecodeStep",
                            (jax.ShapeDtypeStruct((B, num_v_heads * head_v_dim), jnp.bfloat16),
                             jax.ShapeDtypeStruct(conv_state.shape, conv_state.dtype),
                             jax.ShapeDtypeStruct(state.shape, jnp.float32)),
                            input_output_aliases={8: 1, 9: 2}, vmap_method="sequential")
    return call(mixed_qkv, z, a, b, conv_w.astype(jnp.float32), A_log.astype(jnp.float32),
                dt_bias.astype(jnp.float32), norm_w.astype(jnp.float32), conv_state, state,
                num_k_heads=num_k_heads, head_k_dim=head_k_dim, num_v_heads=num_v_heads,
                head_v_dim=head_v_dim, eps=float(eps))


def gdn_ab_projections(x, w_a, w_b):
    """(a, b) = (in_proj_a(x), in_proj_b(x)) of deltanet.py:240-241 in one pass over x:
    x [..., D] bf16, w_a / w_b [Hv, D] bf16 (the [out, in] weight layout) -> [..., Hv] bf16.
    Forward only; under jax.grad the reference's own nnx.Linear calls differentiate."""
    register()
    out = jax.ShapeDtypeStruct((*x.shape[:-1], w_a.shape[0]), jnp.bfloat16)
    call = jax.ffi.ffi_call("OmxGdnAbProj", (out, out), vmap_method="sequential")
    return call(x.astype(jnp.bfloat16), w_a.astype(jnp.bfloat16), w_b.astype(jnp.bfloat16))

