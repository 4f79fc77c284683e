"""GatedDeltaNet layer forward and cached decode on the MI355X kernels.

Mirrors ``GatedDeltaNet.__call__`` (omegalax/models/qwen3_5/deltanet.py:226-306):
the four input projections and the output projection are plain bf16 GEMMs
(torch.nn.functional.linear, i.e. hipBLASLt), and everything between them --
conv + SiLU, gates, L2 norms, GQA, the chunked rule and the gated RMSNorm -- is
one ``gdn_prefill`` call.  Decode runs ``gdn_decode_step`` on a per-layer cache
(conv window + recurrent state), which the reference does not have
(model.py:324-326, text/api.py:128-131); its semantics are those of the
chunked path: a step after prefill(x[:n]) equals prefill(x[:n+1])[n].

Parameters load from Hugging Face Qwen3.5 checkpoints with the reference's key
mapping (loader.py:173-190, 226-307): linear weights stay in the [out, in] layout
F.linear takes, conv1d.weight [C, 1, K] is squeezed to [C, K].
"""
from __future__ import annotations

from dataclasses import dataclass, field
from typing import Mapping

import torch
import torch.nn.functional as F

from .deltanet import ab_proj_supported, gdn_ab_projections, gdn_decode_step, gdn_prefill
from .segments import lengths_to_cu_seqlens, segment_ids_to_cu_seqlens

_PREFIX = "model.language_model.layers."


@dataclass
class GDNConfig:
    """The GDN fields of Qwen3_5TextConfig (config.py:48-53, rms_norm_eps :38)."""
    hidden_size: int
    num_k_heads: int
    head_k_dim: int
    num_v_heads: int
    head_v_dim: int
    conv_kernel: int = 4
    rms_norm_eps: float = 1e-6

    @property
    def conv_dim(self) -> int:
        return 2 * self.num_k_heads * self.head_k_dim + self.num_v_heads * self.head_v_dim

    def dims(self) -> dict:
        return dict(num_k_heads=self.num_k_heads, head_k_dim=self.head_k_dim,
                    num_v_heads=self.num_v_heads, head_v_dim=self.head_v_dim)


@dataclass
class GDNParams:
    """One linear-attention layer's parameters (deltanet.py:174-223)."""
    in_proj_qkv: torch.Tensor   # [conv_dim, D] bf16
    in_proj_z: torch.Tensor     # [Hv*dv, D] bf16
    in_proj_b: torch.Tensor     # [Hv, D] bf16
    in_proj_a: torch.Tensor     # [Hv, D] bf16
    conv_w: torch.Tensor        # [conv_dim, K] fp32
    dt_bias: torch.Tensor       # [Hv] fp32
    A_log: torch.Tensor         # [Hv] fp32
    norm_w: torch.Tensor        # [dv] fp32
    out_proj: torch.Tensor      # [D, Hv*dv] bf16

    def to(self, device) -> "GDNParams":
        return GDNParams(**{k: getattr(self, k).to(device) for k in self.__dataclass_fields__})


def gdn_params_from_hf(tensors: Mapping[str, torch.Tensor], layer_idx: int,
                       prefix: str = _PREFIX) -> GDNParams:
    """Layer ``layer_idx``'s GDN parameters from Hugging Face checkpoint tensors
    (e.g. ``safetensors.torch.load_file``), keys as at loader.py:173-190, 226-234."""
    base = f"{prefix}{layer_idx}.linear_attn."

    def get(name):
        key = base + name
        if key not in tensors:
            raise KeyError(f"checkpoint has no {key}")
        return tensors[key]

    conv = get("conv1d.weight")
    if conv.dim() == 3:  # [C, 1, K] -> [C, K] (loader.py:289)
        conv = conv.squeeze(1)
    lin = lambda name: get(name).to(torch.bfloat16).contiguous()
    f32 = lambda name: get(name).to(torch.float32).contiguous()
    return GDNParams(in_proj_qkv=lin("in_proj_qkv.weight"), in_proj_z=lin("in_proj_z.weight"),
                     in_proj_b=lin("in_proj_b.weight"), in_proj_a=lin("in_proj_a.weight"),
                     conv_w=conv.to(torch.float32).contiguous(), dt_bias=f32("dt_bias"),
                     A_log=f32("A_log"), norm_w=f32("norm.weight"), out_proj=lin("out_proj.weight"))


def gdn_params_to_hf(params: GDNParams, layer_idx: int, prefix: str = _PREFIX) -> dict:
    """The inverse of gdn_params_from_hf (params.py:136-173 write the same keys)."""
    base = f"{prefix}{layer_idx}.linear_attn."
    return {base + "in_proj_qkv.weight": params.in_proj_qkv, base + "in_proj_z.weight": params.in_proj_z,
            base + "in_proj_b.weight": params.in_proj_b, base + "in_proj_a.weight": params.in_proj_a,
            base + "conv1d.weight": params.conv_w[:, None, :], base + "dt_bias": params.dt_bias,
            base + "A_log": params.A_log, base + "norm.weight": params.norm_w,
            base + "out_proj.weight": params.out_proj}


def load_gdn_layers(path: str, layer_ids, device="cuda", prefix: str = _PREFIX) -> dict:
    """{layer: GDNParams} from a safetensors file (no pickle)."""
    from safetensors.torch import load_file
    tensors = load_file(path)
    return {i: gdn_params_from_hf(tensors, i, prefix).to(device) for i in layer_ids}


def _projections(params: GDNParams, cfg: GDNConfig, h):
    lead = h.shape[:-1]
    mixed = F.linear(h, params.in_proj_qkv)
    z = F.linear(h, params.in_proj_z).reshape(*lead, cfg.num_v_heads, cfg.head_v_dim)
    # the two gate projections in one pass over h (deltanet.py:240-241); shapes outside the
    # one-pass kernel's limits take the two library GEMMs, as the other projections do
    if ab_proj_supported(h.shape[-1], params.in_proj_a.shape[0]):
        a, b = gdn_ab_projections(h, params.in_proj_a, params.in_proj_b)
    else:
        a, b = F.linear(h, params.in_proj_a), F.linear(h, params.in_proj_b)
    return mixed, z, a, b


def gated_deltanet_forward(params: GDNParams, cfg: GDNConfig, hidden_BTD: torch.Tensor,
                           attention_mask_BT: torch.Tensor | None = None, *,
                           segment_ids_BT: torch.Tensor | None = None,
                           cu_seqlens: torch.Tensor | None = None) -> torch.Tensor:
    """out_BTD of deltanet.py:226-306 (bf16).

    ``attention_mask_BT`` zeroes padded tokens first, as the reference does when
    T > 1 (:227-228).  ``segment_ids_BT`` (packed documents) or ``cu_seqlens`` (B = 1)
    restart the state and the conv window at every sequence start.
    """
    h = hidden_BTD.to(torch.bfloat16)
    if attention_mask_BT is not None and h.shape[1] > 1:
        h = h * attention_mask_BT[:, :, None].to(h.dtype)
    B, T, D = h.shape
    mixed, z, a, b = _projections(params, cfg, h)
    if segment_ids_BT is not None:
        if cu_seqlens is not None:
            raise ValueError("give segment_ids or cu_seqlens, not both")
        cu_seqlens = segment_ids_to_cu_seqlens(segment_ids_BT)
        mixed, z, a, b = (t.reshape(1, B * T, *t.shape[2:]) for t in (mixed, z, a, b))
    out = gdn_prefill(mixed, z, a, b, params.conv_w, params.A_log, params.dt_bias, params.norm_w,
                      eps=cfg.rms_norm_eps, cu_seqlens=cu_seqlens, **cfg.dims())
    out = out.reshape(B, T, -1)
    return F.linear(out, params.out_proj)


@dataclass
class GDNLayerCache:
    """Decode cache of one linear-attention layer: the last K-1 conv inputs and the
    recurrent state, per sequence."""
    conv_state: torch.Tensor       # [B, conv_dim, K-1] bf16
    recurrent_state: torch.Tensor  # [B, Hv, dk, dv] fp32
    lengths: torch.Tensor = field(default=None)  # [B] int32 tokens seen (host bookkeeping)


def make_gdn_cache(cfg: GDNConfig, num_layers: int, batch_size: int, device="cuda") -> list:
    """Zero caches for ``num_layers`` linear-attention layers (the per-layer pattern of
    qwen3/cache.py:12-25, with the GDN state in place of the KV cache)."""
    caches = []
    for _ in range(num_layers):
        caches.append(GDNLayerCache(
            conv_state=torch.zeros((batch_size, cfg.conv_dim, cfg.conv_kernel - 1), dtype=torch.bfloat16,
                                   device=device),
            recurrent_state=torch.zeros((batch_size, cfg.num_v_heads, cfg.head_k_dim, cfg.head_v_dim),
                                        dtype=torch.float32, device=device),
            lengths=torch.zeros(batch_size, dtype=torch.int32, device=device)))
    return caches


def gated_deltanet_prefill_cache(params: GDNParams, cfg: GDNConfig, hidden_BTD: torch.Tensor,
                                 cache: GDNLayerCache, lengths: torch.Tensor | None = None) -> torch.Tensor:
    """Prefill a right-padded batch into ``cache`` and return out_BTD.

    Row b holds ``lengths[b]`` real tokens followed by padding (all T when None).
    The rows' real tokens run as a varlen batch that starts from the cache's state,
    so each row's conv window and state end at its own last token; padded positions
    of the output are zero.
    """
    h = hidden_BTD.to(torch.bfloat16)
    B, T, D = h.shape
    dev = h.device
    if lengths is None:
        lengths = torch.full((B,), T, dtype=torch.int32, device=dev)
    lengths = lengths.to(device=dev, dtype=torch.int32)
    mixed, z, a, b = _projections(params, cfg, h)
    valid = torch.arange(T, device=dev)[None, :] < lengths[:, None].to(torch.int64)  # [B, T]
    idx = torch.nonzero(valid.reshape(-1), as_tuple=False).flatten()
    pack = lambda t: t.reshape(B * T, *t.shape[2:]).index_select(0, idx).unsqueeze(0)
    cu = lengths_to_cu_seqlens(lengths)
    out_p, fs, cs = gdn_prefill(pack(mixed), pack(z), pack(a), pack(b), params.conv_w, params.A_log,
                                params.dt_bias, params.norm_w, eps=cfg.rms_norm_eps, cu_seqlens=cu,
                                initial_state=cache.recurrent_state, conv_state=cache.conv_state,
                                output_final_state=True, **cfg.dims())
    cache.recurrent_state.copy_(fs)
    cache.conv_state.copy_(cs)
    cache.lengths = (cache.lengths + lengths).to(torch.int32)
    out = torch.zeros((B * T, out_p.shape[-1]), dtype=out_p.dtype, device=dev)
    out.index_copy_(0, idx, out_p[0])
    return F.linear(out.reshape(B, T, -1), params.out_proj)


def gated_deltanet_decode(params: GDNParams, cfg: GDNConfig, hidden_BD: torch.Tensor,
                          cache: GDNLayerCache) -> torch.Tensor:
    """One decode token per sequence: hidden [B, D] -> out [B, D]; updates ``cache``."""
    h = hidden_BD.to(torch.bfloat16)
    mixed, z, a, b = _projections(params, cfg, h)
    out = gdn_decode_step(mixed, z, a, b, params.conv_w, params.A_log, params.dt_bias, params.norm_w,
                          cache.conv_state, cache.recurrent_state, eps=cfg.rms_norm_eps, **cfg.dims())
    cache.lengths = (cache.lengths + 1).to(torch.int32)
    return F.linear(out, params.out_proj)
