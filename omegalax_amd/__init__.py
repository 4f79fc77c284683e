"""omegalax_amd: MI355X (gfx950) GatedDeltaNet path for omegalax's Qwen3.5 layer.

The compute lives in libomx_gdn.so (HIP kernels behind the C ABI of
include/omx_gdn.h); this package is the Python host side that mirrors the
reference's interface (omegalax/models/qwen3_5/deltanet.py).
"""
from .deltanet import (  # noqa: F401
    GDNError, chunk_gated_delta_rule, chunk_gated_delta_rule_bwd, gdn_ab_projections,
    gdn_decode_step, gdn_prefill, gdn_prefill_bwd, qkv_conv_projection,
    recurrent_gated_delta_rule_step,
)
from .layer import (  # noqa: F401
    GDNConfig, GDNLayerCache, GDNParams, gated_deltanet_decode, gated_deltanet_forward,
    gated_deltanet_prefill_cache, gdn_params_from_hf, gdn_params_to_hf, load_gdn_layers,
    make_gdn_cache,
)
from .segments import lengths_to_cu_seqlens, right_pad_lengths, segment_ids_to_cu_seqlens  # noqa: F401

__version__ = "0.1.0"
