"""omegalax_amd: MI355X (gfx950) GatedDeltaNet path for omegalax's Qwen3.5 layer.

The compute lives in libomx_gdn.so (HIP kernels behind the C ABI of
include/omx_gdn.h); this package is the Python host side that mirrors the
reference's interface (omegalax/models/qwen3_5/deltanet.py).
"""
from .deltanet import (  # noqa: F401
    GDNError, chunk_gated_delta_rule, gdn_decode_step, gdn_prefill,
    recurrent_gated_delta_rule_step,
)

__version__ = "0.1.0"
