"""Optional JAX binding of libomx_gdn through XLA FFI custom calls (omegalax_amd.xla.binding).

Needs JAX with ROCm and libomx_gdn_xla.so, which omegalax_amd.build compiles only when
jaxlib's FFI headers are importable; nothing else in the package imports this module.
"""
