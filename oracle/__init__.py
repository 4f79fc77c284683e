"""CPU oracle for the Qwen3.5 GatedDeltaNet path -- TEST INFRASTRUCTURE ONLY.

This package is a from-scratch NumPy restatement of omegalax's gated-delta-rule
path (omegalax/models/qwen3_5/deltanet.py) and of the decode/initial-state
semantics the reference lacks (transformers' modeling_qwen3_5.py torch
functions).  It exists to check the HIP kernels.  Only ``tests/``,
``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of ``bench.py`` may
import it, and only as the checker or the timed CPU baseline -- never as the
product path.  ``omegalax_amd`` must not import anything from here.

Pinning status of each function is listed in ``oracle/gdn_oracle.py``'s
module docstring.
"""
