"""Host-side bf16 rounding for preparing bf16-exact inputs (numpy)."""
from __future__ import annotations

import numpy as np


def round_bf16(x):
    """Round to the nearest bfloat16 (ties to even); returns float32 holding bf16 values."""
    a = np.array(x, dtype=np.float32, copy=True, order="C")
    u = a.view(np.uint32)
    nan = np.isnan(a)
    # uint32 arithmetic: a finite value's sum cannot wrap (it rounds up to inf at most);
    # NaNs, whose sum may wrap, are restored below
    r = (u >> 16) & 1
    r += 0x7FFF
    u += r
    u &= 0xFFFF0000
    if nan.any():
        a[nan] = np.nan
    return a
