"""Host-side bf16 rounding for preparing bf16-exact inputs (numpy)."""
from __future__ import annotations

import numpy as np


def round_bf16(x):
    """Round to the nearest bfloat16 (ties to even); returns float32 holding bf16 values."""
    a = np.ascontiguousarray(np.asarray(x, dtype=np.float32))
    u = a.view(np.uint32).astype(np.uint64)
    u = (u + 0x7FFF + ((u >> 16) & 1)) & 0xFFFF0000
    out = u.astype(np.uint32).view(np.float32)
    return np.where(np.isnan(a), a, out).astype(np.float32)
